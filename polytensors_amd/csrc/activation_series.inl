// Elementwise activations of a degree-K series, one streaming pass.
//
// For u(t) = sum_k u_k t^k the coefficients of f(u(t)) follow from an ODE that
// f satisfies, matched order by order (k y_k = sum_j j u_j d_{k-j} for
// y' = d(y) u'), all in registers:
//   exp      y' = y u'
//   tanh     y' = d u',  d = 1 - y^2
//   sigmoid  y' = d u',  d = y - y^2 (d_0 = e / (1 + e)^2 with e = exp(-|u_0|),
//            so a rounded y_0 = 1 keeps its small derivative)
//   gelu     x Phi(x): P' = p u', p' = -u p u' (p the normal density), y = u (*) P
//   silu     u (*) sigmoid(u)
//   gelu_tanh 0.5 u (*) (1 + tanh(v)),  v = sqrt(2/pi) (u + 0.044715 u^3)
//   log      y_k = n_k - sum_{i<k} (i/k) y_i n_{k-i},  n = u / u_0
//   sin/cos  s' = c u', c' = -s u' (both series formed together)
//   sqrt/rsqrt y = u^p, p = 1/2 or -1/2: k u_0 y_k = sum_{j=1..k} ((p+1) j - k) u_j y_{k-j}
//            (J.C.P. Miller's power recurrence; for p = -1/2 the reference's poly_rsqrt,
//            /root/reference/src/polytensors/_series.py:83-96)
// These equal the reference's plain-range rules -- Faa di Bruno composition of
// the derivatives at u_0 for gelu/tanh/sigmoid
// (/root/reference/src/polytensors/_plain.py:174-259), plain_exp/plain_log
// (_plain.py:153-171) -- and its default-mode jets for silu and gelu_tanh
// (/root/reference/src/polytensors/_activations.py:89-115), up to rounding.
//
// Backward (the native *_backward operations on series): dx = g (*) D with
// D the series of f'(u(t)): gelu D = P + u (*) p; silu D = S + u (*) dS;
// gelu_tanh D = 0.5 (1 + T) + 0.5 u (*) dT (*) q, q = v'(u);
// tanh and sigmoid take the forward OUTPUT series Y (as aten.tanh_backward
// does): D = 1 - Y (*) Y and Y - Y (*) Y (_plain.py:316-325).
//
// Each thread streams one 16-byte vector of every order per step with
// non-temporal accesses (every byte is touched once).
#pragma once

#include <algorithm>

#include "activation_series.h"
#include "series_math.h"

namespace pt {

constexpr int kActThreads = 256;

template <typename A, int K>
__device__ __forceinline__ void sigmoid_series(const A (&u)[K + 1], const A (&ju)[K + 1], A (&y)[K + 1],
                                               A (&d)[K + 1]) {
  const A e = exp_acc(-fabs(u[0]));
  const A inv = A(1) / (A(1) + e);
  y[0] = u[0] >= A(0) ? inv : e * inv;
  d[0] = e * inv * inv;
  output_ode<A, K, true>(ju, y, d);
}

// Phi-series P and density series p of the standard normal along u; w = u (*) p.
template <typename A, int K>
__device__ __forceinline__ void normal_series(const A (&u)[K + 1], const A (&ju)[K + 1], A (&P)[K + 1],
                                              A (&p)[K + 1], A (&w)[K + 1]) {
  P[0] = normal_cdf(u[0]);
  p[0] = normal_density(u[0]);
  w[0] = u[0] * p[0];
#pragma unroll
  for (int k = 1; k <= K; ++k) {
    A s = A(0), r = A(0);
#pragma unroll
    for (int j = 1; j <= k; ++j) {
      s = fma(ju[j], p[k - j], s);
      r = fma(ju[j], w[k - j], r);
    }
    P[k] = s * (A(1) / A(k));
    p[k] = -r * (A(1) / A(k));
    A q = u[0] * p[k];
#pragma unroll
    for (int a = 1; a <= k; ++a) q = fma(u[a], p[k - a], q);
    w[k] = q;
  }
}

// tanh-GELU pieces: T = tanh(v), dT = 1 - T^2, q = v'(u) along u.
template <typename A, int K>
__device__ __forceinline__ void gelu_tanh_series(const A (&u)[K + 1], A (&T)[K + 1], A (&dT)[K + 1],
                                                 A (&q)[K + 1]) {
  constexpr A kC = A(0.79788456080286535588);   // sqrt(2/pi)
  constexpr A kA = A(0.044715);
  A u2[K + 1], u3[K + 1], v[K + 1], jv[K + 1];
  cauchy_mul<A, K>(u, u, u2);
  cauchy_mul<A, K>(u2, u, u3);
#pragma unroll
  for (int k = 0; k <= K; ++k) {
    v[k] = kC * fma(kA, u3[k], u[k]);
    jv[k] = A(k) * v[k];
    q[k] = kC * A(3) * kA * u2[k];
  }
  q[0] += kC;
  tanh_pair(v[0], T[0], dT[0]);
  output_ode<A, K, false>(jv, T, dT);
}

// out = f(u) series (forward) or g (*) f'(.) series (backward), by kind.
template <typename A, int K, bool BWD>
__device__ __forceinline__ void activation_element(int kind, const A (&u)[K + 1], const A (&g)[K + 1],
                                                   A (&out)[K + 1]) {
  A ju[K + 1];
#pragma unroll
  for (int k = 0; k <= K; ++k) ju[k] = A(k) * u[k];
  A D[K + 1];   // backward: the derivative series
  switch (kind) {
    case PT_ACT_EXP: {
      out[0] = exp_acc(u[0]);
#pragma unroll
      for (int k = 1; k <= K; ++k) {
        A s = A(0);
#pragma unroll
        for (int j = 1; j <= k; ++j) s = fma(ju[j], out[k - j], s);
        out[k] = s * (A(1) / A(k));
      }
      return;
    }
    case PT_ACT_LOG: {
      const A inv0 = A(1) / u[0];
      out[0] = log_acc(u[0]);
      A nrm[K + 1];
#pragma unroll
      for (int k = 1; k <= K; ++k) nrm[k] = u[k] * inv0;
#pragma unroll
      for (int k = 1; k <= K; ++k) {
        A s = nrm[k];
#pragma unroll
        for (int i = 1; i < k; ++i) s = fma(-(A(i) / A(k)) * out[i], nrm[k - i], s);
        out[k] = s;
      }
      return;
    }
    case PT_ACT_SIN:
    case PT_ACT_COS: {
      A sn[K + 1], cs[K + 1];
      sn[0] = sin(u[0]);
      cs[0] = cos(u[0]);
#pragma unroll
      for (int k = 1; k <= K; ++k) {
        A a = A(0), b = A(0);
#pragma unroll
        for (int j = 1; j <= k; ++j) {
          a = fma(ju[j], cs[k - j], a);
          b = fma(ju[j], sn[k - j], b);
        }
        sn[k] = a * (A(1) / A(k));
        cs[k] = -b * (A(1) / A(k));
      }
#pragma unroll
      for (int k = 0; k <= K; ++k) out[k] = kind == PT_ACT_SIN ? sn[k] : cs[k];
      return;
    }
    case PT_ACT_SQRT:
    case PT_ACT_RSQRT: {
      const A root = sqrt(u[0]);
      const A p1 = kind == PT_ACT_SQRT ? A(1.5) : A(0.5);   // p + 1
      const A inv0 = A(1) / u[0];
      out[0] = kind == PT_ACT_SQRT ? root : A(1) / root;
#pragma unroll
      for (int k = 1; k <= K; ++k) {
        A s = A(0);
#pragma unroll
        for (int j = 1; j <= k; ++j) s = fma((p1 * A(j) - A(k)) * u[j], out[k - j], s);
        out[k] = s * inv0 * (A(1) / A(k));
      }
      return;
    }
    case PT_ACT_TANH: {
      if constexpr (BWD) {   // u is the forward output Y: D = 1 - Y (*) Y
        cauchy_mul<A, K>(u, u, D);
#pragma unroll
        for (int k = 0; k <= K; ++k) D[k] = -D[k];
        D[0] += A(1);
        break;
      } else {
        A d[K + 1];
        tanh_series<A, K>(u, ju, out, d);
        return;
      }
    }
    case PT_ACT_SIGMOID: {
      if constexpr (BWD) {   // u is the forward output Y: D = Y - Y (*) Y
        cauchy_mul<A, K>(u, u, D);
#pragma unroll
        for (int k = 0; k <= K; ++k) D[k] = u[k] - D[k];
        break;
      } else {
        A d[K + 1];
        sigmoid_series<A, K>(u, ju, out, d);
        return;
      }
    }
    case PT_ACT_SILU: {
      A S[K + 1], dS[K + 1];
      sigmoid_series<A, K>(u, ju, S, dS);
      if constexpr (BWD) {   // D = S + u (*) dS
        cauchy_mul<A, K>(u, dS, D);
#pragma unroll
        for (int k = 0; k <= K; ++k) D[k] += S[k];
        break;
      } else {
        cauchy_mul<A, K>(u, S, out);
        return;
      }
    }
    case PT_ACT_GELU: {
      A P[K + 1], p[K + 1], w[K + 1];
      normal_series<A, K>(u, ju, P, p, w);
      if constexpr (BWD) {   // D = P + u (*) p
#pragma unroll
        for (int k = 0; k <= K; ++k) D[k] = P[k] + w[k];
        break;
      } else {
        cauchy_mul<A, K>(u, P, out);
        return;
      }
    }
    default: {   // PT_ACT_GELU_TANH (the launcher admits no other kind)
      A T[K + 1], dT[K + 1], q[K + 1];
      gelu_tanh_series<A, K>(u, T, dT, q);
      if constexpr (BWD) {   // D = 0.5 (1 + T) + 0.5 u (*) (dT (*) q)
        A r[K + 1], ur[K + 1];
        cauchy_mul<A, K>(dT, q, r);
        cauchy_mul<A, K>(u, r, ur);
#pragma unroll
        for (int k = 0; k <= K; ++k) D[k] = A(0.5) * (T[k] + ur[k]);
        D[0] += A(0.5);
        break;
      } else {   // 0.5 (u + u (*) T)
        cauchy_mul<A, K>(u, T, out);
#pragma unroll
        for (int k = 0; k <= K; ++k) out[k] = A(0.5) * (u[k] + out[k]);
        return;
      }
    }
  }
  if constexpr (BWD) cauchy_mul<A, K>(g, D, out);
}

// One 16-byte vector per order and thread (a block per 256 vectors) measured
// 1.5% faster than a grid capped at 32 blocks per CU striding over the rest;
// the grid-stride loop remains for inputs past kActMaxBlocks blocks.
constexpr int64_t kActMaxBlocks = int64_t(1) << 20;

template <typename T, int K, bool BWD>
__global__ __launch_bounds__(kActThreads) void activation_series_kernel(
    int kind, CPtrs<T, kMaxElementwiseOrders> x, CPtrs<T, kMaxElementwiseOrders> g,
    MPtrs<T, kMaxElementwiseOrders> y, int64_t numel, bool vec) {
  using A = typename AccOf<T>::type;
  constexpr int V = VecWidth<T>::value;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kActThreads;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kActThreads + threadIdx.x;
  int64_t scalar_from = 0;
  if (vec) {
    const int64_t nvec = numel / V;
    for (int64_t i = first; i < nvec; i += stride) {
      Vec<T, V> rx[K + 1], rg[BWD ? K + 1 : 1];
#pragma unroll
      for (int k = 0; k <= K; ++k) rx[k] = load_vec_nt<T, V>(x.p[k] + i * V);
      if constexpr (BWD) {
#pragma unroll
        for (int k = 0; k <= K; ++k) rg[k] = load_vec_nt<T, V>(g.p[k] + i * V);
      }
      A fx[K + 1][V], fg[BWD ? K + 1 : 1][V];
#pragma unroll
      for (int k = 0; k <= K; ++k) unpack_vec(rx[k], fx[k]);
      if constexpr (BWD) {
#pragma unroll
        for (int k = 0; k <= K; ++k) unpack_vec(rg[k], fg[k]);
      }
#pragma unroll
      for (int e = 0; e < V; ++e) {
        A u[K + 1], gv[K + 1], out[K + 1];
#pragma unroll
        for (int k = 0; k <= K; ++k) {
          u[k] = fx[k][e];
          gv[k] = BWD ? fg[BWD ? k : 0][e] : A(0);
        }
        activation_element<A, K, BWD>(kind, u, gv, out);
#pragma unroll
        for (int k = 0; k <= K; ++k) fx[k][e] = out[k];
      }
#pragma unroll
      for (int k = 0; k <= K; ++k) {
        pack_vec(fx[k], rx[k]);
        store_vec_nt<T, V>(y.p[k] + i * V, rx[k]);
      }
    }
    scalar_from = nvec * V;
  }
  for (int64_t i = scalar_from + first; i < numel; i += stride) {
    A u[K + 1], gv[K + 1], out[K + 1];
#pragma unroll
    for (int k = 0; k <= K; ++k) {
      u[k] = to_acc(x.p[k][i]);
      gv[k] = BWD ? to_acc(g.p[k][i]) : A(0);
    }
    activation_element<A, K, BWD>(kind, u, gv, out);
#pragma unroll
    for (int k = 0; k <= K; ++k) y.p[k][i] = from_acc<T>(out[k]);
  }
}

template <typename T, int K>
static int launch_activation_k(const ActArgs& a) {
  constexpr int V = VecWidth<T>::value;
  CPtrs<T, kMaxElementwiseOrders> x{}, g{};
  MPtrs<T, kMaxElementwiseOrders> y{};
  // 16-byte vectors of every order in registers up to 72 values per thread; above that (16-bit
  // types past degree 8) the element-by-element path, which holds one value per order
  bool vec = (K + 1) * V <= 72;
  for (int k = 0; k <= K; ++k) {
    x.p[k] = static_cast<const T*>(a.x[k]);
    y.p[k] = static_cast<T*>(a.y[k]);
    vec = vec && pt_host::aligned16(a.x[k]) && pt_host::aligned16(a.y[k]);
    if (a.backward) {
      g.p[k] = static_cast<const T*>(a.g[k]);
      vec = vec && pt_host::aligned16(a.g[k]);
    }
  }
  const int64_t work = vec ? (a.numel / V + a.numel % V) : a.numel;
  const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>((work + kActThreads - 1) / kActThreads, kActMaxBlocks));
  if (a.backward) {
    activation_series_kernel<T, K, true><<<dim3(blocks), dim3(kActThreads), 0, a.stream>>>(
        a.kind, x, g, y, a.numel, vec);
  } else {
    activation_series_kernel<T, K, false><<<dim3(blocks), dim3(kActThreads), 0, a.stream>>>(
        a.kind, x, g, y, a.numel, vec);
  }
  PT_LAUNCH_CHECK();
  return PT_OK;
}

template <typename T>
int launch_activation(const ActArgs& a) {
  switch (a.degree) {
    case 0: return launch_activation_k<T, 0>(a);
    case 1: return launch_activation_k<T, 1>(a);
    case 2: return launch_activation_k<T, 2>(a);
    case 3: return launch_activation_k<T, 3>(a);
    case 4: return launch_activation_k<T, 4>(a);
    case 5: return launch_activation_k<T, 5>(a);
    case 6: return launch_activation_k<T, 6>(a);
    case 7: return launch_activation_k<T, 7>(a);
    case 8: return launch_activation_k<T, 8>(a);
    case 9: return launch_activation_k<T, 9>(a);
    case 10: return launch_activation_k<T, 10>(a);
    case 11: return launch_activation_k<T, 11>(a);
    case 12: return launch_activation_k<T, 12>(a);
    case 13: return launch_activation_k<T, 13>(a);
    case 14: return launch_activation_k<T, 14>(a);
    case 15: return launch_activation_k<T, 15>(a);
    case 16: return launch_activation_k<T, 16>(a);
    default: break;
  }
  pt_host::set_error("activation series: degree outside 0..PT_MAX_ELEMENTWISE_DEGREE");
  return PT_UNSUPPORTED;
}

}  // namespace pt
