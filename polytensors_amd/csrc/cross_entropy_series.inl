// Cross entropy of a degree-K series of logits, one streaming pass per row.
//
// For a row z(t) = sum_k z_k t^k over C classes, exp(z(t)) = exp(z_0) e(t)
// with e_0 = 1, e_k = sum_{i=1..k} (i/k) z_i e_{k-i} (the exponential-series
// recurrence of /root/reference/src/polytensors/_plain.py:153-159 applied to
// [0, z_1, .., z_K]). Each thread streams its share of the row once, keeping
// a running maximum m of z_0 and the rescaled sums S_k = sum exp(z_0 - m) e_k;
// the per-thread states merge by the same rescaling (wavefront shuffles, then
// LDS across waves). Then, with n_k = S_k / S_0:
//   lse_0 = m + log S_0,
//   lse_k = n_k - sum_{i=1..k-1} (i/k) lse_i n_{k-i}   (log series, _plain.py:162-171),
//   loss_0 = lse_0 - z_0[y],  loss_k = lse_k - z_k[y]  (the log-softmax series at the
//   target, _plain.py:262-273, read by the per-order NLL of _dispatch.py:537-543).
// This equals the reference's route (centre at lse_0, exponentiate, sum, take
// the log series) up to rounding, with a single read of the logits.
#pragma once

#include "cross_entropy_series.h"
#include "series_math.h"

namespace pt {

constexpr int kCeThreads = 256;

template <typename A, int K>
__device__ __forceinline__ void accumulate_element(A x0, const A (&xk)[K + 1], A m, A (&S)[K + 1]) {
  const A p = exp_fast(x0 - m);
  A e[K + 1];
  e[0] = A(1);
#pragma unroll
  for (int k = 1; k <= K; ++k) {
    A s = A(0);
#pragma unroll
    for (int i = 1; i <= k; ++i) s += (A(i) * xk[i]) * e[k - i];
    e[k] = s * (A(1) / A(k));   // a compile-time reciprocal, not a division
  }
  S[0] += p;
#pragma unroll
  for (int k = 1; k <= K; ++k) S[k] += p * e[k];
}

template <typename A, int K>
__device__ __forceinline__ void rescale(A& m, A new_m, A (&S)[K + 1]) {
  if (new_m > m) {
    const A f = exp_fast(m - new_m);   // m = -inf gives 0 (S is zero then anyway)
#pragma unroll
    for (int k = 0; k <= K; ++k) S[k] *= f;
    m = new_m;
  }
}

// One block of THREADS threads per row. Logits are read with non-temporal
// 16-byte loads (each byte is read once; streaming them past the caches lifts
// the kernel from about 74% to 86% of HBM peak on MI355X), two vectors per
// order in flight per thread and iteration. With CAP every logit series is
// first replaced by its softcap cap * tanh(z / cap) (series_math.h), on the fly.
template <typename T, int K, int THREADS, bool CAP>
__global__ __launch_bounds__(THREADS) void cross_entropy_series_row_kernel(
    CPtrs<T> z, int64_t rows, int64_t classes, int64_t row_stride, bool vec_ok,
    const int64_t* __restrict__ target, int64_t ignore_index, MPtrs<typename AccOf<T>::type> loss,
    MPtrs<typename AccOf<T>::type> lse, typename AccOf<T>::type cap, typename AccOf<T>::type inv_cap) {
  using A = typename AccOf<T>::type;
  constexpr int V = VecWidth<T>::value;
  constexpr A kNegInf = -__builtin_huge_val();
  __shared__ A red_m[THREADS / kWave];
  __shared__ A red_s[THREADS / kWave][K + 1];

  const int64_t row = blockIdx.x;
  const int64_t base = row * row_stride;
  A m = kNegInf;
  A S[K + 1];
#pragma unroll
  for (int k = 0; k <= K; ++k) S[k] = A(0);

  int64_t scalar_from = 0;
  if (vec_ok) {
    constexpr int U = 2;
    const int64_t nvec = classes / V;
    int64_t j = threadIdx.x;
    for (; j + (U - 1) * THREADS < nvec; j += U * THREADS) {
      Vec<T, V> a[U][K + 1];
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int k = 0; k <= K; ++k) a[u][k] = load_vec_nt<T, V>(z.p[k] + base + (j + u * THREADS) * V);
      A x[U][V][K + 1];
      A hi = kNegInf;
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int e = 0; e < V; ++e) {
#pragma unroll
          for (int k = 0; k <= K; ++k) x[u][e][k] = to_acc(a[u][k].v[e]);
          if constexpr (CAP) softcap_series<A, K>(x[u][e], cap, inv_cap);
          hi = fmax(hi, x[u][e][0]);
        }
      rescale<A, K>(m, hi, S);
      if (m != kNegInf) {
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int e = 0; e < V; ++e) accumulate_element<A, K>(x[u][e][0], x[u][e], m, S);
      }
    }
    for (; j < nvec; j += THREADS) {
      Vec<T, V> a[K + 1];
#pragma unroll
      for (int k = 0; k <= K; ++k) a[k] = load_vec_nt<T, V>(z.p[k] + base + j * V);
      A x[V][K + 1];
      A hi = kNegInf;
#pragma unroll
      for (int e = 0; e < V; ++e) {
#pragma unroll
        for (int k = 0; k <= K; ++k) x[e][k] = to_acc(a[k].v[e]);
        if constexpr (CAP) softcap_series<A, K>(x[e], cap, inv_cap);
        hi = fmax(hi, x[e][0]);
      }
      rescale<A, K>(m, hi, S);
      if (m != kNegInf) {
#pragma unroll
        for (int e = 0; e < V; ++e) accumulate_element<A, K>(x[e][0], x[e], m, S);
      }
    }
    scalar_from = nvec * V;
  }
  for (int64_t col = scalar_from + threadIdx.x; col < classes; col += THREADS) {
    A x[K + 1];
#pragma unroll
    for (int k = 0; k <= K; ++k) x[k] = to_acc(z.p[k][base + col]);
    if constexpr (CAP) softcap_series<A, K>(x, cap, inv_cap);
    rescale<A, K>(m, x[0], S);
    if (m != kNegInf) accumulate_element<A, K>(x[0], x, m, S);
  }

  // Merge the per-thread (m, S) states: wave, then block.
  const A wm = wave_max(m);
  {
    const A f = (m == kNegInf) ? A(0) : exp_fast(m - wm);
#pragma unroll
    for (int k = 0; k <= K; ++k) S[k] = wave_sum(S[k] * f);
  }
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x % kWave) == 0) {
    red_m[wave] = wm;
#pragma unroll
    for (int k = 0; k <= K; ++k) red_s[wave][k] = S[k];
  }
  __syncthreads();
  if (threadIdx.x != 0) return;

  A M = kNegInf;
#pragma unroll
  for (int w = 0; w < THREADS / kWave; ++w) M = fmax(M, red_m[w]);
  A tot[K + 1];
#pragma unroll
  for (int k = 0; k <= K; ++k) tot[k] = A(0);
#pragma unroll
  for (int w = 0; w < THREADS / kWave; ++w) {
    const A f = (red_m[w] == kNegInf) ? A(0) : exp_acc(red_m[w] - M);
#pragma unroll
    for (int k = 0; k <= K; ++k) tot[k] += red_s[w][k] * f;
  }
  A L[K + 1];
  L[0] = M + log_acc(tot[0]);
  A nrm[K + 1];
#pragma unroll
  for (int k = 1; k <= K; ++k) nrm[k] = tot[k] / tot[0];
#pragma unroll
  for (int k = 1; k <= K; ++k) {
    A s = nrm[k];
#pragma unroll
    for (int i = 1; i < k; ++i) s -= (A(i) / A(k)) * L[i] * nrm[k - i];
    L[k] = s;
  }
  if (lse.p[0] != nullptr) {
#pragma unroll
    for (int k = 0; k <= K; ++k) lse.p[k][row] = L[k];
  }
  const int64_t y = target[row];
  const bool ignored = (y == ignore_index);
  const bool in_range = (y >= 0 && y < classes);
  A zy[K + 1];
#pragma unroll
  for (int k = 0; k <= K; ++k) zy[k] = in_range ? to_acc(z.p[k][base + y]) : A(0);
  if constexpr (CAP) softcap_series<A, K>(zy, cap, inv_cap);
#pragma unroll
  for (int k = 0; k <= K; ++k) {
    A v;
    if (ignored) {
      v = A(0);
    } else if (!in_range) {
      v = __builtin_nan("");   // an out-of-range class index poisons the loss instead of reading past the row
    } else {
      v = L[k] - zy[k];
    }
    loss.p[k][row] = v;
  }
}

// Deterministic reduction of per-row losses: block k sums order k in a fixed
// order and divides by the number of non-ignored targets for the mean.
template <typename A, int K>
__global__ __launch_bounds__(kCeThreads) void cross_entropy_series_reduce_kernel(
    const A* __restrict__ per_row /* [K+1][rows] */, int64_t rows, const int64_t* __restrict__ target,
    int64_t ignore_index, bool mean, MPtrs<A> out) {
  __shared__ A red[kCeThreads / kWave];
  __shared__ A redc[kCeThreads / kWave];
  const int k = blockIdx.x;
  A s = A(0), c = A(0);
  for (int64_t i = threadIdx.x; i < rows; i += kCeThreads) {
    s += per_row[k * rows + i];
    c += (target[i] != ignore_index) ? A(1) : A(0);
  }
  s = wave_sum(s);
  c = wave_sum(c);
  if ((threadIdx.x % kWave) == 0) {
    red[threadIdx.x / kWave] = s;
    redc[threadIdx.x / kWave] = c;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    A ts = A(0), tc = A(0);
#pragma unroll
    for (int w = 0; w < kCeThreads / kWave; ++w) {
      ts += red[w];
      tc += redc[w];
    }
    out.p[k][0] = mean ? ts / tc : ts;
  }
}

template <typename T, int K>
static int launch_ce_k(const CeArgs& a) {
  using A = typename AccOf<T>::type;
  constexpr int V = VecWidth<T>::value;
  CPtrs<T> z{};
  MPtrs<A> loss{}, lse{};
  bool vec_ok = (a.row_stride * static_cast<int64_t>(sizeof(T))) % 16 == 0;
  for (int k = 0; k <= K; ++k) {
    z.p[k] = static_cast<const T*>(a.z[k]);
    vec_ok = vec_ok && pt_host::aligned16(a.z[k]);
    if (a.lse != nullptr) lse.p[k] = static_cast<A*>(a.lse[k]);
  }
  A* per_row = static_cast<A*>(a.workspace);
  for (int k = 0; k <= K; ++k)
    loss.p[k] = a.reduction == PT_REDUCTION_NONE ? static_cast<A*>(a.loss[k]) : per_row + k * a.rows;
  // Long rows (>= 16 vectors per thread at 256 threads) take 512-thread blocks.
  const bool cap = a.softcap > 0.0;
  const A capv = cap ? static_cast<A>(a.softcap) : A(1);
  const A inv_cap = A(1) / capv;
#define PT_CE_LAUNCH(TH, CP)                                                                   \
  cross_entropy_series_row_kernel<T, K, TH, CP><<<dim3(a.rows), dim3(TH), 0, a.stream>>>(     \
      z, a.rows, a.classes, a.row_stride, vec_ok, a.target, a.ignore_index, loss, lse, capv, inv_cap)
  if (a.classes >= 4096 * static_cast<int64_t>(V)) {
    if (cap) PT_CE_LAUNCH(512, true);
    else PT_CE_LAUNCH(512, false);
  } else {
    if (cap) PT_CE_LAUNCH(kCeThreads, true);
    else PT_CE_LAUNCH(kCeThreads, false);
  }
#undef PT_CE_LAUNCH
  PT_LAUNCH_CHECK();
  if (a.reduction != PT_REDUCTION_NONE) {
    MPtrs<A> out{};
    for (int k = 0; k <= K; ++k) out.p[k] = static_cast<A*>(a.loss[k]);
    cross_entropy_series_reduce_kernel<A, K><<<dim3(K + 1), dim3(kCeThreads), 0, a.stream>>>(
        per_row, a.rows, a.target, a.ignore_index, a.reduction == PT_REDUCTION_MEAN, out);
    PT_LAUNCH_CHECK();
  }
  return PT_OK;
}

// ---------------------------------------------------------------------------
// Backward: the gradient series of the per-row losses, dz(t) = J(z(t))^T c(t)
// = c (*) (p - e_y), with p = exp series of (z - lse) the softmax series of the
// row (lse saved by the forward) and c the row's cotangent series; with a
// softcap, dz is further multiplied by the series of 1 - tanh(z / cap)^2.
// Generalises the reference's degree-1 kernel
// /root/reference/src/polytensors/_cross_entropy_kernels.py:58-85 to degree K.
// Ignored rows get zero. One block per row streams z once and writes dz once.
template <typename A, int K, bool CAP>
__device__ __forceinline__ void ce_bwd_element(const A (&x)[K + 1], bool is_target, const A (&lse)[K + 1],
                                               const A (&c)[K + 1], A cap, A inv_cap, A (&dz)[K + 1]) {
  A z[K + 1], dt[K + 1];
#pragma unroll
  for (int k = 0; k <= K; ++k) z[k] = x[k];
  if constexpr (CAP) softcap_series<A, K>(z, cap, inv_cap, dt);
  A ju[K + 1], p[K + 1];
#pragma unroll
  for (int k = 0; k <= K; ++k) ju[k] = A(k) * (z[k] - lse[k]);
  p[0] = exp_acc(z[0] - lse[0]);
#pragma unroll
  for (int k = 1; k <= K; ++k) {
    A s = A(0);
#pragma unroll
    for (int j = 1; j <= k; ++j) s = fma(ju[j], p[k - j], s);
    p[k] = s * (A(1) / A(k));
  }
  if (is_target) p[0] -= A(1);
#pragma unroll
  for (int k = K; k >= 0; --k) {
    A s = c[0] * p[k];
#pragma unroll
    for (int i = 1; i <= k; ++i) s = fma(c[i], p[k - i], s);
    dz[k] = s;
  }
  if constexpr (CAP) {
#pragma unroll
    for (int k = K; k >= 0; --k) {
      A s = dz[0] * dt[k];
#pragma unroll
      for (int i = 1; i <= k; ++i) s = fma(dz[i], dt[k - i], s);
      dz[k] = s;
    }
  }
}

// Two vectors per order in flight per thread (91 VGPRs, 5 waves per SIMD) measure
// about 1% faster than one (59 VGPRs, 8 waves) on the 8192 x 32000 fp32 rows.
constexpr int kCeBwdUnroll = 2;

template <typename T, int K, int THREADS, bool CAP>
__global__ __launch_bounds__(THREADS) void cross_entropy_series_bwd_kernel(
    CPtrs<T> z, int64_t classes, int64_t row_stride, bool vec_ok, const int64_t* __restrict__ target,
    int64_t ignore_index, CPtrs<typename AccOf<T>::type> lse_p, CPtrs<typename AccOf<T>::type> cot_p,
    MPtrs<T> dz, typename AccOf<T>::type cap, typename AccOf<T>::type inv_cap) {
  using A = typename AccOf<T>::type;
  constexpr int V = VecWidth<T>::value;
  const int64_t row = blockIdx.x;
  const int64_t base = row * row_stride, out = row * classes;
  const int64_t y = target[row];
  const bool ignored = (y == ignore_index);
  A lse[K + 1], c[K + 1];
#pragma unroll
  for (int k = 0; k <= K; ++k) {
    lse[k] = lse_p.p[k][row];
    c[k] = ignored ? A(0) : cot_p.p[k][row];
  }
  // U vectors per order in flight per thread and iteration, as in the forward.
  auto vec_step = [&](Vec<T, V> (&a)[K + 1], int64_t j) {
#pragma unroll
    for (int e = 0; e < V; e += 2) {
      A r[2][K + 1];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        A x[K + 1];
#pragma unroll
        for (int k = 0; k <= K; ++k) x[k] = vec_get(a[k], e + h);
        ce_bwd_element<A, K, CAP>(x, j * V + e + h == y, lse, c, cap, inv_cap, r[h]);
      }
#pragma unroll
      for (int k = 0; k <= K; ++k) vec_put2(a[k], e, r[0][k], r[1][k]);
    }
#pragma unroll
    for (int k = 0; k <= K; ++k) store_vec_nt<T, V>(dz.p[k] + out + j * V, a[k]);
  };
  int64_t scalar_from = 0;
  if (vec_ok) {
    constexpr int U = kCeBwdUnroll;
    const int64_t nvec = classes / V;
    int64_t j = threadIdx.x;
    for (; j + (U - 1) * THREADS < nvec; j += U * THREADS) {
      Vec<T, V> a[U][K + 1];
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int k = 0; k <= K; ++k) a[u][k] = load_vec_nt<T, V>(z.p[k] + base + (j + u * THREADS) * V);
#pragma unroll
      for (int u = 0; u < U; ++u) vec_step(a[u], j + u * THREADS);
    }
    for (; j < nvec; j += THREADS) {
      Vec<T, V> a[K + 1];
#pragma unroll
      for (int k = 0; k <= K; ++k) a[k] = load_vec_nt<T, V>(z.p[k] + base + j * V);
      vec_step(a, j);
    }
    scalar_from = nvec * V;
  }
  for (int64_t col = scalar_from + threadIdx.x; col < classes; col += THREADS) {
    A x[K + 1], r[K + 1];
#pragma unroll
    for (int k = 0; k <= K; ++k) x[k] = to_acc(z.p[k][base + col]);
    ce_bwd_element<A, K, CAP>(x, col == y, lse, c, cap, inv_cap, r);
#pragma unroll
    for (int k = 0; k <= K; ++k) dz.p[k][out + col] = from_acc<T>(r[k]);
  }
}

template <typename T, int K>
static int launch_ce_bwd_k(const CeBwdArgs& a) {
  using A = typename AccOf<T>::type;
  constexpr int V = VecWidth<T>::value;
  CPtrs<T> z{};
  CPtrs<A> lse{}, cot{};
  MPtrs<T> dz{};
  bool vec_ok = (a.row_stride * static_cast<int64_t>(sizeof(T))) % 16 == 0 &&
                (a.classes * static_cast<int64_t>(sizeof(T))) % 16 == 0;
  for (int k = 0; k <= K; ++k) {
    z.p[k] = static_cast<const T*>(a.z[k]);
    lse.p[k] = static_cast<const A*>(a.lse[k]);
    cot.p[k] = static_cast<const A*>(a.cot[k]);
    dz.p[k] = static_cast<T*>(a.dz[k]);
    vec_ok = vec_ok && pt_host::aligned16(a.z[k]) && pt_host::aligned16(a.dz[k]);
  }
  const bool cap = a.softcap > 0.0;
  const A capv = cap ? static_cast<A>(a.softcap) : A(1);
  const A inv_cap = A(1) / capv;
#define PT_CE_BWD_LAUNCH(TH, CP)                                                                     \
  cross_entropy_series_bwd_kernel<T, K, TH, CP><<<dim3(a.rows), dim3(TH), 0, a.stream>>>(           \
      z, a.classes, a.row_stride, vec_ok, a.target, a.ignore_index, lse, cot, dz, capv, inv_cap)
  if (a.classes >= 4096 * static_cast<int64_t>(V)) {
    if (cap) PT_CE_BWD_LAUNCH(512, true);
    else PT_CE_BWD_LAUNCH(512, false);
  } else {
    if (cap) PT_CE_BWD_LAUNCH(kCeThreads, true);
    else PT_CE_BWD_LAUNCH(kCeThreads, false);
  }
#undef PT_CE_BWD_LAUNCH
  PT_LAUNCH_CHECK();
  return PT_OK;
}

template <typename T>
int launch_ce_bwd(const CeBwdArgs& a) {
  switch (a.degree) {
    case 0: return launch_ce_bwd_k<T, 0>(a);
    case 1: return launch_ce_bwd_k<T, 1>(a);
    case 2: return launch_ce_bwd_k<T, 2>(a);
    case 3: return launch_ce_bwd_k<T, 3>(a);
    case 4: return launch_ce_bwd_k<T, 4>(a);
    case 5: return launch_ce_bwd_k<T, 5>(a);
    case 6: return launch_ce_bwd_k<T, 6>(a);
    case 7: return launch_ce_bwd_k<T, 7>(a);
    case 8: return launch_ce_bwd_k<T, 8>(a);
    default: break;
  }
  pt_host::set_error("cross-entropy series backward: degree outside 0..PT_MAX_DEGREE");
  return PT_UNSUPPORTED;
}

template <typename T>
int launch_ce(const CeArgs& a) {
  switch (a.degree) {
    case 0: return launch_ce_k<T, 0>(a);
    case 1: return launch_ce_k<T, 1>(a);
    case 2: return launch_ce_k<T, 2>(a);
    case 3: return launch_ce_k<T, 3>(a);
    case 4: return launch_ce_k<T, 4>(a);
    case 5: return launch_ce_k<T, 5>(a);
    case 6: return launch_ce_k<T, 6>(a);
    case 7: return launch_ce_k<T, 7>(a);
    case 8: return launch_ce_k<T, 8>(a);
    default: break;
  }
  pt_host::set_error("cross-entropy series: degree outside 0..PT_MAX_DEGREE");
  return PT_UNSUPPORTED;
}

}  // namespace pt
