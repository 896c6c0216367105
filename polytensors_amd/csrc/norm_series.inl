// RMSNorm / LayerNorm of a degree-K series along the last dimension.
//
// Per row of n elements with coefficients x_0..x_K:
//   RMSNorm:   c_k = x_k
//   LayerNorm: c_k = x_k - mean(x_k)
//   s_k = mean_n( sum_{i+j=k} c_i c_j ),  s_0 += eps
//   r   = rsqrt series of s:  r_0 = 1/sqrt(s_0),
//         r_k = -sum_{i=1..k} ((2k-i)/(2k)) (s_i/s_0) r_{k-i}
//         (the recurrence of /root/reference/src/polytensors/_series.py:83-96,
//          from 2 s r' + s' r = 0)
//   z_k = sum_{i+j=k} c_i r_j,  then y = z (*) w (+ b)  (Cauchy products).
//
// Register path: every coefficient of a row is loaded once into VGPRs with
// 16-byte loads, the K+1 row sums are reduced with DPP and lane exchanges
// within each wave (and LDS across the row's waves), and y is written once:
// one HBM read and one HBM write of the series. Streaming path (rows too long for
// registers, or unaligned rows): the same math re-reading x per pass.
#pragma once

#include <type_traits>

#include "norm_series.h"

namespace pt {

constexpr int kNormThreads = 256;

template <typename A, int K>
__device__ __forceinline__ void rsqrt_series(const A (&sums)[K + 1], A inv_n, A eps,
                                             A (&r)[K + 1]) {
  const A s0 = sums[0] * inv_n + eps;
  r[0] = rsqrt_acc(s0);
  const A inv_s0 = A(1) / s0;
  A u[K + 1];
#pragma unroll
  for (int k = 1; k <= K; ++k) u[k] = (sums[k] * inv_n) * inv_s0;
#pragma unroll
  for (int k = 1; k <= K; ++k) {
    A acc = A(0);
#pragma unroll
    for (int i = 1; i <= k; ++i)
      acc += (A(2 * k - i) / A(2 * k)) * u[i] * r[k - i];
    r[k] = -acc;
  }
}

// sum_{i+j=k} c_i c_j using the symmetry of the square.
template <typename A, int K>
__device__ __forceinline__ A cauchy_square(const A (&c)[K + 1], int k) {
  A half = A(0);
#pragma unroll
  for (int i = 0; i <= K; ++i)
    if (2 * i < k) half += c[i] * c[k - i];
  A mid = (k % 2 == 0) ? c[k / 2] * c[k / 2] : A(0);
  return A(2) * half + mid;
}

// Sum of N values over the `tpr` threads of one row (tpr a multiple of 64,
// uniform across the block): wavefront shuffles, then LDS across the row's waves.
template <typename A, int N>
__device__ __forceinline__ void row_sums_n(A (&v)[N], A* red /* [waves][N] */, int tpr) {
#pragma unroll
  for (int k = 0; k < N; ++k) v[k] = wave_sum(v[k]);
  if (tpr > kWave) {
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x % kWave) == 0) {
#pragma unroll
      for (int k = 0; k < N; ++k) red[wave * N + k] = v[k];
    }
    __syncthreads();
    const int waves = tpr / kWave;
    const int first = (threadIdx.x / tpr) * waves;
#pragma unroll
    for (int k = 0; k < N; ++k) {
      A s = A(0);
      for (int w = 0; w < waves; ++w) s += red[(first + w) * N + k];
      v[k] = s;
    }
  }
}

template <typename A, int K>
__device__ __forceinline__ void row_sums(A (&v)[K + 1], A* red /* [waves][K+1] */, int tpr) {
  row_sums_n<A, K + 1>(v, red, tpr);
}

template <typename A, int K>
__device__ __forceinline__ void apply_affine(A (&z)[K + 1], const A (&w)[K + 1], int w_orders,
                                             const A (&b)[K + 1], int b_orders) {
  if (w_orders == 1) {
#pragma unroll
    for (int k = 0; k <= K; ++k) z[k] *= w[0];
  } else if (w_orders > 1) {
    A out[K + 1];
#pragma unroll
    for (int k = 0; k <= K; ++k) {
      A s = z[0] * w[k];
#pragma unroll
      for (int i = 1; i <= k; ++i) s += z[i] * w[k - i];
      out[k] = s;
    }
#pragma unroll
    for (int k = 0; k <= K; ++k) z[k] = out[k];
  }
  if (b_orders >= 1) {
    z[0] += b[0];
    if (b_orders > 1) {
#pragma unroll
      for (int k = 1; k <= K; ++k) z[k] += b[k];
    }
  }
}

// ---------------------------------------------------------------------------
// Register-resident kernel. `tpr` threads share a row (a multiple of 64; a
// block holds blockDim.x / tpr rows), each thread owns CHUNKS 16-byte vectors
// of every order, kept in their storage type (a bf16 row costs half the
// VGPRs of its float values) and unpacked where used. The arithmetic is kept
// lean so that the kernel stays HBM-bound: the squared series takes one FMA
// per element and order pair (the products c_i c_j with i < j are summed once
// and doubled once per thread), the weight is folded into the coefficients
// before the output Cauchy product, bf16 results are packed two per
// instruction, and the row's rsqrt series costs one division. The series is
// read and written with non-temporal 16-byte accesses: each byte is touched
// once, and streaming it past the caches lifts a read+write stream from about
// 5.4 to 5.8 TB/s on MI355X. Affine terms here are ordinary (one order).
template <typename T, int K, int CHUNKS, bool LAYER>
__global__ __launch_bounds__(1024) void norm_series_reg_kernel(
    CPtrs<T> x, const T* __restrict__ w, const T* __restrict__ b, MPtrs<T> y, int64_t rows, int n,
    int tpr, typename AccOf<T>::type eps, typename AccOf<T>::type inv_n) {
  using A = typename AccOf<T>::type;
  constexpr int V = VecWidth<T>::value;
  __shared__ A red[2][1024 / kWave][K + 1];

  const int tid = threadIdx.x % tpr;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (blockDim.x / tpr) + threadIdx.x / tpr;
  const bool active = row < rows;
  const int64_t base = row * static_cast<int64_t>(n);

  // Every load is issued unconditionally (lanes past the row or past rows read
  // vector 0, which exists) and then masked: a load under a per-lane branch is
  // waited for where the branch ends, which would serialize the loads. The
  // weight and bias vectors are fetched with the input.
  Vec<T, V> raw[CHUNKS][K + 1], wv[CHUNKS], bv[CHUNKS];
  const T* wp = w != nullptr ? w : x.p[0];
  const T* bp = b != nullptr ? b : x.p[0];
#pragma unroll
  for (int ch = 0; ch < CHUNKS; ++ch) {
    const int col = (ch * tpr + tid) * V;
    const bool in = active && col < n;
    const int64_t at = in ? base + col : 0;
#pragma unroll
    for (int k = 0; k <= K; ++k) raw[ch][k] = load_vec_nt<T, V>(x.p[k] + at);
    wv[ch] = load_vec<T, V>(wp + (in ? col : 0));
    bv[ch] = load_vec<T, V>(bp + (in ? col : 0));
  }
#pragma unroll
  for (int ch = 0; ch < CHUNKS; ++ch) {
    const bool in = active && (ch * tpr + tid) * V < n;
#pragma unroll
    for (int k = 0; k <= K; ++k)
#pragma unroll
      for (int e = 0; e < V; ++e) raw[ch][k].v[e] = in ? raw[ch][k].v[e] : from_acc<T>(A(0));
  }

  // mean[k] stays zero for RMSNorm; padding elements are excluded below.
  A mean[K + 1];
#pragma unroll
  for (int k = 0; k <= K; ++k) mean[k] = A(0);
  if constexpr (LAYER) {
#pragma unroll
    for (int ch = 0; ch < CHUNKS; ++ch)
#pragma unroll
      for (int k = 0; k <= K; ++k)
#pragma unroll
        for (int e = 0; e < V; ++e) mean[k] += vec_get(raw[ch][k], e);
    row_sums<A, K>(mean, &red[0][0][0], tpr);
#pragma unroll
    for (int k = 0; k <= K; ++k) mean[k] *= inv_n;
  }

  // cross[k] = sum over i < k - i of c_i c_{k-i};  sq[k] = c_{k/2}^2 (k even).
  A cross[K + 1], sq[K + 1];
#pragma unroll
  for (int k = 0; k <= K; ++k) cross[k] = sq[k] = A(0);
#pragma unroll
  for (int ch = 0; ch < CHUNKS; ++ch) {
    const int col = (ch * tpr + tid) * V;
    if (!(active && col < n)) continue;
#pragma unroll
    for (int e = 0; e < V; ++e) {
      A c[K + 1];
#pragma unroll
      for (int k = 0; k <= K; ++k) c[k] = LAYER ? vec_get(raw[ch][k], e) - mean[k] : vec_get(raw[ch][k], e);
#pragma unroll
      for (int k = 0; k <= K; ++k) {
#pragma unroll
        for (int i = 0; 2 * i < k; ++i) cross[k] = fma(c[i], c[k - i], cross[k]);
        if (k % 2 == 0) sq[k] = fma(c[k / 2], c[k / 2], sq[k]);
      }
    }
  }
  A sums[K + 1];
#pragma unroll
  for (int k = 0; k <= K; ++k) sums[k] = A(2) * cross[k] + sq[k];
  row_sums<A, K>(sums, &red[1][0][0], tpr);

  A r[K + 1];
  rsqrt_series<A, K>(sums, inv_n, eps, r);

  if (!active) return;
#pragma unroll
  for (int ch = 0; ch < CHUNKS; ++ch) {
    const int col = (ch * tpr + tid) * V;
    if (col >= n) continue;
    A wf[V], bf[V];
    unpack_vec(wv[ch], wf);
    unpack_vec(bv[ch], bf);
#pragma unroll
    for (int e = 0; e < V; ++e) {
      wf[e] = w != nullptr ? wf[e] : A(1);
      bf[e] = b != nullptr ? bf[e] : A(0);
    }
    // Elements in pairs: y_k = sum_i (w c_i) r_{k-i}, written over the consumed inputs.
#pragma unroll
    for (int e = 0; e < V; e += 2) {
      A out[2][K + 1];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        A c[K + 1];
#pragma unroll
        for (int k = 0; k <= K; ++k) {
          const A v = vec_get(raw[ch][k], e + h);
          c[k] = (LAYER ? v - mean[k] : v) * wf[e + h];
        }
#pragma unroll
        for (int k = K; k >= 0; --k) {
          A s = c[0] * r[k];
#pragma unroll
          for (int i = 1; i <= k; ++i) s = fma(c[i], r[k - i], s);
          out[h][k] = (k == 0) ? s + bf[e + h] : s;
        }
      }
#pragma unroll
      for (int k = 0; k <= K; ++k) vec_put2(raw[ch][k], e, out[0][k], out[1][k]);
    }
#pragma unroll
    for (int k = 0; k <= K; ++k) store_vec_nt<T, V>(y.p[k] + base + col, raw[ch][k]);
  }
}

// ---------------------------------------------------------------------------
// Streaming kernel: one 256-thread block per row, scalar accesses, any n.
template <typename T, int K, bool LAYER>
__global__ __launch_bounds__(kNormThreads) void norm_series_stream_kernel(
    CPtrs<T> x, CPtrs<T> w, int w_orders, CPtrs<T> b, int b_orders, MPtrs<T> y,
    int64_t rows, int64_t n, typename AccOf<T>::type eps, typename AccOf<T>::type inv_n) {
  using A = typename AccOf<T>::type;
  __shared__ A red[2][kNormThreads / kWave][K + 1];
  const int64_t row = blockIdx.x;
  const int64_t base = row * n;

  A mean[K + 1];
#pragma unroll
  for (int k = 0; k <= K; ++k) mean[k] = A(0);
  if constexpr (LAYER) {
    for (int64_t col = threadIdx.x; col < n; col += kNormThreads)
#pragma unroll
      for (int k = 0; k <= K; ++k) mean[k] += to_acc(x.p[k][base + col]);
    row_sums<A, K>(mean, &red[0][0][0], kNormThreads);
#pragma unroll
    for (int k = 0; k <= K; ++k) mean[k] *= inv_n;
  }

  A sums[K + 1];
#pragma unroll
  for (int k = 0; k <= K; ++k) sums[k] = A(0);
  for (int64_t col = threadIdx.x; col < n; col += kNormThreads) {
    A c[K + 1];
#pragma unroll
    for (int k = 0; k <= K; ++k) c[k] = to_acc(x.p[k][base + col]) - mean[k];
#pragma unroll
    for (int k = 0; k <= K; ++k) sums[k] += cauchy_square<A, K>(c, k);
  }
  row_sums<A, K>(sums, &red[1][0][0], kNormThreads);
  A r[K + 1];
  rsqrt_series<A, K>(sums, inv_n, eps, r);

  for (int64_t col = threadIdx.x; col < n; col += kNormThreads) {
    A c[K + 1], z[K + 1], wv[K + 1], bv[K + 1];
#pragma unroll
    for (int k = 0; k <= K; ++k) c[k] = to_acc(x.p[k][base + col]) - mean[k];
#pragma unroll
    for (int k = 0; k <= K; ++k) {
      if (k < w_orders) wv[k] = to_acc(w.p[k][col]);
      if (k < b_orders) bv[k] = to_acc(b.p[k][col]);
    }
#pragma unroll
    for (int k = 0; k <= K; ++k) {
      A s = c[0] * r[k];
#pragma unroll
      for (int i = 1; i <= k; ++i) s += c[i] * r[k - i];
      z[k] = s;
    }
    apply_affine<A, K>(z, wv, w_orders, bv, b_orders);
#pragma unroll
    for (int k = 0; k <= K; ++k) y.p[k][base + col] = from_acc<T>(z[k]);
  }
}

// ---------------------------------------------------------------------------


template <typename T>
static bool norm_args_aligned(const NormArgs& a) {
  constexpr int V = VecWidth<T>::value;
  if (a.n % V != 0) return false;
  for (int k = 0; k <= a.degree; ++k)
    if (!pt_host::aligned16(a.x[k]) || !pt_host::aligned16(a.y[k])) return false;
  for (int k = 0; k < a.w_orders; ++k)
    if (!pt_host::aligned16(a.w[k])) return false;
  for (int k = 0; k < a.b_orders; ++k)
    if (!pt_host::aligned16(a.b[k])) return false;
  return true;
}

template <typename T, int K, bool LAYER>
static int launch_norm_k(const NormArgs& a) {
  using A = typename AccOf<T>::type;
  constexpr int V = VecWidth<T>::value;
  CPtrs<T> x{}, w{}, b{};
  MPtrs<T> y{};
  for (int k = 0; k <= K; ++k) {
    x.p[k] = static_cast<const T*>(a.x[k]);
    y.p[k] = static_cast<T*>(a.y[k]);
  }
  for (int k = 0; k < a.w_orders; ++k) w.p[k] = static_cast<const T*>(a.w[k]);
  for (int k = 0; k < a.b_orders; ++k) b.p[k] = static_cast<const T*>(a.b[k]);
  const A eps = static_cast<A>(a.eps);
  const A inv_n = A(1) / static_cast<A>(a.n);

  // Register path: ordinary affine terms, aligned rows, and at most kRawBudget
  // VGPRs of raw row data per thread (4 per 16-byte vector) -- the budget under
  // which no instantiation spills in a 1024-thread block (LayerNorm keeps its
  // means live too).
  constexpr int kRawBudget = LAYER ? 32 : 56;
  const bool plain_affine = a.w_orders <= 1 && a.b_orders <= 1;
  if (plain_affine && norm_args_aligned<T>(a) && a.n <= (1 << 30)) {
    const int64_t vecs = a.n / V;
    int chunks = 0;
    for (int c : {1, 2, 4}) {
      if (vecs <= 1024 * c && 4 * (K + 1) * c * static_cast<int>(sizeof(A) / 4) <= kRawBudget) {
        chunks = c;
        break;
      }
    }
    if (chunks > 0) {
      int tpr = static_cast<int>(((vecs + chunks - 1) / chunks + kWave - 1) / kWave * kWave);
      // Several rows share a 256-thread block only when tpr divides it.
      if (tpr > kWave && tpr < 256) tpr = tpr <= 128 ? 128 : 256;
      const int threads = tpr >= 256 ? tpr : 256;
      const int64_t rows_per_block = threads / tpr;
      const int64_t grid = (a.rows + rows_per_block - 1) / rows_per_block;
      const T* wp = a.w_orders ? w.p[0] : nullptr;
      const T* bp = a.b_orders ? b.p[0] : nullptr;
      const int n = static_cast<int>(a.n);
      // Only instantiate the (K, CHUNKS) pairs the budget above can select.
      auto launch = [&](auto chunk_tag) {
        constexpr int C = decltype(chunk_tag)::value;
        if constexpr (4 * (K + 1) * C * static_cast<int>(sizeof(A) / 4) <= kRawBudget) {
          norm_series_reg_kernel<T, K, C, LAYER><<<dim3(grid), dim3(threads), 0, a.stream>>>(
              x, wp, bp, y, a.rows, n, tpr, eps, inv_n);
        }
      };
      if (chunks == 1) launch(std::integral_constant<int, 1>{});
      else if (chunks == 2) launch(std::integral_constant<int, 2>{});
      else launch(std::integral_constant<int, 4>{});
      PT_LAUNCH_CHECK();
      return PT_OK;
    }
  }
  norm_series_stream_kernel<T, K, LAYER><<<dim3(a.rows), dim3(kNormThreads), 0, a.stream>>>(
      x, w, a.w_orders, b, a.b_orders, y, a.rows, a.n, eps, inv_n);
  PT_LAUNCH_CHECK();
  return PT_OK;
}

template <typename T, bool LAYER>
int launch_norm(const NormArgs& a) {
  switch (a.degree) {
    case 0: return launch_norm_k<T, 0, LAYER>(a);
    case 1: return launch_norm_k<T, 1, LAYER>(a);
    case 2: return launch_norm_k<T, 2, LAYER>(a);
    case 3: return launch_norm_k<T, 3, LAYER>(a);
    case 4: return launch_norm_k<T, 4, LAYER>(a);
    case 5: return launch_norm_k<T, 5, LAYER>(a);
    case 6: return launch_norm_k<T, 6, LAYER>(a);
    case 7: return launch_norm_k<T, 7, LAYER>(a);
    case 8: return launch_norm_k<T, 8, LAYER>(a);
    default: break;
  }
  pt_host::set_error("norm series: degree outside 0..PT_MAX_DEGREE");
  return PT_UNSUPPORTED;
}

// ---------------------------------------------------------------------------
// Backward: the gradient series of the normalization, dx(t) = J(x(t))^T g(t)
// (the series of the reference's VJP formula
// /root/reference/src/polytensors/_fused_norm.py:52-56, generalising its
// degree-1 kernel _norm_kernels.py:22-38). With d = x - mean(x) for LayerNorm
// (d = x for RMSNorm), s = mean(d (*) d), r = rsqrt series of s + eps and
// c = sum_row g (*) d:
//   dx = r (*) (g - mean(g)) - (1/n) r (*) r (*) r (*) c (*) d
// (mean(g) is zero for RMSNorm). The affine terms are separate operations under
// autograd. The sums s and c share one row reduction.
template <typename A, int K>
__device__ __forceinline__ void norm_bwd_row_series(const A (&sums)[2 * (K + 1)], A inv_n, A eps,
                                                    A (&r)[K + 1], A (&q)[K + 1]) {
  A s[K + 1], c[K + 1], r2[K + 1], r3[K + 1];
#pragma unroll
  for (int k = 0; k <= K; ++k) {
    s[k] = sums[k];
    c[k] = sums[K + 1 + k];
  }
  rsqrt_series<A, K>(s, inv_n, eps, r);
  // r2 = r (*) r, r3 = r2 (*) r, q = -(1/n) r3 (*) c
#pragma unroll
  for (int k = K; k >= 0; --k) {
    A a = r[0] * r[k];
#pragma unroll
    for (int i = 1; i <= k; ++i) a = fma(r[i], r[k - i], a);
    r2[k] = a;
  }
#pragma unroll
  for (int k = K; k >= 0; --k) {
    A a = r2[0] * r[k];
#pragma unroll
    for (int i = 1; i <= k; ++i) a = fma(r2[i], r[k - i], a);
    r3[k] = a;
  }
#pragma unroll
  for (int k = K; k >= 0; --k) {
    A a = r3[0] * c[k];
#pragma unroll
    for (int i = 1; i <= k; ++i) a = fma(r3[i], c[k - i], a);
    q[k] = -inv_n * a;
  }
}

// Adds one element's d (*) d (half products, doubled later) and g (*) d to the sums.
template <typename A, int K>
__device__ __forceinline__ void norm_bwd_accumulate(const A (&d)[K + 1], const A (&g)[K + 1],
                                                    A (&cross)[K + 1], A (&sq)[K + 1], A (&c)[K + 1]) {
#pragma unroll
  for (int k = 0; k <= K; ++k) {
#pragma unroll
    for (int i = 0; 2 * i < k; ++i) cross[k] = fma(d[i], d[k - i], cross[k]);
    if (k % 2 == 0) sq[k] = fma(d[k / 2], d[k / 2], sq[k]);
#pragma unroll
    for (int i = 0; i <= k; ++i) c[k] = fma(g[i], d[k - i], c[k]);
  }
}

// dx = r (*) (g - mean(g)) + q (*) d for one element.
template <typename A, int K>
__device__ __forceinline__ void norm_bwd_element(const A (&d)[K + 1], const A (&g)[K + 1],
                                                 const A (&r)[K + 1], const A (&q)[K + 1],
                                                 A (&dx)[K + 1]) {
#pragma unroll
  for (int k = K; k >= 0; --k) {
    A a = r[0] * g[k];
#pragma unroll
    for (int i = 1; i <= k; ++i) a = fma(r[i], g[k - i], a);
#pragma unroll
    for (int i = 0; i <= k; ++i) a = fma(q[i], d[k - i], a);
    dx[k] = a;
  }
}

// Register-resident backward: `tpr` threads per row, CHUNKS 16-byte vectors of
// every order of x and g per thread, non-temporal accesses (as the forward kernel).
template <typename T, int K, int CHUNKS, bool LAYER>
__global__ __launch_bounds__(1024) void norm_series_bwd_reg_kernel(
    CPtrs<T> x, CPtrs<T> g, MPtrs<T> dx, int64_t rows, int n, int tpr, typename AccOf<T>::type eps,
    typename AccOf<T>::type inv_n) {
  using A = typename AccOf<T>::type;
  constexpr int V = VecWidth<T>::value;
  __shared__ A red[2][1024 / kWave][2 * (K + 1)];

  const int tid = threadIdx.x % tpr;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (blockDim.x / tpr) + threadIdx.x / tpr;
  const bool active = row < rows;
  const int64_t base = row * static_cast<int64_t>(n);

  Vec<T, V> rx[CHUNKS][K + 1], rg[CHUNKS][K + 1];
#pragma unroll
  for (int ch = 0; ch < CHUNKS; ++ch) {
    const int col = (ch * tpr + tid) * V;
    const bool in = active && col < n;
#pragma unroll
    for (int k = 0; k <= K; ++k) {
      if (in) {
        rx[ch][k] = load_vec_nt<T, V>(x.p[k] + base + col);
        rg[ch][k] = load_vec_nt<T, V>(g.p[k] + base + col);
      } else {
#pragma unroll
        for (int e = 0; e < V; ++e) rx[ch][k].v[e] = rg[ch][k].v[e] = from_acc<T>(A(0));
      }
    }
  }

  // means of x and g (LayerNorm), zero for RMSNorm; padding elements are zeros.
  A mean[2 * (K + 1)];
#pragma unroll
  for (int k = 0; k < 2 * (K + 1); ++k) mean[k] = A(0);
  if constexpr (LAYER) {
#pragma unroll
    for (int ch = 0; ch < CHUNKS; ++ch)
#pragma unroll
      for (int k = 0; k <= K; ++k)
#pragma unroll
        for (int e = 0; e < V; ++e) {
          mean[k] += vec_get(rx[ch][k], e);
          mean[K + 1 + k] += vec_get(rg[ch][k], e);
        }
    row_sums_n<A, 2 * (K + 1)>(mean, &red[0][0][0], tpr);
#pragma unroll
    for (int k = 0; k < 2 * (K + 1); ++k) mean[k] *= inv_n;
  }

  A cross[K + 1], sq[K + 1], c[K + 1];
#pragma unroll
  for (int k = 0; k <= K; ++k) cross[k] = sq[k] = c[k] = A(0);
#pragma unroll
  for (int ch = 0; ch < CHUNKS; ++ch) {
    const int col = (ch * tpr + tid) * V;
    if (!(active && col < n)) continue;
#pragma unroll
    for (int e = 0; e < V; ++e) {
      A d[K + 1], gv[K + 1];
#pragma unroll
      for (int k = 0; k <= K; ++k) {
        d[k] = LAYER ? vec_get(rx[ch][k], e) - mean[k] : vec_get(rx[ch][k], e);
        gv[k] = vec_get(rg[ch][k], e);
      }
      norm_bwd_accumulate<A, K>(d, gv, cross, sq, c);
    }
  }
  A sums[2 * (K + 1)];
#pragma unroll
  for (int k = 0; k <= K; ++k) {
    sums[k] = A(2) * cross[k] + sq[k];
    sums[K + 1 + k] = c[k];
  }
  row_sums_n<A, 2 * (K + 1)>(sums, &red[1][0][0], tpr);
  A r[K + 1], q[K + 1];
  norm_bwd_row_series<A, K>(sums, inv_n, eps, r, q);

  if (!active) return;
#pragma unroll
  for (int ch = 0; ch < CHUNKS; ++ch) {
    const int col = (ch * tpr + tid) * V;
    if (col >= n) continue;
#pragma unroll
    for (int e = 0; e < V; e += 2) {
      A out[2][K + 1];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        A d[K + 1], gv[K + 1];
#pragma unroll
        for (int k = 0; k <= K; ++k) {
          const A xv = vec_get(rx[ch][k], e + h), gk = vec_get(rg[ch][k], e + h);
          d[k] = LAYER ? xv - mean[k] : xv;
          gv[k] = LAYER ? gk - mean[K + 1 + k] : gk;
        }
        norm_bwd_element<A, K>(d, gv, r, q, out[h]);
      }
#pragma unroll
      for (int k = 0; k <= K; ++k) vec_put2(rx[ch][k], e, out[0][k], out[1][k]);
    }
#pragma unroll
    for (int k = 0; k <= K; ++k) store_vec_nt<T, V>(dx.p[k] + base + col, rx[ch][k]);
  }
}

// Streaming backward: one 256-thread block per row, scalar accesses, any n.
template <typename T, int K, bool LAYER>
__global__ __launch_bounds__(kNormThreads) void norm_series_bwd_stream_kernel(
    CPtrs<T> x, CPtrs<T> g, MPtrs<T> dx, int64_t rows, int64_t n, typename AccOf<T>::type eps,
    typename AccOf<T>::type inv_n) {
  using A = typename AccOf<T>::type;
  __shared__ A red[2][kNormThreads / kWave][2 * (K + 1)];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * n;

  A mean[2 * (K + 1)];
#pragma unroll
  for (int k = 0; k < 2 * (K + 1); ++k) mean[k] = A(0);
  if constexpr (LAYER) {
    for (int64_t col = threadIdx.x; col < n; col += kNormThreads)
#pragma unroll
      for (int k = 0; k <= K; ++k) {
        mean[k] += to_acc(x.p[k][base + col]);
        mean[K + 1 + k] += to_acc(g.p[k][base + col]);
      }
    row_sums_n<A, 2 * (K + 1)>(mean, &red[0][0][0], kNormThreads);
#pragma unroll
    for (int k = 0; k < 2 * (K + 1); ++k) mean[k] *= inv_n;
  }
  A cross[K + 1], sq[K + 1], c[K + 1];
#pragma unroll
  for (int k = 0; k <= K; ++k) cross[k] = sq[k] = c[k] = A(0);
  for (int64_t col = threadIdx.x; col < n; col += kNormThreads) {
    A d[K + 1], gv[K + 1];
#pragma unroll
    for (int k = 0; k <= K; ++k) {
      d[k] = to_acc(x.p[k][base + col]) - mean[k];
      gv[k] = to_acc(g.p[k][base + col]);
    }
    norm_bwd_accumulate<A, K>(d, gv, cross, sq, c);
  }
  A sums[2 * (K + 1)];
#pragma unroll
  for (int k = 0; k <= K; ++k) {
    sums[k] = A(2) * cross[k] + sq[k];
    sums[K + 1 + k] = c[k];
  }
  row_sums_n<A, 2 * (K + 1)>(sums, &red[1][0][0], kNormThreads);
  A r[K + 1], q[K + 1];
  norm_bwd_row_series<A, K>(sums, inv_n, eps, r, q);
  for (int64_t col = threadIdx.x; col < n; col += kNormThreads) {
    A d[K + 1], gv[K + 1], out[K + 1];
#pragma unroll
    for (int k = 0; k <= K; ++k) {
      d[k] = to_acc(x.p[k][base + col]) - mean[k];
      gv[k] = to_acc(g.p[k][base + col]) - mean[K + 1 + k];
    }
    norm_bwd_element<A, K>(d, gv, r, q, out);
#pragma unroll
    for (int k = 0; k <= K; ++k) dx.p[k][base + col] = from_acc<T>(out[k]);
  }
}

template <typename T, int K, bool LAYER>
static int launch_norm_bwd_k(const NormBwdArgs& a) {
  using A = typename AccOf<T>::type;
  constexpr int V = VecWidth<T>::value;
  CPtrs<T> x{}, g{};
  MPtrs<T> dx{};
  bool aligned = a.n % V == 0;
  for (int k = 0; k <= K; ++k) {
    x.p[k] = static_cast<const T*>(a.x[k]);
    g.p[k] = static_cast<const T*>(a.g[k]);
    dx.p[k] = static_cast<T*>(a.dx[k]);
    aligned = aligned && pt_host::aligned16(a.x[k]) && pt_host::aligned16(a.g[k]) &&
              pt_host::aligned16(a.dx[k]);
  }
  const A eps = static_cast<A>(a.eps);
  const A inv_n = A(1) / static_cast<A>(a.n);
  // Register path: at most kRawBudget VGPRs of raw x and g per thread (4 per
  // 16-byte vector), under which no instantiation spills in a 1024-thread block.
  constexpr int kRawBudget = LAYER ? 40 : 48;
  if (aligned && a.n <= (1 << 30)) {
    const int64_t vecs = a.n / V;
    int chunks = 0;
    for (int c : {1, 2, 4}) {
      if (vecs <= 1024 * c && 2 * 4 * (K + 1) * c <= kRawBudget) {
        chunks = c;
        break;
      }
    }
    if (chunks > 0) {
      int tpr = static_cast<int>(((vecs + chunks - 1) / chunks + kWave - 1) / kWave * kWave);
      if (tpr > kWave && tpr < 256) tpr = tpr <= 128 ? 128 : 256;
      const int threads = tpr >= 256 ? tpr : 256;
      const int64_t rows_per_block = threads / tpr;
      const int64_t grid = (a.rows + rows_per_block - 1) / rows_per_block;
      const int n = static_cast<int>(a.n);
      auto launch = [&](auto chunk_tag) {
        constexpr int C = decltype(chunk_tag)::value;
        if constexpr (2 * 4 * (K + 1) * C <= kRawBudget) {
          norm_series_bwd_reg_kernel<T, K, C, LAYER><<<dim3(grid), dim3(threads), 0, a.stream>>>(
              x, g, dx, a.rows, n, tpr, eps, inv_n);
        }
      };
      if (chunks == 1) launch(std::integral_constant<int, 1>{});
      else if (chunks == 2) launch(std::integral_constant<int, 2>{});
      else launch(std::integral_constant<int, 4>{});
      PT_LAUNCH_CHECK();
      return PT_OK;
    }
  }
  norm_series_bwd_stream_kernel<T, K, LAYER><<<dim3(a.rows), dim3(kNormThreads), 0, a.stream>>>(
      x, g, dx, a.rows, a.n, eps, inv_n);
  PT_LAUNCH_CHECK();
  return PT_OK;
}

template <typename T, bool LAYER>
int launch_norm_bwd(const NormBwdArgs& a) {
  switch (a.degree) {
    case 0: return launch_norm_bwd_k<T, 0, LAYER>(a);
    case 1: return launch_norm_bwd_k<T, 1, LAYER>(a);
    case 2: return launch_norm_bwd_k<T, 2, LAYER>(a);
    case 3: return launch_norm_bwd_k<T, 3, LAYER>(a);
    case 4: return launch_norm_bwd_k<T, 4, LAYER>(a);
    case 5: return launch_norm_bwd_k<T, 5, LAYER>(a);
    case 6: return launch_norm_bwd_k<T, 6, LAYER>(a);
    case 7: return launch_norm_bwd_k<T, 7, LAYER>(a);
    case 8: return launch_norm_bwd_k<T, 8, LAYER>(a);
    default: break;
  }
  pt_host::set_error("norm series backward: degree outside 0..PT_MAX_DEGREE");
  return PT_UNSUPPORTED;
}

}  // namespace pt
