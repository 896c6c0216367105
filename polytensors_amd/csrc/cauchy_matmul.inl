// Cauchy-product (truncated series) matrix product on MFMA:
//   C_k = sum_{i+j=k} A_i B_j,  k = 0..K,  all orders in one launch.
//
// The reference forms the same product as (K+1)(K+2)/2 separate matmuls plus
// adds (/root/reference/src/polytensors/_plain.py:118-128), reading A_i once
// per pair it appears in. Here one workgroup computes a BM x BN tile of every
// C_k: per contraction chunk of BK it stages the tiles of all orders of A and
// B in LDS once, and each wave then issues the MFMAs of every (i, j) pair with
// i + j <= K into K+1 accumulators, so each staged operand is reused by all
// pairs of its k-diagonals.
//
// The operands' order counts (1 for an ordinary tensor, K+1 for a series) are
// template parameters: the pair set is fixed at compile time, so the MFMA
// sequence has no branches and issues back to back. The next chunk's global
// loads are issued into registers before the current chunk's MFMAs, so their
// latency hides behind the matrix work; the registers are committed to LDS
// between two barriers.
//
// LDS layout: As[order][row][k], Bs[order][col][k], k contiguous. Within a
// chunk the contraction index is permuted: MFMA step s uses k = (lane / M) *
// RUN + s, so each lane reads its RUN operand values of a row with 16-byte LDS
// loads (the same permutation on A and B leaves the product unchanged).
//
// Banks. gfx950 serves a 16-byte LDS access in four passes of 16 lanes,
// {0-3, 12-15, 20-27}, {4-11, 16-19, 28-31} and the same sets plus 32, an
// 8-byte access in two passes of 32 consecutive lanes (measured with a
// two-lane LDS probe and SQ_LDS_BANK_CONFLICT).
// * float64: rows unpadded, 16-byte chunks XOR-swizzled by a function of the
//   row (CauchyLds::fa), chosen under that model so that the operand reads and
//   the 16-byte tile writes of every pass hit 64 distinct banks (B stored
//   [Kd][N], transposed by 8-byte writes, keeps a two-way conflict on those
//   writes). The first layout, a 16-byte row pad, conflicted on all three:
//   bank conflicts fell from 17.4% to 3.4% of the CU cycles, 33.8 -> 32.0 ms
//   at config 2's shape.
// * float32: rows keep a 16-byte pad, which makes the A-operand reads
//   conflict-free under the model; B stored [Kd][N], transposed by 4-byte
//   writes, also swizzles its chunks by (n / 16) % 4, which makes those writes
//   conflict-free and leaves its operand reads two-way in each pass (no XOR
//   swizzle of two row bits frees both). The float64-style unpadded, swizzled A
//   tile also removed the A-tile write conflicts (5.5% -> 3.7% of the CU
//   cycles) but measured 0.5% slower, so float32 keeps the pad.
// tests/test_cauchy_tiles.py replays these layouts under the bank model.
#pragma once

#include <algorithm>

#include "cauchy_matmul.h"
#include "mfma.h"

namespace pt {

template <typename T, bool TRANS_B>
struct CauchyLds {
  static constexpr int BK = 16;
  static constexpr int QV = 16 / static_cast<int>(sizeof(T));   // values per 16-byte chunk
  static constexpr bool kF64 = sizeof(T) == 8;
  static constexpr int LDA = kF64 ? BK : BK + QV;
  static constexpr int LDB = LDA;
  // double: 8 chunks per row, chunk bits (r0^r2, r0^r1, r0^r3); float: padded rows, no swizzle
  __host__ __device__ __forceinline__ static int fa(int r) {
    if constexpr (kF64) return ((r ^ (r >> 2)) & 1) | (((r ^ (r >> 1)) & 1) << 1) | (((r ^ (r >> 3)) & 1) << 2);
    else return 0;
  }
  __host__ __device__ __forceinline__ static int fb(int n) {
    if constexpr (kF64) return fa(n);
    else if constexpr (!TRANS_B) return (n >> 4) & 3;
    else return 0;
  }
};

template <typename T, int K, int AO, int BO, int BM, int BN, int BK, int WAVES_M, int WAVES_N,
          int MIN_WAVES, bool TRANS_B, bool VEC>
__global__ __launch_bounds__(WAVES_M * WAVES_N * kWave) __attribute__((amdgpu_waves_per_eu(MIN_WAVES)))
void cauchy_matmul_kernel(
    CPtrs<T> A, CPtrs<T> B, MPtrs<T> C, int M, int N, int Kd, int64_t a_bs, int64_t b_bs) {
  using MF = Mfma<T>;
  using acc_t = typename MF::acc_t;
  constexpr int THREADS = WAVES_M * WAVES_N * kWave;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int FM = WM / MF::M, FN = WN / MF::N;
  constexpr int RUN = BK / MF::KK;            // contiguous k per lane per chunk
  constexpr int QV = 16 / sizeof(T);          // values per 16-byte LDS read
  constexpr int V = 16 / sizeof(T);           // values per 16-byte global load
  using Lds = CauchyLds<T, TRANS_B>;
  static_assert(BK == Lds::BK, "LDS layout is for 16-deep chunks");
  constexpr int NA = BM * BK / V / THREADS;   // A vectors per thread and order
  constexpr int NB = BN * BK / V / THREADS;   // B vectors per thread and order
  static_assert(FM * MF::M == WM && FN * MF::N == WN, "wave tile must be whole MFMA blocks");
  static_assert(RUN % QV == 0, "chunk must give whole 16-byte runs");
  static_assert(NA * V * THREADS == BM * BK && NB * V * THREADS == BN * BK, "whole vectors per thread");
  static_assert((AO == 1 || AO == K + 1) && (BO == 1 || BO == K + 1), "operand orders are 1 or K+1");

  __shared__ T As[AO][BM][Lds::LDA];
  __shared__ T Bs[BO][BN][Lds::LDB];
  auto achunk = [](int r, int c) { return c ^ Lds::fa(r); };
  auto bchunk = [](int n, int c) { return c ^ Lds::fb(n); };

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int tile_m = blockIdx.y * BM, tile_n = blockIdx.x * BN;
  const int64_t batch = blockIdx.z;

  const T* a_base[AO];
  const T* b_base[BO];
#pragma unroll
  for (int o = 0; o < AO; ++o) a_base[o] = A.p[o] + batch * a_bs;
#pragma unroll
  for (int o = 0; o < BO; ++o) b_base[o] = B.p[o] + batch * b_bs;

  // ---- global -> registers (one chunk), zero outside the matrices ----
  Vec<T, V> ra[AO][NA], rb[BO][NB];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int o = 0; o < AO; ++o)
#pragma unroll
      for (int it = 0; it < NA; ++it) {
        const int v = it * THREADS + threadIdx.x;
        const int gr = tile_m + v / (BK / V), gk = k0 + (v % (BK / V)) * V;
        const T* p = a_base[o] + static_cast<int64_t>(gr) * Kd + gk;
        if constexpr (VEC) {   // Kd % V == 0: a vector is wholly inside or outside
          if (gr < M && gk < Kd) {
            ra[o][it] = load_vec<T, V>(p);
          } else {
#pragma unroll
            for (int e = 0; e < V; ++e) ra[o][it].v[e] = T(0);
          }
        } else {
#pragma unroll
          for (int e = 0; e < V; ++e) ra[o][it].v[e] = (gr < M && gk + e < Kd) ? p[e] : T(0);
        }
      }
#pragma unroll
    for (int o = 0; o < BO; ++o)
#pragma unroll
      for (int it = 0; it < NB; ++it) {
        const int v = it * THREADS + threadIdx.x;
        if constexpr (TRANS_B) {   // B stored [N][Kd]
          const int gn = tile_n + v / (BK / V), gk = k0 + (v % (BK / V)) * V;
          const T* p = b_base[o] + static_cast<int64_t>(gn) * Kd + gk;
          if constexpr (VEC) {
            if (gn < N && gk < Kd) {
              rb[o][it] = load_vec<T, V>(p);
            } else {
#pragma unroll
              for (int e = 0; e < V; ++e) rb[o][it].v[e] = T(0);
            }
          } else {
#pragma unroll
            for (int e = 0; e < V; ++e) rb[o][it].v[e] = (gn < N && gk + e < Kd) ? p[e] : T(0);
          }
        } else {                   // B stored [Kd][N]: a vector runs along n
          const int gk = k0 + v / (BN / V), gn = tile_n + (v % (BN / V)) * V;
          const T* p = b_base[o] + static_cast<int64_t>(gk) * N + gn;
          if constexpr (VEC) {     // N % V == 0
            if (gk < Kd && gn < N) {
              rb[o][it] = load_vec<T, V>(p);
            } else {
#pragma unroll
              for (int e = 0; e < V; ++e) rb[o][it].v[e] = T(0);
            }
          } else {
#pragma unroll
            for (int e = 0; e < V; ++e) rb[o][it].v[e] = (gk < Kd && gn + e < N) ? p[e] : T(0);
          }
        }
      }
  };
  // ---- registers -> LDS (B transposed to [n][k] when stored [Kd][N]) ----
  auto commit = [&]() {
#pragma unroll
    for (int o = 0; o < AO; ++o)
#pragma unroll
      for (int it = 0; it < NA; ++it) {
        const int v = it * THREADS + threadIdx.x;
        const int r = v / (BK / V);
        store_vec<T, V>(&As[o][r][achunk(r, v % (BK / V)) * V], ra[o][it]);
      }
#pragma unroll
    for (int o = 0; o < BO; ++o)
#pragma unroll
      for (int it = 0; it < NB; ++it) {
        const int v = it * THREADS + threadIdx.x;
        if constexpr (TRANS_B) {
          const int n = v / (BK / V);
          store_vec<T, V>(&Bs[o][n][bchunk(n, v % (BK / V)) * V], rb[o][it]);
        } else {
          const int kk = v / (BN / V), nv = (v % (BN / V)) * V;
#pragma unroll
          for (int e = 0; e < V; ++e) Bs[o][nv + e][bchunk(nv + e, kk / QV) * QV + kk % QV] = rb[o][it].v[e];
        }
      }
  };

  acc_t acc[K + 1][FM][FN];
#pragma unroll
  for (int o = 0; o <= K; ++o)
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) acc[o][fm][fn] = MF::zero();

  const int row_a = wm * WM + lane % MF::M;
  const int col_b = wn * WN + lane % MF::N;
  const int kbase = (lane / MF::M) * RUN;
  const int chunks = (Kd + BK - 1) / BK;
  fetch(0);
  for (int c = 0; c < chunks; ++c) {
    __syncthreads();   // every wave is done reading the previous chunk
    commit();
    __syncthreads();
    if (c + 1 < chunks) fetch((c + 1) * BK);   // in flight during this chunk's MFMAs

#pragma unroll
    for (int q = 0; q < RUN / QV; ++q) {
      Vec<T, QV> av[AO][FM], bv[BO][FN];
#pragma unroll
      for (int o = 0; o < AO; ++o)
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
          av[o][fm] = *reinterpret_cast<const Vec<T, QV>*>(
              &As[o][row_a + fm * MF::M][achunk(row_a + fm * MF::M, kbase / QV + q) * QV]);
#pragma unroll
      for (int o = 0; o < BO; ++o)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
          bv[o][fn] = *reinterpret_cast<const Vec<T, QV>*>(
              &Bs[o][col_b + fn * MF::N][bchunk(col_b + fn * MF::N, kbase / QV + q) * QV]);
#pragma unroll
      for (int ss = 0; ss < QV; ++ss) {
#pragma unroll
        for (int k = 0; k <= K; ++k) {
#pragma unroll
          for (int i = 0; i <= k; ++i) {
            const int j = k - i;
            if (i < AO && j < BO) {   // compile-time after unrolling
#pragma unroll
              for (int fm = 0; fm < FM; ++fm)
#pragma unroll
                for (int fn = 0; fn < FN; ++fn)
                  acc[k][fm][fn] = MF::mma(av[i][fm].v[ss], bv[j][fn].v[ss], acc[k][fm][fn]);
            }
          }
        }
      }
    }
  }

  // ---- epilogue: each accumulator register holds one element of C_k ----
#pragma unroll
  for (int o = 0; o <= K; ++o) {
    T* c_base = C.p[o] + batch * static_cast<int64_t>(M) * N;
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const int col = tile_n + wn * WN + fn * MF::N + MF::acc_col(lane);
#pragma unroll
        for (int r = 0; r < MF::ACC; ++r) {
          const int row = tile_m + wm * WM + fm * MF::M + MF::acc_row(lane, r);
          if (row < M && col < N) c_base[static_cast<int64_t>(row) * N + col] = acc[o][fm][fn][r];
        }
      }
  }
}

// Zero orders 1..degree of C (both operands ordinary: only C_0 is a product).
template <typename T>
__global__ __launch_bounds__(256) void cauchy_zero_orders_kernel(MPtrs<T> C, int degree, int64_t count) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int o = 1; o <= degree; ++o)
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride)
      C.p[o][i] = T(0);
}

// Tile shapes: 4 waves in a 2x2 grid. fp32: 64x64 output tiles, one 32x32x2
// MFMA block per wave. fp64: 64x64 tiles (2x2 16x16x4 blocks per wave) up to
// degree 3, and 32x32 tiles (one block per wave) from degree 4, where K+1
// accumulator sets of 2x2 blocks would no longer fit the register file.
// Contraction chunk 16: at most 9 orders of both operands, 92 KB of LDS.
// MIN_WAVES asks the register allocator for two
// waves per SIMD (at most 256 registers per lane) where the accumulators, the
// prefetched chunk and the MFMA operands fit without spilling, and otherwise
// lets a wave use the whole register file.
template <typename T, int K, int AO, int BO>
struct CauchyTile {
  static constexpr bool kSmallTile = sizeof(T) == 8 && K >= 4;
  static constexpr int BM = kSmallTile ? 32 : 64, BN = BM, WAVES_M = 2, WAVES_N = 2;
  static constexpr int BK = 16;
  static constexpr bool kOneSeries = (AO == 1) || (BO == 1);
  static constexpr int kMaxDegreeTwoWaves =
      sizeof(T) == 4 ? (kOneSeries ? 7 : 5) : (kSmallTile ? (kOneSeries ? 8 : 6) : (kOneSeries ? 3 : 2));
  static constexpr int MIN_WAVES = K <= kMaxDegreeTwoWaves ? 2 : 1;
  static_assert(AO * BM * (BK + 16 / sizeof(T)) * sizeof(T) + BO * BN * (BK + 16 / sizeof(T)) * sizeof(T) <=
                    160 * 1024, "LDS budget");
};

template <typename T, int K, int AO, int BO>
static int launch_cauchy_orders(const CauchyArgs& a, const CPtrs<T>& A, const CPtrs<T>& B,
                                const MPtrs<T>& C, bool vec) {
  using Tile = CauchyTile<T, K, AO, BO>;
  const dim3 grid((a.n + Tile::BN - 1) / Tile::BN, (a.m + Tile::BM - 1) / Tile::BM, a.batch);
  const dim3 block(Tile::WAVES_M * Tile::WAVES_N * kWave);
  const int M = static_cast<int>(a.m), N = static_cast<int>(a.n), Kd = static_cast<int>(a.k);
#define PT_CAUCHY_LAUNCH(TB, VV)                                                                   \
  cauchy_matmul_kernel<T, K, AO, BO, Tile::BM, Tile::BN, Tile::BK, Tile::WAVES_M, Tile::WAVES_N, \
                       Tile::MIN_WAVES, TB, VV><<<grid, block, 0, a.stream>>>(A, B, C, M, N, Kd, a.a_bs, a.b_bs)
  if (a.trans_b) {
    if (vec) PT_CAUCHY_LAUNCH(true, true);
    else PT_CAUCHY_LAUNCH(true, false);
  } else {
    if (vec) PT_CAUCHY_LAUNCH(false, true);
    else PT_CAUCHY_LAUNCH(false, false);
  }
#undef PT_CAUCHY_LAUNCH
  PT_LAUNCH_CHECK();
  return PT_OK;
}

template <typename T, int K>
static int launch_cauchy_k(const CauchyArgs& a) {
  constexpr int V = 16 / sizeof(T);
  CPtrs<T> A{}, B{};
  MPtrs<T> C{};
  bool vec = true;
  for (int o = 0; o < a.a_orders; ++o) {
    A.p[o] = static_cast<const T*>(a.a[o]);
    vec = vec && pt_host::aligned16(a.a[o]);
  }
  for (int o = 0; o < a.b_orders; ++o) {
    B.p[o] = static_cast<const T*>(a.b[o]);
    vec = vec && pt_host::aligned16(a.b[o]);
  }
  for (int o = 0; o <= K; ++o) C.p[o] = static_cast<T*>(a.c[o]);
  vec = vec && a.k % V == 0 && a.a_bs % V == 0 && a.b_bs % V == 0 && (a.trans_b || a.n % V == 0);
  const bool a_series = a.a_orders > 1, b_series = a.b_orders > 1;
  if constexpr (K == 0) {
    return launch_cauchy_orders<T, 0, 1, 1>(a, A, B, C, vec);
  } else {
    if (a_series && b_series) return launch_cauchy_orders<T, K, K + 1, K + 1>(a, A, B, C, vec);
    if (a_series) return launch_cauchy_orders<T, K, K + 1, 1>(a, A, B, C, vec);
    if (b_series) return launch_cauchy_orders<T, K, 1, K + 1>(a, A, B, C, vec);
    // Two ordinary operands: C_0 = A_0 B_0 and zero higher orders.
    int st = launch_cauchy_orders<T, 0, 1, 1>(a, A, B, C, vec);
    if (st != PT_OK) return st;
    const int64_t count = a.batch * a.m * a.n;
    const int64_t blocks = std::min<int64_t>((count + 255) / 256, 4096);
    cauchy_zero_orders_kernel<T><<<dim3(blocks), dim3(256), 0, a.stream>>>(C, K, count);
    PT_LAUNCH_CHECK();
    return PT_OK;
  }
}

template <typename T>
int launch_cauchy(const CauchyArgs& a) {
  switch (a.degree) {
    case 0: return launch_cauchy_k<T, 0>(a);
    case 1: return launch_cauchy_k<T, 1>(a);
    case 2: return launch_cauchy_k<T, 2>(a);
    case 3: return launch_cauchy_k<T, 3>(a);
    case 4: return launch_cauchy_k<T, 4>(a);
    case 5: return launch_cauchy_k<T, 5>(a);
    case 6: return launch_cauchy_k<T, 6>(a);
    case 7: return launch_cauchy_k<T, 7>(a);
    case 8: return launch_cauchy_k<T, 8>(a);
    default: break;
  }
  pt_host::set_error("Cauchy matmul: degree outside 0..PT_MAX_DEGREE");
  return PT_UNSUPPORTED;
}

}  // namespace pt
