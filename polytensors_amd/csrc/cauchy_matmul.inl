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
// LDS layout: As[order][row][k], Bs[order][col][k], k contiguous with a
// 16-byte pad per row. Within a chunk the contraction index is permuted: MFMA
// step s uses k = (lane / M) * RUN + s, so each lane reads its RUN operand
// values of a row with 16-byte LDS loads (the same permutation on A and B
// leaves the product unchanged); the 16-byte row pad makes those reads
// bank-conflict-free.
#pragma once

#include "cauchy_matmul.h"
#include "mfma.h"

namespace pt {

template <typename T, int K, int BM, int BN, int BK, int WAVES_M, int WAVES_N, bool TRANS_B, bool VEC>
__global__ __launch_bounds__(WAVES_M * WAVES_N * kWave) void cauchy_matmul_kernel(
    CPtrs<T> A, int a_orders, CPtrs<T> B, int b_orders, MPtrs<T> C, int M, int N, int Kd,
    int64_t a_bs, int64_t b_bs) {
  using MF = Mfma<T>;
  using acc_t = typename MF::acc_t;
  constexpr int THREADS = WAVES_M * WAVES_N * kWave;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int FM = WM / MF::M, FN = WN / MF::N;
  constexpr int RUN = BK / MF::KK;            // contiguous k per lane per chunk
  constexpr int QV = 16 / sizeof(T);          // values per 16-byte LDS read
  constexpr int V = 16 / sizeof(T);           // values per 16-byte global load
  constexpr int LDK = BK + 16 / sizeof(T);    // padded row length
  static_assert(FM * MF::M == WM && FN * MF::N == WN, "wave tile must be whole MFMA blocks");
  static_assert(RUN % QV == 0, "chunk must give whole 16-byte runs");
  static_assert((BM * BK / V) % THREADS == 0 && (BN * BK / V) % THREADS == 0, "whole loads per thread");

  __shared__ T As[K + 1][BM][LDK];
  __shared__ T Bs[K + 1][BN][LDK];

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int tile_m = blockIdx.y * BM, tile_n = blockIdx.x * BN;
  const int64_t batch = blockIdx.z;

  const T* a_base[K + 1];
  const T* b_base[K + 1];
#pragma unroll
  for (int o = 0; o <= K; ++o) {
    a_base[o] = (o < a_orders) ? A.p[o] + batch * a_bs : nullptr;
    b_base[o] = (o < b_orders) ? B.p[o] + batch * b_bs : nullptr;
  }

  acc_t acc[K + 1][FM][FN];
#pragma unroll
  for (int o = 0; o <= K; ++o)
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) acc[o][fm][fn] = MF::zero();

  for (int k0 = 0; k0 < Kd; k0 += BK) {
    __syncthreads();   // the previous chunk's operands are consumed
    // ---- stage A (row-major [M][Kd]) into As[o][r][k] ----
#pragma unroll
    for (int o = 0; o <= K; ++o) {
      if (o >= a_orders) break;
      if constexpr (VEC) {
#pragma unroll
        for (int it = 0; it < BM * BK / V / THREADS; ++it) {
          const int v = it * THREADS + threadIdx.x;
          const int r = v / (BK / V), kv = (v % (BK / V)) * V;
          const int gr = tile_m + r, gk = k0 + kv;
          Vec<T, V> x;
          if (gr < M && gk < Kd) {
            x = load_vec<T, V>(a_base[o] + static_cast<int64_t>(gr) * Kd + gk);
          } else {
#pragma unroll
            for (int e = 0; e < V; ++e) x.v[e] = T(0);
          }
          store_vec<T, V>(&As[o][r][kv], x);
        }
      } else {
        for (int idx = threadIdx.x; idx < BM * BK; idx += THREADS) {
          const int r = idx / BK, kk = idx % BK;
          const int gr = tile_m + r, gk = k0 + kk;
          As[o][r][kk] = (gr < M && gk < Kd) ? a_base[o][static_cast<int64_t>(gr) * Kd + gk] : T(0);
        }
      }
    }
    // ---- stage B into Bs[o][n][k] ----
#pragma unroll
    for (int o = 0; o <= K; ++o) {
      if (o >= b_orders) break;
      if constexpr (TRANS_B) {   // B stored [N][Kd]
        if constexpr (VEC) {
#pragma unroll
          for (int it = 0; it < BN * BK / V / THREADS; ++it) {
            const int v = it * THREADS + threadIdx.x;
            const int n = v / (BK / V), kv = (v % (BK / V)) * V;
            const int gn = tile_n + n, gk = k0 + kv;
            Vec<T, V> x;
            if (gn < N && gk < Kd) {
              x = load_vec<T, V>(b_base[o] + static_cast<int64_t>(gn) * Kd + gk);
            } else {
#pragma unroll
              for (int e = 0; e < V; ++e) x.v[e] = T(0);
            }
            store_vec<T, V>(&Bs[o][n][kv], x);
          }
        } else {
          for (int idx = threadIdx.x; idx < BN * BK; idx += THREADS) {
            const int n = idx / BK, kk = idx % BK;
            const int gn = tile_n + n, gk = k0 + kk;
            Bs[o][n][kk] = (gn < N && gk < Kd) ? b_base[o][static_cast<int64_t>(gn) * Kd + gk] : T(0);
          }
        }
      } else {                   // B stored [Kd][N]: transpose while staging
        if constexpr (VEC) {
#pragma unroll
          for (int it = 0; it < BN * BK / V / THREADS; ++it) {
            const int v = it * THREADS + threadIdx.x;
            const int kk = v / (BN / V), nv = (v % (BN / V)) * V;
            const int gk = k0 + kk, gn = tile_n + nv;
            Vec<T, V> x;
            if (gk < Kd && gn < N) {
              x = load_vec<T, V>(b_base[o] + static_cast<int64_t>(gk) * N + gn);
            } else {
#pragma unroll
              for (int e = 0; e < V; ++e) x.v[e] = T(0);
            }
#pragma unroll
            for (int e = 0; e < V; ++e) Bs[o][nv + e][kk] = x.v[e];
          }
        } else {
          for (int idx = threadIdx.x; idx < BN * BK; idx += THREADS) {
            const int kk = idx / BN, n = idx % BN;
            const int gk = k0 + kk, gn = tile_n + n;
            Bs[o][n][kk] = (gk < Kd && gn < N) ? b_base[o][static_cast<int64_t>(gk) * N + gn] : T(0);
          }
        }
      }
    }
    __syncthreads();

    // ---- MFMAs of every (i, j) pair with i + j <= K ----
    const int row_a = wm * WM + lane % MF::M;
    const int col_b = wn * WN + lane % MF::N;
    const int kbase = (lane / MF::M) * RUN;
#pragma unroll
    for (int q = 0; q < RUN / QV; ++q) {
      Vec<T, QV> av[K + 1][FM], bv[K + 1][FN];
#pragma unroll
      for (int o = 0; o <= K; ++o) {
        if (o < a_orders) {
#pragma unroll
          for (int fm = 0; fm < FM; ++fm)
            av[o][fm] = *reinterpret_cast<const Vec<T, QV>*>(&As[o][row_a + fm * MF::M][kbase + q * QV]);
        }
        if (o < b_orders) {
#pragma unroll
          for (int fn = 0; fn < FN; ++fn)
            bv[o][fn] = *reinterpret_cast<const Vec<T, QV>*>(&Bs[o][col_b + fn * MF::N][kbase + q * QV]);
        }
      }
#pragma unroll
      for (int ss = 0; ss < QV; ++ss) {
#pragma unroll
        for (int k = 0; k <= K; ++k) {
#pragma unroll
          for (int i = 0; i <= k; ++i) {
            const int j = k - i;
            if (i < a_orders && j < b_orders) {
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

// Tile shapes: 64x64 output tiles, 4 waves of 32x32 each (one 32x32x2 fp32
// MFMA block, or 2x2 16x16x4 fp64 blocks), contraction chunk 16 -- 8 for fp64
// at degree 8, whose 9 staged orders of A and B would otherwise pass the
// 160 KB of LDS a workgroup can hold.
template <typename T, int K>
struct CauchyTile {
  static constexpr int BM = 64, BN = 64, WAVES_M = 2, WAVES_N = 2;
  static constexpr int BK = (sizeof(T) == 8 && K >= 8) ? 8 : 16;
  static_assert((K + 1) * (BM + BN) * (BK + 16 / sizeof(T)) * sizeof(T) <= 160 * 1024, "LDS budget");
};

template <typename T, int K>
static int launch_cauchy_k(const CauchyArgs& a) {
  using Tile = CauchyTile<T, K>;
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
  const dim3 grid((a.n + Tile::BN - 1) / Tile::BN, (a.m + Tile::BM - 1) / Tile::BM, a.batch);
  const dim3 block(Tile::WAVES_M * Tile::WAVES_N * kWave);
  const int M = static_cast<int>(a.m), N = static_cast<int>(a.n), Kd = static_cast<int>(a.k);
#define PT_CAUCHY_LAUNCH(TB, VV)                                                                  \
  cauchy_matmul_kernel<T, K, Tile::BM, Tile::BN, Tile::BK, Tile::WAVES_M, Tile::WAVES_N, TB, VV> \
      <<<grid, block, 0, a.stream>>>(A, a.a_orders, B, a.b_orders, C, M, N, Kd, a.a_bs, a.b_bs)
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
