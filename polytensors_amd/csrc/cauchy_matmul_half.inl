// Cauchy-product matrix product of bfloat16 / float16 series on the 16x16x32
// MFMAs of gfx950, fp32 accumulation:
//   C_k = sum_{i+j=k} A_i B_j,  k = 0..K,  all orders in one launch,
// rounded to the storage type once per element (the reference forms the
// (K+1)(K+2)/2 products as separate half-precision matmuls and adds them in
// the storage type, /root/reference/src/polytensors/_plain.py:118-128).
//
// A workgroup of 4 waves owns a 64 x 64 tile of every C_k; each wave a 32 x 32
// block as 2 x 2 MFMA blocks. The product is formed transposed, C^T = B^T A^T:
// with v_mfma_f32_16x16x32 (lane l supplies row l % 16 of the first operand and
// column l % 16 of the second, contraction elements 8 (l / 16) .. + 7;
// accumulator register r of lane l is row 4 (l / 16) + r, column l % 16) the
// accumulator registers of a lane are four consecutive columns of one row of
// C, written with one 8-byte store.
//
// Contraction chunks of 32 are moved into LDS by LDS DMA (buffer loads into
// LDS, half_mfma.h), two buffers: the DMA of chunk c+1 runs during chunk c's
// MFMAs, one barrier per chunk, no staging registers. Tiles are unpadded with
// 16-byte chunks XOR-swizzled per row so that each pass of an operand read hits
// 64 distinct banks. gfx950 serves a 16-byte read (ds_read_b128) in four passes
// of 16 lanes: {0-3, 12-15, 20-27}, {4-11, 16-19, 28-31} and the same two sets
// plus 32 (found with a two-lane LDS probe and the SQ_LDS_BANK_CONFLICT
// counter); an 8-byte read in two passes of 32 consecutive lanes.
// * A (and B stored [n][k]) as [row][32 k], 64-byte rows, chunk ^= F((row / 4) % 4)
//   with F = (0, 2, 3, 1): an operand is one 16-byte read per lane (lane l reads
//   row l % 16, chunk l / 16). With F(q) = q (the first layout) the rows of lanes
//   0-3 and 20-23 shared banks: four conflict cycles per read;
// * B stored [k][n] as [32 k][64 n], 128-byte rows, chunk ^= 2 h(k) with
//   h(k) = (k / 2) % 2 + 2 ((k / 8) % 2): the B^T operand (eight k of one
//   column n per lane) is two ds_read_b64_tr_b16 transpose reads, lane 4j + a
//   of group g addressing row 8g + j (then 8g + 4 + j), columns n0 + 4a .. + 3.
// Rows past M / N and contraction chunks past Kd are out of the DMA's range and
// load as zeros (the launcher requires Kd and, for B stored [k][n], N to be
// multiples of 8, so a 16-byte chunk is wholly inside or outside).
#pragma once

#include <algorithm>

#include "cauchy_matmul.h"
#include "half_mfma.h"

namespace pt {

// Workgroup tile: WMW x WNW waves, each owning FM x FN MFMA blocks of 16 x 16 of every C_k. The
// narrow tile (64 x 64, 4 waves of 32 x 32) leaves LDS for two workgroups per CU; the wide tile
// (128 x 128, 8 waves of 64 x 32) reads a third fewer LDS bytes per MFMA and half the HBM
// re-reads, and fills one CU with its 8 waves when both operands are series of degree <= 4.
template <int AO, int BO, bool WIDE>
struct CauchyHalfTile {
  static constexpr int WMW = 2, WNW = WIDE ? 4 : 2, FM = WIDE ? 4 : 2, FN = 2;
  static constexpr int BM = 16 * FM * WMW, BN = 16 * FN * WNW, BK = 32;
  static constexpr int kWaves = WMW * WNW, kThreads = kWaves * kWave;
  static constexpr size_t LDS = 2ull * (AO * BM + BO * BN) * BK * 2;
  // every order tile of A ([BM][BK]) and of B ([BK][BN] or [BN][BK]) is one 1 KB DMA segment per wave
  static_assert(BM * BK * 2 == 1024 * kWaves && BN * BK * 2 == 1024 * kWaves, "one DMA segment per wave");
};

// physical 16-byte chunk of logical chunk ch in row r of a [row][32] tile / of a [k][BN] tile
// (BN = 64: 128-byte rows, two rows per bank sweep; BN = 128: 256-byte rows, one per sweep)
__host__ __device__ __forceinline__ int cauchy_swz_rows(int r, int ch) { return ch ^ ((0x78 >> (2 * ((r >> 2) & 3))) & 3); }
template <bool WIDE>
__host__ __device__ __forceinline__ int cauchy_swz_k(int k, int ch) {
  if constexpr (WIDE) return ch ^ (2 * ((k & 3) | (((k >> 3) & 1) << 2)));
  return ch ^ (2 * (((k >> 1) & 1) | (((k >> 3) & 1) << 1)));
}

template <typename T, int K, int AO, int BO, bool TRANS_B, bool WIDE>
__global__ __launch_bounds__((CauchyHalfTile<AO, BO, WIDE>::kThreads)) void cauchy_matmul_half_kernel(
    CPtrs<T> A, CPtrs<T> B, MPtrs<T> C, int M, int N, int Kd, int64_t a_bs, int64_t b_bs, int c_vec) {
  using Tile = CauchyHalfTile<AO, BO, WIDE>;
  using MM = HalfMfma<T>;
  constexpr int BM = Tile::BM, BN = Tile::BN, BK = Tile::BK, FM = Tile::FM, FN = Tile::FN;
  constexpr int CPR = BN / 8;   // 16-byte chunks per k row of a [BK][BN] B tile
  static_assert(Tile::LDS <= 160 * 1024, "LDS budget");
  static_assert((AO == 1 || AO == K + 1) && (BO == 1 || BO == K + 1), "operand orders are 1 or K+1");

  __shared__ __attribute__((aligned(16))) T As[2][AO][BM * BK];
  __shared__ __attribute__((aligned(16))) T Bs[2][BO][BN * BK];

  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int c = lane % 16, g = lane / 16;
  const int wm = wave / Tile::WNW, wn = wave % Tile::WNW;
  const int tile_m = blockIdx.y * BM, tile_n = blockIdx.x * BN;
  const int64_t batch = blockIdx.z;
  const int a_bytes = M * Kd * static_cast<int>(sizeof(T));
  const int b_bytes = Kd * N * static_cast<int>(sizeof(T));

  // DMA of chunk k0 into buffer buf: this wave moves segment `wave` (1 KB) of every order tile
  auto issue = [&](int buf, int k0) {
    {   // A: rows 16 wave + lane / 4, physical chunk lane % 4
      const int row = 16 * wave + lane / 4;
      const int lch = cauchy_swz_rows(row, lane % 4);
      const int gm = tile_m + row, gk = k0 + 8 * lch;
      const int voff = (gm < M && gk < Kd) ? (gm * Kd + gk) * static_cast<int>(sizeof(T)) : kBufferOutOfRange;
#pragma unroll
      for (int o = 0; o < AO; ++o)
        lds_dma16(&As[buf][o][512 * wave], buffer_rsrc(A.p[o] + batch * a_bs, a_bytes), voff);
    }
    int voff;
    if constexpr (TRANS_B) {   // B stored [N][Kd]: as A
      const int row = 16 * wave + lane / 4;
      const int lch = cauchy_swz_rows(row, lane % 4);
      const int gn = tile_n + row, gk = k0 + 8 * lch;
      voff = (gn < N && gk < Kd) ? (gn * Kd + gk) * static_cast<int>(sizeof(T)) : kBufferOutOfRange;
    } else {                   // B stored [Kd][N]: k rows (64 / CPR) wave + lane / CPR, physical chunk lane % CPR
      const int kr = (64 / CPR) * wave + lane / CPR;
      const int lch = cauchy_swz_k<WIDE>(kr, lane % CPR);
      const int gk = k0 + kr, gn = tile_n + 8 * lch;
      voff = (gk < Kd && gn < N) ? (gk * N + gn) * static_cast<int>(sizeof(T)) : kBufferOutOfRange;
    }
#pragma unroll
    for (int o = 0; o < BO; ++o)
      lds_dma16(&Bs[buf][o][512 * wave], buffer_rsrc(B.p[o] + batch * b_bs, b_bytes), voff);
  };

  // operand reads: A^T columns (rows of A) and B^T rows (columns of B) of one order
  auto read_a = [&](int buf, int o, int fm) {
    const int row = FM * 16 * wm + 16 * fm + c;
    return *reinterpret_cast<const u32x4*>(&As[buf][o][row * BK + cauchy_swz_rows(row, g) * 8]);
  };
  auto read_b = [&](int buf, int o, int fn) {
    const int n0 = FN * 16 * wn + 16 * fn;
    if constexpr (TRANS_B) {
      const int row = n0 + c;
      return *reinterpret_cast<const u32x4*>(&Bs[buf][o][row * BK + cauchy_swz_rows(row, g) * 8]);
    } else {
      const int j = c / 4, a = c % 4;
      const int k1 = 8 * g + j, k2 = 8 * g + 4 + j;
      const int lch = n0 / 8 + a / 2, e = 4 * (a % 2);
      return lds_read_tr16x2(&Bs[buf][o][k1 * BN + cauchy_swz_k<WIDE>(k1, lch) * 8 + e],
                             &Bs[buf][o][k2 * BN + cauchy_swz_k<WIDE>(k2, lch) * 8 + e]);
    }
  };

  floatx4 acc[K + 1][FM][FN];
#pragma unroll
  for (int o = 0; o <= K; ++o)
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) acc[o][fm][fn] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int chunks = (Kd + BK - 1) / BK;
  issue(0, 0);
  for (int ch = 0; ch < chunks; ++ch) {
    const int buf = ch & 1;
    __builtin_amdgcn_s_waitcnt(0);   // this wave's DMA of chunk ch has landed
    __syncthreads();                 // ... and every wave's; chunk ch-1's buffer is free
    if (ch + 1 < chunks) issue(buf ^ 1, (ch + 1) * BK);

    u32x4 bf[BO][FN];
    if constexpr (!WIDE) {   // every operand of the chunk in registers, products by output order
      u32x4 af[AO][FM];
#pragma unroll
      for (int o = 0; o < AO; ++o)
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) af[o][fm] = read_a(buf, o, fm);
#pragma unroll
      for (int o = 0; o < BO; ++o)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) bf[o][fn] = read_b(buf, o, fn);
#pragma unroll
      for (int k = 0; k <= K; ++k)
#pragma unroll
        for (int i = 0; i <= k; ++i) {
          const int j = k - i;
          if (i < AO && j < BO) {   // compile-time after unrolling
#pragma unroll
            for (int fm = 0; fm < FM; ++fm)
#pragma unroll
              for (int fn = 0; fn < FN; ++fn) acc[k][fm][fn] = MM::mma(bf[j][fn], af[i][fm], acc[k][fm][fn]);
          }
        }
    } else {                 // B operands held, A read one order at a time (register budget of 2 waves/SIMD)
#pragma unroll
      for (int o = 0; o < BO; ++o)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) bf[o][fn] = read_b(buf, o, fn);
#pragma unroll
      for (int i = 0; i < AO; ++i) {
        u32x4 af[FM];
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) af[fm] = read_a(buf, i, fm);
#pragma unroll
        for (int j = 0; j < BO; ++j) {
          if (i + j <= K) {   // compile-time after unrolling
#pragma unroll
            for (int fm = 0; fm < FM; ++fm)
#pragma unroll
              for (int fn = 0; fn < FN; ++fn) acc[i + j][fm][fn] = MM::mma(bf[j][fn], af[fm], acc[i + j][fm][fn]);
          }
        }
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0);

  // ---- epilogue: lane (c, g) holds C[m0 + c][n0 + 4g .. + 3] of each block ----
  const bool vec = c_vec != 0;   // N % 4 == 0 and every C_k 8-byte aligned: 8-byte stores
#pragma unroll
  for (int o = 0; o <= K; ++o) {
    T* base = C.p[o] + batch * static_cast<int64_t>(M) * N;
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const int row = tile_m + FM * 16 * wm + 16 * fm + c;
        const int col = tile_n + FN * 16 * wn + 16 * fn + 4 * g;
        if (row >= M) continue;
        const floatx4 v = acc[o][fm][fn];
        T* p = base + static_cast<int64_t>(row) * N + col;
        if (vec && col + 3 < N) {
          *reinterpret_cast<uint2*>(p) = make_uint2(MM::pack2(v[0], v[1]), MM::pack2(v[2], v[3]));
        } else {
          uint16_t* q = reinterpret_cast<uint16_t*>(p);
          const uint32_t w01 = MM::pack2(v[0], v[1]), w23 = MM::pack2(v[2], v[3]);
          if (col < N) q[0] = static_cast<uint16_t>(w01);
          if (col + 1 < N) q[1] = static_cast<uint16_t>(w01 >> 16);
          if (col + 2 < N) q[2] = static_cast<uint16_t>(w23);
          if (col + 3 < N) q[3] = static_cast<uint16_t>(w23 >> 16);
        }
      }
  }
}

// Zero orders 1..degree of C (both operands ordinary: only C_0 is a product).
template <typename T>
__global__ __launch_bounds__(256) void cauchy_half_zero_orders_kernel(MPtrs<T> C, int degree, int64_t count) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int o = 1; o <= degree; ++o)
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride)
      reinterpret_cast<uint16_t*>(C.p[o])[i] = 0;
}

template <typename T, int K, int AO, int BO, bool WIDE>
static int launch_cauchy_half_tile(const CauchyArgs& a, const CPtrs<T>& A, const CPtrs<T>& B, const MPtrs<T>& C) {
  using Tile = CauchyHalfTile<AO, BO, WIDE>;
  const dim3 grid((a.n + Tile::BN - 1) / Tile::BN, (a.m + Tile::BM - 1) / Tile::BM, a.batch);
  const dim3 block(Tile::kThreads);
  const int M = static_cast<int>(a.m), N = static_cast<int>(a.n), Kd = static_cast<int>(a.k);
  int c_vec = N % 4 == 0;
  for (int o = 0; o <= K; ++o) c_vec = c_vec && reinterpret_cast<uintptr_t>(C.p[o]) % 8 == 0;
  if (a.trans_b)
    cauchy_matmul_half_kernel<T, K, AO, BO, true, WIDE>
        <<<grid, block, 0, a.stream>>>(A, B, C, M, N, Kd, a.a_bs, a.b_bs, c_vec);
  else
    cauchy_matmul_half_kernel<T, K, AO, BO, false, WIDE>
        <<<grid, block, 0, a.stream>>>(A, B, C, M, N, Kd, a.a_bs, a.b_bs, c_vec);
  PT_LAUNCH_CHECK();
  return PT_OK;
}

// The wide tile where its LDS fits, its (K+1) x 32 accumulator registers leave room for the
// operands within 256 (K <= 4), and both output sides span at least two of its tiles.
template <typename T, int K, int AO, int BO>
static int launch_cauchy_half_orders(const CauchyArgs& a, const CPtrs<T>& A, const CPtrs<T>& B, const MPtrs<T>& C) {
  if constexpr (K <= 4 && CauchyHalfTile<AO, BO, true>::LDS <= 160 * 1024) {
    if (a.m >= 256 && a.n >= 256) return launch_cauchy_half_tile<T, K, AO, BO, true>(a, A, B, C);
  }
  return launch_cauchy_half_tile<T, K, AO, BO, false>(a, A, B, C);
}

template <typename T, int K>
static int launch_cauchy_half_k(const CauchyArgs& a) {
  CPtrs<T> A{}, B{};
  MPtrs<T> C{};
  for (int o = 0; o < a.a_orders; ++o) A.p[o] = static_cast<const T*>(a.a[o]);
  for (int o = 0; o < a.b_orders; ++o) B.p[o] = static_cast<const T*>(a.b[o]);
  for (int o = 0; o <= K; ++o) C.p[o] = static_cast<T*>(a.c[o]);
  const bool a_series = a.a_orders > 1, b_series = a.b_orders > 1;
  if constexpr (K == 0) {
    return launch_cauchy_half_orders<T, 0, 1, 1>(a, A, B, C);
  } else {
    if (a_series && b_series) return launch_cauchy_half_orders<T, K, K + 1, K + 1>(a, A, B, C);
    if (a_series) return launch_cauchy_half_orders<T, K, K + 1, 1>(a, A, B, C);
    if (b_series) return launch_cauchy_half_orders<T, K, 1, K + 1>(a, A, B, C);
    const int st = launch_cauchy_half_orders<T, 0, 1, 1>(a, A, B, C);
    if (st != PT_OK) return st;
    const int64_t count = a.batch * a.m * a.n;
    const int64_t blocks = std::min<int64_t>((count + 255) / 256, 4096);
    cauchy_half_zero_orders_kernel<T><<<dim3(blocks), dim3(256), 0, a.stream>>>(C, K, count);
    PT_LAUNCH_CHECK();
    return PT_OK;
  }
}

template <typename T>
int launch_cauchy_half(const CauchyArgs& a) {
  // 16-byte DMA chunks: whole chunks of the contraction (and of N for B stored [k][n]), aligned
  // operands and batch strides, and each batch's matrix addressable with 32-bit offsets
  constexpr int64_t kLimit = int64_t{1} << 30;
  bool ok = a.k % 8 == 0 && (a.trans_b || a.n % 8 == 0) && a.a_bs % 8 == 0 && a.b_bs % 8 == 0 &&
            a.m * a.k * 2 < kLimit && a.k * a.n * 2 < kLimit;
  for (int o = 0; o < a.a_orders; ++o) ok = ok && pt_host::aligned16(a.a[o]);
  for (int o = 0; o < a.b_orders; ++o) ok = ok && pt_host::aligned16(a.b[o]);
  if (!ok) {
    pt_host::set_error(
        "Cauchy matmul (16-bit): needs the contraction size (and n unless trans_b) to be multiples of 8, "
        "16-byte aligned operands and batch strides, and each matrix below 1 GiB");
    return PT_UNSUPPORTED;
  }
  switch (a.degree) {
    case 0: return launch_cauchy_half_k<T, 0>(a);
    case 1: return launch_cauchy_half_k<T, 1>(a);
    case 2: return launch_cauchy_half_k<T, 2>(a);
    case 3: return launch_cauchy_half_k<T, 3>(a);
    case 4: return launch_cauchy_half_k<T, 4>(a);
    case 5: return launch_cauchy_half_k<T, 5>(a);
    case 6: return launch_cauchy_half_k<T, 6>(a);
    case 7: return launch_cauchy_half_k<T, 7>(a);
    case 8: return launch_cauchy_half_k<T, 8>(a);
    default: break;
  }
  pt_host::set_error("Cauchy matmul: degree outside 0..PT_MAX_DEGREE");
  return PT_UNSUPPORTED;
}

}  // namespace pt
