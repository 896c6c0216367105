// Flash-style attention backward of degree-K series with bfloat16 / float16
// operands on the 16x16x32 MFMAs of gfx950 (fp32 accumulation).
//
// The series arithmetic is that of taylor_attention_bwd.inl (the VJP of
// O = softmax(scale Q K^T) V in truncated series arithmetic):
//   P = exp(scale Q (*) K^T - lse),  dP = G (*) V^T,  Delta = rowsum(G (*) O),
//   dS = P (*) (dP - Delta),  dQ = scale dS (*) K,  dK = scale dS^T (*) Q,  dV = P^T (*) G,
// the reference's degree-1 backward for half types
// (/root/reference/src/polytensors/_attention_kernels.py:85-201: half operands,
// fp32 accumulation, _fused_attention.py:72-78) at degree K. Only the MFMA
// operands are 16-bit: Q, K, V and G as stored, and P and dS rounded to the
// storage type for the products that contract them (from degree 5 as a hi + lo
// pair, as the forward's probabilities). Scores, dP, the exponential series,
// dS and every accumulator are fp32; lse and Delta are fp32 series; each
// gradient is rounded to the storage type once.
//
// With v_mfma_f32_16x16x32 (lane l = 16 g + c supplies A row c and B column c,
// contraction elements 8 g .. 8 g + 7; accumulator register r of lane l is row
// 4 g + r, column c) both kernels form the scores so that the probability and
// dS values a lane holds are the B operand of its output product without
// leaving the lane (as the forward's value product does):
// * taylor_attention_bwd_q_half_kernel: 64 queries per workgroup (16 per wave),
//   key blocks of 32 keys with K and V staged row-major in LDS. S^T = K Q^T and
//   dP^T = V G^T per 16-key half: lane (c, g) holds keys 4 g + r (+ 16) of query
//   c, whose lse and Delta are per-lane constants. dQ^T += K^T dS^T contracts the
//   block's 32 keys with lane group g's slots 8 g .. 8 g + 7 standing for keys
//   4 g .. 4 g + 3 and 16 + 4 g .. 16 + 4 g + 3; its A operand (K^T) is two
//   transpose reads (ds_read_b64_tr_b16) of the row-major K tile.
// * taylor_attention_bwd_kv_half_kernel: 64 keys per workgroup (16 per wave),
//   query blocks of 32 queries with Q and G (and their lse and Delta series)
//   staged in LDS. S = Q K^T and dP = G V^T per 16-query half: lane (c, g) holds
//   queries 4 g + r (+ 16) of key c. dV^T += G^T P and dK^T += Q^T dS take their
//   A operands (G^T, Q^T) from transpose reads of the row-major tiles.
// Output accumulators beyond a register budget are split into head-dim slices
// (a grid dimension; each slice recomputes its scores), and dK and dV get one
// pass each when both do not fit. Deterministic (no atomics).
#pragma once

#include "half_mfma.h"
#include "taylor_attention_bwd.inl"
#include "taylor_attention_half.inl"

namespace pt {

template <int K, int D>
struct AttnHalfBwdShape {
  static constexpr int KB = 32;              // keys (dQ kernel) or queries (dK/dV kernel) per block
  static constexpr int DC = (D + 31) / 32;   // 32-wide head-dim chunks of the score contractions
  static constexpr int DB = D / 16;          // 16-wide output blocks
  static constexpr int LD = D + 8;           // tile row: 16-byte aligned, 4 banks of skew per row
  static constexpr size_t LDS = 2ull * (K + 1) * KB * LD * 2 + 2ull * (K + 1) * KB * 4;
  static constexpr bool fits = LDS <= 160 * 1024;
  static constexpr bool split = K >= 5;      // P and dS orders 1..K as hi + lo operand pairs
  // output accumulator registers per lane: the score and dP series, the 16-bit operands and, from
  // degree 5, the lo operands take the rest
  static constexpr int kBudget = K >= 5 ? 96 : 160;
  static constexpr int slices(int outputs) {
    int sl = 1;
    while (sl < DB && outputs * (K + 1) * (DB / sl) * 4 > kBudget) sl *= 2;
    return sl;
  }
  static constexpr int SL_Q = slices(1);
  static constexpr bool kv_fused = 2 * (K + 1) * DB * 4 <= kBudget;   // dK and dV in one pass
  static constexpr int SL_KV = slices(kv_fused ? 2 : 1);
  // How many of `ops` row tiles of the lane (every order, the whole head dim) stay in registers
  // beside `outputs` accumulator series of nb 16-wide blocks and the working set: scores, dP and
  // the series (about 30 (K+1) registers), the lo operands of `packed` split series and the mask
  // values. The bound of 410 keeps every instantiation free of scratch spills (the compiler's
  // resource remarks).
  static constexpr int resident(int ops, int outputs, int nb, int packed, bool masked, int extra = 0) {
    const int fixed = outputs * (K + 1) * nb * 4 + 30 * (K + 1) + (split ? packed * 4 * (K + 1) : 0) +
                      (masked ? 16 : 0) + extra;
    int n = ops;
    while (n > 0 && n * (K + 1) * DC * 4 + fixed > 410) --n;
    return n;
  }
  // whether `rings` operands fit a two-slot chunk ring beside the same working set (else they are
  // loaded chunk by chunk)
  static constexpr bool ring_fits(int rings, int outputs, int nb, int packed, bool masked, int extra) {
    return outputs * (K + 1) * nb * 4 + 30 * (K + 1) + (split ? packed * 4 * (K + 1) : 0) + (masked ? 16 : 0) +
               extra + rings * 2 * (K + 1) * 4 <= 460;
  }
  // the pipelined dK/dV kernel's operands (K, then V for dK) resident or in a ring (masked case,
  // its DMA bookkeeping counted): else the staged kernel runs
  static constexpr bool kv_pipe_regs(int what) {
    const int nops = (what & 2) ? 2 : 1, outs = ((what & 2) ? 1 : 0) + ((what & 1) ? 1 : 0);
    const int extra = (what & 2) ? 32 : 0;
    const int nr = resident(nops, outs, DB, outs, true, extra);
    return nr == nops || ring_fits(nops - nr, outs, DB, outs, true, extra);
  }
  // operands not resident are read one 32-wide chunk ahead through a two-slot ring, except at
  // degree 8 and head dim 128, where the ring's registers make the kernels spill
  static constexpr bool ring = !(K >= 8 && D == 128);
};

// ROWS rows from row `first` (zero from row `limit` on, limit >= 1) of the K+1
// orders of a [*, D] 16-bit series at row_base into an LDS tile [K+1][ROWS][LD].
// Every lane issues all of its 16-byte loads (clamped rows, no branch) before
// its stores.
template <typename T, int K, int D, int ROWS, int LD>
__device__ __forceinline__ void attn_half_stage(T (&tile)[K + 1][ROWS][LD], const CPtrs<T>& src,
                                                int64_t row_base, int first, int limit) {
  constexpr int VPR = D / 8;   // 16-byte vectors per row
  constexpr int N = (K + 1) * ROWS * VPR;
  constexpr int THREADS = kAttnWaves * kWave;
  constexpr int IT = (N + THREADS - 1) / THREADS;
  u32x4 v[IT];
#pragma unroll
  for (int j = 0; j < IT; ++j) {
    const int e = min(static_cast<int>(threadIdx.x) + THREADS * j, N - 1);
    const int o = e / (ROWS * VPR), rem = e % (ROWS * VPR);
    const int row = first + rem / VPR, cv = (rem % VPR) * 8;
    v[j] = *reinterpret_cast<const u32x4*>(order_ptr<K>(src, o) + (row_base + min(row, limit - 1)) * D + cv);
  }
#pragma unroll
  for (int j = 0; j < IT; ++j) {
    const int idx = static_cast<int>(threadIdx.x) + THREADS * j;
    if (N % THREADS == 0 || idx < N) {
      const int o = idx / (ROWS * VPR), rem = idx % (ROWS * VPR);
      const int r = rem / VPR, cv = (rem % VPR) * 8;
      const u32x4 z = {0u, 0u, 0u, 0u};
      *reinterpret_cast<u32x4*>(&tile[o][r][cv]) = first + r < limit ? v[j] : z;
    }
  }
}

// Packs the series w[o][0..3] of one 16-row half into slots 4 h .. 4 h + 3 of the
// 16-bit operands hi[o] (and, when split, the rounding residuals of orders
// 1..K into lo[o]).
template <typename T, int K, bool SPLIT, int NLO>
__device__ __forceinline__ void attn_half_pack(const float (&w)[K + 1][4], int h, u32x4 (&hi)[K + 1],
                                               u32x4 (&lo)[NLO]) {
  using MM = HalfMfma<T>;
#pragma unroll
  for (int o = 0; o <= K; ++o) {
    const uint32_t w01 = MM::pack2(w[o][0], w[o][1]), w23 = MM::pack2(w[o][2], w[o][3]);
    hi[o][2 * h] = w01;
    hi[o][2 * h + 1] = w23;
    if constexpr (SPLIT) {
      if (o >= 1) {
        lo[o][2 * h] = MM::pack2(w[o][0] - MM::lo(w01), w[o][1] - MM::hi(w01));
        lo[o][2 * h + 1] = MM::pack2(w[o][2] - MM::lo(w23), w[o][3] - MM::hi(w23));
      }
    }
  }
}

// acc[k] += sum_{a+b=k} X_b^T W_a for one 16-wide output block: xt[b] the A operands, W the
// packed B operands (hi, and lo for orders 1..K when split).
template <typename T, int K, bool SPLIT, int NLO>
__device__ __forceinline__ void attn_half_series_mma(floatx4 (&acc)[K + 1], const u32x4 (&xt)[K + 1],
                                                     const u32x4 (&hi)[K + 1], const u32x4 (&lo)[NLO]) {
  using MM = HalfMfma<T>;
#pragma unroll
  for (int k = 0; k <= K; ++k) {
#pragma unroll
    for (int a = 0; a <= k; ++a) acc[k] = MM::mma(xt[k - a], hi[a], acc[k]);
    if constexpr (SPLIT) {
#pragma unroll
      for (int a = 1; a <= k; ++a) acc[k] = MM::mma(xt[k - a], lo[a], acc[k]);
    }
  }
}

// Stores the accumulators acc[db][k] of one 16-row output tile: head dims d0 + 16 db + 4 g .. + 3
// of row `row` (8 bytes per order and block), times factor.
template <typename T, int K, int NB>
__device__ __forceinline__ void attn_half_store(const floatx4 (&acc)[NB][K + 1], MPtrs<T>& out, int64_t row,
                                                int d0, int g, float factor) {
  using MM = HalfMfma<T>;
#pragma unroll
  for (int db = 0; db < NB; ++db)
#pragma unroll
    for (int k = 0; k <= K; ++k)
      *reinterpret_cast<uint2*>(out.p[k] + row + d0 + 16 * db + 4 * g) =
          make_uint2(MM::pack2(acc[db][k][0] * factor, acc[db][k][1] * factor),
                     MM::pack2(acc[db][k][2] * factor, acc[db][k][3] * factor));
}

// MASK: 0 no mask, 1 a boolean mask, 2 a boolean mask and the additive mask madd (float) whose
// finite entries it marks.
template <typename T, int K, int D, int SL, int MASK>
__global__ __launch_bounds__(kAttnWaves * kWave) void taylor_attention_bwd_q_half_kernel(
    CPtrs<T> Q, CPtrs<T> Kp, CPtrs<T> Vp, CPtrs<T> G, CPtrs<float> LSE, CPtrs<float> DELTA, MPtrs<T> DQ, int L,
    int S, const uint8_t* __restrict__ mask_all, AttnMaskMap mmap, const float* __restrict__ madd_all,
    const int32_t* __restrict__ ranges_all, int causal, float scale) {
  using Sh = AttnHalfBwdShape<K, D>;
  using MM = HalfMfma<T>;
  constexpr int KB = Sh::KB, DC = Sh::DC, LD = Sh::LD;
  constexpr int DS = D / SL, DBS = DS / 16;
  constexpr bool SPLIT = Sh::split;
  constexpr int NLO = SPLIT ? K + 1 : 1;
  static_assert(Sh::fits, "K/V tiles exceed LDS");
  __shared__ __align__(16) T Ks[K + 1][KB][LD];
  __shared__ __align__(16) T Vs[K + 1][KB][LD];

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int c = lane % 16;   // query column of the score accumulators; A row of the operands
  const int g = lane / 16;   // lane group
  const int nqb = (L + kAttnBM - 1) / kAttnBM;
  const int64_t bh = gridDim.x / (static_cast<int64_t>(nqb) * SL);
  int64_t head;
  int slice, q_block;
  attn_bwd_q_item(blockIdx.x, bh, nqb, SL, head, slice, q_block);
  const int d0 = slice * DS;
  const int64_t mask_index = attn_mask_index(mmap, head);
  const uint8_t* mask = MASK != 0 ? mask_all + mask_index * L * S : nullptr;
  const float* madd = MASK == 2 ? madd_all + mask_index * L * S : nullptr;
  const int32_t* ranges = ranges_all != nullptr ? ranges_all + mask_index * attn_ranges_count(L, S) : nullptr;
  const int my_q = q_block + wave * kAttnQPerWave + c;
  const bool q_ok = my_q < L;
  const int64_t qrow = (head * L + (q_ok ? my_q : L - 1)) * D;
  float lse[K + 1], delta[K + 1];
#pragma unroll
  for (int o = 0; o <= K; ++o) {
    lse[o] = q_ok ? LSE.p[o][head * L + my_q] : 0.f;
    delta[o] = q_ok ? DELTA.p[o][head * L + my_q] : 0.f;
  }
  // operand of the lane's query row, order o, chunk dc: X[my_q][32 dc + 8 g .. + 7] (zero past D)
  auto load_row = [&](const CPtrs<T>& X, int o, int dc) -> u32x4 {
    const bool din = 32 * dc + 8 * g < D;
    return attn_half_load8<T>(X.p[o] + qrow + (din ? 32 * dc + 8 * g : 0), din);
  };
  // The lane's Q and G rows are the same for every key block: resident in registers when they fit
  // beside the accumulators and the score series, else read (from L2) per block.
  constexpr int NRES = Sh::resident(2, 1, DBS, 1, MASK != 0);   // Q, then G
  u32x4 rows[NRES > 0 ? NRES : 1][K + 1][DC];
#pragma unroll
  for (int i = 0; i < NRES; ++i)
#pragma unroll
    for (int o = 0; o <= K; ++o)
#pragma unroll
      for (int dc = 0; dc < DC; ++dc) rows[i][o][dc] = load_row(i == 0 ? Q : G, o, dc);
  u32x4 ring[2][2][K + 1];   // chunk ring of each operand not resident

  floatx4 acc[DBS][K + 1];   // dQ^T series of each 16-wide head-dim block
#pragma unroll
  for (int db = 0; db < DBS; ++db)
#pragma unroll
    for (int o = 0; o <= K; ++o) acc[db][o] = floatx4{0.f, 0.f, 0.f, 0.f};

  // key range: causal and mask-range bounds, lo rounded down to a 32-key block
  int lo = 0, hi = S;
  if (causal) hi = min(S, q_block + kAttnBM);
  if (ranges != nullptr) {
    const int qb = q_block / kAttnRangeBlock;
    lo = ranges[2 * qb] / KB * KB;
    hi = min(hi, static_cast<int>(ranges[2 * qb + 1]));
  }
  const int tj = c / 4, ta = c % 4;   // transpose reads: this lane addresses row 4 g + tj (+ 16), dims + 4 ta

  for (int kb0 = lo; kb0 < hi; kb0 += KB) {
    uint8_t mbyte[2][4];
    float add[2][4];
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kb0 + 16 * kh + 4 * g + r;
        mbyte[kh][r] = MASK != 0 ? attn_mask_byte(mask, Q.p[0], my_q, key, L, S) : uint8_t(1);
        add[kh][r] = MASK == 2 ? attn_mask_add(madd, my_q, key, L, S) : 0.f;
      }
    // chunk 0 of the operands not resident, in flight during the staging
#pragma unroll
    for (int i = NRES; i < 2; ++i)
#pragma unroll
      for (int o = 0; o <= K; ++o)
        if constexpr (Sh::ring) ring[i][0][o] = load_row(i == 0 ? Q : G, o, 0);
    __syncthreads();   // the previous block's products are done with the tiles
    attn_half_stage<T, K, D, KB, LD>(Ks, Kp, head * S, kb0, S);
    attn_half_stage<T, K, D, KB, LD>(Vs, Vp, head * S, kb0, S);
    __syncthreads();

    // ---- S^T_k = sum_{a+b=k} K_b Q_a^T and dP^T_k = sum_{a+b=k} V_b G_a^T (keys x queries) ----
    // (one contraction after the other: their operands are not live together)
    floatx4 sc[2][K + 1], dp[2][K + 1];
    auto contract = [&](floatx4 (&acc)[2][K + 1], const CPtrs<T>& X, int which, const T (&tile)[K + 1][KB][LD]) {
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int o = 0; o <= K; ++o) acc[kh][o] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int dc = 0; dc < DC; ++dc) {
        // resident rows, or the ring: chunk dc + 1 is loaded while chunk dc's products run
        u32x4 xa[K + 1];
        if (Sh::ring && which >= NRES && dc + 1 < DC) {
#pragma unroll
          for (int o = 0; o <= K; ++o) ring[which][(dc + 1) & 1][o] = load_row(X, o, dc + 1);
        }
#pragma unroll
        for (int o = 0; o <= K; ++o)
          xa[o] = which < NRES ? rows[which < NRES ? which : 0][o][dc]
                               : (Sh::ring ? ring[which][dc & 1][o] : load_row(X, o, dc));
        const bool din = 32 * dc + 8 * g < D;
        const int col = din ? 32 * dc + 8 * g : 0;
        const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
          u32x4 top[K + 1];
#pragma unroll
          for (int o = 0; o <= K; ++o) {
            const u32x4 t = *reinterpret_cast<const u32x4*>(&tile[o][16 * kh + c][col]);
            top[o] = din ? t : z;
          }
#pragma unroll
          for (int k = 0; k <= K; ++k)
#pragma unroll
            for (int a = 0; a <= k; ++a) acc[kh][k] = MM::mma(top[k - a], xa[a], acc[kh][k]);
        }
      }
    };
    contract(sc, Q, 0, Ks);
    contract(dp, G, 1, Vs);

    // ---- probability and dS series; dS^T as the B operand (slots 4 kh + r: key 16 kh + 4 g + r) ----
    u32x4 dsb[K + 1], dsl[NLO];
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      float w[K + 1][4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kb0 + 16 * kh + 4 * g + r;
        bool ok = q_ok && key < S;
        if (causal) ok = ok && key <= my_q;
        if constexpr (MASK != 0) ok = ok && mbyte[kh][r] != 0;
        float p[K + 1], ds[K + 1];
        attn_prob_series<float, K>(sc[kh], r, lse, ok, scale, add[kh][r], p);
        attn_ds_series<float, K>(p, dp[kh], r, delta, ds);
#pragma unroll
        for (int o = 0; o <= K; ++o) w[o][r] = ds[o];
      }
      attn_half_pack<T, K, SPLIT, NLO>(w, kh, dsb, dsl);
    }

    // ---- dQ^T_k += sum_{a+b=k} K_b^T dS^T_a (head dim x queries), 32 keys per MFMA ----
#pragma unroll
    for (int db = 0; db < DBS; ++db) {
      u32x4 kt[K + 1];
      const int col = d0 + 16 * db + 4 * ta;
#pragma unroll
      for (int o = 0; o <= K; ++o) kt[o] = lds_read_tr16x2(&Ks[o][4 * g + tj][col], &Ks[o][16 + 4 * g + tj][col]);
      attn_half_series_mma<T, K, SPLIT, NLO>(acc[db], kt, dsb, dsl);
    }
  }

  if (q_ok) attn_half_store<T, K, DBS>(acc, DQ, (head * L + my_q) * D, d0, g, scale);
}

// ---------------------------------------------------------------------------
// Pipelined dQ kernel: the K and V tiles of key block j+1 move by LDS DMA while
// block j's products run (the layout and DMA geometry of the forward's
// pipelined kernel: rows unpadded, 16-byte chunks XOR-swizzled by the row with
// AttnHalfPipe::fs). K is read to the end of a block (the dQ product) and takes
// two buffers; V is read by the dP product only and takes one, refilled once
// every wave is past it:
//   top of block j: this wave's DMAs have landed (s_waitcnt), barrier;
//     DMA K_{j+1} into the other K buffer;
//   S and dP per 16-key half, then P and dS;
//   barrier (every wave is done with V_j); DMA V_{j+1}; (stored tiles) the P / dS stores;
//   dQ += K_j^T dS^T.
// The DMA is hidden from the compiler (lds_dma16), so a compiler-visible load
// issued after one waits for it too (loads complete in order): inside the loop
// only the G chunks, when G is not resident, are loaded, after the K DMA that
// the score products give time to land (issuing the K DMA after the dP product
// instead measured 3% slower at degree 4, head dim 128).
template <int K, int D>
struct AttnHalfBwdPipe {
  using P = AttnHalfPipe<K, D>;
  static constexpr int KB = 32;
  static constexpr size_t tile = static_cast<size_t>(K + 1) * KB * D * 2;
  // (degree 0 and head dim 16 stay on the staged kernels: at degree 0 the compiler places the
  // DMA's buffer resource in vector registers, which the instruction does not take)
  static constexpr bool fits_q = 3 * tile <= 160 * 1024 && D >= 32 && K >= 1;
  static constexpr int OPT = (K + 1) * P::IT;   // DMA operations per wave and tile
};

// DMA operation i (0 <= i < (K+1) IT) of this wave's share of rows first .. first + 31 of a
// head's [rows, D] series into a tile [K+1][32][D] (chunks swizzled with fs; rows past `rows`
// load zeros).
template <typename T, int K, int D>
__device__ __forceinline__ void attn_half_dma_tile(T (&tile)[K + 1][32][D], const CPtrs<T>& src, int64_t head,
                                                   int rows, int first, int lane, int wave, int i) {
  using P = AttnHalfPipe<K, D>;
  constexpr int CH = P::CH, RPS = P::RPS, SEGS = P::SEGS, IT = P::IT;
  const int o = i / IT, it = i % IT;
  const int seg = it * kAttnWaves + wave;
  if (SEGS % kAttnWaves != 0 && seg >= SEGS) return;
  const int row = seg * RPS + lane / CH;
  const int lch = (lane % CH) ^ P::fs(row);
  const BufferRsrc rsrc = buffer_rsrc(src.p[o] + head * rows * D, rows * D * static_cast<int>(sizeof(T)));
  lds_dma16(&tile[o][seg * RPS][0], rsrc, ((first + row) * D + lch * 8) * static_cast<int>(sizeof(T)));
}

// Row operand of a swizzled tile: row `row`, 16-byte logical chunk `ch` (zero when din is false).
template <typename T, int K, int D>
__device__ __forceinline__ u32x4 attn_half_tile_row(const T (&tile)[K + 1][32][D], int o, int row, int ch, bool din) {
  using P = AttnHalfPipe<K, D>;
  const int pch = (ch & (P::CH - 1)) ^ P::fs(row);
  const u32x4 v = *reinterpret_cast<const u32x4*>(&tile[o][row][pch * 8]);
  const u32x4 z = {0u, 0u, 0u, 0u};
  return din ? v : z;
}

// Transposed operand of a swizzled tile: head dims 16 db + c of rows 4 g .. 4 g + 3 and
// 16 + 4 g .. 16 + 4 g + 3 (two ds_read_b64_tr_b16; lane c = 4 tj + ta addresses row 4 g + tj).
template <typename T, int K, int D>
__device__ __forceinline__ u32x4 attn_half_tile_tr(const T (&tile)[K + 1][32][D], int o, int db, int g, int tj,
                                                   int ta) {
  using P = AttnHalfPipe<K, D>;
  const int row0 = 4 * g + tj, row1 = 16 + 4 * g + tj;
  const int lch = 2 * db + ta / 2;
  const int off0 = ((lch ^ P::fs(row0)) * 8) + 4 * (ta % 2);
  const int off1 = ((lch ^ P::fs(row1)) * 8) + 4 * (ta % 2);
  return lds_read_tr16x2(&tile[o][row0][off0], &tile[o][row1][off1]);
}

// STORE: also write the P and dS series of every visited (query, key) pair to PT / DST (the dS
// values as rounded for the dQ product) for taylor_attention_bwd_kv_half_mat_kernel, in 32-key
// blocks: [head][srow / 32 key blocks][L queries][32 positions] 16-bit values, key 16 h + 4 g + r
// of a block at position 8 g + 4 (h ^ q2) + r, q2 = bit 2 of the query (the eight keys a lane
// holds are adjacent), so that a wave's store of a block fills one contiguous kilobyte. The
// consumer's transpose reads of rows 4 g' + j and 4 (g' + 1) + j, the two row groups of one
// 32-lane pass, then fall on the two halves of their chunks instead of the same half (a two-way
// bank conflict on every read). Degrees 1..4 (one 16-bit operand per value).
template <typename T, int K, int D, int MASK, bool STORE>
__global__ __launch_bounds__(kAttnWaves * kWave) void taylor_attention_bwd_q_half_pipe_kernel(
    CPtrs<T> Q, CPtrs<T> Kp, CPtrs<T> Vp, CPtrs<T> G, CPtrs<float> LSE, CPtrs<float> DELTA, MPtrs<T> DQ,
    MPtrs<T> PT, MPtrs<T> DST, int64_t srow, int L, int S, const uint8_t* __restrict__ mask_all, AttnMaskMap mmap,
    const float* __restrict__ madd_all, const int32_t* __restrict__ ranges_all, int causal, float scale) {
  using Sh = AttnHalfBwdShape<K, D>;
  using BP = AttnHalfBwdPipe<K, D>;
  using MM = HalfMfma<T>;
  constexpr int KB = BP::KB, DC = Sh::DC, DB = Sh::DB, OPT = BP::OPT;
  constexpr bool SPLIT = Sh::split;
  constexpr int NLO = SPLIT ? K + 1 : 1;
  static_assert(BP::fits_q, "K/V tiles exceed LDS");
  using Tile = T[K + 1][KB][D];
  __shared__ __attribute__((aligned(16))) Tile Kt[2];
  __shared__ __attribute__((aligned(16))) Tile Vt;

  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int c = lane % 16;
  const int g = lane / 16;
  const int nqb = (L + kAttnBM - 1) / kAttnBM;
  const int64_t bh = gridDim.x / static_cast<int64_t>(nqb);
  int64_t head;
  int slice, q_block;
  attn_bwd_q_item(blockIdx.x, bh, nqb, 1, head, slice, q_block);
  const int64_t mask_index = attn_mask_index(mmap, head);
  const uint8_t* mask = MASK != 0 ? mask_all + mask_index * L * S : nullptr;
  const float* madd = MASK == 2 ? madd_all + mask_index * L * S : nullptr;
  const int32_t* ranges = ranges_all != nullptr ? ranges_all + mask_index * attn_ranges_count(L, S) : nullptr;
  const int my_q = q_block + wave * kAttnQPerWave + c;
  const bool q_ok = my_q < L;
  const int64_t qrow = (head * L + (q_ok ? my_q : L - 1)) * D;
  float lse[K + 1], delta[K + 1];
#pragma unroll
  for (int o = 0; o <= K; ++o) {
    lse[o] = q_ok ? LSE.p[o][head * L + my_q] : 0.f;
    delta[o] = q_ok ? DELTA.p[o][head * L + my_q] : 0.f;
  }
  auto load_row = [&](const CPtrs<T>& X, int o, int dc) -> u32x4 {
    const bool din = 32 * dc + 8 * g < D;
    return attn_half_load8<T>(X.p[o] + qrow + (din ? 32 * dc + 8 * g : 0), din);
  };
  constexpr int NRES = Sh::resident(2, 1, DB, 1, MASK != 0) >= 1 ? Sh::resident(2, 1, DB, 1, MASK != 0) : 1;
  u32x4 rows[NRES][K + 1][DC];   // Q, then G when it fits
#pragma unroll
  for (int i = 0; i < NRES; ++i)
#pragma unroll
    for (int o = 0; o <= K; ++o)
#pragma unroll
      for (int dc = 0; dc < DC; ++dc) rows[i][o][dc] = load_row(i == 0 ? Q : G, o, dc);

  floatx4 acc[DB][K + 1];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int o = 0; o <= K; ++o) acc[db][o] = floatx4{0.f, 0.f, 0.f, 0.f};

  int lo = 0, hi = S;
  if (causal) hi = min(S, q_block + kAttnBM);
  if (ranges != nullptr) {
    const int qb = q_block / kAttnRangeBlock;
    lo = ranges[2 * qb] / KB * KB;
    hi = min(hi, static_cast<int>(ranges[2 * qb + 1]));
  }
  // a workgroup whose rows admit no key keeps one fully masked block (key < hi fails for every
  // key), so the pipeline always has a first block
  if (hi <= lo) lo = hi = 0;
  const int nblocks = max(1, (hi - lo + KB - 1) / KB);
  const int last_kb0 = lo + (nblocks - 1) * KB;
  const int tj = c / 4, ta = c % 4;

  // A block's mask bytes (and additive values) are read one block ahead, right after the barrier
  // that opens the previous block and before that block's DMA: loads complete in issue order, so
  // a read issued at the top of its own block would hold the block for a full memory round trip.
  // (In the stored-tile launches. The recomputing ones, which hold more registers, read them at
  // the top of their block: ahead, their registers made some instantiations spill.)
  constexpr bool kAhead = MASK != 0 && STORE;
  // (one word of mask bytes per half: byte r for key kb0 + 16 kh + 4 g + r)
  uint32_t mnext[2] = {0u, 0u};
  float anext[MASK == 2 ? 2 : 1][4];
  const bool mvec = MASK != 0 && attn_mask_vec(mask, madd, S);
  auto fetch_mask = [&](int kb0) __attribute__((always_inline)) {
    if constexpr (MASK != 0) {
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
        mnext[kh] = attn_mask_word4<MASK == 2>(mask, madd, my_q, kb0 + 16 * kh + 4 * g, L, S, mvec,
                                               anext[MASK == 2 ? kh : 0]);
    }
  };

  // block 0's tiles (after the row loads: the compiler's waits for those would wait for the DMA).
  // The row loads are waited for here, once: otherwise the compiler, which sees them pending at
  // the loop's entry, waits for them inside the loop, on every block, where the count it uses
  // also covers that block's DMAs and the previous block's stores.
  __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
  for (int i = 0; i < OPT; ++i) {
    attn_half_dma_tile<T, K, D>(Kt[0], Kp, head, S, lo, lane, wave, i);
    attn_half_dma_tile<T, K, D>(Vt, Vp, head, S, lo, lane, wave, i);
  }
  if constexpr (kAhead) fetch_mask(lo);

  // The P / dS stores of a block go out after its last DMA, both halves' in one 16-byte store per
  // series and order (2(K+1)), so the next block waits for its DMAs only. A wave with rows issues
  // all of them (their branch skips only a wave without rows). Stored half by half (8 bytes), they
  // also cost the second half a reload of the G rows (the compiler cannot move those loads above
  // the first half's stores): a padding mask's dQ kernel took 5.48 ms that way at degree 4, d 128.
  // Where holding the first half's P operands until the store would spill (there, with a mask, whose
  // values take those registers), they wait in LDS instead, one 8-byte slot per lane and order
  // (10 KB; the tiles leave 40 KB).
  constexpr bool STAGE0 = STORE && MASK != 0 && K >= 4 && D >= 128;
  __shared__ __attribute__((aligned(8))) uint2 pstage[STAGE0 ? kAttnWaves * kWave : 1][K + 1];
  constexpr int kStoresAfterDma = 2 * (K + 1);   // s_waitcnt vmcnt(2(K+1)) expcnt(0) lgkmcnt(0)
  static_assert(!STORE || kStoresAfterDma < 16, "vmcnt field");
  const bool wave_rows = q_block + wave * kAttnQPerWave < L;
  for (int j = 0; j < nblocks; ++j) {
    const int kb0 = lo + j * KB;
    const int next_kb0 = min(kb0 + KB, last_kb0);   // the last block re-loads itself: no branch
    Tile& cur = Kt[j & 1];
    Tile& nxt = Kt[(j + 1) & 1];
    if constexpr (MASK != 0 && !kAhead) fetch_mask(kb0);   // this block's, at its top
    if (STORE && j > 0 && wave_rows) {
      // this wave's DMAs of block j have landed; the tile stores of block j-1 that followed its
      // last DMA, its last 2(K+1) vector memory operations (the counter drops in issue order), may
      // still be in flight
      __builtin_amdgcn_s_waitcnt(kStoresAfterDma);
    } else {
      __builtin_amdgcn_s_waitcnt(0);   // this wave's DMAs of block j have landed (and the mask values)
    }
    __syncthreads();                 // ... and every wave's; block j-1 is done with nxt
    const uint32_t mword[2] = {mnext[0], mnext[1]};
    float add[2][4];
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int r = 0; r < 4; ++r) add[kh][r] = MASK == 2 ? anext[kh][r] : 0.f;
    if constexpr (kAhead) fetch_mask(next_kb0);   // the next block's, ahead of its DMA
#pragma unroll
    for (int i = 0; i < OPT; ++i) attn_half_dma_tile<T, K, D>(nxt, Kp, head, S, next_kb0, lane, wave, i);

    // ---- per 16-key half: S^T = K Q^T, dP^T = V G^T, then the P and dS series ----
    // (the P operands of both halves are held for one store: in registers, or the first half's in
    // LDS where the registers do not allow it)
    u32x4 dsb[K + 1], dsl[NLO], ppk[STORE ? K + 1 : 1];
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      floatx4 sc[K + 1], dp[K + 1];
#pragma unroll
      for (int o = 0; o <= K; ++o) sc[o] = dp[o] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int dc = 0; dc < DC; ++dc) {
        const bool din = 32 * dc + 8 * g < D;
        u32x4 kop[K + 1];
#pragma unroll
        for (int o = 0; o <= K; ++o) kop[o] = attn_half_tile_row<T, K, D>(cur, o, 16 * kh + c, 4 * dc + g, din);
#pragma unroll
        for (int k = 0; k <= K; ++k)
#pragma unroll
          for (int a = 0; a <= k; ++a) sc[k] = MM::mma(kop[k - a], rows[0][a][dc], sc[k]);
      }
#pragma unroll
      for (int dc = 0; dc < DC; ++dc) {
        const bool din = 32 * dc + 8 * g < D;
        u32x4 ga[K + 1], vop[K + 1];
#pragma unroll
        for (int o = 0; o <= K; ++o) {
          ga[o] = NRES >= 2 ? rows[NRES >= 2 ? 1 : 0][o][dc] : load_row(G, o, dc);
          vop[o] = attn_half_tile_row<T, K, D>(Vt, o, 16 * kh + c, 4 * dc + g, din);
        }
#pragma unroll
        for (int k = 0; k <= K; ++k)
#pragma unroll
          for (int a = 0; a <= k; ++a) dp[k] = MM::mma(vop[k - a], ga[a], dp[k]);
      }
      if (kh == 1) {
        // the last read of V_j is behind: V_{j+1} moves during the second half's series, the
        // stores and the dQ products (after them only, it left its latency to the next block's wait)
        __syncthreads();   // every wave is done with V_j
#pragma unroll
        for (int i = 0; i < OPT; ++i) attn_half_dma_tile<T, K, D>(Vt, Vp, head, S, next_kb0, lane, wave, i);
      }
      float w[K + 1][4], wp[STORE ? K + 1 : 1][4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kb0 + 16 * kh + 4 * g + r;
        bool ok = q_ok && key < hi;
        if (causal) ok = ok && key <= my_q;
        if constexpr (MASK != 0) ok = ok && ((mword[kh] >> (8 * r)) & 0xffu) != 0;
        float p[K + 1], ds[K + 1];
        attn_prob_series<float, K>(sc, r, lse, ok, scale, add[kh][r], p);
        attn_ds_series<float, K>(p, dp, r, delta, ds);
#pragma unroll
        for (int o = 0; o <= K; ++o) {
          w[o][r] = ds[o];
          if constexpr (STORE) wp[o][r] = p[o];
        }
      }
      attn_half_pack<T, K, SPLIT, NLO>(w, kh, dsb, dsl);
      if constexpr (STORE) {
        static_assert(!SPLIT, "stored tiles hold one 16-bit value per pair");
        if (STAGE0 && kh == 0) {
#pragma unroll
          for (int o = 0; o <= K; ++o)
            pstage[threadIdx.x][o] = make_uint2(MM::pack2(wp[o][0], wp[o][1]), MM::pack2(wp[o][2], wp[o][3]));
        } else {
#pragma unroll
          for (int o = 0; o <= K; ++o) {
            ppk[o][2 * kh] = MM::pack2(wp[o][0], wp[o][1]);
            ppk[o][2 * kh + 1] = MM::pack2(wp[o][2], wp[o][3]);
          }
        }
      }
    }
    if constexpr (STAGE0) {   // the first half's P operands back from LDS (this lane's own slots)
#pragma unroll
      for (int o = 0; o <= K; ++o) {
        const uint2 h0 = pstage[threadIdx.x][o];
        ppk[o][0] = h0.x;
        ppk[o][1] = h0.y;
      }
    }
    if constexpr (STORE) {
      // the lane's eight keys (4 g + r and 16 + 4 g + r of the block) of its query, at positions
      // 8 g .. 8 g + 7 of the block's 32: one 16-byte store per series and order, a contiguous
      // kilobyte per wave (plain stores: non-temporal ones measured 8% slower)
      __builtin_amdgcn_sched_barrier(0);
      if (q_ok) {
        const int64_t at = ((head * (srow / 32) + kb0 / 32) * L + my_q) * 32 + 8 * g;
        const bool q2 = ((my_q >> 2) & 1) != 0;   // the halves swapped
#pragma unroll
        for (int o = 0; o <= K; ++o) {
          const u32x4 pp = ppk[o], dd = dsb[o];
          *reinterpret_cast<u32x4*>(PT.p[o] + at) = q2 ? u32x4{pp[2], pp[3], pp[0], pp[1]} : pp;
          *reinterpret_cast<u32x4*>(DST.p[o] + at) = q2 ? u32x4{dd[2], dd[3], dd[0], dd[1]} : dd;
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }

    // ---- dQ^T_k += sum_{a+b=k} K_b^T dS^T_a ----
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      u32x4 kt[K + 1];
#pragma unroll
      for (int o = 0; o <= K; ++o) kt[o] = attn_half_tile_tr<T, K, D>(cur, o, db, g, tj, ta);
      attn_half_series_mma<T, K, SPLIT, NLO>(acc[db], kt, dsb, dsl);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);   // the last block's (redundant) DMAs have landed before the workgroup ends

  if (q_ok && DQ.p[0] != nullptr) attn_half_store<T, K, DB>(acc, DQ, (head * L + my_q) * D, 0, g, scale);
}

// WHAT: 1 = dV, 2 = dK, 3 = both. MASK as the dQ kernel's.
template <typename T, int K, int D, int SL, int WHAT, int MASK>
__global__ __launch_bounds__(kAttnWaves * kWave) void taylor_attention_bwd_kv_half_kernel(
    CPtrs<T> Q, CPtrs<T> Kp, CPtrs<T> Vp, CPtrs<T> G, CPtrs<float> LSE, CPtrs<float> DELTA, MPtrs<T> DK,
    MPtrs<T> DV, int L, int S, const uint8_t* __restrict__ mask_all, AttnMaskMap mmap,
    const float* __restrict__ madd_all, const int32_t* __restrict__ ranges_all, int causal, float scale) {
  using Sh = AttnHalfBwdShape<K, D>;
  using MM = HalfMfma<T>;
  constexpr int KB = Sh::KB, DC = Sh::DC, LD = Sh::LD;
  constexpr int DS = D / SL, DBS = DS / 16;
  constexpr bool SPLIT = Sh::split;
  constexpr int NLO = SPLIT ? K + 1 : 1;
  constexpr bool DO_V = (WHAT & 1) != 0, DO_K = (WHAT & 2) != 0;
  static_assert(Sh::fits, "Q/G tiles exceed LDS");
  __shared__ __align__(16) T Qs[K + 1][KB][LD];
  __shared__ __align__(16) T Gs[K + 1][KB][LD];
  __shared__ __align__(16) float Ls[K + 1][KB];
  __shared__ __align__(16) float Ds[K + 1][KB];

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int c = lane % 16;   // key column of the score accumulators; A row of the operands
  const int g = lane / 16;
  const int64_t bh = gridDim.x / (static_cast<int64_t>((S + 63) / 64) * SL);
  int64_t head;
  int slice, kv_block;
  attn_bwd_kv_item(blockIdx.x, bh, SL, head, slice, kv_block);
  const int d0 = slice * DS;
  const int64_t mask_index = attn_mask_index(mmap, head);
  const uint8_t* mask = MASK != 0 ? mask_all + mask_index * L * S : nullptr;
  const float* madd = MASK == 2 ? madd_all + mask_index * L * S : nullptr;
  const int32_t* ranges = ranges_all != nullptr ? ranges_all + mask_index * attn_ranges_count(L, S) : nullptr;
  const int my_k = kv_block + wave * 16 + c;
  const bool k_ok = my_k < S;
  const int64_t krow = (head * S + (k_ok ? my_k : S - 1)) * D;
  auto load_row = [&](const CPtrs<T>& X, int o, int dc) -> u32x4 {
    const bool din = 32 * dc + 8 * g < D;
    return attn_half_load8<T>(X.p[o] + krow + (din ? 32 * dc + 8 * g : 0), din);
  };
  // The lane's K (and, for dK, V) rows are the same for every query block: resident in registers
  // when they fit, else read (from L2) per block.
  constexpr int NRES = Sh::resident(DO_K ? 2 : 1, (DO_K ? 1 : 0) + (DO_V ? 1 : 0), DBS,
                                    (DO_K ? 1 : 0) + (DO_V ? 1 : 0), MASK != 0);   // K, then V
  u32x4 rows[NRES > 0 ? NRES : 1][K + 1][DC];
#pragma unroll
  for (int i = 0; i < NRES; ++i)
#pragma unroll
    for (int o = 0; o <= K; ++o)
#pragma unroll
      for (int dc = 0; dc < DC; ++dc) rows[i][o][dc] = load_row(i == 0 ? Kp : Vp, o, dc);
  u32x4 ring[2][2][K + 1];   // chunk ring of each operand not resident

  floatx4 acc_v[DO_V ? DBS : 1][K + 1], acc_k[DO_K ? DBS : 1][K + 1];
#pragma unroll
  for (int db = 0; db < DBS; ++db)
#pragma unroll
    for (int o = 0; o <= K; ++o) {
      if constexpr (DO_V) acc_v[db][o] = floatx4{0.f, 0.f, 0.f, 0.f};
      if constexpr (DO_K) acc_k[db][o] = floatx4{0.f, 0.f, 0.f, 0.f};
    }

  int lo, hi;
  attn_query_range(L, kv_block, causal, ranges, lo, hi);
  lo = lo / KB * KB;
  const int tj = c / 4, ta = c % 4;

  for (int qb0 = lo; qb0 < hi; qb0 += KB) {
    uint8_t mbyte[2][4];
    float add[2][4];
#pragma unroll
    for (int qh = 0; qh < 2; ++qh)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int q = qb0 + 16 * qh + 4 * g + r;
        mbyte[qh][r] = MASK != 0 ? attn_mask_byte(mask, Q.p[0], q, my_k, L, S) : uint8_t(1);
        add[qh][r] = MASK == 2 ? attn_mask_add(madd, q, my_k, L, S) : 0.f;
      }
    // chunk 0 of the operands not resident, in flight during the staging
#pragma unroll
    for (int i = NRES; i < (DO_K ? 2 : 1); ++i)
#pragma unroll
      for (int o = 0; o <= K; ++o)
        if constexpr (Sh::ring) ring[i][0][o] = load_row(i == 0 ? Kp : Vp, o, 0);
    __syncthreads();   // the previous block's products are done with the tiles
    attn_half_stage<T, K, D, KB, LD>(Qs, Q, head * L, qb0, L);
    attn_half_stage<T, K, D, KB, LD>(Gs, G, head * L, qb0, L);
    for (int idx = threadIdx.x; idx < (K + 1) * KB; idx += kAttnWaves * kWave) {
      const int o = idx / KB, i = idx % KB, q = qb0 + i;
      const int64_t at = head * L + min(q, L - 1);
      const float l = order_ptr<K>(LSE, o)[at], dl = order_ptr<K>(DELTA, o)[at];
      Ls[o][i] = q < L ? l : 0.f;
      Ds[o][i] = q < L ? dl : 0.f;
    }
    __syncthreads();

    // ---- S_k = sum_{a+b=k} Q_a K_b^T and dP_k = sum_{a+b=k} G_a V_b^T (queries x keys) ----
    // (one contraction after the other: their operands are not live together)
    floatx4 sc[2][K + 1], dp[DO_K ? 2 : 1][K + 1];
    auto contract = [&](floatx4 (&acc)[2][K + 1], const CPtrs<T>& X, int which, const T (&tile)[K + 1][KB][LD]) {
#pragma unroll
      for (int qh = 0; qh < 2; ++qh)
#pragma unroll
        for (int o = 0; o <= K; ++o) acc[qh][o] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int dc = 0; dc < DC; ++dc) {
        // resident rows, or the ring: chunk dc + 1 is loaded while chunk dc's products run
        u32x4 xb[K + 1];
        if (Sh::ring && which >= NRES && dc + 1 < DC) {
#pragma unroll
          for (int o = 0; o <= K; ++o) ring[which][(dc + 1) & 1][o] = load_row(X, o, dc + 1);
        }
#pragma unroll
        for (int o = 0; o <= K; ++o)
          xb[o] = which < NRES ? rows[which < NRES ? which : 0][o][dc]
                               : (Sh::ring ? ring[which][dc & 1][o] : load_row(X, o, dc));
        const bool din = 32 * dc + 8 * g < D;
        const int col = din ? 32 * dc + 8 * g : 0;
        const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int qh = 0; qh < 2; ++qh) {
          u32x4 ta_[K + 1];
#pragma unroll
          for (int o = 0; o <= K; ++o) {
            const u32x4 t = *reinterpret_cast<const u32x4*>(&tile[o][16 * qh + c][col]);
            ta_[o] = din ? t : z;
          }
#pragma unroll
          for (int k = 0; k <= K; ++k)
#pragma unroll
            for (int a = 0; a <= k; ++a) acc[qh][k] = MM::mma(ta_[a], xb[k - a], acc[qh][k]);
        }
      }
    };
    contract(sc, Kp, 0, Qs);
    if constexpr (DO_K) contract(dp, Vp, 1, Gs);

    // ---- P and dS series as B operands (slots 4 qh + r: query 16 qh + 4 g + r) ----
    u32x4 pb[K + 1], pl[NLO], dsb[K + 1], dsl[NLO];
#pragma unroll
    for (int qh = 0; qh < 2; ++qh) {
      float wp[K + 1][4], wd[K + 1][4];
      floatx4 l4[K + 1], d4[K + 1];
#pragma unroll
      for (int o = 0; o <= K; ++o) {
        l4[o] = *reinterpret_cast<const floatx4*>(&Ls[o][16 * qh + 4 * g]);
        if constexpr (DO_K) d4[o] = *reinterpret_cast<const floatx4*>(&Ds[o][16 * qh + 4 * g]);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int q = qb0 + 16 * qh + 4 * g + r;
        bool ok = k_ok && q < L;
        if (causal) ok = ok && my_k <= q;
        if constexpr (MASK != 0) ok = ok && mbyte[qh][r] != 0;
        float lse[K + 1], p[K + 1];
#pragma unroll
        for (int o = 0; o <= K; ++o) lse[o] = l4[o][r];
        attn_prob_series<float, K>(sc[qh], r, lse, ok, scale, add[qh][r], p);
#pragma unroll
        for (int o = 0; o <= K; ++o) wp[o][r] = p[o];
        if constexpr (DO_K) {
          float delta[K + 1], ds[K + 1];
#pragma unroll
          for (int o = 0; o <= K; ++o) delta[o] = d4[o][r];
          attn_ds_series<float, K>(p, dp[qh], r, delta, ds);
#pragma unroll
          for (int o = 0; o <= K; ++o) wd[o][r] = ds[o];
        }
      }
      if constexpr (DO_V) attn_half_pack<T, K, SPLIT, NLO>(wp, qh, pb, pl);
      if constexpr (DO_K) attn_half_pack<T, K, SPLIT, NLO>(wd, qh, dsb, dsl);
    }

    // ---- dV^T_k += sum_{a+b=k} G_b^T P_a and dK^T_k += sum_{a+b=k} Q_b^T dS_a, 32 queries per MFMA ----
#pragma unroll
    for (int db = 0; db < DBS; ++db) {
      const int col = d0 + 16 * db + 4 * ta;
      if constexpr (DO_V) {
        u32x4 gt[K + 1];
#pragma unroll
        for (int o = 0; o <= K; ++o) gt[o] = lds_read_tr16x2(&Gs[o][4 * g + tj][col], &Gs[o][16 + 4 * g + tj][col]);
        attn_half_series_mma<T, K, SPLIT, NLO>(acc_v[db], gt, pb, pl);
      }
      if constexpr (DO_K) {
        u32x4 qt[K + 1];
#pragma unroll
        for (int o = 0; o <= K; ++o) qt[o] = lds_read_tr16x2(&Qs[o][4 * g + tj][col], &Qs[o][16 + 4 * g + tj][col]);
        attn_half_series_mma<T, K, SPLIT, NLO>(acc_k[db], qt, dsb, dsl);
      }
    }
  }

  if (!k_ok) return;
  const int64_t row = (head * S + my_k) * D;
  if constexpr (DO_V) attn_half_store<T, K, DBS>(acc_v, DV, row, d0, g, 1.f);
  if constexpr (DO_K) attn_half_store<T, K, DBS>(acc_k, DK, row, d0, g, scale);
}

// Pipelined dK/dV kernel (WHAT as the staged kernel's): the Q and G tiles of query
// block j+1 (and its lse and Delta series) move while block j's products run. A
// tile read to the end of a block takes two buffers, one read by the score
// products only takes one, refilled once every wave is past it:
//   dV (WHAT 1): Q for S (one buffer), G for dV (two);
//   dK (WHAT 2): Q for S and dK (two), G for dP (one);
//   both (WHAT 3): two each.
// The lse and Delta series of block j+1 are loaded at the top of block j (before
// that block's DMA, so that waiting for them does not wait for it) and written to
// LDS once every wave is done with block j's.
template <int K, int D, int WHAT>
struct AttnHalfBwdKvPipe {
  static constexpr int NQ = (WHAT & 2) ? 2 : 1;
  static constexpr int NG = (WHAT & 1) ? 2 : 1;
  static constexpr size_t LDS = (NQ + NG) * AttnHalfBwdPipe<K, D>::tile + 2ull * (K + 1) * 32 * 4;
  static constexpr bool fits = LDS <= 160 * 1024 && D >= 32 && K >= 1;
};

template <typename T, int K, int D, int WHAT, int MASK>
__global__ __launch_bounds__(kAttnWaves * kWave) void taylor_attention_bwd_kv_half_pipe_kernel(
    CPtrs<T> Q, CPtrs<T> Kp, CPtrs<T> Vp, CPtrs<T> G, CPtrs<float> LSE, CPtrs<float> DELTA, MPtrs<T> DK,
    MPtrs<T> DV, int L, int S, const uint8_t* __restrict__ mask_all, AttnMaskMap mmap,
    const float* __restrict__ madd_all, const int32_t* __restrict__ ranges_all, int causal, float scale) {
  using Sh = AttnHalfBwdShape<K, D>;
  using BP = AttnHalfBwdPipe<K, D>;
  using KP = AttnHalfBwdKvPipe<K, D, WHAT>;
  using MM = HalfMfma<T>;
  constexpr int KB = BP::KB, DC = Sh::DC, DB = Sh::DB, OPT = BP::OPT;
  constexpr bool SPLIT = Sh::split;
  constexpr int NLO = SPLIT ? K + 1 : 1;
  constexpr bool DO_V = (WHAT & 1) != 0, DO_K = (WHAT & 2) != 0;
  constexpr int NQ = KP::NQ, NG = KP::NG;
  static_assert(KP::fits, "Q/G tiles exceed LDS");
  using Tile = T[K + 1][KB][D];
  __shared__ __attribute__((aligned(16))) Tile Qt[NQ];
  __shared__ __attribute__((aligned(16))) Tile Gt[NG];
  __shared__ __attribute__((aligned(16))) float Ls[K + 1][KB];
  __shared__ __attribute__((aligned(16))) float Ds[K + 1][KB];

  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int c = lane % 16;
  const int g = lane / 16;
  const int64_t bh = gridDim.x / static_cast<int64_t>((S + 63) / 64);
  int64_t head;
  int slice, kv_block;
  attn_bwd_kv_item(blockIdx.x, bh, 1, head, slice, kv_block);
  const int64_t mask_index = attn_mask_index(mmap, head);
  const uint8_t* mask = MASK != 0 ? mask_all + mask_index * L * S : nullptr;
  const float* madd = MASK == 2 ? madd_all + mask_index * L * S : nullptr;
  const int32_t* ranges = ranges_all != nullptr ? ranges_all + mask_index * attn_ranges_count(L, S) : nullptr;
  const int my_k = kv_block + wave * 16 + c;
  const bool k_ok = my_k < S;
  const int64_t krow = (head * S + (k_ok ? my_k : S - 1)) * D;
  auto load_row = [&](const CPtrs<T>& X, int o, int dc) -> u32x4 {
    const bool din = 32 * dc + 8 * g < D;
    return attn_half_load8<T>(X.p[o] + krow + (din ? 32 * dc + 8 * g : 0), din);
  };
  // K, then V, resident when they fit (the DMA bookkeeping takes about 32 registers more than the
  // staged kernel's staging); the others go through a two-slot chunk ring
  constexpr int NOPS = DO_K ? 2 : 1, OUTS = (DO_K ? 1 : 0) + (DO_V ? 1 : 0), EXTRA = DO_K ? 32 : 0;
  constexpr int NR0 = Sh::resident(NOPS, OUTS, DB, OUTS, MASK != 0, EXTRA);
  // K always resident: loading both K and V chunk by chunk measured 33% slower for the dK pass at
  // degree 4, head dim 128, where the resident K costs a few registers of scratch spill instead
  // (4 to 7, the compiler's resource remarks)
  constexpr int NR = NR0 > 0 ? NR0 : 1;
  constexpr bool RING = NR < NOPS && Sh::ring_fits(NOPS - NR, OUTS, DB, OUTS, MASK != 0, EXTRA + (NR - NR0) * (K + 1) * DC * 4);
  constexpr bool EARLY = NR == NOPS;   // the score products load nothing: the DMA may precede them
  u32x4 rows[NR > 0 ? NR : 1][K + 1][DC];
  u32x4 ring[2][2][K + 1];   // [operand][slot]: step s = 2-slot sequence over (half, chunk)
#pragma unroll
  for (int i = 0; i < NR; ++i)
#pragma unroll
    for (int o = 0; o <= K; ++o)
#pragma unroll
      for (int dc = 0; dc < DC; ++dc) rows[i][o][dc] = load_row(i == 0 ? Kp : Vp, o, dc);

  floatx4 acc_v[DO_V ? DB : 1][K + 1], acc_k[DO_K ? DB : 1][K + 1];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int o = 0; o <= K; ++o) {
      if constexpr (DO_V) acc_v[db][o] = floatx4{0.f, 0.f, 0.f, 0.f};
      if constexpr (DO_K) acc_k[db][o] = floatx4{0.f, 0.f, 0.f, 0.f};
    }

  int lo, hi;
  attn_query_range(L, kv_block, causal, ranges, lo, hi);
  lo = lo / KB * KB;
  // a workgroup whose keys no query admits keeps one fully masked block (q < hi fails)
  if (hi <= lo) lo = hi = 0;
  const int nblocks = max(1, (hi - lo + KB - 1) / KB);
  const int last_qb0 = lo + (nblocks - 1) * KB;
  const int tj = c / 4, ta = c % 4;

  // the lse and Delta series of query rows qb0 .. qb0 + 31 (zero past L): NV values per thread
  constexpr int NV = ((K + 1) * KB + kAttnWaves * kWave - 1) / (kAttnWaves * kWave);
  float lv[NV], dv_[NV];
  auto load_rows = [&](int qb0) {
#pragma unroll
    for (int t = 0; t < NV; ++t) {
      const int idx = min(static_cast<int>(threadIdx.x) + kAttnWaves * kWave * t, (K + 1) * KB - 1);
      const int o = idx / KB, q = qb0 + idx % KB;
      const int64_t at = head * L + min(q, L - 1);
      lv[t] = order_ptr<K>(LSE, o)[at];
      if constexpr (DO_K) dv_[t] = order_ptr<K>(DELTA, o)[at];
    }
  };
  auto store_rows = [&](int qb0) {
#pragma unroll
    for (int t = 0; t < NV; ++t) {
      const int idx = static_cast<int>(threadIdx.x) + kAttnWaves * kWave * t;
      if (((K + 1) * KB) % (kAttnWaves * kWave) == 0 || idx < (K + 1) * KB) {
        const int o = idx / KB, i = idx % KB;
        const bool in = qb0 + i < L;
        Ls[o][i] = in ? lv[t] : 0.f;
        if constexpr (DO_K) Ds[o][i] = in ? dv_[t] : 0.f;
      }
    }
  };

  // block 0: its lse / Delta rows, then its tiles
  load_rows(lo);
  store_rows(lo);
#pragma unroll
  for (int i = 0; i < OPT; ++i) {
    attn_half_dma_tile<T, K, D>(Qt[0], Q, head, L, lo, lane, wave, i);
    attn_half_dma_tile<T, K, D>(Gt[0], G, head, L, lo, lane, wave, i);
  }

  for (int j = 0; j < nblocks; ++j) {
    const int qb0 = lo + j * KB;
    const int next_qb0 = min(qb0 + KB, last_qb0);   // the last block re-loads itself: no branch
    Tile& qcur = Qt[NQ == 2 ? (j & 1) : 0];
    Tile& gcur = Gt[NG == 2 ? (j & 1) : 0];
    uint8_t mbyte[2][4];
    float add[2][4];
#pragma unroll
    for (int qh = 0; qh < 2; ++qh)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int q = qb0 + 16 * qh + 4 * g + r;
        mbyte[qh][r] = MASK != 0 ? attn_mask_byte(mask, Q.p[0], q, my_k, L, S) : uint8_t(1);
        add[qh][r] = MASK == 2 ? attn_mask_add(madd, q, my_k, L, S) : 0.f;
      }
    load_rows(next_qb0);             // block j+1's lse / Delta, ahead of this block's DMA
    __builtin_amdgcn_s_waitcnt(0);   // this wave's DMAs of block j have landed (and the loads above)
    __syncthreads();                 // ... and every wave's; block j-1 is done with the other buffers
    // tiles read to the end of the block: block j+1's into their other buffer, here when the score
    // products load nothing (every row operand resident), else after them with the others (their
    // loads would wait for the DMA)
    auto dma_double = [&]() {
#pragma unroll
      for (int i = 0; i < OPT; ++i) {
        if constexpr (NQ == 2) attn_half_dma_tile<T, K, D>(Qt[(j + 1) & 1], Q, head, L, next_qb0, lane, wave, i);
        if constexpr (NG == 2) attn_half_dma_tile<T, K, D>(Gt[(j + 1) & 1], G, head, L, next_qb0, lane, wave, i);
      }
    };
    if constexpr (EARLY) dma_double();
    // chunk 0 of the operands not resident (no DMA in flight ahead of them)
#pragma unroll
    for (int i = NR; i < NOPS; ++i)
#pragma unroll
      for (int o = 0; o <= K; ++o)
        if constexpr (RING) ring[i][0][o] = load_row(i == 0 ? Kp : Vp, o, 0);

    // ---- per 16-query half: S = Q K^T, dP = G V^T (queries x keys), then the P and dS series ----
    u32x4 pb[K + 1], pl[NLO], dsb[K + 1], dsl[NLO];
#pragma unroll
    for (int qh = 0; qh < 2; ++qh) {
      floatx4 sc[K + 1], dp[DO_K ? K + 1 : 1];
#pragma unroll
      for (int o = 0; o <= K; ++o) {
        sc[o] = floatx4{0.f, 0.f, 0.f, 0.f};
        if constexpr (DO_K) dp[o] = floatx4{0.f, 0.f, 0.f, 0.f};
      }
      // operand `which` of (half qh, chunk dc): resident, or ring step qh DC + dc, whose successor's
      // chunk is loaded now
      auto operand = [&](int which, int dc, u32x4 (&x)[K + 1]) {
        const int st = qh * DC + dc;
        if (RING && which >= NR && st + 1 < 2 * DC) {
#pragma unroll
          for (int o = 0; o <= K; ++o) ring[which][(st + 1) & 1][o] = load_row(which == 0 ? Kp : Vp, o, (dc + 1) % DC);
        }
#pragma unroll
        for (int o = 0; o <= K; ++o)
          x[o] = which < NR ? rows[which < NR ? which : 0][o][dc]
                            : (RING ? ring[which][st & 1][o] : load_row(which == 0 ? Kp : Vp, o, dc));
      };
#pragma unroll
      for (int dc = 0; dc < DC; ++dc) {
        const bool din = 32 * dc + 8 * g < D;
        u32x4 qa[K + 1], kb[K + 1];
        operand(0, dc, kb);
#pragma unroll
        for (int o = 0; o <= K; ++o) qa[o] = attn_half_tile_row<T, K, D>(qcur, o, 16 * qh + c, 4 * dc + g, din);
#pragma unroll
        for (int k = 0; k <= K; ++k)
#pragma unroll
          for (int a = 0; a <= k; ++a) sc[k] = MM::mma(qa[a], kb[k - a], sc[k]);
      }
      if constexpr (DO_K) {
#pragma unroll
        for (int dc = 0; dc < DC; ++dc) {
          const bool din = 32 * dc + 8 * g < D;
          u32x4 ga[K + 1], vb[K + 1];
          operand(1, dc, vb);
#pragma unroll
          for (int o = 0; o <= K; ++o) ga[o] = attn_half_tile_row<T, K, D>(gcur, o, 16 * qh + c, 4 * dc + g, din);
#pragma unroll
          for (int k = 0; k <= K; ++k)
#pragma unroll
            for (int a = 0; a <= k; ++a) dp[k] = MM::mma(ga[a], vb[k - a], dp[k]);
        }
      }
      float wp[K + 1][4], wd[K + 1][4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int q = qb0 + 16 * qh + 4 * g + r;
        bool ok = k_ok && q < hi;
        if (causal) ok = ok && my_k <= q;
        if constexpr (MASK != 0) ok = ok && mbyte[qh][r] != 0;
        // (read per element: the row series of all four elements at once cost registers that spill)
        float lse[K + 1], p[K + 1];
#pragma unroll
        for (int o = 0; o <= K; ++o) lse[o] = Ls[o][16 * qh + 4 * g + r];
        attn_prob_series<float, K>(sc, r, lse, ok, scale, add[qh][r], p);
#pragma unroll
        for (int o = 0; o <= K; ++o) wp[o][r] = p[o];
        if constexpr (DO_K) {
          float delta[K + 1], ds[K + 1];
#pragma unroll
          for (int o = 0; o <= K; ++o) delta[o] = Ds[o][16 * qh + 4 * g + r];
          attn_ds_series<float, K>(p, dp, r, delta, ds);
#pragma unroll
          for (int o = 0; o <= K; ++o) wd[o][r] = ds[o];
        }
      }
      if constexpr (DO_V) attn_half_pack<T, K, SPLIT, NLO>(wp, qh, pb, pl);
      if constexpr (DO_K) attn_half_pack<T, K, SPLIT, NLO>(wd, qh, dsb, dsl);
    }
    __syncthreads();   // every wave is done with the single-buffered tile and this block's lse / Delta
    store_rows(next_qb0);
    if constexpr (!EARLY) dma_double();
#pragma unroll
    for (int i = 0; i < OPT; ++i) {
      if constexpr (NQ == 1) attn_half_dma_tile<T, K, D>(Qt[0], Q, head, L, next_qb0, lane, wave, i);
      if constexpr (NG == 1) attn_half_dma_tile<T, K, D>(Gt[0], G, head, L, next_qb0, lane, wave, i);
    }

    // ---- dV^T_k += sum_{a+b=k} G_b^T P_a, dK^T_k += sum_{a+b=k} Q_b^T dS_a ----
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      if constexpr (DO_V) {
        u32x4 gt[K + 1];
#pragma unroll
        for (int o = 0; o <= K; ++o) gt[o] = attn_half_tile_tr<T, K, D>(gcur, o, db, g, tj, ta);
        attn_half_series_mma<T, K, SPLIT, NLO>(acc_v[db], gt, pb, pl);
      }
      if constexpr (DO_K) {
        u32x4 qt[K + 1];
#pragma unroll
        for (int o = 0; o <= K; ++o) qt[o] = attn_half_tile_tr<T, K, D>(qcur, o, db, g, tj, ta);
        attn_half_series_mma<T, K, SPLIT, NLO>(acc_k[db], qt, dsb, dsl);
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0);   // the last block's (redundant) DMAs have landed before the workgroup ends

  if (!k_ok) return;
  const int64_t row = (head * S + my_k) * D;
  if constexpr (DO_V) attn_half_store<T, K, DB>(acc_v, DV, row, 0, g, 1.f);
  if constexpr (DO_K) attn_half_store<T, K, DB>(acc_k, DK, row, 0, g, scale);
}

// ---------------------------------------------------------------------------
// Stored-tile dK / dV kernel: the dQ kernel has written the P and dS series of
// every visited pair, so each output takes one series product per block (five
// products per pair in all instead of eight, and no exponential series here).
// A workgroup owns KEYS keys (16 per wave: 128 where the tiles fit LDS, so that
// each Q / G tile read serves twice the keys and two waves share each SIMD, else
// 64). Per 32-query block the X tile (G for dV, Q for dK) and the block's stored
// P (or dS) values of the workgroup's keys move by LDS DMA, double-buffered. The
// stored values are the B operand, read by transpose reads (lane c receives key
// c's queries 4 g .. 4 g + 3 and 16 + 4 g ..), and masked by admissibility: a
// pair the dQ kernel did not visit (a block outside its mask range) holds no
// written value.
template <int K, int D, int WHAT, int KEYS>
struct AttnHalfBwdMat {
  static constexpr int KB = 32;
  static constexpr int WAVES = KEYS / 16;
  static constexpr int NOUT = ((WHAT & 1) ? 1 : 0) + ((WHAT & 2) ? 1 : 0);
  static constexpr size_t xtile = static_cast<size_t>(K + 1) * KB * D * 2;
  static constexpr size_t stile = static_cast<size_t>(K + 1) * KB * KEYS * 2;
  static constexpr size_t LDS = 2 * NOUT * (xtile + stile);
  // (128 keys: two waves per SIMD, so at most 256 registers per lane: the output accumulators
  // of one output, up to 160)
  static constexpr bool fits = LDS <= 160 * 1024 && D >= 32 && K >= 1 && K <= 4 &&
                               (KEYS == 64 || NOUT * (K + 1) * (D / 16) * 4 <= 160);
};
template <int K, int D, int WHAT>
constexpr int attn_half_mat_keys() {
  return AttnHalfBwdMat<K, D, WHAT, 128>::fits ? 128 : 64;
}

// DMA operation i (0 <= i < (K+1) ceil(segments / WAVES)) of this wave's share of rows
// first .. first + 31 of a head's [rows, D] series into a tile [K+1][32][D] (as
// attn_half_dma_tile, for a workgroup of WAVES waves).
template <typename T, int K, int D, int WAVES>
__device__ __forceinline__ void attn_half_dma_tile_w(T (&tile)[K + 1][32][D], const CPtrs<T>& src, int64_t head,
                                                     int rows, int first, int lane, int wave, int i) {
  using P = AttnHalfPipe<K, D>;
  constexpr int CH = P::CH, RPS = P::RPS, SEGS = P::SEGS, IT = (SEGS + WAVES - 1) / WAVES;
  const int o = i / IT, it = i % IT;
  const int seg = it * WAVES + wave;
  if (SEGS % WAVES != 0 && seg >= SEGS) return;
  const int row = seg * RPS + lane / CH;
  const int lch = (lane % CH) ^ P::fs(row);
  const BufferRsrc rsrc = buffer_rsrc(src.p[o] + head * rows * D, rows * D * static_cast<int>(sizeof(T)));
  lds_dma16(&tile[o][seg * RPS][0], rsrc, ((first + row) * D + lch * 8) * static_cast<int>(sizeof(T)));
}

// This wave's DMA of one order of a stored tile: its 512 / KEYS query rows (of first .. first + 31)
// of the KEYS keys from key0 (32-key blocks of a head's [srow / 32][rows][32] 16-bit series) into
// LDS [32][KEYS] (row r: positions of keys key0 .. key0 + KEYS - 1 of query first + r). Rows past
// `rows` read the next key block's first rows, or zeros past the head's series: their pairs are
// inadmissible and masked.
// 16-byte chunk swizzle of a stored tile [32][KEYS] in LDS (physical chunk = logical ^ f(row)):
// rows of 256 (128) bytes all start on bank 0 (0 or 32), so the transpose reads of rows
// 4 g .. 4 g + 3 at four chunks would fall on 8 banks; with f the 64 pieces of a read spread
// evenly over the 16 chunks, four to a chunk (SQ_LDS_BANK_CONFLICT had been 28% of the cycles).
template <int KEYS>
__device__ __forceinline__ int attn_stored_swz(int row) {
  return KEYS == 128 ? 4 * (row & 3) : 4 * ((row >> 1) & 1);
}

template <typename T, int K, int KEYS>
__device__ __forceinline__ void attn_half_dma_stored(T (&tile)[K + 1][32][KEYS], const CPtrs<T>& src, int64_t head,
                                                     int rows, int64_t srow, int first, int key0, int lane, int wave,
                                                     int o) {
  constexpr int CPR = KEYS / 8, RPS = 64 / CPR;   // 16-byte chunks per row, rows per 1 KB segment
  const int row = RPS * wave + lane / CPR;
  const int ch = (lane % CPR) ^ attn_stored_swz<KEYS>(row);   // the logical chunk this lane's slot holds
  const int64_t nkb = srow / 32;
  const BufferRsrc rsrc = buffer_rsrc(src.p[o] + head * nkb * rows * 32, static_cast<int>(nkb * rows * 32 * 2));
  const int64_t at = ((key0 / 32 + ch / 4) * static_cast<int64_t>(rows) + first + row) * 32 + 8 * (ch % 4);
  lds_dma16(&tile[o][RPS * wave][0], rsrc, static_cast<int>(at * 2));
}

// Query range [lo, hi) of keys kv_block .. kv_block + KEYS - 1: the union over their 64-key
// range blocks (an empty one, hi <= lo, adds nothing).
template <int KEYS>
__device__ __forceinline__ void attn_query_range_keys(int L, int S, int kv_block, int causal, const int32_t* ranges,
                                                      int& lo, int& hi) {
  attn_query_range(L, kv_block, causal, ranges, lo, hi);
#pragma unroll
  for (int b = 64; b < KEYS; b += 64) {
    if (kv_block + b < S) {
      int l2, h2;
      attn_query_range(L, kv_block + b, causal, ranges, l2, h2);
      if (hi <= lo) {
        lo = l2;
        hi = h2;
      } else if (l2 < h2) {
        lo = min(lo, l2);
        hi = max(hi, h2);
      }
    }
  }
}

template <typename T, int K, int D, int WHAT, int KEYS, bool MASKED>
__global__ __launch_bounds__(KEYS * 4) void taylor_attention_bwd_kv_half_mat_kernel(
    CPtrs<T> Q, CPtrs<T> G, CPtrs<T> PT, CPtrs<T> DST, MPtrs<T> DK, MPtrs<T> DV, int64_t srow, int L, int S,
    const uint8_t* __restrict__ mask_all, AttnMaskMap mmap, const int32_t* __restrict__ ranges_all, int causal,
    float scale) {
  using MT = AttnHalfBwdMat<K, D, WHAT, KEYS>;
  constexpr int KB = MT::KB, DB = D / 16, NOUT = MT::NOUT, WAVES = MT::WAVES;
  constexpr int OPT = (K + 1) * ((AttnHalfPipe<K, D>::SEGS + WAVES - 1) / WAVES);
  constexpr bool DO_V = (WHAT & 1) != 0, DO_K = (WHAT & 2) != 0;
  constexpr int SV = 0, SK = DO_V ? 1 : 0;   // slots of the dV and dK inputs
  static_assert(MT::fits, "tiles exceed LDS");
  using XTile = T[K + 1][KB][D];
  using STile = T[K + 1][KB][KEYS];
  __shared__ __attribute__((aligned(16))) XTile Xt[2][NOUT];
  __shared__ __attribute__((aligned(16))) STile St[2][NOUT];

  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int c = lane % 16;
  const int g = lane / 16;
  const int64_t bh = gridDim.x / static_cast<int64_t>((S + KEYS - 1) / KEYS);
  const int64_t head = blockIdx.x % bh;   // heads fastest: a head's key blocks share an XCD
  const int kv_block = static_cast<int>(blockIdx.x / bh) * KEYS;
  const int64_t mask_index = attn_mask_index(mmap, head);
  const uint8_t* mask = MASKED ? mask_all + mask_index * L * S : nullptr;
  const int32_t* ranges = ranges_all != nullptr ? ranges_all + mask_index * attn_ranges_count(L, S) : nullptr;
  const int my_k = kv_block + wave * 16 + c;
  const bool k_ok = my_k < S;

  floatx4 acc_v[DO_V ? DB : 1][K + 1], acc_k[DO_K ? DB : 1][K + 1];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int o = 0; o <= K; ++o) {
      if constexpr (DO_V) acc_v[db][o] = floatx4{0.f, 0.f, 0.f, 0.f};
      if constexpr (DO_K) acc_k[db][o] = floatx4{0.f, 0.f, 0.f, 0.f};
    }

  int lo, hi;
  attn_query_range_keys<KEYS>(L, S, kv_block, causal, ranges, lo, hi);
  lo = lo / KB * KB;
  if (hi <= lo) lo = hi = 0;   // one fully masked block (q < hi fails): the pipeline always has a first
  const int nblocks = max(1, (hi - lo + KB - 1) / KB);
  const int last_qb0 = lo + (nblocks - 1) * KB;
  const int tj = c / 4, ta = c % 4;

  // (the stored tiles first: with the X-tile DMAs, which some waves skip at head dim 32, ahead of
  // them the compiler placed their buffer resources in vector registers, which the instruction
  // does not take)
  auto dma = [&](int buf, int qb0) {
#pragma unroll
    for (int o = 0; o <= K; ++o) {
      if constexpr (DO_V)
        attn_half_dma_stored<T, K, KEYS>(St[buf][SV], PT, head, L, srow, qb0, kv_block, lane, wave, o);
      if constexpr (DO_K)
        attn_half_dma_stored<T, K, KEYS>(St[buf][SK], DST, head, L, srow, qb0, kv_block, lane, wave, o);
    }
#pragma unroll
    for (int i = 0; i < OPT; ++i) {
      if constexpr (DO_V) attn_half_dma_tile_w<T, K, D, WAVES>(Xt[buf][SV], G, head, L, qb0, lane, wave, i);
      if constexpr (DO_K) attn_half_dma_tile_w<T, K, D, WAVES>(Xt[buf][SK], Q, head, L, qb0, lane, wave, i);
    }
  };
  // a block's mask bytes are read one block ahead, before that block's DMA (loads complete in
  // issue order: read at the top of its own block, they would hold it for a memory round trip)
  uint8_t mnext[MASKED ? 8 : 1];
  auto fetch_mask = [&](int qb0) __attribute__((always_inline)) {
    if constexpr (MASKED) {
#pragma unroll
      for (int s = 0; s < 8; ++s)
        mnext[s] = attn_mask_byte(mask, Q.p[0], qb0 + 16 * (s / 4) + 4 * g + s % 4, my_k, L, S);
    }
  };
  dma(0, lo);
  fetch_mask(lo);

  for (int j = 0; j < nblocks; ++j) {
    const int qb0 = lo + j * KB;
    const int cur = j & 1;
    __builtin_amdgcn_s_waitcnt(0);   // this wave's DMAs of block j have landed (and its mask bytes)
    __syncthreads();                 // ... and every wave's; block j-1 is done with the other buffers
    uint8_t mbyte[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) mbyte[s] = MASKED ? mnext[s] : uint8_t(1);
    fetch_mask(min(qb0 + KB, last_qb0));   // the next block's, ahead of its DMA
    dma(cur ^ 1, min(qb0 + KB, last_qb0));   // block j+1 (the last block re-loads itself: no branch)

    // admissibility of the eight pairs behind the lane's operand slots (slot 4 qh + r: query
    // qb0 + 16 qh + 4 g + r, key my_k), as 16-bit lane masks
    u32x4 keep;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      uint32_t m = 0;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int s = 2 * w + h;
        const int q = qb0 + 16 * (s / 4) + 4 * g + s % 4;
        bool ok = k_ok && q < hi;
        if (causal) ok = ok && my_k <= q;
        if constexpr (MASKED) ok = ok && mbyte[s] != 0;
        m |= ok ? (0xffffu << (16 * h)) : 0u;
      }
      keep[w] = m;
    }
    auto products = [&](floatx4 (&acc)[DB][K + 1], const XTile& xt, const STile& st) {
      u32x4 b[K + 1], none[1];
      // the wave's keys kv_block + 16 wave + c: block wave / 2, key 16 (wave % 2) + c at position
      // 8 (c / 4) + 4 ((wave % 2) ^ q2) + c % 4, q2 = bit 2 of the query row (rows r and r + 16 share
      // it); this lane addresses the four positions of lanes 4 ta ..
      const int r0 = 4 * g + tj, r1 = 16 + 4 * g + tj;
      const int lch = 4 * (wave / 2) + ta, off = 4 * ((wave % 2) ^ ((r0 >> 2) & 1));   // logical chunk, offset
      const int c0 = 8 * (lch ^ attn_stored_swz<KEYS>(r0)) + off, c1 = 8 * (lch ^ attn_stored_swz<KEYS>(r1)) + off;
#pragma unroll
      for (int o = 0; o <= K; ++o) b[o] = lds_read_tr16x2(&st[o][r0][c0], &st[o][r1][c1]) & keep;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        u32x4 x[K + 1];
#pragma unroll
        for (int o = 0; o <= K; ++o) x[o] = attn_half_tile_tr<T, K, D>(xt, o, db, g, tj, ta);
        attn_half_series_mma<T, K, false, 1>(acc[db], x, b, none);
      }
    };
    if constexpr (DO_V) products(acc_v, Xt[cur][SV], St[cur][SV]);
    if constexpr (DO_K) products(acc_k, Xt[cur][SK], St[cur][SK]);
  }
  __builtin_amdgcn_s_waitcnt(0);   // the last block's (redundant) DMAs have landed before the workgroup ends

  if (!k_ok) return;
  const int64_t row = (head * S + my_k) * D;
  if constexpr (DO_V) attn_half_store<T, K, DB>(acc_v, DV, row, 0, g, 1.f);
  if constexpr (DO_K) attn_half_store<T, K, DB>(acc_k, DK, row, 0, g, scale);
}

template <typename T, int K, int D>
static int launch_attention_bwd_half_kd(const AttnBwdArgs& a) {
  using Sh = AttnHalfBwdShape<K, D>;
  static_assert(Sh::fits, "every 16-bit backward shape fits LDS");
  CPtrs<T> q{}, k{}, v{}, o{}, g{};
  CPtrs<float> lse{}, delta_in{};
  MPtrs<float> delta{};
  MPtrs<T> dq{}, dk{}, dv{};
  const int64_t rows = a.bh * a.lq;
  for (int i = 0; i <= K; ++i) {
    q.p[i] = static_cast<const T*>(a.q[i]);
    k.p[i] = static_cast<const T*>(a.k[i]);
    v.p[i] = static_cast<const T*>(a.v[i]);
    o.p[i] = static_cast<const T*>(a.out[i]);
    g.p[i] = static_cast<const T*>(a.grad[i]);
    lse.p[i] = static_cast<const float*>(a.lse[i]);
    delta.p[i] = static_cast<float*>(a.workspace) + i * rows;
    delta_in.p[i] = delta.p[i];
    if (a.dq != nullptr) dq.p[i] = static_cast<T*>(a.dq[i]);
    if (a.dk != nullptr) dk.p[i] = static_cast<T*>(a.dk[i]);
    if (a.dv != nullptr) dv.p[i] = static_cast<T*>(a.dv[i]);
  }
  const int L = static_cast<int>(a.lq), S = static_cast<int>(a.lk);
  const float scale = static_cast<float>(a.scale);
  const int causal = a.causal ? 1 : 0;
  const float* madd = static_cast<const float*>(a.mask_add);
  const int mask_kind = madd != nullptr ? 2 : a.mask != nullptr ? 1 : 0;
  const dim3 block(kAttnWaves * kWave);
  // the DMA's buffer resources span a head's K / V rows and Q / G rows (plus one block) with 32-bit
  // offsets
  const bool q_pipe_ok = a.lk >= 1 && (a.lk + 32) * D * static_cast<int64_t>(sizeof(T)) < (int64_t{1} << 31);
  const bool kv_pipe_ok = a.lq >= 1 && (a.lq + 32) * D * static_cast<int64_t>(sizeof(T)) < (int64_t{1} << 31);
  // Stored tiles (degrees 1..4, the pipelined dQ kernel): the dQ kernel writes the P and dS series,
  // the dK / dV kernels read them (five products per pair instead of eight). Elsewhere the request
  // is a hint and the scores are recomputed.
  const int64_t srow = attention_bwd_half_row(a.lk);
  bool mat = false;
  MPtrs<T> pt{}, dst{};
  CPtrs<T> pt_in{}, dst_in{};
  if constexpr (K >= 1 && K <= 4 && AttnHalfBwdPipe<K, D>::fits_q && Sh::SL_Q == 1 &&
                AttnHalfBwdMat<K, D, 1, 64>::fits && AttnHalfBwdMat<K, D, 2, 64>::fits) {
    mat = a.materialize && rows > 0 && (a.dk != nullptr || a.dv != nullptr) && q_pipe_ok && kv_pipe_ok &&
          (a.lq + 32) * srow * 2 < (int64_t{1} << 31);
    if (mat) {
      const AttnBwdLayout lay = attention_bwd_half_layout(K, a.bh, a.lq, a.lk, true);
      for (int i = 0; i <= K; ++i) {
        pt.p[i] = reinterpret_cast<T*>(static_cast<char*>(a.workspace) + lay.tiles_offset + i * lay.tile_bytes);
        dst.p[i] = reinterpret_cast<T*>(static_cast<char*>(a.workspace) + lay.tiles_offset +
                                        (K + 1 + i) * lay.tile_bytes);
        pt_in.p[i] = pt.p[i];
        dst_in.p[i] = dst.p[i];
      }
    }
  }
  if (rows > 0 && (a.dq != nullptr || ((a.dk != nullptr || a.dv != nullptr) && a.lk > 0))) {
    attn_bwd_delta_kernel<T, K, D><<<dim3(static_cast<unsigned>((rows + 15) / 16)), dim3(256), 0, a.stream>>>(
        g, o, delta, rows);
    PT_LAUNCH_CHECK();
  }
  if ((a.dq != nullptr || mat) && rows > 0) {   // (with stored tiles and no dq the kernel still writes them)
    constexpr int SL = Sh::SL_Q;
    bool done = false;
    if constexpr (AttnHalfBwdPipe<K, D>::fits_q && SL == 1) {
      if (q_pipe_ok) {
        const dim3 grid(static_cast<unsigned>((a.lq + kAttnBM - 1) / kAttnBM * a.bh));
#define PT_ATTN_BWD_Q_HALF_PIPE(MASK, STORE)                                                                 \
  taylor_attention_bwd_q_half_pipe_kernel<T, K, D, MASK, STORE><<<grid, block, 0, a.stream>>>(               \
      q, k, v, g, lse, delta_in, dq, pt, dst, srow, L, S, a.mask, a.mask_map, madd, a.mask_ranges, causal,    \
      scale)
        if (mat) {
          if constexpr (K >= 1 && K <= 4) {
            if (mask_kind == 2) PT_ATTN_BWD_Q_HALF_PIPE(2, true);
            else if (mask_kind == 1) PT_ATTN_BWD_Q_HALF_PIPE(1, true);
            else PT_ATTN_BWD_Q_HALF_PIPE(0, true);
          }
        } else {
          if (mask_kind == 2) PT_ATTN_BWD_Q_HALF_PIPE(2, false);
          else if (mask_kind == 1) PT_ATTN_BWD_Q_HALF_PIPE(1, false);
          else PT_ATTN_BWD_Q_HALF_PIPE(0, false);
        }
#undef PT_ATTN_BWD_Q_HALF_PIPE
        PT_LAUNCH_CHECK();
        done = true;
      }
    }
    if (!done) {
      const dim3 grid(static_cast<unsigned>((a.lq + kAttnBM - 1) / kAttnBM * a.bh * SL));
#define PT_ATTN_BWD_Q_HALF(MASK)                                                                             \
  taylor_attention_bwd_q_half_kernel<T, K, D, SL, MASK><<<grid, block, 0, a.stream>>>(                       \
      q, k, v, g, lse, delta_in, dq, L, S, a.mask, a.mask_map, madd, a.mask_ranges, causal, scale)
      if (mask_kind == 2) PT_ATTN_BWD_Q_HALF(2);
      else if (mask_kind == 1) PT_ATTN_BWD_Q_HALF(1);
      else PT_ATTN_BWD_Q_HALF(0);
#undef PT_ATTN_BWD_Q_HALF
      PT_LAUNCH_CHECK();
    }
  }
  if (mat) {
    if constexpr (K >= 1 && K <= 4 && AttnHalfBwdMat<K, D, 1, 64>::fits && AttnHalfBwdMat<K, D, 2, 64>::fits) {
#define PT_ATTN_BWD_KV_HALF_MAT(WHAT)                                                                        \
  do {                                                                                                       \
    constexpr int KEYS = attn_half_mat_keys<K, D, WHAT>();                                                   \
    const dim3 grid(static_cast<unsigned>((a.lk + KEYS - 1) / KEYS * a.bh)), mblock(KEYS * 4);               \
    if (a.mask != nullptr)                                                                                   \
      taylor_attention_bwd_kv_half_mat_kernel<T, K, D, WHAT, KEYS, true><<<grid, mblock, 0, a.stream>>>(     \
          q, g, pt_in, dst_in, dk, dv, srow, L, S, a.mask, a.mask_map, a.mask_ranges, causal, scale);        \
    else                                                                                                     \
      taylor_attention_bwd_kv_half_mat_kernel<T, K, D, WHAT, KEYS, false><<<grid, mblock, 0, a.stream>>>(    \
          q, g, pt_in, dst_in, dk, dv, srow, L, S, a.mask, a.mask_map, a.mask_ranges, causal, scale);        \
    PT_LAUNCH_CHECK();                                                                                       \
  } while (0)
      bool fused = false;
      if constexpr (AttnHalfBwdMat<K, D, 3, 64>::fits) {
        if (a.dk != nullptr && a.dv != nullptr) {
          PT_ATTN_BWD_KV_HALF_MAT(3);
          fused = true;
        }
      }
      if (!fused) {
        if (a.dv != nullptr) PT_ATTN_BWD_KV_HALF_MAT(1);
        if (a.dk != nullptr) PT_ATTN_BWD_KV_HALF_MAT(2);
      }
#undef PT_ATTN_BWD_KV_HALF_MAT
    }
  } else if ((a.dk != nullptr || a.dv != nullptr) && a.lk > 0) {
    constexpr int SL = Sh::SL_KV;
    const dim3 grid(static_cast<unsigned>((a.lk + 63) / 64 * a.bh * SL));
    const bool pipe_ok = SL == 1 && kv_pipe_ok;   // the pipelined kernel (one slice)
#define PT_ATTN_BWD_KV_HALF_LAUNCH(KERNEL, ...)                                                              \
  do {                                                                                                       \
    if (mask_kind == 2)                                                                                      \
      KERNEL<__VA_ARGS__, 2><<<grid, block, 0, a.stream>>>(                                                  \
          q, k, v, g, lse, delta_in, dk, dv, L, S, a.mask, a.mask_map, madd, a.mask_ranges, causal, scale);  \
    else if (mask_kind == 1)                                                                                 \
      KERNEL<__VA_ARGS__, 1><<<grid, block, 0, a.stream>>>(                                                  \
          q, k, v, g, lse, delta_in, dk, dv, L, S, a.mask, a.mask_map, madd, a.mask_ranges, causal, scale);  \
    else                                                                                                     \
      KERNEL<__VA_ARGS__, 0><<<grid, block, 0, a.stream>>>(                                                  \
          q, k, v, g, lse, delta_in, dk, dv, L, S, a.mask, a.mask_map, madd, a.mask_ranges, causal, scale);  \
    PT_LAUNCH_CHECK();                                                                                       \
  } while (0)
#define PT_ATTN_BWD_KV_HALF(WHAT)                                                                           \
  do {                                                                                                       \
    bool piped = false;                                                                                      \
    if constexpr (SL == 1 && AttnHalfBwdKvPipe<K, D, WHAT>::fits && Sh::kv_pipe_regs(WHAT)) {               \
      if (pipe_ok) {                                                                                         \
        PT_ATTN_BWD_KV_HALF_LAUNCH(taylor_attention_bwd_kv_half_pipe_kernel, T, K, D, WHAT);                 \
        piped = true;                                                                                        \
      }                                                                                                      \
    }                                                                                                        \
    if (!piped) PT_ATTN_BWD_KV_HALF_LAUNCH(taylor_attention_bwd_kv_half_kernel, T, K, D, SL, WHAT);          \
  } while (0)
    // the fused pass writes both outputs: with one of them not wanted (NULL) that one's pass runs alone
    bool fused = false;
    if constexpr (Sh::kv_fused) {
      if (a.dk != nullptr && a.dv != nullptr) {
        PT_ATTN_BWD_KV_HALF(3);
        fused = true;
      }
    }
    if (!fused) {
      if (a.dv != nullptr) PT_ATTN_BWD_KV_HALF(1);
      if (a.dk != nullptr) PT_ATTN_BWD_KV_HALF(2);
    }
#undef PT_ATTN_BWD_KV_HALF
#undef PT_ATTN_BWD_KV_HALF_LAUNCH
  }
  return PT_OK;
}

template <typename T, int K>
static int launch_attention_bwd_half_k(const AttnBwdArgs& a) {
  switch (a.d) {
    case 16: return launch_attention_bwd_half_kd<T, K, 16>(a);
    case 32: return launch_attention_bwd_half_kd<T, K, 32>(a);
    case 64: return launch_attention_bwd_half_kd<T, K, 64>(a);
    case 128: return launch_attention_bwd_half_kd<T, K, 128>(a);
    default: break;
  }
  pt_host::set_error("Taylor attention backward: head dim must be 16, 32, 64 or 128");
  return PT_UNSUPPORTED;
}

template <typename T>
int launch_attention_bwd_half(const AttnBwdArgs& a) {
  switch (a.degree) {
    case 0: return launch_attention_bwd_half_k<T, 0>(a);
    case 1: return launch_attention_bwd_half_k<T, 1>(a);
    case 2: return launch_attention_bwd_half_k<T, 2>(a);
    case 3: return launch_attention_bwd_half_k<T, 3>(a);
    case 4: return launch_attention_bwd_half_k<T, 4>(a);
    case 5: return launch_attention_bwd_half_k<T, 5>(a);
    case 6: return launch_attention_bwd_half_k<T, 6>(a);
    case 7: return launch_attention_bwd_half_k<T, 7>(a);
    case 8: return launch_attention_bwd_half_k<T, 8>(a);
    default: break;
  }
  pt_host::set_error("Taylor attention backward: degree outside 0..PT_MAX_DEGREE");
  return PT_UNSUPPORTED;
}

}  // namespace pt
