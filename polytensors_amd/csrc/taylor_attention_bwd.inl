// Flash-style attention backward of degree-K series on MFMA (gfx950).
//
// The gradient series of attention for an output cotangent series G(t)
// (coefficient j = sum_{k<=j} J_{j-k}^T G_k) is the vector-Jacobian product of
// O = softmax(scale Q K^T) V evaluated in truncated series arithmetic, every
// product a Cauchy product (*) of the orders:
//   P = exp(scale Q (*) K^T - lse)     lse: the forward's log-sum-exp series,
//   dV = P^T (*) G,   dP = G (*) V^T,   Delta = rowsum(G (*) O),
//   dS = P (*) (dP - Delta),   dQ = scale dS (*) K,   dK = scale dS^T (*) Q.
// At degree 1 this is the reference's backward
// (/root/reference/src/polytensors/_attention_kernels.py:85-201 with the
// cotangent swap of _fused_attention.py:267-295), here at any degree. The
// exponential series is P_0 = exp(x_0), P_k = (1/k) sum_{i=1..k} i x_i P_{k-i}
// with x = scale Q (*) K^T - lse (/root/reference/src/polytensors/_plain.py:153-159).
// An inadmissible (query, key) pair and a query row with no admissible key
// (lse_0 = +inf) have P = 0 in every order.
//
// Three kernels, deterministic (no atomics):
// * attn_bwd_delta_kernel: the Delta series of every query row (16 lanes per row).
// * taylor_attention_bwd_q_kernel: the forward's decomposition (64 queries per
//   workgroup, 16 per wave, key blocks of 16 of every order of K and V staged
//   in LDS). Scores and dP are formed transposed (keys x queries) so that dS^T
//   sits in the accumulator registers in the B-operand layout of
//   dQ^T += K^T dS^T; lse and Delta of the lane's query are per-lane constants.
// * taylor_attention_bwd_kv_kernel: the mirror image (64 keys per workgroup, 16
//   per wave, query blocks of 16 with their Q, G, lse and Delta staged in LDS).
//   Scores are queries x keys, so that P and dS are the B operands of
//   dV^T += G^T P and dK^T += Q^T dS.
// Output accumulators beyond a register budget are split into head-dim slices
// (a grid dimension; each slice recomputes its scores), and dK and dV get one
// pass each when both do not fit.
#pragma once

#include "taylor_attention.inl"

namespace pt {

// Head-dim chunks per slice: the most (a power-of-two divisor of db) whose
// accumulators stay within `budget` 32-bit registers per lane.
constexpr int attn_bwd_chunks(int orders, int acc_regs, int outputs, int db, int budget) {
  int n = db;
  while (n > 1 && orders * n * acc_regs * outputs > budget) n /= 2;
  return n;
}

// Launch plan of the backward kernels: accumulator budget of 160 registers per lane.
template <typename T, int K, int D>
struct AttnBwdPlan {
  using A = typename AccOf<T>::type;
  static constexpr int DB = D / 16;
  static constexpr int kAccRegs = 4 * static_cast<int>(sizeof(A) / 4);   // registers per 16x16 accumulator
  static constexpr int kBudget = 160;
  static constexpr bool kv_fused = (K + 1) * DB * kAccRegs * 2 <= kBudget;   // dK and dV in one pass
  static constexpr int NS_KV = attn_bwd_chunks(K + 1, kAccRegs, kv_fused ? 2 : 1, DB, kBudget);
  static constexpr int NS_Q = attn_bwd_chunks(K + 1, kAccRegs, 1, DB, kBudget);
  // the dK/dV kernel on stored P and dS tiles holds no score series: a larger budget
  static constexpr int kMatBudget = 192;
  // fused dK and dV also hold both tile series twice (current and prefetched block)
  static constexpr bool km_fused = (K + 1) * DB * kAccRegs * 2 + 4 * (K + 1) * kAccRegs <= kMatBudget;
  static constexpr int NS_KM = attn_bwd_chunks(K + 1, kAccRegs, km_fused ? 2 : 1, DB, kMatBudget);
  // two whole-head-dim tiles of 16 rows of every order (K and V, or Q and G) and two 16-row
  // accumulator series; where the two tiles do not fit (float64 at head dim 128 from degree 4)
  // they take turns in one buffer, staged one after the other within each block (seq)
  static constexpr size_t tile_bytes = static_cast<size_t>(K + 1) * kAttnBN * AttnShape<T, K, D>::LD * sizeof(T);
  static constexpr size_t acc_bytes = 2ull * (K + 1) * 16 * sizeof(A);
  static constexpr bool seq = 2 * tile_bytes + acc_bytes > 160 * 1024;
  static constexpr size_t kv_lds = (seq ? 1 : 2) * tile_bytes + acc_bytes;
  static constexpr bool fits = kv_lds <= 160 * 1024;
};

// N consecutive values at p (16-byte loads when the run is a whole number of them).
template <typename T, int N>
__device__ __forceinline__ void load_run(const T* p, typename AccOf<T>::type (&out)[N]) {
  constexpr int V = 16 / sizeof(T);
  if constexpr (N % V == 0) {
#pragma unroll
    for (int i = 0; i < N / V; ++i) {
      const Vec<T, V> x = load_vec<T, V>(p + i * V);
#pragma unroll
      for (int e = 0; e < V; ++e) out[i * V + e] = to_acc(x.v[e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < N; ++e) out[e] = to_acc(p[e]);
  }
}

// Delta_k = sum_{a+b=k} rowsum(G_a * O_b) for every query row; 16 lanes per row.
template <typename T, int K, int D>
__global__ __launch_bounds__(256) void attn_bwd_delta_kernel(CPtrs<T> G, CPtrs<T> O,
                                                             MPtrs<typename AccOf<T>::type> Delta,
                                                             int64_t rows) {
  using A = typename AccOf<T>::type;
  constexpr int EPL = D / 16;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 16 + threadIdx.x / 16;
  const int j = threadIdx.x % 16;
  A acc[K + 1];
#pragma unroll
  for (int k = 0; k <= K; ++k) acc[k] = A(0);
  if (row < rows) {
    A g[K + 1][EPL], o[K + 1][EPL];
#pragma unroll
    for (int k = 0; k <= K; ++k) {
      load_run<T, EPL>(G.p[k] + row * D + j * EPL, g[k]);
      load_run<T, EPL>(O.p[k] + row * D + j * EPL, o[k]);
    }
#pragma unroll
    for (int k = 0; k <= K; ++k)
#pragma unroll
      for (int a = 0; a <= k; ++a)
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[k] += g[a][e] * o[k - a][e];
  }
#pragma unroll
  for (int k = 0; k <= K; ++k) {
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) acc[k] += __shfl_xor(acc[k], off, kWave);
  }
  if (row < rows && j == 0) {
#pragma unroll
    for (int k = 0; k <= K; ++k) Delta.p[k][row] = acc[k];
  }
}

// Probability series of one score element from its raw score accumulators
// (unscaled), its additive mask value (0 without one), the row's lse series and
// admissibility.
template <typename A, int K, typename AccT>
__device__ __forceinline__ void attn_prob_series(const AccT (&sc)[K + 1], int r, const A (&lse)[K + 1],
                                                 bool valid, A scale, A add, A (&p)[K + 1]) {
  p[0] = valid ? exp_fast(static_cast<A>(sc[0][r]) * scale + add - lse[0]) : A(0);
  // b_i = i x_i with x_i = scale S_i - lse_i: one fma per order (i scale and i lse_i do not depend
  // on the key, so they leave the key loop)
  A b[K + 1];
#pragma unroll
  for (int i = 1; i <= K; ++i) b[i] = static_cast<A>(sc[i][r]) * (A(i) * scale) - A(i) * lse[i];
#pragma unroll
  for (int k = 1; k <= K; ++k) {
    A t = b[1] * p[k - 1];
#pragma unroll
    for (int i = 2; i <= k; ++i) t += b[i] * p[k - i];
    p[k] = t * (A(1) / A(k));
  }
}

// dS_k = sum_{a+b=k} P_a (dP_b - Delta_b).
template <typename A, int K, typename AccT>
__device__ __forceinline__ void attn_ds_series(const A (&p)[K + 1], const AccT (&dp)[K + 1], int r,
                                               const A (&delta)[K + 1], A (&ds)[K + 1]) {
  A u[K + 1];
#pragma unroll
  for (int b = 0; b <= K; ++b) u[b] = static_cast<A>(dp[b][r]) - delta[b];
#pragma unroll
  for (int k = 0; k <= K; ++k) {
    A t = A(0);
#pragma unroll
    for (int a = 0; a <= k; ++a) t += p[a] * u[k - a];
    ds[k] = t;
  }
}

// Stores the accumulators of one 16-row tile of a [rows, D] output (accumulator
// n of the slice covers head-dim chunk chunk0 + n; register r of lane group h
// holds column 16 (chunk0 + n) + acc_row(h, r) of row `row`).
template <typename T, int K, int NS, typename AccT>
__device__ __forceinline__ void attn_bwd_store(const AccT (&acc)[K + 1][NS], MPtrs<T>& out, int64_t row,
                                               int chunk0, int h, typename AccOf<T>::type factor) {
  using MF = Mfma16<T>;
  constexpr int D16 = 16;
#pragma unroll
  for (int k = 0; k <= K; ++k) {
#pragma unroll
    for (int n = 0; n < NS; ++n) {
      T* dst = out.p[k] + row + (chunk0 + n) * D16;
      if constexpr (sizeof(T) == 4) {
        Vec<T, 4> w;
#pragma unroll
        for (int r = 0; r < 4; ++r) w.v[r] = static_cast<T>(acc[k][n][r] * factor);
        store_vec<T, 4>(dst + 4 * h, w);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[MF::acc_row(h, r)] = static_cast<T>(acc[k][n][r] * factor);
      }
    }
  }
}

// Offset of element (query qi, key ki) of 16 x 16 tile (qt, kt) of one head in
// the P / dS tile buffers (float): tiles are [head][query tile][key tile], and
// within a tile the element sits at (ki % 4) * 64 + (ki / 4) * 16 + qi. The
// producer's lane (query c, lane group h) holds keys 4h + r in register r, so
// one store instruction (fixed r) writes 256 contiguous bytes; the consumer's
// lane (key c, lane group h) needs queries 4h .. 4h + 3 of its key, which are
// consecutive: one 16-byte load (attn_tile_consumer_offset).
// (Host-callable, like the work-item and range helpers below: the index checks
// of the tests replay the producer and consumer addressing on the CPU.)
__host__ __device__ __forceinline__ int64_t attn_tile_base(int64_t head, int qt, int kt, int nqt, int nkt) {
  return ((head * nqt + qt) * nkt + kt) * 256;
}
__host__ __device__ __forceinline__ int64_t attn_tile_offset(int64_t head, int qt, int kt, int nqt, int nkt, int qi,
                                                             int ki) {
  return attn_tile_base(head, qt, kt, nqt, nkt) + (ki % 4) * 64 + (ki / 4) * 16 + qi;
}
// first of the four consecutive values (queries 4h .. 4h + 3 of key c) a consumer lane reads
__host__ __device__ __forceinline__ int64_t attn_tile_consumer_offset(int64_t head, int qt, int kt, int nqt,
                                                                      int nkt, int c, int h) {
  return attn_tile_base(head, qt, kt, nqt, nkt) + (c % 4) * 64 + (c / 4) * 16 + 4 * h;
}

// Work item of workgroup t of the query-side kernel (grid: query blocks x heads x
// slices): head fastest (consecutive workgroups on consecutive XCDs), then
// head-dim slice, then query block, heaviest (last) query block first.
__host__ __device__ __forceinline__ void attn_bwd_q_item(int64_t t, int64_t bh, int nqb, int slices, int64_t& head,
                                                         int& slice, int& q_block) {
  head = t % bh;
  slice = static_cast<int>((t / bh) % slices);
  q_block = (nqb - 1 - static_cast<int>(t / (bh * slices))) * kAttnBM;
}

// Work item of workgroup t of a key-side kernel (grid: 64-key blocks x heads x
// slices): head fastest, then slice, then key block, lightest causal work (the
// last key block) last.
__host__ __device__ __forceinline__ void attn_bwd_kv_item(int64_t t, int64_t bh, int slices, int64_t& head,
                                                          int& slice, int& kv_block) {
  head = t % bh;
  slice = static_cast<int>((t / bh) % slices);
  kv_block = static_cast<int>(t / (bh * slices)) * (kAttnWaves * 16);
}

// Query range [lo, hi) a key workgroup visits: causal (queries from the block's
// first key on) and mask-range bounds, lo rounded down to a 16-query block.
__host__ __device__ __forceinline__ void attn_query_range(int L, int kv_block, int causal, const int32_t* ranges,
                                                          int& lo, int& hi) {
  lo = causal ? kv_block : 0;
  hi = L;
  if (ranges != nullptr) {
    const int nqb = (L + kAttnRangeBlock - 1) / kAttnRangeBlock;
    const int kb = nqb + kv_block / kAttnRangeBlock;
    const int rl = static_cast<int>(ranges[2 * kb]) / 16 * 16, rh = static_cast<int>(ranges[2 * kb + 1]);
    lo = lo > rl ? lo : rl;
    hi = hi < rh ? hi : rh;
  }
}

// Register-staged copy of ROWS rows (from row `first`, zero past `limit`) of the
// K+1 orders of a [*, D] series into an LDS tile [K+1][ROWS][LD]: fetch issues
// the global loads into registers (early, so they are in flight during the
// previous block's MFMAs) and commit writes them to LDS after the barrier.
template <typename T, int K, int D, int ROWS>
struct RowStager {
  static constexpr int V = 16 / sizeof(T);
  static constexpr int VPR = D / V;                // 16-byte vectors per row
  static constexpr int PER_ORDER = ROWS * VPR;     // vectors per order
  static constexpr int THREADS = kAttnWaves * kWave;
  static constexpr int IPO = (PER_ORDER + THREADS - 1) / THREADS;   // per thread and order
  static constexpr int ITERS = (K + 1) * IPO;
  static_assert(ITERS <= 64, "validity bits");
  Vec<T, V> r[ITERS];
  uint64_t valid = 0;   // bit i: vector i is real (in range and below the row limit)

  // Every step handles one order for all lanes (its pointer is a scalar kernel
  // argument), and every lane loads: rows past `limit` (>= 1) and lanes past the
  // order's vectors load a valid duplicate and are dropped at commit. A load
  // under a per-lane branch would be waited for at the branch's end.
  __device__ __forceinline__ void fetch(const CPtrs<T>& src, int64_t row_base, int first, int limit) {
    valid = 0;
#pragma unroll
    for (int o = 0; o <= K; ++o) {
#pragma unroll
      for (int j = 0; j < IPO; ++j) {
        const int i = o * IPO + j;
        const int idx = static_cast<int>(threadIdx.x) + THREADS * j;
        const int e = min(idx, PER_ORDER - 1);
        const int row = first + e / VPR, cv = (e % VPR) * V;
        r[i] = load_vec<T, V>(src.p[o] + (row_base + min(row, limit - 1)) * D + cv);
        valid |= static_cast<uint64_t>(row < limit) << i;
      }
    }
  }
  template <int LD>
  __device__ __forceinline__ void commit(T (&tile)[K + 1][ROWS][LD]) const {
#pragma unroll
    for (int o = 0; o <= K; ++o) {
#pragma unroll
      for (int j = 0; j < IPO; ++j) {
        const int i = o * IPO + j;
        const int idx = static_cast<int>(threadIdx.x) + THREADS * j;
        if (PER_ORDER % THREADS == 0 || idx < PER_ORDER) {
          Vec<T, V> w;
          const bool ok = (valid >> i) & 1u;
#pragma unroll
          for (int e = 0; e < V; ++e) w.v[e] = ok ? r[i].v[e] : T(0);
          store_vec<T, V>(&tile[o][idx / VPR][(idx % VPR) * V], w);
        }
      }
    }
  }
};

// acc[k][n] += sum_{a+b=k} tile[b][row(s)][col(n)] * bop(a, s) for the NS
// head-dim chunks n and the 4 steps s of a 16x16x4 product (A operands from an
// LDS tile [K+1][16][LD]: row acc_row(h, s), column 16 (chunk0 + n) + c; B
// operands bop(a, s) from registers). Step t+1's LDS operands are read while
// step t's MFMAs run.
template <typename T, int K, int NS, int LD, typename AccT, typename BOp>
__device__ __forceinline__ void attn_lds_products(AccT (&acc)[K + 1][NS], const T (&tile)[K + 1][16][LD],
                                                  int chunk0, int c, int h, const BOp& bop) {
  using MF = Mfma16<T>;
  constexpr int STEPS = NS * 4;
  T ring[2][K + 1];
  auto load = [&](T (&dst)[K + 1], int t) {
    const int row = MF::acc_row(h, t % 4), col = (chunk0 + t / 4) * 16 + c;
#pragma unroll
    for (int o = 0; o <= K; ++o) dst[o] = tile[o][row][col];
  };
  load(ring[0], 0);
#pragma unroll
  for (int t = 0; t < STEPS; ++t) {
    if (t + 1 < STEPS) load(ring[(t + 1) & 1], t + 1);
    __builtin_amdgcn_sched_barrier(0);
    const int n = t / 4, sidx = t % 4;
#pragma unroll
    for (int k = 0; k <= K; ++k)
#pragma unroll
      for (int a = 0; a <= k; ++a) acc[k][n] = MF::mma(ring[t & 1][k - a], bop(a, sidx), acc[k][n]);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// The two head-dim contractions of one block, S (chunks 0..DB-1 of the global
// operand) then dP (chunks DB..2DB-1), with the global operand read one chunk
// ahead: chunk c+1 is loaded into the other half of the register ring while
// chunk c's MFMAs run, and the last step loads chunk 0 again for the next
// block. Chunks are taken in pairs so that the ring halves are static
// registers. ring[0] holds chunk 0 on entry and on exit. PHASES = 1 runs the S
// contraction only (chunks 0..DB-1).
//
// RING > 2 (the chunk loop fully unrolled, RING dividing the chunk count): chunk
// c + RING - 1 is loaded while chunk c's MFMAs run, RING - 1 chunks ahead;
// ring[i] holds chunk i (i < RING - 1) on entry and on exit.
template <typename T, int K, int DB, int PHASES = 2, int RING = 2, typename Load, typename StepS, typename StepP>
__device__ __forceinline__ void attn_bwd_contract(Vec<T, 4> (&ring)[RING][K + 1], Load& load, StepS& s_step,
                                                  StepP& p_step) {
  constexpr int NC = PHASES * DB;   // chunks per block
  if constexpr (RING > 2) {
    static_assert(NC % RING == 0, "the ring must divide the chunks of a block");
    constexpr int AHEAD = RING - 1;
#pragma unroll
    for (int cg = 0; cg < NC; ++cg) {
      load(ring[(cg + AHEAD) % RING], (cg + AHEAD) % NC);
      __builtin_amdgcn_sched_barrier(0);
      if (cg < DB) s_step(cg, ring[cg % RING]);
      else p_step(cg - DB, ring[cg % RING]);
      __builtin_amdgcn_sched_barrier(0);
    }
  } else if constexpr (NC == 1) {
    s_step(0, ring[0]);
  } else if constexpr (DB == 1) {   // PHASES == 2: one chunk per phase
    load(ring[1], 1);
    __builtin_amdgcn_sched_barrier(0);
    s_step(0, ring[0]);
    load(ring[0], 0);
    __builtin_amdgcn_sched_barrier(0);
    p_step(0, ring[1]);
  } else {
#pragma unroll 1
    for (int dc = 0; dc < DB; dc += 2) {
      load(ring[1], dc + 1);
      __builtin_amdgcn_sched_barrier(0);
      s_step(dc, ring[0]);
      load(ring[0], (dc + 2) % NC);
      __builtin_amdgcn_sched_barrier(0);
      s_step(dc + 1, ring[1]);
    }
    if constexpr (PHASES == 2) {
#pragma unroll 1
      for (int dc = 0; dc < DB; dc += 2) {
        load(ring[1], DB + dc + 1);
        __builtin_amdgcn_sched_barrier(0);
        p_step(dc, ring[0]);
        load(ring[0], (DB + dc + 2) % NC);
        __builtin_amdgcn_sched_barrier(0);
        p_step(dc + 1, ring[1]);
      }
    }
  }
}

// STORE: also write the P and dS series of every visited 16 x 16 (query, key)
// tile to PT / DST (attn_tile_offset layout) for taylor_attention_bwd_kv_mat_kernel.
// MASK: 0 no mask, 1 a boolean mask, 2 a boolean mask and the additive mask madd
// whose finite entries it marks (the unmasked instantiation holds no mask
// registers: at K = 4, D = 128 four of them cost the causal case 3%).
template <typename T, int K, int D, int NS, bool STORE, int MASK>
__global__ __launch_bounds__(kAttnWaves * kWave) void taylor_attention_bwd_q_kernel(
    CPtrs<T> Q, CPtrs<T> Kp, CPtrs<T> Vp, CPtrs<T> G, CPtrs<typename AccOf<T>::type> LSE,
    CPtrs<typename AccOf<T>::type> DELTA, MPtrs<T> DQ, MPtrs<T> PT, MPtrs<T> DST, int L, int S,
    const uint8_t* __restrict__ mask_all, AttnMaskMap mmap, const typename AccOf<T>::type* __restrict__ madd_all,
    const int32_t* __restrict__ ranges_all, int causal, typename AccOf<T>::type scale) {
  constexpr bool MASKED = MASK != 0, ADD = MASK == 2;
  static_assert(!(ADD && STORE), "an additive mask runs the recomputing path");
  using A = typename AccOf<T>::type;
  using MF = Mfma16<T>;
  using acc_t = typename MF::acc_t;
  constexpr int LD = AttnShape<T, K, D>::LD;
  constexpr int DB = D / 16;
  constexpr int SLICES = DB / NS;
  constexpr int V = 16 / sizeof(T);
  constexpr int QV = 4;
  constexpr bool SEQ = AttnBwdPlan<T, K, D>::seq;   // K and V tiles take turns in one buffer

  __shared__ T tiles[SEQ ? 1 : 2][K + 1][kAttnBN][LD];
  auto& Ks = tiles[0];
  auto& Vs = tiles[SEQ ? 0 : 1];

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int c = lane % 16;
  const int h = lane / 16;
  const int nqb = (L + kAttnBM - 1) / kAttnBM;
  const int64_t bh = gridDim.x / (static_cast<int64_t>(nqb) * SLICES);
  int64_t head;
  int slice, q_block;
  attn_bwd_q_item(blockIdx.x, bh, nqb, SLICES, head, slice, q_block);
  // this head's mask, its block ranges (and additive values)
  const int64_t mask_index = attn_mask_index(mmap, head);
  const uint8_t* mask = mask_all != nullptr ? mask_all + mask_index * L * S : nullptr;
  const int32_t* ranges = ranges_all != nullptr ? ranges_all + mask_index * attn_ranges_count(L, S) : nullptr;
  const typename AccOf<T>::type* madd = madd_all != nullptr ? madd_all + mask_index * L * S : nullptr;
  const int my_q = q_block + wave * kAttnQPerWave + c;
  const bool q_ok = my_q < L;
  const int64_t qoff = (head * L + (q_ok ? my_q : 0)) * D;

  A lse[K + 1], delta[K + 1];
#pragma unroll
  for (int o = 0; o <= K; ++o) {
    lse[o] = q_ok ? LSE.p[o][head * L + my_q] : (o == 0 ? A(__builtin_huge_val()) : A(0));
    delta[o] = q_ok ? DELTA.p[o][head * L + my_q] : A(0);
  }

  acc_t acc[K + 1][NS];
#pragma unroll
  for (int o = 0; o <= K; ++o)
#pragma unroll
    for (int n = 0; n < NS; ++n) acc[o][n] = MF::zero();

  // Global operand chunks c = 0 .. 2 DB - 1: Q[my row] for c < DB, then G[my row]; chunk c
  // covers head dims 16 (c mod DB) + 4h .. +3 of every order.
  auto load_glob = [&](Vec<T, QV>(&buf)[K + 1], int cg) {
    const bool second = cg >= DB;
    const int dc = second ? cg - DB : cg;
#pragma unroll
    for (int o = 0; o <= K; ++o)
      buf[o] = *reinterpret_cast<const Vec<T, QV>*>((second ? G.p[o] : Q.p[o]) + qoff + dc * 16 + 4 * h);
  };
  // Global operand ring: four slots (three chunks ahead; 2.4% faster at K = 4,
  // D = 128 than two) where the float kernels take them without spilling
  // registers (checked per instantiation), else two.
  constexpr int kRing =
      (sizeof(T) == 4 && (2 * DB) % 4 == 0 && (K <= 4 || (K <= 6 && D <= 64) || D == 16)) ? 4 : 2;
  Vec<T, QV> gq[kRing][K + 1];
#pragma unroll
  for (int i = 0; i < (kRing > 2 ? kRing - 1 : 1); ++i) load_glob(gq[i], i);

  int lo, hi;
  attn_key_range(S, q_block, causal, ranges, lo, hi);
  // Key block kb0+16's K and V rows are fetched into registers while block kb0's
  // MFMAs run, where the registers allow (otherwise staged when needed).
  // (registers: accumulators + two staged row sets + operand ring + score series)
  constexpr int kW = static_cast<int>(sizeof(A) / 4);
  constexpr bool kPrefetchStage =
      !SEQ && (K + 1) * NS * 4 * kW + 2 * RowStager<T, K, D, kAttnBN>::ITERS * 4 + 2 * (K + 1) * 4 * kW +
                      2 * (K + 1) * 4 * kW <= 330;
  // rows kb0 .. kb0+15 of every order of one operand into a tile (zero past S)
  auto stage_rows = [&](T(&tile)[K + 1][kAttnBN][LD], const CPtrs<T>& src, int kb0) {
    constexpr int VPR = D / V;
    for (int idx = threadIdx.x; idx < (K + 1) * kAttnBN * VPR; idx += kAttnWaves * kWave) {
      const int o = idx / (kAttnBN * VPR);
      const int rem = idx % (kAttnBN * VPR);
      const int r = rem / VPR, cv = (rem % VPR) * V;
      const int key = kb0 + r;
      Vec<T, V> x;
      if (key < S) {
        x = load_vec<T, V>(order_ptr<K>(src, o) + (head * S + key) * D + cv);
      } else {
#pragma unroll
        for (int e = 0; e < V; ++e) x.v[e] = T(0);
      }
      store_vec<T, V>(&tile[o][r][cv], x);
    }
  };
  RowStager<T, K, D, kAttnBN> stage_k, stage_v;
  if constexpr (kPrefetchStage) {
    if (lo < hi) {
      stage_k.fetch(Kp, head * S, lo, S);
      stage_v.fetch(Vp, head * S, lo, S);
    }
  }
  for (int kb0 = lo; kb0 < hi; kb0 += kAttnBN) {
    uint8_t mbyte[MASKED ? 4 : 1];   // mask bytes of this lane's keys, read ahead of the block's prefetches
    A add[ADD ? 4 : 1] = {};
    if constexpr (MASKED) {
#pragma unroll
      for (int r = 0; r < 4; ++r) mbyte[r] = attn_mask_byte(mask, Q.p[0], my_q, kb0 + MF::acc_row(h, r), L, S);
    }
    if constexpr (ADD) {
#pragma unroll
      for (int r = 0; r < 4; ++r) add[r] = attn_mask_add(madd, my_q, kb0 + MF::acc_row(h, r), L, S);
    }
    __syncthreads();   // the previous block's MFMAs are done with the tiles
    if constexpr (kPrefetchStage) {
      stage_k.commit(Ks);
      stage_v.commit(Vs);
    } else {
      if constexpr (SEQ) {
        stage_rows(Vs, Vp, kb0);   // dP first: V now, K after it
      } else {
        stage_rows(Ks, Kp, kb0);
        stage_rows(Vs, Vp, kb0);
      }
    }
    __syncthreads();

    // S^T_k = sum_{a+b=k} K_b Q_a^T and dP^T_k = sum_{a+b=k} V_b G_a^T (keys x queries)
    acc_t sc[K + 1], dp[K + 1];
#pragma unroll
    for (int o = 0; o <= K; ++o) sc[o] = dp[o] = MF::zero();
    auto s_step = [&](int dc, const Vec<T, QV>(&qa)[K + 1]) {
      Vec<T, QV> kb[K + 1];
#pragma unroll
      for (int o = 0; o <= K; ++o) kb[o] = *reinterpret_cast<const Vec<T, QV>*>(&Ks[o][c][dc * 16 + 4 * h]);
#pragma unroll
      for (int s = 0; s < QV; ++s)
#pragma unroll
        for (int k = 0; k <= K; ++k)
#pragma unroll
          for (int a = 0; a <= k; ++a) sc[k] = MF::mma(kb[k - a].v[s], qa[a].v[s], sc[k]);
    };
    auto p_step = [&](int dc, const Vec<T, QV>(&ga)[K + 1]) {
      Vec<T, QV> vb[K + 1];
#pragma unroll
      for (int o = 0; o <= K; ++o) vb[o] = *reinterpret_cast<const Vec<T, QV>*>(&Vs[o][c][dc * 16 + 4 * h]);
#pragma unroll
      for (int s = 0; s < QV; ++s)
#pragma unroll
        for (int k = 0; k <= K; ++k)
#pragma unroll
          for (int a = 0; a <= k; ++a) dp[k] = MF::mma(vb[k - a].v[s], ga[a].v[s], dp[k]);
    };
    if constexpr (SEQ) {
      // dP^T with the V tile, then the K tile in its place for S^T (and the dQ products)
      for (int dc = 0; dc < DB; ++dc) {
        Vec<T, QV> ga[K + 1];
        load_glob(ga, DB + dc);
        p_step(dc, ga);
      }
      __syncthreads();   // every wave is done with the V tile
      stage_rows(Ks, Kp, kb0);
      __syncthreads();
      for (int dc = 0; dc < DB; ++dc) {
        Vec<T, QV> qa[K + 1];
        load_glob(qa, dc);
        s_step(dc, qa);
      }
    } else {
      attn_bwd_contract<T, K, DB, 2, kRing>(gq, load_glob, s_step, p_step);
    }
    // The next block's K/V rows are fetched after the contraction's global loads (memory
    // waits complete in order), so they overlap the dS series and the dQ products.
    if constexpr (kPrefetchStage) {
      if (kb0 + kAttnBN < hi) {
        stage_k.fetch(Kp, head * S, kb0 + kAttnBN, S);
        stage_v.fetch(Vp, head * S, kb0 + kAttnBN, S);
      }
      __builtin_amdgcn_sched_barrier(0);
    }

    // dS^T in place of the scores
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int key = kb0 + MF::acc_row(h, r);
      bool ok = q_ok && key < S;
      if (causal) ok = ok && key <= my_q;
      if constexpr (MASKED) ok = ok && mbyte[r] != 0;
      A p[K + 1], ds[K + 1];
      attn_prob_series<A, K>(sc, r, lse, ok, scale, ADD ? add[r] : A(0), p);
      attn_ds_series<A, K>(p, dp, r, delta, ds);
#pragma unroll
      for (int o = 0; o <= K; ++o) sc[o][r] = static_cast<T>(ds[o]);
      if constexpr (STORE) {
        static_assert(sizeof(T) == 4, "the tile layout follows the float accumulator layout (acc_row = 4h + r)");
        // (a wave whose 16 queries all lie past L owns no tile)
        if (slice == 0 && q_block + wave * kAttnQPerWave < L) {
          // element (query c, key acc_row(h, r)) of the wave's tile
          const int64_t at = attn_tile_offset(head, q_block / 16 + wave, kb0 / 16, (L + 15) / 16,
                                                  (S + 15) / 16, c, MF::acc_row(h, r));
#pragma unroll
          for (int o = 0; o <= K; ++o) {
            PT.p[o][at] = static_cast<T>(p[o]);
            DST.p[o][at] = static_cast<T>(ds[o]);
          }
        }
      }
    }

    // dQ^T_k += sum_{a+b=k} K_b^T dS^T_a (head dim x queries)
    attn_lds_products<T, K, NS>(acc, Ks, slice * NS, c, h, [&](int a, int sidx) { return sc[a][sidx]; });
  }

  if (q_ok && DQ.p[0] != nullptr) attn_bwd_store<T, K, NS>(acc, DQ, (head * L + my_q) * D, slice * NS, h, scale);
}

// WHAT: 1 = dV, 2 = dK, 3 = both. MASK as the dQ kernel's.
template <typename T, int K, int D, int NS, int WHAT, int MASK>
__global__ __launch_bounds__(kAttnWaves * kWave) void taylor_attention_bwd_kv_kernel(
    CPtrs<T> Q, CPtrs<T> Kp, CPtrs<T> Vp, CPtrs<T> G, CPtrs<typename AccOf<T>::type> LSE,
    CPtrs<typename AccOf<T>::type> DELTA, MPtrs<T> DK, MPtrs<T> DV, int L, int S,
    const uint8_t* __restrict__ mask_all, AttnMaskMap mmap, const typename AccOf<T>::type* __restrict__ madd_all,
    const int32_t* __restrict__ ranges_all, int causal, typename AccOf<T>::type scale) {
  constexpr bool MASKED = MASK != 0, ADD = MASK == 2;
  using A = typename AccOf<T>::type;
  using MF = Mfma16<T>;
  using acc_t = typename MF::acc_t;
  constexpr int LD = AttnShape<T, K, D>::LD;
  constexpr int DB = D / 16;
  constexpr int SLICES = DB / NS;
  constexpr int V = 16 / sizeof(T);
  constexpr int QV = 4;
  constexpr int kBM = 16;                       // queries per block
  constexpr int kBK = kAttnWaves * 16;          // keys per workgroup
  static_assert(kBK == kAttnRangeBlock, "key blocks are the mask-range blocks");
  constexpr bool DO_V = (WHAT & 1) != 0;
  constexpr bool DO_K = (WHAT & 2) != 0;
  constexpr bool SEQ = AttnBwdPlan<T, K, D>::seq;   // Q and G tiles take turns in one buffer
  static_assert(!SEQ || WHAT != 3, "with one tile buffer dK and dV run as separate passes");

  __shared__ T tiles[SEQ ? 1 : 2][K + 1][kBM][LD];
  auto& Qs = tiles[0];
  auto& Gs = tiles[SEQ ? 0 : 1];
  __shared__ A Ls[K + 1][kBM];
  __shared__ A Ds[K + 1][kBM];

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int c = lane % 16;
  const int h = lane / 16;
  const int nkb = (S + kBK - 1) / kBK;
  const int64_t bh = gridDim.x / (static_cast<int64_t>(nkb) * SLICES);
  int64_t head;
  int slice, kv_block;
  attn_bwd_kv_item(blockIdx.x, bh, SLICES, head, slice, kv_block);
  // this head's mask, its block ranges (and additive values)
  const int64_t mask_index = attn_mask_index(mmap, head);
  const uint8_t* mask = mask_all != nullptr ? mask_all + mask_index * L * S : nullptr;
  const int32_t* ranges = ranges_all != nullptr ? ranges_all + mask_index * attn_ranges_count(L, S) : nullptr;
  const typename AccOf<T>::type* madd = madd_all != nullptr ? madd_all + mask_index * L * S : nullptr;
  const int my_k = kv_block + wave * 16 + c;
  const bool k_ok = my_k < S;
  const int64_t koff = (head * S + (k_ok ? my_k : 0)) * D;

  acc_t acc_v[DO_V ? K + 1 : 1][NS], acc_k[DO_K ? K + 1 : 1][NS];
#pragma unroll
  for (int n = 0; n < NS; ++n) {
#pragma unroll
    for (int o = 0; o < (DO_V ? K + 1 : 1); ++o) acc_v[o][n] = MF::zero();
#pragma unroll
    for (int o = 0; o < (DO_K ? K + 1 : 1); ++o) acc_k[o][n] = MF::zero();
  }

  // Global operand chunks c: K[my key] for c < DB, then V[my key] (dK passes).
  auto load_glob = [&](Vec<T, QV>(&buf)[K + 1], int cg) {
    const bool second = cg >= DB;
    const int dc = second ? cg - DB : cg;
#pragma unroll
    for (int o = 0; o <= K; ++o)
      buf[o] = *reinterpret_cast<const Vec<T, QV>*>((second ? Vp.p[o] : Kp.p[o]) + koff + dc * 16 + 4 * h);
  };
  Vec<T, QV> gk[2][K + 1];
  load_glob(gk[0], 0);

  int lo, hi;
  attn_query_range(L, kv_block, causal, ranges, lo, hi);
  for (int qb0 = lo; qb0 < hi; qb0 += kBM) {
    uint8_t mbyte[MASKED ? 4 : 1];   // mask bytes of this lane's queries, read ahead of the block's loads
    A add[ADD ? 4 : 1] = {};
    if constexpr (MASKED) {
#pragma unroll
      for (int r = 0; r < 4; ++r) mbyte[r] = attn_mask_byte(mask, Q.p[0], qb0 + MF::acc_row(h, r), my_k, L, S);
    }
    if constexpr (ADD) {
#pragma unroll
      for (int r = 0; r < 4; ++r) add[r] = attn_mask_add(madd, qb0 + MF::acc_row(h, r), my_k, L, S);
    }
    __syncthreads();
    // rows qb0 .. qb0+15 of every order of one operand into a tile (zero past L)
    auto stage_rows = [&](T(&tile)[K + 1][kBM][LD], const CPtrs<T>& src) {
      constexpr int VPR = D / V;
      for (int idx = threadIdx.x; idx < (K + 1) * kBM * VPR; idx += kAttnWaves * kWave) {
        const int o = idx / (kBM * VPR);
        const int rem = idx % (kBM * VPR);
        const int r = rem / VPR, cv = (rem % VPR) * V;
        const int q = qb0 + r;
        Vec<T, V> x;
        if (q < L) {
          x = load_vec<T, V>(order_ptr<K>(src, o) + (head * L + q) * D + cv);
        } else {
#pragma unroll
          for (int e = 0; e < V; ++e) x.v[e] = T(0);
        }
        store_vec<T, V>(&tile[o][r][cv], x);
      }
    };
    {
      if constexpr (!SEQ) {
        stage_rows(Qs, Q);
        stage_rows(Gs, G);
      } else if constexpr (DO_K) {
        stage_rows(Gs, G);   // dP first: G now, Q after it
      } else {
        stage_rows(Qs, Q);   // S first: Q now, G after it
      }
      for (int idx = threadIdx.x; idx < (K + 1) * kBM; idx += kAttnWaves * kWave) {
        const int o = idx / kBM, r = idx % kBM;
        const int q = qb0 + r;
        Ls[o][r] = q < L ? LSE.p[o][head * L + q] : (o == 0 ? A(__builtin_huge_val()) : A(0));
        Ds[o][r] = q < L ? DELTA.p[o][head * L + q] : A(0);
      }
    }
    __syncthreads();

    // S_k = sum_{a+b=k} Q_a K_b^T and dP_k = sum_{a+b=k} G_a V_b^T (queries x keys)
    acc_t sc[K + 1], dp[DO_K ? K + 1 : 1];
#pragma unroll
    for (int o = 0; o <= K; ++o) sc[o] = MF::zero();
#pragma unroll
    for (int o = 0; o < (DO_K ? K + 1 : 1); ++o) dp[o] = MF::zero();
    auto s_step = [&](int dc, const Vec<T, QV>(&kb)[K + 1]) {
      Vec<T, QV> qa[K + 1];
#pragma unroll
      for (int o = 0; o <= K; ++o) qa[o] = *reinterpret_cast<const Vec<T, QV>*>(&Qs[o][c][dc * 16 + 4 * h]);
#pragma unroll
      for (int s = 0; s < QV; ++s)
#pragma unroll
        for (int k = 0; k <= K; ++k)
#pragma unroll
          for (int a = 0; a <= k; ++a) sc[k] = MF::mma(qa[a].v[s], kb[k - a].v[s], sc[k]);
    };
    auto p_step = [&](int dc, const Vec<T, QV>(&vb)[K + 1]) {
      if constexpr (DO_K) {
        Vec<T, QV> ga[K + 1];
#pragma unroll
        for (int o = 0; o <= K; ++o) ga[o] = *reinterpret_cast<const Vec<T, QV>*>(&Gs[o][c][dc * 16 + 4 * h]);
#pragma unroll
        for (int s = 0; s < QV; ++s)
#pragma unroll
          for (int k = 0; k <= K; ++k)
#pragma unroll
            for (int a = 0; a <= k; ++a) dp[k] = MF::mma(ga[a].v[s], vb[k - a].v[s], dp[k]);
      }
    };
    if constexpr (SEQ) {
      if constexpr (DO_K) {   // dP with the G tile, then the Q tile in its place for S (and dK)
        for (int dc = 0; dc < DB; ++dc) {
          Vec<T, QV> vb[K + 1];
          load_glob(vb, DB + dc);
          p_step(dc, vb);
        }
        __syncthreads();   // every wave is done with the G tile
        stage_rows(Qs, Q);
        __syncthreads();
      }
      for (int dc = 0; dc < DB; ++dc) {
        Vec<T, QV> kb[K + 1];
        load_glob(kb, dc);
        s_step(dc, kb);
      }
    } else {
      attn_bwd_contract<T, K, DB, DO_K ? 2 : 1>(gk, load_glob, s_step, p_step);
    }

    // P in place of the scores (dV), dS in place of dP (dK)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int qr = MF::acc_row(h, r);
      const int q = qb0 + qr;
      bool ok = k_ok && q < L;
      if (causal) ok = ok && my_k <= q;
      if constexpr (MASKED) ok = ok && mbyte[r] != 0;
      A lse[K + 1], p[K + 1];
#pragma unroll
      for (int o = 0; o <= K; ++o) lse[o] = Ls[o][qr];
      attn_prob_series<A, K>(sc, r, lse, ok, scale, ADD ? add[r] : A(0), p);
      if constexpr (DO_K) {
        A delta[K + 1], ds[K + 1];
#pragma unroll
        for (int o = 0; o <= K; ++o) delta[o] = Ds[o][qr];
        attn_ds_series<A, K>(p, dp, r, delta, ds);
#pragma unroll
        for (int o = 0; o <= K; ++o) dp[o][r] = static_cast<T>(ds[o]);
      }
      if constexpr (DO_V) {
#pragma unroll
        for (int o = 0; o <= K; ++o) sc[o][r] = static_cast<T>(p[o]);
      }
    }

    if constexpr (SEQ && DO_V) {   // the G tile in the Q tile's place for the dV products
      __syncthreads();
      stage_rows(Gs, G);
      __syncthreads();
    }

    // dV^T_k += sum_{a+b=k} G_b^T P_a and dK^T_k += sum_{a+b=k} Q_b^T dS_a (head dim x keys)
#pragma unroll
    for (int n = 0; n < NS; ++n) {
      const int col = (slice * NS + n) * 16 + c;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int qr = MF::acc_row(h, s);
        if constexpr (DO_V) {
          T gv[K + 1];
#pragma unroll
          for (int o = 0; o <= K; ++o) gv[o] = Gs[o][qr][col];
#pragma unroll
          for (int k = 0; k <= K; ++k)
#pragma unroll
            for (int a = 0; a <= k; ++a) acc_v[k][n] = MF::mma(gv[k - a], sc[a][s], acc_v[k][n]);
        }
        if constexpr (DO_K) {
          T qv[K + 1];
#pragma unroll
          for (int o = 0; o <= K; ++o) qv[o] = Qs[o][qr][col];
#pragma unroll
          for (int k = 0; k <= K; ++k)
#pragma unroll
            for (int a = 0; a <= k; ++a) acc_k[k][n] = MF::mma(qv[k - a], dp[a][s], acc_k[k][n]);
        }
      }
    }
  }

  if (!k_ok) return;
  const int64_t row = (head * S + my_k) * D;
  if constexpr (DO_V) attn_bwd_store<T, K, NS>(acc_v, DV, row, slice * NS, h, A(1));
  if constexpr (DO_K) attn_bwd_store<T, K, NS>(acc_k, DK, row, slice * NS, h, scale);
}

// dK / dV from the P and dS tiles written by the dQ kernel: per 64-key
// workgroup (16 keys per wave) and query block of 16, dV^T += G^T P and
// dK^T += Q^T dS with G and Q staged in LDS and the tile series read straight
// into the B-operand registers (masked by admissibility: tiles the dQ kernel
// did not visit hold no admissible pair). Two products per pair instead of the
// four of the recomputing kernel. WHAT: 1 = dV, 2 = dK, 3 = both.
template <typename T, int K, int D, int NS, int WHAT, bool MASKED>
__global__ __launch_bounds__(kAttnWaves * kWave) void taylor_attention_bwd_kv_mat_kernel(
    CPtrs<T> Q, CPtrs<T> G, CPtrs<T> PT, CPtrs<T> DST, MPtrs<T> DK, MPtrs<T> DV, int L, int S,
    const uint8_t* __restrict__ mask_all, AttnMaskMap mmap, const int32_t* __restrict__ ranges_all, int causal,
    typename AccOf<T>::type scale) {
  using A = typename AccOf<T>::type;
  using MF = Mfma16<T>;
  using acc_t = typename MF::acc_t;
  constexpr int LD = AttnShape<T, K, D>::LD;
  constexpr int DB = D / 16;
  constexpr int SLICES = DB / NS;
  constexpr int V = 16 / sizeof(T);
  constexpr int kBM = 16;
  constexpr int kBK = kAttnWaves * 16;
  static_assert(kBK == kAttnRangeBlock, "key blocks are the mask-range blocks");
  constexpr bool DO_V = (WHAT & 1) != 0;
  constexpr bool DO_K = (WHAT & 2) != 0;

  __shared__ T Gs[DO_V ? K + 1 : 1][kBM][LD];
  __shared__ T Qs[DO_K ? K + 1 : 1][kBM][LD];

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int c = lane % 16;
  const int h = lane / 16;
  const int nkb = (S + kBK - 1) / kBK;
  const int64_t bh = gridDim.x / (static_cast<int64_t>(nkb) * SLICES);
  int64_t head;
  int slice, kv_block;
  attn_bwd_kv_item(blockIdx.x, bh, SLICES, head, slice, kv_block);
  // this head's mask, its block ranges (and additive values)
  const int64_t mask_index = attn_mask_index(mmap, head);
  const uint8_t* mask = mask_all != nullptr ? mask_all + mask_index * L * S : nullptr;
  const int32_t* ranges = ranges_all != nullptr ? ranges_all + mask_index * attn_ranges_count(L, S) : nullptr;
  const int my_k = kv_block + wave * 16 + c;
  const bool k_ok = my_k < S;
  const int nqt = (L + 15) / 16, nkt = (S + 15) / 16;
  static_assert(sizeof(T) == 4, "the tile layout follows the float accumulator layout (acc_row = 4h + r)");
  const int kt = min(kv_block / 16 + wave, nkt - 1);   // a wave past S reads a valid tile, all masked

  acc_t acc_v[DO_V ? K + 1 : 1][NS], acc_k[DO_K ? K + 1 : 1][NS];
#pragma unroll
  for (int n = 0; n < NS; ++n) {
#pragma unroll
    for (int o = 0; o < (DO_V ? K + 1 : 1); ++o) acc_v[o][n] = MF::zero();
#pragma unroll
    for (int o = 0; o < (DO_K ? K + 1 : 1); ++o) acc_k[o][n] = MF::zero();
  }

  int lo, hi;
  attn_query_range(L, kv_block, causal, ranges, lo, hi);
  // Block qb0+16's rows and tile values are fetched into registers while block
  // qb0's MFMAs run (register double buffering of the staging).
  RowStager<T, K, D, kBM> stage_g, stage_q;
  Vec<T, 4> pn[DO_V ? K + 1 : 1], sn[DO_K ? K + 1 : 1];   // next block's tile values
  auto fetch = [&](int qb) {
    const int64_t at = attn_tile_consumer_offset(head, qb / 16, kt, nqt, nkt, c, h);
#pragma unroll
    for (int o = 0; o <= K; ++o) {
      if constexpr (DO_V) pn[o] = *reinterpret_cast<const Vec<T, 4>*>(PT.p[o] + at);
      if constexpr (DO_K) sn[o] = *reinterpret_cast<const Vec<T, 4>*>(DST.p[o] + at);
    }
    if constexpr (DO_V) stage_g.fetch(G, head * L, qb, L);
    if constexpr (DO_K) stage_q.fetch(Q, head * L, qb, L);
  };
  if (lo < hi) fetch(lo);
  for (int qb0 = lo; qb0 < hi; qb0 += kBM) {
    Vec<T, 4> pv[DO_V ? K + 1 : 1], sv[DO_K ? K + 1 : 1];
#pragma unroll
    for (int o = 0; o <= K; ++o) {
      if constexpr (DO_V) pv[o] = pn[o];
      if constexpr (DO_K) sv[o] = sn[o];
    }
    __syncthreads();   // the previous block's MFMAs are done with the tiles
    if constexpr (DO_V) stage_g.commit(Gs);
    if constexpr (DO_K) stage_q.commit(Qs);
    __syncthreads();
    uint8_t mbyte[MASKED ? 4 : 1];   // mask bytes of this block's queries, read ahead of the prefetch
    if constexpr (MASKED) {
#pragma unroll
      for (int sidx = 0; sidx < 4; ++sidx)
        mbyte[sidx] = attn_mask_byte(mask, Q.p[0], qb0 + MF::acc_row(h, sidx), my_k, L, S);
    }
    if (qb0 + kBM < hi) fetch(qb0 + kBM);
    __builtin_amdgcn_sched_barrier(0);   // keep the prefetch ahead of this block's MFMAs

#pragma unroll
    for (int sidx = 0; sidx < 4; ++sidx) {
      const int q = qb0 + MF::acc_row(h, sidx);
      bool ok = k_ok && q < L;
      if (causal) ok = ok && my_k <= q;
      if constexpr (MASKED) ok = ok && mbyte[sidx] != 0;
#pragma unroll
      for (int o = 0; o <= K; ++o) {
        if constexpr (DO_V) pv[o].v[sidx] = ok ? pv[o].v[sidx] : T(0);
        if constexpr (DO_K) sv[o].v[sidx] = ok ? sv[o].v[sidx] : T(0);
      }
    }

    if constexpr (DO_V)
      attn_lds_products<T, K, NS>(acc_v, Gs, slice * NS, c, h, [&](int a, int sidx) { return pv[a].v[sidx]; });
    if constexpr (DO_K)
      attn_lds_products<T, K, NS>(acc_k, Qs, slice * NS, c, h, [&](int a, int sidx) { return sv[a].v[sidx]; });
  }

  if (!k_ok) return;
  const int64_t row = (head * S + my_k) * D;
  if constexpr (DO_V) attn_bwd_store<T, K, NS>(acc_v, DV, row, slice * NS, h, A(1));
  if constexpr (DO_K) attn_bwd_store<T, K, NS>(acc_k, DK, row, slice * NS, h, scale);
}

template <typename T, int K, int D>
static int launch_attention_bwd_kd(const AttnBwdArgs& a) {
  using A = typename AccOf<T>::type;
  using Plan = AttnBwdPlan<T, K, D>;
  if constexpr (!Plan::fits) {
    pt_host::set_error("Taylor attention backward: degree and head dim exceed the LDS budget for this dtype");
    return PT_UNSUPPORTED;
  } else {
    CPtrs<T> q{}, k{}, v{}, o{}, g{};
    CPtrs<A> lse{}, delta_in{};
    MPtrs<A> delta{};
    MPtrs<T> dq{}, dk{}, dv{};
    const int64_t rows = a.bh * a.lq;
    for (int i = 0; i <= K; ++i) {
      q.p[i] = static_cast<const T*>(a.q[i]);
      k.p[i] = static_cast<const T*>(a.k[i]);
      v.p[i] = static_cast<const T*>(a.v[i]);
      o.p[i] = static_cast<const T*>(a.out[i]);
      g.p[i] = static_cast<const T*>(a.grad[i]);
      lse.p[i] = static_cast<const A*>(a.lse[i]);
      delta.p[i] = static_cast<A*>(a.workspace) + i * rows;
      delta_in.p[i] = delta.p[i];
      if (a.dq != nullptr) dq.p[i] = static_cast<T*>(a.dq[i]);
      if (a.dk != nullptr) dk.p[i] = static_cast<T*>(a.dk[i]);
      if (a.dv != nullptr) dv.p[i] = static_cast<T*>(a.dv[i]);
    }
    const int L = static_cast<int>(a.lq), S = static_cast<int>(a.lk);
    const A scale = static_cast<A>(a.scale);
    const int causal = a.causal ? 1 : 0;
    // the stored-tile path is built for float32 only (the C ABI refuses it for float64); with an
    // additive mask the scores are recomputed
    constexpr bool kCanStore = sizeof(T) == 4;
    if (!kCanStore && a.materialize) {
      pt_host::set_error("Taylor attention backward: materialize is float32 only");
      return PT_UNSUPPORTED;
    }
    const bool materialize = a.materialize && a.mask_add == nullptr;
    const A* madd = static_cast<const A*>(a.mask_add);
    MPtrs<T> pt{}, dst{};
    CPtrs<T> pt_in{}, dst_in{};
    if (materialize) {
      const AttnBwdLayout lay = attention_bwd_layout(sizeof(A), sizeof(T), K, a.bh, a.lq, a.lk);
      for (int i = 0; i <= K; ++i) {
        pt.p[i] = reinterpret_cast<T*>(static_cast<char*>(a.workspace) + lay.tiles_offset + i * lay.tile_bytes);
        dst.p[i] = reinterpret_cast<T*>(static_cast<char*>(a.workspace) + lay.tiles_offset +
                                        (K + 1 + i) * lay.tile_bytes);
        pt_in.p[i] = pt.p[i];
        dst_in.p[i] = dst.p[i];
      }
    }
    if (rows > 0) {
      attn_bwd_delta_kernel<T, K, D><<<dim3(static_cast<unsigned>((rows + 15) / 16)), dim3(256), 0, a.stream>>>(
          g, o, delta, rows);
      PT_LAUNCH_CHECK();
    }
    const bool need_q = a.dq != nullptr || materialize;
    if (need_q && rows > 0) {
      constexpr int SL = Plan::DB / Plan::NS_Q;
      const dim3 grid(static_cast<unsigned>((a.lq + kAttnBM - 1) / kAttnBM * a.bh * SL));
#define PT_ATTN_BWD_Q(STORE, MASK)                                                                     \
  taylor_attention_bwd_q_kernel<T, K, D, Plan::NS_Q, STORE, MASK><<<grid, dim3(kAttnWaves * kWave), 0, a.stream>>>( \
      q, k, v, g, lse, delta_in, dq, pt, dst, L, S, a.mask, a.mask_map, madd, a.mask_ranges, causal, scale)
      const bool masked = a.mask != nullptr;
      if constexpr (kCanStore) {
        if (materialize) {   // (without a dq output the kernel still writes the P and dS tiles)
          if (masked) PT_ATTN_BWD_Q(true, 1);
          else PT_ATTN_BWD_Q(true, 0);
        }
      }
      if (!materialize) {
        if (madd != nullptr) PT_ATTN_BWD_Q(false, 2);
        else if (masked) PT_ATTN_BWD_Q(false, 1);
        else PT_ATTN_BWD_Q(false, 0);
      }
#undef PT_ATTN_BWD_Q
      PT_LAUNCH_CHECK();
    }
    if ((a.dk != nullptr || a.dv != nullptr) && a.lk > 0) {
      const dim3 block(kAttnWaves * kWave);
      // the fused pass writes both outputs: with one of them not wanted (NULL) that one's pass runs alone
      const bool both = a.dk != nullptr && a.dv != nullptr;
#define PT_ATTN_BWD_KV(KERNEL, NS, WHAT, ARGS)                                      \
  do {                                                                              \
    if (a.mask != nullptr) KERNEL<T, K, D, NS, WHAT, true><<<grid, block, 0, a.stream>>> ARGS; \
    else KERNEL<T, K, D, NS, WHAT, false><<<grid, block, 0, a.stream>>> ARGS;                  \
  } while (0)
#define PT_ATTN_BWD_KV_RECOMPUTE(WHAT)                                                                       \
  do {                                                                                                       \
    if (madd != nullptr)                                                                                     \
      taylor_attention_bwd_kv_kernel<T, K, D, Plan::NS_KV, WHAT, 2><<<grid, block, 0, a.stream>>>(           \
          q, k, v, g, lse, delta_in, dk, dv, L, S, a.mask, a.mask_map, madd, a.mask_ranges, causal, scale);              \
    else if (a.mask != nullptr)                                                                              \
      taylor_attention_bwd_kv_kernel<T, K, D, Plan::NS_KV, WHAT, 1><<<grid, block, 0, a.stream>>>(           \
          q, k, v, g, lse, delta_in, dk, dv, L, S, a.mask, a.mask_map, madd, a.mask_ranges, causal, scale);              \
    else                                                                                                     \
      taylor_attention_bwd_kv_kernel<T, K, D, Plan::NS_KV, WHAT, 0><<<grid, block, 0, a.stream>>>(           \
          q, k, v, g, lse, delta_in, dk, dv, L, S, a.mask, a.mask_map, madd, a.mask_ranges, causal, scale);              \
  } while (0)
      if (materialize) {
       if constexpr (kCanStore) {
        constexpr int SL = Plan::DB / Plan::NS_KM;
        const dim3 grid(static_cast<unsigned>((a.lk + 63) / 64 * a.bh * SL));
        bool fused = false;
        if constexpr (Plan::km_fused) {
          if (both) {
            PT_ATTN_BWD_KV(taylor_attention_bwd_kv_mat_kernel, Plan::NS_KM, 3, (q, g, pt_in, dst_in, dk, dv, L, S, a.mask, a.mask_map, a.mask_ranges, causal, scale));
            PT_LAUNCH_CHECK();
            fused = true;
          }
        }
        if (!fused) {
          if (a.dv != nullptr) {
            PT_ATTN_BWD_KV(taylor_attention_bwd_kv_mat_kernel, Plan::NS_KM, 1, (q, g, pt_in, dst_in, dk, dv, L, S, a.mask, a.mask_map, a.mask_ranges, causal, scale));
            PT_LAUNCH_CHECK();
          }
          if (a.dk != nullptr) {
            PT_ATTN_BWD_KV(taylor_attention_bwd_kv_mat_kernel, Plan::NS_KM, 2, (q, g, pt_in, dst_in, dk, dv, L, S, a.mask, a.mask_map, a.mask_ranges, causal, scale));
            PT_LAUNCH_CHECK();
          }
        }
       }
      } else {
        constexpr int SL = Plan::DB / Plan::NS_KV;
        const dim3 grid(static_cast<unsigned>((a.lk + 63) / 64 * a.bh * SL));
        bool fused = false;
        if constexpr (Plan::kv_fused) {
          if (both) {
            PT_ATTN_BWD_KV_RECOMPUTE(3);
            PT_LAUNCH_CHECK();
            fused = true;
          }
        }
        if (!fused) {
          if (a.dv != nullptr) {
            PT_ATTN_BWD_KV_RECOMPUTE(1);
            PT_LAUNCH_CHECK();
          }
          if (a.dk != nullptr) {
            PT_ATTN_BWD_KV_RECOMPUTE(2);
            PT_LAUNCH_CHECK();
          }
        }
      }
#undef PT_ATTN_BWD_KV
#undef PT_ATTN_BWD_KV_RECOMPUTE
    }
    return PT_OK;
  }
}

template <typename T, int K>
static int launch_attention_bwd_k(const AttnBwdArgs& a) {
  switch (a.d) {
    case 16: return launch_attention_bwd_kd<T, K, 16>(a);
    case 32: return launch_attention_bwd_kd<T, K, 32>(a);
    case 64: return launch_attention_bwd_kd<T, K, 64>(a);
    case 128: return launch_attention_bwd_kd<T, K, 128>(a);
    default: break;
  }
  pt_host::set_error("Taylor attention backward: head dim must be 16, 32, 64 or 128");
  return PT_UNSUPPORTED;
}

template <typename T>
int launch_attention_bwd(const AttnBwdArgs& a) {
  switch (a.degree) {
    case 0: return launch_attention_bwd_k<T, 0>(a);
    case 1: return launch_attention_bwd_k<T, 1>(a);
    case 2: return launch_attention_bwd_k<T, 2>(a);
    case 3: return launch_attention_bwd_k<T, 3>(a);
    case 4: return launch_attention_bwd_k<T, 4>(a);
    case 5: return launch_attention_bwd_k<T, 5>(a);
    case 6: return launch_attention_bwd_k<T, 6>(a);
    case 7: return launch_attention_bwd_k<T, 7>(a);
    case 8: return launch_attention_bwd_k<T, 8>(a);
    default: break;
  }
  pt_host::set_error("Taylor attention backward: degree outside 0..PT_MAX_DEGREE");
  return PT_UNSUPPORTED;
}

}  // namespace pt
