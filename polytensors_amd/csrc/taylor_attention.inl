// Flash-style attention forward of degree-K series on MFMA (gfx950).
//
// Per query row, with score series S(t) = scale Q(t) K(t)^T:
//   exp(S(t)) = exp(S_0) e(t),  e_0 = 1,  e_k = sum_{j=1..k} (j/k) S_j e_{k-j}
// (the exponential-series recurrence of /root/reference/src/polytensors/_plain.py:153-159),
//   l_k = sum_keys exp(S_0 - m) e_k,   N_k = sum_keys sum_{a+b=k} exp(S_0 - m) e_a V_b,
//   O(t) = N(t) / l(t):  O_0 = N_0 / l_0,  O_k = (N_k - sum_{j=1..k} l_j O_{k-j}) / l_0,
// which equals softmax(S(t)) V(t) of the reference's decomposition
// (/root/reference/src/polytensors/_decompositions.py:28-43) since the softmax
// series is exp(S(t)) divided by its row sum. The running maximum m uses the
// constant order only and is raised lazily (only when a block's maximum
// exceeds it by more than kRescaleSlack), rescaling l and N by exp(m_old - m_new).
//
// Work decomposition: a workgroup of 4 waves owns 64 query rows of one (batch,
// head); each wave owns 16 queries. Key blocks of 16 keys of every order of K
// and V are staged in LDS. Scores are formed transposed, S^T = K Q^T, with
// 16x16x4 MFMAs (keys on the M side, queries on the N side, head dim
// contracted): the accumulator then holds, per lane, one query column and four
// keys, which is exactly the B operand layout of the value product
// O^T = V^T P^T. So the exponential series is computed in place in the score
// accumulators and fed straight to the PV MFMAs: P never leaves registers.
// Query operands are read from global memory (L2-resident) per 16-wide
// head-dim chunk; within a chunk the head-dim index is permuted so that a lane
// reads its 4 operand values with one 16-byte load (same permutation on K).
// The output accumulators O^T_k (16 head-dim rows x 16 queries per MFMA block)
// stay in registers for the whole key loop.
#pragma once

#include <type_traits>

#include "mfma.h"
#include "taylor_attention.h"

namespace pt {

// 16x16x4 MFMA for float (fp32) and double (fp64): same shape, different accumulator layouts.
template <typename T>
struct Mfma16;

template <>
struct Mfma16<float> {
  using acc_t = floatx4;
  __device__ __forceinline__ static acc_t zero() { return acc_t{0.f, 0.f, 0.f, 0.f}; }
  __device__ __forceinline__ static acc_t mma(float a, float b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
  // accumulator register r of lane l: row 4 (l/16) + r, column l % 16
  __host__ __device__ __forceinline__ static int acc_row(int h, int r) { return 4 * h + r; }
  // the lane group and register holding row i
  __host__ __device__ __forceinline__ static int row_group(int i) { return i / 4; }
  __host__ __device__ __forceinline__ static int row_reg(int i) { return i % 4; }
};

template <>
struct Mfma16<double> {
  using acc_t = doublex4;
  __device__ __forceinline__ static acc_t zero() { return acc_t{0.0, 0.0, 0.0, 0.0}; }
  __device__ __forceinline__ static acc_t mma(double a, double b, acc_t c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
  }
  // accumulator register r of lane l: row 4 r + l/16, column l % 16
  __host__ __device__ __forceinline__ static int acc_row(int h, int r) { return 4 * r + h; }
  __host__ __device__ __forceinline__ static int row_group(int i) { return i % 4; }
  __host__ __device__ __forceinline__ static int row_reg(int i) { return i / 4; }
};


template <typename T>
struct AttnRescale {
  static constexpr float value = 8.0f;   // lazy-rescale slack (natural-log units): p <= e^8
};

// The largest divisor of `per` (vectors per thread of a staging step) up to `most`: the loads
// of a staging step go out in groups of that many.
constexpr int attn_stage_group(int per, int most) {
  int g = most < per ? most : per;
  while (g > 1 && per % g != 0) --g;
  return g < 1 ? 1 : g;
}

template <typename T, int K, int D>
struct AttnShape {
  static constexpr int SL = attn_slices(static_cast<int>(sizeof(T)), K, D);
  static constexpr int DS = D / SL;    // output head dims per slice
  static constexpr int DBS = DS / 16;  // 16-wide output blocks per slice
  // Row stride of the staged K/V tiles: D + 4 values. For floats that is 4 mod 64
  // banks, so the 16 key rows of a 16-byte K-operand read and the 4 key rows of
  // a V-operand read fall on distinct banks; for doubles it keeps rows 32-byte aligned.
  static constexpr int LD = D + 4;
  static constexpr int LDV = DS + 4;   // V tile row: the slice's dims
  static constexpr size_t KT = static_cast<size_t>(K + 1) * kAttnBN * LD;    // K tile values
  static constexpr size_t VT = static_cast<size_t>(K + 1) * kAttnBN * LDV;   // V tile values
  // K and V tiles one after the other in one buffer when both do not fit (staged between the
  // score and value products of each key block)
  static constexpr bool SEQ = (KT + VT) * sizeof(T) > 160 * 1024;
  static constexpr size_t LDS = (SEQ ? (KT > VT ? KT : VT) : KT + VT) * sizeof(T);
  static constexpr bool fits = LDS <= 160 * 1024;
  // Query operands read one head-dim chunk ahead, and the 16-byte vectors per thread whose
  // loads a staging step issues before their LDS stores, where the registers allow
  // (instantiations checked free of scratch spills with the compiler's resource remarks).
  static constexpr int kAccRegs = (K + 1) * DBS * 4 * static_cast<int>(sizeof(T) / 4);
  static constexpr bool kQAhead = K <= 4 && kAccRegs <= 160;
  static constexpr int kStageGroup = kAccRegs > 160 ? 1 : 8;
};

// Shared epilogue: row sums across the 4 lane groups, series quotient
// O_k = (N_k - sum_{j=1..k} l_j O_{k-j}) / l_0, and the lse series.
// Work item of a workgroup in a one-dimensional grid of (query blocks) x (heads).
// Causal work grows with the query block, so the heaviest blocks are issued
// first; consecutive workgroup ids go to consecutive XCDs, and taking the head
// as the fast index gives every XCD an equal share of each query-block level
// (the same eight-head residue class on each XCD, which also keeps its K/V
// rows in that XCD's L2).
// Workgroups are dispatched round-robin over the 8 XCDs (workgroup t to XCD t % 8),
// each with its own L2. Causal: heads run fastest and the heaviest query blocks
// go first across the whole grid, so the launch ends on light blocks. Otherwise
// (query blocks of equal work), when the head count is a multiple of 8, XCD x
// takes heads x, x + 8, ... one after another with all query blocks of a head
// together, which then read the head's K/V rows from one L2 at about the same
// time (1.7% faster on a sliding window; grouping causal blocks this way was
// 8.5% slower, the XCDs ending on heavy blocks).
constexpr int kXcds = 8;
// Work item t of `items` (query blocks x heads).
__device__ __forceinline__ void attn_work_item_at(int L, int causal, int64_t t, int64_t items, int64_t& head,
                                                  int& q_block) {
  const int nqb = (L + kAttnBM - 1) / kAttnBM;
  const int64_t bh = items / nqb;
  if (!causal && bh % kXcds == 0) {
    const int64_t j = t / kXcds;
    head = t % kXcds + kXcds * (j / nqb);
    q_block = (nqb - 1 - static_cast<int>(j % nqb)) * kAttnBM;   // last (in masks, often fullest) first
  } else {
    head = t % bh;
    q_block = (nqb - 1 - static_cast<int>(t / bh)) * kAttnBM;
  }
}
__device__ __forceinline__ void attn_work_item(int L, int causal, int64_t& head, int& q_block) {
  attn_work_item_at(L, causal, blockIdx.x, gridDim.x, head, q_block);
}

// Block ranges of a boolean (L, S) mask, the reference's _mask_ranges
// (/root/reference/src/polytensors/_fused_attention.py:81-99) at this build's
// block sizes: for each 64-row query block the first and one-past-last key
// admissible for any of its rows, then for each 64-key block the first and
// one-past-last query admitting any of its keys; (0, 0) for a block with none.
// The attention kernels skip the key (query) blocks outside these ranges.
// One workgroup per block; the mask is read once per block set.
constexpr int kAttnRangeBlock = 64;

template <int Unused = 0>   // a template: this header is included by several translation units
__global__ __launch_bounds__(256) void attn_mask_ranges_kernel(const uint8_t* __restrict__ masks, int L, int S,
                                                               int32_t* __restrict__ all_ranges) {
  // mask blockIdx.y of the [n, L, S] set, its ranges at blockIdx.y * attn_ranges_count(L, S)
  const uint8_t* __restrict__ mask = masks + static_cast<int64_t>(blockIdx.y) * L * S;
  int32_t* __restrict__ ranges = all_ranges + static_cast<int64_t>(blockIdx.y) * attn_ranges_count(L, S);
  __shared__ int lo_s, hi_s;
  const int nqb = (L + kAttnRangeBlock - 1) / kAttnRangeBlock;
  const int b = blockIdx.x;
  if (threadIdx.x == 0) {
    lo_s = INT32_MAX;
    hi_s = -1;
  }
  __syncthreads();
  int lo = INT32_MAX, hi = -1;
  // 16-byte reads where the rows allow them (S % 16 == 0, aligned mask): a chunk
  // with any nonzero byte gives its first and last such byte from the four words
  const bool vec = S % 16 == 0 && (reinterpret_cast<uintptr_t>(mask) & 15u) == 0;
  auto chunk_bounds = [](const uint4 w, int& first, int& last) {
    const uint32_t v[4] = {w.x, w.y, w.z, w.w};
    first = 16;
    last = -1;
#pragma unroll
    for (int i = 3; i >= 0; --i)
      if (v[i] != 0) first = 4 * i + __builtin_ctz(v[i]) / 8;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (v[i] != 0) last = 4 * i + (31 - __builtin_clz(v[i])) / 8;
  };
  if (vec && b < nqb) {
    const int r0 = b * kAttnRangeBlock, nr = min(kAttnRangeBlock, L - r0);
    const int cpr = S / 16;   // chunks per row
#pragma unroll 8
    for (int idx = threadIdx.x; idx < nr * cpr; idx += 256) {
      const int r = idx / cpr, ch = idx % cpr;
      const uint4 w = *reinterpret_cast<const uint4*>(mask + static_cast<int64_t>(r0 + r) * S + ch * 16);
      int first, last;
      chunk_bounds(w, first, last);
      if (last >= 0) {
        lo = min(lo, ch * 16 + first);
        hi = max(hi, ch * 16 + last);
      }
    }
  } else if (vec) {
    // key block of 64 columns: four 16-byte chunks of each row (all inside S, as S % 16 == 0)
    const int c0 = (b - nqb) * kAttnRangeBlock;
    const int col0 = c0 + (threadIdx.x % 4) * 16;
    if (col0 < S) {
#pragma unroll 8
      for (int r = threadIdx.x / 4; r < L; r += 64) {
        const uint4 w = *reinterpret_cast<const uint4*>(mask + static_cast<int64_t>(r) * S + col0);
        if ((w.x | w.y | w.z | w.w) != 0) {
          lo = min(lo, r);
          hi = max(hi, r);
        }
      }
    }
  } else if (b < nqb) {
    const int r0 = b * kAttnRangeBlock, nr = min(kAttnRangeBlock, L - r0);
    for (int r = 0; r < nr; ++r) {
      const uint8_t* row = mask + static_cast<int64_t>(r0 + r) * S;
#pragma unroll 8
      for (int col = threadIdx.x; col < S; col += 256) {
        if (row[col] != 0) {
          lo = min(lo, col);
          hi = max(hi, col);
        }
      }
    }
  } else {
    const int c0 = (b - nqb) * kAttnRangeBlock, nc = min(kAttnRangeBlock, S - c0);
    const int col = threadIdx.x % kAttnRangeBlock;
    if (col < nc) {
#pragma unroll 8
      for (int r = threadIdx.x / kAttnRangeBlock; r < L; r += 256 / kAttnRangeBlock) {
        if (mask[static_cast<int64_t>(r) * S + c0 + col] != 0) {
          lo = min(lo, r);
          hi = max(hi, r);
        }
      }
    }
  }
#pragma unroll
  for (int off = kWave / 2; off >= 1; off >>= 1) {
    lo = min(lo, __shfl_xor(lo, off, kWave));
    hi = max(hi, __shfl_xor(hi, off, kWave));
  }
  if (threadIdx.x % kWave == 0) {
    atomicMin(&lo_s, lo);   // LDS atomics
    atomicMax(&hi_s, hi);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const bool any = hi_s >= 0;
    ranges[2 * b] = any ? lo_s : 0;
    ranges[2 * b + 1] = any ? hi_s + 1 : 0;
  }
}

// Key range [lo, hi) a query workgroup visits: causal and mask-range bounds,
// lo rounded down to a key block. (Host-callable: the index checks replay it.)
__host__ __device__ __forceinline__ void attn_key_range(int S, int q_block, int causal, const int32_t* ranges,
                                                        int& lo, int& hi) {
  lo = 0;
  hi = S;
  if (causal) hi = S < q_block + kAttnBM ? S : q_block + kAttnBM;
  if (ranges != nullptr) {
    const int qb = q_block / kAttnRangeBlock;
    lo = ranges[2 * qb] / kAttnBN * kAttnBN;
    const int rh = static_cast<int>(ranges[2 * qb + 1]);
    hi = hi < rh ? hi : rh;
  }
}

// Byte (row, col) of an (L, S) boolean mask, read unconditionally: indices are
// clamped into the mask and without a mask a valid dummy byte is read (the
// caller ignores it). Callers issue these reads ahead of their prefetches: a
// load under a per-lane branch, or one issued after a prefetch and used soon,
// makes the compiler wait for every load in flight (memory waits complete in
// order).
__device__ __forceinline__ uint8_t attn_mask_byte(const uint8_t* mask, const void* dummy, int row, int col, int L,
                                                  int S) {
  const uint8_t* base = mask != nullptr ? mask : static_cast<const uint8_t*>(dummy);
  const int64_t at = mask != nullptr ? static_cast<int64_t>(min(row, L - 1)) * S + min(col, S - 1) : 0;
  return base[at];
}

// Value (row, col) of an (L, S) additive mask (the accumulator type), indices clamped into it
// as attn_mask_byte's. Its -inf entries are also 0 in the boolean mask the launch is given, so a
// read value is used for admissible keys only.
template <typename A>
__device__ __forceinline__ A attn_mask_add(const A* madd, int row, int col, int L, int S) {
  return madd[static_cast<int64_t>(min(row, L - 1)) * S + min(col, S - 1)];
}

// The mask bytes of keys k0 .. k0+3 of row `row` (k0 a multiple of 4) as one word, byte r for key
// k0 + r, and with ADD their additive values. Where vec holds (attn_mask_vec: S a multiple of 4,
// the mask 4-byte and the values 16-byte aligned) that is one 4-byte and one 16-byte load: k0 < S
// then implies k0 + 3 < S, and a group at or past S reads the row's last four keys, whose values
// are never used (those keys fail key < hi). Otherwise byte by byte, indices clamped as
// attn_mask_byte's.
template <bool ADD>
__device__ __forceinline__ uint32_t attn_mask_word4(const uint8_t* mask, const float* madd, int row, int k0, int L,
                                                    int S, bool vec, float (&add)[4]) {
  const int64_t at = static_cast<int64_t>(min(row, L - 1)) * S;
  if (vec) {
    const int kc = min(k0, S - 4);
    if constexpr (ADD) {
      const float4 v = *reinterpret_cast<const float4*>(madd + at + kc);
      add[0] = v.x;
      add[1] = v.y;
      add[2] = v.z;
      add[3] = v.w;
    }
    return *reinterpret_cast<const uint32_t*>(mask + at + kc);
  }
  uint32_t w = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t e = at + min(k0 + r, S - 1);
    w |= static_cast<uint32_t>(mask[e]) << (8 * r);
    if constexpr (ADD) add[r] = madd[e];
  }
  return w;
}
__device__ __forceinline__ bool attn_mask_vec(const uint8_t* mask, const float* madd, int S) {
  return mask != nullptr && S % 4 == 0 && (reinterpret_cast<uintptr_t>(mask) & 3) == 0 &&
         (madd == nullptr || (reinterpret_cast<uintptr_t>(madd) & 15) == 0);
}

// E is the head-dim interleave of the output accumulators: accumulator
// g*E + e, register r of lane group h holds column g*16E + E*(4h + r) + e
// (E = 1: the plain 16x16 layout, column 16 db + acc_row(h, r)).
// The accumulators hold NB 16-wide output blocks from head dim d0 on (a slice of the
// D head dims); the lse series is written where write_lse holds (one slice).
template <typename T, int K, int D, typename AccT, int E = 1, int NB = D / 16>
__device__ __forceinline__ void attention_epilogue(AccT (&acc_o)[K + 1][NB],
                                                   typename AccOf<T>::type (&lsum)[K + 1],
                                                   typename AccOf<T>::type m_used, MPtrs<T>& O,
                                                   MPtrs<typename AccOf<T>::type>& LSE, int64_t head,
                                                   int L, int my_q, bool q_ok, int h, int d0 = 0,
                                                   bool write_lse = true) {
  using A = typename AccOf<T>::type;
  using MF = Mfma16<T>;
  constexpr int DB = NB;
  static_assert(E == 1 || NB == D / 16, "interleaved accumulators span the whole head dim");
#pragma unroll
  for (int o = 0; o <= K; ++o) {
    lsum[o] = rows_sum(lsum[o]);
  }
  if (!q_ok) return;
  const bool empty = !(lsum[0] > A(0));
  const A inv_l0 = empty ? A(0) : A(1) / lsum[0];
  if constexpr (E > 1) {
    static_assert(sizeof(T) == 4, "interleaved accumulators are an fp32 layout");
#pragma unroll
    for (int g = 0; g < DB / E; ++g) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        A out[E][K + 1];
#pragma unroll
        for (int e = 0; e < E; ++e) {
#pragma unroll
          for (int k = 0; k <= K; ++k) {
            A t = static_cast<A>(acc_o[k][g * E + e][r]);
#pragma unroll
            for (int j = 1; j <= k; ++j) t -= lsum[j] * out[e][k - j];
            out[e][k] = t * inv_l0;
          }
        }
#pragma unroll
        for (int k = 0; k <= K; ++k) {
          Vec<T, E> w;
#pragma unroll
          for (int e = 0; e < E; ++e) w.v[e] = static_cast<T>(out[e][k]);
          store_vec<T, E>(O.p[k] + (head * L + my_q) * D + g * 16 * E + E * (4 * h + r), w);
        }
      }
    }
  }
#pragma unroll
  for (int db = 0; db < (E == 1 ? DB : 0); ++db) {
    A out[4][K + 1];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
      for (int k = 0; k <= K; ++k) {
        A t = static_cast<A>(acc_o[k][db][r]);
#pragma unroll
        for (int j = 1; j <= k; ++j) t -= lsum[j] * out[r][k - j];
        out[r][k] = t * inv_l0;
      }
    }
    T* orow = nullptr;
#pragma unroll
    for (int k = 0; k <= K; ++k) {
      orow = O.p[k] + (head * L + my_q) * D + d0 + db * 16;
      if constexpr (sizeof(T) == 4) {
        // fp32 layout: registers r = 0..3 hold head-dim columns 4h + r: one 16-byte store
        Vec<T, 4> w;
#pragma unroll
        for (int r = 0; r < 4; ++r) w.v[r] = static_cast<T>(out[r][k]);
        store_vec<T, 4>(orow + 4 * h, w);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) orow[MF::acc_row(h, r)] = static_cast<T>(out[r][k]);
      }
    }
  }
  if (LSE.p[0] != nullptr && h == 0 && write_lse) {
    const int64_t at = head * L + my_q;
    if (empty) {
      LSE.p[0][at] = __builtin_huge_val();
#pragma unroll
      for (int k = 1; k <= K; ++k) LSE.p[k][at] = A(0);
    } else {
      A lse[K + 1], nrm[K + 1];
      lse[0] = m_used + log_acc(lsum[0]);
#pragma unroll
      for (int k = 1; k <= K; ++k) nrm[k] = lsum[k] * inv_l0;
#pragma unroll
      for (int k = 1; k <= K; ++k) {
        A t = nrm[k];
#pragma unroll
        for (int j = 1; j < k; ++j) t -= (A(j) / A(k)) * lse[j] * nrm[k - j];
        lse[k] = t;
      }
#pragma unroll
      for (int k = 0; k <= K; ++k) LSE.p[k][at] = lse[k];
    }
  }
}

// The order-o pointer of a series for a per-lane o: selected among the kernel
// arguments (scalar registers) instead of indexing the argument array, which
// would load the pointer from memory and wait for it before the data load.
template <int K, typename T>
__device__ __forceinline__ const T* order_ptr(const CPtrs<T>& s, int o) {
  const T* p = s.p[0];
#pragma unroll
  for (int i = 1; i <= K; ++i) p = (o == i) ? s.p[i] : p;
  return p;
}

// ADD: an additive (L, S) mask madd is given with the boolean mask of its finite entries; it
// adds to the constant-order scores after scaling.
template <typename T, int K, int D, bool ADD>
__global__ __launch_bounds__(kAttnWaves * kWave) void taylor_attention_fwd_kernel(
    CPtrs<T> Q, int q_orders, CPtrs<T> Kp, int k_orders, CPtrs<T> Vp, int v_orders, MPtrs<T> O,
    MPtrs<typename AccOf<T>::type> LSE, int L, int S, const uint8_t* __restrict__ mask_all, AttnMaskMap mmap,
    const typename AccOf<T>::type* __restrict__ madd_all, const int32_t* __restrict__ ranges_all, int causal,
    typename AccOf<T>::type scale, int chunks, int chunk_keys, typename AccOf<T>::type* __restrict__ part) {
  using A = typename AccOf<T>::type;
  using MF = Mfma16<T>;
  using acc_t = typename MF::acc_t;
  using Shape = AttnShape<T, K, D>;
  constexpr int LD = Shape::LD, LDV = Shape::LDV, SL = Shape::SL, DS = Shape::DS;
  constexpr int DB = D / 16;                  // 16-wide head-dim chunks of the score contraction
  constexpr int DBS = Shape::DBS;             // 16-wide output blocks of this slice
  constexpr int V = 16 / sizeof(T);           // values per 16-byte load
  constexpr int QV = 4;                       // operand values per lane per 16-wide chunk
  constexpr A kNegInf = -__builtin_huge_val();
  constexpr A kSlack = AttnRescale<T>::value;
  static_assert(Shape::fits, "K/V tiles exceed LDS");

  // the K tile (every head dim) and the V tile (the slice's head dims); in one buffer, one after
  // the other within each key block, when both do not fit
  __shared__ __attribute__((aligned(16))) T tiles[Shape::LDS / sizeof(T)];
  T(*Ks)[kAttnBN][LD] = reinterpret_cast<T(*)[kAttnBN][LD]>(&tiles[0]);
  T(*Vs)[kAttnBN][LDV] = reinterpret_cast<T(*)[kAttnBN][LDV]>(&tiles[Shape::SEQ ? 0 : Shape::KT]);

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int c = lane % 16;        // query column of this lane (and key row for K operands)
  const int h = lane / 16;        // lane group
  int64_t head;
  int q_block, slice = 0;
  // key chunks fastest (chunks > 1: each workgroup takes one contiguous share of the key range
  // and writes unnormalised partial sums, attn_split_combine_kernel merges them), then slices,
  // then the work items
  const int chunk = static_cast<int>(blockIdx.x % chunks);
  const int64_t wi = blockIdx.x / chunks, items = gridDim.x / chunks;
  const int nqb = (L + kAttnBM - 1) / kAttnBM;
  const int64_t bh = items / (static_cast<int64_t>(nqb) * SL);
  if constexpr (SL == 1) {
    attn_work_item_at(L, causal, wi, items, head, q_block);
  } else {
    // slices fastest, then heads, heaviest query blocks first
    const int64_t t = wi / SL;
    slice = static_cast<int>(wi % SL);
    head = t % bh;
    q_block = (nqb - 1 - static_cast<int>(t / bh)) * kAttnBM;
  }
  const int d0 = slice * DS;   // first output head dim of this workgroup
  // this head's mask, its block ranges (and additive values)
  const int64_t mask_index = attn_mask_index(mmap, head);
  const uint8_t* mask = mask_all != nullptr ? mask_all + mask_index * L * S : nullptr;
  const int32_t* ranges = ranges_all != nullptr ? ranges_all + mask_index * attn_ranges_count(L, S) : nullptr;
  const typename AccOf<T>::type* madd = madd_all != nullptr ? madd_all + mask_index * L * S : nullptr;
  const int q0 = q_block + wave * kAttnQPerWave;
  const int my_q = q0 + c;
  const bool q_ok = my_q < L;

  // Every pair (a, b) runs unconditionally: an operand with fewer orders reads
  // zeros for the missing ones (selected after a load from a valid address), so
  // no branch splits the MFMA sequence.
  const T* qrow[K + 1];
  bool q_live[K + 1];
#pragma unroll
  for (int o = 0; o <= K; ++o) {
    q_live[o] = q_ok && o < q_orders;
    qrow[o] = Q.p[o < q_orders ? o : 0] + (head * L + (q_ok ? my_q : 0)) * D;
  }

  acc_t acc_o[K + 1][DBS];
#pragma unroll
  for (int o = 0; o <= K; ++o)
#pragma unroll
    for (int db = 0; db < DBS; ++db) acc_o[o][db] = MF::zero();
  A m_used = kNegInf;
  A lsum[K + 1];   // per-lane partial row sums (this lane's keys only)
#pragma unroll
  for (int o = 0; o <= K; ++o) lsum[o] = A(0);

  int lo, hi;
  attn_key_range(S, q_block, causal, ranges, lo, hi);
  if (chunks > 1) {   // this workgroup's share (chunk_keys is a multiple of the key block)
    lo += chunk * chunk_keys;
    hi = min(hi, lo + chunk_keys);
  }

  for (int kb0 = lo; kb0 < hi; kb0 += kAttnBN) {
    uint8_t mbyte[4];
    A add[ADD ? 4 : 1];
#pragma unroll
    for (int r = 0; r < 4; ++r) mbyte[r] = attn_mask_byte(mask, Q.p[0], my_q, kb0 + MF::acc_row(h, r), L, S);
    if constexpr (ADD) {
#pragma unroll
      for (int r = 0; r < 4; ++r) add[r] = attn_mask_add(madd, my_q, kb0 + MF::acc_row(h, r), L, S);
    }
    __syncthreads();
    // ---- stage rows kb0 .. kb0+15 of every order (zero past S / the orders given): K over every
    // head dim, V over the slice's (V after the scores when the two share the buffer) ----
    // Loads go out in groups of kStageGroup vectors per thread before their LDS stores, each
    // from a clamped (valid) address with the value zeroed afterwards: a load under a per-lane
    // branch would be waited for where the branch ends, one round trip per vector.
    auto stage = [&](auto dst, const CPtrs<T>& src, int orders, auto dims_c, int first) {
      constexpr int vpr = decltype(dims_c)::value / V;   // 16-byte vectors per row
      constexpr int total = (K + 1) * kAttnBN * vpr;
      constexpr int threads = kAttnWaves * kWave;
      constexpr int per = (total + threads - 1) / threads;
      constexpr int G = attn_stage_group(per, Shape::kStageGroup);
#pragma unroll 1
      for (int g0 = 0; g0 < per; g0 += G) {
        Vec<T, V> x[G];
        bool live[G];
#pragma unroll
        for (int j = 0; j < G; ++j) {
          const int idx = (g0 + j) * threads + static_cast<int>(threadIdx.x);
          const int o = idx / (kAttnBN * vpr);
          const int rem = idx % (kAttnBN * vpr);
          const int key = kb0 + rem / vpr, cv = (rem % vpr) * V;
          live[j] = (total % threads == 0 || idx < total) && key < S && o < orders;
          const int oc = o < orders ? o : 0, kc = key < S ? key : S - 1;
          x[j] = load_vec<T, V>(order_ptr<K>(src, oc) + (head * S + kc) * D + first + cv);
        }
#pragma unroll
        for (int j = 0; j < G; ++j) {
          const int idx = (g0 + j) * threads + static_cast<int>(threadIdx.x);
          if (total % threads != 0 && idx >= total) continue;
          const int o = idx / (kAttnBN * vpr);
          const int rem = idx % (kAttnBN * vpr);
#pragma unroll
          for (int e = 0; e < V; ++e) x[j].v[e] = live[j] ? x[j].v[e] : T(0);
          store_vec<T, V>(&dst[o][rem / vpr][(rem % vpr) * V], x[j]);
        }
      }
    };
    stage(Ks, Kp, k_orders, std::integral_constant<int, D>{}, 0);
    if constexpr (!Shape::SEQ) stage(Vs, Vp, v_orders, std::integral_constant<int, DS>{}, d0);
    __syncthreads();

    // ---- scores S^T_k = sum_{a+b=k} K_b Q_a^T (keys x queries) ----
    acc_t sc[K + 1];
#pragma unroll
    for (int o = 0; o <= K; ++o) sc[o] = MF::zero();
    // Not unrolled: no register array is indexed by dc, and a rolled loop keeps
    // the code (and compile time) of the high-degree instantiations small. The query
    // operands (global, L2-resident) are read one chunk ahead.
    Vec<T, QV> qn[Shape::kQAhead ? K + 1 : 1];
    if constexpr (Shape::kQAhead) {
#pragma unroll
      for (int o = 0; o <= K; ++o) qn[o] = *reinterpret_cast<const Vec<T, QV>*>(qrow[o] + 4 * h);
    }
#pragma unroll 1
    for (int dc = 0; dc < DB; ++dc) {
      // lane operands: K[key = c][d = 16 dc + 4 h + s], Q[my_q][same d], s = 0..3
      Vec<T, QV> qa[K + 1], kb[K + 1];
      const int dn = !Shape::kQAhead ? dc : dc + 1 < DB ? dc + 1 : dc;   // the next chunk (or this one)
#pragma unroll
      for (int o = 0; o <= K; ++o) {
        if constexpr (Shape::kQAhead) {
          qa[o] = qn[o];
          qn[o] = *reinterpret_cast<const Vec<T, QV>*>(qrow[o] + dn * 16 + 4 * h);
        } else {
          qa[o] = *reinterpret_cast<const Vec<T, QV>*>(qrow[o] + dc * 16 + 4 * h);
        }
#pragma unroll
        for (int e = 0; e < QV; ++e) qa[o].v[e] = q_live[o] ? qa[o].v[e] : T(0);
        kb[o] = *reinterpret_cast<const Vec<T, QV>*>(&Ks[o][c][dc * 16 + 4 * h]);
      }
#pragma unroll
      for (int s = 0; s < QV; ++s) {
#pragma unroll
        for (int k = 0; k <= K; ++k) {
#pragma unroll
          for (int a = 0; a <= k; ++a) sc[k] = MF::mma(kb[k - a].v[s], qa[a].v[s], sc[k]);
        }
      }
    }

    // ---- mask, online maximum of the constant order, exponential series ----
    bool valid[4];
    A s0[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int key = kb0 + MF::acc_row(h, r);
      bool ok = q_ok && key < S;
      if (causal) ok = ok && key <= my_q;
      if (mask != nullptr) ok = ok && mbyte[r] != 0;
      valid[r] = ok;
      A s = static_cast<A>(sc[0][r]) * scale;
      if constexpr (ADD) s += add[r];
      s0[r] = ok ? s : kNegInf;
    }
    A bmax = fmax(fmax(s0[0], s0[1]), fmax(s0[2], s0[3]));
    bmax = rows_max(bmax);
    const bool raise = bmax > m_used + kSlack || (m_used == kNegInf && bmax != kNegInf);
    if (__any(raise)) {
      const A m_new = raise ? bmax : m_used;
      const A alpha = (raise && m_used != kNegInf) ? exp_fast(m_used - m_new) : (raise ? A(0) : A(1));
#pragma unroll
      for (int o = 0; o <= K; ++o) {
        lsum[o] *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc_o[o][db][r] *= alpha;
      }
      m_used = m_new;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const A p = valid[r] ? exp_fast(s0[r] - m_used) : A(0);
      A sk[K + 1], e[K + 1];
#pragma unroll
      for (int o = 1; o <= K; ++o) sk[o] = static_cast<A>(sc[o][r]) * scale;
      e[0] = A(1);
#pragma unroll
      for (int k = 1; k <= K; ++k) {
        A t = A(0);
#pragma unroll
        for (int j = 1; j <= k; ++j) t += (A(j) * sk[j]) * e[k - j];
        e[k] = t * (A(1) / A(k));   // a compile-time reciprocal, not a division
      }
#pragma unroll
      for (int o = 0; o <= K; ++o) {
        const A w = p * e[o];
        lsum[o] += w;
        sc[o][r] = static_cast<T>(w);
      }
    }

    if constexpr (Shape::SEQ) {
      __syncthreads();   // every wave's scores are done with the K tile
      stage(Vs, Vp, v_orders, std::integral_constant<int, DS>{}, d0);
      __syncthreads();
    }

    // ---- O^T_k += sum_{a+b=k} V_b^T E_a^T (head dim x queries) ----
#pragma unroll
    for (int db = 0; db < DBS; ++db) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int key_row = MF::acc_row(h, s);   // key held in score register s by this lane group
        T vb[K + 1];
#pragma unroll
        for (int o = 0; o <= K; ++o) vb[o] = Vs[o][key_row][db * 16 + c];
#pragma unroll
        for (int k = 0; k <= K; ++k) {
#pragma unroll
          for (int a = 0; a <= k; ++a) acc_o[k][db] = MF::mma(vb[k - a], sc[a][s], acc_o[k][db]);
        }
      }
    }
  }

  if (chunks > 1) {
    // partial results of this key share: the row's shift, its row-sum series and the
    // unnormalised output series N_k, all relative to exp(-m_used)
#pragma unroll
    for (int o = 0; o <= K; ++o) {
      lsum[o] = rows_sum(lsum[o]);
    }
    if (!q_ok) return;
    const int64_t rows = bh * L, row = head * L + my_q;
    A* pm = part;                                                   // [chunks][rows]
    A* pl = part + static_cast<int64_t>(chunks) * rows;             // [chunks][K+1][rows]
    A* pn = pl + static_cast<int64_t>(chunks) * (K + 1) * rows;    // [chunks][K+1][rows][D]
    if (h == 0 && slice == 0) {
      pm[chunk * rows + row] = m_used;
#pragma unroll
      for (int o = 0; o <= K; ++o) pl[(static_cast<int64_t>(chunk) * (K + 1) + o) * rows + row] = lsum[o];
    }
#pragma unroll
    for (int o = 0; o <= K; ++o)
#pragma unroll
      for (int db = 0; db < DBS; ++db)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          pn[((static_cast<int64_t>(chunk) * (K + 1) + o) * rows + row) * D + d0 + db * 16 + MF::acc_row(h, r)] =
              static_cast<A>(acc_o[o][db][r]);
    return;
  }
  attention_epilogue<T, K, D, acc_t, 1, DBS>(acc_o, lsum, m_used, O, LSE, head, L, my_q, q_ok, h, d0, slice == 0);
}

// Merges the key shares of a split launch: per row, the shift m = max_c m_c, the weights
// exp(m_c - m), then the row-sum and output series as their weighted sums, the series quotient
// O_k = (N_k - sum_{j=1..k} l_j O_{k-j}) / l_0 and the lse series, as the single-launch epilogue.
// One thread per (row, head dim).
template <typename T, int K>
__global__ __launch_bounds__(256) void attn_split_combine_kernel(const typename AccOf<T>::type* __restrict__ part,
                                                                 int chunks, int64_t rows, int D, MPtrs<T> O,
                                                                 MPtrs<typename AccOf<T>::type> LSE) {
  using A = typename AccOf<T>::type;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= rows * D) return;
  const int64_t row = idx / D;
  const int d = static_cast<int>(idx % D);
  const A* pm = part;
  const A* pl = part + static_cast<int64_t>(chunks) * rows;
  const A* pn = pl + static_cast<int64_t>(chunks) * (K + 1) * rows;
  // (the chunk loops unrolled so that their independent loads are in flight together: the
  // kernel is a few load round trips long)
  A m = -__builtin_huge_val();
#pragma unroll 8
  for (int c = 0; c < chunks; ++c) m = fmax(m, pm[c * rows + row]);
  A l[K + 1], n[K + 1];
#pragma unroll
  for (int o = 0; o <= K; ++o) l[o] = n[o] = A(0);
  if (m != -__builtin_huge_val()) {
#pragma unroll 4
    for (int c = 0; c < chunks; ++c) {
      const A mc = pm[c * rows + row];
      const A w = mc == -__builtin_huge_val() ? A(0) : exp_fast(mc - m);
#pragma unroll
      for (int o = 0; o <= K; ++o) {
        l[o] += w * pl[(static_cast<int64_t>(c) * (K + 1) + o) * rows + row];
        n[o] += w * pn[((static_cast<int64_t>(c) * (K + 1) + o) * rows + row) * D + d];
      }
    }
  }
  const bool empty = !(l[0] > A(0));
  const A inv_l0 = empty ? A(0) : A(1) / l[0];
  A out[K + 1];
#pragma unroll
  for (int k = 0; k <= K; ++k) {
    A t = n[k];
#pragma unroll
    for (int j = 1; j <= k; ++j) t -= l[j] * out[k - j];
    out[k] = t * inv_l0;
    O.p[k][row * D + d] = static_cast<T>(out[k]);
  }
  if (d == 0 && LSE.p[0] != nullptr) {
    if (empty) {
      LSE.p[0][row] = __builtin_huge_val();
#pragma unroll
      for (int k = 1; k <= K; ++k) LSE.p[k][row] = A(0);
    } else {
      A lse[K + 1], nrm[K + 1];
      lse[0] = m + log_acc(l[0]);
#pragma unroll
      for (int k = 1; k <= K; ++k) nrm[k] = l[k] * inv_l0;
#pragma unroll
      for (int k = 1; k <= K; ++k) {
        A t = nrm[k];
#pragma unroll
        for (int j = 1; j < k; ++j) t -= (A(j) / A(k)) * lse[j] * nrm[k - j];
        lse[k] = t;
      }
#pragma unroll
      for (int k = 0; k <= K; ++k) LSE.p[k][row] = lse[k];
    }
  }
}

// ---------------------------------------------------------------------------
// Pipelined fp32 kernel for full-order operands (every operand has K+1 orders),
// key length a multiple of 16, and two K/V tiles within LDS:
// * the K and V tiles of key block j+1 are fetched by LDS DMA
//   (global_load_lds_dwordx4) into the second LDS buffer while block j's PV
//   products run, so staging costs no registers and its latency hides behind
//   MFMAs; one barrier per key block;
// * tiles are stored unpadded with the 16-byte chunks of a key row XOR-swizzled
//   by the row index (physical chunk = chunk ^ (row mod min(16, chunks))), which
//   keeps both the 16-byte K-operand reads and the 4-byte V-operand reads free
//   of bank conflicts;
// * query and key operands of head-dim chunk dc+1 are loaded while chunk dc's
//   MFMAs run;
// * masks are evaluated only on key blocks that cross the causal diagonal (or
//   with an explicit mask); interior blocks skip the per-element tests.
template <int K, int D>
struct AttnPipeShape {
  static constexpr int CH = D / 4;                        // 16-byte chunks per key row
  static constexpr int SWZ = CH < 16 ? CH : 16;           // swizzle period (power of two)
  static constexpr int RPS = 1024 / (D * 4);              // key rows per 1 KB DMA segment
  static constexpr int SEGS = kAttnBN / RPS;              // segments per order tile
  static constexpr size_t LDS = 2ull * 2 * (K + 1) * kAttnBN * D * sizeof(float);
  static constexpr bool fits = LDS <= 160 * 1024;
};

// LDS DMA of the K and V tiles of the key block starting at kb0 into one
// buffer (tiles[kv][order][row][d]): 1 KB segments; lane l writes physical
// chunk l % CH of row l / CH of its segment, loading the logical chunk that the
// row swizzle maps there.
// LDS-DMA operations one wave issues per key block: (K, V) x orders x its share
// of the 1 KB segments of an order tile.
template <int K, int D>
struct AttnDma {
  static constexpr int IT = (AttnPipeShape<K, D>::SEGS + kAttnWaves - 1) / kAttnWaves;
  static constexpr int OPS = 2 * (K + 1) * IT;
};

// Operation i of this wave's share of key block kb0's DMA. Callers pass an i that
// is a constant once their loops are unrolled, so the K/V pointer and the order
// are static indices.
template <int K, int D>
__device__ __forceinline__ void attn_issue_op(float (&buf)[2][K + 1][kAttnBN][D], const CPtrs<float>& Kp,
                                              const CPtrs<float>& Vp, int64_t head, int S, int kb0, int lane,
                                              int wave, int i) {
  using Shape = AttnPipeShape<K, D>;
  constexpr int CH = Shape::CH, SWZ = Shape::SWZ, RPS = Shape::RPS, SEGS = Shape::SEGS, IT = AttnDma<K, D>::IT;
  const int kv = i / ((K + 1) * IT), o = (i / IT) % (K + 1), it = i % IT;
  const int seg = it * kAttnWaves + wave;
  if (SEGS % kAttnWaves != 0 && seg >= SEGS) return;
  const int r = seg * RPS + lane / CH;
  const int lch = (lane % CH) ^ (r % SWZ);
  const float* src = (kv ? Vp.p[o] : Kp.p[o]) + (head * S + kb0 + r) * D + lch * 4;
  __builtin_amdgcn_global_load_lds(src, &buf[kv][o][seg * RPS][0], 16, 0, 0);
}

template <int K, int D>
__device__ __forceinline__ void attn_issue_tile(float (&buf)[2][K + 1][kAttnBN][D], const CPtrs<float>& Kp,
                                                const CPtrs<float>& Vp, int64_t head, int S, int kb0, int lane,
                                                int wave) {
#pragma unroll
  for (int i = 0; i < AttnDma<K, D>::OPS; ++i) attn_issue_op<K, D>(buf, Kp, Vp, head, S, kb0, lane, wave, i);
}

// Word 3 of a raw buffer resource on gfx9-family GPUs (32-bit data format, no swizzle).
constexpr int kBufferRsrcWord3 = 0x00020000;

__device__ __forceinline__ Vec<float, 4> attn_buffer_load4(__amdgpu_buffer_rsrc_t r, uint32_t byte_offset) {
  return __builtin_bit_cast(Vec<float, 4>, __builtin_amdgcn_raw_buffer_load_b128(r, byte_offset, 0, 0));
}

// Four bf16 values (round to nearest even) as the operand of a 16x16x16 bf16 MFMA.
typedef short AttnBf16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ AttnBf16x4 attn_pack_bf16x4(const Vec<float, 4>& v) {
  const uint32_t lo = pack_bf16x2(v.v[0], v.v[1]), hi = pack_bf16x2(v.v[2], v.v[3]);
  return __builtin_bit_cast(AttnBf16x4, (static_cast<uint64_t>(hi) << 32) | lo);
}

// Whether key kb0 + 4h + r (score register r of lane group h in the 16x16x4
// accumulator layout) is admissible for query my_q; mword holds the mask bytes
// of keys kb0 + 4h .. kb0 + 4h + 3.
// Branch-free (bitwise operators): a branch in the loops that call this splits
// their bodies and makes the compiler's memory-counter waits conservative.
__device__ __forceinline__ bool attn_key_ok(uint32_t mword, int kb0, int r, int h, int my_q, bool q_ok, int causal,
                                            bool has_mask) {
  const bool causal_ok = (kb0 + 4 * h + r <= my_q) | (causal == 0);
  const bool mask_ok = (((mword >> (8 * r)) & 0xffu) != 0u) | !has_mask;
  return q_ok & causal_ok & mask_ok;
}

// Operands of head-dim chunk dc: Q[my row][16 dc + 4 h .. +3] from global memory,
// K[key c][same d] from the swizzled LDS tile.
template <int K>
__device__ __forceinline__ void attn_load_q_chunk(Vec<float, 4> (&qn)[K + 1], const float* const (&qrow)[K + 1],
                                                  int dc, int h) {
#pragma unroll
  for (int o = 0; o <= K; ++o) qn[o] = *reinterpret_cast<const Vec<float, 4>*>(qrow[o] + dc * 16 + 4 * h);
}

template <int K, int D>
__device__ __forceinline__ void attn_load_k_chunk(Vec<float, 4> (&kn)[K + 1], const float (&ktile)[K + 1][kAttnBN][D],
                                                  int dc, int c, int h) {
  constexpr int SWZ = AttnPipeShape<K, D>::SWZ;
  const int pchk = (dc * 4 + h) ^ (c % SWZ);
#pragma unroll
  for (int o = 0; o <= K; ++o) kn[o] = *reinterpret_cast<const Vec<float, 4>*>(&ktile[o][c][pchk * 4]);
}

// Head-dim columns per lane in a PV operand read of the pipelined kernel: one
// 16-byte read serves four MFMAs when 16 lanes x 4 columns fit the head dim.
template <int D>
struct AttnPvE {
  static constexpr int value = D >= 64 ? 4 : D / 16;
};

// V operands of PV step (g, s): key row acc_row(h, s), head-dim columns
// g*16E + E*c .. +E-1 of every order (E consecutive floats: one LDS read).
template <int K, int D>
__device__ __forceinline__ void attn_load_v_step(Vec<float, AttnPvE<D>::value> (&vb)[K + 1],
                                                 const float (&vtile)[K + 1][kAttnBN][D], int g, int s, int c,
                                                 int h) {
  constexpr int E = AttnPvE<D>::value, SWZ = AttnPipeShape<K, D>::SWZ;
  const int key_row = Mfma16<float>::acc_row(h, s);
  const int col = g * 16 * E + E * c;
  const int pch = (col / 4) ^ (key_row % SWZ);
#pragma unroll
  for (int o = 0; o <= K; ++o)
    vb[o] = *reinterpret_cast<const Vec<float, E>*>(&vtile[o][key_row][pch * 4 + col % 4]);
}

template <int K, int D>
__global__ __launch_bounds__(kAttnWaves * kWave) void taylor_attention_fwd_pipe_kernel(
    CPtrs<float> Q, CPtrs<float> Kp, CPtrs<float> Vp, MPtrs<float> O, MPtrs<float> LSE, int L, int S,
    const uint8_t* __restrict__ mask_all, AttnMaskMap mmap, const int32_t* __restrict__ ranges_all, int causal,
    float scale) {
  using A = float;
  using MF = Mfma16<float>;
  using acc_t = MF::acc_t;
  using Shape = AttnPipeShape<K, D>;
  constexpr int DB = D / 16;
  constexpr int CH = Shape::CH, SWZ = Shape::SWZ, RPS = Shape::RPS, SEGS = Shape::SEGS;
  constexpr A kNegInf = -__builtin_huge_valf();
  static_assert(Shape::fits, "two K/V tiles exceed LDS");

  // [buffer][0 = K, 1 = V][order][key row][head dim], rows unpadded and chunk-swizzled
  __shared__ __attribute__((aligned(16))) float tiles[2][2][K + 1][kAttnBN][D];

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int c = lane % 16;
  const int h = lane / 16;
  int64_t head;
  int q_block;
  attn_work_item(L, causal, head, q_block);
  // this head's mask, its block ranges (and additive values)
  const int64_t mask_index = attn_mask_index(mmap, head);
  const uint8_t* mask = mask_all != nullptr ? mask_all + mask_index * L * S : nullptr;
  const int32_t* ranges = ranges_all != nullptr ? ranges_all + mask_index * attn_ranges_count(L, S) : nullptr;
  const int q0_wave = q_block + wave * kAttnQPerWave;
  const int my_q = q0_wave + c;
  const bool q_ok = my_q < L;
  const int q_row = q_ok ? my_q : L - 1;   // rows past L read a valid row; their results are dropped

  const float* qrow[K + 1];
#pragma unroll
  for (int o = 0; o <= K; ++o) qrow[o] = Q.p[o] + (head * L + q_row) * D;

  int lo, hi;
  attn_key_range(S, q_block, causal, ranges, lo, hi);
  // a workgroup whose rows admit no key keeps one (fully masked) block, so the
  // pipeline below always has a first block (the launcher requires S >= 16)
  if (hi <= lo) {
    lo = 0;
    hi = kAttnBN;
  }
  const int nblocks = (hi - lo + kAttnBN - 1) / kAttnBN;

  // Mask bits of this lane's keys 4h .. 4h+3 of a key block (the rows of its
  // score registers r = 0..3) are one aligned 32-bit read of the mask row; it
  // is unconditional and branch-free (without a mask it re-reads a valid dummy
  // word), so no load sits behind a branch and the compiler's memory-counter
  // waits stay exact for the prefetches around it.
  const uint8_t* mrow = mask != nullptr ? mask + static_cast<int64_t>(q_row) * S + 4 * h
                                        : reinterpret_cast<const uint8_t*>(Q.p[0]);
  const int mstep = mask != nullptr ? 1 : 0;

  // The shift of the exponentials is a running maximum of the order-0 scores, raised lazily:
  // only when a key block's maximum exceeds it by more than kSlack (so p <= e^kSlack), with the
  // accumulators rescaled on that rare path. The output does not depend on the shift (it cancels
  // in O = N / l).
  constexpr A kSlack = A(8);
  A m_used = kNegInf;

  // the first key block's DMA is issued only now: LDS-DMA loads pending beside
  // ordinary loads make the compiler wait for every load in flight
  attn_issue_tile<K, D>(tiles[0], Kp, Vp, head, S, lo, lane, wave);

  acc_t acc_o[K + 1][DB];
#pragma unroll
  for (int o = 0; o <= K; ++o)
#pragma unroll
    for (int db = 0; db < DB; ++db) acc_o[o][db] = MF::zero();
  A lsum[K + 1];
#pragma unroll
  for (int o = 0; o <= K; ++o) lsum[o] = A(0);

  // Query chunks live in a ring of NQ register slots (chunk dc in slot dc % NQ).
  // With NQ == DB the whole query tile stays resident; otherwise chunk dc+NQ-1
  // (cyclically: every key block reads the same chunks) is fetched while chunk
  // dc's MFMAs run, NQ-1 chunks ahead of its use.
  constexpr int NQ = DB;
  Vec<float, 4> qs[NQ][K + 1];
#pragma unroll
  for (int dc = 0; dc < (NQ == DB ? DB : NQ - 1); ++dc) attn_load_q_chunk<K>(qs[dc], qrow, dc, h);

  for (int j = 0; j < nblocks; ++j) {
    const int buf = j & 1;
    const int kb0 = lo + j * kAttnBN;
    __builtin_amdgcn_s_waitcnt(0);   // this wave's DMA of block j has landed
    __syncthreads();                 // ... and every wave's; block j-1's buffer is free
    const uint32_t mword = *reinterpret_cast<const uint32_t*>(mrow + mstep * kb0);   // used after the scores

    // ---- scores S^T_k = sum_{a+b=k} K_b Q_a^T; key chunk dc+1 read from LDS during chunk dc ----
    // (scheduling barriers keep each chunk's prefetches ahead of its MFMAs; left
    // alone the scheduler sinks them next to their uses)
    acc_t sc[K + 1];
#pragma unroll
    for (int o = 0; o <= K; ++o) sc[o] = MF::zero();
    Vec<float, 4> kq[2][K + 1];
    attn_load_k_chunk<K, D>(kq[0], tiles[buf][0], 0, c, h);
#pragma unroll
    for (int dc = 0; dc < DB; ++dc) {
      if constexpr (NQ < DB) {
        const int ahead = (dc + NQ - 1) % DB;
        attn_load_q_chunk<K>(qs[ahead % NQ], qrow, ahead, h);
      }
      if (dc + 1 < DB) attn_load_k_chunk<K, D>(kq[(dc + 1) & 1], tiles[buf][0], dc + 1, c, h);
      __builtin_amdgcn_sched_barrier(0);
      const Vec<float, 4>(&qa)[K + 1] = qs[dc % NQ];
      const Vec<float, 4>(&kb)[K + 1] = kq[dc & 1];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
#pragma unroll
        for (int k = 0; k <= K; ++k) {
#pragma unroll
          for (int a = 0; a <= k; ++a) sc[k] = MF::mma(kb[k - a].v[s], qa[a].v[s], sc[k]);
        }
      }
    }

    // admissibility is settled before the DMA below is issued, so waiting for
    // the mask word never waits for the DMA
    bool valid[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) valid[r] = attn_key_ok(mword, kb0, r, h, my_q, q_ok, causal, mask != nullptr);


    // ---- running maximum of the order-0 scores (the row's 16 keys of this block are spread over
    // the four lane groups), raised lazily ----
    A bmax = kNegInf;
#pragma unroll
    for (int r = 0; r < 4; ++r) bmax = fmaxf(bmax, valid[r] ? sc[0][r] * scale : kNegInf);
    bmax = rows_max(bmax);
    const bool raise = bmax > m_used + kSlack || (m_used == kNegInf && bmax != kNegInf);
    // a row whose shift is still -inf has accumulated nothing: raising it rescales nothing
    if (__any(raise && m_used != kNegInf)) {
      const A alpha = (raise && m_used != kNegInf) ? exp_fast(m_used - bmax) : A(1);
#pragma unroll
      for (int o = 0; o <= K; ++o) {
        lsum[o] *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          // out of and back into the accumulation registers here, on this rare path, so that the
          // accumulators keep one register class across the loop (no copies per block)
          asm volatile("" : "+a"(acc_o[o][db]));
#pragma unroll
          for (int r = 0; r < 4; ++r) acc_o[o][db][r] *= alpha;
          asm volatile("" : "+a"(acc_o[o][db]));
        }
      }
    }
    if (raise) m_used = bmax;

    // ---- exponential series against the running maximum ----
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const A p = valid[r] ? exp_fast(sc[0][r] * scale - m_used) : A(0);
      A sk[K + 1], e[K + 1];
#pragma unroll
      for (int o = 1; o <= K; ++o) sk[o] = sc[o][r] * scale;
      e[0] = A(1);
#pragma unroll
      for (int k = 1; k <= K; ++k) {
        A t = A(0);
#pragma unroll
        for (int i = 1; i <= k; ++i) t += (A(i) * sk[i]) * e[k - i];
        e[k] = t * (A(1) / A(k));
      }
#pragma unroll
      for (int o = 0; o <= K; ++o) {
        const A w = p * e[o];
        lsum[o] += w;
        sc[o][r] = w;
      }
    }

    // ---- O^T_k += sum_{a+b=k} V_b^T E_a^T ----
    // Step t = (g, s) reads E consecutive head-dim columns of key row 4h+s per
    // lane and order; element e feeds the MFMAs of accumulator g*E + e, whose
    // rows are the columns g*16E + E*m + e. Step t+1's reads (and a share of the
    // next key block's DMA into the other buffer; the last block re-loads
    // itself, so there is no branch) are issued right after step t's first
    // MFMA: with an LDS DMA in flight the compiler waits for every outstanding
    // LDS read before using any, and the rest of step t covers their latency.
    constexpr int PE = AttnPvE<D>::value, STEPS = DB / PE * 4, OPS = AttnDma<K, D>::OPS;
    const int next_kb0 = min(kb0 + kAttnBN, lo + (nblocks - 1) * kAttnBN);
    Vec<float, PE> vq[2][K + 1];
    attn_load_v_step<K, D>(vq[0], tiles[buf][1], 0, 0, c, h);
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
      const int g = t / 4, s = t % 4;
      const Vec<float, PE>(&vb)[K + 1] = vq[t & 1];
      acc_o[0][g * PE] = MF::mma(vb[0].v[0], sc[0][s], acc_o[0][g * PE]);
      __builtin_amdgcn_sched_barrier(0);
      if (t + 1 < STEPS) attn_load_v_step<K, D>(vq[(t + 1) & 1], tiles[buf][1], (t + 1) / 4, (t + 1) % 4, c, h);
#pragma unroll
      for (int i = t * OPS / STEPS; i < (t + 1) * OPS / STEPS; ++i)
        attn_issue_op<K, D>(tiles[buf ^ 1], Kp, Vp, head, S, next_kb0, lane, wave, i);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int e = 0; e < PE; ++e) {
#pragma unroll
        for (int k = 0; k <= K; ++k) {
#pragma unroll
          for (int a = 0; a <= k; ++a) {
            if (e == 0 && k == 0) continue;   // issued above
            acc_o[k][g * PE + e] = MF::mma(vb[k - a].v[e], sc[a][s], acc_o[k][g * PE + e]);
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  __builtin_amdgcn_s_waitcnt(0);   // the last block's (redundant) DMA has landed before the workgroup ends
  // (a row with no visible key has p = 0 everywhere: any finite shift will do)
  attention_epilogue<float, K, D, acc_t, AttnPvE<D>::value>(acc_o, lsum, m_used == kNegInf ? A(0) : m_used, O, LSE,
                                                           head, L, my_q, q_ok, h);
}

template <typename T, int K, int D>
static int launch_attention_kd(const AttnArgs& a) {
  using A = typename AccOf<T>::type;
  if constexpr (!AttnShape<T, K, D>::fits) {
    pt_host::set_error("Taylor attention: degree and head dim exceed the LDS budget for this dtype");
    return PT_UNSUPPORTED;
  } else {
    CPtrs<T> q{}, k{}, v{};
    MPtrs<T> o{};
    MPtrs<A> lse{};
    for (int i = 0; i < a.q_orders; ++i) q.p[i] = static_cast<const T*>(a.q[i]);
    for (int i = 0; i < a.k_orders; ++i) k.p[i] = static_cast<const T*>(a.k[i]);
    for (int i = 0; i < a.v_orders; ++i) v.p[i] = static_cast<const T*>(a.v[i]);
    for (int i = 0; i <= K; ++i) {
      o.p[i] = static_cast<T*>(a.out[i]);
      if (a.lse != nullptr) lse.p[i] = static_cast<A*>(a.lse[i]);
    }
    const dim3 grid(static_cast<unsigned>((a.lq + kAttnBM - 1) / kAttnBM * a.bh));
    if constexpr (sizeof(T) == 4 && AttnPipeShape<K, D>::fits) {
      // the pipelined kernel reads each lane's four mask bytes as one 32-bit word (and takes no
      // additive mask)
      bool pipe = a.mask_add == nullptr && a.q_orders == K + 1 && a.k_orders == K + 1 && a.v_orders == K + 1 && a.lk >= kAttnBN &&
                  a.lk % kAttnBN == 0 && reinterpret_cast<uintptr_t>(a.mask) % 4 == 0 &&
                  a.lk * D * sizeof(float) < (size_t{1} << 31) &&   // 32-bit buffer offsets: per-head keys,
                  (a.mask == nullptr || a.lq * a.lk < (int64_t{1} << 31));   // ... and the whole mask
      for (int i = 0; i <= K && pipe; ++i)
        pipe = pt_host::aligned16(a.q[i]) && pt_host::aligned16(a.k[i]) && pt_host::aligned16(a.v[i]);
      if (pipe) {
        taylor_attention_fwd_pipe_kernel<K, D><<<grid, dim3(kAttnWaves * kWave), 0, a.stream>>>(
            q, k, v, o, lse, static_cast<int>(a.lq), static_cast<int>(a.lk), a.mask, a.mask_map, a.mask_ranges,
            a.causal ? 1 : 0, static_cast<A>(a.scale));
        PT_LAUNCH_CHECK();
        return PT_OK;
      }
    }
    const AttnSplit sp = attention_split(a, sizeof(T) == 8 ? PT_FLOAT64 : PT_FLOAT32);
    const bool split = sp.chunks > 1 && a.workspace != nullptr && a.workspace_bytes >= sp.bytes;
    const int chunks = split ? sp.chunks : 1;
    const dim3 sgrid(grid.x * AttnShape<T, K, D>::SL * chunks);
    const A* madd = static_cast<const A*>(a.mask_add);
#define PT_ATTN_STAGED(ADD)                                                                                  \
  taylor_attention_fwd_kernel<T, K, D, ADD><<<sgrid, dim3(kAttnWaves * kWave), 0, a.stream>>>(               \
      q, a.q_orders, k, a.k_orders, v, a.v_orders, o, lse, static_cast<int>(a.lq), static_cast<int>(a.lk),   \
      a.mask, a.mask_map, madd, a.mask_ranges, a.causal ? 1 : 0, static_cast<A>(a.scale), chunks, split ? sp.chunk_keys : 0, \
      split ? static_cast<A*>(a.workspace) : nullptr)
    if (madd != nullptr) PT_ATTN_STAGED(true);
    else PT_ATTN_STAGED(false);
#undef PT_ATTN_STAGED
    PT_LAUNCH_CHECK();
    if (split) {
      const int64_t rows = a.bh * a.lq, threads = rows * D;
      attn_split_combine_kernel<T, K><<<dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0, a.stream>>>(
          static_cast<const A*>(a.workspace), chunks, rows, static_cast<int>(D), o, lse);
      PT_LAUNCH_CHECK();
    }
    return PT_OK;
  }
}

template <typename T, int K>
static int launch_attention_k(const AttnArgs& a) {
  switch (a.d) {
    case 16: return launch_attention_kd<T, K, 16>(a);
    case 32: return launch_attention_kd<T, K, 32>(a);
    case 64: return launch_attention_kd<T, K, 64>(a);
    case 128: return launch_attention_kd<T, K, 128>(a);
    default: break;
  }
  pt_host::set_error("Taylor attention: head dim must be 16, 32, 64 or 128");
  return PT_UNSUPPORTED;
}

template <typename T>
int launch_attention(const AttnArgs& a) {
  switch (a.degree) {
    case 0: return launch_attention_k<T, 0>(a);
    case 1: return launch_attention_k<T, 1>(a);
    case 2: return launch_attention_k<T, 2>(a);
    case 3: return launch_attention_k<T, 3>(a);
    case 4: return launch_attention_k<T, 4>(a);
    case 5: return launch_attention_k<T, 5>(a);
    case 6: return launch_attention_k<T, 6>(a);
    case 7: return launch_attention_k<T, 7>(a);
    case 8: return launch_attention_k<T, 8>(a);
    default: break;
  }
  pt_host::set_error("Taylor attention: degree outside 0..PT_MAX_DEGREE");
  return PT_UNSUPPORTED;
}

}  // namespace pt
