// Flash-style attention forward of degree-K series with bfloat16 / float16
// operands on the 16x16x32 MFMAs of gfx950 (fp32 accumulation).
//
// The series arithmetic is that of taylor_attention.inl: per query row,
//   exp(S(t)) = exp(S_0) e(t),  e_k = sum_{j=1..k} (j/k) S_j e_{k-j},
//   l_k = sum_keys exp(S_0 - m) e_k,  N_k = sum_keys sum_{a+b=k} exp(S_0 - m) e_a V_b,
//   O_k = (N_k - sum_{j=1..k} l_j O_{k-j}) / l_0,
// the series of the reference's decomposition
// (/root/reference/src/polytensors/_decompositions.py:28-43), as in its degree-1
// fused kernel for half types (/root/reference/src/polytensors/_fused_attention.py:72-78,
// _attention_kernels.py:27-82: half operands, fp32 accumulation). Only the
// MFMA operands are 16-bit: Q, K and V as stored, and the probability series
// P_k = exp(S_0 - m) e_k rounded to the storage type for the value product.
// The row sums l_k add those rounded values (hi + lo where split), so numerator
// and denominator of O = N / l weigh each key alike and O is the exact weighted
// average for the rounded weights. Summed from the fp32 values instead, the
// weights' rounding survives the cancellation in the quotient's higher orders:
// a degree-3 case (d 32, 19 x 13 keys, causal) had order 3 off by 1.05e-2 of its
// scale (6.4e-3 this way), and its key gradient, through the saved output and lse,
// by 2.3e-2 (4.0e-3 this way).
// Scores, the exponential series, the row sums and the output accumulators are
// fp32; the output is rounded to the storage type once, the lse series is fp32.
//
// Work decomposition: a workgroup of 4 waves owns 64 query rows of one head
// (16 per wave); key blocks of 32 keys are staged in LDS, K row-major and V
// transposed (head dim x keys). With v_mfma_f32_16x16x32 (lane l supplies A
// row l % 16 and B column l % 16, contraction elements 8 (l / 16) .. + 7; the
// accumulator register r of lane l is row 4 (l / 16) + r, column l % 16):
// * scores transposed, S^T = K Q^T per 16-key half: lane (c, g) = (l % 16,
//   l / 16) holds keys 4g + r of the half for query c;
// * the value product O^T += V^T P^T contracts the block's 32 keys with lane
//   group g's slots 8g .. 8g + 7 standing for keys 4g .. 4g + 3 and
//   16 + 4g .. 16 + 4g + 3: exactly the eight probabilities the lane holds, so
//   P goes from the score accumulators into the B operand without leaving the
//   lane. The A operand (V^T, the same eight keys of head-dim row c) is two
//   8-byte reads of the transposed V tile.
// The output accumulators O^T_k (16 head dims x 16 queries per block) and, when
// the registers allow, the wave's query tile stay in registers for the whole key
// loop.
#pragma once

#include <type_traits>

#include "half_mfma.h"
#include "taylor_attention.inl"

namespace pt {


template <int K, int D>
struct AttnHalfShape {
  static constexpr int KB = 32;              // keys per block
  static constexpr int DC = (D + 31) / 32;   // 32-wide head-dim chunks of the score contraction
  // Output head-dim slices: the output accumulators of every order at head dim 128 exceed the
  // registers from degree 5 on; two slices (a grid dimension, each recomputing its scores) keep
  // every instantiation free of scratch spills (checked with the compiler's resource remarks).
  static constexpr int SL = D == 128 ? (K >= 8 ? 4 : K >= 5 ? 2 : 1) : 1;
  static constexpr int DS = D / SL;          // output head dims per slice
  static constexpr int DB = DS / 16;         // 16-wide output blocks of the slice
  static constexpr int LDK = D + 8;          // K tile row: 16-byte aligned, 4 banks of skew per row
  // Transposed V tile row (keys): 40 values (20 dwords) make the 8-byte operand reads of 16 rows x
  // two lane groups hit 64 distinct banks; 36 where the larger tile would not fit.
  static constexpr size_t lds_with(int ldv) { return static_cast<size_t>(K + 1) * (KB * LDK + DS * ldv) * 2; }
  static constexpr int LDV = lds_with(40) <= 160 * 1024 ? 40 : 36;
  static constexpr size_t LDS = lds_with(LDV);
  static constexpr bool fits = LDS <= 160 * 1024;
  // Probability orders 1..K as a hi + lo pair of 16-bit operands (two value-product MFMAs each)
  // from degree 5 on. The higher probability coefficients exceed the output coefficients they
  // cancel into by about the factor 10 at high degree, so one rounding of them costs up to 4e-2 of
  // the output order; the pair keeps it near 1e-3. Up to degree 4 one rounding stays below 5e-3.
  static constexpr bool split = K >= 5;
  // The wave's query tile stays in registers when accumulators, tile and working set fit.
  static constexpr bool q_regs = SL == 1 && (K + 1) * DB * 4 + (K + 1) * DC * 4 + 16 * (K + 1) + 64 +
                                                    (split ? 4 * K : 0) <= 448;
};

// Eight 16-bit values (one 16-byte load) at p, or zeros.
template <typename T>
__device__ __forceinline__ u32x4 attn_half_load8(const T* p, bool ok) {
  const u32x4 v = *reinterpret_cast<const u32x4*>(p);
  const u32x4 z = {0u, 0u, 0u, 0u};
  return ok ? v : z;
}

// ADD: an additive (L, S) mask madd (float32 values) is given with the boolean mask of its finite
// entries; it adds to the constant-order scores after scaling.
template <typename T, int K, int D, bool ADD>
__global__ __launch_bounds__(kAttnWaves * kWave) void taylor_attention_fwd_half_kernel(
    CPtrs<T> Q, int q_orders, CPtrs<T> Kp, int k_orders, CPtrs<T> Vp, int v_orders, MPtrs<T> O, MPtrs<float> LSE,
    int L, int S, const uint8_t* __restrict__ mask_all, AttnMaskMap mmap, const int32_t* __restrict__ ranges_all,
    const float* __restrict__ madd_all, int causal, float scale) {
  using Sh = AttnHalfShape<K, D>;
  using MM = HalfMfma<T>;
  constexpr int KB = Sh::KB, DC = Sh::DC, DB = Sh::DB, LDK = Sh::LDK, LDV = Sh::LDV;
  constexpr float kNegInf = -__builtin_huge_valf();
  constexpr float kSlack = MM::kSlack;
  static_assert(Sh::fits, "K/V tiles exceed LDS");

  constexpr int SL = Sh::SL, DS = Sh::DS;
  __shared__ __align__(16) T Ks[K + 1][KB][LDK];
  __shared__ __align__(16) T Vt[K + 1][DS][LDV];

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int c = lane % 16;   // query column (score and output accumulators); key / head-dim row of A operands
  const int g = lane / 16;   // lane group
  int64_t head;
  int q_block, slice = 0;
  if constexpr (SL == 1) {
    attn_work_item(L, causal, head, q_block);
  } else {
    // slices fastest, then heads, heaviest query blocks first
    const int nqb = (L + kAttnBM - 1) / kAttnBM;
    const int64_t bh = gridDim.x / (static_cast<int64_t>(nqb) * SL);
    const int64_t t = blockIdx.x / SL;
    slice = static_cast<int>(blockIdx.x % SL);
    head = t % bh;
    q_block = (nqb - 1 - static_cast<int>(t / bh)) * kAttnBM;
  }
  const int d0 = slice * DS;   // first output head dim of this workgroup
  // this head's mask, its block ranges (and additive values)
  const int64_t mask_index = attn_mask_index(mmap, head);
  const uint8_t* mask = mask_all != nullptr ? mask_all + mask_index * L * S : nullptr;
  const int32_t* ranges = ranges_all != nullptr ? ranges_all + mask_index * attn_ranges_count(L, S) : nullptr;
  const float* madd = ADD ? madd_all + mask_index * L * S : nullptr;
  const int my_q = q_block + wave * kAttnQPerWave + c;
  const bool q_ok = my_q < L;
  const int64_t qrow = (head * L + (q_ok ? my_q : 0)) * D;

  // Query operand of order o, chunk dc: Q[my_q][32 dc + 8 g .. + 7] (zero past D, L or the orders given).
  auto load_q = [&](int o, int dc) -> u32x4 {
    const bool in = q_ok && o < q_orders && 32 * dc + 8 * g < D;
    return attn_half_load8<T>(order_ptr<K>(Q, o < q_orders ? o : 0) + qrow + (in ? 32 * dc + 8 * g : 0), in);
  };
  u32x4 qreg[Sh::q_regs ? K + 1 : 1][Sh::q_regs ? DC : 1];
  if constexpr (Sh::q_regs) {
#pragma unroll
    for (int o = 0; o <= K; ++o)
#pragma unroll
      for (int dc = 0; dc < DC; ++dc) qreg[o][dc] = load_q(o, dc);
  }

  floatx4 acc_o[K + 1][DB];
#pragma unroll
  for (int o = 0; o <= K; ++o)
#pragma unroll
    for (int db = 0; db < DB; ++db) acc_o[o][db] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_used = kNegInf;
  float lsum[K + 1];   // this lane's partial row sums (its keys only)
#pragma unroll
  for (int o = 0; o <= K; ++o) lsum[o] = 0.f;

  // key range: causal and mask-range bounds, lo rounded down to a 32-key block
  int lo = 0, hi = S;
  if (causal) hi = min(S, q_block + kAttnBM);
  if (ranges != nullptr) {
    const int qb = q_block / kAttnRangeBlock;
    lo = ranges[2 * qb] / KB * KB;
    hi = min(hi, static_cast<int>(ranges[2 * qb + 1]));
  }

  for (int kb0 = lo; kb0 < hi; kb0 += KB) {
    uint8_t mbyte[2][4];   // mask bytes of this lane's eight keys, read ahead of the staging loads
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int r = 0; r < 4; ++r) mbyte[kh][r] = attn_mask_byte(mask, Q.p[0], my_q, kb0 + 16 * kh + 4 * g + r, L, S);
    float add[ADD ? 2 : 1][4];   // additive mask values of the same keys
    if constexpr (ADD) {
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int r = 0; r < 4; ++r) add[kh][r] = attn_mask_add(madd, my_q, kb0 + 16 * kh + 4 * g + r, L, S);
    }
    __syncthreads();   // the previous block's products are done with the tiles
    // ---- stage K rows kb0 .. kb0 + 31 of every order, row-major (zero past S / the orders given) ----
    {
      constexpr int VPR = D / 8;   // 16-byte vectors per row
      for (int idx = threadIdx.x; idx < (K + 1) * KB * VPR; idx += kAttnWaves * kWave) {
        const int o = idx / (KB * VPR);
        const int rem = idx % (KB * VPR);
        const int r = rem / VPR, cv = (rem % VPR) * 8;
        const int key = kb0 + r;
        const bool in = key < S && o < k_orders;
        const u32x4 v = attn_half_load8<T>(order_ptr<K>(Kp, o < k_orders ? o : 0) +
                                               (head * S + min(key, S - 1)) * D + cv, in);
        *reinterpret_cast<u32x4*>(&Ks[o][r][cv]) = v;
      }
    }
    // ---- stage V rows transposed: Vt[o][dim - d0][key] for the slice's dims, four keys x eight dims per step ----
    {
      constexpr int DV = DS / 8;
      for (int idx = threadIdx.x; idx < (K + 1) * (KB / 4) * DV; idx += kAttnWaves * kWave) {
        const int o = idx / ((KB / 4) * DV);
        const int rem = idx % ((KB / 4) * DV);
        const int kq = rem % (KB / 4), dv = rem / (KB / 4);   // key quad fastest: adjacent lanes, adjacent keys
        const T* src = order_ptr<K>(Vp, o < v_orders ? o : 0);
        u32x4 x[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int key = kb0 + 4 * kq + j;
          x[j] = attn_half_load8<T>(src + (head * S + min(key, S - 1)) * D + d0 + 8 * dv, key < S && o < v_orders);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          // dim 8 dv + e of keys 4 kq .. 4 kq + 3: the low or high halves of word e / 2
          const int w = e / 2;
          uint32_t lo_w, hi_w;
          if (e % 2 == 0) {
            lo_w = (x[0][w] & 0xffffu) | (x[1][w] << 16);
            hi_w = (x[2][w] & 0xffffu) | (x[3][w] << 16);
          } else {
            lo_w = (x[0][w] >> 16) | (x[1][w] & 0xffff0000u);
            hi_w = (x[2][w] >> 16) | (x[3][w] & 0xffff0000u);
          }
          *reinterpret_cast<uint2*>(&Vt[o][8 * dv + e][4 * kq]) = make_uint2(lo_w, hi_w);
        }
      }
    }
    __syncthreads();

    // ---- scores S^T_k = sum_{a+b=k} K_b Q_a^T for the two 16-key halves (keys x queries) ----
    floatx4 sc[2][K + 1];
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int o = 0; o <= K; ++o) sc[kh][o] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dc = 0; dc < DC; ++dc) {
      u32x4 qa[K + 1];
#pragma unroll
      for (int o = 0; o <= K; ++o) {
        if constexpr (Sh::q_regs) qa[o] = qreg[o][dc];
        else qa[o] = load_q(o, dc);
      }
      const bool din = 32 * dc + 8 * g < D;
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
        u32x4 kop[K + 1];
#pragma unroll
        for (int o = 0; o <= K; ++o) {
          const u32x4 v = *reinterpret_cast<const u32x4*>(&Ks[o][16 * kh + c][din ? 32 * dc + 8 * g : 0]);
          const u32x4 z = {0u, 0u, 0u, 0u};
          kop[o] = din ? v : z;
        }
#pragma unroll
        for (int k = 0; k <= K; ++k)
#pragma unroll
          for (int a = 0; a <= k; ++a) sc[kh][k] = MM::mma(kop[k - a], qa[a], sc[kh][k]);
      }
    }

    // ---- mask, online maximum of the constant order, exponential series ----
    bool valid[2][4];
    float s0[2][4];
    float bmax = kNegInf;
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kb0 + 16 * kh + 4 * g + r;
        bool ok = q_ok && key < S;
        if (causal) ok = ok && key <= my_q;
        if (mask != nullptr) ok = ok && mbyte[kh][r] != 0;
        valid[kh][r] = ok;
        float sv = sc[kh][0][r] * scale;
        if constexpr (ADD) sv += add[kh][r];
        s0[kh][r] = ok ? sv : kNegInf;
        bmax = fmaxf(bmax, s0[kh][r]);
      }
    bmax = rows_max(bmax);
    const bool raise = bmax > m_used + kSlack || (m_used == kNegInf && bmax != kNegInf);
    if (__any(raise)) {
      const float m_new = raise ? bmax : m_used;
      const float alpha = (raise && m_used != kNegInf) ? exp_fast(m_used - m_new) : (raise ? 0.f : 1.f);
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
    u32x4 pb[K + 1];   // probability operands: slots 0..3 keys 4g + r, slots 4..7 keys 16 + 4g + r
    u32x4 pl[Sh::split ? K + 1 : 1];   // lo parts of orders 1..K (split)
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      float w[K + 1][4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = valid[kh][r] ? exp_fast(s0[kh][r] - m_used) : 0.f;
        float sk[K + 1], e[K + 1];
#pragma unroll
        for (int o = 1; o <= K; ++o) sk[o] = sc[kh][o][r] * scale;
        e[0] = 1.f;
#pragma unroll
        for (int k = 1; k <= K; ++k) {
          float t = 0.f;
#pragma unroll
          for (int j = 1; j <= k; ++j) t += (static_cast<float>(j) * sk[j]) * e[k - j];
          e[k] = t * (1.f / static_cast<float>(k));
        }
#pragma unroll
        for (int o = 0; o <= K; ++o) w[o][r] = p * e[o];
      }
#pragma unroll
      for (int o = 0; o <= K; ++o) {
        const uint32_t w01 = MM::pack2(w[o][0], w[o][1]), w23 = MM::pack2(w[o][2], w[o][3]);
        pb[o][2 * kh] = w01;
        pb[o][2 * kh + 1] = w23;
        // the row sums add the weights as rounded for the value products
        lsum[o] = MM::sum2(w23, MM::sum2(w01, lsum[o]));
        if constexpr (Sh::split) {
          if (o >= 1) {   // the rounding residuals as the lo operand
            pl[o][2 * kh] = MM::pack2(w[o][0] - MM::lo(w01), w[o][1] - MM::hi(w01));
            pl[o][2 * kh + 1] = MM::pack2(w[o][2] - MM::lo(w23), w[o][3] - MM::hi(w23));
            lsum[o] = MM::sum2(pl[o][2 * kh + 1], MM::sum2(pl[o][2 * kh], lsum[o]));
          }
        }
      }
    }

    // ---- O^T_k += sum_{a+b=k} V_b^T P_a^T (head dim x queries), 32 keys per MFMA ----
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      u32x4 vop[K + 1];
#pragma unroll
      for (int o = 0; o <= K; ++o) {
        const uint2 first = *reinterpret_cast<const uint2*>(&Vt[o][16 * db + c][4 * g]);
        const uint2 second = *reinterpret_cast<const uint2*>(&Vt[o][16 * db + c][16 + 4 * g]);
        vop[o] = u32x4{first.x, first.y, second.x, second.y};
      }
#pragma unroll
      for (int k = 0; k <= K; ++k) {
#pragma unroll
        for (int a = 0; a <= k; ++a) acc_o[k][db] = MM::mma(vop[k - a], pb[a], acc_o[k][db]);
        if constexpr (Sh::split) {
#pragma unroll
          for (int a = 1; a <= k; ++a) acc_o[k][db] = MM::mma(vop[k - a], pl[a], acc_o[k][db]);
        }
      }
    }
  }

  // ---- epilogue: row sums over the lane groups, series quotient, output and lse series ----
#pragma unroll
  for (int o = 0; o <= K; ++o) {
    lsum[o] = rows_sum(lsum[o]);
  }
  if (!q_ok) return;
  const bool empty = !(lsum[0] > 0.f);
  const float inv_l0 = empty ? 0.f : 1.f / lsum[0];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    float out[4][K + 1];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
      for (int k = 0; k <= K; ++k) {
        float t = acc_o[k][db][r];
#pragma unroll
        for (int j = 1; j <= k; ++j) t -= lsum[j] * out[r][k - j];
        out[r][k] = t * inv_l0;
      }
    }
#pragma unroll
    for (int k = 0; k <= K; ++k) {
      // head dims 16 db + 4 g .. + 3 of this query: one 8-byte store
      *reinterpret_cast<uint2*>(O.p[k] + (head * L + my_q) * D + d0 + 16 * db + 4 * g) =
          make_uint2(MM::pack2(out[0][k], out[1][k]), MM::pack2(out[2][k], out[3][k]));
    }
  }
  if (LSE.p[0] != nullptr && g == 0 && slice == 0) {
    const int64_t at = head * L + my_q;
    if (empty) {
      LSE.p[0][at] = __builtin_huge_valf();
#pragma unroll
      for (int k = 1; k <= K; ++k) LSE.p[k][at] = 0.f;
    } else {
      float lse[K + 1], nrm[K + 1];
      lse[0] = m_used + logf(lsum[0]);
#pragma unroll
      for (int k = 1; k <= K; ++k) nrm[k] = lsum[k] * inv_l0;
#pragma unroll
      for (int k = 1; k <= K; ++k) {
        float t = nrm[k];
#pragma unroll
        for (int j = 1; j < k; ++j) t -= (static_cast<float>(j) / static_cast<float>(k)) * lse[j] * nrm[k - j];
        lse[k] = t;
      }
#pragma unroll
      for (int k = 0; k <= K; ++k) LSE.p[k][at] = lse[k];
    }
  }
}

// ---------------------------------------------------------------------------
// Pipelined 16-bit kernel for full-order operands where two K/V tile buffers
// fit LDS and the working set fits the registers (no head-dim slices):
// * the K and V tiles of key block j+1 are fetched by LDS DMA (buffer loads
//   into LDS) into the second buffer while block j's value products run: no
//   staging registers, one barrier per key block;
// * both tiles are stored row-major and unpadded, the 16-byte chunks of a row
//   XOR-swizzled by the row so that the operand reads hit 64 distinct banks:
//   the K operand is one 16-byte read per lane (16 key rows, one chunk each);
//   the V^T operand comes straight out of the row-major V tile through two
//   ds_read_b64_tr_b16 transpose reads. Within each 16-lane group, the lane
//   4a + b of a transpose read receives element b of the 8-byte pieces addressed
//   by lanes a, a+4, a+8, a+12 (checked on gfx950 with a lane-layout probe);
//   so when lane 4j + a of group g addresses V[4g + j][16 db + 4a ..], lane c of
//   the group receives V[4g + j][16 db + c] for j = 0..3: four keys of its head
//   dim, the operand slots of the value product.
// f(integral_constant<int, I>) for I = B .. E-1 in order: indices that are constants from the
// start, so register arrays indexed by them never go to scratch
template <int B, int E, typename F>
__device__ __forceinline__ void attn_static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    attn_static_for<B + 1, E>(f);
  }
}

// Used at head dim 128 from degree 3, where both kernels run one wave per SIMD. Elsewhere it
// measured slower: at d 64, K 4 its 263 registers cost the pipelined kernel's second wave per
// SIMD (0.54 against 0.38 ms at config 3's other sizes); at d 128, K 1..2 it was 1% slower.
template <int K, int D>
struct AttnHalfPipe {
  static constexpr int KB = 32;
  static constexpr int CH = D * 2 / 16;                 // 16-byte chunks per row
  static constexpr int RPS = 1024 / (D * 2);            // rows per 1 KB DMA segment
  static constexpr int SEGS = KB / RPS;                 // segments per order tile
  static constexpr int IT = (SEGS + kAttnWaves - 1) / kAttnWaves;   // per wave and order tile
  static constexpr int OPS = 2 * (K + 1) * IT;          // DMA operations per wave and key block
  static constexpr int RSH = CH >= 16 ? 0 : CH == 8 ? 1 : CH == 4 ? 2 : 3;   // log2(16 / CH)
  static constexpr size_t LDS = 2ull * 2 * (K + 1) * KB * D * 2;
  static constexpr bool split = AttnHalfShape<K, D>::split;
  static constexpr int R = 4;   // the value products' operand ring: reads run three items ahead
  // registers of the accumulators, query tile, scores, probability operands (hi, lo) and ring
  static constexpr int regs =
      (K + 1) * (D / 16 * 4 + (D + 31) / 32 * 4 + 8 + 4) + 4 * R + (split ? 4 * K : 0);
  static constexpr bool fits = LDS <= 160 * 1024 && regs <= 400;
  // Chunk swizzle of every tile (physical chunk = logical chunk ^ fs(row)). gfx950 serves a
  // 16-byte LDS read in four passes of 16 lanes ({0-3, 12-15, 20-27}, {4-11, 16-19, 28-31}, and
  // those plus 32) and an 8-byte or transpose read in two passes of 32 lanes (measured with a
  // two-lane LDS probe). Under that grouping fs makes both the row reads (one chunk of 16 rows
  // per 16-byte read: K, and the backward's row operands) and the transpose reads (8-byte pieces
  // of 2 chunks of 8 rows per 32 lanes: V, and the backward's transposed operands) hit 64
  // distinct banks at head dims 32, 64 and 128. (A swizzle by the row's low bits, row & (CH-1),
  // which the K tiles had used, left the transpose reads two-way conflicted.)
  __device__ __forceinline__ static int fs(int row) { return CH >= 4 ? 2 * ((row >> RSH) & (CH / 2 - 1)) : 0; }
};

// DMA operation i of this wave's share of key block kb0 into one buffer
// (tiles[kv][order][row][d]); i is a compile-time constant at every call. The
// resource spans exactly this head's S rows: rows past S are out of range and
// load as zeros, so a ragged last key block needs no branch.
template <typename T, int K, int D>
__device__ __forceinline__ void attn_half_issue_op(T (&buf)[2][K + 1][32][D], const CPtrs<T>& Kp,
                                                   const CPtrs<T>& Vp, int64_t head, int S, int kb0, int lane,
                                                   int wave, int i) {
  using P = AttnHalfPipe<K, D>;
  constexpr int CH = P::CH, RPS = P::RPS, SEGS = P::SEGS, IT = P::IT;
  const int kv = i / ((K + 1) * IT), o = (i / IT) % (K + 1), it = i % IT;
  const int seg = it * kAttnWaves + wave;
  if (SEGS % kAttnWaves != 0 && seg >= SEGS) return;
  const int row = seg * RPS + lane / CH;
  const int lch = (lane % CH) ^ P::fs(row);
  const BufferRsrc rsrc = buffer_rsrc((kv ? Vp.p[o] : Kp.p[o]) + head * S * D, S * D * static_cast<int>(sizeof(T)));
  lds_dma16(&buf[kv][o][seg * RPS][0], rsrc, ((kb0 + row) * D + lch * 8) * static_cast<int>(sizeof(T)));
}

// The pipelined kernels' epilogue: the row sums over the lane groups, O_k = (N_k - sum_{j=1..k} l_j
// O_{k-j}) / l_0 into the outputs, and the lse series (+inf and zeros for a row without keys).
template <typename T, int K, int DB>
__device__ __forceinline__ void attn_half_fwd_epilogue(floatx4 (&acc_o)[K + 1][DB], float (&lsum)[K + 1], float m_used,
                                                       MPtrs<T>& O, MPtrs<float>& LSE, int64_t head, int L, int my_q,
                                                       bool q_ok, int g) {
  using MM = HalfMfma<T>;
  constexpr int D = 16 * DB;
#pragma unroll
  for (int o = 0; o <= K; ++o) {
    lsum[o] = rows_sum(lsum[o]);
  }
  if (!q_ok) return;
  const bool empty = !(lsum[0] > 0.f);
  const float inv_l0 = empty ? 0.f : 1.f / lsum[0];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    float out[4][K + 1];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
      for (int k = 0; k <= K; ++k) {
        float t = acc_o[k][db][r];
#pragma unroll
        for (int jj = 1; jj <= k; ++jj) t -= lsum[jj] * out[r][k - jj];
        out[r][k] = t * inv_l0;
      }
    }
#pragma unroll
    for (int k = 0; k <= K; ++k)
      *reinterpret_cast<uint2*>(O.p[k] + (head * L + my_q) * D + 16 * db + 4 * g) =
          make_uint2(MM::pack2(out[0][k], out[1][k]), MM::pack2(out[2][k], out[3][k]));
  }
  if (LSE.p[0] != nullptr && g == 0) {
    const int64_t at = head * L + my_q;
    if (empty) {
      LSE.p[0][at] = __builtin_huge_valf();
#pragma unroll
      for (int k = 1; k <= K; ++k) LSE.p[k][at] = 0.f;
    } else {
      float lse[K + 1], nrm[K + 1];
      lse[0] = m_used + logf(lsum[0]);
#pragma unroll
      for (int k = 1; k <= K; ++k) nrm[k] = lsum[k] * inv_l0;
#pragma unroll
      for (int k = 1; k <= K; ++k) {
        float t = nrm[k];
#pragma unroll
        for (int jj = 1; jj < k; ++jj) t -= (static_cast<float>(jj) / static_cast<float>(k)) * lse[jj] * nrm[k - jj];
        lse[k] = t;
      }
#pragma unroll
      for (int k = 0; k <= K; ++k) LSE.p[k][at] = lse[k];
    }
  }
}

// MASK: 0 none (mask_all and madd_all unused), 1 a boolean mask, 2 an additive mask madd (float32
// values) with the boolean mask of its finite entries. Without a mask no mask memory is read.
template <typename T, int K, int D, int MASK>
__global__ __launch_bounds__(kAttnWaves * kWave) void taylor_attention_fwd_half_pipe_kernel(
    CPtrs<T> Q, CPtrs<T> Kp, CPtrs<T> Vp, MPtrs<T> O, MPtrs<float> LSE, int L, int S,
    const uint8_t* __restrict__ mask_all, AttnMaskMap mmap, const int32_t* __restrict__ ranges_all,
    const float* __restrict__ madd_all, int causal, float scale) {
  using P = AttnHalfPipe<K, D>;
  using MM = HalfMfma<T>;
  constexpr int KB = P::KB, DC = (D + 31) / 32, DB = D / 16, OPS = P::OPS;
  constexpr float kNegInf = -__builtin_huge_valf();
  constexpr float kSlack = MM::kSlack;
  static_assert(P::LDS <= 160 * 1024, "two K/V tiles exceed LDS");

  // two buffers of [0 = K, 1 = V][order][key row][head dim], rows unpadded and chunk-swizzled
  using Tiles = T[2][K + 1][KB][D];
  __shared__ __attribute__((aligned(16))) Tiles tiles[2];

  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int c = lane % 16;
  const int g = lane / 16;
  int64_t head;
  int q_block;
  attn_work_item(L, causal, head, q_block);
  // this head's mask, its block ranges (and additive values)
  const int64_t mask_index = attn_mask_index(mmap, head);
  const uint8_t* mask = mask_all != nullptr ? mask_all + mask_index * L * S : nullptr;
  const int32_t* ranges = ranges_all != nullptr ? ranges_all + mask_index * attn_ranges_count(L, S) : nullptr;
  constexpr bool ADD = MASK == 2;
  // The next block's DMA is issued in shares over the score products, so that it has the
  // exponential series and the value products to land before the next block's wait (over the
  // value products it left 0.98 ms at the config-3 shape, against 0.92). With an additive mask
  // the value products measured faster (1.91 against 2.10 ms on a padding mask).
  constexpr bool dma_in_scores = MASK != 2;
  const float* madd = ADD ? madd_all + mask_index * L * S : nullptr;
  const int my_q = q_block + wave * kAttnQPerWave + c;
  const bool q_ok = my_q < L;
  const int64_t qrow = (head * L + (q_ok ? my_q : L - 1)) * D;

  // the wave's query tile of every order, resident in registers
  u32x4 qreg[K + 1][DC];
#pragma unroll
  for (int o = 0; o <= K; ++o)
#pragma unroll
    for (int dc = 0; dc < DC; ++dc) {
      const bool din = 32 * dc + 8 * g < D;
      qreg[o][dc] = attn_half_load8<T>(Q.p[o] + qrow + (din ? 32 * dc + 8 * g : 0), din);
    }

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

  floatx4 acc_o[K + 1][DB];
#pragma unroll
  for (int o = 0; o <= K; ++o)
#pragma unroll
    for (int db = 0; db < DB; ++db) acc_o[o][db] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_used = kNegInf;
  float iscale[K + 1];   // i scale: the score series' factors in the exponential recurrence
#pragma unroll
  for (int i = 0; i <= K; ++i) iscale[i] = static_cast<float>(i) * scale;
  float lsum[K + 1];
#pragma unroll
  for (int o = 0; o <= K; ++o) lsum[o] = 0.f;

  // the first block's DMA is issued after the query loads: LDS-DMA loads pending
  // beside ordinary loads make the compiler wait for every load in flight
  // The mask bytes (and additive values) of a block are read one block ahead, before that
  // block's DMA is issued: loads complete in order, so a read issued at the top of its own block
  // would hold the block for a full memory round trip (the additive values come from L2 or HBM).
  // (one word of mask bytes per half: byte r for key kb0 + 16 kh + 4 g + r)
  uint32_t mnext[2] = {0u, 0u};
  float anext[ADD ? 2 : 1][4];
  const bool mvec = MASK != 0 && attn_mask_vec(mask, madd, S);
  auto fetch_mask = [&](int kb0) __attribute__((always_inline)) {
    if constexpr (MASK != 0) {
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
        mnext[kh] = attn_mask_word4<ADD>(mask, madd, my_q, kb0 + 16 * kh + 4 * g, L, S, mvec, anext[ADD ? kh : 0]);
    }
  };

#pragma unroll
  for (int i = 0; i < OPS; ++i) attn_half_issue_op<T, K, D>(tiles[0], Kp, Vp, head, S, lo, lane, wave, i);
  fetch_mask(lo);

  // key block j from buffer cur; the DMA of block j+1 into nxt
  auto block = [&](Tiles& cur, Tiles& nxt, int j) __attribute__((always_inline)) {
    const int kb0 = lo + j * KB;
    __builtin_amdgcn_s_waitcnt(0);   // this wave's DMA of block j has landed (and its mask reads)
    __syncthreads();                 // ... and every wave's; block j-1's buffer is free
    const uint32_t mword[2] = {mnext[0], mnext[1]};
    float add[ADD ? 2 : 1][4];   // additive mask values of the same keys
    if constexpr (ADD) {
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int r = 0; r < 4; ++r) add[kh][r] = anext[kh][r];
    }
    fetch_mask(min(kb0 + KB, last_kb0));   // the next block's, ahead of its DMA
    const int next_kb0 = min(kb0 + KB, last_kb0);

    // ---- scores S^T_k = sum_{a+b=k} K_b Q_a^T, two 16-key halves ----
    // Per step (chunk dc, half kh) the K+1 operands K_b (16-byte reads) are read one step ahead,
    // and the products are grouped by output order, S_k's k+1 products back to back: 2-3% faster
    // than operand by operand through a ring (K=4 at d=64 0.383 -> 0.373 ms, K=2 at d=128 0.458 ->
    // 0.448 ms), each accumulator summing in the same order (b ascending). Item t = (step, k)
    // carries its share of the next block's DMA.
    floatx4 sc[2][K + 1];
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int o = 0; o <= K; ++o) sc[kh][o] = floatx4{0.f, 0.f, 0.f, 0.f};
    constexpr int R = P::R;
    constexpr int KT = 2 * DC * (K + 1);
    auto load_k = [&](int t) {
      const int st = t / (K + 1), o = t % (K + 1);
      const int dc = st / 2, kh = st % 2;
      const int row = 16 * kh + c;
      const bool din = 32 * dc + 8 * g < D;
      const int pch = ((4 * dc + g) & (P::CH - 1)) ^ P::fs(row);
      const u32x4 v = *reinterpret_cast<const u32x4*>(&cur[0][o][row][pch * 8]);
      const u32x4 z = {0u, 0u, 0u, 0u};
      return din ? v : z;
    };
    constexpr int NS = 2 * DC;
    u32x4 kop[2][K + 1];
#pragma unroll
    for (int o = 0; o <= K; ++o) kop[0][o] = load_k(o);
    attn_static_for<0, NS>([&](auto sc_) __attribute__((always_inline)) {
      constexpr int st = decltype(sc_)::value;
      constexpr int dc = st / 2, kh = st % 2;
      if constexpr (st + 1 < NS) {
#pragma unroll
        for (int o = 0; o <= K; ++o) kop[(st + 1) & 1][o] = load_k((st + 1) * (K + 1) + o);
      }
      attn_static_for<0, K + 1>([&](auto kc) __attribute__((always_inline)) {
        constexpr int k = decltype(kc)::value;
        constexpr int t = st * (K + 1) + k;
        if constexpr (dma_in_scores) {
          attn_static_for<t * OPS / KT, (t + 1) * OPS / KT>([&](auto ic) __attribute__((always_inline)) {
            attn_half_issue_op<T, K, D>(nxt, Kp, Vp, head, S, next_kb0, lane, wave, decltype(ic)::value);
          });
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int b = 0; b <= k; ++b) sc[kh][k] = MM::mma(kop[st & 1][b], qreg[k - b][dc], sc[kh][k]);
        __builtin_amdgcn_sched_barrier(0);
      });
    });

    // ---- mask, online maximum of the constant order, exponential series ----
    bool valid[2][4];
    float s0[2][4];
    float bmax = kNegInf;
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kb0 + 16 * kh + 4 * g + r;
        bool ok = q_ok && key < hi;
        if (causal) ok = ok && key <= my_q;
        if constexpr (MASK != 0) ok = ok && ((mword[kh] >> (8 * r)) & 0xffu) != 0;
        valid[kh][r] = ok;
        float sv = sc[kh][0][r] * scale;
        if constexpr (ADD) sv += add[kh][r];
        s0[kh][r] = ok ? sv : kNegInf;
        bmax = fmaxf(bmax, s0[kh][r]);
      }
    bmax = rows_max(bmax);
    const bool raise = bmax > m_used + kSlack || (m_used == kNegInf && bmax != kNegInf);
    if (__any(raise)) {
      const float m_new = raise ? bmax : m_used;
      const float alpha = (raise && m_used != kNegInf) ? exp_fast(m_used - m_new) : (raise ? 0.f : 1.f);
#pragma unroll
      for (int o = 0; o <= K; ++o) {
        lsum[o] *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          // out of and back into the accumulation registers here, on this rare path, so that
          // the accumulators keep one register class across the loop (no copies per block)
          asm volatile("" : "+a"(acc_o[o][db]));
#pragma unroll
          for (int r = 0; r < 4; ++r) acc_o[o][db][r] *= alpha;
          asm volatile("" : "+a"(acc_o[o][db]));
        }
      }
      m_used = m_new;
    }
    u32x4 pb[K + 1];
    u32x4 pl[P::split ? K + 1 : 1];   // lo parts of orders 1..K (split)
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      float w[K + 1][4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        // the weights w_k = p e_k directly: w_0 = p, w_k = (1/k) sum_i b_i w_{k-i}, b_i = i scale S_i
        float b[K + 1];
#pragma unroll
        for (int o = 1; o <= K; ++o) b[o] = sc[kh][o][r] * iscale[o];
        w[0][r] = valid[kh][r] ? exp_fast(s0[kh][r] - m_used) : 0.f;
#pragma unroll
        for (int k = 1; k <= K; ++k) {
          float t = b[1] * w[k - 1][r];
#pragma unroll
          for (int i = 2; i <= k; ++i) t = fmaf(b[i], w[k - i][r], t);
          w[k][r] = t * (1.f / static_cast<float>(k));
        }
      }
#pragma unroll
      for (int o = 0; o <= K; ++o) {
        const uint32_t w01 = MM::pack2(w[o][0], w[o][1]), w23 = MM::pack2(w[o][2], w[o][3]);
        pb[o][2 * kh] = w01;
        pb[o][2 * kh + 1] = w23;
        // the row sums add the weights as rounded for the value products
        lsum[o] = MM::sum2(w23, MM::sum2(w01, lsum[o]));
        if constexpr (P::split) {
          if (o >= 1) {
            pl[o][2 * kh] = MM::pack2(w[o][0] - MM::lo(w01), w[o][1] - MM::hi(w01));
            pl[o][2 * kh + 1] = MM::pack2(w[o][2] - MM::lo(w23), w[o][3] - MM::hi(w23));
            lsum[o] = MM::sum2(pl[o][2 * kh + 1], MM::sum2(pl[o][2 * kh], lsum[o]));
          }
        }
      }
    }

    // ---- O^T_k += sum_{a+b=k} V_b^T P_a^T ----
    // Items t = (db, b): one V_b^T operand (two transpose reads) feeds the K+1-b products
    // O_{a+b} += V_b^T P_a^T (and those of the lo parts); the reads run R-1 items ahead. Where the
    // DMA is issued here, a share of the next block's per item (the last block re-loads itself,
    // so there is no branch).
    const int tj = c / 4, ta = c % 4;   // this lane's piece: row 4g + tj (+16), head dims 16 db + 4 ta
    auto load_v = [&](int t) {
      const int db = t / (K + 1), o = t % (K + 1);
      const int row0 = 4 * g + tj, row1 = 16 + 4 * g + tj;
      const int lch = 2 * db + ta / 2;
      const int off0 = ((lch ^ P::fs(row0)) * 8) + 4 * (ta % 2);
      const int off1 = ((lch ^ P::fs(row1)) * 8) + 4 * (ta % 2);
      return lds_read_tr16x2(&cur[1][o][row0][off0], &cur[1][o][row1][off1]);
    };
    constexpr int VT = DB * (K + 1);
    u32x4 vring[R];
#pragma unroll
    for (int t = 0; t < R - 1 && t < VT; ++t) vring[t] = load_v(t);
#pragma unroll
    for (int t = 0; t < VT; ++t) {
      if (t + R - 1 < VT) vring[(t + R - 1) % R] = load_v(t + R - 1);
      if constexpr (!dma_in_scores) {
#pragma unroll
        for (int i = t * OPS / VT; i < (t + 1) * OPS / VT; ++i)
          attn_half_issue_op<T, K, D>(nxt, Kp, Vp, head, S, next_kb0, lane, wave, i);
      }
      __builtin_amdgcn_sched_barrier(0);
      const int db = t / (K + 1), bo = t % (K + 1);
#pragma unroll
      for (int a = 0; a + bo <= K; ++a) acc_o[a + bo][db] = MM::mma(vring[t % R], pb[a], acc_o[a + bo][db]);
      if constexpr (P::split) {
#pragma unroll
        for (int a = 1; a + bo <= K; ++a) acc_o[a + bo][db] = MM::mma(vring[t % R], pl[a], acc_o[a + bo][db]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  for (int j = 0; j < nblocks; ++j) block(tiles[j & 1], tiles[(j + 1) & 1], j);
  __builtin_amdgcn_s_waitcnt(0);   // the last block's (redundant) DMA has landed before the workgroup ends

  attn_half_fwd_epilogue<T, K, DB>(acc_o, lsum, m_used, O, LSE, head, L, my_q, q_ok, g);
}

// Software-pipelined form of the kernel above for degrees 3..4 at head dim 128 (one probability
// operand per order). Iteration j forms key block j+1's scores and, between those products, runs block j's
// exponential series (VALU work that issues while the MFMAs execute), then block j's value
// products. The series of a block is cut into units, one order of one row each, spread evenly
// over the next block's score items.
// Buffers: the K tile of block j+2 goes where block j's K tile was (read by the previous
// iteration's scores), the V tile of block j+1 where block j-1's was; both are issued at the top of
// iteration j and waited for at the top of iteration j+1.
template <int K, int D>
struct AttnHalfSw {
  static constexpr bool fits = AttnHalfPipe<K, D>::fits && !AttnHalfPipe<K, D>::split && D == 128 && K >= 3;
};

template <typename T, int K, int D, int MASK>
__global__ __launch_bounds__(kAttnWaves * kWave) void taylor_attention_fwd_half_sw_kernel(
    CPtrs<T> Q, CPtrs<T> Kp, CPtrs<T> Vp, MPtrs<T> O, MPtrs<float> LSE, int L, int S,
    const uint8_t* __restrict__ mask_all, AttnMaskMap mmap, const int32_t* __restrict__ ranges_all,
    const float* __restrict__ madd_all, int causal, float scale) {
  using P = AttnHalfPipe<K, D>;
  using MM = HalfMfma<T>;
  constexpr int KB = P::KB, DC = (D + 31) / 32, DB = D / 16, OPS = P::OPS, KOPS = OPS / 2;
  constexpr float kNegInf = -__builtin_huge_valf();
  constexpr float kSlack = MM::kSlack;
  constexpr bool ADD = MASK == 2;
  static_assert(P::LDS <= 160 * 1024 && !P::split, "two K/V tiles within LDS, one operand per order");

  using Tiles = T[2][K + 1][KB][D];
  __shared__ __attribute__((aligned(16))) Tiles tiles[2];

  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int c = lane % 16;
  const int g = lane / 16;
  int64_t head;
  int q_block;
  attn_work_item(L, causal, head, q_block);
  const int64_t mask_index = attn_mask_index(mmap, head);
  const uint8_t* mask = mask_all != nullptr ? mask_all + mask_index * L * S : nullptr;
  const int32_t* ranges = ranges_all != nullptr ? ranges_all + mask_index * attn_ranges_count(L, S) : nullptr;
  const float* madd = ADD ? madd_all + mask_index * L * S : nullptr;
  const int my_q = q_block + wave * kAttnQPerWave + c;
  const bool q_ok = my_q < L;
  const int64_t qrow = (head * L + (q_ok ? my_q : L - 1)) * D;

  u32x4 qreg[K + 1][DC];
#pragma unroll
  for (int o = 0; o <= K; ++o)
#pragma unroll
    for (int dc = 0; dc < DC; ++dc) {
      const bool din = 32 * dc + 8 * g < D;
      qreg[o][dc] = attn_half_load8<T>(Q.p[o] + qrow + (din ? 32 * dc + 8 * g : 0), din);
    }

  int lo = 0, hi = S;
  if (causal) hi = min(S, q_block + kAttnBM);
  if (ranges != nullptr) {
    const int qb = q_block / kAttnRangeBlock;
    lo = ranges[2 * qb] / KB * KB;
    hi = min(hi, static_cast<int>(ranges[2 * qb + 1]));
  }
  if (hi <= lo) lo = hi = 0;
  const int nblocks = max(1, (hi - lo + KB - 1) / KB);
  const int last_kb0 = lo + (nblocks - 1) * KB;
  auto kb_of = [&](int j) { return min(lo + j * KB, last_kb0); };   // past the end: the last block again

  floatx4 acc_o[K + 1][DB];
#pragma unroll
  for (int o = 0; o <= K; ++o)
#pragma unroll
    for (int db = 0; db < DB; ++db) acc_o[o][db] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_used = kNegInf;
  float iscale[K + 1];
#pragma unroll
  for (int i = 0; i <= K; ++i) iscale[i] = static_cast<float>(i) * scale;
  float lsum[K + 1];
#pragma unroll
  for (int o = 0; o <= K; ++o) lsum[o] = 0.f;

  // (one word of mask bytes per half: byte r for key kb0 + 16 kh + 4 g + r)
  uint32_t mnext[2] = {0u, 0u};
  float anext[ADD ? 2 : 1][4];
  const bool mvec = MASK != 0 && attn_mask_vec(mask, madd, S);
  auto fetch_mask = [&](int kb0) __attribute__((always_inline)) {
    if constexpr (MASK != 0) {
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
        mnext[kh] = attn_mask_word4<ADD>(mask, madd, my_q, kb0 + 16 * kh + 4 * g, L, S, mvec, anext[ADD ? kh : 0]);
    }
  };

  // ---- scores S^T_k = sum_{a+b=k} K_b Q_a^T of the block in buffer kt, two 16-key halves ----
  // Per step (chunk dc, half kh) the K+1 operands K_b are read one step ahead; the products are
  // grouped by output order, S_k's k+1 products back to back (0.843 against 0.863 ms at the
  // config-3 shape operand by operand). Item t = (step, k) runs extra(t), the other work of the
  // item (DMA shares and series units), before the order's products, which execute while it
  // issues. Each accumulator sums its products in the same order either way (b ascending).
  constexpr int KT = 2 * DC * (K + 1);
  auto scores = [&](Tiles& kt, floatx4 (&s)[2][K + 1], auto&& extra) __attribute__((always_inline)) {
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int o = 0; o <= K; ++o) s[kh][o] = floatx4{0.f, 0.f, 0.f, 0.f};
    auto load_k = [&](int t) {
      const int st = t / (K + 1), o = t % (K + 1);
      const int dc = st / 2, kh = st % 2;
      const int row = 16 * kh + c;
      const bool din = 32 * dc + 8 * g < D;
      const int pch = ((4 * dc + g) & (P::CH - 1)) ^ P::fs(row);
      const u32x4 v = *reinterpret_cast<const u32x4*>(&kt[0][o][row][pch * 8]);
      const u32x4 z = {0u, 0u, 0u, 0u};
      return din ? v : z;
    };
    constexpr int NS = 2 * DC;
    u32x4 kop[2][K + 1];
#pragma unroll
    for (int o = 0; o <= K; ++o) kop[0][o] = load_k(o);
    attn_static_for<0, NS>([&](auto sc_) __attribute__((always_inline)) {
      constexpr int st = decltype(sc_)::value;
      constexpr int dc = st / 2, kh = st % 2;
      if constexpr (st + 1 < NS) {
#pragma unroll
        for (int o = 0; o <= K; ++o) kop[(st + 1) & 1][o] = load_k((st + 1) * (K + 1) + o);
      }
      attn_static_for<0, K + 1>([&](auto kc) __attribute__((always_inline)) {
        constexpr int k = decltype(kc)::value;
        extra(std::integral_constant<int, st * (K + 1) + k>{});
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int b = 0; b <= k; ++b) s[kh][k] = MM::mma(kop[st & 1][b], qreg[k - b][dc], s[kh][k]);
        __builtin_amdgcn_sched_barrier(0);
      });
    });
  };

  // ---- O^T_k += sum_{a+b=k} V_b^T P_a^T of the block in buffer vt ----
  // Grouped by output order as the scores, per 16-wide output block db; the next block's K+1
  // operands (two transpose reads each) are read one per order group, so the reads spread over
  // the products: 1.3% faster than operand by operand through a ring (read all at the group's
  // start, they were 2% slower).
  const int tj = c / 4, ta = c % 4;
  auto values = [&](Tiles& vt, const u32x4 (&pb)[K + 1]) __attribute__((always_inline)) {
    auto load_v = [&](int t) {
      const int db = t / (K + 1), o = t % (K + 1);
      const int row0 = 4 * g + tj, row1 = 16 + 4 * g + tj;
      const int lch = 2 * db + ta / 2;
      const int off0 = ((lch ^ P::fs(row0)) * 8) + 4 * (ta % 2);
      const int off1 = ((lch ^ P::fs(row1)) * 8) + 4 * (ta % 2);
      return lds_read_tr16x2(&vt[1][o][row0][off0], &vt[1][o][row1][off1]);
    };
    u32x4 vop[2][K + 1];
#pragma unroll
    for (int o = 0; o <= K; ++o) vop[0][o] = load_v(o);
    attn_static_for<0, DB>([&](auto dc_) __attribute__((always_inline)) {
      constexpr int db = decltype(dc_)::value;
      attn_static_for<0, K + 1>([&](auto kc) __attribute__((always_inline)) {
        constexpr int k = decltype(kc)::value;
        if constexpr (db + 1 < DB) {   // one operand of the next block db + 1 per order group
          vop[(db + 1) & 1][k] = load_v((db + 1) * (K + 1) + k);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int b = 0; b <= k; ++b) acc_o[k][db] = MM::mma(vop[db & 1][b], pb[k - b], acc_o[k][db]);
        __builtin_amdgcn_sched_barrier(0);
      });
    });
  };

  floatx4 scc[2][K + 1], scn[2][K + 1];   // scores of the block in its series, and of the next

  // prologue: block 0's tiles, block 1's K tile, block 0's mask values; block 0's scores
#pragma unroll
  for (int i = 0; i < OPS; ++i) attn_half_issue_op<T, K, D>(tiles[0], Kp, Vp, head, S, lo, lane, wave, i);
#pragma unroll
  for (int i = 0; i < KOPS; ++i) attn_half_issue_op<T, K, D>(tiles[1], Kp, Vp, head, S, kb_of(1), lane, wave, i);
  fetch_mask(lo);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  scores(tiles[0], scc, [&](auto) {});

  // iteration j: block j's series and value products, block j+1's scores (LAST: none)
  auto step = [&](int j, auto last) __attribute__((always_inline)) {
    constexpr bool LAST = decltype(last)::value;
    Tiles& cur = tiles[j & 1];
    Tiles& nxt = tiles[(j + 1) & 1];
    const int kb0 = lo + j * KB;
    __builtin_amdgcn_s_waitcnt(0);   // this wave's K(j+1), V(j) and mask values of block j have landed
    __syncthreads();                 // ... every wave's; K(j) and V(j-1) are no longer read
    const uint32_t mword[2] = {mnext[0], mnext[1]};
    float add[ADD ? 2 : 1][4];
    if constexpr (ADD) {
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int r = 0; r < 4; ++r) add[kh][r] = anext[kh][r];
    }
    if constexpr (!LAST) fetch_mask(kb_of(j + 1));

    // ---- mask, online maximum of the constant order (rescale on a raise) ----
    bool valid[2][4];
    float s0[2][4];
    float bmax = kNegInf;
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kb0 + 16 * kh + 4 * g + r;
        bool ok = q_ok && key < hi;
        if (causal) ok = ok && key <= my_q;
        if constexpr (MASK != 0) ok = ok && ((mword[kh] >> (8 * r)) & 0xffu) != 0;
        valid[kh][r] = ok;
        float sv = scc[kh][0][r] * scale;
        if constexpr (ADD) sv += add[kh][r];
        s0[kh][r] = ok ? sv : kNegInf;
        bmax = fmaxf(bmax, s0[kh][r]);
      }
    bmax = rows_max(bmax);
    const bool raise = bmax > m_used + kSlack || (m_used == kNegInf && bmax != kNegInf);
    if (__any(raise)) {
      const float m_new = raise ? bmax : m_used;
      const float alpha = (raise && m_used != kNegInf) ? exp_fast(m_used - m_new) : (raise ? 0.f : 1.f);
#pragma unroll
      for (int o = 0; o <= K; ++o) {
        lsum[o] *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          asm volatile("" : "+a"(acc_o[o][db]));
#pragma unroll
          for (int r = 0; r < 4; ++r) acc_o[o][db][r] *= alpha;
          asm volatile("" : "+a"(acc_o[o][db]));
        }
      }
      m_used = m_new;
    }

    // ---- the series in units: unit u is order u % (K+1) of row u / (K+1) (half row / 4, key
    // register row % 4); after the last order of an odd row the row pair is packed ----
    u32x4 pb[K + 1];
    float bser[K + 1];
    float wrow[2][K + 1];
    auto unit = [&](auto uc) __attribute__((always_inline)) {
      constexpr int u = decltype(uc)::value;
      constexpr int row = u / (K + 1), k = u % (K + 1);
      constexpr int kh = row / 4, r = row % 4;
      if constexpr (k == 0) {
#pragma unroll
        for (int o = 1; o <= K; ++o) bser[o] = scc[kh][o][r] * iscale[o];
        wrow[r & 1][0] = valid[kh][r] ? exp_fast(s0[kh][r] - m_used) : 0.f;
      } else {
        float t = bser[1] * wrow[r & 1][k - 1];
#pragma unroll
        for (int i = 2; i <= k; ++i) t = fmaf(bser[i], wrow[r & 1][k - i], t);
        wrow[r & 1][k] = t * (1.f / static_cast<float>(k));
      }
      if constexpr (k == K && (r & 1)) {
        // the row sums add the weights as rounded for the value products
#pragma unroll
        for (int o = 0; o <= K; ++o) {
          const uint32_t w2 = MM::pack2(wrow[0][o], wrow[1][o]);
          pb[o][2 * kh + r / 2] = w2;
          lsum[o] = MM::sum2(w2, lsum[o]);
        }
      }
    };
    constexpr int U = 8 * (K + 1);
    if constexpr (LAST) {
      attn_static_for<0, U>(unit);
    } else {
      const int kb_k = kb_of(j + 2), kb_v = kb_of(j + 1);
      scores(nxt, scn, [&](auto tc) __attribute__((always_inline)) {
        constexpr int t = decltype(tc)::value;
        // K(j+2) into this block's K tile, V(j+1) into the other buffer's V tile
        attn_static_for<t * OPS / KT, (t + 1) * OPS / KT>([&](auto ic) __attribute__((always_inline)) {
          constexpr int i = decltype(ic)::value;
          if constexpr (i < KOPS) attn_half_issue_op<T, K, D>(cur, Kp, Vp, head, S, kb_k, lane, wave, i);
          else attn_half_issue_op<T, K, D>(nxt, Kp, Vp, head, S, kb_v, lane, wave, i);
        });
        attn_static_for<t * U / KT, (t + 1) * U / KT>(unit);
      });
    }
    values(cur, pb);
    if constexpr (!LAST) {
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int o = 0; o <= K; ++o) scc[kh][o] = scn[kh][o];
    }
  };
  for (int j = 0; j + 1 < nblocks; ++j) step(j, std::false_type{});
  step(nblocks - 1, std::true_type{});
  __builtin_amdgcn_s_waitcnt(0);   // the redundant K DMA of the last iterations has landed before the workgroup ends

  attn_half_fwd_epilogue<T, K, DB>(acc_o, lsum, m_used, O, LSE, head, L, my_q, q_ok, g);
}

template <typename T, int K, int D>
static int launch_attention_half_kd(const AttnArgs& a) {
  if constexpr (!AttnHalfShape<K, D>::fits) {
    pt_host::set_error("Taylor attention: degree and head dim exceed the LDS budget for this dtype");
    return PT_UNSUPPORTED;
  } else {
    // 16-byte operand loads and 8-byte output stores
    bool aligned = true;
    for (int i = 0; i < a.q_orders; ++i) aligned = aligned && pt_host::aligned16(a.q[i]);
    for (int i = 0; i < a.k_orders; ++i) aligned = aligned && pt_host::aligned16(a.k[i]);
    for (int i = 0; i < a.v_orders; ++i) aligned = aligned && pt_host::aligned16(a.v[i]);
    for (int i = 0; i <= K; ++i) aligned = aligned && (reinterpret_cast<uintptr_t>(a.out[i]) % 8 == 0);
    PT_REQUIRE(aligned, PT_INVALID_ARGUMENT,
               "Taylor attention: 16-bit operands must be 16-byte aligned and outputs 8-byte aligned");
    CPtrs<T> q{}, k{}, v{};
    MPtrs<T> o{};
    MPtrs<float> lse{};
    const float* madd = static_cast<const float*>(a.mask_add);   // float32 values for 16-bit operands
    for (int i = 0; i < a.q_orders; ++i) q.p[i] = static_cast<const T*>(a.q[i]);
    for (int i = 0; i < a.k_orders; ++i) k.p[i] = static_cast<const T*>(a.k[i]);
    for (int i = 0; i < a.v_orders; ++i) v.p[i] = static_cast<const T*>(a.v[i]);
    for (int i = 0; i <= K; ++i) {
      o.p[i] = static_cast<T*>(a.out[i]);
      if (a.lse != nullptr) lse.p[i] = static_cast<float*>(a.lse[i]);
    }
    if constexpr (AttnHalfPipe<K, D>::fits) {
      // full-order operands and a head's K / V rows (plus one block) addressable with 32-bit offsets
      const int64_t head_bytes = (a.lk + 32) * D * static_cast<int64_t>(sizeof(T));
      const bool pipe = a.q_orders == K + 1 && a.k_orders == K + 1 && a.v_orders == K + 1 && a.lk >= 1 &&
                        head_bytes < (int64_t{1} << 31);
      if (pipe) {
        const dim3 grid(static_cast<unsigned>((a.lq + kAttnBM - 1) / kAttnBM * a.bh));
#define PT_HALF_PIPE(KERNEL, ADDV)                                                                             \
  KERNEL<T, K, D, ADDV><<<grid, dim3(kAttnWaves * kWave), 0, a.stream>>>(                                      \
      q, k, v, o, lse, static_cast<int>(a.lq), static_cast<int>(a.lk), a.mask, a.mask_map, a.mask_ranges, madd, \
      a.causal ? 1 : 0, static_cast<float>(a.scale))
        if constexpr (AttnHalfSw<K, D>::fits) {
          if (madd != nullptr) PT_HALF_PIPE(taylor_attention_fwd_half_sw_kernel, 2);
          else if (a.mask != nullptr) PT_HALF_PIPE(taylor_attention_fwd_half_sw_kernel, 1);
          else PT_HALF_PIPE(taylor_attention_fwd_half_sw_kernel, 0);
        } else {
          if (madd != nullptr) PT_HALF_PIPE(taylor_attention_fwd_half_pipe_kernel, 2);
          else if (a.mask != nullptr) PT_HALF_PIPE(taylor_attention_fwd_half_pipe_kernel, 1);
          else PT_HALF_PIPE(taylor_attention_fwd_half_pipe_kernel, 0);
        }
#undef PT_HALF_PIPE
        PT_LAUNCH_CHECK();
        return PT_OK;
      }
    }
    const dim3 grid(static_cast<unsigned>((a.lq + kAttnBM - 1) / kAttnBM * a.bh * AttnHalfShape<K, D>::SL));
#define PT_HALF_STAGED(ADDV)                                                                                   \
  taylor_attention_fwd_half_kernel<T, K, D, ADDV><<<grid, dim3(kAttnWaves * kWave), 0, a.stream>>>(           \
      q, a.q_orders, k, a.k_orders, v, a.v_orders, o, lse, static_cast<int>(a.lq), static_cast<int>(a.lk),     \
      a.mask, a.mask_map, a.mask_ranges, madd, a.causal ? 1 : 0, static_cast<float>(a.scale))
    if (madd != nullptr) PT_HALF_STAGED(true);
    else PT_HALF_STAGED(false);
#undef PT_HALF_STAGED
    PT_LAUNCH_CHECK();
    return PT_OK;
  }
}

template <typename T, int K>
static int launch_attention_half_k(const AttnArgs& a) {
  switch (a.d) {
    case 16: return launch_attention_half_kd<T, K, 16>(a);
    case 32: return launch_attention_half_kd<T, K, 32>(a);
    case 64: return launch_attention_half_kd<T, K, 64>(a);
    case 128: return launch_attention_half_kd<T, K, 128>(a);
    default: break;
  }
  pt_host::set_error("Taylor attention: head dim must be 16, 32, 64 or 128");
  return PT_UNSUPPORTED;
}

template <typename T>
int launch_attention_half(const AttnArgs& a) {
  switch (a.degree) {
    case 0: return launch_attention_half_k<T, 0>(a);
    case 1: return launch_attention_half_k<T, 1>(a);
    case 2: return launch_attention_half_k<T, 2>(a);
    case 3: return launch_attention_half_k<T, 3>(a);
    case 4: return launch_attention_half_k<T, 4>(a);
    case 5: return launch_attention_half_k<T, 5>(a);
    case 6: return launch_attention_half_k<T, 6>(a);
    case 7: return launch_attention_half_k<T, 7>(a);
    case 8: return launch_attention_half_k<T, 8>(a);
    default: break;
  }
  pt_host::set_error("Taylor attention: degree outside 0..PT_MAX_DEGREE");
  return PT_UNSUPPORTED;
}

}  // namespace pt
