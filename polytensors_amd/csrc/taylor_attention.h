// Launch interface of the Taylor attention kernels (definitions in taylor_attention.inl).
#pragma once

#include <algorithm>

#include "pt_common.h"

namespace pt {

constexpr int kAttnWaves = 4;
constexpr int kAttnQPerWave = 16;
constexpr int kAttnBM = kAttnWaves * kAttnQPerWave;   // query rows per workgroup
constexpr int kAttnBN = 16;                           // keys per block of the fp32/fp64 kernels

// Output head-dim slices of the staged kernel (a grid dimension; each slice's workgroup
// recomputes the scores and accumulates D / SL output dims) where K+1 sets of output
// accumulators over the whole head dim would spill the register file: float64 at head dim 128
// from degree 3 and 64 from degree 6, float32 at head dim 128 from degree 6 (checked with the
// compiler's resource remarks). elem = sizeof(T).
__host__ __device__ constexpr int attn_slices(int elem, int K, int D) {
  return elem == 8 ? (D == 128 ? (K >= 6 ? 4 : K >= 3 ? 2 : 1) : D == 64 && K >= 6 ? 2 : 1)
                   : (D == 128 && K >= 6 ? 2 : 1);
}

// Which of a set of (L, S) masks a head uses: head b (0 .. bh-1) takes mask
// (b / div) * outer + (b % div) * inner. One shared mask: {1, 0, 0}; masks per
// batch over H heads each ([B, 1, L, S]): {H, 1, 0}; per head of each batch
// ([1, H, L, S]): {H, 0, 1}; one per head ([bh, L, S]): {1, 1, 0}.
struct AttnMaskMap {
  int64_t div = 1, outer = 0, inner = 0;
};

__host__ __device__ inline int64_t attn_mask_index(const AttnMaskMap& m, int64_t head) {
  return (head / m.div) * m.outer + (head % m.div) * m.inner;
}

// int32 entries of one mask's block ranges (launch_attention_mask_ranges): a (lo, hi)
// pair per 64-row query block, then per 64-key block.
__host__ __device__ constexpr int64_t attn_ranges_count(int64_t lq, int64_t lk) {
  return 2 * ((lq + 63) / 64 + (lk + 63) / 64);
}

struct AttnArgs {
  int degree;
  const void* const* q;
  int q_orders;
  const void* const* k;
  int k_orders;
  const void* const* v;
  int v_orders;
  void* const* out;
  void* const* lse;
  int64_t bh, lq, lk, d;
  bool causal;
  const uint8_t* mask;
  const int32_t* mask_ranges;   // null, or the block ranges of mask (launch_attention_mask_ranges)
  double scale;
  hipStream_t stream;
  void* workspace = nullptr;   // partial sums of a key-split launch (attention_split), or null
  size_t workspace_bytes = 0;
  // null, or an (L, S) additive mask in the accumulator type (float32/float64 operands only),
  // with mask its finite entries
  const void* mask_add = nullptr;
  AttnMaskMap mask_map{};   // mask (mask_ranges, mask_add) of each head, from a set of masks
};

template <typename T>
int launch_attention(const AttnArgs& a);

// Key split of the staged float32/float64 kernel for launches with few workgroups: `chunks`
// workgroups per work item, each over `chunk_keys` consecutive keys, whose partial sums
// (bytes of workspace) a second kernel merges. chunks = 1: no split. The pipelined float32
// kernel (full-order operands, whole 16-key blocks) and the 16-bit kernels never split.
struct AttnSplit {
  int chunks = 1, chunk_keys = 0;
  size_t bytes = 0;
};

// dtype: PT_FLOAT32 / PT_FLOAT64 (others never split). A launch of fewer than 128 workgroups
// takes up to 256 / workgroups key shares of at least one 16-key block each.
inline AttnSplit attention_split(int dtype, int degree, int q_orders, int k_orders, int v_orders, int64_t bh,
                                 int64_t lq, int64_t lk, int64_t d) {
  AttnSplit sp;
  if (dtype != PT_FLOAT32 && dtype != PT_FLOAT64) return sp;
  const bool full = q_orders == degree + 1 && k_orders == degree + 1 && v_orders == degree + 1;
  if (dtype == PT_FLOAT32 && full && lk >= kAttnBN && lk % kAttnBN == 0) return sp;   // the pipelined kernel
  const int elem = dtype == PT_FLOAT64 ? 8 : 4;
  const int64_t items = (lq + kAttnBM - 1) / kAttnBM * bh * attn_slices(elem, degree, static_cast<int>(d));
  const int64_t nkb = (lk + kAttnBN - 1) / kAttnBN;
  if (items >= 128 || nkb < 2 || items == 0) return sp;
  int64_t chunks = std::min<int64_t>((256 + items - 1) / items, nkb);
  const int64_t per = (nkb + chunks - 1) / chunks;   // key blocks per share
  chunks = (nkb + per - 1) / per;
  if (chunks < 2) return sp;
  sp.chunks = static_cast<int>(chunks);
  sp.chunk_keys = static_cast<int>(per * kAttnBN);
  const int64_t rows = bh * lq;
  sp.bytes = static_cast<size_t>(chunks) * static_cast<size_t>(rows) * static_cast<size_t>(1 + (degree + 1) * (1 + d)) *
             static_cast<size_t>(elem);
  return sp;
}

inline AttnSplit attention_split(const AttnArgs& a, int dtype) {
  return attention_split(dtype, a.degree, a.q_orders, a.k_orders, a.v_orders, a.bh, a.lq, a.lk, a.d);
}

// bfloat16 / float16 operands on the 16x16x32 MFMAs (taylor_attention_half.inl); T = bf16 or _Float16.
template <typename T>
int launch_attention_half(const AttnArgs& a);

// Block ranges of n_masks boolean (L, S) masks ([n_masks, L, S]) into ranges[n_masks *
// attention_mask_ranges_count(L, S)].
int64_t attention_mask_ranges_count(int64_t lq, int64_t lk);
int launch_attention_mask_ranges(const uint8_t* mask, int64_t n_masks, int64_t lq, int64_t lk, int32_t* ranges,
                                 hipStream_t stream);

// Backward: every series has degree+1 orders; dq/dk/dv may be null (not
// computed). workspace holds (degree+1) * bh * lq accumulator-type values.
struct AttnBwdArgs {
  int degree;
  const void* const* q;
  const void* const* k;
  const void* const* v;
  const void* const* out;
  const void* const* lse;
  const void* const* grad;
  void* const* dq;
  void* const* dk;
  void* const* dv;
  void* workspace;
  int64_t bh, lq, lk, d;
  bool causal;
  const uint8_t* mask;
  const int32_t* mask_ranges;
  double scale;
  bool materialize;   // store P and dS tiles in the workspace (5 products per pair instead of 8)
  hipStream_t stream;
  // null, or an (L, S) additive mask in the accumulator type with mask its finite entries (the
  // scores are then recomputed: materialize does not apply)
  const void* mask_add = nullptr;
  AttnMaskMap mask_map{};
};

template <typename T>
int launch_attention_bwd(const AttnBwdArgs& a);
// bfloat16 / float16 operands (16-bit MFMA, fp32 accumulation; lse in float32)
template <typename T>
int launch_attention_bwd_half(const AttnBwdArgs& a);

// Workspace of the backward: the rowsum(G O) series ((K+1) bh lq accumulator
// values), then, when materializing, the P and dS tiles of every order
// ((K+1) x 2 buffers of bh x ceil(lq/16) x ceil(lk/16) tiles of 256 values).
struct AttnBwdLayout {
  size_t delta_bytes, tiles_offset, tile_bytes, total;
};

inline AttnBwdLayout attention_bwd_layout(size_t acc_size, size_t elem_size, int degree, int64_t bh, int64_t lq,
                                          int64_t lk, bool materialize = true) {
  AttnBwdLayout l{};
  l.delta_bytes = static_cast<size_t>(degree + 1) * static_cast<size_t>(bh) * static_cast<size_t>(lq) * acc_size;
  l.tiles_offset = (l.delta_bytes + 255) / 256 * 256;
  const size_t tiles = static_cast<size_t>(bh) * static_cast<size_t>((lq + 15) / 16) * static_cast<size_t>((lk + 15) / 16);
  l.tile_bytes = (tiles * 256 * elem_size + 255) / 256 * 256;
  l.total = materialize ? l.tiles_offset + 2 * static_cast<size_t>(degree + 1) * l.tile_bytes : l.delta_bytes;
  return l;
}

// Workspace of the 16-bit backward: the rowsum(G O) series (float32), then, when storing tiles,
// the P and dS series of every (query, key) pair as 16-bit values [K+1][bh][row / 32][lq][32]
// (32-key blocks; row = attention_bwd_half_row(lk), lk rounded up to a multiple of 128, the keys
// of one workgroup of the reading kernel).
inline int64_t attention_bwd_half_row(int64_t lk) { return (lk + 127) / 128 * 128; }
inline AttnBwdLayout attention_bwd_half_layout(int degree, int64_t bh, int64_t lq, int64_t lk, bool materialize) {
  AttnBwdLayout l{};
  l.delta_bytes = static_cast<size_t>(degree + 1) * static_cast<size_t>(bh) * static_cast<size_t>(lq) * 4;
  l.tiles_offset = (l.delta_bytes + 255) / 256 * 256;
  l.tile_bytes = (static_cast<size_t>(bh) * static_cast<size_t>(lq) * static_cast<size_t>(attention_bwd_half_row(lk)) *
                      2 + 255) / 256 * 256;
  l.total = materialize ? l.tiles_offset + 2 * static_cast<size_t>(degree + 1) * l.tile_bytes : l.delta_bytes;
  return l;
}

}  // namespace pt
