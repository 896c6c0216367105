// Launch interface of the Taylor attention kernels (definitions in taylor_attention.inl).
#pragma once

#include "pt_common.h"

namespace pt {

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
};

template <typename T>
int launch_attention(const AttnArgs& a);

// bfloat16 / float16 operands on the 16x16x32 MFMAs (taylor_attention_half.inl); T = bf16 or _Float16.
template <typename T>
int launch_attention_half(const AttnArgs& a);

// Block ranges of a boolean (L, S) mask into ranges[attention_mask_ranges_count(L, S)].
int64_t attention_mask_ranges_count(int64_t lq, int64_t lk);
int launch_attention_mask_ranges(const uint8_t* mask, int64_t lq, int64_t lk, int32_t* ranges, hipStream_t stream);

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
};

template <typename T>
int launch_attention_bwd(const AttnBwdArgs& a);

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

}  // namespace pt
