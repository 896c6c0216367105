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
  hipStream_t stream;
};

template <typename T>
int launch_attention_bwd(const AttnBwdArgs& a);

}  // namespace pt
