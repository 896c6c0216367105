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
  double scale;
  hipStream_t stream;
};

template <typename T>
int launch_attention(const AttnArgs& a);

}  // namespace pt
