// Launch interface of the Cauchy-product matmul kernels (definitions in cauchy_matmul.inl).
#pragma once

#include "pt_common.h"

namespace pt {

struct CauchyArgs {
  int degree;
  const void* const* a;
  int a_orders;
  const void* const* b;
  int b_orders;
  void* const* c;
  int64_t batch, m, n, k;
  int64_t a_bs, b_bs;
  bool trans_b;
  hipStream_t stream;
};

template <typename T>
int launch_cauchy(const CauchyArgs& a);

// bfloat16 / float16 operands on the 16x16x32 MFMAs (cauchy_matmul_half.inl); T = bf16 or _Float16.
template <typename T>
int launch_cauchy_half(const CauchyArgs& a);

}  // namespace pt
