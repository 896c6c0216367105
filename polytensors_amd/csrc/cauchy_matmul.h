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

}  // namespace pt
