// Launch interface of the norm-series kernels (definitions in norm_series.inl).
#pragma once

#include "pt_common.h"

namespace pt {

struct NormArgs {
  int degree;
  const void* const* x;
  const void* const* w;
  int w_orders;
  const void* const* b;
  int b_orders;
  void* const* y;
  int64_t rows;
  int64_t n;
  double eps;
  hipStream_t stream;
};

template <typename T, bool LAYER>
int launch_norm(const NormArgs& a);

// Gradient series of the normalization (no affine terms): dx = J(x(t))^T g(t).
struct NormBwdArgs {
  int degree;
  const void* const* x;
  const void* const* g;
  void* const* dx;
  int64_t rows;
  int64_t n;
  double eps;
  hipStream_t stream;
};

template <typename T, bool LAYER>
int launch_norm_bwd(const NormBwdArgs& a);

}  // namespace pt
