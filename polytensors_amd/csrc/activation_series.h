// Launch interface of the activation-series kernels (definitions in activation_series.inl).
#pragma once

#include "pt_common.h"

namespace pt {

struct ActArgs {
  int degree;
  int kind;                 // pt_activation
  bool backward;
  const void* const* x;     // forward: input series; backward: the saved series
  const void* const* g;     // backward: gradient series, else null
  void* const* y;
  int64_t numel;
  hipStream_t stream;
};

template <typename T>
int launch_activation(const ActArgs& a);

}  // namespace pt
