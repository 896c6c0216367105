// Launch interface of the elementwise series product / quotient kernels
// (definitions in series_binary.inl).
#pragma once

#include "pt_common.h"

namespace pt {

struct BinaryArgs {
  int degree;
  int op;                   // pt_binary
  const void* const* a;     // K+1 pointers
  const void* const* b;     // K+1 pointers
  void* const* y;
  int64_t numel;
  hipStream_t stream;
};

template <typename T>
int launch_binary(const BinaryArgs& a);

}  // namespace pt
