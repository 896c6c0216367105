// Launch interface of the cross-entropy series kernels (definitions in cross_entropy_series.inl).
#pragma once

#include "pt_common.h"

namespace pt {

struct CeArgs {
  int degree;
  const void* const* z;
  int64_t rows;
  int64_t classes;
  int64_t row_stride;
  const int64_t* target;
  int64_t ignore_index;
  double softcap;   // 0: none
  int reduction;
  void* const* loss;
  void* const* lse;
  void* workspace;
  hipStream_t stream;
};

template <typename T>
int launch_ce(const CeArgs& a);

// Gradient series of the per-row losses: dz = c (*) (softmax(z) - e_y) per row.
struct CeBwdArgs {
  int degree;
  const void* const* z;
  int64_t rows;
  int64_t classes;
  int64_t row_stride;
  const int64_t* target;
  int64_t ignore_index;
  double softcap;             // 0: none
  const void* const* lse;     // K+1 pointers [rows], arithmetic type
  const void* const* cot;     // K+1 pointers [rows], arithmetic type
  void* const* dz;            // K+1 pointers [rows, classes] contiguous
  hipStream_t stream;
};

template <typename T>
int launch_ce_bwd(const CeBwdArgs& a);

}  // namespace pt
