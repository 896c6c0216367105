// C ABI of the cross-entropy series kernels.
#include "cross_entropy_series.h"

namespace {

size_t acc_size(int dtype) { return dtype == PT_FLOAT64 ? sizeof(double) : sizeof(float); }

}  // namespace

extern "C" {

size_t pt_cross_entropy_series_workspace_size(int dtype, int degree, int64_t rows, int reduction) {
  if (reduction == PT_REDUCTION_NONE || rows <= 0 || degree < 0 || degree > PT_MAX_DEGREE) return 0;
  return static_cast<size_t>(degree + 1) * static_cast<size_t>(rows) * acc_size(dtype);
}

int pt_cross_entropy_series_fwd(int dtype, int degree, const void* const* logits, int64_t rows,
                                int64_t classes, int64_t row_stride, const int64_t* target,
                                int64_t ignore_index, double softcap, int reduction, void* const* loss,
                                void* const* lse, void* workspace, void* stream) {
  pt_host::clear_error();
  PT_REQUIRE(degree >= 0 && degree <= PT_MAX_DEGREE, PT_UNSUPPORTED,
             "cross-entropy series: degree must be in 0..8");
  PT_REQUIRE(dtype >= PT_FLOAT32 && dtype <= PT_FLOAT16, PT_UNSUPPORTED,
             "cross-entropy series: unknown dtype code");
  PT_REQUIRE(reduction >= PT_REDUCTION_NONE && reduction <= PT_REDUCTION_SUM, PT_INVALID_ARGUMENT,
             "cross-entropy series: reduction must be 0 (none), 1 (mean) or 2 (sum)");
  PT_REQUIRE(logits != nullptr && loss != nullptr, PT_INVALID_ARGUMENT,
             "cross-entropy series: logits and loss pointer arrays are required");
  PT_REQUIRE(rows >= 0 && classes >= 1 && row_stride >= classes, PT_INVALID_ARGUMENT,
             "cross-entropy series: need rows >= 0, classes >= 1, row_stride >= classes");
  PT_REQUIRE(rows <= INT32_MAX, PT_UNSUPPORTED, "cross-entropy series: rows beyond 2^31-1");
  PT_REQUIRE(softcap >= 0.0 && softcap <= 1e300, PT_INVALID_ARGUMENT,
             "cross-entropy series: softcap must be 0 (none) or a positive finite cap");
  PT_REQUIRE(rows == 0 || target != nullptr, PT_INVALID_ARGUMENT,
             "cross-entropy series: target is required");
  PT_REQUIRE(reduction == PT_REDUCTION_NONE || rows == 0 || workspace != nullptr,
             PT_INVALID_ARGUMENT, "cross-entropy series: a reduction needs the workspace");
  for (int k = 0; k <= degree; ++k) {
    PT_REQUIRE(logits[k] != nullptr && loss[k] != nullptr, PT_INVALID_ARGUMENT,
               "cross-entropy series: null coefficient pointer");
    PT_REQUIRE(lse == nullptr || lse[k] != nullptr, PT_INVALID_ARGUMENT,
               "cross-entropy series: lse array with a null entry");
  }
  PT_REQUIRE(rows > 0 || reduction == PT_REDUCTION_NONE, PT_UNSUPPORTED,
             "cross-entropy series: a reduction over zero rows");
  if (rows == 0) return PT_OK;
  pt::CeArgs a{degree, logits, rows, classes, row_stride, target, ignore_index, softcap, reduction,
               loss, lse, workspace, static_cast<hipStream_t>(stream)};
  switch (dtype) {
    case PT_FLOAT32: return pt::launch_ce<float>(a);
    case PT_FLOAT64: return pt::launch_ce<double>(a);
    case PT_BFLOAT16: return pt::launch_ce<pt::bf16>(a);
    case PT_FLOAT16: return pt::launch_ce<_Float16>(a);
    default: break;
  }
  pt_host::set_error("cross-entropy series: unknown dtype code");
  return PT_UNSUPPORTED;
}

int pt_cross_entropy_series_bwd(int dtype, int degree, const void* const* logits, int64_t rows,
                                int64_t classes, int64_t row_stride, const int64_t* target,
                                int64_t ignore_index, double softcap, const void* const* lse,
                                const void* const* cot, void* const* dz, void* stream) {
  pt_host::clear_error();
  PT_REQUIRE(degree >= 0 && degree <= PT_MAX_DEGREE, PT_UNSUPPORTED,
             "cross-entropy series backward: degree must be in 0..8");
  PT_REQUIRE(dtype >= PT_FLOAT32 && dtype <= PT_FLOAT16, PT_UNSUPPORTED,
             "cross-entropy series backward: unknown dtype code");
  PT_REQUIRE(logits != nullptr && lse != nullptr && cot != nullptr && dz != nullptr, PT_INVALID_ARGUMENT,
             "cross-entropy series backward: logits, lse, cot and dz pointer arrays are required");
  PT_REQUIRE(rows >= 0 && classes >= 1 && row_stride >= classes, PT_INVALID_ARGUMENT,
             "cross-entropy series backward: need rows >= 0, classes >= 1, row_stride >= classes");
  PT_REQUIRE(rows <= INT32_MAX, PT_UNSUPPORTED, "cross-entropy series backward: rows beyond 2^31-1");
  PT_REQUIRE(rows == 0 || target != nullptr, PT_INVALID_ARGUMENT,
             "cross-entropy series backward: target is required");
  PT_REQUIRE(softcap >= 0.0 && softcap <= 1e300, PT_INVALID_ARGUMENT,
             "cross-entropy series backward: softcap must be 0 (none) or a positive finite cap");
  for (int k = 0; k <= degree; ++k)
    PT_REQUIRE(logits[k] != nullptr && lse[k] != nullptr && cot[k] != nullptr && dz[k] != nullptr,
               PT_INVALID_ARGUMENT, "cross-entropy series backward: null coefficient pointer");
  if (rows == 0) return PT_OK;
  pt::CeBwdArgs a{degree, logits, rows, classes, row_stride, target, ignore_index, softcap,
                  lse, cot, dz, static_cast<hipStream_t>(stream)};
  switch (dtype) {
    case PT_FLOAT32: return pt::launch_ce_bwd<float>(a);
    case PT_FLOAT64: return pt::launch_ce_bwd<double>(a);
    case PT_BFLOAT16: return pt::launch_ce_bwd<pt::bf16>(a);
    case PT_FLOAT16: return pt::launch_ce_bwd<_Float16>(a);
    default: break;
  }
  pt_host::set_error("cross-entropy series backward: unknown dtype code");
  return PT_UNSUPPORTED;
}

}  // extern "C"
