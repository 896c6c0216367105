// C ABI of the activation-series kernels.
#include "activation_series.h"

namespace {

int check_activation(int dtype, int degree, int kind, bool backward, const void* const* g,
                     const void* const* x, void* const* y, int64_t numel) {
  PT_REQUIRE(degree >= 0 && degree <= PT_MAX_ELEMENTWISE_DEGREE, PT_UNSUPPORTED,
             "activation series: degree must be in 0..16");
  PT_REQUIRE(dtype >= PT_FLOAT32 && dtype <= PT_FLOAT16, PT_UNSUPPORTED,
             "activation series: unknown dtype code");
  PT_REQUIRE(kind >= PT_ACT_GELU && kind <= PT_ACT_RSQRT, PT_UNSUPPORTED,
             "activation series: unknown activation kind");
  PT_REQUIRE(!backward || kind <= PT_ACT_SILU, PT_UNSUPPORTED,
             "activation series: exp, log, sin, cos, sqrt and rsqrt have no backward entry point (their "
             "gradients are products of forward series)");
  PT_REQUIRE(x != nullptr && y != nullptr && (!backward || g != nullptr), PT_INVALID_ARGUMENT,
             "activation series: pointer arrays are required");
  PT_REQUIRE(numel >= 0, PT_INVALID_ARGUMENT, "activation series: numel must be >= 0");
  for (int k = 0; k <= degree; ++k) {
    PT_REQUIRE(x[k] != nullptr && y[k] != nullptr && (!backward || g[k] != nullptr),
               PT_INVALID_ARGUMENT, "activation series: null coefficient pointer");
  }
  return PT_OK;
}

int dispatch_activation(int dtype, const pt::ActArgs& a) {
  switch (dtype) {
    case PT_FLOAT32: return pt::launch_activation<float>(a);
    case PT_FLOAT64: return pt::launch_activation<double>(a);
    case PT_BFLOAT16: return pt::launch_activation<pt::bf16>(a);
    case PT_FLOAT16: return pt::launch_activation<_Float16>(a);
    default: break;
  }
  pt_host::set_error("activation series: unknown dtype code");
  return PT_UNSUPPORTED;
}

}  // namespace

extern "C" {

int pt_activation_series_fwd(int dtype, int degree, int kind, const void* const* x, void* const* y,
                             int64_t numel, void* stream) {
  pt_host::clear_error();
  int st = check_activation(dtype, degree, kind, false, nullptr, x, y, numel);
  if (st != PT_OK) return st;
  if (numel == 0) return PT_OK;
  pt::ActArgs a{degree, kind, false, x, nullptr, y, numel, static_cast<hipStream_t>(stream)};
  return dispatch_activation(dtype, a);
}

int pt_activation_series_bwd(int dtype, int degree, int kind, const void* const* g,
                             const void* const* saved, void* const* dx, int64_t numel, void* stream) {
  pt_host::clear_error();
  int st = check_activation(dtype, degree, kind, true, g, saved, dx, numel);
  if (st != PT_OK) return st;
  if (numel == 0) return PT_OK;
  pt::ActArgs a{degree, kind, true, saved, g, dx, numel, static_cast<hipStream_t>(stream)};
  return dispatch_activation(dtype, a);
}

}  // extern "C"
