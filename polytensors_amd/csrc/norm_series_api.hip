// C ABI of the RMSNorm / LayerNorm series kernels.
#include "norm_series.h"

namespace {

int check_norm(int dtype, int degree, const void* const* x, const void* const* w,
               int w_orders, const void* const* b, int b_orders, void* const* y,
               int64_t rows, int64_t n, double eps) {
  PT_REQUIRE(degree >= 0 && degree <= PT_MAX_DEGREE, PT_UNSUPPORTED,
             "norm series: degree must be in 0..8");
  PT_REQUIRE(dtype >= PT_FLOAT32 && dtype <= PT_FLOAT16, PT_UNSUPPORTED,
             "norm series: unknown dtype code");
  PT_REQUIRE(x != nullptr && y != nullptr, PT_INVALID_ARGUMENT,
             "norm series: x and y pointer arrays are required");
  PT_REQUIRE(rows >= 0 && n >= 1, PT_INVALID_ARGUMENT,
             "norm series: rows must be >= 0 and n >= 1");
  PT_REQUIRE(rows <= INT32_MAX, PT_UNSUPPORTED, "norm series: rows beyond 2^31-1");
  PT_REQUIRE(w_orders == 0 || w_orders == 1 || w_orders == degree + 1, PT_INVALID_ARGUMENT,
             "norm series: weight_orders must be 0, 1 or degree+1");
  PT_REQUIRE(b_orders == 0 || b_orders == 1 || b_orders == degree + 1, PT_INVALID_ARGUMENT,
             "norm series: bias_orders must be 0, 1 or degree+1");
  PT_REQUIRE(w_orders == 0 || w != nullptr, PT_INVALID_ARGUMENT,
             "norm series: weight pointer array missing");
  PT_REQUIRE(b_orders == 0 || b != nullptr, PT_INVALID_ARGUMENT,
             "norm series: bias pointer array missing");
  PT_REQUIRE(eps >= 0.0, PT_INVALID_ARGUMENT, "norm series: eps must be >= 0");
  for (int k = 0; k <= degree; ++k)
    PT_REQUIRE(x[k] != nullptr && y[k] != nullptr, PT_INVALID_ARGUMENT,
               "norm series: null coefficient pointer");
  return PT_OK;
}

int dispatch_norm(int dtype, bool layer, const pt::NormArgs& a) {
  switch (dtype) {
    case PT_FLOAT32:
      return layer ? pt::launch_norm<float, true>(a) : pt::launch_norm<float, false>(a);
    case PT_FLOAT64:
      return layer ? pt::launch_norm<double, true>(a) : pt::launch_norm<double, false>(a);
    case PT_BFLOAT16:
      return layer ? pt::launch_norm<pt::bf16, true>(a) : pt::launch_norm<pt::bf16, false>(a);
    case PT_FLOAT16:
      return layer ? pt::launch_norm<_Float16, true>(a) : pt::launch_norm<_Float16, false>(a);
    default:
      break;
  }
  pt_host::set_error("norm series: unknown dtype code");
  return PT_UNSUPPORTED;
}

int check_norm_bwd(int dtype, int degree, const void* const* x, const void* const* g, void* const* dx,
                   int64_t rows, int64_t n, double eps) {
  PT_REQUIRE(degree >= 0 && degree <= PT_MAX_DEGREE, PT_UNSUPPORTED,
             "norm series backward: degree must be in 0..8");
  PT_REQUIRE(dtype >= PT_FLOAT32 && dtype <= PT_FLOAT16, PT_UNSUPPORTED,
             "norm series backward: unknown dtype code");
  PT_REQUIRE(x != nullptr && g != nullptr && dx != nullptr, PT_INVALID_ARGUMENT,
             "norm series backward: x, g and dx pointer arrays are required");
  PT_REQUIRE(rows >= 0 && n >= 1, PT_INVALID_ARGUMENT, "norm series backward: rows must be >= 0 and n >= 1");
  PT_REQUIRE(rows <= INT32_MAX, PT_UNSUPPORTED, "norm series backward: rows beyond 2^31-1");
  PT_REQUIRE(eps >= 0.0, PT_INVALID_ARGUMENT, "norm series backward: eps must be >= 0");
  for (int k = 0; k <= degree; ++k)
    PT_REQUIRE(x[k] != nullptr && g[k] != nullptr && dx[k] != nullptr, PT_INVALID_ARGUMENT,
               "norm series backward: null coefficient pointer");
  return PT_OK;
}

int dispatch_norm_bwd(int dtype, bool layer, const pt::NormBwdArgs& a) {
  switch (dtype) {
    case PT_FLOAT32:
      return layer ? pt::launch_norm_bwd<float, true>(a) : pt::launch_norm_bwd<float, false>(a);
    case PT_FLOAT64:
      return layer ? pt::launch_norm_bwd<double, true>(a) : pt::launch_norm_bwd<double, false>(a);
    case PT_BFLOAT16:
      return layer ? pt::launch_norm_bwd<pt::bf16, true>(a) : pt::launch_norm_bwd<pt::bf16, false>(a);
    case PT_FLOAT16:
      return layer ? pt::launch_norm_bwd<_Float16, true>(a) : pt::launch_norm_bwd<_Float16, false>(a);
    default:
      break;
  }
  pt_host::set_error("norm series backward: unknown dtype code");
  return PT_UNSUPPORTED;
}

}  // namespace

extern "C" {

int pt_rms_norm_series_fwd(int dtype, int degree, const void* const* x,
                           const void* const* weight, int weight_orders, void* const* y,
                           int64_t rows, int64_t n, double eps, void* stream) {
  pt_host::clear_error();
  int st = check_norm(dtype, degree, x, weight, weight_orders, nullptr, 0, y, rows, n, eps);
  if (st != PT_OK) return st;
  if (rows == 0) return PT_OK;
  pt::NormArgs a{degree, x, weight, weight_orders, nullptr, 0, y, rows, n, eps,
                 static_cast<hipStream_t>(stream)};
  return dispatch_norm(dtype, false, a);
}

int pt_layer_norm_series_fwd(int dtype, int degree, const void* const* x,
                             const void* const* weight, int weight_orders,
                             const void* const* bias, int bias_orders, void* const* y,
                             int64_t rows, int64_t n, double eps, void* stream) {
  pt_host::clear_error();
  int st = check_norm(dtype, degree, x, weight, weight_orders, bias, bias_orders, y, rows, n,
                      eps);
  if (st != PT_OK) return st;
  if (rows == 0) return PT_OK;
  pt::NormArgs a{degree, x, weight, weight_orders, bias, bias_orders, y, rows, n, eps,
                 static_cast<hipStream_t>(stream)};
  return dispatch_norm(dtype, true, a);
}

int pt_rms_norm_series_bwd(int dtype, int degree, const void* const* x, const void* const* g,
                           void* const* dx, int64_t rows, int64_t n, double eps, void* stream) {
  pt_host::clear_error();
  int st = check_norm_bwd(dtype, degree, x, g, dx, rows, n, eps);
  if (st != PT_OK) return st;
  if (rows == 0) return PT_OK;
  pt::NormBwdArgs a{degree, x, g, dx, rows, n, eps, static_cast<hipStream_t>(stream)};
  return dispatch_norm_bwd(dtype, false, a);
}

int pt_layer_norm_series_bwd(int dtype, int degree, const void* const* x, const void* const* g,
                             void* const* dx, int64_t rows, int64_t n, double eps, void* stream) {
  pt_host::clear_error();
  int st = check_norm_bwd(dtype, degree, x, g, dx, rows, n, eps);
  if (st != PT_OK) return st;
  if (rows == 0) return PT_OK;
  pt::NormBwdArgs a{degree, x, g, dx, rows, n, eps, static_cast<hipStream_t>(stream)};
  return dispatch_norm_bwd(dtype, true, a);
}

}  // extern "C"
