// C ABI of the Cauchy-product matmul kernels.
#include "cauchy_matmul.h"

extern "C" {

int pt_cauchy_matmul(int dtype, int degree, const void* const* a, int a_orders,
                     const void* const* b, int b_orders, void* const* c, int64_t batch, int64_t m,
                     int64_t n, int64_t k, int64_t a_batch_stride, int64_t b_batch_stride,
                     int trans_b, void* stream) {
  pt_host::clear_error();
  PT_REQUIRE(degree >= 0 && degree <= PT_MAX_DEGREE, PT_UNSUPPORTED,
             "Cauchy matmul: degree must be in 0..8");
  PT_REQUIRE(dtype == PT_FLOAT32 || dtype == PT_FLOAT64 || dtype == PT_BFLOAT16 || dtype == PT_FLOAT16,
             PT_UNSUPPORTED, "Cauchy matmul: float32, float64, bfloat16 or float16");
  PT_REQUIRE(a != nullptr && b != nullptr && c != nullptr, PT_INVALID_ARGUMENT,
             "Cauchy matmul: a, b and c pointer arrays are required");
  PT_REQUIRE(a_orders == 1 || a_orders == degree + 1, PT_INVALID_ARGUMENT,
             "Cauchy matmul: a_orders must be 1 or degree+1");
  PT_REQUIRE(b_orders == 1 || b_orders == degree + 1, PT_INVALID_ARGUMENT,
             "Cauchy matmul: b_orders must be 1 or degree+1");
  PT_REQUIRE(batch >= 0 && m >= 0 && n >= 0 && k >= 0, PT_INVALID_ARGUMENT,
             "Cauchy matmul: negative size");
  PT_REQUIRE(a_batch_stride >= 0 && b_batch_stride >= 0, PT_INVALID_ARGUMENT,
             "Cauchy matmul: negative batch stride");
  PT_REQUIRE(m <= INT32_MAX && n <= INT32_MAX && k <= INT32_MAX && batch <= 65535 &&
                 (m + 31) / 32 <= 65535,
             PT_UNSUPPORTED, "Cauchy matmul: sizes beyond the launch grid");
  for (int o = 0; o < a_orders; ++o)
    PT_REQUIRE(a[o] != nullptr, PT_INVALID_ARGUMENT, "Cauchy matmul: null A coefficient");
  for (int o = 0; o < b_orders; ++o)
    PT_REQUIRE(b[o] != nullptr, PT_INVALID_ARGUMENT, "Cauchy matmul: null B coefficient");
  for (int o = 0; o <= degree; ++o)
    PT_REQUIRE(c[o] != nullptr, PT_INVALID_ARGUMENT, "Cauchy matmul: null C coefficient");
  if (batch == 0 || m == 0 || n == 0) return PT_OK;
  pt::CauchyArgs args{degree, a, a_orders, b, b_orders, c, batch, m, n, k,
                      a_batch_stride, b_batch_stride, trans_b != 0, static_cast<hipStream_t>(stream)};
  switch (dtype) {
    case PT_FLOAT32: return pt::launch_cauchy<float>(args);
    case PT_FLOAT64: return pt::launch_cauchy<double>(args);
    case PT_BFLOAT16: return pt::launch_cauchy_half<pt::bf16>(args);
    default: return pt::launch_cauchy_half<_Float16>(args);
  }
}

}  // extern "C"
