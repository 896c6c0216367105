// C ABI of the elementwise series product / quotient kernels.
#include "series_binary.h"

extern "C" {

int pt_series_binary(int dtype, int degree, int op, const void* const* a, const void* const* b,
                     void* const* y, int64_t numel, void* stream) {
  pt_host::clear_error();
  PT_REQUIRE(degree >= 0 && degree <= PT_MAX_ELEMENTWISE_DEGREE, PT_UNSUPPORTED,
             "series product: degree must be in 0..16");
  PT_REQUIRE(dtype >= PT_FLOAT32 && dtype <= PT_FLOAT16, PT_UNSUPPORTED, "series product: unknown dtype code");
  PT_REQUIRE(op == PT_BINARY_MUL || op == PT_BINARY_DIV, PT_UNSUPPORTED, "series product: unknown operation");
  PT_REQUIRE(a != nullptr && b != nullptr && y != nullptr, PT_INVALID_ARGUMENT,
             "series product: pointer arrays are required");
  PT_REQUIRE(numel >= 0, PT_INVALID_ARGUMENT, "series product: numel must be >= 0");
  for (int k = 0; k <= degree; ++k)
    PT_REQUIRE(a[k] != nullptr && b[k] != nullptr && y[k] != nullptr, PT_INVALID_ARGUMENT,
               "series product: null coefficient pointer");
  if (numel == 0) return PT_OK;
  pt::BinaryArgs args{degree, op, a, b, y, numel, static_cast<hipStream_t>(stream)};
  switch (dtype) {
    case PT_FLOAT32: return pt::launch_binary<float>(args);
    case PT_FLOAT64: return pt::launch_binary<double>(args);
    case PT_BFLOAT16: return pt::launch_binary<pt::bf16>(args);
    case PT_FLOAT16: return pt::launch_binary<_Float16>(args);
    default: break;
  }
  pt_host::set_error("series product: unknown dtype code");
  return PT_UNSUPPORTED;
}

}  // extern "C"
