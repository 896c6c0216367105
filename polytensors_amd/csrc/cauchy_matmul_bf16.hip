// Instantiates the 16-bit Cauchy-product matmul kernels for one type.
#include "cauchy_matmul_half.inl"

namespace pt {
template int launch_cauchy_half<bf16>(const CauchyArgs&);
}  // namespace pt
