// Instantiates the Cauchy-product matmul kernels for one type.
#include "cauchy_matmul.inl"

namespace pt {
template int launch_cauchy<double>(const CauchyArgs&);
}  // namespace pt
