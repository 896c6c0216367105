// Instantiates the norm-series kernels for one storage type.
#include "norm_series.inl"

namespace pt {
template int launch_norm<bf16, false>(const NormArgs&);
template int launch_norm<bf16, true>(const NormArgs&);
template int launch_norm_bwd<bf16, false>(const NormBwdArgs&);
template int launch_norm_bwd<bf16, true>(const NormBwdArgs&);
}  // namespace pt
