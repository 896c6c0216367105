// Instantiates the norm-series kernels for one storage type.
#include "norm_series.inl"

namespace pt {
template int launch_norm<_Float16, false>(const NormArgs&);
template int launch_norm<_Float16, true>(const NormArgs&);
template int launch_norm_bwd<_Float16, false>(const NormBwdArgs&);
template int launch_norm_bwd<_Float16, true>(const NormBwdArgs&);
}  // namespace pt
