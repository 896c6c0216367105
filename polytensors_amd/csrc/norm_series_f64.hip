// Instantiates the norm-series kernels for one storage type.
#include "norm_series.inl"

namespace pt {
template int launch_norm<double, false>(const NormArgs&);
template int launch_norm<double, true>(const NormArgs&);
template int launch_norm_bwd<double, false>(const NormBwdArgs&);
template int launch_norm_bwd<double, true>(const NormBwdArgs&);
}  // namespace pt
