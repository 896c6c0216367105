// Instantiates the norm-series kernels for one storage type.
#include "norm_series.inl"

namespace pt {
template int launch_norm<float, false>(const NormArgs&);
template int launch_norm<float, true>(const NormArgs&);
template int launch_norm_bwd<float, false>(const NormBwdArgs&);
template int launch_norm_bwd<float, true>(const NormBwdArgs&);
}  // namespace pt
