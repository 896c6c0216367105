// Instantiates the norm-series kernels for one storage type.
#include "norm_series.inl"

namespace pt {
template int launch_norm<double, false>(const NormArgs&);
template int launch_norm<double, true>(const NormArgs&);
}  // namespace pt
