// Instantiates the cross-entropy series kernels for one storage type.
#include "cross_entropy_series.inl"

namespace pt {
template int launch_ce<float>(const CeArgs&);
template int launch_ce_bwd<float>(const CeBwdArgs&);
}  // namespace pt
