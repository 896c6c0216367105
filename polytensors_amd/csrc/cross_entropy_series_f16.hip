// Instantiates the cross-entropy series kernels for one storage type.
#include "cross_entropy_series.inl"

namespace pt {
template int launch_ce<_Float16>(const CeArgs&);
template int launch_ce_bwd<_Float16>(const CeBwdArgs&);
}  // namespace pt
