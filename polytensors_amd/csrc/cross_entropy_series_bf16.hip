// Instantiates the cross-entropy series kernels for one storage type.
#include "cross_entropy_series.inl"

namespace pt {
template int launch_ce<bf16>(const CeArgs&);
template int launch_ce_bwd<bf16>(const CeBwdArgs&);
}  // namespace pt
