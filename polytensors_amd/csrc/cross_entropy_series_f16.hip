// Instantiates the cross-entropy series kernels for one storage type.
#include "cross_entropy_series.inl"

namespace pt {
template int launch_ce<_Float16>(const CeArgs&);
}  // namespace pt
