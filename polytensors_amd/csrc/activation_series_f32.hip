// Instantiates the activation-series kernels for one storage type.
#include "activation_series.inl"

namespace pt {
template int launch_activation<float>(const ActArgs&);
}  // namespace pt
