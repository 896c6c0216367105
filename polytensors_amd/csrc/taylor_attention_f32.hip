// Instantiates the Taylor attention kernels for one type.
#include "taylor_attention.inl"

namespace pt {
template int launch_attention<float>(const AttnArgs&);
}  // namespace pt
