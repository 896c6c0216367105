// Instantiates the Taylor attention backward kernels for one type.
#include "taylor_attention_bwd.inl"

namespace pt {
template int launch_attention_bwd<float>(const AttnBwdArgs&);
}  // namespace pt
