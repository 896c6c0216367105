// Instantiates the 16-bit Taylor attention backward kernels for one type.
#include "taylor_attention_bwd_half.inl"

namespace pt {
template int launch_attention_bwd_half<bf16>(const AttnBwdArgs&);
}  // namespace pt
