// Instantiates the 16-bit Taylor attention forward kernels for one type.
#include "taylor_attention_half.inl"

namespace pt {
template int launch_attention_half<bf16>(const AttnArgs&);
}  // namespace pt
