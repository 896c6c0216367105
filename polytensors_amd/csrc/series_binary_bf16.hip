// Instantiates the elementwise series product / quotient kernels for one storage type.
#include "series_binary.inl"

namespace pt {
template int launch_binary<bf16>(const BinaryArgs&);
}  // namespace pt
