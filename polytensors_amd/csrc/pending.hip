// Entry points whose kernels are not built yet: they report PT_UNSUPPORTED.
#include "pt_common.h"

extern "C" {

int pt_taylor_attention_fwd(int, int, const void* const*, int, const void* const*, int,
                            const void* const*, int, void* const*, void* const*, int64_t, int64_t,
                            int64_t, int64_t, int, const uint8_t*, double, void*) {
  pt_host::set_error("Taylor attention kernel not built");
  return PT_UNSUPPORTED;
}

}  // extern "C"
