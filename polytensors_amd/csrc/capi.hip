// Library-wide C ABI functions: error reporting and version queries.
#include "pt_common.h"

namespace pt_host {

static thread_local std::string g_last_error;

void set_error(const std::string& message) { g_last_error = message; }
void clear_error() { g_last_error.clear(); }

}  // namespace pt_host

extern "C" {

const char* pt_last_error(void) { return pt_host::g_last_error.c_str(); }

int pt_abi_version(void) { return PT_ABI_VERSION; }

int pt_max_degree(void) { return PT_MAX_DEGREE; }
int pt_max_elementwise_degree(void) { return PT_MAX_ELEMENTWISE_DEGREE; }

}  // extern "C"
