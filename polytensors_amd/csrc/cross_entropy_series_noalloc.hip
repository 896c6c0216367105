// Allocation-free variant of pt_cross_entropy_series_fwd.
//
// A mean or sum reduction first writes the per-row loss series to a scratch
// buffer ((K+1) x rows values of the arithmetic type) and then reduces it in a
// second kernel. Here that buffer is a file-scope device array, `scratch`, of
// PT_CE_NOALLOC_SCRATCH_BYTES, which every GPU the library runs on holds until
// the process ends. Its device address is looked up once per device, with that
// device current (hipGetSymbolAddress), on the entry point's first call there,
// and only that address is handed to the kernels: on the host, `scratch` names
// a host-side stand-in, not device memory. The entry point calls no hipMalloc,
// hipFree or allocating library routine.
//
// Every call on one GPU shares that GPU's array: calls that overlap on one GPU
// (different streams, or host threads) race on it. The row kernel writes every
// per-row value the reduction reads, so nothing needs clearing between calls.
#include <mutex>

#include "cross_entropy_series.h"

static __device__ __align__(256) unsigned char scratch[PT_CE_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
void* g_scratch_ptr[kMaxDevices] = {};   // device address of `scratch` per device ordinal

// The device address of `scratch` on the current device (looked up once per device).
int scratch_address(void** out) {
  int device = -1;
  const hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) {
    pt_host::set_error(std::string("cross-entropy series (no-alloc): hipGetDevice failed: ") +
                       hipGetErrorString(e));
    return PT_DEVICE_ERROR;
  }
  PT_REQUIRE(device >= 0 && device < kMaxDevices, PT_UNSUPPORTED,
             "cross-entropy series (no-alloc): device ordinal beyond 63");
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  if (g_scratch_ptr[device] == nullptr) {
    void* ptr = nullptr;
    const hipError_t s = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (s != hipSuccess || ptr == nullptr) {
      pt_host::set_error(std::string("cross-entropy series (no-alloc): hipGetSymbolAddress(scratch) failed: ") +
                         hipGetErrorString(s));
      return PT_DEVICE_ERROR;
    }
    g_scratch_ptr[device] = ptr;
  }
  *out = g_scratch_ptr[device];
  return PT_OK;
}

}  // namespace

extern "C" {

size_t pt_cross_entropy_series_noalloc_max_bytes(void) { return PT_CE_NOALLOC_SCRATCH_BYTES; }

int pt_cross_entropy_series_fwd_noalloc(int dtype, int degree, const void* const* logits, int64_t rows,
                                        int64_t classes, int64_t row_stride, const int64_t* target,
                                        int64_t ignore_index, double softcap, int reduction, void* const* loss,
                                        void* const* lse, void* stream) {
  pt_host::clear_error();
  const size_t need = pt_cross_entropy_series_workspace_size(dtype, degree, rows, reduction);
  PT_REQUIRE(need <= PT_CE_NOALLOC_SCRATCH_BYTES, PT_UNSUPPORTED,
             "cross-entropy series (no-alloc): the reduction's per-row losses ((degree+1) x rows values) exceed "
             "the 4 MiB scratch buffer; use pt_cross_entropy_series_fwd with a workspace");
  void* workspace = nullptr;
  if (need > 0) {
    const int status = scratch_address(&workspace);
    if (status != PT_OK) return status;
  }
  return pt_cross_entropy_series_fwd(dtype, degree, logits, rows, classes, row_stride, target, ignore_index,
                                     softcap, reduction, loss, lse, workspace, stream);
}

}  // extern "C"
