"""ctypes binding of ``libpolytaylor.so`` (the C ABI declared in ``include/polytaylor.h``).

The library is loaded after torch, so its HIP runtime dependency resolves to the
runtime torch already loaded (one HIP runtime per process: the stream handles
torch hands out are valid in the library). There is no fallback: a missing or
stale library raises ``LibraryMissingError``.
"""

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libpolytaylor.so")
# the operators' PyTorch registration (csrc/torch_ops.cpp), linked with libpolytaylor.so
TORCH_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libpolytaylor_torch.so")
ABI_VERSION = 13

PT_OK, PT_INVALID_ARGUMENT, PT_UNSUPPORTED, PT_DEVICE_ERROR = 0, 1, 2, 3
REDUCTIONS = {"none": 0, "mean": 1, "sum": 2}
# pt_activation codes of include/polytaylor.h
BINARY_OPS = {"mul": 0, "div": 1}
ACTIVATIONS = {"gelu": 0, "gelu_tanh": 1, "tanh": 2, "sigmoid": 3, "silu": 4, "exp": 5, "log": 6, "sin": 7,
               "cos": 8, "sqrt": 9, "rsqrt": 10}

DTYPE_CODES = {
    torch.float32: 0,
    torch.float64: 1,
    torch.bfloat16: 2,
    torch.float16: 3,
}

_c_int, _c_i64, _c_dbl, _c_vp = ctypes.c_int, ctypes.c_int64, ctypes.c_double, ctypes.c_void_p
_c_vpp = ctypes.POINTER(ctypes.c_void_p)
_c_dblp = ctypes.POINTER(ctypes.c_double)

# name -> (restype, argtypes); mirrors include/polytaylor.h.
SIGNATURES = {
    "pt_last_error": (ctypes.c_char_p, []),
    "pt_abi_version": (_c_int, []),
    "pt_max_degree": (_c_int, []),
    "pt_max_elementwise_degree": (_c_int, []),
    "pt_rms_norm_series_fwd": (_c_int, [_c_int, _c_int, _c_vpp, _c_vpp, _c_int, _c_vpp,
                                        _c_i64, _c_i64, _c_dbl, _c_vp]),
    "pt_layer_norm_series_fwd": (_c_int, [_c_int, _c_int, _c_vpp, _c_vpp, _c_int, _c_vpp, _c_int,
                                          _c_vpp, _c_i64, _c_i64, _c_dbl, _c_vp]),
    "pt_cross_entropy_series_fwd": (_c_int, [_c_int, _c_int, _c_vpp, _c_i64, _c_i64, _c_i64, _c_vp,
                                             _c_i64, _c_dbl, _c_int, _c_vpp, _c_vpp, _c_vp, _c_vp]),
    "pt_cross_entropy_series_bwd": (_c_int, [_c_int, _c_int, _c_vpp, _c_i64, _c_i64, _c_i64, _c_vp,
                                             _c_i64, _c_dbl, _c_vpp, _c_vpp, _c_vpp, _c_vp]),
    "pt_cross_entropy_series_workspace_size": (ctypes.c_size_t, [_c_int, _c_int, _c_i64, _c_int]),
    "pt_cross_entropy_series_fwd_noalloc": (_c_int, [_c_int, _c_int, _c_vpp, _c_i64, _c_i64, _c_i64, _c_vp,
                                                     _c_i64, _c_dbl, _c_int, _c_vpp, _c_vpp, _c_vp]),
    "pt_cross_entropy_series_noalloc_max_bytes": (ctypes.c_size_t, []),
    "pt_cauchy_matmul": (_c_int, [_c_int, _c_int, _c_vpp, _c_int, _c_vpp, _c_int, _c_vpp,
                                  _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_vp]),
    "pt_taylor_attention_fwd": (_c_int, [_c_int, _c_int, _c_vpp, _c_int, _c_vpp, _c_int, _c_vpp, _c_int,
                                         _c_vpp, _c_vpp, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_vp,
                                         _c_vp, _c_dbl, _c_vp]),
    "pt_taylor_attention_fwd_workspace_size": (ctypes.c_size_t, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_i64,
                                                                 _c_i64, _c_i64, _c_i64]),
    "pt_taylor_attention_fwd_ws": (_c_int, [_c_int, _c_int, _c_vpp, _c_int, _c_vpp, _c_int, _c_vpp, _c_int,
                                            _c_vpp, _c_vpp, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_vp,
                                            _c_vp, _c_vp, _c_vp, _c_dbl, _c_vp, ctypes.c_size_t, _c_vp]),
    "pt_attention_mask_ranges_count": (_c_i64, [_c_i64, _c_i64]),
    "pt_attention_mask_ranges": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp]),
    "pt_taylor_attention_bwd": (_c_int, [_c_int, _c_int, _c_vpp, _c_vpp, _c_vpp, _c_vpp, _c_vpp, _c_vpp,
                                         _c_vpp, _c_vpp, _c_vpp, _c_vp, _c_int, _c_i64, _c_i64, _c_i64, _c_i64,
                                         _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_dbl, _c_vp]),
    "pt_taylor_attention_bwd_workspace_size": (ctypes.c_size_t, [_c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_int]),
    "pt_stream_copy": (_c_int, [_c_vp, _c_vp, _c_i64, _c_int, _c_int, _c_vp]),
    "pt_stream_read": (_c_int, [_c_vp, _c_i64, _c_int, _c_int, _c_vp, _c_vp]),
    "pt_stream_probe_blocks": (_c_int, []),
    "pt_stream_series": (_c_int, [_c_vpp, _c_int, _c_vpp, _c_int, _c_i64, _c_vp, _c_vp]),
    "pt_stream_series_blocks": (_c_i64, [_c_i64]),
    "pt_complex_to_real": (_c_int, [_c_int, _c_int, _c_vpp, _c_int, _c_dblp, _c_dblp, _c_vpp, _c_i64, _c_vp]),
    "pt_real_to_complex": (_c_int, [_c_int, _c_int, _c_int, _c_vpp, _c_dblp, _c_dblp, _c_vpp, _c_i64, _c_vp]),
    "pt_activation_series_fwd": (_c_int, [_c_int, _c_int, _c_int, _c_vpp, _c_vpp, _c_i64, _c_vp]),
    "pt_activation_series_bwd": (_c_int, [_c_int, _c_int, _c_int, _c_vpp, _c_vpp, _c_vpp, _c_i64, _c_vp]),
    "pt_series_binary": (_c_int, [_c_int, _c_int, _c_int, _c_vpp, _c_vpp, _c_vpp, _c_i64, _c_vp]),
    "pt_rms_norm_series_bwd": (_c_int, [_c_int, _c_int, _c_vpp, _c_vpp, _c_vpp, _c_i64, _c_i64, _c_dbl, _c_vp]),
    "pt_layer_norm_series_bwd": (_c_int, [_c_int, _c_int, _c_vpp, _c_vpp, _c_vpp, _c_i64, _c_i64, _c_dbl, _c_vp]),
}


class LibraryMissingError(RuntimeError):
    """The HIP kernels were not built (run ``python -m polytensors_amd.build``)."""


class KernelError(RuntimeError):
    """A pt_* entry point returned an error status."""


_lock = threading.Lock()
_lib = None


def load():
    """Load and bind the library (once); raises LibraryMissingError if absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise LibraryMissingError(
                f"{LIB_PATH} is missing: build the gfx950 kernels with `python -m polytensors_amd.build`")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (restype, argtypes) in SIGNATURES.items():
            try:
                fn = getattr(lib, name)
            except AttributeError:
                raise LibraryMissingError(f"{LIB_PATH} lacks {name}: it is stale, rebuild it") from None
            fn.restype = restype
            fn.argtypes = argtypes
        if lib.pt_abi_version() != ABI_VERSION:
            raise LibraryMissingError(f"{LIB_PATH} has ABI {lib.pt_abi_version()}, expected {ABI_VERSION}: rebuild it")
        _lib = lib
    return _lib


_torch_ops_loaded = False


def load_torch_ops():
    """Load the C++ operator registration once; False when it is not built (or the kernel
    library it links against is missing or of another ABI)."""
    global _torch_ops_loaded
    if _torch_ops_loaded:
        return True
    if not os.path.exists(TORCH_LIB_PATH):
        return False
    try:
        load()   # the kernel library first, with its ABI check (takes the lock itself)
    except (LibraryMissingError, OSError):
        return False
    with _lock:
        if not _torch_ops_loaded:
            torch.ops.load_library(TORCH_LIB_PATH)
            _torch_ops_loaded = True
    return True


def available():
    try:
        load()
    except (LibraryMissingError, OSError):
        return False
    return True


def max_degree():
    return load().pt_max_degree()


def double_array(values):
    """A host array of doubles."""
    return (ctypes.c_double * max(1, len(values)))(*values)


def ptr_array(tensors):
    """A host array of device pointers (keeps no reference to the tensors)."""
    arr = (ctypes.c_void_p * max(1, len(tensors)))()
    for i, t in enumerate(tensors):
        arr[i] = t.data_ptr()
    return arr


def stream_of(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def check(status, what):
    if status != PT_OK:
        message = load().pt_last_error().decode(errors="replace")
        kind = {PT_INVALID_ARGUMENT: "invalid argument", PT_UNSUPPORTED: "unsupported",
                PT_DEVICE_ERROR: "device error"}.get(status, f"status {status}")
        raise KernelError(f"{what}: {kind}: {message}")
