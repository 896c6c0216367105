"""The C-ABI library loads and exports everything include/polytaylor.h declares (CPU only).

No kernel is launched: the calls below return at argument validation, before
any device work.
"""

import ctypes
import os
import re

import pytest
import torch

from polytensors_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "polytaylor.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pt_[a-z0-9_]+)\s*\(", text)))


def test_library_is_built():
    assert os.path.exists(_lib.LIB_PATH), "build the kernels: python -m polytensors_amd.build"


def test_every_declared_symbol_is_exported_and_bound():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    names = declared_functions()
    assert len(names) >= 9
    for name in names:
        assert hasattr(lib, name), name
    assert sorted(_lib.SIGNATURES) == names


def test_version_queries():
    lib = _lib.load()
    assert lib.pt_abi_version() == _lib.ABI_VERSION
    assert lib.pt_max_degree() == 8
    assert lib.pt_max_elementwise_degree() == 16


def _vpp(n):
    return (ctypes.c_void_p * n)(*([1 << 20] * n))


@pytest.mark.parametrize("entry,args,status,needle", [
    ("pt_rms_norm_series_fwd", lambda: (0, 9, _vpp(10), None, 0, _vpp(10), 4, 8, 1e-5, None), 2, "degree"),
    ("pt_rms_norm_series_fwd", lambda: (7, 1, _vpp(2), None, 0, _vpp(2), 4, 8, 1e-5, None), 2, "dtype"),
    ("pt_rms_norm_series_fwd", lambda: (0, 1, None, None, 0, _vpp(2), 4, 8, 1e-5, None), 1, "required"),
    ("pt_rms_norm_series_fwd", lambda: (0, 1, _vpp(2), None, 3, _vpp(2), 4, 8, 1e-5, None), 1, "weight_orders"),
    ("pt_layer_norm_series_fwd", lambda: (0, 1, _vpp(2), None, 0, None, 1, _vpp(2), 4, 8, 1e-5, None), 1, "bias"),
    ("pt_rms_norm_series_fwd", lambda: (0, 1, _vpp(2), None, 0, _vpp(2), 4, 0, 1e-5, None), 1, "n >= 1"),
    ("pt_stream_copy", lambda: (1 << 20, 1 << 21, 24, 0, 1, None), 1, "multiple of 16"),
    ("pt_stream_copy", lambda: ((1 << 20) + 4, 1 << 21, 32, 0, 1, None), 1, "aligned"),
    ("pt_stream_read", lambda: (1 << 20, 32, 70000, 1, 1 << 21, None), 1, "blocks"),
    ("pt_stream_read", lambda: (1 << 20, 32, 0, 0, None, None), 1, "out"),
    # attention masks: a map of heads to masks, additive masks, mask sets
    ("pt_taylor_attention_fwd_ws", lambda: (0, 1, _vpp(2), 2, _vpp(2), 2, _vpp(2), 2, _vpp(2), None, 1, 16, 16, 64,
                                            0, 1 << 20, None, None, (ctypes.c_int64 * 3)(0, 0, 0), 0.125, None, 0,
                                            None), 1, "mask_map"),
    ("pt_taylor_attention_fwd_ws", lambda: (0, 1, _vpp(2), 2, _vpp(2), 2, _vpp(2), 2, _vpp(2), None, 1, 16, 16, 64,
                                            0, None, None, 1 << 20, None, 0.125, None, 0, None), 1, "boolean mask"),
    ("pt_taylor_attention_bwd", lambda: (0, 1, _vpp(2), _vpp(2), _vpp(2), _vpp(2), _vpp(2), _vpp(2), None, None, None,
                                         1 << 20, 0, 1, 16, 16, 64, 0, 1 << 20, None, None,
                                         (ctypes.c_int64 * 3)(1, -1, 0), 0.125, None), 1, "mask_map"),
    ("pt_attention_mask_ranges", lambda: (1 << 20, 70000, 16, 16, 1 << 21, None), 1, "n_masks"),
])
def test_argument_errors_return_before_launch(entry, args, status, needle):
    lib = _lib.load()
    got = getattr(lib, entry)(*args())
    assert got == status
    assert needle in lib.pt_last_error().decode()


def test_empty_rows_is_a_no_op():
    lib = _lib.load()
    assert lib.pt_rms_norm_series_fwd(0, 2, _vpp(3), None, 0, _vpp(3), 0, 16, 1e-5, None) == 0
    assert lib.pt_last_error().decode() == ""


def test_operator_schemas_match_the_cpp_registration():
    # polytensors_amd/_ops.py states the schemas the C++ extension (csrc/torch_ops.cpp) registers,
    # for the stand-in used when the extension is not built; the two must not drift apart
    from polytensors_amd import _ops

    if not _ops.NATIVE:
        pytest.skip("libpolytaylor_torch.so is not built")
    for name, schema in _ops.SCHEMAS.items():
        got = str(getattr(torch.ops.polytensors_amd, name).default._schema)
        assert got == f"polytensors_amd::{name}{schema}", name


def test_attention_key_split_plan():
    # few workgroups split (config 1: one head of 128 queries); config 3 does not; the pipelined
    # float32 kernel (full orders, whole 16-key blocks) and the 16-bit kernels never split
    lib = _lib.load()
    size = lib.pt_taylor_attention_fwd_workspace_size
    assert size(1, 3, 4, 4, 4, 1, 128, 128, 64) > 0                    # float64, config 1
    assert size(1, 4, 5, 5, 5, 64, 2048, 2048, 128) == 0               # float64, many workgroups
    assert size(0, 3, 4, 4, 4, 1, 128, 128, 64) == 0                   # float32, pipelined kernel
    assert size(0, 3, 4, 4, 4, 1, 128, 70, 64) > 0                     # float32, generic kernel
    assert size(2, 3, 4, 4, 4, 1, 128, 128, 64) == 0                   # bfloat16
    # bytes: chunks x rows x (1 + (K+1)(1+d)) values
    b = size(1, 3, 4, 4, 4, 1, 128, 128, 64)
    assert b % (128 * (1 + 4 * 65) * 8) == 0


def test_attention_backward_workspace_sizes():
    # float32 / float64: the rowsum(G O) series in the accumulator type, plus with materialize the
    # P and dS tiles (2 (K+1) bh ceil(L/16) ceil(S/16) tiles of 256 values); 16-bit: the series in
    # float32, plus at degrees 1..4 dense 16-bit tiles [2 (K+1)][bh][L][S rounded up to 128]
    lib = _lib.load()
    size = lib.pt_taylor_attention_bwd_workspace_size
    r256 = lambda x: (x + 255) // 256 * 256
    bh, L, S = 3, 100, 70
    for code, acc in ((0, 4), (1, 8)):
        assert size(code, 2, bh, L, S, 0) == 3 * bh * L * acc
    tiles32 = r256(bh * 7 * 5 * 256 * 4)
    assert size(0, 2, bh, L, S, 1) == r256(3 * bh * L * 4) + 2 * 3 * tiles32
    for code in (2, 3):   # bfloat16, float16
        assert size(code, 2, bh, L, S, 0) == 3 * bh * L * 4
        assert size(code, 2, bh, L, S, 1) == r256(3 * bh * L * 4) + 2 * 3 * r256(bh * L * 128 * 2)
        assert size(code, 0, bh, L, S, 1) == bh * L * 4            # degree 0: recomputed, series only
        assert size(code, 5, bh, L, S, 1) == 6 * bh * L * 4        # degrees 5..8: recomputed
        assert size(code, 4, bh, L, 129, 1) == r256(5 * bh * L * 4) + 2 * 5 * r256(bh * L * 256 * 2)
    assert size(0, 9, bh, L, S, 0) == 0 and size(0, 2, -1, L, S, 0) == 0   # out of range
