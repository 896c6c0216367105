"""The allocation-free cross-entropy entry point (pt_cross_entropy_series_fwd_noalloc).

It runs the kernels of pt_cross_entropy_series_fwd with the library's file-scope
scratch array in place of a caller workspace, so its results must equal that
entry point's bit for bit. Two calls in a row, the second on a smaller input,
check that the shared array carries nothing from one call into the next. Calls
go through the C ABI (ctypes), as a binding that cannot allocate would make them.
"""

import ctypes

import pytest
import torch

from polytensors_amd import _lib

PT_UNSUPPORTED = 2


def _series(rows, classes, degree, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    z = [(torch.randn(rows, classes, generator=g, dtype=torch.float64) * (2.0 if k == 0 else 0.5 ** k)).to(dtype)
         for k in range(degree + 1)]
    y = torch.randint(0, classes, (rows,), generator=g)
    y[::5] = -100
    return z, y


def _run(lib, noalloc, z, y, reduction, degree):
    acc = torch.float64 if z[0].dtype == torch.float64 else torch.float32
    rows = z[0].shape[0]
    loss = torch.full((degree + 1, rows) if reduction == 0 else (degree + 1,), float("nan"), dtype=acc,
                      device=z[0].device)
    lse = torch.full((degree + 1, rows), float("nan"), dtype=acc, device=z[0].device)
    code = _lib.DTYPE_CODES[z[0].dtype]
    args = (code, degree, _lib.ptr_array(z), rows, z[0].shape[1], z[0].stride(0), y.data_ptr(), -100, 0.0,
            reduction, _lib.ptr_array(list(loss.unbind(0))), _lib.ptr_array(list(lse.unbind(0))))
    stream = _lib.stream_of(z[0].device)
    if noalloc:
        status = lib.pt_cross_entropy_series_fwd_noalloc(*args, stream)
    else:
        ws = torch.empty(max(1, lib.pt_cross_entropy_series_workspace_size(code, degree, rows, reduction)),
                         dtype=torch.uint8, device=z[0].device)
        status = lib.pt_cross_entropy_series_fwd(*args, ws.data_ptr(), stream)
    _lib.check(status, "cross_entropy_series_fwd" + ("_noalloc" if noalloc else ""))
    torch.cuda.synchronize()
    return loss, lse


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.bfloat16])
def test_noalloc_equals_the_workspace_entry_point_on_two_calls(dtype):
    lib = _lib.load()
    # second call smaller: fewer rows, classes and orders than the first
    for rows, classes, degree, seed in [(3000, 1000, 4, 1), (257, 300, 2, 2)]:
        z, y = _series(rows, classes, degree, dtype, seed)
        z, y = [c.cuda() for c in z], y.cuda()
        for reduction in (1, 2, 0):
            want = _run(lib, False, z, y, reduction, degree)
            got = _run(lib, True, z, y, reduction, degree)
            print(f"[noalloc] {dtype} rows={rows} classes={classes} degree={degree} reduction={reduction}",
                  flush=True)
            assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])
            assert torch.isfinite(got[0]).all()


def test_noalloc_refuses_reductions_beyond_its_scratch_array():
    # (4 + 1) x 300000 float32 per-row losses are 6 MB > 4 MiB: refused before any device work
    lib = _lib.load()
    assert lib.pt_cross_entropy_series_noalloc_max_bytes() == 4 << 20
    ptrs = (ctypes.c_void_p * 5)(*([1 << 20] * 5))
    status = lib.pt_cross_entropy_series_fwd_noalloc(0, 4, ptrs, 300000, 32000, 32000, 1 << 21, -100, 0.0, 1,
                                                     ptrs, None, None)
    assert status == PT_UNSUPPORTED
    assert "scratch" in lib.pt_last_error().decode()


@pytest.mark.gpu
@pytest.mark.parametrize("reduction", [1, 2])
def test_noalloc_under_hip_graph_capture(reduction):
    # the callers it is for: a HIP graph holding the no-alloc call. One eager call first (it
    # looks up the scratch array's device address; capture records only the kernels). The graph
    # must hold kernel nodes only (no memset), and each replay, with the inputs rewritten in place
    # and eager work between replays, must equal the workspace entry point on those inputs.
    import ctypes as C

    lib = _lib.load()
    degree, rows, classes = 3, 1500, 700
    z, y = _series(rows, classes, degree, torch.float32, 7)
    z, y = [c.cuda() for c in z], y.cuda()
    loss = torch.empty(degree + 1, dtype=torch.float32, device="cuda")
    lse = torch.empty(degree + 1, rows, dtype=torch.float32, device="cuda")
    zp, lp, sp = _lib.ptr_array(z), _lib.ptr_array(list(loss.unbind(0))), _lib.ptr_array(list(lse.unbind(0)))

    def call():
        _lib.check(lib.pt_cross_entropy_series_fwd_noalloc(0, degree, zp, rows, classes, classes, y.data_ptr(), -100,
                                                            0.0, reduction, lp, sp, _lib.stream_of(z[0].device)),
                   "cross_entropy_series_fwd_noalloc")

    call()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph(keep_graph=True)
    with torch.cuda.graph(graph):
        call()
    hip = C.CDLL("libamdhip64.so.7")
    raw, count = C.c_void_p(graph.raw_cuda_graph()), C.c_size_t(0)
    assert hip.hipGraphGetNodes(raw, None, C.byref(count)) == 0 and count.value >= 1
    nodes = (C.c_void_p * count.value)()
    assert hip.hipGraphGetNodes(raw, nodes, C.byref(count)) == 0
    kinds = set()
    for i in range(count.value):
        kind = C.c_int(-1)
        hip.hipGraphNodeGetType(C.c_void_p(nodes[i]), C.byref(kind))
        kinds.add(kind.value)
    assert kinds == {0}, f"graph node types {kinds} (0 = kernel)"
    graph.instantiate()
    for replay in range(3):
        g = torch.Generator(device="cuda").manual_seed(100 + replay)
        for c in z:   # new inputs in place (eager work between replays)
            c.copy_(torch.randn(c.shape, generator=g, device="cuda"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = _run(lib, False, z, y, reduction, degree)
        print(f"[noalloc graph] reduction={reduction} replay={replay}", flush=True)
        assert torch.equal(loss, want[0]) and torch.equal(lse, want[1])
