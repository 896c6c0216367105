"""The streaming probes that measure the HBM ceiling (pt_stream_copy / pt_stream_read).

They are measurement kernels, not part of the series path: checked here so the
ceiling the bench reports comes from kernels that really move every byte.
"""

import numpy as np
import pytest
import torch

from polytensors_amd import _lib

pytestmark = pytest.mark.gpu


def _words(nbytes, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(-2 ** 31, 2 ** 31 - 1, (nbytes // 4,), generator=g, dtype=torch.int64).to(torch.int32)


@pytest.mark.parametrize("nbytes", [0, 16, 4096 + 48, 1 << 20, (3 << 20) + 16 * 7])
@pytest.mark.parametrize("blocks", [0, 1, 3, 1024])
@pytest.mark.parametrize("chunked", [0, 1])
def test_copy_moves_every_byte(nbytes, blocks, chunked):
    host = _words(nbytes, nbytes + blocks)
    src = host.cuda()
    dst = torch.full_like(src, -1)
    lib = _lib.load()
    _lib.check(lib.pt_stream_copy(src.data_ptr(), dst.data_ptr(), nbytes, blocks, chunked, _lib.stream_of(src.device)),
               "stream copy")
    torch.cuda.synchronize()
    assert torch.equal(dst.cpu(), host)


@pytest.mark.parametrize("nbytes", [0, 16, 4096 + 48, 1 << 20, (3 << 20) + 16 * 7])
@pytest.mark.parametrize("blocks", [0, 1, 3, 1024])
@pytest.mark.parametrize("chunked", [0, 1])
def test_read_checksum_covers_every_word(nbytes, blocks, chunked):
    host = _words(nbytes, 7 * nbytes + blocks)
    src = host.cuda()
    lib = _lib.load()
    grid = blocks or lib.pt_stream_probe_blocks()
    out = torch.full((grid,), 12345, dtype=torch.int32, device="cuda")
    _lib.check(lib.pt_stream_read(src.data_ptr(), nbytes, blocks, chunked, out.data_ptr(), _lib.stream_of(src.device)),
               "stream read")
    torch.cuda.synchronize()
    got = np.bitwise_xor.reduce(out.cpu().numpy().view(np.uint32)) if grid else 0
    want = np.bitwise_xor.reduce(host.numpy().view(np.uint32)) if nbytes else np.uint32(0)
    assert int(got) == int(want)


@pytest.mark.parametrize("nbytes", [0, 16, 4096 + 48, (1 << 20) + 16 * 5])
@pytest.mark.parametrize("ns,nd", [(1, 1), (5, 5), (10, 5), (5, 0), (18, 9)])
def test_series_pattern_touches_every_vector(nbytes, ns, nd):
    # every destination receives the XOR of the sources at each vector; without destinations the
    # per-block words XOR to that of every source word
    srcs_host = [_words(nbytes, 100 * nbytes + 3 * s + ns) for s in range(ns)]
    srcs = [h.cuda() for h in srcs_host]
    dsts = [torch.full((nbytes // 4,), -1, dtype=torch.int32, device="cuda") for _ in range(nd)]
    lib = _lib.load()
    blocks = max(1, lib.pt_stream_series_blocks(nbytes))
    out = torch.full((blocks,), 12345, dtype=torch.int32, device="cuda")
    _lib.check(lib.pt_stream_series(_lib.ptr_array(srcs), ns, _lib.ptr_array(dsts) if nd else None, nd, nbytes,
                                    out.data_ptr(), _lib.stream_of(out.device)), "stream series")
    torch.cuda.synchronize()
    x = np.zeros(nbytes // 4, dtype=np.uint32)
    for h in srcs_host:
        x ^= h.numpy().view(np.uint32)
    for d in dsts:
        assert np.array_equal(d.cpu().numpy().view(np.uint32), x)
    if nd == 0 and nbytes:
        assert int(np.bitwise_xor.reduce(out.cpu().numpy().view(np.uint32))) == int(np.bitwise_xor.reduce(x))
