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
