"""CPU replay of the float32 / float64 Cauchy matmul's LDS tiles (no GPU).

`csrc/cauchy_matmul.inl` stages each contraction chunk of 16 into As[order][row][k]
and Bs[order][col][k] (CauchyLds: float64 rows unpadded with 16-byte chunks
XOR-swizzled by the row, float32 rows padded by 16 bytes, float32 B stored
[Kd][N] swizzled by (n / 16) % 4). This replay performs every tile write of one
chunk (the 16-byte commits of A and of B stored [N][Kd], the scalar transposing
writes of B stored [Kd][N]) and every operand read of every wave, at the tile
shapes the launcher uses, and checks that

* each (row, k) element has its own LDS word and is read back by the lane whose
  MFMA operand needs it (lane l: row l % M, k = (l / M) RUN + step);
* under the measured gfx950 bank model (tests/lds_banks.py) the float64 operand
  reads and 16-byte writes and the float32 A-operand reads are free of bank
  conflicts. Two costs remain by design: the float64 transposing writes of B
  stored [Kd][N] (2 cycles per write at 32-row tiles, 6 at 64-row tiles, as in
  the first, padded layout), and the float32 B-operand reads of B stored [Kd][N]
  (4 cycles per read), whose swizzle keeps the float32 transposing writes
  conflict-free instead: no XOR swizzle of two row bits makes both free.
"""

import pytest

from tests.lds_banks import conflict_cycles

BK = 16


def fa(dtype_bytes, r):   # CauchyLds::fa
    if dtype_bytes == 8:
        return ((r ^ (r >> 2)) & 1) | (((r ^ (r >> 1)) & 1) << 1) | (((r ^ (r >> 3)) & 1) << 2)
    return 0


def fb(dtype_bytes, trans_b, n):   # CauchyLds::fb
    if dtype_bytes == 8:
        return fa(8, n)
    return 0 if trans_b else (n >> 4) & 3


def layout(es, trans_b):
    qv = 16 // es
    ld = BK if es == 8 else BK + qv

    def a_addr(r, k):
        return (r * ld + ((k // qv) ^ fa(es, r)) * qv + k % qv) * es

    def b_addr(n, k):
        return (n * ld + ((k // qv) ^ fb(es, trans_b, n)) * qv + k % qv) * es
    return qv, a_addr, b_addr


CASES = [  # (element bytes, BM, MFMA M, KK, B stored [N][Kd])
    (8, 32, 16, 4, False), (8, 32, 16, 4, True), (8, 64, 16, 4, False),
    (4, 64, 32, 2, False), (4, 64, 32, 2, True),
]


@pytest.mark.parametrize("es,bm,m,kk,trans_b", CASES)
def test_tiles_are_bijective_and_reads_get_their_operands(es, bm, m, kk, trans_b):
    qv, a_addr, b_addr = layout(es, trans_b)
    for addr in (a_addr, b_addr):
        words = {addr(r, k) for r in range(bm) for k in range(BK)}
        assert len(words) == bm * BK   # one word per element
    run = BK // kk
    # lane l reads row l % m, k = (l / m) run + q qv + s: the 16-byte read at k0 = (l / m) run + q qv
    for lane in range(64):
        for q in range(run // qv):
            k0 = (lane // m) * run + q * qv
            assert [a_addr(lane % m, k0) + es * s for s in range(qv)] == [a_addr(lane % m, k0 + s) for s in range(qv)]


@pytest.mark.parametrize("es,bm,m,kk,trans_b", CASES)
def test_bank_conflicts(es, bm, m, kk, trans_b):
    qv, a_addr, b_addr = layout(es, trans_b)
    run, v, threads = BK // kk, 16 // es, 256
    waves_m = 2
    wm_rows = bm // waves_m
    assert wm_rows % m == 0
    for side, addr in (("a", a_addr), ("b", b_addr)):
        for base in range(0, bm, m):
            for q in range(run // qv):
                cycles = conflict_cycles([addr(base + l % m, (l // m) * run + q * qv) for l in range(64)], 16)
                if es == 4 and side == "b" and not trans_b:
                    assert cycles == 4
                else:
                    assert cycles == 0, (side, base, q)
    writes = 0   # 16-byte commits of A (and of B stored [N][Kd]): thread v -> row v / (BK/V), chunk v % (BK/V)
    for addr in (a_addr, b_addr) if trans_b else (a_addr,):
        for w0 in range(0, bm * BK // v, 64):
            writes += conflict_cycles([addr((w0 + l) // (BK // v), ((w0 + l) % (BK // v)) * v) for l in range(64)], 16)
    if es == 8:
        assert writes == 0
    if not trans_b and es == 8:   # transposing 8-byte writes: thread v -> k = v / (BN/V), n = (v % (BN/V)) V + e
        for w0 in range(0, bm * BK // v, 64):
            for e in range(v):
                lanes = [b_addr(((w0 + l) % (bm // v)) * v + e, (w0 + l) // (bm // v)) for l in range(64)]
                assert conflict_cycles(lanes, 8) <= (2 if bm == 32 else 6)


def test_first_float64_layout_conflicted():
    # the padded, unswizzled float64 tile (rows of 18 doubles) that measured 17.4% conflict cycles
    def addr(r, k):
        return (r * 18 + k) * 8
    assert conflict_cycles([addr(l % 16, (l // 16) * 4) for l in range(64)], 16) > 0
