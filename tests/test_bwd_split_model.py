"""The backward's split tiles, restated on the CPU.

When the fused backward (both sides in one launch) fills at most all of the GPU's slots
(bwd_split_tiles in csrc/fpa_bwd_fused.hip), the heaviest half of the key tiles and of the query tiles
run as two items each: a key tile's query blocks from its diagonal block ib0 up to ibs = ib0 + max(2,
(NB - ib0) / 2) and from ibs on; a query tile's key blocks from jbmax down to jbs = jbmax + 1 - max(2,
(jbmax + 1) / 2) and below jbs.  This file checks on the CPU, over ragged and exact lengths, that
the halves partition each tile's block range, that the diagonal blocks of all four waves stay in the
first half, that both halves are non-empty, that the host's cost split matches the kernels' ranges,
and that fpa_bwd_workspace_bytes grows by exactly the partial-sum regions.  The GPU results of the
split backward are compared with the unsplit launches and the oracle in tests/test_gpu_parity.py.
"""
import os
import sys

import pytest

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "first-passage-attention_amd"))

NW, BT, G = 4, 128, 64
CUS, FILL, FUSED_MAX = 256, 100, 1024


def kv_wpe(dtype, D):
    return 1 if (D >= 128 or (dtype == 1 and D >= 64)) else 2


def fused(dtype, D):
    return D < 256 and not (dtype == 1 and D == 64)   # kv_wpe == q_wpe, one dK/dV part, not fp32 D64


def split_tiles(BH, T, dtype, D):
    nt = (T + BT - 1) // BT
    if not fused(dtype, D) or nt < 4 or 3 * nt > FUSED_MAX or 100 * 2 * nt * BH > FILL * CUS * kv_wpe(dtype, D):
        return 0, 0
    return nt // 2, nt // 2


def kv_range(kt, NB, half):
    ib0 = kt * BT // G
    ibs = ib0 + max(2, (NB - ib0) // 2)
    return (ib0, NB) if half == 0 else (ib0, ibs) if half == 1 else (ibs, NB)


def q_range(qt, NB, half):
    jbmax = min(NB - 1, (qt * BT + BT - 1) // G)
    jbs = jbmax + 1 - max(2, (jbmax + 1) // 2)
    return (0, jbmax + 1) if half == 0 else (jbs, jbmax + 1) if half == 1 else (0, jbs)


SHAPES = [(1, 3, 1000, 0, 32), (2, 4, 600, 0, 64), (3, 5, 777, 1, 16), (1, 1, 513, 0, 16), (1, 1, 4100, 0, 128),
          (1, 2, 777, 1, 32), (1, 4, 4096, 0, 64), (1, 1, 16384, 0, 64), (4, 12, 2048, 0, 64), (1, 2, 385, 0, 64)]


@pytest.mark.parametrize("B,H,T,dtype,D", SHAPES)
def test_halves_partition_each_tile(B, H, T, dtype, D):
    nt, NB = (T + BT - 1) // BT, (T + G - 1) // G
    nks, nqs = split_tiles(B * H, T, dtype, D)
    for kt in range(nks):
        lo, hi = kv_range(kt, NB, 0)
        a, b = kv_range(kt, NB, 1), kv_range(kt, NB, 2)
        assert a[0] == lo and a[1] == b[0] and b[1] == hi and a[0] < a[1] < b[1]
        for w in range(NW):  # each wave's diagonal block (keys kt*BT + 32w ...) is in the first half
            kw0 = kt * BT + 32 * w
            if kw0 < T:
                assert a[0] <= kw0 // G < a[1]
        nnear = max(2, (NB - lo) // 2)   # the host's cost split
        assert (a[1] - a[0], b[1] - b[0]) == (nnear, NB - lo - nnear)
        assert (kt + 1) * BT <= T        # split keys are all below T
    for qt in range(nt - nqs, nt):
        lo, hi = q_range(qt, NB, 0)
        a, b = q_range(qt, NB, 1), q_range(qt, NB, 2)
        assert b[0] == lo and b[1] == a[0] and a[1] == hi and b[0] < b[1] < a[1]
        for w in range(NW):
            qw0 = qt * BT + 32 * w
            if qw0 < T:
                assert a[0] <= qw0 // G < a[1]
        nblk = hi - lo
        nnear = max(2, nblk // 2)
        assert (a[1] - a[0], b[1] - b[0]) == (nnear, nblk - nnear)
    assert 2 * nt + nks + nqs <= FUSED_MAX


def _lib():
    from fpa import _lib as lib_mod
    if not os.path.exists(lib_mod.LIB_PATH):
        pytest.skip("libfpa.so is not built")
    return lib_mod.lib()


def a64(n):
    return (n + 63) // 64 * 64


@pytest.mark.parametrize("B,H,T,dtype,D", SHAPES)
def test_workspace_bytes_hold_the_partials(B, H, T, dtype, D):
    L = _lib()
    BH, TP = B * H, (T + G - 1) // G * G
    NB, NK32, nt = TP // G, (T + 31) // 32, (T + BT - 1) // BT
    nks, nqs = split_tiles(BH, T, dtype, D)
    KS, QS = nks * BT, (nt - nqs) * BT if nqs else T
    floats = (a64(8 * BH * TP) + 2 * a64(BH * TP) + a64(BH * NB * G * G) + a64(BH * NB * NB) + a64(2 * BH * NK32)
              + a64(2 * BH * KS * 2 * D) + a64(2 * BH * KS * 2) + a64(2 * BH * (T - QS) * D) + a64(2 * BH * (T - QS)))
    assert L.fpa_bwd_workspace_bytes(B, H, T, D, dtype) == 4 * floats


def test_split_only_where_the_launch_is_short():
    assert split_tiles(12, 2048, 0, 64) == (8, 8)    # B1 H12 T2048: 384 items, 75% of the 512 slots
    assert split_tiles(16, 2048, 0, 64) == (8, 8)    # B1 H16: 512 items, all of them
    assert split_tiles(24, 2048, 0, 64) == (0, 0)    # B2 H12: 768 items
    assert split_tiles(8, 2048, 0, 64) == (8, 8)     # B1 H8: 256 items
    assert split_tiles(4, 4096, 0, 64) == (16, 16)
    assert split_tiles(48, 2048, 0, 64) == (0, 0)    # cfg2
    assert split_tiles(2, 1300, 1, 64) == (0, 0)     # fp32 D64 runs the two sides as two launches
    assert split_tiles(1, 384, 0, 64) == (0, 0)      # three tiles
