"""The forward's work items with split row tiles, restated on the CPU.

fpa_fwd_kernel (csrc/fpa_fwd.h) takes its item from the workgroup id through xcd_work_item
(csrc/fpa_common.h): a per-head item index k, 0 the heaviest.  With ns split row tiles per head
(fwd_split_tiles in csrc/fpa_fwd.hip: half of the row tiles when the launch's workgroups fill at
most 70% of the slots), items 3i and 3i + 1 are the two halves of the key range of row-tile rank i
(part B: tiles jsplit .. jtmax, part A: tiles below jsplit) and item 3i + 2 is rank ns + i whole; the
items after 3 ns are the remaining ranks.  This file emulates that index arithmetic and checks, over
shapes with and without heads in multiples of 8 and ragged T, that every row tile is covered exactly
once (whole, or as parts A and B), that part A stays below every diagonal block of its rows, that
the split rows are rows rs0 .. T-1, and that the library's fpa_fwd_workspace_bytes sizes exactly
what the items write.  The GPU results of the split forward are compared with the unsplit forward
and the oracle in tests/test_gpu_parity.py.
"""
import os
import sys

import pytest

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "first-passage-attention_amd"))

NW, BM, BN, G = 4, 128, 64, 64
XCD_CUS, CUS = 32, 256
FILL = 70                            # FPA_FWD_SPLIT_FILL
WPE16, WPE32 = 3, 2                  # FPA_FWD_WPE, FPA_FWD_WPE32


def wpe(dtype, D):
    return 2 if D == 128 else 1 if D > 128 else (WPE16 if dtype == 0 else (3 if D <= 32 else WPE32))


def split_tiles(BH, T, dtype, D):
    nqt = (T + BM - 1) // BM
    if nqt < 4 or 100 * BH * nqt > FILL * CUS * wpe(dtype, D):
        return 0
    return nqt // 2


def snake_index(k, n, ncu, slots):
    s, c = divmod(k, ncu)
    return s * ncu + (ncu - 1 - c) if (s & 1) and s < slots and (s + 1) * ncu <= n else k


def xcd_work_item(L, BH, ntiles, slots):
    if BH % 8 == 0:
        xcd, hpx = L & 7, BH >> 3
        k = snake_index(L >> 3, ntiles * hpx, XCD_CUS, slots) if slots > 1 else L >> 3
        return k // hpx, (k % hpx) * 8 + xcd
    if slots > 1:
        L = (snake_index(L >> 3, (ntiles * BH) >> 3, XCD_CUS, slots) << 3) | (L & 7)
    return L // BH, L % BH


def decode(k, ns):
    if k < 3 * ns:
        i, j = divmod(k, 3)
        return (ns + i, 0) if j == 2 else (i, j + 1)
    return k - ns, 0


SHAPES = [  # (B, H, T, dtype, D)
    (4, 12, 2048, 0, 64), (2, 8, 4096, 1, 128), (1, 12, 16381, 0, 64), (2, 12, 2048, 0, 64),
    (1, 3, 1000, 0, 32), (3, 5, 777, 1, 16), (1, 1, 513, 0, 16), (1, 1, 4100, 0, 128), (2, 1, 600, 1, 256),
    (8, 12, 2048, 0, 64), (16, 12, 2048, 0, 64), (1, 2, 384, 0, 64), (1, 2, 385, 1, 64),
]


@pytest.mark.parametrize("B,H,T,dtype,D", SHAPES)
def test_items_cover_every_row_tile_once(B, H, T, dtype, D):
    BH, nqt, nkt = B * H, (T + BM - 1) // BM, (T + BN - 1) // BN
    ns = split_tiles(BH, T, dtype, D)
    assert 2 * ns <= nqt
    NB = (T + G - 1) // G
    seen = {}
    for L in range(BH * (nqt + ns)):
        k, bh = xcd_work_item(L, BH, nqt + ns, wpe(dtype, D))
        assert 0 <= k < nqt + ns and 0 <= bh < BH
        rank, part = decode(k, ns)
        assert (part != 0) == (rank < ns)
        qt = nqt - 1 - rank
        key = (bh, qt, part)
        assert key not in seen
        seen[key] = L
        q0 = qt * BM
        jtmax = min(nkt - 1, (q0 + BM - 1) // BN)
        jsplit = (jtmax + 1) >> 1
        if part:
            assert q0 >= (nqt - ns) * BM  # rows rs0 .. T-1
            for w in range(NW):  # every active wave's diagonal block lies in part B
                qw0 = q0 + 32 * w
                if qw0 < T:
                    ib = qw0 // G
                    assert jsplit <= ib <= jtmax and ib < NB
            assert jsplit >= 1 and (jsplit - 1) * BN + BN - 1 < q0  # part A: full tiles before every row
    expect = {(bh, qt, p) for bh in range(BH) for qt in range(nqt)
              for p in ((1, 2) if nqt - 1 - qt < ns else (0,))}
    assert set(seen) == expect


def _lib():
    from fpa import _lib as lib_mod
    if not os.path.exists(lib_mod.LIB_PATH):
        pytest.skip("libfpa.so is not built")
    return lib_mod.lib()


@pytest.mark.parametrize("B,H,T,dtype,D", SHAPES)
def test_workspace_bytes_match_the_split(B, H, T, dtype, D):
    L = _lib()
    BH, nqt = B * H, (T + BM - 1) // BM
    ns = split_tiles(BH, T, dtype, D)
    got = L.fpa_fwd_workspace_bytes(B, H, T, D, dtype)
    if ns == 0:
        assert got == 0
        return
    rows = BH * (T - (nqt - ns) * BM)
    esz = 2 if dtype == 0 else 4
    assert got == (rows * D * esz + 255) // 256 * 256 + 16 * rows


def test_split_only_where_the_launch_is_short():
    assert split_tiles(24, 2048, 0, 64) == 8        # B2 H12: 384 workgroups, 768 slots
    assert split_tiles(32, 2048, 0, 64) == 8        # B2 H16: 512 workgroups
    assert split_tiles(36, 2048, 0, 64) == 0        # B3 H12: 576 workgroups
    assert split_tiles(48, 2048, 0, 64) == 0        # cfg2: 768 workgroups
    assert split_tiles(16, 4096, 1, 128) == 0       # cfg3: 512 workgroups, 512 slots
    assert split_tiles(12, 16381, 0, 64) == 0       # cfg4
    assert split_tiles(2, 384, 0, 64) == 0          # three row tiles
