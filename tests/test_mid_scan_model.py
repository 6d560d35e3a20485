"""The middle-block sums of the backward's dphi, both ways the combine takes them, on the CPU.

For query block U of a head the combine needs, with c_b the largest a = -phi log2(e) / tau over block
b, cmid(i, j) the largest c_b over blocks j+1 .. i-1 and V(i, j) = 2^{cmid(i, j)} M(i, j) the table
the key side writes (M the middle-block soft-min sum of a block pair),

    2^{c_U} sum_{j < U < i} M(i, j) = sum_{j < U < i} 2^{c_U - cmid(i, j)} V(i, j).

Below 160 blocks per head the combine adds that over every pair (stepping the pair index without a
division, four pairs per thread at a time); from 160 blocks on a separate pass (one wave of 64 lanes
per query block i) first turns row i into prefix sums Q_i(U), each relative to m_U = max(c_U ..
c_{i-1}), and stores them times 2^{c_U - m_U}, so that the combine adds sum_{i > U} of those.  This file
restates both in float64 lane by lane as the kernels run them (the lane segments, the down pass
with parked m_U, the affine-map scan across lanes, the up pass) and checks them against the direct
sum, including rows shorter than a wave, rows that do not divide into 64 segments and a wide
spread of c.  The GPU runs of both forms are compared with the float64 oracle in
tests/test_gpu_configs.py.
"""
import numpy as np
import pytest

LANES = 256  # threads of a combine workgroup
WAVE = 64


def range_max(c):
    """rm[j, i] = max(c[j+1 .. i-1]) for j + 1 < i."""
    NB = len(c)
    rm = np.full((NB, NB), -np.inf)
    for j in range(NB):
        run = -np.inf
        for i in range(j + 2, NB):
            run = max(run, c[i - 1])
            rm[j, i] = run
    return rm


def direct(c, V, U, rm):
    NB = len(c)
    return sum(2.0 ** (c[U] - rm[j, i]) * V[i, j] for i in range(U + 1, NB) for j in range(U))


def combine_pairs(c, V, U):
    """The combine's pair loop: thread tid takes pairs idx = tid, tid + 256, ... (ib, jb) stepped
    without a division, four at a time; per-thread sums added in thread order."""
    NB = len(c)
    npairs = U * (NB - 1 - U)
    scanA = np.full(NB, -np.inf)                                   # max over [j, U)
    scanA[:U] = np.maximum.accumulate(c[:U][::-1])[::-1]
    scanB = np.full(NB, -np.inf)                                   # max over (U, i]
    scanB[U + 1:] = np.maximum.accumulate(c[U + 1:])
    dq, dr = LANES // U, LANES - (LANES // U) * U
    total = 0.0
    for tid in range(LANES):
        ib, jb, acc, idx = U + 1 + tid // U, tid % U, 0.0, tid
        while idx < npairs:
            for r in range(4):
                if idx + r * LANES < npairs:
                    assert (ib, jb) == (U + 1 + (idx + r * LANES) // U, (idx + r * LANES) % U)
                    cm = max(scanA[jb + 1], c[U], scanB[ib - 1])
                    acc += 2.0 ** (c[U] - cm) * V[ib, jb]
                jb += dr
                ib += dq
                if jb >= U:
                    jb -= U
                    ib += 1
            idx += 4 * LANES
        total += acc
    return total


def mid_pass(c, V):
    """fpa_bwd_mid_kernel on one head: Q[U, i] = 2^{c_U - m_U} Q_i(U) in the upper triangle."""
    NB = len(c)
    Q = np.zeros((NB, NB))
    for i in range(2, NB):
        n = i - 1
        k = (n + WAVE - 1) // WAVE
        seg = [(min(l * k, n), min(min(l * k, n) + k, n)) for l in range(WAVE)]
        smax = [max(c[lo:hi], default=-np.inf) for lo, hi in seg]
        mhi = [max(max(smax[l + 1:], default=-np.inf), c[i - 1]) for l in range(WAVE)]
        maps, mlo = [], []
        for l, (lo, hi) in enumerate(seg):  # down pass: Q(hi) = A Q(lo) + B, m_U parked
            A, B, mn = 1.0, 0.0, mhi[l]
            for U in range(hi - 1, lo - 1, -1):
                m = max(c[U], mn)
                B += V[i, U] * A
                A *= 2.0 ** (mn - m)
                if U > lo:
                    Q[U, i] = m
                mn = m
            maps.append((A, B))
            mlo.append(mn)
        q_in, B_run = [], 0.0
        for l in range(WAVE):  # inclusive scan of the maps; the value entering each segment
            q_in.append(B_run if l else 0.0)
            B_run = maps[l][0] * B_run + maps[l][1]
        for l, (lo, hi) in enumerate(seg):  # up pass
            q, m = q_in[l], mlo[l]
            for U in range(lo, hi):
                mn = Q[U + 1, i] if U + 1 < hi else mhi[l]
                q = 2.0 ** (mn - m) * q + V[i, U]
                Q[U + 1, i] = 2.0 ** (c[U + 1] - mn) * q
                m = mn
    return Q


def combine_prefix(c, Q, U):
    return sum(Q[U, i] for i in range(U + 1, len(c)))


@pytest.mark.parametrize("NB,spread,seed", [(3, 1.0, 0), (9, 30.0, 1), (70, 5.0, 2), (131, 60.0, 3), (200, 20.0, 4)])
def test_middle_block_sums_both_ways(NB, spread, seed):
    rng = np.random.default_rng(seed)
    c = rng.normal(0.0, spread, NB)
    V = rng.normal(0.0, 1.0, (NB, NB))
    V[np.triu_indices(NB, -1)] = np.nan  # only j <= i - 2 is ever written by the key side
    Q = mid_pass(c, np.nan_to_num(V, nan=0.0) * np.tril(np.ones((NB, NB)), -2))
    rm = range_max(c)
    for U in range(1, NB - 1):
        ref = direct(c, V, U, rm)
        for got in (combine_pairs(c, V, U), combine_prefix(c, Q, U)):
            assert abs(got - ref) <= 1e-10 * (1.0 + abs(ref)), (NB, U, got, ref)


def test_prefix_factors_never_exceed_one():
    """Every factor the prefix pass multiplies by is 2^{m_{U+1} - m_U} <= 1 (m is a suffix maximum), so
    a wide spread of a cannot overflow the running sums."""
    rng = np.random.default_rng(7)
    for _ in range(20):
        c = rng.normal(0.0, 200.0, 50)
        for i in range(2, 50):
            m = [max(c[U:i]) for U in range(i)]
            assert all(m[U + 1] <= m[U] for U in range(i - 1))
