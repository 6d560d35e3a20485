"""Numpy model of the blockwise algorithm that the HIP kernels implement.

This is test infrastructure: it states, position by position, the decomposition
the kernels in ``first-passage-attention_amd/csrc`` compute (block statistics,
the per-pair range minimum from those statistics, and the four-part soft-min
gradient for phi), so that ``tests/test_blockwise_model.py`` can check the
decomposition itself against the dense oracle on the CPU, at any block size G,
before the kernels are run on a GPU.

Notation (one head, base-2 logs, il2 = log2(e) / tau, a_u = -phi_u * il2):
positions are cut into blocks of G; block b covers [b*G, b*G + G).
  PRE_t  = min phi[sb .. t]          PREL_t = log2 sum 2^a[sb .. t]
  SUF_s  = min phi(s .. eb)          SUFL_s = log2 sum 2^a(s .. eb)   (+inf / -inf if empty)
  BMIN_b = min phi over block b      BLSE_b = log2 sum 2^a over block b
For a pair t in block i, s in block j < i the range (s, t] is
  (s, end of j) + blocks j+1..i-1 + [start of i, t], so
  X_ts = min(SUF_s, MID_ij, PRE_t),  Z_ts = 2^SUFL_s + 2^MIDL_ij + 2^PREL_t.
Pairs inside one block use the in-block range directly.
"""
import math

import numpy as np

LOG2E = 1.4426950408889634


def lse2(x):
    x = np.asarray(x, np.float64)
    if x.size == 0:
        return -np.inf
    m = x.max()
    if m == -np.inf:
        return -np.inf
    return m + math.log2(np.exp2(x - m).sum())


def lse2_pair(a, b):
    m = max(a, b)
    if m == -np.inf:
        return -np.inf
    return m + math.log2(2.0 ** (a - m) + 2.0 ** (b - m))


def block_stats(phi, tau, G):
    T = len(phi)
    NB = -(-T // G)
    TP = NB * G
    ph = np.full(TP, np.inf)
    ph[:T] = phi
    il2 = LOG2E / tau
    a = np.where(np.isfinite(ph), -ph * il2, -np.inf)
    PRE, PREL, SUF, SUFL = (np.empty(TP) for _ in range(4))
    BMIN, BLSE = np.empty(NB), np.empty(NB)
    for b in range(NB):
        sb, eb = b * G, b * G + G
        for p in range(sb, eb):
            PRE[p] = ph[sb:p + 1].min()
            PREL[p] = lse2(a[sb:p + 1])
            SUF[p] = ph[p + 1:eb].min() if p + 1 < eb else np.inf
            SUFL[p] = lse2(a[p + 1:eb])
        BMIN[b] = ph[sb:eb].min()
        BLSE[b] = lse2(a[sb:eb])
    return dict(G=G, NB=NB, il2=il2, a=a, ph=ph, PRE=PRE, PREL=PREL, SUF=SUF, SUFL=SUFL,
                BMIN=BMIN, BLSE=BLSE, BMAXA=-BMIN * il2)


def mid_stats(st, j, i):
    """MID (min phi), MIDL (log2 sum 2^a) and CMID (max a) over blocks j+1 .. i-1."""
    mid, midl, cmid = np.inf, -np.inf, -np.inf
    for m in range(j + 1, i):
        mid = min(mid, st["BMIN"][m])
        midl = lse2_pair(midl, st["BLSE"][m])
        cmid = max(cmid, st["BMAXA"][m])
    return mid, midl, cmid


def pair_min(st, t, s):
    """X_ts = min_{s<u<=t} phi_u from block statistics (or in-block for the same block)."""
    G = st["G"]
    i, j = t // G, s // G
    if i == j:
        return st["ph"][s + 1:t + 1].min() if t > s else np.inf
    mid = mid_stats(st, j, i)[0]
    return min(st["SUF"][s], mid, st["PRE"][t])


def forward(q, k, v, phi, psi, beta, G, tau=1.0):
    """One head: (o, lse2) with the bias built from block statistics."""
    T, D = q.shape
    st = block_stats(phi, tau, G)
    X = np.full((T, T), np.inf)
    for t in range(T):
        for s in range(t):
            X[t, s] = pair_min(st, t, s)
    x = X - psi[None, :]
    bias = np.where(np.tril(np.ones((T, T), bool), -1), beta * np.minimum(x, 0.0), 0.0)
    z = (q @ k.T / math.sqrt(D) + bias) * LOG2E
    z = np.where(np.tril(np.ones((T, T), bool)), z, -np.inf)
    m = z.max(-1, keepdims=True)
    p = np.exp2(z - m)
    l = p.sum(-1, keepdims=True)
    return (p / l) @ v, (m + np.log2(l))[:, 0], X, st


def backward(q, k, v, phi, psi, beta, do, G, tau=1.0):
    """One head: (o, dq, dk, dv, dphi, dpsi, dbeta) through the blockwise decomposition."""
    T, D = q.shape
    o, lse, X, st = forward(q, k, v, phi, psi, beta, G, tau)
    NB, a = st["NB"], st["a"]
    x = X - psi[None, :]
    strict = np.tril(np.ones((T, T), bool), -1)
    z = (q @ k.T / math.sqrt(D) + np.where(strict, beta * np.minimum(x, 0.0), 0.0)) * LOG2E
    p = np.where(np.tril(np.ones((T, T), bool)), np.exp2(z - lse[:, None]), 0.0)
    dp = do @ v.T
    delta = (do * o).sum(-1)
    ds = p * (dp - delta[:, None])
    dq, dk, dv = ds @ k / math.sqrt(D), ds.T @ q / math.sqrt(D), p.T @ do
    gmat = np.where(strict & (x <= 0), ds, 0.0)
    dpsi = -beta * gmat.sum(0)
    dbeta = np.where(strict, ds * np.minimum(x, 0.0), 0.0).sum()

    # ---- soft-min gradient of phi, four parts ----
    W, R = np.zeros(NB * G), np.zeros(NB * G)
    Tb = np.zeros((NB, NB))
    C = np.where(np.isfinite(st["SUF"]), -st["SUF"] * st["il2"], -np.inf)   # max a over (s, eb)
    c_row = -st["PRE"] * st["il2"]                                         # max a over [sb, t]
    for i in range(NB):
        for j in range(i):
            _, midl, cmid = mid_stats(st, j, i)
            for s in range(j * G, min(j * G + G, T)):
                rs = max(C[s], cmid)
                if rs == -np.inf:           # column contributes neither to W nor to Tb
                    continue
                acc = 0.0
                for t in range(i * G, min(i * G + G, T)):
                    zc = 2.0 ** (st["SUFL"][s] - rs) + 2.0 ** (midl - rs) + 2.0 ** (st["PREL"][t] - rs)
                    acc += gmat[t, s] / zc
                W[s] += 2.0 ** (C[s] - rs) * acc
                if i > j + 1:
                    Tb[i, j] += 2.0 ** (cmid - rs) * acc
            for t in range(i * G, min(i * G + G, T)):
                ct = c_row[t]
                mterm = 2.0 ** (midl - ct) + 2.0 ** (st["PREL"][t] - ct)
                for s in range(j * G, j * G + G):
                    if s >= T:
                        continue
                    R[t] += gmat[t, s] / (2.0 ** (st["SUFL"][s] - ct) + mterm)
    dphi = np.zeros(T)
    for U in range(NB):
        sb = U * G
        cU = st["BMAXA"][U]
        S = 0.0
        for i in range(U + 1, NB):
            for j in range(U):
                cmid = mid_stats(st, j, i)[2]
                S += 2.0 ** (cU - cmid) * Tb[i, j]
        diag = diag_part(gmat, a, sb, min(sb + G, T))
        for u in range(sb, min(sb + G, T)):
            p1 = sum(2.0 ** (a[u] - C[s]) * W[s] for s in range(sb, u))
            p2 = sum(2.0 ** (a[u] - c_row[t]) * R[t] for t in range(u, min(sb + G, T)))
            p3 = 2.0 ** (a[u] - cU) * S
            dphi[u] = beta * (p1 + p2 + p3 + diag[u - sb])
    return o, dq, dk, dv, dphi, dpsi, dbeta


def diag_part(gmat, a, sb, eb):
    """sum over s < u <= t inside [sb, eb) of g_ts 2^{a_u} / Z_ts, by per-column recurrences.

    For column s: lz(u) = log2 sum_{s<u'<=u} 2^{a_u'} (running), rho(u) = 2^{lz(u) - lz(u+1)},
    lam(u) = g_us + rho(u) lam(u+1) (reverse), contribution 2^{a_u - lz(u)} lam(u) to u.
    """
    n = eb - sb
    out = np.zeros(n)
    for s in range(sb, eb - 1):
        lz = np.empty(n)
        run = -np.inf
        for u in range(s + 1, eb):
            run = lse2_pair(run, a[u])
            lz[u - sb] = run
        lam = 0.0
        for u in range(eb - 1, s, -1):
            rho = 2.0 ** (lz[u - sb] - lz[u + 1 - sb]) if u + 1 < eb else 0.0
            lam = gmat[u, s] + rho * lam
            out[u - sb] += 2.0 ** (a[u] - lz[u - sb]) * lam
    return out
