"""CPU oracle for First Passage Attention (FPA).

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or, for ``cpu_baseline``, as the thing timed on the host CPU).  The
product path (``impl="hip"``) never calls it.

What it restates (reference ``kernel.py`` of yliu-fort/first-passage-attention):

* ``kernel.py:3-8`` / ``README.md:11-13`` -- the definition.  For query ``t`` and
  key ``s <= t`` of a head, ``b_ts = beta * min(0, min_{s<u<=t} phi_u - psi_s)``
  with ``b_tt = 0``; ``o_t = sum_s softmax_s(q_t.k_s / sqrt(D) + b_ts) v_s``.
* ``kernel.py:23-24`` -- arithmetic in float64 if any operand is float64, else
  float32.
* ``kernel.py:31-41`` -- the hard range minimum and the soft range minimum
  ``-tau * log sum_{s<u<=t} exp(-phi_u / tau)`` (finite ``-1e30`` sentinel on the
  empty ranges so that autograd never sees ``inf - inf``).
* ``kernel.py:44-54`` -- the straight-through combination: the value is the hard
  minimum, the gradient is the soft minimum's; ``clamp(max=0)`` passes the
  gradient at equality.
* ``kernel.py:57-64`` -- causal softmax attention with autocast off.

* ``kernel.py:502-509`` -- the layer's Field: ``(delta, g, h) = x W^T + b`` in fp32
  (float64 for float64 x), ``W = cumsum_t delta``, ``phi = W + g``, ``psi = W + h``
  (:func:`field_phi_psi`; :func:`field_by_loops` restates it with loops for tiny shapes).

Two independent formulations live here so that tests can pin one with the
other: :func:`fpa_forward` / :func:`fpa_grads` (dense tensors + autograd, the
reference's own formulation) and :func:`explicit_grads` (closed-form gradient
formulas evaluated with loops, after ``test.py:66-84``).  :func:`bias_by_loops`
and :func:`attention_by_loops` are brute-force restatements for tiny shapes.
"""
import math

import numpy as np
import torch

LOG2E = 1.4426950408889634
SENTINEL = 1e30  # kernel.py:39


def compute_dtype(*xs):
    """float64 if any operand is float64, else float32 (kernel.py:23-24)."""
    return torch.float64 if any(x.dtype == torch.float64 for x in xs) else torch.float32


def _strict_upper(T, device):
    """mask[s, u] = u > s: the keys' ranges (s, t] start strictly after s."""
    idx = torch.arange(T, device=device)
    return idx[None, :] > idx[:, None]


def range_min(phi):
    """X[..., t, s] = min_{s<u<=t} phi_u, +inf where the range is empty (kernel.py:31-34)."""
    T = phi.shape[-1]
    grid = phi.unsqueeze(-2).expand(*phi.shape[:-1], T, T)           # [s, u] -> phi_u
    grid = torch.where(_strict_upper(T, phi.device), grid, torch.full_like(grid, math.inf))
    run = torch.cummin(grid, dim=-1).values                          # [s, t] = min over (s, t]
    return run.transpose(-1, -2)


def range_softmin(phi, tau):
    """L[..., t, s] = -tau * log sum_{s<u<=t} exp(-phi_u/tau) (kernel.py:37-41)."""
    T = phi.shape[-1]
    grid = (-phi / tau).unsqueeze(-2).expand(*phi.shape[:-1], T, T)
    grid = torch.where(_strict_upper(T, phi.device), grid, torch.full_like(grid, -SENTINEL))
    return (-tau * torch.logcumsumexp(grid, dim=-1)).transpose(-1, -2)


def first_passage_bias(phi, psi, beta, tau=1.0):
    """(B, H, T, T) bias indexed [t, s]; straight-through soft-min gradient (kernel.py:44-54)."""
    if not tau > 0:
        raise ValueError("tau must be positive")
    dt = compute_dtype(phi, psi)
    phi, psi = phi.to(dt), psi.to(dt)
    if torch.is_tensor(beta):
        beta = beta.reshape(-1, 1, 1)
    soft = range_softmin(phi, tau)
    hard = range_min(phi).detach()
    x = hard + (soft - soft.detach()) - psi.unsqueeze(-2)
    return beta * torch.clamp(x, max=0.0)


def causal_attention(q, k, v, bias):
    """Causal softmax attention with an additive bias, autocast off (kernel.py:57-64)."""
    dt = compute_dtype(q, bias)
    T, D = q.shape[-2], q.shape[-1]
    with torch.autocast(device_type=q.device.type, enabled=False):
        logits = torch.matmul(q.to(dt), k.to(dt).transpose(-1, -2).contiguous()) / math.sqrt(D)
        logits = logits + bias.to(dt)
        causal = torch.ones(T, T, dtype=torch.bool, device=q.device).tril()
        logits = logits.masked_fill(~causal, -math.inf)
        return torch.matmul(torch.softmax(logits, dim=-1), v.to(dt)).to(q.dtype)


def fpa_forward(q, k, v, phi, psi, beta, tau=1.0):
    """Dense FPA output (the reference's ``impl="reference"`` path)."""
    return causal_attention(q, k, v, first_passage_bias(phi, psi, beta, tau))


def fpa_grads(q, k, v, phi, psi, beta, do, tau=1.0, dtype=torch.float64):
    """(o, dq, dk, dv, dphi, dpsi, dbeta) of <o, do> by autograd, in ``dtype`` on the CPU.

    beta may be a scalar or an (H,) tensor; dbeta is always returned with shape (H,).
    """
    H = q.shape[1]
    b = beta if torch.is_tensor(beta) else torch.tensor(float(beta))
    b = b.reshape(-1)
    if b.numel() == 1:
        b = b.expand(H)
    args = [t.detach().cpu().to(dtype).requires_grad_() for t in (q, k, v, phi, psi)]
    bb = b.detach().cpu().to(dtype).contiguous().requires_grad_()
    o = fpa_forward(*args, bb, tau=tau)
    grads = torch.autograd.grad(o, args + [bb], do.detach().cpu().to(dtype))
    return [o.detach()] + [g.detach() for g in grads]


def fpa_grads_stored(q, k, v, phi, psi, beta, do, tau=1.0, store=torch.float16, dtype=torch.float64,
                     o_stored=None):
    """fpa_grads with Delta_t = sum_d dO_td O~_td taken from O~, the forward output rounded to ``store``.

    That is the Delta the reference's _bwd_delta (kernel.py:165-174) computes, from the output
    tensor the forward stored in the input dtype (and so does the HIP prep kernel).  With it
    dS_ts = P_ts (dP_ts - Delta~_t), the exact dS plus P_ts (Delta_t - Delta~_t); P_ts is the
    derivative of the row's log-sum-exp lse_t by S_ts, so the gradients of
    <o, dO> + sum_t (Delta_t - Delta~_t) lse_t, with the coefficients held fixed, are these.
    o is returned exact.  With store = dtype the result is fpa_grads'.  ``o_stored``, when given, is
    the stored output itself (the forward's result, with its own rounding) and replaces O~.
    """
    H, T, D = q.shape[1], q.shape[2], q.shape[3]
    b = beta if torch.is_tensor(beta) else torch.tensor(float(beta))
    b = b.reshape(-1)
    if b.numel() == 1:
        b = b.expand(H)
    args = [t.detach().cpu().to(dtype).requires_grad_() for t in (q, k, v, phi, psi)]
    bb = b.detach().cpu().to(dtype).contiguous().requires_grad_()
    qd, kd, vd, ph, ps = args
    logits = torch.matmul(qd, kd.transpose(-1, -2)) / math.sqrt(D) + first_passage_bias(ph, ps, bb, tau)
    causal = torch.ones(T, T, dtype=torch.bool).tril()
    logits = logits.masked_fill(~causal, -math.inf)
    lse = torch.logsumexp(logits, dim=-1)
    o = torch.matmul(torch.exp(logits - lse.unsqueeze(-1)), vd)
    dod = do.detach().cpu().to(dtype)
    delta = (dod * o.detach()).sum(-1)
    os_ = o.detach().to(store) if o_stored is None else o_stored.detach().cpu()
    delta_stored = (dod * os_.to(dtype)).sum(-1)
    loss = (o * dod).sum() + ((delta - delta_stored) * lse).sum()
    grads = torch.autograd.grad(loss, args + [bb])
    return [o.detach()] + [g.detach() for g in grads]


def dbeta_terms(q, k, v, phi, psi, beta, do, tau=1.0, dtype=torch.float64):
    """Per head, dbeta = sum_{s<=t} dS_ts min(0, x_ts) and the magnitude A of what it is made of.

    x_ts = min phi(s, t] - psi_s: the bias's value is beta * min(0, x) (kernel.py:44-54), so
    d bias / d beta = min(0, x); the reference's _bwd_kv adds dS x over its key blocks at
    kernel.py:227, 249.  dS_ts = P_ts dP_ts - P_ts Delta_t with dP = dO V^T and Delta_t = sum_d dO_td
    O_td.  A = sum |P_ts min(0, x_ts)| (|dP_ts| + |Delta_t|) bounds how far relative errors of at most e
    in every dP_ts and Delta_t (the arithmetic's own rounding, or the rounding of the stored output
    that Delta is taken from) can move dbeta: by at most e * A.  Where the two products cancel (A much
    larger than |dbeta|), rounding at the level of the arithmetic alone moves dbeta by that much.
    Returns (dbeta, A), each of shape (H,).
    """
    H, T, D = q.shape[1], q.shape[2], q.shape[3]
    b = beta if torch.is_tensor(beta) else torch.tensor(float(beta))
    b = b.reshape(-1)
    if b.numel() == 1:
        b = b.expand(H)
    qd, kd, vd, ph, ps, dod = [t.detach().cpu().to(dtype) for t in (q, k, v, phi, psi, do)]
    xm = (range_min(ph) - ps.unsqueeze(-2)).clamp(max=0.0)  # [t, s]; empty range: +inf -> 0
    causal = torch.ones(T, T, dtype=torch.bool).tril()
    logits = torch.matmul(qd, kd.transpose(-1, -2)) / math.sqrt(D) + b.detach().cpu().to(dtype).reshape(-1, 1, 1) * xm
    p = torch.softmax(logits.masked_fill(~causal, -math.inf), dim=-1)
    dp = torch.matmul(dod, vd.transpose(-1, -2))
    delta = (dod * torch.matmul(p, vd)).sum(-1, keepdim=True)
    px = (p * xm).masked_fill(~causal, 0.0)
    return (px * (dp - delta)).sum((0, 2, 3)), (px.abs() * (dp.abs() + delta.abs())).sum((0, 2, 3))

def fpa_grads_chunked(q, k, v, phi, psi, beta, do, tau=1.0, dtype=torch.float64, device=None,
                      max_elems=1 << 27):
    """fpa_grads computed over chunks of query rows, for shapes whose (T, T) tensors are too big.

    Same definition (kernel.py:23-64) and the same straight-through autograd formulation: for the
    query rows t in [t0, t1) of one chunk, keys s < t0 see the ranges (s, t] split at t0,

        min_{s<u<=t} phi_u            = min(SUF_s, PRE_t),   SUF_s = min_{s<u<t0} phi_u,  PRE_t = min_{t0<=u<=t} phi_u
        log sum_{s<u<=t} e^{-phi_u/tau} = logaddexp(LS_s, LP_t)  (the same split of the log-sum-exp)

    and keys t0 <= s < t1 use the dense formulation restricted to the chunk.  The loss <o, do> is a
    sum over rows, so each chunk is differentiated on its own and the gradients of k, v, phi, psi
    and beta accumulate over chunks.  The arithmetic runs in ``dtype`` on ``device`` (default: q's
    device), so the full-size configurations can be checked in float64 on the GPU; a pass holds at
    most about ``max_elems`` elements per (t, s) tensor.  Returns CPU tensors like fpa_grads.
    """
    dev = torch.device(device) if device is not None else q.device
    B, H, T, D = q.shape
    b = beta if torch.is_tensor(beta) else torch.tensor(float(beta))
    b = b.reshape(-1)
    if b.numel() == 1:
        b = b.expand(H)
    cast = lambda t: t.detach().to(dev, dtype).reshape((B * H,) + tuple(t.shape[2:])).contiguous()  # noqa: E731
    Q, K, V, PHI, PSI, DO = (cast(t) for t in (q, k, v, phi, psi, do))
    BETA = b.detach().to(dev, dtype).contiguous()
    out = [torch.empty_like(Q)] + [torch.zeros_like(x) for x in (Q, K, V, PHI, PSI)]
    dbeta = torch.zeros(H, dtype=dtype, device=dev)
    scale = 1.0 / math.sqrt(D)
    rows = max(1, max_elems // T)                      # (head, query row) pairs per pass
    G = max(1, min(B * H, rows // min(T, 256)))        # heads per pass (chunks of at least 256 rows)
    C = max(1, min(T, rows // G))                      # query rows per chunk
    for h0 in range(0, B * H, G):
        h1 = min(B * H, h0 + G)
        heads = torch.arange(h0, h1, device=dev) % H
        leaves = [x[h0:h1].clone().requires_grad_() for x in (Q, K, V, PHI, PSI)]
        bet = BETA.clone().requires_grad_()
        q_, k_, v_, ph, ps = leaves
        for t0 in range(0, T, C):
            t1 = min(T, t0 + C)
            a = -ph[:, :t1] / tau
            bh = bet[heads].view(-1, 1, 1)
            # Hard range minimum (no gradient: straight-through, kernel.py:44-54).
            with torch.no_grad():
                xin = range_min(ph[:, t0:t1])                                   # (G, C, C), keys in the chunk
                if t0 > 0:
                    pre = torch.cummin(ph[:, t0:t1], dim=-1).values             # min over [t0, t]
                    suf = torch.flip(torch.cummin(torch.flip(ph[:, :t0], [-1]), dim=-1).values, [-1])
                    suf = torch.cat([suf[:, 1:], torch.full_like(suf[:, :1], math.inf)], dim=-1)  # (s, t0)
                    xpre = torch.minimum(suf.unsqueeze(-2), pre.unsqueeze(-1))  # (G, C, t0)
                    hard = torch.cat([xpre, xin], dim=-1)
                else:
                    hard = xin
            # Soft range minimum (carries the gradient), with the reference's finite sentinel.
            sin = range_softmin(ph[:, t0:t1], tau)
            if t0 > 0:
                lp = torch.logcumsumexp(a[:, t0:t1], dim=-1)
                ls = torch.flip(torch.logcumsumexp(torch.flip(a[:, :t0], [-1]), dim=-1), [-1])
                ls = torch.cat([ls[:, 1:], torch.full_like(ls[:, :1], -SENTINEL)], dim=-1)
                spre = -tau * torch.logaddexp(ls.unsqueeze(-2), lp.unsqueeze(-1))
                soft = torch.cat([spre, sin], dim=-1)
            else:
                soft = sin
            x = hard + (soft - soft.detach()) - ps[:, :t1].unsqueeze(-2)
            bias = bh * torch.clamp(x, max=0.0)
            logits = torch.matmul(q_[:, t0:t1], k_[:, :t1].transpose(-1, -2).contiguous()) * scale + bias
            tt = torch.arange(t0, t1, device=dev).view(-1, 1)
            ss = torch.arange(0, t1, device=dev).view(1, -1)
            logits = logits.masked_fill(ss > tt, -math.inf)
            o_c = torch.matmul(torch.softmax(logits, dim=-1), v_[:, :t1])
            out[0][h0:h1, t0:t1] = o_c.detach()
            (o_c * DO[h0:h1, t0:t1]).sum().backward()
        for i, leaf in enumerate(leaves):
            out[i + 1][h0:h1] = leaf.grad
        dbeta += bet.grad
    shp4, shp3 = (B, H, T, D), (B, H, T)
    res = [out[0].view(shp4), out[1].view(shp4), out[2].view(shp4), out[3].view(shp4),
           out[4].view(shp3), out[5].view(shp3), dbeta]
    return [r.cpu() for r in res]


# ----------------------------------------------------------------------------
# Brute-force restatements used to pin the dense oracle on tiny shapes.
# ----------------------------------------------------------------------------

def bias_by_loops(phi, psi, beta):
    """Loop-by-loop bias from the definition (after test.py:33-42)."""
    phi, psi = np.asarray(phi, np.float64), np.asarray(psi, np.float64)
    beta = np.broadcast_to(np.asarray(beta, np.float64).reshape(-1), (phi.shape[1],))
    B, H, T = phi.shape
    out = np.zeros((B, H, T, T))
    for b in range(B):
        for h in range(H):
            for t in range(T):
                for s in range(t):
                    m = min(phi[b, h, s + 1:t + 1])
                    out[b, h, t, s] = beta[h] * min(0.0, m - psi[b, h, s])
    return out


def attention_by_loops(q, k, v, bias):
    """Row-by-row causal softmax with the bias (after test.py:51-63)."""
    q, k, v, bias = (np.asarray(x, np.float64) for x in (q, k, v, bias))
    B, H, T, D = q.shape
    o = np.zeros_like(q)
    for b in range(B):
        for h in range(H):
            for t in range(T):
                z = k[b, h, :t + 1] @ q[b, h, t] / math.sqrt(D) + bias[b, h, t, :t + 1]
                z = np.exp(z - z.max())
                o[b, h, t] = (z / z.sum()) @ v[b, h, :t + 1]
    return o


def explicit_grads(q, k, v, phi, psi, beta, do, tau=1.0):
    """Closed-form gradients, loops over (t, s) for the bias terms (after test.py:66-84).

    Softmax backward: dS = P * (dP - rowsum(dO * O)); dq = dS k / sqrt(D);
    dk = dS^T q / sqrt(D); dv = P^T dO.  Bias terms, with gate g_ts = [x_ts <= 0]
    and x_ts = min_{s<u<=t} phi_u - psi_s:
      dpsi_s -= beta * g * dS_ts;  dbeta += min(0, x_ts) * dS_ts;
      dphi_u += beta * g * dS_ts * softmax_{u' in (s, t]}(-phi_u'/tau)[u].
    """
    q, k, v, phi, psi, do = (np.asarray(x, np.float64) for x in (q, k, v, phi, psi, do))
    B, H, T, D = q.shape
    beta = np.broadcast_to(np.asarray(beta, np.float64).reshape(-1), (H,))
    bias = bias_by_loops(phi, psi, beta)
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    dphi, dpsi, dbeta = np.zeros_like(phi), np.zeros_like(psi), np.zeros(H)
    o = np.zeros_like(q)
    for b in range(B):
        for h in range(H):
            z = q[b, h] @ k[b, h].T / math.sqrt(D) + bias[b, h]
            z = np.where(np.tril(np.ones((T, T), bool)), z, -np.inf)
            p = np.exp(z - z.max(-1, keepdims=True))
            p /= p.sum(-1, keepdims=True)
            o[b, h] = p @ v[b, h]
            dp = do[b, h] @ v[b, h].T
            ds = p * (dp - (do[b, h] * o[b, h]).sum(-1, keepdims=True))
            dq[b, h] = ds @ k[b, h] / math.sqrt(D)
            dk[b, h] = ds.T @ q[b, h] / math.sqrt(D)
            dv[b, h] = p.T @ do[b, h]
            for t in range(T):
                for s in range(t):
                    rng = phi[b, h, s + 1:t + 1]
                    x = rng.min() - psi[b, h, s]
                    gate = 1.0 if x <= 0 else 0.0
                    w = np.exp(-(rng - rng.min()) / tau)
                    w /= w.sum()
                    dphi[b, h, s + 1:t + 1] += beta[h] * gate * ds[t, s] * w
                    dpsi[b, h, s] -= beta[h] * gate * ds[t, s]
                    dbeta[h] += min(0.0, x) * ds[t, s]
    return [o, dq, dk, dv, dphi, dpsi, dbeta]


# ----------------------------------------------------------------------------
# Seeded inputs (the distributions of BASELINE.json / reference test.py:108-117)
# ----------------------------------------------------------------------------

def make_inputs(B, H, T, D, dtype=torch.float16, seed=0, phi_scale=1.0, ties=False,
                psi_noise=0.5, beta="uniform", drift=0.0):
    """Seeded CPU inputs (q, k, v, phi, psi, beta, do).

    q, k, v, do ~ N(0, 1) cast to ``dtype``; phi = phi_scale * cumsum N(0, 1) - drift * t
    (rounded when ``ties``); psi = phi + psi_noise * N(0, 1); beta = U(0,1) + 0.5
    ("uniform"), ones ("ones") or softplus(N(0, 1)) ("softplus").
    """
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(B, H, T, D, generator=g).to(dtype) for _ in range(3))
    phi = torch.randn(B, H, T, generator=g).cumsum(-1) * phi_scale
    if drift:
        phi = phi - drift * torch.arange(T, dtype=phi.dtype)
    if ties:
        phi = torch.round(phi)
    psi = phi + psi_noise * torch.randn(B, H, T, generator=g)
    if beta == "uniform":
        b = torch.rand(H, generator=g) + 0.5
    elif beta == "ones":
        b = torch.ones(H)
    elif beta == "softplus":
        b = torch.nn.functional.softplus(torch.randn(H, generator=g))
    else:
        raise ValueError(beta)
    do = torch.randn(B, H, T, D, generator=g).to(dtype)
    return q, k, v, phi, psi, b, do


def field_phi_psi(x, weight, bias, n_heads):
    """phi, psi (B, H, T) of Field.forward (kernel.py:502-509) in float64, differentiable in x,
    weight and bias: lin = x W^T + b viewed as (B, T, 3, H) = (delta, g, h); W = cumsum_t delta."""
    B, T, _ = x.shape
    lin = x.double() @ weight.double().T + bias.double()
    d, g, h = lin.view(B, T, 3, n_heads).permute(2, 0, 3, 1)
    w = d.cumsum(-1)
    return w + g, w + h


def field_by_loops(x, weight, bias, n_heads):
    """field_phi_psi with explicit loops (tiny shapes only): output o = j * H + h of the
    projection is delta (j = 0), g (j = 1) or h (j = 2) of head h."""
    x, weight, bias = (np.asarray(a.detach().double()) for a in (x, weight, bias))
    B, T, C = x.shape
    phi = np.zeros((B, n_heads, T))
    psi = np.zeros((B, n_heads, T))
    for b in range(B):
        for hh in range(n_heads):
            run = 0.0
            for t in range(T):
                lin = [sum(x[b, t, c] * weight[j * n_heads + hh, c] for c in range(C)) + bias[j * n_heads + hh]
                       for j in range(3)]
                run += lin[0]
                phi[b, hh, t] = run + lin[1]
                psi[b, hh, t] = run + lin[2]
    return torch.from_numpy(phi), torch.from_numpy(psi)


def rel_err(x, ref):
    """max |x - ref| / max |ref| (reference test.py:120-121)."""
    x = torch.as_tensor(x).double().cpu()
    ref = torch.as_tensor(ref).double().cpu()
    return ((x - ref).abs().max() / ref.abs().max().clamp(min=1e-30)).item()
