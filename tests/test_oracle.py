"""Pins the CPU oracle (oracle/fpa_oracle.py) against brute force, closed forms and invariants.

Mirrors the definition tests of the reference (test.py:45-105): the oracle is only
trusted because these pass.
"""
import math

import numpy as np
import pytest
import torch

from oracle import fpa_oracle as O


def random_field(B, H, T, seed, ties=False):
    g = torch.Generator().manual_seed(seed)
    phi = torch.randn(B, H, T, generator=g, dtype=torch.float64).cumsum(-1)
    if ties:
        phi = torch.round(phi)
    psi = phi + 0.5 * torch.randn(B, H, T, generator=g, dtype=torch.float64)
    beta = torch.rand(H, generator=g, dtype=torch.float64) + 0.5
    return phi, psi, beta


@pytest.mark.parametrize("ties", [False, True])
def test_bias_is_the_definition(ties):
    phi, psi, beta = random_field(2, 3, 12, seed=1 + ties, ties=ties)
    got = O.first_passage_bias(phi, psi, beta).numpy()
    assert np.array_equal(got, O.bias_by_loops(phi, psi, beta))


def test_attention_is_softmax_with_the_bias():
    B, H, T, D = 2, 3, 10, 8
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(B, H, T, D, generator=g, dtype=torch.float64) for _ in range(3))
    phi, psi, beta = random_field(B, H, T, seed=4)
    want = O.attention_by_loops(q, k, v, O.bias_by_loops(phi, psi, beta))
    got = O.fpa_forward(q, k, v, phi, psi, beta).numpy()
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("tau,scale,ties", [(0.7, 1.0, False), (1.0, 40.0, False), (0.25, 1.0, True)])
def test_gradients_match_the_closed_form(tau, scale, ties):
    B, H, T, D = 1, 2, 11, 4
    q, k, v, phi, psi, beta, do = O.make_inputs(B, H, T, D, dtype=torch.float64, seed=5,
                                                phi_scale=scale, ties=ties)
    got = O.fpa_grads(q, k, v, phi, psi, beta, do, tau=tau)
    want = O.explicit_grads(q, k, v, phi, psi, beta, do, tau=tau)
    for name, a, b in zip(("o", "dq", "dk", "dv", "dphi", "dpsi", "dbeta"), got, want):
        assert np.allclose(a.numpy(), b, rtol=1e-9, atol=1e-11), name


def test_gradient_of_the_bias_alone():
    """After reference test.py:66-84: d<bias, G>/d(phi, psi, beta) against loops."""
    B, H, T, tau = 1, 2, 9, 0.7
    phi, psi, beta = random_field(B, H, T, seed=5)
    G = torch.randn(B, H, T, T, generator=torch.Generator().manual_seed(6), dtype=torch.float64)
    args = [t.clone().requires_grad_() for t in (phi, psi, beta)]
    dphi, dpsi, dbeta = torch.autograd.grad((O.first_passage_bias(*args, tau=tau) * G).sum(), args)
    e_phi, e_psi, e_beta = np.zeros((B, H, T)), np.zeros((B, H, T)), np.zeros(H)
    for h in range(H):
        for t in range(T):
            for s in range(t):
                rng = phi[0, h, s + 1:t + 1].numpy()
                x = rng.min() - psi[0, h, s].item()
                gate = 1.0 if x <= 0 else 0.0
                w = np.exp(-(rng - rng.min()) / tau)
                e_phi[0, h, s + 1:t + 1] += beta[h].item() * gate * G[0, h, t, s].item() * w / w.sum()
                e_psi[0, h, s] -= beta[h].item() * gate * G[0, h, t, s].item()
                e_beta[h] += min(0.0, x) * G[0, h, t, s].item()
    for got, want in ((dphi, e_phi), (dpsi, e_psi), (dbeta, e_beta)):
        assert np.allclose(got.numpy(), want, rtol=1e-10, atol=1e-12)


def test_causal():
    B, H, T, D, t0 = 1, 2, 16, 8, 9
    g = torch.Generator().manual_seed(7)
    q, k, v = (torch.randn(B, H, T, D, generator=g, dtype=torch.float64) for _ in range(3))
    phi, psi, beta = random_field(B, H, T, seed=8)
    o = O.fpa_forward(q, k, v, phi, psi, beta)
    later = [t.clone() for t in (q, k, v, phi, psi)]
    for t in later:
        t[:, :, t0 + 1:] = torch.randn(t[:, :, t0 + 1:].shape, generator=g, dtype=torch.float64) * 10
    o2 = O.fpa_forward(*later, beta)
    assert torch.equal(o[:, :, :t0 + 1], o2[:, :, :t0 + 1])


def test_bias_never_rises():
    phi, psi, beta = random_field(2, 3, 24, seed=10)
    b = O.first_passage_bias(phi, psi, beta)
    T = phi.shape[-1]
    keys = torch.ones(T, T, dtype=torch.bool).tril()[:-1]
    assert (b[:, :, 1:][..., keys] <= b[:, :, :-1][..., keys]).all()


def test_zero_beta_is_plain_causal_attention():
    """beta = 0 removes the bias: the output is causal softmax attention (torch SDPA)."""
    q, k, v, phi, psi, _, _ = O.make_inputs(2, 3, 33, 16, dtype=torch.float64, seed=21)
    o = O.fpa_forward(q, k, v, phi, psi, torch.zeros(3, dtype=torch.float64))
    want = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True)
    assert torch.allclose(o, want, rtol=1e-12, atol=1e-12)


def test_small_tau_gradient_goes_to_the_argmin():
    """As tau -> 0 the soft-min weight concentrates on the argmin of phi over (s, t]."""
    phi = torch.tensor([[[0.0, 3.0, 1.0, 2.0, -1.0, 0.5]]], dtype=torch.float64)
    psi = torch.full_like(phi, 10.0)          # every gate open
    beta = torch.ones(1, dtype=torch.float64)
    G = torch.zeros(1, 1, 6, 6, dtype=torch.float64)
    G[0, 0, 3, 0] = 1.0                       # pair (t=3, s=0): range (0, 3] = {3, 1, 2}, argmin u=2
    p = phi.clone().requires_grad_()
    (dphi,) = torch.autograd.grad((O.first_passage_bias(p, psi, beta, tau=1e-3) * G).sum(), [p])
    want = torch.zeros_like(phi)
    want[0, 0, 2] = 1.0
    assert torch.allclose(dphi, want, atol=1e-12)


def test_tau_must_be_positive():
    phi, psi, beta = random_field(1, 1, 4, seed=0)
    with pytest.raises(ValueError, match="tau must be positive"):
        O.first_passage_bias(phi, psi, beta, tau=0.0)


def test_field_oracle_is_the_loop_definition():
    """field_phi_psi (tensor form) against field_by_loops (projection and running sum by hand)."""
    g = torch.Generator().manual_seed(3)
    x, w, b = torch.randn(2, 7, 5, generator=g), torch.randn(9, 5, generator=g), torch.randn(9, generator=g)
    phi, psi = O.field_phi_psi(x, w, b, 3)
    lphi, lpsi = O.field_by_loops(x, w, b, 3)
    assert torch.allclose(phi, lphi, rtol=1e-12, atol=1e-12)
    assert torch.allclose(psi, lpsi, rtol=1e-12, atol=1e-12)


def test_field_oracle_special_cases():
    """With zero weights phi and psi are t * bias_delta + bias_g / bias_h; with a single position
    there is no sum, phi = delta + g."""
    x = torch.randn(1, 6, 4)
    w = torch.zeros(6, 4)
    b = torch.tensor([1.0, -2.0, 0.5, 3.0, 0.25, -1.0])  # delta (h0, h1), g (h0, h1), h (h0, h1)
    phi, psi = O.field_phi_psi(x, w, b, 2)
    t = torch.arange(1, 7, dtype=torch.float64)
    assert torch.allclose(phi[0, 0], 1.0 * t + 0.5) and torch.allclose(phi[0, 1], -2.0 * t + 3.0)
    assert torch.allclose(psi[0, 0], 1.0 * t + 0.25) and torch.allclose(psi[0, 1], -2.0 * t - 1.0)
    x1 = torch.randn(1, 1, 4, dtype=torch.float64)
    w1 = torch.randn(3, 4, dtype=torch.float64)
    b1 = torch.randn(3, dtype=torch.float64)
    p1, s1 = O.field_phi_psi(x1, w1, b1, 1)
    lin = x1[0, 0] @ w1.T + b1
    assert torch.allclose(p1[0, 0, 0], lin[0] + lin[1]) and torch.allclose(s1[0, 0, 0], lin[0] + lin[2])


@pytest.mark.parametrize("B,H,T,D,tau,scale,ties,drift,max_elems", [
    (2, 3, 150, 16, 1.0, 1.0, False, 0.0, 1 << 27),   # one pass: the dense formulation
    (2, 3, 150, 16, 1.0, 1.0, False, 0.0, 150 * 400),  # two heads per pass
    (1, 2, 300, 32, 0.7, 3.0, True, 0.0, 300 * 40),   # chunks of 40 rows, ties, tau 0.7
    (1, 1, 257, 16, 2.0, 40.0, False, 0.0, 257 * 7),  # chunks of 7 rows (ragged), phi scale 40
    (1, 2, 280, 16, 0.25, 1.0, False, 0.2, 280 * 64),  # steep drift: deep-prefix minima, small tau
])
def test_chunked_oracle_is_the_dense_oracle(B, H, T, D, tau, scale, ties, drift, max_elems):
    """fpa_grads_chunked (query rows in chunks, keys before a chunk through the split range
    minimum and log-sum-exp) gives the dense oracle's outputs and gradients to 1e-12."""
    q, k, v, phi, psi, beta, do = O.make_inputs(B, H, T, D, dtype=torch.float32, seed=17, phi_scale=scale,
                                                ties=ties, drift=drift)
    ref = O.fpa_grads(q, k, v, phi, psi, beta, do, tau=tau)
    got = O.fpa_grads_chunked(q, k, v, phi, psi, beta, do, tau=tau, max_elems=max_elems)
    for name, x, r in zip(("o", "dq", "dk", "dv", "dphi", "dpsi", "dbeta"), got, ref):
        assert x.shape == r.shape, name
        assert O.rel_err(x, r) <= 1e-12, (name, O.rel_err(x, r))



def test_stored_output_oracle():
    """fpa_grads_stored: with no rounding it is fpa_grads; with the output stored in fp16 the gradients
    move by exactly the closed-form change of dS, P_ts (Delta_t - Delta~_t), pushed through
    dq = dS k / sqrt(D) and dk = dS^T q / sqrt(D); dv (P^T dO) does not move."""
    B, H, T, D = 1, 2, 40, 16
    q, k, v, phi, psi, beta, do = O.make_inputs(B, H, T, D, dtype=torch.float16, seed=77, phi_scale=2.0)
    exact = O.fpa_grads(q, k, v, phi, psi, beta, do, tau=0.7)
    same = O.fpa_grads_stored(q, k, v, phi, psi, beta, do, tau=0.7, store=torch.float64)
    for x, y in zip(exact, same):
        assert torch.allclose(x, y, rtol=1e-11, atol=1e-12)
    st = O.fpa_grads_stored(q, k, v, phi, psi, beta, do, tau=0.7, store=torch.float16)
    # Closed form of the change, from the float64 forward by the loop definition.
    qd, kd, vd, dod = (t.double().numpy() for t in (q, k, v, do))
    bias = O.bias_by_loops(phi.double().numpy(), psi.double().numpy(), beta.double().numpy())
    for h in range(H):
        z = qd[0, h] @ kd[0, h].T / np.sqrt(D) + bias[0, h]
        z = np.where(np.tril(np.ones((T, T), bool)), z, -np.inf)
        p = np.exp(z - z.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        o = p @ vd[0, h]
        o16 = o.astype(np.float16).astype(np.float64)
        change = p * ((dod[0, h] * o).sum(-1) - (dod[0, h] * o16).sum(-1))[:, None]
        assert np.abs(change).max() > 0  # the rounding does change dS
        dq_change = change @ kd[0, h] / np.sqrt(D)
        dk_change = change.T @ qd[0, h] / np.sqrt(D)
        assert np.allclose(st[1][0, h].numpy() - exact[1][0, h].numpy(), dq_change, rtol=1e-6, atol=1e-12)
        assert np.allclose(st[2][0, h].numpy() - exact[2][0, h].numpy(), dk_change, rtol=1e-6, atol=1e-12)
        assert np.allclose(st[3][0, h].numpy(), exact[3][0, h].numpy(), rtol=1e-11, atol=1e-12)
    # o_stored: the stored output given directly.  The exact output rounded to fp16 gives the same
    # gradients as store=float16; any other output moves dS by P_ts (Delta_t - Delta~_t) with
    # Delta~ from it, through dq as above.
    given = O.fpa_grads_stored(q, k, v, phi, psi, beta, do, tau=0.7, o_stored=exact[0].to(torch.float16))
    for x, y in zip(st, given):
        assert torch.equal(x, y)
    g = torch.Generator().manual_seed(5)
    o_other = exact[0] + 1e-3 * torch.randn(exact[0].shape, generator=g, dtype=torch.float64)
    other = O.fpa_grads_stored(q, k, v, phi, psi, beta, do, tau=0.7, store=torch.float64, o_stored=o_other)
    for h in range(H):
        z = qd[0, h] @ kd[0, h].T / np.sqrt(D) + bias[0, h]
        z = np.where(np.tril(np.ones((T, T), bool)), z, -np.inf)
        p = np.exp(z - z.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        change = p * ((dod[0, h] * (p @ vd[0, h])).sum(-1) - (dod[0, h] * o_other[0, h].numpy()).sum(-1))[:, None]
        assert np.allclose(other[1][0, h].numpy() - exact[1][0, h].numpy(), change @ kd[0, h] / np.sqrt(D),
                           rtol=1e-6, atol=1e-12)
        assert np.allclose(other[3][0, h].numpy(), exact[3][0, h].numpy(), rtol=1e-11, atol=1e-12)


@pytest.mark.parametrize("seed,scale,sign", [(5, 1.0, 1.0), (6, 4.0, -1.0), (7, 0.3, 1.0)])
def test_dbeta_terms(seed, scale, sign):
    """dbeta_terms: its dbeta is autograd's (through the straight-through bias), and its magnitude is the
    loop definition's sum_{s<t} |min(0, x_ts) P_ts| (|dP_ts| + |Delta_t|) with P, dP and Delta from the
    closed-form softmax backward (the pairs s = t add 0: the bias is 0 there); it bounds |dbeta|."""
    B, H, T, D = 1, 2, 23, 16
    q, k, v, phi, psi, beta, do = O.make_inputs(B, H, T, D, dtype=torch.float32, seed=seed, phi_scale=scale)
    beta = sign * beta
    tot, mag = O.dbeta_terms(q, k, v, phi, psi, beta, do, tau=0.8)
    ref = O.fpa_grads(q, k, v, phi, psi, beta, do, tau=0.8)[6]
    assert O.rel_err(tot, ref) <= 1e-12
    assert (mag >= tot.abs() - 1e-12).all()
    qd, kd, vd, dod, ph, ps = (t.double().numpy() for t in (q, k, v, do, phi, psi))
    bias = O.bias_by_loops(ph, ps, beta.double().numpy())
    for h in range(H):
        z = qd[0, h] @ kd[0, h].T / np.sqrt(D) + bias[0, h]
        z = np.where(np.tril(np.ones((T, T), bool)), z, -np.inf)
        p = np.exp(z - z.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        dp = dod[0, h] @ vd[0, h].T
        delta = (dod[0, h] * (p @ vd[0, h])).sum(-1)
        loop = sum(abs(min(0.0, ph[0, h, s + 1:t + 1].min() - ps[0, h, s]) * p[t, s]) * (abs(dp[t, s]) + abs(delta[t]))
                   for t in range(T) for s in range(t))
        assert abs(mag[h].item() - loop) <= 1e-12 * loop
