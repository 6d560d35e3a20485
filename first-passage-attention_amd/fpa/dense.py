"""Dense PyTorch path of the API: ``impl="reference"``.

The reference exposes its own definition as ``impl="reference"`` (kernel.py:20-64,
465-466); this module provides the same path for the drop-in API.  It materialises
(B, H, T, T) tensors, runs on any device, in float64 when any operand is float64
and float32 otherwise, with autocast disabled.  The hard range minimum gives the
value; the soft range minimum -tau*log sum exp(-phi/tau) gives the gradient for phi.
"""
import math

import torch

_EMPTY = 1e30  # finite stand-in for "no term" in the soft minimum (keeps autograd NaN-free)


def _work_dtype(*xs):
    return torch.float64 if any(x.dtype == torch.float64 for x in xs) else torch.float32


def _keys_window(T, device):
    """w[s, u] = True where u lies in the key range (s, ...]."""
    i = torch.arange(T, device=device)
    return i.view(1, T) > i.view(T, 1)


def _hard_range_min(phi):
    T = phi.shape[-1]
    vals = torch.where(_keys_window(T, phi.device), phi.unsqueeze(-2), phi.new_full((), math.inf))
    return vals.cummin(dim=-1).values.transpose(-1, -2)


def _soft_range_min(phi, tau):
    T = phi.shape[-1]
    vals = torch.where(_keys_window(T, phi.device), (-phi / tau).unsqueeze(-2), phi.new_full((), -_EMPTY))
    return (-tau * vals.logcumsumexp(dim=-1)).transpose(-1, -2)


def first_passage_bias(phi, psi, beta, tau=1.0):
    """The (B, H, T, T) bias indexed [t, s] of phi, psi (B, H, T) and beta (H,)."""
    if not tau > 0:
        raise ValueError("tau must be positive")
    dt = _work_dtype(phi, psi)
    phi, psi = phi.to(dt), psi.to(dt)
    if torch.is_tensor(beta):
        beta = beta.reshape(-1, 1, 1)
    soft = _soft_range_min(phi, tau)
    x = _hard_range_min(phi).detach() + (soft - soft.detach()) - psi.unsqueeze(-2)
    return beta * x.clamp(max=0.0)


def causal_attention(q, k, v, bias):
    dt = _work_dtype(q, bias)
    T = q.shape[-2]
    with torch.autocast(device_type=q.device.type, enabled=False):
        logits = (q.to(dt) @ k.to(dt).transpose(-1, -2).contiguous()) * q.shape[-1] ** -0.5 + bias.to(dt)
        allowed = torch.ones(T, T, dtype=torch.bool, device=q.device).tril()
        logits = logits.masked_fill(~allowed, -math.inf)
        return (logits.softmax(-1) @ v.to(dt)).to(q.dtype)
