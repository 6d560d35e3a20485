"""First Passage Attention on MI355X (gfx950): the drop-in Python surface.

Same surface as the reference module ``kernel`` of yliu-fort/first-passage-attention
(kernel.py:44, 458-530): ``first_passage_attention``, ``first_passage_bias``,
``Field`` and ``FirstPassageAttention``.  ``impl="hip"`` runs the hand-written
gfx950 kernels of ``libfpa.so`` (``"triton"`` is accepted as an alias so code written
against the reference runs unchanged); ``impl="reference"`` is the dense PyTorch
definition; ``impl=None`` picks ``"hip"`` for GPU tensors and ``"reference"`` otherwise.
"""
import math

import torch
from torch import nn
from torch.nn import functional as F

from . import dense
from .dense import first_passage_bias

__all__ = ["first_passage_attention", "first_passage_bias", "Field", "FirstPassageAttention"]

_HIP_NAMES = ("hip", "triton")


def _pow2(n):
    return n >= 16 and n & (n - 1) == 0


def _check_hip(q, k, v, phi, psi, beta, tau, impl, block):
    """The reference's validation (kernel.py:463-486, same order and messages); returns beta as (H,)."""
    if impl not in _HIP_NAMES:
        raise ValueError(f"unknown implementation {impl!r}")
    if q.dim() != 4 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError("q, k and v must have the same shape (B, H, T, D)")
    if q.dtype not in (torch.float16, torch.float32) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k and v must all be fp16 or all fp32")
    B, H, T, D = q.shape
    if phi.shape != (B, H, T) or psi.shape != (B, H, T):
        raise ValueError("phi and psi must have shape (B, H, T)")
    if not _pow2(D) or not _pow2(block):
        raise ValueError("the head dimension and the block must be powers of two >= 16")
    if not torch.is_tensor(beta):
        beta = torch.tensor(float(beta), device=q.device)
    beta = beta.reshape(-1)
    if beta.numel() == 1:
        beta = beta.expand(H)
    if beta.shape != (H,):
        raise ValueError("beta must have shape (H,) or a single value")
    if not tau > 0:
        raise ValueError("tau must be positive")
    if not q.is_cuda:
        raise RuntimeError("impl='hip' needs q, k, v on a ROCm GPU")
    # The kernels dereference every pointer on q's device: a tensor elsewhere (a CPU beta, say)
    # is refused here, before any launch.
    for name, t in (("k", k), ("v", v), ("phi", phi), ("psi", psi), ("beta", beta)):
        if t.device != q.device:
            raise ValueError(f"{name} is on {t.device}, but q is on {q.device}: impl='hip' needs every "
                             "tensor on the same GPU")
    return beta


def first_passage_attention(q, k, v, phi, psi, beta, tau=1.0, impl=None, block=64):
    """o (B, H, T, D) of q, k, v (B, H, T, D), phi, psi (B, H, T) and beta (H,).

    impl: "hip" (q, k, v all fp16 or all fp32; D a power of two >= 16), "reference"
    (any device), or None for "hip" on GPU tensors and "reference" otherwise.
    block: validated like the reference's (a power of two >= 16); the HIP kernels
    choose their own tiles, so it does not change the result.
    Validation order and messages follow kernel.py:463-486.
    """
    if impl is None:
        impl = "hip" if q.is_cuda else "reference"
    if impl == "reference":
        return dense.causal_attention(q, k, v, first_passage_bias(phi, psi, beta, tau))
    beta = _check_hip(q, k, v, phi, psi, beta, tau, impl, block)
    from ._hip import FirstPassageAttentionHIP  # loads libfpa.so; raises if it is missing
    return FirstPassageAttentionHIP.apply(q, k, v, phi.float(), psi.float(), beta.float(), tau)


def _attention_packed(qkv, phi, psi, beta, tau, impl, block):
    """The layer's attention on its projection output qkv (B, T, 3, H, D): o as (B, T, H, D).

    On the HIP kernels q, k, v are read as strided views of qkv, o is written in (B, T, H, D)
    order and the backward writes d(qkv) in qkv's own layout, so the layer copies nothing
    around the attention (the reference pads and copies, kernel.py:380-384, 527)."""
    q, k, v = qkv.permute(2, 0, 3, 1, 4)
    if impl is None:
        impl = "hip" if qkv.is_cuda else "reference"
    if impl == "reference":
        return first_passage_attention(q, k, v, phi, psi, beta, tau, impl, block).transpose(1, 2)
    beta = _check_hip(q, k, v, phi, psi, beta, tau, impl, block)
    from ._hip import FirstPassageAttentionPackedHIP
    return FirstPassageAttentionPackedHIP.apply(qkv, phi.float(), psi.float(), beta.float(), tau)


class Field(nn.Module):
    """phi = W + g, psi = W + h with W = cumsum(delta), and beta = softplus(beta_raw), per head,
    from x (B, T, d_model); delta, g and h are linear maps of x computed in fp32 (kernel.py:492-509).

    impl (not in the reference's signature; keyword only, default None): "hip" runs the projection
    and the cumulative sum, and their gradient, on the HIP kernels (x fp16 or fp32 on the GPU, at
    most 32 heads) and raises for inputs outside that; "reference" runs them in PyTorch; None picks
    "hip" for GPU tensors it covers and "reference" otherwise (float64 x, CPU tensors, more than
    32 heads)."""

    def __init__(self, d_model, n_heads, beta_init=1.0, *, impl=None):
        super().__init__()
        self.n_heads = n_heads
        if impl is not None and impl not in _HIP_NAMES and impl != "reference":
            raise ValueError(f"unknown implementation {impl!r}")
        self.impl = impl
        self.proj = nn.Linear(d_model, 3 * n_heads)
        # inverse softplus, so that softplus(beta_raw) == beta_init
        self.beta_raw = nn.Parameter(torch.full((n_heads,), beta_init + math.log(-math.expm1(-beta_init))))

    def _hip(self, x):
        covered = (x.is_cuda and x.dtype in (torch.float16, torch.float32) and x.dim() == 3
                   and self.n_heads <= 32 and self.proj.weight.device == x.device)
        if self.impl is None:
            return covered
        if self.impl in _HIP_NAMES:
            if not covered:
                raise ValueError("Field with impl='hip' needs x (B, T, C) fp16 or fp32 and its weights on one "
                                 "ROCm GPU, and at most 32 heads")
            return True
        return False

    def forward(self, x):
        if self._hip(x):
            from ._hip import FieldHIP  # loads libfpa.so; raises if it is missing
            phi, psi = FieldHIP.apply(x, self.proj.weight, self.proj.bias, self.n_heads)
            return phi, psi, F.softplus(self.beta_raw)
        B, T, _ = x.shape
        dt = torch.float64 if x.dtype == torch.float64 else torch.float32
        with torch.autocast(device_type=x.device.type, enabled=False):
            lin = F.linear(x.to(dt), self.proj.weight.to(dt), self.proj.bias.to(dt))
        delta, g, h = lin.view(B, T, 3, self.n_heads).permute(2, 0, 3, 1)
        w = delta.cumsum(dim=-1)
        return w + g, w + h, F.softplus(self.beta_raw)


class FirstPassageAttention(nn.Module):
    """Multi-head causal FPA without positional encoding: x (B, T, d_model) -> (B, T, d_model)
    (kernel.py:512-530)."""

    def __init__(self, d_model, n_heads, tau=1.0, beta_init=1.0, impl=None, block=64):
        super().__init__()
        if d_model % n_heads:
            raise ValueError("d_model must be a multiple of n_heads")
        self.h, self.d = n_heads, d_model // n_heads
        self.tau, self.impl, self.block = tau, impl, block
        self.qkv = nn.Linear(d_model, 3 * d_model, bias=False)
        self.out = nn.Linear(d_model, d_model, bias=False)
        # The layer's impl picks the attention kernels; its Field uses the HIP prologue where that covers
        # the input (GPU, at most 32 heads) and the PyTorch projection otherwise, as the reference does.
        self.field = Field(d_model, n_heads, beta_init, impl="reference" if impl == "reference" else None)

    def forward(self, x):
        B, T, _ = x.shape
        qkv = self.qkv(x).view(B, T, 3, self.h, self.d)
        phi, psi, beta = self.field(x)
        o = _attention_packed(qkv, phi, psi, beta, self.tau, self.impl, self.block)  # (B, T, H, D)
        return self.out(o.reshape(B, T, -1))
