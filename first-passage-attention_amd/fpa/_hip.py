"""Autograd Function that runs First Passage Attention on the gfx950 HIP kernels.

Replaces the reference's ``_FirstPassageAttention`` (kernel.py:415-451): the forward
enqueues the block statistics and the forward kernel (``fpa_fwd``), the backward
enqueues the five backward kernels (``fpa_bwd``).  torch allocates every output
and scratch buffer; the kernels run on torch's current stream with no host sync.
Unlike the reference, q/k/v and do are read through their strides (no padding to a
multiple of the block and no ``.contiguous()`` copy for the layer's permuted views);
a tensor is copied only when its head dimension is not contiguous or its rows are
not 16-byte aligned.
"""
import contextlib
import functools

import torch

from . import _lib


@functools.lru_cache(maxsize=256)
def _fwd_floats(B, H, T):
    """(lse floats, state floats) of a forward of this shape."""
    L = _lib.lib()
    return L.fpa_lse_floats(B, H, T), L.fpa_state_floats(B, H, T)


@functools.lru_cache(maxsize=256)
def _bwd_ws_bytes(B, H, T, D, dtype):
    return _lib.lib().fpa_bwd_workspace_bytes(B, H, T, D, dtype)


@functools.lru_cache(maxsize=256)
def _fwd_ws_bytes(B, H, T, D, dtype):
    return _lib.lib().fpa_fwd_workspace_bytes(B, H, T, D, dtype)


def _rows_ok(t):
    ce = 8 if t.dtype == torch.float16 else 4
    s = t.stride()
    return (s[3] == 1 and t.data_ptr() % 16 == 0 and all(x % ce == 0 for x in s[:3])
            and 0 <= s[2] * 64 * t.element_size() < 2 ** 31)


def device_guard(dev):
    """torch.cuda.device(dev), or nothing to enter when dev is already the current device."""
    if dev.index is None or dev.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(dev)


def rows(t):
    """t itself when the kernels can read it through its strides, else a contiguous copy."""
    return t if _rows_ok(t) else t.contiguous()


class FwdBuffers:
    """Outputs and saved state of one forward call (all allocated by torch on q's device)."""

    def __init__(self, q, o=None):
        B, H, T, D = q.shape
        dev = q.device
        self.o = torch.empty((B, H, T, D), dtype=q.dtype, device=dev) if o is None else o
        n_lse, n_state = _fwd_floats(B, H, T)
        both = torch.empty(n_lse + n_state, dtype=torch.float32, device=dev)  # one allocation, two regions
        self.lse, self.state = both[:n_lse], both[n_lse:]
        # Scratch of the split row tiles (none for most shapes), needed only while the call runs.
        nws = _fwd_ws_bytes(B, H, T, D, _lib.dtype_code(q.dtype))
        self.ws = workspace(dev, nws) if nws else None


# Scratch kept per (device, stream) and grown on demand: a call's kernels run in stream order, so
# the next forward or backward on the same stream may reuse the same bytes.  Under HIP graph
# capture a fresh tensor is taken instead (from the graph's private pool, alive as long as the
# graph), so a later growth of the cache never frees memory that a captured graph still uses.
_WS_CACHE = {}


def workspace(dev, nbytes):
    """A uint8 device tensor of at least nbytes for one forward or backward call on the current stream."""
    if torch.cuda.is_current_stream_capturing():
        return torch.empty(nbytes, dtype=torch.uint8, device=dev)
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), torch.cuda.current_stream(dev).cuda_stream)
    ws = _WS_CACHE.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        _WS_CACHE[key] = ws
    return ws


def release_workspaces():
    """Drop the cached backward scratch (torch's allocator gets the memory back)."""
    _WS_CACHE.clear()


class BwdBuffers:
    """Gradients and scratch of one backward call."""

    def __init__(self, q, dqkv=None):
        B, H, T, D = q.shape
        dev = q.device
        if dqkv is None:  # one allocation for the three
            self.dq, self.dk, self.dv = torch.empty((3, B, H, T, D), dtype=q.dtype, device=dev).unbind(0)
        else:  # strided views of one (B, T, 3, H, D) buffer
            self.dq, self.dk, self.dv = dqkv.permute(2, 0, 3, 1, 4)
        n = B * H * T
        f = torch.empty(2 * n + H, dtype=torch.float32, device=dev)  # dphi, dpsi, dbeta in one allocation
        self.dphi, self.dpsi = f[:n].view(B, H, T), f[n:2 * n].view(B, H, T)
        self.dbeta = f[2 * n:]
        self.ws = workspace(dev, _bwd_ws_bytes(B, H, T, D, _lib.dtype_code(q.dtype)))


def fwd_args(q, k, v, phi, psi, beta, tau, out):
    """FpaFwdArgs for fpa_fwd (q/k/v already passed through rows(); phi, psi, beta float32)."""
    B, H, T, D = q.shape
    o, ws = out.o, out.ws
    return _lib.FpaFwdArgs.from_buffer_copy(_lib.FWD_PACK.pack(
        B, H, T, D, _lib.dtype_code(q.dtype), float(tau),
        q.data_ptr(), *q.stride(), k.data_ptr(), *k.stride(), v.data_ptr(), *v.stride(),
        phi.data_ptr(), *phi.stride(), psi.data_ptr(), *psi.stride(), beta.data_ptr(),
        o.data_ptr(), *o.stride(), out.lse.data_ptr(), out.state.data_ptr(), 0,
        ws.data_ptr() if ws is not None else 0))


def bwd_args(q, k, v, beta, tau, fwd, do, grads):
    """FpaBwdArgs for fpa_bwd."""
    B, H, T, D = q.shape
    o, dq, dk, dv = fwd.o, grads.dq, grads.dk, grads.dv
    return _lib.FpaBwdArgs.from_buffer_copy(_lib.BWD_PACK.pack(
        B, H, T, D, _lib.dtype_code(q.dtype), float(tau),
        q.data_ptr(), *q.stride(), k.data_ptr(), *k.stride(), v.data_ptr(), *v.stride(), beta.data_ptr(),
        o.data_ptr(), *o.stride(), do.data_ptr(), *do.stride(), fwd.lse.data_ptr(), fwd.state.data_ptr(),
        dq.data_ptr(), *dq.stride(), dk.data_ptr(), *dk.stride(), dv.data_ptr(), *dv.stride(),
        grads.dphi.data_ptr(), grads.dpsi.data_ptr(), grads.dbeta.data_ptr(), grads.ws.data_ptr(), 0))


def run_fwd(args, device):
    _lib.check(_lib.lib().fpa_fwd(args, _lib.stream_of(device)))


def run_bwd(args, device):
    _lib.check(_lib.lib().fpa_bwd(args, _lib.stream_of(device)))


def run_bwd_noalloc(args, device):
    """fpa_bwd_noalloc: the backward on the library's static per-GPU scratch (args.workspace unused)."""
    _lib.check(_lib.lib().fpa_bwd_noalloc(args, _lib.stream_of(device)))


class _Saved:
    def __init__(self, o, lse, state):
        self.o, self.lse, self.state = o, lse, state


class FirstPassageAttentionHIP(torch.autograd.Function):
    """o = FPA(q, k, v, phi, psi, beta); phi/psi/beta are float32, beta is (H,)."""

    @staticmethod
    def forward(ctx, q, k, v, phi, psi, beta, tau):
        q, k, v = rows(q), rows(k), rows(v)
        beta = beta.contiguous()
        dev = q.device
        with device_guard(dev):
            out = FwdBuffers(q)
            run_fwd(fwd_args(q, k, v, phi, psi, beta, tau, out), dev)
        ctx.save_for_backward(q, k, v, out.o, out.lse, out.state, beta)
        ctx.tau = float(tau)
        return out.o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse, state, beta = ctx.saved_tensors
        dev = q.device
        do = rows(do.to(q.dtype))
        with device_guard(dev):
            grads = BwdBuffers(q)
            run_bwd(bwd_args(q, k, v, beta, ctx.tau, _Saved(o, lse, state), do, grads), dev)
        return grads.dq, grads.dk, grads.dv, grads.dphi, grads.dpsi, grads.dbeta, None


class FirstPassageAttentionPackedHIP(torch.autograd.Function):
    """The layer's path: qkv (B, T, 3, H, D) -> o (B, T, H, D); the backward returns d(qkv) in
    qkv's layout.  The kernels read and write every tensor through its strides, so there is no
    copy on either side of the attention."""

    @staticmethod
    def forward(ctx, qkv, phi, psi, beta, tau):
        B, T, _, H, D = qkv.shape
        q, k, v = (rows(t) for t in qkv.permute(2, 0, 3, 1, 4))
        beta = beta.contiguous()
        dev = qkv.device
        with device_guard(dev):
            o_bthd = torch.empty((B, T, H, D), dtype=qkv.dtype, device=dev)
            out = FwdBuffers(q, o=o_bthd.permute(0, 2, 1, 3))
            run_fwd(fwd_args(q, k, v, phi, psi, beta, tau, out), dev)
        ctx.save_for_backward(q, k, v, out.o, out.lse, out.state, beta)
        ctx.tau = float(tau)
        return o_bthd

    @staticmethod
    def backward(ctx, do_bthd):
        q, k, v, o, lse, state, beta = ctx.saved_tensors
        B, H, T, D = q.shape
        dev = q.device
        do = rows(do_bthd.to(q.dtype).permute(0, 2, 1, 3))
        with device_guard(dev):
            dqkv = torch.empty((B, T, 3, H, D), dtype=q.dtype, device=dev)
            grads = BwdBuffers(q, dqkv=dqkv)
            run_bwd(bwd_args(q, k, v, beta, ctx.tau, _Saved(o, lse, state), do, grads), dev)
        return dqkv, grads.dphi, grads.dpsi, grads.dbeta, None


class FieldHIP(torch.autograd.Function):
    """Field's projection and cumulative sum (kernel.py:502-509) on the HIP kernels:
    x (B, T, C) fp16 or fp32 -> phi, psi (B, H, T) fp32, computed in fp32 like the reference.
    The backward gives dx (x's dtype), d(weight) and d(bias) in a fixed summation order."""

    @staticmethod
    def forward(ctx, x, weight, bias, n_heads):
        B, T, C = x.shape
        for name, t in (("weight", weight), ("bias", bias)):
            if t.device != x.device:
                raise ValueError(f"Field {name} is on {t.device}, but x is on {x.device}")
        if x.stride(2) != 1:
            x = x.contiguous()
        w = weight.float().contiguous()
        b = bias.float().contiguous()
        L = _lib.lib()
        dev = x.device
        with device_guard(dev):
            phi = torch.empty((B, n_heads, T), dtype=torch.float32, device=dev)
            psi = torch.empty_like(phi)
            ws = torch.empty(L.fpa_field_workspace_bytes(B, T, C, n_heads), dtype=torch.uint8, device=dev)
            a = _lib.FpaFieldFwdArgs()
            a.B, a.T, a.C, a.H = B, T, C, n_heads
            a.dtype = _lib.dtype_code(x.dtype)
            a.x, a.sx = _lib.ptr(x), (x.stride(0), x.stride(1))
            a.weight, a.bias = _lib.ptr(w), _lib.ptr(b)
            a.phi, a.psi, a.workspace = _lib.ptr(phi), _lib.ptr(psi), _lib.ptr(ws)
            _lib.check(L.fpa_field_fwd(a, _lib.stream_of(dev)))
        ctx.save_for_backward(x, w, ws)
        ctx.n_heads = n_heads
        ctx.wdtype, ctx.bdtype = weight.dtype, bias.dtype
        return phi, psi

    @staticmethod
    def backward(ctx, dphi, dpsi):
        x, w, ws = ctx.saved_tensors
        B, T, C = x.shape
        H = ctx.n_heads
        dev = x.device
        zeros = None
        if dphi is None or dpsi is None:
            zeros = torch.zeros((B, H, T), dtype=torch.float32, device=dev)
        dphi = zeros if dphi is None else dphi.float().contiguous()
        dpsi = zeros if dpsi is None else dpsi.float().contiguous()
        L = _lib.lib()
        with device_guard(dev):
            dx = torch.empty_like(x) if ctx.needs_input_grad[0] else None
            dw = torch.empty_like(w)
            db = torch.empty(w.shape[0], dtype=torch.float32, device=dev)
            a = _lib.FpaFieldBwdArgs()
            a.B, a.T, a.C, a.H = B, T, C, H
            a.dtype = _lib.dtype_code(x.dtype)
            a.x, a.sx = _lib.ptr(x), (x.stride(0), x.stride(1))
            a.weight, a.dphi, a.dpsi = _lib.ptr(w), _lib.ptr(dphi), _lib.ptr(dpsi)
            a.dx = _lib.ptr(dx) if dx is not None else None
            a.sdx = (dx.stride(0), dx.stride(1)) if dx is not None else (0, 0)
            a.dweight, a.dbias, a.workspace = _lib.ptr(dw), _lib.ptr(db), _lib.ptr(ws)
            _lib.check(L.fpa_field_bwd(a, _lib.stream_of(dev)))
        return dx, dw.to(ctx.wdtype), db.to(ctx.bdtype), None
