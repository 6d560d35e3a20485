"""CPU tests of the host side: the C ABI library, the Python surface and the dense path.

No GPU work here: the library is loaded and its exports and size queries are checked,
argument validation is exercised (it returns before any launch), and the
``impl="reference"`` path and the layer are checked against the oracle on the CPU.
"""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

import fpa
from fpa import _lib
from oracle import fpa_oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fpa.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(fpa_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = declared_functions()
    assert names, "no functions parsed from include/fpa.h"
    for n in names:
        assert hasattr(L, n), n
    assert L.fpa_abi_version() == _lib.ABI_VERSION


def test_struct_layout_matches_header(tmp_path):
    """The ctypes mirrors have the layout gcc gives the structs of include/fpa.h."""
    import shutil
    import subprocess
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    lines = []
    for cls, cname in ((_lib.FpaFwdArgs, "FpaFwdArgs"), (_lib.FpaBwdArgs, "FpaBwdArgs"),
                       (_lib.FpaFieldFwdArgs, "FpaFieldFwdArgs"), (_lib.FpaFieldBwdArgs, "FpaFieldBwdArgs")):
        lines.append(f'printf("{cname} sizeof %zu\\n", sizeof({cname}));')
        for n, _ in cls._fields_:
            lines.append(f'printf("{cname} {n} %zu\\n", offsetof({cname}, {n}));')
    src = tmp_path / "layout.c"
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "fpa.h"\nint main(void){\n'
                   + "\n".join(lines) + "\nreturn 0;}\n")
    exe = tmp_path / "layout"
    subprocess.run([cc, "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    for line in filter(None, out):
        cname, field, val = line.split()
        cls = getattr(_lib, cname)
        got = ctypes.sizeof(cls) if field == "sizeof" else getattr(cls, field).offset
        assert got == int(val), (cname, field, got, val)


def test_packed_args_equal_the_ctypes_structs():
    """fwd_args / bwd_args fill the argument structs with one struct.pack; the bytes are those of the
    same structs filled field by field through the ctypes mirrors (whose layout is checked against
    the header above), for strided tensors and with and without a forward workspace."""
    from fpa import _hip
    g = torch.Generator().manual_seed(0)
    base = torch.randn(2, 5, 3, 3, 16, generator=g).half()  # (B, T, 3, H, D)
    q, k, v = base.permute(2, 0, 3, 1, 4)  # (B, H, T, D) = (2, 3, 5, 16) views with the layer's strides
    do, o = torch.randn(2, 3, 5, 16).half(), torch.randn(2, 3, 5, 16).half()
    phi, psi = torch.randn(2, 3, 9)[..., :5], torch.randn(2, 3, 5)
    beta = torch.randn(3)

    class Buf:
        pass
    fb = Buf()
    fb.o, fb.lse, fb.state = o, torch.empty(64), torch.empty(32)
    gb = Buf()
    gb.dq, gb.dk, gb.dv = torch.empty((3, 2, 3, 5, 16), dtype=torch.float16).unbind(0)
    gb.dphi, gb.dpsi, gb.dbeta, gb.ws = torch.empty(2, 3, 5), torch.empty(2, 3, 5), torch.empty(3), torch.empty(8)
    S4 = ctypes.c_int64 * 4
    S3 = ctypes.c_int64 * 3
    for ws in (None, torch.empty(16)):
        fb.ws = ws
        a = _lib.FpaFwdArgs()
        a.B, a.H, a.T, a.D, a.dtype, a.tau = 2, 3, 5, 16, 0, 0.75
        a.q, a.sq, a.k, a.sk, a.v, a.sv = q.data_ptr(), S4(*q.stride()), k.data_ptr(), S4(*k.stride()), v.data_ptr(), S4(*v.stride())
        a.phi, a.sphi, a.psi, a.spsi = phi.data_ptr(), S3(*phi.stride()), psi.data_ptr(), S3(*psi.stride())
        a.beta, a.o, a.so = beta.data_ptr(), o.data_ptr(), S4(*o.stride())
        a.lse, a.state, a.phases = fb.lse.data_ptr(), fb.state.data_ptr(), 0
        a.workspace = ws.data_ptr() if ws is not None else None
        assert bytes(_hip.fwd_args(q, k, v, phi, psi, beta, 0.75, fb)) == bytes(a)
    b = _lib.FpaBwdArgs()
    b.B, b.H, b.T, b.D, b.dtype, b.tau = 2, 3, 5, 16, 0, 0.75
    b.q, b.sq, b.k, b.sk, b.v, b.sv = q.data_ptr(), S4(*q.stride()), k.data_ptr(), S4(*k.stride()), v.data_ptr(), S4(*v.stride())
    b.beta, b.o, b.so, b.dout, b.sdo = beta.data_ptr(), o.data_ptr(), S4(*o.stride()), do.data_ptr(), S4(*do.stride())
    b.lse, b.state = fb.lse.data_ptr(), fb.state.data_ptr()
    b.dq, b.sdq, b.dk, b.sdk = gb.dq.data_ptr(), S4(*gb.dq.stride()), gb.dk.data_ptr(), S4(*gb.dk.stride())
    b.dv, b.sdv = gb.dv.data_ptr(), S4(*gb.dv.stride())
    b.dphi, b.dpsi, b.dbeta, b.workspace, b.phases = (gb.dphi.data_ptr(), gb.dpsi.data_ptr(), gb.dbeta.data_ptr(),
                                                      gb.ws.data_ptr(), 0)
    assert bytes(_hip.bwd_args(q, k, v, beta, 0.75, fb, do, gb)) == bytes(b)


def test_size_queries():
    L = _lib.lib()
    B, H, T = 2, 3, 100
    TP, NB = 128, 2
    assert L.fpa_lse_floats(B, H, T) == 2 * B * H * TP
    assert L.fpa_state_floats(B, H, T) == 10 * B * H * TP + 2 * B * H * NB
    ws = L.fpa_bwd_workspace_bytes(B, H, T, 64, 0)
    assert ws % 256 == 0 and ws >= 4 * (3 * B * H * TP + B * H * NB * 64 * 64)


@pytest.mark.parametrize("field,value,code,msg", [
    ("tau", 0.0, _lib.FPA_ERR_INVALID, "tau must be positive"),
    ("D", 24, _lib.FPA_ERR_INVALID, "the head dimension and the block must be powers of two >= 16"),
    ("dtype", 7, _lib.FPA_ERR_INVALID, "q, k and v must all be fp16 or all fp32"),
    ("D", 512, _lib.FPA_ERR_UNSUPPORTED, "head dimension 512 is not built"),
    ("T", 0, _lib.FPA_ERR_INVALID, "q, k and v must have the same shape (B, H, T, D)"),
    ("T", 8388609, _lib.FPA_ERR_UNSUPPORTED, "T must be at most 8388608"),
    ("B", 65536, _lib.FPA_ERR_UNSUPPORTED, "B and H must each be at most 65535"),
    ("H", 65536, _lib.FPA_ERR_UNSUPPORTED, "B and H must each be at most 65535"),
])
def test_c_abi_validation(field, value, code, msg):
    L = _lib.lib()
    a = _lib.FpaFwdArgs()
    a.B, a.H, a.T, a.D, a.dtype, a.tau = 1, 1, 16, 64, 0, 1.0
    setattr(a, field, value)
    assert L.fpa_fwd(a, None) == code
    assert msg in L.fpa_last_error().decode()


@pytest.mark.parametrize("B,H,T,D", [(1, 1, 8388608, 64), (65535, 2, 64, 16), (1, 1, 64, 256)])
def test_c_abi_accepts_the_envelope(B, H, T, D):
    """Shapes at the edges of what the kernels take (T = 2^23, B * H > 65535, D = 256) pass
    validation: with NULL tensors the first complaint is about q, after every shape check."""
    L = _lib.lib()
    for dtype in (0, 1):
        a = _lib.FpaFwdArgs()
        a.B, a.H, a.T, a.D, a.dtype, a.tau = B, H, T, D, dtype, 1.0
        assert L.fpa_fwd(a, None) == _lib.FPA_ERR_INVALID
        assert L.fpa_last_error().decode() == "q is NULL"


def test_c_abi_rejects_unaligned_rows():
    L = _lib.lib()
    a = _lib.FpaFwdArgs()
    a.B, a.H, a.T, a.D, a.dtype, a.tau = 1, 1, 16, 64, 0, 1.0
    a.q = a.k = a.v = a.o = ctypes.c_void_p(16 * 1024)
    a.sq[:] = a.sk[:] = a.sv[:] = a.so[:] = (1024, 1024, 64, 1)
    a.sq[2] = 3   # t stride not a multiple of 8 halves
    assert L.fpa_fwd(a, None) == _lib.FPA_ERR_INVALID
    assert "16-byte aligned" in L.fpa_last_error().decode()


def test_c_abi_rejects_huge_row_stride():
    L = _lib.lib()
    a = _lib.FpaFwdArgs()
    a.B, a.H, a.T, a.D, a.dtype, a.tau = 1, 1, 16, 64, 0, 1.0
    a.q = a.k = a.v = a.o = ctypes.c_void_p(16 * 1024)
    a.sq[:] = a.sk[:] = a.sv[:] = a.so[:] = (1 << 26, 1 << 26, 1 << 25, 1)  # 64 rows span >= 2^31 bytes
    assert L.fpa_fwd(a, None) == _lib.FPA_ERR_INVALID
    assert "row stride is out of range" in L.fpa_last_error().decode()


def test_python_validation_order_and_messages():
    q = torch.zeros(1, 2, 8, 16, dtype=torch.float16)
    phi = psi = torch.zeros(1, 2, 8)
    beta = torch.ones(2)
    f = fpa.first_passage_attention
    with pytest.raises(ValueError, match="unknown implementation 'cuda'"):
        f(q, q, q, phi, psi, beta, impl="cuda")
    with pytest.raises(ValueError, match="same shape"):
        f(q, q[:, :1], q, phi, psi, beta, impl="hip")
    with pytest.raises(ValueError, match="fp16 or all fp32"):
        f(q, q.float(), q, phi, psi, beta, impl="hip")
    with pytest.raises(ValueError, match=r"phi and psi must have shape \(B, H, T\)"):
        f(q, q, q, phi[:, :1], psi, beta, impl="hip")
    with pytest.raises(ValueError, match="powers of two"):
        f(q, q, q, phi, psi, beta, impl="hip", block=24)
    with pytest.raises(ValueError, match=r"beta must have shape \(H,\)"):
        f(q, q, q, phi, psi, torch.ones(3), impl="hip")
    with pytest.raises(ValueError, match="tau must be positive"):
        f(q, q, q, phi, psi, beta, tau=-1.0, impl="hip")
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        f(q, q, q, phi, psi, beta, impl="hip")
    with pytest.raises(ValueError, match="multiple of n_heads"):
        fpa.FirstPassageAttention(30, 4)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_dense_path_matches_the_oracle(dtype):
    q, k, v, phi, psi, beta, do = O.make_inputs(2, 3, 40, 8, dtype=dtype, seed=3, phi_scale=5.0)
    a = [t.to(dtype if t.dim() == 4 else torch.float64).clone().requires_grad_() for t in (q, k, v, phi, psi)]
    b = beta.double().requires_grad_()
    o = fpa.first_passage_attention(*a, b, tau=0.6, impl="reference")
    got = [o] + list(torch.autograd.grad(o, a + [b], do.to(dtype)))
    ref = O.fpa_grads(q, k, v, phi, psi, beta, do, tau=0.6)
    tol = 1e-12 if dtype == torch.float64 else 2e-5
    for name, x, r in zip(("o", "dq", "dk", "dv", "dphi", "dpsi", "dbeta"), got, ref):
        assert O.rel_err(x.detach(), r) <= tol, name


def test_impl_none_on_cpu_is_the_dense_path():
    q, k, v, phi, psi, beta, _ = O.make_inputs(1, 2, 20, 16, dtype=torch.float64, seed=4)
    o1 = fpa.first_passage_attention(q, k, v, phi, psi, beta)
    o2 = fpa.first_passage_attention(q, k, v, phi, psi, beta, impl="reference")
    assert torch.equal(o1, o2)


def test_kernel_module_alias():
    import kernel
    assert kernel.first_passage_attention is fpa.first_passage_attention
    assert kernel.FirstPassageAttention is fpa.FirstPassageAttention


def _layer(impl, d_model=64, n_heads=4, T=50, seed=0):
    torch.manual_seed(seed)
    layer = fpa.FirstPassageAttention(d_model, n_heads, impl=impl)
    x = torch.randn(2, T, d_model, generator=torch.Generator().manual_seed(seed + 1))
    return layer, x


def test_layer_causal():
    """After test.py:184-190."""
    layer, x = _layer("reference")
    t0 = 30
    x2 = x.clone()
    x2[:, t0 + 1:] = torch.randn(x2[:, t0 + 1:].shape) * 5
    with torch.no_grad():
        assert torch.allclose(layer(x)[:, :t0 + 1], layer(x2)[:, :t0 + 1], rtol=0, atol=1e-6)


def test_layer_gradients():
    """After test.py:193-197."""
    layer, x = _layer("reference")
    layer(x).square().mean().backward()
    for name, p in layer.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad).all() and p.grad.abs().max() > 0, name


def test_field_initial_beta():
    f = fpa.Field(16, 3, beta_init=0.7)
    _, _, beta = f(torch.randn(1, 5, 16))
    assert torch.allclose(beta, torch.full((3,), 0.7), atol=1e-6)


def test_field_matches_definition():
    """phi = cumsum(delta) + g, psi = cumsum(delta) + h from one fp32 projection."""
    torch.manual_seed(5)
    f = fpa.Field(12, 2)
    x = torch.randn(2, 9, 12)
    phi, psi, _ = f(x)
    lin = x @ f.proj.weight.T + f.proj.bias
    d, g, h = lin.view(2, 9, 3, 2).permute(2, 0, 3, 1)
    assert torch.allclose(phi, d.cumsum(-1) + g, atol=1e-5)
    assert torch.allclose(psi, d.cumsum(-1) + h, atol=1e-5)


def _field_args(**kw):
    a = _lib.FpaFieldFwdArgs()
    a.B, a.T, a.C, a.H, a.dtype = 2, 100, 48, 4, _lib.FPA_F32
    a.x, a.sx = 4096, (4800, 48)
    a.weight, a.bias, a.phi, a.psi, a.workspace = 8192, 8192, 8192, 8192, 1 << 20
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("field,value,code,msg", [
    ("B", 0, _lib.FPA_ERR_INVALID, "B, T, C >= 1"),
    ("H", 33, _lib.FPA_ERR_UNSUPPORTED, "at most 32 heads"),
    ("dtype", 7, _lib.FPA_ERR_INVALID, "fp16 or fp32"),
    ("x", None, _lib.FPA_ERR_INVALID, "non-NULL"),
    ("workspace", (1 << 20) + 64, _lib.FPA_ERR_INVALID, "256-byte aligned"),
])
def test_field_c_abi_validation(field, value, code, msg):
    """fpa_field_fwd rejects bad arguments before any launch (no GPU needed)."""
    L = _lib.lib()
    rc = L.fpa_field_fwd(_field_args(**{field: value}), None)
    assert rc == code
    assert msg in L.fpa_last_error().decode()


@pytest.mark.parametrize("B,T,ok", [
    (1, 2**31 - 16, True),     # T rounded up to 16 is 2^31 - 16: taken (then stopped by the NULL x)
    (1, 2**31 - 15, False),    # rounds up to 2^31: refused before any launch
    (2, 2**30 - 8, False),     # B * TL = 2^31
    (2, 2**30 - 16, True),
])
def test_field_c_abi_length_bound(B, T, ok):
    """B * TL (T rounded up to 16) must stay below 2^31, the bound the Field kernels' position
    arithmetic is written for (their scans step in 64-bit positions, so the last chunk of a length
    near 2^31 does not wrap); no GPU needed: refused or stopped before any launch."""
    L = _lib.lib()
    rc = L.fpa_field_fwd(_field_args(B=B, T=T, x=None), None)
    err = L.fpa_last_error().decode()
    if ok:
        assert rc == _lib.FPA_ERR_INVALID and "non-NULL" in err, (rc, err)
    else:
        assert rc == _lib.FPA_ERR_UNSUPPORTED and "too large" in err, (rc, err)


def test_field_workspace_size():
    """The projection as B*3H rows of T rounded up to 16 floats, plus the dW / dbias partials (at most
    64 splits of the positions)."""
    L = _lib.lib()
    up = lambda n: (n + 63) // 64 * 64
    for B, T, C, H in ((8, 2048, 768, 12), (3, 257, 70, 5), (1, 1, 16, 1)):
        S = min(64, (B * T + 255) // 256)
        TL = (T + 15) // 16 * 16
        assert L.fpa_field_workspace_bytes(B, T, C, H) == 4 * (up(B * 3 * H * TL) + up(S * 3 * H * (C + 1)))


def test_library_is_built_from_these_sources():
    """libfpa.so carries the hash of the sources it was built from, and it is the hash of the sources
    in the tree (the loader refuses a stale library)."""
    from fpa._srchash import source_hash
    L = _lib.lib()
    assert L.fpa_source_hash().decode() == source_hash()
    assert len(source_hash()) == 16


def test_tuning_flags_change_the_baked_hash(monkeypatch):
    """A library built with extra FPA_HIPCC_FLAGS carries the source hash plus a digest of the flags,
    so the loader refuses it unless FPA_ALLOW_TUNING_BUILD=1 (no tuning build passes for a normal one)."""
    import importlib.util
    import os
    from fpa._srchash import source_hash
    spec = importlib.util.spec_from_file_location(
        "fpa_build_t", os.path.join(os.path.dirname(_lib.__file__), "..", "build.py"))
    b = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(b)
    monkeypatch.delenv("FPA_HIPCC_FLAGS", raising=False)
    assert b._baked_hash() == source_hash()
    monkeypatch.setenv("FPA_HIPCC_FLAGS", "-DFPA_KV_CLASSES=0")
    tuned = b._baked_hash()
    assert tuned.startswith(source_hash() + "+") and len(tuned) == 16 + 1 + 8
    monkeypatch.setenv("FPA_HIPCC_FLAGS", "-DFPA_KV_CLASSES=1")
    assert b._baked_hash() != tuned


def test_field_impl_is_validated():
    with pytest.raises(ValueError, match="unknown implementation"):
        fpa.Field(16, 2, impl="cuda")
    layer = fpa.FirstPassageAttention(64, 2, impl="hip")
    assert layer.field.impl is None  # the layer's Field picks HIP or PyTorch per input
