"""The layer's Field prologue on the HIP kernels (fpa_field_fwd / fpa_field_bwd) against the
float64 definition of kernel.py:502-509 (oracle.field_phi_psi) and its autograd gradient.

Tolerances: phi, psi, dW, dbias and fp32 dx within 1e-5 of the largest reference value (fp32
accumulation over C features and T positions); fp16 dx within 2e-3 (its rounding).
"""
import pytest
import torch

import fpa
from oracle import fpa_oracle as O

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def hip():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from fpa import _hip, _lib
    _lib.lib()
    return _hip


def _rel(x, r):
    return ((x.double().cpu() - r).abs().max() / r.abs().max().clamp(min=1e-30)).item()


def _case(hip, x, H, seed):
    """(phi, psi, dx, dW, db) from the HIP kernels and from the float64 definition."""
    g = torch.Generator().manual_seed(seed)
    B, T, C = x.shape
    w = torch.randn(3 * H, C, generator=g) / C ** 0.5
    b = torch.randn(3 * H, generator=g)
    dphi, dpsi = torch.randn(B, H, T, generator=g), torch.randn(B, H, T, generator=g)
    dev = "cuda"
    xd = x.to(dev).requires_grad_()
    wd, bd = w.to(dev).requires_grad_(), b.to(dev).requires_grad_()
    phi, psi = hip.FieldHIP.apply(xd, wd, bd, H)
    dx, dw, db = torch.autograd.grad((phi, psi), (xd, wd, bd), (dphi.to(dev), dpsi.to(dev)))
    xr = x.detach().double().requires_grad_()
    wr, br = w.double().requires_grad_(), b.double().requires_grad_()
    rphi, rpsi = O.field_phi_psi(xr, wr, br, H)
    rdx, rdw, rdb = torch.autograd.grad((rphi, rpsi), (xr, wr, br), (dphi.double(), dpsi.double()))
    return (phi, psi, dx, dw, db), (rphi.detach(), rpsi.detach(), rdx, rdw, rdb)


@pytest.mark.parametrize("B,T,C,H,dtype", [
    (2, 100, 48, 4, torch.float32),
    (1, 1, 16, 1, torch.float32),
    (3, 257, 70, 5, torch.float32),
    (2, 300, 96, 12, torch.float16),
    (1, 64, 768, 32, torch.float32),
    (2, 45, 70, 3, torch.float16),     # C not a multiple of 4: the one-element-per-lane kernels in fp16
    # Four-feature-aligned x, by output count NO = 3H: the staged projection takes NO <= 48 (tiles 1-3),
    # proj16 NO > 48 (NT = 4 up to 64 outputs, NT = 6 beyond); the merged dx + dW launch has one
    # instantiation per output range (<3,1> NO <= 12, <6,1> <= 16, <6,2> <= 24, <9,2> <= 32, <9,3> <= 36,
    # <12,3> <= 48, <24,4> <= 64, <24,6> beyond).
    (2, 33, 20, 6, torch.float32),     # staged (NO 18): chunk of 20 features, waves with 16 and 4; dxdw <6,2>
    (3, 50, 36, 2, torch.float32),     # staged (NO 6): waves with 16, 16 and 4 features; dxdw <3,1>
    (1, 60, 40, 5, torch.float32),     # staged (NO 15); dxdw <6,1>
    (2, 50, 44, 9, torch.float16),     # staged (NO 27), fp16, C % 16 = 12; dxdw <9,2>
    (2, 77, 88, 14, torch.float32),    # staged (NO 42), C % 16 = 8; dxdw <12,3>
    (2, 70, 100, 20, torch.float32),   # proj16 NT = 4 (NO 60), last step of 4 features; dxdw <24,4>
    (1, 90, 52, 17, torch.float16),    # proj16 NT = 4 (NO 51), fp16, last step of 4 features; dxdw <24,4>
    (1, 40, 72, 24, torch.float32),    # proj16 NT = 6 (NO 72), last step of 8 features; dxdw <24,6>
    (1, 200, 768, 32, torch.float16),  # 96 outputs: six 16-wide tiles in fp16
])
def test_field_matches_the_definition(hip, B, T, C, H, dtype):
    _say(f"[field] B{B} T{T} C{C} H{H} {dtype}")
    x = torch.randn(B, T, C, generator=torch.Generator().manual_seed(B * 1000 + T)).to(dtype)
    got, ref = _case(hip, x, H, seed=T + C)
    for name, a, r in zip(("phi", "psi", "dx", "dW", "dbias"), got, ref):
        assert a.dtype == (dtype if name == "dx" else torch.float32), name
        assert torch.isfinite(a).all(), name
        tol = 2e-3 if (name == "dx" and dtype == torch.float16) else 1e-5
        assert _rel(a, r) <= tol, (name, _rel(a, r))


@pytest.mark.parametrize("C,H", [(64, 4), (70, 4), (64, 8), (100, 20)])
def test_field_without_dx(hip, C, H):
    """x that needs no gradient: the backward skips dx (a NULL dx in the C ABI) and still gives dW
    and dbias, for aligned (C = 64, 100: the dW kernel with 1, 2 and 4 output tiles) and unaligned
    (C = 70) features."""
    _say(f"[field] no dx, C={C} H={H}")
    B, T = 2, 90
    g = torch.Generator().manual_seed(C)
    x = torch.randn(B, T, C, generator=g)
    w = torch.randn(3 * H, C, generator=g) / C ** 0.5
    b = torch.randn(3 * H, generator=g)
    dphi, dpsi = torch.randn(B, H, T, generator=g), torch.randn(B, H, T, generator=g)
    dev = "cuda"
    wd, bd = w.to(dev).requires_grad_(), b.to(dev).requires_grad_()
    phi, psi = hip.FieldHIP.apply(x.to(dev), wd, bd, H)
    dw, db = torch.autograd.grad((phi, psi), (wd, bd), (dphi.to(dev), dpsi.to(dev)))
    wr, br = w.double().requires_grad_(), b.double().requires_grad_()
    rphi, rpsi = O.field_phi_psi(x.double(), wr, br, H)
    rdw, rdb = torch.autograd.grad((rphi, rpsi), (wr, br), (dphi.double(), dpsi.double()))
    for name, a, r in (("phi", phi, rphi.detach()), ("psi", psi, rpsi.detach()), ("dW", dw, rdw), ("dbias", db, rdb)):
        assert _rel(a, r) <= 1e-5, (name, _rel(a, r))


def test_field_strided_x_and_determinism(hip):
    """x as a view with a row stride wider than C (the features of a larger tensor), and two runs
    bit-identical."""
    _say("[field] strided x, determinism")
    base = torch.randn(2, 130, 80, generator=torch.Generator().manual_seed(9))
    x = base[:, :, 8:72]
    assert x.stride() == (130 * 80, 80, 1)
    got, ref = _case(hip, x, 3, seed=10)
    for name, a, r in zip(("phi", "psi", "dx", "dW", "dbias"), got, ref):
        assert _rel(a, r) <= 1e-5, (name, _rel(a, r))
    again, _ = _case(hip, x, 3, seed=10)
    assert all(torch.equal(a, b) for a, b in zip(got, again))


def test_field_lm_shape_against_fp32_torch(hip):
    """The cfg5 LM shape (B8 T2048 C768 H12, fp32 x): phi, psi and the gradients against the
    reference's own fp32 formulation on the GPU."""
    _say("[field] B8 T2048 C768 H12 fp32 against torch fp32")
    dev = "cuda"
    g = torch.Generator().manual_seed(11)
    B, T, C, H = 8, 2048, 768, 12
    x = torch.randn(B, T, C, generator=g).to(dev).requires_grad_()
    f = fpa.Field(C, H, impl="hip").to(dev)
    r = fpa.Field(C, H, impl="reference").to(dev)
    r.load_state_dict(f.state_dict())
    dphi, dpsi = torch.randn(B, H, T, generator=g).to(dev), torch.randn(B, H, T, generator=g).to(dev)
    outs = []
    for m in (f, r):
        phi, psi, _ = m(x)
        grads = torch.autograd.grad((phi, psi), (x, m.proj.weight, m.proj.bias), (dphi, dpsi))
        outs.append([phi.detach(), psi.detach()] + [t.detach() for t in grads])
    for name, a, b in zip(("phi", "psi", "dx", "dW", "dbias"), *outs):
        err = ((a - b).abs().max() / b.abs().max()).item()
        assert err <= 1e-4, (name, err)


def test_layer_uses_the_field_kernels(hip):
    """The layer on the GPU with impl=None runs Field through the kernels and matches the
    reference layer (fp32)."""
    _say("[field] layer impl=None vs reference")
    torch.manual_seed(12)
    dev = "cuda"
    m = fpa.FirstPassageAttention(64, 4).to(dev)
    r = fpa.FirstPassageAttention(64, 4, impl="reference").to(dev)
    r.load_state_dict(m.state_dict())
    assert m.field._hip(torch.empty(1, 1, 64, device=dev))
    x = torch.randn(2, 90, 64, device=dev)
    ya, yb = m(x), r(x)
    ga = torch.autograd.grad(ya.sum(), list(m.parameters()))
    gb = torch.autograd.grad(yb.sum(), list(r.parameters()))
    assert ((ya - yb).norm() / yb.norm()).item() <= 1e-4
    for a, b in zip(ga, gb):
        assert ((a - b).norm() / b.norm().clamp(min=1e-30)).item() <= 1e-4
