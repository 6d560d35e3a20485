"""The shape envelope of the HIP path: head dimension 256, more than 65535 heads in a launch, lengths
past 131072, and the ``block`` argument.

The reference takes any power-of-two head dimension >= 16 and any length (kernel.py:454-455,
476-477, 400 of the reference) with per-head grids (NB, H, B) (kernel.py:408, 439).  Here D = 256
runs in both dtypes (single-buffered tiles in fp32, the key side split over parts of D), heads go on
grid axes (H, B), and T is taken up to 2^19.  Parity is against the float64 oracle where it is
affordable; at T > 131072 two size-independent properties stand in for it: causality (rows and
gradients of a prefix do not depend on what follows once dO is zero there) and a per-row float64
restatement of the forward for rows at the far end.
"""
import math
import sys

import pytest
import torch

from oracle import fpa_oracle as O
from test_gpu_parity import NAMES, check, run_hip

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def fpa():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    import fpa as m
    from fpa import _lib
    _lib.lib()  # loud failure if libfpa.so is missing
    return m


@pytest.mark.parametrize("B,H,T,scale,dtype,seed", [
    (1, 2, 200, 1.0, torch.float16, 400),
    (1, 2, 130, 1.0, torch.float32, 401),
    (1, 1, 150, 40.0, torch.float16, 402),
    (2, 1, 70, 1.0, torch.float32, 403),
])
def test_head_dim_256(fpa, B, H, T, scale, dtype, seed):
    _say(f"[envelope] D=256 B={B} H={H} T={T} scale={scale} {dtype} seed={seed}")
    q, k, v, phi, psi, beta, do = O.make_inputs(B, H, T, 256, dtype=dtype, seed=seed, phi_scale=scale)
    kern = run_hip(fpa, q, k, v, phi, psi, beta, do)
    check(kern, O.fpa_grads(q, k, v, phi, psi, beta, do), dtype)
    again = run_hip(fpa, q, k, v, phi, psi, beta, do)
    assert all(torch.equal(x, y) for x, y in zip(kern, again))


@pytest.mark.parametrize("B,H,T,D,dtype,seed", [
    (2050, 32, 20, 16, torch.float16, 410),   # B * H = 65600: heads pinned per XCD
    (32769, 2, 9, 16, torch.float32, 411),    # B * H = 65538: not a multiple of 8
])
def test_more_than_65535_heads(fpa, B, H, T, D, dtype, seed):
    """Every head of a launch with B * H > 65535 against the float64 oracle (run on the GPU)."""
    _say(f"[envelope] B={B} H={H} (B*H={B * H}) T={T} D={D} {dtype}")
    q, k, v, phi, psi, beta, do = O.make_inputs(B, H, T, D, dtype=dtype, seed=seed)
    kern = run_hip(fpa, q, k, v, phi, psi, beta, do)
    ref = O.fpa_grads_chunked(q, k, v, phi, psi, beta, do, device="cuda")
    check(kern, ref, dtype)


def _row_reference(q, k, v, phi, psi, beta, t):
    """o_t of one head in float64 from the definition (kernel.py:23-64 of the reference): the bias
    of key s <= t is beta * min(0, min_{s<u<=t} phi_u - psi_s), 0 for s = t."""
    qd, kd, vd = (x.double() for x in (q, k, v))
    ph, ps = phi[: t + 1].double(), psi[: t + 1].double()
    # m[s] = min phi over (s, t]: a reversed running minimum of phi[1 .. t], then +inf at s = t.
    m = torch.flip(torch.cummin(torch.flip(ph[1:], [0]), 0).values, [0])
    m = torch.cat([m, torch.tensor([math.inf], dtype=torch.float64)])
    bias = float(beta) * torch.clamp(m - ps, max=0.0)
    s = kd[: t + 1] @ qd[t] / math.sqrt(q.shape[-1]) + bias
    p = torch.softmax(s, 0)
    return p @ vd[: t + 1]


@pytest.mark.parametrize("T", [131269, 1048641, 8388608])
def test_length_beyond_131072(fpa, T):
    """T = 131269 (2052 blocks of 64), T = 1048641 (16386 blocks: past the LDS staging of the mid pass)
    and T = 8388608 (131072 blocks, the largest the library takes: 64 GiB of block-pair sums), one head,
    fp16 D16.

    With dO zero on every row >= T0 = 320, each output and gradient of positions < T0 equals that
    of the T0-long problem on the same prefix (which is itself checked against the oracle) and
    every gradient of positions >= T0 is zero.  The far rows of o are checked against a float64
    restatement of the definition, one row at a time."""
    T0, D = 320, 16
    _say(f"[envelope] T={T} (NB={(T + 63) // 64}), prefix T0={T0}, D={D} fp16")
    q, k, v, phi, psi, beta, do = O.make_inputs(1, 1, T, D, dtype=torch.float16, seed=420, beta="ones")
    do[:, :, T0:] = 0
    big = run_hip(fpa, q, k, v, phi, psi, beta, do)
    pre = [x[:, :, :T0].contiguous() for x in (q, k, v, phi, psi)]
    small = run_hip(fpa, *pre, beta, do[:, :, :T0].contiguous())
    check(small, O.fpa_grads(*pre, beta, do[:, :, :T0]), torch.float16)
    for name, xb, xs in zip(NAMES, big, small):
        assert torch.isfinite(xb).all(), name
        if name == "dbeta":
            assert torch.allclose(xb, xs, rtol=1e-6, atol=0), (name, xb, xs)
            continue
        head = xb[:, :, :T0]
        err = (head.double() - xs.double()).abs().max().item() / max(xs.double().abs().max().item(), 1e-30)
        assert err <= 1e-6, (name, err)
        if name != "o":
            assert (xb[:, :, T0:] == 0).all(), name
    o = big[0][0, 0]
    for t in (T - 1, T - 1000, T // 2 + 17, 131072):
        ref = _row_reference(q[0, 0], k[0, 0], v[0, 0], phi[0, 0], psi[0, 0], 1.0, t)
        err = (o[t].double() - ref).abs().max().item() / ref.abs().max().item()
        assert err <= 2e-3, (t, err)


def test_block_argument_is_a_no_op(fpa):
    """The HIP kernels fix their own tiling; block = 16, 32, 64 (the reference's test matrix,
    test.py:134-147) validate and give bit-identical outputs and gradients."""
    _say("[envelope] block in (16, 32, 64)")
    q, k, v, phi, psi, beta, do = O.make_inputs(1, 2, 200, 64, dtype=torch.float16, seed=430)
    runs = []
    for block in (16, 32, 64):
        dev = "cuda"
        a = [t.to(dev).clone().requires_grad_() for t in (q, k, v, phi, psi, beta)]
        o = fpa.first_passage_attention(*a, impl="hip", block=block)
        grads = torch.autograd.grad(o, a, do.to(dev))
        runs.append([o.detach().cpu()] + [g.cpu() for g in grads])
    for other in runs[1:]:
        assert all(torch.equal(x, y) for x, y in zip(runs[0], other))
