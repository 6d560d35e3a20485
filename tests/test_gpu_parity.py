"""Parity of the HIP kernels (impl="hip", libfpa.so) with the float64 CPU oracle.

Mirrors the kernel tests of the reference (test.py:134-214): every output and gradient
must be finite, have the reference's dtype (o, dq, dk, dv in the input dtype; dphi,
dpsi, dbeta float32) and be within max|x - ref| / max|ref| <= 2e-3 (fp16; 1e-2 for
dbeta) or 2e-4 (fp32) of the float64 oracle; repeated runs must be bit-identical.
"""
import sys

import pytest
import torch

from oracle import fpa_oracle as O

pytestmark = pytest.mark.gpu

NAMES = ("o", "dq", "dk", "dv", "dphi", "dpsi", "dbeta")
TOL = {torch.float16: 2e-3, torch.float32: 2e-4}
TOL_DBETA_FP16 = 1e-2


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


def run_hip(fpa, q, k, v, phi, psi, beta, do, tau=1.0):
    dev = "cuda"
    a = [t.to(dev).clone().requires_grad_() for t in (q, k, v, phi, psi, beta)]
    o = fpa.first_passage_attention(*a, tau=tau, impl="hip")
    grads = torch.autograd.grad(o, a, do.to(dev))
    torch.cuda.synchronize()
    return [o.detach().cpu()] + [g.detach().cpu() for g in grads]


def check(kern, ref, dtype, names=NAMES):
    for name, x, r in zip(names, kern, ref):
        want_dtype = dtype if name in ("o", "dq", "dk", "dv") else torch.float32
        assert x.dtype == want_dtype, (name, x.dtype)
        assert torch.isfinite(x).all(), name
        tol = TOL_DBETA_FP16 if (name == "dbeta" and dtype == torch.float16) else TOL[dtype]
        # An exactly-zero reference (e.g. dq, dk, dphi of a single row) is checked absolutely.
        err = O.rel_err(x, r) if r.abs().max() > 0 else x.double().abs().max().item()
        assert err <= tol, (name, err)


# (B, H, T, D, phi_scale, ties, dtype, seed, tau): the reference's CASES (test.py:134-147)
# plus head dimensions 16..128 in both dtypes, ragged and tiny T, and tau != 1.
CASES = [
    (1, 2, 64, 64, 1.0, False, torch.float16, 100, 1.0),
    (2, 3, 100, 64, 1.0, False, torch.float16, 101, 1.0),
    (1, 2, 128, 64, 1.0, False, torch.float16, 102, 1.0),
    (1, 2, 96, 64, 40.0, False, torch.float16, 103, 1.0),
    (1, 2, 96, 64, 1.0, True, torch.float16, 104, 1.0),
    (1, 2, 80, 32, 1.0, False, torch.float16, 110, 1.0),
    (1, 2, 100, 64, 1.0, False, torch.float32, 111, 1.0),
    (1, 2, 96, 16, 40.0, False, torch.float32, 112, 1.0),
    (2, 4, 512, 64, 1.0, False, torch.float16, 105, 1.0),
    (1, 2, 2048, 64, 1.0, False, torch.float16, 106, 1.0),
    (1, 2, 2048, 64, 1.0, False, torch.float32, 200, 1.0),
    (1, 2, 1000, 64, 40.0, False, torch.float32, 201, 1.0),
    (1, 2, 300, 128, 1.0, False, torch.float16, 300, 1.0),
    (1, 2, 300, 128, 1.0, False, torch.float32, 301, 1.0),
    (1, 3, 257, 16, 1.0, False, torch.float16, 302, 1.0),
    (1, 1, 3, 32, 1.0, False, torch.float16, 303, 1.0),
    (1, 2, 7, 32, 1.0, False, torch.float32, 304, 1.0),
    (2, 2, 65, 64, 3.0, True, torch.float16, 305, 0.7),
    (1, 2, 700, 32, 1.0, False, torch.float16, 306, 2.0),
    # edge shapes: a single row; exactly one block; B*H = 15 (no XCD pinning) and 16 (pinned)
    (1, 1, 1, 32, 1.0, False, torch.float16, 307, 1.0),
    (1, 2, 64, 128, 1.0, False, torch.float32, 308, 1.0),
    (3, 5, 130, 64, 1.0, False, torch.float16, 309, 1.0),
    (2, 8, 200, 32, 3.0, True, torch.float32, 310, 1.0),
]


@pytest.mark.parametrize("B,H,T,D,scale,ties,dtype,seed,tau", CASES)
def test_kernel_matches_the_oracle(fpa, B, H, T, D, scale, ties, dtype, seed, tau):
    _say(f"[parity] B={B} H={H} T={T} D={D} scale={scale} ties={ties} {dtype} seed={seed} tau={tau}")
    q, k, v, phi, psi, beta, do = O.make_inputs(B, H, T, D, dtype=dtype, seed=seed, phi_scale=scale, ties=ties)
    kern = run_hip(fpa, q, k, v, phi, psi, beta, do, tau)
    ref = O.fpa_grads(q, k, v, phi, psi, beta, do, tau=tau)
    check(kern, ref, dtype)


def test_kernel_temperature(fpa):
    """After test.py:162-167: tau = 0.25, fp32."""
    _say("[parity] temperature tau=0.25")
    q, k, v, phi, psi, beta, do = O.make_inputs(1, 2, 72, 32, dtype=torch.float32, seed=11)
    check(run_hip(fpa, q, k, v, phi, psi, beta, do, 0.25), O.fpa_grads(q, k, v, phi, psi, beta, do, tau=0.25),
          torch.float32)


def test_kernel_deterministic(fpa):
    """After test.py:170-174: two runs are bit-identical (no unordered atomics)."""
    _say("[determinism] B=2 H=2 T=96 D=32 fp16, and B=1 H=2 T=600 D=64 fp16")
    for shape, seed in (((2, 2, 96, 32), 12), ((1, 2, 600, 64), 13)):
        inp = O.make_inputs(*shape, seed=seed)
        runs = [run_hip(fpa, *inp) for _ in range(2)]
        assert all(torch.equal(x, y) for x, y in zip(*runs))


def _unsplit_ws_bytes(B, H, T):
    """Backward workspace bytes of a shape whose fused launch splits no tile."""
    a64 = lambda n: (n + 63) // 64 * 64  # noqa: E731
    BH, TP = B * H, (T + 63) // 64 * 64
    NB, NK32 = TP // 64, (T + 31) // 32
    return 4 * (a64(8 * BH * TP) + 2 * a64(BH * TP) + a64(BH * NB * 4096) + a64(BH * NB * NB) + a64(2 * BH * NK32))


def _bwd_runs(q, k, v, phi, psi, beta, do, phase_sets):
    """dq, dk, dv, dphi, dpsi, dbeta of the HIP backward run once per set of fpa_bwd phases."""
    from fpa import _hip
    dev = torch.device("cuda")
    fb = _hip.FwdBuffers(q)
    _hip.run_fwd(_hip.fwd_args(q, k, v, phi, psi, beta, 1.0, fb), dev)
    gb = _hip.BwdBuffers(q)
    ba = _hip.bwd_args(q, k, v, beta, 1.0, fb, do, gb)
    outs = []
    for phases in phase_sets:
        for ph in phases:
            ba.phases = ph
            _hip.run_bwd(ba, dev)
        torch.cuda.synchronize()
        outs.append([t.clone() for t in (gb.dq, gb.dk, gb.dv, gb.dphi, gb.dpsi, gb.dbeta)])
    return outs


def test_fused_backward_matches_separate_launches(fpa):
    """The backward's key and query sides run as one launch; launched one by one through the
    phases bitmask they give bit-identical gradients (head counts with and without the per-XCD
    head placement, a ragged T, and fp32 D128; shapes whose fused launch does not split tiles)."""
    from fpa import _hip, _lib
    dev = torch.device("cuda")
    for (B, H, T, D, dtype), seed in (((2, 4, 300, 64, torch.float16), 14), ((1, 3, 333, 64, torch.float16), 15),
                                      ((1, 2, 260, 128, torch.float32), 16), ((1, 2, 200, 64, torch.float32), 17)):
        _say(f"[fused] B{B} H{H} T{T} D{D} {dtype}")
        q, k, v, phi, psi, beta, do = (t.to(dev) for t in O.make_inputs(B, H, T, D, dtype=dtype, seed=seed))
        assert _hip._bwd_ws_bytes(B, H, T, D, _lib.dtype_code(dtype)) == _unsplit_ws_bytes(B, H, T)
        outs = _bwd_runs(q, k, v, phi, psi, beta, do, ((0,), (_lib.FPA_BWD_DELTA, _lib.FPA_BWD_KEYS,
                                                                _lib.FPA_BWD_QUERIES, _lib.FPA_BWD_PHI | _lib.FPA_BWD_BETA)))
        assert all(torch.equal(x, y) for x, y in zip(*outs))


BWD_SPLIT_CASES = [  # (B, H, T, D, dtype, beta, seed): shapes whose fused backward splits its heaviest tiles
    (2, 4, 600, 64, torch.float16, None, 51),                  # B*H = 8: heads pinned to XCDs
    (1, 3, 1000, 32, torch.float16, (-0.7, 0.0, 1.3), 52),
    (1, 2, 777, 32, torch.float32, None, 53),
    (1, 1, 4100, 128, torch.float16, None, 54),
    (1, 1, 513, 16, torch.float16, None, 55),
    (1, 4, 4096, 64, torch.float16, None, 56),
]


@pytest.mark.parametrize("B,H,T,D,dtype,beta,seed", BWD_SPLIT_CASES)
def test_split_backward(fpa, B, H, T, D, dtype, beta, seed):
    """When the fused backward fills at most all of the slots, the heaviest half of its key tiles and of
    its query tiles run as two items each over halves of their block range, and a merge kernel adds the
    partial sums before the combine.  Launched one side at a time (phases), the backward runs every tile
    whole: the gradients agree to rounding.  Through the split path the gradients agree with the oracle
    (for fp16 the oracle fed the kernel's own stored output, as in test_split_forward)."""
    from fpa import _hip, _lib
    _say(f"[bwd split] B{B} H{H} T{T} D{D} {dtype}")
    q, k, v, phi, psi, b0, do = O.make_inputs(B, H, T, D, dtype=dtype, seed=seed, psi_noise=1.0)
    beta = torch.tensor(beta) if beta is not None else b0
    dev = torch.device("cuda")
    assert _hip._bwd_ws_bytes(B, H, T, D, _lib.dtype_code(dtype)) > _unsplit_ws_bytes(B, H, T)
    qd, kd, vd, pd, sd, bd, dod = (t.to(dev) for t in (q, k, v, phi, psi, beta, do))
    split, whole = _bwd_runs(qd, kd, vd, pd, sd, bd, dod, ((0,), (_lib.FPA_BWD_DELTA, _lib.FPA_BWD_KEYS,
                                                                 _lib.FPA_BWD_QUERIES, _lib.FPA_BWD_PHI)))
    tol = 1e-3 if dtype == torch.float16 else 1e-5
    for name, x, y in zip(NAMES[1:], split, whole):
        assert O.rel_err(x.cpu(), y.cpu()) <= (1e-2 if name == "dbeta" and dtype == torch.float16 else tol), name
    kern = run_hip(fpa, q, k, v, phi, psi, beta, do)
    ref = O.fpa_grads_chunked(q, k, v, phi, psi, beta, do, device="cuda")
    if dtype == torch.float16:
        ref = ref[:1] + list(O.fpa_grads_stored(q, k, v, phi, psi, beta, do, o_stored=kern[0])[1:])
    check(kern, ref, dtype)


SPLIT_CASES = [  # (B, H, T, D, dtype, beta, seed): shapes whose forward splits its heaviest row tiles
    (1, 3, 1000, 32, torch.float16, (-0.7, 0.0, 1.3), 41),
    (3, 5, 777, 16, torch.float32, None, 42),
    (1, 1, 4100, 128, torch.float16, None, 43),
    (2, 1, 600, 256, torch.float32, None, 44),
    (1, 2, 700, 64, torch.float16, None, 45),
    (1, 1, 513, 16, torch.float16, None, 46),      # fp16 D16: two 16-byte chunks per row in the merge
    (2, 4, 1000, 64, torch.float16, None, 47),     # B*H = 8: heads pinned to XCDs, items per XCD
    (1, 2, 1100, 128, torch.float32, None, 48),    # fp32 D128: K, V single-buffered (two workgroups per CU)
]


@pytest.mark.parametrize("B,H,T,D,dtype,beta,seed", SPLIT_CASES)
def test_split_forward(fpa, B, H, T, D, dtype, beta, seed):
    """When the launch is short of workgroups the forward runs the heaviest row tiles as two halves of
    their key range and a merge kernel combines them.  Without a workspace every row tile runs
    whole: o agrees to rounding (each half rounds its P and its normalised o on its own) and so does
    the row's lse (m + log2 l).  Through the split path o agrees with the float64 oracle and, for
    fp16, the gradients with the oracle fed the kernel's own stored output (Delta from the fp16 o, as
    the reference's _bwd_delta takes it, kernel.py:165-174): on the first case that rounding alone
    moves the exact dbeta by 1.7e-2, with or without the split."""
    from fpa import _hip, _lib
    _say(f"[split] B{B} H{H} T{T} D{D} {dtype}")
    dev = torch.device("cuda")
    q, k, v, phi, psi, b0, do = O.make_inputs(B, H, T, D, dtype=dtype, seed=seed, psi_noise=1.0)
    beta = torch.tensor(beta) if beta is not None else b0
    assert _hip._fwd_ws_bytes(B, H, T, D, _lib.dtype_code(dtype)) > 0
    qd, kd, vd, pd, sd, bd = (t.to(dev) for t in (q, k, v, phi, psi, beta))
    outs = []
    for split in (True, False):
        fb = _hip.FwdBuffers(qd)
        fa = _hip.fwd_args(qd, kd, vd, pd, sd, bd, 1.0, fb)
        assert bool(fa.workspace) and fb.ws is not None
        if not split:
            fa.workspace = None
        _hip.run_fwd(fa, dev)
        torch.cuda.synchronize()
        TP = fb.lse.numel() // (2 * B * H)
        lse = fb.lse.view(2, B * H, TP)[:, :, :T]
        outs.append((fb.o.clone(), lse[0] + lse[1] if dtype == torch.float32 else lse[0].clone()))
    (o_s, l_s), (o_w, l_w) = outs
    assert O.rel_err(o_s.cpu(), o_w.cpu()) <= (1e-3 if dtype == torch.float16 else 1e-6)
    assert (l_s - l_w).abs().max().item() <= (1e-3 if dtype == torch.float16 else 1e-5 * (1 + l_w.abs().max().item()))
    kern = run_hip(fpa, q, k, v, phi, psi, beta, do)
    ref = O.fpa_grads_chunked(q, k, v, phi, psi, beta, do, device="cuda")
    if dtype == torch.float16:
        ref = ref[:1] + list(O.fpa_grads_stored(q, k, v, phi, psi, beta, do, o_stored=kern[0])[1:])
    check(kern, ref, dtype)


def test_negative_and_zero_beta(fpa):
    """beta <= 0 flips / removes the bias; the kernels take the sign per head."""
    _say("[parity] beta = (-0.7, 0, 1.3)")
    q, k, v, phi, psi, _, do = O.make_inputs(1, 3, 150, 32, dtype=torch.float32, seed=31)
    beta = torch.tensor([-0.7, 0.0, 1.3])
    check(run_hip(fpa, q, k, v, phi, psi, beta, do), O.fpa_grads(q, k, v, phi, psi, beta, do), torch.float32)


@pytest.mark.parametrize("drift", [0.0, 0.01])
def test_signed_beta_many_blocks(fpa, drift):
    """beta (-0.7, 0, 1.3) over 16 blocks in fp16: the per-key classes of both backward sides (per-key
    bias, per-key soft-min denominators, open gate) are voted per block and must hold for either sign
    of beta and for beta = 0."""
    _say(f"[parity] beta = (-0.7, 0, 1.3), T=1000 D64 fp16, drift {drift}")
    q, k, v, phi, psi, _, do = O.make_inputs(1, 3, 1000, 64, dtype=torch.float16, seed=33, drift=drift)
    beta = torch.tensor([-0.7, 0.0, 1.3])
    check(run_hip(fpa, q, k, v, phi, psi, beta, do), O.fpa_grads(q, k, v, phi, psi, beta, do), torch.float16)


def test_fp32_large_logits(fpa):
    """fp32 with beta < 0 over a long phi walk: the bias is positive and the logits reach several hundred
    (base 2).  The backward forms P from the forward's running maximum and log2 sum, so its P is the
    forward's to a few ulps: dv (P^T dO) is held to 1e-5, every other gradient to the fp32 bound.
    dbeta, a sum of dS x over rows of dS that sum to zero, is also held to the oracle fed the kernel's
    own stored output (``fpa_grads_stored``: Delta taken from that output, everything else exact), the
    quantity the reference's backward computes (kernel.py:165-174); measured 9e-6 against the exact
    oracle and 4e-5 against the stored-output one."""
    _say("[parity] fp32 beta < 0, T=1531 D64, phi scale 4")
    q, k, v, phi, psi, _, do = O.make_inputs(1, 2, 1531, 64, dtype=torch.float32, seed=2005, phi_scale=4.0,
                                             psi_noise=0.1)
    beta = torch.tensor([-0.9, -1.3])
    kern = run_hip(fpa, q, k, v, phi, psi, beta, do, tau=0.5)
    ref = O.fpa_grads(q, k, v, phi, psi, beta, do, tau=0.5)
    check(kern, ref, torch.float32)
    assert O.rel_err(kern[3], ref[3]) <= 1e-5, ("dv", O.rel_err(kern[3], ref[3]))
    stored = O.fpa_grads_stored(q, k, v, phi, psi, beta, do, tau=0.5, store=torch.float32, o_stored=kern[0])
    err = O.rel_err(kern[6], stored[6])
    _say(f"[parity] fp32 large logits: dbeta vs stored-output oracle {err:.2e}, vs exact {O.rel_err(kern[6], ref[6]):.2e}")
    assert err <= TOL[torch.float32], ("dbeta", err)


def test_scalar_beta_and_strided_views(fpa):
    """beta given as a Python float; q, k, v as permuted views of one (B, T, 3, H, D) tensor."""
    _say("[parity] scalar beta, permuted q/k/v views")
    B, H, T, D = 2, 3, 130, 32
    g = torch.Generator().manual_seed(41)
    qkv = torch.randn(B, T, 3, H, D, generator=g).half()
    q, k, v = qkv.permute(2, 0, 3, 1, 4)
    _, _, _, phi, psi, _, do = O.make_inputs(B, H, T, D, seed=42)
    dev = "cuda"
    qkv_d = qkv.to(dev).requires_grad_()
    qd, kd, vd = qkv_d.permute(2, 0, 3, 1, 4)
    pd, sd = phi.to(dev).requires_grad_(), psi.to(dev).requires_grad_()
    o = fpa.first_passage_attention(qd, kd, vd, pd, sd, 0.8, impl="hip")
    dqkv, dphi, dpsi = torch.autograd.grad(o, [qkv_d, pd, sd], do.to(dev))
    ref = O.fpa_grads(q, k, v, phi, psi, torch.tensor(0.8), do)
    dq, dk, dv = dqkv.cpu().permute(2, 0, 3, 1, 4)
    got = [o.detach().cpu(), dq, dk, dv, dphi.cpu(), dpsi.cpu()]
    for name, x, r in zip(NAMES, got, ref):
        assert torch.isfinite(x).all(), name
        assert O.rel_err(x, r) <= TOL[torch.float16], (name, O.rel_err(x, r))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_bench_shape_heads(fpa, dtype):
    """The north-star shape B4 H12 T2048 D64 runs whole on the GPU; two of its 48 heads are
    checked against the oracle (FPA is independent per head)."""
    _say(f"[parity] B4 H12 T2048 D64 {dtype}, heads (0,0) and (3,11)")
    B, H, T, D = 4, 12, 2048, 64
    q, k, v, phi, psi, _, do = O.make_inputs(B, H, T, D, dtype=dtype, seed=0, psi_noise=1.0)
    beta = torch.ones(H)
    kern = run_hip(fpa, q, k, v, phi, psi, beta, do)
    for b, h in ((0, 0), (3, 11)):
        sl = lambda t: t[b:b + 1, h:h + 1]  # noqa: E731
        ref = O.fpa_grads(sl(q), sl(k), sl(v), sl(phi), sl(psi), beta[h:h + 1], sl(do))
        got = [sl(x) for x in kern[:6]]
        for name, x, r in zip(NAMES[:6], got, ref[:6]):
            assert torch.isfinite(x).all(), name
            assert O.rel_err(x, r) <= TOL[dtype], (name, b, h, O.rel_err(x, r))
    assert torch.isfinite(kern[6]).all()


def test_layer_kernel_matches_the_reference(fpa):
    """After test.py:200-214: the FirstPassageAttention layer, hip vs the dense path, fp32."""
    _say("[layer] fp32 hip vs reference")
    out = []
    for impl in ("hip", "reference"):
        torch.manual_seed(0)
        layer = fpa.FirstPassageAttention(64, 4, impl=impl).cuda()
        x = torch.randn(2, 50, 64, generator=torch.Generator().manual_seed(1)).cuda()
        y = layer(x)
        loss = y.float().square().mean()
        out.append([y.detach().float()] + list(torch.autograd.grad(loss, list(layer.parameters()))))
    for a, b in zip(*out):
        assert ((a - b).norm() / b.norm()).item() <= 1e-4


def test_layer_kernel_fp16_autocast(fpa):
    """After test.py:200-214 with amp: fp16 autocast, relative norm <= 5e-3."""
    _say("[layer] fp16 autocast hip vs fp32 reference")
    out = []
    for impl, amp in (("hip", True), ("reference", True)):
        torch.manual_seed(0)
        layer = fpa.FirstPassageAttention(64, 4, impl=impl).cuda()
        x = torch.randn(2, 50, 64, generator=torch.Generator().manual_seed(1)).cuda()
        with torch.autocast("cuda", dtype=torch.float16, enabled=amp):
            y = layer(x)
        loss = y.float().square().mean()
        out.append([y.detach().float()] + list(torch.autograd.grad(loss, list(layer.parameters()))))
    for a, b in zip(*out):
        assert ((a - b).norm() / b.norm()).item() <= 5e-3


def test_steep_drift_and_small_tau(fpa):
    """phi with a steep downward drift and a small tau: block log-sum-exp spreads above 100
    binades (the exact form of the key side's soft-min denominators) and query blocks far above
    the key blocks' references (the clamped product form); fp32 for the tight tolerance."""
    _say("[parity] B1 H2 T1500 D64 fp32 drift 0.2, tau 0.1 and 1.0")
    for tau in (0.1, 1.0):
        q, k, v, phi, psi, beta, do = O.make_inputs(1, 2, 1500, 64, dtype=torch.float32, seed=51, drift=0.2)
        check(run_hip(fpa, q, k, v, phi, psi, beta, do, tau), O.fpa_grads(q, k, v, phi, psi, beta, do, tau=tau),
              torch.float32)


def test_cfg3_shape_head(fpa):
    """The fp32 wide-head shape B2 H8 T4096 D128 (beta = softplus) runs whole; one head is
    checked against the oracle at the fp32 tolerance."""
    _say("[parity] B2 H8 T4096 D128 fp32, head (1,5)")
    B, H, T, D = 2, 8, 4096, 128
    q, k, v, phi, psi, beta, do = O.make_inputs(B, H, T, D, dtype=torch.float32, seed=3, psi_noise=1.0,
                                                beta="softplus")
    kern = run_hip(fpa, q, k, v, phi, psi, beta, do)
    for x in kern:
        assert torch.isfinite(x).all()
    b, h = 1, 5
    sl = lambda t: t[b:b + 1, h:h + 1]  # noqa: E731
    ref = O.fpa_grads(sl(q), sl(k), sl(v), sl(phi), sl(psi), beta[h:h + 1], sl(do))
    for name, x, r in zip(NAMES[:6], [sl(x) for x in kern[:6]], ref[:6]):
        assert O.rel_err(x, r) <= TOL[torch.float32], (name, O.rel_err(x, r))


def test_cfg4_shape_prefix(fpa):
    """The long ragged shape B1 H12 T16381 D64 fp16 with phi drift -0.01 t runs whole, twice
    with bit-identical results.  Rows t < 2048 depend only on keys s <= t, so o and dq of those
    rows are checked against the oracle run on the 2048-long prefix of one head."""
    _say("[parity] B1 H12 T16381 D64 fp16 drift 0.01, prefix of head 7")
    B, H, T, D = 1, 12, 16381, 64
    q, k, v, phi, psi, _, do = O.make_inputs(B, H, T, D, dtype=torch.float16, seed=4, psi_noise=1.0, drift=0.01)
    beta = torch.ones(H)
    runs = [run_hip(fpa, q, k, v, phi, psi, beta, do) for _ in range(2)]
    assert all(torch.equal(x, y) for x, y in zip(*runs))
    for x in runs[0]:
        assert torch.isfinite(x).all()
    h, P = 7, 2048
    sl = lambda t: t[:, h:h + 1, :P]  # noqa: E731
    ref = O.fpa_grads(sl(q), sl(k), sl(v), sl(phi), sl(psi), beta[h:h + 1], sl(do))
    for name, idx in (("o", 0), ("dq", 1)):
        assert O.rel_err(sl(runs[0][idx]), ref[idx]) <= TOL[torch.float16], (name, O.rel_err(sl(runs[0][idx]), ref[idx]))


def test_large_scores(fpa):
    """q and k scaled by 60 in fp16: row maxima of q.k reach 1.4e5, far outside the usual range,
    which stresses how -lse and -Delta enter the score accumulators.  o is held to the exact oracle
    and every gradient to the oracle fed the kernel's own stored output (Delta taken from the fp16
    output, as the reference's _bwd_delta does, kernel.py:165-174; against the exact gradients that
    rounding alone moves dphi by 1.7e-2), at the fp16 bounds, except dphi.  The fp32 score
    accumulators hold values near 1.4e5 (an ulp of 0.008), so each logit carries a rounding of a few
    1e-3 (base 2) and P of a few 1e-3 relative, in any fp32 evaluation of these scores (the
    reference's `tl.dot` accumulates in fp32 too); dphi, a soft-min-weighted sum of gated dS over
    pairs whose rows cancel, takes that as 3.7e-3 and is held to 1e-2."""
    _say("[parity] B1 H2 T256 D64 fp16, q and k x60")
    q, k, v, phi, psi, beta, do = O.make_inputs(1, 2, 256, 64, dtype=torch.float16, seed=61)
    q, k = (q.float() * 60).half(), (k.float() * 60).half()
    kern = run_hip(fpa, q, k, v, phi, psi, beta, do)
    exact = O.fpa_grads(q, k, v, phi, psi, beta, do)
    stored = O.fpa_grads_stored(q, k, v, phi, psi, beta, do, o_stored=kern[0])
    ref = [exact[0]] + stored[1:]
    errs = {name: O.rel_err(x, r) for name, x, r in zip(NAMES, kern, ref)}
    _say("[parity] large-score errors (stored-output oracle) " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()))
    check([x for n, x in zip(NAMES, kern) if n != "dphi"], [r for n, r in zip(NAMES, ref) if n != "dphi"],
          torch.float16, names=[n for n in NAMES if n != "dphi"])
    assert torch.isfinite(kern[4]).all() and errs["dphi"] <= 1e-2, ("dphi", errs["dphi"])


@pytest.mark.parametrize("T", [300, 700])
def test_graph_replay_matches_eager(fpa, T):
    """The forward and backward captured in one HIP graph: three replays, with eager work and
    synchronisations between them, each give outputs bit-identical to the eager call (the
    library records no memset nodes).  At T = 700 the forward splits its heaviest row tiles and
    runs its merge kernel on a workspace taken from the graph's pool."""
    _say(f"[graph] B1 H2 T{T} D64 fp16, capture and three replays")
    q, k, v, phi, psi, beta, do = O.make_inputs(1, 2, T, 64, dtype=torch.float16, seed=71)
    dev = "cuda"
    leaves = [t.to(dev).clone().requires_grad_() for t in (q, k, v, phi, psi, beta)]
    dod = do.to(dev)

    def step():
        o = fpa.first_passage_attention(*leaves, impl="hip")
        return [o] + list(torch.autograd.grad(o, leaves, dod))

    eager = [t.detach().clone() for t in step()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = step()
    for r in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(x, y) for x, y in zip(static, eager)), r
        step()  # eager work between replays
        torch.cuda.synchronize()


def test_block_is_a_no_op(fpa):
    """block (the reference's kernel block, test.py:134-147 varies it over 16/32/64) does not change
    the HIP kernels' results: block = 16, 32, 64 and 128 give bit-identical outputs and gradients."""
    _say("[parity] block 16/32/64/128 bit-identical, B1 H2 T200 D32 fp16")
    q, k, v, phi, psi, beta, do = O.make_inputs(1, 2, 200, 32, dtype=torch.float16, seed=81)
    runs = []
    for block in (16, 32, 64, 128):
        a = [t.cuda().clone().requires_grad_() for t in (q, k, v, phi, psi, beta)]
        o = fpa.first_passage_attention(*a, impl="hip", block=block)
        runs.append([o.detach()] + list(torch.autograd.grad(o, a, do.cuda())))
    for other in runs[1:]:
        assert all(torch.equal(x, y) for x, y in zip(runs[0], other))


def test_tensors_on_another_device_are_refused(fpa):
    """beta (or k, phi, ...) on the CPU with q on the GPU raises ValueError before any launch, as the
    reference's Triton launch refuses a host tensor."""
    _say("[api] CPU beta / CPU phi with GPU q")
    q, k, v, phi, psi, beta, _ = O.make_inputs(1, 2, 64, 32, dtype=torch.float16, seed=82)
    qd, kd, vd, phid, psid = (t.cuda() for t in (q, k, v, phi, psi))
    with pytest.raises(ValueError, match="beta is on cpu"):
        fpa.first_passage_attention(qd, kd, vd, phid, psid, beta, impl="hip")
    with pytest.raises(ValueError, match="phi is on cpu"):
        fpa.first_passage_attention(qd, kd, vd, phi, psid, beta.cuda(), impl="hip")
    with pytest.raises(ValueError, match="k is on cpu"):
        fpa.first_passage_attention(qd, k, vd, phid, psid, beta.cuda(), impl="hip")
    torch.cuda.synchronize()


def test_layer_with_more_heads_than_the_field_kernels(fpa):
    """FirstPassageAttention(2048, 64, impl="hip"): 64 heads of D = 32.  The attention runs on the HIP
    kernels and the Field prologue (HIP kernels up to 32 heads) on PyTorch; output and parameter
    gradients match the dense layer in fp32."""
    _say("[layer] 64 heads (d_model 2048, D 32), fp32 hip vs reference")
    out = []
    for impl in ("hip", "reference"):
        torch.manual_seed(0)
        layer = fpa.FirstPassageAttention(2048, 64, impl=impl).cuda()
        x = torch.randn(1, 40, 2048, generator=torch.Generator().manual_seed(1)).cuda()
        y = layer(x)
        loss = y.float().square().mean()
        out.append([y.detach().float()] + list(torch.autograd.grad(loss, list(layer.parameters()))))
    for a, b in zip(*out):
        assert ((a - b).norm() / b.norm()).item() <= 1e-4
