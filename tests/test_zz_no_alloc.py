"""fpa_bwd_noalloc: the backward on the library's static scratch gives fpa_bwd's results.

Three calls in a row through the C ABI, each with a smaller problem than the one before (the scratch
keeps the previous call's contents; the first call's fused launch splits its heaviest tiles and adds
their halves through the scratch), each compared bit for bit with fpa_bwd on a torch-allocated
workspace; a problem whose scratch need exceeds the static array is refused before any launch.
"""
import sys

import pytest
import torch

from oracle import fpa_oracle as O

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _both(B, H, T, D, dtype, seed):
    from fpa import _hip, _lib
    dev = torch.device("cuda")
    q, k, v, phi, psi, beta, do = (t.to(dev) for t in O.make_inputs(B, H, T, D, dtype=dtype, seed=seed))
    fb = _hip.FwdBuffers(q)
    _hip.run_fwd(_hip.fwd_args(q, k, v, phi, psi, beta, 1.0, fb), dev)
    outs = []
    for runner in (_hip.run_bwd, _hip.run_bwd_noalloc):
        gb = _hip.BwdBuffers(q)
        gb.dq.fill_(7.0)  # stale values must not survive
        ba = _hip.bwd_args(q, k, v, beta, 1.0, fb, do, gb)
        if runner is _hip.run_bwd_noalloc:
            ba.workspace = None  # unused by the no-allocation entry point
        runner(ba, dev)
        torch.cuda.synchronize()
        outs.append([t.clone() for t in (gb.dq, gb.dk, gb.dv, gb.dphi, gb.dpsi, gb.dbeta)])
    ref = O.fpa_grads(q, k, v, phi, psi, beta, do)
    return outs, ref


def test_noalloc_backward_matches_fpa_bwd():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    for (B, H, T, D, dtype), seed in (((1, 3, 1000, 32, torch.float16), 90), ((2, 3, 300, 64, torch.float16), 91),
                                      ((1, 2, 100, 32, torch.float32), 92)):
        _say(f"[noalloc] B{B} H{H} T{T} D{D} {dtype}")
        (with_ws, noalloc), ref = _both(B, H, T, D, dtype, seed)
        for name, x, y in zip(("dq", "dk", "dv", "dphi", "dpsi", "dbeta"), with_ws, noalloc):
            assert torch.equal(x, y), name
        tol = 2e-3 if dtype == torch.float16 else 2e-4
        for name, x, r in zip(("dq", "dk", "dv", "dphi", "dpsi"), noalloc, ref[1:6]):
            assert O.rel_err(x.cpu(), r) <= tol, (name, O.rel_err(x.cpu(), r))


def test_noalloc_refuses_a_problem_beyond_its_scratch():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from fpa import _hip, _lib
    _say("[noalloc] oversized problem refused")
    L = _lib.lib()
    B, H, T, D = 16, 16, 4096, 64
    assert L.fpa_bwd_workspace_bytes(B, H, T, D, _lib.FPA_F16) > _lib.NOALLOC_SCRATCH_BYTES
    a = _lib.FpaBwdArgs()
    a.B, a.H, a.T, a.D, a.dtype, a.tau = B, H, T, D, _lib.FPA_F16, 1.0
    with pytest.raises(_lib.FpaError, match="more than the"):
        _lib.check(L.fpa_bwd_noalloc(a, None))
