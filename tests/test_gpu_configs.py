"""Whole-tensor parity of the HIP kernels at every BASELINE.json attention configuration.

Every element of all seven outputs (o, dq, dk, dv, dphi, dpsi, dbeta) over every head is compared
with the float64 oracle, as the reference's kernel tests compare every element
(test.py:150-159).  At these sizes the oracle is ``fpa_grads_chunked`` (query rows in chunks,
pinned to the dense oracle on the CPU by tests/test_oracle.py) run in float64 on the GPU; the
first test checks that its GPU run agrees with its CPU run.  Bounds (max |x - ref| / max |ref|,
reference test.py:18-20): 2e-3 fp16 (1e-2 for dbeta), 2e-4 fp32.
"""
import sys

import pytest
import torch

from baseline_configs import CONFIGS, make_config
from oracle import fpa_oracle as O

pytestmark = pytest.mark.gpu

NAMES = ("o", "dq", "dk", "dv", "dphi", "dpsi", "dbeta")
TOL = {torch.float16: 2e-3, torch.float32: 2e-4}


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def fpa():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    import fpa as m
    from fpa import _lib
    _lib.lib()
    return m


def run_hip(fpa, q, k, v, phi, psi, beta, do, tau=1.0):
    a = [t.cuda().clone().requires_grad_() for t in (q, k, v, phi, psi, beta)]
    o = fpa.first_passage_attention(*a, tau=tau, impl="hip")
    grads = torch.autograd.grad(o, a, do.cuda())
    torch.cuda.synchronize()
    return [o.detach()] + [g.detach() for g in grads]


def compare(name, kern, ref, dtype):
    errs = {}
    for n, x, r in zip(NAMES, kern, ref):
        want = dtype if n in ("o", "dq", "dk", "dv") else torch.float32
        assert x.dtype == want, (n, x.dtype)
        assert x.shape == r.shape, (n, x.shape, r.shape)
        assert torch.isfinite(x).all(), n
        errs[n] = O.rel_err(x.cpu(), r)
    _say(f"[{name}] " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()))
    for n, e in errs.items():
        tol = 1e-2 if (n == "dbeta" and dtype == torch.float16) else TOL[dtype]
        assert e <= tol, (name, n, e)


def test_chunked_oracle_on_the_gpu_is_the_cpu_oracle():
    """The float64 oracle gives the same numbers on the GPU as on the CPU (chunks of 50 rows)."""
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    _say("[oracle] chunked float64 oracle, GPU against CPU, B2 H2 T300 D32")
    q, k, v, phi, psi, beta, do = O.make_inputs(2, 2, 300, 32, dtype=torch.float32, seed=90, drift=0.05)
    cpu = O.fpa_grads(q, k, v, phi, psi, beta, do)
    gpu = O.fpa_grads_chunked(q, k, v, phi, psi, beta, do, device="cuda", max_elems=300 * 50)
    for n, x, r in zip(NAMES, gpu, cpu):
        assert O.rel_err(x, r) <= 1e-12, (n, O.rel_err(x, r))


def test_cfg1_exact(fpa):
    """BASELINE config 1 at its exact specification: B1 H2 T256 D32 fp32, beta = 1, loss o.sum(),
    seed 0 (the reference's CPU-runnable case, here on the HIP kernels)."""
    _say("[cfg1] B1 H2 T256 D32 fp32, dO = 1, seed 0")
    inp = make_config("cfg1")
    compare("cfg1", run_hip(fpa, *inp), O.fpa_grads(*inp), torch.float32)


@pytest.mark.parametrize("random_do", [False, True], ids=["loss_sum", "random_do"])
def test_cfg2_all_heads(fpa, random_do):
    """BASELINE config 2 (the bench shape), all 48 heads: with the config's loss o.float().sum()
    (dO = 1) and with a random dO."""
    _say(f"[cfg2] B4 H12 T2048 D64 fp16, all heads, random_do={random_do}")
    inp = make_config("cfg2", random_do=random_do)
    kern = run_hip(fpa, *inp)
    ref = O.fpa_grads_chunked(*inp, device="cuda")
    compare("cfg2", kern, ref, torch.float16)


def test_cfg3_all_heads(fpa):
    """B2 H8 T4096 D128 fp32, beta = softplus(N(0, 1)), all 16 heads."""
    _say("[cfg3] B2 H8 T4096 D128 fp32, all heads")
    inp = make_config("cfg3")
    kern = run_hip(fpa, *inp)
    ref = O.fpa_grads_chunked(*inp, device="cuda")
    compare("cfg3", kern, ref, torch.float32)


def test_cfg4_full_length(fpa):
    """B1 H12 T16381 D64 fp16 with phi drift -0.01 t (range minima from deep
    prefixes, 256 blocks per head, a ragged last block), the whole length of all 12 heads; a second
    run is bit-identical."""
    _say("[cfg4] B1 H12 T16381 D64 fp16 drift 0.01, all heads, full length")
    inp = make_config("cfg4")
    kern = run_hip(fpa, *inp)
    again = run_hip(fpa, *inp)
    assert all(torch.equal(x, y) for x, y in zip(kern, again))
    del again
    ref = O.fpa_grads_chunked(*inp, device="cuda")
    compare("cfg4", kern, ref, torch.float16)


@pytest.mark.parametrize("T", [159 * 64 + 1, 160 * 64 - 5, 192 * 64 + 33])
def test_middle_block_sums_both_ways(fpa, T):
    """The middle-block soft-min sums of dphi are taken over every (query block, key block) pair
    around each block up to 159 blocks per head, and from per-row prefix sums of the middle-block
    table (a separate pass over each row) from 160 blocks on: both sides of the switch and one
    length well past it, each with a ragged last block, drift (range minima from deep prefixes) and
    beta of either sign, in fp32 against the float64 oracle."""
    _say(f"[mid] B1 H3 T{T} D16 fp32, beta (0.8, -0.6, 1.4), drift 0.01")
    q, k, v, phi, psi, _, do = O.make_inputs(1, 3, T, 16, dtype=torch.float32, seed=T, drift=0.01)
    beta = torch.tensor([0.8, -0.6, 1.4])
    kern = run_hip(fpa, q, k, v, phi, psi, beta, do)
    ref = O.fpa_grads_chunked(q, k, v, phi, psi, beta, do, device="cuda")
    compare(f"mid T{T}", kern, ref, torch.float32)
