"""A seeded sweep of mixed shapes and inputs through the HIP kernels against the float64 oracle.

The fixed cases (test_gpu_parity.py) follow the reference's test matrix (test.py:134-147); this
sweep draws further combinations from one seeded generator: ragged lengths, every head
dimension up to 128, both dtypes, beta of either sign or zero per head, tau, the phi scale and
drift, and the psi noise, which together move the backward's per-block decisions (per-key bias
and soft-min classes, open gates, product or exact soft-min forms) around.  The bounds are the
reference's (test.py:18-20): max |x - ref| / max |ref| <= 2e-3 in fp16 (1e-2 for dbeta) and 2e-4
in fp32.

The draws stay in the reference's data model (psi = phi + noise of at most 0.5, phi scale up to 4):
dbeta is sum_ts dS_ts b_ts / beta, and every row of dS sums to zero, so its relative error grows
with sum |dS b| / |dbeta|.  With psi noise 2, phi scale 8 and tau 0.5 that ratio reaches 2.5e4 and a
float32 evaluation misses the bound as well (6e-3 against 2e-4), so such inputs test conditioning
rather than the kernels.

In fp16 the backward's Delta_t = sum_d dO_td O_td reads the output as stored, in fp16, as the
reference's _bwd_delta does (kernel.py:165-174); that rounding alone moves dphi by up to 3e-3 of
its largest value on some draws (it is not a kernel error: against a float64 reference that takes
the same rounded output, the kernels agree to 4e-5 there).  So fp16 gradients are checked against
``fpa_grads_stored``, the float64 gradients with Delta from the output rounded to fp16; o against
the exact forward.  dbeta sums dS_ts b_ts, whose rows cancel, so on some draws it moves by several
percent when the stored output is rounded (the exact and the stored references differ by that
much); an fp16 output one unit off in a few places moves it as far again, so fp16 dbeta is held
to the larger of the usual bound and twice that measured sensitivity.
"""
import random
import sys

import pytest
import torch

from oracle import fpa_oracle as O
from test_gpu_parity import NAMES, TOL, TOL_DBETA_FP16, check, run_hip

pytestmark = pytest.mark.gpu


def _cases(n=16, seed=2026):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        out.append(dict(
            B=rng.choice([1, 2]), H=rng.choice([1, 2, 3]),
            T=rng.choice([1, 37, 64, 129, 200, 333, 512, 701]),
            D=rng.choice([16, 32, 64, 128]),
            dtype=rng.choice(["f16", "f32"]),
            beta=rng.choice(["positive", "negative", "mixed", "zero"]),
            tau=rng.choice([0.5, 1.0, 2.0]),
            phi_scale=rng.choice([0.3, 1.0, 4.0]),
            drift=rng.choice([0.0, 0.02]),
            psi_noise=rng.choice([0.1, 0.25, 0.5]),
            seed=1000 + i))
    return out


CASES = _cases()


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


@pytest.mark.parametrize("case", CASES, ids=[f"c{i}" for i in range(len(CASES))])
def test_sweep_matches_the_oracle(fpa, case):
    c = case
    dtype = torch.float16 if c["dtype"] == "f16" else torch.float32
    _say(f"[sweep] {c}")
    q, k, v, phi, psi, _, do = O.make_inputs(c["B"], c["H"], c["T"], c["D"], dtype=dtype, seed=c["seed"],
                                             phi_scale=c["phi_scale"], psi_noise=c["psi_noise"], drift=c["drift"])
    g = torch.Generator().manual_seed(c["seed"])
    mag = torch.rand(c["H"], generator=g) + 0.5
    if c["beta"] == "positive":
        beta = mag
    elif c["beta"] == "negative":
        beta = -mag
    elif c["beta"] == "mixed":
        beta = mag * torch.tensor([(-1.0) ** h for h in range(c["H"])])
    else:
        beta = torch.zeros(c["H"])
    kern = run_hip(fpa, q, k, v, phi, psi, beta, do, tau=c["tau"])
    exact = O.fpa_grads(q, k, v, phi, psi, beta, do, tau=c["tau"])
    if dtype == torch.float32:
        check(kern, exact, dtype)
        return
    ref = O.fpa_grads_stored(q, k, v, phi, psi, beta, do, tau=c["tau"], store=torch.float16)
    check(kern[:6], ref[:6], dtype)
    db, db_ref, db_exact = kern[6], ref[6], exact[6]
    assert db.dtype == torch.float32 and torch.isfinite(db).all()
    scale = db_ref.abs().max().item()
    sens = (db_ref - db_exact).abs().max().item() / scale
    err = O.rel_err(db, db_ref)
    _say(f"  dbeta err {err:.2e}, sensitivity to the stored output {sens:.2e}")
    assert err <= max(TOL_DBETA_FP16, 2 * sens), ("dbeta", err, sens)
