"""A seeded sweep of mixed shapes and inputs through the HIP kernels against the float64 oracle.

The fixed cases (test_gpu_parity.py) follow the reference's test matrix (test.py:134-147); this
sweep draws further combinations from one seeded generator: ragged lengths, every head
dimension up to 256, both dtypes, beta of either sign or zero per head, tau, the phi scale and
drift, and the psi noise, which together move the backward's per-block decisions (per-key bias
and soft-min classes, open gates, product or exact soft-min forms) around.  The bounds are the
reference's (test.py:18-20): max |x - ref| / max |ref| <= 2e-3 in fp16 (1e-2 for dbeta) and 2e-4
in fp32.

The backward's Delta_t = sum_d dO_td O_td reads the output as the forward stored it, as the
reference's _bwd_delta does (kernel.py:165-174).  In fp16 that output is rounded to fp16, and
dbeta and dphi, sums of dS_ts over many pairs whose rows cancel (every row of dS sums to zero),
move by up to several percent from that rounding alone on some draws.  So fp16 gradients are
checked against ``fpa_grads_stored`` given the kernel's own output (the float64 gradients with
Delta from that output, everything else exact); fp32 gradients, whose output rounding is at the
level of the backward's own fp32 arithmetic, against the exact gradients; o against the exact
forward.

The draws stay in the reference's data model (psi = phi + noise of at most 0.5, phi scale up to 4).
With beta < 0 the bias is positive and grows with the range of the walk: at T = 1531 and phi scale 4
the logits and lse reach 630 (base 2).  dbeta is a sum over every causal pair of dS_ts min(0, x_ts),
dS = P dP - P Delta, and on some draws those products cancel by orders of magnitude (A / |dbeta| from
5e3 to 5e5 with A = sum |P min(0, x)| (|dP| + |Delta|), ``oracle.dbeta_terms``): rounding at the level
of the arithmetic then moves dbeta past a relative bound with nothing wrong.  So dbeta of each head may
also differ by KAPPA * A, an error of KAPPA relative to every product it is made of: 2^-14 in fp16, 2^-24
(one unit of fp32 roundoff) in fp32.  Over 348 draws (these and a wider one-off sweep) the most any head
needed beyond the relative bound was 4.6e-6 A in fp16 (B1 H1 T17, dbeta 4.5e-2 from the stored-output
oracle with A / |dbeta| = 6.5e3) and 4.4e-9 A in fp32 (T383, beta < 0, 7.7e-3 with A / |dbeta| = 4.9e5);
a wrong or missing term would move dbeta by a fraction of A.
"""
import random
import sys

import pytest
import torch

from oracle import fpa_oracle as O
from test_gpu_parity import NAMES, TOL, TOL_DBETA_FP16, check, run_hip

# dbeta is a sum over every causal pair of dS_ts min(0, x_ts), dS = P dP - P Delta, whose products
# cancel by orders of magnitude on some draws.  Relative errors e in dP and Delta move it by at most
# e * A (oracle.dbeta_terms), so besides the reference's relative bound each head may differ by KAPPA * A:
# 2^-14 in fp16 and 2^-24 in fp32, each at least 13 times what any of 348 draws needed.
KAPPA = {torch.float16: 2.0 ** -14, torch.float32: 2.0 ** -24}


def check_dbeta(x, ref, mag, dtype):
    tol = TOL_DBETA_FP16 if dtype == torch.float16 else TOL[dtype]
    err = (x.double() - ref.double()).abs()
    bound = tol * ref.double().abs().max() + KAPPA[dtype] * mag.double()
    need = ((err - tol * ref.double().abs().max()) / mag.double().clamp(min=1e-300)).max().item()
    print(f"[sweep] dbeta rel {O.rel_err(x, ref):.2e}, beyond the relative bound {need:.2e} of A", flush=True)
    assert torch.isfinite(x).all() and (err <= bound).all(), ("dbeta", err.tolist(), bound.tolist())

pytestmark = pytest.mark.gpu


def _cases(n=16, seed=2026, lengths=(1, 37, 64, 129, 200, 333, 512, 701), first=1000,
           betas=("positive", "negative", "mixed", "zero"), dims=(16, 32, 64, 128), ties=False,
           dtypes=("f16", "f32"), taus=(0.5, 1.0, 2.0), scales=(0.3, 1.0, 4.0)):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        out.append(dict(
            B=rng.choice([1, 2]), H=rng.choice([1, 2, 3]),
            T=rng.choice(lengths),
            D=rng.choice(dims),
            dtype=rng.choice(dtypes),
            beta=rng.choice(betas),
            tau=rng.choice(taus),
            phi_scale=rng.choice(scales),
            drift=rng.choice([0.0, 0.02]),
            psi_noise=rng.choice([0.1, 0.25, 0.5]),
            ties=ties,
            seed=first + i))
    return out


# Short and ragged lengths; six draws over 16 to 32 blocks (more off-diagonal blocks per tile, so
# every per-block class occurs), beta > 0; six draws at D = 256 (the single-wave-per-SIMD kernels); six
# with phi rounded to integers (equal values inside ranges: tied minima and equal soft-min weights); four
# long fp16 draws with beta of either sign; six at extreme temperatures (tau 0.1: the soft-min weights
# near one-hot over spans of a few units of phi; tau 8: near-uniform); four long fp32 draws with
# negative or mixed beta; then a wider draw of 100 over lengths up to 2500 and every head dimension, and
# 25 long draws at tau 0.1 to 8 (six of these have dbeta sums that cancel by 5e3 to 5e5); then 24 at phi
# scales 10 to 40 (soft-min spreads past the product form's range and the in-block recurrence's single
# reference).
CASES = (_cases() + _cases(n=6, seed=7, lengths=(1000, 1531, 2048), first=2000, betas=("positive",))
         + _cases(n=6, seed=11, lengths=(3, 65, 190, 449, 640), first=3000, dims=(256,))
         + _cases(n=6, seed=13, lengths=(97, 256, 511, 800), first=4000, ties=True)
         + _cases(n=4, seed=17, lengths=(1000, 1531, 2048), first=5000, betas=("negative", "mixed"), dtypes=("f16",))
         + _cases(n=6, seed=19, lengths=(64, 300, 777), first=6000, betas=("positive", "mixed"), taus=(0.1, 8.0))
         + _cases(n=4, seed=23, lengths=(1000, 1531, 2048), first=7000, betas=("negative", "mixed"), dtypes=("f32",),
                  dims=(16, 32, 64))
         + _cases(n=100, seed=31337, lengths=(1, 17, 63, 65, 127, 129, 255, 383, 385, 511, 640, 897, 1025, 1500, 2047,
                                             2500), first=90000, dims=(16, 32, 64, 128, 256))
         + _cases(n=25, seed=31339, lengths=(450, 999, 1800), first=92000, taus=(0.1, 0.25, 4.0, 8.0))
         + _cases(n=24, seed=41, lengths=(33, 100, 257, 600, 1100), first=93000, dims=(16, 32, 64, 128, 256),
                  taus=(0.3, 1.0, 3.0), scales=(10.0, 20.0, 40.0)))


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
                                             phi_scale=c["phi_scale"], psi_noise=c["psi_noise"], drift=c["drift"],
                                             ties=c["ties"])
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
    mag = O.dbeta_terms(q, k, v, phi, psi, beta, do, tau=c["tau"])[1]
    if dtype == torch.float32:
        check(kern[:6], exact[:6], dtype)
        check_dbeta(kern[6], exact[6], mag, dtype)
        return
    check(kern[:1], exact[:1], dtype)
    ref = O.fpa_grads_stored(q, k, v, phi, psi, beta, do, tau=c["tau"], o_stored=kern[0])
    check(kern[:6], [exact[0]] + ref[1:6], dtype, NAMES[:6])
    check_dbeta(kern[6], ref[6], mag, dtype)
