"""The blockwise decomposition used by the HIP kernels, checked against the dense oracle.

Runs entirely on the CPU in float64: block statistics, the per-pair range minimum
from them, and the four-part soft-min gradient (key block, query block, middle
blocks, in-block recurrence) must reproduce the oracle's output and all gradients.
"""
import numpy as np
import pytest
import torch

import blockwise_model as M
from oracle import fpa_oracle as O

CASES = [  # T, G, phi_scale, ties, tau, drift
    (37, 8, 1.0, False, 1.0, 0.0),
    (50, 8, 40.0, False, 1.0, 0.0),
    (45, 8, 1.0, True, 0.7, 0.0),
    (64, 16, 1.0, False, 0.25, 0.0),
    (41, 8, 1.0, False, 1.0, 0.3),
    (7, 8, 1.0, False, 1.0, 0.0),
    (24, 8, 3.0, False, 2.0, -0.5),
]


@pytest.mark.parametrize("T,G,scale,ties,tau,drift", CASES)
def test_blockwise_matches_oracle(T, G, scale, ties, tau, drift):
    q, k, v, phi, psi, beta, do = O.make_inputs(1, 2, T, 8, dtype=torch.float64, seed=T + G,
                                                phi_scale=scale, ties=ties, drift=drift)
    ref = O.fpa_grads(q, k, v, phi, psi, beta, do, tau=tau)
    for h in range(2):
        got = M.backward(q[0, h].numpy(), k[0, h].numpy(), v[0, h].numpy(), phi[0, h].numpy(),
                         psi[0, h].numpy(), beta[h].item(), do[0, h].numpy(), G, tau)
        want = [ref[0][0, h], ref[1][0, h], ref[2][0, h], ref[3][0, h], ref[4][0, h],
                ref[5][0, h], ref[6][h]]
        for name, a, b in zip(("o", "dq", "dk", "dv", "dphi", "dpsi", "dbeta"), got, want):
            b = b.numpy()
            err = np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)
            assert err < 1e-9, (name, h, err)
