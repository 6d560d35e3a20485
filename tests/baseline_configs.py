"""The BASELINE.json workloads as seeded CPU tensors (the same recipe as bench.py).

A CPU ``torch.Generator().manual_seed(seed)`` draws, in this order, q, k, v, a random dO (drawn
even when the loss fixes dO, so every config sees the same stream), the phi increments and the psi
noise, then beta for "softplus" configs.  phi = cumsum_t N(0, 1) - drift * t; psi = phi + N(0, 1).
"""
import torch

CONFIGS = {
    # name: B, H, T, D, dtype, beta, drift, loss
    "cfg1": dict(B=1, H=2, T=256, D=32, dtype=torch.float32, beta="ones", drift=0.0, loss="sum"),
    "cfg2": dict(B=4, H=12, T=2048, D=64, dtype=torch.float16, beta="ones", drift=0.0, loss="sum"),
    "cfg3": dict(B=2, H=8, T=4096, D=128, dtype=torch.float32, beta="softplus", drift=0.0, loss="sum"),
    "cfg4": dict(B=1, H=12, T=16381, D=64, dtype=torch.float16, beta="ones", drift=0.01, loss="sum"),
}


def make_config(name, seed=0, random_do=False):
    """(q, k, v, phi, psi, beta, do) of BASELINE config `name`.  do is the gradient of the config's loss
    (o.sum() / o.float().sum(): all ones), or the drawn N(0, 1) dO when random_do."""
    c = CONFIGS[name]
    B, H, T, D, dt = c["B"], c["H"], c["T"], c["D"], c["dtype"]
    g = torch.Generator().manual_seed(seed)
    q, k, v, do = (torch.randn(B, H, T, D, generator=g).to(dt) for _ in range(4))
    phi = torch.randn(B, H, T, generator=g).cumsum(-1) - c["drift"] * torch.arange(T, dtype=torch.float32)
    psi = phi + torch.randn(B, H, T, generator=g)
    if c["beta"] == "ones":
        beta = torch.ones(H)
    else:
        beta = torch.nn.functional.softplus(torch.randn(H, generator=g))
    if not random_do:
        do = torch.ones_like(do)
    return q, k, v, phi, psi, beta, do
