"""The cfg5 LM harness model (fpa.lm.FPADecoder) built on the FirstPassageAttention layer."""
import pytest
import torch

from fpa.lm import FPADecoder

TINY = dict(vocab=500, d_model=64, n_heads=4, layers=2, d_mlp=128)


def _tokens(B, T, vocab, seed):
    return torch.randint(0, vocab, (B, T + 1), generator=torch.Generator().manual_seed(seed))


def test_tiny_lm_step_on_cpu():
    """Reference-path training step: finite loss near log(vocab) at init, tied head, every
    parameter gets a gradient."""
    torch.manual_seed(0)
    m = FPADecoder(**TINY, impl="reference")
    assert m.head.weight is m.emb.weight
    loss = m.loss(_tokens(2, 40, TINY["vocab"], 1))
    assert torch.isfinite(loss)
    assert abs(loss.item() - torch.log(torch.tensor(float(TINY["vocab"]))).item()) < 1.0
    loss.backward()
    for n, p in m.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad).all(), n


@pytest.mark.gpu
def test_tiny_lm_hip_matches_reference():
    """The same model and tokens with the HIP kernels and with the dense path (fp32, ragged
    T = 80): loss and every parameter gradient agree to a relative norm of 1e-4."""
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    print("[lm] tiny decoder fp32 hip vs reference, B2 T80", flush=True)
    tok = _tokens(2, 80, TINY["vocab"], 2).cuda()
    out = []
    for impl in ("hip", "reference"):
        torch.manual_seed(0)
        m = FPADecoder(**TINY, impl=impl).cuda()
        loss = m.loss(tok)
        grads = torch.autograd.grad(loss, list(m.parameters()))
        out.append([loss.detach()] + [g.detach() for g in grads])
    for a, b in zip(*out):
        assert torch.isfinite(a).all()
        assert ((a - b).norm() / b.norm().clamp(min=1e-30)).item() <= 1e-4
