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


@pytest.mark.gpu
def test_cfg5_full_size_step():
    """BASELINE config 5 at full size: the 12-layer d768 H12 decoder (MLP 3072, vocab 32000) on B8 x
    T2048 random tokens under fp16 autocast.  One forward + backward: the loss is finite and within
    1 of ln(32000) (random init), every parameter gets a finite, non-zero gradient, and a second step
    from the same seed gives a bit-identical loss and bit-identical attention-layer gradients."""
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    print("[lm] cfg5 full size: 12 layers d768 H12, B8 T2048, fp16 autocast", flush=True)
    tok = _tokens(8, 2048, 32000, 5).cuda()
    runs = []
    for _ in range(2):
        torch.manual_seed(0)
        m = FPADecoder(32000, 768, 12, 12, 3072, impl="hip").cuda()
        with torch.autocast("cuda", dtype=torch.float16):
            loss = m.loss(tok)
        loss.backward()
        torch.cuda.synchronize()
        grads = {n: p.grad.detach().clone() for n, p in m.named_parameters()}
        runs.append((loss.detach().clone(), grads))
        del m
    loss, grads = runs[0]
    assert torch.isfinite(loss)
    assert abs(loss.item() - torch.log(torch.tensor(32000.0)).item()) < 1.0, loss.item()
    for n, g in grads.items():
        assert torch.isfinite(g).all() and g.abs().max() > 0, n
    assert torch.equal(runs[0][0], runs[1][0])
    for n in grads:
        if ".attn." in n:
            assert torch.equal(runs[0][1][n], runs[1][1][n]), n


@pytest.mark.gpu
def test_cfg5_layer_hip_matches_dense_at_full_size():
    """One FirstPassageAttention block of the cfg5 model (d768, 12 heads) at B8 x T2048 under fp16
    autocast: output and every parameter gradient of the HIP layer against the dense layer with the
    same weights, to a relative norm of 5e-3 (the reference's autocast bound, test.py:200-214)."""
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    import fpa
    print("[lm] cfg5 layer at B8 T2048 d768 H12: hip vs dense, fp16 autocast", flush=True)
    x = torch.randn(8, 2048, 768, generator=torch.Generator().manual_seed(6)).cuda()
    out = []
    for impl in ("hip", "reference"):
        torch.manual_seed(0)
        layer = fpa.FirstPassageAttention(768, 12, impl=impl).cuda()
        with torch.autocast("cuda", dtype=torch.float16):
            y = layer(x)
        # A sum, not a mean: the mean over 12.6M outputs puts the fp16 gradients of both paths in
        # the subnormal range, where neither is accurate.  The comparison is scale-free.
        loss = y.float().square().sum()
        out.append([y.detach().float()] + [g.detach() for g in torch.autograd.grad(loss, list(layer.parameters()))])
        del layer, y, loss
        torch.cuda.empty_cache()
    for i, (a, b) in enumerate(zip(*out)):
        assert torch.isfinite(a).all(), i
        assert ((a - b).norm() / b.norm()).item() <= 5e-3, (i, ((a - b).norm() / b.norm()).item())
