"""A pre-norm decoder language model built on the FirstPassageAttention layer.

The training-step workload of the build's LM measurements: token embedding, `layers` blocks of
[LayerNorm -> FirstPassageAttention -> residual, LayerNorm -> GELU MLP -> residual], a final
LayerNorm and an output head tied to the embedding.  The reference ships the attention layer
(kernel.py:512-530) but no model around it; this one has the usual GPT-2-small shape (d_model 768,
12 heads, MLP 3072) so that a step exercises the layer at the size it is meant for.
"""
import torch
import torch.nn as nn
import torch.nn.functional as F

from . import FirstPassageAttention


class DecoderBlock(nn.Module):
    def __init__(self, d_model, n_heads, d_mlp, impl=None):
        super().__init__()
        self.ln1 = nn.LayerNorm(d_model)
        self.attn = FirstPassageAttention(d_model, n_heads, impl=impl)
        self.ln2 = nn.LayerNorm(d_model)
        self.fc1 = nn.Linear(d_model, d_mlp)
        self.fc2 = nn.Linear(d_mlp, d_model)

    def forward(self, x):
        x = x + self.attn(self.ln1(x))
        return x + self.fc2(F.gelu(self.fc1(self.ln2(x))))


class FPADecoder(nn.Module):
    """tokens (B, T) int64 -> logits (B, T, vocab)."""

    def __init__(self, vocab=32000, d_model=768, n_heads=12, layers=12, d_mlp=3072, impl=None):
        super().__init__()
        self.vocab = vocab
        self.emb = nn.Embedding(vocab, d_model)
        self.blocks = nn.ModuleList(DecoderBlock(d_model, n_heads, d_mlp, impl) for _ in range(layers))
        self.ln = nn.LayerNorm(d_model)
        self.head = nn.Linear(d_model, vocab, bias=False)
        self.head.weight = self.emb.weight
        nn.init.normal_(self.emb.weight, std=0.02)

    def forward(self, tokens):
        x = self.emb(tokens)
        for blk in self.blocks:
            x = blk(x)
        return self.head(self.ln(x))

    def loss(self, tokens):
        """Next-token cross entropy of tokens (B, T + 1): inputs tokens[:, :-1], targets tokens[:, 1:].

        The log-softmax reads the (fp16 under autocast) logits and works and writes in fp32 itself, so
        no fp32 copy of the logits is made first (the same values as cross_entropy on logits.float());
        autocast is off around it, since it would otherwise make that copy."""
        logits = self(tokens[:, :-1])
        with torch.autocast(device_type=logits.device.type, enabled=False):
            logp = torch.log_softmax(logits.reshape(-1, self.vocab), -1, dtype=torch.float32)
            return F.nll_loss(logp, tokens[:, 1:].reshape(-1))
