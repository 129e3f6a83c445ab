"""A single-GPU restatement of mini-megatron's GPT (test and benchmark harness only).

Same module structure and forward as the reference model at TP = PP = 1:
model/embedding.py:5-16 (token + position embedding), model/transformer.py:8-112
(pre-LN decoder layers: qkv and output projections, causal SDPA, GELU MLP;
final LayerNorm; lm_head), model/loss.py:4-15 (masked mean cross-entropy).  The
linear layers call F.linear from classes named *Linear, as the reference's
ColumnParallelLinear / RowParallelLinear do (parallel/tensor_parallel.py:55,79).
Initialisation follows parallel/tensor_parallel.py:9-10 (N(0, 0.02)).
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F


class ColumnLinear(nn.Module):
    def __init__(self, n_in: int, n_out: int):
        super().__init__()
        self.weight = nn.Parameter(torch.empty(n_out, n_in).normal_(0.0, 0.02))

    def forward(self, x):
        return F.linear(x, self.weight)


class RowLinear(ColumnLinear):
    pass


class Block(nn.Module):
    def __init__(self, h: int, heads: int, ffn: int):
        super().__init__()
        self.heads = heads
        self.ln1 = nn.LayerNorm(h)
        self.qkv = ColumnLinear(h, 3 * h)
        self.o = RowLinear(h, h)
        self.ln2 = nn.LayerNorm(h)
        self.fc1 = ColumnLinear(h, ffn)
        self.fc2 = RowLinear(ffn, h)

    def forward(self, x):
        b, s, h = x.shape
        qkv = self.qkv(self.ln1(x)).reshape(b, s, 3, self.heads, h // self.heads)
        q, k, v = (t.transpose(1, 2) for t in qkv.unbind(2))
        a = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        x = x + self.o(a.transpose(1, 2).reshape(b, s, h))
        return x + self.fc2(F.gelu(self.fc1(self.ln2(x))))


class GPT(nn.Module):
    def __init__(self, vocab: int, h: int, heads: int, ffn: int, layers: int, seq: int):
        super().__init__()
        self.wte = nn.Parameter(torch.empty(vocab, h).normal_(0.0, 0.02))
        self.wpe = nn.Embedding(seq, h)
        self.layers = nn.ModuleList(Block(h, heads, ffn) for _ in range(layers))
        self.ln_f = nn.LayerNorm(h)
        self.lm_head = ColumnLinear(h, vocab)

    def forward(self, ids, labels, mask):
        x = F.embedding(ids, self.wte) + self.wpe(torch.arange(ids.shape[-1], device=ids.device))
        for blk in self.layers:
            x = blk(x)
        logits = self.lm_head(self.ln_f(x))
        loss = F.cross_entropy(logits.reshape(-1, logits.shape[-1]), labels.reshape(-1),
                               reduction="none")
        return logits, (loss * mask.reshape(-1)).sum() / mask.sum()


def tiny(device, seed: int = 0) -> GPT:
    torch.manual_seed(seed)
    return GPT(vocab=512, h=128, heads=4, ffn=512, layers=2, seq=64).to(device)


def batch(device, b: int = 2, s: int = 64, vocab: int = 512, seed: int = 1):
    g = torch.Generator(device="cpu").manual_seed(seed)
    ids = torch.randint(0, vocab, (b, s + 1), generator=g)
    return ids[:, :-1].to(device), ids[:, 1:].to(device), torch.ones(b, s, device=device)
