"""GPT parameter sets of mini-megatron's model family, for sizing and benchmarks.

Registration order follows mini-megatron's model (what ``model.parameters()``
yields, hence the order of ``param_groups`` and of ``state_dict`` ids):
Embedding (model/embedding.py:8-9: token table [V, H], position table [P, H]),
then per decoder layer (model/transformer.py:54-57) ln1.weight, ln1.bias,
attn.qkv.weight [3H, H], attn.o.weight [H, H], ln2.weight, ln2.bias,
mlp.fc1.weight [F, H], mlp.fc2.weight [H, F] (linears are bias-free,
transformer.py:22-23,42-43), then ln_f.weight, ln_f.bias and an untied lm_head
[V, H] (transformer.py:95-99; main.py:172).
"""
from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class GPTShape:
    name: str
    layers: int
    hidden: int
    heads: int
    ffn: int
    vocab: int
    positions: int

    def tensors(self) -> list[tuple[str, tuple[int, ...]]]:
        H, F, V, P = self.hidden, self.ffn, self.vocab, self.positions
        out = [("embedding.token_embedding.weight", (V, H)),
               ("embedding.position_embedding.weight", (P, H))]
        for i in range(self.layers):
            pre = f"decoder.layers.{i}."
            out += [(pre + "ln1.weight", (H,)), (pre + "ln1.bias", (H,)),
                    (pre + "attn.qkv.weight", (3 * H, H)), (pre + "attn.o.weight", (H, H)),
                    (pre + "ln2.weight", (H,)), (pre + "ln2.bias", (H,)),
                    (pre + "mlp.fc1.weight", (F, H)), (pre + "mlp.fc2.weight", (H, F))]
        out += [("ln_f.weight", (H,)), ("ln_f.bias", (H,)), ("lm_head.weight", (V, H))]
        return out

    def numel(self) -> int:
        total = 0
        for _, shape in self.tensors():
            n = 1
            for d in shape:
                n *= d
            total += n
        return total


GPT_125M = GPTShape("gpt-125m", layers=12, hidden=768, heads=12, ffn=3072, vocab=50257,
                    positions=1024)
GPT_350M = GPTShape("gpt-350m", layers=24, hidden=1024, heads=16, ffn=4096, vocab=50257,
                    positions=1024)
GPT_1P3B = GPTShape("gpt-1.3b", layers=24, hidden=2048, heads=16, ffn=8192, vocab=50257,
                    positions=2048)
GPT_6P7B = GPTShape("gpt-6.7b", layers=32, hidden=4096, heads=32, ffn=16384, vocab=50257,
                    positions=2048)

SHAPES = {s.name: s for s in (GPT_125M, GPT_350M, GPT_1P3B, GPT_6P7B)}


def init_kind(name: str) -> str:
    """How a tensor is initialised: LayerNorm weights 1, biases 0, the rest N(0, 0.02)."""
    if name.endswith(".bias"):
        return "zeros"
    if ".ln" in name or name.startswith("ln_f"):
        return "ones"
    return "normal"
