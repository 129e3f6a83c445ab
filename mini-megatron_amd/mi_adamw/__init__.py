"""mi_adamw: MI355X-native fused clip + AdamW optimizer step for mini-megatron.

``FusedAdamW`` is a drop-in for the ``torch.optim.AdamW`` that mini-megatron's
training loop builds (main.py:177) and steps (main.py:209); ``clip_grad_norm_``
is a drop-in for ``torch.nn.utils.clip_grad_norm_``.  Both run hand-written
HIP kernels for gfx950 through the C ABI of libmi_adamw.so
(include/mi_adamw.h); there is no CPU or torch fallback.
"""
from .optimizer import FusedAdamW, DEFAULT_CHUNK_ELEMS
from .clip import clip_grad_norm_
from ._lib import version, MiAdamwError

AdamW = FusedAdamW

__all__ = ["FusedAdamW", "AdamW", "clip_grad_norm_", "version", "MiAdamwError",
           "DEFAULT_CHUNK_ELEMS"]
