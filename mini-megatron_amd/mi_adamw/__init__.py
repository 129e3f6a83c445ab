"""mi_adamw: MI355X-native fused clip + AdamW optimizer step for mini-megatron.

``FusedAdamW`` is a drop-in for the ``torch.optim.AdamW`` that mini-megatron's
training loop builds (main.py:177) and steps (main.py:209); ``clip_grad_norm_``
is a drop-in for ``torch.nn.utils.clip_grad_norm_``.  Both run hand-written
HIP kernels for gfx950 through the C ABI of libmi_adamw.so
(include/mi_adamw.h); there is no CPU or torch fallback.  ``bf16_weights``
feeds the step's bf16 model copy to the linear layers of a bf16-autocast
forward in place of autocast's per-forward weight casts.
"""
from .optimizer import FusedAdamW, DEFAULT_CHUNK_ELEMS
from .clip import clip_grad_norm_
from .bf16_forward import bf16_weights, linear_layers
from ._lib import version, MiAdamwError
from .zero import ZeroRangeStep, dp_prescale, shard_bounds

AdamW = FusedAdamW

__all__ = ["FusedAdamW", "AdamW", "clip_grad_norm_", "bf16_weights", "linear_layers", "version",
           "MiAdamwError", "DEFAULT_CHUNK_ELEMS", "ZeroRangeStep", "dp_prescale", "shard_bounds"]
