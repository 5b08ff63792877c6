"""BF16 residual stream with FP32 master parameters (the counterpart of WarpState's
``ops/residual_experiment.py:25-58``).

Under BF16 autocast the embedding table and the depth modulation enter the forward as
BF16 casts of their FP32 masters, so the residual stream, and with it every residual add,
is BF16: x <- r(x + r(projection)), the arithmetic of the fused residual epilogue. The
casts are differentiable, so gradients reach the FP32 masters, and the optimizer, the
state dict and every other parameter are unchanged. Calls outside BF16 autocast run the
original forward.
"""

from __future__ import annotations

import torch
from torch.func import functional_call

_CAST = ("embed.weight", "depth_scale", "depth_bias")


class _Detached(torch.nn.Module):
    """Holds the model for ``functional_call`` and runs its original forward. It is kept
    only by the patched forward's closure, never registered on the model, so the model's
    state dict keeps its keys."""

    def __init__(self, model: torch.nn.Module, forward):
        super().__init__()
        self.model = model
        self.run = forward

    def forward(self, *args, **kwargs):
        return self.run(*args, **kwargs)


def apply_bf16_residuals(model: torch.nn.Module) -> None:
    """Make the residual stream BF16 inside BF16 autocast. Apply after placing the model
    and loading weights, before any DDP wrapper."""
    if getattr(model, "_bf16_residuals", False):
        raise ValueError("BF16 residual execution has already been applied")
    masters = {name: model.get_parameter(name) for name in _CAST}
    if any(p.dtype != torch.float32 for p in masters.values()):
        raise ValueError("BF16 residual execution requires FP32 master parameters")
    original = model.forward
    holder = _Detached(model, original)

    def forward(input_ids, targets=None, *, return_logits=True):
        kind = input_ids.device.type
        if not (torch.is_autocast_enabled(kind)
                and torch.get_autocast_dtype(kind) == torch.bfloat16):
            return original(input_ids, targets, return_logits=return_logits)
        # functional_call swaps the casts in for the call and restores the masters after
        # it, also when the forward raises.
        casts = {"model." + name: p.to(torch.bfloat16) for name, p in masters.items()}
        return functional_call(holder, casts, (input_ids,),
                               {"targets": targets, "return_logits": return_logits},
                               strict=False)

    model.forward = forward
    model._bf16_residuals = True
