"""BF16 residual stream with FP32 master parameters (the counterpart of WarpState's
``ops/residual_experiment.py:25-58``).

Under BF16 autocast the embedding table and the depth modulation enter the forward as
BF16 casts of their FP32 masters, so the residual stream, and with it every residual add,
is BF16: x <- r(x + r(projection)), the arithmetic of the fused residual epilogue. The
casts are differentiable, so gradients reach the FP32 masters, and the optimizer, the
state dict and every other parameter are unchanged. Calls outside BF16 autocast run the
original forward.

Design: each cast parameter is addressed by its owning module's parameter slot. For the
duration of one call the slot holds the BF16 cast; a ``finally`` puts the FP32 master
back, also when the forward raises. No module is added to the model, so the state dict
keeps its keys.
"""

from __future__ import annotations

from contextlib import contextmanager

import torch

# The parameters whose values enter the residual stream (warpstate/model.py: the token
# embedding, tied with the LM head, and the per-depth scale and bias).
_STREAM_PARAMETERS = ("embed.weight", "depth_scale", "depth_bias")


def _slot(model: torch.nn.Module, name: str) -> tuple[torch.nn.Module, str]:
    """(owning module, attribute) of a dotted parameter name."""
    owner_name, _, attr = name.rpartition(".")
    return (model.get_submodule(owner_name) if owner_name else model), attr


@contextmanager
def _bf16_slots(slots):
    """Put r(master) into each (module, attribute, master) slot, restore the masters on
    exit."""
    try:
        for module, attr, master in slots:
            # Written into the parameter table directly: Module.__setattr__ would refuse a
            # non-Parameter tensor for a registered parameter name.
            module._parameters[attr] = master.to(torch.bfloat16)
        yield
    finally:
        for module, attr, master in slots:
            module._parameters[attr] = master


def _bf16_autocast(device_type: str) -> bool:
    return (torch.is_autocast_enabled(device_type)
            and torch.get_autocast_dtype(device_type) == torch.bfloat16)


def apply_bf16_residuals(model: torch.nn.Module) -> None:
    """Make the residual stream BF16 inside BF16 autocast. Apply after placing the model
    and loading weights, before any DDP wrapper."""
    if getattr(model, "_bf16_residuals", False):
        raise ValueError("BF16 residual execution has already been applied")
    slots = []
    for name in _STREAM_PARAMETERS:
        module, attr = _slot(model, name)
        slots.append((module, attr, module._parameters[attr]))
    if any(master.dtype != torch.float32 for _, _, master in slots):
        raise ValueError("BF16 residual execution requires FP32 master parameters")
    unpatched = model.forward

    def forward(input_ids, targets=None, *, return_logits=True):
        if not _bf16_autocast(input_ids.device.type):
            return unpatched(input_ids, targets, return_logits=return_logits)
        with _bf16_slots(slots):
            return unpatched(input_ids, targets, return_logits=return_logits)

    model.forward = forward
    model._bf16_residuals = True
