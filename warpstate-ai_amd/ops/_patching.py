"""Forward replacement shared by the model adapters of this package.

An adapter swaps a module's bound ``forward`` for a dispatcher that sends a call to an
accelerated body only when the call qualifies (training, gradients on, a CUDA input under
BF16 autocast, plus whatever the adapter adds) and to the module's original forward
otherwise. Parameters, buffers, submodules and the state dict are left alone, so the
patched model saves, loads and evaluates exactly like the unpatched one.
"""

from __future__ import annotations

from typing import Callable

import torch

Accelerated = Callable[[torch.nn.Module, torch.Tensor, Callable], torch.Tensor]
Predicate = Callable[[torch.nn.Module, torch.Tensor], bool]


def bf16_autocast_training(module: torch.nn.Module, x: torch.Tensor) -> bool:
    """True for a training-mode call with gradients enabled on a CUDA tensor inside BF16
    autocast: the calls the reference's adapters accelerate (ops/matmul_execution.py:357-360,
    ops/activation_execution.py:233-236)."""
    return (module.training and torch.is_grad_enabled() and x.is_cuda
            and torch.is_autocast_enabled("cuda")
            and torch.get_autocast_dtype("cuda") == torch.bfloat16)


def install_forward(module: torch.nn.Module, accelerated: Accelerated,
                    eligible: Predicate = bf16_autocast_training) -> None:
    """Replace ``module.forward`` by a dispatcher: ``accelerated(module, x, original)`` for
    eligible calls, ``original(x)`` for the rest. ``accelerated`` receives the original
    forward so that it can still decline a call it cannot serve."""
    original = module.forward

    def forward(x, _module=module, _original=original):
        if eligible(_module, x):
            return accelerated(_module, x, _original)
        return _original(x)

    module.forward = forward
