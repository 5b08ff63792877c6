"""Opt-in BF16 SwiGLU and RMSNorm execution on gfx950 without replacing parameters.

Call surface of WarpState's ``ops/activation_execution.py``. Eager execution keeps the
model's BF16 rounding boundaries; compiled execution (``eager_rounding=False``) keeps
BF16 kernel inputs and outputs but elides the intermediate casts. Normalization
statistics and master-parameter gradients stay FP32. CPU, evaluation and non-BF16 paths
stay original. Kernels are the HIP row kernels of ``libwarpstate_hip.so``.
"""

from __future__ import annotations

import torch

from ops import _hip


@torch.library.custom_op("warpstate::bf16_swiglu", mutates_args=())
def bf16_swiglu(packed: torch.Tensor, eager_rounding: bool = True) -> torch.Tensor:
    """SwiGLU of a contiguous BF16 [*, 2*hidden] projection (ops/activation_execution.py:58-70)."""
    hidden = packed.shape[-1] // 2
    output = torch.empty((*packed.shape[:-1], hidden), device=packed.device, dtype=packed.dtype)
    rows = output.numel() // hidden
    _hip.call("ws_swiglu_forward", packed.data_ptr(), output.data_ptr(), rows, hidden,
              int(eager_rounding), _hip.stream(packed))
    return output


@bf16_swiglu.register_fake
def _bf16_swiglu_fake(packed, eager_rounding=True):
    return packed.new_empty((*packed.shape[:-1], packed.shape[-1] // 2))


@torch.library.custom_op("warpstate::bf16_swiglu_backward", mutates_args=())
def _swiglu_backward(packed: torch.Tensor, grad: torch.Tensor,
                     eager_rounding: bool) -> torch.Tensor:
    """dUp | dGate from the packed projection and the SwiGLU output gradient
    (ops/activation_execution.py:73-81)."""
    grad = grad.contiguous()
    output = torch.empty_like(packed)
    hidden = packed.shape[-1] // 2
    _hip.call("ws_swiglu_backward", packed.data_ptr(), grad.data_ptr(), output.data_ptr(),
              grad.numel() // hidden, hidden, int(eager_rounding), _hip.stream(packed))
    return output


@_swiglu_backward.register_fake
def _swiglu_backward_fake(packed, grad, eager_rounding):
    return torch.empty_like(packed)


def _swiglu_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[0])
    ctx.eager_rounding = inputs[1]


def _swiglu_autograd(ctx, grad):
    return _swiglu_backward(ctx.saved_tensors[0], grad, ctx.eager_rounding), None


bf16_swiglu.register_autograd(_swiglu_autograd, setup_context=_swiglu_setup)


@torch.library.custom_op("warpstate::bf16_rmsnorm", mutates_args=())
def bf16_rmsnorm(x: torch.Tensor, weight: torch.Tensor,
                 eps: float, eager_rounding: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    """BF16 RMSNorm with FP32 statistics; also returns the saved row rsqrts
    (ops/activation_execution.py:161-173)."""
    width = x.shape[-1]
    rows = x.numel() // width
    output = torch.empty_like(x)
    rstd = torch.empty((rows,), device=x.device, dtype=torch.float32)
    _hip.call("ws_rmsnorm_forward", x.data_ptr(), weight.data_ptr(), output.data_ptr(),
              rstd.data_ptr(), rows, width, float(eps), int(eager_rounding), _hip.stream(x))
    return output, rstd


@bf16_rmsnorm.register_fake
def _bf16_rmsnorm_fake(x, weight, eps, eager_rounding=True):
    rows = x.numel() // x.shape[-1]
    return torch.empty_like(x), x.new_empty((rows,), dtype=torch.float32)


@torch.library.custom_op("warpstate::bf16_rmsnorm_backward", mutates_args=())
def _rms_backward(x: torch.Tensor, weight: torch.Tensor, rstd: torch.Tensor,
                  grad: torch.Tensor, eager_rounding: bool) -> tuple[torch.Tensor, torch.Tensor]:
    """dX (BF16) and the FP32 weight gradient (ops/activation_execution.py:176-194)."""
    grad = grad.contiguous()
    x = x.contiguous()
    width = x.shape[-1]
    rows = x.numel() // width
    output = torch.empty_like(x)
    weight_grad = torch.empty_like(weight)
    partial = torch.empty((_hip.query("ws_rmsnorm_backward_partial_floats", rows, width),),
                          device=x.device, dtype=torch.float32)
    _hip.call("ws_rmsnorm_backward", x.data_ptr(), weight.data_ptr(), rstd.data_ptr(),
              grad.data_ptr(), output.data_ptr(), weight_grad.data_ptr(), partial.data_ptr(),
              rows, width, int(eager_rounding), _hip.stream(x))
    return output, weight_grad


@_rms_backward.register_fake
def _rms_backward_fake(x, weight, rstd, grad, eager_rounding):
    return torch.empty_like(x), torch.empty_like(weight)


def _rms_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[0], inputs[1], output[1])
    ctx.mark_non_differentiable(output[1])
    ctx.eager_rounding = inputs[3]


def _rms_autograd(ctx, grad, _grad_rstd):
    x, weight, rstd = ctx.saved_tensors
    dx, dw = _rms_backward(x, weight, rstd, grad, ctx.eager_rounding)
    return dx, dw, None, None


bf16_rmsnorm.register_autograd(_rms_autograd, setup_context=_rms_setup)


_MODES = {"baseline": (), "swiglu": ("swiglu",), "rmsnorm": ("rmsnorm",),
          "all": ("swiglu", "rmsnorm")}


def _fused_swiglu_forward(module, x, _original):
    """up_gate, then the SwiGLU row kernel on the packed projection, then down."""
    act = bf16_swiglu(module.up_gate(x).contiguous(),
                      eager_rounding=not torch.compiler.is_compiling())
    return module.down(act)


def _rms_input_ok(module, x) -> bool:
    """Training calls the RMSNorm row kernels take: a non-empty contiguous BF16 CUDA tensor
    whose rows fit the kernels (at most 8192 features)."""
    return (module.training and torch.is_grad_enabled() and x.is_cuda
            and x.dtype == torch.bfloat16 and x.is_contiguous() and x.numel() > 0
            and 0 < x.shape[-1] <= 8192)


def _fused_rms_forward(module, x, _original):
    return bf16_rmsnorm(x, module.weight, module.eps,
                        eager_rounding=not torch.compiler.is_compiling())[0]


def apply_activation_execution(model: torch.nn.Module, mode: str = "baseline") -> None:
    """Send the SwiGLU and/or RMSNorm modules' training forwards to the HIP row kernels
    (ops/activation_execution.py:212-253); ``baseline`` changes nothing. The FP32 parameter
    objects and the state dict stay as they are, and other calls keep the original path.
    Eager calls keep eager BF16 rounding; traced calls use the compiled arithmetic."""
    from warpstate.model import RMSNorm, SwiGLU

    from ops._patching import bf16_autocast_training, install_forward

    if mode not in _MODES:
        raise ValueError(f"Unknown activation execution mode: {mode}")
    if getattr(model, "_activation_execution_mode", "baseline") != "baseline":
        raise ValueError("Activation execution has already been applied")
    if mode == "baseline":
        return
    if any(p.dtype != torch.float32 for p in model.parameters()):
        raise ValueError("Activation execution requires FP32 master parameters")
    routes = {"swiglu": (SwiGLU, _fused_swiglu_forward, bf16_autocast_training),
              "rmsnorm": (RMSNorm, _fused_rms_forward, _rms_input_ok)}
    selected = [routes[name] for name in _MODES[mode]]
    for module in model.modules():
        for kind, body, eligible in selected:
            if isinstance(module, kind):
                install_forward(module, body, eligible)
                break
    model._activation_execution_mode = mode
