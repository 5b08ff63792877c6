"""Route a WarpState model's training step through the fused HIP GEMMs (additive adapter).

``apply_fused_execution(model)`` replaces, for eligible training calls, the parts of each
core and of the loss that the fused kernels of ``ops.fused_execution`` cover:

* ``project``: norm1 -> in_proj -> sigmoid on the gate slice (warpstate/model.py:107-112,
  :120-121, :174) becomes one ``rmsnorm_gate_mm`` (RMSNorm row pass, projection with the
  sigmoid in its epilogue);
* the attention output projection with its residual add (warpstate/model.py:177) and
  the SwiGLU block with its residual add (warpstate/model.py:52-60, :178) become
  ``residual_mm`` and ``launch_swiglu_mm`` + ``residual_mm``;
* the chunked tied-head loss (warpstate/model.py:316-334) becomes the fused
  cross-entropy (``linear_cross_entropy``), whose logits never reach HBM.

The backward of each piece is one autograd function built from the fused backward kernels:
the gate-sigmoid backward, the SwiGLU backward fused on the dAct GEMM and the RMSNorm
backward, with the plain input-gradient GEMMs on hipBLASLt (``dgrad_mm``). The projection weights' gradients are accumulated straight into the FP32
masters' ``.grad`` with the FP32-accumulating GEMM, G += f32(r(dY^T X))
(test_gradient_execution.py:243-246), in one grouped launch for the MLP's two weights;
the function returns no gradient for them, so no BF16 weight gradient is materialised
and autograd's own accumulation is bypassed for these parameters (one GPU: there is no
gradient-bucket hook to feed). Every other parameter (norm weights, the tied head, the
embedding and depth modulation) gets its gradient through autograd as usual.

A core call is eligible in training mode with gradients on, under BF16 autocast, on a BF16
CUDA residual stream (``ops.residual_experiment.apply_bf16_residuals``) and bias-free
projections; everything else runs the original forwards. The token mixer between the
projections (``core.mix``) is the model's own code.
"""

from __future__ import annotations

import torch

from ops import fused_execution as fx
from ops._patching import bf16_autocast_training

BF16 = torch.bfloat16


def _grad_buffer(param: torch.Tensor) -> torch.Tensor:
    """The FP32 master's ``.grad``, created as zeros on first use."""
    if param.grad is None:
        param.grad = torch.zeros_like(param, memory_format=torch.contiguous_format)
    grad = param.grad
    if grad.dtype != torch.float32 or not grad.is_contiguous():
        raise ValueError("Fused execution accumulates into contiguous FP32 .grad buffers")
    return grad


class _NormProjection(torch.autograd.Function):
    """P = r(RMSNorm(x) @ W^T) with r(sigmoid) on the gate columns, for x [rows, d] BF16,
    the FP32 norm weight [d] and the FP32 master W [n, d]."""

    @staticmethod
    def forward(ctx, x, norm_weight, weight, eps, gate):
        w = weight.to(BF16)
        normed = torch.empty_like(x)
        out, rstd = fx.rmsnorm_gate_mm(x, norm_weight.contiguous(), eps, w, gate, normed=normed)
        ctx.save_for_backward(x, norm_weight, rstd, normed, w, out)
        ctx.weight, ctx.gate = weight, gate
        return out

    @staticmethod
    def backward(ctx, dout):
        x, norm_weight, rstd, normed, w, out = ctx.saved_tensors
        from ops.activation_execution import _rms_backward

        dp = fx.sigmoid_backward_cols(dout.contiguous(), out, ctx.gate)
        dy = fx.dgrad_mm(dp, w)
        if ctx.needs_input_grad[2]:
            fx.mm_accumulate_(_grad_buffer(ctx.weight), dp.T, normed, True)
        dx, dnorm = _rms_backward(x, norm_weight, rstd, dy, True)
        return dx, dnorm, None, None, None


class _ResidualProjection(torch.autograd.Function):
    """r(R + r(A @ W^T)) for A [rows, k] BF16, the FP32 master W [n, k] and R [rows, n]."""

    @staticmethod
    def forward(ctx, a, weight, residual):
        w = weight.to(BF16)
        ctx.save_for_backward(a, w)
        ctx.weight = weight
        return fx.residual_mm(a, w, residual)

    @staticmethod
    def backward(ctx, dout):
        a, w = ctx.saved_tensors
        dout = dout.contiguous()
        if ctx.needs_input_grad[1]:
            fx.mm_accumulate_(_grad_buffer(ctx.weight), dout.T, a, True)
        return fx.dgrad_mm(dout, w) if ctx.needs_input_grad[0] else None, None, dout


class _SwiGLUBlock(torch.autograd.Function):
    """R + down(silu(gate) * up) with (up | gate) = h @ W_upgate^T, in two launches (the
    paired projection with the SwiGLU epilogue, then the down projection with the residual
    epilogue), eager BF16 rounding throughout."""

    @staticmethod
    def forward(ctx, h, w_upgate, w_down, residual):
        from ops.matmul_epilogue import launch_swiglu_mm

        wug, wd = w_upgate.to(BF16), w_down.to(BF16)
        packed, act = launch_swiglu_mm(h, wug.T, "tiled", (128, 128, 32, 8, 3), True)
        ctx.save_for_backward(h, wug, wd, packed, act)
        ctx.weights = (w_upgate, w_down)
        return fx.residual_mm(act, wd, residual)

    @staticmethod
    def backward(ctx, dout):
        h, wug, wd, packed, act = ctx.saved_tensors
        w_upgate, w_down = ctx.weights
        dout = dout.contiguous()
        dpacked = fx.swiglu_backward_mm(dout, wd, packed, True)
        groups = []
        if ctx.needs_input_grad[2]:
            groups.append((_grad_buffer(w_down), dout.T, act))
        if ctx.needs_input_grad[1]:
            groups.append((_grad_buffer(w_upgate), dpacked.T, h))
        fx.mm_accumulate_group_(groups, True)
        dh = fx.dgrad_mm(dpacked, wug) if ctx.needs_input_grad[0] else None
        return dh, None, None, dout


def _core_eligible(core, x: torch.Tensor) -> bool:
    return (bf16_autocast_training(core, x) and x.dtype == BF16 and x.numel() > 0
            and all(m.bias is None for m in (core.in_proj, core.out_proj, core.ffn.up_gate,
                                             core.ffn.down)))


def _fused_core_forward(core, x: torch.Tensor) -> torch.Tensor:
    """One core on rows of the BF16 residual stream: the same rounding points as the
    eager forward under BF16 autocast, in five launches plus the mixer."""
    from ops.activation_execution import bf16_rmsnorm

    d = core.in_proj.in_features
    rows = x.reshape(-1, d).contiguous()
    p = _NormProjection.apply(rows, core.norm1.weight, core.in_proj.weight,
                              float(core.norm1.eps), (3 * d, 4 * d))
    q, k, v, gate, u = p.view(*x.shape[:-1], 5 * d).chunk(5, dim=-1)
    mixed = core.mix(q, k, v, gate, u).reshape(-1, d).to(BF16).contiguous()
    rows = _ResidualProjection.apply(mixed, core.out_proj.weight, rows)
    h, _rstd = bf16_rmsnorm(rows, core.norm2.weight, float(core.norm2.eps), True)
    rows = _SwiGLUBlock.apply(h, core.ffn.up_gate.weight, core.ffn.down.weight, rows)
    return rows.view(x.shape)


def apply_fused_execution(model: torch.nn.Module) -> None:
    """Patch every core of ``model.cores`` and the model's ``chunked_loss``; apply once,
    to a model with FP32 master parameters, before compiling or wrapping it."""
    if getattr(model, "_fused_execution", False):
        raise ValueError("Fused execution has already been applied")
    if any(p.dtype != torch.float32 for p in model.parameters()):
        raise ValueError("Fused execution requires FP32 master parameters")
    for core in model.cores:
        original = core.forward

        def core_forward(x, _core=core, _original=original):
            if _core_eligible(_core, x):
                return _fused_core_forward(_core, x)
            return _original(x)

        core.forward = core_forward
    original_loss = model.chunked_loss

    def chunked_loss(x, targets):
        if not bf16_autocast_training(model, x):
            return original_loss(x, targets)
        mean, _per_token = fx.linear_cross_entropy(x.reshape(-1, x.shape[-1]),
                                                   model.embed.weight, targets.reshape(-1))
        return mean

    model.chunked_loss = chunked_loss
    model._fused_execution = True
