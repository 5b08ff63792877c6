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
  cross-entropy (``linear_cross_entropy``), which never holds the full [rows, vocab]
  logits in HBM (one row chunk's BF16 logits at a time in its one-pass mode).

Each core piece is a registered operator (``warpstate::fused_norm_projection``,
``warpstate::fused_residual_projection``, ``warpstate::fused_swiglu_block``) with a fake
implementation and an autograd formula whose backward is another operator, so the patched
core compiles with ``torch.compile(fullgraph=True)`` as the reference compiles its cores
(run_40b.py:430-438). The backward operators are built from the fused backward kernels
(the gate-sigmoid backward, the SwiGLU backward fused on the dAct GEMM, the RMSNorm
backward) and ``dgrad_mm`` for the input gradients. A projection weight's gradient is
f32(r(dY^T X)) from the FP32-accumulating GEMM (the MLP's two in one grouped launch),
returned through autograd like the reference's BF16 dW (test_gradient_execution.py:243-246):
autograd's accumulation into the FP32 master's ``.grad``, and any gradient hook (DDP's),
see it as usual.

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
F32 = torch.float32
Tensor = torch.Tensor
custom_op = torch.library.custom_op


# --- norm1 -> in_proj -> gate sigmoid ------------------------------------------------------

@custom_op("warpstate::fused_norm_projection", mutates_args=())
def fused_norm_projection(x: Tensor, norm_weight: Tensor, weight: Tensor, eps: float,
                          gate_begin: int, gate_end: int
                          ) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """(P, rstd, y, W_bf16) for rows x [rows, d] BF16, the FP32 norm weight [d] and the
    FP32 master W [n, d]: y = RMSNorm(x) in BF16, P = r(y @ W^T) with r(sigmoid) on columns
    [gate_begin, gate_end). y and the BF16 weight are kept for the backward."""
    w = weight.to(BF16)
    normed = torch.empty_like(x)
    out, rstd = fx.rmsnorm_gate_mm(x, norm_weight.contiguous(), eps, w, (gate_begin, gate_end),
                                   normed=normed)
    return out, rstd, normed, w


@fused_norm_projection.register_fake
def _norm_projection_fake(x, norm_weight, weight, eps, gate_begin, gate_end):
    return (x.new_empty((x.shape[0], weight.shape[0])), x.new_empty((x.shape[0],), dtype=F32),
            torch.empty_like(x), weight.new_empty(weight.shape, dtype=BF16))


@custom_op("warpstate::fused_norm_projection_backward", mutates_args=())
def fused_norm_projection_backward(dout: Tensor, x: Tensor, norm_weight: Tensor, rstd: Tensor,
                                   normed: Tensor, w: Tensor, out: Tensor, gate_begin: int,
                                   gate_end: int) -> tuple[Tensor, Tensor, Tensor]:
    """(dx, d norm_weight, dW): dP through the gate sigmoid, dy = r(dP @ W),
    dW = f32(r(dP^T y)), then the RMSNorm backward with the saved rstd."""
    from ops.activation_execution import _rms_backward

    dp = fx.sigmoid_backward_cols(dout.contiguous(), out, (gate_begin, gate_end))
    dy = fx.dgrad_mm(dp, w)
    dw = torch.zeros(w.shape, dtype=F32, device=w.device)
    fx.mm_accumulate_(dw, dp.T, normed, True)
    dx, dnorm = _rms_backward(x, norm_weight, rstd, dy, True)
    return dx, dnorm, dw


@fused_norm_projection_backward.register_fake
def _norm_projection_backward_fake(dout, x, norm_weight, rstd, normed, w, out, gate_begin,
                                   gate_end):
    return (torch.empty_like(x), norm_weight.new_empty(norm_weight.shape, dtype=F32),
            w.new_empty(w.shape, dtype=F32))


def _norm_projection_setup(ctx, inputs, output):
    x, norm_weight, _weight, _eps, gate_begin, gate_end = inputs
    out, rstd, normed, w = output
    ctx.save_for_backward(x, norm_weight, rstd, normed, w, out)
    ctx.gate = (gate_begin, gate_end)


def _norm_projection_autograd(ctx, dout, _drstd, _dnormed, _dw):
    x, norm_weight, rstd, normed, w, out = ctx.saved_tensors
    dx, dnorm, dweight = fused_norm_projection_backward(dout, x, norm_weight, rstd, normed, w,
                                                        out, *ctx.gate)
    return dx, dnorm, dweight, None, None, None


fused_norm_projection.register_autograd(_norm_projection_autograd,
                                        setup_context=_norm_projection_setup)


# --- projection + residual -----------------------------------------------------------------

@custom_op("warpstate::fused_residual_projection", mutates_args=())
def fused_residual_projection(a: Tensor, weight: Tensor, residual: Tensor
                              ) -> tuple[Tensor, Tensor]:
    """(r(R + r(A @ W^T)), W_bf16) for A [rows, k] BF16, the FP32 master W [n, k] and the
    BF16 residual R [rows, n]."""
    w = weight.to(BF16)
    return fx.residual_mm(a, w, residual), w


@fused_residual_projection.register_fake
def _residual_projection_fake(a, weight, residual):
    return torch.empty_like(residual), weight.new_empty(weight.shape, dtype=BF16)


@custom_op("warpstate::fused_residual_projection_backward", mutates_args=())
def fused_residual_projection_backward(dout: Tensor, a: Tensor, w: Tensor
                                       ) -> tuple[Tensor, Tensor]:
    """(dA, dW): dA = r(dOut @ W), dW = f32(r(dOut^T A))."""
    dout = dout.contiguous()
    dw = torch.zeros(w.shape, dtype=F32, device=w.device)
    fx.mm_accumulate_(dw, dout.T, a, True)
    return fx.dgrad_mm(dout, w), dw


@fused_residual_projection_backward.register_fake
def _residual_projection_backward_fake(dout, a, w):
    return torch.empty_like(a), w.new_empty(w.shape, dtype=F32)


def _residual_projection_setup(ctx, inputs, output):
    a, _weight, _residual = inputs
    ctx.save_for_backward(a, output[1])


def _residual_projection_autograd(ctx, dout, _dw):
    a, w = ctx.saved_tensors
    da, dweight = fused_residual_projection_backward(dout, a, w)
    return da, dweight, dout


fused_residual_projection.register_autograd(_residual_projection_autograd,
                                            setup_context=_residual_projection_setup)


# --- SwiGLU block + residual ---------------------------------------------------------------

@custom_op("warpstate::fused_swiglu_block", mutates_args=())
def fused_swiglu_block(h: Tensor, w_upgate: Tensor, w_down: Tensor, residual: Tensor
                       ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(R + down(silu(gate) * up), packed, act, W_upgate_bf16, W_down_bf16) with
    (up | gate) = h @ W_upgate^T: the paired projection with the SwiGLU epilogue, then the
    down projection with the residual epilogue, eager BF16 rounding throughout. The paired
    projection runs on the persistent grid (the same bits as the tiled one, 2-4 % faster at
    the layer's shapes)."""
    from ops.matmul_epilogue import launch_swiglu_mm

    wug, wd = w_upgate.to(BF16), w_down.to(BF16)
    packed, act = launch_swiglu_mm(h, wug.T, "persistent", (128, 128, 32, 8, 3), True)
    return fx.residual_mm(act, wd, residual), packed, act, wug, wd


@fused_swiglu_block.register_fake
def _swiglu_block_fake(h, w_upgate, w_down, residual):
    rows, two_h = h.shape[0], w_upgate.shape[0]
    return (torch.empty_like(residual), h.new_empty((rows, two_h)),
            h.new_empty((rows, two_h // 2)), w_upgate.new_empty(w_upgate.shape, dtype=BF16),
            w_down.new_empty(w_down.shape, dtype=BF16))


@custom_op("warpstate::fused_swiglu_block_backward", mutates_args=())
def fused_swiglu_block_backward(dout: Tensor, h: Tensor, packed: Tensor, act: Tensor,
                                wug: Tensor, wd: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """(dh, dW_upgate, dW_down): dPacked from the dAct GEMM with the SwiGLU backward in its
    epilogue, both weight gradients in one grouped FP32-accumulating launch, and
    dh = r(dPacked @ W_upgate)."""
    dout = dout.contiguous()
    dpacked = fx.swiglu_backward_mm(dout, wd, packed, True)
    g_upgate = torch.zeros(wug.shape, dtype=F32, device=wug.device)
    g_down = torch.zeros(wd.shape, dtype=F32, device=wd.device)
    fx.mm_accumulate_group_([(g_down, dout.T, act), (g_upgate, dpacked.T, h)], True)
    return fx.dgrad_mm(dpacked, wug), g_upgate, g_down


@fused_swiglu_block_backward.register_fake
def _swiglu_block_backward_fake(dout, h, packed, act, wug, wd):
    return (torch.empty_like(h), wug.new_empty(wug.shape, dtype=F32),
            wd.new_empty(wd.shape, dtype=F32))


def _swiglu_block_setup(ctx, inputs, output):
    _out, packed, act, wug, wd = output
    ctx.save_for_backward(inputs[0], packed, act, wug, wd)


def _swiglu_block_autograd(ctx, dout, _dpacked, _dact, _dwug, _dwd):
    h, packed, act, wug, wd = ctx.saved_tensors
    dh, g_upgate, g_down = fused_swiglu_block_backward(dout, h, packed, act, wug, wd)
    return dh, g_upgate, g_down, dout


fused_swiglu_block.register_autograd(_swiglu_block_autograd, setup_context=_swiglu_block_setup)


# --- the adapter ---------------------------------------------------------------------------

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
    p = fused_norm_projection(rows, core.norm1.weight, core.in_proj.weight,
                              float(core.norm1.eps), 3 * d, 4 * d)[0]
    q, k, v, gate, u = p.view(*x.shape[:-1], 5 * d).chunk(5, dim=-1)
    mixed = core.mix(q, k, v, gate, u).reshape(-1, d).to(BF16).contiguous()
    rows = fused_residual_projection(mixed, core.out_proj.weight, rows)[0]
    h, _rstd = bf16_rmsnorm(rows, core.norm2.weight, float(core.norm2.eps), True)
    rows = fused_swiglu_block(h, core.ffn.up_gate.weight, core.ffn.down.weight, rows)[0]
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
