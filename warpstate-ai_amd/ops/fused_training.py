"""Route a WarpState model's training step through the fused HIP GEMMs (additive adapter).

``apply_fused_execution(model)`` attaches each core at the finest boundary it offers.

A core that exposes the ``project`` / ``mix`` seams runs as a whole through three fused
operators, for eligible training calls:

* ``project``: norm1 -> in_proj -> sigmoid on the gate slice (warpstate/model.py:107-112,
  :120-121, :174) becomes one ``rmsnorm_gate_mm`` (RMSNorm row pass, projection with the
  sigmoid in its epilogue);
* the attention output projection with its residual add (warpstate/model.py:177) and
  the SwiGLU block with its residual add (warpstate/model.py:52-60, :178) become
  ``residual_mm`` and ``launch_swiglu_mm`` + ``residual_mm``.

A core in the reference's own layout (``WarpStateCore.forward`` as one method,
warpstate/model.py:114-178: ``_split`` around in_proj, the gate sigmoid and both residual
adds inline) is attached module by module: its RMSNorm modules go to the RMSNorm row
kernel, its bias-free Linear modules to this library's GEMM, and its SwiGLU module to the
paired projection with the SwiGLU epilogue plus the down GEMM. What needs the seams (the
gate sigmoid in the projection's epilogue, the residual adds in the projections'
epilogues) stays in the core's own code.

The tied-head loss (warpstate/model.py:316-334) becomes the fused cross-entropy
(``linear_cross_entropy``), which never holds the full [rows, vocab] logits in HBM (one
row chunk's BF16 logits at a time in its one-pass mode): through a ``chunked_loss`` seam,
or else by wrapping the model's forward in the style of ops/loss_experiment.py:44-52.

Every piece is a registered operator with a fake implementation and an autograd formula
whose backward is another operator, so patched cores compile with
``torch.compile(fullgraph=True)`` as the reference compiles its cores
(run_40b.py:430-438). The backward operators are built from the fused backward kernels
(the gate-sigmoid backward, the SwiGLU backward fused on the dAct GEMM, the RMSNorm
backward) and ``dgrad_mm`` for the input gradients. A projection weight's gradient is
f32(r(dY^T X)), the reference's BF16 weight gradient widened to FP32
(test_gradient_execution.py:243-246), written by the FP32 GEMM epilogue in one pass into a
fresh buffer (the MLP's two in one grouped launch) and returned through autograd:
autograd's accumulation into the FP32 master's ``.grad``, and any gradient hook (DDP's),
see it as usual.

A call is eligible in training mode with gradients on, under BF16 autocast, on CUDA; the
core operators and the RMSNorm modules also need a BF16 residual stream
(``ops.residual_experiment.apply_bf16_residuals``), and projections must be bias-free.
Everything else runs the original forwards.
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
    dw = fx.mm_f32(dp.T, normed)
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
    return fx.dgrad_mm(dout, w), fx.mm_f32(dout.T, a)


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
    g_down, g_upgate = fx.mm_f32_group([(dout.T, act), (dpacked.T, h)])
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


# --- module-level pieces (models whose cores expose no seams) --------------------------------

@custom_op("warpstate::fused_linear", mutates_args=())
def fused_linear(a: Tensor, weight: Tensor) -> tuple[Tensor, Tensor]:
    """(r(A @ W^T), W_bf16) for rows A [rows, k] BF16 and the FP32 master W [n, k]: a
    bias-free nn.Linear under BF16 autocast on this library's GEMM."""
    w = weight.to(BF16)
    return fx.mm(a, w.T), w


@fused_linear.register_fake
def _linear_fake(a, weight):
    return a.new_empty((a.shape[0], weight.shape[0])), weight.new_empty(weight.shape, dtype=BF16)


@custom_op("warpstate::fused_linear_backward", mutates_args=())
def fused_linear_backward(dout: Tensor, a: Tensor, w: Tensor) -> tuple[Tensor, Tensor]:
    """(dA, dW): dA = r(dOut @ W), dW = f32(r(dOut^T A)) written in one FP32 pass."""
    dout = dout.contiguous()
    return fx.dgrad_mm(dout, w), fx.mm_f32(dout.T, a)


@fused_linear_backward.register_fake
def _linear_backward_fake(dout, a, w):
    return torch.empty_like(a), w.new_empty(w.shape, dtype=F32)


def _linear_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[0], output[1])


def _linear_autograd(ctx, dout, _dw):
    a, w = ctx.saved_tensors
    return fused_linear_backward(dout, a, w)


fused_linear.register_autograd(_linear_autograd, setup_context=_linear_setup)


@custom_op("warpstate::fused_swiglu_mlp", mutates_args=())
def fused_swiglu_mlp(h: Tensor, w_upgate: Tensor, w_down: Tensor
                     ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(down(silu(gate) * up), packed, act, W_upgate_bf16, W_down_bf16): the SwiGLU module
    (warpstate/model.py:52-60) as the paired projection with the SwiGLU epilogue and the
    down projection, eager BF16 rounding; the caller keeps its own residual add."""
    from ops.matmul_epilogue import launch_swiglu_mm

    wug, wd = w_upgate.to(BF16), w_down.to(BF16)
    packed, act = launch_swiglu_mm(h, wug.T, "persistent", (128, 128, 32, 8, 3), True)
    return fx.mm(act, wd.T), packed, act, wug, wd


@fused_swiglu_mlp.register_fake
def _swiglu_mlp_fake(h, w_upgate, w_down):
    rows, two_h = h.shape[0], w_upgate.shape[0]
    return (h.new_empty((rows, w_down.shape[0])), h.new_empty((rows, two_h)),
            h.new_empty((rows, two_h // 2)), w_upgate.new_empty(w_upgate.shape, dtype=BF16),
            w_down.new_empty(w_down.shape, dtype=BF16))


def _swiglu_mlp_setup(ctx, inputs, output):
    _out, packed, act, wug, wd = output
    ctx.save_for_backward(inputs[0], packed, act, wug, wd)


def _swiglu_mlp_autograd(ctx, dout, _dpacked, _dact, _dwug, _dwd):
    h, packed, act, wug, wd = ctx.saved_tensors
    return fused_swiglu_block_backward(dout, h, packed, act, wug, wd)


fused_swiglu_mlp.register_autograd(_swiglu_mlp_autograd, setup_context=_swiglu_mlp_setup)


def _rows_bf16(x: Tensor) -> Tensor:
    return x.reshape(-1, x.shape[-1]).to(BF16).contiguous()


def _linear_forward(module, x, original):
    if module.bias is not None:
        return original(x)
    out = fused_linear(_rows_bf16(x), module.weight)[0]
    return out.view(*x.shape[:-1], module.out_features)


def _swiglu_forward(module, x, original):
    if module.up_gate.bias is not None or module.down.bias is not None:
        return original(x)
    out = fused_swiglu_mlp(_rows_bf16(x), module.up_gate.weight, module.down.weight)[0]
    return out.view(*x.shape[:-1], module.down.out_features)


def _rms_forward(module, x, original):
    from ops.activation_execution import bf16_rmsnorm

    if not (x.dtype == BF16 and x.is_contiguous() and 0 < x.shape[-1] <= 8192):
        return original(x)  # an FP32 residual stream keeps the original FP32 arithmetic
    return bf16_rmsnorm(x, module.weight, float(module.eps), True)[0]


class _HiddenReady(Exception):
    """Carries the final norm's output out of the model's own forward."""

    def __init__(self, hidden):
        super().__init__()
        self.hidden = hidden


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


def _attach_modules(core) -> None:
    """Module-level routing of a core without seams (the reference's WarpStateCore layout,
    warpstate/model.py:114-178): its RMSNorm modules, bias-free Linear modules and SwiGLU
    module, each for eligible calls only. The gate sigmoid and the residual adds stay inline
    in the core's forward, so they are not fused."""
    from warpstate.model import RMSNorm, SwiGLU

    from ops._patching import install_forward

    inside_swiglu = set()
    for module in core.modules():
        if isinstance(module, SwiGLU):
            install_forward(module, _swiglu_forward)
            inside_swiglu.update(id(m) for m in module.modules())
    for module in core.modules():
        if isinstance(module, RMSNorm):
            install_forward(module, _rms_forward)
        elif isinstance(module, torch.nn.Linear) and id(module) not in inside_swiglu:
            install_forward(module, _linear_forward)


def _attach_core(core) -> None:
    """Core-level routing of a core that exposes the ``project`` / ``mix`` seams: the
    RMSNorm-prologue projection with the gate sigmoid and both residual epilogues fused."""
    original = core.forward

    def core_forward(x, _core=core, _original=original):
        if _core_eligible(_core, x):
            return _fused_core_forward(_core, x)
        return _original(x)

    core.forward = core_forward


def _loss_eligible(model, input_ids: Tensor) -> bool:
    return (model.training and torch.is_grad_enabled() and input_ids.is_cuda
            and torch.is_autocast_enabled("cuda")
            and torch.get_autocast_dtype("cuda") == BF16)


def _attach_loss(model) -> None:
    """The tied-head loss through the fused cross-entropy. A model with a ``chunked_loss``
    seam has it replaced; otherwise the model's forward is wrapped in the style of
    ops/loss_experiment.py:44-52: a training call with targets and return_logits=False runs
    the model's own forward up to ``final_norm`` (a forward hook takes its output and stops
    the forward there, before the logits exist) and the fused loss on that hidden state."""
    if hasattr(model, "chunked_loss"):
        original_loss = model.chunked_loss

        def chunked_loss(x, targets):
            if not bf16_autocast_training(model, x):
                return original_loss(x, targets)
            mean, _per_token = fx.linear_cross_entropy(x.reshape(-1, x.shape[-1]),
                                                       model.embed.weight, targets.reshape(-1))
            return mean

        model.chunked_loss = chunked_loss
        return
    original_forward = model.forward

    def forward(input_ids, targets=None, *, return_logits=True):
        if targets is None or return_logits or not _loss_eligible(model, input_ids):
            return original_forward(input_ids, targets, return_logits=return_logits)

        def stop(_module, _inputs, output):
            raise _HiddenReady(output)

        handle = model.final_norm.register_forward_hook(stop)
        try:
            original_forward(input_ids, None, return_logits=True)
        except _HiddenReady as ready:
            hidden = ready.hidden
        else:
            raise RuntimeError("the model's forward did not reach final_norm")
        finally:
            handle.remove()
        mean, _per_token = fx.linear_cross_entropy(hidden.reshape(-1, hidden.shape[-1]),
                                                   model.embed.weight, targets.reshape(-1))
        return None, mean

    model.forward = forward


def apply_fused_execution(model: torch.nn.Module) -> None:
    """Route ``model``'s cores and tied-head loss through the fused kernels; apply once, to
    a model with FP32 master parameters, before compiling or wrapping it.

    Each core is attached at the finest boundary it offers: a core with the ``project`` /
    ``mix`` seams runs as a whole through the fused core operators; any other core (the
    reference's layout) has its RMSNorm, Linear and SwiGLU modules routed one by one. The
    loss replaces ``chunked_loss`` when the model has one, else wraps ``forward``."""
    if getattr(model, "_fused_execution", False):
        raise ValueError("Fused execution has already been applied")
    if any(p.dtype != torch.float32 for p in model.parameters()):
        raise ValueError("Fused execution requires FP32 master parameters")
    seams = [callable(getattr(c, "mix", None)) and callable(getattr(c, "project", None))
             for c in model.cores]
    for core, has_seams in zip(model.cores, seams):
        if has_seams:
            _attach_core(core)
        else:
            _attach_modules(core)
    if not all(seams):
        from ops._patching import install_forward

        install_forward(model.final_norm, _rms_forward)
    _attach_loss(model)
    model._fused_execution = True
