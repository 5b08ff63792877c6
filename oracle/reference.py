"""CPU restatement of WarpState's BF16 matmul hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import
this module, and only as the checker (or the timed CPU baseline); no product code path
calls it. Every function runs PyTorch CPU operators on BF16 / FP32 CPU tensors at the
rounding points of the reference's eager ``aten`` path (cited per function, paths relative
to gtausa197-svg/WarpState-AI). ``r(.)`` below is round-to-nearest-even to BF16.

Pinning (tests/test_oracle.py): each function is checked against closed forms, special
cases and a float64 brute force with an independent integer-arithmetic BF16 rounding
(tests/golden/bf16_numpy.py) on small inputs, plus the known-answer fixtures in
tests/golden/. The reference ships no stored vectors; its own tests pin self-consistency
(their fixtures are seeded closed-form comparisons), which these checks restate.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

BF16 = torch.bfloat16
F32 = torch.float32


def mm(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """C = r(sum_k f32(a) f32(b)): the ``aten`` branch of launch_mm
    (ops/matmul_kernels.py:185-186), torch.mm on BF16 CPU tensors."""
    return torch.mm(a, b)


def mm_f32_reference(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """The FP32-dot reference the reference's tests compare against,
    r(f32(a) @ f32(b)) (test_matmul_epilogue.py:76)."""
    return (a.float() @ b.float()).to(BF16)


def swiglu_mm(a: torch.Tensor, b: torch.Tensor, eager_rounding: bool) -> tuple[torch.Tensor, torch.Tensor]:
    """(packed, act) of launch_swiglu_mm's ``aten`` path (ops/matmul_epilogue.py:119-126):
    packed = r(a @ b); up, gate = halves; act = F.silu(gate) * up in BF16 when eager,
    else r(silu(f32 gate) * f32 up)."""
    packed = torch.mm(a, b)
    up, gate = packed.chunk(2, dim=-1)
    if eager_rounding:
        act = F.silu(gate) * up
    else:
        act = (F.silu(gate.float()) * up.float()).to(BF16)
    return packed, act


def swiglu(packed: torch.Tensor, eager_rounding: bool) -> torch.Tensor:
    """SwiGLU of a packed projection (ops/activation_execution.py:22-33)."""
    up, gate = packed.chunk(2, dim=-1)
    if eager_rounding:
        return F.silu(gate) * up
    return (F.silu(gate.float()) * up.float()).to(BF16)


def swiglu_backward(packed: torch.Tensor, grad: torch.Tensor, eager_rounding: bool) -> torch.Tensor:
    """(dUp | dGate) of SwiGLU (ops/activation_execution.py:36-55).

    Eager: autograd of ``F.silu(gate) * up`` on BF16 tensors (warpstate/model.py:59-60),
    i.e. dUp = r(dy r(silu(g))), dGate = r(r(dy up) sig(g) (1 + g (1 - sig(g)))).
    Compiled arithmetic (not eager): the same expressions in FP32 without the inner casts.
    """
    if eager_rounding:
        source = packed.detach().clone().requires_grad_(True)
        up, gate = source.chunk(2, dim=-1)
        out = F.silu(gate) * up
        (result,) = torch.autograd.grad(out, source, grad)
        return result
    up, gate = (half.float() for half in packed.chunk(2, dim=-1))
    dy = grad.float()
    sig = 1.0 / (1.0 + torch.exp(-gate))
    silu = gate / (1.0 + torch.exp(-gate))
    dgate = (dy * up) * sig * (1 + gate * (1 - sig))
    return torch.cat([(dy * silu).to(BF16), dgate.to(BF16)], dim=-1)


def rms_rstd(x: torch.Tensor, eps: float) -> torch.Tensor:
    """rsqrt(mean(f32(x)^2) + eps) per row (warpstate/model.py:26-27)."""
    wide = x.float()
    return torch.rsqrt(wide.pow(2).mean(dim=-1) + eps)


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm.forward on BF16 x with FP32 weight (warpstate/model.py:25-28):
    r(r(f32(x) rstd) r(w))."""
    wide = x.float()
    wide = wide * torch.rsqrt(wide.pow(2).mean(dim=-1, keepdim=True) + eps)
    return wide.to(x.dtype) * weight.to(x.dtype)


def rmsnorm_fp32_product(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """The BF16 RMSNorm kernel without eager rounding (ops/activation_execution.py:96-110,
    ROUND = False: the compiled path): r(f32(x) rstd w), the product in FP32 and one BF16
    rounding on the store."""
    wide = x.float()
    rstd = torch.rsqrt(wide.pow(2).mean(dim=-1, keepdim=True) + eps)
    return (wide * rstd * weight.float()).to(x.dtype)


def rmsnorm_gate_projection(x, norm_weight, eps, weight, gate):
    """RMSNorm -> in_proj -> sigmoid on the gate slice
    (warpstate/model.py:120-121, :109, :174): out = r(y @ W^T) with
    out[:, gate] = r(sigmoid(out[:, gate]))."""
    y = rmsnorm(x, norm_weight, eps)
    out = torch.mm(y, weight.T)
    begin, end = gate
    if end > begin:
        out[:, begin:end] = torch.sigmoid(out[:, begin:end])
    return out


def residual_projection(h, weight, residual):
    """x + down(h) in BF16 (warpstate/model.py:178 under ops/residual_experiment.py:25-58):
    r(R + r(h @ W^T))."""
    return residual + torch.mm(h, weight.T)


def accumulate_weight_grad(g, a, b, round_bf16=True):
    """G + f32(r(a @ b)) (test_gradient_execution.py:243-246); without the BF16 rounding,
    G + f32(a) @ f32(b) (ops/benchmark_gradient_accumulation.py:141-144)."""
    if round_bf16:
        return g + torch.mm(a, b).float()
    return g + a.float() @ b.float()


def mlp_backward(x, w_upgate, w_down, packed, act, dy, g_upgate, g_down, eager_rounding=True):
    """Backward of down(silu(gate) * up) as the reference's registered autograd composes it
    (ops/matmul_execution.py:236-244, :314-319): dAct = r(dY @ W_down),
    dPacked = SwiGLU backward, dX = r(dPacked @ W_upgate), and FP32 accumulation
    G += f32(r(dW)). Returns (dX, dPacked, G_upgate', G_down')."""
    dact = torch.mm(dy, w_down)
    dpacked = swiglu_backward(packed, dact, eager_rounding)
    dx = torch.mm(dpacked, w_upgate)
    g_down = accumulate_weight_grad(g_down, dy.T, act)
    g_upgate = accumulate_weight_grad(g_upgate, dpacked.T, x)
    return dx, dpacked, g_upgate, g_down


def linear_cross_entropy(hidden, weight, targets, chunk: int = 1024):
    """Tied-head loss of WarpStateLM.forward (warpstate/model.py:316-334) with
    ``_full_loss`` semantics (ops/loss_experiment.py:14-19).

    Returns (per-token loss [rows] f32, mean, valid count, dhidden [rows, d] BF16 of mean).
    Each chunk recomputes BF16 logits r(h @ W^T) and takes F.cross_entropy on their FP32
    values; ignored targets (-100) contribute 0.
    """
    hidden = hidden.detach()
    rows = hidden.shape[0]
    count = targets.ne(-100).sum().clamp_min(1)
    leaf = hidden.clone().requires_grad_(True)
    losses = []
    total = torch.zeros((), dtype=F32)
    for start in range(0, rows, chunk):
        h = leaf[start:start + chunk]
        y = targets[start:start + chunk]
        logits = F.linear(h, weight).float()
        per = F.cross_entropy(logits, y, ignore_index=-100, reduction="none")
        losses.append(per.detach())
        total = total + per.sum()
    mean = total / count
    (dhidden,) = torch.autograd.grad(mean, leaf)
    return torch.cat(losses), mean.detach(), int(targets.ne(-100).sum()), dhidden


def linear_cross_entropy_weight_grad(hidden, weight, targets, chunk: int = 1024,
                                     grad_mean: float = 1.0):
    """FP32 gradient of the mean tied-head loss with respect to the head weight
    [vocab, d], accumulated chunk by chunk as the reference's autocast path does it
    (warpstate/model.py:321-331; BF16 weight gradient per F.linear call, then FP32
    AccumulateGrad as in test_gradient_execution.py:243-246):
    dW += f32(r(G_c^T @ h_c)) with G_c = r(grad_mean (softmax - onehot) / count), zero rows
    for ignored targets.
    """
    count = max(int(targets.ne(-100).sum()), 1)
    dweight = torch.zeros(weight.shape, dtype=F32)
    with torch.no_grad():
        for start in range(0, hidden.shape[0], chunk):
            h = hidden[start:start + chunk]
            y = targets[start:start + chunk]
            logits = F.linear(h, weight).float()
            soft = torch.softmax(logits, dim=-1)
            valid = y.ne(-100)
            onehot = torch.zeros_like(soft)
            onehot[valid.nonzero().squeeze(1), y[valid]] = 1.0
            g = ((soft - onehot) * (grad_mean / count)) * valid.unsqueeze(1)
            dweight += torch.mm(g.to(BF16).T, h).float()
    return dweight


def rmsnorm_gate_projection_backward(x, norm_weight, eps, weight, gate, dout, weight_grad):
    """Backward of RMSNorm -> in_proj -> gate sigmoid (warpstate/model.py:22-28, :109,
    :174) as CPU autograd composes it on BF16 tensors, with the projection weight's BF16
    gradient accumulated into FP32 (test_gradient_execution.py:243-246).
    Returns (dx BF16, d norm_weight FP32, weight_grad').
    """
    xl = x.detach().clone().requires_grad_(True)
    wl = norm_weight.detach().clone().requires_grad_(True)
    y = rmsnorm(xl, wl, eps)
    yl = y.detach().requires_grad_(True)
    wt = weight.detach().clone().requires_grad_(True)
    p = torch.mm(yl, wt.T)
    begin, end = gate
    out = torch.cat([p[:, :begin], torch.sigmoid(p[:, begin:end]), p[:, end:]], dim=1)
    out.backward(dout)
    y.backward(yl.grad)
    return xl.grad, wl.grad, weight_grad + wt.grad.float()
