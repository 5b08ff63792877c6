"""Independent numpy restatement of the hot path's arithmetic, used to pin the oracle.

Nothing here calls torch: BF16 round-to-nearest-even is done on the integer bit patterns
of FP32 values, and the matrix products are exact float64 sums rounded once to BF16, so a
mistake in the torch-based oracle (``oracle/reference.py``) cannot be repeated here by
construction. Each function names the reference lines whose semantics it restates (paths
relative to gtausa197-svg/WarpState-AI).
"""

from __future__ import annotations

import numpy as np


# --- BF16 bit-level conversions -------------------------------------------------------

def f32_to_bf16_bits(x) -> np.ndarray:
    """FP32 -> BF16 bit pattern, round to nearest, ties to even (NaN kept quiet)."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = np.isnan(x)
    out = rounded.astype(np.uint16)
    out[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return out


def bf16_bits_to_f32(bits) -> np.ndarray:
    bits = np.ascontiguousarray(np.asarray(bits, dtype=np.uint16))
    return (bits.astype(np.uint32) << 16).view(np.float32)


def r32(x) -> np.ndarray:
    """Round FP32 values to BF16, returned as FP32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def r64(x) -> np.ndarray:
    """Round float64 values directly to BF16 (one rounding: 8 significant bits, ties to
    even), returned as float64. Finite normal range only."""
    x = np.asarray(x, dtype=np.float64)
    mant, exp = np.frexp(x)           # x = mant * 2**exp, 0.5 <= |mant| < 1
    return np.ldexp(np.rint(mant * 256.0) / 256.0, exp)


# --- Hot-path functions ------------------------------------------------------------------

def mm(a, b) -> np.ndarray:
    """r(sum_k a b) with an exact float64 sum (ops/matmul_kernels.py:81-108, the FP32-dot
    reference of test_matmul_epilogue.py:76 without accumulation error)."""
    return r64(np.asarray(a, np.float64) @ np.asarray(b, np.float64))


def silu32(g):
    g = np.asarray(g, np.float32)
    return (g / (np.float32(1) + np.exp(-g))).astype(np.float32)


def sigmoid32(x):
    x = np.asarray(x, np.float32)
    return (np.float32(1) / (np.float32(1) + np.exp(-x))).astype(np.float32)


def swiglu(packed, eager_rounding: bool) -> np.ndarray:
    """act from a BF16-valued packed projection (up | gate), warpstate/model.py:59-60 and
    ops/matmul_epilogue.py:119-126: eager r(r(silu(g)) up), else r(silu(g) up)."""
    packed = np.asarray(packed, np.float32)
    h = packed.shape[-1] // 2
    up, gate = packed[..., :h], packed[..., h:]
    s = silu32(gate)
    if eager_rounding:
        s = r32(s)
    return r32(s * up)


def swiglu_backward(packed, grad, eager_rounding: bool) -> np.ndarray:
    """(dUp | dGate), ops/activation_execution.py:36-55: dUp = r(dy s), dGate =
    r(r?(dy up) sig (1 + g (1 - sig))) with s = r?(silu(g))."""
    packed = np.asarray(packed, np.float32)
    dy = np.asarray(grad, np.float32)
    h = packed.shape[-1] // 2
    up, gate = packed[..., :h], packed[..., h:]
    sig = sigmoid32(gate)
    s = silu32(gate)
    dsilu = dy * up
    if eager_rounding:
        s = r32(s)
        dsilu = r32(dsilu)
    dgate = (dsilu * sig) * (np.float32(1) + gate * (np.float32(1) - sig))
    return np.concatenate([r32(dy * s), r32(dgate)], axis=-1)


def rms_rstd(x, eps) -> np.ndarray:
    """1 / sqrt(mean(x^2) + eps) per row in float64 (warpstate/model.py:26-27)."""
    x = np.asarray(x, np.float64)
    return 1.0 / np.sqrt((x * x).mean(axis=-1) + eps)


def rmsnorm(x, weight, eps) -> np.ndarray:
    """r(r(x rstd) r(w)) (warpstate/model.py:25-28 on BF16 x, FP32 weight)."""
    x = np.asarray(x, np.float32)
    rstd = rms_rstd(x, eps).astype(np.float32)
    z = r32(x * rstd[:, None])
    return r32(z * r32(np.asarray(weight, np.float32)))


def rmsnorm_gate_projection(x, norm_weight, eps, weight, gate) -> np.ndarray:
    """RMSNorm -> in_proj -> sigmoid of the gate columns (warpstate/model.py:109,120-121,
    174): out = r(y W^T), out[:, gate] = r(sigmoid(out[:, gate]))."""
    y = rmsnorm(x, norm_weight, eps)
    out = mm(y, np.asarray(weight, np.float64).T).astype(np.float32)
    begin, end = gate
    out[:, begin:end] = r32(sigmoid32(out[:, begin:end]))
    return out


def residual_projection(h, weight, residual) -> np.ndarray:
    """r(R + r(h W^T)) (warpstate/model.py:178 with BF16 residuals)."""
    proj = mm(h, np.asarray(weight, np.float64).T).astype(np.float32)
    return r32(np.asarray(residual, np.float32) + proj)


def accumulate(g, a, b, round_bf16=True) -> np.ndarray:
    """G + f32(r(a b)) (test_gradient_execution.py:243-246), or G + a b without the BF16
    rounding; the sum rounds once to FP32."""
    prod = np.asarray(a, np.float64) @ np.asarray(b, np.float64)
    if round_bf16:
        prod = r64(prod)
    return (np.asarray(g, np.float64) + prod).astype(np.float32)


def linear_cross_entropy(hidden, weight, targets):
    """Per-token loss, mean over valid tokens, valid count and dHidden of the mean for the
    tied LM head (warpstate/model.py:316-334, ops/loss_experiment.py:14-19): BF16 logits
    r(h E^T) in FP32, logsumexp minus the target logit, -100 ignored;
    dh = r(r((softmax - onehot) / count) E)."""
    logits = mm(hidden, np.asarray(weight, np.float64).T)        # BF16-valued, float64
    targets = np.asarray(targets, np.int64)
    valid = targets != -100
    count = int(valid.sum())
    mx = logits.max(axis=1, keepdims=True)
    lse = (mx[:, 0] + np.log(np.exp(logits - mx).sum(axis=1)))
    safe = np.where(valid, targets, 0)
    tgt = logits[np.arange(len(targets)), safe]
    loss = np.where(valid, lse - tgt, 0.0)
    mean = loss.sum() / max(count, 1)
    soft = np.exp(logits - lse[:, None])
    soft[np.arange(len(targets)), safe] -= 1.0
    soft[~valid] = 0.0
    grad_logits = r64(soft / max(count, 1))
    dh = r64(grad_logits @ np.asarray(weight, np.float64))
    return loss, mean, count, dh
