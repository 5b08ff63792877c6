"""CPU restatement of the packed attention-backward gradient layout -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` may import this module, as the checker; no product code path calls it.
It restates the arithmetic of the reference's fused layout kernels
(ops/backward_layout.py:116-186, the two-stage profile kernels of
ops/backward_layout_baseline.py:25-104 and :107-201 compute the same values) in numpy
FP32 with an exactly rounded FP32 fused multiply-add, so a GPU result can be checked bit
for bit. The reference compiles those kernels with FP contraction on; the contracted
pairs used here are the four multiply-adds whose product has a single use:

  q_e = fma(q_e, cos_e, r(q_o sin_o) + 0)          q = q_memory + q_local
  q_o = fma(q_o, cos_o, r(-q_e sin_e) + 0)
  k   = fma(k_write, fma(-tanh_k, tanh_k, 1), k_local)
  k_e = fma(k_e, cos_e, bf16(r(k_o sin_o) + 0))    k_o likewise with -k_e sin_e
  gate = r(fma(dy, local, -r(dy r(memory scale))) r(gate r(1 - gate)))
  u   = r(u_write fma(-tanh_u, tanh_u, 1))

with (e, o) = (2i, 2i + 1) a rotary lane pair, r() FP32 rounding, and every section
rounded to BF16 (nearest-even) on output.

Pinning (tests/test_layout_oracle.py): ``fma32`` against exact rational arithmetic and
Dekker's exact product error; the layout against the reference's own CPU tests
(test_backward_layout.py:16-65: pair direction and packing, the RoPE vector-Jacobian
product through autograd, the observable BF16 rounding of the key's half-term, the gate
derivative through autograd, u packing) and against the independent eager expression
within the reference's tolerance. Parity unpinned: which multiply-adds the CUDA compiler
actually contracts in the reference's kernels (no CUDA toolchain or device here); the
choice above is the one whose products each have a single use.
"""

from __future__ import annotations

import numpy as np
import torch


def _f32(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32)


def fma32(a, b, c) -> np.ndarray:
    """Correctly rounded FP32 a * b + c (round to nearest even).

    a * b is exact in float64 (two 24-bit significands); the float64 sum s = RN64(ab + c)
    then differs from the exact sum by an error e that TwoSum recovers exactly. Rounding s
    to FP32 gives the correctly rounded result unless s lies exactly halfway between two
    FP32 values while e != 0; then the exact sum lies on e's side of the midpoint."""
    a64, b64, c64 = (np.asarray(v, dtype=np.float32).astype(np.float64) for v in (a, b, c))
    p = a64 * b64
    s = p + c64
    bb = s - p
    e = (p - (s - bb)) + (c64 - bb)
    r = s.astype(np.float32)
    r64 = r.astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        toward = np.where(s > r64, np.float32(np.inf), np.float32(-np.inf)).astype(np.float32)
        other = np.nextafter(r, toward)
        mid = (r64 + other.astype(np.float64)) * 0.5
        tie = (s == mid) & (e != 0) & np.isfinite(s)
        up = np.maximum(r, other)
        down = np.minimum(r, other)
    return np.where(tie, np.where(e > 0, up, down), r).astype(np.float32)


def _bf16(x: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16)


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().to("cpu", torch.float32).numpy()


def _plus_zero(x: np.ndarray) -> np.ndarray:
    return (x + np.float32(0.0)).astype(np.float32)


def _rotary(v: np.ndarray, cos: np.ndarray, sin: np.ndarray, round_half: bool) -> np.ndarray:
    """fma(v, cos, half) with half_e = r(v_o sin_o) + 0, half_o = r(-v_e sin_e) + 0, the
    half-term optionally rounded to BF16 first."""
    half = np.empty_like(v)
    half[..., 0::2] = _plus_zero(v[..., 1::2] * sin[..., 1::2])
    half[..., 1::2] = _plus_zero(-v[..., 0::2] * sin[..., 0::2])
    if round_half:
        half = _np(_bf16(half))
    return fma32(v, np.broadcast_to(cos, v.shape), half)


def backward_layout(inputs, scale: float | None = None) -> torch.Tensor:
    """The packed gradient [B, N*C, 5*H*D] BF16 = [q | k | v | gate | u] for a
    ``LayoutInputs``-ordered tuple of CPU tensors (ops/backward_layout.py:87-113 for the
    sections, :116-186 for the arithmetic)."""
    (q_memory, q_local, sin, cos, k_write, tanh_k, k_local, v_local, grad_y, memory, local,
     gate, u_write, tanh_u) = inputs
    b, n, h, c, d = q_memory.shape
    scale = np.float32(d ** -0.5 if scale is None else scale)
    f = {name: _np(t) for name, t in zip(
        ("qm", "ql", "sin", "cos", "kw", "tk", "kl", "dy", "mem", "loc", "gate", "uw", "tu"),
        (q_memory, q_local, sin, cos, k_write, tanh_k, k_local, grad_y, memory, local, gate,
         u_write, tanh_u))}
    q = (f["qm"] + f["ql"]).astype(np.float32)
    q_out = _rotary(q, f["cos"], f["sin"], round_half=False)
    kw = np.swapaxes(f["kw"], -1, -2)
    k = fma32(kw, fma32(-f["tk"], f["tk"], np.float32(1.0)), f["kl"])
    k_out = _rotary(k, f["cos"], f["sin"], round_half=True)
    dy = f["dy"].reshape(b, n, c, h, d).transpose(0, 1, 3, 2, 4)
    scaled = (dy * (f["mem"] * scale).astype(np.float32)).astype(np.float32)
    pre = fma32(dy, f["loc"], -scaled)
    gate_out = (pre * (f["gate"] * (np.float32(1.0) - f["gate"]))).astype(np.float32)
    u_out = (f["uw"] * fma32(-f["tu"], f["tu"], np.float32(1.0))).astype(np.float32)

    def token_major(x: torch.Tensor) -> torch.Tensor:
        return x.transpose(2, 3).reshape(b, n * c, h * d)

    sections = [_bf16(q_out), _bf16(k_out), v_local.to("cpu"), _bf16(gate_out), _bf16(u_out)]
    return torch.cat([token_major(x) for x in sections], dim=-1)
