"""Packed BF16 attention-backward gradient layout on gfx950 (isolated, not a training adapter).

The step before the input projection's backward GEMMs: from the saved per-head tensors
of one attention core, build the token-major packed gradient ``[B, N*C, 5*H*D]`` =
``[q | k | v | gate | u]`` that is the A operand of the projection's dgrad and wgrad. It
restates ops/backward_layout.py: the inverse rotary embedding of the query and key
gradients (with the key's rotated half-term rounded to BF16 first), the tanh backward of
the key and u writes, and the gate's sigmoid-weighted gradient. Only layouts and
pointwise arithmetic change; no reduction, GEMM or parameter gradient is touched.

All saved tensors are contiguous ``[batch, chunks, heads, chunk_size, head_dim]`` BF16,
except ``k_write`` ``[B, N, H, D, C]`` (transposed), ``grad_y`` ``[B, N*C, H*D]``
(token-major) and the FP32 ``sin``/``cos`` tables ``[C, D]``.
"""

from __future__ import annotations

from typing import NamedTuple

import torch

from ops import _hip

PROFILE_SHAPE = (4, 16, 32, 128, 64)
ALGORITHMS = ("profile", "paired", "single")


class LayoutInputs(NamedTuple):
    q_memory: torch.Tensor
    q_local: torch.Tensor
    sin: torch.Tensor
    cos: torch.Tensor
    k_write: torch.Tensor
    tanh_k: torch.Tensor
    k_local: torch.Tensor
    v_local: torch.Tensor
    grad_y: torch.Tensor
    memory: torch.Tensor
    local: torch.Tensor
    gate: torch.Tensor
    u_write: torch.Tensor
    tanh_u: torch.Tensor


def _expected(name: str, shape: tuple[int, ...]) -> tuple[tuple[int, ...], torch.dtype]:
    b, n, h, c, d = shape
    if name in ("sin", "cos"):
        return (c, d), torch.float32
    if name == "k_write":
        return (b, n, h, d, c), torch.bfloat16
    if name == "grad_y":
        return (b, n * c, h * d), torch.bfloat16
    return shape, torch.bfloat16


def validate_inputs(inputs: LayoutInputs, *, cuda: bool = False) -> tuple[int, ...]:
    """Shape/dtype/contiguity contract of every saved tensor (ops/backward_layout.py:41-65);
    returns (B, N, H, C, D)."""
    if not isinstance(inputs, LayoutInputs):
        raise TypeError("Expected named LayoutInputs")
    shape = tuple(inputs.q_memory.shape)
    if len(shape) != 5 or min(shape) < 1 or shape[-1] % 2:
        raise ValueError("Expected positive [B,N,H,C,D] with an even head dimension")
    device = inputs.q_memory.device
    if cuda and device.type != "cuda":
        raise ValueError("HIP layout kernels require CUDA (ROCm) tensors")
    for name, tensor in zip(inputs._fields, inputs, strict=True):
        wanted, dtype = _expected(name, shape)
        if tuple(tensor.shape) != wanted or tensor.dtype != dtype:
            raise ValueError(f"{name} must have shape {wanted} and dtype {dtype}")
        if tensor.device != device or not tensor.is_contiguous():
            raise ValueError(f"{name} must be contiguous on {device}")
    return shape


def make_inputs(shape=PROFILE_SHAPE, *, device="cpu", seed=817) -> LayoutInputs:
    """Deterministic synthetic saved tensors (ops/backward_layout.py:68-84): N(0, 0.1^2)
    BF16 values, tanh/sigmoid-range saved activations, and the model's rope tables. Draws
    happen in the reference's order, so a seed gives the reference's values."""
    from warpstate.model import rope_cos_sin

    b, n, h, c, d = shape
    gen = torch.Generator(device=device).manual_seed(seed)

    def draw(dims=shape, scale=0.1):
        return torch.randn(dims, device=device, dtype=torch.bfloat16, generator=gen) * scale

    cos, sin = rope_cos_sin(c, d, torch.device(device), torch.float32)
    q_memory, q_local = draw(), draw()
    k_write = draw((b, n, h, d, c))
    tanh_k = draw(scale=1).float().tanh().bfloat16()
    k_local, v_local = draw(), draw()
    grad_y = draw((b, n * c, h * d))
    memory, local = draw(), draw()
    gate = draw(scale=1).float().sigmoid().bfloat16()
    u_write = draw()
    tanh_u = draw(scale=1).float().tanh().bfloat16()
    return LayoutInputs(q_memory, q_local, sin, cos, k_write, tanh_k, k_local, v_local, grad_y,
                        memory, local, gate, u_write, tanh_u)


def _token_major(value: torch.Tensor) -> torch.Tensor:
    b, n, h, c, d = value.shape
    return value.transpose(2, 3).reshape(b, n * c, h * d)


def _inverse_rotary(value: torch.Tensor) -> torch.Tensor:
    """Lane pair (a, b) -> (b, -a): the transpose of rotate_half."""
    pairs = value.unflatten(-1, (-1, 2))
    return torch.stack((pairs[..., 1], -pairs[..., 0]), dim=-1).flatten(-2)


def reference_layout(inputs: LayoutInputs) -> torch.Tensor:
    """Independent eager tensor expression of all five sections with both BF16 boundaries
    (ops/backward_layout.py:87-113). Eager FP32 ops round every product separately, so
    it agrees with the kernels within a BF16 ulp, not bit for bit."""
    b, n, h, c, d = validate_inputs(inputs)
    f = {name: value.float() for name, value in zip(inputs._fields, inputs, strict=True)}
    q = f["q_memory"] + f["q_local"]
    k = f["k_write"].transpose(-2, -1) * (1 - f["tanh_k"] ** 2) + f["k_local"]
    q_out = (_inverse_rotary(q * f["sin"]) + q * f["cos"]).bfloat16()
    k_half = _inverse_rotary(k * f["sin"]).bfloat16()
    k_out = (k_half.float() + k * f["cos"]).bfloat16()
    dy = f["grad_y"].view(b, n, c, h, d).transpose(2, 3)
    gate = f["gate"]
    gate_out = ((dy * f["local"] - dy * (f["memory"] * d ** -0.5))
                * (gate * (1 - gate))).bfloat16()
    u_out = (f["u_write"] * (1 - f["tanh_u"] ** 2)).bfloat16()
    return torch.cat([_token_major(x) for x in (q_out, k_out, inputs.v_local, gate_out, u_out)],
                     dim=-1)


def _storage(tensor: torch.Tensor) -> int:
    return tensor.untyped_storage().data_ptr()


def prepare_layout(inputs: LayoutInputs, algorithm="paired", *, block=512, warps=4,
                   output=None, scratch=None):
    """Validate once and return a launch callable that allocates nothing
    (ops/backward_layout.py:213-270).

    ``block`` and ``warps`` keep the reference's accepted values; on gfx950 the kernel's
    work split is fixed (one 256-thread workgroup per head and block of up to 16 tokens),
    so they do not change the launch. The three algorithms give identical bits: "single"
    is one pass, "paired" a q/k pass then a v/gate/u pass, and "profile" the reference's
    two-kernel baseline that round-trips q and the key's rotated half-term through two
    head-major BF16 scratch tensors (PROFILE_SHAPE only, as in the reference).
    Callers must keep the inputs', output's and scratch's storage stable.
    """
    b, n, h, c, d = validate_inputs(inputs, cuda=True)
    if algorithm not in ALGORITHMS:
        raise ValueError(f"Unknown backward layout algorithm: {algorithm}")
    if block not in (128, 256, 512, 1024) or warps not in (4, 8):
        raise ValueError("Use block 128/256/512/1024 with 4/8 warps")
    shape = (b, n * c, 5 * h * d)
    device = inputs.q_memory.device
    if output is None:
        output = torch.empty(shape, dtype=torch.bfloat16, device=device)
    if (tuple(output.shape) != shape or output.dtype != torch.bfloat16
            or output.device != device or not output.is_contiguous()):
        raise ValueError("Output must be a contiguous BF16 packed gradient on the input device")
    if any(_storage(output) == _storage(value) for value in inputs):
        raise ValueError("Output may not alias a saved input")
    scratch_q = scratch_k = None
    if algorithm == "profile":
        if (b, n, h, c, d) != PROFILE_SHAPE:
            raise ValueError("The exact profiled baseline supports PROFILE_SHAPE only")
        if scratch is None:
            scratch = (torch.empty_like(inputs.q_memory), torch.empty_like(inputs.q_memory))
        if (len(scratch) != 2 or any(value.shape != inputs.q_memory.shape
                                     or value.dtype != torch.bfloat16 or value.device != device
                                     or not value.is_contiguous() for value in scratch)):
            raise ValueError("The profile baseline needs two contiguous BF16 scratch tensors")
        scratch_q, scratch_k = scratch
        taken = {_storage(value) for value in (*inputs, output)}
        if (_storage(scratch_q) in taken or _storage(scratch_k) in taken
                or _storage(scratch_q) == _storage(scratch_k)):
            raise ValueError("Scratch tensors may not alias inputs, output, or one another")
    code = ALGORITHMS.index(algorithm)
    pointers = [value.data_ptr() for value in inputs]
    extra = (output.data_ptr(), b, n, h, c, d, d ** -0.5, code, _hip.ptr(scratch_q),
             _hip.ptr(scratch_k))

    def operation():
        _hip.call("ws_backward_layout", *pointers, *extra, _hip.stream(output))
        return output

    return operation


def launch_layout(inputs: LayoutInputs, algorithm="paired", *, block=512, warps=4,
                  output=None, scratch=None) -> torch.Tensor:
    """One checked launch; timed loops should call prepare_layout once instead."""
    return prepare_layout(inputs, algorithm, block=block, warps=warps,
                          output=output, scratch=scratch)()
