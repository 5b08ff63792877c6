"""BF16 paired FFN projections with a SwiGLU epilogue, on gfx950.

Call surface of WarpState's ``ops/matmul_epilogue.py``. The training adapter owns autograd
and keeps the FP32 master parameters. Both projection halves are rounded to BF16 before the
activation, and the packed projection is returned for the backward pass, so fusing saves a
projection read, not its storage (ops/matmul_epilogue.py:1-7).

The HIP kernel stages one A panel and the two weight panels (up columns j, gate columns
H + j) of each output tile in LDS, accumulates both halves in FP32 on the MFMA units, and in
registers rounds both to BF16, stores them into the packed output, applies
g / (1 + e^-g) to the rounded gate, optionally rounds it (``eager_rounding``) and stores
r(silu * up).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from ops import _hip

SUPPORTED_TILES = (
    (64, 64, 32, 4, 3),
    (64, 64, 64, 4, 2),
    (128, 64, 32, 8, 3),
    (64, 128, 32, 8, 3),
    (128, 64, 32, 4, 3),
    (64, 128, 32, 4, 3),
    (128, 128, 32, 8, 3),
)


def launch_swiglu_mm(a: torch.Tensor, b: torch.Tensor, algorithm: str = "tiled",
                     tile=SUPPORTED_TILES[0], eager_rounding: bool = False
                     ) -> tuple[torch.Tensor, torch.Tensor]:
    """Return packed ``a @ b`` and SwiGLU, both BF16 and row-contiguous.

    ``a`` has shape [M,K], ``b`` [K,2H] with up in columns [0,H) and gate in [H,2H).
    Positive-stride layouts are supported. ``tile`` is (block_m, block_n, block_k,
    num_warps, num_stages) with block_n counting columns of *each* half.
    ``eager_rounding`` controls only the BF16 rounding of the SiLU output before the
    multiply; the projection rounding always remains. ``aten`` is the reference execution
    with the same rounding choices (ops/matmul_epilogue.py:86-142).
    """
    from ops.matmul_kernels import normalize_tile

    if algorithm not in ("aten", "tiled", "persistent"):
        raise ValueError(f"Unknown SwiGLU matmul algorithm: {algorithm}")
    if a.ndim != 2 or b.ndim != 2 or a.shape[1] != b.shape[0]:
        raise ValueError("SwiGLU matmul expects compatible [M,K] and [K,2H] matrices")
    if min(a.shape) <= 0 or b.shape[1] <= 0 or b.shape[1] % 2:
        raise ValueError("SwiGLU matmul requires positive dimensions and an even packed width")
    if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
        raise ValueError("SwiGLU matmul requires BF16 operands")
    if a.device != b.device or any(stride <= 0 for tensor in (a, b) for stride in tensor.stride()):
        raise ValueError("SwiGLU matmul requires the same device and positive strides")
    block_m, block_n, block_k, _warps, stages = normalize_tile(tile)
    if (block_m + 2 * block_n) * block_k * 2 * stages > 96 * 1024:
        raise ValueError("Paired SwiGLU tile exceeds the conservative 96 KiB shared-memory budget")
    if algorithm == "aten":
        packed = torch.mm(a, b)
        up, gate = packed.chunk(2, dim=-1)
        if eager_rounding:
            output = F.silu(gate) * up
        else:
            output = (F.silu(gate.float()) * up.float()).to(torch.bfloat16)
        return packed, output
    if a.device.type != "cuda":
        raise ValueError("Custom SwiGLU matmul kernels require CUDA")
    rows, reduction = a.shape
    hidden = b.shape[1] // 2
    tile_code = _hip.tile_code(block_m, 2 * block_n)
    if tile_code == 0:
        # A weight given as a row-major [K, 2H] B (N-contiguous) is copied K-contiguous
        # first: the 256 x 256 paired kernel reads it 10-15 % faster that way.
        from ops.fused_execution import k_contiguous_b

        b = k_contiguous_b(b, rows)
    packed = torch.empty((rows, 2 * hidden), dtype=torch.bfloat16, device=a.device)
    output = torch.empty((rows, hidden), dtype=torch.bfloat16, device=a.device)
    # block_n counts one half, so the paired request covers block_m x 2*block_n outputs.
    _hip.call("ws_swiglu_mm", a.data_ptr(), a.stride(0), a.stride(1), b.data_ptr(),
              b.stride(0), b.stride(1), packed.data_ptr(), output.data_ptr(), rows, hidden,
              reduction, int(eager_rounding), _hip.algorithm_code(algorithm), tile_code,
              _hip.stream(a))
    return packed, output
