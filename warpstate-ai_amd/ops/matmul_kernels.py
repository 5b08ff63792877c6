"""BF16 matrix kernels for MI355X (gfx950); autograd and policy selection belong to callers.

Call surface of WarpState's ``ops/matmul_kernels.py`` (tile tuples, dispatch signatures,
``launch_mm`` and the ``warpstate::persistent_tma_mm`` operator), backed by hand-written
HIP kernels in ``libwarpstate_hip.so`` instead of Triton. Kernels accumulate in FP32 on the
MFMA units and return BF16; ``aten`` keeps the process's BLAS (``torch.mm``).

Algorithms (ops/matmul_kernels.py:19):
  * ``tiled``: one workgroup per output tile;
  * ``persistent``: one resident workgroup per CU slot, striding over tiles;
  * ``persistent_tma``: the persistent kernel under the reference's TMA preconditions
    (unit inner stride, 16-byte rows and offsets), which it keeps as errors.

Tiles keep the reference's five-field form and validation. On this hardware the
(block_m, block_n) request picks the macro-tile: at least 128x128 outputs select the
256x256 eight-wave tile, smaller requests the 128x128 four-wave tile; block_k, warps and
stages are validated and recorded but the kernels use BK=64 with an LDS double buffer.
"""

from collections.abc import Mapping
import json

import torch

from ops import _hip

ALGORITHMS = ("aten", "tiled", "persistent", "persistent_tma")
TILE_FIELDS = ("block_m", "block_n", "block_k", "num_warps", "num_stages")
DEFAULT_TILE = (128, 128, 32, 4, 3)
TUNING_TILES = (
    (64, 128, 64, 4, 3),
    DEFAULT_TILE,
    (128, 256, 32, 8, 3),
    (256, 128, 32, 8, 3),
    (128, 128, 64, 4, 2),
)
_SHARED_BUDGET = 96 * 1024


def normalize_tile(tile=None):
    """Validate a five-integer tile tuple or named JSON object (ops/matmul_kernels.py:31-50)."""
    if tile is None:
        tile = DEFAULT_TILE
    if isinstance(tile, Mapping):
        if set(tile) != set(TILE_FIELDS):
            raise ValueError("Tile must contain exactly " + ", ".join(TILE_FIELDS))
        tile = tuple(tile[field] for field in TILE_FIELDS)
    if not isinstance(tile, (tuple, list)) or len(tile) != 5:
        raise ValueError("Tile must be (block_m, block_n, block_k, num_warps, num_stages)")
    if any(type(value) is not int for value in tile):
        raise ValueError("Tile values must be integers")
    block_m, block_n, block_k, warps, stages = tile
    for value in (block_m, block_n, block_k):
        if value < 16 or value > 256 or value & (value - 1):
            raise ValueError("Matrix tile dimensions must be powers of two between 16 and 256")
    if warps not in (4, 8) or stages not in (1, 2, 3, 4):
        raise ValueError("Supported launch settings are 4/8 warps and 1–4 stages")
    if (block_m + block_n) * block_k * 2 * stages > _SHARED_BUDGET:
        raise ValueError("BF16 operand pipeline exceeds the conservative 96 KiB shared-memory budget")
    return (block_m, block_n, block_k, warps, stages)


def tile_dict(tile):
    return dict(zip(TILE_FIELDS, normalize_tile(tile), strict=True))


def matrix_signature(a, b):
    """Serializable dispatch signature (ops/matmul_kernels.py:57-65)."""
    if a.ndim != 2 or b.ndim != 2 or a.shape[1] != b.shape[0]:
        raise ValueError("Expected compatible two-dimensional matrix operands")
    if a.dtype != b.dtype:
        raise ValueError("Matrix operands must have matching dtypes")
    return {"m": a.shape[0], "n": b.shape[1], "k": a.shape[1],
            "a_stride": list(a.stride()), "b_stride": list(b.stride()),
            "dtype": str(a.dtype).removeprefix("torch.")}


def policy_key(a, b):
    return json.dumps(matrix_signature(a, b), sort_keys=True, separators=(",", ":"))


def _launch(a, b, algorithm, tile):
    """Run the HIP GEMM on the current stream into a new row-contiguous BF16 output.

    An N-contiguous B (the weight of an input-gradient GEMM) is first copied to a
    K-contiguous layout when A's rows amortize the copy; the product is unchanged."""
    from ops.fused_execution import k_contiguous_b

    block_m, block_n = tile[0], tile[1]
    if _hip.tile_code(block_m, block_n) == 0:
        b = k_contiguous_b(b, a.shape[0])
    m, k = a.shape
    n = b.shape[1]
    output = torch.empty((m, n), device=a.device, dtype=torch.bfloat16)
    _hip.call("ws_mm", a.data_ptr(), a.stride(0), a.stride(1), b.data_ptr(), b.stride(0),
              b.stride(1), output.data_ptr(), m, n, k, _hip.algorithm_code(algorithm),
              _hip.tile_code(block_m, block_n), _hip.stream(a))
    return output


@torch.library.custom_op("warpstate::persistent_tma_mm", mutates_args=())
def _tma_mm(a: torch.Tensor, b: torch.Tensor, bm: int, bn: int, bk: int,
            warps: int, stages: int) -> torch.Tensor:
    """Opaque launch boundary of the persistent aligned-operand kernel
    (ops/matmul_kernels.py:135-159)."""
    return _launch(a, b, "persistent_tma", (bm, bn, bk, warps, stages))


@_tma_mm.register_fake
def _tma_mm_fake(a, b, bm, bn, bk, warps, stages):
    return torch.empty((a.shape[0], b.shape[1]), device=a.device, dtype=torch.bfloat16)


def launch_mm(a, b, algorithm="aten", tile=None):
    """Return BF16 ``a @ b`` on the GPU; caller supplies any autograd registration.

    Supports positive 2D strides, including ordinary transposed weights and transposed
    output gradients. No inputs are modified (ops/matmul_kernels.py:167-205).
    """
    if algorithm not in ALGORITHMS:
        raise ValueError("Unknown matrix algorithm: " + str(algorithm))
    if a.ndim != 2 or b.ndim != 2 or a.shape[1] != b.shape[0]:
        raise ValueError("Expected compatible two-dimensional matrix operands")
    if a.device != b.device or not a.is_cuda:
        raise ValueError("Matrix kernels require operands on the same CUDA device")
    if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
        raise ValueError("Matrix kernels require BF16 inputs")
    if min(a.shape[0], a.shape[1], b.shape[1]) < 1 or min(*a.stride(), *b.stride()) < 1:
        raise ValueError("Matrix kernels require positive dimensions and strides")
    if algorithm == "aten":
        return torch.mm(a, b)
    tile = normalize_tile(tile)
    if algorithm == "persistent_tma":
        if (min(a.stride()) != 1 or min(b.stride()) != 1
                or max(a.stride()) * 2 % 16 or max(b.stride()) * 2 % 16):
            raise ValueError("TMA operands require an innermost stride of one and 16-byte-aligned rows")
        if a.storage_offset() * 2 % 16 or b.storage_offset() * 2 % 16:
            raise ValueError("TMA operands require 16-byte-aligned storage offsets")
        return _tma_mm(a, b, *tile)
    return _launch(a, b, algorithm, tile)
