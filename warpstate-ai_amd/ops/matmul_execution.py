"""Opt-in, shape-specific BF16 matrix execution with ordinary autograd ownership, on gfx950.

Call surface of WarpState's ``ops/matmul_execution.py``: the strict JSON plan
(``warpstate-matmul-plan-v1``), exact (kind, m, n, k, strides) selection, the registered
operators ``warpstate::{selected_matrix_kernel, planned_mm, selected_swiglu_kernel,
selected_swiglu_gradient_kernel, planned_swiglu_mm}`` with their autograd and fake
implementations, and model patching. Plans are validated and registered once, before
compiling cores or constructing DDP. Selected shapes launch the HIP kernels of
``libwarpstate_hip.so``; unselected shapes use ATen. CPU and evaluation paths stay
original; FP32 parameter casts stay inside each visible forward graph.
"""

from __future__ import annotations

from dataclasses import dataclass
import hashlib
import json
import os
from pathlib import Path

import torch
from torch.library import custom_op

PLAN_FORMAT = "warpstate-matmul-plan-v1"
_DEFAULT_TILE = (64, 64, 32, 4, 3)
_TILE_FIELDS = ("block_m", "block_n", "block_k", "num_warps", "num_stages")
_PLANS: dict[str, "MatmulPlan"] = {}
_PACKAGE = Path(__file__).resolve().parents[1]


@dataclass(frozen=True)
class MatmulEntry:
    kind: str
    m: int
    n: int
    k: int
    a_stride: tuple[int, int]
    b_stride: tuple[int, int]
    algorithm: str
    tile: tuple[int, int, int, int, int]
    name: str = ""

    @property
    def key(self):
        return (self.kind, self.m, self.n, self.k, *self.a_stride, *self.b_stride)

    def as_dict(self):
        return {"kind": self.kind, "m": self.m, "n": self.n, "k": self.k,
                "a_stride": list(self.a_stride), "b_stride": list(self.b_stride),
                "dtype": "bfloat16", "algorithm": self.algorithm,
                "tile": dict(zip(_TILE_FIELDS, self.tile, strict=True)), "name": self.name}


@dataclass(frozen=True)
class MatmulPlan:
    entries: tuple[MatmulEntry, ...]
    sha256: str
    source_hashes: tuple[tuple[str, str], ...]
    registry_key: str
    description: str = ""

    @property
    def metadata(self):
        """Serializable provenance for runtime records and resume signatures."""
        return {"format": PLAN_FORMAT, "sha256": self.sha256,
                "source_sha256": dict(self.source_hashes),
                "entries": [entry.as_dict() for entry in self.entries]}

    def select(self, kind, m, n, k, a_stride, b_stride):
        """Pure shape/layout lookup; no device work or filesystem access."""
        wanted = (kind, m, n, k, *a_stride, *b_stride)
        return next((entry for entry in self.entries if entry.key == wanted), None)


def _positive_integer(value, name):
    if isinstance(value, bool) or not isinstance(value, int) or value < 1:
        raise ValueError(f"{name} must be a positive integer")
    return value


def _stride(value, name):
    if not isinstance(value, list) or len(value) != 2:
        raise ValueError(f"{name} must contain two positive integer strides")
    return tuple(_positive_integer(item, name) for item in value)


def _no_duplicate_json_keys(pairs):
    document = {}
    for key, value in pairs:
        if key in document:
            raise ValueError(f"Duplicate JSON key: {key}")
        document[key] = value
    return document


def _implementation_hashes(has_fused_swiglu):
    """SHA-256 of this implementation's own sources, keyed like the reference's files.

    The HIP sources behind the kernels are part of the provenance, so a kernel change
    changes the execution signature just as a Triton source change does in the reference
    (ops/matmul_execution.py:96-102).
    """
    names = {"ops/matmul_execution.py": _PACKAGE / "ops" / "matmul_execution.py",
             "ops/matmul_kernels.py": _PACKAGE / "ops" / "matmul_kernels.py",
             "csrc/gemm.h": _PACKAGE / "csrc" / "gemm.h",
             "csrc/mm.hip": _PACKAGE / "csrc" / "mm.hip"}
    if has_fused_swiglu:
        names["ops/matmul_epilogue.py"] = _PACKAGE / "ops" / "matmul_epilogue.py"
        names["ops/activation_execution.py"] = _PACKAGE / "ops" / "activation_execution.py"
        names["csrc/rowops.h"] = _PACKAGE / "csrc" / "rowops.h"
    return tuple((name, hashlib.sha256(path.read_bytes()).hexdigest())
                 for name, path in sorted(names.items()))


def matmul_plan_from_dict(document: dict) -> MatmulPlan:
    """Validate a source recipe; later selection only uses immutable data
    (ops/matmul_execution.py:105-169)."""
    from ops.matmul_kernels import normalize_tile

    if not isinstance(document, dict):
        raise ValueError("Matmul plan must be a JSON object")
    if set(document) - {"format", "description", "entries"}:
        raise ValueError("Unknown matmul plan fields")
    if document.get("format") != PLAN_FORMAT:
        raise ValueError(f"Matmul plan format must be {PLAN_FORMAT}")
    description = document.get("description", "")
    if not isinstance(description, str):
        raise ValueError("Matmul plan description must be a string")
    if not isinstance(document.get("entries"), list):
        raise ValueError("Matmul plan entries must be a list")
    allowed = {"kind", "m", "n", "k", "a_stride", "b_stride", "dtype", "algorithm", "tile", "name"}
    entries, seen = [], set()
    for index, row in enumerate(document["entries"]):
        if not isinstance(row, dict) or set(row) - allowed:
            raise ValueError(f"Unknown fields in matmul entry {index}")
        if row.get("kind") not in {"mm", "swiglu"}:
            raise ValueError("Matmul entry kind must be mm or swiglu")
        if row.get("dtype") != "bfloat16":
            raise ValueError("Matmul plans support BF16 operands only")
        if row.get("algorithm") not in {"aten", "tiled", "persistent", "persistent_tma"}:
            raise ValueError("Unknown matmul algorithm")
        if row["kind"] == "swiglu" and row["algorithm"] == "persistent_tma":
            raise ValueError("Fused SwiGLU does not yet support the persistent_tma algorithm")
        dimensions = tuple(_positive_integer(row.get(name), name) for name in ("m", "n", "k"))
        if row["kind"] == "swiglu" and dimensions[1] % 2:
            raise ValueError("Fused SwiGLU output width must be even")
        name = row.get("name", "")
        if not isinstance(name, str):
            raise ValueError("Matmul entry name must be a string")
        tile_document = row.get("tile", dict(zip(_TILE_FIELDS, _DEFAULT_TILE, strict=True)))
        if not isinstance(tile_document, dict) or set(tile_document) != set(_TILE_FIELDS):
            raise ValueError("Matmul tile must specify block_m/block_n/block_k/num_warps/num_stages")
        for field, value in tile_document.items():
            _positive_integer(value, field)
        tile = tuple(normalize_tile(tile_document))
        if row["kind"] == "swiglu":
            block_m, block_n, block_k, _warps, stages = tile
            if (block_m + 2 * block_n) * block_k * 2 * stages > 96 * 1024:
                raise ValueError("Fused SwiGLU tile exceeds the conservative shared-memory budget")
        entry = MatmulEntry(row["kind"], *dimensions,
                            _stride(row.get("a_stride"), "a_stride"),
                            _stride(row.get("b_stride"), "b_stride"),
                            row["algorithm"], tile, name)
        if entry.key in seen:
            raise ValueError("Duplicate matmul shape/layout entry")
        seen.add(entry.key)
        entries.append(entry)
    canonical = {"format": PLAN_FORMAT, "description": description,
                 "entries": [entry.as_dict() for entry in entries]}
    digest = hashlib.sha256(
        json.dumps(canonical, sort_keys=True, separators=(",", ":")).encode()).hexdigest()
    hashes = _implementation_hashes(any(entry.kind == "swiglu" for entry in entries))
    registry_key = hashlib.sha256((digest + json.dumps(hashes)).encode()).hexdigest()
    plan = MatmulPlan(tuple(entries), digest, hashes, registry_key, description)
    existing = _PLANS.get(registry_key)
    if existing is not None and existing != plan:
        raise RuntimeError("Matmul plan registry identity collision")
    _PLANS[registry_key] = plan
    return plan


def _workspace() -> Path:
    """Directory plans must live under: $WARPSTATE_WORKSPACE, else this checkout's parent."""
    configured = os.environ.get("WARPSTATE_WORKSPACE")
    return Path(configured).expanduser().resolve() if configured else _PACKAGE.parents[1]


def load_matmul_plan(path: str | Path) -> MatmulPlan:
    """Load once before training; no recipes or hashes are read during forward."""
    path = Path(path).expanduser().resolve()
    if not path.is_relative_to(_workspace()):
        raise ValueError("Matmul plan must remain inside the WarpState workspace")
    document = json.loads(path.read_text(), object_pairs_hook=_no_duplicate_json_keys)
    return matmul_plan_from_dict(document)


def _choice(a, b, plan_key, kind="mm"):
    """Eligible plan entry for these operands, or None (ops/matmul_execution.py:182-198)."""
    if (a.ndim != 2 or b.ndim != 2 or not a.is_cuda or not b.is_cuda
            or a.device != b.device or a.dtype != torch.bfloat16
            or b.dtype != torch.bfloat16 or a.shape[1] != b.shape[0]
            or a.numel() == 0 or b.numel() == 0
            or any(stride <= 0 for stride in (*a.stride(), *b.stride()))):
        return None
    entry = _PLANS[plan_key].select(kind, a.shape[0], b.shape[1], a.shape[1],
                                    a.stride(), b.stride())
    if entry is not None and entry.algorithm == "persistent_tma":
        # Sliced views may lose the aligned base that the aligned-operand kernel assumes.
        if (min(a.stride()) != 1 or min(b.stride()) != 1
                or max(a.stride()) * 2 % 16 or max(b.stride()) * 2 % 16
                or a.storage_offset() * 2 % 16 or b.storage_offset() * 2 % 16):
            return None
    return entry


@custom_op("warpstate::selected_matrix_kernel", mutates_args=())
def _selected_matrix_kernel(a: torch.Tensor, b: torch.Tensor, plan_key: str) -> torch.Tensor:
    """Opaque launch, keeping the outer operator's registered autograd."""
    from ops.matmul_kernels import launch_mm

    entry = _choice(a, b, plan_key)
    if entry is None or entry.algorithm == "aten":
        return torch.mm(a, b)
    return launch_mm(a, b, entry.algorithm, entry.tile)


@_selected_matrix_kernel.register_fake
def _selected_matrix_kernel_fake(a, b, plan_key):
    return torch.empty((a.shape[0], b.shape[1]), dtype=a.dtype, device=a.device)


@custom_op("warpstate::planned_mm", mutates_args=())
def _planned_mm(a: torch.Tensor, b: torch.Tensor, plan_key: str) -> torch.Tensor:
    entry = _choice(a, b, plan_key)
    if entry is None or entry.algorithm == "aten":
        return torch.mm(a, b)
    return _selected_matrix_kernel(a, b, plan_key)


@_planned_mm.register_fake
def _planned_mm_fake(a, b, plan_key):
    return torch.empty((a.shape[0], b.shape[1]), dtype=a.dtype, device=a.device)


def _mm_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[0], inputs[1])
    ctx.plan_key = inputs[2]


def _mm_backward(ctx, grad):
    """dA = g @ b^T and dB = (g^T @ a)^T, in Linear's dW orientation
    (ops/matmul_execution.py:236-244)."""
    a, b = ctx.saved_tensors
    grad = grad.contiguous()
    da = _planned_mm(grad, b.T, ctx.plan_key) if ctx.needs_input_grad[0] else None
    db = _planned_mm(grad.T, a, ctx.plan_key).T if ctx.needs_input_grad[1] else None
    return da, db, None


_planned_mm.register_autograd(_mm_backward, setup_context=_mm_setup)


def planned_matmul(a: torch.Tensor, b: torch.Tensor, plan: MatmulPlan) -> torch.Tensor:
    """Autograd-enabled entry point, also useful for isolated correctness checks."""
    return _planned_mm(a, b, plan.registry_key)


@custom_op("warpstate::selected_swiglu_kernel", mutates_args=())
def _selected_swiglu_kernel(a: torch.Tensor, weight: torch.Tensor, plan_key: str,
                            eager_rounding: bool) -> tuple[torch.Tensor, torch.Tensor]:
    """Takes the native-layout BF16 weight [2H, K]; the projection view B = W^T is formed
    at launch (ops/matmul_execution.py:255-271)."""
    from ops.matmul_epilogue import launch_swiglu_mm

    b = weight.T
    entry = _choice(a, b, plan_key, "swiglu")
    if entry is None or entry.algorithm == "aten":
        return launch_swiglu_mm(a, b, "aten", _DEFAULT_TILE, eager_rounding)
    return launch_swiglu_mm(a, b, entry.algorithm, entry.tile, eager_rounding)


@_selected_swiglu_kernel.register_fake
def _selected_swiglu_kernel_fake(a, weight, plan_key, eager_rounding):
    packed = torch.empty((a.shape[0], weight.shape[0]), dtype=a.dtype, device=a.device)
    activation = torch.empty((a.shape[0], weight.shape[0] // 2), dtype=a.dtype, device=a.device)
    return packed, activation


@custom_op("warpstate::selected_swiglu_gradient_kernel", mutates_args=())
def _selected_swiglu_gradient_kernel(packed: torch.Tensor, grad: torch.Tensor,
                                     eager_rounding: bool) -> torch.Tensor:
    from ops.activation_execution import _swiglu_backward

    return _swiglu_backward(packed, grad, eager_rounding)


@_selected_swiglu_gradient_kernel.register_fake
def _selected_swiglu_gradient_kernel_fake(packed, grad, eager_rounding):
    return torch.empty_like(packed)


@custom_op("warpstate::planned_swiglu_mm", mutates_args=())
def _planned_swiglu_mm(a: torch.Tensor, b: torch.Tensor, plan_key: str,
                       eager_rounding: bool) -> tuple[torch.Tensor, torch.Tensor]:
    from ops.matmul_epilogue import launch_swiglu_mm

    entry = _choice(a, b, plan_key, "swiglu")
    if entry is not None and entry.algorithm != "aten":
        return _selected_swiglu_kernel(a, b.T, plan_key, eager_rounding)
    algorithm = entry.algorithm if entry is not None else "aten"
    tile = entry.tile if entry is not None else _DEFAULT_TILE
    return launch_swiglu_mm(a, b, algorithm, tile, eager_rounding)


@_planned_swiglu_mm.register_fake
def _planned_swiglu_mm_fake(a, b, plan_key, eager_rounding):
    packed = torch.empty((a.shape[0], b.shape[1]), dtype=a.dtype, device=a.device)
    activation = torch.empty((a.shape[0], b.shape[1] // 2), dtype=a.dtype, device=a.device)
    return packed, activation


def _fused_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[0], inputs[1], output[0])
    ctx.plan_key = inputs[2]
    ctx.eager_rounding = inputs[3]
    ctx.mark_non_differentiable(output[0])


def _fused_backward(ctx, _packed_grad, grad):
    """SwiGLU backward, then dX and dW of the packed projection
    (ops/matmul_execution.py:314-319)."""
    a, b, packed = ctx.saved_tensors
    projection_grad = _selected_swiglu_gradient_kernel(packed, grad, ctx.eager_rounding)
    da = _planned_mm(projection_grad, b.T, ctx.plan_key) if ctx.needs_input_grad[0] else None
    db = _planned_mm(projection_grad.T, a, ctx.plan_key).T if ctx.needs_input_grad[1] else None
    return da, db, None, None


_planned_swiglu_mm.register_autograd(_fused_backward, setup_context=_fused_setup)


def _linear_has_choices(module, plan):
    width, output = module.in_features, module.out_features
    return any(entry.kind == "mm" and (
        (entry.n == output and entry.k == width)      # forward
        or (entry.n == width and entry.k == output)   # dX
        or (entry.m == output and entry.n == width)   # dW
    ) for entry in plan.entries)


def apply_matmul_execution(model: torch.nn.Module, plan: MatmulPlan) -> None:
    """Patch bias-free Linear and SwiGLU forwards inside ``model.cores``; apply before core
    compilation and DDP (ops/matmul_execution.py:334-388). CPU/evaluation paths stay
    original and parameters are never replaced by cached BF16 views."""
    from warpstate.model import SwiGLU

    if not isinstance(plan, MatmulPlan):
        raise TypeError("Load a MatmulPlan before applying matrix execution")
    if getattr(model, "_matmul_execution_plan", None) is not None:
        raise ValueError("Matmul execution has already been applied")
    if any(parameter.dtype != torch.float32 for parameter in model.parameters()):
        raise ValueError("Matmul execution requires FP32 master parameters")
    if plan.registry_key not in _PLANS:
        raise ValueError("Matmul plan is not registered in this process")
    model._matmul_execution_plan = plan
    if not plan.entries:
        return
    has_fused = any(entry.kind == "swiglu" and entry.algorithm != "aten" for entry in plan.entries)

    def bf16_training(module, x):
        return (module.training and torch.is_grad_enabled() and x.is_cuda
                and torch.is_autocast_enabled("cuda")
                and torch.get_autocast_dtype("cuda") == torch.bfloat16)

    for core in model.cores:
        for module in core.modules():
            original = module.forward
            if (isinstance(module, torch.nn.Linear) and module.bias is None
                    and _linear_has_choices(module, plan)):
                def linear_forward(x, _module=module, _original=original):
                    if not bf16_training(_module, x):
                        return _original(x)
                    a = x.reshape(-1, x.shape[-1]).to(torch.bfloat16)
                    b = _module.weight.to(torch.bfloat16).T
                    output = _planned_mm(a, b, plan.registry_key)
                    return output.reshape(*x.shape[:-1], _module.out_features)
                module.forward = linear_forward
            elif (isinstance(module, SwiGLU) and has_fused and any(
                    entry.kind == "swiglu" and entry.n == module.up_gate.out_features
                    and entry.k == module.up_gate.in_features for entry in plan.entries)):
                def swiglu_forward(x, _module=module, _original=original):
                    if not bf16_training(_module, x) or _module.up_gate.bias is not None:
                        return _original(x)
                    a = x.reshape(-1, x.shape[-1]).to(torch.bfloat16)
                    b = _module.up_gate.weight.to(torch.bfloat16).T
                    entry = _choice(a, b, plan.registry_key, "swiglu")
                    if entry is None or entry.algorithm == "aten":
                        return _original(x)
                    _, activation = _planned_swiglu_mm(
                        a, b, plan.registry_key, not torch.compiler.is_compiling())
                    activation = activation.reshape(*x.shape[:-1], _module.down.in_features)
                    return _module.down(activation)
                module.forward = swiglu_forward
