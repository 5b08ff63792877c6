"""Plan-selected BF16 GEMMs behind registered operators, for gfx950.

Interface (kept so that plans, compiled graphs and callers written for WarpState's
``ops/matmul_execution.py`` work unchanged): the ``warpstate-matmul-plan-v1`` document and
its validation messages, ``MatmulEntry`` / ``MatmulPlan``, ``matmul_plan_from_dict``,
``load_matmul_plan``, ``planned_matmul``, ``apply_matmul_execution``, and the operators
``warpstate::{selected_matrix_kernel, planned_mm, selected_swiglu_kernel,
selected_swiglu_gradient_kernel, planned_swiglu_mm}`` with their schemas, fake tensors and
autograd formulas.

How it works here:
* A plan is parsed once into immutable entries plus a dictionary from the exact
  (kind, m, n, k, a strides, b strides) key to its entry, so selection during a forward is
  one lookup. Plans are registered in a process-wide table under a key that covers the
  plan's canonical JSON and the SHA-256 of the sources that execute it (Python and HIP).
* The operators decide on the host, before any launch, whether a call is served by a HIP
  kernel of ``libwarpstate_hip.so`` or by ATen (no entry, an ``aten`` entry, CPU operands,
  or operands that lost the alignment an aligned-load entry needs).
* The weight-gradient GEMM of every projection is issued as dY^T @ X, the nn.Linear dW
  orientation the tuner measures, and its transpose is returned as the gradient of B = W^T.
"""

from __future__ import annotations

from dataclasses import dataclass, field
import hashlib
import json
import os
from pathlib import Path

import torch
from torch.library import custom_op

from ops._patching import install_forward

PLAN_FORMAT = "warpstate-matmul-plan-v1"
_TILE_FIELDS = ("block_m", "block_n", "block_k", "num_warps", "num_stages")
_DEFAULT_TILE = (64, 64, 32, 4, 3)
_KINDS = ("mm", "swiglu")
_ALGORITHMS = ("aten", "tiled", "persistent", "persistent_tma")
_DOCUMENT_FIELDS = frozenset({"format", "description", "entries"})
_ENTRY_FIELDS = frozenset({"kind", "m", "n", "k", "a_stride", "b_stride", "dtype",
                           "algorithm", "tile", "name"})
_PACKAGE = Path(__file__).resolve().parents[1]
# Sources whose bytes are part of a plan's identity: the Python that selects and launches
# and the HIP that computes. Fused SwiGLU plans add the epilogue's modules.
_SOURCES = ("ops/matmul_execution.py", "ops/matmul_kernels.py", "csrc/gemm.h",
            "csrc/gemm_fast.h", "csrc/mm.hip")
_SWIGLU_SOURCES = ("ops/matmul_epilogue.py", "ops/activation_execution.py", "csrc/rowops.h")

_PLANS: dict[str, "MatmulPlan"] = {}


@dataclass(frozen=True)
class MatmulEntry:
    """One selected shape/layout: operation kind, sizes, element strides of A [m, k] and
    B [k, n], the algorithm and its five-field tile."""
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
    def key(self) -> tuple:
        return (self.kind, self.m, self.n, self.k, *self.a_stride, *self.b_stride)

    def as_dict(self) -> dict:
        return {"kind": self.kind, "m": self.m, "n": self.n, "k": self.k,
                "a_stride": list(self.a_stride), "b_stride": list(self.b_stride),
                "dtype": "bfloat16", "algorithm": self.algorithm,
                "tile": dict(zip(_TILE_FIELDS, self.tile, strict=True)), "name": self.name}


@dataclass(frozen=True)
class MatmulPlan:
    """A validated plan: entries in document order, the canonical digest, the source
    digests and the registry key. ``select`` reads a prebuilt index only."""
    entries: tuple[MatmulEntry, ...]
    sha256: str
    source_hashes: tuple[tuple[str, str], ...]
    registry_key: str
    description: str = ""
    _index: dict = field(init=False, repr=False, compare=False, hash=False)

    def __post_init__(self):
        object.__setattr__(self, "_index", {entry.key: entry for entry in self.entries})

    @property
    def metadata(self) -> dict:
        """The plan's provenance as plain JSON values (for run records and resume
        signatures)."""
        return {"format": PLAN_FORMAT, "sha256": self.sha256,
                "source_sha256": dict(self.source_hashes),
                "entries": [entry.as_dict() for entry in self.entries]}

    def select(self, kind, m, n, k, a_stride, b_stride) -> MatmulEntry | None:
        return self._index.get((kind, m, n, k, *a_stride, *b_stride))


# --- reading a plan document ------------------------------------------------------------

def _require(condition: bool, message: str) -> None:
    if not condition:
        raise ValueError(message)


def _count(value, name: str) -> int:
    """A positive int (bool is not accepted as an int)."""
    _require(type(value) is int and value >= 1, f"{name} must be a positive integer")
    return value


def _strides(value, name: str) -> tuple[int, int]:
    _require(isinstance(value, list) and len(value) == 2,
             f"{name} must contain two positive integer strides")
    return (_count(value[0], name), _count(value[1], name))


def _tile(row: dict, kind: str) -> tuple[int, int, int, int, int]:
    from ops.matmul_kernels import normalize_tile

    document = row.get("tile")
    if document is None and "tile" not in row:
        return normalize_tile(dict(zip(_TILE_FIELDS, _DEFAULT_TILE)))
    _require(isinstance(document, dict) and set(document) == set(_TILE_FIELDS),
             "Matmul tile must specify block_m/block_n/block_k/num_warps/num_stages")
    for name in _TILE_FIELDS:
        _count(document[name], name)
    tile = normalize_tile(document)
    if kind == "swiglu":
        # block_n counts one half of the pair: A plus two B panels per stage.
        bm, bn, bk, _warps, stages = tile
        _require((bm + 2 * bn) * bk * 2 * stages <= 96 * 1024,
                 "Fused SwiGLU tile exceeds the conservative shared-memory budget")
    return tile


def _entry(index: int, row) -> MatmulEntry:
    _require(isinstance(row, dict) and set(row) <= _ENTRY_FIELDS,
             f"Unknown fields in matmul entry {index}")
    kind, algorithm = row.get("kind"), row.get("algorithm")
    _require(kind in _KINDS, "Matmul entry kind must be mm or swiglu")
    _require(row.get("dtype") == "bfloat16", "Matmul plans support BF16 operands only")
    _require(algorithm in _ALGORITHMS, "Unknown matmul algorithm")
    _require(not (kind == "swiglu" and algorithm == "persistent_tma"),
             "Fused SwiGLU does not yet support the persistent_tma algorithm")
    m, n, k = (_count(row.get(name), name) for name in ("m", "n", "k"))
    _require(kind != "swiglu" or n % 2 == 0, "Fused SwiGLU output width must be even")
    name = row.get("name", "")
    _require(isinstance(name, str), "Matmul entry name must be a string")
    tile = _tile(row, kind)
    return MatmulEntry(kind, m, n, k, _strides(row.get("a_stride"), "a_stride"),
                       _strides(row.get("b_stride"), "b_stride"), algorithm, tile, name)


def _digest(text: str) -> str:
    return hashlib.sha256(text.encode()).hexdigest()


def _source_hashes(with_swiglu: bool) -> tuple[tuple[str, str], ...]:
    names = _SOURCES + (_SWIGLU_SOURCES if with_swiglu else ())
    return tuple((name, hashlib.sha256((_PACKAGE / name).read_bytes()).hexdigest())
                 for name in sorted(names))


def matmul_plan_from_dict(document: dict) -> MatmulPlan:
    """Validate a plan document and register it (ops/matmul_execution.py:105-169).

    Errors are ``ValueError`` with the reference's messages, raised in its order: document
    shape, format, description, entries; then per entry its fields, kind, dtype,
    algorithm, sizes, name, tile and strides; then duplicate keys."""
    _require(isinstance(document, dict), "Matmul plan must be a JSON object")
    _require(set(document) <= _DOCUMENT_FIELDS, "Unknown matmul plan fields")
    _require(document.get("format") == PLAN_FORMAT, f"Matmul plan format must be {PLAN_FORMAT}")
    description = document.get("description", "")
    _require(isinstance(description, str), "Matmul plan description must be a string")
    rows = document.get("entries")
    _require(isinstance(rows, list), "Matmul plan entries must be a list")
    entries: list[MatmulEntry] = []
    keys: set[tuple] = set()
    for index, row in enumerate(rows):
        entry = _entry(index, row)
        _require(entry.key not in keys, "Duplicate matmul shape/layout entry")
        keys.add(entry.key)
        entries.append(entry)
    canonical = json.dumps({"format": PLAN_FORMAT, "description": description,
                            "entries": [entry.as_dict() for entry in entries]},
                           sort_keys=True, separators=(",", ":"))
    sha = _digest(canonical)
    sources = _source_hashes(any(entry.kind == "swiglu" for entry in entries))
    plan = MatmulPlan(tuple(entries), sha, sources, _digest(sha + json.dumps(sources)),
                      description)
    registered = _PLANS.setdefault(plan.registry_key, plan)
    if registered != plan:
        raise RuntimeError("Matmul plan registry identity collision")
    return plan


def _workspace() -> Path:
    """Root under which plan files must live: $WARPSTATE_WORKSPACE when set, otherwise the
    directory that holds this checkout."""
    configured = os.environ.get("WARPSTATE_WORKSPACE")
    return Path(configured).expanduser().resolve() if configured else _PACKAGE.parents[1]


def _reject_duplicate_keys(pairs: list) -> dict:
    document: dict = {}
    for key, value in pairs:
        _require(key not in document, f"Duplicate JSON key: {key}")
        document[key] = value
    return document


def load_matmul_plan(path: str | Path) -> MatmulPlan:
    """Read, validate and register a plan file; call before compiling or training, since
    forwards only consult registered plans."""
    path = Path(path).expanduser().resolve()
    _require(path.is_relative_to(_workspace()),
             "Matmul plan must remain inside the WarpState workspace")
    return matmul_plan_from_dict(json.loads(path.read_text(),
                                            object_pairs_hook=_reject_duplicate_keys))


# --- selection -------------------------------------------------------------------------

def _launchable(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Operands a HIP kernel can take at all: two non-empty BF16 CUDA matrices on one
    device with matching inner sizes and positive strides."""
    return (a.ndim == 2 and b.ndim == 2 and a.is_cuda and b.is_cuda and a.device == b.device
            and a.dtype == torch.bfloat16 and b.dtype == torch.bfloat16
            and a.shape[1] == b.shape[0] and a.numel() > 0 and b.numel() > 0
            and min(*a.stride(), *b.stride()) > 0)


def _aligned_rows(t: torch.Tensor) -> bool:
    """Unit inner stride, 16-byte row pitch and a 16-byte-aligned storage offset: what the
    aligned-load (``persistent_tma``) kernels assume. A view sliced out of an aligned
    allocation can keep its shape and strides and still fail the offset test."""
    return (min(t.stride()) == 1 and max(t.stride()) * 2 % 16 == 0
            and t.storage_offset() * 2 % 16 == 0)


def _choice(a, b, plan_key, kind="mm"):
    """The entry that serves these operands, or None for ATen (ops/matmul_execution.py:182-198)."""
    if not _launchable(a, b):
        return None
    entry = _PLANS[plan_key].select(kind, a.shape[0], b.shape[1], a.shape[1],
                                    a.stride(), b.stride())
    if entry is not None and entry.algorithm == "persistent_tma":
        if not (_aligned_rows(a) and _aligned_rows(b)):
            return None
    return entry


def _served(entry: MatmulEntry | None) -> bool:
    return entry is not None and entry.algorithm != "aten"


# --- registered operators ---------------------------------------------------------------

@custom_op("warpstate::selected_matrix_kernel", mutates_args=())
def _selected_matrix_kernel(a: torch.Tensor, b: torch.Tensor, plan_key: str) -> torch.Tensor:
    """The GEMM launch as one opaque node, so that compiled autograd re-traces the outer
    operator's backward without looking inside the kernel call."""
    from ops.matmul_kernels import launch_mm

    entry = _choice(a, b, plan_key)
    return launch_mm(a, b, entry.algorithm, entry.tile) if _served(entry) else torch.mm(a, b)


@_selected_matrix_kernel.register_fake
def _(a, b, plan_key):
    return a.new_empty((a.shape[0], b.shape[1]))


@custom_op("warpstate::planned_mm", mutates_args=())
def _planned_mm(a: torch.Tensor, b: torch.Tensor, plan_key: str) -> torch.Tensor:
    """r(a @ b): selected shapes through the opaque kernel node, the rest through ATen."""
    if _served(_choice(a, b, plan_key)):
        return _selected_matrix_kernel(a, b, plan_key)
    return torch.mm(a, b)


@_planned_mm.register_fake
def _(a, b, plan_key):
    return a.new_empty((a.shape[0], b.shape[1]))


def _save_operands(ctx, inputs, output):
    a, b, ctx.plan_key = inputs
    ctx.save_for_backward(a, b)


def _operand_grads(ctx, grad_out, a, b, plan_key):
    """(dA, dB) of C = A @ B: dA = G B^T, and dB from the dW-oriented product G^T A,
    transposed back (ops/matmul_execution.py:236-244)."""
    da = _planned_mm(grad_out, b.T, plan_key) if ctx.needs_input_grad[0] else None
    db = _planned_mm(grad_out.T, a, plan_key).T if ctx.needs_input_grad[1] else None
    return da, db


def _mm_backward(ctx, grad):
    a, b = ctx.saved_tensors
    return (*_operand_grads(ctx, grad.contiguous(), a, b, ctx.plan_key), None)


_planned_mm.register_autograd(_mm_backward, setup_context=_save_operands)


def planned_matmul(a: torch.Tensor, b: torch.Tensor, plan: MatmulPlan) -> torch.Tensor:
    """``a @ b`` through ``warpstate::planned_mm`` with autograd."""
    return _planned_mm(a, b, plan.registry_key)


def _paired(a, b, entry, eager_rounding):
    from ops.matmul_epilogue import launch_swiglu_mm

    if _served(entry):
        return launch_swiglu_mm(a, b, entry.algorithm, entry.tile, eager_rounding)
    tile = entry.tile if entry is not None else _DEFAULT_TILE
    return launch_swiglu_mm(a, b, "aten", tile, eager_rounding)


def _paired_fake(rows, width, like):
    return like.new_empty((rows, width)), like.new_empty((rows, width // 2))


@custom_op("warpstate::selected_swiglu_kernel", mutates_args=())
def _selected_swiglu_kernel(a: torch.Tensor, weight: torch.Tensor, plan_key: str,
                            eager_rounding: bool) -> tuple[torch.Tensor, torch.Tensor]:
    """(packed, act) from the nn.Linear-layout weight [2H, K]: B = W^T is formed inside,
    so that a compiled graph passes the same BF16 weight here and to the saved-for-backward
    slot (ops/matmul_execution.py:255-271)."""
    b = weight.T
    return _paired(a, b, _choice(a, b, plan_key, "swiglu"), eager_rounding)


@_selected_swiglu_kernel.register_fake
def _(a, weight, plan_key, eager_rounding):
    return _paired_fake(a.shape[0], weight.shape[0], a)


@custom_op("warpstate::selected_swiglu_gradient_kernel", mutates_args=())
def _selected_swiglu_gradient_kernel(packed: torch.Tensor, grad: torch.Tensor,
                                     eager_rounding: bool) -> torch.Tensor:
    """dUp | dGate of the packed projection (the SwiGLU backward row kernel)."""
    from ops.activation_execution import _swiglu_backward

    return _swiglu_backward(packed, grad, eager_rounding)


@_selected_swiglu_gradient_kernel.register_fake
def _(packed, grad, eager_rounding):
    return torch.empty_like(packed)


@custom_op("warpstate::planned_swiglu_mm", mutates_args=())
def _planned_swiglu_mm(a: torch.Tensor, b: torch.Tensor, plan_key: str,
                       eager_rounding: bool) -> tuple[torch.Tensor, torch.Tensor]:
    """(packed, act) of the paired projection with the SwiGLU epilogue."""
    entry = _choice(a, b, plan_key, "swiglu")
    if _served(entry):
        return _selected_swiglu_kernel(a, b.T, plan_key, eager_rounding)
    return _paired(a, b, entry, eager_rounding)


@_planned_swiglu_mm.register_fake
def _(a, b, plan_key, eager_rounding):
    return _paired_fake(a.shape[0], b.shape[1], a)


def _save_paired(ctx, inputs, output):
    a, b, ctx.plan_key, ctx.eager_rounding = inputs
    packed = output[0]
    ctx.save_for_backward(a, b, packed)
    ctx.mark_non_differentiable(packed)


def _fused_backward(ctx, _packed_grad, grad):
    """Through the activation to dPacked, then dA and dB of the packed projection
    (ops/matmul_execution.py:314-319)."""
    a, b, packed = ctx.saved_tensors
    dpacked = _selected_swiglu_gradient_kernel(packed, grad, ctx.eager_rounding)
    return (*_operand_grads(ctx, dpacked, a, b, ctx.plan_key), None, None)


_planned_swiglu_mm.register_autograd(_fused_backward, setup_context=_save_paired)


# --- model patching --------------------------------------------------------------------

def _linear_has_choices(module: torch.nn.Linear, plan: MatmulPlan) -> bool:
    """Whether any ``mm`` entry can serve one of the Linear's three GEMMs, given as
    (m, n, k) with None for the token count: the forward [*, in] x [in, out], the input
    gradient [*, out] x [out, in] and the weight gradient [out, *] x [*, in]."""
    d_in, d_out = module.in_features, module.out_features
    gemms = ((None, d_out, d_in), (None, d_in, d_out), (d_out, d_in, None))
    return any(entry.kind == "mm"
               and all(want is None or want == got
                       for want, got in zip(gemm, (entry.m, entry.n, entry.k)))
               for entry in plan.entries for gemm in gemms)


def _rows(x: torch.Tensor) -> torch.Tensor:
    return x.reshape(-1, x.shape[-1]).to(torch.bfloat16)


def _planned_linear(plan_key: str):
    def run(module, x, _original):
        out = _planned_mm(_rows(x), module.weight.to(torch.bfloat16).T, plan_key)
        return out.reshape(*x.shape[:-1], module.out_features)
    return run


def _planned_swiglu(plan_key: str):
    def run(module, x, original):
        if module.up_gate.bias is not None:
            return original(x)
        a = _rows(x)
        b = module.up_gate.weight.to(torch.bfloat16).T
        if not _served(_choice(a, b, plan_key, "swiglu")):
            return original(x)
        # Eager calls keep the eager BF16 rounding of the SiLU; traced calls follow the
        # compiled arithmetic.
        _packed, act = _planned_swiglu_mm(a, b, plan_key, not torch.compiler.is_compiling())
        return module.down(act.reshape(*x.shape[:-1], module.down.in_features))
    return run


def apply_matmul_execution(model: torch.nn.Module, plan: MatmulPlan) -> None:
    """Route the bias-free Linear and SwiGLU modules of ``model.cores`` through the plan
    (ops/matmul_execution.py:334-388). Apply before compiling cores and before DDP.

    Only training calls with gradients on CUDA tensors under BF16 autocast change path;
    CPU and evaluation calls run the original forwards. Parameters stay the FP32 masters:
    each forward casts them to BF16 inside the visible graph, so gradients reach the
    masters through ordinary casts."""
    from warpstate.model import SwiGLU

    if not isinstance(plan, MatmulPlan):
        raise TypeError("Load a MatmulPlan before applying matrix execution")
    if getattr(model, "_matmul_execution_plan", None) is not None:
        raise ValueError("Matmul execution has already been applied")
    if any(p.dtype != torch.float32 for p in model.parameters()):
        raise ValueError("Matmul execution requires FP32 master parameters")
    if plan.registry_key not in _PLANS:
        raise ValueError("Matmul plan is not registered in this process")
    model._matmul_execution_plan = plan
    swiglu = [e for e in plan.entries if e.kind == "swiglu"]
    # SwiGLU modules are routed when the plan launches some fused kernel and has a SwiGLU
    # entry of the module's widths; an ``aten`` entry then still selects the original.
    fused_widths = ({(e.n, e.k) for e in swiglu}
                    if any(e.algorithm != "aten" for e in swiglu) else set())
    for core in model.cores:
        for module in core.modules():
            if (isinstance(module, torch.nn.Linear) and module.bias is None
                    and _linear_has_choices(module, plan)):
                install_forward(module, _planned_linear(plan.registry_key))
            elif (isinstance(module, SwiGLU) and (module.up_gate.out_features,
                                                  module.up_gate.in_features) in fused_widths):
                install_forward(module, _planned_swiglu(plan.registry_key))
