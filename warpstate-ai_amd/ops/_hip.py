"""ctypes binding of ``libwarpstate_hip.so``, the C ABI declared in ``include/warpstate_hip.h``.

Every call passes raw device pointers, element strides and sizes, and the HIP stream of
PyTorch's current stream on the calling thread. A non-zero status becomes a
``RuntimeError`` carrying the library's message. There is no fallback: when the library
is missing, every kernel entry point raises.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIBRARY_PATH = Path(__file__).resolve().parents[1] / "lib" / "libwarpstate_hip.so"

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float

# name -> (restype, argtypes); mirrors include/warpstate_hip.h.
SIGNATURES = {
    "ws_last_error": (ctypes.c_char_p, []),
    "ws_version": (ctypes.c_char_p, []),
    "ws_mm": (_i32, [_c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _i64,
                     _i32, _i32, _c_void_p]),
    "ws_swiglu_mm": (_i32, [_c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _c_void_p, _c_void_p,
                            _i64, _i64, _i64, _i32, _i32, _i32, _c_void_p]),
    "ws_swiglu_forward": (_i32, [_c_void_p, _c_void_p, _i64, _i64, _i32, _c_void_p]),
    "ws_swiglu_backward": (_i32, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i32, _c_void_p]),
    "ws_rmsnorm_forward": (_i32, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _f32,
                                  _i32, _c_void_p]),
    "ws_rmsnorm_backward_partial_floats": (_i64, [_i64, _i64]),
    "ws_rmsnorm_backward": (_i32, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                   _c_void_p, _c_void_p, _i64, _i64, _i32, _c_void_p]),
    "ws_rmsnorm_backward_static": (_i32, [_c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                          _c_void_p, _c_void_p, _i64, _i64, _i32, _c_void_p]),
    "ws_rmsnorm_backward_static_max_partial_floats": (_i64, []),
    "ws_transpose_bf16": (_i32, [_c_void_p, _i64, _c_void_p, _i64, _i64, _c_void_p]),
    "ws_rmsnorm_gate_mm": (_i32, [_c_void_p, _i64, _c_void_p, _f32, _c_void_p, _c_void_p,
                                  _c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _i64, _i64,
                                  _i64, _c_void_p]),
    "ws_sigmoid_backward_cols": (_i32, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _i64, _i64,
                                        _i64, _i64, _i64, _c_void_p]),
    "ws_residual_mm": (_i32, [_c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _c_void_p, _i64,
                              _c_void_p, _i64, _i64, _i64, _c_void_p]),
    "ws_swiglu_backward_mm": (_i32, [_c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _c_void_p,
                                     _c_void_p, _i64, _i64, _i64, _i32, _c_void_p]),
    "ws_mm_accumulate_workspace_floats": (_i64, [_i64, _i64, _i64, _i64]),
    "ws_mm_accumulate_f32": (_i32, [_c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _c_void_p, _i64,
                                    _i64, _i64, _i64, _i32, _c_void_p, _i64, _c_void_p]),
    "ws_mm_accumulate_group_workspace_floats": (_i64, [_c_void_p, _i32, _i64]),
    "ws_mm_accumulate_f32_group": (_i32, [_c_void_p, _i32, _i64, _i32, _c_void_p, _c_void_p]),
    "ws_mm_store_f32": (_i32, [_c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _c_void_p, _i64,
                               _i64, _i64, _i64, _i32, _c_void_p, _i64, _c_void_p]),
    "ws_mm_store_f32_group": (_i32, [_c_void_p, _i32, _i64, _i32, _c_void_p, _c_void_p]),
    "ws_linear_ce_parts": (_i64, [_i64]),
    "ws_linear_ce_forward": (_i32, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _i64, _i64, _i64,
                                    _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                    _c_void_p, _c_void_p, _c_void_p, _c_void_p]),
    "ws_linear_ce_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "ws_linear_ce_backward": (_i32, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _c_void_p,
                                     _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64,
                                     _c_void_p, _i64, _c_void_p, _i64, _c_void_p, _i64,
                                     _c_void_p, _c_void_p]),
    "ws_linear_ce_fused": (_i32, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _c_void_p, _i64,
                                  _i64, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                  _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p,
                                  _i64, _c_void_p, _i64, _c_void_p]),
    "ws_linear_ce_fused_backward": (_i32, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p,
                                           _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64,
                                           _i64, _i64, _c_void_p, _i64, _c_void_p, _i64,
                                           _c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p]),
    "ws_linear_ce_combine": (_i32, [_c_void_p] * 8 + [_i64, _i64, _c_void_p]),
    "ws_linear_ce_logit_grad": (_i32, [_c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p,
                                       _c_void_p, _i64, _i64, _i64, _c_void_p]),
    "ws_backward_layout": (_i32, [_c_void_p] * 15 + [_i64] * 5 + [_f32, _i32, _c_void_p,
                                                                   _c_void_p, _c_void_p]),
}


class AccumulateProblem(ctypes.Structure):
    """``ws_accumulate_problem``: one weight gradient of a grouped accumulation."""
    _fields_ = [("a", _c_void_p), ("a_s0", _i64), ("a_s1", _i64),
                ("b", _c_void_p), ("b_s0", _i64), ("b_s1", _i64),
                ("g", _c_void_p), ("ldg", _i64), ("m", _i64), ("n", _i64)]


def problem_table(rows) -> ctypes.Array:
    """A ``ws_accumulate_problem`` array from (a, a_s0, a_s1, b, b_s0, b_s1, g, ldg, m, n)
    tuples of pointers and element counts."""
    return (AccumulateProblem * len(rows))(*[AccumulateProblem(*r) for r in rows])


_lock = threading.Lock()
_library = None


def library() -> ctypes.CDLL:
    """Load the shared library once; raise if it has not been built."""
    global _library
    if _library is None:
        with _lock:
            if _library is None:
                if not LIBRARY_PATH.exists():
                    raise RuntimeError(
                        f"HIP extension not built: {LIBRARY_PATH} is missing "
                        "(run __graft_entry__.build())")
                lib = ctypes.CDLL(str(LIBRARY_PATH))
                for name, (restype, argtypes) in SIGNATURES.items():
                    function = getattr(lib, name)
                    function.restype = restype
                    function.argtypes = argtypes
                _library = lib
    return _library


def call(name: str, *args) -> None:
    """Invoke a status-returning entry point; raise RuntimeError on failure."""
    lib = library()
    status = getattr(lib, name)(*args)
    if status != 0:
        message = lib.ws_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed (status {status}): {message}")


def query(name: str, *args) -> int:
    return int(getattr(library(), name)(*args))


def stream(tensor: torch.Tensor) -> int:
    """HIP stream handle of the calling thread's current stream on the tensor's device."""
    return torch.cuda.current_stream(tensor.device).cuda_stream


def ptr(tensor: torch.Tensor | None) -> int | None:
    return None if tensor is None else tensor.data_ptr()


def algorithm_code(algorithm: str) -> int:
    return {"tiled": 0, "persistent": 1, "persistent_tma": 2}[algorithm]


def tile_code(block_m: int, block_n: int) -> int:
    """Macro-tile for a requested (block_m, block_n): 0 = 256x256, 1 = 128x128.

    Requests of at least 128x128 outputs use the 256x256 8-wave tile; smaller requests
    use the 128x128 4-wave tile that keeps two workgroups per CU.
    """
    return 0 if block_m * block_n >= 128 * 128 else 1
