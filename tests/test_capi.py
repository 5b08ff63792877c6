"""The C-ABI library loads on a CPU-only host and exports every symbol its header declares.

No compute entry point is called here (there is no GPU); the size queries, which do no
device work, are checked against their documented formulas.
"""
import ctypes
import re
from pathlib import Path

import pytest

from ops import _hip

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))


def declared_symbols():
    names = set()
    for header in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names.update(re.findall(r"\b(ws_[a-z0-9_]+)\s*\(", text))
    return names


def test_header_declares_the_entry_points():
    names = declared_symbols()
    assert {"ws_mm", "ws_swiglu_mm", "ws_rmsnorm_gate_mm", "ws_residual_mm",
            "ws_swiglu_backward_mm", "ws_mm_accumulate_f32", "ws_linear_ce_forward",
            "ws_linear_ce_backward", "ws_last_error"} <= names


def test_library_exports_every_declared_symbol_and_binding_matches():
    if not _hip.LIBRARY_PATH.exists():
        pytest.fail(f"{_hip.LIBRARY_PATH} missing: run __graft_entry__.build()")
    lib = ctypes.CDLL(str(_hip.LIBRARY_PATH))
    names = declared_symbols()
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    # The ctypes signature table covers exactly the declared entry points.
    assert set(_hip.SIGNATURES) == names


def test_queries_without_device_work():
    lib = _hip.library()
    assert lib.ws_version().startswith(b"warpstate-hip")
    assert _hip.query("ws_linear_ce_parts", 32768) == 2 * 128
    assert _hip.query("ws_mm_accumulate_workspace_floats", 10, 20, 64, 1) == 0
    # At least the even slices; at least one 256 x 256 partial block per piece of the
    # single (stream-K shared) tile.
    assert _hip.query("ws_mm_accumulate_workspace_floats", 10, 20, 64, 4) >= 800
    assert _hip.query("ws_mm_accumulate_workspace_floats", 10, 20, 64, 4) % 65536 == 0
    # One partial weight-gradient row per 64-row block.
    assert _hip.query("ws_rmsnorm_backward_partial_floats", 10, 64) == 64
    assert _hip.query("ws_rmsnorm_backward_partial_floats", 16384, 2048) == 512 * 2048
    # One 4096-row chunk of BF16 logit gradients plus two FP32 dHidden partial slices.
    assert _hip.query("ws_linear_ce_workspace_bytes", 16384, 32768, 2048, 4096) == \
        256 + 4096 * 32768 * 2 + 2 * 4096 * 2048 * 4


def test_invalid_arguments_are_rejected_before_any_launch():
    """Argument validation runs on the host and reports through ws_last_error."""
    with pytest.raises(RuntimeError, match="positive"):
        _hip.call("ws_mm", 16, 8, 1, 16, 8, 1, 16, 0, 8, 8, 0, 0, None)
    with pytest.raises(RuntimeError, match="algorithm"):
        _hip.call("ws_mm", 16, 8, 1, 16, 8, 1, 16, 8, 8, 8, 7, 0, None)
    with pytest.raises(RuntimeError, match="gate column range"):
        _hip.call("ws_rmsnorm_gate_mm", 16, 8, 16, 1e-6, 16, 16, 16, 1, 8, 16, 8, 8, 8, 6, 9, None)
    # A 256-row tile of the output must span less than 2 GiB (32-bit tile offsets).
    with pytest.raises(RuntimeError, match="row stride"):
        _hip.call("ws_mm", 16, 8, 1, 16, 8, 1, 16, 16, 4_200_000, 8, 0, 0, None)
    with pytest.raises(RuntimeError, match="row stride"):
        _hip.call("ws_mm_accumulate_f32", 16, 8, 1, 16, 8, 1, 16, 2_100_000, 16, 8, 8, 1, None,
                  1, None)


def test_grouped_accumulation_arguments_are_rejected_before_any_launch():
    """Group size, per-gradient shapes and overlapping gradients are checked on the host."""
    gpu_ptr = 1 << 20  # never dereferenced: every call below fails validation first

    def row(g, m, n, ldg=None):
        return (gpu_ptr, 8, 1, gpu_ptr, 8, 1, g, ldg or n, m, n)

    table = _hip.problem_table([row(gpu_ptr, 8, 8)] * 5)
    with pytest.raises(RuntimeError, match="group size 5"):
        _hip.call("ws_mm_accumulate_f32_group", table, 5, 8, 1, None, None)
    with pytest.raises(RuntimeError, match="group size 0"):
        _hip.call("ws_mm_accumulate_f32_group", table, 0, 8, 1, None, None)
    with pytest.raises(RuntimeError, match="null problem table"):
        _hip.call("ws_mm_accumulate_f32_group", None, 1, 8, 1, None, None)
    with pytest.raises(RuntimeError, match="positive"):
        _hip.call("ws_mm_accumulate_f32_group", _hip.problem_table([row(gpu_ptr, 0, 8)]), 1, 8,
                  1, None, None)
    with pytest.raises(RuntimeError, match="row stride"):
        _hip.call("ws_mm_accumulate_f32_group",
                  _hip.problem_table([row(gpu_ptr, 8, 8, 2_100_000)]), 1, 8, 1, None, None)
    # The second gradient starts inside the first one's last row.
    overlapping = _hip.problem_table([row(gpu_ptr, 8, 8), row(gpu_ptr + 4 * (7 * 8 + 4), 8, 8)])
    with pytest.raises(RuntimeError, match="overlap"):
        _hip.call("ws_mm_accumulate_f32_group", overlapping, 2, 8, 1, None, None)


def test_grouped_workspace_query():
    """Whole rounds need no workspace; the shared tiles need one 256 x 256 FP32 block per
    piece; a group that falls back needs what its largest single split needs."""
    def rows(*shapes):
        return _hip.problem_table([(1 << 20, 8, 1, 1 << 20, 8, 1, 1 << 20, n, m, n)
                                   for m, n in shapes])

    q = lambda t, c, k: _hip.query("ws_mm_accumulate_group_workspace_floats", t, c, k)
    assert q(None, 1, 64) == 0
    # 2048 x 2048 twice at k = 16384: 128 tiles, no whole round; each falls back to 2
    # even splits (256 tiles), which need 2 x 2048 x 2048 floats.
    assert q(rows((2048, 2048), (2048, 2048)), 2, 16384) >= 2 * 2048 * 2048
    need = q(rows((2048, 5632), (11264, 2048)), 2, 16384)
    assert need > 0 and need % 65536 == 0


def test_grouped_fallback_splits_follow_auto_splits():
    """A group with fewer tiles than compute units falls back to one call per gradient,
    each split by the library's port of ops.fused_execution.auto_splits: the group's
    workspace is the largest of those single calls' workspaces."""
    from ops.fused_execution import auto_splits

    cus = 256  # the query's device count on a host without a GPU
    for k in (512, 4096, 16384):
        for shapes in ([(2048, 5632)], [(300, 264), (520, 130)], [(1024, 1024), (4096, 512)]):
            rows = _hip.problem_table([(1 << 20, 8, 1, 1 << 20, 8, 1, 1 << 20, n, m, n)
                                       for m, n in shapes])
            tiles = sum(-(-m // 256) * -(-n // 256) for m, n in shapes)
            assert tiles < cus
            want = max(_hip.query("ws_mm_accumulate_workspace_floats", m, n, k,
                                  auto_splits(m, n, k, cus)) for m, n in shapes)
            assert _hip.query("ws_mm_accumulate_group_workspace_floats", rows, len(shapes), k) == want


def test_static_rmsnorm_backward_refuses_wide_rows_before_any_launch():
    """The allocation-free RMSNorm backward takes rows of at most 8192 columns, the widest
    any of its row kernels takes. The check runs before any device call."""
    gpu_ptr = 1 << 20  # never dereferenced
    with pytest.raises(RuntimeError, match="at most 8192 columns"):
        _hip.call("ws_rmsnorm_backward_static", gpu_ptr, gpu_ptr, gpu_ptr, gpu_ptr, gpu_ptr,
                  gpu_ptr, 8, 8200, 1, None)


def test_rmsnorm_backward_partial_rows_per_width():
    """Partial weight-gradient rows: one per 32 rows up to 2048 columns; wider rows take one
    block per row with 4 to 32 rows per block, the most that leaves at least 512 blocks."""
    q = lambda rows, d: _hip.query("ws_rmsnorm_backward_partial_floats", rows, d)
    assert q(16384, 2048) == 512 * 2048 and q(33, 100) == 2 * 100
    assert q(16384, 4096) == 512 * 4096   # 32 rows per block
    assert q(4096, 8192) == 512 * 8192    # 8 rows per block
    assert q(1000, 2056) == 250 * 2056    # 4 rows per block (fewer than 512 blocks)
    assert q(65536, 4096) == 2048 * 4096  # 32 rows per block


def test_transpose_refuses_shapes_beyond_its_grid_before_any_launch():
    """The weight transpose runs 64-row blocks along the grid's y dimension; more rows than
    65535 blocks cover are refused with an error before any device call, as are strides
    shorter than a row."""
    gpu_ptr = 1 << 20  # never dereferenced
    with pytest.raises(RuntimeError, match="exceeds 4194240"):
        _hip.call("ws_transpose_bf16", gpu_ptr, 8, gpu_ptr, 65535 * 64 + 1, 8, None)
    with pytest.raises(RuntimeError, match="invalid transpose shape"):
        _hip.call("ws_transpose_bf16", gpu_ptr, 4, gpu_ptr, 8, 8, None)
