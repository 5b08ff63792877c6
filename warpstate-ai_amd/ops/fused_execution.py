"""Fused BF16 GEMMs of the WarpState training step on gfx950 (additive entry points).

The reference composes these from separate operators; here each is one GEMM launch whose
prologue or epilogue does the extra work in registers:

* ``rmsnorm_gate_mm``: RMSNorm (warpstate/model.py:22-28) before the fused input
  projection (warpstate/model.py:93,109), with sigmoid on the gate column range
  (warpstate/model.py:174) in the GEMM's epilogue. A row pass (x read once, held in
  registers) writes the normalized rows y and rstd; the GEMM then reads y. y has to reach
  HBM anyway, as the saved input of the projection's weight gradient, and its per-element
  BF16 roundings r(r(x rstd) r(w)) keep rstd from being factored out of the product.
* ``residual_mm``: down projection plus the BF16 residual add (warpstate/model.py:178,
  ops/residual_experiment.py:25-58).
* ``swiglu_backward_mm``: the down projection's input gradient (ops/matmul_execution.py:239)
  with the SwiGLU backward (ops/activation_execution.py:36-55) as its epilogue.
* ``mm_accumulate_``: weight-gradient GEMM accumulated into an FP32 buffer,
  G += f32(r(dW)) (test_gradient_execution.py:243-246).
* ``linear_cross_entropy_*``: the tied LM head with fused cross-entropy
  (warpstate/model.py:316-334, ops/loss_experiment.py:14-19); the full [rows, vocab]
  logits never exist in HBM (the two-pass mode keeps them in registers only; the one-pass
  mode holds one row chunk's BF16 logits in its workspace at a time).
* ``mlp_backward``: the SwiGLU MLP backward at training shape built from the above.
"""

from __future__ import annotations

import torch

from ops import _hip

# Rows per LM-head backward chunk. At d = 2048 one 8192-row chunk's dHidden GEMM is 256
# tiles, one full round on 256 CUs without a vocabulary split; its BF16 logit gradients
# take 512 MiB at vocab 32768 (config 5: 5 % faster than 4096-row chunks, both with and
# without stored logits).
DEFAULT_CE_CHUNK_ROWS = 8192


def _check_bf16_cuda(*tensors):
    for tensor in tensors:
        if not tensor.is_cuda:
            raise ValueError("Fused matrix kernels require CUDA tensors")
        if tensor.dtype != torch.bfloat16:
            raise ValueError("Fused matrix kernels require BF16 operands")


def _check_buffer(t: torch.Tensor, shape: tuple, dtype: torch.dtype, device: torch.device,
                  name: str, contiguous: bool = True) -> None:
    """A caller-supplied output or workspace must have exactly the shape, dtype and device
    the launch writes, and be contiguous (or, with ``contiguous=False``, have a unit
    column stride), so that no kernel writes outside it."""
    if tuple(t.shape) != tuple(shape) or t.dtype != dtype or t.device != device:
        raise ValueError(f"{name} must be a {str(dtype).removeprefix('torch.')} tensor of "
                         f"shape {list(shape)} on {device}")
    if contiguous and not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if not contiguous and t.ndim == 2 and t.stride(1) != 1:
        raise ValueError(f"{name} must have a unit column stride")


# Rows of A from which a transposed copy of an N-contiguous B pays for itself: the copy
# moves 4 |B| bytes once, the GEMM reads B's tiles once per 256-row block of A.
TRANSPOSE_MIN_ROWS = 1024


def transpose(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Contiguous ``x.T`` of a 2-D BF16 CUDA tensor with unit column stride (HIP kernel)."""
    _check_bf16_cuda(x)
    if x.ndim != 2 or x.stride(1) != 1:
        raise ValueError("transpose expects a 2-D tensor with unit column stride")
    rows, cols = x.shape
    if out is None:
        out = torch.empty((cols, rows), dtype=x.dtype, device=x.device)
    _hip.call("ws_transpose_bf16", x.data_ptr(), x.stride(0), out.data_ptr(), rows, cols,
              _hip.stream(x))
    return out


def k_contiguous_b(b: torch.Tensor, rows_a: int) -> torch.Tensor:
    """B [K, N] as a view whose reduction dim is contiguous: when B is N-contiguous (a
    weight in an input-gradient GEMM, dX = dY @ W, or a forward weight stored [K, N]
    row-major) and A has enough rows to amortize it, a transposed copy W^T [N, K] viewed
    as [K, N]; otherwise B itself. The copy is exact, so results are the same bits."""
    if (rows_a >= TRANSPOSE_MIN_ROWS and b.stride(1) == 1 and b.stride(0) >= b.shape[1]
            and b.shape[0] > 1):
        return transpose(b).T
    return b


def mm(a: torch.Tensor, b: torch.Tensor, algorithm: str = "tiled", tile: int = 0) -> torch.Tensor:
    """r(a @ b) with the HIP GEMM; `tile` 0 = 256x256, 1 = 128x128."""
    _check_bf16_cuda(a, b)
    if a.ndim != 2 or b.ndim != 2 or a.shape[1] != b.shape[0]:
        raise ValueError(f"Expected a [M, K] and b [K, N], got {list(a.shape)} and {list(b.shape)}")
    if tile == 0:
        b = k_contiguous_b(b, a.shape[0])
    m, k = a.shape
    n = b.shape[1]
    out = torch.empty((m, n), dtype=torch.bfloat16, device=a.device)
    _hip.call("ws_mm", a.data_ptr(), a.stride(0), a.stride(1), b.data_ptr(), b.stride(0),
              b.stride(1), out.data_ptr(), m, n, k, _hip.algorithm_code(algorithm), tile,
              _hip.stream(a))
    return out


def dgrad_mm(grad: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """Input gradient r(grad @ weight) of a bias-free projection: grad [M, N] (the output's
    gradient) and the BF16 weight [N, K] in nn.Linear layout; returns [M, K]
    (ops/matmul_execution.py:239).

    This library's GEMM (``ws_mm``, FP32 accumulation, one BF16 rounding) on the
    persistent grid (one workgroup per CU looping over the tiles: 2.5-3.5 % faster than a
    workgroup per tile at 16384 x 2048 x 9216 / x 11264, bit-identical), with the weight
    first copied K-contiguous by the HIP transpose kernel (``k_contiguous_b``) when grad
    has enough rows to amortize the copy.
    """
    _check_bf16_cuda(grad, weight)
    if grad.dim() != 2 or weight.dim() != 2 or grad.shape[1] != weight.shape[0]:
        raise ValueError("Expected grad [M, N] and weight [N, K]")
    return mm(grad, weight, "persistent")


def rmsnorm_gate_mm(x: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                    weight: torch.Tensor, gate: tuple[int, int] = (0, 0),
                    out: torch.Tensor | None = None, rstd: torch.Tensor | None = None,
                    normed: torch.Tensor | None = None
                    ) -> tuple[torch.Tensor, torch.Tensor]:
    """``(r(RMSNorm(x) @ weight.T) with sigmoid on columns [gate), rstd)``.

    x [M, K] BF16 with unit column stride; norm_weight [K] FP32; weight [N, K] BF16 in
    nn.Linear layout; gate = (begin, end) output columns that get r(sigmoid(.)).
    ``normed`` [M, K] BF16 receives the normalized operand RMSNorm(x) (the saved input of
    the projection's weight gradient); it is allocated when not given.
    """
    _check_bf16_cuda(x, weight)
    if x.ndim != 2 or weight.ndim != 2 or x.shape[1] != weight.shape[1]:
        raise ValueError("Expected x [M, K] and weight [N, K]")
    if x.stride(1) != 1:
        raise ValueError("The RMSNorm prologue needs a unit column stride")
    if norm_weight.dtype != torch.float32 or not norm_weight.is_contiguous():
        raise ValueError("RMSNorm weight must be a contiguous FP32 vector")
    m, k = x.shape
    n = weight.shape[0]
    if norm_weight.shape != (k,) or norm_weight.device != x.device:
        raise ValueError("RMSNorm weight must have one FP32 value per feature, on x's device")
    if not 0 <= gate[0] <= gate[1] <= n:
        raise ValueError(f"gate columns {tuple(gate)} outside [0, {n}]")
    if out is None:
        out = torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    _check_buffer(out, (m, n), torch.bfloat16, x.device, "out")
    if rstd is None:
        rstd = torch.empty((m,), dtype=torch.float32, device=x.device)
    _check_buffer(rstd, (m,), torch.float32, x.device, "rstd")
    if normed is None:
        normed = torch.empty((m, k), dtype=torch.bfloat16, device=x.device)
    _check_buffer(normed, (m, k), torch.bfloat16, x.device, "normed")
    # A weight stored [K, N] (N-contiguous B) is copied K-contiguous first, as for dX.
    b = k_contiguous_b(weight.T, m)
    _hip.call("ws_rmsnorm_gate_mm", x.data_ptr(), x.stride(0), norm_weight.data_ptr(),
              float(eps), rstd.data_ptr(), normed.data_ptr(), b.data_ptr(), b.stride(0),
              b.stride(1), out.data_ptr(), m, n, k, int(gate[0]), int(gate[1]), _hip.stream(x))
    return out, rstd


def sigmoid_backward_cols(dout: torch.Tensor, out: torch.Tensor, gate: tuple[int, int],
                          dp: torch.Tensor | None = None) -> torch.Tensor:
    """Gradient of the projection before the gate sigmoid: dout with columns [gate)
    replaced by r(dout (1 - out) out). ``dp=dout`` rewrites only the gate columns in place."""
    _check_bf16_cuda(dout, out)
    if dout.shape != out.shape or dout.stride(1) != 1 or out.stride(1) != 1:
        raise ValueError("dout and out must be matching [M, N] tensors with unit column stride")
    if dp is None:
        dp = torch.empty_like(dout)
    _check_buffer(dp, dout.shape, torch.bfloat16, dout.device, "dp", contiguous=False)
    rows, cols = dout.shape
    if not 0 <= gate[0] <= gate[1] <= cols:
        raise ValueError(f"gate columns {tuple(gate)} outside [0, {cols}]")
    _hip.call("ws_sigmoid_backward_cols", dout.data_ptr(), dout.stride(0), out.data_ptr(),
              out.stride(0), dp.data_ptr(), dp.stride(0), rows, cols, int(gate[0]),
              int(gate[1]), _hip.stream(dout))
    return dp


def rmsnorm_gate_mm_backward(x: torch.Tensor, norm_weight: torch.Tensor, rstd: torch.Tensor,
                             normed: torch.Tensor, weight: torch.Tensor, gate: tuple[int, int],
                             out: torch.Tensor, dout: torch.Tensor, weight_grad: torch.Tensor,
                             eager_rounding: bool = True, in_place: bool = False
                             ) -> tuple[torch.Tensor, torch.Tensor]:
    """Backward of ``rmsnorm_gate_mm``: returns (dx BF16 [M, K], d norm_weight FP32 [K]) and
    accumulates the projection weight's gradient, weight_grad [N, K] += f32(r(dP^T y)).

    dP is dout through the gate sigmoid (``sigmoid_backward_cols``; ``in_place`` reuses
    dout's storage), dy = r(dP @ W) (``dgrad_mm``, ops/matmul_execution.py:239), then the RMSNorm
    backward of ops/activation_execution.py:113-158 with the saved rstd.
    """
    from ops.activation_execution import _rms_backward

    dp = sigmoid_backward_cols(dout, out, gate, dout if in_place else None)
    dy = dgrad_mm(dp, weight)
    mm_accumulate_(weight_grad, dp.T, normed, True)
    dx, dnorm = _rms_backward(x, norm_weight, rstd, dy, eager_rounding)
    return dx, dnorm


def residual_mm(a: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """r(residual + r(a @ weight.T)); a [M, K], weight [N, K], residual [M, N] (unit
    column stride)."""
    _check_bf16_cuda(a, weight, residual)
    m, k = a.shape
    n = weight.shape[0]
    if weight.shape[1] != k or residual.shape != (m, n) or residual.stride(1) != 1:
        raise ValueError("Expected a [M, K], weight [N, K] and a row-major residual [M, N]")
    if out is None:
        out = torch.empty((m, n), dtype=torch.bfloat16, device=a.device)
    _check_buffer(out, (m, n), torch.bfloat16, a.device, "out")
    b = k_contiguous_b(weight.T, m)
    _hip.call("ws_residual_mm", a.data_ptr(), a.stride(0), a.stride(1), b.data_ptr(),
              b.stride(0), b.stride(1), residual.data_ptr(), residual.stride(0),
              out.data_ptr(), m, n, k, _hip.stream(a))
    return out


def swiglu_backward_mm(grad: torch.Tensor, down_weight: torch.Tensor, packed: torch.Tensor,
                       eager_rounding: bool = True,
                       out: torch.Tensor | None = None) -> torch.Tensor:
    """dPacked [M, 2H] from dY [M, d], the down weight [d, H] (nn.Linear layout) and the
    saved packed projection [M, 2H] (contiguous)."""
    _check_bf16_cuda(grad, down_weight, packed)
    m, k = grad.shape
    h = down_weight.shape[1]
    if down_weight.shape[0] != k or packed.shape != (m, 2 * h) or not packed.is_contiguous():
        raise ValueError("Expected dY [M, d], down weight [d, H], contiguous packed [M, 2H]")
    if out is None:
        out = torch.empty((m, 2 * h), dtype=torch.bfloat16, device=grad.device)
    _check_buffer(out, (m, 2 * h), torch.bfloat16, grad.device, "out")
    down_weight = k_contiguous_b(down_weight, m)
    _hip.call("ws_swiglu_backward_mm", grad.data_ptr(), grad.stride(0), grad.stride(1),
              down_weight.data_ptr(), down_weight.stride(0), down_weight.stride(1),
              packed.data_ptr(), out.data_ptr(), m, h, k, int(eager_rounding), _hip.stream(grad))
    return out


def auto_splits(m: int, n: int, k: int, cus: int = 256, tile: int = 256,
                max_splits: int = 4, min_k_tiles: int = 16) -> int:
    """Split-K factor for an [m, n] output with reduction k: the one (fewest on ties) that
    fills the last round of 256 x 256 tiles on ``cus`` compute units best, keeping at
    least ``min_k_tiles`` 64-wide k-tiles per split. With at least as many tiles as compute
    units the library turns any factor above 1 into a balanced split (whole rounds of tiles
    direct, the remaining tiles' k-range shared by all compute units)."""
    tiles = -(-m // tile) * -(-n // tile)
    best, best_eff = 1, 0.0
    for s in range(1, max_splits + 1):
        if s > 1 and -(-k // 64) // s < min_k_tiles:
            break
        work = tiles * s
        eff = work / (-(-work // cus) * cus)
        if eff > best_eff + 1e-9:
            best, best_eff = s, eff
    return best


def mm_accumulate_(g: torch.Tensor, a: torch.Tensor, b: torch.Tensor, round_bf16: bool = True,
                   splits: int | None = None, workspace: torch.Tensor | None = None,
                   _entry: str = "ws_mm_accumulate_f32") -> torch.Tensor:
    """G += f32(r(a @ b)) (or G += a @ b in FP32 when ``round_bf16`` is False), in place.

    G is FP32 [M, N] with unit column stride. ``splits`` > 1 lets the reduction be split
    through an FP32 workspace (``ws_mm_accumulate_workspace_floats`` floats): balanced
    stream-K shares for vector operand layouts, ``splits`` even slices otherwise (None:
    chosen by ``auto_splits``)."""
    _check_bf16_cuda(a, b)
    if g.dtype != torch.float32 or g.stride(1) != 1:
        raise ValueError("Gradient buffer must be FP32 with unit column stride")
    m, k = a.shape
    n = b.shape[1]
    if g.shape != (m, n) or b.shape[0] != k:
        raise ValueError("Gradient buffer shape must match a @ b")
    if splits is None:
        splits = auto_splits(m, n, k, torch.cuda.get_device_properties(g.device).multi_processor_count)
    need = _hip.query("ws_mm_accumulate_workspace_floats", m, n, k, splits)
    if need and (workspace is None or workspace.numel() < need):
        workspace = torch.empty((need,), dtype=torch.float32, device=g.device)
    _hip.call(_entry, a.data_ptr(), a.stride(0), a.stride(1), b.data_ptr(),
              b.stride(0), b.stride(1), g.data_ptr(), g.stride(0), m, n, k, int(round_bf16),
              None if not need else workspace.data_ptr(), splits, _hip.stream(a))
    return g


def mm_f32(a: torch.Tensor, b: torch.Tensor, round_bf16: bool = True,
           out: torch.Tensor | None = None, splits: int | None = None) -> torch.Tensor:
    """f32(r(a @ b)) as a new FP32 [M, N] tensor (``out`` when given), written in one pass
    by the FP32 GEMM epilogue without reading or clearing the buffer
    (``ws_mm_store_f32``): the BF16 weight gradient of F.linear widened to FP32.
    ``splits`` as in ``mm_accumulate_``."""
    m, n = a.shape[0], b.shape[1]
    if out is None:
        out = torch.empty((m, n), dtype=torch.float32, device=a.device)
    return mm_accumulate_(out, a, b, round_bf16, splits, _entry="ws_mm_store_f32")


def mm_accumulate_group_(items, round_bf16: bool = True,
                         workspace: torch.Tensor | None = None,
                         _entry: str = "ws_mm_accumulate_f32_group") -> None:
    """G_i += f32(r(a_i @ b_i)) for up to four (G_i, a_i, b_i) with the same reduction
    length, in place and in one launch (``ws_mm_accumulate_f32_group``): the tiles of all
    gradients share the GPU, so a gradient with fewer 256 x 256 tiles than compute units
    does not leave the rest idle. Each G_i is FP32 with unit column stride; the G_i must
    not overlap."""
    rows = []
    k = None
    for g, a, b in items:
        _check_bf16_cuda(a, b)
        if g.dtype != torch.float32 or g.stride(1) != 1:
            raise ValueError("Gradient buffer must be FP32 with unit column stride")
        m, ka = a.shape
        n = b.shape[1]
        if g.shape != (m, n) or b.shape[0] != ka:
            raise ValueError("Gradient buffer shape must match a @ b")
        if k is not None and ka != k:
            raise ValueError("Grouped gradients must share the reduction length")
        k = ka
        rows.append((a.data_ptr(), a.stride(0), a.stride(1), b.data_ptr(), b.stride(0),
                     b.stride(1), g.data_ptr(), g.stride(0), m, n))
    if not rows:
        return
    table = _hip.problem_table(rows)
    first = items[0][0]
    need = _hip.query("ws_mm_accumulate_group_workspace_floats", table, len(rows), k)
    if need and (workspace is None or workspace.numel() < need):
        workspace = torch.empty((need,), dtype=torch.float32, device=first.device)
    _hip.call(_entry, table, len(rows), k, int(round_bf16),
              None if not need else workspace.data_ptr(), _hip.stream(items[0][1]))


def mm_f32_group(pairs, round_bf16: bool = True) -> list[torch.Tensor]:
    """[f32(r(a_i @ b_i))] for up to four (a_i, b_i) with the same reduction length, as new
    FP32 tensors written in one launch without clearing (``ws_mm_store_f32_group``): the
    weight gradients of one backward stage sharing the GPU's tiles."""
    outs = [torch.empty((a.shape[0], b.shape[1]), dtype=torch.float32, device=a.device)
            for a, b in pairs]
    mm_accumulate_group_([(g, a, b) for g, (a, b) in zip(outs, pairs)], round_bf16,
                         _entry="ws_mm_store_f32_group")
    return outs


class CrossEntropyState:
    """Per-call buffers of the fused LM-head cross-entropy, in one of three modes:

    * default: the forward keeps only row statistics; the backward recomputes each chunk's
      logits with a GEMM whose epilogue forms the logit gradients;
    * ``fused``: the forward computes, chunk by chunk, the loss and the gradients for a
      unit upstream gradient (``ws_linear_ce_fused``: one logits GEMM per row, whose BF16
      logits live only in the one-chunk workspace); the backward scales them by the actual
      upstream gradient. Needs ``d``; ``weight_grad`` also keeps the head weight's
      unit gradient (FP32 [vocab, d]);
    * ``store_logits``: the forward keeps the full BF16 logits ([rows, vocab]) and the
      backward reads them instead of recomputing the logits GEMM.
    """

    def __init__(self, rows, vocab, device, chunk_rows=DEFAULT_CE_CHUNK_ROWS, d=None,
                 store_logits=False, fused=False, weight_grad=False):
        if fused and store_logits:
            raise ValueError("A cross-entropy state is either fused or stores the logits")
        if fused and d is None:
            raise ValueError("A fused cross-entropy state needs the hidden width d")
        parts = _hip.query("ws_linear_ce_parts", vocab)
        f32 = dict(dtype=torch.float32, device=device)
        self.part_max = torch.empty((rows, parts), **f32)
        self.part_sum = torch.empty((rows, parts), **f32)
        self.target_logit = torch.empty((rows,), **f32)
        self.lse = torch.empty((rows,), **f32)
        self.loss = torch.empty((rows,), **f32)
        self.mean = torch.empty((), **f32)
        self.count = torch.empty((), dtype=torch.int64, device=device)
        self.rows, self.vocab, self.d = rows, vocab, d
        self.chunk_rows = min(chunk_rows, rows)
        self.logits = (torch.empty((rows, vocab), dtype=torch.bfloat16, device=device)
                       if store_logits else None)
        self.fused = fused
        self.dhidden_unit = (torch.empty((rows, d), dtype=torch.bfloat16, device=device)
                             if fused else None)
        self.dweight_unit = (torch.empty((vocab, d), **f32) if fused and weight_grad else None)
        self.weight_t = None
        self.workspace = None
        if d is not None:
            self.backward_workspace(d)

    def backward_workspace(self, d):
        """The chunk workspace (scale, one chunk of BF16 logits / logit gradients, split-K
        partials), allocated once per hidden width; 256-byte aligned by the allocator."""
        need = _hip.query("ws_linear_ce_workspace_bytes", self.rows, self.vocab, d,
                          self.chunk_rows)
        if self.workspace is None or self.workspace.numel() < need:
            self.workspace = torch.empty((need,), dtype=torch.uint8, device=self.lse.device)
        return self.workspace


def _check_ce(hidden, weight, targets):
    _check_bf16_cuda(hidden, weight)
    if hidden.ndim != 2 or weight.ndim != 2 or hidden.shape[1] != weight.shape[1]:
        raise ValueError("Expected hidden [rows, d] and weight [vocab, d]")
    if hidden.stride(1) != 1 or weight.stride(1) != 1:
        raise ValueError("LM-head operands need a unit column stride")
    if targets.dtype != torch.int64 or targets.shape != (hidden.shape[0],) or not targets.is_contiguous():
        raise ValueError("Targets must be a contiguous int64 vector, one per row")


def _check_state(state: CrossEntropyState, rows: int, vocab: int, device) -> None:
    """The state's buffers are indexed by the operands' rows and vocabulary: a state built
    for another shape or device would be written out of bounds, so it is refused."""
    if not isinstance(state, CrossEntropyState):
        raise TypeError("state must be a CrossEntropyState")
    if (state.rows, state.vocab) != (rows, vocab):
        raise ValueError(f"CrossEntropyState was built for {state.rows} rows and vocabulary "
                         f"{state.vocab}, not {rows} and {vocab}")
    if state.lse.device != device:
        raise ValueError("CrossEntropyState buffers are on another device")
    parts = _hip.query("ws_linear_ce_parts", vocab)
    for name, buffer, shape, dtype in (("part_max", state.part_max, (rows, parts), torch.float32),
                                       ("part_sum", state.part_sum, (rows, parts), torch.float32),
                                       ("target_logit", state.target_logit, (rows,), torch.float32),
                                       ("lse", state.lse, (rows,), torch.float32),
                                       ("loss", state.loss, (rows,), torch.float32),
                                       ("mean", state.mean, (), torch.float32),
                                       ("count", state.count, (), torch.int64)):
        _check_buffer(buffer, shape, dtype, device, "state." + name)
    if state.logits is not None:
        _check_buffer(state.logits, (rows, vocab), torch.bfloat16, device, "state.logits")
    if state.fused:
        _check_buffer(state.dhidden_unit, (rows, state.d), torch.bfloat16, device,
                      "state.dhidden_unit")
        if state.dweight_unit is not None:
            _check_buffer(state.dweight_unit, (vocab, state.d), torch.float32, device,
                          "state.dweight_unit")
    if not 1 <= state.chunk_rows <= rows:
        raise ValueError("CrossEntropyState chunk_rows must lie in [1, rows]")


def linear_cross_entropy_forward(hidden: torch.Tensor, weight: torch.Tensor,
                                 targets: torch.Tensor, state: CrossEntropyState | None = None
                                 ) -> CrossEntropyState:
    """Per-token loss, lse, mean over valid tokens and their count, for hidden [rows, d],
    weight [vocab, d] and int64 targets (-100 ignored)."""
    _check_ce(hidden, weight, targets)
    rows, d = hidden.shape
    vocab = weight.shape[0]
    if state is None:
        state = CrossEntropyState(rows, vocab, hidden.device)
    _check_state(state, rows, vocab, hidden.device)
    if state.fused:
        if state.d != d:
            raise ValueError(f"The fused CrossEntropyState was built for d={state.d}, not {d}")
        workspace = state.backward_workspace(d)
        weight_t = transpose(weight) if rows >= TRANSPOSE_MIN_ROWS else None
        # Kept for the backward's two-pass fallback (an upstream gradient that is not a
        # power of two).
        state.weight_t = weight_t
        if state.dweight_unit is not None:
            state.dweight_unit.zero_()
        _hip.call("ws_linear_ce_fused", hidden.data_ptr(), hidden.stride(0), weight.data_ptr(),
                  weight.stride(0), _hip.ptr(weight_t), targets.data_ptr(), rows, vocab, d,
                  state.part_max.data_ptr(), state.part_sum.data_ptr(),
                  state.target_logit.data_ptr(), state.lse.data_ptr(), state.loss.data_ptr(),
                  state.mean.data_ptr(), state.count.data_ptr(), workspace.data_ptr(),
                  state.chunk_rows, state.dhidden_unit.data_ptr(), state.dhidden_unit.stride(0),
                  _hip.ptr(state.dweight_unit),
                  0 if state.dweight_unit is None else state.dweight_unit.stride(0),
                  _hip.stream(hidden))
        return state
    _hip.call("ws_linear_ce_forward", hidden.data_ptr(), hidden.stride(0), weight.data_ptr(),
              weight.stride(0), targets.data_ptr(), rows, vocab, d, state.part_max.data_ptr(),
              state.part_sum.data_ptr(), state.target_logit.data_ptr(), state.lse.data_ptr(),
              state.loss.data_ptr(), state.mean.data_ptr(), state.count.data_ptr(),
              _hip.ptr(state.logits), _hip.stream(hidden))
    return state


def linear_cross_entropy_backward(hidden: torch.Tensor, weight: torch.Tensor,
                                  targets: torch.Tensor, state: CrossEntropyState,
                                  grad_mean: torch.Tensor,
                                  out: torch.Tensor | None = None,
                                  weight_grad: torch.Tensor | None = None) -> torch.Tensor:
    """dHidden [rows, d] BF16 of ``mean`` given its FP32 scalar gradient.

    ``weight_grad`` (FP32 [vocab, d], unit column stride), when given, accumulates the tied
    head weight's gradient chunk by chunk: weight_grad += f32(r(G_chunk^T @ hidden_chunk)).
    """
    _check_ce(hidden, weight, targets)
    rows, d = hidden.shape
    vocab = weight.shape[0]
    _check_state(state, rows, vocab, hidden.device)
    if grad_mean.numel() != 1 or grad_mean.device != hidden.device:
        raise ValueError("grad_mean must be one value on the operands' device")
    grad_mean = grad_mean.reshape(1).to(torch.float32).contiguous()
    if out is None:
        out = torch.empty((rows, d), dtype=torch.bfloat16, device=hidden.device)
    _check_buffer(out, (rows, d), torch.bfloat16, hidden.device, "out", contiguous=False)
    if weight_grad is not None:
        _check_buffer(weight_grad, (vocab, d), torch.float32, hidden.device, "weight_grad",
                      contiguous=state.fused)
    if state.fused:
        if state.d != d:
            raise ValueError(f"The fused CrossEntropyState was built for d={state.d}, not {d}")
        if weight_grad is not None and state.dweight_unit is None:
            raise ValueError("This fused CrossEntropyState was built without weight_grad")
        _hip.call("ws_linear_ce_fused_backward", hidden.data_ptr(), hidden.stride(0),
                  weight.data_ptr(), weight.stride(0), _hip.ptr(state.weight_t),
                  targets.data_ptr(), state.lse.data_ptr(), state.count.data_ptr(),
                  grad_mean.data_ptr(), rows, vocab, d, state.backward_workspace(d).data_ptr(),
                  state.chunk_rows, state.dhidden_unit.data_ptr(), state.dhidden_unit.stride(0),
                  None if weight_grad is None else state.dweight_unit.data_ptr(),
                  out.data_ptr(), out.stride(0), _hip.ptr(weight_grad), _hip.stream(hidden))
        return out
    workspace = state.backward_workspace(d)
    # The dHidden GEMM reads the head weight along the vocabulary: give it W^T rows.
    weight_t = transpose(weight) if rows >= TRANSPOSE_MIN_ROWS else None
    _hip.call("ws_linear_ce_backward", hidden.data_ptr(), hidden.stride(0), weight.data_ptr(),
              weight.stride(0), None if weight_t is None else weight_t.data_ptr(),
              targets.data_ptr(), state.lse.data_ptr(), state.count.data_ptr(),
              grad_mean.data_ptr(), rows, vocab, d, workspace.data_ptr(), state.chunk_rows,
              out.data_ptr(), out.stride(0),
              None if weight_grad is None else weight_grad.data_ptr(),
              0 if weight_grad is None else weight_grad.stride(0), _hip.ptr(state.logits),
              _hip.stream(hidden))
    return out


def _bf16_rows(t: torch.Tensor) -> torch.Tensor:
    """BF16 copy (or the tensor itself) with a unit column stride, as the kernels take."""
    t = t.to(torch.bfloat16)
    return t if t.stride(-1) == 1 else t.contiguous()


class LinearCrossEntropy(torch.autograd.Function):
    """(mean, per-token loss) of cross-entropy over r(hidden @ weight.T), the tied LM head
    of warpstate/model.py:316-334, with gradients to ``hidden`` and ``weight``.

    ``hidden`` [rows, d] and ``weight`` [vocab, d] may be BF16 or FP32; FP32 operands are
    rounded to BF16 first, as F.linear under BF16 autocast does. The weight's gradient is
    accumulated in FP32 chunk by chunk, sum_c f32(r(G_c^T h_c)); an FP32 weight (the
    master parameter) receives that FP32 sum, a BF16 weight its BF16 rounding. The
    per-token loss is not differentiable.

    ``mode`` picks how the gradients are formed when they are needed:
    ``"fused"`` (default) computes them in the forward for a unit upstream gradient, while
    each chunk's logits are at hand (one logits GEMM per row), and the backward scales them;
    that is exact for an upstream gradient 2^e with |e| <= 32. Any other upstream gradient
    (for example a loss divided by 3 microbatches) makes the backward run the two-pass
    backward on top, a second logits GEMM plus the dHidden and weight GEMMs again, about
    twice the LM head's cost. ``"two_pass"`` keeps only row statistics in the forward and
    always recomputes the logits in the backward: the right choice when such upstream
    gradients are expected."""

    @staticmethod
    def forward(ctx, hidden, weight, targets, chunk_rows=DEFAULT_CE_CHUNK_ROWS, mode="fused"):
        if mode not in ("fused", "two_pass"):
            raise ValueError(f"mode must be 'fused' or 'two_pass', not {mode!r}")
        h, w = _bf16_rows(hidden), _bf16_rows(weight)
        wants = ctx.needs_input_grad
        fused = mode == "fused" and (wants[0] or wants[1])
        state = CrossEntropyState(h.shape[0], w.shape[0], h.device, chunk_rows, d=h.shape[1],
                                  fused=fused, weight_grad=fused and wants[1])
        linear_cross_entropy_forward(h, w, targets, state)
        ctx.save_for_backward(h, w, targets)
        ctx.state = state
        ctx.dtypes = (hidden.dtype, weight.dtype)
        ctx.mark_non_differentiable(state.loss)
        return state.mean.clone(), state.loss

    @staticmethod
    def backward(ctx, grad_mean, _grad_loss):
        h, w, targets = ctx.saved_tensors
        if grad_mean is None:
            grad_mean = torch.zeros((), dtype=torch.float32, device=h.device)
        want_h, want_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        weight_grad = (torch.zeros(w.shape, dtype=torch.float32, device=w.device)
                       if want_w else None)
        dh = linear_cross_entropy_backward(h, w, targets, ctx.state, grad_mean,
                                           weight_grad=weight_grad)
        hidden_dtype, weight_dtype = ctx.dtypes
        return (dh.to(hidden_dtype) if want_h else None,
                weight_grad.to(weight_dtype) if want_w else None, None, None, None)


@torch.compiler.disable
def linear_cross_entropy(hidden, weight, targets, chunk_rows=DEFAULT_CE_CHUNK_ROWS,
                         mode="fused"):
    """(mean, per-token loss) of the fused LM head, with autograd to hidden and weight
    (``mode``: see ``LinearCrossEntropy``). Under torch.compile it runs eagerly (a graph
    break), with its own buffers."""
    return LinearCrossEntropy.apply(hidden, weight, targets, chunk_rows, mode)


def mlp_backward(x: torch.Tensor, w_upgate: torch.Tensor, w_down: torch.Tensor,
                 packed: torch.Tensor, act: torch.Tensor, dy: torch.Tensor,
                 g_upgate: torch.Tensor, g_down: torch.Tensor, eager_rounding: bool = True,
                 dw_splits: int | None = None,
                 dpacked: torch.Tensor | None = None) -> torch.Tensor:
    """Backward of y = down(silu(gate) * up) with (up | gate) = x @ w_upgate.T.

    x [M, d], w_upgate [2H, d], w_down [d, H] (nn.Linear layouts, BF16), packed [M, 2H] and
    act [M, H] saved from the forward, dy [M, d]. Accumulates G_down [d, H] += f32(r(dY^T act))
    and G_upgate [2H, d] += f32(r(dPacked^T x)); returns dX [M, d]. Restates
    ops/matmul_execution.py:236-244 and :314-319 with the SwiGLU backward fused on the
    dAct GEMM. ``dpacked`` (contiguous BF16 [M, 2H]), when given, receives the gradient of
    the packed projection.
    """
    dpacked = swiglu_backward_mm(dy, w_down, packed, eager_rounding, out=dpacked)
    dx = dgrad_mm(dpacked, w_upgate)
    if dw_splits is None:
        # Both weight gradients reduce over the tokens: one launch fills the GPU with them.
        mm_accumulate_group_([(g_down, dy.T, act), (g_upgate, dpacked.T, x)], True)
    else:
        mm_accumulate_(g_down, dy.T, act, True, dw_splits)
        mm_accumulate_(g_upgate, dpacked.T, x, True, dw_splits)
    return dx
