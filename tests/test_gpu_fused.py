"""GPU parity of the fused GEMMs against the CPU oracle at reduced sizes.

* paired SwiGLU GEMM: test_matmul_epilogue.py:54-84 restated (shapes, tiles, schedules,
  both roundings; projection vs FP32 dot; activation recomputed from the returned packed);
* RMSNorm-prologue projection with gate sigmoid, residual epilogue, SwiGLU-backward
  epilogue, FP32 weight-gradient accumulation (plain and split-K), the MLP backward, and
  the fused LM-head cross-entropy (loss, mean, count, dHidden).
Bars: BF16 max|d|/max|ref| <= 1e-2 and rel-RMS <= 3e-3; FP32 ||d||/||ref|| <= 1e-3;
counts bit-exact.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from metrics import assert_bf16_close, assert_f32_close, max_rel, rel_l2
from oracle import reference as oracle

pytestmark = pytest.mark.gpu


def _gen(seed):
    return torch.Generator("cpu").manual_seed(seed)


@pytest.mark.parametrize("algorithm", ["tiled", "persistent"])
@pytest.mark.parametrize("eager_rounding", [False, True])
@pytest.mark.parametrize("shape", [(13, 46, 31), (128, 256, 128), (257, 192, 193), (512, 1024, 256),
                                   (300, 272, 200), (520, 528, 1000)])
@pytest.mark.parametrize("tile", [(64, 64, 32, 4, 3), (128, 128, 32, 8, 3)])
def test_swiglu_projection_and_activation(algorithm, eager_rounding, shape, tile):
    """(M, 2H, K). The last two shapes take the 256 x 256 paired kernel (K a multiple of 8)
    with every edge ragged: partial row tiles, a half width H that is not a multiple of
    the 128 columns a paired tile holds per half, and a partial last k-tile."""
    from ops.matmul_epilogue import launch_swiglu_mm

    m, packed_width, k = shape
    gen = _gen(561)
    a = (torch.randn(m, k, generator=gen) * 0.1).bfloat16()
    b = (torch.randn(packed_width, k, generator=gen) * 0.1).bfloat16().T
    packed, act = launch_swiglu_mm(a.cuda(), b.cuda(), algorithm, tile, eager_rounding)
    torch.cuda.synchronize()
    want_packed, want_act = oracle.swiglu_mm(a, b, eager_rounding)
    assert packed.is_contiguous() and act.is_contiguous()
    assert_bf16_close(packed, want_packed, "packed")
    assert_bf16_close(act, want_act, "act")
    accumulated = oracle.mm_f32_reference(a, b)
    assert rel_l2(packed, accumulated) < 1e-3
    # The activation must consume the returned rounded projection.
    torch.testing.assert_close(act.cpu(), oracle.swiglu(packed.cpu(), eager_rounding),
                               rtol=0.01, atol=2e-4)


def test_swiglu_zero_gate_weights_give_exact_zero():
    from ops.matmul_epilogue import launch_swiglu_mm

    gen = _gen(3)
    a = torch.randn(256, 128, generator=gen).bfloat16()
    w = torch.randn(512, 128, generator=gen).bfloat16()
    w[256:] = 0  # gate half
    packed, act = launch_swiglu_mm(a.cuda(), w.cuda().T, "tiled", (128, 128, 32, 8, 3), True)
    torch.cuda.synchronize()
    assert torch.count_nonzero(act).item() == 0
    assert torch.count_nonzero(packed[:, 256:]).item() == 0


@pytest.mark.parametrize("m,d,n,gate", [(512, 256, 576, (384, 512)), (300, 2048, 1152, (768, 1024)),
                                        (1024, 2048, 9216, (6144, 8192)),
                                        # rows held in registers with a partial last chunk
                                        (200, 1000, 512, (256, 512)), (130, 3072, 512, (0, 256))])
def test_rmsnorm_gate_projection(m, d, n, gate):
    from ops.benchmark_configs import rms_projection_inputs
    from ops.fused_execution import rmsnorm_gate_mm

    inp = rms_projection_inputs(m=m, d=d, n=n, gate=gate, seed=0)
    out, rstd = rmsnorm_gate_mm(inp["x"].cuda(), inp["norm_weight"].cuda(), inp["eps"],
                                inp["w"].cuda(), gate)
    torch.cuda.synchronize()
    want = oracle.rmsnorm_gate_projection(inp["x"], inp["norm_weight"], inp["eps"], inp["w"], gate)
    assert_bf16_close(out, want, "rms gate projection")
    assert_f32_close(rstd.cpu(), oracle.rms_rstd(inp["x"], inp["eps"]), "rstd")
    gate_vals = out[:, gate[0]:gate[1]].float()
    assert gate_vals.min().item() >= 0.0 and gate_vals.max().item() <= 1.0


def test_rmsnorm_gate_zero_weight_is_half_on_gate():
    from ops.fused_execution import rmsnorm_gate_mm

    gen = _gen(9)
    x = torch.randn(256, 512, generator=gen).bfloat16().cuda()
    w = torch.zeros(640, 512, dtype=torch.bfloat16, device="cuda")
    nw = torch.ones(512, device="cuda")
    out, _ = rmsnorm_gate_mm(x, nw, 1e-6, w, (256, 384))
    torch.cuda.synchronize()
    expect = torch.zeros(256, 640)
    expect[:, 256:384] = 0.5
    assert torch.equal(out.float().cpu(), expect)


@pytest.mark.parametrize("m,ffn,d", [(512, 1408, 512), (300, 5632, 2048), (64, 200, 72)])
def test_residual_projection(m, ffn, d):
    from ops.benchmark_configs import down_residual_inputs
    from ops.fused_execution import residual_mm

    inp = down_residual_inputs(m=m, ffn=ffn, d=d, seed=0)
    out = residual_mm(inp["h"].cuda(), inp["w_down"].cuda(), inp["residual"].cuda())
    torch.cuda.synchronize()
    assert_bf16_close(out, oracle.residual_projection(inp["h"], inp["w_down"], inp["residual"]),
                      "residual")


@pytest.mark.parametrize("m,ffn,d", [(128, 384, 260), (264, 512, 516)])
def test_residual_projection_width_4_mod_8(m, ffn, d):
    """Output widths with N % 8 == 4: the staged epilogue writes the last 4 columns of a
    row as a half (8-byte) piece and reads the residual the same way."""
    from ops.benchmark_configs import down_residual_inputs
    from ops.fused_execution import residual_mm

    inp = down_residual_inputs(m=m, ffn=ffn, d=d, seed=3)
    out = residual_mm(inp["h"].cuda(), inp["w_down"].cuda(), inp["residual"].cuda())
    torch.cuda.synchronize()
    assert_bf16_close(out, oracle.residual_projection(inp["h"], inp["w_down"], inp["residual"]),
                      "residual N % 8 == 4")
    zero = residual_mm(inp["h"].cuda(), torch.zeros_like(inp["w_down"]).cuda(), inp["residual"].cuda())
    torch.cuda.synchronize()
    assert torch.equal(zero.cpu(), inp["residual"])


def test_rmsnorm_gate_projection_width_4_mod_8():
    from ops.benchmark_configs import rms_projection_inputs
    from ops.fused_execution import rmsnorm_gate_mm

    gate = (256, 388)
    inp = rms_projection_inputs(m=200, d=256, n=516, gate=gate, seed=5)
    out, _ = rmsnorm_gate_mm(inp["x"].cuda(), inp["norm_weight"].cuda(), inp["eps"],
                             inp["w"].cuda(), gate)
    torch.cuda.synchronize()
    want = oracle.rmsnorm_gate_projection(inp["x"], inp["norm_weight"], inp["eps"], inp["w"], gate)
    assert_bf16_close(out, want, "rms gate projection N % 8 == 4")


def test_residual_zero_weight_returns_residual_bitwise():
    from ops.fused_execution import residual_mm

    gen = _gen(4)
    h = torch.randn(384, 640, generator=gen).bfloat16().cuda()
    r = torch.randn(384, 512, generator=gen).bfloat16().cuda()
    out = residual_mm(h, torch.zeros(512, 640, dtype=torch.bfloat16, device="cuda"), r)
    torch.cuda.synchronize()
    assert torch.equal(out, r)


def _mlp_case(m, d, ffn, seed=0):
    from ops.benchmark_configs import mlp_backward_inputs

    inp = mlp_backward_inputs(m=m, d=d, ffn=ffn, seed=seed)
    packed, act = oracle.swiglu_mm(inp["x"], inp["w_upgate"].T, True)
    return inp, packed, act


@pytest.mark.parametrize("eager_rounding", [True, False])
@pytest.mark.parametrize("m,d,ffn", [(512, 512, 704), (256, 2048, 1408), (100, 72, 40)])
def test_swiglu_backward_epilogue(eager_rounding, m, d, ffn):
    from ops.fused_execution import swiglu_backward_mm

    inp, packed, _act = _mlp_case(m, d, ffn)
    dpacked = swiglu_backward_mm(inp["dy"].cuda(), inp["w_down"].cuda(), packed.cuda(),
                                 eager_rounding)
    torch.cuda.synchronize()
    dact = oracle.mm(inp["dy"], inp["w_down"])
    want = oracle.swiglu_backward(packed, dact, eager_rounding)
    assert_bf16_close(dpacked[:, :ffn], want[:, :ffn], "dUp")
    assert_bf16_close(dpacked[:, ffn:], want[:, ffn:], "dGate")


@pytest.mark.parametrize("splits", [1, 3])
@pytest.mark.parametrize("layout", ["dw", "nn", "nt"])
def test_weight_gradient_fp32_accumulation(splits, layout):
    from ops.fused_execution import mm_accumulate_

    gen = _gen(901)
    tokens, n_out, n_in = 1024, 384, 320
    dy = torch.randn(tokens, n_out, generator=gen).bfloat16()
    x = torch.randn(tokens, n_in, generator=gen).bfloat16()
    g = torch.randn(n_out, n_in, generator=gen) * 1e-2
    if layout == "dw":
        a, b = dy.T, x
    elif layout == "nn":
        a, b = dy.T.contiguous(), x
    else:
        a, b = dy.T.contiguous(), x.T.contiguous().T
    ga, gb = a.cuda(), b.cuda()
    assert ga.stride() == a.stride() and gb.stride() == b.stride()
    gg = g.cuda()
    mm_accumulate_(gg, ga, gb, True, splits)
    torch.cuda.synchronize()
    assert_f32_close(gg.cpu(), oracle.accumulate_weight_grad(g, a, b), f"{layout} splits={splits}")


def test_balanced_accumulation_whole_rounds_plus_shared_tiles():
    """272 output tiles on a 256-CU GPU: 256 run whole and accumulate directly, the last
    tile row's k-range is shared by all CUs and summed from FP32 partials. Rows from both
    regions match the oracle, and the whole buffer matches the unsplit path."""
    from ops.fused_execution import mm_accumulate_

    gen = _gen(77)
    tokens, n_out, n_in = 1024, 17 * 256, 16 * 256
    dy = torch.randn(tokens, n_out, generator=gen).bfloat16()
    x = torch.randn(tokens, n_in, generator=gen).bfloat16()
    g = torch.randn(n_out, n_in, generator=gen) * 1e-2
    a, b = dy.cuda().T, x.cuda()
    balanced, plain = g.cuda(), g.cuda()
    mm_accumulate_(balanced, a, b, True, 2)
    mm_accumulate_(plain, a, b, True, 1)
    torch.cuda.synchronize()
    rows = torch.cat([torch.arange(0, 64), torch.arange(16 * 256, 17 * 256)])
    want = oracle.accumulate_weight_grad(g[rows], dy.T[rows], x)
    assert_f32_close(balanced.cpu()[rows], want, "balanced, sampled rows")
    assert_f32_close(balanced.cpu(), plain.cpu(), "balanced vs unsplit")


@pytest.mark.parametrize("round_bf16,tokens", [(True, 1000), (False, 1000), (True, 520)])
def test_balanced_accumulation_ragged_tiles(round_bf16, tokens):
    """The balanced split with ragged rows, columns and k: 17 x 16 tiles whose last row
    and column of tiles are partial, 1000-long reduction (the last k-tile partial). Both
    widths are multiples of 8, so the M/N-contiguous operands take the fast loader and the
    balanced plan (other widths take the generic loader and even slices). With 520 tokens
    the 16 shared tiles hold 16 x 9 = 144 k-tiles, fewer than the 256 workgroups."""
    from ops.fused_execution import mm_accumulate_

    gen = _gen(79)
    n_out, n_in = 17 * 256 - 96, 16 * 256 - 40
    dy = torch.randn(tokens, n_out, generator=gen).bfloat16()
    x = torch.randn(tokens, n_in, generator=gen).bfloat16()
    g = torch.randn(n_out, n_in, generator=gen) * 1e-2
    balanced = g.cuda()
    mm_accumulate_(balanced, dy.cuda().T, x.cuda(), round_bf16, 2)
    torch.cuda.synchronize()
    rows = torch.cat([torch.arange(0, 32), torch.arange(n_out - 200, n_out)])
    want = oracle.accumulate_weight_grad(g[rows], dy.T[rows], x, round_bf16)
    assert_f32_close(balanced.cpu()[rows], want, f"balanced ragged round={round_bf16}")


@pytest.mark.parametrize("round_bf16", [True, False])
def test_balanced_accumulation_ragged_edges(round_bf16):
    """Ragged rows, columns and k (47 k-tiles, the last one partial) in even k-slices."""
    from ops.fused_execution import mm_accumulate_

    gen = _gen(78)
    tokens, n_out, n_in = 3000, 300, 264
    dy = torch.randn(tokens, n_out, generator=gen).bfloat16()
    x = torch.randn(tokens, n_in, generator=gen).bfloat16()
    g = torch.randn(n_out, n_in, generator=gen) * 1e-2
    gg = g.cuda()
    mm_accumulate_(gg, dy.cuda().T, x.cuda(), round_bf16, 2)
    torch.cuda.synchronize()
    assert_f32_close(gg.cpu(), oracle.accumulate_weight_grad(g, dy.T, x, round_bf16),
                     f"ragged round={round_bf16}")


def _group_case(seed, tokens, shapes, mn_layout=True):
    """(G, a, b) triples on the GPU: a = dY^T, b = X with `tokens` rows (the weight-gradient
    layout, both operands M/N-contiguous) or, with mn_layout False, a K-contiguous a."""
    gen = _gen(seed)
    cases = []
    for n_out, n_in in shapes:
        dy = torch.randn(tokens, n_out, generator=gen).bfloat16()
        x = torch.randn(tokens, n_in, generator=gen).bfloat16()
        g = torch.randn(n_out, n_in, generator=gen) * 1e-2
        a = dy.cuda().T if mn_layout else dy.T.contiguous().cuda()
        cases.append((g, dy.T, x, g.cuda(), a, x.cuda()))
    return cases


@pytest.mark.parametrize("round_bf16", [True, False])
def test_grouped_accumulation_shares_tiles_across_gradients(round_bf16):
    """Three gradients in one launch: 128 + 144 + 4 = 276 tiles on 256 CUs, so the first
    256 run whole and the last 20 (16 of the second gradient, all 4 of the third) share
    the k-range; ragged rows, columns and k (520 tokens: the last k-tile partial). Widths
    are multiples of 8 (fast loader, one launch). The whole tiles match the unsplit call
    bit for bit: the same tile computation, only scheduled differently."""
    from ops.fused_execution import mm_accumulate_, mm_accumulate_group_

    cases = _group_case(81, 520, [(2000, 4000), (4000, 2104), (296, 296)])
    plain = [gg.clone() for _, _, _, gg, _, _ in cases]
    for (_, _, _, _, ga, gb), gp in zip(cases, plain):
        mm_accumulate_(gp, ga, gb, round_bf16, 1)
    mm_accumulate_group_([(gg, ga, gb) for _, _, _, gg, ga, gb in cases], round_bf16)
    torch.cuda.synchronize()
    for i, (g, a, b, gg, _, _) in enumerate(cases):
        assert_f32_close(gg.cpu(), oracle.accumulate_weight_grad(g, a, b, round_bf16),
                         f"gradient {i} round={round_bf16}")
    assert torch.equal(cases[0][3], plain[0])  # all 128 tiles of the first run whole


def test_grouped_accumulation_of_one_matches_the_balanced_call_bitwise():
    """A group of one runs the same balanced plan as ws_mm_accumulate_f32 with splits > 1."""
    from ops.fused_execution import mm_accumulate_, mm_accumulate_group_

    (g, a, b, gg, ga, gb), = _group_case(82, 1024, [(17 * 256 - 96, 16 * 256 - 40)])
    single = gg.clone()
    mm_accumulate_group_([(gg, ga, gb)], True)
    mm_accumulate_(single, ga, gb, True, 2)
    torch.cuda.synchronize()
    assert torch.equal(gg, single)
    rows = torch.cat([torch.arange(0, 32), torch.arange(g.shape[0] - 200, g.shape[0])])
    assert_f32_close(gg.cpu()[rows], oracle.accumulate_weight_grad(g[rows], a[rows], b),
                     "group of one, sampled rows")


@pytest.mark.parametrize("case", ["few_tiles", "mixed_layouts"])
def test_grouped_accumulation_falls_back_to_single_launches(case):
    """Fewer tiles than CUs, or operand layouts that differ between the gradients: each
    gradient then takes ws_mm_accumulate_f32 with its own split."""
    from ops.fused_execution import mm_accumulate_group_

    if case == "few_tiles":
        cases = _group_case(83, 3000, [(300, 264), (520, 130)])
    else:
        cases = (_group_case(84, 1024, [(4096, 4096)]) +
                 _group_case(85, 1024, [(1024, 2048)], mn_layout=False))
    mm_accumulate_group_([(gg, ga, gb) for _, _, _, gg, ga, gb in cases], True)
    torch.cuda.synchronize()
    for i, (g, a, b, gg, _, _) in enumerate(cases):
        assert_f32_close(gg.cpu(), oracle.accumulate_weight_grad(g, a, b), f"{case} gradient {i}")


@pytest.mark.parametrize("round_bf16", [True, False])
@pytest.mark.parametrize("case", ["whole_tiles", "balanced", "even_slices", "generic"])
def test_fp32_store_equals_accumulation_into_zeros_bitwise(case, round_bf16):
    """ws_mm_store_f32 writes G = f32(r(A @ B)) without reading G: on every path (whole
    tiles, balanced stream-K, even split-K slices, the generic loader) it equals
    accumulation into a zeroed buffer bit for bit, whatever G held before (here NaN)."""
    from ops.fused_execution import mm_accumulate_, mm_f32

    shapes = {"whole_tiles": (1024, 16 * 256, 16 * 256, 1),
              "balanced": (1000, 17 * 256 - 96, 16 * 256 - 40, 2),
              "even_slices": (3000, 304, 264, 2),
              "generic": (700, 300, 262, 2)}
    tokens, n_out, n_in, splits = shapes[case]
    gen = _gen(91)
    dy = torch.randn(tokens, n_out, generator=gen).bfloat16().cuda()
    x = torch.randn(tokens, n_in, generator=gen).bfloat16().cuda()
    want = torch.zeros(n_out, n_in, device="cuda")
    mm_accumulate_(want, dy.T, x, round_bf16, splits)
    got = torch.full((n_out, n_in), float("nan"), device="cuda")
    mm_accumulate_(got, dy.T, x, round_bf16, splits, _entry="ws_mm_store_f32")
    fresh = mm_f32(dy.T, x, round_bf16, splits=splits)
    torch.cuda.synchronize()
    assert torch.equal(got, want) and torch.equal(fresh, want)
    rows = torch.arange(0, n_out, 37)
    assert_f32_close(got.cpu()[rows], oracle.accumulate_weight_grad(
        torch.zeros(len(rows), n_in), dy.cpu().T[rows], x.cpu(), round_bf16), f"store {case}")


def test_grouped_fp32_store_equals_grouped_accumulation_into_zeros_bitwise():
    """ws_mm_store_f32_group on the MLP's two weight gradients (one launch, shared tiles)
    equals the grouped accumulation into zeroed buffers bit for bit."""
    from ops.fused_execution import mm_accumulate_group_, mm_f32_group

    cases = _group_case(86, 520, [(2000, 4000), (4000, 2104), (296, 296)])
    zeros = [torch.zeros_like(gg) for _, _, _, gg, _, _ in cases]
    mm_accumulate_group_([(z, ga, gb) for z, (_, _, _, _, ga, gb) in zip(zeros, cases)], True)
    got = mm_f32_group([(ga, gb) for _, _, _, _, ga, gb in cases])
    torch.cuda.synchronize()
    for i, (z, out) in enumerate(zip(zeros, got)):
        assert torch.equal(z, out), i


def test_weight_gradient_zero_upstream_leaves_buffer_bitwise():
    from ops.fused_execution import mm_accumulate_

    gen = _gen(2)
    g = torch.randn(256, 192, generator=gen).cuda()
    before = g.clone()
    x = torch.randn(512, 192, generator=gen).bfloat16().cuda()
    mm_accumulate_(g, torch.zeros(512, 256, dtype=torch.bfloat16, device="cuda").T, x)
    torch.cuda.synchronize()
    assert torch.equal(g, before)


@pytest.mark.parametrize("m,n,k", [(2048, 1536, 768), (100, 384, 200), (1100, 520, 264)])
def test_input_gradient_gemm(m, n, k):
    """dgrad_mm: r(grad @ W) with W [N, K] in nn.Linear layout (this library's GEMM on
    the K-contiguous copy of W from 1024 rows on, on W as given below that)."""
    from ops.fused_execution import dgrad_mm, mm

    g = torch.Generator().manual_seed(m + n + k)
    grad = torch.randn(m, n, generator=g).bfloat16()
    w = (torch.randn(n, k, generator=g) * 0.05).bfloat16()
    dx = dgrad_mm(grad.cuda(), w.cuda())
    torch.cuda.synchronize()
    want = oracle.mm(grad, w)
    assert dx.shape == (m, k) and dx.dtype == torch.bfloat16
    assert_bf16_close(dx, want, "dgrad_mm")
    assert_bf16_close(mm(grad.cuda(), w.cuda()), want, "mm on the same operands")
    with pytest.raises(ValueError):
        dgrad_mm(grad.cuda(), w.cuda().T.contiguous())


def test_mlp_backward_matches_oracle():
    from ops.fused_execution import mlp_backward

    m, d, ffn = 512, 256, 352
    inp, packed, act = _mlp_case(m, d, ffn)
    g_up, g_down = inp["g_upgate"].cuda(), inp["g_down"].cuda()
    dx = mlp_backward(inp["x"].cuda(), inp["w_upgate"].cuda(), inp["w_down"].cuda(),
                      packed.cuda(), act.cuda(), inp["dy"].cuda(), g_up, g_down)
    torch.cuda.synchronize()
    want_dx, _dp, want_gup, want_gdown = oracle.mlp_backward(
        inp["x"], inp["w_upgate"], inp["w_down"], packed, act, inp["dy"],
        inp["g_upgate"], inp["g_down"])
    assert_bf16_close(dx, want_dx, "dX")
    assert_f32_close(g_up.cpu(), want_gup, "G_upgate")
    assert_f32_close(g_down.cpu(), want_gdown, "G_down")


@pytest.mark.parametrize("rows,d,vocab,chunk", [(512, 256, 1024, 256), (3000, 384, 2052, 1024)])
def test_linear_cross_entropy_stored_logits_match_recompute_bitwise(rows, d, vocab, chunk):
    """The forward's stored BF16 logits are r(hidden @ W^T); the backward that reads them
    gives the recomputing backward's loss, dHidden and head-weight gradient bit for bit
    (2052 columns: a last 4-column piece in both the store and the gradient pass)."""
    from ops.fused_execution import (CrossEntropyState, linear_cross_entropy_backward,
                                     linear_cross_entropy_forward)

    gen = _gen(404)
    h = torch.randn(rows, d, generator=gen).bfloat16()
    w = (torch.randn(vocab, d, generator=gen) * 0.05).bfloat16()
    t = torch.randint(0, vocab, (rows,), generator=gen)
    t[::7] = -100
    hc, wc, tc = h.cuda(), w.cuda(), t.cuda()
    grad = torch.full((), 0.7, device="cuda")
    got = []
    for store in (False, True):
        state = CrossEntropyState(rows, vocab, hc.device, chunk_rows=chunk, store_logits=store)
        linear_cross_entropy_forward(hc, wc, tc, state)
        gw = torch.zeros(vocab, d, device="cuda")
        dh = linear_cross_entropy_backward(hc, wc, tc, state, grad, weight_grad=gw)
        got.append((state, dh, gw))
    torch.cuda.synchronize()
    (a, dha, gwa), (b, dhb, gwb) = got
    for name in ("loss", "lse", "mean", "count"):
        assert torch.equal(getattr(a, name), getattr(b, name)), name
    valid = tc != -100  # the target logit is written for valid rows only
    assert torch.equal(a.target_logit[valid], b.target_logit[valid])
    assert torch.equal(dha, dhb) and torch.equal(gwa, gwb)
    assert_bf16_close(b.logits, oracle.mm(h, w.T), "stored logits")


@pytest.mark.parametrize("m,d,vocab,chunk", [(512, 256, 1024, 2048), (300, 512, 4096, 128),
                                             (1024, 2048, 8192, 512), (1001, 256, 1030, 256),
                                             (998, 128, 2048, 300)])
def test_linear_cross_entropy(m, d, vocab, chunk):
    """Against the oracle; the last two cases have row counts that are not a multiple of 4
    (the mean's and count's last piece) and 10 or 16 statistics partials per row (one part
    per lane, or 16-byte pieces)."""
    from ops.benchmark_configs import lm_head_inputs
    from ops.fused_execution import CrossEntropyState, linear_cross_entropy_backward, \
        linear_cross_entropy_forward

    inp = lm_head_inputs(m=m, d=d, vocab=vocab, seed=0)
    h, w, t = inp["hidden"].cuda(), inp["weight"].cuda(), inp["targets"].cuda()
    state = CrossEntropyState(m, vocab, h.device, chunk_rows=chunk)
    linear_cross_entropy_forward(h, w, t, state)
    dh = linear_cross_entropy_backward(h, w, t, state, torch.ones((), device="cuda"))
    torch.cuda.synchronize()
    loss, mean, count, dhidden = oracle.linear_cross_entropy(inp["hidden"], inp["weight"],
                                                             inp["targets"])
    assert int(state.count.item()) == count
    assert_f32_close(state.loss.cpu(), loss, "per-token loss")
    assert abs(state.mean.item() - mean.item()) <= 1e-3 * abs(mean.item())
    ignored = inp["targets"] == -100
    assert torch.count_nonzero(state.loss.cpu()[ignored]).item() == 0
    assert torch.count_nonzero(dh.cpu()[ignored]).item() == 0
    assert_bf16_close(dh, dhidden, "dHidden")


def test_linear_cross_entropy_zero_weight_and_all_ignored():
    from ops.fused_execution import linear_cross_entropy_backward, linear_cross_entropy_forward

    gen = _gen(12)
    vocab = 2048
    h = torch.randn(256, 128, generator=gen).bfloat16().cuda()
    w = torch.zeros(vocab, 128, dtype=torch.bfloat16, device="cuda")
    t = torch.randint(0, vocab, (256,), generator=gen).cuda()
    state = linear_cross_entropy_forward(h, w, t)
    dh = linear_cross_entropy_backward(h, w, t, state, torch.ones((), device="cuda"))
    torch.cuda.synchronize()
    assert torch.allclose(state.loss.cpu(), torch.full((256,), math.log(vocab)), rtol=1e-6, atol=1e-5)
    assert torch.count_nonzero(dh).item() == 0
    t_all = torch.full((256,), -100, dtype=torch.int64, device="cuda")
    w2 = torch.randn(vocab, 128, generator=gen).bfloat16().cuda()
    state = linear_cross_entropy_forward(h, w2, t_all)
    dh = linear_cross_entropy_backward(h, w2, t_all, state, torch.ones((), device="cuda"))
    torch.cuda.synchronize()
    assert state.mean.item() == 0.0 and state.count.item() == 0.0
    assert torch.count_nonzero(state.loss).item() == 0 and torch.count_nonzero(dh).item() == 0


@pytest.mark.parametrize("shape", [(3, 224), (2, 32, 256), (257, 14336), (5, 46), (7, 100)])
@pytest.mark.parametrize("eager_rounding", [True, False])
def test_standalone_swiglu_forward_backward(shape, eager_rounding):
    from ops.activation_execution import bf16_swiglu

    gen = _gen(947)
    source = torch.randn(shape, generator=gen).bfloat16()
    actual = source.cuda().requires_grad_()
    out = bf16_swiglu(actual, eager_rounding=eager_rounding)
    grad = torch.randn(out.shape, generator=gen).bfloat16()
    out.backward(grad.cuda())
    torch.cuda.synchronize()
    flat = source.reshape(-1, shape[-1])
    assert_bf16_close(out.reshape(-1, shape[-1] // 2), oracle.swiglu(flat, eager_rounding), "swiglu")
    want = oracle.swiglu_backward(flat, grad.reshape(-1, shape[-1] // 2), eager_rounding)
    assert_bf16_close(actual.grad.reshape(-1, shape[-1]), want, "swiglu grad")


@pytest.mark.parametrize("shape", [(3, 24), (2, 16, 128), (257, 2048), (1, 2048), (39, 1024),
                                   (100, 512), (65, 1536), (8, 2000), (4, 40, 1000)])
def test_standalone_rmsnorm_forward_backward(shape):
    from ops.activation_execution import bf16_rmsnorm

    gen = _gen(949)
    weight = torch.rand(shape[-1], generator=gen) * 1.9 + 0.1
    source = torch.randn(shape, generator=gen).bfloat16()
    x_ref = source.clone().requires_grad_()
    w_ref = weight.clone().requires_grad_()
    expected = oracle.rmsnorm(x_ref, w_ref, 1e-5)
    grad = torch.randn(shape, generator=gen).bfloat16()
    expected.backward(grad)
    x = source.cuda().requires_grad_()
    w = weight.cuda().requires_grad_()
    out, rstd = bf16_rmsnorm(x, w, 1e-5, True)
    out.backward(grad.cuda())
    torch.cuda.synchronize()
    assert_bf16_close(out, expected.detach(), "rmsnorm")
    assert_bf16_close(x.grad, x_ref.grad, "rmsnorm dx")
    assert w.grad.dtype == torch.float32
    assert rel_l2(w.grad, w_ref.grad) <= 3e-3


@pytest.mark.parametrize("eager_rounding", [True, False])
def test_standalone_swiglu_vector_and_scalar_kernels_agree_bitwise(eager_rounding):
    """The standalone SwiGLU forward and backward take 16-byte pieces of 8 columns when the
    hidden width is a multiple of 8 and the buffers are 16-byte aligned, and one element per
    thread otherwise (here: the same values in views 2 bytes past the boundary). The
    arithmetic per element is the same, so the bits are."""
    from ops import _hip

    gen = _gen(961)
    rows, h = 300, 1024
    packed = torch.randn(rows, 2 * h, generator=gen).bfloat16().cuda()
    dy = torch.randn(rows, h, generator=gen).bfloat16().cuda()

    def shifted(t):
        buf = torch.empty(t.numel() + 8, dtype=t.dtype, device=t.device)
        view = buf[1:1 + t.numel()].view(t.shape)
        view.copy_(t)
        return view

    def run(pk, g):
        out = shifted(torch.empty(rows, h, dtype=torch.bfloat16, device="cuda")) \
            if pk.data_ptr() % 16 else torch.empty(rows, h, dtype=torch.bfloat16, device="cuda")
        dpk = shifted(torch.empty_like(packed)) if pk.data_ptr() % 16 else torch.empty_like(packed)
        _hip.call("ws_swiglu_forward", pk.data_ptr(), out.data_ptr(), rows, h,
                  int(eager_rounding), _hip.stream(pk))
        _hip.call("ws_swiglu_backward", pk.data_ptr(), g.data_ptr(), dpk.data_ptr(), rows, h,
                  int(eager_rounding), _hip.stream(pk))
        return out.clone(), dpk.clone()

    vec_out, vec_d = run(packed, dy)
    sp, sg = shifted(packed), shifted(dy)
    assert sp.data_ptr() % 16 == 2
    sc_out, sc_d = run(sp, sg)
    torch.cuda.synchronize()
    assert torch.equal(vec_out, sc_out) and torch.equal(vec_d, sc_d)


@pytest.mark.parametrize("shape", [(37, 64), (257, 2048), (40, 4096), (9, 8192), (33, 1001),
                                   (5, 8200), (3, 20)])
def test_standalone_rmsnorm_forward_without_eager_rounding(shape):
    """The compiled-path forward (eager_rounding=False: r(x rstd w) with the product in FP32)
    against the oracle, at widths of the register kernels (up to 8192), the two-pass vector
    kernel (8200) and the scalar kernel (widths not a multiple of 8)."""
    from ops.activation_execution import bf16_rmsnorm

    gen = _gen(959)
    weight = torch.rand(shape[-1], generator=gen) * 1.9 + 0.1
    x = torch.randn(shape, generator=gen).bfloat16()
    with torch.no_grad():
        out, rstd = bf16_rmsnorm(x.cuda(), weight.cuda(), 1e-5, False)
    torch.cuda.synchronize()
    assert_bf16_close(out, oracle.rmsnorm_fp32_product(x, weight, 1e-5), "rmsnorm, FP32 product")
    assert_f32_close(rstd.cpu(), oracle.rms_rstd(x.reshape(-1, shape[-1]), 1e-5), "rstd")


@pytest.mark.parametrize("shape", [(3, 20), (5, 100), (33, 27), (9, 1001), (70, 4100),
                                   (2, 3, 8190)])
def test_standalone_rmsnorm_backward_any_width(shape):
    """Widths that are not a multiple of 8 (the generic row kernel and, for odd widths, the
    one-column-at-a-time weight reduction) against the oracle through autograd, as the
    reference's RMSNorm takes any width."""
    from ops.activation_execution import bf16_rmsnorm

    gen = _gen(951)
    weight = torch.rand(shape[-1], generator=gen) * 1.9 + 0.1
    source = torch.randn(shape, generator=gen).bfloat16()
    x_ref = source.clone().requires_grad_()
    w_ref = weight.clone().requires_grad_()
    expected = oracle.rmsnorm(x_ref, w_ref, 1e-5)
    grad = torch.randn(shape, generator=gen).bfloat16()
    expected.backward(grad)
    x = source.cuda().requires_grad_()
    w = weight.cuda().requires_grad_()
    out, _rstd = bf16_rmsnorm(x, w, 1e-5, True)
    out.backward(grad.cuda())
    torch.cuda.synchronize()
    assert_bf16_close(out, expected.detach(), "rmsnorm")
    assert_bf16_close(x.grad, x_ref.grad, "rmsnorm dx")
    assert rel_l2(w.grad, w_ref.grad) <= 3e-3


@pytest.mark.parametrize("eager_rounding", [True, False])
def test_rmsnorm_backward_unaligned_rows_match_aligned(eager_rounding):
    """x and the incoming gradient as views 2 bytes past a 16-byte boundary take the generic
    row kernel; aligned copies of the same values take the vector kernel. The weight
    gradient sums the same values in the same order, so it is bitwise equal; dX is within
    the oracle's bars (its row dot product is summed in another order)."""
    from ops.activation_execution import _rms_backward

    gen = _gen(955)
    rows, d = 100, 2048
    x = torch.randn(rows, d, generator=gen).bfloat16()
    grad = torch.randn(rows, d, generator=gen).bfloat16()
    weight = (torch.rand(d, generator=gen) * 1.9 + 0.1).cuda()
    rstd = (1.0 / x.float().pow(2).mean(-1).add(1e-5).sqrt()).cuda()
    flat_x = torch.zeros(rows * d + 8, dtype=torch.bfloat16, device="cuda")
    flat_g = torch.zeros_like(flat_x)
    xv = flat_x[1:1 + rows * d].view(rows, d)
    gv = flat_g[1:1 + rows * d].view(rows, d)
    xv.copy_(x.cuda())
    gv.copy_(grad.cuda())
    assert xv.data_ptr() % 16 == 2 and xv.is_contiguous() and gv.is_contiguous()
    dx_u, dw_u = _rms_backward(xv, weight, rstd, gv, eager_rounding)
    dx_a, dw_a = _rms_backward(x.cuda(), weight, rstd, grad.cuda(), eager_rounding)
    torch.cuda.synchronize()
    assert torch.equal(dw_u, dw_a)
    assert_bf16_close(dx_u, dx_a.cpu(), "dx, unaligned against aligned")
    if eager_rounding:
        x_ref = x.clone().requires_grad_()
        w_ref = weight.cpu().clone().requires_grad_()
        oracle.rmsnorm(x_ref, w_ref, 1e-5).backward(grad)
        assert_bf16_close(dx_u, x_ref.grad, "dx, unaligned against the oracle")


def test_forward_weights_stored_k_by_n_match_the_native_layout(monkeypatch):
    """Forward weights stored [K, N] row-major (the reference's second measured layout, an
    N-contiguous B) are copied K-contiguous by the transpose kernel before the fused
    projections, and give the native [N, K] layout's bits: the RMSNorm-prologue projection,
    the residual projection and the paired SwiGLU projection."""
    from ops import _hip
    from ops.fused_execution import residual_mm, rmsnorm_gate_mm
    from ops.matmul_epilogue import launch_swiglu_mm

    gen = _gen(957)
    m, k, n = 1024, 384, 640
    x = torch.randn(m, k, generator=gen).bfloat16().cuda()
    nw = (torch.rand(k, generator=gen) * 1.9 + 0.1).cuda()
    w = (torch.randn(n, k, generator=gen) * 0.05).bfloat16().cuda()
    r = torch.randn(m, n, generator=gen).bfloat16().cuda()
    w_kn = w.T.contiguous()
    calls, real = [], _hip.call
    monkeypatch.setattr(_hip, "call", lambda name, *a: (calls.append(name), real(name, *a))[1])
    pairs = [
        (lambda: rmsnorm_gate_mm(x, nw, 1e-6, w, (128, 256))[0],
         lambda: rmsnorm_gate_mm(x, nw, 1e-6, w_kn.T, (128, 256))[0], "ws_rmsnorm_gate_mm"),
        (lambda: residual_mm(x, w, r), lambda: residual_mm(x, w_kn.T, r), "ws_residual_mm"),
        (lambda: launch_swiglu_mm(x, w.T, "persistent", (128, 128, 32, 8, 3), True),
         lambda: launch_swiglu_mm(x, w_kn, "persistent", (128, 128, 32, 8, 3), True),
         "ws_swiglu_mm"),
    ]
    for native, stored_kn, entry in pairs:
        calls.clear()
        want = native()
        assert calls == [entry], calls
        calls.clear()
        got = stored_kn()
        assert calls == ["ws_transpose_bf16", entry], calls
        torch.cuda.synchronize()
        for g, e in zip(got if isinstance(got, tuple) else (got,),
                        want if isinstance(want, tuple) else (want,)):
            assert torch.equal(g, e), entry


@pytest.mark.parametrize("offset", [1, 3])
def test_rmsnorm_forward_with_unaligned_weight_view(offset):
    """An FP32 norm weight that is a view at a 4- or 12-byte offset into a flat parameter
    buffer (not 16-byte aligned): the row kernels must not read it as 16-byte vectors, and
    the standalone forward and the fused projection's row pass still match the oracle."""
    from ops.activation_execution import bf16_rmsnorm
    from ops.fused_execution import rmsnorm_gate_mm

    gen = _gen(953)
    d, rows = 2048, 67
    weight = torch.rand(d, generator=gen) * 1.9 + 0.1
    x = torch.randn(rows, d, generator=gen).bfloat16()
    flat = torch.zeros(d + 8, device="cuda")
    w = flat[offset:offset + d]
    w.copy_(weight.cuda())
    assert w.data_ptr() % 16 != 0 and w.is_contiguous()
    with torch.no_grad():
        out, _ = bf16_rmsnorm(x.cuda(), w, 1e-5, True)
    torch.cuda.synchronize()
    assert_bf16_close(out, oracle.rmsnorm(x, weight, 1e-5), "rmsnorm, unaligned weight")
    proj = (torch.randn(256, d, generator=gen) * 0.02).bfloat16()
    got, _ = rmsnorm_gate_mm(x.cuda(), w, 1e-5, proj.cuda(), (64, 128))
    torch.cuda.synchronize()
    want = oracle.rmsnorm_gate_projection(x, weight, 1e-5, proj, (64, 128))
    assert_bf16_close(got, want, "projection, unaligned weight")


@pytest.mark.parametrize("rows,d,vocab,chunk", [(512, 256, 1024, 4096), (3000, 384, 2048, 1024)])
def test_linear_cross_entropy_head_weight_gradient(rows, d, vocab, chunk):
    """The tied head weight's FP32 gradient accumulated chunk by chunk, against the
    oracle with the same chunking; dHidden is unchanged by asking for it."""
    from ops.benchmark_configs import lm_head_inputs
    from ops.fused_execution import (CrossEntropyState, linear_cross_entropy_backward,
                                     linear_cross_entropy_forward)

    inp = lm_head_inputs(m=rows, d=d, vocab=vocab, seed=4)
    hidden, weight, targets = (inp[k].cuda() for k in ("hidden", "weight", "targets"))
    state = CrossEntropyState(rows, vocab, hidden.device, chunk_rows=chunk)
    linear_cross_entropy_forward(hidden, weight, targets, state)
    one = torch.ones((), device="cuda")
    dh_plain = linear_cross_entropy_backward(hidden, weight, targets, state, one)
    wgrad = torch.zeros(vocab, d, device="cuda")
    dh = linear_cross_entropy_backward(hidden, weight, targets, state, one, weight_grad=wgrad)
    torch.cuda.synchronize()
    assert torch.equal(dh, dh_plain)
    want = oracle.linear_cross_entropy_weight_grad(inp["hidden"], inp["weight"], inp["targets"],
                                                   chunk=min(chunk, rows))
    assert_f32_close(wgrad.cpu(), want, "head weight gradient")


@pytest.mark.parametrize("in_place", [False, True])
@pytest.mark.parametrize("m,d,n,gate", [(512, 256, 576, (384, 512)), (1024, 2048, 9216, (6144, 8192))])
def test_rmsnorm_gate_projection_backward(m, d, n, gate, in_place):
    """QKV backward: gate sigmoid backward, dY through W, FP32 wgrad, RMSNorm backward."""
    from ops.benchmark_configs import rms_projection_inputs
    from ops.fused_execution import rmsnorm_gate_mm, rmsnorm_gate_mm_backward

    inp = rms_projection_inputs(m=m, d=d, n=n, gate=gate, seed=2)
    gen = _gen(12)
    dout = (torch.randn(m, n, generator=gen) * 1e-2).bfloat16()
    g0 = torch.randn(n, d, generator=gen) * 1e-4
    x, nw, w = inp["x"].cuda(), inp["norm_weight"].cuda(), inp["w"].cuda()
    normed = torch.empty_like(x)
    out, rstd = rmsnorm_gate_mm(x, nw, inp["eps"], w, gate, normed=normed)
    g = g0.cuda()
    dx, dnw = rmsnorm_gate_mm_backward(x, nw, rstd, normed, w, gate, out, dout.cuda(), g,
                                       in_place=in_place)
    torch.cuda.synchronize()
    assert_bf16_close(normed, oracle.rmsnorm(inp["x"], inp["norm_weight"], inp["eps"]), "normed")
    want_dx, want_dnw, want_g = oracle.rmsnorm_gate_projection_backward(
        inp["x"], inp["norm_weight"], inp["eps"], inp["w"], gate, dout, g0)
    assert_bf16_close(dx, want_dx, "dx")
    assert rel_l2(dnw, want_dnw) <= 3e-3
    assert_f32_close(g.cpu(), want_g, "W_in gradient")


def _assert_equal_where_normal(a, b, name):
    """Bitwise equality on the elements where both values are zero or normal; elements that
    are subnormal in either (where scaling by a power of two need not commute with rounding)
    only need to agree within one unit of the smallest normal number."""
    tiny = torch.finfo(torch.float32).tiny
    fa, fb = a.float(), b.float()
    sub = ((fa.abs() < tiny) & (fa != 0)) | ((fb.abs() < tiny) & (fb != 0))
    assert torch.equal(a[~sub], b[~sub]), name
    assert bool(((fa[sub] - fb[sub]).abs() <= tiny).all()), name


@pytest.mark.parametrize("rows,d,vocab,chunk", [(512, 256, 1024, 256), (3000, 384, 2052, 1024),
                                                (700, 136, 1030, 512), (1001, 128, 2048, 256)])
def test_fused_cross_entropy_matches_the_two_pass_backward(rows, d, vocab, chunk):
    """The one-pass fused loss (chunk logits kept in the workspace, gradients formed while
    they are there) gives, for a unit upstream gradient, the two-pass loss, dHidden and
    head-weight gradient bit for bit; another upstream gradient scales them. Shapes cover a
    last 4-column piece (2052) and a vocabulary the stored-logits epilogue cannot take (1030,
    which recomputes the chunk's logits)."""
    from ops.fused_execution import (CrossEntropyState, linear_cross_entropy_backward,
                                     linear_cross_entropy_forward)

    gen = _gen(405)
    h = torch.randn(rows, d, generator=gen).bfloat16()
    w = (torch.randn(vocab, d, generator=gen) * 0.05).bfloat16()
    t = torch.randint(0, vocab, (rows,), generator=gen)
    t[::5] = -100
    hc, wc, tc = h.cuda(), w.cuda(), t.cuda()
    for g in (1.0, 0.25, 0.75, 2.0 ** 20, 2.0 ** -20, 2.0 ** 40):
        grad = torch.full((), g, device="cuda")
        got = []
        for fused in (False, True):
            state = CrossEntropyState(rows, vocab, hc.device, chunk_rows=chunk, d=d,
                                      fused=fused, weight_grad=fused)
            linear_cross_entropy_forward(hc, wc, tc, state)
            # Bit-exact comparisons start from zero (the fused pass adds its chunk sum to
            # the buffer at the end, the two-pass backward chunk by chunk).
            gw = torch.full((vocab, d), 0.0 if g != 0.75 else 0.5, device="cuda")
            dh = linear_cross_entropy_backward(hc, wc, tc, state, grad, weight_grad=gw)
            got.append((state, dh, gw))
        torch.cuda.synchronize()
        (a, dha, gwa), (b, dhb, gwb) = got
        for name in ("loss", "lse", "mean", "count"):
            assert torch.equal(getattr(a, name), getattr(b, name)), name
        # A power of two 2^e with |e| <= 32 scales the unit gradients exactly wherever both
        # results are normal numbers; 0.75 and 2^40 run the two-pass backward (chosen on
        # the device) and so match it exactly too.
        _assert_equal_where_normal(dha, dhb, f"fused dHidden, upstream {g}")
        if g != 0.75:
            _assert_equal_where_normal(gwa, gwb, f"fused dW, upstream {g}")
        else:
            assert_f32_close(gwb.cpu(), gwa.cpu(), "fused dW, upstream 0.75")
    want_loss, _mean, count, want_dh = oracle.linear_cross_entropy(h, w, t)
    assert int(b.count.item()) == count
    assert_f32_close(b.loss.cpu(), want_loss, "fused per-token loss")


def test_cross_entropy_combine_and_logit_gradient_entry_points():
    """ws_linear_ce_combine recomputes the forward's second phase from its partials (same
    bits); ws_linear_ce_logit_grad turns BF16 logits into the oracle's logit gradients."""
    from ops import _hip
    from ops.fused_execution import CrossEntropyState, linear_cross_entropy_forward

    rows, d, vocab = 640, 256, 2048
    gen = _gen(406)
    h = torch.randn(rows, d, generator=gen).bfloat16()
    w = (torch.randn(vocab, d, generator=gen) * 0.05).bfloat16()
    t = torch.randint(0, vocab, (rows,), generator=gen)
    t[::9] = -100
    hc, wc, tc = h.cuda(), w.cuda(), t.cuda()
    state = linear_cross_entropy_forward(hc, wc, tc)
    again = CrossEntropyState(rows, vocab, hc.device)
    _hip.call("ws_linear_ce_combine", state.part_max.data_ptr(), state.part_sum.data_ptr(),
              state.target_logit.data_ptr(), tc.data_ptr(), again.lse.data_ptr(),
              again.loss.data_ptr(), again.mean.data_ptr(), again.count.data_ptr(), rows, vocab,
              _hip.stream(hc))
    logits = oracle.mm(h, w.T)
    count = int(t.ne(-100).sum())
    scale = torch.full((1,), 0.5 / count, device="cuda")
    out = torch.empty(rows, vocab, dtype=torch.bfloat16, device="cuda")
    gl = logits.cuda()
    _hip.call("ws_linear_ce_logit_grad", gl.data_ptr(), vocab, tc.data_ptr(),
              state.lse.data_ptr(), scale.data_ptr(), out.data_ptr(), vocab, rows, vocab,
              _hip.stream(hc))
    torch.cuda.synchronize()
    for name in ("lse", "loss", "mean", "count"):
        assert torch.equal(getattr(state, name), getattr(again, name)), name
    soft = torch.softmax(logits.float(), dim=-1)
    onehot = torch.zeros_like(soft)
    valid = t.ne(-100)
    onehot[valid.nonzero().squeeze(1), t[valid]] = 1.0
    want = ((soft - onehot) * (0.5 / count) * valid.unsqueeze(1)).bfloat16()
    assert_bf16_close(out, want, "logit gradients")
    assert torch.count_nonzero(out.cpu()[~valid]).item() == 0


@pytest.mark.parametrize("rows,cols,gate", [(16384, 9216, (6144, 8192)), (37, 80, (13, 61)),
                                            (1000, 264, (0, 264)), (3, 24, (8, 8)),
                                            (257, 1032, (515, 1029))])
@pytest.mark.parametrize("mode", ["in_place", "out_of_place", "unaligned"])
def test_sigmoid_backward_cols_bits(rows, cols, gate, mode):
    """dP = r((dout (1 - s)) s) on the gate columns and dout elsewhere, bit for bit against
    the same FP32 expression on the CPU: in place (only the gate columns' 8-column groups
    are touched, the others keep their bits), into a fresh buffer, and with views 2 bytes
    off a 16-byte boundary (the one-element path)."""
    from ops.fused_execution import sigmoid_backward_cols

    gen = _gen(31)
    dout = (torch.randn(rows, cols, generator=gen) * 1e-2).bfloat16()
    s = torch.rand(rows, cols, generator=gen).bfloat16()
    lo, hi = gate
    want = dout.clone()
    g, sv = dout[:, lo:hi].float(), s[:, lo:hi].float()
    want[:, lo:hi] = ((g * (1.0 - sv)) * sv).bfloat16()
    print(f"sigmoid backward {rows}x{cols} gate={gate} {mode}", flush=True)
    if mode == "unaligned":
        def shifted(t):
            buf = torch.empty(t.numel() + 8, dtype=t.dtype, device="cuda")
            view = buf[1:1 + t.numel()].view(t.shape)
            view.copy_(t.cuda())
            return view
        d, o = shifted(dout), shifted(s)
        got = sigmoid_backward_cols(d, o, gate)
    elif mode == "in_place":
        d = dout.cuda()
        got = sigmoid_backward_cols(d, s.cuda(), gate, d)
        assert got.data_ptr() == d.data_ptr()
    else:
        got = sigmoid_backward_cols(dout.cuda(), s.cuda(), gate)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu().view(torch.int16), want.view(torch.int16))
