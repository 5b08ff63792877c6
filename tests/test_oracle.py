"""Pins the CPU oracle (oracle/reference.py) before any GPU result is judged against it.

Each oracle function is checked against (a) the committed known-answer fixtures in
tests/golden/fixtures.npz, produced by an independent numpy restatement with exact float64
products and integer BF16 rounding (tests/golden/bf16_numpy.py); (b) closed forms and
special cases the mathematics fixes (zero weights, all-ignored targets, exact-integer
products, invariances); and (c) for the derivatives, float64 autograd of the unrounded
formula. The reference's own CPU tests that pin these functions are restated where they
apply (test_matmul_epilogue.py:12-24, test_loss_execution.py:15-58,
test_gradient_execution.py:219-256). Each check is chosen so that a plausible slip (up and
gate swapped, a dropped rounding, a transposed operand, a wrong denominator) fails it.
"""
import math
import sys
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import bf16_numpy as ref  # noqa: E402

from oracle import reference as oracle  # noqa: E402

FIX = np.load(Path(__file__).resolve().parent / "golden" / "fixtures.npz")


def t16(name):
    """Fixture BF16 array (uint16 bits) as a torch bfloat16 tensor."""
    return torch.from_numpy(FIX[name].astype(np.int16)).view(torch.bfloat16)


def as_bits(tensor):
    return tensor.contiguous().view(torch.int16).numpy().view(np.uint16)


def ulp_diff(actual, expected_bits):
    """|difference| in BF16 units in the last place (same-sign values)."""
    a = as_bits(actual).astype(np.int32)
    e = expected_bits.astype(np.int32)
    sa = np.where(a & 0x8000, -(a & 0x7FFF), a & 0x7FFF)
    se = np.where(e & 0x8000, -(e & 0x7FFF), e & 0x7FFF)
    return np.abs(sa - se)


def assert_bf16_bits_close(actual, expected_bits, max_frac=0.02, max_ulp=1):
    """Equal bit patterns except a small fraction that differ by at most `max_ulp` ULP
    (FP32 accumulation order versus the exact sum, or libm versus numpy exp)."""
    d = ulp_diff(actual, expected_bits)
    assert d.max() <= max_ulp, f"max ulp {d.max()}"
    assert (d > 0).mean() <= max_frac, f"mismatch fraction {(d > 0).mean():.4f}"


# --- GEMM ---------------------------------------------------------------------------

def test_mm_matches_exact_products_rounded_once():
    out = oracle.mm(t16("mm_a"), t16("mm_b"))
    assert_bf16_bits_close(out, FIX["mm_c"], max_frac=0.01)


def test_mm_exact_on_integer_operands_and_transposes():
    gen = torch.Generator().manual_seed(5)
    a = torch.randint(-3, 4, (37, 53), generator=gen).bfloat16()
    b = torch.randint(-3, 4, (53, 29), generator=gen).bfloat16()
    exact = (a.double() @ b.double()).bfloat16()
    assert torch.equal(oracle.mm(a, b), exact)
    # (a b)^T = b^T a^T pins operand order.
    assert torch.equal(oracle.mm(b.T, a.T), exact.T)


def test_mm_f32_reference_matches_exact_products_rounded_once():
    """r(f32(a) @ f32(b)) against the fixture's exact float64 products rounded once: the
    FP32 sum differs from the exact one by far less than half a BF16 ulp, so at most one
    ulp on a small fraction of ties."""
    out = oracle.mm_f32_reference(t16("mm_a"), t16("mm_b"))
    assert out.dtype == torch.bfloat16
    assert_bf16_bits_close(out, FIX["mm_c"], max_frac=0.01)


def test_mm_f32_reference_exact_on_integer_operands_and_order():
    gen = torch.Generator().manual_seed(6)
    a = torch.randint(-4, 5, (19, 67), generator=gen).bfloat16()
    b = torch.randint(-4, 5, (67, 23), generator=gen).bfloat16()
    exact = (a.double() @ b.double()).bfloat16()
    assert torch.equal(oracle.mm_f32_reference(a, b), exact)
    assert torch.equal(oracle.mm_f32_reference(b.T, a.T), exact.T)
    # A sum whose exact value needs more than BF16's 8 bits is rounded once at the end:
    # 257 = 256 + 1 rounds to 256 (ties to even), while per-term BF16 rounding would not
    # change it; 255 + 2 = 257 -> 256 and 256 + 3 = 259 -> 260.
    a2 = torch.tensor([[255.0, 2.0], [256.0, 3.0]]).bfloat16()
    b2 = torch.tensor([[1.0], [1.0]]).bfloat16()
    assert oracle.mm_f32_reference(a2, b2).float().flatten().tolist() == [256.0, 260.0]


# --- Paired SwiGLU GEMM --------------------------------------------------------------

@pytest.mark.parametrize("eager", [True, False])
def test_swiglu_mm_fixture(eager):
    packed, act = oracle.swiglu_mm(t16("sw_x"), t16("sw_w").T, eager)
    assert_bf16_bits_close(packed, FIX["sw_packed"], max_frac=0.01)
    # The activation of the *oracle's* packed must equal the closed form bit-exactly up to
    # libm/numpy exp ulps; the fixture activation comes from the fixture packed.
    key = "sw_act_eager" if eager else "sw_act_compiled"
    same = torch.equal(packed, t16("sw_packed"))
    assert_bf16_bits_close(act, FIX[key], max_frac=0.01 if same else 0.03,
                           max_ulp=1 if same else 2)


@pytest.mark.parametrize("eager_rounding", [False, True])
def test_swiglu_mm_reference_closed_form(eager_rounding):
    """test_matmul_epilogue.py:12-24: packed = a @ b, act = the model's closed form."""
    torch.manual_seed(554)
    a = torch.randn(7, 31, dtype=torch.bfloat16)
    b = torch.randn(46, 31, dtype=torch.bfloat16).T
    packed, act = oracle.swiglu_mm(a, b, eager_rounding)
    expected = a @ b
    up, gate = expected.chunk(2, dim=-1)
    wanted = F.silu(gate) * up if eager_rounding else (F.silu(gate.float()) * up.float()).bfloat16()
    assert torch.equal(packed, expected) and torch.equal(act, wanted)


def test_swiglu_up_is_first_half_and_zero_gate_gives_zero():
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(16, 8, generator=gen).bfloat16()
    w = torch.randn(24, 8, generator=gen).bfloat16()
    w[12:] = 0  # gate rows
    _, act = oracle.swiglu_mm(x, w.T, True)
    assert torch.count_nonzero(act) == 0
    w2 = torch.randn(24, 8, generator=gen).bfloat16()
    w2[:12] = 0  # up rows
    _, act2 = oracle.swiglu_mm(x, w2.T, True)
    assert torch.count_nonzero(act2) == 0


def test_eager_rounding_changes_only_the_silu_rounding():
    gen = torch.Generator().manual_seed(9)
    packed = torch.randn(64, 256, generator=gen).bfloat16()
    eager, compiled = oracle.swiglu(packed, True), oracle.swiglu(packed, False)
    assert not torch.equal(eager, compiled)
    assert_bf16_bits_close(eager, ref.f32_to_bf16_bits(ref.swiglu(packed.float().numpy(), True)))
    assert_bf16_bits_close(compiled, ref.f32_to_bf16_bits(ref.swiglu(packed.float().numpy(), False)))


# --- SwiGLU backward -----------------------------------------------------------------

@pytest.mark.parametrize("eager", [True, False])
def test_swiglu_backward_fixture(eager):
    out = oracle.swiglu_backward(t16("sw_packed"), t16("swb_dy"), eager)
    assert_bf16_bits_close(out, FIX["swb_eager" if eager else "swb_compiled"], max_frac=0.02)


def test_swiglu_backward_equals_float64_autograd():
    gen = torch.Generator().manual_seed(11)
    packed = torch.randn(32, 64, generator=gen).bfloat16()
    dy = torch.randn(32, 32, generator=gen).bfloat16()
    src = packed.double().requires_grad_(True)
    up, gate = src.chunk(2, dim=-1)
    (gate * torch.sigmoid(gate) * up).backward(dy.double())
    for eager in (True, False):
        got = oracle.swiglu_backward(packed, dy, eager).double()
        rel = (got - src.grad).norm() / src.grad.norm()
        assert rel < 5e-3, rel


# --- RMSNorm-prologue projection -----------------------------------------------------

def test_rms_rstd_and_gate_projection_fixture():
    x, nw, w = t16("rms_x"), torch.from_numpy(FIX["rms_nw"]), t16("rms_w")
    eps = float(FIX["rms_eps"][0])
    gate = tuple(int(v) for v in FIX["rms_gate"])
    rstd = oracle.rms_rstd(x, eps)
    np.testing.assert_allclose(rstd.numpy(), FIX["rms_rstd"], rtol=2e-6)
    out = oracle.rmsnorm_gate_projection(x, nw, eps, w, gate)
    assert_bf16_bits_close(out, FIX["rms_out"], max_frac=0.02, max_ulp=2)


def test_rmsnorm_zero_weight_gives_half_in_gate_and_zero_elsewhere():
    gen = torch.Generator().manual_seed(4)
    x = torch.randn(9, 64, generator=gen).bfloat16()
    nw = torch.randn(64, generator=gen) * 0.1 + 1
    out = oracle.rmsnorm_gate_projection(x, nw, 1e-6, torch.zeros(40, 64, dtype=torch.bfloat16), (8, 20))
    assert torch.all(out[:, 8:20] == 0.5)
    assert torch.count_nonzero(out[:, :8]) == 0 and torch.count_nonzero(out[:, 20:]) == 0


def test_rmsnorm_zero_row_and_scale_invariance():
    gen = torch.Generator().manual_seed(6)
    x = torch.randn(8, 128, generator=gen).bfloat16()
    x[3] = 0
    nw = torch.randn(128, generator=gen) * 0.1 + 1
    y = oracle.rmsnorm(x, nw, 1e-6)
    assert torch.count_nonzero(y[3]) == 0
    # Multiplying a row by 4 is exact in BF16 and leaves RMSNorm unchanged (eps aside).
    y4 = oracle.rmsnorm(x * 4, nw, 1e-12)
    y1 = oracle.rmsnorm(x, nw, 1e-12)
    assert torch.equal(y4, y1)
    # Unit weight: every nonzero row has mean square 1 up to BF16 rounding.
    ms = oracle.rmsnorm(x, torch.ones(128), 0.0).float().pow(2).mean(dim=1)
    assert torch.allclose(ms[torch.arange(8) != 3], torch.ones(7), atol=1e-2)


def test_rmsnorm_fp32_product_against_float64_and_special_cases():
    """The compiled-path RMSNorm (no eager rounding) is the float64 closed form rounded once
    to BF16: every element within one BF16 rounding of it. A zero row and a zero weight give
    exact zeros; scaling a row by 4 (exact in BF16) leaves it unchanged when eps is
    negligible; and it differs from the eager form, which rounds x rstd and w first."""
    gen = torch.Generator().manual_seed(8)
    x = torch.randn(16, 200, generator=gen).bfloat16()
    x[5] = 0
    nw = torch.randn(200, generator=gen) * 0.1 + 1
    y = oracle.rmsnorm_fp32_product(x, nw, 1e-6)
    x64 = x.double()
    want = x64 * torch.rsqrt(x64.pow(2).mean(-1, keepdim=True) + 1e-6) * nw.double()
    ulp = want.abs().clamp_min(1e-30) * 2.0 ** -8
    assert bool(((y.double() - want).abs() <= ulp).all())
    assert torch.count_nonzero(y[5]) == 0
    assert torch.count_nonzero(oracle.rmsnorm_fp32_product(x, torch.zeros(200), 1e-6)) == 0
    assert torch.equal(oracle.rmsnorm_fp32_product(x * 4, nw, 1e-12),
                       oracle.rmsnorm_fp32_product(x, nw, 1e-12))
    assert not torch.equal(y, oracle.rmsnorm(x, nw, 1e-6))


# --- Residual epilogue ---------------------------------------------------------------

def test_residual_fixture_and_zero_weight_identity():
    out = oracle.residual_projection(t16("res_h"), t16("res_w"), t16("res_r"))
    assert_bf16_bits_close(out, FIX["res_out"], max_frac=0.02)
    zero = oracle.residual_projection(t16("res_h"), torch.zeros_like(t16("res_w")), t16("res_r"))
    assert torch.equal(zero, t16("res_r"))


# --- FP32 weight-gradient accumulation -----------------------------------------------

def test_accumulate_fixture_both_modes():
    g = torch.from_numpy(FIX["acc_g"])
    a, b = t16("acc_a"), t16("acc_b")
    got = oracle.accumulate_weight_grad(g.clone(), a, b, True)
    exp = FIX["acc_round"]
    # One BF16 ULP of the product at most, in a few elements (FP32 sum order).
    np.testing.assert_allclose(got.numpy(), exp, rtol=0, atol=np.abs(exp - FIX["acc_g"]).max() * 2 ** -7)
    assert np.mean(got.numpy() != exp) < 0.02
    direct = oracle.accumulate_weight_grad(g.clone(), a, b, False)
    np.testing.assert_allclose(direct.numpy(), FIX["acc_direct"], rtol=1e-5, atol=1e-5)
    assert not torch.equal(got, direct)


def test_accumulate_zero_gradient_is_identity_and_matches_reference_rule():
    g = torch.randn(12, 16)
    dy = torch.zeros(8, 12, dtype=torch.bfloat16)
    x = torch.randn(8, 16, dtype=torch.bfloat16)
    assert torch.equal(oracle.accumulate_weight_grad(g, dy.T, x), g)
    # test_gradient_execution.py:243-246: reference.add_((derivative.T @ inputs).float()).
    torch.manual_seed(901)
    dy = torch.randn(8, 12, dtype=torch.bfloat16)
    want = g + (dy.T @ x).float()
    assert torch.equal(oracle.accumulate_weight_grad(g, dy.T, x), want)


def test_mlp_backward_matches_float64_autograd():
    from ops.benchmark_configs import mlp_backward_inputs

    inp = mlp_backward_inputs(m=64, d=48, ffn=40, seed=3)
    x, wug, wd, dy = inp["x"], inp["w_upgate"], inp["w_down"], inp["dy"] * 100
    packed, act = oracle.swiglu_mm(x, wug.T, True)
    g_up, g_down = torch.zeros(80, 48), torch.zeros(48, 40)
    dx, dpacked, g_up, g_down = oracle.mlp_backward(x, wug, wd, packed, act, dy, g_up, g_down)
    xd = x.double().requires_grad_(True)
    wugd = wug.double().requires_grad_(True)
    wdd = wd.double().requires_grad_(True)
    up, gate = (xd @ wugd.T).chunk(2, dim=-1)
    y = (gate * torch.sigmoid(gate) * up) @ wdd.T
    y.backward(dy.double())
    for got, want in ((dx, xd.grad), (g_up, wugd.grad), (g_down, wdd.grad)):
        rel = (got.double() - want).norm() / want.norm()
        assert rel < 2e-2, rel


# --- LM-head cross-entropy -------------------------------------------------------------

def test_linear_cross_entropy_fixture():
    loss, mean, count, dh = oracle.linear_cross_entropy(t16("ce_hidden"), t16("ce_weight"),
                                                        torch.from_numpy(FIX["ce_targets"]))
    assert count == int(FIX["ce_count"][0]) == 57
    np.testing.assert_allclose(loss.numpy(), FIX["ce_loss"], rtol=2e-5, atol=2e-5)
    assert math.isclose(mean.item(), float(FIX["ce_mean"][0]), rel_tol=2e-5)
    assert_bf16_bits_close(dh, FIX["ce_dhidden"], max_frac=0.03)
    assert torch.all(loss[torch.from_numpy(FIX["ce_targets"]) == -100] == 0)


def test_linear_cross_entropy_zero_weight_is_log_vocab():
    hidden = torch.randn(40, 16).bfloat16()
    weight = torch.zeros(64, 16, dtype=torch.bfloat16)
    targets = torch.randint(0, 64, (40,))
    targets[:5] = -100
    loss, mean, count, dh = oracle.linear_cross_entropy(hidden, weight, targets, chunk=7)
    assert count == 35
    assert torch.allclose(loss[5:], torch.full((35,), math.log(64)), atol=1e-6)
    assert torch.all(loss[:5] == 0)
    assert abs(mean.item() - math.log(64)) < 1e-6
    assert torch.count_nonzero(dh) == 0


def test_linear_cross_entropy_all_ignored_and_chunk_invariance():
    """test_loss_execution.py:15-58: the chunked loss equals the full loss, the
    all-masked mean is 0 with zero gradients."""
    gen = torch.Generator().manual_seed(572)
    hidden = torch.randn(30, 16, generator=gen).bfloat16()
    weight = (torch.randn(48, 16, generator=gen) * 0.3).bfloat16()
    targets = torch.randint(0, 48, (30,), generator=gen)
    full = oracle.linear_cross_entropy(hidden, weight, targets, chunk=1024)
    chunked = oracle.linear_cross_entropy(hidden, weight, targets, chunk=3)
    assert torch.equal(full[0], chunked[0])
    assert torch.allclose(full[1], chunked[1], rtol=1e-6)
    full_logits = F.linear(hidden, weight).float()
    ref_full = F.cross_entropy(full_logits, targets, reduction="sum") / targets.ne(-100).sum()
    assert torch.allclose(full[1], ref_full, rtol=1e-6)
    ignored = torch.full_like(targets, -100)
    loss, mean, count, dh = oracle.linear_cross_entropy(hidden, weight, ignored, chunk=4)
    assert count == 0 and mean.item() == 0.0
    assert torch.count_nonzero(loss) == 0 and torch.count_nonzero(dh) == 0


def test_fixture_reference_itself_is_consistent_with_brute_force_small_vocab():
    """The numpy CE restatement against a pure-Python loop on a 5 x 6 case."""
    rng = np.random.default_rng(1)
    h = ref.r32(rng.standard_normal((5, 4)).astype(np.float32))
    e = ref.r32(rng.standard_normal((6, 4)).astype(np.float32))
    t = np.array([0, 5, -100, 2, 3])
    loss, mean, count, _ = ref.linear_cross_entropy(h, e, t)
    for i in range(5):
        logits = [float(ref.r64(sum(float(h[i, k]) * float(e[j, k]) for k in range(4)))) for j in range(6)]
        want = 0.0 if t[i] == -100 else math.log(sum(math.exp(v) for v in logits)) - logits[t[i]]
        assert math.isclose(loss[i], want, rel_tol=1e-12, abs_tol=1e-12)
    assert count == 4


def test_head_weight_grad_matches_float64_autograd_and_special_cases():
    gen = torch.Generator().manual_seed(31)
    hidden = torch.randn(70, 24, generator=gen).bfloat16()
    weight = (torch.randn(96, 24, generator=gen) * 0.2).bfloat16()
    targets = torch.randint(0, 96, (70,), generator=gen)
    targets[::9] = -100
    got = oracle.linear_cross_entropy_weight_grad(hidden, weight, targets, chunk=32)
    w64 = weight.double().requires_grad_(True)
    logits = hidden.double() @ w64.T
    loss = F.cross_entropy(logits, targets, ignore_index=-100, reduction="sum") / targets.ne(-100).sum()
    loss.backward()
    rel = (got.double() - w64.grad).norm() / w64.grad.norm()
    assert rel < 2e-2, rel
    # Ignored rows contribute nothing; all ignored gives an exactly zero gradient.
    assert torch.count_nonzero(oracle.linear_cross_entropy_weight_grad(
        hidden, weight, torch.full_like(targets, -100))) == 0
    # Chunking only changes where the BF16 rounding happens.
    other = oracle.linear_cross_entropy_weight_grad(hidden, weight, targets, chunk=1024)
    assert (other - got).norm() / got.norm() < 5e-3


def test_rmsnorm_gate_backward_matches_float64_autograd():
    gen = torch.Generator().manual_seed(41)
    x = torch.randn(40, 64, generator=gen).bfloat16()
    nw = torch.randn(64, generator=gen) * 0.1 + 1
    w = (torch.randn(48, 64, generator=gen) * 0.1).bfloat16()
    dout = torch.randn(40, 48, generator=gen).bfloat16()
    gate = (16, 32)
    dx, dnw, g = oracle.rmsnorm_gate_projection_backward(x, nw, 1e-6, w, gate, dout,
                                                         torch.zeros(48, 64))
    x64 = x.double().requires_grad_(True)
    nw64 = nw.double().requires_grad_(True)
    w64 = w.double().requires_grad_(True)
    y = x64 * torch.rsqrt(x64.pow(2).mean(-1, keepdim=True) + 1e-6) * nw64
    p = y @ w64.T
    out = torch.cat([p[:, :16], torch.sigmoid(p[:, 16:32]), p[:, 32:]], dim=1)
    out.backward(dout.double())
    for got, want in ((dx, x64.grad), (dnw, nw64.grad), (g, w64.grad)):
        assert ((got.double() - want).norm() / want.norm()) < 2e-2
    # The gate columns' gradient vanishes with the sigmoid's derivative: a zero dout on the
    # other columns leaves the weight gradient zero on those rows.
    d2 = dout.clone()
    d2[:, :16] = 0
    d2[:, 32:] = 0
    _, _, g2 = oracle.rmsnorm_gate_projection_backward(x, nw, 1e-6, w, gate, d2, torch.zeros(48, 64))
    assert torch.count_nonzero(g2[:16]) == 0 and torch.count_nonzero(g2[32:]) == 0
