"""GPU results against the committed known-answer fixtures (tests/golden/fixtures.npz).

The fixtures hold ragged-shape inputs and expected outputs computed by the independent
numpy restatement (exact float64 products, integer BF16 rounding); every HIP entry point
of the hot path is run on them through the C ABI. Bars: BF16 max|d|/max|ref| <= 1e-2 and
rel-RMS <= 3e-3; FP32 accumulators ||d||/||ref|| <= 1e-3; valid-token count bit-exact.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from metrics import assert_bf16_close, assert_f32_close

pytestmark = pytest.mark.gpu

FIX = np.load(Path(__file__).resolve().parent / "golden" / "fixtures.npz")


def t16(name, device="cuda"):
    return torch.from_numpy(FIX[name].astype(np.int16)).view(torch.bfloat16).to(device)


def f32(name, device="cuda"):
    return torch.from_numpy(FIX[name]).to(device)


@pytest.mark.parametrize("layout", ["nn", "nt", "tn", "tt"])
@pytest.mark.parametrize("algorithm", ["tiled", "persistent"])
def test_mm_fixture_all_layouts(layout, algorithm):
    from ops.matmul_kernels import launch_mm

    a, b = t16("mm_a"), t16("mm_b")
    if layout[0] == "t":
        a = a.T.contiguous().T
    if layout[1] == "t":
        b = b.T.contiguous().T
    out = launch_mm(a, b, algorithm, (128, 128, 32, 4, 3))
    torch.cuda.synchronize()
    assert_bf16_close(out, t16("mm_c", "cpu"), f"mm {layout}")


@pytest.mark.parametrize("eager", [True, False])
def test_swiglu_mm_fixture(eager):
    from ops.matmul_epilogue import launch_swiglu_mm

    packed, act = launch_swiglu_mm(t16("sw_x"), t16("sw_w").T, "tiled", (128, 128, 32, 8, 3), eager)
    torch.cuda.synchronize()
    assert_bf16_close(packed, t16("sw_packed", "cpu"), "packed")
    assert_bf16_close(act, t16("sw_act_eager" if eager else "sw_act_compiled", "cpu"), "act")


@pytest.mark.parametrize("eager", [True, False])
def test_swiglu_backward_fixture(eager):
    from ops.activation_execution import _swiglu_backward

    out = _swiglu_backward(t16("sw_packed"), t16("swb_dy"), eager)
    torch.cuda.synchronize()
    assert_bf16_close(out, t16("swb_eager" if eager else "swb_compiled", "cpu"), "swiglu bwd")


def test_swiglu_backward_epilogue_fixture():
    from ops.fused_execution import swiglu_backward_mm

    out = swiglu_backward_mm(t16("swbm_g"), t16("swbm_w_down"), t16("sw_packed"), True)
    torch.cuda.synchronize()
    assert_bf16_close(out, t16("swbm_dpacked", "cpu"), "swiglu bwd epilogue")


def test_rmsnorm_gate_projection_fixture():
    from ops.fused_execution import rmsnorm_gate_mm

    gate = tuple(int(v) for v in FIX["rms_gate"])
    out, rstd = rmsnorm_gate_mm(t16("rms_x"), f32("rms_nw"), float(FIX["rms_eps"][0]),
                                t16("rms_w"), gate)
    torch.cuda.synchronize()
    assert_bf16_close(out, t16("rms_out", "cpu"), "rms gate projection")
    assert_f32_close(rstd.cpu(), f32("rms_rstd", "cpu"), "rstd")


def test_residual_fixture():
    from ops.fused_execution import residual_mm

    out = residual_mm(t16("res_h"), t16("res_w"), t16("res_r"))
    torch.cuda.synchronize()
    assert_bf16_close(out, t16("res_out", "cpu"), "residual")


@pytest.mark.parametrize("round_bf16", [True, False])
@pytest.mark.parametrize("splits", [1, 2])
def test_accumulate_fixture(round_bf16, splits):
    from ops.fused_execution import mm_accumulate_

    g = f32("acc_g").clone()
    mm_accumulate_(g, t16("acc_a"), t16("acc_b"), round_bf16, splits)
    torch.cuda.synchronize()
    want = f32("acc_round" if round_bf16 else "acc_direct", "cpu")
    assert_f32_close(g.cpu(), want, "accumulate")


def test_linear_cross_entropy_fixture():
    from ops.fused_execution import linear_cross_entropy_backward, linear_cross_entropy_forward

    hidden, weight = t16("ce_hidden"), t16("ce_weight")
    targets = torch.from_numpy(FIX["ce_targets"]).cuda()
    state = linear_cross_entropy_forward(hidden, weight, targets)
    dh = linear_cross_entropy_backward(hidden, weight, targets, state, torch.ones((), device="cuda"))
    torch.cuda.synchronize()
    assert int(state.count.item()) == int(FIX["ce_count"][0])
    np.testing.assert_allclose(state.loss.cpu().numpy(), FIX["ce_loss"], rtol=1e-3, atol=1e-4)
    assert abs(state.mean.item() - float(FIX["ce_mean"][0])) <= 1e-4 * abs(float(FIX["ce_mean"][0]))
    assert torch.all(state.loss.cpu()[targets.cpu() == -100] == 0)
    assert_bf16_close(dh, t16("ce_dhidden", "cpu"), "dhidden")
