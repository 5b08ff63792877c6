"""Error metrics shared by the parity tests.

Tolerances (stated once, used everywhere):
* BF16 outputs: max|d| / max|ref| <= 1e-2 against the CPU oracle (FP32-accumulated);
  rel-RMS < 3e-3 as in the reference's own GEMM tests (test_matmul_kernels.py:161-163).
* FP32 gradient accumulators: ||d|| / ||ref|| <= 1e-3.
* Integer results (targets, counts): bit-exact.
"""
import torch

BF16_MAX_REL = 1e-2
BF16_REL_RMS = 3e-3
F32_REL_L2 = 1e-3


def max_rel(actual, expected):
    a, e = actual.float().cpu(), expected.float().cpu()
    return ((a - e).abs().max() / e.abs().max().clamp_min(1e-30)).item()


def rel_rms(actual, expected):
    a, e = actual.float().cpu(), expected.float().cpu()
    return ((a - e).square().mean().sqrt() / e.square().mean().sqrt().clamp_min(1e-30)).item()


def rel_l2(actual, expected):
    a, e = actual.double().cpu(), expected.double().cpu()
    return ((a - e).norm() / e.norm().clamp_min(1e-30)).item()


def assert_bf16_close(actual, expected, what=""):
    assert actual.dtype == torch.bfloat16, what
    assert actual.shape == expected.shape, what
    assert torch.isfinite(actual.float()).all(), what
    mr, rr = max_rel(actual, expected), rel_rms(actual, expected)
    assert mr <= BF16_MAX_REL and rr <= BF16_REL_RMS, f"{what}: max_rel={mr:.3e} rel_rms={rr:.3e}"


def assert_f32_close(actual, expected, what=""):
    assert actual.dtype == torch.float32, what
    r = rel_l2(actual, expected)
    assert r <= F32_REL_L2, f"{what}: rel_l2={r:.3e}"
