"""Pins of the layout oracle (oracle/layout.py) and the host contract of ops.backward_layout.

``fma32`` is checked against exact rational arithmetic and Dekker's exact product error.
The layout restates the reference's own CPU tests (test_backward_layout.py:16-99) and is
compared with the independent eager expression within the reference's CUDA tolerance
(test_backward_layout.py:120-125).
"""
from fractions import Fraction
import math

import numpy as np
import pytest
import torch

from oracle.layout import backward_layout, fma32
from ops.backward_layout import (ALGORITHMS, PROFILE_SHAPE, LayoutInputs, make_inputs,
                                 prepare_layout, reference_layout, validate_inputs)


def round_to_f32(q: Fraction) -> np.float32:
    """Exact round-to-nearest-even of a rational to FP32 (normal and subnormal range)."""
    if q == 0:
        return np.float32(0.0)
    sign = -1 if q < 0 else 1
    q = abs(q)
    e = q.numerator.bit_length() - q.denominator.bit_length()
    if Fraction(2) ** e > q:
        e -= 1
    ulp = Fraction(2) ** (max(e, -126) - 23)
    scaled = q / ulp
    whole = scaled.numerator // scaled.denominator
    rest = scaled - whole
    if rest > Fraction(1, 2) or (rest == Fraction(1, 2) and whole % 2):
        whole += 1
    return np.float32(sign * float(whole * ulp))


def exact(x) -> Fraction:
    return Fraction(float(np.float32(x)))


def test_fma32_matches_exact_rounding_on_random_and_tie_cases():
    rng = np.random.default_rng(5)
    a = (rng.standard_normal(3000) * np.exp2(rng.integers(-30, 30, 3000))).astype(np.float32)
    b = (rng.standard_normal(3000) * np.exp2(rng.integers(-30, 30, 3000))).astype(np.float32)
    c = (rng.standard_normal(3000) * np.exp2(rng.integers(-60, 60, 3000))).astype(np.float32)
    # Midpoint cases: (1 + 2^-12)^2 = 1 + 2^-11 + 2^-24 is halfway between two FP32 values;
    # a tiny c decides the direction, which a double rounding through float64 loses.
    t = np.float32(1 + 2.0 ** -12)
    a = np.concatenate([a, [t, t, -t, t]]).astype(np.float32)
    b = np.concatenate([b, [t, t, t, t]]).astype(np.float32)
    c = np.concatenate([c, [2.0 ** -60, -2.0 ** -60, 2.0 ** -60, 0.0]]).astype(np.float32)
    got = fma32(a, b, c)
    want = np.array([round_to_f32(exact(x) * exact(y) + exact(z)) for x, y, z in zip(a, b, c)],
                    dtype=np.float32)
    assert np.array_equal(got, want)
    assert got[-4] == np.float32(1 + 2.0 ** -11 + 2.0 ** -23)  # rounded up past the midpoint
    assert got[-3] == np.float32(1 + 2.0 ** -11)               # rounded down
    assert got[-1] == np.float32(1 + 2.0 ** -11)               # exact tie: to even
    # A float64 sum rounded once more to FP32 gets the first case wrong.
    naive = (t.astype(np.float64) * t + 2.0 ** -60).astype(np.float32)
    assert naive != got[-4]


def test_fma32_recovers_the_exact_product_error():
    """fma(a, b, -r(ab)) is the exact error ab - r(ab) (representable in FP32)."""
    rng = np.random.default_rng(9)
    a = rng.standard_normal(10000).astype(np.float32)
    b = rng.standard_normal(10000).astype(np.float32)
    p = (a * b).astype(np.float32)
    err = fma32(a, b, -p)
    assert np.array_equal(err.astype(np.float64), a.astype(np.float64) * b - p.astype(np.float64))
    assert np.count_nonzero(err) > 9000


def token_major(value):
    b, n, h, c, d = value.shape
    return value.permute(0, 1, 3, 2, 4).reshape(b, n * c, h * d)


def with_distinct_tables(inputs, seed=799):
    gen = torch.Generator().manual_seed(seed)
    return inputs._replace(sin=torch.randn(inputs.sin.shape, generator=gen),
                           cos=torch.randn(inputs.cos.shape, generator=gen))


def test_pair_direction_and_projection_packing():
    inputs = make_inputs((1, 2, 2, 3, 4))
    value = torch.arange(1, 49, dtype=torch.bfloat16).reshape(inputs.q_memory.shape)
    inputs = inputs._replace(q_memory=value, q_local=torch.zeros_like(value),
                             k_write=torch.zeros_like(inputs.k_write), k_local=value,
                             v_local=value + 1, sin=torch.ones_like(inputs.sin),
                             cos=torch.zeros_like(inputs.cos))
    wanted = token_major(torch.stack((value[..., 1::2], -value[..., ::2]), -1).flatten(-2))
    for layout in (backward_layout(inputs), reference_layout(inputs)):
        q, k, v, _, _ = layout.chunk(5, -1)
        assert torch.equal(q, wanted) and torch.equal(k, wanted)
        assert torch.equal(v, token_major(value + 1))


def test_q_matches_model_rope_vjp_with_unequal_pair_coefficients():
    from warpstate.model import apply_rope

    inputs = with_distinct_tables(make_inputs((2, 3, 2, 7, 6), seed=921))
    original = torch.zeros_like(inputs.q_memory, dtype=torch.float32, requires_grad=True)
    gradient, = torch.autograd.grad(apply_rope(original, inputs.cos, inputs.sin), original,
                                    grad_outputs=inputs.q_memory.float() + inputs.q_local.float())
    expected = token_major(gradient.bfloat16())
    # The eager expression rounds like autograd: bit for bit.
    assert torch.equal(reference_layout(inputs).chunk(5, -1)[0], expected)
    # The contracted arithmetic differs by at most one BF16 step, and rarely.
    q = backward_layout(inputs).chunk(5, -1)[0]
    torch.testing.assert_close(q, expected, rtol=2 ** -7, atol=1e-6)
    assert (q == expected).float().mean() > 0.97


def test_model_rope_helpers_match_their_definitions():
    from warpstate.model import rope_cos_sin, rotate_half

    x = torch.arange(8.0).reshape(1, 8)
    assert torch.equal(rotate_half(x), torch.tensor([[-1.0, 0, -3, 2, -5, 4, -7, 6]]))
    cos, sin = rope_cos_sin(5, 6, torch.device("cpu"), torch.float64)
    t = torch.arange(5.0, dtype=torch.float64)[:, None]
    inv = 1.0 / 10000 ** (torch.tensor([0.0, 2.0, 4.0], dtype=torch.float64) / 6)
    angle = (t * inv).repeat_interleave(2, dim=-1)
    torch.testing.assert_close(cos, angle.cos(), rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(sin, angle.sin(), rtol=1e-6, atol=1e-6)
    assert torch.equal(cos[:, 0::2], cos[:, 1::2]) and torch.equal(sin[0], torch.zeros(6, dtype=torch.float64))


def test_k_intermediate_bf16_rounding_is_observable():
    inputs = make_inputs((1, 2, 2, 7, 16), seed=19)
    k = (inputs.k_write.transpose(-2, -1).float() * (1 - inputs.tanh_k.float().square())
         + inputs.k_local.float())
    sine = k * inputs.sin
    unrounded = torch.stack((sine[..., 1::2], -sine[..., ::2]), -1).flatten(-2)
    wrong = token_major((unrounded + k * inputs.cos).bfloat16())
    assert torch.any(backward_layout(inputs).chunk(5, -1)[1] != wrong)
    assert torch.any(reference_layout(inputs).chunk(5, -1)[1] != wrong)


def test_gate_matches_independent_autograd_and_u_packing():
    inputs = make_inputs((1, 2, 2, 3, 4), seed=987)
    inputs = inputs._replace(tanh_u=torch.zeros_like(inputs.tanh_u))
    gate = inputs.gate.float().requires_grad_()
    blended = gate * inputs.local.float() + (1 - gate) * inputs.memory.float() / 2
    dy = inputs.grad_y.reshape(1, 2, 3, 2, 4).permute(0, 1, 3, 2, 4).float()
    derivative, = torch.autograd.grad(blended, gate, grad_outputs=dy)
    expected = token_major((derivative * gate * (1 - gate)).bfloat16())
    for layout in (backward_layout(inputs), reference_layout(inputs)):
        _, _, _, actual, u = layout.chunk(5, -1)
        torch.testing.assert_close(actual, expected, rtol=0.01, atol=1e-6)
        assert torch.equal(u, token_major(inputs.u_write))


def test_u_and_k_tanh_backward_closed_forms():
    """With sin = 0 and cos = 1: k = bf16(k_write (1 - tanh^2) + k_local), q = bf16(q_m + q_l);
    a zero tanh leaves u = u_write exactly and a tanh of +-1 zeroes it."""
    inputs = make_inputs((1, 1, 2, 4, 6), seed=3)
    ones = torch.ones_like(inputs.tanh_u)
    inputs = inputs._replace(sin=torch.zeros_like(inputs.sin), cos=torch.ones_like(inputs.cos),
                             tanh_u=torch.where(torch.arange(6) % 2 == 0, ones, -ones))
    q, k, _, _, u = backward_layout(inputs).chunk(5, -1)
    assert torch.equal(u, torch.zeros_like(u))
    assert torch.equal(q, token_major((inputs.q_memory.float() + inputs.q_local.float()).bfloat16()))
    kf = (inputs.k_write.transpose(-2, -1).double() * (1 - inputs.tanh_k.double() ** 2)
          + inputs.k_local.double())
    # fma(kw, fma(-t, t, 1), kl) is within an FP32 rounding of the exact value.
    torch.testing.assert_close(k.float(), token_major(kf.bfloat16()).float(), rtol=2 ** -7,
                               atol=0)


def one_pair(**values):
    """Inputs of shape (1, 1, 1, 1, 2) (one rotary pair) with the given lane values."""
    inputs = make_inputs((1, 1, 1, 1, 2), seed=0)
    fields = {}
    for name, tensor in zip(inputs._fields, inputs, strict=True):
        value = values.get(name, (0.0, 0.0))
        fields[name] = torch.tensor(value, dtype=tensor.dtype).reshape(tensor.shape)
    return LayoutInputs(**fields)


def test_bf16_midpoint_cases_pin_the_half_term_rounding_and_the_contraction():
    """Closed forms chosen to sit on BF16 midpoints, so one FP32 ulp decides the result.

    X = 2^-8 + 2^-20: q_e = bf16(1 + X) rounds up to 1 + 2^-7, while the key's half-term
    is rounded first, bf16(X) = 2^-8, and bf16(1 + 2^-8) ties to 1. For q's multiply-add,
    the product p = (1 + 2^-12)(2 + 3 2^-13) = P0 + 3 2^-25 (P0 a multiple of 2^-22) plus
    the half-term h = (1 + 2^-8) - P0 is 1 + 2^-8 + 3 2^-25: fused, it rounds to
    1 + 2^-8 + 2^-23 and then up to 1 + 2^-7; with p rounded first (down, to P0) the sum
    is the BF16 midpoint 1 + 2^-8 exactly, which ties down to 1."""
    x = 2.0 ** -8 + 2.0 ** -20
    inputs = one_pair(q_memory=(1.0, 1.0), k_local=(1.0, 1.0), sin=(0.0, x), cos=(1.0, 1.0))
    q, k, _, _, _ = backward_layout(inputs).chunk(5, -1)
    assert q.flatten().tolist() == [1.0 + 2.0 ** -7, 1.0]
    assert k.flatten().tolist() == [1.0, 1.0]
    p0 = 2.0 + 2.0 ** -11 + 2.0 ** -12 + 2.0 ** -13
    h = (1.0 + 2.0 ** -8) - p0
    assert np.float32(h) == h and (1 + 2.0 ** -12) * (2 + 3 * 2.0 ** -13) == p0 + 3 * 2.0 ** -25
    inputs = one_pair(q_memory=(1.0, 1.0), q_local=(2.0 ** -12, 0.0), sin=(0.0, h),
                      cos=(2.0 + 3 * 2.0 ** -13, 1.0))
    q = backward_layout(inputs).chunk(5, -1)[0]
    assert q.flatten().tolist() == [1.0 + 2.0 ** -7, 1.0]
    # The same inputs with the product rounded before the add give the tie value.
    unfused = np.float32(np.float32(np.float32(1 + 2.0 ** -12) * np.float32(2 + 3 * 2.0 ** -13))
                         + np.float32(h))
    assert float(torch.tensor(float(unfused)).bfloat16()) == 1.0


def test_gate_and_u_closed_forms():
    """gate = 1/2 makes gate (1 - gate) = 1/4; with memory = 0 the gradient is
    bf16(dy local / 4), with local = 0 it is bf16(-dy memory scale / 4); tanh_u = 1/2 gives
    u = bf16(0.75 u_write). Every product here is exact."""
    dy, loc, mem, uw = (0.75, -1.5), (3.0, 0.25), (5.0, -2.0), (1.25, -3.0)
    base = dict(gate=(0.5, 0.5), grad_y=dy, u_write=uw, tanh_u=(0.5, -0.5))
    g1, u = [s.flatten().tolist() for s in
             backward_layout(one_pair(local=loc, **base)).chunk(5, -1)[3:]]
    assert g1 == [dy[0] * loc[0] / 4, dy[1] * loc[1] / 4]
    assert u == [0.75 * uw[0], 0.75 * uw[1]]
    scale = 2 ** -0.5  # head_dim 2; the product is not exact, so compare in FP32 first
    g2 = backward_layout(one_pair(memory=mem, **base)).chunk(5, -1)[3].flatten()
    want = [float(torch.tensor(-(dy[i] * np.float32(mem[i] * np.float32(scale))) / 4,
                               dtype=torch.float32).bfloat16()) for i in range(2)]
    assert g2.tolist() == want
    assert float(g2[0]) < 0 and float(g2[1]) < 0  # -dy memory: 0.75 * 5 and -1.5 * -2 > 0


@pytest.mark.parametrize("shape,seed", [((1, 2, 3, 7, 10), 455), ((2, 3, 2, 16, 64), 455),
                                        ((1, 1, 1, 1, 2), 1), ((1, 2, 1, 41, 8), 77)])
def test_oracle_agrees_with_eager_expression_within_reference_tolerance(shape, seed):
    inputs = with_distinct_tables(make_inputs(shape, seed=seed), seed=seed + 1)
    actual, expected = backward_layout(inputs), reference_layout(inputs)
    for value, wanted in zip(actual.chunk(5, -1), expected.chunk(5, -1), strict=True):
        assert torch.isfinite(value).all()
        error = (value.float() - wanted.float()).norm() / wanted.float().norm().clamp_min(1e-20)
        assert float(error) < 0.002
        torch.testing.assert_close(value, wanted, rtol=0.015, atol=1e-4)
    # v is a copy.
    assert torch.equal(actual.chunk(5, -1)[2], token_major(inputs.v_local))


def test_make_inputs_is_deterministic_and_shaped():
    a = make_inputs((1, 2, 2, 3, 4), seed=5)
    b = make_inputs((1, 2, 2, 3, 4), seed=5)
    c = make_inputs((1, 2, 2, 3, 4), seed=6)
    assert all(torch.equal(x, y) for x, y in zip(a, b, strict=True))
    assert not torch.equal(a.q_memory, c.q_memory)
    assert validate_inputs(a) == (1, 2, 2, 3, 4)
    assert float(a.tanh_k.abs().max()) <= 1 and 0 <= float(a.gate.min()) <= float(a.gate.max()) <= 1


@pytest.mark.parametrize("case", ["dtype", "k_shape", "rope_dtype", "strides", "device", "odd_head"])
def test_contract_rejects_unsupported_inputs(case):
    inputs = make_inputs((1, 2, 2, 3, 4))
    if case == "dtype":
        inputs = inputs._replace(q_memory=inputs.q_memory.float())
    elif case == "k_shape":
        inputs = inputs._replace(k_write=inputs.k_write[..., :-1])
    elif case == "rope_dtype":
        inputs = inputs._replace(sin=inputs.sin.bfloat16())
    elif case == "strides":
        inputs = inputs._replace(v_local=inputs.v_local.transpose(1, 2))
    elif case == "device":
        inputs = inputs._replace(gate=torch.empty(inputs.gate.shape, device="meta",
                                                  dtype=torch.bfloat16))
    else:
        inputs = inputs._replace(q_memory=inputs.q_memory[..., :-1])
    with pytest.raises(ValueError):
        validate_inputs(inputs)


def test_contract_requires_named_inputs_and_a_gpu():
    with pytest.raises(TypeError):
        validate_inputs(tuple(make_inputs((1, 1, 1, 1, 2))))
    with pytest.raises(ValueError, match="require CUDA"):
        prepare_layout(make_inputs((1, 1, 1, 1, 2)))
    assert ALGORITHMS == ("profile", "paired", "single") and math.prod(PROFILE_SHAPE) == 2 ** 24
    assert LayoutInputs._fields[:4] == ("q_memory", "q_local", "sin", "cos")


def test_benchmark_distinguishes_signed_zero_and_serializes_nonfinite_outputs():
    import json

    from ops.backward_layout_benchmark import output_errors

    expected = torch.zeros((1, 1, 10), dtype=torch.bfloat16)
    actual = expected.clone()
    actual[0, 0, 0] = -0.0
    report = output_errors(actual, expected)
    assert report["q"]["unequal"] == 0
    assert report["q"]["bitwise_unequal"] == 1
    actual[0, 0, 3] = float("nan")
    report = output_errors(actual, expected)
    assert not report["k"]["finite"] and report["k"]["relative_rms"] is None
    json.dumps(report, allow_nan=False)
