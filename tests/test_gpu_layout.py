"""GPU parity of the packed attention-backward gradient layout (ws_backward_layout).

The HIP result must equal the oracle's bits (oracle/layout.py restates the kernel
arithmetic exactly), agree with the eager tensor expression within the reference's
tolerance (test_backward_layout.py:120-125), leave the inputs untouched, and give the same
bits under all three algorithms.
"""
import pytest
import torch

from oracle.layout import backward_layout
from ops.backward_layout import (PROFILE_SHAPE, launch_layout, make_inputs, prepare_layout,
                                 reference_layout)

pytestmark = pytest.mark.gpu


def cuda_inputs(shape, seed, distinct_tables=True):
    inputs = make_inputs(shape, device="cuda", seed=seed)
    if distinct_tables:  # distinct pair coefficients catch a wrong rotary lane
        gen = torch.Generator(device="cuda").manual_seed(seed + 1)
        inputs = inputs._replace(
            sin=torch.randn(inputs.sin.shape, device="cuda", generator=gen),
            cos=torch.randn(inputs.cos.shape, device="cuda", generator=gen))
    return inputs


def cpu(inputs):
    return type(inputs)(*(value.cpu() for value in inputs))


def assert_bits(actual, expected):
    assert actual.shape == expected.shape and actual.dtype == torch.bfloat16
    diff = actual.view(torch.int16) != expected.view(torch.int16)
    if diff.any():
        section = (diff.nonzero()[0, -1] // (actual.shape[-1] // 5)).item()
        raise AssertionError(f"{int(diff.sum())} elements differ, first in section {section}")


@pytest.mark.parametrize("algorithm", ["paired", "single"])
@pytest.mark.parametrize("shape", [(1, 2, 3, 7, 10), (2, 3, 2, 16, 64), (1, 1, 1, 1, 2),
                                   (1, 2, 1, 41, 8), (1, 1, 2, 9, 2048), (2, 1, 3, 130, 64),
                                   (1, 2, 1, 40, 1024), (1, 1, 2, 256, 64)])
def test_matches_oracle_bits_and_eager_tolerance(algorithm, shape):
    print(f"layout {algorithm} {shape}", flush=True)
    inputs = cuda_inputs(shape, seed=455)
    saved = [value.clone() for value in inputs]
    actual = launch_layout(inputs, algorithm)
    torch.cuda.synchronize()
    assert actual.is_contiguous() and actual.shape == (shape[0], shape[1] * shape[3],
                                                       5 * shape[2] * shape[4])
    assert_bits(actual.cpu(), backward_layout(cpu(inputs)))
    expected = reference_layout(inputs)
    for value, wanted in zip(actual.chunk(5, -1), expected.chunk(5, -1), strict=True):
        assert torch.isfinite(value).all()
        error = (value.float() - wanted.float()).norm() / wanted.float().norm().clamp_min(1e-20)
        assert float(error) < 0.002
        torch.testing.assert_close(value, wanted, rtol=0.015, atol=1e-4)
    assert all(torch.equal(value, original) for value, original in zip(inputs, saved, strict=True))


def test_unaligned_views_take_the_element_path():
    """Inputs at a 2-byte offset (not 16-byte aligned) still give the oracle's bits."""
    shape = (1, 2, 2, 16, 64)
    base = make_inputs(shape, device="cuda", seed=3)

    def shifted(value):
        flat = torch.empty(value.numel() + 1, dtype=value.dtype, device="cuda")
        view = flat[1:].view(value.shape)
        view.copy_(value)
        return view

    inputs = type(base)(*(shifted(v) if v.dtype == torch.bfloat16 else v for v in base))
    assert inputs.q_memory.data_ptr() % 16 != 0
    assert_bits(launch_layout(inputs, "single").cpu(), backward_layout(cpu(inputs)))


def test_profile_shape_algorithms_agree_bitwise_with_each_other_and_the_oracle():
    print("layout profile shape", flush=True)
    inputs = make_inputs(PROFILE_SHAPE, device="cuda", seed=817)
    scratch = tuple(torch.empty_like(inputs.q_memory) for _ in range(2))
    baseline = launch_layout(inputs, "profile", scratch=scratch).clone()
    for algorithm in ("paired", "single"):
        assert torch.equal(launch_layout(inputs, algorithm, block=512).view(torch.int16),
                           baseline.view(torch.int16))
    assert_bits(baseline.cpu(), backward_layout(cpu(inputs)))
    # The scratch holds the final q (head-major) after the first profile pass.
    q = baseline.chunk(5, -1)[0].view(4, 16, 128, 32, 64).transpose(2, 3)
    assert torch.equal(scratch[0], q)


def test_preallocated_output_and_repeat_calls():
    inputs = cuda_inputs((2, 2, 2, 32, 64), seed=11)
    out = torch.full((2, 64, 5 * 128), float("nan"), dtype=torch.bfloat16, device="cuda")
    operation = prepare_layout(inputs, "paired", output=out)
    first = operation().clone()
    assert operation() is out and torch.equal(out, first)
    assert torch.isfinite(out).all()


def test_aliasing_and_profile_contract_errors():
    inputs = make_inputs((1, 2, 2, 3, 4), device="cuda")
    shared = torch.zeros(48 + 240, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="alias"):
        prepare_layout(inputs._replace(v_local=shared[:48].view(1, 2, 2, 3, 4)),
                       output=shared[48:].view(1, 6, 40))
    with pytest.raises(ValueError, match="PROFILE_SHAPE"):
        prepare_layout(inputs, "profile")
    with pytest.raises(ValueError, match="Unknown backward layout algorithm"):
        prepare_layout(inputs, "fused")
    with pytest.raises(ValueError, match="block"):
        prepare_layout(inputs, block=64)


def test_profile_scratch_cannot_alias():
    inputs = make_inputs(PROFILE_SHAPE, device="cuda")
    scratch = torch.empty_like(inputs.q_memory)
    for values in ((scratch, scratch), (inputs.q_local, scratch)):
        with pytest.raises(ValueError, match="Scratch tensors may not alias"):
            prepare_layout(inputs, "profile", scratch=values)
