"""GPU parity of the plain BF16 GEMM (launch_mm / ws_mm) against the CPU oracle.

Restates test_matmul_kernels.py:147-188 (odd shapes, all four operand layouts, both
schedules, inputs never modified) and adds aligned shapes that take the vector loaders,
both macro-tiles and the persistent_tma path. Bar: max|d|/max|ref| <= 1e-2 and
rel-RMS < 3e-3 against the oracle, and near-bit agreement with the FP32-dot reference.
"""
import pytest
import torch

from metrics import assert_bf16_close, max_rel
from oracle import reference as oracle

pytestmark = pytest.mark.gpu

LAYOUTS = [(False, False), (False, True), (True, False), (True, True)]


def _operands(m, n, k, layouts, seed, device="cuda", scale=1.0):
    gen = torch.Generator("cpu").manual_seed(seed)
    a = (torch.randn((k, m) if layouts[0] else (m, k), generator=gen) * scale).bfloat16()
    b = (torch.randn((n, k) if layouts[1] else (k, n), generator=gen) * scale).bfloat16()
    a = a.T if layouts[0] else a
    b = b.T if layouts[1] else b
    ga, gb = a.to(device), b.to(device)
    assert ga.stride() == a.stride() and gb.stride() == b.stride()
    return a, b, ga, gb


@pytest.mark.parametrize("algorithm", ["tiled", "persistent"])
@pytest.mark.parametrize("layouts", LAYOUTS)
@pytest.mark.parametrize("tile", [(128, 128, 32, 4, 3), (64, 64, 32, 4, 3)])
def test_odd_shapes_and_transposed_operands(algorithm, layouts, tile):
    from ops.matmul_kernels import launch_mm

    a, b, ga, gb = _operands(97, 113, 129, layouts, 77)
    ga_copy, gb_copy = ga.clone(), gb.clone()
    out = launch_mm(ga, gb, algorithm, tile)
    torch.cuda.synchronize()
    assert out.is_contiguous() and out.shape == (97, 113)
    assert_bf16_close(out, oracle.mm(a, b), f"{algorithm} {layouts} {tile}")
    assert torch.equal(ga, ga_copy) and torch.equal(gb, gb_copy)


@pytest.mark.parametrize("layouts", LAYOUTS)
@pytest.mark.parametrize("shape", [(256, 384, 512), (520, 264, 200), (1024, 2048, 1024),
                                   (264, 260, 136), (300, 516, 256)])
@pytest.mark.parametrize("tile", [(128, 128, 32, 4, 3), (64, 64, 32, 4, 3)])
def test_aligned_shapes_vector_loaders(layouts, shape, tile):
    from ops.matmul_kernels import launch_mm

    m, n, k = shape
    a, b, ga, gb = _operands(m, n, k, layouts, 561)
    out = launch_mm(ga, gb, "tiled", tile)
    torch.cuda.synchronize()
    assert_bf16_close(out, oracle.mm(a, b), f"{shape} {layouts} {tile}")
    # FP32 accumulation: agreement with r(f32 a @ f32 b) up to rare last-bit flips.
    ref32 = oracle.mm_f32_reference(a, b)
    assert max_rel(out, ref32) <= 8e-3
    assert (out.cpu() != ref32).float().mean().item() < 0.02


@pytest.mark.parametrize("layouts", LAYOUTS)
def test_persistent_tma_layouts_with_masked_output_tiles(layouts):
    from ops.matmul_kernels import launch_mm

    a, b, ga, gb = _operands(96, 112, 128, layouts, 3)
    out = launch_mm(ga, gb, "persistent_tma")
    torch.cuda.synchronize()
    assert_bf16_close(out, oracle.mm(a, b), f"tma {layouts}")


def test_strided_view_uses_generic_loader():
    from ops.matmul_kernels import launch_mm

    gen = torch.Generator("cpu").manual_seed(11)
    a = torch.randn(48, 40, generator=gen).bfloat16()
    b_full = torch.randn(40, 70, generator=gen).bfloat16()
    b = b_full[:, ::2]
    out = launch_mm(a.cuda(), b_full.cuda()[:, ::2], "tiled", (128, 128, 32, 4, 3))
    torch.cuda.synchronize()
    assert_bf16_close(out, oracle.mm(a, b), "strided")


def test_exact_small_integer_products():
    """Integer-valued operands: every partial sum is exact in FP32, so the result must equal
    the exact product bit for bit (pins the MFMA fragment and output layouts)."""
    from ops.matmul_kernels import launch_mm

    gen = torch.Generator("cpu").manual_seed(5)
    for m, n, k in [(64, 64, 64), (256, 256, 128), (300, 260, 72)]:
        a = torch.randint(-3, 4, (m, k), generator=gen).bfloat16()
        b = torch.randint(-3, 4, (k, n), generator=gen).bfloat16()
        exact = (a.double() @ b.double()).bfloat16()
        for tile in [(128, 128, 32, 4, 3), (64, 64, 32, 4, 3)]:
            out = launch_mm(a.cuda(), b.cuda(), "tiled", tile)
            torch.cuda.synchronize()
            assert torch.equal(out.cpu(), exact), (m, n, k, tile)
            outt = launch_mm(a.T.contiguous().cuda().T, b.T.contiguous().cuda().T, "tiled", tile)
            torch.cuda.synchronize()
            assert torch.equal(outt.cpu(), exact), (m, n, k, tile, "transposed")


@pytest.mark.parametrize("shape,stride_pad", [((64, 64), 0), ((1000, 2056), 8), ((37, 91), 5),
                                              ((2048, 11264), 0), ((8, 8), 0), ((24, 520), 16),
                                              ((11264, 2048), 0), ((9216, 2048), 0),
                                              ((2048, 5632), 8), ((40, 12), 4)])
def test_transpose_is_bit_exact(shape, stride_pad):
    """The weight-layout transpose used by the input-gradient GEMMs moves bits only: the
    register kernel (rows, columns and stride multiples of 8, including partial 64 x 256
    tiles) and the LDS kernel (any other shape)."""
    from ops.fused_execution import transpose

    rows, cols = shape
    gen = torch.Generator("cpu").manual_seed(21)
    full = torch.randn(rows, cols + stride_pad, generator=gen).bfloat16().cuda()
    x = full[:, :cols]
    out = transpose(x)
    torch.cuda.synchronize()
    assert out.shape == (cols, rows) and out.is_contiguous()
    assert torch.equal(out.cpu(), x.cpu().T.contiguous())


def test_input_gradient_layout_uses_transposed_weight_and_matches():
    """dX = dY @ W with W N-contiguous and many rows takes the transposed-weight path; the
    result must match the oracle as any other layout does."""
    from ops.fused_execution import k_contiguous_b
    from ops.matmul_kernels import launch_mm

    gen = torch.Generator("cpu").manual_seed(8)
    dy = torch.randn(2048, 640, generator=gen).bfloat16()
    w = (torch.randn(640, 384, generator=gen) * 0.05).bfloat16()
    gdy, gw = dy.cuda(), w.cuda()
    assert k_contiguous_b(gw, 2048).stride() == (1, 640)
    out = launch_mm(gdy, gw, "tiled", (128, 128, 32, 4, 3))
    torch.cuda.synchronize()
    assert_bf16_close(out, oracle.mm(dy, w), "dX with transposed weight")
