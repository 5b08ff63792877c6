"""Bit-exact GPU checks of the 256 x 256 GEMM's four operand layouts at the k-tile counts
its pipelines treat specially.

Integer-valued BF16 operands in [-3, 3] make every FP32 partial sum an integer below 2^24,
so any summation order gives the exact product, and the BF16 output must equal the
exactly rounded product bit for bit (the reference's layout test,
test_matmul_kernels.py:147-188, holds its kernels to a BF16 bar on random data; exact
operands pin the fragment, stage and output indexing here). The shapes cover one to five
64-wide k-tiles (with both operands K-contiguous, B runs through three LDS stages and its
first two k-tiles are issued before the loop; with both M/N-contiguous, the next k-tile's
loads are issued at the top of each k-tile), a ragged last k-tile, ragged row and column
tiles, and a reduction long enough for the stages to wrap many times. Every width is a
multiple of 8, so every operand takes a vector loader and the launch the 256 x 256 path.
"""
import pytest
import torch

from ops import _hip

pytestmark = pytest.mark.gpu

SHAPES = [(256, 256, 64), (256, 256, 128), (256, 512, 192), (512, 256, 256), (256, 256, 320),
          (264, 520, 200), (520, 264, 1000)]
# (A M-contiguous, B N-contiguous): False = K-contiguous.
LAYOUTS = [(False, False), (False, True), (True, False), (True, True)]


def _int_operand(rows, cols, gen):
    return torch.randint(-3, 4, (rows, cols), generator=gen).bfloat16()


@pytest.mark.parametrize("layouts", LAYOUTS)
@pytest.mark.parametrize("shape", SHAPES)
def test_fast_gemm_exact_integer_products(shape, layouts):
    m, n, k = shape
    gen = torch.Generator("cpu").manual_seed(m * 7 + n * 3 + k)
    a, b = _int_operand(m, k, gen), _int_operand(k, n, gen)
    exact = (a.float() @ b.float()).bfloat16()
    ga = a.T.contiguous().cuda().T if layouts[0] else a.cuda()
    gb = b.cuda() if layouts[1] else b.T.contiguous().cuda().T
    assert (ga.stride(0) == 1) == layouts[0] and (gb.stride(1) == 1) == layouts[1]
    out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    print(f"fast gemm {shape} layouts={layouts}", flush=True)
    _hip.call("ws_mm", ga.data_ptr(), ga.stride(0), ga.stride(1), gb.data_ptr(), gb.stride(0),
              gb.stride(1), out.data_ptr(), m, n, k, 0, 0, _hip.stream(ga))
    torch.cuda.synchronize()
    got = out.cpu()
    assert torch.equal(got, exact), (shape, layouts, (got != exact).sum().item())


@pytest.mark.parametrize("round_bf16", [False, True])
@pytest.mark.parametrize("tokens", [520, 1000])
def test_balanced_accumulation_exact_integer_products(round_bf16, tokens):
    """G += a @ b over the balanced stream-K plan (272 tiles: 256 whole, 16 shared by all
    workgroups, pieces of one or a few k-tiles) with integer-valued G and operands: the
    FP32 result is exact, so it equals G + the exact product (rounded to BF16 first when
    round_bf16) bit for bit, whatever the split."""
    from ops.fused_execution import mm_accumulate_

    gen = torch.Generator("cpu").manual_seed(tokens + int(round_bf16))
    n_out, n_in = 17 * 256, 16 * 256
    dy, x = _int_operand(tokens, n_out, gen), _int_operand(tokens, n_in, gen)
    g = torch.randint(-100, 101, (n_out, n_in), generator=gen).float()
    product = dy.float().T @ x.float()
    want = g + (product.bfloat16().float() if round_bf16 else product)
    gg = g.cuda()
    print(f"balanced accumulate tokens={tokens} round_bf16={round_bf16}", flush=True)
    mm_accumulate_(gg, dy.cuda().T, x.cuda(), round_bf16, 2)
    torch.cuda.synchronize()
    got = gg.cpu()
    assert torch.equal(got, want), (tokens, round_bf16, (got != want).sum().item())
