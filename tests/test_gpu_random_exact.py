"""Seeded random shapes, operand layouts and leading dimensions through the GEMM entry
points, checked bit for bit.

Integer-valued BF16 operands in [-3, 3] make every FP32 partial sum an exact integer, so
any tiling, split or summation order gives the exact product; outputs are then compared
with the exactly rounded product, not within a tolerance. Shapes are drawn from 1 to
1100 in each dimension (multiples of 8 and not, so the vector loaders, the generic
loader and ragged edge tiles all occur), operands are K- or M/N-contiguous with padded
leading dimensions, and each case names itself before it runs. The cases cover:

* ``ws_mm`` (tiled and persistent grids, both tile sizes) against r(A B);
* the FP32 weight-gradient accumulation, single and grouped (automatic and forced
  splits), against G + r(A B) and G + A B;
* the residual epilogue against r(R + r(A B)) with an integer residual;
* the paired SwiGLU projection's packed output against r(A B) (its activation is
  nonlinear and is checked against the oracle within the BF16 bars instead).
"""
import random

import pytest
import torch

from metrics import assert_bf16_close
from oracle import reference as oracle
from ops import _hip

pytestmark = pytest.mark.gpu

CASES = 24


def _ints(rows, cols, gen):
    return torch.randint(-3, 4, (rows, cols), generator=gen).bfloat16()


def _dim(rng):
    """1..1100: a third multiples of 8 (vector loaders), a third multiples of 256
    (whole tiles), a third anything."""
    kind = rng.randrange(3)
    if kind == 0:
        return 8 * rng.randint(1, 137)
    if kind == 1:
        return 256 * rng.randint(1, 4)
    return rng.randint(1, 1100)


def _place(x, mn_contiguous, pad, device="cuda"):
    """x [R, C] on the GPU as a view with unit column stride (or, when mn_contiguous, unit
    row stride) and a leading dimension padded by ``pad`` elements."""
    r, c = x.shape
    if mn_contiguous:
        buf = torch.zeros((c, r + pad), dtype=x.dtype, device=device)
        buf[:, :r] = x.T.to(device)
        return buf[:, :r].T
    buf = torch.zeros((r, c + pad), dtype=x.dtype, device=device)
    buf[:, :c] = x.to(device)
    return buf[:, :c]


def _case(seed):
    rng = random.Random(seed)
    m, n, k = _dim(rng), _dim(rng), _dim(rng)
    a_mn, b_n = rng.random() < 0.5, rng.random() < 0.5
    pad_a, pad_b = rng.choice([0, 0, 8, 3]), rng.choice([0, 0, 8, 5])
    return rng, m, n, k, a_mn, b_n, pad_a, pad_b


@pytest.mark.parametrize("seed", range(CASES))
def test_random_mm_exact(seed):
    rng, m, n, k, a_mn, b_n, pad_a, pad_b = _case(1000 + seed)
    algorithm, tile = rng.choice([(0, 0), (1, 0), (0, 1), (1, 1)])
    gen = torch.Generator("cpu").manual_seed(seed)
    a, b = _ints(m, k, gen), _ints(k, n, gen)
    exact = (a.float() @ b.float()).bfloat16()
    ga, gb = _place(a, a_mn, pad_a), _place(b.T, not b_n, pad_b).T
    print(f"ws_mm seed={seed} m={m} n={n} k={k} a_mn={a_mn} b_n={b_n} pads={pad_a},{pad_b} "
          f"algorithm={algorithm} tile={tile} strides={ga.stride()},{gb.stride()}", flush=True)
    out = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    _hip.call("ws_mm", ga.data_ptr(), ga.stride(0), ga.stride(1), gb.data_ptr(), gb.stride(0),
              gb.stride(1), out.data_ptr(), m, n, k, algorithm, tile, _hip.stream(ga))
    torch.cuda.synchronize()
    got = out.cpu()
    assert torch.equal(got, exact), (seed, (got != exact).sum().item())


@pytest.mark.parametrize("seed", range(CASES))
def test_random_accumulate_exact(seed):
    """G += f32(r(dY^T X)) (or the unrounded product) in the weight-gradient layout: dY
    [T, N] and X [T, K] token-major, so both GEMM operands are M/N-contiguous views, or
    copies made K-contiguous; single calls with automatic or forced splits, and a group of
    two or three gradients sharing the token count."""
    from ops.fused_execution import mm_accumulate_, mm_accumulate_group_

    rng = random.Random(2000 + seed)
    tokens = _dim(rng)
    members = 1 if rng.random() < 0.5 else rng.randint(2, 3)
    round_bf16 = rng.random() < 0.7
    gen = torch.Generator("cpu").manual_seed(100 + seed)
    items, wants = [], []
    for _ in range(members):
        n_out, n_in = _dim(rng), _dim(rng)
        dy, x = _ints(tokens, n_out, gen), _ints(tokens, n_in, gen)
        g = torch.randint(-100, 101, (n_out, n_in), generator=gen).float()
        product = dy.float().T @ x.float()
        wants.append(g + (product.bfloat16().float() if round_bf16 else product))
        k_contig = rng.random() < 0.3
        a = _place(dy.T, False, 0) if k_contig else _place(dy, False, rng.choice([0, 8])).T
        b = _place(x.T, False, 0).T if k_contig else _place(x, False, rng.choice([0, 8]))
        items.append((g.cuda(), a, b))
    shapes = [(tuple(g.shape), a.stride(), b.stride()) for g, a, b in items]
    if members == 1:
        splits = rng.choice([None, 1, 2, 3])
        print(f"accumulate seed={seed} tokens={tokens} {shapes} round={round_bf16} "
              f"splits={splits}", flush=True)
        mm_accumulate_(items[0][0], items[0][1], items[0][2], round_bf16, splits)
    else:
        print(f"accumulate group seed={seed} tokens={tokens} {shapes} round={round_bf16}",
              flush=True)
        mm_accumulate_group_(items, round_bf16)
    torch.cuda.synchronize()
    for (g, _, _), want in zip(items, wants):
        got = g.cpu()
        assert torch.equal(got, want), (seed, (got != want).sum().item())


@pytest.mark.parametrize("seed", range(CASES // 2))
def test_random_residual_exact(seed):
    from ops.fused_execution import residual_mm

    rng, m, n, k, _a_mn, _b_n, _pa, _pb = _case(3000 + seed)
    gen = torch.Generator("cpu").manual_seed(200 + seed)
    h, w = _ints(m, k, gen), _ints(n, k, gen)
    r = torch.randint(-300, 301, (m, n), generator=gen).bfloat16()
    want = (r.float() + (h.float() @ w.float().T).bfloat16().float()).bfloat16()
    print(f"residual seed={seed} m={m} n={n} k={k}", flush=True)
    out = residual_mm(h.cuda(), w.cuda(), r.cuda())
    torch.cuda.synchronize()
    got = out.cpu()
    assert torch.equal(got, want), (seed, (got != want).sum().item())


@pytest.mark.parametrize("seed", range(CASES // 2))
def test_random_paired_swiglu(seed):
    from ops.matmul_epilogue import launch_swiglu_mm

    rng = random.Random(4000 + seed)
    m, h, k = _dim(rng), max(1, _dim(rng) // 2), _dim(rng)
    algorithm = rng.choice(["tiled", "persistent"])
    tile = rng.choice([(128, 128, 32, 8, 3), (64, 64, 32, 4, 3)])
    eager = rng.random() < 0.5
    gen = torch.Generator("cpu").manual_seed(300 + seed)
    x, w = _ints(m, k, gen), _ints(2 * h, k, gen)
    print(f"paired swiglu seed={seed} m={m} h={h} k={k} {algorithm} {tile} eager={eager}",
          flush=True)
    packed, act = launch_swiglu_mm(x.cuda(), w.cuda().T, algorithm, tile, eager)
    torch.cuda.synchronize()
    assert torch.equal(packed.cpu(), (x.float() @ w.float().T).bfloat16()), seed
    # Small-integer gates drive the sigmoid into saturation; scale them into its curved
    # range for the activation check.
    xs = (torch.randn(m, k, generator=gen)).bfloat16()
    ws = (torch.randn(2 * h, k, generator=gen) * 0.05).bfloat16()
    packed, act = launch_swiglu_mm(xs.cuda(), ws.cuda().T, algorithm, tile, eager)
    torch.cuda.synchronize()
    want_packed, want_act = oracle.swiglu_mm(xs, ws.T, eager)
    assert_bf16_close(packed, want_packed, f"packed seed={seed}")
    assert_bf16_close(act, want_act, f"act seed={seed}")
