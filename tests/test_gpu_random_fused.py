"""Seeded random shapes through the fused entry points, against the CPU oracle.

Each case draws its sizes (1 to about 1100 per GEMM dimension; vocabularies up to 3000,
multiples of 8 and not), prints them, and checks the HIP path against the oracle at the
bars of the fixed-shape tests (BF16 max|d|/max|ref| <= 1e-2 and rel-RMS <= 3e-3, FP32
||d||/||ref|| <= 1e-3, counts exact):

* the RMSNorm-prologue projection with a random gate column range;
* the dAct GEMM with the SwiGLU backward epilogue, both roundings;
* the fused LM-head cross-entropy in its two-pass and one-pass modes (loss, mean, count,
  dHidden), random chunk sizes and ignored targets;
* the FP32 store GEMMs against accumulation into zeroed buffers, bit for bit.
"""
import random

import pytest
import torch

from metrics import assert_bf16_close, assert_f32_close
from oracle import reference as oracle

pytestmark = pytest.mark.gpu

CASES = 12


def _dim(rng, lo=1, hi=1100):
    kind = rng.randrange(3)
    if kind == 0:
        return max(lo, 8 * rng.randint(1, hi // 8))
    if kind == 1:
        return max(lo, 256 * rng.randint(1, max(1, hi // 256)))
    return rng.randint(lo, hi)


@pytest.mark.parametrize("seed", range(CASES))
def test_random_rmsnorm_gate_projection(seed):
    from ops.fused_execution import rmsnorm_gate_mm

    rng = random.Random(5000 + seed)
    m, d, n = _dim(rng), _dim(rng, 8), _dim(rng)
    lo = rng.randint(0, n)
    hi = rng.randint(lo, n)
    gen = torch.Generator("cpu").manual_seed(seed)
    x = torch.randn(m, d, generator=gen).bfloat16()
    nw = torch.rand(d, generator=gen) * 1.9 + 0.1
    w = (torch.randn(n, d, generator=gen) * 0.05).bfloat16()
    print(f"rms gate projection seed={seed} m={m} d={d} n={n} gate=({lo}, {hi})", flush=True)
    out, rstd = rmsnorm_gate_mm(x.cuda(), nw.cuda(), 1e-6, w.cuda(), (lo, hi))
    torch.cuda.synchronize()
    assert_bf16_close(out, oracle.rmsnorm_gate_projection(x, nw, 1e-6, w, (lo, hi)), "projection")
    assert_f32_close(rstd.cpu(), oracle.rms_rstd(x, 1e-6), "rstd")


@pytest.mark.parametrize("seed", range(CASES))
def test_random_swiglu_backward_gemm(seed):
    from ops.fused_execution import swiglu_backward_mm

    rng = random.Random(6000 + seed)
    m, h, k = _dim(rng), max(1, _dim(rng) // 2), _dim(rng)
    eager = rng.random() < 0.5
    gen = torch.Generator("cpu").manual_seed(50 + seed)
    dy = (torch.randn(m, k, generator=gen) * 0.1).bfloat16()
    w_down = (torch.randn(k, h, generator=gen) * 0.05).bfloat16()
    packed = torch.randn(m, 2 * h, generator=gen).bfloat16()
    print(f"swiglu backward gemm seed={seed} m={m} h={h} k={k} eager={eager}", flush=True)
    got = swiglu_backward_mm(dy.cuda(), w_down.cuda(), packed.cuda(), eager)
    torch.cuda.synchronize()
    want = oracle.swiglu_backward(packed, oracle.mm(dy, w_down), eager)
    assert_bf16_close(got, want, "dPacked")


@pytest.mark.parametrize("seed", range(CASES))
def test_random_linear_cross_entropy(seed):
    from ops.fused_execution import (CrossEntropyState, linear_cross_entropy_backward,
                                     linear_cross_entropy_forward)

    rng = random.Random(7000 + seed)
    rows, d = _dim(rng), _dim(rng, 8, 512)
    vocab = rng.choice([_dim(rng, 8, 3000), rng.randint(2, 3000)])
    chunk = rng.choice([64, 256, 1024, 8192])
    fused = rng.random() < 0.5
    gen = torch.Generator("cpu").manual_seed(70 + seed)
    hidden = torch.randn(rows, d, generator=gen).bfloat16()
    weight = (torch.randn(vocab, d, generator=gen) * 0.05).bfloat16()
    targets = torch.randint(0, vocab, (rows,), generator=gen, dtype=torch.int64)
    targets[torch.rand(rows, generator=gen) < 0.1] = -100
    print(f"cross entropy seed={seed} rows={rows} d={d} vocab={vocab} chunk={chunk} "
          f"fused={fused}", flush=True)
    h, w, t = hidden.cuda(), weight.cuda(), targets.cuda()
    state = CrossEntropyState(rows, vocab, h.device, chunk_rows=chunk, d=d, fused=fused)
    linear_cross_entropy_forward(h, w, t, state)
    dh = linear_cross_entropy_backward(h, w, t, state, torch.ones((), device="cuda"))
    torch.cuda.synchronize()
    loss, mean, count, dh_ref = oracle.linear_cross_entropy(hidden, weight, targets, chunk)
    assert int(state.count.item()) == count
    assert_f32_close(state.loss.cpu(), loss, "loss")
    assert abs(state.mean.item() - mean.item()) <= 1e-3 * abs(mean.item()) + 1e-6
    assert_bf16_close(dh, dh_ref, "dHidden")


@pytest.mark.parametrize("seed", range(CASES))
def test_random_fp32_store_matches_accumulation_into_zeros(seed):
    from ops.fused_execution import mm_accumulate_, mm_accumulate_group_, mm_f32, mm_f32_group

    rng = random.Random(8000 + seed)
    tokens = _dim(rng)
    round_bf16 = rng.random() < 0.7
    gen = torch.Generator("cpu").manual_seed(80 + seed)
    pairs = []
    for _ in range(rng.randint(1, 3)):
        n_out, n_in = _dim(rng), _dim(rng)
        dy = torch.randn(tokens, n_out, generator=gen).bfloat16().cuda()
        x = torch.randn(tokens, n_in, generator=gen).bfloat16().cuda()
        pairs.append((dy.T, x))
    print(f"fp32 store seed={seed} tokens={tokens} "
          f"{[(tuple(a.shape), tuple(b.shape)) for a, b in pairs]} round={round_bf16}", flush=True)
    if len(pairs) == 1:
        (a, b), = pairs
        splits = rng.choice([1, 2, 3])
        got = [mm_f32(a, b, round_bf16, splits=splits)]
        want = [mm_accumulate_(torch.zeros(a.shape[0], b.shape[1], device="cuda"), a, b,
                               round_bf16, splits)]
    else:
        got = mm_f32_group(pairs, round_bf16)
        want = [torch.zeros(a.shape[0], b.shape[1], device="cuda") for a, b in pairs]
        mm_accumulate_group_([(g, a, b) for g, (a, b) in zip(want, pairs)], round_bf16)
    torch.cuda.synchronize()
    for g, w in zip(got, want):
        assert torch.equal(g, w), seed
    a, b = pairs[0]
    ref = oracle.accumulate_weight_grad(torch.zeros(a.shape[0], b.shape[1]), a.cpu(), b.cpu(),
                                        round_bf16)
    assert_f32_close(got[0].cpu(), ref, "FP32 gradient against the oracle")
