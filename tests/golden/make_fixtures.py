"""Write ``tests/golden/fixtures.npz``: small known-answer vectors for the hot path.

Inputs come from numpy's seeded PCG64 generator, rounded to BF16; expected outputs come
from ``bf16_numpy`` (exact float64 products rounded once, integer-arithmetic BF16
rounding), never from torch or from the reference's code. BF16 arrays are stored as
uint16 bit patterns. Shapes are ragged on purpose (odd M, N, K; partial tiles).

Run from the repository root:  python tests/golden/make_fixtures.py
"""

from __future__ import annotations

from pathlib import Path

import numpy as np

import bf16_numpy as ref

OUT = Path(__file__).resolve().parent / "fixtures.npz"


def bf(rng, shape, std=1.0, mean=0.0):
    return ref.r32((rng.standard_normal(shape) * std + mean).astype(np.float32))


def bits(x):
    return ref.f32_to_bf16_bits(x)


def main():
    rng = np.random.default_rng(20250601)
    f = {}
    # Plain GEMM, the reference's ragged test shape (test_matmul_kernels.py:147-165).
    a, b = bf(rng, (97, 129)), bf(rng, (129, 113))
    f.update(mm_a=bits(a), mm_b=bits(b), mm_c=bits(ref.mm(a, b)))
    # Paired SwiGLU GEMM: x [130, 72], packed weight [2*88, 72] (up rows first).
    x, w = bf(rng, (130, 72)), bf(rng, (176, 72), 0.1)
    packed = ref.mm(x, w.T).astype(np.float32)
    f.update(sw_x=bits(x), sw_w=bits(w), sw_packed=bits(packed),
             sw_act_eager=bits(ref.swiglu(packed, True)),
             sw_act_compiled=bits(ref.swiglu(packed, False)))
    # Standalone SwiGLU backward on that packed projection.
    dy = bf(rng, (130, 88))
    f.update(swb_dy=bits(dy), swb_eager=bits(ref.swiglu_backward(packed, dy, True)),
             swb_compiled=bits(ref.swiglu_backward(packed, dy, False)))
    # Down-projection dgrad with the SwiGLU backward epilogue: dact = r(g @ W_down),
    # W_down in nn.Linear layout [d, H].
    g, w_down = bf(rng, (130, 40)), bf(rng, (40, 88), 0.1)
    dact = ref.mm(g, w_down).astype(np.float32)
    f.update(swbm_g=bits(g), swbm_w_down=bits(w_down),
             swbm_dpacked=bits(ref.swiglu_backward(packed, dact, True)))
    # RMSNorm-prologue projection with gate sigmoid.
    x = bf(rng, (80, 256))
    nw = (rng.standard_normal(256) * 0.1 + 1.0).astype(np.float32)
    w = bf(rng, (200, 256), 0.05)
    gate = np.array([64, 136], dtype=np.int64)
    f.update(rms_x=bits(x), rms_nw=nw, rms_w=bits(w), rms_gate=gate,
             rms_eps=np.array([1e-6], np.float32),
             rms_rstd=ref.rms_rstd(x, 1e-6).astype(np.float32),
             rms_out=bits(ref.rmsnorm_gate_projection(x, nw, 1e-6, w, tuple(gate))))
    # Residual epilogue.
    h, w, r = bf(rng, (72, 160)), bf(rng, (136, 160), 0.05), bf(rng, (72, 136))
    f.update(res_h=bits(h), res_w=bits(w), res_r=bits(r),
             res_out=bits(ref.residual_projection(h, w, r)))
    # FP32 weight-gradient accumulation G += f32(r(a @ b)) and without rounding.
    gbuf = (rng.standard_normal((48, 80)) * 1e-2).astype(np.float32)
    a, b = bf(rng, (48, 100)), bf(rng, (100, 80))
    f.update(acc_g=gbuf, acc_a=bits(a), acc_b=bits(b),
             acc_round=ref.accumulate(gbuf, a, b, True),
             acc_direct=ref.accumulate(gbuf, a, b, False))
    # LM head cross-entropy: hidden [64, 128], tied weight [vocab 300, 128], 7 ignored.
    hid, emb = bf(rng, (64, 128)), bf(rng, (300, 128), 0.05)
    tg = rng.integers(0, 300, 64).astype(np.int64)
    tg[rng.permutation(64)[:7]] = -100
    loss, mean, count, dh = ref.linear_cross_entropy(hid, emb, tg)
    f.update(ce_hidden=bits(hid), ce_weight=bits(emb), ce_targets=tg,
             ce_loss=loss.astype(np.float32), ce_mean=np.array([mean], np.float64),
             ce_count=np.array([count], np.int64), ce_dhidden=bits(dh))
    np.savez_compressed(OUT, **f)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(f)} arrays)")


if __name__ == "__main__":
    main()
