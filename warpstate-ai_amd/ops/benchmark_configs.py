"""Seeded synthetic inputs of the hot-path benchmark configurations (CPU tensors).

Every tensor is drawn from ``torch.Generator('cpu').manual_seed(seed)`` in FP32 ``randn``,
in the order listed, scaled, then cast to BF16, so CPU and GPU runs see identical inputs.
Weights use nn.Linear / nn.Embedding layouts ([out, in]). Sizes default to the benchmark
shapes and shrink for tests through the keyword arguments.

1. SwiGLU gate/up: X [4096, 1024] ~ N(0,1); W_gate, W_up [2816, 1024] ~ N(0, 0.02), packed
   as [W_up; W_gate] (up columns first, warpstate/model.py:59).
2. RMSNorm-prologue projection: X [16384, 2048] ~ N(0,1); norm weight 1 + N(0, 0.1) FP32;
   eps 1e-6; W [9216, 2048] ~ N(0, 0.02) = Q, K, V (3 x 16 heads x 128), gate [6144, 8192),
   memory-write [8192, 9216).
3. Down + residual: A, B [16384, 5632] ~ N(0,1), H = r(silu(A) * B); W_down [2048, 5632]
   ~ N(0, 0.02); R [16384, 2048] ~ N(0,1).
4. MLP backward (d 2048, ffn 5632): X [16384, 2048] ~ N(0,1); W_up, W_gate [5632, 2048]
   ~ N(0, 0.02) packed [11264, 2048]; W_down [2048, 5632] ~ N(0, 0.02); dY [16384, 2048]
   ~ N(0, 1e-2); G_down [2048, 5632], G_upgate [11264, 2048] FP32 ~ N(0, 1e-4).
5. LM head: hidden [16384, 2048] ~ N(0,1); W [32768, 2048] ~ N(0, 0.02); targets uniform in
   [0, 32768) int64, then round(0.05 M) positions of a permutation set to -100.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def _normal(gen, shape, std=1.0, mean=0.0):
    return torch.randn(shape, generator=gen, dtype=torch.float32) * std + mean


def _bf16(t):
    return t.to(torch.bfloat16)


def swiglu_forward_inputs(m=4096, d=1024, h=2816, seed=0):
    gen = torch.Generator("cpu").manual_seed(seed)
    x = _bf16(_normal(gen, (m, d)))
    w_gate = _bf16(_normal(gen, (h, d), 0.02))
    w_up = _bf16(_normal(gen, (h, d), 0.02))
    return {"x": x, "w_upgate": torch.cat([w_up, w_gate], dim=0).contiguous()}


def rms_projection_inputs(m=16384, d=2048, n=9216, gate=(6144, 8192), seed=0):
    gen = torch.Generator("cpu").manual_seed(seed)
    x = _bf16(_normal(gen, (m, d)))
    norm_weight = _normal(gen, (d,), 0.1, 1.0)
    w = _bf16(_normal(gen, (n, d), 0.02))
    return {"x": x, "norm_weight": norm_weight, "eps": 1e-6, "w": w, "gate": gate}


def down_residual_inputs(m=16384, ffn=5632, d=2048, seed=0):
    gen = torch.Generator("cpu").manual_seed(seed)
    a = _bf16(_normal(gen, (m, ffn)))
    b = _bf16(_normal(gen, (m, ffn)))
    h = F.silu(a) * b
    del a, b
    w_down = _bf16(_normal(gen, (d, ffn), 0.02))
    residual = _bf16(_normal(gen, (m, d)))
    return {"h": h, "w_down": w_down, "residual": residual}


def mlp_backward_inputs(m=16384, d=2048, ffn=5632, seed=0):
    """Raw inputs; the saved packed projection r(X W_upgate^T) and activation are derived
    by the caller (they are forward outputs)."""
    gen = torch.Generator("cpu").manual_seed(seed)
    x = _bf16(_normal(gen, (m, d)))
    w_up = _bf16(_normal(gen, (ffn, d), 0.02))
    w_gate = _bf16(_normal(gen, (ffn, d), 0.02))
    w_down = _bf16(_normal(gen, (d, ffn), 0.02))
    dy = _bf16(_normal(gen, (m, d), 1e-2))
    g_down = _normal(gen, (d, ffn), 1e-4)
    g_upgate = _normal(gen, (2 * ffn, d), 1e-4)
    return {"x": x, "w_upgate": torch.cat([w_up, w_gate], dim=0).contiguous(),
            "w_down": w_down, "dy": dy, "g_down": g_down, "g_upgate": g_upgate}


def lm_head_inputs(m=16384, d=2048, vocab=32768, ignore_fraction=0.05, seed=0):
    gen = torch.Generator("cpu").manual_seed(seed)
    hidden = _bf16(_normal(gen, (m, d)))
    weight = _bf16(_normal(gen, (vocab, d), 0.02))
    targets = torch.randint(0, vocab, (m,), generator=gen, dtype=torch.int64)
    ignored = torch.randperm(m, generator=gen)[:round(ignore_fraction * m)]
    targets[ignored] = -100
    return {"hidden": hidden, "weight": weight, "targets": targets}


# Algorithmic FLOPs per configuration at its benchmark shape (2 M N K per GEMM; the
# LM head counts logits forward and dHidden, not the recomputed logits).
def flops_swiglu_forward(m, d, h):
    return 2 * m * d * 2 * h


def flops_rms_projection(m, d, n):
    return 2 * m * d * n


def flops_down_residual(m, ffn, d):
    return 2 * m * ffn * d


def flops_mlp_backward(m, d, ffn):
    return 2 * m * d * ffn + 2 * m * 2 * ffn * d + 2 * d * ffn * m + 2 * 2 * ffn * d * m


def flops_lm_head(m, d, vocab):
    return 4 * m * d * vocab
