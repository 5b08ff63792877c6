"""Module types of the hot path and a small LM built from them (see package docstring).

RMSNorm, SwiGLU, the residual adds and the chunked tied-head loss follow the numerics of
warpstate/model.py:15-28, :52-60, :177-178 and :316-334; the token mixer between
``in_proj`` and ``out_proj`` is a placeholder.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.utils.checkpoint import checkpoint

from .config import WarpStateConfig


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-5):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # FP32 statistics, BF16-rounded normalized value times the cast weight.
        wide = x.float()
        wide = wide * torch.rsqrt(wide.pow(2).mean(dim=-1, keepdim=True) + self.eps)
        return wide.to(x.dtype) * self.weight.to(x.dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """Interleaved rotary pairing (warpstate/model.py:31-34): lane pair (2i, 2i+1) maps
    (a, b) to (-b, a)."""
    pairs = x.unflatten(-1, (-1, 2))
    return torch.stack((-pairs[..., 1], pairs[..., 0]), dim=-1).flatten(-2)


def rope_cos_sin(length: int, dim: int, device: torch.device, dtype: torch.dtype
                 ) -> tuple[torch.Tensor, torch.Tensor]:
    """[length, dim] rotary tables with each frequency repeated for its lane pair
    (warpstate/model.py:37-42): angle(t, 2i) = angle(t, 2i+1) = t / 10000^(2i/dim)."""
    positions = torch.arange(length, device=device, dtype=torch.float32)
    exponents = torch.arange(0, dim, 2, device=device, dtype=torch.float32) / dim
    angles = positions[:, None] * (1.0 / (10000 ** exponents))[None, :]
    angles = angles.repeat_interleave(2, dim=-1)
    return angles.cos().to(dtype), angles.sin().to(dtype)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [B, N, H, C, D] with [C, D] tables (warpstate/model.py:45-49)."""
    return x * cos + rotate_half(x) * sin


class SwiGLU(nn.Module):
    """Packed projection: up in output columns [0, hidden), gate in [hidden, 2 hidden)."""

    def __init__(self, dim: int, hidden: int):
        super().__init__()
        self.up_gate = nn.Linear(dim, hidden * 2, bias=False)
        self.down = nn.Linear(hidden, dim, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        up, gate = self.up_gate(x).chunk(2, dim=-1)
        return self.down(F.silu(gate) * up)


class WarpStateCore(nn.Module):
    """One core: norm1 -> in_proj -> (q, k, v, sigmoid(g), u) -> token mixer -> out_proj
    with a residual add, then norm2 -> SwiGLU with a residual add
    (warpstate/model.py:93-96, :107-112, :120-121, :174-178).

    ``project`` and ``mix`` are the two halves of the token path: the fused-execution
    adapter replaces ``project`` (RMSNorm prologue, projection and gate sigmoid in one
    GEMM launch) and keeps ``mix``.
    """

    def __init__(self, cfg: WarpStateConfig):
        super().__init__()
        d = cfg.d_model
        self.norm1 = RMSNorm(d, cfg.rms_eps)
        self.in_proj = nn.Linear(d, 5 * d, bias=False)
        self.out_proj = nn.Linear(d, d, bias=False)
        self.norm2 = RMSNorm(d, cfg.rms_eps)
        self.ffn = SwiGLU(d, cfg.ffn_hidden)

    def project(self, x: torch.Tensor) -> tuple[torch.Tensor, ...]:
        """(q, k, v, sigmoid(g), u): the five d-wide slices of in_proj(norm1(x)), the fourth
        through the gate sigmoid."""
        q, k, v, g, u = self.in_proj(self.norm1(x)).chunk(5, dim=-1)
        return q, k, v, torch.sigmoid(g), u

    def mix(self, q, k, v, gate, u) -> torch.Tensor:
        """Placeholder token mixer (gate-weighted blend of v and a tanh of the other
        slices) standing in for the reference's chunked attention and memory."""
        return gate * v + (1 - gate) * torch.tanh(q * k + u)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x + self.out_proj(self.mix(*self.project(x)))
        return x + self.ffn(self.norm2(x))


class WarpStateLM(nn.Module):
    def __init__(self, cfg: WarpStateConfig):
        super().__init__()
        cfg.validate()
        self.cfg = cfg
        self.embed = nn.Embedding(cfg.vocab_size, cfg.d_model)
        self.cores = nn.ModuleList([WarpStateCore(cfg) for _ in range(cfg.n_cores)])
        self.depth_scale = nn.Parameter(torch.zeros(cfg.logical_depth, cfg.d_model))
        self.depth_bias = nn.Parameter(torch.zeros(cfg.logical_depth, cfg.d_model))
        self.final_norm = RMSNorm(cfg.d_model, cfg.rms_eps)
        for module in self.modules():
            if isinstance(module, (nn.Linear, nn.Embedding)):
                nn.init.normal_(module.weight, mean=0.0, std=0.02)

    def features(self, input_ids: torch.Tensor) -> torch.Tensor:
        """Embedding, the depth loop over the shared cores and the final norm
        (warpstate/model.py:303-313)."""
        x = self.embed(input_ids)
        for depth in range(self.cfg.logical_depth):
            x = x * (1.0 + self.depth_scale[depth]) + self.depth_bias[depth]
            core = self.cores[depth % self.cfg.n_cores]
            if self.training and self.cfg.gradient_checkpointing:
                x = checkpoint(core, x, use_reentrant=False)
            else:
                x = core(x)
        return self.final_norm(x)

    def chunked_loss(self, x: torch.Tensor, targets: torch.Tensor) -> torch.Tensor:
        """Mean cross-entropy of the tied head over valid targets, one loss_chunk_size row
        block of FP32 logits at a time (warpstate/model.py:314-334)."""
        hidden = x.reshape(-1, x.size(-1))
        labels = targets.reshape(-1)
        loss = x.new_zeros((), dtype=torch.float32)
        step = self.cfg.loss_chunk_size
        for start in range(0, labels.numel(), step):
            logits = F.linear(hidden[start:start + step], self.embed.weight).float()
            loss = loss + F.cross_entropy(logits, labels[start:start + step], reduction="sum")
        return loss / labels.ne(-100).sum().clamp_min(1)

    def forward(self, input_ids, targets=None, *, return_logits=True):
        x = self.features(input_ids)
        if targets is not None and not return_logits:
            return None, self.chunked_loss(x, targets)
        logits = F.linear(x, self.embed.weight)
        if targets is None:
            return logits
        return logits, F.cross_entropy(logits.reshape(-1, logits.size(-1)), targets.reshape(-1))
