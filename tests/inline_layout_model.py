"""A test-side language model in the layout of the reference's ``WarpStateCore`` and
``WarpStateLM`` (warpstate/model.py:114-178, :302-334): each core is one ``forward`` with
``_split`` around ``in_proj``, the gate sigmoid and both residual adds inline, and the
chunked tied-head loss inline in the LM's forward. It has none of the ``project`` /
``mix`` / ``chunked_loss`` seams of the package's stand-in model, so it shows what the
fused adapter can attach to without them. The token mixer between ``_split`` and
``out_proj`` is a placeholder for the reference's chunked attention and memory (it is
not on the GEMM hot path).
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.utils.checkpoint import checkpoint

from warpstate.config import WarpStateConfig
from warpstate.model import RMSNorm, SwiGLU


class InlineCore(nn.Module):
    def __init__(self, cfg: WarpStateConfig):
        super().__init__()
        d = cfg.d_model
        self.heads = cfg.n_heads
        self.norm1 = RMSNorm(d, cfg.rms_eps)
        self.in_proj = nn.Linear(d, 5 * d, bias=False)
        self.out_proj = nn.Linear(d, d, bias=False)
        self.norm2 = RMSNorm(d, cfg.rms_eps)
        self.ffn = SwiGLU(d, cfg.ffn_hidden)

    def _split(self, z: torch.Tensor) -> tuple[torch.Tensor, ...]:
        b, t, _ = z.shape
        return tuple(part.view(b, t, self.heads, -1) for part in self.in_proj(z).chunk(5, dim=-1))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        b, t, d = x.shape
        z = self.norm1(x)
        q, k, v, g, u = self._split(z)
        gate = torch.sigmoid(g)
        y = (gate * v + (1 - gate) * torch.tanh(q * k + u)).reshape(b, t, d)
        x = x + self.out_proj(y)
        x = x + self.ffn(self.norm2(x))
        return x


class InlineLM(nn.Module):
    def __init__(self, cfg: WarpStateConfig):
        super().__init__()
        cfg.validate()
        self.cfg = cfg
        self.embed = nn.Embedding(cfg.vocab_size, cfg.d_model)
        self.cores = nn.ModuleList([InlineCore(cfg) for _ in range(cfg.n_cores)])
        self.depth_scale = nn.Parameter(torch.zeros(cfg.logical_depth, cfg.d_model))
        self.depth_bias = nn.Parameter(torch.zeros(cfg.logical_depth, cfg.d_model))
        self.final_norm = RMSNorm(cfg.d_model, cfg.rms_eps)
        for module in self.modules():
            if isinstance(module, (nn.Linear, nn.Embedding)):
                nn.init.normal_(module.weight, mean=0.0, std=0.02)

    def forward(self, input_ids, targets=None, *, return_logits=True):
        x = self.embed(input_ids)
        for depth in range(self.cfg.logical_depth):
            x = x * (1.0 + self.depth_scale[depth]) + self.depth_bias[depth]
            core = self.cores[depth % self.cfg.n_cores]
            if self.training and self.cfg.gradient_checkpointing:
                x = checkpoint(core, x, use_reentrant=False)
            else:
                x = core(x)
        x = self.final_norm(x)
        if targets is not None and not return_logits:
            hidden = x.reshape(-1, x.size(-1))
            labels = targets.reshape(-1)

            def chunk_loss(h, w, y):
                return F.cross_entropy(F.linear(h, w).float(), y, reduction="sum")

            loss = x.new_zeros((), dtype=torch.float32)
            step = self.cfg.loss_chunk_size
            for start in range(0, labels.numel(), step):
                args = (hidden[start:start + step], self.embed.weight, labels[start:start + step])
                if self.training and torch.is_grad_enabled():
                    loss = loss + checkpoint(chunk_loss, *args, use_reentrant=False)
                else:
                    loss = loss + chunk_loss(*args)
            return None, loss / labels.ne(-100).sum().clamp_min(1)
        logits = F.linear(x, self.embed.weight)
        if targets is None:
            return logits
        return logits, F.cross_entropy(logits.reshape(-1, logits.size(-1)), targets.reshape(-1))
