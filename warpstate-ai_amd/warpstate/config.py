"""Model hyperparameters with the field names of warpstate/config.py:9-21."""
from __future__ import annotations

from dataclasses import dataclass


@dataclass
class WarpStateConfig:
    vocab_size: int = 32768
    d_model: int = 1280
    n_heads: int = 20
    n_cores: int = 4
    logical_depth: int = 16
    ffn_hidden: int = 4480
    chunk_size: int = 128
    dropout: float = 0.0
    rms_eps: float = 1e-5
    gradient_checkpointing: bool = True
    parallel_memory: bool = False
    loss_chunk_size: int = 128

    def validate(self) -> None:
        if self.d_model % self.n_heads or self.logical_depth < self.n_cores:
            raise ValueError("invalid WarpState configuration")
        if self.chunk_size <= 0 or self.n_cores <= 0 or self.loss_chunk_size <= 0:
            raise ValueError("invalid WarpState configuration")

    @property
    def head_dim(self) -> int:
        return self.d_model // self.n_heads
