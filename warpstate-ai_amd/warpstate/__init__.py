"""Minimal model shim: the module types the hot path patches and composes.

This is not WarpState's model. It keeps the names the hot-path modules look up
(``warpstate.model.RMSNorm`` / ``SwiGLU``, ``model.cores`` with ``in_proj``, ``out_proj``,
``norm1``, ``norm2``, ``ffn``) so plan application and activation patching can be exercised
end to end; its token mixer is a gated elementwise placeholder for the reference's
chunked attention and recurrent memory, which are outside this hot path.
"""
from .config import WarpStateConfig
from .model import WarpStateLM

__all__ = ["WarpStateConfig", "WarpStateLM"]
