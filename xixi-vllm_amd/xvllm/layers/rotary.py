"""Rotary embedding module and its fp32 cos||sin table
(reference ``rotary.py:7-62``)."""
from __future__ import annotations

import torch
from torch import nn

from . import ops  # noqa: F401


def build_cos_sin_cache(head_dim: int, max_position_embeddings: int, rope_theta: float) -> torch.Tensor:
    """[max_pos, head_dim] fp32 table: cos of the NeoX half-split angles in the
    first head_dim/2 columns, sin in the rest.  inv_freq_i = theta^(-2i/D),
    angle = pos * inv_freq_i, all in fp32 in that order (rotary.py:13-20)."""
    exponent = torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim
    inv_freq = 1.0 / (rope_theta ** exponent)
    pos = torch.arange(max_position_embeddings, dtype=torch.float)
    ang = pos[:, None] * inv_freq[None, :]
    return torch.cat((ang.cos(), ang.sin()), dim=-1)


class RotaryEmbedding(nn.Module):
    def __init__(self, head_dim: int, rotary_dim: int, max_position_embeddings: int, rope_theta: float) -> None:
        super().__init__()
        self.head_dim = head_dim
        assert rotary_dim == head_dim, "rotary_dim must equal head_dim (full rotation)"
        self.register_buffer(
            "cos_sin_cache", build_cos_sin_cache(head_dim, max_position_embeddings, rope_theta), persistent=False
        )

    def _apply(self, fn, recurse: bool = True):
        out = super()._apply(fn, recurse)
        if self.cos_sin_cache.dtype != torch.float32:  # the kernel reads an fp32 table
            self.cos_sin_cache = self.cos_sin_cache.to(torch.float32)
        return out

    def forward(self, positions: torch.Tensor, query: torch.Tensor, key: torch.Tensor):
        return torch.ops.vllm.rotary_embedding(query, key, positions, self.cos_sin_cache, self.head_dim)
