"""SiluAndMul module (reference ``activation.py:6-8``)."""
from __future__ import annotations

import torch
from torch import nn

from . import ops  # noqa: F401


class SiluAndMul(nn.Module):
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return torch.ops.vllm.silu_and_mul(x)
