"""Dense GEMMs of the decoder on PyTorch (hipBLASLt), and a split-K form for
the two whose output goes straight into a residual add + RMSNorm (o_proj and
down_proj, reference src/compute/models/qwen3.py:64,115 feeding the norms of
:150,:152).

At decode batch sizes an [M, K] x [K, 4096] GEMM has few output tiles for 256
CUs: hipBLASLt runs o_proj (K 4096) and down_proj (K 12288) of Qwen3-8B at
M 64 at 1.8-2.8 TB/s.  Cut along K into P slices, the same weights run as a
batched GEMM of P times the tiles (one bmm over strided views, no copies),
each slice's fp32 product kept apart; the norm kernel that consumes them sums
the P partials, rounds to bf16 (the value the unsplit GEMM would have
written) and continues as fused_add_rmsnorm.  The partials cost P x M x N x 4
extra bytes of reads in the norm, small next to the weights at these M.

Measured on MI355X, graph replay, weights streaming from HBM (us):

    M 64:  o_proj 12.1 -> 9.6 (P 4), down_proj 36.8 -> 23.6 (P 4)
    M 128: o_proj 19.2 -> 12.3 (P 4), down_proj 66.1 -> 30.2 (P 4)
    M 256: o_proj 18.9 -> 17.0 (P 4, not worth the partial reads),
           down_proj 55.1 -> 44.1 (P 4)
    M 8:   o_proj 11.8 -> 8.4 (P 4), down_proj 20.7 -> 21.2 (P 4: no gain)
"""
from __future__ import annotations

from typing import NamedTuple

import torch
import torch.nn.functional as F


class PartialSums(NamedTuple):
    """fp32 partial products [P, M, N] of one split-K GEMM; their sum is the
    GEMM's output."""

    parts: torch.Tensor

    def materialize(self) -> torch.Tensor:
        """The bf16 [M, N] output of the unsplit GEMM (for callers outside
        the decoder's norm chain)."""
        return self.parts.sum(0).to(torch.bfloat16)


def split_factor(m: int, n: int, k: int) -> int:
    """K slices for an [m, k] x [k, n] GEMM feeding a norm (1: no split)."""
    if n > 8192 or k % (4 * 64):
        return 1
    if k >= 8192:
        return 4 if 16 <= m <= 256 else 1
    if k >= 4096:
        return 4 if m <= 128 else 1
    return 1


def linear_into_norm(x: torch.Tensor, w: torch.Tensor, split: bool = True):
    """x [M, K] @ w[N, K]^T for a consumer that accepts PartialSums (the
    residual add + RMSNorm of the next norm): the split-K partials when
    split_factor picks a split, else the plain bf16 product."""
    m, k = x.shape
    n = w.shape[0]
    p = split_factor(m, n, k) if split else 1
    if p == 1 or x.stride(1) != 1 or w.stride(1) != 1:
        return F.linear(x, w)
    xs, ws = split_k_views(x, w, p)
    return PartialSums(torch.bmm(xs, ws, out_dtype=torch.float32))


def split_k_views(x: torch.Tensor, w: torch.Tensor, p: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Slice p of x [M, K] and of w [N, K] along K as batched-GEMM operands,
    views only: x -> [P, M, K/P], w -> [P, K/P, N] (w^T's slices)."""
    m, k = x.shape
    n = w.shape[0]
    return x.view(m, p, k // p).transpose(0, 1), w.view(n, p, k // p).permute(1, 2, 0)
