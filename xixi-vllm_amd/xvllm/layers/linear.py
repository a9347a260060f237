"""Dense GEMMs of the decoder on PyTorch (hipBLASLt), and a split-K form for
the two whose output goes straight into a residual add + RMSNorm (o_proj and
down_proj, reference src/compute/models/qwen3.py:64,115 feeding the norms of
:150,:152).

At decode batch sizes an [M, K] x [K, 4096] GEMM has few output tiles for 256
CUs: hipBLASLt runs Qwen3-8B's o_proj (K 4096) and down_proj (K 12288) at
1.4-2.7 TB/s between M 32 and 256.  Cut along K into P slices, the same
weights run as a batched GEMM with P times the tiles (one bmm over strided
views, no copies), each slice's fp32 product kept apart; the norm kernel
that consumes them sums the P partials, rounds to bf16 (the value the
unsplit GEMM would have written) and continues as fused_add_rmsnorm.  The
partials cost P x M x N x 4 bytes of extra reads in the norm, which the
table below charges against the GEMM's gain.

Measured on MI355X, graph replay, more than 1 GB of weights cycled so that
none is served from the 256 MB last-level cache (us; unsplit -> split):

    down_proj  M 32: 28.2 -> 22.6 (P 4)   M 64: 37.5 -> 25.0 (P 4)
               M 128: 66.2 -> 27.3 (P 8)  M 256: 54.4 -> 36.0 (P 8)
               M 1, 8: no gain
    o_proj     M 1, 8: 15.3 -> 10.1 (P 4)  M 128: 24.2 -> 15.6 (P 8)
               M 32, 64, 256: gains below the partials' extra reads

The other two GEMMs stay unsplit (same measurement, bmm over the same views):
gate_up (K 4096, N 24576) M 32-128: 45-51 unsplit, no split faster; M 256:
65.5 -> 59.6 (P 2), less than its 50 MB of fp32 partials cost to write and
read back.  qkv (N 6144) M 64: 17.5 -> 15.4 (P 4), M 128: 25.0 -> 17.7,
M 256: 39.3 -> 23.1; its consumer is the fused q/k-norm + RoPE + KV-store
kernel, which would need a partial-summing form for gains of a few us per
layer at the largest serving batches.
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
    if n > 8192 or k % (8 * 64):
        return 1
    if k >= 8192:
        return 4 if 32 <= m < 96 else 8 if 96 <= m <= 256 else 1
    if k >= 4096:
        return 4 if m <= 16 else 8 if 96 <= m <= 192 else 1
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
