"""Dense GEMMs of the decoder: PyTorch (hipBLASLt) with a split-K form for
the two whose output goes straight into a residual add + RMSNorm (o_proj and
down_proj, reference src/compute/models/qwen3.py:64,115 feeding the norms of
:150,:152), and, opt-in for decode batches of at most 64 rows of a model with
packed weights, the weight-streaming gfx950 kernel (xv_dense_gemm) over
packed weight tiles: gate_up fused with SiLU-and-mul, down and o as split-K
partials for the same norm (dense_gemm and the streamed_* helpers at the end
of this file; measured 11-27 % faster than the hipBLASLt forms below at M 8
and 64, weights streamed from HBM).  The split-K measurements below are the
hipBLASLt path, the default.

At decode batch sizes an [M, K] x [K, 4096] GEMM has few output tiles for 256
CUs: hipBLASLt runs Qwen3-8B's o_proj (K 4096) and down_proj (K 12288) at
1.4-2.7 TB/s between M 32 and 256.  Cut along K into P slices, the same
weights run as a batched GEMM with P times the tiles (one bmm over strided
views, no copies), each slice's fp32 product kept apart; the norm kernel
that consumes them sums the P partials, rounds to bf16 (the value the
unsplit GEMM would have written) and continues as fused_add_rmsnorm.  The
partials cost P x M x N x 4 bytes of extra reads in the norm, which the
table below charges against the GEMM's gain.

The split per shape and batch size is SPLIT_TABLE, measured for the Qwen3-8B
and Qwen3-32B weights; the first measurements, which set split_rule for other
shapes (MI355X, graph replay, more than 1 GB of weights cycled so that none is
served from the 256 MB last-level cache; us, unsplit -> split):

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

import bisect
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


# The fastest K split per decode graph bucket (SPLIT_BUCKETS) for the o_proj
# and down_proj weights of Qwen3-8B ([4096, 4096], [4096, 12288]) and
# Qwen3-32B ([5120, 8192], [5120, 25600]), measured on MI355X by
# `python -m xvllm.layers.split_tune` (the GEMM plus the norm that sums its
# partials, graph replay, weights cycled past the last-level cache).
# hipBLASLt's kernel choice makes the best split jump between neighbouring
# sizes, so the table is taken as measured.  At Qwen3-32B's M 32 it runs
# o_proj unsplit (27.6 us against 54.2 at P 4) and down_proj at P 2 (80.1
# against 89.1 us).  Other shapes use split_rule.
SPLIT_BUCKETS = (1, 2, 4, 8, 16, 32, 48, 64, 80, 96, 112, 128, 144, 160, 176, 192, 208, 224, 240, 256)
SPLIT_TABLE = {
    (4096, 4096): (4, 4, 4, 4, 4, 1, 1, 2, 2, 2, 2, 2, 2, 4, 2, 4, 2, 4, 2, 4),
    (4096, 12288): (1, 1, 1, 1, 1, 4, 4, 4, 4, 4, 8, 8, 8, 8, 8, 8, 8, 8, 8, 8),
    (5120, 8192): (1, 1, 1, 1, 1, 1, 8, 8, 1, 2, 4, 2, 2, 8, 2, 8, 4, 8, 4, 8),
    (5120, 25600): (2, 2, 2, 2, 2, 2, 8, 8, 8, 4, 8, 8, 8, 8, 8, 8, 4, 8, 8, 8),
}


def split_rule(m: int, n: int, k: int) -> int:
    """K slices for a shape outside SPLIT_TABLE (the Qwen3-8B measurements
    above, generalised by K)."""
    if n > 8192 or k % (8 * 64):
        return 1
    if k >= 8192:
        return 4 if 32 <= m < 96 else 8 if 96 <= m <= 256 else 1
    if k >= 4096:
        return 4 if m <= 16 else 8 if 96 <= m <= 192 else 1
    return 1


def split_factor(m: int, n: int, k: int) -> int:
    """K slices for an [m, k] x [k, n] GEMM feeding a norm (1: no split):
    SPLIT_TABLE's entry for the smallest bucket of at least m rows, else
    split_rule; above 256 rows, 1."""
    if m < 1 or m > SPLIT_BUCKETS[-1]:
        return 1
    row = SPLIT_TABLE.get((n, k))
    if row is None:
        return split_rule(m, n, k)
    return row[bisect.bisect_left(SPLIT_BUCKETS, m)]


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


# Output forms of xv_dense_gemm (csrc/dense_gemm.hip).
GEMM_BF16, GEMM_PARTS, GEMM_SILU_MUL = 0, 1, 2


class PackedWeight(NamedTuple):
    """A [N, K] weight in the tile order the decode GEMM kernel streams:
    16-row x 64-column tiles of 2 KB, each in the kernel's lane order (see
    pack_weight), row blocks outermost."""

    data: torch.Tensor  # bf16, N * K elements
    n: int
    k: int


def pack_weight(w: torch.Tensor) -> PackedWeight:
    """Pack w [N, K] (N % 16 == 0, K % 64 == 0) for dense_gemm: tile (nb, sg)
    holds, for lane l = 16 g + r (r < 16, g < 4), w[16 nb + r, 64 sg + 8 g + e]
    at 8 l + e and w[16 nb + r, 64 sg + 32 + 8 g + e] at 512 + 8 l + e."""
    n, k = w.shape
    if n % 16 or k % 64:
        raise ValueError(f"pack_weight: [{n}, {k}] is not a whole number of 16 x 64 tiles")
    t = w.reshape(n // 16, 16, k // 64, 2, 4, 8)  # [nb, r, sg, half, g, e]
    return PackedWeight(t.permute(0, 2, 3, 4, 1, 5).contiguous().view(-1), n, k)


def dense_gemm(x: torch.Tensor, w: PackedWeight, mode: int = GEMM_BF16, *, col_tiles: int = 4, waves: int = 4,
               parts: int = 1):
    """x [M, K] @ w^T on the weight-streaming gfx950 kernel (M <= 64), w packed
    by pack_weight.

    mode GEMM_BF16: bf16 [M, N].  GEMM_PARTS: PartialSums of a K split over
    `parts` ([P, M, N] fp32).  GEMM_SILU_MUL: w is the gate/up weight [2I, K]
    (gate rows first) and the result is bf16 silu(x w_gate^T) * (x w_up^T),
    [M, I], the two products rounded to bf16 first as the unfused GEMM stores
    them.  col_tiles x 16 weight rows per wave (1, 2 or 4; even for
    GEMM_SILU_MUL), `waves` (4 or 8) waves per workgroup over the same K.
    Raises on shapes or layouts the kernel does not take."""
    from .. import _C
    from .._torch_glue import ptr, require_bf16, require_cuda, stream_of

    require_cuda(x)
    require_bf16(x)
    require_bf16(w.data)
    m, k = x.shape
    n = w.n
    if x.stride(1) != 1:
        raise ValueError("dense_gemm: x needs unit stride along K")
    if w.k != k:
        raise ValueError(f"dense_gemm: x {tuple(x.shape)} and w [{w.n}, {w.k}] disagree on K")
    if w.data.numel() != w.n * w.k or not w.data.is_contiguous() or w.n % 16 or w.k % 64:
        raise ValueError(f"dense_gemm: packed weight holds {w.data.numel()} elements "
                         f"(contiguous: {w.data.is_contiguous()}), not whole 16 x 64 tiles of [{w.n}, {w.k}]")
    if mode == GEMM_PARTS:
        out = torch.empty((parts, m, n), dtype=torch.float32, device=x.device)
        os_, ps = n, m * n
    else:
        out = torch.empty((m, n // 2 if mode == GEMM_SILU_MUL else n), dtype=torch.bfloat16, device=x.device)
        os_, ps = out.shape[1], 0
    _C.check(
        _C.lib().xv_dense_gemm(ptr(x), x.stride(0), ptr(w.data), ptr(out), os_, ps, m, n, k, mode, col_tiles, waves,
                               parts, stream_of(x)),
        "xv_dense_gemm",
    )
    return PartialSums(out) if mode == GEMM_PARTS else out


# Batches of up to this many rows take the weight-streaming kernel when the
# model holds packed weights (pack_decode_weights): decode batches, and also
# prefill chunks this short (the same products); larger batches stay on
# hipBLASLt over the [N, K] weights.
STREAM_MAX_ROWS = 64


def stream_parts(k: int) -> int:
    """K slices of a split-K streamed GEMM (the most of 8, 4, 2, 1 that cut K
    into whole 4-step rounds)."""
    for p in (8, 4, 2, 1):
        if k % (p * 256) == 0:
            return p
    return 0


def streamable(w: torch.Tensor, mode: int) -> bool:
    """Whether w [N, K] fits the shapes the streamed decode GEMMs use:
    gate/up + SiLU with 2 tiles x 4 waves (2I % 128), split-K partials with
    1 tile x 8 waves (N % 128)."""
    n, k = w.shape
    if mode == GEMM_SILU_MUL:
        return n % 128 == 0 and k % 256 == 0
    return n % 128 == 0 and stream_parts(k) > 0


def stream_rows(x: torch.Tensor) -> bool:
    """Whether activations x [M, K] can take a streamed decode GEMM: at most
    STREAM_MAX_ROWS rows, unit stride along K, 16-byte aligned rows (other
    layouts stay on hipBLASLt)."""
    return (0 < x.shape[0] <= STREAM_MAX_ROWS and x.stride(1) == 1 and x.stride(0) % 8 == 0
            and x.data_ptr() % 16 == 0)


def streamed_silu_mul(x: torch.Tensor, w: PackedWeight) -> torch.Tensor:
    """silu(x w_gate^T) * (x w_up^T) of a decode batch, bf16 [M, I]."""
    return dense_gemm(x, w, GEMM_SILU_MUL, col_tiles=2, waves=4)


def streamed_into_norm(x: torch.Tensor, w: PackedWeight) -> PartialSums:
    """x @ w^T of a decode batch as split-K PartialSums for the next residual
    add + RMSNorm, K cut P = 8 ways where it allows; up to 32 rows, K slices
    under 1024 elements are halved instead (measured: Qwen3-8B o_proj at
    M 8, P 4 7.3 us against P 8 7.8; down_proj P 8 at every M)."""
    p = stream_parts(w.k)
    if x.shape[0] <= 32 and w.k // p < 1024 and p > 1:
        p //= 2
    return dense_gemm(x, w, GEMM_PARTS, col_tiles=1, waves=8, parts=p)
