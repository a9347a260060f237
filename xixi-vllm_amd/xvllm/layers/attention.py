"""``vllm::attention`` custom op (reference ``src/compute/layers/attention.py:13-143``):
stores this step's K/V at ``slot_mapping`` (kv_ops.store_kvcache), then runs
paged GQA decode attention or varlen causal prefill attention, both as gfx950
HIP kernels.  Same signature, same module-global ``attention_context`` pool
handle, same ``AttnInputs`` record.
"""
from __future__ import annotations

import math
from contextlib import contextmanager
from dataclasses import dataclass
from typing import NamedTuple, Optional

import torch
import torch.nn as nn

from .. import _C
from .._torch_glue import aligned16, ptr, require_bf16, require_cuda, stream_of
from ..kv_ops import store_kvcache


@dataclass
class CascadePlan:
    """Shared-prefix groups of a decode batch (device int32 tensors): row b's
    first prefix_tokens[b] tokens are its group's shared blocks; group g's
    record group_info[g] is (first index into group_rows, rows, first batch
    row, prefix tokens).  num_groups and max_prefix_blocks fix the prefix
    pass's grid (empty groups allowed)."""
    prefix_tokens: torch.Tensor
    group_info: torch.Tensor
    group_rows: torch.Tensor
    num_groups: int
    max_prefix_blocks: int


class AttnInputs(NamedTuple):
    slot_mapping: torch.Tensor
    is_prefill: bool
    cu_seqlens_q: Optional[torch.Tensor] = None
    cu_seqlens_k: Optional[torch.Tensor] = None
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    block_tables: Optional[torch.Tensor] = None
    cache_seqlens: Optional[torch.Tensor] = None
    cascade: Optional[CascadePlan] = None  # decode only: shared-prefix groups (no reference counterpart)


@dataclass
class AttnMetadata:
    kv_cache: torch.Tensor  # [2, L, NB, BS, Hkv, D]
    # fp8 (e4m3fn) pools only: the dequantisation scales of K and V (this
    # build's optional pool format; the reference's pool holds the model dtype)
    k_scale: float = 1.0
    v_scale: float = 1.0


# Active metadata, innermost context last (the reference keeps one module
# global, attention.py:29-40; a stack gives the same nesting behaviour).
_META_STACK: list[AttnMetadata] = []


@contextmanager
def attention_context(meta: AttnMetadata):
    """Makes `meta.kv_cache` the pool that vllm::attention reads and writes
    for the duration of the block (nesting restores the outer one)."""
    _META_STACK.append(meta)
    try:
        yield meta
    finally:
        _META_STACK.pop()


def kv_scales() -> tuple[float, float]:
    """(k_scale, v_scale) of the active pool (1, 1 for a bf16 pool)."""
    if not _META_STACK:
        raise RuntimeError("vllm::attention needs an active attention_context(AttnMetadata(kv_cache=...))")
    m = _META_STACK[-1]
    return m.k_scale, m.v_scale


def _layer_caches(layer_id: int) -> tuple[torch.Tensor, torch.Tensor]:
    if not _META_STACK:
        raise RuntimeError("vllm::attention needs an active attention_context(AttnMetadata(kv_cache=...))")
    pool = _META_STACK[-1].kv_cache
    return pool[0, layer_id], pool[1, layer_id]


_WORKSPACE: dict[tuple[str, int | None], torch.Tensor] = {}


# Workspaces replaced by a larger one stay allocated: a hipGraph captured
# earlier keeps the old pointer and replays onto it.
_RETIRED: list[torch.Tensor] = []


def decode_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Per-device decode workspace, grown on demand outside graph capture (the
    kernels need no initial contents: partial counts and partials are written
    before they are read).  The size query never decreases with the batch, so
    a decode graph set captured largest bucket first allocates it once; a
    workspace that is outgrown anyway is kept alive for the graphs that hold
    it.  Calls on one device share it: they must be ordered on one stream."""
    key = (device.type, device.index)
    ws = _WORKSPACE.get(key)
    if ws is None or ws.numel() < nbytes:
        if ws is not None:
            _RETIRED.append(ws)
        with torch.inference_mode(False):  # a plain tensor: later callers outside inference mode may use it
            ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _WORKSPACE[key] = ws
    return ws


def _q_view(q: torch.Tensor, num_heads: int, head_dim: int) -> tuple[torch.Tensor, int, int]:
    q3 = q.view(q.shape[0], num_heads, head_dim) if q.dim() == 2 else q
    if q3.stride(-1) != 1 or q3.stride(0) % 8 or q3.stride(1) % 8 or not aligned16(q3):
        q3 = q3.contiguous()
    return q3, q3.stride(0), q3.stride(1)


def paged_decode_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    cache_seqlens: torch.Tensor,
    num_qo_heads: int,
    num_kv_heads: int,
    head_dim: int,
    softmax_scale: float | None = None,
    out: torch.Tensor | None = None,
    *,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
) -> torch.Tensor:
    """Causal decode over the paged cache: q [B, Hq*D] (or [B, Hq, D]),
    k_cache/v_cache [NB, BS, Hkv, D], block_tables int32 [B, max_blocks],
    cache_seqlens int32 [B] (0 = padding row) -> [B, Hq*D].  An fp8 cache
    (torch.float8_e4m3fn, written by store_kvcache with the same scales)
    attends to k_cache * k_scale and v_cache * v_scale."""
    require_cuda(q, k_cache, v_cache, block_tables, cache_seqlens)
    fp8 = k_cache.dtype == torch.float8_e4m3fn
    require_bf16(q, *(() if fp8 else (k_cache, v_cache)))
    if fp8 and v_cache.dtype != torch.float8_e4m3fn:
        raise TypeError("k_cache and v_cache must share one dtype")
    q3, qs0, qs1 = _q_view(q, num_qo_heads, head_dim)
    bsz = q3.shape[0]
    nb, page, hkv, d = k_cache.shape
    assert hkv == num_kv_heads and d == head_dim and v_cache.stride() == k_cache.stride()
    bt = block_tables if block_tables.dtype == torch.int32 else block_tables.to(torch.int32)
    if bt.stride(-1) != 1:
        bt = bt.contiguous()
    sl = cache_seqlens.to(torch.int32).contiguous()
    assert bt.shape[0] >= bsz and sl.shape[0] >= bsz
    if out is None:
        out = torch.empty((bsz, num_qo_heads * head_dim), dtype=q.dtype, device=q.device)
    L = _C.lib()
    max_blocks = bt.shape[1]
    ws_bytes = L.xv_paged_decode_workspace_size(bsz, num_qo_heads, num_kv_heads, max_blocks, page, head_dim)
    ws = decode_workspace(q.device, ws_bytes)
    scale = 1.0 / math.sqrt(head_dim) if softmax_scale is None else softmax_scale
    if fp8:
        _C.check(
            L.xv_paged_decode_attention_fp8(
                ptr(q3), qs0, qs1, ptr(k_cache), ptr(v_cache), k_cache.stride(0), k_cache.stride(1),
                k_cache.stride(2), ptr(bt), bt.stride(0), ptr(sl), ptr(out), out.stride(0), ptr(ws), ws.numel(),
                bsz, num_qo_heads, num_kv_heads, head_dim, page, max_blocks, float(scale), float(k_scale),
                float(v_scale), stream_of(q),
            ),
            "xv_paged_decode_attention_fp8",
        )
        return out
    _C.check(
        L.xv_paged_decode_attention(
            ptr(q3), qs0, qs1, ptr(k_cache), ptr(v_cache), k_cache.stride(0), k_cache.stride(1),
            k_cache.stride(2), ptr(bt), bt.stride(0), ptr(sl), ptr(out), out.stride(0), ptr(ws), ws.numel(),
            bsz, num_qo_heads, num_kv_heads, head_dim, page, max_blocks, float(scale), stream_of(q),
        ),
        "xv_paged_decode_attention",
    )
    return out


_CASCADE_WS: dict[tuple[str, int | None], torch.Tensor] = {}


def cascade_decode_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    cache_seqlens: torch.Tensor,
    plan: CascadePlan,
    num_qo_heads: int,
    num_kv_heads: int,
    head_dim: int,
    softmax_scale: float | None = None,
    out: torch.Tensor | None = None,
    *,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
) -> torch.Tensor:
    """paged_decode_attention with the shared prefixes of `plan` read once per
    group (xv_cascade_decode_attention, or _fp8 on an fp8 cache with the
    scales of paged_decode_attention).  Same output as the plain decode up
    to fp32 summation order."""
    require_cuda(q, k_cache, v_cache, block_tables, cache_seqlens, plan.prefix_tokens)
    fp8 = k_cache.dtype == torch.float8_e4m3fn
    require_bf16(q, *(() if fp8 else (k_cache, v_cache)))
    if fp8 and v_cache.dtype != torch.float8_e4m3fn:
        raise TypeError("k_cache and v_cache must share one dtype")
    q3, qs0, qs1 = _q_view(q, num_qo_heads, head_dim)
    bsz = q3.shape[0]
    nb, page, hkv, d = k_cache.shape
    assert hkv == num_kv_heads and d == head_dim and v_cache.stride() == k_cache.stride()
    bt = block_tables if block_tables.dtype == torch.int32 else block_tables.to(torch.int32)
    if bt.stride(-1) != 1:
        bt = bt.contiguous()
    sl = cache_seqlens.to(torch.int32).contiguous()
    if out is None:
        out = torch.empty((bsz, num_qo_heads * head_dim), dtype=q.dtype, device=q.device)
    L = _C.lib()
    max_blocks = bt.shape[1]
    nbytes = L.xv_cascade_decode_workspace_size(bsz, num_qo_heads, num_kv_heads, max_blocks, page, head_dim)
    key = (q.device.type, q.device.index)
    ws = _CASCADE_WS.get(key)
    if ws is None or ws.numel() < nbytes:
        if ws is not None:
            _RETIRED.append(ws)  # a recorded graph may still hold it
        with torch.inference_mode(False):  # a plain tensor: later callers outside inference mode may use it
            ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=q.device)
        _CASCADE_WS[key] = ws
    scale = 1.0 / math.sqrt(head_dim) if softmax_scale is None else softmax_scale
    args = (
        ptr(q3), qs0, qs1, ptr(k_cache), ptr(v_cache), k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
        ptr(bt), bt.stride(0), ptr(sl), ptr(plan.prefix_tokens), ptr(plan.group_info), ptr(plan.group_rows),
        plan.num_groups, min(plan.max_prefix_blocks, max_blocks), ptr(out), out.stride(0), ptr(ws), ws.numel(),
        bsz, num_qo_heads, num_kv_heads, head_dim, page, max_blocks, float(scale),
    )
    if fp8:
        _C.check(L.xv_cascade_decode_attention_fp8(*args, float(k_scale), float(v_scale), stream_of(q)),
                 "xv_cascade_decode_attention_fp8")
    else:
        _C.check(L.xv_cascade_decode_attention(*args, stream_of(q)), "xv_cascade_decode_attention")
    return out


def prefill_attention(
    q: torch.Tensor,
    k: torch.Tensor | None,
    v: torch.Tensor | None,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    max_seqlen_q: int,
    num_qo_heads: int,
    num_kv_heads: int,
    head_dim: int,
    k_cache: torch.Tensor | None = None,
    v_cache: torch.Tensor | None = None,
    block_tables: torch.Tensor | None = None,
    softmax_scale: float | None = None,
    max_seqlen_k: int = 0,
    kv_scale: tuple[float, float] | None = None,
) -> torch.Tensor:
    """Varlen causal attention, bottom-right aligned.  With block_tables the
    keys come from the paged cache (cached prefix + this chunk), otherwise
    from k/v rows cu_seqlens_k[b] .. cu_seqlens_k[b+1].  An fp8 paged cache
    needs max_seqlen_k and its (k_scale, v_scale) (default: the active
    attention_context's)."""
    q3, qs0, qs1 = _q_view(q, num_qo_heads, head_dim)
    require_cuda(q3, cu_seqlens_q, cu_seqlens_k)
    require_bf16(q3)
    bsz = cu_seqlens_q.shape[0] - 1
    cuq = cu_seqlens_q.to(torch.int32).contiguous()
    cuk = cu_seqlens_k.to(torch.int32).contiguous()
    out = torch.empty((q3.shape[0], num_qo_heads * head_dim), dtype=q.dtype, device=q.device)
    scale = 1.0 / math.sqrt(head_dim) if softmax_scale is None else softmax_scale
    if block_tables is not None and k_cache is not None and k_cache.dtype == torch.float8_e4m3fn:
        # fp8 pages: the sequences' keys dequantized into varlen bf16 rows, then the dense path
        k_scale, v_scale = kv_scales() if kv_scale is None else kv_scale
        if max_seqlen_k <= 0:
            raise ValueError("prefill over an fp8 paged cache needs max_seqlen_k (the longest key run)")
        hkv = k_cache.shape[2]
        bt = block_tables.to(torch.int32)
        if bt.stride(-1) != 1:
            bt = bt.contiguous()
        rows = bsz * int(max_seqlen_k)
        kd = torch.empty((max(rows, 1), hkv, head_dim), dtype=torch.bfloat16, device=q.device)
        vd = torch.empty_like(kd)
        _C.check(
            _C.lib().xv_gather_kv_fp8(
                ptr(k_cache), ptr(v_cache), k_cache.stride(0), k_cache.stride(1), k_cache.stride(2), ptr(bt),
                bt.stride(0), k_cache.shape[1], ptr(cuk), bsz, int(max_seqlen_k), hkv, head_dim, float(k_scale),
                float(v_scale), ptr(kd), ptr(vd), kd.stride(0), stream_of(q),
            ),
            "xv_gather_kv_fp8",
        )
        return prefill_attention(q, kd, vd, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, num_qo_heads, num_kv_heads,
                                 head_dim, softmax_scale=softmax_scale)
    if block_tables is not None:
        assert k_cache is not None and v_cache is not None
        require_bf16(k_cache, v_cache)
        bt = block_tables.to(torch.int32)
        if bt.stride(-1) != 1:
            bt = bt.contiguous()
        kd = vd = None
        kvs0 = kvs1 = 0
        kc, vc = k_cache, v_cache
        ps, ts, hs = k_cache.stride(0), k_cache.stride(1), k_cache.stride(2)
        page = k_cache.shape[1]
        bts = bt.stride(0)
    else:
        k3 = k.view(k.shape[0], num_kv_heads, head_dim) if k.dim() == 2 else k
        v3 = v.view(v.shape[0], num_kv_heads, head_dim) if v.dim() == 2 else v
        if (k3.stride() != v3.stride() or k3.stride(-1) != 1 or k3.stride(0) % 8 or k3.stride(1) % 8
                or not aligned16(k3) or not aligned16(v3)):
            k3, v3 = k3.contiguous(), v3.contiguous()
        require_bf16(k3, v3)
        kd, vd = k3, v3
        kvs0, kvs1 = k3.stride(0), k3.stride(1)
        kc = vc = bt = None
        ps = ts = hs = bts = 0
        page = 16
    _C.check(
        _C.lib().xv_prefill_attention(
            ptr(q3), qs0, qs1, ptr(kd), ptr(vd), kvs0, kvs1, ptr(kc), ptr(vc), ps, ts, hs, ptr(bt), bts,
            ptr(cuq), ptr(cuk), ptr(out), out.stride(0), bsz, int(max_seqlen_q), num_qo_heads, num_kv_heads,
            head_dim, page, float(scale), stream_of(q),
        ),
        "xv_prefill_attention",
    )
    return out


@torch.library.custom_op("vllm::attention", mutates_args=())
def attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    slot_mapping: Optional[torch.Tensor],
    is_prefill: bool,
    cu_seqlens_q: Optional[torch.Tensor],
    cu_seqlens_k: Optional[torch.Tensor],
    max_seqlen_q: int,
    max_seqlen_k: int,
    block_tables: Optional[torch.Tensor],
    cache_seqlens: Optional[torch.Tensor],
    layer_id: int,
    num_qo_heads: int,
    num_kv_heads: int,
    head_dim: int,
) -> torch.Tensor:
    k_cache, v_cache = _layer_caches(layer_id)
    k3 = k.view(-1, num_kv_heads, head_dim)
    v3 = v.view(-1, num_kv_heads, head_dim)
    ks, vs = kv_scales()
    if slot_mapping is not None:  # None: this step's K/V are already in the cache (fused store)
        store_kvcache(k3, v3, k_cache, v_cache, slot_mapping, k_scale=ks, v_scale=vs)  # paged view, in place
    if is_prefill:
        if block_tables is not None:
            return prefill_attention(
                q, None, None, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, num_qo_heads, num_kv_heads,
                head_dim, k_cache=k_cache, v_cache=v_cache, block_tables=block_tables, max_seqlen_k=max_seqlen_k,
                kv_scale=(ks, vs),
            )
        return prefill_attention(
            q, k3, v3, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, num_qo_heads, num_kv_heads, head_dim
        )
    return paged_decode_attention(
        q, k_cache, v_cache, block_tables, cache_seqlens, num_qo_heads, num_kv_heads, head_dim,
        k_scale=ks, v_scale=vs,
    )


@attention.register_fake
def _attention_fake(
    q, k, v, slot_mapping, is_prefill, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
    max_seqlen_k, block_tables, cache_seqlens, layer_id, num_qo_heads,
    num_kv_heads, head_dim,
):
    return torch.empty((q.shape[0], num_qo_heads * head_dim), dtype=q.dtype, device=q.device)


def kv_cache_of(layer_id: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(k_cache, v_cache) [NB, BS, Hkv, D] views of the active pool for a layer."""
    return _layer_caches(layer_id)


class Attention(nn.Module):
    def __init__(self, num_heads: int, head_dim: int, num_kv_heads: int, layer_id: int = 0) -> None:
        super().__init__()
        self.num_heads, self.num_kv_heads, self.head_dim = num_heads, num_kv_heads, head_dim
        self.layer_id = layer_id

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, attn: AttnInputs) -> torch.Tensor:
        if attn.cascade is not None and not attn.is_prefill:
            # shared-prefix decode: the plan does not fit the vllm::attention schema
            k_cache, v_cache = _layer_caches(self.layer_id)
            ks, vs = kv_scales()
            if attn.slot_mapping is not None:
                store_kvcache(k.view(-1, self.num_kv_heads, self.head_dim), v.view(-1, self.num_kv_heads, self.head_dim),
                              k_cache, v_cache, attn.slot_mapping, k_scale=ks, v_scale=vs)
            return cascade_decode_attention(q, k_cache, v_cache, attn.block_tables, attn.cache_seqlens, attn.cascade,
                                            self.num_heads, self.num_kv_heads, self.head_dim, k_scale=ks, v_scale=vs)
        return torch.ops.vllm.attention(
            q, k, v, attn.slot_mapping, attn.is_prefill, attn.cu_seqlens_q, attn.cu_seqlens_k,
            attn.max_seqlen_q, attn.max_seqlen_k, attn.block_tables, attn.cache_seqlens,
            self.layer_id, self.num_heads, self.num_kv_heads, self.head_dim,
        )
