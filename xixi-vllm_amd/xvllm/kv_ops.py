"""KV store by slot mapping (reference ``src/compute/kv_ops.py:35-62``)."""
from __future__ import annotations

import torch

from . import _C
from ._torch_glue import aligned16, ptr, require_bf16, require_cuda, stream_of


def store_kvcache(
    key: torch.Tensor,
    value: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    *,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
) -> None:
    """k_cache[slot[i]] = key[i]; v_cache[slot[i]] = value[i]; slot -1 is skipped.

    An fp8 cache (torch.float8_e4m3fn, this build's optional pool format)
    stores e4m3fn(key * (1/k_scale)) and e4m3fn(value * (1/v_scale)); the
    scales are ignored for a bf16 cache.

    key/value: [N, Hkv, D].  The kernel reads strided views directly when
    every head row starts 16-byte aligned with a unit last stride (the q/k/v
    views of a fused qkv GEMM output); any other layout is first copied to a
    fresh contiguous tensor, as the reference does for every input
    (kv_ops.py:42-45).  k_cache/v_cache: paged [NB, BS, Hkv, D] views of the
    pool (any strides, written in place) or flat [num_slots, Hkv, D].
    """
    require_cuda(key, value, k_cache, v_cache, slot_mapping)
    fp8 = k_cache.dtype == torch.float8_e4m3fn
    require_bf16(key, value, *(() if fp8 else (k_cache, v_cache)))
    if fp8 and v_cache.dtype != torch.float8_e4m3fn:
        raise TypeError("k_cache and v_cache must share one dtype")
    n, num_heads, head_dim = key.shape
    assert slot_mapping.numel() == n
    if head_dim % 8:
        raise ValueError(f"head_dim must be a multiple of 8 (16-byte rows), got {head_dim}")

    def readable(t):
        if t.stride(-1) != 1 or t.stride(0) % 8 or t.stride(1) % 8 or not aligned16(t):
            return t.clone(memory_format=torch.contiguous_format)  # fresh, aligned allocation
        return t

    key, value = readable(key), readable(value)
    kc, vc = k_cache, v_cache
    if kc.stride() != vc.stride() or kc.shape != vc.shape:
        raise ValueError("k_cache and v_cache must share one layout")
    if kc.dim() == 4:  # [NB, BS, Hkv, D]
        assert kc.shape[2] == num_heads and kc.shape[3] == head_dim
        ps, ts, hs, bs = kc.stride(0), kc.stride(1), kc.stride(2), kc.shape[1]
    else:  # [num_slots, Hkv, D]
        kc = kc.view(-1, num_heads, head_dim)
        vc = vc.view(-1, num_heads, head_dim)
        ps, ts, hs, bs = kc.stride(0), 0, kc.stride(1), 1
    slots = slot_mapping if slot_mapping.dtype == torch.int32 else slot_mapping.to(torch.int32)
    slots = slots.contiguous()
    if fp8:
        _C.check(
            _C.lib().xv_store_kvcache_fp8(
                ptr(key), key.stride(0), key.stride(1), ptr(value), value.stride(0), value.stride(1),
                ptr(kc), ptr(vc), ps, ts, hs, bs, ptr(slots), n, num_heads, head_dim,
                float(k_scale), float(v_scale), stream_of(key),
            ),
            "xv_store_kvcache_fp8",
        )
        return
    _C.check(
        _C.lib().xv_store_kvcache(
            ptr(key), key.stride(0), key.stride(1), ptr(value), value.stride(0), value.stride(1),
            ptr(kc), ptr(vc), ps, ts, hs, bs, ptr(slots), n, num_heads, head_dim,
            stream_of(key),
        ),
        "xv_store_kvcache",
    )
