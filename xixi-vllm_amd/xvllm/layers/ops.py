"""torch.library custom ops with the names and signatures of xixi-vllm's
``src/compute/layers/ops.py`` (``vllm::silu_and_mul``, ``vllm::rotary_embedding``,
``vllm::rmsnorm``, ``vllm::fused_add_rmsnorm``), each running a gfx950 HIP
kernel through the C ABI, plus ``xv::qk_norm_rope``, the fused Qwen3 q/k
head-norm + RoPE used by ``Qwen3Attention._split_norm_rope``.

Fake (meta) implementations are registered for every op, as the reference does.
"""
from __future__ import annotations

import torch

from .. import _C
from .._torch_glue import aligned16, ptr, require_bf16, require_cuda, stream_of


def _rows_view(x: torch.Tensor, hidden: int) -> tuple[torch.Tensor, int, int, int, int]:
    """Express x[..., hidden] as (n_outer, n_inner) rows with two strides, copying
    only when the layout cannot be described that way."""
    if x.stride(-1) == 1 and aligned16(x):
        if x.dim() == 2 and x.stride(0) % 8 == 0:
            return x, x.shape[0], 1, x.stride(0), 0
        if x.dim() == 3 and x.stride(0) % 8 == 0 and x.stride(1) % 8 == 0:
            return x, x.shape[0], x.shape[1], x.stride(0), x.stride(1)
        if x.dim() == 1:
            return x, 1, 1, hidden, 0
    xc = x.reshape(-1, hidden).contiguous()
    return xc, xc.shape[0], 1, hidden, 0


@torch.library.custom_op("vllm::silu_and_mul", mutates_args=())
def silu_and_mul(x: torch.Tensor) -> torch.Tensor:
    """out = silu(x[:, :I]) * x[:, I:]  (reference ops.py:20-23)."""
    require_cuda(x)
    require_bf16(x)
    inter = x.shape[-1] // 2
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or not aligned16(x2):
        x2 = x2.contiguous()
    out = torch.empty(x.shape[:-1] + (inter,), dtype=x.dtype, device=x.device)
    _C.check(
        _C.lib().xv_silu_and_mul(ptr(x2), x2.stride(0), ptr(out), inter, x2.shape[0], inter, stream_of(x)),
        "xv_silu_and_mul",
    )
    return out


@silu_and_mul.register_fake
def _silu_and_mul_fake(x: torch.Tensor) -> torch.Tensor:
    return torch.empty((x.shape[0], x.shape[1] // 2), dtype=x.dtype, device=x.device)


def _head_view(t: torch.Tensor) -> tuple[torch.Tensor, int, int]:
    """[T, H, D] view with unit last stride and 16-byte aligned rows."""
    if t.stride(-1) != 1 or t.stride(0) % 8 or t.stride(1) % 8 or not aligned16(t):
        t = t.contiguous()
    return t, t.stride(0), t.stride(1)


@torch.library.custom_op("vllm::rotary_embedding", mutates_args=())
def rotary_embedding(
    q: torch.Tensor,
    k: torch.Tensor,
    positions: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    head_size: int,
) -> tuple[torch.Tensor, torch.Tensor]:
    """NeoX RoPE from the fp32 cos||sin table, new q/k tensors (reference ops.py:31-51)."""
    require_cuda(q, k, positions, cos_sin_cache)
    require_bf16(q, k)
    n = q.shape[0]
    q3, qs0, qs1 = _head_view(q.reshape(n, -1, head_size) if q.dim() == 2 else q)
    k3, ks0, ks1 = _head_view(k.reshape(n, -1, head_size) if k.dim() == 2 else k)
    if cos_sin_cache.dtype != torch.float32:
        raise TypeError("cos_sin_cache must be float32 (reference rotary.py:41-51)")
    pos = positions.to(torch.int64).contiguous()
    csc = cos_sin_cache.contiguous()
    qo = torch.empty(q3.shape, dtype=q.dtype, device=q.device)
    ko = torch.empty(k3.shape, dtype=k.dtype, device=k.device)
    _C.check(
        _C.lib().xv_rotary_embedding(
            ptr(q3), qs0, qs1, ptr(k3), ks0, ks1, ptr(pos), ptr(csc), ptr(qo), ptr(ko),
            n, q3.shape[1], k3.shape[1], head_size, stream_of(q),
        ),
        "xv_rotary_embedding",
    )
    return qo.view(q.shape), ko.view(k.shape)


@rotary_embedding.register_fake
def _rotary_embedding_fake(q, k, positions, cos_sin_cache, head_size):
    return torch.empty_like(q), torch.empty_like(k)


@torch.library.custom_op("vllm::rmsnorm", mutates_args=())
def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm over the last dim into a new tensor (reference ops.py:59-64)."""
    require_cuda(x, weight)
    require_bf16(x, weight)
    hidden = weight.shape[0]
    xv, n_outer, n_inner, s_outer, s_inner = _rows_view(x, hidden)
    w = weight.contiguous()
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    _C.check(
        _C.lib().xv_rmsnorm(ptr(xv), s_outer, s_inner, ptr(w), ptr(out), n_outer, n_inner, hidden,
                            float(eps), stream_of(x)),
        "xv_rmsnorm",
    )
    return out


@rmsnorm.register_fake
def _rmsnorm_fake(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    return torch.empty_like(x)


@torch.library.custom_op("vllm::fused_add_rmsnorm", mutates_args=("x", "residual"))
def fused_add_rmsnorm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float) -> None:
    """In place: residual <- x + residual; x <- rmsnorm(residual) (reference ops.py:72-79)."""
    require_cuda(x, residual, weight)
    require_bf16(x, residual, weight)
    hidden = weight.shape[0]
    for t, name in ((x, "x"), (residual, "residual")):
        if t.dim() != 2 or t.stride(-1) != 1 or t.stride(0) % 8 or not aligned16(t):
            raise ValueError(f"fused_add_rmsnorm needs a 2-D row-major {name} with 16-byte aligned rows")
    w = weight.contiguous()
    _C.check(
        _C.lib().xv_fused_add_rmsnorm(ptr(x), x.stride(0), ptr(residual), residual.stride(0), ptr(w),
                                      x.shape[0], hidden, float(eps), stream_of(x)),
        "xv_fused_add_rmsnorm",
    )


@fused_add_rmsnorm.register_fake
def _fused_add_rmsnorm_fake(x, residual, weight, eps) -> None:
    return None


@torch.library.custom_op("xv::fused_add_rmsnorm_parts", mutates_args=("residual",))
def fused_add_rmsnorm_parts(parts: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                            eps: float) -> torch.Tensor:
    """fused_add_rmsnorm on the fp32 partial sums [P, T, H] of a split-K GEMM:
    x = bf16(parts.sum(0)); residual <- x + residual; returns rmsnorm(residual)."""
    require_cuda(parts, residual, weight)
    require_bf16(residual, weight)
    if parts.dtype != torch.float32 or parts.dim() != 3 or parts.stride(-1) != 1 or not aligned16(parts):
        raise ValueError("fused_add_rmsnorm_parts needs fp32 partial sums [P, T, H], rows contiguous")
    if residual.dim() != 2 or residual.stride(-1) != 1 or residual.stride(0) % 8 or not aligned16(residual):
        raise ValueError("fused_add_rmsnorm_parts needs a 2-D row-major residual with 16-byte aligned rows")
    p, t, hidden = parts.shape
    if residual.shape != (t, hidden) or weight.shape[0] != hidden:
        raise ValueError(f"shapes: parts {tuple(parts.shape)}, residual {tuple(residual.shape)}, weight {tuple(weight.shape)}")
    out = torch.empty((t, hidden), dtype=residual.dtype, device=residual.device)
    w = weight.contiguous()
    _C.check(
        _C.lib().xv_fused_add_rmsnorm_parts(ptr(parts), parts.stride(0), parts.stride(1), p, ptr(out), hidden,
                                            ptr(residual), residual.stride(0), ptr(w), t, hidden, float(eps),
                                            stream_of(residual)),
        "xv_fused_add_rmsnorm_parts",
    )
    return out


@fused_add_rmsnorm_parts.register_fake
def _fused_add_rmsnorm_parts_fake(parts, residual, weight, eps) -> torch.Tensor:
    return residual.new_empty(residual.shape)


@torch.library.custom_op("xv::qk_norm_rope", mutates_args=())
def qk_norm_rope(
    q: torch.Tensor,
    k: torch.Tensor,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    eps: float,
    positions: torch.Tensor,
    cos_sin_cache: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-head RMSNorm of q [T, Hq, D] and k [T, Hkv, D] followed by NeoX RoPE,
    one kernel (reference qwen3.py:117-128: rmsnorm, rmsnorm, rotary_embedding)."""
    require_cuda(q, k, q_weight, k_weight, positions, cos_sin_cache)
    require_bf16(q, k, q_weight, k_weight)
    q3, qs0, qs1 = _head_view(q)
    k3, ks0, ks1 = _head_view(k)
    n, hq, d = q3.shape
    pos = positions.to(torch.int64).contiguous()
    qo = torch.empty((n, hq, d), dtype=q.dtype, device=q.device)
    ko = torch.empty(k3.shape, dtype=k.dtype, device=k.device)
    _C.check(
        _C.lib().xv_qk_norm_rope(
            ptr(q3), qs0, qs1, ptr(k3), ks0, ks1, ptr(q_weight.contiguous()), ptr(k_weight.contiguous()),
            float(eps), ptr(pos), ptr(cos_sin_cache.contiguous()), ptr(qo), ptr(ko), n, hq, k3.shape[1], d,
            stream_of(q),
        ),
        "xv_qk_norm_rope",
    )
    return qo, ko


@qk_norm_rope.register_fake
def _qk_norm_rope_fake(q, k, q_weight, k_weight, eps, positions, cos_sin_cache):
    return torch.empty(q.shape, dtype=q.dtype, device=q.device), torch.empty(k.shape, dtype=k.dtype, device=k.device)


def _cache_strides(cache: torch.Tensor) -> tuple[int, int, int, int]:
    """(page, token, head strides, block size) of a paged [NB, BS, Hkv, D] cache view."""
    assert cache.dim() == 4 and cache.stride(-1) == 1
    return cache.stride(0), cache.stride(1), cache.stride(2), cache.shape[1]


@torch.library.custom_op("xv::qk_norm_rope_store", mutates_args=("k_cache", "v_cache"))
def qk_norm_rope_store(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    eps: float,
    positions: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
) -> torch.Tensor:
    """Decode-step fusion: q/k head RMSNorm + RoPE; q returned [T, Hq, D], k (roped)
    and v written into the paged caches at slot_mapping (reference
    qwen3.py:117-128 followed by kv_ops.store_kvcache).  fp8 caches
    (torch.float8_e4m3fn) store e4m3fn(x / scale), as store_kvcache does."""
    require_cuda(q, k, v, k_cache, v_cache, slot_mapping)
    fp8 = k_cache.dtype == torch.float8_e4m3fn
    require_bf16(q, k, v, *(() if fp8 else (k_cache, v_cache)))
    if fp8 and v_cache.dtype != torch.float8_e4m3fn:
        raise TypeError("k_cache and v_cache must share one dtype")
    q3, qs0, qs1 = _head_view(q)
    k3, ks0, ks1 = _head_view(k)
    v3, vs0, vs1 = _head_view(v)
    n, hq, d = q3.shape
    ps, ts, hs, bs = _cache_strides(k_cache)
    assert v_cache.stride() == k_cache.stride()
    slots = slot_mapping.to(torch.int32).contiguous()
    pos = positions.to(torch.int64).contiguous()
    qo = torch.empty((n, hq, d), dtype=q.dtype, device=q.device)
    if fp8:
        _C.check(
            _C.lib().xv_qk_norm_rope_store_fp8(
                ptr(q3), qs0, qs1, ptr(k3), ks0, ks1, ptr(v3), vs0, vs1, ptr(q_weight.contiguous()),
                ptr(k_weight.contiguous()), float(eps), ptr(pos), ptr(cos_sin_cache.contiguous()), ptr(qo),
                ptr(k_cache), ptr(v_cache), ps, ts, hs, bs, ptr(slots), n, hq, k3.shape[1], d, float(k_scale),
                float(v_scale), stream_of(q),
            ),
            "xv_qk_norm_rope_store_fp8",
        )
        return qo
    _C.check(
        _C.lib().xv_qk_norm_rope_store(
            ptr(q3), qs0, qs1, ptr(k3), ks0, ks1, ptr(v3), vs0, vs1, ptr(q_weight.contiguous()),
            ptr(k_weight.contiguous()), float(eps), ptr(pos), ptr(cos_sin_cache.contiguous()), ptr(qo),
            ptr(k_cache), ptr(v_cache), ps, ts, hs, bs, ptr(slots), n, hq, k3.shape[1], d, stream_of(q),
        ),
        "xv_qk_norm_rope_store",
    )
    return qo


@qk_norm_rope_store.register_fake
def _qk_norm_rope_store_fake(q, k, v, q_weight, k_weight, eps, positions, cos_sin_cache, k_cache, v_cache,
                             slot_mapping, k_scale=1.0, v_scale=1.0):
    return torch.empty(q.shape, dtype=q.dtype, device=q.device)
