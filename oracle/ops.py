"""numpy restatement of the reference hot-path ops (TEST INFRASTRUCTURE ONLY).

Inputs/outputs are numpy arrays.  bf16 tensors are passed as float32 arrays
holding bf16-representable values; outputs are float64 (attention) or fp32
rounded to bf16 where the reference writes bf16.
"""
from __future__ import annotations

import math

import numpy as np

from .bf16 import round_bf16


# ---------------------------------------------------------------- KV store
def store_kvcache(key, value, k_cache, v_cache, slot_mapping) -> None:
    """k_cache.view(-1,Hkv,D)[slot[i]] = key[i]; slot -1 skipped.
    Reference: src/compute/kv_ops.py:8-32 (kernel), :35-62 (wrapper)."""
    kc = k_cache.reshape(-1, *key.shape[1:])
    vc = v_cache.reshape(-1, *value.shape[1:])
    for i, s in enumerate(np.asarray(slot_mapping).tolist()):
        if s == -1:
            continue
        kc[s] = key[i]
        vc[s] = value[i]


def slots_for_range(block_table, start: int, end: int, block_size: int) -> list[int]:
    """Physical slot of every token in [start, end): bt[p // BS] * BS + p % BS.
    Reference: src/data/sequence.py:26-51 (and batch.py:123 for one decode token)."""
    return [block_table[p // block_size] * block_size + p % block_size for p in range(start, end)]


# ---------------------------------------------------------------- attention
def gather_paged(cache, block_table, n_tokens: int):
    """Rows 0..n_tokens-1 of one sequence from a paged cache [NB, BS, Hkv, D]."""
    bs = cache.shape[1]
    p = np.arange(n_tokens)
    pages = np.asarray(block_table)[p // bs]
    return np.asarray(cache)[pages, p % bs]


def _attend(q, k, v, mask=None, scale=None):
    """q [Nq, Hq, D], k/v [Nk, Hkv, D] -> [Nq, Hq, D] float64; q head h uses kv
    head h // (Hq/Hkv) (GQA); mask [Nq, Nk] True = visible."""
    nq, hq, d = q.shape
    hkv = k.shape[1]
    grp = hq // hkv
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    q64, k64, v64 = (np.asarray(a, np.float64) for a in (q, k, v))
    out = np.zeros((nq, hq, d))
    for h in range(hq):
        s = (q64[:, h, :] @ k64[:, h // grp, :].T) * scale
        if mask is not None:
            s = np.where(mask, s, -np.inf)
        m = s.max(axis=1, keepdims=True)
        m = np.where(np.isfinite(m), m, 0.0)
        p = np.exp(s - m)
        den = p.sum(axis=1, keepdims=True)
        out[:, h, :] = np.where(den > 0, (p @ v64[:, h // grp, :]) / np.where(den > 0, den, 1), 0.0)
    return out


def paged_decode_attention(q, k_cache, v_cache, block_tables, cache_seqlens, scale=None):
    """Decode: every sequence's single query attends to all cache_seqlens[b]
    cached tokens (the new one included).  Padding rows (seqlen 0) give 0.
    Reference: src/compute/layers/attention.py:91-99 (flash_attn_with_kvcache,
    causal, cache_seqlens = pos+1 per batch.py:124)."""
    bsz, hq, d = q.shape
    out = np.zeros((bsz, hq, d))
    for b in range(bsz):
        n = int(cache_seqlens[b])
        if n <= 0:
            continue
        k = gather_paged(k_cache, block_tables[b], n)
        v = gather_paged(v_cache, block_tables[b], n)
        out[b] = _attend(q[b : b + 1], k, v, scale=scale)[0]
    return out


def prefill_attention(q, cu_q, cu_k, k=None, v=None, k_cache=None, v_cache=None, block_tables=None, scale=None):
    """Varlen causal attention, bottom-right aligned: query i of a sequence with
    q_len queries and k_len keys sees keys j <= k_len - q_len + i.  Keys come
    from k/v rows cu_k[b]:cu_k[b+1] or, with block_tables, from the paged cache.
    Reference: src/compute/layers/attention.py:74-90 (flash_attn_varlen_func,
    causal=True, block_table when batch.py:172-179 has_cache)."""
    out = np.zeros(q.shape, dtype=np.float64)
    bsz = len(cu_q) - 1
    for b in range(bsz):
        q0, q1 = int(cu_q[b]), int(cu_q[b + 1])
        klen = int(cu_k[b + 1] - cu_k[b])
        if block_tables is not None:
            kb = gather_paged(k_cache, block_tables[b], klen)
            vb = gather_paged(v_cache, block_tables[b], klen)
        else:
            kb = k[int(cu_k[b]) : int(cu_k[b + 1])]
            vb = v[int(cu_k[b]) : int(cu_k[b + 1])]
        nq = q1 - q0
        if nq == 0:
            continue
        qi = np.arange(nq)[:, None]
        kj = np.arange(klen)[None, :]
        mask = kj <= (klen - nq) + qi
        out[q0:q1] = _attend(q[q0:q1], kb, vb, mask=mask, scale=scale)
    return out


# ---------------------------------------------------------------- norms
def rmsnorm(x, w, eps):
    """x * rsqrt(mean(x^2) + eps) * w over the last dim, fp32, bf16 output.
    Reference: src/compute/layers/ops.py:59-64 (flashinfer rmsnorm)."""
    x32 = np.asarray(x, np.float32)
    ms = np.mean(x32.astype(np.float64) ** 2, axis=-1, keepdims=True)
    r = (x32 / np.sqrt(ms + eps)) * np.asarray(w, np.float32)
    return round_bf16(r.astype(np.float32))


def fused_add_rmsnorm(x, residual, w, eps):
    """Returns (x_out, residual_out): residual_out = bf16(x + residual),
    x_out = rmsnorm of the fp32 sum.  Reference: src/compute/layers/ops.py:72-79,
    layernorm.py:16-20."""
    s = np.asarray(x, np.float32) + np.asarray(residual, np.float32)
    return rmsnorm(s, w, eps), round_bf16(s)


# ---------------------------------------------------------------- RoPE
def build_cos_sin_cache(head_dim: int, max_pos: int, theta: float):
    """[max_pos, D] fp32: cos || sin of pos * theta^(-2i/D).
    Reference: src/compute/layers/rotary.py:7-20 (evaluated in float64 here,
    then rounded to fp32)."""
    i = np.arange(0, head_dim, 2, dtype=np.float64)
    inv = 1.0 / (theta ** (i / head_dim))
    ang = np.arange(max_pos, dtype=np.float64)[:, None] * inv[None, :]
    return np.concatenate([np.cos(ang), np.sin(ang)], axis=-1).astype(np.float32)


def rope_neox(x, positions, cos_sin):
    """x [T, H, D]: o1 = x1 cos - x2 sin, o2 = x2 cos + x1 sin (NeoX half split),
    cos/sin rows from the table.  Reference: src/compute/layers/ops.py:31-51
    (apply_rope_with_cos_sin_cache, is_neox=True)."""
    d = x.shape[-1]
    cs = np.asarray(cos_sin, np.float32)[np.asarray(positions)]
    c = cs[:, None, : d // 2].astype(np.float64)
    s = cs[:, None, d // 2 :].astype(np.float64)
    x64 = np.asarray(x, np.float64)
    x1, x2 = x64[..., : d // 2], x64[..., d // 2 :]
    return round_bf16(np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1).astype(np.float32))


def qk_norm_rope(q, k, qw, kw, eps, positions, cos_sin):
    """Qwen3 _split_norm_rope: per-head RMSNorm (bf16 result) then NeoX RoPE.
    Reference: src/compute/models/qwen3.py:117-128."""
    return (rope_neox(rmsnorm(q, qw, eps), positions, cos_sin),
            rope_neox(rmsnorm(k, kw, eps), positions, cos_sin))


# ---------------------------------------------------------------- activation
def silu_and_mul(x):
    """silu(x[:, :I]) * x[:, I:], bf16 output.  Reference: src/compute/layers/ops.py:20-23."""
    x64 = np.asarray(x, np.float64)
    i = x.shape[-1] // 2
    g, u = x64[..., :i], x64[..., i:]
    return round_bf16((g / (1.0 + np.exp(-g)) * u).astype(np.float32))


# ---------------------------------------------------------------- fp8 pages
# The optional fp8 pool format of this build (the reference's pool holds the
# model dtype, src/compute/kv_pool.py:49-51): OCP float8 e4m3fn, sign, 4
# exponent bits (bias 7), 3 mantissa bits, no infinities, 0x7f / 0xff NaN.
def fp8_e4m3fn_values() -> np.ndarray:
    """float32 value of each of the 256 codes, from the format definition."""
    c = np.arange(256)
    s, e, m = c >> 7, (c >> 3) & 15, c & 7
    mag = np.where(e == 0, m * 2.0**-9, (1.0 + m / 8.0) * 2.0 ** (e - 7))
    v = np.where(s == 1, -mag, mag)
    v = np.where((e == 15) & (m == 7), np.nan, v)
    return v.astype(np.float32)


def quantize_fp8(x, inv_scale: float) -> np.ndarray:
    """e4m3fn codes of float32(x) * float32(inv_scale): round to nearest, ties
    to the even code, except that a tie at 464 (halfway from the largest value
    448 to the next binade's 480) gives 448; |product| > 464 and NaN give NaN
    (0x7f, sign kept for the product)."""
    p = (np.asarray(x, np.float32) * np.float32(inv_scale)).astype(np.float32)
    pos = fp8_e4m3fn_values()[:127].astype(np.float64)  # codes 0..126 ascending: 0 .. 448
    a = np.abs(p.astype(np.float64))
    hi = np.clip(np.searchsorted(pos, a, side="left"), 0, 126)  # first value >= a
    lo = np.clip(hi - 1, 0, 126)
    d_lo, d_hi = a - pos[lo], pos[hi] - a
    code = np.where(d_lo < d_hi, lo, np.where(d_hi < d_lo, hi, np.where(lo % 2 == 0, lo, hi)))
    code = np.where(a > 448.0, np.where(a <= 464.0, 126, 127), code)
    code = np.where(np.isnan(a), 127, code)
    sign = np.signbit(p) & ~np.isnan(p)
    return (code | np.where(sign, 0x80, 0)).astype(np.uint8)


def dequantize_fp8(codes, scale: float) -> np.ndarray:
    """float64 values the decode attends to: value(code) * scale."""
    return fp8_e4m3fn_values()[np.asarray(codes, np.uint8)].astype(np.float64) * float(scale)
