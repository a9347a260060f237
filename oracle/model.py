"""numpy restatement of one Qwen3 decoder layer at decode time, plus the final
norm and the greedy LM head (TEST INFRASTRUCTURE ONLY).

Follows src/compute/models/qwen3.py:112-153 (layer wiring), :187-208 (final
norm), :117-128 (q/k norm + RoPE) and src/compute/layers/attention.py:43-100
(store, then causal paged decode).  bf16 rounding is applied where the
reference's ops write bf16 tensors (GEMM outputs, norm outputs, RoPE, SiLU,
attention output); arithmetic inside an op is float64.
"""
from __future__ import annotations

import numpy as np

from . import ops as O
from .bf16 import round_bf16


def linear(x, w):
    """bf16 GEMM x @ w.T with an fp32-accumulated, bf16-rounded result."""
    return round_bf16((np.asarray(x, np.float64) @ np.asarray(w, np.float64).T).astype(np.float32))


def decode_layer(w: dict, hidden, residual, positions, k_cache, v_cache, block_tables, seqlens, slots, cos_sin,
                 hq: int, hkv: int, d: int, eps: float, kv_fp8: tuple | None = None):
    """One decoder layer for a decode batch.  Mutates k_cache/v_cache (stores
    this step's K/V).  Returns dict(attn=attention output [B, Hq*D],
    hidden=layer output, residual=residual stream).  kv_fp8 = (k_scale,
    v_scale): the caches hold dequantized fp8 pages (this build's optional
    pool format), and this step's K/V are stored as the fp8 store rounds them."""
    if residual is None:
        x, residual = O.rmsnorm(hidden, w["input_layernorm"], eps), round_bf16(hidden)
    else:
        x, residual = O.fused_add_rmsnorm(hidden, residual, w["input_layernorm"], eps)
    qkv = linear(x, w["qkv_proj"])
    t = qkv.shape[0]
    q = qkv[:, : hq * d].reshape(t, hq, d)
    k = qkv[:, hq * d : (hq + hkv) * d].reshape(t, hkv, d)
    v = qkv[:, (hq + hkv) * d :].reshape(t, hkv, d)
    q, k = O.qk_norm_rope(q, k, w["q_norm"], w["k_norm"], eps, positions, cos_sin)
    if kv_fp8 is not None:
        ks, vs = (np.float32(x) for x in kv_fp8)
        k = O.dequantize_fp8(O.quantize_fp8(k, np.float32(1.0) / ks), ks)
        v = O.dequantize_fp8(O.quantize_fp8(v, np.float32(1.0) / vs), vs)
    O.store_kvcache(k, v, k_cache, v_cache, slots)
    attn = round_bf16(O.paged_decode_attention(q, k_cache, v_cache, block_tables, seqlens).astype(np.float32))
    attn = attn.reshape(t, hq * d)
    h, residual = post_attention(w, attn, residual, eps)
    return {"attn": attn, "hidden": h, "residual": residual}


def post_attention(w: dict, attn, residual, eps: float):
    """The rest of a decoder layer after attention (qwen3.py:66-72, 143-153):
    o_proj, fused add + post-attention RMSNorm, gate_up, SiLU-and-mul, down.
    Returns (layer output, residual stream)."""
    h = linear(attn, w["o_proj"])
    h, residual = O.fused_add_rmsnorm(h, residual, w["post_attention_layernorm"], eps)
    gu = linear(h, w["gate_up_proj"])
    return linear(O.silu_and_mul(gu), w["down_proj"]), residual


def final_logits(hidden, residual, norm_w, lm_head, eps):
    """Final fused add + RMSNorm (qwen3.py:205-206) then the LM head GEMM."""
    x, _ = O.fused_add_rmsnorm(hidden, residual, norm_w, eps)
    return x, linear(x, lm_head)
