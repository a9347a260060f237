"""Qwen3 dense decoder wired onto the xvllm operator API, one GPU (the
reference's tp=1, pp=1 case of src/compute/models/qwen3.py:44-238).

Per layer: input RMSNorm (fused with the residual add after layer 0), fused
qkv GEMM, per-head q/k RMSNorm + NeoX RoPE (one kernel, `xv::qk_norm_rope`),
`vllm::attention` (KV store + paged decode / prefill), o GEMM, fused add +
RMSNorm, gate_up GEMM, SiLU-and-mul, down GEMM.  GEMMs run on PyTorch
(hipBLASLt), except at decode batch sizes (at most 64 rows) once
pack_decode_weights has made packed copies of gate_up, down and o: then the
gate_up GEMM + SiLU-and-mul is one weight-streaming kernel, and down and o
are streamed as split-K partials into the next norm.  Weights are plain
tensors (random init for the benchmarks; the reference's checkpoint loader is
out of scope).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from ..config import head_dim as _head_dim
from ..config import rope_theta as _rope_theta
from ..layers import Attention, AttnInputs, RMSNorm, RotaryEmbedding
from ..layers.attention import kv_cache_of, kv_scales
from ..layers.linear import (GEMM_PARTS, GEMM_SILU_MUL, linear_into_norm, pack_weight, stream_rows, streamable,
                             streamed_into_norm, streamed_silu_mul)
from ..layers import ops as _ops  # noqa: F401  (registers the custom ops)
from ..sampler import sample


class StalePackedWeights(RuntimeError):
    """A weight was written or replaced after pack_decode_weights copied it:
    the streamed decode GEMMs would read the old values."""


def _weight_stamp(*params) -> tuple:
    return tuple((p._version, p.data_ptr()) for p in params)


def _check_stamp(module, stamp: tuple, *params) -> None:
    """Raise when a packed weight's source changed since it was packed
    (in-place writes through the Parameter bump its version; assigning a new
    tensor moves its data pointer).  Writes through `.data` bypass the version
    counter and are not seen."""
    if _weight_stamp(*params) != stamp:
        raise StalePackedWeights(f"{type(module).__name__}: weights changed after pack_decode_weights; "
                                 "call model.pack_decode_weights(False) then pack_decode_weights() again "
                                 "(outside graph capture; re-capture the decode graphs)")


class Qwen3MLP(nn.Module):
    def __init__(self, hidden: int, inter: int):
        super().__init__()
        self.gate_up_proj = nn.Parameter(torch.empty(2 * inter, hidden))  # [gate; up] (linear.py:297-304)
        self.down_proj = nn.Parameter(torch.empty(hidden, inter))
        self.split_k = True
        self.packed = None  # (gate_up, down) PackedWeights for decode batches

    def forward(self, x):
        """SiLU-MLP; the down GEMM may return PartialSums (split-K) for the
        next residual add + RMSNorm."""
        if self.packed is not None and self.split_k and stream_rows(x):
            _check_stamp(self, self._stamp, self.gate_up_proj, self.down_proj)
            return streamed_into_norm(streamed_silu_mul(x, self.packed[0]), self.packed[1])
        return linear_into_norm(torch.ops.vllm.silu_and_mul(F.linear(x, self.gate_up_proj)), self.down_proj,
                                self.split_k)

    def pack(self, enabled: bool = True):
        if not enabled:
            self.packed = None
        elif self.packed is None and streamable(self.gate_up_proj, GEMM_SILU_MUL) and streamable(self.down_proj,
                                                                                                   GEMM_PARTS):
            self.packed = (pack_weight(self.gate_up_proj.data), pack_weight(self.down_proj.data))
            self._stamp = _weight_stamp(self.gate_up_proj, self.down_proj)


class Qwen3Attention(nn.Module):
    def __init__(self, cfg, layer_id: int):
        super().__init__()
        self.num_heads = cfg.num_attention_heads
        self.num_kv_heads = cfg.num_key_value_heads
        self.head_dim = _head_dim(cfg)
        self.q_size = self.num_heads * self.head_dim
        self.kv_size = self.num_kv_heads * self.head_dim
        self.qkv_proj = nn.Parameter(torch.empty(self.q_size + 2 * self.kv_size, cfg.hidden_size))
        self.o_proj = nn.Parameter(torch.empty(cfg.hidden_size, self.q_size))
        self.q_norm = RMSNorm(self.head_dim, cfg.rms_norm_eps)
        self.k_norm = RMSNorm(self.head_dim, cfg.rms_norm_eps)
        self.rotary_emb = RotaryEmbedding(self.head_dim, self.head_dim, cfg.max_position_embeddings, _rope_theta(cfg))
        self.attn = Attention(self.num_heads, self.head_dim, self.num_kv_heads, layer_id=layer_id)
        self.eps = cfg.rms_norm_eps
        self.split_k = True
        self.packed_o = None  # o_proj PackedWeight for decode batches

    def forward(self, positions, hidden, attn: AttnInputs):
        """qkv -> q/k norm + RoPE -> attention -> o GEMM (PartialSums when
        split along K, for post_attention_layernorm)."""
        qkv = F.linear(hidden, self.qkv_proj)
        if not attn.is_prefill:
            # decode: norm + RoPE + KV store in one kernel, attention reads the cache
            q, k, v = self._split_norm_rope_store(positions, qkv, attn.slot_mapping)
            o = self.attn(q.view(q.shape[0], self.q_size), k, v, attn._replace(slot_mapping=None))
        else:
            q, k, v = self._split_norm_rope(positions, qkv)
            o = self.attn(q.view(q.shape[0], self.q_size), k, v, attn)
        if self.packed_o is not None and self.split_k and stream_rows(o):
            _check_stamp(self, self._stamp, self.o_proj)
            return streamed_into_norm(o, self.packed_o)
        return linear_into_norm(o, self.o_proj, self.split_k)

    def pack(self, enabled: bool = True):
        if not enabled:
            self.packed_o = None
        elif self.packed_o is None and streamable(self.o_proj, GEMM_PARTS):
            self.packed_o = pack_weight(self.o_proj.data)
            self._stamp = _weight_stamp(self.o_proj)

    def _views(self, qkv):
        t = qkv.shape[0]
        q = qkv[:, : self.q_size].view(t, self.num_heads, self.head_dim)
        k = qkv[:, self.q_size : self.q_size + self.kv_size].view(t, self.num_kv_heads, self.head_dim)
        v = qkv[:, self.q_size + self.kv_size :].view(t, self.num_kv_heads, self.head_dim)
        return q, k, v

    def _split_norm_rope_store(self, positions, qkv, slot_mapping):
        q, k, v = self._views(qkv)
        k_cache, v_cache = kv_cache_of(self.attn.layer_id)
        ks, vs = kv_scales()
        q = torch.ops.xv.qk_norm_rope_store(
            q, k, v, self.q_norm.weight, self.k_norm.weight, self.eps, positions, self.rotary_emb.cos_sin_cache,
            k_cache, v_cache, slot_mapping, ks, vs,
        )
        return q, k, v

    def _split_norm_rope(self, positions, qkv):
        """split -> per-head q/k RMSNorm -> RoPE (reference qwen3.py:117-128),
        the two norms and the rotation as one kernel reading the qkv views."""
        q, k, v = self._views(qkv)
        q, k = torch.ops.xv.qk_norm_rope(
            q, k, self.q_norm.weight, self.k_norm.weight, self.eps, positions, self.rotary_emb.cos_sin_cache
        )
        return q, k, v


class Qwen3DecoderLayer(nn.Module):
    def __init__(self, cfg, layer_id: int):
        super().__init__()
        self.self_attn = Qwen3Attention(cfg, layer_id)
        self.mlp = Qwen3MLP(cfg.hidden_size, cfg.intermediate_size)
        self.input_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)

    def forward(self, positions, hidden, residual, attn: AttnInputs):
        """(hidden, residual) -> (hidden, residual) as the reference layer
        (qwen3.py:149-153), except that the returned hidden may be the
        PartialSums of the split-K down GEMM: the next layer's input norm (or
        the final norm) consumes them; PartialSums.materialize() gives the
        bf16 tensor."""
        hidden, residual = self.input_layernorm(hidden, residual)
        hidden = self.self_attn(positions, hidden, attn)
        hidden, residual = self.post_attention_layernorm(hidden, residual)
        return self.mlp(hidden), residual


class Qwen3Model(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.embed_tokens = nn.Parameter(torch.empty(cfg.vocab_size, cfg.hidden_size))
        self.layers = nn.ModuleList([Qwen3DecoderLayer(cfg, i) for i in range(cfg.num_hidden_layers)])
        self.norm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)

    def forward(self, input_ids, positions, attn: AttnInputs):
        h, residual = F.embedding(input_ids, self.embed_tokens), None
        for layer in self.layers:
            h, residual = layer(positions, h, residual, attn)
        return self.norm(h, residual)[0]


class Qwen3ForCausalLM(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.config = cfg
        self.model = Qwen3Model(cfg)
        self.lm_head = nn.Parameter(torch.empty(cfg.vocab_size, cfg.hidden_size))

    def forward(self, input_ids, positions, attn: AttnInputs):
        return self.model(input_ids, positions, attn)

    def set_split_k(self, enabled: bool):
        """Split-K for o_proj / down_proj at decode batch sizes (on by default)."""
        for m in self.modules():
            if isinstance(m, (Qwen3Attention, Qwen3MLP)):
                m.split_k = enabled
        return self

    @torch.no_grad()
    def pack_decode_weights(self, enabled: bool = True):
        """Packed copies of every layer's gate_up, down and o weights for the
        weight-streaming decode GEMMs; layers that have them keep them (the
        graphs captured over them stay valid).  enabled=False drops them: only
        when no captured graph still uses them.  Call once the weights are
        final: the copies do not follow later writes (an eager forward raises
        StalePackedWeights when a packed weight was written in place or
        replaced since).  They add packed_decode_bytes() to the weights,
        (2 I H + I H + H Hq D) x 2 bytes per layer (Qwen3-8B: 335 MB per
        layer, 12.1 GB; the Qwen3-32B shape: 56 GB): size the KV pool after
        packing, or pass that figure as KVPool.auto_num_blocks' reserve_bytes."""
        for m in self.modules():
            if isinstance(m, (Qwen3Attention, Qwen3MLP)):
                m.pack(enabled)
        return self

    def packed_decode_bytes(self) -> int:
        """Bytes pack_decode_weights adds (counted for the layers whose
        weights the streamed GEMMs take)."""
        total = 0
        for m in self.modules():
            if isinstance(m, Qwen3MLP) and streamable(m.gate_up_proj, GEMM_SILU_MUL) and streamable(m.down_proj,
                                                                                                  GEMM_PARTS):
                total += (m.gate_up_proj.numel() + m.down_proj.numel()) * m.gate_up_proj.element_size()
            elif isinstance(m, Qwen3Attention) and streamable(m.o_proj, GEMM_PARTS):
                total += m.o_proj.numel() * m.o_proj.element_size()
        return total

    def compute_logits(self, hidden):
        return F.linear(hidden, self.lm_head)

    def argmax(self, hidden):
        """Greedy ids (reference vocab_parallel.py:180-216): argmax of the bf16
        logits, lowest id on ties, by the sampler kernel."""
        logits = self.compute_logits(hidden)
        return sample(logits, None, all_greedy=True)

    @torch.no_grad()
    def random_init_(self, std: float = 0.02, seed: int = 0):
        """Weights ~ N(0, std) (norm weights 1), drawn on the parameters' device."""
        g = torch.Generator(device=self.lm_head.device).manual_seed(seed)
        for name, p in self.named_parameters():
            if name.endswith("norm.weight"):
                p.fill_(1.0)
            else:
                p.normal_(0.0, std, generator=g)
        return self
