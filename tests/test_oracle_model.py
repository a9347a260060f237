"""Pins oracle/model.py (the checker of the config-1 GPU test) against things
other than itself:

- an independent implementation of the same decoder layer: transformers'
  Qwen3DecoderLayer / Qwen3RMSNorm (float64, eager attention, the past keys
  and values of each sequence gathered from the paged cache into its
  DynamicCache).  It fixes the qkv split order, the q/k head norms, the NeoX
  rotation, the GQA head map, the residual contract and the gate/up order;
- closed forms: zero o_proj / down_proj leave the layer output 0 and the
  residual equal to the input (the first layer's (norm(x), x) rule); one-hot
  qkv rows make q, k, v known copies of the normed input, so the stored V and
  the split are fixed; a context of one token returns that token's V per
  head; an identity LM head returns the normed hidden state.
"""
import numpy as np
import pytest
import torch

import oracle.model as OM
import oracle.ops as O
from oracle.bf16 import round_bf16

H, HQ, HKV, D, FFN, EPS, THETA = 256, 4, 2, 128, 512, 1e-6, 1e6
rng = np.random.default_rng(5)


def _bf(a):
    return round_bf16(np.asarray(a, np.float32))


def _weights(scale_out=3.0):
    """Weights whose op outputs are O(1), so that wiring mistakes show above
    the bf16 rounding of the residual stream."""
    n = lambda shape, std: _bf(rng.standard_normal(shape) * std)
    return {
        "qkv_proj": n(((HQ + 2 * HKV) * D, H), 1 / np.sqrt(H)),
        "o_proj": n((H, HQ * D), scale_out / np.sqrt(HQ * D)),
        "gate_up_proj": n((2 * FFN, H), 1 / np.sqrt(H)),
        "down_proj": n((H, FFN), scale_out / np.sqrt(FFN)),
        "q_norm": _bf(1 + 0.1 * rng.standard_normal(D)),
        "k_norm": _bf(1 + 0.1 * rng.standard_normal(D)),
        "input_layernorm": _bf(1 + 0.1 * rng.standard_normal(H)),
        "post_attention_layernorm": _bf(1 + 0.1 * rng.standard_normal(H)),
        "norm": _bf(1 + 0.1 * rng.standard_normal(H)),
    }


def _paged_case(ctx, page=16, pool=64):
    need = [(c + page - 1) // page for c in ctx]
    perm = rng.permutation(pool)
    bt = np.full((len(ctx), max(need)), -1, np.int32)
    o = 0
    for b, n in enumerate(need):
        bt[b, :n] = perm[o : o + n]
        o += n
    kc = _bf(rng.standard_normal((pool, page, HKV, D)))
    vc = _bf(rng.standard_normal((pool, page, HKV, D)))
    pos = np.array([c - 1 for c in ctx], np.int64)
    slots = np.array([bt[b, p // page] * page + p % page for b, p in enumerate(pos)], np.int32)
    return bt, kc, vc, pos, slots


def _run_oracle(w, hidden, residual, ctx, bt, kc, vc, pos, slots):
    cs = O.build_cos_sin_cache(D, 4096, THETA)
    return OM.decode_layer(w, hidden, residual, pos, kc, vc, bt, np.array(ctx), slots, cs, HQ, HKV, D, EPS)


def _hf_layer(w):
    from transformers import Qwen3Config
    from transformers.models.qwen3 import modeling_qwen3 as M

    cfg = Qwen3Config(hidden_size=H, intermediate_size=FFN, num_attention_heads=HQ, num_key_value_heads=HKV,
                      head_dim=D, rms_norm_eps=EPS, max_position_embeddings=4096, num_hidden_layers=1,
                      rope_parameters={"rope_type": "default", "rope_theta": THETA}, vocab_size=1000)
    cfg._attn_implementation = "eager"
    layer = M.Qwen3DecoderLayer(cfg, 0).to(torch.float64).eval()
    rope = M.Qwen3RotaryEmbedding(cfg).to(torch.float64)
    t = lambda a: torch.from_numpy(np.asarray(a, np.float64))
    qkv = t(w["qkv_proj"])
    with torch.no_grad():
        a = layer.self_attn
        a.q_proj.weight.copy_(qkv[: HQ * D])
        a.k_proj.weight.copy_(qkv[HQ * D : (HQ + HKV) * D])
        a.v_proj.weight.copy_(qkv[(HQ + HKV) * D :])
        a.o_proj.weight.copy_(t(w["o_proj"]))
        a.q_norm.weight.copy_(t(w["q_norm"]))
        a.k_norm.weight.copy_(t(w["k_norm"]))
        layer.mlp.gate_proj.weight.copy_(t(w["gate_up_proj"][:FFN]))
        layer.mlp.up_proj.weight.copy_(t(w["gate_up_proj"][FFN:]))
        layer.mlp.down_proj.weight.copy_(t(w["down_proj"]))
        layer.input_layernorm.weight.copy_(t(w["input_layernorm"]))
        layer.post_attention_layernorm.weight.copy_(t(w["post_attention_layernorm"]))
    return cfg, layer, rope


def test_decode_layer_matches_transformers_qwen3():
    from transformers.cache_utils import DynamicCache

    w = _weights()
    ctx = [1, 7, 40]
    bt, kc, vc, pos, slots = _paged_case(ctx)
    hidden = _bf(rng.standard_normal((len(ctx), H)))
    ref = _run_oracle(w, hidden, None, ctx, bt, kc.copy(), vc.copy(), pos, slots)
    kc_after, vc_after = kc.copy(), vc.copy()
    _run_oracle(w, hidden, None, ctx, bt, kc_after, vc_after, pos, slots)
    cfg, layer, rope = _hf_layer(w)
    seen = {}
    layer.self_attn.o_proj.register_forward_pre_hook(lambda m, a: seen.__setitem__("attn", a[0].clone()))
    for b, c in enumerate(ctx):
        cache = DynamicCache(config=cfg)
        if c > 1:  # the sequence's earlier tokens, as stored (normed and rotated K)
            kp = O.gather_paged(kc, bt[b], c - 1)  # [c-1, HKV, D]
            vp = O.gather_paged(vc, bt[b], c - 1)
            cache.update(torch.from_numpy(kp.astype(np.float64)).permute(1, 0, 2)[None],
                         torch.from_numpy(vp.astype(np.float64)).permute(1, 0, 2)[None], 0)
        x = torch.from_numpy(hidden[b : b + 1].astype(np.float64))[None]
        pid = torch.tensor([[c - 1]])
        with torch.no_grad():
            out = layer(x, attention_mask=None, position_ids=pid, past_key_values=cache, use_cache=True,
                        position_embeddings=rope(x, pid))
        out = out[0] if isinstance(out, tuple) else out
        # attention output (o_proj input): q/k norm, rotation, GQA, softmax over the context
        np.testing.assert_allclose(ref["attn"][b], seen["attn"].numpy().reshape(-1), rtol=2e-2, atol=2e-2)
        # this step's K and V, as the oracle stored them at the sequence's slot
        k_new = cache.layers[0].keys[0, :, c - 1].numpy()
        v_new = cache.layers[0].values[0, :, c - 1].numpy()
        page, off = divmod(int(slots[b]), 16)
        np.testing.assert_allclose(kc_after[page, off], k_new, rtol=2e-2, atol=2e-2)
        np.testing.assert_allclose(vc_after[page, off], v_new, rtol=1e-2, atol=1e-2)
        # layer output: the oracle returns (mlp out, residual) whose sum is the decoder's output
        delta_hf = out.numpy().reshape(-1) - hidden[b].astype(np.float64)
        delta_or = (ref["hidden"][b].astype(np.float64) + ref["residual"][b]) - hidden[b]
        assert np.abs(delta_hf).mean() > 0.3  # the residual does not hide the layer's contribution
        np.testing.assert_allclose(delta_or, delta_hf, rtol=3e-2, atol=3e-2)


def test_final_logits_match_transformers_norm():
    from transformers.models.qwen3 import modeling_qwen3 as M

    w = _weights()
    hid, res = _bf(rng.standard_normal((3, H))), _bf(rng.standard_normal((3, H)))
    lm = _bf(rng.standard_normal((50, H)) / np.sqrt(H))
    x, logits = OM.final_logits(hid, res, w["norm"], lm, EPS)
    norm = M.Qwen3RMSNorm(H, eps=EPS).to(torch.float64)
    with torch.no_grad():
        norm.weight.copy_(torch.from_numpy(w["norm"].astype(np.float64)))
        xr = norm(torch.from_numpy((hid.astype(np.float64) + res)))
    np.testing.assert_allclose(x, xr.numpy(), rtol=1e-2, atol=1e-2)
    np.testing.assert_allclose(logits, xr.numpy() @ lm.T.astype(np.float64), rtol=2e-2, atol=2e-2)
    # identity LM head: the logits are the normed state itself
    _, ident = OM.final_logits(hid, res, w["norm"], np.eye(H, dtype=np.float32), EPS)
    np.testing.assert_array_equal(ident, x)


def test_zero_output_projections_pass_the_residual_through():
    """o_proj = down_proj = 0: the layer output is exactly 0 and the residual
    is the input (first layer: (norm(x), x); later layers: bf16(x + r))."""
    w = _weights()
    w["o_proj"] = np.zeros_like(w["o_proj"])
    w["down_proj"] = np.zeros_like(w["down_proj"])
    ctx = [5, 17]
    bt, kc, vc, pos, slots = _paged_case(ctx)
    hidden = _bf(rng.standard_normal((2, H)))
    ref = _run_oracle(w, hidden, None, ctx, bt, kc, vc, pos, slots)
    assert not ref["hidden"].any()
    np.testing.assert_array_equal(ref["residual"], hidden)
    r_in = _bf(rng.standard_normal((2, H)))
    ref2 = _run_oracle(w, hidden, r_in, ctx, bt, kc, vc, pos, slots)
    assert not ref2["hidden"].any()
    np.testing.assert_array_equal(ref2["residual"], _bf(hidden + r_in))


def test_one_hot_qkv_fixes_the_split_and_single_token_attention():
    """qkv row r copies column m(r) of the normed input x (m distinct per
    part), so q, k, v are known: the stored V at the step's slot is exactly
    x[m(v rows)], and with a context of one token every query head h returns
    the V of kv head h // (HQ // HKV)."""
    w = _weights()
    rows = (HQ + 2 * HKV) * D
    cols = (np.arange(rows) * 7 + 3) % H
    onehot = np.zeros((rows, H), np.float32)
    onehot[np.arange(rows), cols] = 1.0
    w["qkv_proj"] = onehot
    ctx = [1, 1, 1]
    bt, kc, vc, pos, slots = _paged_case(ctx)
    hidden = _bf(rng.standard_normal((3, H)))
    ref = _run_oracle(w, hidden, None, ctx, bt, kc, vc, pos, slots)
    x = O.rmsnorm(hidden, w["input_layernorm"], EPS)
    v_rows = cols[(HQ + HKV) * D :]
    v_want = x[:, v_rows].reshape(3, HKV, D)
    for b in range(3):
        page, off = divmod(int(slots[b]), 16)
        np.testing.assert_array_equal(vc[page, off], v_want[b])
        attn = ref["attn"][b].reshape(HQ, D)
        for h in range(HQ):
            np.testing.assert_array_equal(attn[h], v_want[b, h // (HQ // HKV)])
    # K: the normed, rotated copy of its rows (position 0: the rotation is the identity)
    k_rows = cols[HQ * D : (HQ + HKV) * D]
    k_want = O.rmsnorm(x[:, k_rows].reshape(3, HKV, D), w["k_norm"], EPS)
    for b in range(3):
        page, off = divmod(int(slots[b]), 16)
        np.testing.assert_array_equal(kc[page, off], k_want[b])
