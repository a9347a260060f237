"""fp8 (OCP e4m3fn) KV pages, this build's optional pool format (the
reference's pool holds the model dtype, src/compute/kv_pool.py:49-51): the
store is bit-exact against the oracle's quantizer (itself pinned against
torch's float8_e4m3fn cast in tests/test_oracle.py), and the decode attention
matches the oracle's attention over the dequantized pages within rtol/atol
2e-2 (bf16 output, fp32 accumulate), the tolerance of the bf16 path."""
import math

import numpy as np
import pytest
import torch

import oracle.ops as O
from helpers import f32, gen, make_paged, randn_bf16

pytestmark = pytest.mark.gpu

RTOL = ATOL = 2e-2


def _close(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert np.isfinite(got).all(), "non-finite output"
    err = np.abs(got - want) - (ATOL + RTOL * np.abs(want))
    assert (err <= 0).all(), f"max excess {err.max():.4g} at {np.unravel_index(err.argmax(), err.shape)}"


def _to_fp8(codes: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(codes)).view(torch.float8_e4m3fn)


@pytest.mark.parametrize("n,layout,ks,vs", [(37, "nhd", 1.0, 1.0), (300, "nhd", 0.05, 0.2), (64, "hnd", 0.013, 3.0),
                                            (1, "hnd", 1.0, 0.5)])
def test_store_kvcache_fp8_bitexact(dev, n, layout, ks, vs):
    """Random injective slots with padding (-1) tokens; values scaled so some
    products pass the format's range (NaN codes) and some underflow to
    subnormals and zero; untouched slots keep their old bytes."""
    from xvllm.kv_ops import store_kvcache

    g = gen(n)
    hkv, d, nb, page = 8, 128, 40, 16
    key = randn_bf16((n, hkv, d), g, std=3.0)
    val = randn_bf16((n, hkv, d), g, std=3.0)
    slots = torch.randperm(nb * page, generator=g)[:n].to(torch.int32)
    slots[::5] = -1
    init = np.random.default_rng(n).integers(0, 256, (2, nb, page, hkv, d), dtype=np.uint8)
    if layout == "nhd":
        store = torch.from_numpy(init.copy())
        kc, vc = store[0], store[1]
    else:  # head-major memory, the reference's logical [NB, BS, Hkv, D] view
        store = torch.from_numpy(np.ascontiguousarray(init.transpose(0, 1, 3, 2, 4)))
        kc, vc = store[0].transpose(1, 2), store[1].transpose(1, 2)
    want_k, want_v = init[0].copy(), init[1].copy()
    sl = slots.numpy()
    kq = O.quantize_fp8(f32(key), np.float32(1.0) / np.float32(ks))
    vq = O.quantize_fp8(f32(val), np.float32(1.0) / np.float32(vs))
    for i, s in enumerate(sl):
        if s >= 0:
            want_k[s // page, s % page] = kq[i]
            want_v[s // page, s % page] = vq[i]
    sg = store.to(dev)
    if layout == "nhd":
        kg, vg = sg[0].view(torch.float8_e4m3fn), sg[1].view(torch.float8_e4m3fn)
    else:
        kg, vg = sg[0].view(torch.float8_e4m3fn).transpose(1, 2), sg[1].view(torch.float8_e4m3fn).transpose(1, 2)
    store_kvcache(key.to(dev), val.to(dev), kg, vg, slots.to(dev), k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    got = sg.cpu().numpy()
    if layout == "hnd":
        got = got.transpose(0, 1, 3, 2, 4)
    assert np.array_equal(got[0], want_k)
    assert np.array_equal(got[1], want_v)


def _fp8_case(ctx, hq, hkv, g, ks, vs, layout="nhd"):
    d = 128
    need = sum((c + 15) // 16 for c in ctx)
    kc, vc, bt, sl = make_paged(ctx, int(need * 1.25) + 4, hkv, d, g)  # unused rows NaN
    kq = O.quantize_fp8(f32(kc), np.float32(1.0) / np.float32(ks))
    vq = O.quantize_fp8(f32(vc), np.float32(1.0) / np.float32(vs))
    q = randn_bf16((len(ctx), hq, d), g)
    want = O.paged_decode_attention(f32(q), O.dequantize_fp8(kq, ks), O.dequantize_fp8(vq, vs), bt.numpy(), sl.numpy())
    if layout == "nhd":
        kg, vg = _to_fp8(kq), _to_fp8(vq)
    else:
        kg = _to_fp8(kq.transpose(0, 2, 1, 3)).transpose(1, 2)
        vg = _to_fp8(vq.transpose(0, 2, 1, 3)).transpose(1, 2)
    return q, kg, vg, bt, sl, want


@pytest.mark.parametrize(
    "hq,hkv,ctx,layout",
    [
        (32, 8, [1, 17, 300, 513, 16, 2048, 0, 77], "nhd"),  # Qwen3-8B heads, pad row (0)
        (32, 8, [1, 17, 300, 513, 16, 2048, 0, 77], "hnd"),
        (16, 8, [128, 511, 256, 300], "nhd"),                 # group 2
        (64, 8, [1000, 33, 4096], "hnd"),                     # group 8
        (8, 8, [5, 260], "nhd"),                              # MHA
        (32, 8, [2060], "nhd"),                               # 33 partials per head
    ],
)
def test_paged_decode_fp8(dev, hq, hkv, ctx, layout):
    from xvllm.layers.attention import paged_decode_attention

    g = gen(hq + len(ctx) + 1000)
    ks, vs = 1.0 / 32, 1.0 / 16
    q, kg, vg, bt, sl, want = _fp8_case(ctx, hq, hkv, g, ks, vs, layout)
    d = 128
    kd, vd = (kg.to(dev), vg.to(dev)) if layout == "nhd" else (None, None)
    if layout == "hnd":  # keep the head-major memory order on the device
        kd = kg.transpose(1, 2).contiguous().to(dev).transpose(1, 2)
        vd = vg.transpose(1, 2).contiguous().to(dev).transpose(1, 2)
    out = paged_decode_attention(q.view(len(ctx), -1).to(dev), kd, vd, bt.to(dev), sl.to(dev), hq, hkv, d,
                                 k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    _close(f32(out).reshape(len(ctx), hq, d), want)


def test_paged_decode_fp8_config2_full_size(dev):
    """Config 2's batch (B 64, ctx U[512, 4096]) on fp8 pages; a sample of rows
    against the oracle, every row finite."""
    from xvllm.layers.attention import paged_decode_attention

    g = gen(2025)
    ctx = torch.randint(512, 4097, (64,), generator=g).tolist()
    need = sum((c + 15) // 16 for c in ctx)
    kc, vc, bt, sl = make_paged(ctx, math.ceil(need * 1.25), 8, 128, g, fill_nan=False)
    kq, vq = O.quantize_fp8(f32(kc), 8.0), O.quantize_fp8(f32(vc), 8.0)
    q = randn_bf16((64, 32, 128), g)
    out = paged_decode_attention(q.view(64, -1).to(dev), _to_fp8(kq).to(dev), _to_fp8(vq).to(dev), bt.to(dev),
                                 sl.to(dev), 32, 8, 128, k_scale=0.125, v_scale=0.125)
    got = f32(out).reshape(64, 32, 128)
    rows = [0, 31, 63]
    want = O.paged_decode_attention(f32(q)[rows], O.dequantize_fp8(kq, 0.125), O.dequantize_fp8(vq, 0.125),
                                    bt.numpy()[rows], sl.numpy()[rows])
    _close(got[rows], want)
    assert np.isfinite(got).all()


def test_fp8_store_then_decode_round_trip(dev):
    """store_kvcache (fp8) then paged_decode_attention (fp8) over the same
    pool: equal to the oracle on the quantized values of the stored rows."""
    from xvllm.kv_ops import store_kvcache
    from xvllm.layers.attention import paged_decode_attention

    g = gen(77)
    hq, hkv, d, page = 32, 8, 128, 16
    ctx = [40, 129, 7]
    need = [(c + page - 1) // page for c in ctx]
    nb = sum(need) + 2
    perm = torch.randperm(nb, generator=g)
    bt = torch.full((3, max(need)), -1, dtype=torch.int32)
    o = 0
    for b, n in enumerate(need):
        bt[b, :n] = perm[o : o + n].to(torch.int32)
        o += n
    T = sum(ctx)
    key, val = randn_bf16((T, hkv, d), g), randn_bf16((T, hkv, d), g)
    slots = torch.tensor([int(bt[b, p // page]) * page + p % page for b, c in enumerate(ctx) for p in range(c)],
                         dtype=torch.int32)
    kc = torch.zeros((nb, page, hkv, d), dtype=torch.float8_e4m3fn, device=dev)
    vc = torch.zeros_like(kc)
    ks, vs = 0.02, 0.04
    store_kvcache(key.to(dev), val.to(dev), kc, vc, slots.to(dev), k_scale=ks, v_scale=vs)
    q = randn_bf16((3, hq, d), g)
    sl = torch.tensor(ctx, dtype=torch.int32)
    out = paged_decode_attention(q.view(3, -1).to(dev), kc, vc, bt.to(dev), sl.to(dev), hq, hkv, d,
                                 k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    kq = kc.cpu().view(torch.uint8).numpy()
    vq = vc.cpu().view(torch.uint8).numpy()
    want = O.paged_decode_attention(f32(q), O.dequantize_fp8(kq, ks), O.dequantize_fp8(vq, vs), bt.numpy(), sl.numpy())
    _close(f32(out).reshape(3, hq, d), want)
    # and the stored codes are the oracle's
    kq_want = O.quantize_fp8(f32(key), np.float32(1.0) / np.float32(ks))
    sls = slots.numpy()
    assert np.array_equal(kq.reshape(-1, hkv, d)[sls], kq_want)


def test_qk_norm_rope_store_fp8_equals_bf16_store_then_quantize(dev):
    """The fused decode store into an fp8 cache writes exactly the fp8 codes
    of what the bf16 fused store writes (roped k and v, rounded to bf16),
    and returns the same q."""
    import xvllm.layers.ops  # noqa: F401
    from xvllm.layers.rotary import build_cos_sin_cache

    g = gen(91)
    t, hq, hkv, d, nb, page = 37, 32, 8, 128, 12, 16
    qkv = randn_bf16((t, (hq + 2 * hkv) * d), g, std=2.0).to(dev)
    q = qkv[:, : hq * d].view(t, hq, d)
    k = qkv[:, hq * d : (hq + hkv) * d].view(t, hkv, d)
    v = qkv[:, (hq + hkv) * d :].view(t, hkv, d)
    qw, kw = randn_bf16((d,), g, 0.1, 1.0).to(dev), randn_bf16((d,), g, 0.1, 1.0).to(dev)
    pos = torch.randint(0, 4096, (t,), generator=g).to(dev)
    cs = build_cos_sin_cache(d, 4096, 1e6).to(dev)
    slots = torch.randperm(nb * page, generator=g)[:t].to(torch.int32)
    slots[::6] = -1
    slots = slots.to(dev)
    kb = torch.zeros((nb, page, hkv, d), dtype=torch.bfloat16, device=dev)
    vb = torch.zeros_like(kb)
    k8 = torch.zeros((nb, page, hkv, d), dtype=torch.float8_e4m3fn, device=dev)
    v8 = torch.zeros_like(k8)
    ks, vs = 0.03, 0.5
    qa = torch.ops.xv.qk_norm_rope_store(q, k, v, qw, kw, 1e-6, pos, cs, kb, vb, slots)
    qb = torch.ops.xv.qk_norm_rope_store(q, k, v, qw, kw, 1e-6, pos, cs, k8, v8, slots, ks, vs)
    torch.cuda.synchronize()
    assert torch.equal(qa.view(torch.int16), qb.view(torch.int16))
    sl = slots.cpu().numpy()
    sl = sl[sl >= 0]
    kq = O.quantize_fp8(f32(kb).reshape(-1, hkv, d)[sl], np.float32(1.0) / np.float32(ks))
    vq = O.quantize_fp8(f32(vb).reshape(-1, hkv, d)[sl], np.float32(1.0) / np.float32(vs))
    assert np.array_equal(k8.cpu().view(torch.uint8).numpy().reshape(-1, hkv, d)[sl], kq)
    assert np.array_equal(v8.cpu().view(torch.uint8).numpy().reshape(-1, hkv, d)[sl], vq)


def test_chunked_prefill_over_fp8_pages(dev):
    """Chunked prefill whose keys (cached prefix + chunk) come from fp8 pages
    through the block tables: the oracle's causal attention over the
    dequantized pages, within the bf16 tolerance."""
    from xvllm.layers.attention import prefill_attention

    g = gen(123)
    hq, hkv, d, page = 32, 8, 128, 16
    pre, new = [40, 0, 300, 17], [24, 33, 1, 64]
    klens = [p_ + n_ for p_, n_ in zip(pre, new)]
    need = [(k_ + page - 1) // page for k_ in klens]
    kc, vc, bt, _ = make_paged(klens, sum(need) + 5, hkv, d, g)
    ks, vs = 0.05, 0.1
    kq = O.quantize_fp8(f32(kc), np.float32(1.0) / np.float32(ks))
    vq = O.quantize_fp8(f32(vc), np.float32(1.0) / np.float32(vs))
    q = randn_bf16((sum(new), hq, d), g)
    cu_q = torch.tensor([0] + np.cumsum(new).tolist(), dtype=torch.int32)
    cu_k = torch.tensor([0] + np.cumsum(klens).tolist(), dtype=torch.int32)
    out = prefill_attention(q.view(sum(new), -1).to(dev), None, None, cu_q.to(dev), cu_k.to(dev), max(new), hq, hkv,
                            d, k_cache=_to_fp8(kq).to(dev), v_cache=_to_fp8(vq).to(dev), block_tables=bt.to(dev),
                            max_seqlen_k=max(klens), kv_scale=(ks, vs))
    torch.cuda.synchronize()
    want = O.prefill_attention(f32(q), cu_q.numpy(), cu_k.numpy(), k_cache=O.dequantize_fp8(kq, ks),
                               v_cache=O.dequantize_fp8(vq, vs), block_tables=bt.numpy())
    _close(f32(out).reshape(-1, hq, d), want)


def test_config1_layer_decode_on_fp8_pool(dev):
    """Config 1's decoder layer with an fp8 pool (scales 1/16 and 1/8): the
    layer stores this step's K/V as fp8 and attends over fp8 pages; the
    oracle layer on the dequantized pages (its store rounds K/V the same
    way) matches the attention output and the layer output at the bf16
    tolerance."""
    from test_gpu_model import D, EPS, FFN, HIDDEN, HKV, HQ, _layer_case
    import oracle.model as OM
    from xvllm.config import Qwen3Shape
    from xvllm.layers.attention import AttnInputs, AttnMetadata, attention_context
    from xvllm.layers.rotary import build_cos_sin_cache
    from xvllm.models.qwen3 import Qwen3DecoderLayer

    ctx, bt, w, kc, vc, hidden, pos, slots = _layer_case(seed=5)
    ks, vs = 1.0 / 16, 1.0 / 8
    kq = O.quantize_fp8(f32(kc), np.float32(1.0) / np.float32(ks))
    vq = O.quantize_fp8(f32(vc), np.float32(1.0) / np.float32(vs))
    cfg = Qwen3Shape(HIDDEN, HQ, HKV, D, FFN, 1, max_position_embeddings=4096)
    with torch.device(dev):
        layer = Qwen3DecoderLayer(cfg, 0).to(torch.bfloat16)
        layer.self_attn.rotary_emb.cos_sin_cache = build_cos_sin_cache(D, 4096, 1e6).to(dev)
    with torch.no_grad():
        for name, mod in (("qkv_proj", layer.self_attn), ("o_proj", layer.self_attn), ("gate_up_proj", layer.mlp),
                          ("down_proj", layer.mlp)):
            getattr(mod, name).copy_(w[name])
        layer.self_attn.q_norm.weight.copy_(w["q_norm"])
        layer.self_attn.k_norm.weight.copy_(w["k_norm"])
        layer.input_layernorm.weight.copy_(w["input_layernorm"])
        layer.post_attention_layernorm.weight.copy_(w["post_attention_layernorm"])
    pool = torch.stack([_to_fp8(kq), _to_fp8(vq)])[:, None].to(dev)
    attn_in = AttnInputs(slot_mapping=slots.to(dev), is_prefill=False,
                         cache_seqlens=torch.tensor(ctx, dtype=torch.int32, device=dev), block_tables=bt.to(dev))
    captured = {}
    orig = layer.self_attn.attn.forward

    def spy(q, k, v, a):
        captured["attn"] = orig(q, k, v, a)
        return captured["attn"]

    layer.self_attn.attn.forward = spy
    with torch.no_grad(), attention_context(AttnMetadata(pool, k_scale=ks, v_scale=vs)):
        h, res = layer(pos.to(dev), hidden.to(dev), None, attn_in)
    torch.cuda.synchronize()
    cs = O.build_cos_sin_cache(D, 4096, 1e6)
    wn = {k2: f32(v2) for k2, v2 in w.items()}
    kcn, vcn = O.dequantize_fp8(kq, ks), O.dequantize_fp8(vq, vs)
    ref = OM.decode_layer(wn, f32(hidden), None, pos.numpy(), kcn, vcn, bt.numpy(), np.array(ctx), slots.numpy(), cs,
                          HQ, HKV, D, EPS, kv_fp8=(ks, vs))
    _close(f32(captured["attn"]), ref["attn"])
    h_ref, r_ref = OM.post_attention(wn, f32(captured["attn"]), f32(hidden), EPS)
    _close(f32(h), h_ref)
    _close(f32(res), r_ref)
