"""Config 1 (Qwen3-0.6B-shaped single decoder layer, one decode step, B 8,
ctx U[128,512], 16-token pages from a random permutation of a 512-page pool)
through the xvllm model code against the numpy oracle; and the decode body
under hipGraph replay against eager execution."""
import numpy as np
import pytest
import torch

import oracle.model as OM
import oracle.ops as O
from helpers import f32, gen, randn_bf16

pytestmark = pytest.mark.gpu

HIDDEN, HQ, HKV, D, FFN, V, EPS = 1024, 16, 8, 128, 3072, 151936, 1e-6


def _close(got, want, rtol=2e-2, atol=2e-2):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert np.isfinite(got).all()
    ok = np.abs(got - want) <= atol + rtol * np.abs(want)
    assert ok.all(), f"{(~ok).sum()} of {ok.size} outside tolerance, max err {np.abs(got - want).max():.3g}"


def _layer_case(seed=0, bsz=8):
    g = gen(seed)
    ctx = torch.randint(128, 513, (bsz,), generator=g).tolist()
    pool = 512
    perm = torch.randperm(pool, generator=g)
    need = [(c + 15) // 16 for c in ctx]
    bt = torch.full((bsz, max(need)), -1, dtype=torch.int32)
    o = 0
    for b, n in enumerate(need):
        bt[b, :n] = perm[o : o + n].to(torch.int32)
        o += n
    w = {
        "qkv_proj": randn_bf16(((HQ + 2 * HKV) * D, HIDDEN), g, 0.02),
        "o_proj": randn_bf16((HIDDEN, HQ * D), g, 0.02),
        "gate_up_proj": randn_bf16((2 * FFN, HIDDEN), g, 0.02),
        "down_proj": randn_bf16((HIDDEN, FFN), g, 0.02),
        "q_norm": randn_bf16((D,), g, 0.1, 1.0),
        "k_norm": randn_bf16((D,), g, 0.1, 1.0),
        "input_layernorm": randn_bf16((HIDDEN,), g, 0.1, 1.0),
        "post_attention_layernorm": randn_bf16((HIDDEN,), g, 0.1, 1.0),
        "norm": randn_bf16((HIDDEN,), g, 0.1, 1.0),
        "lm_head": randn_bf16((V, HIDDEN), g, 0.02),
    }
    kc = randn_bf16((pool, 16, HKV, D), g)
    vc = randn_bf16((pool, 16, HKV, D), g)
    hidden = randn_bf16((bsz, HIDDEN), g)
    pos = torch.tensor([c - 1 for c in ctx], dtype=torch.int64)
    slots = torch.tensor([int(bt[b, p // 16]) * 16 + p % 16 for b, p in enumerate(pos.tolist())], dtype=torch.int32)
    return ctx, bt, w, kc, vc, hidden, pos, slots


def test_config1_single_layer_decode(dev):
    from xvllm.config import Qwen3Shape
    from xvllm.layers.attention import AttnInputs, AttnMetadata, attention_context
    from xvllm.layers.rotary import build_cos_sin_cache
    from xvllm.models.qwen3 import Qwen3DecoderLayer
    from xvllm.sampler import sample

    ctx, bt, w, kc, vc, hidden, pos, slots = _layer_case()
    cfg = Qwen3Shape(HIDDEN, HQ, HKV, D, FFN, 1, max_position_embeddings=4096)
    with torch.device(dev):
        layer = Qwen3DecoderLayer(cfg, 0).to(torch.bfloat16)
        layer.self_attn.rotary_emb.cos_sin_cache = build_cos_sin_cache(D, 4096, 1e6).to(dev)
    with torch.no_grad():
        layer.self_attn.qkv_proj.copy_(w["qkv_proj"])
        layer.self_attn.o_proj.copy_(w["o_proj"])
        layer.mlp.gate_up_proj.copy_(w["gate_up_proj"])
        layer.mlp.down_proj.copy_(w["down_proj"])
        layer.self_attn.q_norm.weight.copy_(w["q_norm"])
        layer.self_attn.k_norm.weight.copy_(w["k_norm"])
        layer.input_layernorm.weight.copy_(w["input_layernorm"])
        layer.post_attention_layernorm.weight.copy_(w["post_attention_layernorm"])
    pool = torch.stack([kc, vc])[:, None].to(dev)  # [2, 1 layer, NB, BS, Hkv, D]
    attn_in = AttnInputs(slot_mapping=slots.to(dev), is_prefill=False, cache_seqlens=torch.tensor(ctx, dtype=torch.int32, device=dev),
                         block_tables=bt.to(dev))
    captured = {}
    orig = layer.self_attn.attn.forward

    def spy(q, k, v, a):
        captured["attn"] = orig(q, k, v, a)
        return captured["attn"]

    layer.self_attn.attn.forward = spy
    with torch.no_grad(), attention_context(AttnMetadata(pool)):
        h, res = layer(pos.to(dev), hidden.to(dev), None, attn_in)
        norm_w = w["norm"].to(dev)
        x = h.clone()
        r = res.clone()
        torch.ops.vllm.fused_add_rmsnorm(x, r, norm_w, EPS)
        logits = torch.nn.functional.linear(x, w["lm_head"].to(dev))
        ids = sample(logits, None, all_greedy=True)
    torch.cuda.synchronize()

    cs = O.build_cos_sin_cache(D, 4096, 1e6)
    kcn, vcn = f32(kc), f32(vc)
    wn = {k2: f32(v2) for k2, v2 in w.items()}
    ref = OM.decode_layer(wn, f32(hidden), None, pos.numpy(), kcn, vcn, bt.numpy(), np.array(ctx), slots.numpy(), cs,
                          HQ, HKV, D, EPS)
    # 1. attention output: the oracle's whole layer up to attention (q/k norm,
    #    RoPE, store, paged decode) from the same inputs, every element
    _close(f32(captured["attn"]), ref["attn"])
    # 2. layer output and residual: the oracle's post-attention block on the
    #    device's attention output (so bf16 rounding differences of the
    #    attention do not compound into the MLP), every element
    h_ref, r_ref = OM.post_attention(wn, f32(captured["attn"]), f32(hidden), EPS)
    _close(f32(h), h_ref)
    _close(f32(res), r_ref)
    # 3. final norm and LM head on the device's layer output, every element
    xr, logits_r = OM.final_logits(f32(h), f32(res), wn["norm"], wn["lm_head"], EPS)
    _close(f32(x), xr)
    _close(f32(logits), OM.linear(f32(x), wn["lm_head"]))
    # 4. end to end, the whole chain against the oracle's own chain
    xr_e2e, _ = OM.final_logits(ref["hidden"], ref["residual"], wn["norm"], wn["lm_head"], EPS)
    rel = np.linalg.norm(f32(x) - xr_e2e) / np.linalg.norm(xr_e2e)
    assert rel < 1e-2, f"end-to-end relative L2 error {rel:.3g}"
    # 5. the KV store wrote this step's V (the oracle's V from its own GEMM:
    #    equal up to the bf16 rounding of the qkv product)
    np.testing.assert_allclose(f32(pool[1, 0]).reshape(-1, HKV, D)[slots.numpy()],
                               vcn.reshape(-1, HKV, D)[slots.numpy()], rtol=1e-2, atol=1e-2)
    # 6. greedy ids of every row bit-exact: the C oracle sampler on the device's logits
    import oracle.sampler as S

    bits = logits.view(torch.int16).cpu().numpy().view(np.uint16)
    want = S.sample(bits, None, None, None, None, None, 1)
    assert np.array_equal(ids.cpu().numpy(), want), f"{ids.cpu().numpy()} vs {want}"
    # and the oracle's own logits pick the same token where their top-2 margin exceeds the tolerance
    top2 = np.sort(logits_r, axis=1)[:, -2:]
    sure = (top2[:, 1] - top2[:, 0]) > 0.05
    assert np.array_equal(ids.cpu().numpy()[sure], np.argmax(logits_r, axis=1)[sure])


@pytest.mark.parametrize("m", [1, 5, 17, 64])
def test_config1_streamed_post_attention(dev, m):
    """The weight-streaming decode GEMMs (packed o, gate_up + SiLU, down as
    split-K partials into the norms) on the config-1 layer, every element
    against the oracle's post-attention block on the same inputs, at decode
    batches 1, 5, 17 and 64; and an in-place weight write after packing
    raises instead of reading the stale packed copy."""
    from xvllm.config import Qwen3Shape
    from xvllm.layers.linear import PartialSums
    from xvllm.models.qwen3 import Qwen3DecoderLayer, StalePackedWeights

    _, _, w, _, _, _, _, _ = _layer_case(seed=m)
    g = gen(100 + m)
    attn = randn_bf16((m, HQ * D), g)
    hidden = randn_bf16((m, HIDDEN), g)
    cfg = Qwen3Shape(HIDDEN, HQ, HKV, D, FFN, 1, max_position_embeddings=4096)
    with torch.device(dev):
        layer = Qwen3DecoderLayer(cfg, 0).to(torch.bfloat16)
    with torch.no_grad():
        layer.self_attn.o_proj.copy_(w["o_proj"])
        layer.mlp.gate_up_proj.copy_(w["gate_up_proj"])
        layer.mlp.down_proj.copy_(w["down_proj"])
        layer.post_attention_layernorm.weight.copy_(w["post_attention_layernorm"])
    layer.self_attn.pack()
    layer.mlp.pack()
    assert layer.self_attn.packed_o is not None and layer.mlp.packed is not None
    from xvllm.layers.linear import streamed_into_norm

    with torch.no_grad():
        a, res = attn.to(dev), hidden.to(dev).clone()
        o = streamed_into_norm(a, layer.self_attn.packed_o)
        assert isinstance(o, PartialSums)
        x, res = layer.post_attention_layernorm(o, res)
        h = layer.mlp(x)
        assert isinstance(h, PartialSums), "the MLP did not take the streamed path"
        h = h.materialize()
    torch.cuda.synchronize()
    wn = {k2: f32(v2) for k2, v2 in w.items()}
    h_ref, r_ref = OM.post_attention(wn, f32(attn), f32(hidden), EPS)
    _close(f32(res), r_ref)
    _close(f32(h), h_ref)
    with torch.no_grad():
        layer.mlp.down_proj.mul_(1.0)  # an in-place write after packing
        with pytest.raises(StalePackedWeights):
            layer.mlp(x)


def test_decode_graph_replay_matches_eager(dev):
    """A 2-layer random Qwen3-0.6B-shaped model: hipGraph replays of the decode
    body (several, with eager work and new metadata in between) equal eager runs."""
    from xvllm.batch import SeqSchedule
    from xvllm.config import Qwen3Shape
    from xvllm.kv_pool import KVPool
    from xvllm.model_runner import ModelRunner
    from xvllm.models import Qwen3ForCausalLM

    cfg = Qwen3Shape(HIDDEN, HQ, HKV, D, FFN, 2, vocab_size=4096, max_position_embeddings=4096)
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(dev):
            model = Qwen3ForCausalLM(cfg).random_init_(seed=1)
            kv = KVPool(cfg, num_blocks=256, block_size=16, device=dev, dtype=torch.bfloat16)
    finally:
        torch.set_default_dtype(torch.float32)
    kv.kv_cache.normal_()
    runner = ModelRunner(model, kv, max_num_seqs=16, context_len=1024, device=dev)
    g = gen(5)
    for step in range(3):
        bsz = [5, 16, 3][step]
        perm = torch.randperm(256, generator=g).tolist()
        seqs = []
        for i in range(bsz):
            c = int(torch.randint(1, 200, (1,), generator=g))
            n = (c + 15) // 16
            seqs.append(SeqSchedule(seq_id=100 * step + i, token_ids=[int(torch.randint(0, 4096, (1,), generator=g))],
                                    num_cached_tokens=c - 1, block_table=perm[i * 13 : i * 13 + n]))
        pad = runner.graph_runner._pad_bs(bsz)
        runner.batch.build_decode(seqs, pad_to=pad)
        snapshot = kv.kv_cache.clone()
        g_hidden = runner.decode_hidden(bsz).clone()
        torch.cuda.synchronize()
        kv.kv_cache.copy_(snapshot)
        with torch.inference_mode():
            e_hidden = runner._decode_body(bsz)[:bsz].clone()
        torch.cuda.synchronize()
        assert torch.equal(g_hidden, e_hidden), f"step {step}: graph replay differs from eager"
        assert torch.isfinite(g_hidden.float()).all()
    runner.destroy()


def test_serving_loop_reads_back_the_sampled_ids(dev):
    """A few continuous-batching steps of a 2-layer random Qwen3-shaped model
    (prefill chunks, then decode rows with a prefill in the same step): every
    id read back on the host equals the id sampled on the device in that step,
    and decode steps feed them back as input.  Regression: the side-stream D2H
    copy of the ids must be ordered after their join on the compute stream."""
    from xvllm.batch import SeqSchedule
    from xvllm.config import Qwen3Shape
    from xvllm.kv_pool import KVPool
    from xvllm.model_runner import ModelRunner
    from xvllm.models import Qwen3ForCausalLM

    V = 4096
    cfg = Qwen3Shape(HIDDEN, HQ, HKV, D, FFN, 2, vocab_size=V, max_position_embeddings=4096)
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(dev):
            model = Qwen3ForCausalLM(cfg).random_init_(seed=3)
            kv = KVPool(cfg, num_blocks=512, block_size=16, device=dev, dtype=torch.bfloat16)
    finally:
        torch.set_default_dtype(torch.float32)
    runner = ModelRunner(model, kv, max_num_seqs=32, max_num_batched_tokens=2048, context_len=1024, device=dev)
    staged = {}
    orig = runner._stage_samples

    def spy(p, d):  # keep the device-side ids of the step
        staged["p"] = None if p is None else p.clone()
        staged["d"] = None if d is None else d.clone()
        return orig(p, d)

    runner._stage_samples = spy
    g = gen(9)
    free = list(range(512))
    seqs = []
    for i in range(12):
        n = int(torch.randint(20, 120, (1,), generator=g))
        seqs.append(dict(id=i, toks=torch.randint(0, V, (n,), generator=g).tolist(), cached=0, bt=[]))
    busy = torch.randn(4096, 4096, device=dev)
    for step in range(12):
        decodes, prefills = [], []
        for s in seqs:
            if s["cached"] >= len(s["toks"]) - 1 and s["cached"] > 0:  # prompt done: decode the last token
                if (s["cached"] + 1 + 15) // 16 > len(s["bt"]):
                    s["bt"].append(free.pop())
                decodes.append(SeqSchedule(s["id"], [s["toks"][-1]], s["cached"], list(s["bt"])))
        for s in seqs[: 4 + step]:
            if s["cached"] == 0:  # whole prompt as one prefill chunk
                s["bt"] = [free.pop() for _ in range((len(s["toks"]) + 15) // 16)]
                prefills.append(SeqSchedule(s["id"], s["toks"], 0, list(s["bt"])))
        for _ in range(6):  # a busy compute stream makes a misordered copy visible
            busy = busy @ busy * 1e-3
        n_p, n_d = runner.run_forward(decodes, prefills)
        p_ids, d_ids = runner.read_samples(n_p, n_d)
        torch.cuda.synchronize()
        want_d = [] if staged["d"] is None else staged["d"].view(-1).tolist()
        want_p = [] if staged["p"] is None else staged["p"].view(-1).tolist()
        assert d_ids == want_d and p_ids == want_p, f"step {step}"
        assert all(0 <= t < V for t in d_ids + p_ids)
        for s, t in zip(decodes, d_ids):
            rec = seqs[s.seq_id]
            rec["cached"] += 1
            rec["toks"].append(t)
        for s, t in zip(prefills, p_ids):
            rec = seqs[s.seq_id]
            rec["cached"] = len(rec["toks"])
            rec["toks"].append(t)
    runner.destroy()
