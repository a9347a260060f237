"""Shared-prefix (cascade) decode attention on the GPU, through the C ABI:
groups of rows whose block tables share leading blocks read those blocks
once per group (prefix pass) and merge with their own suffix.  Checked
against the numpy oracle (plain paged decode over each row's whole table)
and against the plain decode kernel on the same inputs, for several group
layouts, block sizes and GQA groups, including a row whose suffix is empty,
rows outside every group, empty trailing groups, and decode graphs that
carry the cascade plan."""

import numpy as np
import pytest
import torch

import oracle.ops as O
from helpers import f32, gen, randn_bf16

pytestmark = pytest.mark.gpu


def _close(got, want, rtol=2e-2, atol=2e-2):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert np.isfinite(got).all()
    err = np.abs(got - want) - (atol + rtol * np.abs(want))
    assert (err <= 0).all(), f"max excess {err.max():.4g} at {np.unravel_index(err.argmax(), err.shape)}"


def _shared_case(g, ctx, shares, block, pool_extra=4):
    """Block tables where the rows of each (rows, n_blocks) in `shares` start
    with the same n_blocks pages; every other page distinct."""
    bsz = len(ctx)
    need = [(c + block - 1) // block for c in ctx]
    width = max(need)
    total = sum(need) + pool_extra
    perm = torch.randperm(total, generator=g).tolist()
    bt = torch.full((bsz, width), -1, dtype=torch.int32)
    o = 0
    for b, n in enumerate(need):
        bt[b, :n] = torch.tensor(perm[o : o + n], dtype=torch.int32)
        o += n
    for rows, n in shares:
        for r in rows[1:]:
            bt[r, :n] = bt[rows[0], :n]
    return bt, total


def _plan(bt, ctx, block, dev, groups=4, max_prefix_blocks=None, min_blocks=1, max_rows=16):
    from xvllm.layers.attention import CascadePlan
    from xvllm.prefix_cache import cascade_groups

    mp = max_prefix_blocks or bt.shape[1]
    pre, info, rows = cascade_groups(bt.numpy(), np.asarray(ctx), block, max_rows=max_rows, min_blocks=min_blocks,
                                     max_groups=groups, max_prefix_blocks=mp)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)
    rows_t = t(rows) if len(rows) else torch.zeros(1, dtype=torch.int32, device=dev)
    return CascadePlan(t(pre), t(info), rows_t, groups, mp), pre


@pytest.mark.parametrize(
    "hq,hkv,block,ctx,shares",
    [
        # G 4, 16-token blocks: a 5-row group over 20 blocks (row 2's suffix empty), a 3-row group, loners
        (32, 8, 16, [500, 700, 320, 321, 1000, 150, 130, 200, 77, 1, 0, 640],
         [([0, 1, 2, 3, 4], 20), ([5, 6, 7], 7)]),
        # G 8 (Qwen3-32B heads), 256-token blocks
        (64, 8, 256, [600, 1024, 513, 700, 2000, 300], [([0, 1, 2, 3], 2), ([4, 5], 1)]),
        # G 2, a group of 40 rows: cut into runs of 128 / G = 64 -> one group; and an odd block size
        (16, 8, 48, [100 + 7 * i for i in range(40)], [(list(range(40)), 2)]),
        # MHA, one group, blocks of 32
        (8, 8, 32, [96, 200, 64, 65], [([0, 1, 2, 3], 2)]),
    ],
)
def test_cascade_decode_matches_oracle_and_plain_decode(dev, hq, hkv, block, ctx, shares):
    from xvllm.layers.attention import cascade_decode_attention, paged_decode_attention

    print(f"cascade hq {hq} hkv {hkv} block {block} B {len(ctx)}", flush=True)
    g = gen(hq * block + len(ctx))
    d = 128
    bt, pool = _shared_case(g, ctx, shares, block)
    kc, vc = randn_bf16((pool, block, hkv, d), g), randn_bf16((pool, block, hkv, d), g)
    q = randn_bf16((len(ctx), hq, d), g)
    sl = torch.tensor(ctx, dtype=torch.int32)
    plan, pre = _plan(bt, ctx, block, dev, max_rows=128 // (hq // hkv))
    assert (pre > 0).sum() >= 2
    args = (q.view(len(ctx), -1).to(dev), kc.to(dev), vc.to(dev), bt.to(dev), sl.to(dev))
    out = cascade_decode_attention(*args, plan, hq, hkv, d)
    plain = paged_decode_attention(*args, hq, hkv, d)
    torch.cuda.synchronize()
    want = O.paged_decode_attention(f32(q), f32(kc), f32(vc), bt.numpy(), sl.numpy())
    _close(f32(out).reshape(len(ctx), hq, d), want)
    _close(f32(out), f32(plain), rtol=1e-2, atol=1e-2)
    assert (f32(out)[np.asarray(ctx) == 0] == 0).all()


CASES = [
    (32, 8, 16, [500, 700, 320, 321, 1000, 150, 130, 200, 77, 1, 0, 640], [([0, 1, 2, 3, 4], 20), ([5, 6, 7], 7)]),
    (64, 8, 256, [600, 1024, 513, 700, 2000, 300], [([0, 1, 2, 3], 2), ([4, 5], 1)]),
    (16, 8, 48, [100 + 7 * i for i in range(40)], [(list(range(40)), 2)]),
    (8, 8, 32, [96, 200, 64, 65], [([0, 1, 2, 3], 2)]),
]


@pytest.mark.parametrize("layout", ["nhd", "hnd"])
@pytest.mark.parametrize("hq,hkv,block,ctx,shares", CASES)
def test_cascade_decode_fp8_matches_oracle_and_plain_decode(dev, hq, hkv, block, ctx, shares, layout):
    """fp8 (e4m3fn) pages: the cascade against the oracle over the
    dequantized pages and against the plain fp8 decode, both page orders."""
    from xvllm.layers.attention import cascade_decode_attention, paged_decode_attention

    print(f"cascade fp8 {layout} hq {hq} hkv {hkv} block {block} B {len(ctx)}", flush=True)
    g = gen(7 * hq + block + len(ctx))
    d, ks, vs = 128, 0.05, 0.3
    bt, pool = _shared_case(g, ctx, shares, block)
    kc, vc = randn_bf16((pool, block, hkv, d), g), randn_bf16((pool, block, hkv, d), g)
    kq = O.quantize_fp8(f32(kc), np.float32(1.0) / np.float32(ks))
    vq = O.quantize_fp8(f32(vc), np.float32(1.0) / np.float32(vs))

    def on_dev(codes):
        t = torch.from_numpy(np.ascontiguousarray(codes)).view(torch.float8_e4m3fn).to(dev)
        return t.transpose(1, 2).contiguous().transpose(1, 2) if layout == "hnd" else t

    q = randn_bf16((len(ctx), hq, d), g)
    sl = torch.tensor(ctx, dtype=torch.int32)
    plan, pre = _plan(bt, ctx, block, dev, max_rows=128 // (hq // hkv))
    assert (pre > 0).sum() >= 2
    args = (q.view(len(ctx), -1).to(dev), on_dev(kq), on_dev(vq), bt.to(dev), sl.to(dev))
    out = cascade_decode_attention(*args, plan, hq, hkv, d, k_scale=ks, v_scale=vs)
    plain = paged_decode_attention(*args, hq, hkv, d, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    want = O.paged_decode_attention(f32(q), O.dequantize_fp8(kq, ks), O.dequantize_fp8(vq, vs), bt.numpy(),
                                    sl.numpy())
    _close(f32(out).reshape(len(ctx), hq, d), want)
    _close(f32(out), f32(plain), rtol=1e-2, atol=1e-2)
    assert (f32(out)[np.asarray(ctx) == 0] == 0).all()


def test_cascade_empty_groups_and_no_groups(dev):
    """A plan with only trailing empty groups (no row shares anything) and a
    plan whose one group is followed by empty ones: both equal the plain decode."""
    from xvllm.layers.attention import cascade_decode_attention, paged_decode_attention

    g = gen(31)
    hq, hkv, d, block = 32, 8, 128, 16
    ctx = [300, 40, 900, 17]
    for shares in ([], [([0, 2], 10)]):
        bt, pool = _shared_case(g, ctx, shares, block)
        kc, vc = randn_bf16((pool, block, hkv, d), g), randn_bf16((pool, block, hkv, d), g)
        q = randn_bf16((len(ctx), hq, d), g)
        sl = torch.tensor(ctx, dtype=torch.int32)
        plan, pre = _plan(bt, ctx, block, dev, groups=3)
        assert (pre > 0).sum() == (2 if shares else 0)
        args = (q.view(len(ctx), -1).to(dev), kc.to(dev), vc.to(dev), bt.to(dev), sl.to(dev))
        out = cascade_decode_attention(*args, plan, hq, hkv, d)
        plain = paged_decode_attention(*args, hq, hkv, d)
        torch.cuda.synchronize()
        _close(f32(out), f32(plain), rtol=1e-2, atol=1e-2)


def test_cascade_config5_full_size(dev):
    """Config 5's attention: B 32 x 32768, rows 0..15 sharing 512 blocks of
    16 tokens (8192 tokens), group 8; cascade against the plain decode on
    every row and the oracle on rows from both halves."""
    from test_gpu_config5 import BSZ, CTX, HKV, HQ, config5_block_tables
    from xvllm.layers.attention import cascade_decode_attention, paged_decode_attention

    bt, unique = config5_block_tables()
    g = torch.Generator(device=dev).manual_seed(9)
    d = 128
    kc = torch.randn((unique, 16, HKV, d), generator=g, device=dev).to(torch.bfloat16)
    vc = torch.randn((unique, 16, HKV, d), generator=g, device=dev).to(torch.bfloat16)
    q = torch.randn((BSZ, HQ * d), generator=g, device=dev).to(torch.bfloat16)
    sl = torch.full((BSZ,), CTX, dtype=torch.int32)
    plan, pre = _plan(bt, [CTX] * BSZ, 16, dev, groups=2, max_prefix_blocks=512, min_blocks=16)
    assert pre[:16].tolist() == [8192] * 16 and not pre[16:].any()
    btd, sld = bt.to(dev), sl.to(dev)
    out = cascade_decode_attention(q, kc, vc, btd, sld, plan, HQ, HKV, d)
    plain = paged_decode_attention(q, kc, vc, btd, sld, HQ, HKV, d)
    torch.cuda.synchronize()
    _close(f32(out), f32(plain), rtol=1e-2, atol=1e-2)
    for r in (0, 15, 16):
        pages = btd[r].long()
        want = O.paged_decode_attention(f32(q[r : r + 1].cpu()).reshape(1, HQ, d), f32(kc[pages].cpu()),
                                        f32(vc[pages].cpu()), np.arange(CTX // 16, dtype=np.int32)[None, :],
                                        np.array([CTX]))
        _close(f32(out[r : r + 1].cpu()).reshape(1, HQ, d), want)


def test_cascade_config5_full_size_fp8(dev):
    """Config 5's attention on fp8 pages (scales 0.125): cascade against the
    plain fp8 decode on every row and the oracle over the dequantized pages on
    rows from both halves."""
    from test_gpu_config5 import BSZ, CTX, HKV, HQ, config5_block_tables
    from xvllm.layers.attention import cascade_decode_attention, paged_decode_attention

    bt, unique = config5_block_tables()
    g = torch.Generator(device=dev).manual_seed(10)
    d, sc = 128, 0.125
    kc = (torch.randn((unique, 16, HKV, d), generator=g, device=dev) / sc).to(torch.float8_e4m3fn)
    vc = (torch.randn((unique, 16, HKV, d), generator=g, device=dev) / sc).to(torch.float8_e4m3fn)
    q = torch.randn((BSZ, HQ * d), generator=g, device=dev).to(torch.bfloat16)
    sl = torch.full((BSZ,), CTX, dtype=torch.int32)
    plan, pre = _plan(bt, [CTX] * BSZ, 16, dev, groups=2, max_prefix_blocks=512, min_blocks=16)
    assert pre[:16].tolist() == [8192] * 16 and not pre[16:].any()
    btd, sld = bt.to(dev), sl.to(dev)
    out = cascade_decode_attention(q, kc, vc, btd, sld, plan, HQ, HKV, d, k_scale=sc, v_scale=sc)
    plain = paged_decode_attention(q, kc, vc, btd, sld, HQ, HKV, d, k_scale=sc, v_scale=sc)
    torch.cuda.synchronize()
    _close(f32(out), f32(plain), rtol=1e-2, atol=1e-2)
    for r in (0, 15, 16):
        pages = btd[r].long()
        kr = O.dequantize_fp8(kc[pages].cpu().view(torch.uint8).numpy(), sc)
        vr = O.dequantize_fp8(vc[pages].cpu().view(torch.uint8).numpy(), sc)
        want = O.paged_decode_attention(f32(q[r : r + 1].cpu()).reshape(1, HQ, d), kr, vr,
                                        np.arange(CTX // 16, dtype=np.int32)[None, :], np.array([CTX]))
        _close(f32(out[r : r + 1].cpu()).reshape(1, HQ, d), want)


@pytest.mark.parametrize("kv_dtype", ["bf16", "fp8"])
def test_cascade_decode_graphs_match_eager(dev, kv_dtype):
    """A 2-layer model whose decode batch shares prefixes (rows 0..5 the same
    12 blocks): the runner's decode graphs carry the cascade plan; replays
    equal eager runs and equal a runner without cascade within bf16
    tolerance (relative L2 after two layers); a batch with no sharing runs
    through the same graphs.  Also on an fp8 pool (scales 0.25)."""
    from xvllm.batch import SeqSchedule
    from xvllm.config import Qwen3Shape
    from xvllm.kv_pool import KVPool
    from xvllm.model_runner import ModelRunner
    from xvllm.models import Qwen3ForCausalLM

    cfg = Qwen3Shape(1024, 16, 8, 128, 3072, 2, vocab_size=4096, max_position_embeddings=4096)
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(dev):
            model = Qwen3ForCausalLM(cfg).random_init_(seed=4)
            if kv_dtype == "fp8":
                kv = KVPool(cfg, num_blocks=600, block_size=16, device=dev, dtype=torch.float8_e4m3fn,
                            k_scale=0.25, v_scale=0.25)
            else:
                kv = KVPool(cfg, num_blocks=600, block_size=16, device=dev, dtype=torch.bfloat16)
    finally:
        torch.set_default_dtype(torch.float32)
    if kv_dtype == "fp8":
        kv.kv_cache.copy_((torch.randn(kv.kv_cache.shape, device=dev) * 4).to(torch.float8_e4m3fn))
    else:
        kv.kv_cache.normal_()
    casc = ModelRunner(model, kv, max_num_seqs=16, context_len=1024, device=dev, cascade_groups=2,
                       cascade_max_prefix_blocks=32, cascade_min_blocks=4, cascade_min_shared_bytes=0)
    gated = ModelRunner(model, kv, max_num_seqs=16, context_len=1024, device=dev, cascade_groups=2,
                        cascade_max_prefix_blocks=32, cascade_min_blocks=4)
    plain = ModelRunner(model, kv, max_num_seqs=16, context_len=1024, device=dev)
    g = gen(17)
    for step, (bs, shared) in enumerate(((9, 6), (4, 0), (13, 6))):
        perm = torch.randperm(600, generator=g).tolist()
        prefix = perm[:12]
        seqs, o = [], 12
        for i in range(bs):
            c = int(torch.randint(200, 400, (1,), generator=g))
            n = (c + 15) // 16
            btab = prefix + perm[o : o + n - 12] if i < shared else perm[o : o + n]
            o += n
            seqs.append(SeqSchedule(seq_id=100 * step + i, token_ids=[int(torch.randint(0, 4096, (1,), generator=g))],
                                    num_cached_tokens=c - 1, block_table=btab))
        snap = kv.kv_cache.clone()
        # the default gate: 12 shared blocks are far below the bytes where the cascade pays
        gated.batch.build_decode(seqs, pad_to=gated.graph_runner._pad_bs(bs))
        assert gated.batch.cascade_rows == 0 and not gated._use_cascade()
        casc.batch.build_decode(seqs, pad_to=casc.graph_runner._pad_bs(bs))
        assert casc.batch.cascade_rows == shared and casc._use_cascade() == (shared > 0)
        h_graph = casc.decode_hidden(bs).clone()
        torch.cuda.synchronize()
        kv.kv_cache.copy_(snap)
        with torch.inference_mode():
            h_eager = casc._decode_body(bs)[:bs].clone()
        torch.cuda.synchronize()
        assert torch.equal(h_graph, h_eager), f"step {step}: cascade graph replay differs from eager"
        kv.kv_cache.copy_(snap)
        plain.batch.build_decode(seqs, pad_to=plain.graph_runner._pad_bs(bs))
        h_plain = plain.decode_hidden(bs).clone()
        torch.cuda.synchronize()
        # two layers of bf16 rounding after attention outputs that differ in
        # fp32 summation order: compared in relative L2 (the attention itself
        # is checked element by element above)
        hg, hp = f32(h_graph).astype(np.float64), f32(h_plain).astype(np.float64)
        assert np.linalg.norm(hg - hp) / np.linalg.norm(hp) < 1e-2, step
    casc.destroy()
    gated.destroy()
    plain.destroy()
