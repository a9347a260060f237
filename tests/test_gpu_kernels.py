"""GPU parity of every hot-path kernel against the CPU oracle, through the
C ABI (xvllm ops are thin ctypes wrappers).  Tolerances: bit-exact for the KV
store; rtol/atol 2e-2 (bf16 output, fp32 accumulate) for attention and norms."""
import math

import numpy as np
import pytest
import torch

import oracle.ops as O
import xvllm.layers.ops  # noqa: F401  (registers the vllm:: and xv:: ops)
from helpers import f32, gen, make_paged, randn_bf16

pytestmark = pytest.mark.gpu

RTOL = ATOL = 2e-2


def _close(got, want, rtol=RTOL, atol=ATOL):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert np.isfinite(got).all(), "non-finite output"
    err = np.abs(got - want) - (atol + rtol * np.abs(want))
    assert (err <= 0).all(), f"max excess {err.max():.4g} at {np.unravel_index(err.argmax(), err.shape)}"


@pytest.mark.parametrize(
    "n,hkv,d,strided",
    [(37, 8, 128, False), (64, 8, 128, True), (5, 2, 64, False), (7, 4, 128, False), (1, 8, 128, True)],
)
def test_store_kvcache_bitexact(dev, n, hkv, d, strided):
    from xvllm.kv_ops import store_kvcache

    g = gen(1)
    nb, page = 16, 16
    if strided:  # k/v as views of a fused qkv row, like Qwen3Attention
        qkv = randn_bf16((n, (32 + 2 * hkv) * d), g)
        key = qkv[:, 32 * d : (32 + hkv) * d].view(n, hkv, d)
        val = qkv[:, (32 + hkv) * d :].view(n, hkv, d)
    else:
        key, val = randn_bf16((n, hkv, d), g), randn_bf16((n, hkv, d), g)
    slots = torch.randperm(nb * page, generator=g)[:n].to(torch.int32)
    slots[::7] = -1
    kc = randn_bf16((nb, page, hkv, d), g)
    vc = randn_bf16((nb, page, hkv, d), g)
    kc_ref, vc_ref = kc.clone(), vc.clone()
    O.store_kvcache(key, val, kc_ref, vc_ref, slots)  # torch tensors index like numpy here
    kg, vg = kc.to(dev), vc.to(dev)
    store_kvcache(key.to(dev), val.to(dev), kg.view(-1, hkv, d), vg.view(-1, hkv, d), slots.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(kg.cpu().view(torch.int16), kc_ref.view(torch.int16))
    assert torch.equal(vg.cpu().view(torch.int16), vc_ref.view(torch.int16))


@pytest.mark.parametrize(
    "hq,hkv,ctx",
    [
        (32, 8, [1, 17, 300, 513, 16, 2048, 0, 77]),  # Qwen3-8B heads, pad row (0)
        (16, 8, [128, 511, 256, 300]),                 # Qwen3-0.6B heads (group 2)
        (64, 8, [1000, 33, 4096]),                     # Qwen3-32B heads (group 8)
        (8, 8, [5, 260]),                              # MHA
    ],
)
def test_paged_decode_attention(dev, hq, hkv, ctx):
    from xvllm.layers.attention import paged_decode_attention

    g = gen(hq + len(ctx))
    d = 128
    need = sum((c + 15) // 16 for c in ctx)
    kc, vc, bt, sl = make_paged(ctx, int(need * 1.25) + 4, hkv, d, g)
    q = randn_bf16((len(ctx), hq, d), g)
    want = O.paged_decode_attention(f32(q), f32(kc), f32(vc), bt.numpy(), sl.numpy())
    out = paged_decode_attention(q.view(len(ctx), -1).to(dev), kc.to(dev), vc.to(dev), bt.to(dev), sl.to(dev), hq, hkv, d)
    torch.cuda.synchronize()
    _close(f32(out).reshape(len(ctx), hq, d), want)


def test_paged_decode_config2_full_size(dev):
    """Config 2 at full size (B 64, ctx U[512,4096]); a sample of rows is
    checked against the oracle, every row for finiteness."""
    from xvllm.layers.attention import paged_decode_attention

    g = gen(2024)
    ctx = torch.randint(512, 4097, (64,), generator=g).tolist()
    need = sum((c + 15) // 16 for c in ctx)
    kc, vc, bt, sl = make_paged(ctx, math.ceil(need * 1.25), 8, 128, g, fill_nan=False)
    q = randn_bf16((64, 32, 128), g)
    out = paged_decode_attention(q.view(64, -1).to(dev), kc.to(dev), vc.to(dev), bt.to(dev), sl.to(dev), 32, 8, 128)
    got = f32(out).reshape(64, 32, 128)
    rows = [0, 17, 63]
    want = O.paged_decode_attention(f32(q)[rows], f32(kc), f32(vc), bt.numpy()[rows], sl.numpy()[rows])
    _close(got[rows], want)
    assert np.isfinite(got).all()


def test_paged_decode_many_short_sequences(dev):
    """256 sequences of 0..40 tokens: wave ranges cross many segments shorter
    than the page pipeline, with empty (padding) rows among them."""
    from xvllm.layers.attention import paged_decode_attention

    g = gen(77)
    ctx = torch.randint(0, 41, (256,), generator=g).tolist()
    ctx[5] = ctx[200] = 0
    need = sum((c + 15) // 16 for c in ctx)
    kc, vc, bt, sl = make_paged(ctx, int(need * 1.25) + 4, 8, 128, g)
    q = randn_bf16((256, 32, 128), g)
    want = O.paged_decode_attention(f32(q), f32(kc), f32(vc), bt.numpy(), sl.numpy())
    out = paged_decode_attention(q.view(256, -1).to(dev), kc.to(dev), vc.to(dev), bt.to(dev), sl.to(dev), 32, 8, 128)
    torch.cuda.synchronize()
    _close(f32(out).reshape(256, 32, 128), want)


def test_paged_decode_batch_above_256(dev):
    """B 300: two launches of the kernel pair (256 + 44 sequences) on one
    workspace, with padding rows on both sides of the cut."""
    from xvllm.layers.attention import paged_decode_attention

    g = gen(300)
    ctx = torch.randint(0, 200, (300,), generator=g).tolist()
    ctx[255] = ctx[256] = 0
    ctx[299] = 1
    need = sum((c + 15) // 16 for c in ctx)
    kc, vc, bt, sl = make_paged(ctx, int(need * 1.25) + 4, 8, 128, g)
    q = randn_bf16((300, 32, 128), g)
    want = O.paged_decode_attention(f32(q), f32(kc), f32(vc), bt.numpy(), sl.numpy())
    out = paged_decode_attention(q.view(300, -1).to(dev), kc.to(dev), vc.to(dev), bt.to(dev), sl.to(dev), 32, 8, 128)
    torch.cuda.synchronize()
    _close(f32(out).reshape(300, 32, 128), want)


@pytest.mark.parametrize("ctxlen,bsz", [(32768, 2), (131072, 1)])
def test_paged_decode_single_long_sequence(dev, ctxlen, bsz):
    """A few sequences of 32k / 128k tokens (block tables of 2048 / 8192
    pages): every wave streams part of one sequence, and the merge combines
    up to max_blocks / min-range partials per head.  K/V drawn on the device;
    checked against a plain fp32 torch softmax attention over the gathered
    keys (the numpy oracle is too slow at this length)."""
    from xvllm.layers.attention import paged_decode_attention

    g = torch.Generator(device=dev).manual_seed(ctxlen)
    hq, hkv, d = 32, 8, 128
    npg = ctxlen // 16
    pool = bsz * npg + 3
    kc = torch.randn((pool, 16, hkv, d), generator=g, device=dev).to(torch.bfloat16)
    vc = torch.randn((pool, 16, hkv, d), generator=g, device=dev).to(torch.bfloat16)
    perm = torch.randperm(pool, generator=gen(ctxlen))[: bsz * npg].to(torch.int32)
    bt = perm.view(bsz, npg).to(dev)
    sl = torch.full((bsz,), ctxlen, dtype=torch.int32, device=dev)
    sl[-1] = ctxlen - 9
    q = torch.randn((bsz, hq * d), generator=g, device=dev).to(torch.bfloat16)
    out = paged_decode_attention(q, kc, vc, bt, sl, hq, hkv, d)
    torch.cuda.synchronize()
    for r in range(bsz):
        # reference on the GPU in fp32 (exact softmax over the gathered keys)
        n = int(sl[r])
        pages = bt[r].long()
        k = kc[pages].reshape(-1, hkv, d)[:n].float()
        v = vc[pages].reshape(-1, hkv, d)[:n].float()
        qr = q[r].view(hq, d).float()
        kh = k.repeat_interleave(hq // hkv, dim=1)  # [n, hq, d]
        vh = v.repeat_interleave(hq // hkv, dim=1)
        s = torch.einsum("hd,nhd->hn", qr, kh) / math.sqrt(d)
        want = torch.einsum("hn,nhd->hd", torch.softmax(s, dim=-1), vh)
        _close(f32(out[r].cpu()).reshape(1, hq, d), want.cpu().numpy().reshape(1, hq, d))
    assert torch.isfinite(out.float()).all()


def test_paged_decode_long_ranges(dev):
    """B 64 x ctx 8192: each wave streams ~256 pages, crossing page-id table
    windows.  K/V are drawn on the device; the oracle gets only the pages of
    the checked rows."""
    from xvllm.layers.attention import paged_decode_attention

    g = torch.Generator(device=dev).manual_seed(5)
    bsz, ctxlen, hq, hkv, d = 64, 8192, 32, 8, 128
    npg = ctxlen // 16
    pool = bsz * npg + 7
    kc = torch.randn((pool, 16, hkv, d), generator=g, device=dev).to(torch.bfloat16)
    vc = torch.randn((pool, 16, hkv, d), generator=g, device=dev).to(torch.bfloat16)
    perm = torch.randperm(pool, generator=gen(6))[: bsz * npg].to(torch.int32)
    bt = perm.view(bsz, npg).to(dev)
    sl = torch.full((bsz,), ctxlen, dtype=torch.int32, device=dev)
    sl[3] = ctxlen - 5
    q = torch.randn((bsz, hq * d), generator=g, device=dev).to(torch.bfloat16)
    out = paged_decode_attention(q, kc, vc, bt, sl, hq, hkv, d)
    torch.cuda.synchronize()
    rows = [0, 3, 40, 63]
    for r in rows:
        pages = bt[r].long()
        kr, vr = f32(kc[pages].cpu()), f32(vc[pages].cpu())
        want = O.paged_decode_attention(f32(q[r : r + 1].cpu()).reshape(1, hq, d), kr, vr,
                                        np.arange(npg, dtype=np.int32)[None, :], np.array([int(sl[r])]))
        _close(f32(out[r : r + 1].cpu()).reshape(1, hq, d), want)
    assert torch.isfinite(out.float()).all()


@pytest.mark.parametrize("rows,hidden", [(7, 4096), (64, 1024), (33, 128), (3, 5120), (2, 4104)])
def test_rmsnorm(dev, rows, hidden):
    g = gen(rows)
    x = randn_bf16((rows, hidden), g)
    w = randn_bf16((hidden,), g, std=0.1, mean=1.0)
    out = torch.ops.vllm.rmsnorm(x.to(dev), w.to(dev), 1e-6)
    _close(f32(out), O.rmsnorm(f32(x), f32(w), 1e-6))


def test_rmsnorm_head_view(dev):
    """q/k head norm on a [T, H, D] view of a fused qkv row (no copy)."""
    g = gen(5)
    t, hq, d = 9, 32, 128
    qkv = randn_bf16((t, 48 * d), g).to(dev)
    q = qkv[:, : hq * d].view(t, hq, d)
    w = randn_bf16((d,), g, std=0.1, mean=1.0)
    out = torch.ops.vllm.rmsnorm(q, w.to(dev), 1e-6)
    _close(f32(out), O.rmsnorm(f32(q), f32(w), 1e-6))


@pytest.mark.parametrize("rows,hidden", [(7, 4096), (64, 1024), (1, 5120)])
def test_fused_add_rmsnorm(dev, rows, hidden):
    g = gen(rows + 1)
    x, r = randn_bf16((rows, hidden), g), randn_bf16((rows, hidden), g)
    w = randn_bf16((hidden,), g, std=0.1, mean=1.0)
    xg, rg = x.to(dev), r.to(dev)
    torch.ops.vllm.fused_add_rmsnorm(xg, rg, w.to(dev), 1e-6)
    want_x, want_r = O.fused_add_rmsnorm(f32(x), f32(r), f32(w), 1e-6)
    # the residual sum of two bf16 values rounded once is exact to the bit
    assert np.array_equal(f32(rg), want_r)
    _close(f32(xg), want_x)


def _rope_inputs(g, t, hq, hkv, d=128, max_pos=32768):
    qkv = randn_bf16((t, (hq + 2 * hkv) * d), g)
    pos = torch.randint(0, max_pos, (t,), generator=g)
    cs = torch.from_numpy(O.build_cos_sin_cache(d, max_pos, 1e6))
    return qkv, pos, cs


def test_rotary_embedding(dev):
    g = gen(11)
    t, hq, hkv, d = 19, 32, 8, 128
    qkv, pos, cs = _rope_inputs(g, t, hq, hkv)
    qg = qkv.to(dev)
    q = qg[:, : hq * d].view(t, hq, d)
    k = qg[:, hq * d : (hq + hkv) * d].view(t, hkv, d)
    qo, ko = torch.ops.vllm.rotary_embedding(q, k, pos.to(dev), cs.to(dev), d)
    _close(f32(qo), O.rope_neox(f32(q), pos.numpy(), cs.numpy()))
    _close(f32(ko), O.rope_neox(f32(k), pos.numpy(), cs.numpy()))


@pytest.mark.parametrize("t,hq,hkv", [(23, 32, 8), (8, 16, 8), (3, 64, 8)])
def test_qk_norm_rope(dev, t, hq, hkv):
    import xvllm.layers.ops  # noqa: F401

    g = gen(t * hq)
    d = 128
    qkv, pos, cs = _rope_inputs(g, t, hq, hkv)
    qw = randn_bf16((d,), g, std=0.1, mean=1.0)
    kw = randn_bf16((d,), g, std=0.1, mean=1.0)
    qg = qkv.to(dev)
    q = qg[:, : hq * d].view(t, hq, d)
    k = qg[:, hq * d : (hq + hkv) * d].view(t, hkv, d)
    qo, ko = torch.ops.xv.qk_norm_rope(q, k, qw.to(dev), kw.to(dev), 1e-6, pos.to(dev), cs.to(dev))
    wq, wk = O.qk_norm_rope(f32(q), f32(k), f32(qw), f32(kw), 1e-6, pos.numpy(), cs.numpy())
    _close(f32(qo), wq)
    _close(f32(ko), wk)


@pytest.mark.parametrize("t,inter", [(5, 3072), (64, 12288), (3, 8)])
def test_silu_and_mul(dev, t, inter):
    g = gen(t)
    x = randn_bf16((t, 2 * inter), g)
    out = torch.ops.vllm.silu_and_mul(x.to(dev))
    _close(f32(out), O.silu_and_mul(f32(x)))


# ------------------------------------------------------------------ prefill attention
@pytest.mark.parametrize(
    "hq,hkv,qlens,klens,paged",
    [
        (32, 8, [37, 128, 1, 64], [37, 128, 1, 64], False),     # plain prefill (q_len == k_len)
        (32, 8, [17, 64, 100], [300, 64, 612], True),           # chunked prefill over a cached prefix
        (16, 8, [70, 5], [70, 200], True),                      # Qwen3-0.6B heads
        (64, 8, [33], [129], True),                             # group 8
        (8, 8, [20, 0, 9], [20, 0, 40], False),                 # MHA, an empty sequence
        (32, 8, [777, 64], [777, 64], False),                   # long prompt: many tiles, odd tail
        (32, 8, [300, 129], [2100, 1129], True),                # long chunks over long cached prefixes
        (16, 8, [161], [1000], True),                           # group 2, 64-query blocks
        (32, 8, [64, 64, 1, 64, 0, 64], [64, 64, 1, 64, 0, 64], False),  # equal work: tie order
        (32, 8, [50, 20, 50, 20], [80, 20, 80, 50], True),      # mixed work with ties
        (32, 8, [5, 3] * 35, [5, 3] * 35, False),               # 70 sequences: batch above 64
    ],
)
def test_prefill_attention(dev, hq, hkv, qlens, klens, paged):
    from xvllm.layers.attention import prefill_attention

    g = gen(sum(qlens) + hq)
    d = 128
    cu_q = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(klens)]).astype(np.int32)
    q = randn_bf16((int(cu_q[-1]), hq, d), g)
    if paged:
        need = sum((c + 15) // 16 for c in klens)
        kc, vc, bt, _ = make_paged(klens, need + 5, hkv, d, g)
        want = O.prefill_attention(f32(q), cu_q, cu_k, k_cache=f32(kc), v_cache=f32(vc), block_tables=bt.numpy())
        out = prefill_attention(q.to(dev), None, None, torch.from_numpy(cu_q).to(dev), torch.from_numpy(cu_k).to(dev),
                                max(qlens), hq, hkv, d, k_cache=kc.to(dev), v_cache=vc.to(dev), block_tables=bt.to(dev))
    else:
        k = randn_bf16((int(cu_k[-1]), hkv, d), g)
        v = randn_bf16((int(cu_k[-1]), hkv, d), g)
        want = O.prefill_attention(f32(q), cu_q, cu_k, k=f32(k), v=f32(v))
        out = prefill_attention(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(cu_q).to(dev),
                                torch.from_numpy(cu_k).to(dev), max(qlens), hq, hkv, d)
    torch.cuda.synchronize()
    _close(f32(out).reshape(-1, hq, d), want)


# ------------------------------------------------------------------ sampler
def _sampler_case(g, b, v, std=2.0, ties=False):
    if ties == "flat":
        std = 0.004
    x = torch.randn((b, v), generator=g) * std
    if ties is True:
        x = torch.round(x * 4) / 4  # few distinct values: ties everywhere
    if ties == "massive":
        x = torch.round(torch.randn((b, v), generator=g)) / 2  # ~7 values, tie groups of up to ~58k ids
    return x.to(torch.bfloat16)


@pytest.mark.parametrize(
    "name,b,v,flags,temp,top_p,top_k,min_p,ties",
    [
        ("greedy", 8, 151936, 1, 1.0, 1.0, 0, 0.0, False),
        ("greedy_ties", 4, 4096, 1, 1.0, 1.0, 0, 0.0, True),
        ("temperature", 8, 151936, 0, 0.7, 1.0, 0, 0.0, False),
        ("topk50_topp0.9", 16, 151936, 2 | 4, 0.7, 0.9, 50, 0.0, False),
        ("topp0.95", 8, 151936, 4, 1.0, 0.95, 0, 0.0, False),
        ("minp", 8, 151936, 8, 1.0, 1.0, 0, 0.1, False),
        ("all_filters_ties", 8, 32000, 2 | 4 | 8, 0.8, 0.8, 300, 0.02, True),
        ("odd_vocab", 5, 1003, 2 | 4, 1.1, 0.6, 7, 0.0, False),
        # near-flat rows: the bucket scale adapts to the row's span
        ("flat_topp", 4, 151936, 4, 1.0, 0.5, 0, 0.0, "flat"),
        ("flat_topk", 4, 151936, 2 | 4, 1.0, 0.9, 20000, 0.0, "flat"),
        ("flat_topp0.95_b32", 32, 151936, 4, 1.0, 0.95, 0, 0.0, "flat"),
        ("flat_all_odd_vocab", 6, 151935, 2 | 4 | 8, 1.0, 0.7, 30000, 0.3, "flat"),
        ("flat_minp", 4, 151936, 8, 0.5, 1.0, 0, 0.9, "flat"),
        # tie groups larger than LDS: the boundary bucket overflows -> the row-wide radix-select path
        ("ties_fallback_topp", 4, 151936, 4, 1.0, 0.5, 0, 0.0, "massive"),
        ("ties_fallback_topk", 4, 151936, 2 | 4, 1.0, 0.9, 20000, 0.0, "massive"),
        ("ties_fallback_all_odd_vocab", 6, 151935, 2 | 4 | 8, 0.8, 0.7, 30000, 0.3, "massive"),
        ("ties_fallback_minp", 4, 151936, 8, 1.0, 1.0, 0, 0.5, "massive"),
    ],
)
@pytest.mark.parametrize("multi_wg", [True, False], ids=["multi_wg", "one_wg"])
def test_sampler_bitexact(dev, name, b, v, flags, temp, top_p, top_k, min_p, ties, multi_wg):
    import oracle.sampler as S
    from xvllm.sampler import sample

    g = gen(b * 7 + v)
    logits = _sampler_case(g, b, v, ties=ties)
    temps = torch.full((b,), temp)
    temps[::3] = 0.0 if name not in ("greedy", "greedy_ties") else temp  # mixed greedy rows
    tps = torch.full((b,), top_p)
    tks = torch.full((b,), top_k if top_k else v, dtype=torch.int32)
    mps = torch.full((b,), min_p)
    u = torch.rand(b, generator=g)
    u[0] = 0.0
    want = S.sample(logits.view(torch.int16).numpy().view(np.uint16), temps.numpy(), tps.numpy(), tks.numpy(),
                    mps.numpy(), u.numpy(), flags)
    got = sample(logits.to(dev), temps.to(dev), tps.to(dev), tks.to(dev), mps.to(dev), u.to(dev),
                 all_greedy=bool(flags & 1), use_top_k=bool(flags & 2), use_top_p=bool(flags & 4),
                 use_min_p=bool(flags & 8), multi_workgroup=multi_wg)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), want), f"{got.cpu().numpy()} vs {want}"


@pytest.mark.parametrize("b", [32, 64])
def test_sampler_chain_cut_cases_bitexact(dev, b):
    """The multi-workgroup path's cut on its own cases, against the C oracle:
    near-flat rows whose top-p cut splits a tie group of one key (under and
    over the 512 ids the per-key cut ranks itself; the sort takes the larger),
    wide rows, min-p cuts and both together, seeded uniforms, B 32 and 64."""
    import oracle.sampler as S
    from xvllm.sampler import sample

    rng = np.random.default_rng(77 + b)
    v = 151936
    for case, (std, temp, top_p, min_p, flags) in enumerate([
            (0.05, 1.0, 0.95, 0.0, 4), (0.002, 1.0, 0.9, 0.0, 4), (0.01, 0.7, 0.6, 0.0, 4),
            (1.0, 1.0, 0.9, 0.0, 4), (3.0, 0.8, 0.99, 0.0, 4), (0.05, 1.0, 1.0, 0.97, 8),
            (0.3, 1.0, 1.0, 0.5, 8), (0.02, 1.0, 0.8, 0.99, 4 | 8), (1.0, 0.5, 0.7, 0.01, 4 | 8)]):
        x = (rng.standard_normal((b, v)) * std).astype(np.float32)
        logits = torch.from_numpy(x).to(torch.bfloat16)
        temps = torch.full((b,), temp)
        tps = torch.from_numpy(np.clip(rng.normal(top_p, 0.02, b), 0.05, 1.0).astype(np.float32)) \
            if top_p < 1.0 else torch.ones(b)
        mps = torch.full((b,), min_p)
        u = torch.from_numpy(rng.random(b).astype(np.float32))
        want = S.sample(logits.view(torch.int16).numpy().view(np.uint16), temps.numpy(), tps.numpy(), None,
                        mps.numpy(), u.numpy(), flags)
        print(f"chain cut case {case}: std {std} T {temp} p {top_p} min_p {min_p} B {b}", flush=True)
        got = sample(logits.to(dev), temps.to(dev), tps.to(dev), None, mps.to(dev), u.to(dev),
                     use_top_p=bool(flags & 4), use_min_p=bool(flags & 8))
        assert np.array_equal(got.cpu().numpy(), want), (case, np.nonzero(got.cpu().numpy() != want)[0][:8])


def test_sampler_nan_rows_paths_agree(dev):
    """Rows with NaN logits (some, all) and a row of equal logits: the
    multi-workgroup path gives the ids of the one-workgroup path."""
    from xvllm.sampler import sample

    g = gen(5)
    b, v = 6, 151936
    logits = _sampler_case(g, b, v, std=1.0)
    logits[0, ::7] = float("nan")
    logits[1] = float("nan")
    logits[2] = 0.25
    logits[3, :100] = float("nan")
    logits[3, 5000] = float("inf")
    logits[4, 70001] = logits[4, 90001] = float("nan")  # greedy row: torch.argmax takes NaN id 70001
    temps = torch.tensor([1.0, 0.8, 1.0, 0.7, 0.0, 1.3])
    tps = torch.full((b,), 0.9)
    tks = torch.full((b,), 40, dtype=torch.int32)
    u = torch.rand(b, generator=g)
    for kw in (dict(use_top_p=True), dict(use_top_k=True, use_top_p=True),
               dict(use_top_k=True, use_top_p=True, max_top_k=40), {}):
        args = (logits.to(dev), temps.to(dev), tps.to(dev), tks.to(dev), None, u.to(dev))
        got = sample(*args, **kw)
        want = sample(*args, **kw, multi_workgroup=False)
        assert torch.equal(got, want), (kw, got, want)
        assert int(got[4]) == 70001, kw


def test_sampler_many_draws_bitexact(dev):
    """One row, 256 stratified uniforms: every draw equals the oracle's."""
    import oracle.sampler as S
    from xvllm.sampler import sample

    g = gen(99)
    v, n = 151936, 256
    row = _sampler_case(g, 1, v, std=1.0)
    logits = row.repeat(n, 1)
    u = (torch.arange(n, dtype=torch.float32) + 0.5) / n
    args = dict(temps=torch.full((n,), 0.7), tps=torch.full((n,), 0.9), tks=torch.full((n,), 50, dtype=torch.int32))
    want = S.sample(logits.view(torch.int16).numpy().view(np.uint16), args["temps"].numpy(), args["tps"].numpy(),
                    args["tks"].numpy(), None, u.numpy(), 2 | 4)
    got = sample(logits.to(dev), args["temps"].to(dev), args["tps"].to(dev), args["tks"].to(dev), None, u.to(dev),
                 use_top_k=True, use_top_p=True)
    assert np.array_equal(got.cpu().numpy(), want)


@pytest.mark.parametrize("hnd", [False, True])
def test_qk_norm_rope_store_matches_separate_ops(dev, hnd):
    """Fused decode kernel == qk_norm_rope followed by store_kvcache, bit for bit,
    into a reference-layout pool and into a head-major (strided) pool view."""
    from xvllm.kv_ops import store_kvcache

    g = gen(77)
    t, hq, hkv, d, nb = 13, 32, 8, 128, 12
    qkv, pos, cs = _rope_inputs(g, t, hq, hkv)
    qw = randn_bf16((d,), g, std=0.1, mean=1.0).to(dev)
    kw = randn_bf16((d,), g, std=0.1, mean=1.0).to(dev)
    qg = qkv.to(dev)
    q = qg[:, : hq * d].view(t, hq, d)
    k = qg[:, hq * d : (hq + hkv) * d].view(t, hkv, d)
    v = qg[:, (hq + hkv) * d :].view(t, hkv, d)
    slots = torch.randperm(nb * 16, generator=g)[:t].to(torch.int32)
    slots[3] = -1

    def pool():
        if hnd:  # physical [NB, Hkv, BS, D] seen as [NB, BS, Hkv, D]
            return randn_bf16((nb, hkv, 16, d), g).to(dev).permute(0, 2, 1, 3)
        return randn_bf16((nb, 16, hkv, d), g).to(dev)

    kc1, vc1 = pool(), pool()
    kc2, vc2 = kc1.clone(), vc1.clone()
    qo, ko = torch.ops.xv.qk_norm_rope(q, k, qw, kw, 1e-6, pos.to(dev), cs.to(dev))
    store_kvcache(ko, v, kc1, vc1, slots.to(dev))
    qf = torch.ops.xv.qk_norm_rope_store(q, k, v, qw, kw, 1e-6, pos.to(dev), cs.to(dev), kc2, vc2, slots.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(qf, qo)
    assert torch.equal(kc2, kc1) and torch.equal(vc2, vc1)


def test_paged_decode_merge_ignores_stale_workspace(dev):
    """The merge reads the first partial rows of a head speculatively; rows
    past the head's partial count hold whatever an earlier call left, here
    NaN bit patterns (0xFF bytes) in the whole workspace.  Batches whose
    sequences split into 1 to 6 partials must still be finite and correct."""
    from xvllm.layers.attention import decode_workspace, paged_decode_attention

    g = gen(93)
    for bsz, lo, hi in [(4, 2000, 4097), (16, 300, 4097), (64, 512, 4097)]:
        ctx = torch.randint(lo, hi, (bsz,), generator=g).tolist()
        need = sum((c + 15) // 16 for c in ctx)
        kc, vc, bt, sl = make_paged(ctx, int(need * 1.25) + 4, 8, 128, g)
        q = randn_bf16((bsz, 32, 128), g)
        args = (q.view(bsz, -1).to(dev), kc.to(dev), vc.to(dev), bt.to(dev), sl.to(dev), 32, 8, 128)
        paged_decode_attention(*args)  # sizes the workspace
        decode_workspace(dev, 1).fill_(255)
        out = paged_decode_attention(*args)
        torch.cuda.synchronize()
        print(f"stale workspace: B {bsz} ctx [{lo},{hi})", flush=True)
        assert torch.isfinite(out.float()).all()
        rows = list(range(0, bsz, max(1, bsz // 8)))
        want = O.paged_decode_attention(f32(q)[rows], f32(kc), f32(vc), bt.numpy()[rows], sl.numpy()[rows])
        _close(f32(out).reshape(bsz, 32, 128)[rows], want)


def test_paged_decode_workspace_reuse_across_batches(dev):
    """Calls of different batch sizes share the per-device workspace: split
    partials of one call must never be taken for the arrival counters of the
    next, and each call leaves the counters at zero."""
    from xvllm.layers.attention import paged_decode_attention

    g = gen(91)
    for bsz, lo, hi in [(8, 600, 3000), (256, 1, 300), (64, 200, 2500), (3, 4000, 4097), (256, 30, 900)]:
        ctx = torch.randint(lo, hi, (bsz,), generator=g).tolist()
        need = sum((c + 15) // 16 for c in ctx)
        kc, vc, bt, sl = make_paged(ctx, int(need * 1.25) + 4, 8, 128, g)
        q = randn_bf16((bsz, 32, 128), g)
        rows = list(range(0, bsz, max(1, bsz // 8)))
        want = O.paged_decode_attention(f32(q)[rows], f32(kc), f32(vc), bt.numpy()[rows], sl.numpy()[rows])
        out = paged_decode_attention(q.view(bsz, -1).to(dev), kc.to(dev), vc.to(dev), bt.to(dev), sl.to(dev),
                                     32, 8, 128)
        torch.cuda.synchronize()
        print(f"workspace reuse: B {bsz} ctx [{lo},{hi})", flush=True)
        assert torch.isfinite(out.float()).all()
        _close(f32(out).reshape(bsz, 32, 128)[rows], want)


# ------------------------------------------------------------------ config 3 at full size
def test_config3_elementwise_full_size(dev):
    """Config 3 shapes (T 8192, Qwen3-8B width) through each fused kernel; 64
    seeded rows checked against the oracle (every op is row-wise), the whole
    output checked finite, the residual of add+RMSNorm bit-exact."""
    import xvllm.layers.ops  # noqa: F401
    from xvllm.layers.rotary import build_cos_sin_cache

    g = gen(33)
    T, H, I, HQ_, HKV_, D_ = 8192, 4096, 12288, 32, 8, 128
    rows = torch.randperm(T, generator=g)[:64].sort().values
    r = rows.numpy()
    # residual-add + RMSNorm
    x, res = randn_bf16((T, H), g), randn_bf16((T, H), g)
    w = randn_bf16((H,), g, 0.1, 1.0)
    xd, rd = x.to(dev), res.to(dev)
    torch.ops.vllm.fused_add_rmsnorm(xd, rd, w.to(dev), 1e-6)
    torch.cuda.synchronize()
    want_x, want_r = O.fused_add_rmsnorm(f32(x)[r], f32(res)[r], f32(w), 1e-6)
    assert torch.isfinite(xd.float()).all()
    _close(f32(xd.cpu())[r], want_x)
    assert np.array_equal(f32(rd.cpu())[r], want_r)
    del x, res, xd, rd
    # q/k RMSNorm + RoPE (theta 1e6, positions U[0, 32768))
    q, k = randn_bf16((T, HQ_, D_), g), randn_bf16((T, HKV_, D_), g)
    qw, kw = randn_bf16((D_,), g, 0.1, 1.0), randn_bf16((D_,), g, 0.1, 1.0)
    pos = torch.randint(0, 32768, (T,), generator=g)
    cs = build_cos_sin_cache(D_, 32768, 1e6)
    qo, ko = torch.ops.xv.qk_norm_rope(q.to(dev), k.to(dev), qw.to(dev), kw.to(dev), 1e-6, pos.to(dev), cs.to(dev))
    torch.cuda.synchronize()
    want_q, want_k = O.qk_norm_rope(f32(q)[r], f32(k)[r], f32(qw), f32(kw), 1e-6, pos.numpy()[r], cs.numpy())
    for got, want in ((qo, want_q), (ko, want_k)):
        assert torch.isfinite(got.float()).all()
        _close(f32(got.cpu())[r], want)
    del q, k, qo, ko
    # SiLU(gate) * up at width 12288
    xg = randn_bf16((T, 2 * I), g)
    out = torch.ops.vllm.silu_and_mul(xg.to(dev))
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    _close(f32(out.cpu())[r], O.silu_and_mul(f32(xg)[r]))


@pytest.mark.parametrize("b,v", [(1, 151936), (7, 4099), (64, 151936), (300, 32000)])
def test_greedy_multi_workgroup_bitexact(dev, b, v):
    """All-greedy batches spread each row over several workgroups (one 64-bit
    atomic max per wave).  Against the C oracle and torch.argmax (the
    reference's greedy): ties at the maximum (lowest id wins), -0 vs +0
    (equal), NaN entries (the lowest NaN id wins), an all-NaN row (id 0); and a
    second call on the same workspace (its slots must have been cleared)."""
    import oracle.sampler as S
    from xvllm.sampler import sample

    g = gen(b + v)
    x = torch.round(torch.randn((b, v), generator=g) * 4) / 4  # few distinct values: ties at the max
    x = x.to(torch.bfloat16)
    bits = x.view(torch.int16)
    if b >= 7:
        bits[1, :] = torch.tensor(0x7FC0, dtype=torch.int16)  # all-NaN row
        bits[2, :] = torch.tensor(-32768, dtype=torch.int16)  # all -0.0 ...
        bits[2, 5:9] = 0                                      # ... a few +0.0 after the first ids
        bits[3, ::5] = torch.tensor(0x7FC0, dtype=torch.int16)  # NaNs among values
        bits[4, v - 3] = torch.tensor(0x7FC0, dtype=torch.int16)  # one NaN near the end
        bits[5, v // 2 :: 97] = torch.tensor(-64, dtype=torch.int16)  # 0xFFC0: negative-sign NaNs
    for call in range(2):
        xs = x if call == 0 else x.flip(1).contiguous()
        want = S.sample(xs.view(torch.int16).numpy().view(np.uint16), np.zeros(b, np.float32), None, None, None,
                        None, 1)
        got = sample(xs.to(dev), None, all_greedy=True)
        torch.cuda.synchronize()
        assert np.array_equal(got.cpu().numpy(), want), f"call {call}: {got.cpu().numpy()[:8]} vs {want[:8]}"
        assert np.array_equal(want, xs.argmax(-1).numpy())


def test_decode_graphs_largest_first_share_one_workspace(dev):
    """Decode-attention graphs captured for buckets 256 .. 1 (largest first, as
    the graph runner does) on the shared workspace, then replayed in mixed
    order with eager calls between: every replay equals the eager result, and
    no capture regrew the workspace (a regrown one would leave the earlier
    graphs replaying onto freed memory)."""
    import xvllm.layers.attention as A
    from xvllm.layers.attention import paged_decode_attention

    g = torch.Generator(device=dev).manual_seed(11)
    hq, hkv, d, maxb = 32, 8, 128, 256
    pool = 2048
    kc = torch.randn((pool, 16, hkv, d), generator=g, device=dev).to(torch.bfloat16)
    vc = torch.randn((pool, 16, hkv, d), generator=g, device=dev).to(torch.bfloat16)
    buckets = [256, 240, 128, 96, 64, 1]
    ctx = torch.randint(1, 16 * 8, (256,), generator=torch.Generator().manual_seed(12)).to(torch.int32).to(dev)
    bt = torch.randint(0, pool, (256, maxb), generator=g, device=dev).to(torch.int32)
    q = torch.randn((256, hq * d), generator=g, device=dev).to(torch.bfloat16)
    outs, graphs = {}, {}
    first_ws = None
    for bs in buckets:
        out = torch.empty((bs, hq * d), dtype=torch.bfloat16, device=dev)
        paged_decode_attention(q[:bs], kc, vc, bt[:bs], ctx[:bs], hq, hkv, d, out=out)  # warm-up, sizes the workspace
        torch.cuda.synchronize()
        ws = A._WORKSPACE[(dev.type, dev.index)]
        first_ws = first_ws if first_ws is not None else ws.data_ptr()
        assert ws.data_ptr() == first_ws, f"workspace regrown at bucket {bs}"
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            paged_decode_attention(q[:bs], kc, vc, bt[:bs], ctx[:bs], hq, hkv, d, out=out)
        outs[bs], graphs[bs] = out, gr
    for bs in [256, 1, 240, 64, 256, 96, 128, 256]:
        want = paged_decode_attention(q[:bs], kc, vc, bt[:bs], ctx[:bs], hq, hkv, d)
        graphs[bs].replay()
        torch.cuda.synchronize()
        assert torch.equal(outs[bs], want), f"replay of bucket {bs}"


def test_sampler_one_workspace_sampled_and_greedy_calls_interleaved(dev):
    """One workspace sized for 64 rows serves sampled calls (multi-workgroup
    path, which writes the top of the workspace) and all-greedy calls (whose
    per-row lines at the bottom must be zero) in any order and batch size:
    greedy ids equal the argmax (lowest id on ties), sampled ids equal the
    one-workgroup path's."""
    from xvllm import _C
    from xvllm._torch_glue import ptr, stream_of
    from xvllm.sampler import sample

    L = _C.lib()
    V = 151936
    ws = torch.zeros(L.xv_sampler_workspace_size(64, V), dtype=torch.uint8, device=dev)
    g = gen(321)

    def call(logits, flags, temps=None, tps=None, tks=None, u=None):
        out = torch.empty(logits.shape[0], dtype=torch.int64, device=dev)
        rc = L.xv_sample(ptr(logits), logits.stride(0), logits.shape[0], V, ptr(temps), ptr(tps), ptr(tks), None,
                         ptr(u), flags, ptr(out), ptr(ws), ws.numel(), stream_of(logits))
        assert rc == 0
        return out

    for bs, kind in [(8, "sampled"), (64, "greedy"), (32, "sampled"), (48, "greedy"), (64, "sampled"), (64, "greedy")]:
        logits = _sampler_case(g, bs, V, std=1.0).to(dev)
        if kind == "greedy":
            got = call(logits, _C.XV_SAMPLE_ALL_GREEDY)
            x = logits.float()
            want = (x == x.max(dim=1, keepdim=True).values).float().argmax(dim=1)  # lowest id holding the max
        else:
            temps = torch.full((bs,), 0.7, device=dev)
            tps = torch.full((bs,), 0.9, device=dev)
            tks = torch.full((bs,), 50, dtype=torch.int32, device=dev)
            u = torch.rand(bs, generator=g).to(dev)
            got = call(logits, _C.XV_SAMPLE_USE_TOP_K | _C.XV_SAMPLE_USE_TOP_P, temps, tps, tks, u)
            want = sample(logits, temps, tps, tks, None, u, use_top_k=True, use_top_p=True, multi_workgroup=False)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (bs, kind)


def test_sampler_large_batches_bitexact(dev):
    """Sampled batches of 129-513 rows (the multi-workgroup chain up to 512
    rows, one workgroup per row past it): seeded top-k / top-p / min-p mixes
    with greedy rows, flat and tied rows and NaN entries, equal to the C
    oracle on every row."""
    import oracle.sampler as S
    from xvllm.sampler import sample

    rng = np.random.default_rng(4242)
    for case, (b, flags, kind, v) in enumerate([(129, 4, "flat", 151936), (200, 2 | 4, "normal", 151936),
                                                (256, 4 | 8, "ties", 151936), (256, 2 | 4 | 8, "normal", 151936),
                                                (160, 0, "wide", 151936), (256, 4, "massive", 151936),
                                                (384, 4 | 8, "normal", 32000), (512, 2 | 4, "ties", 32000),
                                                (513, 4, "flat", 32000)]):
        std = {"flat": 0.05, "normal": 1.0, "wide": 4.0, "ties": 1.0, "massive": 1.0}[kind]
        x = rng.standard_normal((b, v)).astype(np.float32) * std
        if kind == "ties":
            x = np.round(x * 4) / 4
        if kind == "massive":
            x = np.round(x) / 2
        x[rng.random((b, v)) < 0.0005] = np.nan
        logits = torch.from_numpy(x).to(torch.bfloat16)
        temps = torch.from_numpy(rng.uniform(0.3, 1.5, b).astype(np.float32))
        temps[torch.from_numpy(rng.random(b) < 0.2)] = 0.0
        tps = torch.from_numpy(rng.uniform(0.3, 0.99, b).astype(np.float32))
        tks = torch.from_numpy(rng.integers(1, 3000, b).astype(np.int32))
        mps = torch.from_numpy(rng.uniform(0.0, 0.3, b).astype(np.float32))
        u = torch.from_numpy(rng.random(b).astype(np.float32))
        want = S.sample(logits.view(torch.int16).numpy().view(np.uint16), temps.numpy(), tps.numpy(), tks.numpy(),
                        mps.numpy(), u.numpy(), flags)
        print(f"large-batch case {case}: b {b} flags {flags} {kind}", flush=True)
        got = sample(logits.to(dev), temps.to(dev), tps.to(dev), tks.to(dev), mps.to(dev), u.to(dev),
                     use_top_k=bool(flags & 2), use_top_p=bool(flags & 4), use_min_p=bool(flags & 8))
        assert np.array_equal(got.cpu().numpy(), want), (case, np.nonzero(got.cpu().numpy() != want)[0][:8])


def test_sampler_randomized_configurations_bitexact(dev):
    """40 seeded random configurations (batch 1-40, vocabularies 1003 / 4099 /
    32000 / 151936, any mix of top-k / top-p / min-p, temperatures with some
    greedy rows, logits from narrow to wide, coarse ties, massive ties and a
    sprinkle of NaN): both paths equal the C oracle on every row."""
    import oracle.sampler as S
    from xvllm.sampler import sample

    rng = np.random.default_rng(2024)
    for case in range(40):
        b = int(rng.integers(1, 41))
        v = int(rng.choice([1003, 4099, 32000, 151936]))
        flags = int(rng.choice([0, 2, 4, 8, 2 | 4, 4 | 8, 2 | 8, 2 | 4 | 8]))
        kind = rng.choice(["narrow", "normal", "wide", "ties", "massive"])
        std = {"narrow": 0.02, "normal": 1.0, "wide": 4.0, "ties": 1.0, "massive": 1.0}[kind]
        x = rng.standard_normal((b, v)).astype(np.float32) * std
        if kind == "ties":
            x = np.round(x * 4) / 4
        if kind == "massive":
            x = np.round(x) / 2
        if rng.random() < 0.2:
            x[rng.random((b, v)) < 0.001] = np.nan
        logits = torch.from_numpy(x).to(torch.bfloat16)
        temps = torch.from_numpy(rng.uniform(0.3, 1.5, b).astype(np.float32))
        temps[torch.from_numpy(rng.random(b) < 0.2)] = 0.0  # some greedy rows
        tps = torch.from_numpy(rng.uniform(0.3, 0.99, b).astype(np.float32))
        tks = torch.from_numpy(rng.integers(1, min(v, 3000), b).astype(np.int32))
        mps = torch.from_numpy(rng.uniform(0.0, 0.3, b).astype(np.float32))
        u = torch.from_numpy(rng.random(b).astype(np.float32))
        want = S.sample(logits.view(torch.int16).numpy().view(np.uint16), temps.numpy(), tps.numpy(), tks.numpy(),
                        mps.numpy(), u.numpy(), flags)
        args = (logits.to(dev), temps.to(dev), tps.to(dev), tks.to(dev), mps.to(dev), u.to(dev))
        kw = dict(use_top_k=bool(flags & 2), use_top_p=bool(flags & 4), use_min_p=bool(flags & 8))
        for mw in (True, False):
            got = sample(*args, **kw, multi_workgroup=mw).cpu().numpy()
            assert np.array_equal(got, want), (case, b, v, flags, kind, mw)


@pytest.mark.parametrize(
    "name,b,v,flags,top_k,kind",
    [
        ("k50_p0.9", 64, 151936, 2 | 4, 50, None),
        ("k1", 8, 151936, 2, 1, None),
        ("k64_minp", 16, 151936, 2 | 8, 64, None),
        ("k20_all", 32, 151936, 2 | 4 | 8, 20, "ties"),
        ("k64_massive_ties", 8, 151936, 2 | 4, 64, "massive"),
        ("k40_flat", 8, 151936, 2 | 4, 40, "flat"),
        ("k7_odd_vocab", 5, 1003, 2 | 4, 7, None),
        ("k33_vocab_4099", 128, 4099, 2 | 4 | 8, 33, None),
        ("k64_odd_vocab_b128", 128, 151935, 2 | 4, 64, None),
        ("k50_b256", 256, 151936, 2 | 4, 50, None),                # above the chain's 128 rows
        ("k16_b300_v32000", 300, 32000, 2 | 4 | 8, 16, "ties"),
    ],
)
def test_sampler_topk_path_bitexact(dev, name, b, v, flags, top_k, kind):
    """The two-launch top-k path (max_top_k <= 64): per-row k in [1, top_k],
    mixed greedy rows, NaN entries and a row of NaN only, equal to the C
    oracle; rows outside the bound (k 0 = whole vocabulary, k above 64) are
    still exact."""
    import oracle.sampler as S
    from xvllm.sampler import sample

    g = gen(b * 13 + v + top_k)
    logits = _sampler_case(g, b, v, std=1.0, ties=True if kind == "ties" else (kind or False))
    if b >= 4:
        logits[1, ::11] = float("nan")
        logits[2] = float("nan")
    temps = torch.rand(b, generator=g) + 0.4
    temps[::5] = 0.0  # greedy rows
    tps = torch.rand(b, generator=g) * 0.6 + 0.35
    tks = torch.randint(1, top_k + 1, (b,), generator=g, dtype=torch.int32)
    tks[0] = top_k
    mps = torch.rand(b, generator=g) * 0.2
    u = torch.rand(b, generator=g)
    u[0] = 0.0
    kw = dict(use_top_k=True, use_top_p=bool(flags & 4), use_min_p=bool(flags & 8))
    want = S.sample(logits.view(torch.int16).numpy().view(np.uint16), temps.numpy(), tps.numpy(), tks.numpy(),
                    mps.numpy(), u.numpy(), flags)
    got = sample(logits.to(dev), temps.to(dev), tps.to(dev), tks.to(dev), mps.to(dev), u.to(dev), **kw,
                 max_top_k=top_k)
    torch.cuda.synchronize()
    print(f"top-k path {name}", flush=True)
    assert np.array_equal(got.cpu().numpy(), want), f"{got.cpu().numpy()} vs {want}"
    # the flag is a claim about every row: rows that break it are still sampled exactly
    if b >= 3:
        tks2 = tks.clone()
        tks2[1] = 0
        tks2[2 % b] = 100
        want2 = S.sample(logits.view(torch.int16).numpy().view(np.uint16), temps.numpy(), tps.numpy(), tks2.numpy(),
                         mps.numpy(), u.numpy(), flags)
        got2 = sample(logits.to(dev), temps.to(dev), tps.to(dev), tks2.to(dev), mps.to(dev), u.to(dev), **kw,
                      max_top_k=top_k)
        assert np.array_equal(got2.cpu().numpy(), want2), f"{got2.cpu().numpy()} vs {want2}"


def test_sampler_topk_path_randomized_bitexact(dev):
    """30 seeded random top-k configurations with every k in [1, 64]: the
    top-k path equals the C oracle on every row."""
    import oracle.sampler as S
    from xvllm.sampler import sample

    rng = np.random.default_rng(77)
    for case in range(30):
        b = int(rng.integers(1, 129))
        v = int(rng.choice([1003, 4099, 32000, 151936]))
        flags = 2 | int(rng.choice([0, 4, 8, 4 | 8]))
        kind = rng.choice(["narrow", "normal", "wide", "ties", "massive"])
        std = {"narrow": 0.02, "normal": 1.0, "wide": 4.0, "ties": 1.0, "massive": 1.0}[kind]
        x = rng.standard_normal((b, v)).astype(np.float32) * std
        if kind == "ties":
            x = np.round(x * 4) / 4
        if kind == "massive":
            x = np.round(x) / 2
        if rng.random() < 0.2:
            x[rng.random((b, v)) < 0.001] = np.nan
        logits = torch.from_numpy(x).to(torch.bfloat16)
        temps = torch.from_numpy(rng.uniform(0.3, 1.5, b).astype(np.float32))
        temps[torch.from_numpy(rng.random(b) < 0.2)] = 0.0
        tps = torch.from_numpy(rng.uniform(0.3, 0.99, b).astype(np.float32))
        kmax = int(rng.integers(1, 65))
        tks = torch.from_numpy(rng.integers(1, kmax + 1, b).astype(np.int32))
        mps = torch.from_numpy(rng.uniform(0.0, 0.3, b).astype(np.float32))
        u = torch.from_numpy(rng.random(b).astype(np.float32))
        want = S.sample(logits.view(torch.int16).numpy().view(np.uint16), temps.numpy(), tps.numpy(), tks.numpy(),
                        mps.numpy(), u.numpy(), flags)
        got = sample(logits.to(dev), temps.to(dev), tps.to(dev), tks.to(dev), mps.to(dev), u.to(dev),
                     use_top_k=True, use_top_p=bool(flags & 4), use_min_p=bool(flags & 8),
                     max_top_k=int(tks.max())).cpu().numpy()
        assert np.array_equal(got, want), (case, b, v, flags, kind, kmax)


@pytest.mark.parametrize("path", ["topk", "chain", "greedy"])
def test_sampler_unaligned_rows_with_infinities_bitexact(dev, path):
    """Logit rows that do not start on a 16-byte boundary (a column-offset
    view with an odd row stride, so every segment kernel takes its id-by-id
    loads) holding +inf, -inf and NaN: the top-k path, the multi-workgroup
    chain and the all-greedy path equal the C oracle on every row.  Rows
    whose largest logit scales to a non-finite value (+inf, -inf, or a
    finite logit past fp32's range at T 0.45) give every candidate mass 0,
    and the draw takes the first candidate in rank order."""
    import oracle.sampler as S
    from xvllm.sampler import sample

    g = gen(4242 + len(path))
    b, v = 40, 50021
    base = _sampler_case(g, b, v + 3, std=1.0)
    base[0, 1 + 7] = float("inf")             # one +inf: it takes all the mass
    base[1, 1 : 1 + v // 2] = float("-inf")   # half the row at -inf
    base[2, 1 + 100 : 1 + 200] = float("nan")
    base[3, 1:] = float("-inf")               # -inf only but one finite logit
    base[3, 1 + 4321] = 0.5
    base[4, 1 + 9] = base[4, 1 + 90] = float("inf")  # two +inf: the lower id leads
    base[5, 1:] = float("nan")                # NaN only
    base[6, 1 + 40000 :] = float("-inf")
    base[7, 1 + 555] = base[7, 1 + 556] = 3.0e38  # finite, but past fp32's range once divided by T
    base[8, 1] = float("nan")                     # -inf only but a NaN in front
    base[8, 2:] = float("-inf")
    logits = base.to(dev)[:, 1 : 1 + v]       # rows start 2 bytes past 16-byte alignment
    assert logits.data_ptr() % 16 != 0 and logits.stride(0) == v + 3
    bits = base[:, 1 : 1 + v].contiguous().view(torch.int16).numpy().view(np.uint16)
    temps = torch.rand(b, generator=g) + 0.4
    tps = torch.rand(b, generator=g) * 0.5 + 0.45
    tks = torch.randint(1, 65, (b,), generator=g, dtype=torch.int32)
    mps = torch.rand(b, generator=g) * 0.2
    u = torch.rand(b, generator=g)
    temps[7] = 0.45
    if path == "greedy":
        temps.zero_()
        flags, kw = 1, dict(all_greedy=True)
    elif path == "topk":
        temps[::6] = 0.0
        flags, kw = 2 | 4 | 8, dict(use_top_k=True, use_top_p=True, use_min_p=True, max_top_k=64)
    else:
        temps[::6] = 0.0
        flags, kw = 4 | 8, dict(use_top_p=True, use_min_p=True)
    want = S.sample(bits, temps.numpy(), tps.numpy(), tks.numpy(), mps.numpy(), u.numpy(), flags)
    got = sample(logits, temps.to(dev), tps.to(dev), tks.to(dev), mps.to(dev), u.to(dev), **kw)
    torch.cuda.synchronize()
    print(f"unaligned rows {path}", flush=True)
    assert np.array_equal(got.cpu().numpy(), want), f"{got.cpu().numpy()} vs {want}"


@pytest.mark.parametrize("path", ["topk", "chain", "one_workgroup"])
def test_sampler_parameter_edges_bitexact(dev, path):
    """Sampling parameters at their edges, row by row: top-p 0, 1e-9 and 1;
    min-p 1 and 1.5 (only the largest logit reaches it); top-k V, above V,
    negative and 1; temperatures just above the greedy threshold (1.1e-5) and
    very large (1e4, near-flat masses); uniforms 0 and just below 1.  Every
    path equals the C oracle."""
    import oracle.sampler as S
    from xvllm.sampler import sample

    g = gen(515 + len(path))
    b, v = 24, 32000
    logits = _sampler_case(g, b, v, std=1.5)
    temps = torch.full((b,), 0.8)
    tps = torch.full((b,), 0.9)
    tks = torch.full((b,), 40, dtype=torch.int32)
    mps = torch.full((b,), 0.05)
    u = torch.rand(b, generator=g)
    tps[0], tps[1], tps[2] = 0.0, 1e-9, 1.0
    mps[3], mps[4] = 1.0, 1.5
    temps[5], temps[6], temps[7] = 1.1e-5, 1e4, 3.0
    u[8], u[9] = 0.0, float(np.nextafter(np.float32(1), np.float32(0)))
    tps[10], mps[10] = 1.0, 0.0                       # no cut but top-k
    logits[11] = logits[11, 0]                        # one value repeated: a single tie group
    temps[12] = 1e4
    tps[12] = 0.999
    if path == "topk":  # every k within the path's bound
        tks[13], tks[14] = 1, 64
        flags, kw = 2 | 4 | 8, dict(use_top_k=True, use_top_p=True, use_min_p=True, max_top_k=64)
    else:
        tks[13], tks[14], tks[15], tks[16] = v, v + 5, -3, 1
        flags, kw = 2 | 4 | 8, dict(use_top_k=True, use_top_p=True, use_min_p=True)
        if path == "one_workgroup":
            kw["multi_workgroup"] = False
    want = S.sample(logits.view(torch.int16).numpy().view(np.uint16), temps.numpy(), tps.numpy(), tks.numpy(),
                    mps.numpy(), u.numpy(), flags)
    got = sample(logits.to(dev), temps.to(dev), tps.to(dev), tks.to(dev), mps.to(dev), u.to(dev), **kw)
    torch.cuda.synchronize()
    print(f"parameter edges {path}", flush=True)
    assert np.array_equal(got.cpu().numpy(), want), f"{got.cpu().numpy()} vs {want}"


@pytest.mark.parametrize("v", [1, 2, 7, 9, 33])
def test_sampler_tiny_vocabularies_bitexact(dev, v):
    """Vocabularies smaller than one 8-id vector or a few of them: the greedy,
    top-k, multi-workgroup and one-workgroup paths equal the C oracle."""
    import oracle.sampler as S
    from xvllm.sampler import sample

    g = gen(808 + v)
    b = 6
    logits = _sampler_case(g, b, v, std=1.0)
    if v > 2:
        logits[1, 1] = float("nan")
    temps = torch.rand(b, generator=g) + 0.5
    temps[0] = 0.0
    tps = torch.full((b,), 0.8)
    tks = torch.full((b,), 3, dtype=torch.int32)
    mps = torch.full((b,), 0.05)
    u = torch.rand(b, generator=g)
    bits = logits.view(torch.int16).numpy().view(np.uint16)
    cases = [(1, dict(all_greedy=True)),
             (2 | 4 | 8, dict(use_top_k=True, use_top_p=True, use_min_p=True, max_top_k=3)),
             (2 | 4 | 8, dict(use_top_k=True, use_top_p=True, use_min_p=True)),
             (4, dict(use_top_p=True, multi_workgroup=False))]
    for flags, kw in cases:
        t = torch.zeros(b) if flags == 1 else temps
        want = S.sample(bits, t.numpy(), tps.numpy(), tks.numpy(), mps.numpy(), u.numpy(), flags)
        got = sample(logits.to(dev), t.to(dev), tps.to(dev), tks.to(dev), mps.to(dev), u.to(dev), **kw)
        torch.cuda.synchronize()
        print(f"tiny vocabulary {v} {kw}", flush=True)
        assert np.array_equal(got.cpu().numpy(), want), (kw, got.cpu().numpy(), want)


def test_sampler_topk_path_many_rows_agrees(dev):
    """1800 rows at V 151936 with max_top_k 64 (past the 1514 rows the top-k
    path's lists fit while the sampled region was sized for 128 rows): the
    top-k path gives the ids of the one-workgroup path, which the oracle pins
    elsewhere."""
    from xvllm.sampler import sample

    g = gen(1800)
    b, v = 1800, 151936
    logits = _sampler_case(g, b, v, std=1.0).to(dev)
    temps = (torch.rand(b, generator=g) + 0.4).to(dev)
    tps = (torch.rand(b, generator=g) * 0.5 + 0.45).to(dev)
    tks = torch.randint(1, 65, (b,), generator=g, dtype=torch.int32).to(dev)
    u = torch.rand(b, generator=g).to(dev)
    kw = dict(use_top_k=True, use_top_p=True)
    got = sample(logits, temps, tps, tks, None, u, **kw, max_top_k=64)
    want = sample(logits, temps, tps, tks, None, u, **kw, multi_workgroup=False)
    torch.cuda.synchronize()
    print("top-k path 1800 rows", flush=True)
    assert torch.equal(got, want), torch.nonzero(got != want)[:8].flatten().tolist()


@pytest.mark.parametrize("nbytes,shape", [(16, 0), (4096 * 16 + 48, 0), (4096 * 16 + 48, 1), (3 << 20, 1)])
def test_stream_copy(dev, nbytes, shape):
    """The benchmark's copy yardstick copies exactly (both launch shapes, a
    ragged tail) and writes nothing past the end."""
    from xvllm import _C

    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=dev)
    dst = torch.zeros(nbytes + 64, dtype=torch.uint8, device=dev)
    _C.check(_C.lib().xv_stream_copy(src.data_ptr(), dst.data_ptr(), nbytes, shape,
                                     torch.cuda.current_stream().cuda_stream), "xv_stream_copy")
    torch.cuda.synchronize()
    assert torch.equal(dst[:nbytes], src)
    assert int(dst[nbytes:].count_nonzero()) == 0


def _expected_parts(ctx: int, hkv: int, max_blocks: int, slots: int = 1024) -> list[int]:
    """Partials per kv head of one sequence (B 1, 16-token blocks), from the
    range rule: the host bound lmin = max(4, ceil(max_blocks / 128)) pages
    (129 partial slots at B 1) gives max_parts = ceil(max_blocks / lmin) + 1
    slots and waves = min(slots, ceil(hkv * max_blocks / lmin)); the kernel
    takes ranges of L = max(4, ceil(np / (max_parts - 1)), ceil(total /
    waves)) pages over the flattened (kv head, page) space, np the sequence's
    pages."""
    lmin = max(4, -(-max_blocks // 128))
    max_parts = -(-max_blocks // lmin) + 1
    np_ = -(-ctx // 16)
    total = hkv * np_
    waves = min(slots, -(-(hkv * max_blocks) // lmin))
    L = max(4, -(-np_ // (max_parts - 1)), -(-total // waves))
    return [(h * np_ + np_ - 1) // L - (h * np_) // L + 1 for h in range(hkv)]


@pytest.mark.parametrize("ctx,nparts", [(2048, 32), (2060, 33), (4096, 64), (4100, 65)])
def test_paged_decode_merge_partial_count_boundaries(dev, ctx, nparts):
    """One sequence whose kv-head segments split into exactly 32, 33, 64 and
    65 partials: the merge's batch boundaries (32 partials per batch of
    loads, two batches in flight).  The partial counts the kernel recorded are
    read back from the workspace (its first B x Hkv int32 words) and must be
    the expected ones, so each case really sits on its boundary."""
    from xvllm.layers.attention import decode_workspace, paged_decode_attention

    hq, hkv, d = 32, 8, 128
    assert set(_expected_parts(ctx, hkv, (ctx + 15) // 16)) == {nparts}
    g = gen(ctx)
    need = (ctx + 15) // 16
    kc, vc, bt, sl = make_paged([ctx], need + 8, hkv, d, g)
    q = randn_bf16((1, hq, d), g)
    out = paged_decode_attention(q.view(1, -1).to(dev), kc.to(dev), vc.to(dev), bt.to(dev), sl.to(dev), hq, hkv, d)
    torch.cuda.synchronize()
    ws = decode_workspace(dev, 0)
    recorded = ws[: hkv * 4].view(torch.int32).cpu().tolist()
    assert recorded == [nparts] * hkv
    want = O.paged_decode_attention(f32(q), f32(kc), f32(vc), bt.numpy(), sl.numpy())
    _close(f32(out).reshape(1, hq, d), want)


@pytest.mark.parametrize("ctx,width", [(512, 2048), (100, 4096), (4100, 8192)])
def test_paged_decode_ranges_follow_actual_lengths(dev, ctx, width):
    """A block table far wider than the sequence (a graph captured for long
    contexts, a cascade suffix): the ranges follow the sequence's own pages,
    not the table width, so short rows still spread over many waves.  The
    recorded partial counts equal the rule's and the output the oracle's."""
    from xvllm.layers.attention import decode_workspace, paged_decode_attention

    hq, hkv, d = 32, 8, 128
    want_parts = _expected_parts(ctx, hkv, width)
    g = gen(ctx + width)
    need = (ctx + 15) // 16
    kc, vc, bt, sl = make_paged([ctx], need + 8, hkv, d, g)
    wide = torch.full((1, width), -1, dtype=torch.int32)
    wide[:, : bt.shape[1]] = bt
    q = randn_bf16((1, hq, d), g)
    out = paged_decode_attention(q.view(1, -1).to(dev), kc.to(dev), vc.to(dev), wide.to(dev), sl.to(dev), hq, hkv, d)
    torch.cuda.synchronize()
    ws = decode_workspace(dev, 0)
    assert ws[: hkv * 4].view(torch.int32).cpu().tolist() == want_parts
    want = O.paged_decode_attention(f32(q), f32(kc), f32(vc), bt.numpy(), sl.numpy())
    _close(f32(out).reshape(1, hq, d), want)
