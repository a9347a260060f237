"""Paged decode attention over seeded random configurations, through the C
ABI, against the numpy oracle: GQA group, kv heads, cache block size, batch,
context lengths (empty and one-token rows included), block tables wider than
the rows need (a graph captured for long contexts), both page memory orders,
and bf16 or fp8 (e4m3fn) pages.  Pool rows no sequence uses hold NaN, so a
read past a row's end shows in the output.  The cascade (shared-prefix)
decode gets the same treatment with random groups of rows sharing leading
blocks, and prefill / chunked prefill with random query and cached-prefix
lengths.  Tolerance rtol/atol 2e-2 (bf16 output, fp32 accumulate); fp8
pages are compared with the oracle over the dequantized pages."""
import numpy as np
import pytest
import torch

import oracle.ops as O
from helpers import f32, make_paged, randn_bf16

pytestmark = pytest.mark.gpu


def _close(got, want, rtol=2e-2, atol=2e-2):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert np.isfinite(got).all(), "non-finite output"
    err = np.abs(got - want) - (atol + rtol * np.abs(want))
    assert (err <= 0).all(), f"max excess {err.max():.4g} at {np.unravel_index(err.argmax(), err.shape)}"


def _draw(rng: np.random.Generator) -> dict:
    group = int(rng.choice([1, 2, 4, 8]))
    hkv = int(rng.choice([1, 2, 8])) if group < 8 else int(rng.choice([1, 8]))
    block = int(rng.choice([16, 32, 64, 256]))
    bsz = int(rng.integers(1, 25))
    ctx = rng.integers(0, 3001, bsz)
    ctx[rng.random(bsz) < 0.1] = 0
    ctx[rng.random(bsz) < 0.1] = 1
    if ctx.max() == 0:
        ctx[0] = int(rng.integers(1, 3001))
    return {"group": group, "hkv": hkv, "block": block, "ctx": [int(c) for c in ctx],
            "wide": int(rng.choice([0, 0, 1, 8])), "layout": str(rng.choice(["nhd", "hnd"])),
            "fp8": bool(rng.random() < 0.35)}


@pytest.mark.parametrize("seed", range(48))
def test_paged_decode_random_configurations(dev, seed):
    from xvllm.layers.attention import paged_decode_attention

    rng = np.random.default_rng(1000 + seed)
    c = _draw(rng)
    print(f"decode random seed {seed}: {c}", flush=True)
    hq, hkv, block, ctx, d = c["group"] * c["hkv"], c["hkv"], c["block"], c["ctx"], 128
    g = torch.Generator().manual_seed(seed)
    need = [(n + block - 1) // block for n in ctx]
    kc, vc, bt, sl = make_paged(ctx, sum(need) + 3, hkv, d, g, page=block)
    if c["wide"]:  # a table wider than any row needs: the unused entries hold -1
        wide = torch.full((len(ctx), bt.shape[1] * (c["wide"] + 1) + 5), -1, dtype=torch.int32)
        wide[:, : bt.shape[1]] = bt
        bt = wide
    q = randn_bf16((len(ctx), hq, d), g)
    kw = {}
    if c["fp8"]:
        ks, vs = 0.05, 0.3
        kq = O.quantize_fp8(f32(kc), np.float32(1.0) / np.float32(ks))  # NaN rows stay NaN codes
        vq = O.quantize_fp8(f32(vc), np.float32(1.0) / np.float32(vs))
        kref, vref = O.dequantize_fp8(kq, ks), O.dequantize_fp8(vq, vs)
        kd = torch.from_numpy(np.ascontiguousarray(kq)).view(torch.float8_e4m3fn)
        vd = torch.from_numpy(np.ascontiguousarray(vq)).view(torch.float8_e4m3fn)
        kw = {"k_scale": ks, "v_scale": vs}
    else:
        kref, vref, kd, vd = f32(kc), f32(vc), kc, vc
    kd, vd = kd.to(dev), vd.to(dev)
    if c["layout"] == "hnd":  # [block][kv head][token][d] in memory, the same logical view
        kd, vd = kd.transpose(1, 2).contiguous().transpose(1, 2), vd.transpose(1, 2).contiguous().transpose(1, 2)
    want = O.paged_decode_attention(f32(q), kref, vref, bt.numpy(), sl.numpy())
    out = paged_decode_attention(q.view(len(ctx), -1).to(dev), kd, vd, bt.to(dev), sl.to(dev), hq, hkv, d, **kw)
    torch.cuda.synchronize()
    got = f32(out).reshape(len(ctx), hq, d)
    _close(got, want)
    assert (got[np.asarray(ctx) == 0] == 0).all()


@pytest.mark.parametrize("seed", range(16))
def test_cascade_decode_random_configurations(dev, seed):
    from test_gpu_cascade import _plan, _shared_case
    from xvllm.layers.attention import cascade_decode_attention

    rng = np.random.default_rng(2000 + seed)
    group = int(rng.choice([1, 2, 4, 8]))
    hkv = int(rng.choice([2, 8]))
    hq, d = group * hkv, 128
    block = int(rng.choice([16, 32, 256]))
    bsz = int(rng.integers(2, 21))
    ctx = [int(x) for x in rng.integers(1, 2500, bsz)]
    rows = rng.permutation(bsz).tolist()
    shares, o = [], 0
    for _ in range(int(rng.integers(1, 4))):  # up to three groups of 2..6 rows
        m = int(rng.integers(2, 7))
        if o + m > bsz:
            break
        grp = rows[o : o + m]
        o += m
        nb = max(1, min(ctx[r] for r in grp) // block)  # blocks every member has fully written
        shares.append((grp, int(rng.integers(1, nb + 1))))
    fp8 = bool(rng.random() < 0.4)
    print(f"cascade random seed {seed}: G {group} hkv {hkv} block {block} B {bsz} groups "
          f"{[(len(r), n) for r, n in shares]} fp8 {fp8}", flush=True)
    g = torch.Generator().manual_seed(seed)
    bt, pool = _shared_case(g, ctx, shares, block)
    kc, vc = randn_bf16((pool, block, hkv, d), g), randn_bf16((pool, block, hkv, d), g)
    q = randn_bf16((bsz, hq, d), g)
    sl = torch.tensor(ctx, dtype=torch.int32)
    plan, pre = _plan(bt, ctx, block, dev, groups=4, max_rows=128 // group)
    kw = {}
    if fp8:
        ks, vs = 0.05, 0.3
        kq = O.quantize_fp8(f32(kc), np.float32(1.0) / np.float32(ks))
        vq = O.quantize_fp8(f32(vc), np.float32(1.0) / np.float32(vs))
        kref, vref = O.dequantize_fp8(kq, ks), O.dequantize_fp8(vq, vs)
        kd = torch.from_numpy(np.ascontiguousarray(kq)).view(torch.float8_e4m3fn)
        vd = torch.from_numpy(np.ascontiguousarray(vq)).view(torch.float8_e4m3fn)
        kw = {"k_scale": ks, "v_scale": vs}
    else:
        kref, vref, kd, vd = f32(kc), f32(vc), kc, vc
    want = O.paged_decode_attention(f32(q), kref, vref, bt.numpy(), sl.numpy())
    out = cascade_decode_attention(q.view(bsz, -1).to(dev), kd.to(dev), vd.to(dev), bt.to(dev), sl.to(dev), plan,
                                   hq, hkv, d, **kw)
    torch.cuda.synchronize()
    _close(f32(out).reshape(bsz, hq, d), want)


@pytest.mark.parametrize("seed", range(24))
def test_prefill_random_configurations(dev, seed):
    """Prefill and chunked prefill: dense q/k/v rows, or a cached prefix plus
    the chunk read through block tables of a random block size and page
    order, bf16 or fp8 pages (gathered into bf16 rows first)."""
    from xvllm.layers.attention import prefill_attention

    rng = np.random.default_rng(3000 + seed)
    group = int(rng.choice([1, 2, 4, 8]))
    hkv = int(rng.choice([1, 2, 8])) if group < 8 else 8
    hq, d = group * hkv, 128
    bsz = int(rng.integers(1, 9))
    qlens = [int(x) for x in rng.integers(0, 400, bsz)]
    paged = bool(rng.random() < 0.7)
    pre = [int(x) for x in rng.integers(0, 1500, bsz)] if paged else [0] * bsz
    if max(qlens) == 0:
        qlens[0] = 1
    klens = [p_ + q_ for p_, q_ in zip(pre, qlens)]
    block = int(rng.choice([16, 32, 64, 256]))
    layout = str(rng.choice(["nhd", "hnd"]))
    fp8 = paged and bool(rng.random() < 0.35)
    print(f"prefill random seed {seed}: G {group} hkv {hkv} q {qlens} k {klens} paged {paged} block {block} "
          f"{layout} fp8 {fp8}", flush=True)
    g = torch.Generator().manual_seed(seed)
    cu_q = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(klens)]).astype(np.int32)
    q = randn_bf16((int(cu_q[-1]), hq, d), g)
    tq, tk = torch.from_numpy(cu_q).to(dev), torch.from_numpy(cu_k).to(dev)
    if paged:
        need = sum((c + block - 1) // block for c in klens)
        kc, vc, bt, _ = make_paged(klens, need + 3, hkv, d, g, page=block)
        kw = {}
        if fp8:
            ks, vs = 0.05, 0.3
            kq = O.quantize_fp8(f32(kc), np.float32(1.0) / np.float32(ks))
            vq = O.quantize_fp8(f32(vc), np.float32(1.0) / np.float32(vs))
            kref, vref = O.dequantize_fp8(kq, ks), O.dequantize_fp8(vq, vs)
            kd = torch.from_numpy(np.ascontiguousarray(kq)).view(torch.float8_e4m3fn)
            vd = torch.from_numpy(np.ascontiguousarray(vq)).view(torch.float8_e4m3fn)
            kw = {"max_seqlen_k": max(klens), "kv_scale": (ks, vs)}
        else:
            kref, vref, kd, vd = f32(kc), f32(vc), kc, vc
        kd, vd = kd.to(dev), vd.to(dev)
        if layout == "hnd":
            kd, vd = kd.transpose(1, 2).contiguous().transpose(1, 2), vd.transpose(1, 2).contiguous().transpose(1, 2)
        want = O.prefill_attention(f32(q), cu_q, cu_k, k_cache=kref, v_cache=vref, block_tables=bt.numpy())
        out = prefill_attention(q.to(dev), None, None, tq, tk, max(qlens), hq, hkv, d, k_cache=kd, v_cache=vd,
                                block_tables=bt.to(dev), **kw)
    else:
        k = randn_bf16((int(cu_k[-1]), hkv, d), g)
        v = randn_bf16((int(cu_k[-1]), hkv, d), g)
        want = O.prefill_attention(f32(q), cu_q, cu_k, k=f32(k), v=f32(v))
        out = prefill_attention(q.to(dev), k.to(dev), v.to(dev), tq, tk, max(qlens), hq, hkv, d)
    torch.cuda.synchronize()
    _close(f32(out).reshape(-1, hq, d), want)
