#!/usr/bin/env python3
"""Benchmark of the decode hot path on one MI355X.

Workload: paged GQA decode attention at the Qwen3-8B
attention shape -- 32 q heads / 8 kv heads, head_dim 128, bf16, batch 64,
context lengths U[512, 4096], 16-token pages, block tables a random
permutation of a pool 1.25x the pages needed, in KVPool's default page
memory order ([page][kv head][token][d]; the reference's order is timed
beside it in `sweep`).  One "step" is one decode
attention call over the batch (split-KV kernel + split merge).  Four layers'
worth of KV pools are cycled so that a step never finds its KV in the 256 MB
MALL, as in a real multi-layer decode step.

Prints one JSON line.  value = algorithmic HBM bytes per call / time per call
(GB/s), the K timed calls captured in one HIP graph as the decode step runs
them (the same calls launched one by one from Python are reported beside).
roofline uses the same numbers against the 8 TB/s HBM peak.
cpu_baseline = the numpy oracle (tests' checker) timed on a bounded sample of
the same workload on the host, one thread.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "xixi-vllm_amd"))

HBM_PEAK_GBS = 8000.0
# HBM bytes per paged_decode_kernel launch at config 2, from rocprofv3 --pmc
# FETCH_SIZE / WRITE_SIZE scaled by a 1 GiB copy (profiles/paged_decode_attention_config2.md):
# 2 x 319019.9 KiB read (FETCH_SIZE counts half on this part) + 1722.5 KiB written;
# on fp8 pages 2 x 160178.0 + 2831.6 KiB.
MEASURED_TRAFFIC_BYTES = int((2 * 319019.9 + 1722.5) * 1024)
MEASURED_TRAFFIC_BYTES_FP8 = int((2 * 160178.0 + 2831.6) * 1024)
HQ, HKV, D, PAGE = 32, 8, 128, 16


def algo_bytes(ctx: list[int], hq=HQ, hkv=HKV, d=D, kv_elem: int = 2) -> int:
    """sum ctx*Hkv*D*2(K,V)*kv_elem B + q and o (2*B*Hq*D*2B) + block-table ints
    + seqlens (kv_elem 2: bf16 pages, 1: fp8 pages)."""
    kv = sum(ctx) * hkv * d * 2 * kv_elem
    qo = 2 * len(ctx) * hq * d * 2
    bt = sum((c + PAGE - 1) // PAGE for c in ctx) * 4
    return kv + qo + bt + 4 * len(ctx)


FP8_SCALE = 0.125  # fp8 pages: N(0,1) values stored as e4m3fn(x * 8), k_scale = v_scale = 1/8


def make_case(torch, ctx: list[int], layers: int, dev, seed: int, layout: str = "hnd", fp8: bool = False):
    """Per layer: q, K pool, V pool, block tables, seqlens.  layout "hnd" (the
    default KVPool order) stores [NB, Hkv, BS, D] and passes the transposed
    view with the reference's logical shape [NB, BS, Hkv, D]; "nhd" is the
    reference's memory order.  fp8: e4m3fn pages (the optional pool format)."""
    g = torch.Generator().manual_seed(seed)
    need = [(c + PAGE - 1) // PAGE for c in ctx]
    pool = math.ceil(1.25 * sum(need))
    max_blocks = max(need)
    cases = []
    for layer in range(layers):
        perm = torch.randperm(pool, generator=g)
        bt = torch.full((len(ctx), max_blocks), -1, dtype=torch.int32)
        o = 0
        for b, n in enumerate(need):
            bt[b, :n] = perm[o : o + n].to(torch.int32)
            o += n
        gd = torch.Generator(device=dev).manual_seed(seed * 100 + layer)
        shape = (pool, PAGE, HKV, D) if layout == "nhd" else (pool, HKV, PAGE, D)
        kc = torch.randn(shape, generator=gd, device=dev).to(torch.bfloat16)
        vc = torch.randn(shape, generator=gd, device=dev).to(torch.bfloat16)
        if fp8:
            kc = (kc.float() / FP8_SCALE).to(torch.float8_e4m3fn)
            vc = (vc.float() / FP8_SCALE).to(torch.float8_e4m3fn)
        if layout == "hnd":
            kc, vc = kc.transpose(1, 2), vc.transpose(1, 2)
        q = torch.randn((len(ctx), HQ * D), generator=gd, device=dev).to(torch.bfloat16)
        cases.append((q, kc, vc, bt.to(dev), torch.tensor(ctx, dtype=torch.int32, device=dev)))
    return cases


def _scales(kc) -> dict:
    import torch

    return {"k_scale": FP8_SCALE, "v_scale": FP8_SCALE} if kc.dtype == torch.float8_e4m3fn else {}


def time_decode(torch, cases, steps: int, warmup: int):
    """Timed region of the headline: `steps` decode-attention calls (cycling
    the KV pools) captured in one HIP graph, as the decode step runs them, and
    replayed once between two syncs.  `warmup` calls run eagerly first (they
    also size the decode workspace).  Returns (ms per call from HIP events,
    wall seconds of the replay, ms per call of the same calls launched
    eagerly from Python)."""
    from xvllm.layers.attention import paged_decode_attention

    outs = [torch.empty_like(c[0]) for c in cases]

    def step(i):
        q, kc, vc, bt, sl = cases[i % len(cases)]
        paged_decode_attention(q, kc, vc, bt, sl, HQ, HKV, D, out=outs[i % len(cases)], **_scales(kc))

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # the same calls launched one by one from Python (reported beside)
    e0.record()
    for i in range(steps):
        step(i)
    e1.record()
    torch.cuda.synchronize()
    eager_ms = e0.elapsed_time(e1) / steps
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(steps):
            step(i)
    graph.replay()  # first replay: uploads the graph
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record()
    graph.replay()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return e0.elapsed_time(e1) / steps, wall, eager_ms


def time_decode_graph(torch, cases, iters: int = 48) -> float:
    """Device time per decode-attention call (us), calls captured in a HIP
    graph as the decode step runs them, cycling the cases' KV pools."""
    from xvllm.layers.attention import paged_decode_attention

    outs = [torch.empty_like(c[0]) for c in cases]
    i = [0]

    def call():
        q, kc, vc, bt, sl = cases[i[0] % len(cases)]
        paged_decode_attention(q, kc, vc, bt, sl, HQ, HKV, D, out=outs[i[0] % len(cases)], **_scales(kc))
        i[0] += 1

    return _time(torch, call, iters=iters, warmup=len(cases))


def _time(torch, fn, iters=50, warmup=5):
    """Device time per call of fn (us): `iters` calls captured in one HIP
    graph and replayed, so host-side launch cost (Python op wrappers) never
    leaves the GPU idle between kernels."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(iters):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    graph.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters * 1e3  # us


MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16


def prefill_suite(torch, dev, iters: int = 20) -> dict:
    """Prefill attention tile (MFMA-bound) at the Qwen3-8B attention shape:
    causal flops = 4*Hq*D*sum(visible keys per query) against the dense bf16
    MFMA peak.  Cases: a plain causal batch with config-4 prompt lengths
    (16 sequences, U[128, 2048]); a chunked prefill of 512 new tokens per
    sequence over a paged cached prefix U[512, 2048]; one 8192-token prompt."""
    from xvllm.layers.attention import prefill_attention

    g = torch.Generator(device=dev).manual_seed(11)
    gc = torch.Generator().manual_seed(11)
    rnd = lambda *shape: torch.randn(shape, generator=g, device=dev).to(torch.bfloat16)
    out = {}

    def rec(name, us, flops, tokens):
        tf = flops / (us * 1e-6) / 1e12
        out[name] = {"us": round(us, 1), "TFLOP/s": round(tf, 1), "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
                     "flops": flops, "q_tokens": tokens}

    def dense_case(qlens):
        cu = torch.tensor([0] + list(torch.tensor(qlens).cumsum(0).tolist()), dtype=torch.int32, device=dev)
        T = int(cu[-1])
        qkv = rnd(T, (HQ + 2 * HKV) * D)
        q = qkv[:, : HQ * D]
        k = qkv[:, HQ * D : (HQ + HKV) * D].view(T, HKV, D)
        v = qkv[:, (HQ + HKV) * D :].view(T, HKV, D)
        fn = lambda: prefill_attention(q, k, v, cu, cu, max(qlens), HQ, HKV, D)
        flops = 4 * HQ * D * sum(L * (L + 1) // 2 for L in qlens)
        return fn, flops, T

    qlens = torch.randint(128, 2049, (16,), generator=gc).tolist()
    fn, fl, T = dense_case(qlens)
    rec("prefill_causal_16seq_U128_2048", _time(torch, fn, iters), fl, T)
    fn, fl, T = dense_case([8192])
    rec("prefill_causal_1seq_8192", _time(torch, fn, iters), fl, T)
    # chunked prefill: 512 new tokens over a cached prefix, keys through the block table
    pre = torch.randint(512, 2049, (16,), generator=gc).tolist()
    new = [512] * 16
    klens = [p_ + n_ for p_, n_ in zip(pre, new)]
    need = [(k_ + PAGE - 1) // PAGE for k_ in klens]
    nb = sum(need) + 8
    kc, vc = rnd(nb, PAGE, HKV, D), rnd(nb, PAGE, HKV, D)
    perm = torch.randperm(nb, generator=gc)
    bt = torch.full((16, max(need)), -1, dtype=torch.int32)
    o_ = 0
    for b, n_ in enumerate(need):
        bt[b, :n_] = perm[o_ : o_ + n_].to(torch.int32)
        o_ += n_
    bt = bt.to(dev)
    cu_q = torch.tensor([0] + torch.tensor(new).cumsum(0).tolist(), dtype=torch.int32, device=dev)
    cu_k = torch.tensor([0] + torch.tensor(klens).cumsum(0).tolist(), dtype=torch.int32, device=dev)
    q = rnd(sum(new), HQ * D)
    fn = lambda: prefill_attention(q, None, None, cu_q, cu_k, 512, HQ, HKV, D, k_cache=kc, v_cache=vc,
                                   block_tables=bt)
    fl = 4 * HQ * D * sum(sum(p_ + i + 1 for i in range(n_)) for p_, n_ in zip(pre, new))
    rec("chunked_prefill_16x512_over_U512_2048_paged", _time(torch, fn, iters), fl, sum(new))
    return out


def copy_ceiling_us(torch, dev, nbytes: int) -> float:
    """Time per call (us) of the library's streaming copy moving nbytes in
    all (half read, half written), the better of its two launch shapes,
    cycling over buffer sets that together exceed the 256 MB MALL: what a
    plain transfer of a kernel's byte count reaches on this part."""
    from xvllm import _C

    half = (nbytes // 2) // 16 * 16
    nsets = max(2, -(-(640 << 20) // (2 * half)))
    bufs = [(torch.empty(half, dtype=torch.uint8, device=dev).fill_(1), torch.empty(half, dtype=torch.uint8, device=dev))
            for _ in range(nsets)]
    best = float("inf")
    for shape in (0, 1):
        it = [0]

        def step():
            src, dst = bufs[it[0] % nsets]
            it[0] += 1
            _C.check(_C.lib().xv_stream_copy(src.data_ptr(), dst.data_ptr(), half, shape,
                                             torch.cuda.current_stream().cuda_stream), "xv_stream_copy")
        best = min(best, _time(torch, step))
    del bufs
    return best


def kernel_suite(torch, dev) -> dict:
    """Config 3 (fused elementwise/reduction set at Qwen3-8B width over 8192
    tokens), the sampler and the streamed decode GEMMs, each against its
    algorithmic HBM bytes."""
    import xvllm.layers.ops  # noqa: F401
    from xvllm.kv_ops import store_kvcache
    from xvllm.layers.rotary import build_cos_sin_cache
    from xvllm.sampler import sample

    g = torch.Generator(device=dev).manual_seed(3)
    T, H, HQ_, HKV_, D_, I = 8192, 4096, 32, 8, 128, 12288
    rnd = lambda *shape: torch.randn(shape, generator=g, device=dev).to(torch.bfloat16)
    out = {}

    def rec(name, us, nbytes, ceiling=False):
        out[name] = {"us": round(us, 2), "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "bytes": nbytes}
        if ceiling:
            cu = copy_ceiling_us(torch, dev, nbytes)
            out[name]["copy_us"] = round(cu, 2)
            out[name]["frac_of_copy"] = round(cu / us, 4)

    # Each op cycles through enough input sets that one set plus the others
    # exceed the 256 MB MALL: every call streams its operands from HBM.
    def cycle(fns):
        it = [0]

        def step():
            fns[it[0] % len(fns)]()
            it[0] += 1
        return step

    w = (torch.randn(H, generator=g, device=dev) * 0.1 + 1).to(torch.bfloat16)
    sets = [(rnd(T, H), rnd(T, H)) for _ in range(2)]
    rec("fused_add_rmsnorm_T8192_H4096",
        _time(torch, cycle([lambda x=x, r=r: torch.ops.vllm.fused_add_rmsnorm(x, r, w, 1e-6) for x, r in sets])),
        T * H * 2 * 4 + H * 2, ceiling=True)
    del sets
    qw = (torch.randn(D_, generator=g, device=dev) * 0.1 + 1).to(torch.bfloat16)
    kw = (torch.randn(D_, generator=g, device=dev) * 0.1 + 1).to(torch.bfloat16)
    cs = build_cos_sin_cache(D_, 32768, 1e6).to(dev)
    fns = []
    for _ in range(3):
        qkv = rnd(T, (HQ_ + 2 * HKV_) * D_)
        q = qkv[:, : HQ_ * D_].view(T, HQ_, D_)
        k = qkv[:, HQ_ * D_ : (HQ_ + HKV_) * D_].view(T, HKV_, D_)
        pos = torch.randint(0, 32768, (T,), generator=g, device=dev)
        fns.append(lambda q=q, k=k, pos=pos: torch.ops.xv.qk_norm_rope(q, k, qw, kw, 1e-6, pos, cs))
    rec("qk_norm_rope_T8192_32q8kv", _time(torch, cycle(fns)), T * (HQ_ + HKV_) * D_ * 2 * 2 + 8 * T + T * D_ * 4,
        ceiling=True)
    del fns, qkv, q, k
    xs = [rnd(T, 2 * I) for _ in range(2)]
    rec("silu_and_mul_T8192_I12288", _time(torch, cycle([lambda x=x: torch.ops.vllm.silu_and_mul(x) for x in xs])),
        T * 3 * I * 2, ceiling=True)
    del xs
    nb = 1024
    fns = []
    for _ in range(5):
        kk, vv = rnd(T, HKV_, D_), rnd(T, HKV_, D_)
        kc = torch.zeros((nb, PAGE, HKV_, D_), dtype=torch.bfloat16, device=dev)
        vc = torch.zeros_like(kc)
        slots = torch.randperm(nb * PAGE, generator=g, device=dev)[:T].to(torch.int32)
        fns.append(lambda kk=kk, vv=vv, kc=kc, vc=vc, slots=slots:
                   store_kvcache(kk, vv, kc.view(-1, HKV_, D_), vc.view(-1, HKV_, D_), slots))
    rec("store_kvcache_T8192", _time(torch, cycle(fns)), 2 * T * HKV_ * D_ * 2 * 2 + 4 * T, ceiling=True)
    del fns, kc, vc, kk, vv
    V = 151936
    for bsz in (64, 256):
        logits = rnd(bsz, V)
        temps = torch.full((bsz,), 0.7, device=dev)
        tps = torch.full((bsz,), 0.9, device=dev)
        tks = torch.full((bsz,), 50, dtype=torch.int32, device=dev)
        u = torch.rand(bsz, generator=g, device=dev)
        rec(f"sampler_greedy_B{bsz}", _time(torch, lambda: sample(logits, temps, all_greedy=True), 20), bsz * V * 2)
        # max_top_k as the serving loop passes it (the reference's Batch.max_top_k)
        rec(f"sampler_k50_p0.9_B{bsz}", _time(torch, lambda: sample(logits, temps, tps, tks, None, u, use_top_k=True,
                                                                    use_top_p=True, max_top_k=50), 20), bsz * V * 2)
        if bsz in (64, 256):  # the same call without the bound: the histogram chain / one workgroup per row
            rec(f"sampler_k50_p0.9_B{bsz}_no_max_top_k",
                _time(torch, lambda: sample(logits, temps, tps, tks, None, u, use_top_k=True, use_top_p=True), 20),
                bsz * V * 2)
    # config 5's sampling: top-p 0.95 at T 1.0 over near-flat logits (as a
    # random-init LM head gives): the boundary bucket overflows LDS and the
    # row-wide radix-select path runs
    bsz = 32
    logits = (torch.randn(bsz, V, generator=g, device=dev) * 0.05).to(torch.bfloat16)
    temps = torch.ones(bsz, device=dev)
    tps = torch.full((bsz,), 0.95, device=dev)
    u = torch.rand(bsz, generator=g, device=dev)
    rec("sampler_p0.95_flat_B32", _time(torch, lambda: sample(logits, temps, tps, None, None, u, use_top_p=True), 20),
        bsz * V * 2)
    # Decode GEMMs on the weight-streaming kernel (packed weights, enough
    # weight sets cycled to pass 600 MB: past the 256 MB MALL, as the model's
    # 15 GB of weights are) against hipBLASLt over the [N, K]
    # weights (the unsplit GEMM + SiLU-and-mul kernel for gate_up, the split-K
    # bmm it replaced for down / o).  Bytes: weights + x + output.
    from xvllm.layers.linear import pack_weight, split_k_views, streamed_into_norm, streamed_silu_mul
    import torch.nn.functional as F
    for name, n, k in (("gate_up_silu", 2 * I, H), ("down_parts", H, I), ("o_parts", H, HQ_ * D_)):
        nset = max(2, -(-600_000_000 // (n * k * 2)))
        ws = [rnd(n, k) for _ in range(nset)]
        pws = [pack_weight(w_) for w_ in ws]
        for m in (8, 64):
            x = rnd(m, k)
            if name == "gate_up_silu":
                fn = lambda r, x=x: streamed_silu_mul(x, pws[r % nset])
                ref = lambda r, x=x: torch.ops.vllm.silu_and_mul(F.linear(x, ws[r % nset]))
                ob = m * n // 2 * 2
            else:
                p = streamed_into_norm(x, pws[0]).parts.shape[0]
                fn = lambda r, x=x: streamed_into_norm(x, pws[r % nset])
                ref = lambda r, x=x, p=p: torch.bmm(*split_k_views(x, ws[r % nset], p), out_dtype=torch.float32)
                ob = p * m * n * 4
            for tag, f in (("", fn), ("_hipblaslt", ref)):
                it = [0]

                def step(f=f):
                    f(it[0])
                    it[0] += 1
                rec(f"decode_gemm_{name}_M{m}{tag}", _time(torch, step), n * k * 2 + m * k * 2 + ob)
        del ws, pws
    return out


def decode_e2e(torch, dev, ctx: list[int], steps: int = 20, sampled: bool = False, fp8: bool = False,
               model=None, stream_gemms: bool = False):
    """Qwen3-8B (36 layers, random bf16 weights ~N(0,0.02)) decode step at the
    given per-sequence contexts: hipGraph replay of the decode body + LM head +
    sampler, steady state (metadata staged once).  fp8: the KV pool in the
    optional fp8 (e4m3fn) page format.  stream_gemms: the runner's opt-in
    weight-streaming decode GEMMs (packed copies of gate_up / down / o beside
    the weights; their bytes are reported).  Returns (record, model)."""
    from xvllm.batch import SeqSchedule
    from xvllm.config import QWEN3_8B
    from xvllm.kv_pool import KVPool
    from xvllm.model_runner import ModelRunner
    from xvllm.models import Qwen3ForCausalLM

    cfg = QWEN3_8B
    bsz = len(ctx)
    need = [(c + PAGE - 1) // PAGE for c in ctx]
    pool = math.ceil(1.25 * sum(need))
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(dev):
            if model is None:
                model = Qwen3ForCausalLM(cfg).random_init_(seed=0).set_split_k(SPLIT_K)
            if fp8:
                kv = KVPool(cfg, num_blocks=pool, block_size=PAGE, device=dev, dtype=torch.float8_e4m3fn,
                            k_scale=FP8_SCALE, v_scale=FP8_SCALE)
            else:
                kv = KVPool(cfg, num_blocks=pool, block_size=PAGE, device=dev, dtype=torch.bfloat16)
    finally:
        torch.set_default_dtype(torch.float32)
    if fp8:  # N(0, 1) values in fp8 at scale 1/8, one layer at a time
        for i in range(2):
            for layer in range(kv.num_layers):
                view = kv.kv_cache[i, layer]
                view.copy_((torch.randn(view.shape, device=dev) / FP8_SCALE).to(torch.float8_e4m3fn))
    else:
        kv.kv_cache.normal_()
    max_ctx = max(ctx) + 1
    runner = ModelRunner(model, kv, max_num_seqs=bsz, context_len=max_ctx, device=dev,
                         stream_decode_gemms=stream_gemms)
    g = torch.Generator().manual_seed(11)
    perm = torch.randperm(pool, generator=g).tolist()
    seqs, o = [], 0
    for i, c in enumerate(ctx):
        seqs.append(SeqSchedule(seq_id=i, token_ids=[int(torch.randint(0, cfg.vocab_size, (1,), generator=g))],
                                num_cached_tokens=c - 1, block_table=perm[o : o + need[i]],
                                temperature=0.7 if sampled else 0.0, top_p=0.9 if sampled else None,
                                top_k=50 if sampled else None))
        o += need[i]
    runner.batch.build_decode(seqs, pad_to=runner.graph_runner._pad_bs(bsz))

    def step():
        runner.decode_hidden(bsz)
        return runner.decode_sample(bsz)

    for _ in range(3):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        ids = step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    wbytes = sum(p.numel() for n, p in model.named_parameters() if "embed_tokens" not in n) * 2
    kvbytes = sum(ctx) * cfg.num_hidden_layers * cfg.num_key_value_heads * 128 * 2 * (1 if fp8 else 2)
    roof_ms = (wbytes + kvbytes) / (HBM_PEAK_GBS * 1e9) * 1e3
    runner.destroy()
    del kv, runner
    packed = model.packed_decode_bytes() if stream_gemms else 0
    if stream_gemms:
        model.pack_decode_weights(False)  # the runner's graphs are gone: drop the packed copies
    assert ids.shape[0] == bsz
    return {"batch": bsz, "mean_ctx": round(sum(ctx) / bsz, 1), "sampling": "T0.7/k50/p0.9" if sampled else "greedy",
            "kv_pages": "fp8 e4m3fn" if fp8 else "bf16",
            "dense_gemms": ("weight-streaming kernel at <= 64 rows (opt-in), packed weight copies of "
                            f"{packed} B beside the weights") if stream_gemms else "PyTorch / hipBLASLt",
            "ms_per_step": round(ms, 4), "tok_per_s": round(bsz / (ms * 1e-3), 1),
            "roofline_ms": round(roof_ms, 4), "roofline_tok_per_s": round(bsz / (roof_ms * 1e-3), 1),
            "frac_of_roofline": round(roof_ms / ms, 4), "weight_bytes": wbytes, "kv_bytes": kvbytes}, model


def decode_config5(torch, dev, steps: int = 8, warmup: int = 2, pool_layers: int = 8, attention: str = "gated",
                   model=None, fp8: bool = False):
    """Config 5: Qwen3-32B-shaped decode (64 layers, hidden 5120, 64 q / 8 kv
    heads, FFN 25600, random bf16 weights ~N(0,0.02)), batch 32 at context
    32768; 16 requests share an 8192-token random-token prefix, 16 are
    independent; top-p 0.95 (T 1.0) over the 151936 vocab with seeded draws.

    The run goes through xvllm.serving.serve: its page ledger admits the 32
    prompts in order, and the radix prefix cache hands the 15 later shared
    requests the 512 prefix pages the first one published, so the timed
    decode steps read shared pages that came from the cache.  The prompts'
    prefill (32 x 32k tokens through 64 layers) is not run: the pool holds
    synthetic N(0,1) K/V (`serve(prefilled=True)`), and each request decodes
    from its last prompt token.  The timed region is `steps` whole serving
    steps (decode graph + LM head + sampler graphs, read-back of the ids, the
    ledger's bookkeeping; one step in flight) after `warmup` steps, timed on
    the device's timeline between events recorded after each step's launches
    (idle time between steps included).
    The 64 layers' KV (275 GB per sequence, 243 GB of unique pages) does not
    fit beside the 64 GB of weights, so the pool holds `pool_layers` layers and
    layer i reads pool layer i % pool_layers: every layer streams the same
    bytes in the same pattern as with a full pool (what this leaves out: the
    real memory footprint and the TLB reach of 243 GB).  attention: "gated"
    is the runner as served (cascade groups staged, the measured gate of
    xvllm.prefix_cache choosing cascade or plain decode per step: the 8192
    shared tokens pass it), "plain" a runner without cascade groups,
    "cascade" the cascade forced.  fp8: the pool in the optional fp8
    (e4m3fn) page format."""
    from xvllm.config import QWEN3_32B
    from xvllm.kv_pool import KVPool
    from xvllm.model_runner import ModelRunner
    from xvllm.models import Qwen3ForCausalLM
    from xvllm.serving import serve

    cfg = QWEN3_32B
    bsz, ctx, prefix, shared = 32, 32768, 8192, 16
    gen = warmup + steps
    npg, ppg = ctx // PAGE, prefix // PAGE
    g = torch.Generator().manual_seed(55)
    pre_toks = torch.randint(0, cfg.vocab_size, (prefix,), generator=g).tolist()
    prompts = []
    for i in range(bsz):
        own = torch.randint(0, cfg.vocab_size, (ctx - (prefix if i < shared else 0),), generator=g).tolist()
        prompts.append((pre_toks + own) if i < shared else own)
    pages = bsz * ((ctx + gen + PAGE - 1) // PAGE) + 16
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(dev):
            if model is None:
                model = Qwen3ForCausalLM(cfg).random_init_(seed=0).set_split_k(SPLIT_K)
            if fp8:
                kv = KVPool(cfg, num_blocks=pages, block_size=PAGE, device=dev, dtype=torch.float8_e4m3fn,
                            num_layers=pool_layers, k_scale=FP8_SCALE, v_scale=FP8_SCALE)
            else:
                kv = KVPool(cfg, num_blocks=pages, block_size=PAGE, device=dev, dtype=torch.bfloat16,
                            num_layers=pool_layers)
    finally:
        torch.set_default_dtype(torch.float32)
    if fp8:
        for i in range(2):
            for layer in range(kv.num_layers):
                view = kv.kv_cache[i, layer]
                view.copy_((torch.randn(view.shape, device=dev) / FP8_SCALE).to(torch.float8_e4m3fn))
    else:
        kv.kv_cache.normal_()
    if attention not in ("gated", "plain", "cascade"):
        raise ValueError(f"attention {attention!r}")
    casc = {} if attention == "plain" else dict(cascade_groups=2, cascade_max_prefix_blocks=ppg,
                                                cascade_min_blocks=64)
    if attention == "cascade":
        casc["cascade_min_shared_bytes"] = 0
    runner = ModelRunner(model, kv, max_num_seqs=bsz, context_len=ctx + gen, device=dev,
                         sample_modes=(4,), **casc)
    runner.generator = torch.Generator(device=dev).manual_seed(5)
    seen = {}

    def after_forward(r, n_p, n_d):
        seen["cascade_rows"] = getattr(r.batch, "cascade_rows", 0)

    outs, st = serve(runner, prompts, gen, sampling=dict(temperature=1.0, top_p=0.95), max_num_seqs=bsz,
                     prefilled=True, timing_events=True, after_forward=after_forward)
    runner.destroy()
    assert st.hit_tokens == (shared - 1) * prefix, st.hit_tokens
    assert all(len(o) == gen for o in outs) and st.steps == gen
    cascade = seen["cascade_rows"] > 0
    if attention != "plain":  # 8192 shared tokens (32 / 16 MiB per layer) pass the gate
        assert seen["cascade_rows"] == shared, seen
    # device timeline from the end of the last warm-up step's launches to the
    # end of the last step's: the host's read-back clock would count the final
    # step's release of every request's pages (~15 ms of host bookkeeping), and
    # a slow host (a profiler's) could shift its starting point
    ev = st.step_events
    ms = ev[warmup - 1].elapsed_time(ev[-1]) / steps
    wbytes = sum(p.numel() for n, p in model.named_parameters() if "embed_tokens" not in n) * 2
    per_tok_layer = cfg.num_key_value_heads * 128 * 2 * (1 if fp8 else 2)
    mean_ctx = ctx + warmup + (steps + 1) / 2  # contexts of the timed steps (prompt + tokens so far)
    kv_seq = int(bsz * mean_ctx * cfg.num_hidden_layers * per_tok_layer)
    unique_tok = bsz * mean_ctx - (shared - 1) * prefix
    kv_unique = int(unique_tok * cfg.num_hidden_layers * per_tok_layer)
    kv_read = kv_unique if cascade else kv_seq  # per-step KV bytes the decode streams
    roof_ms = (wbytes + kv_read) / (HBM_PEAK_GBS * 1e9) * 1e3
    del kv
    torch.cuda.empty_cache()
    return {"model": "Qwen3-32B-shaped (64 layers, 64q/8kv, FFN 25600)", "batch": bsz, "context": ctx,
            "shared_prefix": f"{shared} requests x {prefix} tokens; {st.hit_tokens} prompt tokens' pages handed out "
                             "by the serving ledger's radix prefix cache",
            "attention": ("cascade (shared blocks read once per kv head)" if cascade else "plain paged decode")
                         + (", chosen by the runner's gate" if attention == "gated" else ", forced"),
            "kv_pages": "fp8 e4m3fn" if fp8 else "bf16", "path": "xvllm.serving.serve(prefilled=True)",
            "sampling": "top-p 0.95 (T 1.0)", "kv_pool_layers": pool_layers, "timed_steps": steps,
            "ms_per_step": round(ms, 3), "tok_per_s": round(bsz / (ms * 1e-3), 1), "weight_bytes": wbytes,
            "kv_bytes_per_seq": kv_seq, "kv_bytes_unique_pages": kv_unique, "kv_bytes_read_per_step": kv_read,
            "roofline_ms": round(roof_ms, 3), "frac_of_roofline": round(roof_ms / ms, 4),
            "achieved_GB/s": round((wbytes + kv_read) / (ms * 1e-3) / 1e9, 1)}, model


def cascade_sweep(torch, dev, iters: int = 10) -> dict:
    """Shared-prefix decode attention alone, plain against cascade, at the
    Qwen3-32B attention shape (64 q / 8 kv heads, head-major 16-token pages),
    B 32 at 32768 and at 32777 tokens: `rows` requests share the first
    `prefix` tokens (the same pages), the rest of the KV is per request.  At
    32768 tokens (2048 whole pages per row) the plain decode's stream-K ranges
    start every row's prefix at the same moment, so the rows' reads of a
    shared page arrive together and the last-level cache serves the repeats;
    one more page (32777, as a serving run's contexts fall) shifts the rows
    against each other.  Two layers of KV are cycled so that a call does not
    find the previous call's pages in the last-level cache.  us per call (one
    layer), bf16 and fp8 pages."""
    import numpy as np

    from xvllm.layers.attention import CascadePlan, cascade_decode_attention, paged_decode_attention
    from xvllm.prefix_cache import cascade_groups

    hq, hkv, d, bsz = 64, 8, 128, 32
    g = torch.Generator(device=dev).manual_seed(3)
    q = torch.randn((bsz, hq * d), generator=g, device=dev).to(torch.bfloat16)
    out = {}
    cases = [(ctx, rows, prefix) for ctx in (32768, 32777)
             for rows, prefix in ((16, 2048), (32, 2048), (16, 4096), (32, 4096), (16, 8192), (32, 8192),
                                  (16, 24576), (32, 24576), (32, 32512))]
    for ctx, rows, prefix in cases:
        sl = torch.full((bsz,), ctx, dtype=torch.int32, device=dev)
        npg, ppg = (ctx + PAGE - 1) // PAGE, prefix // PAGE
        unique = ppg + rows * (npg - ppg) + (bsz - rows) * npg
        perm = torch.randperm(unique, generator=torch.Generator().manual_seed(1)).to(torch.int32)
        bt = torch.empty((bsz, npg), dtype=torch.int32)
        o = ppg
        for b in range(bsz):
            own = npg - ppg if b < rows else npg
            if b < rows:
                bt[b, :ppg] = perm[:ppg]
            bt[b, npg - own:] = perm[o:o + own]
            o += own
        pre, info, grp = cascade_groups(bt.numpy(), sl.cpu().numpy(), PAGE, max_rows=128 // (hq // hkv),
                                        min_blocks=16, max_groups=2, max_prefix_blocks=ppg)
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)
        plan = CascadePlan(t(pre), t(info), t(grp) if len(grp) else torch.zeros(1, dtype=torch.int32, device=dev),
                           2, ppg)
        btd = bt.to(dev)
        rec = {}
        for fp8 in (False, True):
            caches = []
            for _ in range(2):
                kv = torch.randn((2, unique, hkv, PAGE, d), generator=g, device=dev)
                kv = (kv / FP8_SCALE).to(torch.float8_e4m3fn) if fp8 else kv.to(torch.bfloat16)
                caches.append((kv[0].transpose(1, 2), kv[1].transpose(1, 2)))
            kw = _scales(caches[0][0])
            for name, fn in (("plain", lambda k, v: paged_decode_attention(q, k, v, btd, sl, hq, hkv, d, **kw)),
                             ("cascade", lambda k, v: cascade_decode_attention(q, k, v, btd, sl, plan, hq, hkv, d,
                                                                                **kw))):
                for _ in range(2):
                    for k, v in caches:
                        fn(k, v)
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(iters):
                    for k, v in caches:
                        fn(k, v)
                e1.record()
                torch.cuda.synchronize()
                rec[f"{'fp8' if fp8 else 'bf16'}_{name}_us"] = round(e0.elapsed_time(e1) / (2 * iters) * 1e3, 1)
            del caches
            torch.cuda.empty_cache()
        out[f"ctx{ctx}_rows{rows}_prefix{prefix}"] = rec
    return out


MFMA_BF16_PEAK_TFLOPS = 2500.0


def serving_roofline(cfg, st, wbytes: int, kv_elem: int = 2) -> dict:
    """Roofline time of a serving run, step by step: each step reads the
    weights once and its decode rows' KV (Sum ctx x L x Hkv x D x 2 x kv_elem
    bytes) against 8 TB/s, plus its prefill flops (the layer GEMMs'
    2 x params per token, causal attention's 4 x Hq x D x L per query-key
    pair, the LM head's 2 x V x H per sampled prompt) against the 2.5 PFLOP/s
    dense bf16 MFMA peak; summed over the steps."""
    h, hq, hkv, d, ffn, layers = (cfg.hidden_size, cfg.num_attention_heads, cfg.num_key_value_heads, 128,
                                  cfg.intermediate_size, cfg.num_hidden_layers)
    layer_params = h * (hq + 2 * hkv) * d + hq * d * h + 3 * h * ffn
    gemm_per_tok = 2 * layer_params * layers
    attn_per_pair = 4 * hq * d * layers
    lm_per_row = 2 * cfg.vocab_size * h
    kv_tok = layers * hkv * d * 2 * kv_elem
    t_bytes = t_flops = 0.0
    for n_d, ctx_sum, n_pt, pairs, n_ps in st.step_work:
        t_bytes += (wbytes + ctx_sum * kv_tok) / (HBM_PEAK_GBS * 1e9)
        t_flops += (n_pt * gemm_per_tok + pairs * attn_per_pair + n_ps * lm_per_row) / (MFMA_BF16_PEAK_TFLOPS * 1e12)
    roof = t_bytes + t_flops
    dec = [w for w in st.step_work if w[0]]
    return {"roofline_s": round(roof, 4), "roofline_hbm_s": round(t_bytes, 4), "roofline_mfma_s": round(t_flops, 4),
            "frac_of_roofline": round(roof / st.wall_s, 4),
            "mean_decode_ctx": round(sum(w[1] for w in dec) / max(1, sum(w[0] for w in dec)), 1),
            "roofline_rule": "sum over steps of (weights + decode KV bytes) / 8 TB/s + prefill flops / 2.5 PFLOP/s"}


def serve_e2e(torch, dev, *, sampled: bool, n_req: int = 256, gen: int = 256, seed: int = 0,
              max_num_seqs: int = 256, max_num_batched_tokens: int = 8192, model=None, fp8: bool = False) -> dict:
    """Config 4: Qwen3-8B (random bf16 weights ~N(0,0.02)) serving 256 requests
    with random-token prompts of U[128, 2048] tokens, each generating `gen`
    tokens (EOS ignored), under continuous batching with the reference
    scheduler's default policy (xvllm.serving: every running sequence decodes
    one token per step, the leftover of the 8192-token budget goes to prefill
    chunks, at most one of them partial; max 256 sequences).  Decode and its
    LM head + sampler run under hipGraph; prefill eagerly.  Sampled runs use
    T 0.7 / top-k 50 / top-p 0.9 with draws from a seeded generator."""
    from xvllm.config import QWEN3_8B
    from xvllm.kv_pool import KVPool
    from xvllm.model_runner import ModelRunner
    from xvllm.models import Qwen3ForCausalLM
    from xvllm.serving import serve

    cfg = QWEN3_8B
    g = torch.Generator().manual_seed(seed + 404)
    plens = torch.randint(128, 2049, (n_req,), generator=g).tolist()
    prompts = [torch.randint(0, cfg.vocab_size, (n,), generator=g).tolist() for n in plens]
    max_len = max(plens) + gen
    pages_needed = sum((n + gen + PAGE - 1) // PAGE for n in plens)
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(dev):
            if model is None:
                model = Qwen3ForCausalLM(cfg).random_init_(seed=0).set_split_k(SPLIT_K)
            if fp8:  # the optional fp8 (e4m3fn) page format
                kv = KVPool(cfg, num_blocks=pages_needed + 16, block_size=PAGE, device=dev,
                            dtype=torch.float8_e4m3fn, k_scale=FP8_SCALE, v_scale=FP8_SCALE)
            else:
                kv = KVPool(cfg, num_blocks=pages_needed + 16, block_size=PAGE, device=dev, dtype=torch.bfloat16)
    finally:
        torch.set_default_dtype(torch.float32)
    samp = dict(temperature=0.7, top_p=0.9, top_k=50) if sampled else None
    modes = (2 | 4 | 16,) if sampled else ()  # the sampled run's sampler graphs, recorded up front
    runner = ModelRunner(model, kv, max_num_seqs=max_num_seqs, max_num_batched_tokens=max_num_batched_tokens,
                         context_len=max_len, device=dev, sample_modes=modes)
    runner.generator = torch.Generator(device=dev).manual_seed(seed + 7) if sampled else None
    outs, st = serve(runner, prompts, gen, sampling=samp, max_num_seqs=max_num_seqs,
                     max_num_batched_tokens=max_num_batched_tokens)
    runner.destroy()
    del kv
    torch.cuda.empty_cache()
    out_tokens = sum(len(o) for o in outs)
    assert out_tokens == n_req * gen
    wbytes = sum(p.numel() for n, p in model.named_parameters() if "embed_tokens" not in n) * 2
    roof = serving_roofline(cfg, st, wbytes, kv_elem=1 if fp8 else 2)
    return {"requests": n_req, "prompt_tokens": sum(plens), "generated_tokens": out_tokens, "steps": st.steps,
            "sampling": "T0.7/k50/p0.9" if sampled else "greedy", "kv_pages": "fp8 e4m3fn" if fp8 else "bf16",
            "wall_s": round(st.wall_s, 3),
            "output_tok_per_s": round(out_tokens / st.wall_s, 1),
            "total_tok_per_s": round((out_tokens + sum(plens)) / st.wall_s, 1),
            "host_s_before_sync": round(st.host_s, 3),
            "mean_decode_batch": round(st.decode_tokens / max(1, st.steps), 1),
            "prefix_cache_hit_tokens": st.hit_tokens, **roof,
            "roofline_output_tok_per_s": round(out_tokens / roof["roofline_s"], 1),
            "policy": "decode-first mixed, 8192-token budget, max 256 seqs, 16-token pages, radix prefix cache"}, model


def cpu_baseline(ctx_all: list[int], budget_s: float = 12.0) -> dict:
    """The oracle's multi-threaded torch restatement (oracle.threaded, pinned
    against the numpy oracle) on every usable host core: the whole config-2
    batch (one call's worth of sequences, fp32 K/V in a paged pool with a
    random block permutation), repeated until the time budget is used."""
    import torch
    from concurrent.futures import ThreadPoolExecutor

    import oracle.threaded as TH

    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    g = torch.Generator().manual_seed(7)
    need = [(c + PAGE - 1) // PAGE for c in ctx_all]
    nb = sum(need)
    kc = torch.randn((nb, PAGE, HKV, D), generator=g)
    vc = torch.randn((nb, PAGE, HKV, D), generator=g)
    perm = torch.randperm(nb, generator=g)
    bt = torch.zeros((len(ctx_all), max(need)), dtype=torch.int64)
    o = 0
    for b, n in enumerate(need):
        bt[b, :n] = perm[o : o + n]
        o += n
    q = torch.randn((len(ctx_all), HQ, D), generator=g)
    prev = torch.get_num_threads()
    torch.set_num_threads(1)  # one thread per task; the pool supplies the parallelism
    t_used, reps = 0.0, 0
    try:
        with ThreadPoolExecutor(max_workers=cores) as pool:
            TH.paged_decode_attention(q, kc, vc, bt, ctx_all, pool=pool)  # untimed first call
            while t_used < budget_s:
                t0 = time.perf_counter()
                TH.paged_decode_attention(q, kc, vc, bt, ctx_all, pool=pool)
                t_used += time.perf_counter() - t0
                reps += 1
    finally:
        torch.set_num_threads(prev)
    return {
        "value": algo_bytes(ctx_all) * reps / t_used / 1e9,
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"oracle.threaded (torch fp32, one sequence per task on {cores} host threads), the full config-2 "
                  f"batch ({len(ctx_all)} sequences, {sum(ctx_all)} tokens) x {reps} calls, {t_used:.1f} s timed "
                  f"(input generation excluded)",
        "host_cpus": os.cpu_count(),
        "host_cpus_usable": cores,
    }


def _torch_threads():
    import torch

    return torch.get_num_threads()


def cpu_baseline_rows(budget_s: float = 1.0) -> dict:
    """The oracle (the CPU restatement of each reference op) timed on the host,
    one thread, on bounded samples of the config-3 / prefill / sampler
    workloads; each row is repeated until `budget_s` is used, after one
    untimed call."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    import oracle.ops as O
    import oracle.sampler as S

    rng = np.random.default_rng(8)
    out = {}

    def run(name, fn, units, unit, sample):
        fn()  # first call (page-in of numpy's temporaries) untimed
        t_used, n = 0.0, 0
        while t_used < budget_s:
            t0 = time.perf_counter()
            fn()
            t_used += time.perf_counter() - t0
            n += 1
        out[name] = {"value": round(units * n / t_used, 3), "unit": unit, "cores": 1, "kind": "port",
                     "sample": f"{sample}, {n} repetitions, {t_used:.1f} s"}

    r = lambda *sh: rng.standard_normal(sh, dtype=np.float32)
    with threadpool_limits(limits=1):
        T = 1024
        k, v = r(T, HKV, D), r(T, HKV, D)
        kc, vc = np.zeros((1024, PAGE, HKV, D), np.float32), np.zeros((1024, PAGE, HKV, D), np.float32)
        slots = rng.permutation(1024 * PAGE)[:T]
        run("store_kvcache", lambda: O.store_kvcache(k, v, kc.reshape(-1, HKV, D), vc.reshape(-1, HKV, D), slots),
            (2 * T * HKV * D * 2 * 2 + 4 * T) / 1e9, "GB/s", f"{T} tokens x 8 kv heads x 128")
        x, res, w = r(128, 4096), r(128, 4096), r(4096)
        run("fused_add_rmsnorm", lambda: O.fused_add_rmsnorm(x, res, w, 1e-6), 128 * 4096 * 2 * 4 / 1e9, "GB/s",
            "128 rows x 4096")
        q, kk, qw, kw = r(256, HQ, D), r(256, HKV, D), r(D), r(D)
        pos, cs = rng.integers(0, 32768, 256), O.build_cos_sin_cache(D, 32768, 1e6)
        run("qk_norm_rope", lambda: O.qk_norm_rope(q, kk, qw, kw, 1e-6, pos, cs),
            256 * (HQ + HKV) * D * 2 * 2 / 1e9, "GB/s", "256 tokens x (32 + 8) heads x 128")
        xg = r(64, 2 * 12288)
        run("silu_and_mul", lambda: O.silu_and_mul(xg), 64 * 3 * 12288 * 2 / 1e9, "GB/s", "64 rows x 12288")
        L = 512
        qp, kp, vp = r(L, HQ, D), r(L, HKV, D), r(L, HKV, D)
        cu = np.array([0, L], np.int32)
        run("prefill_attention", lambda: O.prefill_attention(qp, cu, cu, k=kp, v=vp),
            4 * HQ * D * L * (L + 1) / 2 / 1e12, "TFLOP/s", f"one causal {L}-token prompt, 32 q / 8 kv heads")
        V = 151936
        bits = (rng.standard_normal((4, V)).astype(np.float32) * 2).view(np.uint32) >> 16
        logits = bits.astype(np.uint16)
        t = np.full(4, 0.7, np.float32)
        run("sampler_k50_p0.9", lambda: S.sample(logits, t, np.full(4, 0.9, np.float32), np.full(4, 50, np.int32),
                                                 None, rng.random(4).astype(np.float32), 2 | 4),
            4 * V * 2 / 1e9, "GB/s", "4 rows x 151936 (C oracle)")
        run("sampler_greedy", lambda: S.sample(logits, np.zeros(4, np.float32), None, None, None, None, 1),
            4 * V * 2 / 1e9, "GB/s", "4 rows x 151936 (C oracle)")
    return out


# split-K o_proj / down_proj at decode batch sizes (xvllm.layers.linear); --no-split-k turns it off
SPLIT_K = True


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-suite", action="store_true", help="skip the config-3 kernel set and the sampler")
    ap.add_argument("--no-e2e", action="store_true", help="skip the Qwen3-8B decode tok/s measurement")
    ap.add_argument("--e2e-only", action="store_true", help="only the Qwen3-8B decode step (for profiling)")
    ap.add_argument("--prefill-only", action="store_true", help="only the prefill attention cases (for profiling)")
    ap.add_argument("--suite-only", action="store_true", help="only the config-3 kernel set and the sampler")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill attention cases")
    ap.add_argument("--no-serve", action="store_true", help="skip config 4 (256 requests, greedy and sampled)")
    ap.add_argument("--serve-only", action="store_true", help="only config 4 (for profiling)")
    ap.add_argument("--config5", action="store_true",
                    help="also run config 5 with the plain decode forced and on fp8 pages (the runner as served, "
                         "its gate choosing the decode, runs by default)")
    ap.add_argument("--no-config5", action="store_true", help="skip config 5 (Qwen3-32B-shaped long-context decode)")
    ap.add_argument("--config5-only", action="store_true", help="only config 5 (for profiling)")
    ap.add_argument("--cascade-only", action="store_true",
                    help="only the shared-prefix sweep: plain against cascade decode attention")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 1 GiB device copy (HBM counter calibration for rocprofv3 --pmc)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-split-k", action="store_true", help="plain o_proj / down_proj GEMMs in the model runs")
    ap.add_argument("--kv-dtype", choices=("bf16", "fp8"), default="bf16",
                    help="KV page format of the headline calls (fp8: the pool's optional e4m3fn pages, for profiling)")
    ap.add_argument("--layout", choices=("hnd", "nhd"), default="hnd",
                    help="KV page memory order of the headline (hnd: KVPool's default; nhd: the reference's)")
    args = ap.parse_args()
    global SPLIT_K
    SPLIT_K = not args.no_split_k
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only (no multi-GPU path); run with --gpus 1"}))
        return 2

    import torch

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        return 1
    dev = torch.device("cuda:0")
    if args.calibrate_copy:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "copy", "bytes_read": 1 << 30, "bytes_written": 1 << 30, "launches": 5}))
        return 0
    g = torch.Generator().manual_seed(args.seed)
    ctx = torch.randint(512, 4097, (64,), generator=g).tolist()
    if args.e2e_only:
        rec, model = decode_e2e(torch, dev, ctx, steps=args.steps)
        rec8, model = decode_e2e(torch, dev, ctx, steps=args.steps, fp8=True, model=model)
        print(json.dumps({"decode_e2e": rec, "decode_e2e_fp8": rec8}))
        return 0
    if args.config5_only:
        c5, model = decode_config5(torch, dev)
        c5p, model = decode_config5(torch, dev, attention="plain", model=model)
        c58, model = decode_config5(torch, dev, model=model, fp8=True)
        c58p, model = decode_config5(torch, dev, attention="plain", model=model, fp8=True)
        print(json.dumps({"config5": c5, "config5_plain": c5p, "config5_fp8": c58, "config5_plain_fp8": c58p}))
        return 0
    if args.cascade_only:
        print(json.dumps({"cascade_sweep": cascade_sweep(torch, dev)}))
        return 0
    if args.serve_only:
        greedy, model = serve_e2e(torch, dev, sampled=False)
        sampled, model = serve_e2e(torch, dev, sampled=True, model=model)
        greedy8, model = serve_e2e(torch, dev, sampled=False, model=model, fp8=True)
        print(json.dumps({"serve_greedy": greedy, "serve_sampled": sampled, "serve_greedy_fp8": greedy8}))
        return 0
    if args.prefill_only:
        print(json.dumps(prefill_suite(torch, dev, iters=args.steps)))
        return 0
    if args.suite_only:
        print(json.dumps(kernel_suite(torch, dev)))
        return 0
    fp8 = args.kv_dtype == "fp8"
    cases = make_case(torch, ctx, layers=4, dev=dev, seed=args.seed + 1, layout=args.layout, fp8=fp8)
    ms, wall, eager_ms = time_decode(torch, cases, args.steps, args.warmup)
    nbytes = algo_bytes(ctx, kv_elem=1 if fp8 else 2)
    gbs = nbytes / (ms * 1e-3) / 1e9

    sweep = {}
    if not args.no_sweep:
        # config 2's batch sweep at ctx 2048, and one long single-sequence decode
        for bsz, clen in ((1, 2048), (8, 2048), (64, 2048), (256, 2048), (1, 32768)):
            c2 = [clen] * bsz
            cs = make_case(torch, c2, layers=4 if bsz <= 64 else 2, dev=dev, seed=args.seed + bsz)
            m2 = time_decode_graph(torch, cs) * 1e-3
            sweep[f"B{bsz}_ctx{clen}"] = {"us": round(m2 * 1e3, 2), "GB/s": round(algo_bytes(c2) / (m2 * 1e-3) / 1e9, 1),
                                          "frac": round(algo_bytes(c2) / (m2 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
            del cs
        torch.cuda.empty_cache()
        # the KV pool's memory order: config 2 in the other page layout, timed
        # the same way as the headline (one graph of K calls)
        other = "nhd" if args.layout == "hnd" else "hnd"
        cs = make_case(torch, ctx, layers=4, dev=dev, seed=args.seed + 1, layout=other)
        m2, _, _ = time_decode(torch, cs, args.steps, 20)
        sweep[f"config2_{other}_pages"] = {"us": round(m2 * 1e3, 2), "GB/s": round(nbytes / (m2 * 1e-3) / 1e9, 1),
                                           "frac": round(nbytes / (m2 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        del cs
        torch.cuda.empty_cache()
        # the pool's fp8 (e4m3fn) format: config 2 on fp8 pages in the headline's page order, timed
        # the same way; GB/s counts the fp8 bytes, bf16_equiv_GB/s the bf16 path's bytes in that time
        cs = make_case(torch, ctx, layers=4, dev=dev, seed=args.seed + 1, layout=args.layout, fp8=True)
        m2, _, _ = time_decode(torch, cs, args.steps, 20)
        nb8 = algo_bytes(ctx, kv_elem=1)
        sweep["config2_fp8_pages"] = {"us": round(m2 * 1e3, 2), "GB/s": round(nb8 / (m2 * 1e-3) / 1e9, 1),
                                      "frac": round(nb8 / (m2 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                      "bf16_equiv_GB/s": round(nbytes / (m2 * 1e-3) / 1e9, 1)}
        del cs
        torch.cuda.empty_cache()

    line = {
        "metric": "decode attn HBM GB/s (% of 8 TB/s) + decode tok/s, Qwen3-8B bs=64, 1 GPU",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/K/V, random page permutation)",
        "config": {
            "workload": "config 2: paged GQA decode attention, Hq 32 / Hkv 8 / D 128, B 64, ctx U[512,4096], 16-token pages",
            "batch": 64,
            "total_ctx_tokens": sum(ctx),
            "kv_pools_cycled": 4,
            "kv_pages": "fp8 e4m3fn" if fp8 else "bf16",
            "kv_page_layout": args.layout + (" (KVPool default: [page][kv head][token][d] in memory, the reference's"
                                             " logical [page][token][kv head][d] view)" if args.layout == "hnd"
                                             else " (the reference's memory order)"),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": MEASURED_TRAFFIC_BYTES_FP8 if fp8 else MEASURED_TRAFFIC_BYTES,
            "algorithmic_bytes_per_call": nbytes,
            "kernel": f"paged_decode_kernel<4, {'true' if fp8 else 'false'}> + merge_parts_kernel (one call)",
        },
        "sweep": sweep,
        "wall_s_timed_region": round(wall, 4),
        "timing": "HIP graph of the K calls, replayed once between syncs (the decode step runs them in a graph)",
        "ms_per_step_eager_launch": round(eager_ms, 5),
    }
    if not args.no_suite:
        line["kernels"] = kernel_suite(torch, dev)
    if not args.no_prefill:
        line["prefill"] = prefill_suite(torch, dev)
    if not args.no_e2e:
        del cases
        torch.cuda.empty_cache()
        line["decode_e2e"], model = decode_e2e(torch, dev, ctx)
        line["decode_tok_per_s"] = line["decode_e2e"]["tok_per_s"]
        # the same step on an fp8 (e4m3fn) KV pool, the pool's optional page format
        line["decode_e2e_fp8"], model = decode_e2e(torch, dev, ctx, fp8=True, model=model)
        # the opt-in weight-streaming decode GEMMs (12.1 GB of packed weights beside the 16.4 GB of weights)
        line["decode_e2e_streamed_gemms"], model = decode_e2e(torch, dev, ctx, model=model, stream_gemms=True)
        del model
        torch.cuda.empty_cache()
    if not args.no_config5:
        torch.cuda.empty_cache()
        line["config5"], model = decode_config5(torch, dev)
        if args.config5:
            line["config5_plain"], model = decode_config5(torch, dev, attention="plain", model=model)
            line["config5_fp8"], model = decode_config5(torch, dev, model=model, fp8=True)
            line["config5_plain_fp8"], model = decode_config5(torch, dev, attention="plain", model=model, fp8=True)
        del model
        torch.cuda.empty_cache()
    if not args.no_serve:
        torch.cuda.empty_cache()
        line["serve_greedy"], model = serve_e2e(torch, dev, sampled=False)
        line["serve_sampled"], model = serve_e2e(torch, dev, sampled=True, model=model)
        line["serve_greedy_fp8"], model = serve_e2e(torch, dev, sampled=False, model=model, fp8=True)
        del model
        torch.cuda.empty_cache()
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(ctx)
        line["cpu_baseline_rows"] = cpu_baseline_rows()
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
