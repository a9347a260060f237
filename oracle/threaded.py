"""Multi-threaded CPU restatement of the paged decode attention (TEST
INFRASTRUCTURE ONLY): the same computation as ``oracle.ops.paged_decode_attention``
(reference src/compute/layers/attention.py:91-99, flash_attn_with_kvcache,
causal, cache_seqlens = pos+1 per batch.py:124) in torch fp32 on the host, one
sequence per task over a pool of host threads.  It exists to time the CPU
baseline on all of a host's cores; tests/test_oracle.py pins it against the
numpy restatement.
"""
from __future__ import annotations

import math
from concurrent.futures import ThreadPoolExecutor

import torch


def _one(q, k_cache, v_cache, pages, n, scale, out_row):
    """q [Hq, D]; pages: this sequence's block ids; writes out_row [Hq, D]."""
    nb, bs, hkv, d = k_cache.shape
    hq = q.shape[0]
    k = k_cache.index_select(0, pages).reshape(-1, hkv, d)[:n]  # [n, Hkv, D]
    v = v_cache.index_select(0, pages).reshape(-1, hkv, d)[:n]
    qg = q.view(hkv, hq // hkv, d)  # q head h -> kv head h // G
    s = torch.einsum("hgd,nhd->hgn", qg, k) * scale
    p = torch.softmax(s, dim=-1)
    out_row.copy_(torch.einsum("hgn,nhd->hgd", p, v).reshape(hq, d))


def paged_decode_attention(q, k_cache, v_cache, block_tables, cache_seqlens, scale=None, threads=1,
                           pool: ThreadPoolExecutor | None = None):
    """q [B, Hq, D], k_cache / v_cache [NB, BS, Hkv, D] (float32 torch tensors),
    block_tables int [B, max_blocks], cache_seqlens int [B] -> [B, Hq, D] fp32;
    padding rows (seqlen 0) give 0.  Sequences run as tasks on `pool` (or a pool
    of `threads` host threads); each task's torch ops run single-threaded."""
    bsz, hq, d = q.shape
    bs = k_cache.shape[1]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    out = torch.zeros((bsz, hq, d), dtype=torch.float32)
    bt = torch.as_tensor(block_tables, dtype=torch.int64)
    sl = [int(x) for x in cache_seqlens]
    own = pool is None
    if own:
        pool = ThreadPoolExecutor(max_workers=threads)
    try:
        futs = [pool.submit(_one, q[b], k_cache, v_cache, bt[b, : (sl[b] + bs - 1) // bs], sl[b], scale, out[b])
                for b in range(bsz) if sl[b] > 0]
        for f in futs:
            f.result()
    finally:
        if own:
            pool.shutdown()
    return out
