"""GPU parity of the paged kernels at cache block sizes other than 16 (the
reference's default kvcache_block_size is 256, src/config.py:66-67), the KV
store on layouts the kernel cannot read in place and at config-3 size, and
the decode merge at the partial counts where its batching changes."""
import math

import numpy as np
import pytest
import torch

import oracle.ops as O
from helpers import f32, gen, make_paged, randn_bf16

pytestmark = pytest.mark.gpu

RTOL = ATOL = 2e-2


def _close(got, want, rtol=RTOL, atol=ATOL):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert np.isfinite(got).all(), "non-finite output"
    err = np.abs(got - want) - (atol + rtol * np.abs(want))
    assert (err <= 0).all(), f"max excess {err.max():.4g} at {np.unravel_index(err.argmax(), err.shape)}"


@pytest.mark.parametrize("block", [32, 256, 48])
@pytest.mark.parametrize("hnd", [False, True], ids=["nhd", "hnd"])
def test_paged_decode_block_sizes(dev, block, hnd):
    """Blocks of 32 / 256 / 48 tokens (three 16-token pages each): a
    sequence's 16-token page p lies in block bt[p * 16 // BS]; NaN in every
    unused slot, contexts that end inside and on block boundaries."""
    from xvllm.layers.attention import paged_decode_attention

    print(f"decode block {block} hnd {hnd}", flush=True)
    g = gen(block + hnd)
    hq, hkv, d = 32, 8, 128
    ctx = [1, block, block + 1, 3 * block - 5, 700, 0, 2049, 16]
    need = sum((c + block - 1) // block for c in ctx)
    kc, vc, bt, sl = make_paged(ctx, need + 3, hkv, d, g, page=block)
    q = randn_bf16((len(ctx), hq, d), g)
    want = O.paged_decode_attention(f32(q), f32(kc), f32(vc), bt.numpy(), sl.numpy())
    kg, vg = kc.to(dev), vc.to(dev)
    if hnd:  # [NB, Hkv, BS, D] memory, viewed as [NB, BS, Hkv, D]
        kg = kg.transpose(1, 2).contiguous().transpose(1, 2)
        vg = vg.transpose(1, 2).contiguous().transpose(1, 2)
    out = paged_decode_attention(q.view(len(ctx), -1).to(dev), kg, vg, bt.to(dev), sl.to(dev), hq, hkv, d)
    torch.cuda.synchronize()
    _close(f32(out).reshape(len(ctx), hq, d), want)


@pytest.mark.parametrize("block", [256, 32])
def test_prefill_paged_block_sizes(dev, block):
    """Chunked prefill over cached prefixes read through BS-token blocks."""
    from xvllm.layers.attention import prefill_attention

    print(f"prefill block {block}", flush=True)
    g = gen(7 * block)
    hq, hkv, d = 32, 8, 128
    qlens, klens = [17, 64, 300, 1], [300, 64, 1100, 257]
    cu_q = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(klens)]).astype(np.int32)
    q = randn_bf16((int(cu_q[-1]), hq, d), g)
    need = sum((c + block - 1) // block for c in klens)
    kc, vc, bt, _ = make_paged(klens, need + 2, hkv, d, g, page=block)
    want = O.prefill_attention(f32(q), cu_q, cu_k, k_cache=f32(kc), v_cache=f32(vc), block_tables=bt.numpy())
    out = prefill_attention(q.to(dev), None, None, torch.from_numpy(cu_q).to(dev), torch.from_numpy(cu_k).to(dev),
                            max(qlens), hq, hkv, d, k_cache=kc.to(dev), v_cache=vc.to(dev), block_tables=bt.to(dev))
    torch.cuda.synchronize()
    _close(f32(out).reshape(-1, hq, d), want)


def test_store_kvcache_block_256_and_unaligned_inputs(dev):
    """The store into a 256-token-block pool (slot = block * 256 + offset) and
    key/value views the kernel cannot read in place (rows 2 bytes off a
    16-byte boundary, a non-unit last stride): copied first, as the reference
    makes its inputs contiguous (kv_ops.py:42-45); bit-exact either way."""
    from xvllm.kv_ops import store_kvcache

    g = gen(256)
    n, hkv, d, nb, bs = 50, 8, 128, 6, 256
    base = randn_bf16((n * hkv * d + 1,), g)
    key = base[1:].view(n, hkv, d)                                 # 2-byte offset rows
    val = randn_bf16((n, d, hkv), g).transpose(1, 2)               # last stride != 1
    slots = torch.randperm(nb * bs, generator=g)[:n].to(torch.int32)
    slots[3] = -1
    kc, vc = randn_bf16((nb, bs, hkv, d), g), randn_bf16((nb, bs, hkv, d), g)
    kr, vr = kc.clone(), vc.clone()
    O.store_kvcache(key, val, kr, vr, slots)
    kg, vg = kc.to(dev), vc.to(dev)
    store_kvcache(base.to(dev)[1:].view(n, hkv, d), val.to(dev), kg, vg, slots.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(kg.cpu().view(torch.int16), kr.view(torch.int16))
    assert torch.equal(vg.cpu().view(torch.int16), vr.view(torch.int16))


def test_store_kvcache_config3_full_size(dev):
    """Config 3's store: T 8192 tokens, Hkv 8, into a 16-token-page cache by a
    random injective slot map over 1024 pages; bit-exact against the oracle's
    scatter (done with numpy fancy indexing: injective slots)."""
    from xvllm.kv_ops import store_kvcache

    g = gen(8192)
    t, hkv, d, nb = 8192, 8, 128, 1024
    key, val = randn_bf16((t, hkv, d), g), randn_bf16((t, hkv, d), g)
    slots = torch.randperm(nb * 16, generator=g)[:t].to(torch.int32)
    kc, vc = randn_bf16((nb, 16, hkv, d), g), randn_bf16((nb, 16, hkv, d), g)
    kr, vr = kc.clone(), vc.clone()
    kr.view(-1, hkv, d)[slots.long()] = key  # the oracle's loop, vectorised (slots are distinct)
    vr.view(-1, hkv, d)[slots.long()] = val
    kg, vg = kc.to(dev), vc.to(dev)
    store_kvcache(key.to(dev), val.to(dev), kg, vg, slots.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(kg.cpu().view(torch.int16), kr.view(torch.int16))
    assert torch.equal(vg.cpu().view(torch.int16), vr.view(torch.int16))
    # the loop oracle on a slice agrees with the vectorised scatter
    k2 = kc.clone()
    O.store_kvcache(key[:64], val[:64], k2, vc.clone(), slots[:64])
    assert torch.equal(k2.view(-1, hkv, d)[slots[:64].long()], key[:64])


@pytest.mark.parametrize("parts", [32, 33, 64, 65, 97])
def test_paged_decode_merge_partial_count_boundaries(dev, parts):
    """One sequence of 4 * parts 16-token pages at Hq 32 / Hkv 8: ranges of 4
    pages (the minimum) split each kv head's segment into exactly `parts`
    partials, read back from the workspace's count table.  32 and 64 are the
    ends of the merge's load batches, 33 and 65 start a new one, 97 uses the
    second weight register."""
    from xvllm.layers import attention as A

    print(f"merge parts {parts}", flush=True)
    g = gen(parts)
    hq, hkv, d = 32, 8, 128
    ctx = [64 * parts]  # 4 pages per partial
    kc, vc, bt, sl = make_paged(ctx, 4 * parts + 3, hkv, d, g)
    q = randn_bf16((1, hq, d), g)
    want = O.paged_decode_attention(f32(q), f32(kc), f32(vc), bt.numpy(), sl.numpy())
    out = A.paged_decode_attention(q.view(1, -1).to(dev), kc.to(dev), vc.to(dev), bt.to(dev), sl.to(dev), hq, hkv, d)
    torch.cuda.synchronize()
    ws = A._WORKSPACE[(dev.type, dev.index)]
    counts = ws[: 4 * hkv].cpu().view(torch.int32).tolist()
    total = 8 * 4 * parts
    if math.ceil(total / 4) <= 1024:  # ranges of exactly 4 pages while they fit the resident waves
        assert counts == [parts] * hkv, counts
    _close(f32(out).reshape(1, hq, d), want)


def test_store_kvcache_multi_unit_waves_with_padding(dev):
    """2049 tokens (4098 64-chunk units: the two-units-per-wave path, with an
    odd unit count so the last wave has one) and padding slots (-1)."""
    from xvllm.kv_ops import store_kvcache

    g = gen(2049)
    t, hkv, d, nb = 2049, 8, 128, 200
    key, val = randn_bf16((t, hkv, d), g), randn_bf16((t, hkv, d), g)
    slots = torch.randperm(nb * 16, generator=g)[:t].to(torch.int32)
    slots[::5] = -1
    slots[-1] = -1
    kc, vc = randn_bf16((nb, 16, hkv, d), g), randn_bf16((nb, 16, hkv, d), g)
    kr, vr = kc.clone(), vc.clone()
    keep = slots >= 0
    kr.view(-1, hkv, d)[slots[keep].long()] = key[keep]
    vr.view(-1, hkv, d)[slots[keep].long()] = val[keep]
    kg, vg = kc.to(dev), vc.to(dev)
    store_kvcache(key.to(dev), val.to(dev), kg, vg, slots.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(kg.cpu().view(torch.int16), kr.view(torch.int16))
    assert torch.equal(vg.cpu().view(torch.int16), vr.view(torch.int16))
