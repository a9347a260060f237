"""Step metadata (reference src/compute/batch.py:111-179, src/data/sequence.py:26-51)
as the kernels see it on the device: decode rows (input id = last token,
position = cached tokens, slot = bt[pos // 16] * 16 + pos % 16, cache_seqlens =
pos + 1), rows padded up to a graph bucket (slot -1, seqlen 0, block table -1),
prefill chunks (ids, positions, slots, cu_seqlens_q/k, has_cache), all
bit-exact; and the staging buffers shared by a step's decode and prefill."""
import numpy as np
import pytest
import torch

import oracle.ops as O
from helpers import gen

pytestmark = pytest.mark.gpu


def _seqs(g, n, pool, *, decode):
    from xvllm.batch import SeqSchedule

    perm = torch.randperm(pool, generator=g).tolist()
    out, o = [], 0
    for i in range(n):
        cached = int(torch.randint(0, 300, (1,), generator=g))
        new = 1 if decode else int(torch.randint(1, 70, (1,), generator=g))
        pages = (cached + new + 15) // 16
        toks = torch.randint(0, 151936, (new,), generator=g).tolist()
        out.append(SeqSchedule(seq_id=100 + i, token_ids=toks, num_cached_tokens=cached,
                               block_table=perm[o : o + pages]))
        o += pages
    return out


def _batch(dev):
    from xvllm.batch import Batch

    return Batch(max_bs=16, max_tokens=2048, max_blocks=32, vocab_size=151936, device=dev, block_size=16)


def test_decode_metadata_and_bucket_padding(dev):
    g = gen(71)
    b = _batch(dev)
    seqs = _seqs(g, 5, 200, decode=True)
    b.build_decode(seqs, pad_to=8)
    torch.cuda.synchronize()
    pos = np.array([s.num_cached_tokens for s in seqs])
    slots = np.array([O.slots_for_range(s.block_table, p, p + 1, 16)[0] for s, p in zip(seqs, pos)])
    assert np.array_equal(b.input_ids[:5].cpu().numpy(), [s.token_ids[-1] for s in seqs])
    assert np.array_equal(b.positions[:5].cpu().numpy(), pos)
    assert np.array_equal(b.slot_mapping[:5].cpu().numpy(), slots)
    assert np.array_equal(b.cache_seqlens[:5].cpu().numpy(), pos + 1)
    bt = b.block_tables.cpu().numpy()
    for i, s in enumerate(seqs):
        k = len(s.block_table)
        assert np.array_equal(bt[i, :k], s.block_table) and (bt[i, k:] == -1).all()
    assert (b.slot_mapping[5:8].cpu().numpy() == -1).all()
    assert (b.cache_seqlens[5:8].cpu().numpy() == 0).all()
    assert (bt[5:8] == -1).all()
    # next step: every sequence one token further (a new page for some), one fewer sequence
    for s in seqs:
        s.num_cached_tokens += 1
        if s.num_cached_tokens // 16 >= len(s.block_table):
            s.block_table = s.block_table + [199 - s.seq_id]
    b.build_decode(seqs[:4], pad_to=4)
    torch.cuda.synchronize()
    bt = b.block_tables.cpu().numpy()
    for i, s in enumerate(seqs[:4]):
        p = s.num_cached_tokens
        assert int(b.slot_mapping[i]) == O.slots_for_range(s.block_table, p, p + 1, 16)[0]
        assert np.array_equal(bt[i, : len(s.block_table)], s.block_table)


def test_prefill_metadata(dev):
    g = gen(72)
    b = _batch(dev)
    seqs = _seqs(g, 4, 300, decode=False)
    seqs[1].num_cached_tokens = 0  # one sequence without a cached prefix
    nt, max_q, max_k, has_cache = b.build_prefill(seqs)
    torch.cuda.synchronize()
    lens = [len(s.token_ids) for s in seqs]
    ends = [s.num_cached_tokens + n for s, n in zip(seqs, lens)]
    assert nt == sum(lens) and max_q == max(lens) and max_k == max(ends) and has_cache
    assert np.array_equal(b.input_ids[:nt].cpu().numpy(), sum((s.token_ids for s in seqs), []))
    pos = np.concatenate([np.arange(s.num_cached_tokens, e) for s, e in zip(seqs, ends)])
    assert np.array_equal(b.positions[:nt].cpu().numpy(), pos)
    slots = sum((O.slots_for_range(s.block_table, s.num_cached_tokens, e, 16) for s, e in zip(seqs, ends)), [])
    assert np.array_equal(b.slot_mapping[:nt].cpu().numpy(), slots)
    assert np.array_equal(b.cu_seqlens_q[:5].cpu().numpy(), np.concatenate([[0], np.cumsum(lens)]))
    assert np.array_equal(b.cu_seqlens_k[:5].cpu().numpy(), np.concatenate([[0], np.cumsum(ends)]))


def test_decode_then_prefill_in_one_step_keeps_decode_metadata(dev):
    """A step stages its decode rows, enqueues work that reads them, then stages
    its prefill chunks through the same pinned buffers: the decode work must
    still see the decode rows (regression: the host overwrote the staging
    buffers before the non-blocking H2D copies ran)."""
    g = gen(73)
    b = _batch(dev)
    a = torch.randn(4096, 4096, device=dev)
    for trial in range(5):
        dec = _seqs(g, 6, 200, decode=True)
        pre = _seqs(g, 3, 200, decode=False)
        for _ in range(8):  # keep the stream busy so the H2D copies run late
            a = a @ a * 1e-3
        b.build_decode(dec)
        seen_ids = b.input_ids[:6].clone()
        seen_slots = b.slot_mapping[:6].clone()
        b.build_prefill(pre)
        torch.cuda.synchronize()
        assert seen_ids.cpu().tolist() == [s.token_ids[-1] for s in dec], f"trial {trial}"
        want = [O.slots_for_range(s.block_table, s.num_cached_tokens, s.num_cached_tokens + 1, 16)[0] for s in dec]
        assert seen_slots.cpu().tolist() == want, f"trial {trial}"
