"""Host logic of the step metadata (reference src/compute/batch.py:111-251,
src/data/sequence.py:26-51) on the CPU: the same Batch code with its buffers
on the CPU device.  Decode rows, bucket padding, incremental block-table rows,
prefill chunks and the sampling-parameter normalisation, all exact; the slot
map is checked against the oracle's slots_for_range."""
import numpy as np
import torch

import oracle.ops as O
from helpers import gen

CPU = torch.device("cpu")
V = 151936


def _seqs(g, n, pool, *, decode, seq0=100):
    from xvllm.batch import SeqSchedule

    perm = torch.randperm(pool, generator=g).tolist()
    out, o = [], 0
    for i in range(n):
        cached = int(torch.randint(0, 300, (1,), generator=g))
        new = 1 if decode else int(torch.randint(1, 70, (1,), generator=g))
        pages = (cached + new + 15) // 16
        toks = torch.randint(0, V, (new,), generator=g).tolist()
        out.append(SeqSchedule(seq_id=seq0 + i, token_ids=toks, num_cached_tokens=cached,
                               block_table=perm[o : o + pages]))
        o += pages
    return out


def _batch():
    from xvllm.batch import Batch

    return Batch(max_bs=16, max_tokens=2048, max_blocks=32, vocab_size=V, device=CPU, block_size=16)


def test_decode_rows_and_bucket_padding():
    g = gen(81)
    b = _batch()
    seqs = _seqs(g, 5, 200, decode=True)
    b.build_decode(seqs, pad_to=8)
    pos = np.array([s.num_cached_tokens for s in seqs])
    assert b.input_ids[:5].tolist() == [s.token_ids[-1] for s in seqs]
    assert np.array_equal(b.positions[:5].numpy(), pos)
    want = [O.slots_for_range(s.block_table, p, p + 1, 16)[0] for s, p in zip(seqs, pos)]
    assert b.slot_mapping[:5].tolist() == want
    assert np.array_equal(b.cache_seqlens[:5].numpy(), pos + 1)
    bt = b.block_tables.numpy()
    for i, s in enumerate(seqs):
        k = len(s.block_table)
        assert bt[i, :k].tolist() == s.block_table and (bt[i, k:] == -1).all()
    # padding rows up to the bucket: slot -1, seqlen 0, block table -1
    assert (b.slot_mapping[5:8].numpy() == -1).all()
    assert (b.cache_seqlens[5:8].numpy() == 0).all()
    assert (bt[5:8] == -1).all()


def test_decode_inputs_fed_from_the_previous_steps_ids():
    """Rows with src_row >= 0 take their input id from the previous step's
    sampled ids (a device tensor) by a gather, clamped into [0, vocab); the
    other rows keep their host ids; a source row past the previous step's ids
    or a missing previous step raises."""
    import dataclasses

    import pytest

    g = gen(84)
    b = _batch()
    seqs = _seqs(g, 6, 200, decode=True)
    prev = torch.tensor([11, 22, V + 5, 44, -3, 66], dtype=torch.int64)  # two ids a bad sampler could leave
    src = [3, -1, 0, 2, -1, 4]
    fed = [dataclasses.replace(s, token_ids=[0] if r >= 0 else s.token_ids, src_row=r) for s, r in zip(seqs, src)]
    b.build_decode(fed, prev_ids=prev)
    want = [min(max(int(prev[r]), 0), V - 1) if r >= 0 else s.token_ids[-1] for s, r in zip(seqs, src)]
    assert b.input_ids[:6].tolist() == want
    assert b.input_ids[3] == V - 1 and b.input_ids[5] == 0  # clamped
    with pytest.raises(ValueError, match="previous step"):
        b.build_decode(fed)
    with pytest.raises(ValueError, match="source row"):
        b.build_decode(fed, prev_ids=prev[:3])


def test_block_table_rows_grow_append_only_and_follow_new_owners():
    g = gen(82)
    b = _batch()
    seqs = _seqs(g, 4, 300, decode=True)
    b.build_decode(seqs)
    for step in range(40):  # one token per step; a new page every 16 tokens
        for s in seqs:
            s.num_cached_tokens += 1
            if s.num_cached_tokens // 16 >= len(s.block_table):
                s.block_table = s.block_table + [250 + s.seq_id % 50]
        if step == 20:  # row 2 changes owner: a different sequence takes the slot
            seqs[2] = _seqs(g, 1, 300, decode=True, seq0=900)[0]
        b.build_decode(seqs)
        bt = b.block_tables.numpy()
        for i, s in enumerate(seqs):
            k = len(s.block_table)
            assert bt[i, :k].tolist() == s.block_table and (bt[i, k:] == -1).all(), (step, i)
            p = s.num_cached_tokens
            assert int(b.slot_mapping[i]) == O.slots_for_range(s.block_table, p, p + 1, 16)[0]


def test_prefill_chunks():
    g = gen(83)
    b = _batch()
    seqs = _seqs(g, 4, 300, decode=False)
    seqs[1].num_cached_tokens = 0  # one sequence without a cached prefix
    nt, max_q, max_k, has_cache = b.build_prefill(seqs)
    lens = [len(s.token_ids) for s in seqs]
    ends = [s.num_cached_tokens + n for s, n in zip(seqs, lens)]
    assert (nt, max_q, max_k, has_cache) == (sum(lens), max(lens), max(ends), True)
    assert b.input_ids[:nt].tolist() == sum((s.token_ids for s in seqs), [])
    pos = np.concatenate([np.arange(s.num_cached_tokens, e) for s, e in zip(seqs, ends)])
    assert np.array_equal(b.positions[:nt].numpy(), pos)
    slots = sum((list(O.slots_for_range(s.block_table, s.num_cached_tokens, e, 16)) for s, e in zip(seqs, ends)), [])
    assert b.slot_mapping[:nt].tolist() == slots
    assert b.cu_seqlens_q[:5].tolist() == [0, *np.cumsum(lens).tolist()]
    assert b.cu_seqlens_k[:5].tolist() == [0, *np.cumsum(ends).tolist()]
    # fresh prompts only: no cached prefix, no block-table pass
    fresh = _seqs(g, 2, 300, decode=False, seq0=500)
    for s in fresh:
        s.num_cached_tokens = 0
    assert b.build_prefill(fresh)[3] is False


def test_sampling_parameter_normalisation():
    """top_k None / <= 0 -> V and capped at V, top_p None -> 1, min_p None -> 0,
    greedy = temperature <= 1e-5, and the use_* switches (batch.py:217-251)."""
    from xvllm.batch import SeqSchedule

    b = _batch()
    mk = lambda i, **kw: SeqSchedule(seq_id=i, token_ids=[1], num_cached_tokens=3, block_table=[i], **kw)
    seqs = [mk(0, temperature=0.0), mk(1, temperature=0.7, top_k=50, top_p=0.9),
            mk(2, temperature=1.0, top_k=0, min_p=0.05), mk(3, temperature=1e-6, top_k=V + 10),
            mk(4, temperature=0.8, top_k=-3, top_p=None)]
    b.build_decode(seqs)
    assert np.allclose(b.temperatures[:5].numpy(), [0.0, 0.7, 1.0, 1e-6, 0.8])
    assert b.top_ks[:5].tolist() == [V, 50, V, V, V]
    assert np.allclose(b.top_ps[:5].numpy(), [1.0, 0.9, 1.0, 1.0, 1.0])
    assert np.allclose(b.min_ps[:5].numpy(), [0.0, 0.0, 0.05, 0.0, 0.0])
    assert (b.all_greedy, b.any_greedy, b.use_top_k, b.use_top_p, b.use_min_p, b.max_top_k) == \
        (False, True, True, True, True, V)
    greedy = [mk(i, temperature=0.0) for i in range(3)]
    b.build_decode(greedy)
    assert (b.all_greedy, b.use_top_k, b.use_top_p, b.use_min_p, b.max_top_k) == (True, False, False, False, 0)


def test_graph_buckets_and_padding():
    """Decode graph buckets 1, 2, 4, 8, 16, 32, ... up to max_bs (max_bs
    included), and a batch pads to the smallest bucket that holds it
    (cuda_graph.py:38-52)."""
    from xvllm.cuda_graph import HipGraphRunner

    for max_bs in (1, 5, 16, 100, 256):
        bs = HipGraphRunner.make_bs_list(max_bs)
        assert bs == sorted(set(bs)) and bs[-1] == max_bs and all(b <= max_bs for b in bs)
        r = HipGraphRunner(bs, CPU)
        for n in range(1, max_bs + 1):
            p = r._pad_bs(n)
            assert p >= n and p in bs and not any(n <= b < p for b in bs)
    assert HipGraphRunner.make_bs_list(256)[:6] == [1, 2, 4, 8, 16, 32]


def test_staging_rejects_bad_pages_positions_and_ids():
    """With the pool size known, a page id outside the pool, a position past
    the block table or an input id outside the vocabulary raises on the host
    before anything is staged for a kernel; padding rows are staged greedy."""
    import pytest

    from xvllm.batch import Batch, SeqSchedule

    def mk():
        return Batch(max_bs=16, max_tokens=2048, max_blocks=32, vocab_size=V, device=CPU, block_size=16,
                     num_blocks=100)

    ok = SeqSchedule(1, [5], 20, [3, 4])
    mk().build_decode([ok], pad_to=2)
    for bad in (SeqSchedule(1, [5], 20, [3, 100]),       # page past the pool
                SeqSchedule(1, [5], 20, [-1, 4]),        # negative page
                SeqSchedule(1, [5], 32, [3, 4]),         # position 32 has no page
                SeqSchedule(1, [V], 20, [3, 4]),         # id outside the vocabulary
                SeqSchedule(1, [5], 20, list(range(33)))):  # more blocks than a row holds
        with pytest.raises(ValueError):
            mk().build_decode([bad])
    with pytest.raises(ValueError):
        mk().build_prefill([SeqSchedule(1, list(range(40)), 0, [3, 4])])   # 40 tokens, 2 pages
    with pytest.raises(ValueError):
        mk().build_prefill([SeqSchedule(1, [1, 2, 3], 0, [150])])
    # an appended page is checked too
    b = mk()
    b.build_decode([SeqSchedule(7, [5], 31, [3, 4])])
    with pytest.raises(ValueError):
        b.build_decode([SeqSchedule(7, [5], 32, [3, 4, 999])])
    # padding rows sample greedily
    b = mk()
    b.temperatures.fill_(0.7)
    b.build_decode([SeqSchedule(1, [5], 20, [3, 4], temperature=0.9)], pad_to=4)
    assert b.temperatures[:4].tolist() == pytest.approx([0.9, 0.0, 0.0, 0.0])
