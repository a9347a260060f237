"""The serving page ledger and its radix prefix cache on the CPU
(reference src/data/kv.py:40-119, block_manager.py, radix_index.py):

- unit cases: a hit reuses the cached prefix pages (never the block of the
  last token), publishing on fill and on finish, cached pages come back on a
  later hit, eviction frees only unpinned leaves, the fit rule counts
  reclaimable pages as the reference's _fit_prefix does;
- serve() over a fake runner that keeps each page's token contents: every
  position a step attends to holds that sequence's own token (so a hit reads
  the right pages and no page owned by a live sequence is ever handed to
  another), the ledger's invariants hold after every step, and the outputs
  with the prefix cache equal those without it while fewer tokens are
  prefilled.
"""
from collections import deque

import numpy as np
import pytest
import torch

from xvllm.kv_manager import KVManager, KVPoolExhausted

BS = 4


def toks(n, base=0):
    return [base + i for i in range(n)]


def test_hit_reuses_prefix_pages_and_never_the_last_block():
    m = KVManager(32, BS)
    a = toks(13)  # 4 blocks, 3 full
    bt_a, c_a = m.allocate(0, a)
    assert c_a == 0 and len(bt_a) == 4
    m.publish(0, a, bt_a, 13)  # prefill done: 3 full blocks published
    assert m.published_blocks(0) == 3
    # same first 8 tokens: two blocks hit
    b = a[:8] + [99] * 5
    bt_b, c_b = m.allocate(1, b)
    assert bt_b[:2] == bt_a[:2] and c_b == 8 and not set(bt_b[2:]) & set(bt_a)
    # a prompt equal to a's first 12 tokens: its last token's block is recomputed
    bt_c, c_c = m.allocate(2, a[:12])
    assert bt_c[:2] == bt_a[:2] and c_c == 8 and bt_c[2] != bt_a[2]
    m.check({0: bt_a, 1: bt_b, 2: bt_c})
    assert m.ref[bt_a[0]] == 3


def test_finish_keeps_published_pages_cached_for_a_later_hit():
    m = KVManager(16, BS)
    a = toks(10)
    bt, _ = m.allocate(0, a)
    a2 = a + [50, 51, 52]            # three generated tokens, the last one's KV unwritten
    bt.append(m.append_page(0))
    m.deallocate(0, a2, bt, 12)      # 12 tokens written: 3 full blocks published
    m.check({})
    assert m.cached == set(bt[:3]) and m.num_free == 16 - 3
    # the last sampled token's block (tokens 12..15) was not published
    bt2, c2 = m.allocate(1, a2 + [7, 7, 7, 7])
    assert bt2[:3] == bt[:3] and c2 == 12
    m.check({1: bt2})
    assert not m.cached


def test_eviction_takes_only_unpinned_leaves_lru():
    m = KVManager(8, BS)
    a, b = toks(9), toks(9, 1000)
    bt_a, _ = m.allocate(0, a)
    m.deallocate(0, a, bt_a, 8)           # 2 blocks cached
    bt_b, _ = m.allocate(1, b)
    m.publish(1, b, bt_b, 8)              # b's 2 blocks published, pinned by the live sequence 1
    assert m.num_free == 3 and len(m.cached) == 2  # a's third page went back to free
    # 4 fresh pages needed with 2 free: a's cached leaf goes, b's pinned one stays
    c = toks(16, 5000)
    assert m.can_allocate(c)
    bt_c, _ = m.allocate(2, c)
    assert not set(bt_c) & set(bt_b)
    assert set(bt_a[:2]) & set(bt_c)  # a's whole leaf was evicted, one of its pages reused
    m.check({1: bt_b, 2: bt_c})
    # nothing left to evict: b is pinned
    with pytest.raises(KVPoolExhausted):
        m.append_page(2)
        m.append_page(2)


def test_duplicate_blocks_stop_publishing_and_stay_reclaimable():
    """Two sequences compute the same blocks before either publishes: the
    second keeps its own pages (tables stay append-only) and publishes
    nothing; after the first ends, its cached pages are not pinned by the
    second, so an allocation can reclaim them."""
    m = KVManager(9, BS)
    a = toks(9)
    bt0, _ = m.allocate(0, a)
    bt1, c1 = m.allocate(1, a)
    assert c1 == 0 and not set(bt0) & set(bt1)
    m.publish(0, a, bt0, 9)
    m.publish(1, a, bt1, 9)  # blocks held under seq 0's pages: seq 1 stops publishing
    assert m.cache.cached_pages() == set(bt0[:2])
    m.deallocate(0, a, bt0, 9)
    m.check({1: bt1})
    assert m.cached == set(bt0[:2])
    bt2, _ = m.allocate(2, toks(20, 300))  # 4 free + the 2 cached pages of seq 0
    assert set(bt0[:2]) & set(bt2)
    m.check({1: bt1, 2: bt2})
    m.deallocate(1, a, bt1, 9)
    m.check({2: bt2})


def test_fit_counts_reclaimable_pages_like_the_reference():
    m = KVManager(6, BS)
    a = toks(9)
    bt_a, _ = m.allocate(0, a)                # 3 pages
    m.deallocate(0, a, bt_a, 8)               # 2 cached, 4 free
    # 6 blocks, 2 of them a hit: 4 fresh from 4 free -> fits
    assert m.can_allocate(a[:8] + toks(13, 900))
    # 7 blocks with no hit: 4 free + 2 reclaimable < 7
    assert not m.can_allocate(toks(28, 700))
    # 6 blocks with no hit: 4 free + 2 reclaimable (the cached pages outside the hit)
    assert m.can_allocate(toks(24, 700))


def test_without_prefix_cache_nothing_is_shared():
    m = KVManager(16, BS, prefix_cache=False)
    a = toks(9)
    bt_a, _ = m.allocate(0, a)
    m.publish(0, a, bt_a, 9)
    bt_b, c = m.allocate(1, a)
    assert c == 0 and not set(bt_a) & set(bt_b)
    m.deallocate(0, a, bt_a, 9)
    assert m.num_free == 16 - 3 and not m.cached


class _FakeBatch:
    def forget_rows(self):
        pass


class _FakeKV:
    def __init__(self, n):
        self.num_blocks = n


class FakeRunner:
    """Stands in for ModelRunner on the host: keeps the token id whose KV each
    slot holds, checks that every position a scheduled row attends to holds
    that sequence's own token, and samples a deterministic function of the
    whole context (so outputs do not depend on which pages held it)."""

    def __init__(self, num_pages, block_size, vocab=1000):
        self.block_size, self.kv, self.batch = block_size, _FakeKV(num_pages), _FakeBatch()
        self.slots = np.full(num_pages * block_size, -1, np.int64)
        self.vocab = vocab
        self.ctx = {}   # seq id -> tokens whose KV it has written
        self._pending = deque()  # (prefill ids, decode ids) of launched steps not read back
        self._last = []          # the last launched step's ids, decode rows first (the device's copy)
        self.launched_steps = 0

    def _check_and_write(self, s, new_tokens):
        bs = self.block_size
        bt = np.asarray(s.block_table, np.int64)
        start = s.num_cached_tokens
        ctx = self.ctx.setdefault(s.seq_id, [])
        # the cached positions: hit pages (first use) or this sequence's own earlier writes
        if start and not ctx:
            ctx.extend(self._hit_tokens.pop(s.seq_id)[:start])
        assert len(ctx) == start, (s.seq_id, len(ctx), start)
        pos = np.arange(start)
        got = self.slots[bt[pos // bs] * bs + pos % bs]
        assert np.array_equal(got, np.asarray(ctx[:start])), f"seq {s.seq_id}: a cached page lost its contents"
        pos = np.arange(start, start + len(new_tokens))
        self.slots[bt[pos // bs] * bs + pos % bs] = new_tokens
        ctx.extend(new_tokens)
        return int(sum((i + 1) * t for i, t in enumerate(ctx)) % self.vocab)

    def run_forward(self, decodes, prefills):
        # a device-fed decode input is the previous launched step's id of that row
        d = [self._check_and_write(s, [self._last[s.src_row]] if s.src_row >= 0 else s.token_ids) for s in decodes]
        p = [self._check_and_write(s, s.token_ids) for s in prefills]
        self._pending.append((p, d))
        self._last = d + p
        self.launched_steps += 1
        return len(p), len(d)

    def read_samples(self, n_p, n_d):
        p, d = self._pending.popleft()
        assert (len(p), len(d)) == (n_p, n_d)
        return p, d


def _workload(seed, n_req=24, vocab=1000):
    rng = np.random.default_rng(seed)
    shared = [rng.integers(0, vocab, int(rng.integers(5, 40))).tolist() for _ in range(3)]
    prompts = []
    for _ in range(n_req):
        k = int(rng.integers(0, 4))
        own = rng.integers(0, vocab, int(rng.integers(1, 30))).tolist()
        prompts.append((shared[k] if k < 3 else []) + own)
    prompts.append(list(prompts[0]))  # an exact repeat: the full-prompt-hit case
    prompts.append(shared[0][: (len(shared[0]) // BS) * BS])  # a prompt of whole blocks, all cached
    return prompts


_ORIG_ALLOC = KVManager.allocate


def _recording(monkeypatch, runner):
    """Make the ledger tell the fake runner each admitted prompt's tokens
    (what its hit pages must hold)."""
    runner._hit_tokens = {}

    def spy_alloc(self, sid, tokens):
        got = _ORIG_ALLOC(self, sid, tokens)
        if got is not None:
            runner._hit_tokens[sid] = list(tokens)
        return got

    monkeypatch.setattr(KVManager, "allocate", spy_alloc)


def _live_check(kvm, live):
    kvm.check({r.rid: r.bt for r in live})


@pytest.mark.parametrize("overlap", [False, True])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_serve_with_prefix_cache_matches_without(monkeypatch, seed, overlap):
    from xvllm import serving

    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **k: None)
    prompts = _workload(seed)
    gen = 7
    pages = sum((len(p) + gen + BS - 1) // BS for p in prompts)
    outs = {}
    for pc in (False, True):
        runner = FakeRunner(pages, BS)
        _recording(monkeypatch, runner)
        outs[pc] = serving.serve(runner, prompts, gen, max_num_seqs=6, max_num_batched_tokens=40,
                                 prefix_cache=pc, overlap=overlap, after_step=_live_check)
    assert outs[True][0] == outs[False][0]
    assert all(len(o) == gen for o in outs[True][0])
    st_on, st_off = outs[True][1], outs[False][1]
    assert st_off.hit_tokens == 0 and st_on.hit_tokens > 0
    assert st_on.prefill_tokens + st_on.hit_tokens == st_off.prefill_tokens


@pytest.mark.parametrize("overlap", [False, True])
@pytest.mark.parametrize("prefix_cache", [False, True])
def test_serve_under_page_pressure(monkeypatch, prefix_cache, overlap):
    """A pool only as large as the pages of the max_num_seqs largest
    requests: prompts wait for pages, cached pages are evicted for later
    prompts, no live page is ever reused, and the outputs equal those of a
    pool that holds everything."""
    from xvllm import serving

    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **k: None)
    prompts = _workload(5, n_req=40)
    gen, seqs = 5, 4
    demand = sorted(((len(p) + gen + BS - 1) // BS for p in prompts), reverse=True)
    small = sum(demand[:seqs])
    evicted = []
    orig_take = KVManager._take

    def spy_take(self):
        before = len(self.cached)
        p = orig_take(self)
        if len(self.cached) < before:
            evicted.append(p)
        return p

    monkeypatch.setattr(KVManager, "_take", spy_take)
    runner = FakeRunner(small, BS)
    _recording(monkeypatch, runner)
    outs, st = serving.serve(runner, prompts, gen, max_num_seqs=seqs, max_num_batched_tokens=32,
                             prefix_cache=prefix_cache, overlap=overlap, after_step=_live_check)
    big = FakeRunner(sum(demand), BS)
    _recording(monkeypatch, big)
    want, _ = serving.serve(big, prompts, gen, max_num_seqs=seqs, max_num_batched_tokens=32, prefix_cache=False,
                            overlap=False)
    assert outs == want
    if prefix_cache:
        assert evicted, "the run never had to evict a cached page"
        assert st.hit_tokens > 0
    with pytest.raises(ValueError, match="live requests may need"):
        serving.serve(FakeRunner(small - 1, BS), prompts, gen, max_num_seqs=seqs)


@pytest.mark.parametrize("prefilled", [False, True])
def test_overlapped_serving_keeps_one_step_in_flight(monkeypatch, prefilled):
    """With overlap, every step after the first is launched before the
    previous one is read back, decode inputs after a prefill or decode come
    from the device (src_row), and the outputs equal the one-step-at-a-time
    loop's."""
    from xvllm import serving

    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **k: None)
    prompts = _workload(3, n_req=20)
    gen = 6
    pages = sum((len(p) + gen + BS - 1) // BS for p in prompts)
    runs = {}
    for overlap in (False, True):
        runner = FakeRunner(pages, BS)
        _recording(monkeypatch, runner)
        if prefilled:  # the pool "holds" every prompt token but the last
            orig = runner._check_and_write

            def fill_then_check(s, toks, runner=runner, orig=orig):
                if s.seq_id not in runner.ctx:
                    bt = np.asarray(s.block_table, np.int64)
                    pos = np.arange(s.num_cached_tokens)
                    prompt = runner._hit_tokens[s.seq_id]
                    runner.slots[bt[pos // BS] * BS + pos % BS] = prompt[: s.num_cached_tokens]
                    runner.ctx[s.seq_id] = list(prompt[: s.num_cached_tokens])
                return orig(s, toks)

            runner._check_and_write = fill_then_check
        depth, fed = [], []
        orig_run = runner.run_forward

        def spy(decodes, prefills, runner=runner, orig_run=orig_run, depth=depth, fed=fed):
            depth.append(len(runner._pending))
            fed.extend(s.src_row >= 0 for s in decodes)
            return orig_run(decodes, prefills)

        runner.run_forward = spy
        outs, st = serving.serve(runner, prompts, gen, max_num_seqs=8, max_num_batched_tokens=48, overlap=overlap,
                                 prefilled=prefilled, after_step=_live_check)
        runs[overlap] = (outs, st, depth, fed)
    assert runs[True][0] == runs[False][0]
    assert all(len(o) == gen for o in runs[True][0])
    _, st, depth, fed = runs[True]
    assert depth[0] == 0 and all(d == 1 for d in depth[1:]), depth
    assert sum(fed) == st.decode_tokens - (len(prompts) if prefilled else 0)
    assert max(runs[False][2]) == 0 and not any(runs[False][3])
