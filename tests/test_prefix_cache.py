"""Host logic of the radix prefix cache and of the cascade grouping, on the
CPU: matches are the longest cached full-block prefixes (never the block of
a prompt's last token), inserts share existing pages and split edges, pins
protect nodes from eviction, eviction is least-recently-used by leaf; the
decode grouping equals a brute force over the block tables."""
import itertools

import numpy as np
import pytest

from xvllm.prefix_cache import RadixPrefixCache, block_hash, cascade_groups, chain_hashes

BS = 4


def test_block_hash_chain_matches_its_definition():
    import xxhash

    toks = list(range(10))
    h0 = xxhash.xxh64(np.asarray(toks[:4], np.int32).tobytes()).intdigest()
    h1x = xxhash.xxh64()
    h1x.update(h0.to_bytes(8, "little"))
    h1x.update(np.asarray(toks[4:8], np.int32).tobytes())
    assert chain_hashes(toks, 4, 2) == [h0, h1x.intdigest()]
    assert block_hash(toks[:4]) == h0
    # the same block after a different prefix hashes differently
    assert chain_hashes([9, 9, 9, 9] + toks[4:8], 4, 2)[1] != h1x.intdigest()


def test_match_insert_split_and_dedupe():
    c = RadixPrefixCache(BS)
    a = list(range(100, 113))            # 13 tokens: 3 full blocks
    pages_a, node_a = c.insert(a, [10, 11, 12, 13])
    assert pages_a == [10, 11, 12]
    # a prompt sharing two blocks: match gives their pages
    b = a[:8] + [7, 7, 7, 7, 7]
    assert c.match(b) == [10, 11]
    # the block of the last token is never matched: a prompt equal to a's first 12 tokens
    assert c.match(a[:12]) == [10, 11]
    assert c.match(a[:13]) == [10, 11, 12]
    # inserting b splits a's edge and keeps the tree's pages for the shared blocks
    pages_b, node_b = c.insert(b, [20, 21, 22, 23])
    assert pages_b == [10, 11, 22]
    assert c.match(a) == [10, 11, 12] and c.match(b + [0]) == [10, 11, 22]
    assert c.cached_pages() == {10, 11, 12, 22}
    # nothing shared: no match
    assert c.match([1, 2, 3, 4, 5, 6]) == []


def test_pins_protect_and_eviction_is_lru_by_leaf():
    c = RadixPrefixCache(BS)
    a = list(range(12))
    b = a[:4] + [50] * 8
    d = [77] * 12
    c.insert(a, [1, 2, 3])
    c.insert(b, [1, 5, 6])
    c.insert(d, [7, 8, 9])
    na = c.node_of(a)
    c.pin(na)
    c.match(d)  # d becomes the most recent
    freed = c.evict(1)
    assert freed == [5, 6]  # b's leaf: unpinned and least recently used
    freed = c.evict(10)
    assert sorted(freed) == [7, 8, 9]  # a's path is pinned
    c.unpin(na)
    assert sorted(c.evict(10)) == [1, 2, 3]
    assert c.cached_pages() == set()


def _brute_groups(bt, sl, bs, max_rows, min_blocks, max_prefix):
    """Every bucket of rows with equal first page (in row order, cut into runs
    of max_rows): its longest common leading run of pages within every row's
    full blocks."""
    live = [r for r in range(len(sl)) if sl[r] > 0]
    out = []
    firsts = sorted({bt[r][0] for r in live}, key=lambda p: min(r for r in live if bt[r][0] == p))
    for p in firsts:
        rows = [r for r in live if bt[r][0] == p]
        for c0 in range(0, len(rows), max_rows):
            part = rows[c0 : c0 + max_rows]
            if len(part) < 2:
                continue
            lim = min(min(sl[r] // bs for r in part), max_prefix, len(bt[0]))
            n = 0
            while n < lim and all(bt[r][n] == bt[part[0]][n] for r in part):
                n += 1
            if n >= min_blocks:
                out.append((n, tuple(part)))
    return out


@pytest.mark.parametrize("seed", range(6))
def test_cascade_groups_equal_brute_force(seed):
    rng = np.random.default_rng(seed)
    B, W, bs = 40, 12, 16
    bt = rng.integers(0, 10_000, (B, W)).astype(np.int32)
    # planted shared prefixes of various lengths among random rows
    for _ in range(5):
        rows = rng.choice(B, rng.integers(2, 9), replace=False)
        n = rng.integers(1, W)
        bt[rows, :n] = bt[rows[0], :n]
    sl = rng.integers(0, W * bs + 1, B)
    max_rows = int(rng.integers(2, 6))
    pre, info, rows = cascade_groups(bt, sl, bs, max_rows=max_rows, min_blocks=2, max_groups=100, max_prefix_blocks=9)
    want = _brute_groups(bt.tolist(), sl.tolist(), bs, max_rows, 2, 9)
    got = [(int(info[g, 3] // bs), tuple(rows[info[g, 0] : info[g, 0] + info[g, 1]].tolist()))
           for g in range(100) if info[g, 1] > 0]
    for g in range(100):
        if info[g, 1]:
            assert info[g, 2] == rows[info[g, 0]] and (pre[rows[info[g, 0] : info[g, 0] + info[g, 1]]] == info[g, 3]).all()
    assert sorted(got) == sorted(want)
    grouped = set(rows.tolist())
    assert all(pre[r] == 0 for r in range(B) if r not in grouped)
    # every group's rows really share those pages, and each row's prefix is written
    for n, part in got:
        assert all((bt[r, :n] == bt[part[0], :n]).all() and sl[r] >= n * bs for r in part)


def test_cascade_groups_keep_the_largest_and_pad_the_records():
    bt = np.array([[1, 2, 3, 4]] * 3 + [[9, 8, 7, 6]] * 2 + [[5, 5, 5, 5]], np.int32)
    sl = np.array([64] * 6)
    pre, info, rows = cascade_groups(bt, sl, 16, max_rows=16, min_blocks=1, max_groups=1, max_prefix_blocks=4)
    assert info.tolist() == [[0, 3, 0, 64]] and rows.tolist() == [0, 1, 2]
    assert pre.tolist() == [64, 64, 64, 0, 0, 0]
    pre, info, rows = cascade_groups(bt, sl, 16, max_rows=16, min_blocks=1, max_groups=4, max_prefix_blocks=2)
    assert info.tolist() == [[0, 3, 0, 32], [3, 2, 3, 32], [0, 0, 0, 0], [0, 0, 0, 0]]
    assert pre.tolist() == [32] * 5 + [0]


def test_cascade_gate_takes_the_cascade_only_past_the_measured_bytes():
    """Batch decode builds stage shared-prefix groups only when they share at
    least the gate's bytes of KV per layer; below it the batch runs plain."""
    import torch

    from xvllm.batch import Batch, SeqSchedule
    from xvllm.prefix_cache import CASCADE_MIN_SHARED_BYTES, cascade_pays

    tok_bytes = 8 * 128 * 2 * 2  # Qwen3 kv heads x head dim x (K, V) x bf16
    shared = [list(range(0, 32))]
    info = np.array([[0, 4, 0, 32 * 16], [0, 0, 0, 0]], np.int32)
    assert not cascade_pays(info, tok_bytes)
    big = np.array([[0, 4, 0, 8192 * 2], [0, 3, 4, 8192]], np.int32)
    assert cascade_pays(big, tok_bytes)  # 24576 tokens x 4 KB = 100 MB
    assert not cascade_pays(np.zeros((2, 4), np.int32), tok_bytes, 0)
    assert CASCADE_MIN_SHARED_BYTES == 8 << 20
    for gate, want in ((None, 0), (0, 4)):
        b = Batch(max_bs=8, max_tokens=64, max_blocks=64, vocab_size=100, device=torch.device("cpu"), block_size=16,
                  num_blocks=512, cascade_groups=2, cascade_min_blocks=4, cascade_token_bytes=tok_bytes,
                  cascade_min_shared_bytes=gate)
        seqs = [SeqSchedule(i, [1], 40 * 16 - 1, shared[0] + list(range(100 + 10 * i, 108 + 10 * i)))
                for i in range(4)]
        b.build_decode(seqs)
        assert b.cascade_rows == want
        assert int(b.cascade.prefix_tokens[:4].sum()) == (4 * 32 * 16 if want else 0)
