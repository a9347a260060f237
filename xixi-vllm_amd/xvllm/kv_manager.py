"""Page ledger of one KV pool for serving, with the radix prefix cache
(reference src/data/kv.py:15-119 over src/data/block_manager.py:33-176 and the
radix backend, src/data/prefix/radix_index.py:20-129).

Every page is in exactly one state:
- free: on the free list, no owner;
- used: owned by ref > 0 live sequences (a page is shared only as a
  prefix-cache hit, so ref > 1 implies the page is held by the tree);
- cached: ref 0 but held by the radix tree, reusable by a later hit and
  reclaimable by evicting its (unpinned) leaf.

The sequence-facing calls follow KVManager's:
- `allocate` = `_fit_prefix` + `allocate` (kv.py:40-84): the longest cached
  full-block prefix of the prompt is reused when the fresh pages the rest
  needs fit in free pages plus cached pages outside the hit; the hit pages
  are acquired (used: ref + 1; cached: back to used) and the sequence pins
  the tree node its hit ends in.  The block of the prompt's last token is
  never matched, so at least that token is computed and sampled; this closes
  the reference's full-prompt-hit case (scheduler.py:110-115 admits such a
  prompt with nothing to prefill).
- `append_page` = `may_append` (block_manager.py:168-176).
- `publish` = `sync_prefix` (kv.py:91-101): the blocks filled since the last
  call go into the tree and the sequence pins the new end of its path.
- `deallocate` (kv.py:102-119): publishes (unless told not to), unpins, and
  returns each page to cached (held by the tree) or free.

Deliberate differences:
- Only blocks whose KV has been written are published: the reference's
  deallocate counts the last sampled token, whose KV no step wrote, into its
  full blocks (kv.py:103, sequence.py:130-131).
- A block the tree already holds under another page (two sequences computed
  the same block before either published it) is not swapped into the
  publishing sequence's table, as radix_index.py:79-88 does: block tables stay
  append-only while a sequence runs (the decode graphs' staged tables are
  only ever extended).  That sequence publishes nothing from then on, and its
  duplicate pages are freed when it ends.  So every page on the tree path a
  live sequence pins is one it holds (ref > 0), and every cached page
  (ref 0) is in an unpinned subtree, reclaimable by eviction.
- Eviction frees unpinned leaves least recently used first when the free
  list is empty, as the reference's reclaim_fn route does; there is no second
  LRU of cached page ids (block_manager.py:47-48), since every cached page is
  in the tree.
"""
from __future__ import annotations

from collections import deque

import numpy as np

from .prefix_cache import RadixPrefixCache, block_hash


class KVPoolExhausted(RuntimeError):
    """No free page and nothing the prefix cache can give back."""


class KVManager:
    def __init__(self, num_pages: int, block_size: int, *, prefix_cache: bool = True) -> None:
        if num_pages <= 0:
            raise ValueError(f"num_pages must be > 0, got {num_pages}")
        if block_size <= 0:
            raise ValueError(f"block_size must be > 0, got {block_size}")
        self.num_pages, self.block_size = num_pages, block_size
        self.ref = np.zeros(num_pages, np.int32)
        self.free: deque[int] = deque(range(num_pages))
        self.cached: set[int] = set()
        self.cache = RadixPrefixCache(block_size) if prefix_cache else None
        self._hashes: dict[int, list[int]] = {}   # seq -> chain hashes of its published blocks
        self._pin: dict[int, object] = {}         # seq -> tree node it pins
        self._prompt_chain: dict[int, list[int]] = {}  # seq -> hashes of its prompt blocks, from admission
        self._stopped: set[int] = set()           # seqs that found their blocks cached under other pages
        self.hit_blocks = 0                       # blocks reused by allocate, over the ledger's life

    # ------------------------------------------------------------ state
    @property
    def num_free(self) -> int:
        return len(self.free)

    @property
    def num_available(self) -> int:
        """Free pages plus cached pages a fresh allocation may reclaim."""
        return len(self.free) + len(self.cached)

    def _chain(self, tokens, n_blocks: int, start: int = 0, prev: int = -1) -> list[int]:
        bs = self.block_size
        out = []
        for i in range(start, n_blocks):
            prev = block_hash(tokens[i * bs : (i + 1) * bs], prev)
            out.append(prev)
        return out

    def _take(self) -> int:
        """One page for a fresh block: from the free list, else by evicting
        unpinned leaves of the prefix cache."""
        if not self.free and self.cache is not None and self.cached:
            for p in self.cache.evict(1):
                if self.ref[p] == 0:
                    self.cached.discard(p)
                    self.free.append(p)
        if not self.free:
            raise KVPoolExhausted(f"all {self.num_pages} KV pages are in use")
        p = self.free.popleft()
        self.ref[p] = 1
        return p

    # ------------------------------------------------------------ sequences
    def fit_prefix(self, tokens) -> tuple[list[int], list[int]] | None:
        """(hit pages, chain hashes of the prompt's blocks but the last
        token's) when a prompt of `tokens` fits, else None (kv.py:40-55)."""
        bs = self.block_size
        need = (len(tokens) + bs - 1) // bs
        hit, hashes = [], []
        if self.cache is not None and len(tokens) > bs:
            hashes = self._chain(tokens, (len(tokens) - 1) // bs)
            hit = self.cache.match_hashes(hashes)
        reclaimable = sum(1 for p in hit if p in self.cached)
        other_cached = len(self.cached) - reclaimable
        if len(self.free) + other_cached >= need - len(hit):
            return hit, hashes
        return None

    def can_allocate(self, tokens) -> bool:
        return self.fit_prefix(tokens) is not None

    def allocate(self, seq_id: int, tokens) -> tuple[list[int], int] | None:
        """Pages for a new sequence's prompt: (block table, tokens whose KV the
        reused prefix pages already hold), or None when it does not fit."""
        if seq_id in self._hashes:
            raise ValueError(f"sequence {seq_id} already holds pages")
        fit = self.fit_prefix(tokens)
        if fit is None:
            return None
        hit, hashes = fit
        need = (len(tokens) + self.block_size - 1) // self.block_size
        for p in hit:
            if self.ref[p] == 0:
                self.cached.discard(p)
            self.ref[p] += 1
        table = list(hit) + [self._take() for _ in range(need - len(hit))]
        self._hashes[seq_id] = hashes[: len(hit)]
        self._prompt_chain[seq_id] = hashes
        if hit:
            node = self.cache.node_of_hashes(hashes[: len(hit)])
            self.cache.pin(node)
            self._pin[seq_id] = node
        self.hit_blocks += len(hit)
        return table, len(hit) * self.block_size

    def append_page(self, seq_id: int) -> int:
        """One more page for a running sequence (its next token starts a block)."""
        if seq_id not in self._hashes:
            raise ValueError(f"sequence {seq_id} holds no pages")
        return self._take()

    def published_blocks(self, seq_id: int) -> int:
        return len(self._hashes.get(seq_id, ()))

    def publish(self, seq_id: int, tokens, block_table: list[int], num_cached: int) -> None:
        """Put the sequence's full blocks whose KV is written (the first
        num_cached tokens of `tokens`) into the prefix cache (kv.py:91-101)."""
        if self.cache is None:
            return
        hashes = self._hashes[seq_id]
        full = min(num_cached // self.block_size, len(block_table))
        if full <= len(hashes) or seq_id in self._stopped:
            return
        known = self._prompt_chain.get(seq_id, ())
        if len(known) > len(hashes):  # computed at admission
            hashes.extend(known[len(hashes) : full])
        if full > len(hashes):
            hashes.extend(self._chain(tokens, full, len(hashes), hashes[-1] if hashes else -1))
        held = self.cache.match_hashes(hashes)
        if held != list(block_table[: len(held)]):  # the tree holds one of these blocks under another page
            self._stopped.add(seq_id)
            return
        _, node = self.cache.insert_hashes(hashes, block_table[:full])
        # pages the tree holds now and no live sequence owns cannot exist here:
        # the inserted pages are this sequence's own (ref >= 1)
        old = self._pin.pop(seq_id, None)
        self.cache.pin(node)
        if old is not None:
            self.cache.unpin(old)
        self._pin[seq_id] = node

    def deallocate(self, seq_id: int, tokens, block_table: list[int], num_cached: int, *,
                   publish: bool = True) -> None:
        """Release a finished (or preempted, publish=False) sequence's pages."""
        if publish:
            self.publish(seq_id, tokens, block_table, num_cached)
        node = self._pin.pop(seq_id, None)
        if node is not None:
            self.cache.unpin(node)
        self._hashes.pop(seq_id, None)
        self._prompt_chain.pop(seq_id, None)
        self._stopped.discard(seq_id)
        bt = np.asarray(block_table, np.int64)
        if bt.size == 0:
            return
        np.subtract.at(self.ref, bt, 1)  # a table lists a page once, but count repeats right anyway
        if (self.ref[bt] < 0).any():
            p = int(bt[np.argmax(self.ref[bt] < 0)])
            raise AssertionError(f"page {p} released more often than it was taken")
        released = dict.fromkeys(bt[self.ref[bt] == 0].tolist())  # in table order, once each
        if self.cache is None:
            self.free.extend(released)
            return
        held = self.cache.held(released)
        self.cached |= held
        self.free.extend(p for p in released if p not in held)

    # ------------------------------------------------------------ checks
    def check(self, live_tables: dict[int, list[int]] | None = None) -> None:
        """Assert the ledger's invariants (tests call this between steps):
        every page in exactly one of free / used / cached; a cached page is
        held by the tree; a page owned by several sequences is held by the
        tree; with `live_tables`, each page's ref equals the live tables that
        hold it."""
        free = set(self.free)
        assert len(free) == len(self.free), "a page is on the free list twice"
        used = set(np.nonzero(self.ref > 0)[0].tolist())
        assert not (free & used) and not (free & self.cached) and not (used & self.cached)
        assert len(free) + len(used) + len(self.cached) == self.num_pages, "a page is in no state"
        if self.cache is not None:
            assert all(self.cache.holds(p) for p in self.cached)
            assert all(self.cache.holds(p) for p in np.nonzero(self.ref > 1)[0].tolist())
        if live_tables is not None:
            cnt = np.zeros(self.num_pages, np.int64)
            for t in live_tables.values():
                np.add.at(cnt, np.asarray(t, np.int64), 1)
            assert np.array_equal(cnt, self.ref), "page refs differ from the live block tables"
