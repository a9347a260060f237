"""Radix prefix cache over KV pages, and the shared-prefix groups of a decode
batch that the cascade decode reads once per group.

The cache follows the reference's radix prefix index
(src/data/prefix/radix_index.py:20-129, radix_tree.py:45-185): a compressed
radix tree keyed by the chain hashes of full token blocks
(h_i = xxh64(tokens_i | h_{i-1}), hash_util.py:16-30), valued by the page ids
that hold those blocks; live sequences pin the nodes on their path, and only
unpinned leaves are evicted, least recently used first, a whole leaf at a
time.  A prompt that hits the tree reuses the pages of its longest cached
full-block prefix (at most all blocks but the one holding its last token, so
that the last token is still computed and sampled).

`cascade_groups` works on the page ids of a decode batch directly: rows whose
block tables start with the same pages share those blocks, whoever mapped
them.
"""
from __future__ import annotations

import heapq
import time
from dataclasses import dataclass, field

import numpy as np

try:
    import xxhash
except ImportError:  # pragma: no cover - the image ships xxhash
    xxhash = None


def block_hash(tokens, prev: int = -1) -> int:
    """Chain hash of one full block: xxh64 over the previous hash (8 bytes,
    little endian, absent for the first block) then the block's int32 token ids."""
    if xxhash is None:
        raise ImportError("xxhash is required for the prefix cache")
    h = xxhash.xxh64()
    if prev != -1:
        h.update(int(prev).to_bytes(8, "little", signed=False))
    h.update(np.asarray(tokens, dtype=np.int32).tobytes())
    return h.intdigest()


def chain_hashes(tokens, block_size: int, n_blocks: int) -> list[int]:
    out, h = [], -1
    for i in range(n_blocks):
        h = block_hash(tokens[i * block_size : (i + 1) * block_size], h)
        out.append(h)
    return out


@dataclass(eq=False)
class _Node:
    key: tuple = ()            # block hashes of this edge
    pages: tuple = ()          # page ids of those blocks
    parent: "_Node | None" = None
    children: dict = field(default_factory=dict)  # first hash of a child's key -> child
    refs: int = 0
    last_use: float = 0.0


class RadixPrefixCache:
    def __init__(self, block_size: int) -> None:
        self.block_size = block_size
        self.root = _Node(refs=1)
        self._page_node: dict[int, _Node] = {}

    # ------------------------------------------------------------ lookup
    def _walk(self, hashes: list[int], touch: bool) -> tuple[list[int], _Node, int]:
        """(pages of the longest cached prefix of `hashes`, the node it ends
        in, blocks matched inside that node's edge)."""
        node, pages, i = self.root, [], 0
        now = time.monotonic()
        while i < len(hashes):
            child = node.children.get(hashes[i])
            if child is None:
                break
            n = 0
            while n < len(child.key) and i + n < len(hashes) and child.key[n] == hashes[i + n]:
                n += 1
            if touch:
                child.last_use = now
            pages.extend(child.pages[:n])
            i += n
            if n < len(child.key):
                return pages, child, n
            node = child
        return pages, node, len(node.key)

    def match(self, tokens) -> list[int]:
        """Page ids of the longest cached full-block prefix of `tokens`,
        leaving the block of the last token out (it must be computed)."""
        n_blocks = max(0, (len(tokens) - 1) // self.block_size)
        if n_blocks == 0:
            return []
        return self.match_hashes(chain_hashes(tokens, self.block_size, n_blocks))

    def match_hashes(self, hashes: list[int]) -> list[int]:
        """Page ids of the longest cached prefix of a block-hash chain."""
        pages, _, _ = self._walk(hashes, touch=True)
        return pages

    # ------------------------------------------------------------ insert
    def _split(self, node: _Node, at: int) -> _Node:
        """Cut node's edge after `at` blocks; returns the new upper node."""
        up = _Node(key=node.key[:at], pages=node.pages[:at], parent=node.parent, refs=node.refs,
                   last_use=node.last_use)
        up.parent.children[up.key[0]] = up
        node.key, node.pages, node.parent = node.key[at:], node.pages[at:], up
        up.children = {node.key[0]: node}
        for p in up.pages:
            self._page_node[p] = up
        return up

    def insert(self, tokens, pages) -> tuple[list[int], "_Node"]:
        """Publish the full blocks of `tokens` held in `pages` (the sequence's
        block table).  Returns (the page ids the tree holds for those blocks,
        the deepest node): where the tree already caches a block, its page
        replaces the sequence's (the caller frees the duplicate)."""
        n_blocks = len(tokens) // self.block_size
        return self.insert_hashes(chain_hashes(tokens, self.block_size, n_blocks), pages)

    def insert_hashes(self, hashes: list[int], pages) -> tuple[list[int], "_Node"]:
        """insert() over the blocks' chain hashes (one per page of `pages`)."""
        n_blocks = len(hashes)
        node, i, out = self.root, 0, []
        now = time.monotonic()
        while i < n_blocks:
            child = node.children.get(hashes[i])
            if child is None:
                leaf = _Node(key=tuple(hashes[i:]), pages=tuple(pages[i:n_blocks]), parent=node, last_use=now)
                node.children[leaf.key[0]] = leaf
                for p in leaf.pages:
                    self._page_node[p] = leaf
                out.extend(leaf.pages)
                return out, leaf
            n = 0
            while n < len(child.key) and i + n < n_blocks and child.key[n] == hashes[i + n]:
                n += 1
            child.last_use = now
            if n < len(child.key):
                child = self._split(child, n)
            out.extend(child.pages)
            i += n
            node = child
        return out, node

    # ------------------------------------------------------------ pins
    def node_of(self, tokens) -> _Node:
        """The node a sequence with these (cached) tokens pins."""
        n_blocks = len(tokens) // self.block_size
        return self.node_of_hashes(chain_hashes(tokens, self.block_size, n_blocks))

    def node_of_hashes(self, hashes: list[int]) -> _Node:
        """The node that ends the cached path of `hashes` (split there if the
        path ends inside an edge); the root when nothing matches."""
        _, node, n = self._walk(hashes, touch=False)
        if node is not self.root and n < len(node.key):
            node = self._split(node, n)
        return node

    def pin(self, node: _Node) -> None:
        while node is not self.root:
            node.refs += 1
            node = node.parent

    def unpin(self, node: _Node) -> None:
        while node is not self.root:
            node.refs -= 1
            assert node.refs >= 0
            node = node.parent

    def cached_pages(self) -> set[int]:
        return set(self._page_node)

    def holds(self, page: int) -> bool:
        return page in self._page_node

    def held(self, pages) -> set[int]:
        """The pages of `pages` the tree holds."""
        return self._page_node.keys() & set(pages)

    # ------------------------------------------------------------ eviction
    def evict(self, n_pages: int) -> list[int]:
        """Free unpinned leaves, least recently used first, a whole leaf at a
        time, until n_pages pages are returned (or nothing more can go); a
        parent left without children becomes a candidate in turn."""
        freed: list[int] = []
        if n_pages <= 0:
            return freed
        heap, stack, seq = [], [self.root], 0
        while stack:  # the tree's nodes, not its pages: a walk per call
            n = stack.pop()
            if n.children:
                stack.extend(n.children.values())
            elif n is not self.root and n.refs == 0:
                heap.append((n.last_use, seq, n))
                seq += 1
        heapq.heapify(heap)
        while len(freed) < n_pages and heap:
            _, _, leaf = heapq.heappop(heap)
            freed.extend(leaf.pages)
            for p in leaf.pages:
                del self._page_node[p]
            parent = leaf.parent
            del parent.children[leaf.key[0]]
            if parent is not self.root and not parent.children and parent.refs == 0:
                heapq.heappush(heap, (parent.last_use, seq, parent))
                seq += 1
        return freed


# Shared bytes per layer (sum over a batch's groups of prefix tokens x kv bytes
# per token) from which the cascade decode pays.  Measured on MI355X at the
# Qwen3-32B attention shape (64 q / 8 kv heads, B 32 rows of 32777 tokens, us
# per layer, plain -> cascade, bf16 pages): 16 rows sharing 2048 tokens
# (8 MiB) 670 -> 665, 4096 tokens 663 -> 644, 8192 tokens 661 -> 614, 24576
# tokens 677 -> 473; fp8 pages: 2048 tokens (4 MiB) 362 -> 365, 4096 tokens
# (8 MiB) 360 -> 354, 8192 tokens 361 -> 339.  Below 8 MiB the prefix pass
# and the second merge cost what the saved reads give back.  (At exactly
# 32768 tokens, 2048 whole pages per row, the plain decode's stream-K ranges
# start every row's prefix together and the last-level cache serves the
# rows' repeat reads of a shared page: plain then wins up to 8192 shared
# tokens, 607 against 620 at 16 rows.  One more token breaks that alignment,
# and serving contexts are almost never so aligned.)
CASCADE_MIN_SHARED_BYTES = 8 << 20


def cascade_pays(group_info: np.ndarray, token_bytes: int, min_shared_bytes: int = CASCADE_MIN_SHARED_BYTES) -> bool:
    """Whether a batch's shared-prefix groups (cascade_groups' group_info)
    share enough KV per layer for the cascade decode to beat the plain one."""
    info = np.asarray(group_info)
    live = info[:, 1] > 1
    return bool(live.any()) and int(info[live, 3].astype(np.int64).sum()) * token_bytes >= min_shared_bytes


def cascade_groups(block_tables: np.ndarray, seqlens: np.ndarray, block_size: int, *, max_rows: int,
                   min_blocks: int, max_groups: int, max_prefix_blocks: int):
    """Shared-prefix groups of a decode batch from its block tables.

    Rows (with seqlen > 0) whose tables start with the same page are
    candidates; a group's prefix is the longest run of leading pages common
    to all its rows, limited to blocks every row has fully written
    (seqlen // block_size) and to max_prefix_blocks.  Buckets larger than
    max_rows are cut into runs of max_rows rows; groups whose prefix is
    shorter than min_blocks are dropped, and the max_groups groups with the
    most shared blocks x (rows - 1) are kept.

    Returns (prefix_tokens [B] int32, group_info [max_groups, 4] int32,
    group_rows) as numpy arrays: group g's record is (first index into
    group_rows, rows, first batch row, prefix tokens); trailing groups are
    empty (0 rows).
    """
    bt = np.asarray(block_tables)
    sl = np.asarray(seqlens).astype(np.int64)
    B = sl.shape[0]
    prefix = np.zeros(B, np.int32)
    live = np.nonzero(sl > 0)[0]
    buckets: dict[int, list[int]] = {}
    for r in live:
        buckets.setdefault(int(bt[r, 0]), []).append(int(r))
    groups = []
    for rows in buckets.values():
        for c in range(0, len(rows), max_rows):
            part = rows[c : c + max_rows]
            if len(part) < 2:
                continue
            full = int(min(sl[part] // block_size))
            lim = min(full, max_prefix_blocks, bt.shape[1])
            sub = bt[part, :lim]
            same = np.all(sub == sub[0], axis=0)
            n = lim if same.all() else int(np.argmin(same))
            if n >= min_blocks:
                groups.append((n * (len(part) - 1), n, part))
    groups.sort(key=lambda t: -t[0])
    groups = groups[:max_groups]
    info = np.zeros((max_groups, 4), np.int32)
    rows_out = []
    for g, (_, n, part) in enumerate(groups):
        prefix[part] = n * block_size
        info[g] = (len(rows_out), len(part), part[0], n * block_size)
        rows_out.extend(part)
    return prefix, info, np.asarray(rows_out, np.int32)
