"""Static device buffers and their pinned host mirrors for one engine step
(reference src/compute/batch.py:37-251): decode / prefill metadata, block
tables and sampling parameters, staged on the host with numpy and copied
H2D without blocking, so that graph replays read them in place.

Decode metadata per sequence (batch.py:119-124): input id = last token,
position = num_cached_tokens, slot = bt[pos // BS] * BS + pos % BS,
cache_seqlens = pos + 1.  Rows padded up to a graph bucket get slot -1,
seqlen 0 and block table -1 (batch.py:133-136), and temperature 0, so that a
sampler graph recorded for the bucket treats them as greedy rows.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch


@dataclass
class SeqSchedule:
    """What the model runner needs of one scheduled sequence (the fields of the
    reference's wire record, src/data/batch.py:81-98)."""
    seq_id: int
    token_ids: list[int]            # decode: [last token]; prefill: this chunk's tokens
    num_cached_tokens: int
    block_table: list[int]
    temperature: float = 0.0
    top_p: float | None = None
    top_k: int | None = None
    min_p: float | None = None
    need_sample: bool = True
    # decode rows only: when >= 0, the input id is row src_row of the previous
    # step's sampled ids, still on the device (token_ids is then a placeholder)
    src_row: int = -1


def slots_for_range(block_table, start: int, end: int, block_size: int) -> np.ndarray:
    """Physical slot of every token position in [start, end) (sequence.py:26-51)."""
    p = np.arange(start, end, dtype=np.int64)
    bt = np.asarray(block_table, dtype=np.int64)
    return (bt[p // block_size] * block_size + p % block_size).astype(np.int32)


def _pinned(shape, dtype, fill=None, pin=True):
    t = torch.empty(shape, dtype=dtype, pin_memory=pin)
    if fill is not None:
        t.fill_(fill)
    return t


class Batch:
    def __init__(self, *, max_bs: int, max_tokens: int, max_blocks: int, vocab_size: int,
                 device: torch.device, block_size: int, num_blocks: int | None = None,
                 cascade_groups: int = 0, cascade_max_prefix_blocks: int = 0, cascade_min_blocks: int = 16,
                 cascade_max_rows: int = 16, cascade_token_bytes: int = 0,
                 cascade_min_shared_bytes: int | None = None) -> None:
        """`num_blocks`: pages in the KV pool; when given, every page id and
        slot staged for the device is checked against it on the host (a bad
        one raises ValueError instead of reaching a kernel).
        `cascade_groups` > 0: decode builds also stage the batch's
        shared-prefix groups (at most that many, of at most cascade_max_rows
        rows, prefixes of cascade_min_blocks .. cascade_max_prefix_blocks
        blocks) for the cascade decode, when they share at least
        cascade_min_shared_bytes of KV per layer (prefix tokens x
        cascade_token_bytes; default prefix_cache.CASCADE_MIN_SHARED_BYTES);
        otherwise the build stages no groups and cascade_rows is 0."""
        self.num_blocks = num_blocks
        self.max_bs, self.max_tokens, self.max_blocks = max_bs, max_tokens, max_blocks
        self.vocab_size, self.device, self.block_size = vocab_size, device, block_size
        gpu = lambda shape, dt, fill=0: torch.full(shape, fill, dtype=dt, device=device)
        self.input_ids = gpu((max_tokens,), torch.int64)
        self.positions = gpu((max_tokens,), torch.int64)
        self.slot_mapping = gpu((max_tokens,), torch.int32, -1)
        self.cache_seqlens = gpu((max_bs,), torch.int32)
        self.cu_seqlens_q = gpu((max_bs + 1,), torch.int32)
        self.cu_seqlens_k = gpu((max_bs + 1,), torch.int32)
        self.block_tables = gpu((max_bs, max_blocks), torch.int32, -1)
        self.temperatures = gpu((max_bs,), torch.float32)
        self.top_ps = gpu((max_bs,), torch.float32)
        self.top_ks = gpu((max_bs,), torch.int32)
        self.min_ps = gpu((max_bs,), torch.float32)
        self.all_greedy, self.any_greedy = True, False
        self.use_top_k = self.use_top_p = self.use_min_p = False
        self.max_top_k = 0
        # pinned host staging (plain host memory when the buffers live on the CPU,
        # which runs the same host logic without a GPU)
        pin = torch.device(device).type == "cuda"
        self._h_ids = _pinned((max_tokens,), torch.int64, pin=pin)
        self._h_pos = _pinned((max_tokens,), torch.int64, pin=pin)
        self._h_slot = _pinned((max_tokens,), torch.int32, -1, pin=pin)
        self._h_csl = _pinned((max_bs,), torch.int32, pin=pin)
        self._h_cuq = _pinned((max_bs + 1,), torch.int32, pin=pin)
        self._h_cuk = _pinned((max_bs + 1,), torch.int32, pin=pin)
        self._h_bt = _pinned((max_bs, max_blocks), torch.int32, -1, pin=pin)
        self._h_samp = _pinned((4, max_bs), torch.float32, pin=pin)
        self._h_topk = _pinned((max_bs,), torch.int32, pin=pin)
        self._h_feed = _pinned((2, max_bs), torch.int64, pin=pin)  # (batch row, source row) of device-fed ids
        self._feed = gpu((2, max_bs), torch.int64)
        self._bt_np = self._h_bt.numpy()
        self._row_len = np.full(max_bs, -1, dtype=np.int64)   # entries of each host row in sync
        self._row_sid = np.full(max_bs, -1, dtype=np.int64)   # sequence that owns the row
        self._samp_key = None
        # the pinned staging buffers feed non-blocking H2D copies: a build
        # waits for the previous build's copies before overwriting them (a
        # step that runs decode and prefill stages both into the same buffers)
        self._h2d_done = torch.cuda.Event() if torch.device(device).type == "cuda" else None
        self._h2d_pending = False
        # shared-prefix groups of the decode batch (static buffers a graph can hold)
        self.cascade = None
        self._casc_cfg = (cascade_groups, cascade_max_prefix_blocks or max_blocks, cascade_min_blocks,
                          cascade_max_rows)
        from .prefix_cache import CASCADE_MIN_SHARED_BYTES

        self._casc_gate = (cascade_token_bytes, CASCADE_MIN_SHARED_BYTES if cascade_min_shared_bytes is None
                           else cascade_min_shared_bytes)
        self.cascade_rows = 0  # rows in shared-prefix groups in the last decode build
        if cascade_groups > 0:
            from .layers.attention import CascadePlan

            self.cascade = CascadePlan(gpu((max_bs,), torch.int32), gpu((cascade_groups, 4), torch.int32),
                                       gpu((max_bs,), torch.int32), cascade_groups, self._casc_cfg[1])
            self._h_casc = _pinned((2 * max_bs + 4 * cascade_groups,), torch.int32, pin=pin)

    def _wait_staging(self) -> None:
        if self._h2d_pending:
            self._h2d_done.synchronize()
            self._h2d_pending = False

    def _staged(self) -> None:
        if self._h2d_done is not None:
            self._h2d_done.record()
            self._h2d_pending = True

    # ------------------------------------------------------------ block tables
    def _sync_block_tables(self, seqs: list[SeqSchedule]) -> None:
        """Bring host rows up to date (append-only growth writes one entry) and
        copy the used rows H2D in one transfer (batch.py:181-215)."""
        bt = self._bt_np
        dirty = False
        for i, s in enumerate(seqs):
            k = len(s.block_table)
            if self._row_sid[i] == s.seq_id and self._row_len[i] == k:
                continue
            if k > self.max_blocks:
                raise ValueError(f"sequence {s.seq_id}: {k} blocks, the batch holds at most {self.max_blocks}")
            if self._row_sid[i] == s.seq_id and self._row_len[i] == k - 1 and k > 0:
                bt[i, k - 1] = s.block_table[-1]
                self._check_pages(s.seq_id, bt[i, k - 1 : k])
            else:
                bt[i, :k] = s.block_table
                bt[i, k:] = -1
                self._check_pages(s.seq_id, bt[i, :k])
            self._row_sid[i], self._row_len[i] = s.seq_id, k
            dirty = True
        if dirty:
            n = len(seqs)
            self.block_tables[:n].copy_(self._h_bt[:n], non_blocking=True)

    def forget_rows(self) -> None:
        """Drop the record of which sequence's table each host row holds, so
        that the next build writes every row whole (a new run may reuse a
        sequence id with another table)."""
        self._row_sid[:] = -1
        self._row_len[:] = -1

    def _check_pages(self, seq_id: int, pages: np.ndarray) -> None:
        if self.num_blocks is not None and pages.size and (pages.min() < 0 or pages.max() >= self.num_blocks):
            raise ValueError(f"sequence {seq_id}: page id outside [0, {self.num_blocks}) in its block table")

    def _sync_sampling(self, seqs: list[SeqSchedule]) -> None:
        key = tuple((s.seq_id, s.temperature, s.top_p, s.top_k, s.min_p) for s in seqs)
        if key == self._samp_key:
            return
        self._samp_key = key
        n = len(seqs)
        v = self.vocab_size
        t = np.array([s.temperature for s in seqs], np.float32)
        p = np.array([1.0 if s.top_p is None else s.top_p for s in seqs], np.float32)
        k = np.array([v if (s.top_k is None or s.top_k <= 0) else min(s.top_k, v) for s in seqs], np.int32)
        m = np.array([0.0 if s.min_p is None else s.min_p for s in seqs], np.float32)
        h = self._h_samp.numpy()
        h[0, :n], h[1, :n], h[2, :n] = t, p, m
        self._h_topk.numpy()[:n] = k
        self.temperatures[:n].copy_(self._h_samp[0, :n], non_blocking=True)
        self.top_ps[:n].copy_(self._h_samp[1, :n], non_blocking=True)
        self.min_ps[:n].copy_(self._h_samp[2, :n], non_blocking=True)
        self.top_ks[:n].copy_(self._h_topk[:n], non_blocking=True)
        self.all_greedy = bool(np.all(t <= 1e-5))
        self.any_greedy = bool(np.any(t <= 1e-5))
        self.use_top_k = bool(np.any(k < v))
        self.use_top_p = bool(np.any(p < 1.0))
        self.use_min_p = bool(np.any(m > 0.0))
        self.max_top_k = int(k.max()) if self.use_top_k else 0

    # ------------------------------------------------------------ decode
    def build_decode(self, seqs: list[SeqSchedule], *, pad_to: int | None = None,
                     prev_ids: torch.Tensor | None = None) -> None:
        """Stage a decode batch.  Rows with src_row >= 0 take their input id
        from prev_ids[src_row] (the previous step's sampled ids, on the
        device) by a gather on the current stream, clamped into [0, vocab) so
        that an id the host has not yet checked can never index past the
        embedding; the host checks every id when it reads them back."""
        n = len(seqs)
        self._wait_staging()
        self._sync_block_tables(seqs)
        pos = np.fromiter((s.num_cached_tokens for s in seqs), np.int64, n)
        src = np.fromiter((s.src_row for s in seqs), np.int64, n)
        fed = src >= 0
        ids = np.fromiter((0 if s.src_row >= 0 else s.token_ids[-1] for s in seqs), np.int64, n)
        if fed.any():
            if prev_ids is None:
                raise ValueError("decode rows take ids from the previous step, but it left none on the device")
            if int(src.max()) >= prev_ids.numel():
                raise ValueError(f"source row {int(src.max())} past the previous step's {prev_ids.numel()} ids")
        short = pos // self.block_size >= self._row_len[:n]
        if short.any() or (pos < 0).any():
            i = int(np.argmax(short | (pos < 0)))
            raise ValueError(f"sequence {seqs[i].seq_id}: position {int(pos[i])} has no page in its block table")
        if ((ids < 0) | (ids >= self.vocab_size)).any():
            raise ValueError(f"decode input id outside [0, {self.vocab_size})")
        rows = np.arange(n)
        slot = self._bt_np[rows, pos // self.block_size].astype(np.int64) * self.block_size + pos % self.block_size
        self._h_ids.numpy()[:n] = ids
        self._h_pos.numpy()[:n] = pos
        self._h_slot.numpy()[:n] = slot
        self._h_csl.numpy()[:n] = pos + 1
        self.input_ids[:n].copy_(self._h_ids[:n], non_blocking=True)
        self.positions[:n].copy_(self._h_pos[:n], non_blocking=True)
        self.slot_mapping[:n].copy_(self._h_slot[:n], non_blocking=True)
        self.cache_seqlens[:n].copy_(self._h_csl[:n], non_blocking=True)
        if fed.any():
            rows = np.nonzero(fed)[0]
            k = rows.size
            feed = self._h_feed.numpy()
            feed[0, :k], feed[1, :k] = rows, src[rows]
            self._feed[:, :k].copy_(self._h_feed[:, :k], non_blocking=True)
            got = prev_ids.view(-1).index_select(0, self._feed[1, :k]).clamp_(0, self.vocab_size - 1)
            self.input_ids.index_copy_(0, self._feed[0, :k], got)
        self._sync_sampling(seqs)
        if self.cascade is not None:
            self._stage_cascade(n, pos + 1, pad_to or n)
        if pad_to is not None and pad_to > n:
            self.slot_mapping[n:pad_to].fill_(-1)
            self.cache_seqlens[n:pad_to].zero_()
            self.block_tables[n:pad_to].fill_(-1)
            self.temperatures[n:pad_to].zero_()  # padding rows sample greedily (cheapest path)
            self._row_sid[n:pad_to] = -1
            self._row_len[n:pad_to] = -1
        self._staged()

    def _stage_cascade(self, n: int, seqlens: np.ndarray, rows: int) -> None:
        from .prefix_cache import cascade_groups, cascade_pays

        groups, max_pre, min_blocks, max_rows = self._casc_cfg
        pre, info, grp_rows = cascade_groups(self._bt_np[:n], seqlens, self.block_size, max_rows=max_rows,
                                             min_blocks=min_blocks, max_groups=groups, max_prefix_blocks=max_pre)
        if len(grp_rows) and not cascade_pays(info, *self._casc_gate):
            pre[:], info[:], grp_rows = 0, 0, grp_rows[:0]  # the plain decode is faster for this batch
        h = self._h_casc.numpy()
        mb, ng = self.max_bs, len(grp_rows)
        h[:rows] = 0
        h[:n] = pre
        h[mb : mb + 4 * groups] = info.reshape(-1)
        h[mb + 4 * groups : mb + 4 * groups + ng] = grp_rows
        self.cascade_rows = ng
        c = self.cascade
        c.prefix_tokens[:rows].copy_(self._h_casc[:rows], non_blocking=True)
        c.group_info.view(-1).copy_(self._h_casc[mb : mb + 4 * groups], non_blocking=True)
        if ng:
            c.group_rows[:ng].copy_(self._h_casc[mb + 4 * groups : mb + 4 * groups + ng], non_blocking=True)

    # ------------------------------------------------------------ prefill
    def build_prefill(self, seqs: list[SeqSchedule]) -> tuple[int, int, int, bool]:
        self._wait_staging()
        ids, pos, slot = self._h_ids.numpy(), self._h_pos.numpy(), self._h_slot.numpy()
        cuq, cuk = self._h_cuq.numpy(), self._h_cuk.numpy()
        cuq[0] = cuk[0] = 0
        nt = max_q = max_k = 0
        for i, s in enumerate(seqs):
            start, n = s.num_cached_tokens, len(s.token_ids)
            end = start + n
            ids[nt : nt + n] = s.token_ids
            pos[nt : nt + n] = np.arange(start, end)
            if (end + self.block_size - 1) // self.block_size > len(s.block_table):
                raise ValueError(f"sequence {s.seq_id}: positions up to {end} need more pages than its block table")
            slot[nt : nt + n] = slots_for_range(s.block_table, start, end, self.block_size)
            self._check_pages(s.seq_id, np.asarray(s.block_table[: (end + self.block_size - 1) // self.block_size]))
            cuq[i + 1], cuk[i + 1] = cuq[i] + n, cuk[i] + end
            max_q, max_k = max(max_q, n), max(max_k, end)
            nt += n
        bs = len(seqs)
        if nt and ((ids[:nt] < 0) | (ids[:nt] >= self.vocab_size)).any():
            raise ValueError(f"prefill input id outside [0, {self.vocab_size})")
        self.input_ids[:nt].copy_(self._h_ids[:nt], non_blocking=True)
        self.positions[:nt].copy_(self._h_pos[:nt], non_blocking=True)
        self.slot_mapping[:nt].copy_(self._h_slot[:nt], non_blocking=True)
        self.cu_seqlens_q[: bs + 1].copy_(self._h_cuq[: bs + 1], non_blocking=True)
        self.cu_seqlens_k[: bs + 1].copy_(self._h_cuk[: bs + 1], non_blocking=True)
        has_cache = int(cuk[bs]) > int(cuq[bs])
        if has_cache:
            self._sync_block_tables(seqs)
        self._sync_sampling(seqs)
        self._staged()
        return nt, max_q, max_k, has_cache
