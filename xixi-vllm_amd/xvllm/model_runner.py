"""Per-step driver on one GPU (reference src/compute/model_runner.py:23-312):
decode (hipGraph replay per batch bucket, or eager) then prefill, sampling,
and an asynchronous D2H copy of the sampled ids on a side stream.

Unlike the reference, whose sampler runs eagerly after the decode graph
(model_runner.py:206), the LM head and the sampler of a decode step replay
as a second graph per (batch bucket, sampling mode): the mode is the set of
kernel switches the batch's parameters select (all greedy, top-k / top-p /
min-p in use, every top-k at most 64), so a graph is only replayed for
batches it was recorded for.  Sampling parameters and the uniform draws are
static buffers written before the replay."""
from __future__ import annotations

from collections import deque

import torch

from . import _C
from .batch import Batch, SeqSchedule
from .config import head_dim as _head_dim
from .cuda_graph import HipGraphRunner
from .kv_pool import KVPool
from .layers.attention import AttnInputs, AttnMetadata, attention_context
from .sampler import Sampler, reserve_workspace, sample


class SampledIdOutOfRange(RuntimeError):
    """A sampled id read back on the host lies outside [0, vocab): fed back as
    the next step's input it would index past the embedding table."""


def sample_mode(batch: Batch) -> int:
    """The xv_sample flag set the staged batch selects (the reference's
    host-side switches, batch.py:217-251)."""
    if batch.all_greedy:
        return _C.XV_SAMPLE_ALL_GREEDY
    f = 0
    if batch.use_top_k:
        f |= _C.XV_SAMPLE_USE_TOP_K
        if 0 < batch.max_top_k <= 64:
            f |= _C.XV_SAMPLE_TOP_K_LE_64
    if batch.use_top_p:
        f |= _C.XV_SAMPLE_USE_TOP_P
    if batch.use_min_p:
        f |= _C.XV_SAMPLE_USE_MIN_P
    return f


class ModelRunner:
    def __init__(self, model, kv: KVPool, sampler: Sampler | None = None, *, max_num_seqs: int = 256,
                 max_num_batched_tokens: int = 8192, context_len: int = 4096, device=None,
                 enforce_eager: bool = False, sample_modes: tuple[int, ...] = (), cascade_groups: int = 0,
                 cascade_max_prefix_blocks: int = 0, cascade_min_blocks: int = 16,
                 cascade_min_shared_bytes: int | None = None, stream_decode_gemms: bool = False) -> None:
        """`sample_modes`: sampling modes (see `sample_mode`) whose decode
        sampler graphs are recorded up front besides the all-greedy one;
        other modes are recorded at their first use.
        `cascade_groups` > 0: decode steps find up to that many groups of rows
        whose block tables share leading pages (a prefix cache's shared
        blocks) and read those pages once per group (cascade decode);
        cascade_max_prefix_blocks bounds the shared blocks per group (default:
        the whole table) and sizes the prefix pass.  A step takes the cascade
        only when its groups share at least cascade_min_shared_bytes of KV
        per layer (default prefix_cache.CASCADE_MIN_SHARED_BYTES, the measured
        point below which the plain decode is faster); the runner records a
        plain and a cascade decode graph per bucket and replays the one the
        staged batch selects.
        `stream_decode_gemms` (off by default: the dense GEMMs stay on
        PyTorch / hipBLASLt): pack the model's gate_up / down / o weights
        (model.pack_decode_weights) so that decode batches of at most 64 rows
        run them on the weight-streaming kernel; the weights must be final.
        The packed copies take model.packed_decode_bytes() of device memory
        (Qwen3-8B: 12.1 GB) beside the weights, which a KV pool sized before
        this runner does not see: size it with that figure as reserve_bytes.
        Packed copies an earlier runner made are kept either way (its graphs
        read them), and every runner of the model then uses them."""
        self.model = model
        if stream_decode_gemms and hasattr(model, "pack_decode_weights"):
            model.pack_decode_weights()
        self.kv = kv
        self.sampler = sampler or Sampler()
        self.generator: torch.Generator | None = None  # source of the sampler's uniform draws
        self.device = device or kv.device
        self.block_size = kv.block_size
        cfg = model.config
        self.hidden_size = cfg.hidden_size
        self._meta = AttnMetadata(kv_cache=kv.kv_cache, k_scale=getattr(kv, "k_scale", 1.0),
                                  v_scale=getattr(kv, "v_scale", 1.0))
        n_model_layers = len(model.model.layers)
        if kv.num_layers < n_model_layers:  # layer aliasing: layer i reads pool layer i % pool layers
            for i, layer in enumerate(model.model.layers):
                layer.self_attn.attn.layer_id = i % kv.num_layers
        self.max_bs = min(max_num_seqs, 256)
        max_blocks = (context_len + self.block_size - 1) // self.block_size
        self.batch = Batch(max_bs=self.max_bs, max_tokens=max(max_num_batched_tokens, self.max_bs),
                           max_blocks=max_blocks, vocab_size=cfg.vocab_size, device=self.device,
                           block_size=self.block_size, num_blocks=kv.num_blocks, cascade_groups=cascade_groups,
                           cascade_max_prefix_blocks=cascade_max_prefix_blocks, cascade_min_blocks=cascade_min_blocks,
                           cascade_max_rows=max(1, 128 // (cfg.num_attention_heads // cfg.num_key_value_heads)),
                           cascade_token_bytes=cfg.num_key_value_heads * _head_dim(cfg) * 2 * kv.dtype.itemsize,
                           cascade_min_shared_bytes=cascade_min_shared_bytes)
        self.vocab_size = cfg.vocab_size
        act_dtype = torch.bfloat16 if kv.dtype == torch.float8_e4m3fn else kv.dtype  # activations stay bf16
        self._decode_out = torch.zeros(self.max_bs, self.hidden_size, dtype=act_dtype, device=self.device)
        self._decode_ids = torch.zeros(self.max_bs, dtype=torch.int64, device=self.device)
        self._uniforms = torch.zeros(self.max_bs, dtype=torch.float32, device=self.device)
        self._copy_stream = torch.cuda.Stream(device=self.device)
        # two read-back slots (pinned ids + the event of their copy): a step's
        # ids may still wait to be read while the next step is launched
        self._readback = [(torch.empty(self.max_bs * 2, dtype=torch.int64, pin_memory=True), torch.cuda.Event())
                          for _ in range(2)]
        self._readback_next = 0
        self._pending: deque = deque()  # (slot, n_p, n_d) of launched steps not read back yet
        self._last_ids: torch.Tensor | None = None  # the last launched step's sampled ids, on the device
        self.launched_steps = 0  # steps staged for read-back so far (device-fed inputs name the last one)
        self.graph_runner: HipGraphRunner | None = None
        self.cascade_graph_runner: HipGraphRunner | None = None
        self._sample_graphs: dict[tuple[int, int], torch.cuda.CUDAGraph] = {}
        if not enforce_eager:
            # every workspace a graph will hold is allocated before the first capture
            reserve_workspace(self.device, self.max_bs, cfg.vocab_size)
            self.graph_runner = HipGraphRunner(HipGraphRunner.make_bs_list(self.max_bs), self.device)
            with torch.inference_mode():
                self.graph_runner.capture(lambda bs: self._decode_body(bs, cascade=False))
                if self.batch.cascade is not None:
                    self.cascade_graph_runner = HipGraphRunner(self.graph_runner.bs_list, self.device)
                    self.cascade_graph_runner.capture(lambda bs: self._decode_body(bs, cascade=True))
                for mode in dict.fromkeys((_C.XV_SAMPLE_ALL_GREEDY, *sample_modes)):
                    for bs in reversed(self.graph_runner.bs_list):
                        self._sample_graph(bs, mode)

    # ------------------------------------------------------------ decode
    def _use_cascade(self) -> bool:
        """Whether the staged decode batch has shared-prefix groups worth the
        cascade decode (the batch build applies the measured gate)."""
        return self.batch.cascade is not None and self.batch.cascade_rows > 0

    def _decode_attn(self, bs: int, cascade: bool) -> AttnInputs:
        return AttnInputs(slot_mapping=self.batch.slot_mapping[:bs], is_prefill=False,
                          cache_seqlens=self.batch.cache_seqlens[:bs], block_tables=self.batch.block_tables[:bs],
                          cascade=self.batch.cascade if cascade else None)

    def _decode_body(self, bs: int, cascade: bool | None = None) -> torch.Tensor:
        """The decode forward over the staged batch; cascade None: as the
        staged batch selects."""
        if cascade is None:
            cascade = self._use_cascade()
        with attention_context(self._meta):
            out = self.model(self.batch.input_ids[:bs], self.batch.positions[:bs], self._decode_attn(bs, cascade))
        self._decode_out[:bs] = out
        return self._decode_out[:bs]

    @torch.inference_mode()
    def decode_hidden(self, bs: int) -> torch.Tensor:
        """Final hidden states of the decode batch whose metadata is staged."""
        if self.graph_runner is not None and bs <= self.max_bs:
            runner = self.cascade_graph_runner if self._use_cascade() else self.graph_runner
            hidden, _ = runner.replay(bs)
            return hidden[:bs]
        return self._decode_body(bs)

    def _run_decode(self, seqs: list[SeqSchedule]) -> torch.Tensor:
        bs = len(seqs)
        pad_to = self.graph_runner._pad_bs(bs) if self.graph_runner is not None and bs <= self.max_bs else None
        self.batch.build_decode(seqs, pad_to=pad_to, prev_ids=self._last_ids)
        if pad_to is None:
            return self._sample_logits(self.decode_hidden(bs), bs)
        self.decode_hidden(bs)
        return self.decode_sample(bs)

    # ------------------------------------------------------------ decode sampling graphs
    def _sample_body(self, bs: int, mode: int) -> None:
        """LM head + sampler over the first bs rows of the decode output into
        the static id buffer, with the staged parameters and uniforms."""
        logits = self.model.compute_logits(self._decode_out[:bs])
        b = self.batch
        greedy = bool(mode & _C.XV_SAMPLE_ALL_GREEDY)
        sample(logits, None if greedy else b.temperatures[:bs], b.top_ps[:bs], b.top_ks[:bs], b.min_ps[:bs],
               None if greedy else self._uniforms[:bs], all_greedy=greedy,
               use_top_k=bool(mode & _C.XV_SAMPLE_USE_TOP_K), use_top_p=bool(mode & _C.XV_SAMPLE_USE_TOP_P),
               use_min_p=bool(mode & _C.XV_SAMPLE_USE_MIN_P),
               max_top_k=64 if mode & _C.XV_SAMPLE_TOP_K_LE_64 else 0, out=self._decode_ids[:bs])

    def _sample_graph(self, bs: int, mode: int) -> torch.cuda.CUDAGraph:
        """The sampler graph of bucket bs in `mode`, recorded on first use
        (after one eager run that sizes the GEMM's library workspace; the
        sampler workspace was reserved for max_bs rows beforehand)."""
        key = (bs, mode)
        graph = self._sample_graphs.get(key)
        if graph is None:
            torch.cuda.synchronize(self.device)
            self._sample_body(bs, mode)
            torch.cuda.synchronize(self.device)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool=self.graph_runner._mempool):
                self._sample_body(bs, mode)
            torch.cuda.synchronize(self.device)
            self._sample_graphs[key] = graph
        return graph

    @torch.inference_mode()
    def decode_sample(self, bs: int) -> torch.Tensor:
        """Ids [bs] of the decode rows whose hidden states are in the decode
        output, by the sampler graph of bs's bucket and the staged mode.  Rows
        past bs up to the bucket are padding, staged greedy by build_decode."""
        size = self.graph_runner.bucket(bs)
        mode = sample_mode(self.batch)
        if not mode & _C.XV_SAMPLE_ALL_GREEDY:  # rows past bs are greedy padding: no draw
            self._uniforms[:bs].uniform_(generator=self.generator)
        self._sample_graph(size, mode).replay()
        return self._decode_ids[:bs]

    # ------------------------------------------------------------ prefill
    def _run_prefill(self, seqs: list[SeqSchedule]) -> torch.Tensor | None:
        nt, max_q, max_k, has_cache = self.batch.build_prefill(seqs)
        bs = len(seqs)
        attn = AttnInputs(slot_mapping=self.batch.slot_mapping[:nt], is_prefill=True,
                          cu_seqlens_q=self.batch.cu_seqlens_q[: bs + 1], cu_seqlens_k=self.batch.cu_seqlens_k[: bs + 1],
                          max_seqlen_q=max_q, max_seqlen_k=max_k,
                          block_tables=self.batch.block_tables[:bs] if has_cache else None)
        with attention_context(self._meta):
            hidden = self.model(self.batch.input_ids[:nt], self.batch.positions[:nt], attn)
        if not any(s.need_sample for s in seqs):
            return torch.zeros(bs, dtype=torch.int64, device=self.device)
        last = self.batch.cu_seqlens_q[1 : bs + 1].long() - 1
        return self._sample_logits(hidden[last], bs)

    # ------------------------------------------------------------ sampling
    def _sample_logits(self, hidden: torch.Tensor, bs: int) -> torch.Tensor:
        if self.batch.all_greedy:
            return self.model.argmax(hidden)
        logits = self.model.compute_logits(hidden)
        b = self.batch
        # drawn like the graph path's (uniform_ from the same generator), into a
        # buffer of its own: a decode sampler graph may still read _uniforms
        u = torch.empty(bs, dtype=torch.float32, device=self.device).uniform_(generator=self.generator)
        return self.sampler(logits, b.temperatures[:bs], top_ps=b.top_ps[:bs], top_ks=b.top_ks[:bs],
                            min_ps=b.min_ps[:bs], generator=self.generator, all_greedy=b.all_greedy,
                            any_greedy=b.any_greedy,
                            use_top_k=b.use_top_k, use_top_p=b.use_top_p, use_min_p=b.use_min_p,
                            max_top_k=b.max_top_k, uniforms=u)

    @torch.inference_mode()
    def run_forward(self, decodes: list[SeqSchedule], prefills: list[SeqSchedule]) -> tuple[int, int]:
        d = self._run_decode(decodes) if decodes else None
        p = self._run_prefill(prefills) if prefills else None
        return self._stage_samples(p, d)

    def _stage_samples(self, p, d) -> tuple[int, int]:
        """Queue this step's sampled ids for the host: decode rows first, then
        prefill rows, joined on the device (kept as the next step's source of
        device-fed decode inputs) and moved by one non-blocking copy on the
        side stream into a free read-back slot, so the next step's launches
        do not wait for it.  At most two steps may wait to be read back."""
        n_d = 0 if d is None else d.numel()
        n_p = 0 if p is None else p.numel()
        if len(self._pending) >= len(self._readback):
            raise RuntimeError("two steps' ids are already waiting to be read back")
        slot = self._readback_next
        self._readback_next = (slot + 1) % len(self._readback)
        cpu, event = self._readback[slot]
        side = self._copy_stream
        ids = None
        if n_d + n_p:
            if cpu.numel() < n_d + n_p:
                cpu = torch.empty(n_d + n_p, dtype=torch.int64, pin_memory=True)
                self._readback[slot] = (cpu, event)
            ids = torch.cat([t.view(-1) for t in (d, p) if t is not None])
        # the copy may start only after everything that produces `ids`,
        # the join included, has run on the compute stream
        side.wait_stream(torch.cuda.current_stream())
        if ids is not None:
            with torch.cuda.stream(side):
                cpu[: n_d + n_p].copy_(ids, non_blocking=True)
            ids.record_stream(side)  # made on the compute stream, read on the side stream
        event.record(side)
        self._last_ids = ids
        self._pending.append((slot, n_p, n_d))
        self.launched_steps += 1
        return n_p, n_d

    def read_samples(self, n_p: int, n_d: int) -> tuple[list[int], list[int]]:
        """(prefill ids, decode ids) of the oldest launched step not read back
        yet.  Every id is checked against [0, vocab) on the host before it is
        returned; a wrong id raises here (the device-fed decode inputs of a
        step launched meanwhile were clamped into range)."""
        if not self._pending:
            raise RuntimeError("no launched step is waiting to be read back")
        slot, pp, dd = self._pending.popleft()
        if (pp, dd) != (n_p, n_d):
            raise ValueError(f"the oldest waiting step has {dd} decode + {pp} prefill rows, not {n_d} + {n_p}")
        cpu, event = self._readback[slot]
        event.synchronize()
        ids = cpu[: n_d + n_p].tolist()
        bad = [(i, t) for i, t in enumerate(ids) if not 0 <= t < self.vocab_size]
        if bad:
            raise SampledIdOutOfRange(f"{len(bad)} sampled ids outside [0, {self.vocab_size}): "
                                      f"first (row, id) {bad[:4]} of {n_d} decode + {n_p} prefill rows")
        return ids[n_d:], ids[:n_d]

    def destroy(self) -> None:
        self._sample_graphs.clear()
        if self.graph_runner is not None:
            self.graph_runner.destroy()
            self.graph_runner = None
        if self.cascade_graph_runner is not None:
            self.cascade_graph_runner.destroy()
            self.cascade_graph_runner = None
