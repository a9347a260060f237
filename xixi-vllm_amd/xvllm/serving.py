"""Continuous batching over one ModelRunner on one GPU: the default step
policy of the reference scheduler (src/control/scheduler.py:58-154) reduced
to what drives the decode hot path, over the page ledger and radix prefix
cache of xvllm.kv_manager (src/data/kv.py:15-119).

Each step, every running sequence decodes one token (its last sampled one);
the rest of the token budget goes to prefill chunks of waiting prompts in
arrival order, at most one of them partial, and a step that has no decode
rows takes no trailing partial chunk.  A prompt's pages are taken when it is
admitted (reusing the pages of its longest cached full-block prefix, whose
tokens are then not prefilled again), a decode page when its first token is
written.  Once a step's ids are read back, the blocks it filled are
published to the prefix cache (sync_prefix, scheduler.py:185); a finished
sequence publishes and releases its pages (scheduler.py:194-205), the
published ones staying cached for later prompts until a fresh allocation
evicts them.  Generation stops after `gen` tokens per request (EOS is not
checked).  Every id the runner reads back is range-checked on the host.

One step in flight (overlap=True, the default): step N+1 is scheduled and
launched before step N's ids are read back, so the host's read-back,
bookkeeping and staging run while the device computes.  What step N+1 needs
of step N is known without its ids (which sequences run, their positions and
pages: generation is counted, not stopped by a token), except the decode
input ids themselves, which the runner takes from step N's sampled ids on
the device (SeqSchedule.src_row).  Publishing, releasing finished sequences
and the host's id check then trail the launches by one step.  overlap=False
reads each step back before the next is scheduled (the reference's order).

This is the measurement driver of configs 4 and 5, not the reference's
Scheduler: no preemption and no stop strings.  The pool must hold the pages
of the max_num_seqs largest requests (checked up front): a prompt that does
not fit yet waits for running requests to finish, and none is ever preempted.
"""
from __future__ import annotations

import time
from collections import deque
from dataclasses import dataclass, field
from typing import Callable

import torch

from .batch import SeqSchedule
from .kv_manager import KVManager


@dataclass(eq=False)
class Request:
    rid: int
    prompt: list[int]
    tokens: list[int] = field(default_factory=list)   # prompt + generated tokens read back so far
    bt: list[int] = field(default_factory=list)
    cached: int = 0              # positions whose KV steps already read back have written
    pos: int = 0                 # positions whose KV launched steps write (cached + those in flight)
    n_out: int = 0               # generated tokens of launched steps
    src: tuple[int, int] | None = None  # (step, row) of its newest sampled id while only the device has it
    hit: int = 0                 # prompt tokens whose KV came from the prefix cache
    admitted: bool = False
    finished: bool = False

    @property
    def out(self) -> list[int]:
        return self.tokens[len(self.prompt):]


@dataclass
class ServeStats:
    steps: int = 0
    decode_tokens: int = 0
    prefill_tokens: int = 0
    hit_tokens: int = 0          # prompt tokens served from the prefix cache
    host_s: float = 0.0          # host time scheduling and launching steps
    wall_s: float = 0.0
    step_end_s: list[float] = field(default_factory=list)  # when each step's ids were read back, since the start
    # a timing event recorded on the compute stream after each step's launches
    # (device-timeline step times: elapsed_time between two of them)
    step_events: list = field(default_factory=list)
    # per step: (decode rows, sum of their context lengths incl. the new token,
    # prefill tokens, prefill attention query-key pairs under the causal mask,
    # prefill rows sampled)
    step_work: list[tuple[int, int, int, int, int]] = field(default_factory=list)


@dataclass
class _Step:
    serial: int
    n_p: int
    n_d: int
    dreqs: list[Request]
    preqs: list[tuple[Request, int, bool]]  # (request, chunk tokens, prompt done)


def serve(runner, prompts: list[list[int]], gen: int, *, sampling: dict | None = None,
          max_num_seqs: int = 256, max_num_batched_tokens: int = 8192, num_pages: int | None = None,
          prefix_cache: bool = True, prefilled: bool = False, kv_manager: KVManager | None = None,
          overlap: bool = True, timing_events: bool = False,
          after_forward: Callable[[object, int, int], None] | None = None,
          after_step: Callable[[KVManager, list[Request]], None] | None = None
          ) -> tuple[list[list[int]], ServeStats]:
    """Generate `gen` tokens for every prompt; returns (outputs, stats).

    sampling: SeqSchedule fields shared by every request (temperature,
    top_p, top_k, min_p); greedy when None.  num_pages: pages of the pool
    handed out (default: all of the runner's pool).  prefix_cache: reuse
    cached prompt prefixes (the page ledger's radix cache); kv_manager: a
    ledger to use (and keep) instead of a new one.  overlap: keep one step in
    flight (module docstring).  timing_events: record a timing event after
    each step's launches (ServeStats.step_events), so that step times can be
    read on the device's timeline, which a slow host (a profiler's) cannot
    shorten the way it can shift read-back times.
    prefilled: the pool already holds the KV of every prompt token but the
    last (synthetic pages for a long-context decode measurement, whose prefill
    would dominate the run): admission allocates and matches pages as usual
    and publishes the prompt's full blocks at once, and each request starts
    decoding from its last prompt token; the first generated token comes from
    that decode step.
    after_forward(runner, n_prefill, n_decode) runs after each step's
    launches, before its ids are read back (tests use it to check the step on
    the device); after_step(ledger, live requests) after each step's
    read-back and bookkeeping.  Neither may launch steps of its own while a
    step is in flight (with overlap, use overlap=False for such hooks)."""
    samp = dict(sampling or {"temperature": 0.0})
    page = runner.block_size
    pool = runner.kv.num_blocks if num_pages is None else num_pages
    kvm = kv_manager or KVManager(pool, page, prefix_cache=prefix_cache)
    if kvm.num_pages > runner.kv.num_blocks:
        raise ValueError(f"the ledger hands out {kvm.num_pages} pages, the pool holds {runner.kv.num_blocks}")
    # at most max_num_seqs requests hold pages at once, and every page no live
    # request holds is free or reclaimable: admission may wait, never deadlock
    demand = sorted(((len(p) + gen + page - 1) // page for p in prompts), reverse=True)
    if sum(demand[:max_num_seqs]) > kvm.num_pages:
        raise ValueError(f"{min(max_num_seqs, len(prompts))} live requests may need {sum(demand[:max_num_seqs])} "
                         f"pages, the ledger holds {kvm.num_pages}")
    if gen < 1:
        raise ValueError(f"gen must be >= 1, got {gen}")
    runner.batch.forget_rows()  # block-table rows staged by an earlier run are not this run's
    reqs = [Request(i, list(p), list(p)) for i, p in enumerate(prompts)]
    waiting = deque(reqs)        # prompts not fully prefilled (admitted or not)
    running: list[Request] = []  # prefill done, not released
    in_flight: deque[_Step] = deque()
    st = ServeStats()
    serial = 0
    launched_at = None           # runner.launched_steps right after this run's last launch

    def admit(r: Request) -> bool:
        got = kvm.allocate(r.rid, r.prompt)
        if got is None:
            return False
        r.bt, r.cached = got
        r.pos = r.hit = r.cached
        r.admitted = True
        st.hit_tokens += r.cached
        if prefilled:
            r.cached = r.pos = len(r.prompt) - 1
            kvm.publish(r.rid, r.tokens, r.bt, r.cached)
        return True

    def schedule() -> _Step | None:
        nonlocal serial, launched_at
        if prefilled:  # admitted requests go straight to decoding
            active = sum(1 for r in running if r.n_out < gen)
            while waiting and active < max_num_seqs and admit(waiting[0]):
                running.append(waiting.popleft())
                active += 1
        decodes, dreqs = [], []
        for r in running:  # one token per running sequence (its last token)
            if r.n_out >= gen:
                continue  # done; released once its last step is read back
            if r.pos // page >= len(r.bt):
                r.bt.append(kvm.append_page(r.rid))
            if r.src is None:
                decodes.append(SeqSchedule(r.rid, [r.tokens[-1]], r.pos, r.bt, **samp))
            else:  # the previous step sampled it and only the device has it yet
                if r.src[0] != serial - 1 or runner.launched_steps != launched_at:
                    raise RuntimeError("a decode input must come from the step launched just before")
                decodes.append(SeqSchedule(r.rid, [0], r.pos, r.bt, src_row=r.src[1], **samp))
            dreqs.append(r)
        used = len(decodes)
        prefills, preqs = [], []
        for r in [] if prefilled else list(waiting):
            if len(decodes) + len(prefills) >= max_num_seqs:
                break
            remaining = max_num_batched_tokens - used
            if remaining <= 0:
                break
            if not r.admitted and not admit(r):  # pages at admission (the reference's _try_alloc)
                break
            need = len(r.prompt) - r.pos
            if remaining < need and prefills and not decodes:
                break  # prefill-first steps take no trailing partial chunk
            chunk = min(need, remaining)
            done = r.pos + chunk == len(r.prompt)
            prefills.append(SeqSchedule(r.rid, r.prompt[r.pos : r.pos + chunk], r.pos, r.bt,
                                        need_sample=done, **samp))
            preqs.append((r, chunk, done))
            used += chunk
            if not done:
                break  # at most one partial chunk per step
        if not decodes and not prefills:
            return None
        pairs = sum(c * r.pos + c * (c + 1) // 2 for r, c, _ in preqs)
        st.step_work.append((len(decodes), sum(r.pos + 1 for r in dreqs), used - len(decodes), pairs,
                             sum(1 for _, _, done in preqs if done)))
        n_p, n_d = runner.run_forward(decodes, prefills)
        launched_at = runner.launched_steps
        if timing_events:
            ev = torch.cuda.Event(enable_timing=True)
            ev.record()
            st.step_events.append(ev)
        step = _Step(serial, n_p, n_d, dreqs, preqs)
        # what the launched step writes and samples (its ids arrive later)
        for row, r in enumerate(dreqs):
            r.pos += 1
            r.n_out += 1
            r.src = (serial, row)
        for i, (r, chunk, done) in enumerate(preqs):
            r.pos += chunk
            if done:
                r.n_out += 1
                r.src = (serial, n_d + i)
                waiting.remove(r)
                running.append(r)
        serial += 1
        st.steps += 1
        st.decode_tokens += len(decodes)
        st.prefill_tokens += used - len(decodes)
        if after_forward is not None:
            after_forward(runner, len(prefills), len(decodes))
        return step

    def read_back(step: _Step) -> None:
        p_ids, d_ids = runner.read_samples(step.n_p, step.n_d)
        for row, (r, tok) in enumerate(zip(step.dreqs, d_ids)):
            r.tokens.append(tok)
            r.cached += 1
            if r.src == (step.serial, row):
                r.src = None
        for i, ((r, chunk, done), tok) in enumerate(zip(step.preqs, p_ids)):
            r.cached += chunk
            if done:
                r.tokens.append(tok)
                if r.src == (step.serial, step.n_d + i):
                    r.src = None
        for r in [*step.dreqs, *(r for r, _, _ in step.preqs)]:
            if r.cached // page > kvm.published_blocks(r.rid):
                kvm.publish(r.rid, r.tokens, r.bt, r.cached)
        for r in [r for r in step.dreqs + [r for r, _, done in step.preqs if done] if len(r.out) >= gen]:
            running.remove(r)
            r.finished = True
            kvm.deallocate(r.rid, r.tokens, r.bt, r.cached)
        if after_step is not None:
            after_step(kvm, [r for r in reqs if r.admitted and not r.finished])
        st.step_end_s.append(time.perf_counter() - t0)

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while waiting or running or in_flight:
        h0 = time.perf_counter()
        step = schedule() if (waiting or any(r.n_out < gen for r in running)) else None
        st.host_s += time.perf_counter() - h0
        if step is not None:
            in_flight.append(step)
        elif not in_flight:
            raise RuntimeError("no request can be scheduled (the pool cannot hold the next prompt)")
        if in_flight and (not overlap or step is None or len(in_flight) > 1):
            read_back(in_flight.popleft())
    torch.cuda.synchronize()
    st.wall_s = time.perf_counter() - t0
    return [r.out for r in reqs], st
