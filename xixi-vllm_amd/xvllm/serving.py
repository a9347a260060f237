"""Continuous batching over one ModelRunner on one GPU: the default step
policy of the reference scheduler (src/control/scheduler.py:58-154) reduced
to what drives the decode hot path.

Each step, every running sequence decodes one token (its last sampled one);
the rest of the token budget goes to prefill chunks of waiting prompts in
arrival order, at most one of them partial, and a step that has no decode
rows takes no trailing partial chunk.  A prompt's pages are taken when it is
admitted, a decode page when its first token is written.  Generation stops
after `gen` tokens per request (EOS is not checked).  Every id the runner
reads back is range-checked on the host before it is fed back.

This is the measurement driver of config 4, not the reference's
Scheduler/KVManager: no preemption, no prefix cache, no stop strings.
"""
from __future__ import annotations

import time
from collections import deque
from dataclasses import dataclass, field
from typing import Callable

import torch

from .batch import SeqSchedule


@dataclass
class Request:
    rid: int
    prompt: list[int]
    out: list[int] = field(default_factory=list)
    bt: list[int] = field(default_factory=list)
    cached: int = 0


@dataclass
class ServeStats:
    steps: int = 0
    decode_tokens: int = 0
    prefill_tokens: int = 0
    host_s: float = 0.0
    wall_s: float = 0.0


def serve(runner, prompts: list[list[int]], gen: int, *, sampling: dict | None = None,
          max_num_seqs: int = 256, max_num_batched_tokens: int = 8192, num_pages: int | None = None,
          after_forward: Callable[[object, int, int], None] | None = None) -> tuple[list[list[int]], ServeStats]:
    """Generate `gen` tokens for every prompt; returns (outputs, stats).

    sampling: SeqSchedule fields shared by every request (temperature,
    top_p, top_k, min_p); greedy when None.  num_pages: pages of the pool
    handed out (default: all of the runner's pool).  after_forward(runner,
    n_prefill, n_decode) runs after each step's launches, before its ids are
    read back (tests use it to check the step on the device)."""
    samp = dict(sampling or {"temperature": 0.0})
    page = runner.block_size
    pool = runner.kv.num_blocks if num_pages is None else num_pages
    need_pages = sum((len(p) + gen + page - 1) // page for p in prompts)
    if need_pages > pool:
        raise ValueError(f"the requests need {need_pages} pages, the pool holds {pool}")
    free = list(range(pool))[::-1]
    reqs = [Request(i, list(p)) for i, p in enumerate(prompts)]
    waiting = deque(reqs)
    running: deque = deque()
    st = ServeStats()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while waiting or running:
        h0 = time.perf_counter()
        decodes, dreqs = [], []
        for r in running:  # one token per running sequence (its last sampled token)
            if len(decodes) >= max_num_seqs:
                break
            pos = r.cached
            if pos // page >= len(r.bt):
                r.bt.append(free.pop())
            decodes.append(SeqSchedule(r.rid, [r.out[-1]], pos, r.bt, **samp))
            dreqs.append(r)
        used = len(decodes)
        prefills, preqs = [], []
        for r in list(waiting):
            if len(decodes) + len(prefills) >= max_num_seqs:
                break
            remaining = max_num_batched_tokens - used
            if remaining <= 0:
                break
            if not r.bt:  # all of the prompt's pages at admission (the reference allocates at _try_alloc)
                r.bt = [free.pop() for _ in range((len(r.prompt) + page - 1) // page)]
            need = len(r.prompt) - r.cached
            if remaining < need and prefills and not decodes:
                break  # prefill-first steps take no trailing partial chunk
            chunk = min(need, remaining)
            done = r.cached + chunk == len(r.prompt)
            prefills.append(SeqSchedule(r.rid, r.prompt[r.cached : r.cached + chunk], r.cached, r.bt,
                                        need_sample=done, **samp))
            preqs.append((r, chunk, done))
            used += chunk
            if not done:
                break  # at most one partial chunk per step
        n_p, n_d = runner.run_forward(decodes, prefills)
        if after_forward is not None:
            after_forward(runner, len(prefills), len(decodes))
        st.host_s += time.perf_counter() - h0
        p_ids, d_ids = runner.read_samples(n_p, n_d)
        st.steps += 1
        st.decode_tokens += len(decodes)
        for r, tok in zip(dreqs, d_ids):
            r.cached += 1
            r.out.append(tok)
        for (r, chunk, done), tok in zip(preqs, p_ids):
            r.cached += chunk
            st.prefill_tokens += chunk
            if done:
                r.out.append(tok)
                waiting.remove(r)
                running.append(r)
        for r in [r for r in running if len(r.out) >= gen]:
            running.remove(r)
            free.extend(r.bt)
    torch.cuda.synchronize()
    st.wall_s = time.perf_counter() - t0
    return [r.out for r in reqs], st
