"""Batched token sampler with the interface of xixi-vllm's
``src/compute/sampler.py:20-119`` (``Sampler.forward``), running the gfx950
radix-select sampling kernel (one workgroup per row).

Semantics follow the reference: temperature <= 1e-5 rows (or ``all_greedy``)
take ``torch.argmax`` of the logits (a NaN counts as the maximum, so the
lowest NaN id wins; otherwise the lowest id on ties).  Sampled rows drop NaN
logits, where the reference's softmax would make the whole row NaN; otherwise
the logits are scaled by 1/temperature and filtered by top-k, then top-p
and min-p over the renormalised top-k set, keeping at least the best token.
The reference draws with ``torch.multinomial`` / exponential noise; here the
draw is an explicit uniform per row (``uniforms``, or ``torch.rand`` from
``generator`` when omitted) used as an inverse CDF over the kept tokens in
ascending id order with exact fixed-point masses, so a given uniform always
yields the same token -- the same distribution as the reference, made
reproducible.
"""
from __future__ import annotations

import torch
from torch import nn

from . import _C
from ._torch_glue import ptr, require_bf16, require_cuda, stream_of


_WORKSPACE: dict[tuple[str, int | None], torch.Tensor] = {}

# Workspaces replaced by a larger one stay allocated until the process ends:
# a hipGraph captured on an earlier one keeps its pointer and replays onto it.
_RETIRED: list[torch.Tensor] = []


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Per-device sampler workspace, zero-filled once and grown on demand (the
    kernels leave it zero after every call).  Growing must happen outside
    graph capture: callers that capture size it first with `reserve_workspace`
    for their largest batch (the size query never decreases with the batch).
    Calls on one device share it and must be ordered on one stream."""
    key = (device.type, device.index)
    ws = _WORKSPACE.get(key)
    if ws is None or ws.numel() < nbytes:
        if ws is not None:
            _RETIRED.append(ws)
        with torch.inference_mode(False):  # a plain tensor: later callers outside inference mode may use it
            ws = torch.zeros(max(nbytes, 4096), dtype=torch.uint8, device=device)
        _WORKSPACE[key] = ws
    return ws


def reserve_workspace(device: torch.device, max_batch: int, vocab: int) -> torch.Tensor:
    """Allocate the sampler workspace for every call of up to `max_batch`
    rows over `vocab` ids, before any graph that samples is captured."""
    return _workspace(torch.device(device), _C.lib().xv_sampler_workspace_size(max_batch, vocab))


def sample(
    logits: torch.Tensor,
    temperatures: torch.Tensor | None,
    top_ps: torch.Tensor | None = None,
    top_ks: torch.Tensor | None = None,
    min_ps: torch.Tensor | None = None,
    uniforms: torch.Tensor | None = None,
    *,
    all_greedy: bool = False,
    use_top_k: bool = False,
    use_top_p: bool = False,
    use_min_p: bool = False,
    out: torch.Tensor | None = None,
    multi_workgroup: bool = True,
    max_top_k: int = 0,
) -> torch.Tensor:
    """Raw entry: bf16 logits [B, V] -> int64 ids [B] (graph-capturable).

    With `multi_workgroup` (the default) the kernels get a workspace and split
    each row over several workgroups; without it one workgroup takes a row.
    `max_top_k` is the largest top-k of any row, as the reference's
    ``Batch.max_top_k``; at most 64 selects the two-launch top-k path.  All
    of these give the same ids."""
    require_cuda(logits)
    require_bf16(logits)
    if logits.stride(-1) != 1:
        logits = logits.contiguous()
    bsz, vocab = logits.shape
    flags = 0
    if all_greedy:
        flags |= _C.XV_SAMPLE_ALL_GREEDY
    if use_top_k:
        flags |= _C.XV_SAMPLE_USE_TOP_K
    if use_top_p:
        flags |= _C.XV_SAMPLE_USE_TOP_P
    if use_min_p:
        flags |= _C.XV_SAMPLE_USE_MIN_P
    if use_top_k and 0 < max_top_k <= 64:
        flags |= _C.XV_SAMPLE_TOP_K_LE_64

    def prep(t, dt):
        if t is None:
            return None
        require_cuda(t)
        t = t.to(dt)
        return t if t.is_contiguous() else t.contiguous()

    temps = prep(temperatures, torch.float32)
    tps, tks, mps, us = prep(top_ps, torch.float32), prep(top_ks, torch.int32), prep(min_ps, torch.float32), prep(uniforms, torch.float32)
    if out is None:
        out = torch.empty(bsz, dtype=torch.int64, device=logits.device)
    L = _C.lib()
    ws = _workspace(logits.device, L.xv_sampler_workspace_size(bsz, vocab)) if multi_workgroup else None
    _C.check(
        L.xv_sample(
            ptr(logits), logits.stride(0), bsz, vocab, ptr(temps), ptr(tps), ptr(tks), ptr(mps), ptr(us), flags,
            ptr(out), ptr(ws), ws.numel() if ws is not None else 0, stream_of(logits),
        ),
        "xv_sample",
    )
    return out


class Sampler(nn.Module):
    def forward(
        self,
        logits: torch.Tensor,
        temperatures: torch.Tensor,
        top_ps: torch.Tensor | None = None,
        top_ks: torch.Tensor | None = None,
        min_ps: torch.Tensor | None = None,
        generator: torch.Generator | None = None,
        *,
        all_greedy: bool = False,
        any_greedy: bool = False,
        use_top_k: bool = False,
        use_top_p: bool = False,
        use_min_p: bool = False,
        max_top_k: int = 0,
        uniforms: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """Returns [batch] token ids.  ``any_greedy`` is accepted for interface
        parity (the kernel checks each row's temperature itself); ``max_top_k``
        at most 64 selects the kernels' top-k path."""
        del any_greedy
        if uniforms is None and not all_greedy:
            uniforms = torch.rand(logits.shape[0], generator=generator, device=logits.device)
        return sample(
            logits, temperatures, top_ps, top_ks, min_ps, uniforms,
            all_greedy=all_greedy, use_top_k=use_top_k, use_top_p=use_top_p, use_min_p=use_min_p,
            max_top_k=max_top_k,
        )
