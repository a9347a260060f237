"""Small helpers turning torch tensors into the raw arguments of the C ABI."""
from __future__ import annotations

import torch


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def require_cuda(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("xvllm ops run on the GPU only (HIP kernels); got a CPU tensor")


def require_bf16(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and t.dtype != torch.bfloat16:
            raise TypeError(f"xvllm kernels take bfloat16 activations, got {t.dtype}")


def aligned16(t: torch.Tensor) -> bool:
    return t.data_ptr() % 16 == 0
