"""Shared seeded input builders for the parity tests."""
from __future__ import annotations

import numpy as np
import torch


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def randn_bf16(shape, g, std=1.0, mean=0.0):
    """fp32 draw then bf16 cast (how every synthetic input here is made)."""
    return (torch.randn(shape, generator=g) * std + mean).to(torch.bfloat16)


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().to("cpu", torch.float32).numpy()


def make_paged(ctx_lens, num_blocks_pool, hkv, d, g, page=16, fill_nan=True):
    """Random-permutation block tables over a pool; unused pool rows hold NaN
    so any read past a sequence end shows up in the output."""
    ctx_lens = [int(c) for c in ctx_lens]
    need = [(c + page - 1) // page for c in ctx_lens]
    assert sum(need) <= num_blocks_pool
    perm = torch.randperm(num_blocks_pool, generator=g).tolist()
    max_blocks = max(max(need), 1)
    bt = torch.full((len(ctx_lens), max_blocks), -1, dtype=torch.int32)
    o = 0
    for b, n in enumerate(need):
        bt[b, :n] = torch.tensor(perm[o : o + n], dtype=torch.int32)
        o += n
    kc = randn_bf16((num_blocks_pool, page, hkv, d), g)
    vc = randn_bf16((num_blocks_pool, page, hkv, d), g)
    if fill_nan:
        valid = torch.zeros(num_blocks_pool, page, dtype=torch.bool)
        for b, c in enumerate(ctx_lens):
            for p in range(c):
                valid[bt[b, p // page], p % page] = True
        kc[~valid] = float("nan")
        vc[~valid] = float("nan")
    return kc, vc, bt, torch.tensor(ctx_lens, dtype=torch.int32)
