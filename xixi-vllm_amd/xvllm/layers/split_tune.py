"""Measure the K split of the two GEMMs that feed a residual add + RMSNorm
(o_proj and down_proj) per decode batch size, and print the table
xvllm.layers.linear.SPLIT_TABLE holds.

    python -m xvllm.layers.split_tune [--shapes 4096x4096,4096x12288,...]

For every weight shape [N, K] and decode graph bucket M, each K split P in
1, 2, 4, 8 (those that cut K into 64-element multiples; the norm sums at
most 8 partials) runs the GEMM
(F.linear for P 1, else the batched GEMM over split views that
linear_into_norm issues) followed by the norm that consumes it
(vllm::fused_add_rmsnorm, or xv::fused_add_rmsnorm_parts summing the P fp32
partials), 20 pairs captured in a graph and replayed, with enough weight
copies cycled that no call finds its weights in the 256 MB last-level cache.
The fastest P per (N, K, M) is the table entry.  Needs a GPU.
"""
from __future__ import annotations

import argparse
import json

import torch
import torch.nn.functional as F

from .linear import split_k_views

BUCKETS = (1, 2, 4, 8, 16, 32, 48, 64, 80, 96, 112, 128, 144, 160, 176, 192, 208, 224, 240, 256)
SHAPES = ((4096, 4096), (4096, 12288), (5120, 8192), (5120, 25600))  # Qwen3-8B / -32B o_proj, down_proj


def _graph_us(fn, iters: int = 20) -> float:
    for i in range(3):
        fn(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(iters):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    g.replay()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) / iters * 1e3


def measure(n: int, k: int, buckets=BUCKETS, device="cuda") -> dict[int, dict[int, float]]:
    """us of GEMM + norm per (M, P) for an [N, K] weight."""
    from . import ops  # noqa: F401  (registers the vllm:: / xv:: ops)

    dev = torch.device(device)
    nsets = max(2, int(2e9 // (n * k * 2)) + 1)
    ws = [torch.randn(n, k, device=dev, dtype=torch.bfloat16) for _ in range(nsets)]
    w_norm = torch.ones(n, device=dev, dtype=torch.bfloat16)
    out: dict[int, dict[int, float]] = {}
    for m in buckets:
        x = torch.randn(m, k, device=dev, dtype=torch.bfloat16)
        res = torch.randn(m, n, device=dev, dtype=torch.bfloat16)
        row = {}
        for p in (1, 2, 4, 8):
            if k % (p * 64):
                continue
            if p == 1:
                def step(i, x=x, res=res):
                    y = F.linear(x, ws[i % nsets])
                    torch.ops.vllm.fused_add_rmsnorm(y, res, w_norm, 1e-6)
            else:
                views = [split_k_views(x, w, p) for w in ws]

                def step(i, views=views, res=res):
                    parts = torch.bmm(*views[i % nsets], out_dtype=torch.float32)
                    torch.ops.xv.fused_add_rmsnorm_parts(parts, res, w_norm, 1e-6)
            row[p] = round(_graph_us(step), 2)
        out[m] = row
    del ws
    torch.cuda.empty_cache()
    return out


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--shapes", default=",".join(f"{n}x{k}" for n, k in SHAPES),
                    help="comma-separated NxK weight shapes")
    args = ap.parse_args()
    table = {}
    for spec in args.shapes.split(","):
        n, k = (int(v) for v in spec.lower().split("x"))
        res = measure(n, k)
        best = {m: min(row, key=row.get) for m, row in res.items()}
        for m, row in res.items():
            print(f"[{n}, {k}] M {m}: " + "  ".join(f"P{p} {us}" for p, us in row.items()) + f"  -> P {best[m]}",
                  flush=True)
        table[f"{n}x{k}"] = best
    print(json.dumps(table))


if __name__ == "__main__":
    main()
