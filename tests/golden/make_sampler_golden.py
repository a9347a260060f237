"""Write tests/golden/sampler_ref.npz: the distributions xixi-vllm's own
Sampler (src/compute/sampler.py) samples from, for seeded bf16 logits.

Run in the build container only (needs /root/reference):
    python tests/golden/make_sampler_golden.py

The reference file is loaded by path (it imports only torch).  Its RNG calls
are intercepted to record what it samples from, so the fixture holds the
exact renormalised probabilities per token id:
  * top-k / top-p paths: torch.multinomial(probs over ordered candidates) with
    the candidate ids from torch.topk / torch.sort, mapped back to ids;
  * min-p-only path: torch.multinomial(probs over the vocabulary);
  * temperature-only path: the softmax fed to the Gumbel-max draw.
The fixture stores inputs (raw bf16 bits, per-row parameters) and outputs
(probabilities per id); nothing of the reference's source is stored.
"""
from __future__ import annotations

import importlib.util
import sys
import types
from pathlib import Path

import numpy as np
import torch

REF = Path("/root/reference/src/compute/sampler.py")
OUT = Path(__file__).resolve().parent / "sampler_ref.npz"


def load_ref():
    spec = importlib.util.spec_from_file_location("xixi_ref_sampler", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


class Recorder:
    """Stands in for the module's `torch` name; records the last candidate ids
    and the probabilities handed to the sampling draw."""

    def __init__(self):
        self.cand = None
        self.probs = None

    def __getattr__(self, name):
        return getattr(torch, name)

    def topk(self, x, k, dim=-1):
        v, i = torch.topk(x, k, dim=dim)
        self.cand = i.clone()
        return v, i

    def sort(self, x, descending=False, dim=-1):
        v, i = torch.sort(x, descending=descending, dim=dim, stable=True)
        self.cand = i.clone()
        return v, i

    def multinomial(self, p, n, generator=None):
        self.probs = p.clone()
        return torch.multinomial(p, n, generator=generator)

    def softmax(self, x, dim=-1):
        r = torch.softmax(x, dim=dim)
        self.softmax_out = r.clone()
        return r


def main():
    mod = load_ref()
    rec = Recorder()
    mod.torch = rec
    sampler = mod.Sampler()
    V = 4000
    g = torch.Generator().manual_seed(1234)
    cases = []
    # (temperature, top_p, top_k, min_p, use_top_k, use_top_p, use_min_p, logit std)
    specs = [
        (0.7, 0.9, 50, 0.0, True, True, False, 3.0),
        (1.0, 0.95, V, 0.0, False, True, False, 2.0),
        (0.5, 1.0, 20, 0.0, True, False, False, 2.0),
        (1.0, 1.0, V, 0.1, False, False, True, 2.0),
        (0.8, 0.8, 100, 0.05, True, True, True, 3.0),
        (1.3, 0.5, V, 0.0, False, True, False, 1.0),
        (1.0, 1.0, V, 0.0, False, False, False, 2.0),
        (0.9, 0.7, V, 0.2, False, True, True, 4.0),
    ]
    rows_logits, rows_probs, rows_params = [], [], []
    for (t, p, k, m, uk, up, um, std) in specs:
        for rep in range(2):
            logits = (torch.randn(1, V, generator=g) * std).to(torch.bfloat16)
            temps = torch.tensor([t], dtype=torch.float32)
            rec.cand = rec.probs = None
            rec.softmax_out = None
            sampler.forward(
                logits, temps, top_ps=torch.tensor([p]), top_ks=torch.tensor([k], dtype=torch.int32),
                min_ps=torch.tensor([m]), generator=torch.Generator().manual_seed(0),
                all_greedy=False, any_greedy=False, use_top_k=uk, use_top_p=up, use_min_p=um,
                max_top_k=k if uk else 0,
            )
            full = np.zeros(V, dtype=np.float64)
            if uk or up:
                pr = rec.probs[0].double()
                pr = pr / pr.sum()
                full[rec.cand[0].numpy()] = pr.numpy()
            elif um:
                pr = rec.probs[0].double()
                full[:] = (pr / pr.sum()).numpy()
            else:
                full[:] = rec.softmax_out[0].double().numpy()
            flags = (2 if uk else 0) | (4 if up else 0) | (8 if um else 0)
            rows_logits.append(logits.view(torch.int16).numpy()[0].astype(np.uint16))
            rows_probs.append(full)
            rows_params.append((t, p, k, m, flags))
    np.savez_compressed(
        OUT,
        logits_bits=np.stack(rows_logits),
        probs=np.stack(rows_probs).astype(np.float32),
        temp=np.array([r[0] for r in rows_params], np.float32),
        top_p=np.array([r[1] for r in rows_params], np.float32),
        top_k=np.array([r[2] for r in rows_params], np.int32),
        min_p=np.array([r[3] for r in rows_params], np.float32),
        flags=np.array([r[4] for r in rows_params], np.int32),
    )
    print(f"wrote {OUT} ({len(rows_params)} rows)")


if __name__ == "__main__":
    sys.exit(main())
