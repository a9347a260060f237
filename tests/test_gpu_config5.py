"""Config 5 at full size on the GPU: Qwen3-32B attention shape (64 q / 8 kv
heads, group 8), batch 32 at context 32768, requests 0..15 sharing an
8192-token prefix mapped to the same KV pages (as a radix prefix cache maps
them), 16..31 independent; top-p 0.95 at T 1.0 over the 151936 vocabulary
with seeded draws.

- Attention: rows on both sides of the shared/independent split against the
  numpy oracle on their gathered pages; every row finite.
- Sampler: ids of all 32 rows bit-exact against the C oracle on the device's
  own logits (a random-init LM head over random hidden states) and uniforms.
"""
import numpy as np
import pytest
import torch

import oracle.ops as O
import oracle.sampler as S
from helpers import f32, gen

pytestmark = pytest.mark.gpu

BSZ, CTX, PREFIX, SHARED, HQ, HKV, D, V = 32, 32768, 8192, 16, 64, 8, 128, 151936


def _close(got, want, rtol=2e-2, atol=2e-2):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert np.isfinite(got).all()
    err = np.abs(got - want) - (atol + rtol * np.abs(want))
    assert (err <= 0).all(), f"max excess {err.max():.4g}"


def config5_block_tables(seed=55):
    """[32, 2048] page ids over the unique pages: rows < 16 start with the
    same 512 prefix pages."""
    npg, ppg = CTX // 16, PREFIX // 16
    unique = ppg + SHARED * (npg - ppg) + (BSZ - SHARED) * npg
    perm = torch.randperm(unique, generator=gen(seed)).to(torch.int32)
    bt = torch.empty((BSZ, npg), dtype=torch.int32)
    o = ppg
    for i in range(BSZ):
        if i < SHARED:
            bt[i, :ppg] = perm[:ppg]
            bt[i, ppg:] = perm[o : o + npg - ppg]
            o += npg - ppg
        else:
            bt[i] = perm[o : o + npg]
            o += npg
    return bt, unique


def test_config5_shared_prefix_decode_attention(dev):
    from xvllm.layers.attention import paged_decode_attention

    bt, unique = config5_block_tables()
    assert torch.equal(bt[0, : PREFIX // 16], bt[SHARED - 1, : PREFIX // 16])
    g = torch.Generator(device=dev).manual_seed(5)
    kc = torch.randn((unique, 16, HKV, D), generator=g, device=dev).to(torch.bfloat16)
    vc = torch.randn((unique, 16, HKV, D), generator=g, device=dev).to(torch.bfloat16)
    q = torch.randn((BSZ, HQ * D), generator=g, device=dev).to(torch.bfloat16)
    sl = torch.full((BSZ,), CTX, dtype=torch.int32, device=dev)
    btd = bt.to(dev)
    out = paged_decode_attention(q, kc, vc, btd, sl, HQ, HKV, D)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    for r in (0, 15, 16, 31):
        print(f"config5 attention row {r}", flush=True)
        pages = btd[r].long()
        kr, vr = f32(kc[pages].cpu()), f32(vc[pages].cpu())
        want = O.paged_decode_attention(f32(q[r : r + 1].cpu()).reshape(1, HQ, D), kr, vr,
                                        np.arange(CTX // 16, dtype=np.int32)[None, :], np.array([CTX]))
        _close(f32(out[r : r + 1].cpu()).reshape(1, HQ, D), want)


def test_config5_top_p_sampler_bitexact(dev):
    from xvllm.sampler import sample

    g = torch.Generator(device=dev).manual_seed(7)
    hidden = torch.randn((BSZ, 5120), generator=g, device=dev).to(torch.bfloat16)
    lm_head = (torch.randn((V, 5120), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    logits = torch.nn.functional.linear(hidden, lm_head)
    del lm_head
    temps = torch.ones(BSZ, device=dev)
    top_p = torch.full((BSZ,), 0.95, device=dev)
    u = torch.rand(BSZ, generator=g, device=dev)
    ids = sample(logits, temps, top_p, None, None, u, use_top_p=True)
    ids1 = sample(logits, temps, top_p, None, None, u, use_top_p=True, multi_workgroup=False)
    torch.cuda.synchronize()
    bits = logits.view(torch.int16).cpu().numpy().view(np.uint16)
    want = S.sample(bits, np.ones(BSZ, np.float32), np.full(BSZ, 0.95, np.float32), None, None,
                    u.cpu().numpy(), 4)
    assert np.array_equal(ids.cpu().numpy(), want)
    assert np.array_equal(ids1.cpu().numpy(), want)
