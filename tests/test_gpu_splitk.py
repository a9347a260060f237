"""Split-K o_proj / down_proj feeding the residual add + RMSNorm, on the GPU:
the partial-sum norm kernel equals fused_add_rmsnorm on the bf16 sum of the
partials bit for bit, the split GEMM + norm equals the unsplit chain within
the bf16 tolerance at the Qwen3-8B and -32B o_proj / down_proj shapes and
decode batch sizes (every split the measured table picks there), and a decode
step of a Qwen3-8B-width model (graphs, two layers) agrees with split-K off."""

import numpy as np
import pytest
import torch

import oracle.ops as O
import xvllm.layers.ops  # noqa: F401  (registers the vllm:: and xv:: ops)
from helpers import f32, gen, randn_bf16

pytestmark = pytest.mark.gpu


def _close(got, want, rtol=2e-2, atol=2e-2):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert np.isfinite(got).all()
    err = np.abs(got - want) - (atol + rtol * np.abs(want))
    assert (err <= 0).all(), f"max excess {err.max():.4g} at {np.unravel_index(err.argmax(), err.shape)}"


@pytest.mark.parametrize("nparts,rows,hidden", [(1, 7, 4096), (4, 64, 4096), (8, 3, 5120), (3, 256, 4096),
                                                (2, 33, 1024), (5, 1, 4104)])
def test_parts_norm_equals_fused_add_rmsnorm_on_the_sum(dev, nparts, rows, hidden):
    print(f"parts norm P {nparts} rows {rows} hidden {hidden}", flush=True)
    g = gen(nparts * 1000 + rows)
    parts = torch.randn((nparts, rows, hidden), generator=g) * 0.5
    r = randn_bf16((rows, hidden), g)
    w = randn_bf16((hidden,), g, std=0.1, mean=1.0)
    # the sum in the kernel's order (part 0 first), rounded to bf16 once
    acc = parts[0].clone()
    for p in range(1, nparts):
        acc += parts[p]
    x = acc.to(torch.bfloat16)
    xg, rg = x.to(dev), r.clone().to(dev)
    torch.ops.vllm.fused_add_rmsnorm(xg, rg, w.to(dev), 1e-6)
    rp = r.clone().to(dev)
    out = torch.ops.xv.fused_add_rmsnorm_parts(parts.to(dev), rp, w.to(dev), 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(rp, rg), "residual differs from fused_add_rmsnorm on the summed x"
    assert torch.equal(out, xg), "normalised rows differ from fused_add_rmsnorm on the summed x"
    want_x, want_r = O.fused_add_rmsnorm(f32(x), f32(r), f32(w), 1e-6)
    assert np.array_equal(f32(rp), want_r)
    _close(f32(out), want_x)


def test_parts_norm_rejects_bad_arguments(dev):
    r = torch.zeros((4, 4096), dtype=torch.bfloat16, device=dev)
    w = torch.ones(4096, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        torch.ops.xv.fused_add_rmsnorm_parts(torch.zeros((2, 4, 4096), device=dev, dtype=torch.bfloat16), r, w, 1e-6)
    with pytest.raises(ValueError):
        torch.ops.xv.fused_add_rmsnorm_parts(torch.zeros((2, 5, 4096), device=dev), r, w, 1e-6)
    with pytest.raises(RuntimeError):  # more than 8 partials: the kernel refuses
        torch.ops.xv.fused_add_rmsnorm_parts(torch.zeros((9, 4, 4096), device=dev), r, w, 1e-6)


@pytest.mark.parametrize("m,n,k", [(m, n, k) for n, k in ((4096, 4096), (4096, 12288)) for m in (8, 64, 128, 256)]
                         + [(m, n, k) for n, k in ((5120, 8192), (5120, 25600)) for m in (8, 32, 48, 96, 200)])
def test_split_linear_into_norm_matches_unsplit(dev, m, n, k):
    from xvllm.layers.layernorm import RMSNorm
    from xvllm.layers.linear import PartialSums, linear_into_norm, split_factor

    print(f"split-K M {m} N {n} K {k} P {split_factor(m, n, k)}", flush=True)
    g = gen(m + k)
    x = randn_bf16((m, k), g).to(dev)
    wt = (randn_bf16((n, k), g) * 0.02).to(torch.bfloat16).to(dev)
    r = randn_bf16((m, n), g).to(dev)
    norm = RMSNorm(n).to(dev).to(torch.bfloat16)
    y = linear_into_norm(x, wt)
    assert isinstance(y, PartialSums) == (split_factor(m, n, k) > 1)
    r1 = r.clone()
    h1, r1 = norm(y, r1)
    r2 = r.clone()
    h2, r2 = norm(torch.nn.functional.linear(x, wt), r2)
    torch.cuda.synchronize()
    _close(f32(r1), f32(r2))
    _close(f32(h1), f32(h2))
    if isinstance(y, PartialSums):
        _close(f32(y.materialize()), f32(torch.nn.functional.linear(x, wt)))


def test_split_k_decode_step_matches_unsplit(dev):
    """Two Qwen3-8B-width layers (hidden 4096, FFN 12288, 32/8 heads), a
    decode batch of 64 through the runner's graphs: split-K on and off give
    the same final hidden within bf16 tolerance (relative L2), and the split
    run's graph replay equals its eager run."""
    from xvllm.batch import SeqSchedule
    from xvllm.config import Qwen3Shape
    from xvllm.kv_pool import KVPool
    from xvllm.model_runner import ModelRunner
    from xvllm.models import Qwen3ForCausalLM

    cfg = Qwen3Shape(4096, 32, 8, 128, 12288, 2, vocab_size=4096, max_position_embeddings=8192)
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(dev):
            model = Qwen3ForCausalLM(cfg).random_init_(seed=6)
            kv = KVPool(cfg, num_blocks=64 * 40, block_size=16, device=dev, dtype=torch.bfloat16)
    finally:
        torch.set_default_dtype(torch.float32)
    kv.kv_cache.normal_()
    runner = ModelRunner(model, kv, max_num_seqs=64, context_len=1024, device=dev, stream_decode_gemms=True)
    g = gen(23)
    perm = torch.randperm(64 * 40, generator=g).tolist()
    seqs, o = [], 0
    for i in range(64):
        c = int(torch.randint(100, 600, (1,), generator=g))
        n = (c + 15) // 16
        seqs.append(SeqSchedule(seq_id=i, token_ids=[int(torch.randint(0, 4096, (1,), generator=g))],
                                num_cached_tokens=c - 1, block_table=perm[o : o + n]))
        o += n
    snap = kv.kv_cache.clone()
    out = {}
    for split in (True, False):
        model.set_split_k(split)
        kv.kv_cache.copy_(snap)
        runner.batch.build_decode(seqs, pad_to=64)
        with torch.inference_mode():
            out[split, "eager"] = runner._decode_body(64)[:64].clone()
        torch.cuda.synchronize()
    model.set_split_k(True)
    kv.kv_cache.copy_(snap)
    runner.batch.build_decode(seqs, pad_to=runner.graph_runner._pad_bs(64))
    graph = runner.decode_hidden(64).clone()
    torch.cuda.synchronize()
    assert torch.equal(graph, out[True, "eager"]), "split-K graph replay differs from its eager run"
    a, b = f32(out[True, "eager"]).astype(np.float64), f32(out[False, "eager"]).astype(np.float64)
    assert np.isfinite(a).all()
    rel = np.linalg.norm(a - b) / np.linalg.norm(b)
    assert rel < 1e-2, f"split-K vs unsplit relative L2 {rel:.3g}"
    runner.destroy()
