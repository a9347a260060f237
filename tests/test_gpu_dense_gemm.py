"""Weight-streaming decode GEMM (xv_dense_gemm) against a torch fp32 product
of the same bf16 operands: bf16 output (rtol/atol 1e-2: one bf16 rounding of
an fp32 sum), fp32 split-K partials (their sum within 1e-4 relative), and
the gate/up projection fused with SiLU-and-mul, all over weights in
the packed tile order (pack_weight, itself checked element by element on
the CPU) (reference
src/compute/layers/activation.py:6-8 over the bf16-rounded products,
rtol/atol 2e-2).  Row counts cover every 16-row tile count and ragged last
tiles; the Qwen3-8B shapes run at M 64."""
import pytest
import torch

pytestmark = pytest.mark.gpu

SHAPES = [(6144, 4096, 2, 8, 1), (4096, 4096, 4, 4, 4), (4096, 12288, 2, 8, 2), (256, 1024, 2, 4, 1),
          (512, 2048, 1, 8, 8), (1024, 4096, 1, 4, 2)]


def _operands(m, n, k, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((m, k), generator=g).to(torch.bfloat16)
    w = (torch.randn((n, k), generator=g) * 0.02).to(torch.bfloat16)
    return x, w


def _close(got, want, rtol, atol):
    err = (got - want).abs() - (atol + rtol * want.abs())
    assert torch.isfinite(got).all()
    assert (err <= 0).all(), f"max excess {err.max().item():.4g}"


@pytest.mark.parametrize("m", [1, 5, 16, 17, 33, 48, 64])
@pytest.mark.parametrize("shape", SHAPES)
def test_dense_gemm_bf16_and_parts(dev, m, shape):
    from xvllm.layers.linear import GEMM_BF16, GEMM_PARTS, dense_gemm, pack_weight

    n, k, ct, wv, p = shape
    print(f"dense gemm m {m} n {n} k {k} tiles {ct} waves {wv} parts {p}", flush=True)
    x, w = _operands(m, n, k, m * 7 + n)
    want = x.float() @ w.float().T
    xd, wd = x.to(dev), pack_weight(w.to(dev))
    out = dense_gemm(xd, wd, GEMM_BF16, col_tiles=ct, waves=wv)
    _close(out.float().cpu(), want, 1e-2, 1e-2)
    ps = dense_gemm(xd, wd, GEMM_PARTS, col_tiles=ct, waves=wv, parts=p)
    assert ps.parts.shape == (p, m, n)
    _close(ps.parts.sum(0).cpu(), want, 1e-4, 1e-3)


@pytest.mark.parametrize("m", [1, 9, 32, 64])
@pytest.mark.parametrize("tiles_waves", [(4, 4), (2, 8), (2, 4)])
def test_dense_gemm_silu_mul(dev, m, tiles_waves):
    from xvllm.layers.linear import GEMM_SILU_MUL, dense_gemm, pack_weight

    inter, k = 1024, 4096
    ct, wv = tiles_waves
    print(f"dense gemm silu m {m} I {inter} tiles {ct} waves {wv}", flush=True)
    x, w = _operands(m, 2 * inter, k, m + 3)
    gu = (x.float() @ w.float().T).to(torch.bfloat16).float()
    g, u = gu[:, :inter], gu[:, inter:]
    want = g * torch.sigmoid(g) * u
    out = dense_gemm(x.to(dev), pack_weight(w.to(dev)), GEMM_SILU_MUL, col_tiles=ct, waves=wv)
    assert out.shape == (m, inter)
    _close(out.float().cpu(), want, 2e-2, 2e-2)


def test_dense_gemm_strided_rows(dev):
    """x as a row-strided view (a slice of a wider buffer)."""
    from xvllm.layers.linear import GEMM_BF16, dense_gemm, pack_weight

    x, w = _operands(24, 512, 2048, 5)
    wide = torch.zeros((24, 2048 + 64), dtype=torch.bfloat16)
    wide[:, 32 : 32 + 2048] = x
    xv = wide.to(dev)[:, 32 : 32 + 2048]
    out = dense_gemm(xv, pack_weight(w.to(dev)), GEMM_BF16, col_tiles=4, waves=4)
    _close(out.float().cpu(), x.float() @ w.float().T, 1e-2, 1e-2)
