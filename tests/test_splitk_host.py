"""Split-K host logic on the CPU: the K-slice views of x and w are the
operands whose batched product sums to x @ w^T (checked in float64 against
the plain product, including the slice order), and the split table only
splits the shapes it was measured on."""
import pytest
import torch

from xvllm.layers.linear import split_factor, split_k_views


@pytest.mark.parametrize("m,n,k,p", [(5, 12, 32, 4), (3, 8, 24, 3), (1, 16, 64, 8), (7, 6, 10, 2)])
def test_split_views_sum_to_the_product(m, n, k, p):
    g = torch.Generator().manual_seed(m * n + k)
    x = torch.randn(m, k, generator=g, dtype=torch.float64)
    w = torch.randn(n, k, generator=g, dtype=torch.float64)
    xs, ws = split_k_views(x, w, p)
    assert xs.shape == (p, m, k // p) and ws.shape == (p, k // p, n)
    assert xs.data_ptr() == x.data_ptr() and ws.data_ptr() == w.data_ptr()  # views, no copies
    parts = torch.bmm(xs, ws)
    torch.testing.assert_close(parts.sum(0), x @ w.T)
    # slice i is the i-th contiguous K range
    i = p - 1
    lo, hi = i * (k // p), (i + 1) * (k // p)
    torch.testing.assert_close(parts[i], x[:, lo:hi] @ w[:, lo:hi].T)


def test_split_table():
    from xvllm.layers.linear import SPLIT_BUCKETS, SPLIT_TABLE, split_rule

    # measured shapes: the entry of the smallest bucket holding m rows
    assert [split_factor(m, 4096, 4096) for m in (1, 8, 16, 32, 64, 128, 256)] == [4, 4, 4, 1, 2, 2, 4]
    assert [split_factor(m, 4096, 12288) for m in (8, 16, 32, 64, 128, 256, 512)] == [1, 1, 4, 4, 8, 8, 1]
    assert [split_factor(m, 5120, 8192) for m in (1, 32, 33, 48, 200)] == [1, 1, 8, 8, 4]
    assert [split_factor(m, 5120, 25600) for m in (1, 32, 64, 96)] == [2, 2, 8, 4]
    for (n, k), row in SPLIT_TABLE.items():
        assert len(row) == len(SPLIT_BUCKETS)
        assert all(p in (1, 2, 4, 8) and k % (p * 64) == 0 for p in row)  # the norm sums at most 8 partials
    # other shapes: the rule
    assert [split_factor(m, 4096, 8192) for m in (16, 32, 128)] == [split_rule(m, 4096, 8192) for m in (16, 32, 128)]
    # prefill-sized M, wide outputs and short K never split
    assert split_factor(8192, 4096, 12288) == 1
    assert split_factor(64, 24576, 4096) == 1
    assert split_factor(64, 1024, 3072) == 1
    assert split_factor(128, 4096, 4352) == 1  # K not a multiple of 8 x 64
    assert split_factor(0, 4096, 4096) == 1
