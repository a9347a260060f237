"""Pins the CPU oracle (the checker of every GPU parity test) against things
other than itself: the reference's own sampler distributions (golden fixture
written by tests/golden/make_sampler_golden.py), closed forms, invariants,
special cases and brute force on tiny inputs.

Parity status per oracle function:
  store_kvcache, slots_for_range      pinned (closed-form scatter / brute force)
  paged_decode_attention              pinned (dense softmax identities, GQA map, paging invariance)
  prefill_attention                   pinned (bottom-right causal == per-query decode)
  rmsnorm, fused_add_rmsnorm          pinned (unit RMS, scale invariance, exact residual sum)
  build_cos_sin_cache, rope_neox      pinned (closed form, rotation group law, norm preservation)
  silu_and_mul                        pinned (closed form)
  sampler (C)                         pinned (reference golden distributions + special cases + chi-square)
The reference's RNG stream (torch.multinomial / exponential_) is not
reproduced: draws are explicit uniforms (parity unpinned for the stream
itself, by design).
"""
import math
from pathlib import Path

import numpy as np
import pytest

import oracle.ops as O
import oracle.sampler as S
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits, round_bf16

GOLD = Path(__file__).resolve().parent / "golden" / "sampler_ref.npz"
rng = np.random.default_rng(0)


# ------------------------------------------------------------------ bf16
def test_bf16_round_trip_and_rne():
    x = np.array([1.0, 1.00390625, 1.005859375, -2.5, 3.0e38, 1e-40], np.float32)
    b = f32_to_bf16_bits(x)
    assert bf16_bits_to_f32(b)[0] == 1.0
    # 1 + 2^-8 is a tie between 1 and 1+2^-7: round to even -> 1.0
    assert bf16_bits_to_f32(b)[1] == 1.0
    assert bf16_bits_to_f32(b)[2] == np.float32(1.0078125)
    assert np.array_equal(round_bf16(round_bf16(x)), round_bf16(x))


# ------------------------------------------------------------------ KV store
def test_store_kvcache_scatter():
    n, h, d = 6, 2, 8
    key = rng.standard_normal((n, h, d)).astype(np.float32)
    val = rng.standard_normal((n, h, d)).astype(np.float32)
    kc = np.zeros((4, 4, h, d), np.float32)
    vc = np.zeros_like(kc)
    slots = np.array([3, -1, 0, 15, 7, -1])
    O.store_kvcache(key, val, kc, vc, slots)
    flat = kc.reshape(-1, h, d)
    for i, s in enumerate(slots):
        if s >= 0:
            assert np.array_equal(flat[s], key[i])
    assert np.count_nonzero(np.abs(flat).sum(axis=(1, 2))) == 4  # the two -1 slots wrote nothing


def test_slots_for_range():
    bt = [5, 2, 9]
    assert O.slots_for_range(bt, 0, 3, 4) == [20, 21, 22]
    assert O.slots_for_range(bt, 3, 9, 4) == [23, 8, 9, 10, 11, 36]
    assert O.slots_for_range(bt, 4, 4, 4) == []


# ------------------------------------------------------------------ attention
def _rand_paged(ctx, hkv, d, page=16, extra=3):
    need = sum((c + page - 1) // page for c in ctx)
    nb = need + extra
    perm = rng.permutation(nb)
    bt = -np.ones((len(ctx), max((c + page - 1) // page for c in ctx)), np.int64)
    o = 0
    for b, c in enumerate(ctx):
        n = (c + page - 1) // page
        bt[b, :n] = perm[o : o + n]
        o += n
    kc = rng.standard_normal((nb, page, hkv, d)).astype(np.float32)
    vc = rng.standard_normal((nb, page, hkv, d)).astype(np.float32)
    return kc, vc, bt


def test_decode_single_token_returns_v():
    kc, vc, bt = _rand_paged([1], 2, 8)
    q = rng.standard_normal((1, 4, 8)).astype(np.float32)
    out = O.paged_decode_attention(q, kc, vc, bt, np.array([1]))
    page, off = bt[0, 0], 0
    for h in range(4):
        np.testing.assert_allclose(out[0, h], vc[page, off, h // 2], rtol=1e-12)


def test_decode_equal_keys_average_v_and_gqa_map():
    ctx = [37]
    kc, vc, bt = _rand_paged(ctx, 2, 8)
    kc[:] = 0.5  # all keys equal -> uniform weights -> mean of V
    q = rng.standard_normal((1, 6, 8)).astype(np.float32)
    out = O.paged_decode_attention(q, kc, vc, bt, np.array(ctx))
    rows = O.gather_paged(vc, bt[0], 37)
    for h in range(6):
        np.testing.assert_allclose(out[0, h], rows[:, h // 3].astype(np.float64).mean(axis=0), rtol=1e-10)


def test_decode_matches_logsumexp_formula_and_paging_invariance():
    ctx = [50, 17]
    kc, vc, bt = _rand_paged(ctx, 2, 16)
    q = rng.standard_normal((2, 4, 16)).astype(np.float32)
    out = O.paged_decode_attention(q, kc, vc, bt, np.array(ctx))
    for b, c in enumerate(ctx):
        k = O.gather_paged(kc, bt[b], c).astype(np.float64)
        v = O.gather_paged(vc, bt[b], c).astype(np.float64)
        for h in range(4):
            s = k[:, h // 2] @ q[b, h].astype(np.float64) / 4.0
            lse = np.log(np.exp(s - s.max()).sum()) + s.max()
            np.testing.assert_allclose(out[b, h], np.exp(s - lse) @ v[:, h // 2], rtol=1e-10)
    # re-permuting the pool (same logical content) gives the same answer
    perm = rng.permutation(kc.shape[0])
    inv = np.argsort(perm)
    out2 = O.paged_decode_attention(q, kc[perm], vc[perm], np.where(bt >= 0, inv[np.maximum(bt, 0)], -1), np.array(ctx))
    np.testing.assert_allclose(out, out2, rtol=1e-12)


def test_padding_row_is_zero():
    kc, vc, bt = _rand_paged([5, 1], 1, 8)
    out = O.paged_decode_attention(np.ones((2, 1, 8), np.float32), kc, vc, bt, np.array([5, 0]))
    assert np.all(out[1] == 0)


def test_prefill_bottom_right_causal_equals_per_query_decode():
    """A chunk of q_len queries over k_len keys: query i equals a decode over
    the first k_len - q_len + i + 1 keys (bottom-right aligned causal)."""
    ctx_k, q_len = [40, 23], [7, 23]
    kc, vc, bt = _rand_paged(ctx_k, 2, 8)
    cu_q = np.concatenate([[0], np.cumsum(q_len)])
    cu_k = np.concatenate([[0], np.cumsum(ctx_k)])
    q = rng.standard_normal((cu_q[-1], 4, 8)).astype(np.float32)
    out = O.prefill_attention(q, cu_q, cu_k, k_cache=kc, v_cache=vc, block_tables=bt)
    for b in range(2):
        for i in range(q_len[b]):
            vis = ctx_k[b] - q_len[b] + i + 1
            want = O.paged_decode_attention(q[cu_q[b] + i][None], kc, vc, bt[b : b + 1], np.array([vis]))
            np.testing.assert_allclose(out[cu_q[b] + i], want[0], rtol=1e-10)
    # dense k/v path agrees with the paged path
    kd = np.concatenate([O.gather_paged(kc, bt[b], ctx_k[b]) for b in range(2)])
    vd = np.concatenate([O.gather_paged(vc, bt[b], ctx_k[b]) for b in range(2)])
    out_d = O.prefill_attention(q, cu_q, cu_k, k=kd, v=vd)
    np.testing.assert_allclose(out, out_d, rtol=1e-12)


# ------------------------------------------------------------------ norms
def test_rmsnorm_unit_rms_and_scale_invariance():
    x = rng.standard_normal((5, 64)).astype(np.float32)
    y = O.rmsnorm(x, np.ones(64, np.float32), 0.0)
    np.testing.assert_allclose(np.sqrt((y.astype(np.float64) ** 2).mean(-1)), 1.0, rtol=1e-2)
    np.testing.assert_allclose(O.rmsnorm(4 * x, np.ones(64, np.float32), 0.0), y, rtol=1e-6)
    w = rng.standard_normal(64).astype(np.float32)
    np.testing.assert_allclose(O.rmsnorm(x, w, 0.0), round_bf16(y * w), rtol=1e-2, atol=1e-2)


def test_fused_add_rmsnorm_residual_is_exact_sum():
    x = round_bf16(rng.standard_normal((3, 32)).astype(np.float32))
    r = round_bf16(rng.standard_normal((3, 32)).astype(np.float32))
    xo, ro = O.fused_add_rmsnorm(x, r, np.ones(32, np.float32), 1e-6)
    np.testing.assert_array_equal(ro, round_bf16(x + r))
    np.testing.assert_allclose(xo, O.rmsnorm(x + r, np.ones(32, np.float32), 1e-6))


# ------------------------------------------------------------------ RoPE
def test_cos_sin_cache_closed_form():
    cs = O.build_cos_sin_cache(128, 64, 1e6)
    i = 5
    ang = 17 * (1e6 ** (-2 * i / 128))
    assert abs(cs[17, i] - math.cos(ang)) < 1e-6 and abs(cs[17, 64 + i] - math.sin(ang)) < 1e-6
    assert np.all(cs[0, :64] == 1) and np.all(cs[0, 64:] == 0)


def test_rope_identity_norm_and_group_law():
    d = 128
    cs = O.build_cos_sin_cache(d, 512, 1e6)
    x = round_bf16(rng.standard_normal((4, 3, d)).astype(np.float32))
    np.testing.assert_array_equal(O.rope_neox(x, np.zeros(4, np.int64), cs), x)  # position 0
    y = O.rope_neox(x, np.array([1, 7, 100, 511]), cs).astype(np.float64)
    n0 = x[..., :64] ** 2 + x[..., 64:] ** 2
    n1 = y[..., :64] ** 2 + y[..., 64:] ** 2
    np.testing.assert_allclose(n1, n0, rtol=2e-2, atol=2e-2)
    # complex form: (x1 + i x2) * e^{i angle}
    c = x[..., :64].astype(np.float64) + 1j * x[..., 64:]
    ang = np.array([1, 7, 100, 511])[:, None, None] * (1e6 ** (-np.arange(0, d, 2) / d))[None, None, :]
    z = c * np.exp(1j * ang)
    np.testing.assert_allclose(y[..., :64], z.real, atol=2e-2)
    np.testing.assert_allclose(y[..., 64:], z.imag, atol=2e-2)


# ------------------------------------------------------------------ activation
def test_silu_and_mul_closed_form():
    x = np.array([[0.0, 1.0, -3.0, 2.0, 5.0, 7.0]], np.float32)
    y = O.silu_and_mul(x)
    want = np.array([0.0, 1 / (1 + math.exp(-1)) * 7, -3 / (1 + math.exp(3)) * 7][:1] + [0] * 0)
    np.testing.assert_allclose(y[0, 0], 0.0)
    np.testing.assert_allclose(y[0, 1], round_bf16(np.float32(1 / (1 + math.exp(-1.0)) * 5.0)), rtol=1e-6)
    np.testing.assert_allclose(y[0, 2], round_bf16(np.float32(-3 / (1 + math.exp(3.0)) * 7.0)), rtol=1e-6)


# ------------------------------------------------------------------ sampler
def test_exp2_accuracy():
    for x in np.linspace(-60, 0, 2001):
        got = S.exp2(np.float32(x))
        want = 2.0 ** float(np.float32(x))
        assert abs(got - want) <= 2e-7 * want + 1e-38


def test_sampler_matches_reference_distributions():
    """Kept set and renormalised probabilities equal those the reference's
    Sampler hands to its random draw (fixture from the reference itself)."""
    z = np.load(GOLD)
    for r in range(z["logits_bits"].shape[0]):
        p = S.probs(z["logits_bits"][r], z["temp"][r], z["top_p"][r], z["top_k"][r], z["min_p"][r], z["flags"][r])
        ref = z["probs"][r].astype(np.float64)
        vals = bf16_bits_to_f32(z["logits_bits"][r])
        # Equal logits at the cut-off may be kept in either order (torch.topk /
        # sort leave it open; this sampler keeps the lower ids): compare the kept
        # logit values with their probabilities, and exact membership elsewhere.
        mine = sorted(zip(vals[p > 0], p[p > 0]))
        theirs = sorted(zip(vals[ref > 0], ref[ref > 0]))
        assert len(mine) == len(theirs), f"row {r}: kept {len(mine)} vs reference {len(theirs)}"
        np.testing.assert_array_equal([m[0] for m in mine], [t[0] for t in theirs], err_msg=f"row {r}")
        np.testing.assert_allclose([m[1] for m in mine], [t[1] for t in theirs], rtol=1e-4, atol=1e-7, err_msg=f"row {r}")
        boundary = min(m[0] for m in mine)
        strict = vals > boundary
        assert np.array_equal((p > 0) & strict, (ref > 0) & strict), f"row {r}"


def test_sampler_special_cases():
    v = 1000
    bits = f32_to_bf16_bits(rng.standard_normal((1, v)).astype(np.float32) * 2)
    best = int(np.argmax(bf16_bits_to_f32(bits[0])))
    one = lambda **kw: int(S.sample(bits, [kw.get("t", 1.0)], [kw.get("p", 1.0)], [kw.get("k", v)],
                                    [kw.get("m", 0.0)], [kw.get("u", 0.5)], kw.get("f", 0))[0])
    assert one(t=0.0) == best                      # greedy
    assert one(f=1) == best                        # all-greedy flag
    for u in (0.0, 0.3, 0.999999):
        assert one(k=1, f=2, u=u) == best          # top-k 1 is greedy
        assert one(p=1e-9, f=4, u=u) == best       # top-p ~0 keeps only the best
        assert one(m=1.0, f=8, u=u) == best        # min-p 1 keeps only the max
    # ties: greedy picks the lowest index
    tb = np.full((1, 16), f32_to_bf16_bits(np.array([1.0], np.float32))[0], np.uint16)
    assert int(S.sample(tb, [0.0], None, None, None, [0.5], 0)[0]) == 0
    # inverse CDF in ascending id order: u -> 0 picks the smallest kept id
    kept = np.nonzero(S.probs(bits[0], 1.0, 0.5, v, 0.0, 4) > 0)[0]
    assert one(p=0.5, f=4, u=0.0) == kept.min()
    assert one(p=0.5, f=4, u=0.9999999) == kept.max()


def test_sampler_draw_frequencies_chi_square():
    """Stratified uniforms reproduce the kept-set probabilities."""
    v = 64
    bits = f32_to_bf16_bits(rng.standard_normal((1, v)).astype(np.float32))
    n = 20000
    u = (np.arange(n) + 0.5) / n
    ids = S.sample(np.repeat(bits, n, 0), np.full(n, 0.8), np.full(n, 0.9), np.full(n, 20), np.zeros(n), u, 2 | 4)
    p = S.probs(bits[0], 0.8, 0.9, 20, 0.0, 2 | 4)
    freq = np.bincount(ids, minlength=v) / n
    np.testing.assert_allclose(freq, p, atol=2.0 / n + 1e-12)


def test_sampler_greedy_is_torch_argmax():
    """The reference's greedy id is ``logits.argmax(-1)`` on the bf16 logits
    (src/compute/sampler.py:48,61,91): the lowest index on ties, -0 equal to
    +0, and a NaN counts as the maximum (the lowest NaN index wins)."""
    import torch

    v = 777
    x = rng.standard_normal((10, v)).astype(np.float32)
    x[0, 5] = x[0, 600] = np.nan                  # NaN among values: the first NaN
    x[1, :] = np.nan                              # all NaN: 0
    x[2, :] = 0.0
    x[2, 3] = -0.0                                # zeros of both signs: 0
    x[3, :] = -np.inf                             # all -inf: 0
    x[4, 100] = np.inf
    x[4, 700] = np.nan                            # NaN beats +inf
    x[5, 9] = x[5, 20] = 50.0                     # ties: the lower id
    x[6, v - 1] = np.nan                          # NaN in the last slot
    bits = f32_to_bf16_bits(x)
    want = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).argmax(-1).numpy()
    for flags, temps in ((1, None), (0, np.zeros(10, np.float32))):
        got = S.sample(bits, temps, None, None, None, np.full(10, 0.5, np.float32), flags)
        np.testing.assert_array_equal(got, want)


def test_threaded_decode_attention_equals_numpy_oracle():
    """The multi-threaded torch restatement used for the CPU baseline computes
    what the numpy oracle computes (fp32 against float64), padding rows included."""
    import torch

    import oracle.ops as O
    import oracle.threaded as TH

    rng = np.random.default_rng(5)
    ctx = [1, 17, 300, 0, 64]
    hq, hkv, d, bs = 32, 8, 128, 16
    need = [(c + bs - 1) // bs for c in ctx]
    nb = sum(need) + 3
    kc = rng.standard_normal((nb, bs, hkv, d)).astype(np.float32)
    vc = rng.standard_normal((nb, bs, hkv, d)).astype(np.float32)
    perm = rng.permutation(nb)
    bt = np.full((len(ctx), max(need)), -1, np.int64)
    o = 0
    for b, n in enumerate(need):
        bt[b, :n] = perm[o : o + n]
        o += n
    q = rng.standard_normal((len(ctx), hq, d)).astype(np.float32)
    want = O.paged_decode_attention(q, kc, vc, bt, np.array(ctx))
    got = TH.paged_decode_attention(torch.from_numpy(q), torch.from_numpy(kc), torch.from_numpy(vc),
                                    np.where(bt < 0, 0, bt), ctx, threads=4).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)
    assert not got[3].any()


def test_fp8_codec_equals_torch_float8_e4m3fn():
    """The fp8 format of the optional pool: the decode table and the
    quantizer (round to nearest even, NaN past the range) equal torch's
    float8_e4m3fn cast, over a dense sweep of float32 bit patterns and the
    special values."""
    import torch

    import oracle.ops as O

    codes = torch.arange(256, dtype=torch.uint8)
    want = codes.view(torch.float8_e4m3fn).float().numpy()
    got = O.fp8_e4m3fn_values()
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[~np.isnan(got)], want[~np.isnan(want)])
    i = np.arange(1 << 20, dtype=np.uint64)
    x = (i * 4096 + 77 * (i & 3)).astype(np.uint32).view(np.float32)
    x = np.concatenate([x, np.float32([0.0, -0.0, 448.0, 456.0, 463.99, 464.0, 480.0, -464.0, 2.0**-10,
                                       3 * 2.0**-10, 2.0**-9 * 1.5, 2.0**-9 * 2.5, 1e-30, -1e-30])])
    fin = np.isfinite(x)
    tq = torch.from_numpy(x[fin].copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    oq = O.quantize_fp8(x[fin], 1.0)
    assert np.array_equal(oq, tq), np.where(oq != tq)[0][:5]
    # a non-unit scale: one fp32 multiply before the rounding
    y = np.random.default_rng(0).standard_normal(4096).astype(np.float32) * 3
    inv = np.float32(1.0) / np.float32(0.37)
    tq = (torch.from_numpy(y) * torch.tensor(inv)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(O.quantize_fp8(y, inv), tq)
