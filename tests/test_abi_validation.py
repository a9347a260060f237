"""Host-side argument checks of the C ABI, run without a GPU: every call below
is malformed (bad sizes, misaligned pointers, strides not in 16-byte units, a
short workspace), so the entry point returns hipErrorInvalidValue before any
HIP call; pointers are fake and never dereferenced.  Also the workspace-size
queries, which are pure host arithmetic."""
import ctypes as C

import pytest

INVALID = 1  # hipErrorInvalidValue
A = 0x10000  # a 16-byte aligned fake address
U = A + 8    # 8 bytes off


@pytest.fixture(scope="module")
def lib():
    from xvllm import _C

    if not _C.lib_path().exists():
        pytest.fail("libxv_kernels.so is not built (run __graft_entry__.build())")
    return _C.lib()


def _decode(lib, **kw):
    a = dict(q=A, qst=4096, qsh=128, kc=A, vc=A, ps=16384, ts=1024, hs=128, bt=A, bts=256, sl=A, out=A, ost=4096,
             ws=A, wsb=1 << 30, B=64, Hq=32, Hkv=8, D=128, BS=16, maxb=256, scale=0.088)
    a.update(kw)
    return lib.xv_paged_decode_attention(a["q"], a["qst"], a["qsh"], a["kc"], a["vc"], a["ps"], a["ts"], a["hs"],
                                         a["bt"], a["bts"], a["sl"], a["out"], a["ost"], a["ws"], a["wsb"], a["B"],
                                         a["Hq"], a["Hkv"], a["D"], a["BS"], a["maxb"], a["scale"], None)


def test_decode_rejects_bad_layouts(lib):
    for kw in (dict(D=64), dict(BS=24), dict(BS=0), dict(BS=8), dict(Hq=12), dict(Hq=128), dict(q=U), dict(kc=U), dict(qst=4100),
               dict(ts=1028), dict(out=A + 2), dict(ost=4097), dict(ws=None), dict(wsb=1024), dict(maxb=0)):
        assert _decode(lib, **kw) == INVALID, kw
    assert _decode(lib, B=0) == 0  # nothing to do


def _prefill(lib, **kw):
    a = dict(q=A, qst=4096, qsh=128, k=A, v=A, kvst=1024, kvsh=128, kc=None, vc=None, ps=0, ts=0, hs=0, bt=None,
             bts=0, cuq=A, cuk=A, out=A, ost=4096, B=4, maxq=512, Hq=32, Hkv=8, D=128, BS=16, scale=0.088)
    a.update(kw)
    return lib.xv_prefill_attention(a["q"], a["qst"], a["qsh"], a["k"], a["v"], a["kvst"], a["kvsh"], a["kc"],
                                    a["vc"], a["ps"], a["ts"], a["hs"], a["bt"], a["bts"], a["cuq"], a["cuk"],
                                    a["out"], a["ost"], a["B"], a["maxq"], a["Hq"], a["Hkv"], a["D"], a["BS"],
                                    a["scale"], None)


def test_prefill_rejects_bad_layouts(lib):
    for kw in (dict(D=64), dict(Hq=24), dict(k=None), dict(k=U), dict(kvst=1020), dict(q=U), dict(qsh=130),
               dict(out=A + 4), dict(ost=4098), dict(bt=A, kc=A, vc=A, BS=40), dict(bt=A, kc=None, vc=A),
               dict(bt=A, kc=U, vc=A, BS=16), dict(maxq=32 * 65536)):
        assert _prefill(lib, **kw) == INVALID, kw
    assert _prefill(lib, B=0) == 0 and _prefill(lib, maxq=0) == 0


def test_elementwise_entry_points_reject_bad_layouts(lib):
    s = None
    # store: head_dim not a multiple of 8, misaligned key, cache stride not in 16-byte units
    assert lib.xv_store_kvcache(A, 1024, 128, A, 1024, 128, A, A, 16384, 1024, 128, 16, A, 4, 8, 100, s) == INVALID
    assert lib.xv_store_kvcache(U, 1024, 128, A, 1024, 128, A, A, 16384, 1024, 128, 16, A, 4, 8, 128, s) == INVALID
    assert lib.xv_store_kvcache(A, 1024, 128, A, 1024, 128, A, A, 16384, 1020, 128, 16, A, 4, 8, 128, s) == INVALID
    # norms: hidden not a multiple of 8 / too long, misaligned rows or strides
    assert lib.xv_rmsnorm(A, 4096, 0, A, A, 4, 1, 4100, C.c_float(1e-6), s) == INVALID
    assert lib.xv_rmsnorm(A, 4096, 0, A, A, 4, 1, 32768, C.c_float(1e-6), s) == INVALID
    assert lib.xv_rmsnorm(U, 4096, 0, A, A, 4, 1, 4096, C.c_float(1e-6), s) == INVALID
    assert lib.xv_fused_add_rmsnorm(A, 4100, A, 4096, A, 4, 4096, C.c_float(1e-6), s) == INVALID
    assert lib.xv_fused_add_rmsnorm(A, 4096, U, 4096, A, 4, 4096, C.c_float(1e-6), s) == INVALID
    # split-K parts norm: 0 or 9 parts, a part stride not in 16-byte units, misaligned residual
    f = C.c_float(1e-6)
    assert lib.xv_fused_add_rmsnorm_parts(A, 16384, 4096, 0, A, 4096, A, 4096, A, 4, 4096, f, s) == INVALID
    assert lib.xv_fused_add_rmsnorm_parts(A, 16384, 4096, 9, A, 4096, A, 4096, A, 4, 4096, f, s) == INVALID
    assert lib.xv_fused_add_rmsnorm_parts(A, 16386, 4096, 2, A, 4096, A, 4096, A, 4, 4096, f, s) == INVALID
    assert lib.xv_fused_add_rmsnorm_parts(A, 16384, 4096, 2, A, 4096, U, 4096, A, 4, 4096, f, s) == INVALID
    # RoPE: head_dim other than 128, misaligned q
    assert lib.xv_rotary_embedding(A, 4096, 128, A, 1024, 128, A, A, A, A, 4, 32, 8, 64, s) == INVALID
    assert lib.xv_rotary_embedding(U, 4096, 128, A, 1024, 128, A, A, A, A, 4, 32, 8, 128, s) == INVALID
    assert lib.xv_qk_norm_rope(A, 4096, 130, A, 1024, 128, A, A, C.c_float(1e-6), A, A, A, A, 4, 32, 8, 128,
                               s) == INVALID
    # SiLU-and-mul: inter_size not a multiple of 8, misaligned output
    assert lib.xv_silu_and_mul(A, 24576, A, 12288, 4, 12290, s) == INVALID
    assert lib.xv_silu_and_mul(A, 24576, U, 12288, 4, 12288, s) == INVALID
    # sampler: bad sizes, sampled rows without temperatures
    assert lib.xv_sample(A, 100, 4, 200, A, None, None, None, None, 0, A, None, 0, s) == INVALID
    assert lib.xv_sample(A, 151936, 4, 151936, None, None, None, None, None, 0, A, None, 0, s) == INVALID
    assert lib.xv_sample(A, 151936, 4, 0, A, None, None, None, None, 0, A, None, 0, s) == INVALID


def test_workspace_sizes(lib):
    ws = lambda b, hq, hkv, maxb: lib.xv_paged_decode_workspace_size(b, hq, hkv, maxb, 16, 128)
    # the partial budget keeps every batch within ~32 MB of partials plus counters
    for b in (1, 8, 64, 256, 300, 1000):
        for maxb in (1, 128, 2048, 8192):
            assert 256 <= ws(b, 32, 8, maxb) <= (33 << 20), (b, maxb)
    assert ws(0, 32, 8, 128) == 256
    # one long sequence: up to 129 partials per head
    assert ws(1, 32, 8, 8192) >= 32 * 129 * 129 * 4
    sw = lambda b, v: lib.xv_sampler_workspace_size(b, v)
    assert sw(0, 151936) == 256 and sw(64, 151936) % 256 == 0
    assert sw(64, 151936) >= 64 * 8192 * 8  # the per-row candidate lists
    assert sw(256, 151936) >= sw(64, 151936)


def test_decode_workspace_never_shrinks_with_batch(lib):
    """Decode graphs are captured largest bucket first on one shared workspace:
    a smaller bucket must never need more (a regrown workspace would leave the
    earlier graphs replaying onto freed memory)."""
    for hq, hkv in ((32, 8), (16, 8), (64, 8), (8, 8)):
        for maxb in (1, 8, 128, 256, 296, 2048, 8192):
            prev = 0
            for b in range(1, 300):
                cur = lib.xv_paged_decode_workspace_size(b, hq, hkv, maxb, 16, 128)
                assert cur >= prev, (hq, hkv, maxb, b)
                prev = cur


def test_sampler_workspace_never_shrinks_with_batch(lib):
    for v in (1003, 32000, 151936):
        prev = 0
        for b in range(1, 300):
            cur = lib.xv_sampler_workspace_size(b, v)
            assert cur >= prev and cur >= b * 128, (v, b)
            prev = cur


def test_stream_copy_rejects_bad_arguments(lib):
    for args in ((A, A, 24, 0), (U, A, 32, 0), (A, U, 32, 1), (A, A, -16, 0), (A, A, 32, 2)):
        assert lib.xv_stream_copy(*args, None) == INVALID, args
    assert lib.xv_stream_copy(A, A, 0, 0, None) == 0  # nothing to do


def test_fp8_entry_points_reject_bad_arguments(lib):
    def dec(**kw):
        a = dict(q=A, kc=A, vc=A, ps=16384, ts=1024, hs=128, B=64, BS=16, ks=1.0, vs=1.0)
        a.update(kw)
        return lib.xv_paged_decode_attention_fp8(a["q"], 4096, 128, a["kc"], a["vc"], a["ps"], a["ts"], a["hs"], A, 256,
                                                 A, A, 4096, A, 1 << 30, a["B"], 32, 8, 128, a["BS"], 256, 0.088,
                                                 a["ks"], a["vs"], None)
    for kw in (dict(ts=1032), dict(hs=136), dict(kc=U), dict(ks=0.0), dict(vs=-1.0), dict(ks=float("inf")),
               dict(vs=float("nan")), dict(BS=8)):
        assert dec(**kw) == INVALID, kw
    assert dec(B=0) == 0

    def casc(**kw):
        a = dict(kc=A, ps=16384, ts=1024, hs=128, B=64, ks=1.0, vs=1.0, pre=A)
        a.update(kw)
        return lib.xv_cascade_decode_attention_fp8(A, 4096, 128, a["kc"], A, a["ps"], a["ts"], a["hs"], A, 256, A,
                                                   a["pre"], A, A, 2, 16, A, 4096, A, 1 << 30, a["B"], 32, 8, 128, 16,
                                                   256, 0.088, a["ks"], a["vs"], None)
    for kw in (dict(ts=1032), dict(hs=136), dict(kc=U), dict(ks=0.0), dict(vs=float("nan")), dict(pre=0),
               dict(B=257)):
        assert casc(**kw) == INVALID, kw
    assert casc(B=0) == 0


def test_cascade_rejects_prefixes_beyond_its_chunk_table(lib):
    """The prefix pass holds at most 32 chunks of 2048 pages (1M tokens of
    shared prefix): longer prefixes are rejected before any launch."""
    for fn, extra in ((lib.xv_cascade_decode_attention, ()), (lib.xv_cascade_decode_attention_fp8, (1.0, 1.0))):
        blocks = 65536 // 16 + 1  # 256-token blocks: one block over 1M tokens
        rc = fn(A, 4096, 128, A, A, 256 * 1024, 1024, 128, A, blocks, A, A, A, A, 1, blocks,
                A, 4096, A, 1 << 45, 1, 32, 8, 128, 256, blocks, 0.088, *extra, None)
        assert rc == INVALID

    def store(**kw):
        a = dict(k=A, kc=A, ps=16384, ts=1024, hs=128, n=8, hkv=8, d=128, ks=1.0, vs=1.0)
        a.update(kw)
        return lib.xv_store_kvcache_fp8(a["k"], 1024, 128, A, 1024, 128, a["kc"], A, a["ps"], a["ts"], a["hs"], 16, A,
                                        a["n"], a["hkv"], a["d"], a["ks"], a["vs"], None)
    for kw in (dict(k=U), dict(kc=A + 4), dict(ts=1028), dict(ks=0.0), dict(vs=float("inf")), dict(hkv=2, d=128),
               dict(d=12)):
        assert store(**kw) == INVALID, kw
    assert store(n=0) == 0


def test_fp8_model_entry_points_reject_bad_arguments(lib):
    def rope(**kw):
        a = dict(D=128, ks=1.0, vs=1.0, T=4)
        a.update(kw)
        return lib.xv_qk_norm_rope_store_fp8(A, 6144, 128, A, 6144, 128, A, 6144, 128, A, A, 1e-6, A, A, A, A, A,
                                             16384, 1024, 128, 16, A, a["T"], 32, 8, a["D"], a["ks"], a["vs"], None)
    for kw in (dict(D=64), dict(ks=0.0), dict(vs=float("inf"))):
        assert rope(**kw) == INVALID, kw
    assert rope(T=0) == 0

    def gather(**kw):
        a = dict(kc=A, ts=1024, out=A, ost=1024, B=4, D=128, ks=1.0)
        a.update(kw)
        return lib.xv_gather_kv_fp8(a["kc"], A, 16384, a["ts"], 128, A, 64, 16, A, a["B"], 512, 8, a["D"], a["ks"],
                                    1.0, a["out"], A, a["ost"], None)
    for kw in (dict(kc=A + 4), dict(ts=1028), dict(out=U), dict(ost=512), dict(D=64), dict(ks=-1.0)):
        assert gather(**kw) == INVALID, kw
    assert gather(B=0) == 0


def _gemm(lib, **kw):
    a = dict(x=A, xs=4096, w=A, out=A, os=6144, ps=0, m=64, n=6144, k=4096, mode=0, ct=2, wv=4, p=1)
    a.update(kw)
    return lib.xv_dense_gemm(a["x"], a["xs"], a["w"], a["out"], a["os"], a["ps"], a["m"], a["n"], a["k"], a["mode"],
                             a["ct"], a["wv"], a["p"], None)


def test_dense_gemm_rejects_bad_arguments(lib):
    for kw in (dict(m=65), dict(m=-1), dict(n=6144 + 16), dict(k=4096 + 64), dict(ct=3), dict(wv=2), dict(p=0),
               dict(p=2), dict(mode=3), dict(mode=2, ct=1), dict(x=U), dict(w=U), dict(xs=4100), dict(xs=2048),
               dict(os=6143), dict(os=1024), dict(out=A + 4), dict(mode=1, p=4, ps=64 * 6144 - 4),
               dict(mode=1, p=4, out=A + 8, ps=64 * 6144), dict(mode=1, p=8, k=4096 + 256, ps=64 * 6144)):
        assert _gemm(lib, **kw) == INVALID, kw
    assert _gemm(lib, m=0) == 0  # nothing to do


def test_pack_weight_tile_order():
    """pack_weight against its definition, element by element with explicit
    index arithmetic: tile (nb, sg), lane l = 16 g + r, element e."""
    import numpy as np
    import torch

    from xvllm.layers.linear import pack_weight

    n, k = 48, 192
    w = torch.zeros((n, k), dtype=torch.bfloat16)
    ids = np.arange(n * k).reshape(n, k)
    wi = torch.from_numpy(ids.astype(np.int32))
    packed = pack_weight(wi.view(n, k)).data.numpy()
    assert packed.shape == (n * k,)
    for nb in range(n // 16):
        for sg in range(k // 64):
            base = (nb * (k // 64) + sg) * 1024
            for l in range(64):
                r, g = l % 16, l // 16
                for e in range(8):
                    assert packed[base + 8 * l + e] == ids[16 * nb + r, 64 * sg + 8 * g + e]
                    assert packed[base + 512 + 8 * l + e] == ids[16 * nb + r, 64 * sg + 32 + 8 * g + e]
    assert sorted(packed.tolist()) == list(range(n * k))  # a permutation
    with pytest.raises(ValueError):
        pack_weight(w[:, :100])
