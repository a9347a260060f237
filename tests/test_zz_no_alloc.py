"""The allocation-free decode entry point, xv_paged_decode_attention_noalloc,
called through the C ABI: its workspace is the library's static device array
instead of a caller buffer.  On the GPU its outputs equal those of
xv_paged_decode_attention (same kernels, bit-exact) on two calls in a row,
the second with a smaller batch, so the second call runs on the contents the
first left in the shared array; on the CPU, a call whose workspace would
exceed the array is rejected before the device is touched."""
import ctypes as C
import math

import pytest
import torch

from helpers import gen, make_paged, randn_bf16

INVALID = 1  # hipErrorInvalidValue


def _lib():
    from xvllm import _C

    if not _C.lib_path().exists():
        pytest.fail("libxv_kernels.so is not built (run __graft_entry__.build())")
    return _C.lib()


def test_noalloc_rejects_workspace_beyond_its_array():
    L = _lib()
    A = 0x10000
    # B 256 x Hq 128 needs more than the 48 MiB array (at least 3 partials per head)
    need = L.xv_paged_decode_workspace_size(256, 128, 16, 4096, 16, 128)
    assert need > 48 << 20
    rc = L.xv_paged_decode_attention_noalloc(A, 16384, 128, A, A, 262144, 2048, 128, A, 4096, A, A, 16384,
                                             256, 128, 16, 128, 16, 4096, 0.088, None)
    assert rc == INVALID
    # argument errors are reported the same way as by the workspace entry point
    assert L.xv_paged_decode_attention_noalloc(A, 4096, 128, A, A, 16384, 1024, 128, A, 256, A, A, 4096,
                                               64, 32, 8, 64, 16, 256, 0.088, None) == INVALID
    assert L.xv_paged_decode_attention_noalloc(A, 4096, 128, A, A, 16384, 1024, 128, A, 256, A, A, 4096,
                                               0, 32, 8, 128, 16, 256, 0.088, None) == 0


def _call(L, fn, q, kc, vc, bt, sl, out, hq, hkv, ws=None):
    stream = torch.cuda.current_stream().cuda_stream
    args = [q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1),
            kc.stride(2), bt.data_ptr(), bt.stride(0), sl.data_ptr(), out.data_ptr(), out.stride(0)]
    if ws is not None:
        args += [ws.data_ptr(), ws.numel()]
    args += [q.shape[0], hq, hkv, 128, kc.shape[1], bt.shape[1], 1.0 / math.sqrt(128), stream]
    return getattr(L, fn)(*args)


@pytest.mark.gpu
def test_noalloc_equals_workspace_entry_point(dev):
    L = _lib()
    hq, hkv = 32, 8
    for call, (bsz, lo, hi) in enumerate(((64, 512, 4097), (8, 1, 3000))):
        print(f"noalloc call {call}: B {bsz}", flush=True)
        g = gen(900 + call)
        ctx = torch.randint(lo, hi, (bsz,), generator=g).tolist()
        ctx[bsz // 2] = 0  # a padding row
        need = sum((c + 15) // 16 for c in ctx)
        kc, vc, bt, sl = make_paged(ctx, math.ceil(need * 1.25) + 4, hkv, 128, g, fill_nan=False)
        q = randn_bf16((bsz, hq, 128), g).to(dev)
        kc, vc, bt, sl = kc.to(dev), vc.to(dev), bt.to(dev), sl.to(dev)
        ws_bytes = L.xv_paged_decode_workspace_size(bsz, hq, hkv, bt.shape[1], 16, 128)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        want = torch.empty((bsz, hq * 128), dtype=torch.bfloat16, device=dev)
        got = torch.full_like(want, float("nan"))
        assert _call(L, "xv_paged_decode_attention", q, kc, vc, bt, sl, want, hq, hkv, ws=ws) == 0
        assert _call(L, "xv_paged_decode_attention_noalloc", q, kc, vc, bt, sl, got, hq, hkv) == 0
        torch.cuda.synchronize()
        assert torch.isfinite(want.float()).all()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"call {call}"
