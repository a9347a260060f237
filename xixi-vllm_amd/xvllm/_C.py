"""ctypes binding of libxv_kernels.so (the C ABI in include/xv_kernels.h).

The library is loaded lazily on first use; a missing library raises
immediately -- there is no CPU or PyTorch fallback for any op.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

_LIB: C.CDLL | None = None

i32, i64, f32, vp, sz = C.c_int, C.c_int64, C.c_float, C.c_void_p, C.c_size_t

# name -> (restype, argtypes); must match include/xv_kernels.h exactly
SIGNATURES: dict[str, tuple] = {
    "xv_error_string": (C.c_char_p, [i32]),
    "xv_abi_version": (i32, []),
    "xv_store_kvcache": (i32, [vp, i64, i64, vp, i64, i64, vp, vp, i64, i64, i64, i32, vp, i64, i32, i32, vp]),
    "xv_store_kvcache_fp8": (
        i32, [vp, i64, i64, vp, i64, i64, vp, vp, i64, i64, i64, i32, vp, i64, i32, i32, f32, f32, vp]
    ),
    "xv_paged_decode_workspace_size": (sz, [i32, i32, i32, i32, i32, i32]),
    "xv_paged_decode_attention": (
        i32,
        [vp, i64, i64, vp, vp, i64, i64, i64, vp, i64, vp, vp, i64, vp, sz,
         i32, i32, i32, i32, i32, i32, f32, vp],
    ),
    "xv_paged_decode_attention_fp8": (
        i32,
        [vp, i64, i64, vp, vp, i64, i64, i64, vp, i64, vp, vp, i64, vp, sz,
         i32, i32, i32, i32, i32, i32, f32, f32, f32, vp],
    ),
    "xv_paged_decode_attention_noalloc": (
        i32,
        [vp, i64, i64, vp, vp, i64, i64, i64, vp, i64, vp, vp, i64,
         i32, i32, i32, i32, i32, i32, f32, vp],
    ),
    "xv_cascade_decode_workspace_size": (sz, [i32, i32, i32, i32, i32, i32]),
    "xv_cascade_decode_attention": (
        i32,
        [vp, i64, i64, vp, vp, i64, i64, i64, vp, i64, vp, vp, vp, vp, i32, i32, vp, i64, vp, sz,
         i32, i32, i32, i32, i32, i32, f32, vp],
    ),
    "xv_cascade_decode_attention_fp8": (
        i32,
        [vp, i64, i64, vp, vp, i64, i64, i64, vp, i64, vp, vp, vp, vp, i32, i32, vp, i64, vp, sz,
         i32, i32, i32, i32, i32, i32, f32, f32, f32, vp],
    ),
    "xv_prefill_attention": (
        i32,
        [vp, i64, i64, vp, vp, i64, i64, vp, vp, i64, i64, i64, vp, i64, vp, vp, vp, i64,
         i32, i32, i32, i32, i32, i32, f32, vp],
    ),
    "xv_rmsnorm": (i32, [vp, i64, i64, vp, vp, i64, i64, i32, f32, vp]),
    "xv_fused_add_rmsnorm": (i32, [vp, i64, vp, i64, vp, i64, i32, f32, vp]),
    "xv_fused_add_rmsnorm_parts": (i32, [vp, i64, i64, i32, vp, i64, vp, i64, vp, i64, i32, f32, vp]),
    "xv_rotary_embedding": (i32, [vp, i64, i64, vp, i64, i64, vp, vp, vp, vp, i64, i32, i32, i32, vp]),
    "xv_qk_norm_rope": (
        i32, [vp, i64, i64, vp, i64, i64, vp, vp, f32, vp, vp, vp, vp, i64, i32, i32, i32, vp]
    ),
    "xv_qk_norm_rope_store": (
        i32, [vp, i64, i64, vp, i64, i64, vp, i64, i64, vp, vp, f32, vp, vp, vp, vp, vp, i64, i64, i64, i32, vp,
              i64, i32, i32, i32, vp]
    ),
    "xv_qk_norm_rope_store_fp8": (
        i32, [vp, i64, i64, vp, i64, i64, vp, i64, i64, vp, vp, f32, vp, vp, vp, vp, vp, i64, i64, i64, i32, vp,
              i64, i32, i32, i32, f32, f32, vp]
    ),
    "xv_gather_kv_fp8": (
        i32, [vp, vp, i64, i64, i64, vp, i64, i32, vp, i32, i32, i32, i32, f32, f32, vp, vp, i64, vp]
    ),
    "xv_silu_and_mul": (i32, [vp, i64, vp, i64, i64, i32, vp]),
    "xv_dense_gemm": (i32, [vp, i64, vp, vp, i64, i64, i32, i32, i32, i32, i32, i32, i32, vp]),
    "xv_stream_copy": (i32, [vp, vp, i64, i32, vp]),
    "xv_sampler_workspace_size": (sz, [i32, i32]),
    "xv_sample": (i32, [vp, i64, i32, i32, vp, vp, vp, vp, vp, i32, vp, vp, sz, vp]),
}

XV_SAMPLE_ALL_GREEDY = 1
XV_SAMPLE_USE_TOP_K = 2
XV_SAMPLE_USE_TOP_P = 4
XV_SAMPLE_USE_MIN_P = 8
XV_SAMPLE_TOP_K_LE_64 = 16


def lib_path() -> Path:
    return Path(__file__).resolve().parent / "libxv_kernels.so"


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        p = lib_path()
        if not p.exists():
            raise ImportError(
                f"{p} is missing: build the HIP kernels first "
                "(python xixi-vllm_amd/build.py or __graft_entry__.build())"
            )
        L = C.CDLL(str(p))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def check(code: int, what: str) -> None:
    if code != 0:
        msg = lib().xv_error_string(code)
        raise RuntimeError(f"{what} failed: hip error {code} ({msg.decode() if msg else '?'})")
