"""xvllm: MI355X-native decode hot path behind the operator API of xixi-vllm's
``src/compute`` package (attention backend, RMSNorm, rotary, activation, KV
store and pool, sampler, decode-graph runner).

Every op runs a hand-written HIP kernel for gfx950 from ``libxv_kernels.so``
through its C ABI (``include/xv_kernels.h``); there is no fallback path.
"""
__all__ = ["ops_available"]


def ops_available() -> bool:
    from . import _C

    return _C.lib_path().exists()
