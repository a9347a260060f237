"""The C-ABI library loads and exports every entry point include/xv_kernels.h
declares, with the argument counts the Python binding uses (no GPU calls)."""
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "xv_kernels.h"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    decls = {}
    for m in re.finditer(r"\b(xv_\w+)\s*\(([^)]*)\)\s*;", text):
        args = [a for a in m.group(2).split(",") if a.strip() and a.strip() != "void"]
        decls[m.group(1)] = len(args)
    return decls


def test_header_declares_entry_points():
    d = _declared()
    for name in ("xv_store_kvcache", "xv_paged_decode_attention", "xv_prefill_attention", "xv_rmsnorm",
                 "xv_fused_add_rmsnorm", "xv_rotary_embedding", "xv_qk_norm_rope", "xv_silu_and_mul", "xv_sample"):
        assert name in d


def test_library_exports_every_declared_symbol():
    from xvllm import _C

    if not _C.lib_path().exists():
        pytest.fail("libxv_kernels.so is not built (run __graft_entry__.build())")
    lib = _C.lib()
    for name, nargs in _declared().items():
        assert hasattr(lib, name), f"{name} not exported"
        assert name in _C.SIGNATURES, f"{name} has no Python binding"
        assert len(_C.SIGNATURES[name][1]) == nargs, f"{name}: binding has {len(_C.SIGNATURES[name][1])} args, header {nargs}"
    assert lib.xv_abi_version() >= 1
