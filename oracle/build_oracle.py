"""Compile the oracle's C restatement (oracle/csrc/*.c) into oracle/_build/liboracle.so.
TEST INFRASTRUCTURE ONLY."""
from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
OUT = HERE / "_build" / "liboracle.so"


def build() -> Path:
    OUT.parent.mkdir(parents=True, exist_ok=True)
    srcs = sorted(str(p) for p in (HERE / "csrc").glob("*.c"))
    cmd = ["gcc", "-O2", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", "-o", str(OUT), *srcs, "-lm"]
    subprocess.run(cmd, check=True)
    return OUT


if __name__ == "__main__":
    print(build())
