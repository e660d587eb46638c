"""Compile the C oracle (oracle/jq_oracle.c) into oracle/_build/libjq_oracle.so with gcc.

Test infrastructure only. The reference ships no C/C++ source for this path (its kernels are
Metal and Python), so there is no reference build under oracle/_ref.
"""
from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "jq_oracle.c"
OUT = HERE / "_build" / "libjq_oracle.so"


def build() -> Path:
    OUT.parent.mkdir(exist_ok=True)
    if OUT.exists() and OUT.stat().st_mtime >= SRC.stat().st_mtime:
        return OUT
    cmd = ["gcc", "-O2", "-ffp-contract=off", "-fPIC", "-shared", str(SRC), "-o", str(OUT)]
    subprocess.run(cmd, check=True)
    return OUT


if __name__ == "__main__":
    print(build())
