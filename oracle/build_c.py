"""Build oracle/_c/liboracle_c.so (the C restatement of the int4 dequant, OpenMP) with gcc.
Test infrastructure only: tests, smoke() and bench.py's cpu_baseline load it."""

from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
OUT = HERE / "_c" / "liboracle_c.so"


def build(verbose: bool = False) -> Path:
    OUT.parent.mkdir(exist_ok=True)
    cmd = ["gcc", "-O3", "-fPIC", "-shared", "-fopenmp", "-std=c11", str(HERE / "dequant.c"), "-o", str(OUT)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"gcc failed for the C oracle:\n{res.stderr}")
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    build(verbose=True)
