"""Build recipe for the CPU oracle (test infrastructure only).

Compiles ``oracle/qasr_oracle.c`` with gcc into ``oracle/_build/libqasr_oracle.so``.

Flags: ``-ffp-contract=off -fno-fast-math`` so a*b+c is never fused unless the
source calls fmaf (Rust never contracts), and ``-march=x86-64-v3`` so fmaf is
the hardware FMA (same result as libm's, faster) and the lane loops vectorise
without reassociation. ``build(native=True)`` makes the CPU-baseline copy
(``libqasr_oracle_native.so``, ``-march=native``, the reference's
``target-cpu=native``) on the host that times it.

The reference itself (Rust) cannot be built here: no cargo/rustc in the image,
so there is no ``oracle/_ref`` build; the restatement plus closed-form and
integer checks in tests/ pin the oracle instead.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "qasr_oracle.c"
OUT_DIR = HERE / "_build"
SO = OUT_DIR / "libqasr_oracle.so"
# the CPU-baseline copy, compiled for the host it runs on (-march=native); it is
# built where it is timed and never travels
NATIVE_SO = OUT_DIR / "libqasr_oracle_native.so"

CFLAGS = ["-O3", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
          "-Wall", "-Wextra", "-Wno-unused-parameter"]
PORTABLE = "-march=x86-64-v3"
NATIVE = "-march=native"


def build(native: bool = False) -> Path:
    """Compiles the oracle. ``native``: the timed CPU-baseline copy for this
    host (``-march=native``); otherwise the portable checker (x86-64-v3)."""
    cc = shutil.which("gcc") or shutil.which("cc")
    if not cc:
        raise RuntimeError("gcc not found; cannot build the CPU oracle")
    OUT_DIR.mkdir(exist_ok=True)
    out = NATIVE_SO if native else SO
    tmp = out.with_suffix(f".so.tmp{os.getpid()}")
    cmd = [cc, *CFLAGS, NATIVE if native else PORTABLE, str(SRC), "-o", str(tmp), "-lm", "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("oracle build failed: " + " ".join(cmd))
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build())
