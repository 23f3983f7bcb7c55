"""Build recipe for the gfx950 kernel library.

Compiles every ``csrc/*.hip`` with hipcc for gfx950 and produces, in-tree:

* ``qwenasr_amd/libqasr_hip.so`` -- shared library the Python and C++ hosts load;
* ``qwenasr_amd/libqasr_hip.a``  -- static archive for a host that links it
  statically (a Rust ``build.rs`` would add ``cargo:rustc-link-lib=static=qasr_hip``
  plus ``amdhip64``).

Run ``python -m qwenasr_amd.build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
SO = PKG / "libqasr_hip.so"
ARCHIVE = PKG / "libqasr_hip.a"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))

ARCH = "gfx950"

# -ffp-contract=off keeps every a*b+c a separate multiply and add unless the
# source calls fmaf, so elementwise epilogues round exactly as written.
# Packed-fp32 instruction selection is disabled (v_pk_* f32 forms).
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def _hipcc() -> str:
    p = ROCM / "bin" / "hipcc"
    if p.exists():
        return str(p)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found; the gfx950 library cannot be built")
    return found


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def build(verbose: bool = False) -> Path:
    """Compile all kernels and link the shared and static libraries."""
    hipcc = _hipcc()
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    objs = [BUILD / (s.stem + ".o") for s in srcs]

    def compile_one(pair):
        src, obj = pair
        cmd = [hipcc, *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        _run(cmd)

    workers = min(len(srcs), max(1, (os.cpu_count() or 4)))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        list(ex.map(compile_one, zip(srcs, objs)))

    tmp_so = SO.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp_so),
          *map(str, objs)])
    os.replace(tmp_so, SO)

    if ARCHIVE.exists():
        ARCHIVE.unlink()
    _run(["ar", "rcs", str(ARCHIVE), *map(str, objs)])
    build_cpp_tests(hipcc, verbose)
    return SO


ROOT = PKG.parent
CPP_TESTS = ROOT / "tests" / "cpp"
CPP_TEST_BIN = CPP_TESTS / "_build" / "test_kernels"


def build_cpp_tests(hipcc: str | None = None, verbose: bool = False) -> Path:
    """Builds the C++ host-mirror test against the static archive (so the
    binary carries its own copy of the kernels: the static-link path a Rust
    build.rs would use)."""
    hipcc = hipcc or _hipcc()
    CPP_TEST_BIN.parent.mkdir(exist_ok=True)
    obj = CPP_TEST_BIN.with_suffix(".o")
    tmp = CPP_TEST_BIN.with_suffix(".tmp")
    # compile and link separately: hipcc applies ``-x hip`` to every input
    # that follows a .cpp source, which would include the archive
    cmds = [[hipcc, f"--offload-arch={ARCH}", "-O2", "-std=c++17", "-Wall", "-I", str(ROOT / "include"),
             "-c", str(CPP_TESTS / "test_kernels.cpp"), "-o", str(obj)],
            [hipcc, f"--offload-arch={ARCH}", str(obj), str(ARCHIVE), "-o", str(tmp)]]
    for cmd in cmds:
        if verbose:
            print(" ".join(cmd), flush=True)
        _run(cmd)
    os.replace(tmp, CPP_TEST_BIN)
    return CPP_TEST_BIN


if __name__ == "__main__":
    out = build(verbose="-v" in sys.argv)
    print(out)
