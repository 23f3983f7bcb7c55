"""The C++ host mirror (include/qwen_asr/kernels.hpp) and its restatement of the
reference's kernel unit tests (tests/cpp/test_kernels.cpp), run on the GPU.
The binary links the static archive libqasr_hip.a."""
from __future__ import annotations

import subprocess

import pytest

from qwenasr_amd import build

pytestmark = pytest.mark.gpu


def test_cpp_kernel_tests_pass():
    assert build.CPP_TEST_BIN.exists(), "C++ test not built (run __graft_entry__.build())"
    r = subprocess.run([str(build.CPP_TEST_BIN)], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    print(r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = [l for l in r.stdout.splitlines() if l.startswith("test ")]
    assert len(lines) == 16 and all(l.endswith("ok") for l in lines)
