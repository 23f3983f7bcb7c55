"""The no-allocation lm_head argmax entry point against the workspace one.

qasr_lm_head_int8_argmax_noalloc_f32 keeps its per-workgroup candidates in a
device array the library holds, instead of a caller workspace. Called through
the C ABI twice in a row -- the second call with a smaller vocabulary and
hidden size, so it runs on array contents the first call left -- it must give
the same token index and logits, bit for bit, as
qasr_lm_head_int8_argmax_f32 with a workspace on the same inputs. Plus the
error paths: a vocabulary above the stated maximum, an unsupported hidden
size.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _ptr(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _run(dev, r, vocab, hidden, nan_rows=()):
    from qwenasr_amd import _lib

    so = _lib.lib()
    w = torch.from_numpy(r.integers(-127, 128, (vocab, hidden), dtype=np.int8)).to(dev)
    s = torch.from_numpy((1e-3 + 1e-3 * r.random(vocab)).astype(np.float32)).to(dev)
    x = torch.from_numpy(r.standard_normal(hidden).astype(np.float32)).to(dev)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ws = torch.empty(so.qasr_lm_head_argmax_workspace_bytes(vocab) // 8 + 1, dtype=torch.float64, device=dev)
    idx_a = torch.full((1,), -7, dtype=torch.int32, device=dev)
    idx_b = torch.full((1,), -7, dtype=torch.int32, device=dev)
    lg_a = torch.full((vocab,), float("nan"), device=dev)
    lg_b = torch.full((vocab,), float("nan"), device=dev)
    print(f"[no_alloc] vocab {vocab} hidden {hidden}: workspace entry", flush=True)
    _lib.call("qasr_lm_head_int8_argmax_f32", _ptr(idx_a), _ptr(lg_a), _ptr(x), _ptr(w), _ptr(s), 1, hidden,
              vocab, _ptr(ws), ws.numel() * 8, st)
    print(f"[no_alloc] vocab {vocab} hidden {hidden}: no-alloc entry", flush=True)
    _lib.call("qasr_lm_head_int8_argmax_noalloc_f32", _ptr(idx_b), _ptr(lg_b), _ptr(x), _ptr(w), _ptr(s), 1,
              hidden, vocab, st)
    torch.cuda.synchronize()
    assert torch.equal(lg_a, lg_b)
    assert int(idx_a.item()) == int(idx_b.item())
    assert 0 <= int(idx_b.item()) < vocab
    return int(idx_b.item())


def test_noalloc_lm_head_equals_workspace_entry_twice(dev):
    r = np.random.default_rng(71)
    first = _run(dev, r, 151936, 2048)   # the 1.7B lm_head: 37984 candidates
    second = _run(dev, r, 5003, 1024)    # smaller: the array still holds the first call's candidates
    assert first >= 0 and second >= 0


def test_noalloc_lm_head_rejects_what_it_cannot_hold(dev):
    from qwenasr_amd import _lib

    so = _lib.lib()
    idx = torch.zeros(1, dtype=torch.int32, device=dev)
    x = torch.zeros(1024, device=dev)
    w = torch.zeros(16, dtype=torch.int8, device=dev)  # never read: rejected before any launch
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    big = 262144 + 4
    rc = so.qasr_lm_head_int8_argmax_noalloc_f32(_ptr(idx), _ptr(x), _ptr(x), _ptr(w), _ptr(x), 1, 1024, big, st)
    assert rc == _lib.QASR_ERR_INVALID_ARG, rc
    assert b"262144" in so.qasr_last_error()
    rc = so.qasr_lm_head_int8_argmax_noalloc_f32(_ptr(idx), _ptr(x), _ptr(x), _ptr(w), _ptr(x), 1, 1000, 16, st)
    assert rc == _lib.QASR_ERR_UNSUPPORTED, rc
    torch.cuda.synchronize()


_CAPTURE_SCRIPT = r'''
import ctypes, sys
import numpy as np
import torch
sys.path.insert(0, sys.argv[1])
from qwenasr_amd import _lib

P = lambda t: ctypes.c_void_p(t.data_ptr())
dev = torch.device("cuda:0")
so = _lib.lib()
vocab, hidden = 65536, 1024
r = np.random.default_rng(5)
w = torch.from_numpy(r.integers(-127, 128, (vocab, hidden), dtype=np.int8)).to(dev)
s = torch.from_numpy((1e-3 + 1e-3 * r.random(vocab)).astype(np.float32)).to(dev)
x = torch.from_numpy(r.standard_normal(hidden).astype(np.float32)).to(dev)
ws = torch.empty(so.qasr_lm_head_argmax_workspace_bytes(vocab) // 8 + 1, dtype=torch.float64, device=dev)
idx_g = torch.full((1,), -7, dtype=torch.int32, device=dev)
lg_g = torch.full((vocab,), float("nan"), device=dev)
idx_e = torch.full((1,), -7, dtype=torch.int32, device=dev)
lg_e = torch.full((vocab,), float("nan"), device=dev)
torch.cuda.synchronize()

def workspace_form():
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.call("qasr_lm_head_int8_argmax_f32", P(idx_e), P(lg_e), P(x), P(w), P(s), 1, hidden, vocab,
              P(ws), ws.numel() * 8, st)

print("[no_alloc capture] first no-alloc call of the process, inside graph capture", flush=True)
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.call("qasr_lm_head_int8_argmax_noalloc_f32", P(idx_g), P(lg_g), P(x), P(w), P(s), 1, hidden,
              vocab, st)
torch.cuda.synchronize()
for replay in range(3):
    if replay:
        x.copy_(torch.from_numpy(r.standard_normal(hidden).astype(np.float32)).to(dev))  # eager work
        idx_g.fill_(-7)
        lg_g.fill_(float("nan"))
    torch.cuda.synchronize()
    print(f"[no_alloc capture] replay {replay}", flush=True)
    g.replay()
    torch.cuda.synchronize()
    workspace_form()
    torch.cuda.synchronize()
    assert torch.equal(lg_g, lg_e), f"replay {replay}: logits differ"
    assert int(idx_g.item()) == int(idx_e.item()), f"replay {replay}: {idx_g.item()} != {idx_e.item()}"
    assert 0 <= int(idx_g.item()) < vocab
print("[no_alloc capture] ok", flush=True)
'''


def test_noalloc_first_call_under_graph_capture_in_a_fresh_process(dev):
    """The scratch address lookup happens on a device's first call. Made for the
    first time inside a graph capture, in a process that has not called the
    entry point before, the captured kernels must still equal the workspace
    form on every replay (three replays, new inputs written eagerly between
    them)."""
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, "-c", _CAPTURE_SCRIPT, str(root)], capture_output=True, text=True,
                       timeout=300)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0, r.stderr[-2000:]
    assert "[no_alloc capture] ok" in r.stdout
