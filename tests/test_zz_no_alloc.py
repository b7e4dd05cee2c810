"""dr_matmul_noalloc, the matmul entry point that allocates nothing (its split-K workspace is the library's own static
device array), against dr_matmul with a caller workspace, through the C ABI: two calls in a row, the second with a
smaller input, each bit for bit the same as dr_matmul's output; a launch that needs more workspace than the static
array holds is refused before anything is enqueued; the first call on a device, which clears the array's counters, is
refused under stream capture (checked in a fresh process, where that call is the first); calls captured in a HIP graph
after an eager one replay bit for bit as dr_matmul's."""

import ctypes
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from common.testing import same
from dense_reader import _lib, linear
from oracle import dense_oracle as O


def _fake_launch(m, k, n):
    L = _lib.Launch()  # pointers that are never read: the call is refused on the host
    L.x, L.y, L.m, L.k, L.ldx, L.ldy, L.nseg = 16, 16, m, k, k, n, 1
    s = L.seg[0]
    s.fmt, s.n, s.n_pad, s.codes, s.exps = 0, n, n, 16, 16
    return L


def test_noalloc_refuses_beyond_its_scratch():
    lib = _lib.lib()
    cap = lib.dr_scratch_bytes()
    L = _fake_launch(32, 14336, 32768)  # 1024 tiles x 2 K splits x 32 rows of partial sums: 8.4 MB
    need = lib.dr_workspace_bytes(ctypes.byref(L))
    assert need > cap, (need, cap)
    assert lib.dr_matmul_noalloc(ctypes.byref(L)) == _lib.DR_ERANGE
    assert lib.dr_matmul_noalloc(ctypes.byref(_lib.Launch())) == _lib.DR_EINVAL


def _noalloc(x, w, scale, **kw):
    L, y, keep = linear._launch(x, w, scale, **kw)
    L.stream = torch.cuda.current_stream(x.device).cuda_stream
    need = _lib.lib().dr_workspace_bytes(ctypes.byref(L))
    assert 0 < need <= _lib.lib().dr_scratch_bytes(), need  # (the case exercises the static workspace)
    _lib.check(_lib.lib().dr_matmul_noalloc(ctypes.byref(L)), "dr_matmul_noalloc")
    del keep
    return y


@pytest.mark.gpu
def test_noalloc_equals_matmul(device):
    g = torch.Generator().manual_seed(400)
    # (rows, K, N, format, residual + fp32 out): a split-K MFMA launch, then a smaller split-K GEMV launch
    for m, k, n, fmt, res in ((8, 14336, 4096, linear.bfloat8_b, True), (1, 9216, 320, linear.bfloat4_b, False)):
        wt = O.matrix(n, k, 401 + m)
        tw, _ = linear.native_weight(device, wt, fmt)
        x = O.x_input(m, k, 402 + m).to(torch.bfloat16).reshape(1, 1, m, k).to(device.torch)
        opts = {}
        if res:
            r = torch.randn(m, n, generator=g).to(torch.bfloat16).reshape(1, 1, m, n).to(device.torch)
            opts = {"residual": r, "out32": True}
        want = linear.matmul(x, tw, None, **opts)
        for rep in range(2):
            got = _noalloc(x, tw, None, **opts)
            torch.cuda.synchronize()
            same(f"noalloc rows {m} K {k} N {n} call {rep} against dr_matmul", got.cpu(), want.cpu())


_FIRST_UNDER_CAPTURE = r"""
import ctypes, sys
sys.path.insert(0, sys.argv[1]); sys.path.insert(0, sys.argv[2])
import torch
from dense_reader import _lib, linear
from oracle import dense_oracle as O
dev = linear.dev.open_device(0)
m, k, n = 1, 9216, 320
tw, _ = linear.native_weight(dev, O.matrix(n, k, 411), linear.bfloat8_b)
x = O.x_input(m, k, 412).to(torch.bfloat16).reshape(1, 1, m, k).cuda()
L, y, keep = linear._launch(x, tw, None)
need = _lib.lib().dr_workspace_bytes(ctypes.byref(L))
assert need > 0, need
s = torch.cuda.Stream()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g, stream=s):
    L.stream = torch.cuda.current_stream().cuda_stream
    first = _lib.lib().dr_matmul_noalloc(ctypes.byref(L))
    y.zero_()  # (the graph is not empty)
torch.cuda.synchronize()
L.stream = torch.cuda.current_stream().cuda_stream
eager = _lib.lib().dr_matmul_noalloc(ctypes.byref(L))
torch.cuda.synchronize()
print("first-under-capture", first, "eager", eager, flush=True)
"""


@pytest.mark.gpu
def test_noalloc_first_call_under_capture_refused(tmp_path):
    """In a fresh process (so the call is the device's first), dr_matmul_noalloc under stream capture is refused with
    DR_EINVAL and enqueues nothing (the capture ends with an empty graph); the next, eager call succeeds."""
    root = Path(__file__).resolve().parents[1]
    script = tmp_path / "first.py"
    script.write_text(_FIRST_UNDER_CAPTURE)
    r = subprocess.run([sys.executable, str(script), str(root / "tensix-kernels_amd"), str(root)], capture_output=True,
                       text=True, timeout=100)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    line = [s for s in r.stdout.splitlines() if s.startswith("first-under-capture")][-1].split()
    assert int(line[1]) == _lib.DR_EINVAL and int(line[3]) == _lib.DR_OK, line


@pytest.mark.gpu
def test_noalloc_in_a_graph(device):
    """After an eager call, dr_matmul_noalloc calls captured in a HIP graph (a split-K GEMV and a split-K MFMA launch)
    replay three times, with eager work between the replays, each bit for bit the same as dr_matmul's output."""
    cases = []
    for m, k, n in ((1, 9216, 320), (8, 14336, 1024)):
        tw, _ = linear.native_weight(device, O.matrix(n, k, 420 + m), linear.bfloat8_b)
        x = O.x_input(m, k, 421 + m).to(torch.bfloat16).reshape(1, 1, m, k).to(device.torch)
        want = linear.matmul(x, tw, None).cpu()
        _noalloc(x, tw, None)  # (the eager call: the device's scratch is set up outside any capture)
        cases.append((x, tw, want))
    torch.cuda.synchronize()
    outs = [torch.zeros(1, 1, x.shape[-2], tw.n, dtype=torch.bfloat16, device=device.torch) for x, tw, _ in cases]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for (x, tw, _), y in zip(cases, outs):
            L, _y, keep = linear._launch(x, tw, None, out=y)
            L.stream = torch.cuda.current_stream().cuda_stream
            _lib.check(_lib.lib().dr_matmul_noalloc(ctypes.byref(L)), "dr_matmul_noalloc")
    for rep in range(3):
        for y in outs:
            y.fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        for (x, tw, want), y in zip(cases, outs):
            same(f"noalloc in a graph, rows {x.shape[-2]} K {tw.k}: replay {rep} against dr_matmul", y.cpu(), want)
        linear.matmul(cases[0][0], cases[0][1], None)  # (eager work between the replays)
        torch.cuda.synchronize()
