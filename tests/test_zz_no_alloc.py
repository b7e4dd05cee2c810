"""dr_matmul_noalloc, the matmul entry point that allocates nothing (its split-K workspace is the library's own static
device array), against dr_matmul with a caller workspace, through the C ABI: two calls in a row, the second with a
smaller input, each bit for bit the same as dr_matmul's output; a launch that needs more workspace than the static
array holds is refused before anything is enqueued."""

import ctypes

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
