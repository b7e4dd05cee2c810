"""The int4 group-scale matmul (int4/w4a16.py) on the GPU against the CPU oracle, after XylolabsInc/tensix-kernels
int4/tests/test_int4.py, test for test.

Random codes in -7..7 and bf16 group scales (G = 32); x with a few outlier channels. Reference: x rounded to bf16 times
q * s in float64 (the device's weight exactly). Bars, relative Frobenius error and PCC above 0.9999:
- the matmul: below 1 % (the reference's bar for both of its fidelities; there is one arithmetic here);
- the dequantized bfloat8_b weight: below 2 % (its block-float rounding);
- the packed codes and scales: byte for byte the oracle's layout;
- repeated calls and the Tensix work-split options: bit for bit.
"""

import numpy as np
import pytest
import torch

from common import device as cdev
from common.testing import check, same
from dense_reader import linear
from int4 import w4a16
from oracle import dense_oracle as O

pytestmark = pytest.mark.gpu


def make_case(n, k, seed):
    g = torch.Generator().manual_seed(seed)
    codes = torch.randint(-7, 8, (n, k), generator=g).to(torch.int8)
    scales = (torch.rand(n, k // 32, generator=g) * 0.01 + 0.001).to(torch.bfloat16)
    return codes, scales


def make_x(device, k, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(1, k, generator=g)
    x[:, torch.randperm(k, generator=g)[:8]] *= 20  # a few outlier channels
    x = x.to(torch.bfloat16)
    return x, x.reshape(1, 1, 1, k).to(device.torch)


def host(y, n):
    return y.float().cpu().reshape(-1, y.shape[-1])[:1, :n]


def test_layout(device):
    n, k = 200, 320
    codes, scales = make_case(n, k, 1)
    wq = w4a16.int4_weight(device, codes)
    same("int4 codes: the oracle's layout", wq["t"].cpu(),
         torch.from_numpy(O.int4_layout(codes.numpy(), wq["n_pad"], wq["k_pad"])))
    ts = w4a16.group_scales(device, scales)
    want = O.int4_scales_layout(scales.view(torch.int16).numpy().view(np.uint16), ts.shape[0] * 16, wq["k_pad"])
    same("int4 group scales: the oracle's order", ts.reshape(-1).view(torch.int16).cpu(),
         torch.from_numpy(want.view(np.int16)))


@pytest.mark.parametrize("fid", ["hifi4", "hifi2"])
def test_matmul(device, fid):
    for k, n in ((1024, 1152), (3072, 1024), (4096, 4096)):
        codes, scales = make_case(n, k, k + n)
        wq = w4a16.int4_weight(device, codes)
        ts = w4a16.group_scales(device, scales)
        x, tx = make_x(device, k, n)
        ref = O.int4_ref(x, codes, scales)
        y = host(w4a16.w4a16_linear(tx, wq, ts, fidelity=fid), n)
        check(f"int4 {fid} K {k} N {n}", y, ref)
        same(f"int4 {fid} K {k} N {n}: the work-split options change nothing",
             host(w4a16.w4a16_linear(tx, wq, ts, split=False, cores_per_bank=2, fidelity=fid), n), y)


@pytest.mark.parametrize("k", [2048, 4096])
def test_rows(device, k):
    """Several rows through the C ABI (two a pass, the last pass partial): each row against the oracle and against the
    one-token call on that row, bit for bit (the rows of a pass are summed in the same order as a lone row); at K = 2048
    the launches take 256-k chunks, at 4096 512-k chunks."""
    n = 1056
    codes, scales = make_case(n, k, 21)
    wq = w4a16.int4_weight(device, codes)
    ts = w4a16.group_scales(device, scales)
    g = torch.Generator().manual_seed(22)
    x = torch.randn(5, k, generator=g).to(torch.bfloat16)
    tx = x.to(device.torch)
    for m in (2, 3, 5):
        y = w4a16.rows_matmul(tx[:m], wq, ts).float().cpu()
        check(f"int4 {m} rows K {k} N {n}", y, O.int4_ref(x[:m], codes, scales))
        for r in range(m):
            one = host(w4a16.w4a16_linear(tx[r].reshape(1, 1, 1, k), wq, ts), n)
            same(f"int4 {m} rows: row {r} against the one-token call", y[r : r + 1], one)


def test_fewer_banks(device):
    k, n = 1024, 1024
    banks = cdev.dram_banks(device)
    fewer = max(1, banks // 2)
    codes, scales = make_case(n, k, 7)
    wq = w4a16.int4_weight(device, codes, max_banks=fewer)
    assert wq["banks"] == fewer
    ts = w4a16.group_scales(device, scales)
    x, tx = make_x(device, k, 8)
    check(f"int4 weight over {fewer} of {banks} banks", host(w4a16.w4a16_linear(tx, wq, ts), n),
          O.int4_ref(x, codes, scales))


def test_dequantize(device):
    k, n = 2048, 1152
    codes, scales = make_case(n, k, 9)
    wq = w4a16.int4_weight(device, codes)
    ts = w4a16.group_scales(device, scales)
    wd = w4a16.dequantize(wq, ts)
    got = linear.held(wd, n).cpu().float()
    w = O.int4_dequantized(codes, scales).T.float()
    check("dequantized bfloat8_b weight against q * s", got, w, rel=0.02)
    same("dequantized bfloat8_b weight: the oracle's bfloat8_b rounding of q * s", got,
         torch.from_numpy(O.held(w, "bfp8")).float())
    again = w4a16.dequantize(wq, ts, out=wd)
    same("dequantize into a given output: the same values", linear.held(again, n).cpu(), got)
