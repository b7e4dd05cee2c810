"""A seeded sweep over the MoE layer's shapes on the GPU (moe8.gate_up / down for one row, gate_up_rows / down_rows
for several), every case against the oracle's float64 layer (moe_oracle.layer): experts E, slots k, H and I on and off
the 256-K padding, each activation, with and without the gate/up bias, bfloat4_b packs and kblock packs, one or two
loaders. Bars as the MoE tests' (moe/tests/test_moe.py): relative Frobenius error below 1 % and PCC above 0.9999 for
h and y; rows past R zero; each case called twice, bit for bit.
"""

import numpy as np
import pytest
import torch

from common.testing import check, same
from moe import moe8
from oracle import dense_oracle as O
from oracle import moe_oracle as MO

pytestmark = pytest.mark.gpu

BF = torch.bfloat16
CASES = 30


def _case(i):
    r = np.random.default_rng(7000 + i)
    E = int(r.choice([2, 4, 8, 16, 32]))
    c = {"i": i, "E": E, "k": int(r.integers(1, min(E, 8) + 1)), "H": int(r.choice([256, 480, 1024, 1056, 2880])),
         "I": int(r.choice([64, 96, 256, 512, 1440])), "act": str(r.choice(["silu", "gelu_tanh", "swiglu_oai"])),
         "bias": bool(r.integers(2)), "kblock": bool(r.integers(2)), "loaders": int(r.integers(1, 3)),
         "rows": int(r.choice([0, 2, 5, 17]))}
    while c["E"] * c["H"] * c["I"] > 16 * 1024 * 1024:  # (the oracle's float64 experts stay small)
        c["I"] = {1440: 512, 512: 256, 256: 96}.get(c["I"], 64)
        if c["I"] == 64:
            c["H"] = min(c["H"], 1024)
    return c


def _grid(w, kblock):
    """w's values on the BFP4_b grid (kblock: shared exponents along K), bf16 [K, N]."""
    return torch.from_numpy(MO.held_kblock(w.numpy()) if kblock else O.held(w, "bfp4")).float().to(BF)


def _host(t, cols):
    return t.float().cpu().reshape(-1, t.shape[-1])[:, :cols]


@pytest.mark.parametrize("i", range(CASES))
def test_moe_sweep(device, i):
    c = _case(i)
    print(f"case {c}", flush=True)
    E, k, H, I, act = c["E"], c["k"], c["H"], c["I"], c["act"]
    g = torch.Generator().manual_seed(8000 + i)
    scale = 0.1 if act == "swiglu_oai" else 0.02
    gu = torch.stack([_grid(torch.randn(H, 2 * I, generator=g) * scale, c["kblock"]) for _ in range(E)])
    dn = torch.stack([_grid(torch.randn(I, H, generator=g) * 0.02, c["kblock"]) for _ in range(E)])
    gb = torch.randn(E, 2 * I, generator=g) * 0.5 if c["bias"] else None
    P = moe8.pack(device, gu, dn, kblock=c["kblock"], gu_bias=gb)
    # (a bias or column groups need two loaders, as the reference's gate_up asserts)
    ld = c["loaders"] if gb is None and moe8.gu_groups(I // 32, P["banks"])[0] == 1 else 2
    name = f"moe sweep {i} E {E} k {k} H {H} I {I} {act} bias {c['bias']} kblock {c['kblock']} loaders {ld}"
    gbn = None if gb is None else gb.float().numpy()

    # one row: k slots of distinct experts
    ids = torch.randperm(E, generator=g)[:k]
    wts = torch.softmax(torch.randn(k, generator=g), 0).to(BF)
    x = torch.randn(1, H, generator=g)
    x[:, torch.randperm(H, generator=g)[:8]] *= 20
    x = x.to(BF)
    y64, h64 = MO.layer(x.float().numpy()[0], gu.float().numpy(), dn.float().numpy(), ids.tolist(),
                        wts.float().numpy(), act, gbn)
    tid = ids.to(torch.int16).reshape(1, 1, 1, k).to(device.torch)
    twt = wts.reshape(1, 1, 1, k).to(device.torch)
    tx = x.reshape(1, 1, 1, H).to(device.torch)

    def decode():
        th = moe8.gate_up(tx, P, tid, twt, k, act=act, loaders=ld)
        ty = moe8.down(th, P, tid, k, loaders=ld)
        return _host(th, k * I)[:1], _host(ty, H)[:1]

    h, y = decode()
    h2, y2 = decode()
    same(f"{name}: h repeated", h2, h)
    same(f"{name}: y repeated", y2, y)
    check(f"{name}: h", h, torch.from_numpy(h64).reshape(1, -1))
    check(f"{name}: y", y, torch.from_numpy(y64).reshape(1, -1))

    R = c["rows"]
    if R == 0:
        return
    rid = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(R)])
    rw = torch.softmax(torch.randn(R, k, generator=g), 1).to(BF)
    xr = torch.randn(R, H, generator=g).to(BF)
    u = MO.union(rid.numpy(), E)
    yref = torch.zeros(R, H, dtype=torch.float64)
    href = torch.zeros(R, len(u) * I, dtype=torch.float64)
    for r in range(R):
        yr, hr = MO.layer(xr[r].float().numpy(), gu.float().numpy(), dn.float().numpy(), rid[r].tolist(),
                          rw[r].float().numpy(), act, gbn)
        yref[r] = torch.from_numpy(yr)
        for s, e in enumerate(rid[r].tolist()):
            q = u.index(e)
            href[r, q * I:(q + 1) * I] = torch.from_numpy(hr[s * I:(s + 1) * I])
    tid = rid.to(torch.int16).reshape(1, 1, R, k).to(device.torch)
    twt = rw.reshape(1, 1, R, k).to(device.torch)
    tx = xr.reshape(1, 1, R, H).to(device.torch)
    th = moe8.gate_up_rows(tx, P, tid, twt, k, R, act=act, loaders=ld)
    ty = moe8.down_rows(th, P, tid, k, R, loaders=ld)
    check(f"{name} rows {R}: h", _host(th, len(u) * I)[:R], href)
    yall = _host(ty, H)
    check(f"{name} rows {R}: y", yall[:R], yref)
    same(f"{name} rows {R}: rows past R zero", yall[R:32], torch.zeros(max(0, min(32, yall.shape[0]) - R), H))
