"""The MoE ops (moe/moe8.py) on the GPU against the CPU oracle, after XylolabsInc/tensix-kernels
moe/tests/test_moe.py, test for test.

Experts are random matrices on the BFP4_b grid (so the packed weights hold them exactly); x has a few outlier
channels. Bars, relative Frobenius error and PCC above 0.9999 against the oracle's float64 layer:
- the conversion: the GPU pack holds bfp4_tiles' values bit for bit (the reference compares with ttnn's conversion);
- gate_up and down (one row) below 1 % for h and y, for each activation; two loaders against one, other cores per
  bank, a split share of 0.6 and uint32 ids against the default, bit for bit; ids past E give zeros / add nothing;
- a gate/up bias and column groups (two banks) against the oracle; column groups with one loader refused; the same
  with kblock packs (shared exponents along K), whose GPU pack holds the oracle's kblock values bit for bit;
- gate_up_rows and down_rows (R rows, each with its own experts) below 1 %, rows past R zero; a row of the rows ops
  equals the one-row ops on that row bit for bit where one expert set is shared;
- the same ops at the reference's default fidelity (hifi2): below 1.6 % (one arithmetic here: the same results);
- route: the picks equal the oracle's (the lower id among equal keys) and each weight within 1 bf16 ulp of it or
  within 2^-29 (times the scale), over random rows with ties and fixed edge rows;
- the pack cache: prepack then pack_cached gives the same outputs as pack bit for bit; a mismatched call is refused;
  repack_down equals a fresh pack at the new split;
- a HIP graph of route, gate_up and down, replayed several times, equals the eager calls.
"""

import ctypes
import shutil
import tempfile
from pathlib import Path

import pytest
import torch

from common.testing import check, raises, same
from dense_reader import _lib, linear
from moe import moe8
from oracle import dense_oracle as O
from oracle import moe_oracle as MO

pytestmark = pytest.mark.gpu

E, H, I, K = 16, 1024, 512, 4
BF = torch.bfloat16
REL = 0.01
REL_HIFI2 = 0.016
FID = "hifi4"


def on_grid(w, kblock=False):
    """w's values on the BFP4_b grid (the oracle's held values; kblock: the grid of 16 consecutive K), float32 [K, N]."""
    return torch.from_numpy(MO.held_kblock(w.numpy()) if kblock else O.held(w, "bfp4")).float()


_EXPERTS = {}


def experts(seed, gu_scale=0.02, kblock=False):
    key = (seed, gu_scale, kblock)
    if key not in _EXPERTS:
        g = torch.Generator().manual_seed(seed)
        gu = torch.stack([on_grid(torch.randn(H, 2 * I, generator=g) * gu_scale, kblock).to(BF) for _ in range(E)])
        dn = torch.stack([on_grid(torch.randn(I, H, generator=g) * 0.02, kblock).to(BF) for _ in range(E)])
        _EXPERTS[key] = (gu, dn)
    return _EXPERTS[key]


def make_x(rows, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, H, generator=g)
    x[:, torch.randperm(H, generator=g)[:8]] *= 20
    return x.to(BF)


def decode_inputs(device, seed, ids32=False):
    g = torch.Generator().manual_seed(100 + seed)
    ids = torch.randperm(E, generator=g)[:K]
    wts = torch.softmax(torch.randn(K, generator=g), 0).to(BF)
    x = make_x(1, seed)
    idt = torch.int32 if ids32 else torch.int16
    tid = ids.to(idt).reshape(1, 1, 1, K).to(device.torch)
    twt = wts.reshape(1, 1, 1, K).to(device.torch)
    tx = x.reshape(1, 1, 1, H).to(device.torch)
    return ids, wts, x, tid, twt, tx


def host(t, cols):
    return t.float().cpu().reshape(-1, t.shape[-1])[:, :cols]


def oracle(x, gu, dn, ids, wts, act, gb=None):
    y, h = MO.layer(x.float().numpy()[0], gu.float().numpy(), dn.float().numpy(), ids.tolist(),
                    wts.float().numpy(), act, None if gb is None else gb.float().numpy())
    return torch.from_numpy(y).reshape(1, -1), torch.from_numpy(h).reshape(1, -1)


def test_conversion(device):
    """The GPU pack of a weight holds bfp4_tiles' values bit for bit (zeros and a denormal included)."""
    g = torch.Generator().manual_seed(0)
    w = torch.randn(256, 512, generator=g) * 0.02
    w[3, 5], w[7, 9] = 0.0, -1e-30
    tiles = moe8.bfp4_tiles(w)
    v = torch.from_numpy(moe8.bfp4_values(tiles).transpose(0, 2, 1, 3).reshape(256, 512).copy())
    tw, _ = linear.native_weight(device, w.t().contiguous(), linear.bfloat4_b, sharded=False)
    same("bfp4_tiles against the GPU pack's held values", v, linear.held(tw).float().cpu())


def decode_case(device, fid, rel):
    for act, scale in (("silu", 0.02), ("gelu_tanh", 0.02), ("swiglu_oai", 0.1)):
        gu, dn = experts(1, scale)
        P = moe8.pack(device, gu, dn)
        ids, wts, x, tid, twt, tx = decode_inputs(device, 2)
        ry, rh = oracle(x, gu, dn, ids, wts, act)
        outs = {}
        for loaders in (1, 2):
            th = moe8.gate_up(tx, P, tid, twt, K, act=act, loaders=loaders, fidelity=fid)
            ty = moe8.down(th, P, tid, K, loaders=loaders, fidelity=fid)
            outs[loaders] = (host(th, K * I)[:1], host(ty, H)[:1])
            check(f"{act} gate_up h, {fid}, loaders {loaders}", outs[loaders][0], rh, rel=rel)
            check(f"{act} down y, {fid}, loaders {loaders}", outs[loaders][1], ry, rel=rel)
        same(f"{act} h: two loaders against one", outs[2][0], outs[1][0])
        same(f"{act} y: two loaders against one", outs[2][1], outs[1][1])
        if act == "silu" and fid == FID:
            cpb = 2 if P["cpb"] != 2 else 1
            th = moe8.gate_up(tx, P, tid, twt, K, act=act, cpb=cpb, fidelity=fid)
            same(f"h with {cpb} cores a bank against the pack's {P['cpb']}", host(th, K * I)[:1], outs[2][0])
            try:
                moe8.SPLIT_SHARE = 0.6
                th = moe8.gate_up(tx, P, tid, twt, K, act=act, fidelity=fid)
                ty = moe8.down(th, P, tid, K, fidelity=fid)
                same("h with a split share of 0.6", host(th, K * I)[:1], outs[2][0])
                same("y with a split share of 0.6", host(ty, H)[:1], outs[2][1])
            finally:
                moe8.SPLIT_SHARE = 0.5
            _, _, _, tid32, twt32, tx32 = decode_inputs(device, 2, ids32=True)
            th = moe8.gate_up(tx32, P, tid32, twt32, K, act=act, ids32=True, fidelity=fid)
            ty = moe8.down(th, P, tid32, K, ids32=True, fidelity=fid)
            same("h with uint32 ids", host(th, K * I)[:1], outs[2][0])
            same("y with uint32 ids", host(ty, H)[:1], outs[2][1])


def test_decode(device):
    decode_case(device, FID, REL)


def test_ids_past_experts(device):
    """A slot whose id is not below E chooses no expert: its h columns are zeros and down adds nothing for it."""
    gu, dn = experts(1)
    P = moe8.pack(device, gu, dn)
    ids, wts, x, tid, twt, tx = decode_inputs(device, 3)
    bad = tid.clone()
    bad[..., 1] = E + 5
    th = moe8.gate_up(tx, P, bad, twt, K)
    h = host(th, K * I)
    assert torch.count_nonzero(h[:, I : 2 * I]) == 0
    keep = [0, 2, 3]
    ry, rh = oracle(x, gu, dn, ids[keep], wts[keep], "silu")
    check("h with an id past E: the other slots", h.reshape(K, I)[keep].reshape(1, -1), rh)
    check("y with an id past E: the other slots", host(moe8.down(th, P, bad, K), H), ry)


def rows_inputs(device, R, seed, ids32=False):
    g = torch.Generator().manual_seed(200 + seed)
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(R)])
    wts = torch.softmax(torch.randn(R, K, generator=g), -1).to(BF)
    x = make_x(R, seed)
    idt = torch.int32 if ids32 else torch.int16
    tid = ids.to(idt).reshape(1, 1, R, K).to(device.torch)
    twt = wts.reshape(1, 1, R, K).to(device.torch)
    tx = x.reshape(1, 1, R, H).to(device.torch)
    return ids, wts, x, tid, twt, tx


def rows_case(device, gu, dn, P, R, act="silu", gb=None, loaders=(1,), seed=0, ids32=False, fid=FID):
    ids, wts, x, tid, twt, tx = rows_inputs(device, R, seed, ids32)
    u = MO.union(ids.numpy(), E)
    ref = torch.zeros(R, H, dtype=torch.float64)
    href = torch.zeros(R, len(u) * I, dtype=torch.float64)
    for r in range(R):
        yr, hr = oracle(x[r : r + 1], gu, dn, ids[r], wts[r], act, gb)
        ref[r] = yr[0]
        for s, e in enumerate(ids[r].tolist()):
            q = u.index(e)
            href[r, q * I : (q + 1) * I] = hr[0, s * I : (s + 1) * I]
    outs = []
    for ld in loaders:
        th = moe8.gate_up_rows(tx, P, tid, twt, K, R, act=act, loaders=ld, ids32=ids32, fidelity=fid)
        ty = moe8.down_rows(th, P, tid, K, R, loaders=ld, ids32=ids32, fidelity=fid)
        hd = host(th, len(u) * I)[:R]
        yall = host(ty, H)
        name = f"rows {R} ({act}{', bias' if gb is not None else ''}{', uint32 ids' if ids32 else ''}), {fid}, loaders {ld}"
        bar = REL if fid == "hifi4" else REL_HIFI2
        check(f"{name}: h", hd, href, rel=bar)
        check(f"{name}: y", yall[:R], ref, rel=bar)
        same(f"{name}: rows past R zero", yall[R:32], torch.zeros(32 - R, H))
        same(f"{name}: h rows past R zero", host(th, th.shape[-1])[R:32], torch.zeros(32 - R, th.shape[-1]))
        outs.append((hd, yall))
    for (h1, y1), (h2, y2), ld in zip(outs, outs[1:], loaders[1:]):
        same(f"rows {R}: h with {ld} loaders against {loaders[0]}", h2, h1)
        same(f"rows {R}: y with {ld} loaders against {loaders[0]}", y2, y1)
    return outs


def test_bias_groups(device):
    gu, dn = experts(3, 0.1)
    g = torch.Generator().manual_seed(4)
    gb = torch.randn(E, 2 * I, generator=g) * 0.5
    # two banks: 2 * ceil(16 / 2) = 16 tiles of an expert a bank in the reference's dest: two column groups
    P = moe8.pack(device, gu, dn, banks=2, gu_bias=gb)
    assert moe8.gu_groups(I // 32, 2)[0] == 2
    for act in ("swiglu_oai", "silu"):
        ids, wts, x, tid, twt, tx = decode_inputs(device, 5)
        ry, rh = oracle(x, gu, dn, ids, wts, act, gb)
        th = moe8.gate_up(tx, P, tid, twt, K, act=act, loaders=2, fidelity=FID)
        ty = moe8.down(th, P, tid, K, loaders=2, fidelity=FID)
        check(f"{act} with a bias and column groups, {FID}: h", host(th, K * I)[:1], rh, rel=REL)
        check(f"{act} with a bias and column groups, {FID}: y", host(ty, H)[:1], ry, rel=REL)
    raises("column groups with one loader", AssertionError, lambda: moe8.gate_up(tx, P, tid, twt, K, loaders=1))
    rows_case(device, gu, dn, P, 6, act="swiglu_oai", gb=gb, loaders=(1, 2), seed=6)


def test_kblock_pack(device):
    """The GPU kblock pack (dr_pack, DR_BFP4_KB) read back by dr_unpack holds the oracle's kblock values bit for bit:
    zeros, a tiny value, a group with one large value, and a K past the last full 256 (padded with zeros)."""
    lib = _lib.lib()
    for k, n in ((256, 512), (1120, 96)):
        g = torch.Generator().manual_seed(k)
        w = torch.randn(k, n, generator=g) * 0.02
        w[3, 5], w[7, 9] = 0.0, -1e-30
        w[40:56, 17] *= 300
        k_pad, n_pad = -(-k // linear.KALIGN) * linear.KALIGN, -(-n // 32) * 32
        fmt = moe8.DR_BFP4_KB
        codes = torch.zeros(lib.dr_codes_bytes(fmt, k_pad, n_pad), dtype=torch.uint8, device=device.torch)
        exps = torch.zeros(lib.dr_exps_bytes(fmt, k_pad, n_pad), dtype=torch.uint8, device=device.torch)
        wd = w.t().contiguous().to(device.torch)
        out = torch.full((k, n_pad), float("nan"), device=device.torch)
        _lib.check(lib.dr_pack(wd.data_ptr(), k, n, k, fmt, None, codes.data_ptr(), exps.data_ptr(), n_pad, k_pad,
                               device.stream()), "dr_pack")
        _lib.check(lib.dr_unpack(codes.data_ptr(), exps.data_ptr(), fmt, n, k, n_pad, k_pad, out.data_ptr(), n_pad,
                                 device.stream()), "dr_unpack")
        same(f"kblock pack {k} x {n}", out[:, :n].cpu(), torch.from_numpy(MO.held_kblock(w.numpy())))
    raises("dr_matmul refuses a kblock weight", Exception, lambda: _kblock_matmul(device))


def _kblock_matmul(device):
    """a dense launch of a kblock segment: dr_matmul takes only the four dense formats (DR_EINVAL raises)."""
    L = _lib.Launch()
    x = torch.zeros(1, 256, dtype=BF, device=device.torch)
    y = torch.zeros(1, 32, dtype=BF, device=device.torch)
    codes = torch.zeros(4096, dtype=torch.uint8, device=device.torch)
    L.x, L.m, L.k, L.ldx, L.y, L.ldy, L.nseg = x.data_ptr(), 1, 256, 256, y.data_ptr(), 32, 1
    s0 = L.seg[0]
    s0.fmt, s0.n, s0.n_pad, s0.codes, s0.exps = moe8.DR_BFP4_KB, 32, 32, codes.data_ptr(), codes.data_ptr()
    L.stream = torch.cuda.current_stream(device.torch).cuda_stream
    _lib.check(_lib.lib().dr_matmul(ctypes.byref(L)), "dr_matmul")


def test_kblock_ragged_k(device):
    """kblock packs where K is not a multiple of 256 (H = 2880 for gate/up, I = 1440 for down: the last exponent
    groups half padding): one row on the GEMV and 3 rows on the MFMA kernels against the oracle, silu and
    swiglu_oai."""
    Eg, Hg, Ig, kg = 8, 2880, 1440, 3
    g = torch.Generator().manual_seed(51)
    gu = torch.stack([on_grid(torch.randn(Hg, 2 * Ig, generator=g) * 0.05, True).to(BF) for _ in range(Eg)])
    dn = torch.stack([on_grid(torch.randn(Ig, Hg, generator=g) * 0.02, True).to(BF) for _ in range(Eg)])
    P = moe8.pack(device, gu, dn, kblock=True)
    R = 3
    ids = torch.stack([torch.randperm(Eg, generator=g)[:kg] for _ in range(R)])
    wts = torch.softmax(torch.randn(R, kg, generator=g), -1).to(BF)
    x = torch.randn(R, Hg, generator=g).to(BF)
    tid = ids.to(torch.int16).reshape(1, 1, R, kg).to(device.torch)
    twt = wts.reshape(1, 1, R, kg).to(device.torch)
    tx = x.reshape(1, 1, R, Hg).to(device.torch)
    for act in ("silu", "swiglu_oai"):
        refs = [oracle(x[r : r + 1], gu, dn, ids[r], wts[r], act) for r in range(R)]
        th = moe8.gate_up(tx[:, :, :1].contiguous(), P, tid, twt, kg, act=act, loaders=2)
        ty = moe8.down(th, P, tid, kg)
        check(f"kblock, K past 256-multiples, {act}, one row: h", host(th, kg * Ig)[:1], refs[0][1], rel=REL)
        check(f"kblock, K past 256-multiples, {act}, one row: y", host(ty, Hg)[:1], refs[0][0], rel=REL)
        u = MO.union(ids.numpy(), Eg)
        th = moe8.gate_up_rows(tx, P, tid, twt, kg, R, act=act)
        ty = moe8.down_rows(th, P, tid, kg, R)
        href = torch.zeros(R, len(u) * Ig, dtype=torch.float64)
        for r in range(R):
            for s_, e in enumerate(ids[r].tolist()):
                q = u.index(e)
                href[r, q * Ig : (q + 1) * Ig] = refs[r][1][0, s_ * Ig : (s_ + 1) * Ig]
        check(f"kblock, K past 256-multiples, {act}, {R} rows: h", host(th, len(u) * Ig)[:R], href, rel=REL)
        check(f"kblock, K past 256-multiples, {act}, {R} rows: y", host(ty, Hg)[:R],
              torch.cat([refs[r][0] for r in range(R)]), rel=REL)


def test_bias_groups_kblock(device):
    """The reference's kblock case (each shared exponent over 16 consecutive K at one N): a bias and column groups,
    one row for each activation, the rows ops at 6 rows (the MFMA kernels) and 2 rows (the GEMV's two-row pass), and
    the router inside gate/up equal to route then gate_up, all on the kblock pack against the oracle."""
    gu, dn = experts(3, 0.1, kblock=True)
    g = torch.Generator().manual_seed(4)
    gb = torch.randn(E, 2 * I, generator=g) * 0.5
    P = moe8.pack(device, gu, dn, banks=2, gu_bias=gb, kblock=True)
    assert P["kblock"] and moe8.gu_groups(I // 32, 2)[0] == 2
    for act in ("swiglu_oai", "silu"):
        ids, wts, x, tid, twt, tx = decode_inputs(device, 5)
        ry, rh = oracle(x, gu, dn, ids, wts, act, gb)
        th = moe8.gate_up(tx, P, tid, twt, K, act=act, loaders=2, fidelity=FID)
        ty = moe8.down(th, P, tid, K, loaders=2, fidelity=FID)
        check(f"{act} with a bias, column groups and K blocks, {FID}: h", host(th, K * I)[:1], rh, rel=REL)
        check(f"{act} with a bias, column groups and K blocks, {FID}: y", host(ty, H)[:1], ry, rel=REL)
    raises("column groups with one loader", AssertionError, lambda: moe8.gate_up(tx, P, tid, twt, K, loaders=1))
    rows_case(device, gu, dn, P, 6, act="swiglu_oai", gb=gb, loaders=(1, 2), seed=6)
    rows_case(device, gu, dn, P, 2, act="silu", gb=gb, seed=7)
    rows_case(device, gu, dn, P, 20, act="silu", gb=gb, seed=8)
    # the router inside gate/up on a kblock pack (32 experts: the router takes E a multiple of 32): ids, weights, h
    # and down's y the same as route then gate_up
    Er, Hr, Ir = 32, 256, 64
    g = torch.Generator().manual_seed(9)
    gur = torch.stack([on_grid(torch.randn(Hr, 2 * Ir, generator=g) * 0.05, True).to(BF) for _ in range(Er)])
    dnr = torch.stack([on_grid(torch.randn(Ir, Hr, generator=g) * 0.02, True).to(BF) for _ in range(Er)])
    Pr = moe8.pack(device, gur, dnr, kblock=True)
    lg = (torch.randn(1, 1, 1, Er, generator=g) * 2).to(device.torch)
    xr = torch.randn(1, 1, 1, Hr, generator=g).to(BF).to(device.torch)
    outs = []
    for fused in (False, True):
        ids = torch.full((1, 1, 1, K), 1234, dtype=torch.int16, device=device.torch)
        w = torch.full((1, 1, 1, K), float("nan"), dtype=BF, device=device.torch)
        if fused:
            h = moe8.route_gate_up(lg, xr, Pr, ids, w, K, act="silu", loaders=2)
        else:
            moe8.route(lg, ids, w, K)
            h = moe8.gate_up(xr, Pr, ids, w, K, act="silu", loaders=2)
        y = moe8.down(h, Pr, ids, K)
        outs.append([t.cpu() for t in (ids, w.view(torch.int16), h, y)])
    for name, a, b in zip(("ids", "weights", "h", "y"), outs[1], outs[0]):
        same(f"kblock, the router inside gate/up: {name}", a, b)
    ids0 = outs[0][0].reshape(-1).long()
    ry, rh = oracle(xr.cpu().reshape(1, Hr), gur, dnr, ids0, outs[0][1].view(BF).reshape(-1), "silu")
    check("kblock, routed h against the oracle", host(outs[0][2], K * Ir)[:1], rh, rel=REL)
    check("kblock, routed y against the oracle", host(outs[0][3], Hr)[:1], ry, rel=REL)


def test_rows(device):
    gu, dn = experts(7)
    P = moe8.pack(device, gu, dn)
    rows_case(device, gu, dn, P, 1, seed=1)
    rows_case(device, gu, dn, P, 2, seed=4)
    rows_case(device, gu, dn, P, 5, loaders=(1, 2), seed=2)
    rows_case(device, gu, dn, P, 32, act="gelu_tanh", seed=3)
    rows_case(device, gu, dn, P, 5, seed=2, ids32=True)
    rows_case(device, gu, dn, P, 17, seed=8)
    rows_case(device, gu, dn, P, 24, seed=9)  # (gate_up: the last rows of one 32-row pass)
    rows_case(device, gu, dn, P, 25, seed=10)  # (gate_up: two passes of 16 rows again)


def test_rows_one_row_equals_decode(device):
    """With one row and its own k experts, the rows ops order the slots by expert id: h's blocks are the decode h's
    slots in that order, bit for bit, and y equals the decode y to rounding (the experts are summed in another
    order)."""
    gu, dn = experts(7)
    P = moe8.pack(device, gu, dn)
    ids, wts, x, tid, twt, tx = decode_inputs(device, 9)
    hd = host(moe8.gate_up(tx, P, tid, twt, K), K * I).reshape(K, I)
    hr = host(moe8.gate_up_rows(tx, P, tid, twt, K, 1), K * I)[:1].reshape(K, I)
    order = torch.argsort(ids)
    same("rows h (one row) against the decode h in expert order", hr, hd[order])


def test_hifi2(device):
    """The ops at the reference's default fidelity, against REL_HIFI2."""
    decode_case(device, "hifi2", REL_HIFI2)
    gu, dn = experts(7)
    P = moe8.pack(device, gu, dn)
    rows_case(device, gu, dn, P, 5, loaders=(1, 2), seed=2, fid="hifi2")
    rows_case(device, gu, dn, P, 32, act="gelu_tanh", seed=3, fid="hifi2")


def ulps(a, b):
    """|a - b| in bf16 ulps of b (bf16 tensors)."""
    return (a.view(torch.int16).to(torch.int32) - b.view(torch.int16).to(torch.int32)).abs()


def edge_rows(e, k, g):
    """32 rows of logits [32, e] that a range or sign error shows in: all equal, near 0, tiny, large, huge, ties at the
    k-th place, two values, signs mixed, the rest random."""
    rows = [
        torch.zeros(e),
        torch.full((e,), 1.5),
        torch.full((e,), -2.0),
        torch.randn(e, generator=g) * 1e-3,
        torch.randn(e, generator=g) * 1e-6,
        torch.randn(e, generator=g) * 40,
        torch.randn(e, generator=g) * 1e3,
    ]
    t = torch.randn(e, generator=g)
    t[: 2 * k] = 2.5
    rows.append(t)
    t = torch.randn(e, generator=g)
    t[torch.randperm(e, generator=g)[: k + 3]] = 1.25
    rows.append(t)
    rows.append(torch.where(torch.rand(e, generator=g) < 0.5, torch.tensor(-1.0), torch.tensor(1.0)))
    rows.append(torch.randn(e, generator=g).abs())
    rows.append(-torch.randn(e, generator=g).abs())
    while len(rows) < 32:
        rows.append(torch.randn(e, generator=g) * float(2 ** (len(rows) % 7 - 3)))
    return torch.stack(rows)


def route_case(device, g, name, kind, R, k, ids32=False, bias=False, edge=False, **opts):
    e = 128
    lg = edge_rows(e, k, g) if edge else torch.randn(R, e, generator=g) * 3
    if not edge:
        lg[::2] = lg[::2].to(BF).float()  # ties in the even rows
    R = lg.shape[0]
    tl = lg.reshape(1, 1, R, e).to(device.torch)
    kk = k + (opts.get("slot") is not None)
    idt = torch.int32 if ids32 else torch.int16
    ti = torch.full((1, 1, R, kk), 7, dtype=idt, device=device.torch)
    tw = torch.full((1, 1, R, kk), 7.0, dtype=BF, device=device.torch)
    b, tb = None, None
    if bias:
        b = torch.randn(e, generator=g) * 0.1
        tb = b.reshape(1, 1, 1, e).to(device.torch)
    moe8.route(tl, ti, tw, k, kind=kind, bias=tb, ids32=ids32, **opts)
    gi = ti.cpu().reshape(R, kk).long() & (0xFFFFFFFF if ids32 else 0xFFFF)
    gw = tw.cpu().reshape(R, kk)
    ri, rw = MO.route(lg.numpy(), k, kind, None if b is None else b.numpy(), **opts)
    same(f"route {name}: picks", gi, torch.tensor(ri))
    rw = torch.tensor(rw, dtype=torch.float64)
    tol = 2.0**-29 * max(1.0, opts.get("scale", 1.0))
    bad = (ulps(gw, rw.to(BF)) > 1) & ((gw.double() - rw).abs() > tol)
    ok = int(bad.sum()) == 0
    print(f"{'ok  ' if ok else 'FAIL'} route {name}: weights within 1 bf16 ulp or {tol:.0e}: {int(bad.sum())} off")
    assert ok, name


def test_route(device):
    g = torch.Generator().manual_seed(3)
    route_case(device, g, "softmax R 1 k 8", "softmax", 1, 8)
    route_case(device, g, "softmax R 4 k 6 uint32", "softmax", 4, 6, ids32=True)
    route_case(device, g, "softmax edge rows k 8", "softmax", 32, 8, edge=True)
    route_case(device, g, "sigmoid + bias R 4 k 8", "sigmoid", 4, 8, bias=True)
    route_case(device, g, "sigmoid + bias edge rows k 6 uint32", "sigmoid", 32, 6, ids32=True, bias=True, edge=True)
    route_case(device, g, "sigmoid, no bias, R 4 k 8", "sigmoid", 4, 8)
    route_case(device, g, "sigmoid, no bias, not normalized, edge rows", "sigmoid", 32, 8, edge=True, norm=False)
    route_case(
        device, g, "sigmoid + bias, groups 8/4, scale 2.5, slot", "sigmoid", 8, 8, bias=True,
        groups=(8, 4), scale=2.5, slot=128,
    )


def test_route_gate_up_fused(device):
    """route_gate_up (the token routed inside the gate/up launch) against route then gate_up: ids, weights, the shared
    gate, h, and down's y on them bit for bit, over the router's options (softmax; uint32 ids; sigmoid with a bias and
    a scale; groups; a slot inside and past the experts; a shared gate column), and replayed in a HIP graph."""
    Ef, Hf, If = 64, 512, 256
    g = torch.Generator().manual_seed(41)
    gu = (torch.randn(Ef, Hf, 2 * If, generator=g) * 0.02).to(BF)
    dn = (torch.randn(Ef, If, Hf, generator=g) * 0.02).to(BF)
    gb = (torch.randn(Ef, 2 * If, generator=g) * 0.1).to(BF)
    P = moe8.pack(device, gu, dn, gu_bias=gb)
    x = torch.randn(1, 1, 1, Hf, generator=g).to(BF).to(device.torch)
    bias = (torch.randn(Ef, generator=g) * 0.5).to(device.torch)
    cases = [
        ("softmax k 4", 4, {}),
        ("softmax k 8 uint32", 8, {"ids32": True}),
        ("sigmoid + bias k 6 scale 2.5", 6, {"kind": "sigmoid", "bias": bias, "scale": 2.5}),
        ("sigmoid + bias groups 8/4 k 8", 8, {"kind": "sigmoid", "bias": bias, "groups": (8, 4)}),
        ("softmax k 4 slot 5", 4, {"slot": 5}),
        ("softmax k 3 slot past E", 3, {"slot": Ef + 3}),
        ("softmax k 4 shared gate", 4, {"shared": True}),
    ]
    for name, k, opts in cases:
        opts = dict(opts)
        kk = k + ("slot" in opts)
        idt = torch.int32 if opts.get("ids32") else torch.int16
        width = Ef + (1 if opts.get("shared") else 0)
        lg = (torch.randn(1, 1, 1, width, generator=g) * 2).to(device.torch)
        lg[..., 7] = lg[..., 9]  # (a tie)
        outs = []
        for fused in (False, True):
            ids = torch.full((1, 1, 1, kk), 1234, dtype=idt, device=device.torch)
            w = torch.full((1, 1, 1, kk), float("nan"), dtype=BF, device=device.torch)
            o = dict(opts)
            sh = torch.zeros(1, 1, 1, 1, dtype=BF, device=device.torch) if o.pop("shared", False) else None
            if fused:
                h = moe8.route_gate_up(lg, x, P, ids, w, k, act="swiglu_oai", loaders=2, shared=sh, **o)
            else:
                moe8.route(lg, ids, w, k, experts=Ef, shared=sh, **o)
                h = moe8.gate_up(x, P, ids, w, kk, act="swiglu_oai", loaders=2, ids32=o.get("ids32", False))
            y = moe8.down(h, P, ids, kk, ids32=o.get("ids32", False))
            outs.append([t.cpu() for t in (ids, w.view(torch.int16), h, y)] + ([sh.cpu()] if sh is not None else []))
        for label, a, b in zip(("ids", "weights", "h", "y", "shared gate"), outs[0], outs[1]):
            same(f"route_gate_up {name}: {label} against route then gate_up", b, a)
    # a HIP graph of route_gate_up and down, replayed three times with eager work between, against the eager result
    k = 4
    lg = (torch.randn(1, 1, 1, Ef, generator=g) * 2).to(device.torch)
    ids = torch.zeros(1, 1, 1, k, dtype=torch.int16, device=device.torch)
    w = torch.zeros(1, 1, 1, k, dtype=BF, device=device.torch)
    want_h = moe8.route_gate_up(lg, x, P, ids, w, k, act="silu", loaders=2)
    want_y = moe8.down(want_h, P, ids, k).clone()
    want_h = want_h.clone()
    ids.zero_()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gh = moe8.route_gate_up(lg, x, P, ids, w, k, act="silu", loaders=2)
        gy = moe8.down(gh, P, ids, k)
    for i in range(3):
        ids.zero_()
        graph.replay()
        torch.cuda.synchronize()
        same(f"route_gate_up graph replay {i}: h", gh.cpu(), want_h.cpu())
        same(f"route_gate_up graph replay {i}: y", gy.cpu(), want_y.cpu())


def test_route_shared_gate(device):
    """shared: sigmoid of the logits' column E (a shared expert's gate folded into the router's matmul), in bf16."""
    g = torch.Generator().manual_seed(11)
    R, e = 5, 64
    lg = torch.randn(R, e + 1, generator=g) * 2
    ti = torch.zeros(1, 1, R, 4, dtype=torch.int16, device=device.torch)
    tw = torch.zeros(1, 1, R, 4, dtype=BF, device=device.torch)
    sh = torch.zeros(1, 1, R, 1, dtype=BF, device=device.torch)
    moe8.route(lg.reshape(1, 1, R, e + 1).to(device.torch), ti, tw, 4, experts=e, shared=sh)
    want = torch.sigmoid(lg[:, e].double()).to(BF)
    assert int(ulps(sh.cpu().reshape(R), want).max()) <= 1
    ri, _ = MO.route(lg[:, :e].numpy(), 4)
    same("route with a shared gate column: picks", ti.cpu().reshape(R, 4).long(), torch.tensor(ri))


def test_pack_cache(device):
    gu, dn = experts(9)
    banks = moe8.dev.dram_banks(device)
    tmp = Path(tempfile.mkdtemp(prefix="moe8-cache-"))
    try:
        cache = tmp / "layer0"
        cpb = moe8._clamp_cpb(device, banks, 3)
        assert moe8.prepack(gu, dn, cache, banks, cpb) is True
        assert moe8.prepack(gu, dn, cache, banks, cpb) is False
        ids, wts, x, tid, twt, tx = decode_inputs(device, 8)
        P0 = moe8.pack(device, gu, dn)
        P1 = moe8.pack_cached(device, cache)
        h0, h1 = moe8.gate_up(tx, P0, tid, twt, K), moe8.gate_up(tx, P1, tid, twt, K)
        same("pack_cached against pack: h", host(h1, K * I), host(h0, K * I))
        same("pack_cached against pack: y", host(moe8.down(h1, P1, tid, K), H), host(moe8.down(h0, P0, tid, K), H))
        other = experts(10)
        raises("a cache of other weights", moe8.PackCacheMismatch, lambda: moe8.prepack(*other, cache, banks, cpb))
        raises("a cache of another split", moe8.PackCacheMismatch, lambda: moe8.pack_cached(device, cache, cores_per_bank=1))
        assert moe8.repack_down(cache, cores_per_bank=1) is True
        P2 = moe8.pack_cached(device, cache, cores_per_bank=1)
        P3 = moe8.pack(device, gu, dn, cores_per_bank=1)
        same("repack_down against a fresh pack: y", host(moe8.down(h0, P2, tid, K), H), host(moe8.down(h0, P3, tid, K), H))
        P4 = moe8.pack(device, gu, dn, cache=tmp / "layer1")
        same("pack with cache= against pack: the packed codes", P4["gu"].cpu(), P0["gu"].cpu())
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


def test_split_k_decode_loop(device):
    """gate_up and down of an H = I = 2880 layer, both split K (their workgroups meet in one shared workspace), in a
    decode loop of three steps on other experts and another x each: every step's h and y equal the same step run on a
    fresh workspace, bit for bit (down's partial sums never land where gate_up's counters are), and the first step's
    h the oracle's."""
    Hb = Ib = 2880
    Eb = 8
    g = torch.Generator().manual_seed(30)
    gu = (torch.randn(Eb, Hb, 2 * Ib, generator=g) * 0.02).to(BF)
    dn = (torch.randn(Eb, Ib, Hb, generator=g) * 0.02).to(BF)
    P = moe8.pack(device, gu, dn)
    steps = []
    for s in range(3):
        ids = torch.randperm(Eb, generator=g)[:K]
        wts = torch.softmax(torch.randn(K, generator=g), 0).to(BF)
        x = torch.randn(1, Hb, generator=g).to(BF)
        steps.append((ids, wts, x, ids.to(torch.int16).reshape(1, 1, 1, K).to(device.torch),
                      wts.reshape(1, 1, 1, K).to(device.torch), x.reshape(1, 1, 1, Hb).to(device.torch)))

    def step(st):
        th = moe8.gate_up(st[5], P, st[3], st[4], K)
        ty = moe8.down(th, P, st[3], K)
        return host(th, K * Ib)[:1], host(ty, Hb)[:1]

    loop = [step(st) for st in steps]
    for i, st in enumerate(steps):
        linear._WORKSPACE.clear()
        h, y = step(st)
        same(f"decode loop step {i}: h against the step alone", loop[i][0], h)
        same(f"decode loop step {i}: y against the step alone", loop[i][1], y)
    ids, wts, x = steps[0][:3]
    held_gu = torch.stack([torch.from_numpy(O.held(gu[e].float(), "bfp4")) for e in ids.tolist()])
    _, rh = MO.layer(x.float().numpy()[0], held_gu.double().numpy(), torch.zeros(K, Ib, 1).double().numpy(),
                     list(range(K)), wts.float().numpy(), "silu")
    check("decode loop step 0: h against the oracle", loop[0][0], torch.from_numpy(rh).reshape(1, -1), rel=REL)
    # down (16-column tiles in four K splits at this shape) on its own input: the step's bf16 h times the held rows
    hd = loop[0][0].double().reshape(K, Ib)
    ry = sum(hd[s] @ torch.from_numpy(O.held(dn[e].float(), "bfp4")).double() for s, e in enumerate(ids.tolist()))
    check("decode loop step 0: y against the oracle on the step's h", loop[0][1], ry.reshape(1, -1).float(), rel=REL)


def test_graph_replay(device):
    """route, gate_up and down captured in one HIP graph, replayed several times with eager work between, equal the
    eager calls each time."""
    gu, dn = experts(1)
    P = moe8.pack(device, gu, dn)
    g = torch.Generator().manual_seed(12)
    lg = torch.full((1, 1, 1, 32), -1e9)  # (the router takes a multiple of 32 experts: columns past E never win)
    lg[..., :E] = torch.randn(E, generator=g) * 2
    lg = lg.to(device.torch)
    tid = torch.zeros(1, 1, 1, K, dtype=torch.int16, device=device.torch)
    twt = torch.zeros(1, 1, 1, K, dtype=BF, device=device.torch)
    x = make_x(1, 13).reshape(1, 1, 1, H).to(device.torch)

    def layer():
        moe8.route(lg, tid, twt, K)
        return moe8.down(moe8.gate_up(x, P, tid, twt, K), P, tid, K)

    want = layer().clone()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = layer()
    for i in range(4):
        tid.zero_()
        graph.replay()
        torch.cuda.synchronize()
        same(f"graph replay {i}: y", out.cpu(), want.cpu())
        layer()  # eager work between the replays
        torch.cuda.synchronize()
