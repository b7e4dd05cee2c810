"""A seeded sweep over the matmul's option space on the GPU, every case against the CPU oracle.

The config tests pin each benchmarked shape; this sweep covers the combinations between them: formats, rows on either
kernel (1-2 GEMV, 3-32 MFMA, past 32 in passes), K with and without padding and split K, N off the tile width, bf16
and fp32 column scales, the GLU (interleaved or two weights, silu or gelu_tanh, with or without scales), the residual
in both modes with and without the fp32 output, the fp32 output alone, col0 into a wider output, block lists of mixed
formats with per-block scales, and top-k records (bf16 keys or fp32 scores, a record a tile or groups of tiles). Expected values come
from the oracle alone (oracle.held of the float weights, oracle.ref in float64, oracle.tile_topk's ranking of the op's
own output), with the reference's bars (linear.py / test_dense_reader.py: 1 % relative Frobenius error and PCC 0.9999
for bf16 outputs, 0.1 % for fp32 outputs, records bit for bit); every case is also called twice and must repeat bit
for bit. A second sweep runs the top-k merge on seeded random records against the oracle's host merge.
"""

import numpy as np
import pytest
import torch

from common.testing import check, same
from dense_reader import linear
from oracle import dense_oracle as O

pytestmark = pytest.mark.gpu

FMTS = {"bfp8": linear.bfloat8_b, "bfp4": linear.bfloat4_b, "bf16": linear.bfloat16}
KS = (96, 256, 480, 1024, 1056, 2048, 2080, 4096, 4352, 6144, 9216)
NS_ = (32, 48, 96, 200, 256, 480, 544, 1024, 1056)
MS = (1, 2, 3, 4, 5, 8, 13, 16, 17, 24, 31, 32, 33, 40)
KINDS = ("plain", "scale", "glu", "residual", "out32", "col0", "blocks", "topk")
CASES = 200


def _case(i):
    """Case i: a dict of the options, drawn from a generator seeded by i (the same cases on every run)."""
    r = np.random.default_rng(1000 + i)
    kind = KINDS[i % len(KINDS)]
    c = {"i": i, "kind": kind, "fmt": str(r.choice(list(FMTS))), "k": int(r.choice(KS)), "n": int(r.choice(NS_)),
         "m": int(r.choice(MS))}
    if kind in ("glu", "blocks"):
        c["m"] = min(c["m"], 32)
    if kind == "scale":
        c["f32"] = bool(r.integers(2))
    if kind == "glu":
        c["n"] = 32 * int(r.integers(1, 18))  # whole gate/up tile pairs
        c["two"] = bool(r.integers(2))
        c["act"] = str(r.choice(["swiglu", "geglu"]))
        c["scaled"] = bool(r.integers(2))
    if kind == "residual":
        c["mode"] = str(r.choice(["epilogue", "preload"]))
        c["out32"] = bool(r.integers(2))
    if kind == "col0":
        c["col0"] = int(r.integers(0, 4))
        c["extra"] = int(r.integers(0, 3))
    if kind == "blocks":
        nb = int(r.integers(2, 5))
        c["blocks"] = [(str(r.choice(list(FMTS))), int(r.choice((32, 64, 96, 160, 256))), bool(r.integers(2)))
                       for _ in range(nb)]
        c["k"] = min(c["k"], 4352)
    if kind == "topk":
        c["m"] = min(c["m"], 32)
        c["rows"] = int(r.integers(1, c["m"] + 1))
        c["kk"] = int(r.choice([1, 2, 5, 8, 16, 32]))
        c["cut"] = int(r.integers(0, 40)) if r.integers(2) else 0  # (valid columns: n - cut)
        c["base"] = int(r.integers(0, 5000))
        c["slots"] = int(r.choice([0, 3, 7]))  # (0: a record a tile; else tiles ranked in groups)
        c["fp32"] = bool(r.integers(2))  # (fp32 scores, or the reference's bf16 keys)
    if c["k"] >= 9216:
        c["n"] = min(c["n"], 256)  # (a split-K case: the oracle's float64 product stays small)
    return c


def _x(dev, m, k, seed):
    x = O.x_input(m, k, seed)
    return x, x.to(torch.bfloat16).reshape(1, 1, m, k).to(dev.torch)


def _weight(dev, n, k, fmt, seed):
    """A packed weight and the oracle's held values of it, [K, n] float."""
    wt = O.matrix(n, k, seed)
    tw = linear.native_weight(dev, wt, FMTS[fmt])[0]
    return tw, torch.from_numpy(O.held(wt.T.contiguous(), fmt)).float()


def _scales(dev, n, seed, f32):
    """Column scales in U(0.5, 1.5): the tensor the op takes and the values it holds (bf16 rounds them)."""
    s = torch.rand(n, generator=torch.Generator().manual_seed(seed)) + 0.5
    ts = linear.scale_tensor(dev, s, dtype=linear.float32 if f32 else linear.bfloat16)
    return ts, (s if f32 else s.to(torch.bfloat16).float())


def _host(y, m, n, c0=0):
    return y.float().cpu().reshape(-1, y.shape[-1])[:m, c0:c0 + n]


def _ref64(x, h, s=None):
    y = x.to(torch.bfloat16).double() @ h.double()
    return y * s.double()[None, :] if s is not None else y


def _twice(name, fn):
    """fn() twice: the second result must equal the first bit for bit."""
    a = fn()
    b = fn()
    same(f"{name}: repeated call", a, b)
    return a


@pytest.mark.parametrize("i", range(CASES))
def test_sweep(device, i):
    c = _case(i)
    print(f"case {c}", flush=True)
    kind, fmt, k, n, m = c["kind"], c["fmt"], c["k"], c["n"], c["m"]
    x, tx = _x(device, m, k, 2000 + i)
    name = f"sweep {i} {kind} {fmt} M {m} K {k} N {n}"
    if kind == "plain":
        tw, h = _weight(device, n, k, fmt, 3000 + i)
        y = _twice(name, lambda: _host(linear.matmul(tx, tw, None), m, n))
        check(name, y, _ref64(x, h).float())
    elif kind == "scale":
        tw, h = _weight(device, n, k, fmt, 3000 + i)
        ts, s = _scales(device, n, 4000 + i, c["f32"])
        y = _twice(name, lambda: _host(linear.matmul(tx, tw, ts), m, n))
        check(f"{name} scales fp32 {c['f32']}", y, _ref64(x, h, s).float())
    elif kind == "glu":
        gw, uw = O.matrix(n, k, 3000 + i), O.matrix(n, k, 3500 + i)
        hg = torch.from_numpy(O.held(gw.T.contiguous(), fmt)).float()
        hu = torch.from_numpy(O.held(uw.T.contiguous(), fmt)).float()
        sg = su = None
        kw = {"glu": True, "glu_act": {"swiglu": 0, "geglu": 1}[c["act"]]}
        if c["two"]:
            tg = linear.native_weight(device, gw, FMTS[fmt])[0]
            tu = linear.native_weight(device, uw, FMTS[fmt])[0]
            tsg = None
            if c["scaled"]:
                tsg, sg = _scales(device, n, 4000 + i, True)
                tsu, su = _scales(device, n, 4500 + i, True)
                kw["scale_up"] = tsu
            call = lambda: _host(linear.matmul(tx, tg, tsg, w_up=tu, **kw), m, n)  # noqa: E731
        else:
            ti = linear.native_weight(device, linear.interleave_glu(gw, uw), FMTS[fmt])[0]
            tsi = None
            if c["scaled"]:
                _, sg = _scales(device, n, 4000 + i, True)
                _, su = _scales(device, n, 4500 + i, True)
                both = torch.stack([sg.reshape(-1, 32), su.reshape(-1, 32)], 1).reshape(-1)
                tsi = linear.scale_tensor(device, both, dtype=linear.float32)
            call = lambda: _host(linear.matmul(tx, ti, tsi, **kw), m, n)  # noqa: E731
        y = _twice(name, call)
        check(f"{name} {c['act']} two weights {c['two']} scaled {c['scaled']}", y,
              O.glu_ref(_ref64(x, hg, sg), _ref64(x, hu, su), c["act"]))
    elif kind == "residual":
        tw, h = _weight(device, n, k, fmt, 3000 + i)
        res = torch.randn(m, n, generator=torch.Generator().manual_seed(5000 + i)).to(torch.bfloat16)
        tr = res.reshape(1, 1, m, n).to(device.torch)
        want = (_ref64(x, h) + res.double()).float()
        y = _twice(name, lambda: _host(linear.matmul(tx, tw, None, residual=tr, residual_mode=c["mode"],
                                                     out32=c["out32"]), m, n))
        if c["out32"]:
            check(f"{name} residual {c['mode']} fp32 out", y, want, rel=1e-3, pcc=0.999999)
        else:
            check(f"{name} residual {c['mode']}", y, want)
    elif kind == "out32":
        tw, h = _weight(device, n, k, fmt, 3000 + i)
        y = _twice(name, lambda: _host(linear.matmul(tx, tw, None, out32=True), m, n))
        check(f"{name} fp32 out", y, _ref64(x, h).float(), rel=1e-3, pcc=0.999999)
    elif kind == "col0":
        tw, h = _weight(device, n, k, fmt, 3000 + i)
        c0, width = c["col0"], 32 * (c["col0"] + c["extra"]) + n
        out = torch.full((1, 1, m, width), 7.0, dtype=torch.bfloat16, device=device.torch)
        linear.matmul(tx, tw, None, out=out, col0=c0)
        y = out.float().cpu().reshape(m, width)
        check(f"{name} col0 {c0}", y[:, 32 * c0:32 * c0 + n], _ref64(x, h).float())
        rest = torch.cat([y[:, :32 * c0], y[:, 32 * c0 + n:]], 1)
        same(f"{name} col0 {c0}: the other columns untouched", rest, torch.full_like(rest, 7.0))
    elif kind == "topk":
        tw, h = _weight(device, n, k, fmt, 3000 + i)
        rows, kk, base, slots, f32 = c["rows"], c["kk"], c["base"], c["slots"], c["fp32"]
        nv = max(1, n - c["cut"])
        recs = linear.topk_slots(n, slots)
        r = linear.topk_result(device, recs, rows, kk)
        spec = {"r": r, "k": kk, "rows": rows, "slot0": 0, "base": base, "n": nv, "write_y": True, "slots": slots,
                "fp32": f32}
        g = linear.launch_plan(tx, tw, None, topk=spec)["tiles_per_record"]
        y = _host(linear.matmul(tx, tw, None, topk=spec), m, n)
        check(f"{name} top-k: y", y, _ref64(x, h).float())
        words = r.cpu().reshape(recs, -1)
        yf = None
        if f32:  # the fp32 scores the records rank: the same sums, written by an fp32-output call
            yf = _host(linear.matmul(tx, tw, None, out32=True), m, n)
            check(f"{name} top-k: fp32 scores", yf, _ref64(x, h).float(), rel=1e-3, pcc=0.999999)
            same(f"{name} top-k: fp32 scores rounded to bf16 equal y", yf.to(torch.bfloat16).float(), y)
            yf = yf[:rows].numpy()
        want = O.tile_topk(y[:rows].numpy(), rows, kk, nv, base, fp32=f32, yf=yf, width=32 * g)
        same(f"{name} top-k rows {rows} k {kk} valid {nv} groups of {g} fp32 {f32}: records against the oracle's "
             f"ranking of y", words, torch.from_numpy(want.view(np.int32)))
        r2 = linear.topk_result(device, recs, rows, kk)
        linear.matmul(tx, tw, None, topk={**spec, "r": r2})
        same(f"{name} top-k: repeated call", r2.cpu().reshape(recs, -1), words)
    else:  # blocks
        entries, wants, col, singles = [], [], 0, []
        for j, (bf, bn, scaled) in enumerate(c["blocks"]):
            tw, h = _weight(device, bn, k, bf, 3000 + 10 * i + j)
            ts, s = _scales(device, bn, 4000 + 10 * i + j, True) if scaled else (None, None)
            entries.append((tw, col // 32, ts) if scaled else (tw, col // 32))
            singles.append((tw, col // 32, ts))
            wants.append((col, bn, _ref64(x, h, s).float()))
            col += 32 * (-(-bn // 32)) + 32 * (j % 2)  # (every other block leaves a tile of gap)
        # (the gaps between blocks are never written: only the blocks' columns are compared)
        cols = torch.cat([torch.arange(c0, c0 + bn) for c0, bn, _ in wants])
        y = linear.matmul(tx, entries, None).float().cpu().reshape(m, -1)
        same(f"{name}: repeated call", y[:, cols], linear.matmul(tx, entries, None).float().cpu().reshape(m, -1)[:, cols])
        for j, (c0, bn, want) in enumerate(wants):
            check(f"{name} block {j} {c['blocks'][j]}", y[:, c0:c0 + bn], want)
        one = torch.zeros(1, 1, m, y.shape[1], dtype=torch.bfloat16, device=device.torch)
        for tw, t0, ts in singles:
            linear.matmul(tx, tw, ts, out=one, col0=t0)
        for j, (c0, bn, _) in enumerate(wants):
            same(f"{name} block {j}: against one call per block", y[:, c0:c0 + bn],
                 one.float().cpu().reshape(m, -1)[:, c0:c0 + bn])


MERGE_CASES = 60


@pytest.mark.parametrize("i", range(MERGE_CASES))
def test_merge_sweep(device, i):
    """dr_topk_merge on seeded random records (record counts 1-9000, 1-32 rows, k 1-32, k_out 1-64, bf16 keys or fp32
    scores; few distinct values, normal values or a ramp; slots unsorted or sorted within each record as the matmul
    writes them) against the oracle's host merge, bit for bit."""
    from test_dense_reader import _records

    r = np.random.default_rng(9000 + i)
    nrec = int(r.choice([1, 3, 17, 100, 517, 1024, 4008, 9000]))
    rows = int(r.choice([1, 2, 3, 4, 7, 16, 32]))
    k = int(r.choice([1, 2, 4, 5, 8, 16, 32]))
    if rows * k > 256:
        k = max(1, 256 // rows)
    k_out = int(r.choice([1, 8, 16, 31, 32, 33, 64]))
    fp32 = bool(r.integers(2))
    kind = int(r.integers(3))
    values = (np.array([-3.0, -1.0, 0.0, 0.5, 1.0, 2.0, 3.0], np.float32) if kind == 0 else
              r.standard_normal(5000).astype(np.float32) if kind == 1 else np.arange(200, dtype=np.float32) / 7)
    t = _records(nrec, rows, k, fp32, int(r.integers(1 << 30)), values)
    name = f"merge sweep {i}: records {nrec} rows {rows} k {k} k_out {k_out} fp32 {fp32} values {kind}"
    if r.integers(2):  # each record's slots sorted best first, as the matmul writes them
        w = t.numpy().view(np.uint32).reshape(nrec, 2, rows, k).copy()
        order = np.argsort(-w[:, 0].view(np.float32), axis=2, kind="stable") if fp32 else \
            np.argsort(-w[:, 0].astype(np.int64), axis=2, kind="stable")
        w[:, 0] = np.take_along_axis(w[:, 0], order, 2)
        w[:, 1] = np.take_along_axis(w[:, 1], order, 2)
        t = torch.from_numpy(w.reshape(nrec, -1).view(np.int32))
        name += " sorted"
    print(name, flush=True)
    hv, hi = linear.records_host(t, rows, k, fp32=fp32)
    wv, wi = O.global_topk(hv.numpy(), hi.numpy(), k_out)
    gv, gi = linear.topk_merge(t.reshape(1, 1, nrec, -1).to(device.torch), rows, k, k_out=k_out, fp32=fp32)
    same(f"{name}: values", gv.cpu(), torch.from_numpy(wv))
    same(f"{name}: ids", gi.cpu().long(), torch.from_numpy(wi))
