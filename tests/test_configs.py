"""Every benchmarked configuration at its full shape, through the kernel the bench times, against the CPU oracle.

The shapes are the benchmark's (bench.py CONFIGS; the north star NS and C1-C5): weights W ~ N(0, 0.02) [out, in],
x with the reference tests' outlier channels (test_dense_reader.py:28-39), fp32 column scales U(0.5, 1.5). Each test
first asks the library which kernel the call runs (linear.launch_plan, the C ABI's dr_launch_plan) and asserts it is
the benchmarked one, then checks the output:

- the held values are the GPU's unpack (dr_unpack) of the packed weight, five of its 32-column tiles compared bit for
  bit with the oracle's own conversion of the same matrix (the rest is the same kernel on more tiles);
- the matmul against x (bf16) @ held in float64 (oracle.ref, test_dense_reader.py:56-58), with the reference's bars:
  relative Frobenius error below 1 % and PCC above 0.9999 for bf16 outputs, 0.1 % for fp32 outputs
  (test_dense_reader.py:104-136);
- bit for bit where two launches must agree (a block list and one call per block, repeated calls, graph replays);
- top-k records (test_dense_reader.py:139-157, with BASELINE's bar for fp32 scores): the ids of every record exact
  except at float64 scores tied within 1e-3 relative, the record values equal to the output at their ids.
"""

import numpy as np
import pytest
import torch

from common.testing import check, same
from dense_reader import linear
from oracle import dense_oracle as O

pytestmark = pytest.mark.gpu

FMT = {"bfp8": linear.bfloat8_b, "bfp4": linear.bfloat4_b, "bf16": linear.bfloat16}


def x_input(device, m, k, seed):
    x = O.x_input(m, k, seed)
    return x, x.to(torch.bfloat16).reshape(1, 1, m, k).to(device.torch)


def host(y, m, n):
    return y.float().cpu().reshape(-1, y.shape[-1])[:m, :n]


def pinned_held(tw, wt, fmt, n, div=None):
    """The weight's held values [K, n] (the GPU's unpack), with the first, the last and three random 32-column tiles
    compared bit for bit with the oracle's conversion of wt [n, K] (divided by div [n] first, as col_scale does)."""
    h = linear.held(tw, n).cpu()
    tiles = -(-n // 32)
    rng = np.random.default_rng(n * 7 + tw.k)
    for t in sorted({0, tiles - 1, *rng.integers(0, tiles, 3).tolist()}):
        c0, c1 = 32 * t, min(32 * t + 32, n)
        src = wt[c0:c1] if div is None else wt[c0:c1] / div[c0:c1, None]
        want = torch.from_numpy(O.held(src.T.contiguous(), fmt))[:, : c1 - c0]
        same(f"{fmt} K {tw.k} N {n}: held tile {t} against the oracle", h[:, c0:c1], want)
    return h


def ref64(x, h, scale=None):
    """x rounded to bf16 times h in float64 (times the column scales), left in float64."""
    y = x.to(torch.bfloat16).double() @ h.double()
    return y * scale.double()[None, :] if scale is not None else y


def uniform_scales(n, seed):
    return torch.rand(n, generator=torch.Generator().manual_seed(seed)) + 0.5


def assert_plan(p, **want):
    got = {k: p[k] for k in want}
    print(f"plan: {p}", flush=True)
    assert got == want, (got, want, p)


# --- NS: the north star, bfloat8_b M=1 (and 2) K=4096 N=14336 ---------------------------------------------------------


@pytest.fixture(scope="module")
def ns_weights(device):
    k, n = 4096, 14336
    wts = [O.matrix(n, k, 100 + i) for i in range(3)]
    tws = [linear.native_weight(device, w, linear.bfloat8_b)[0] for w in wts]
    held = [pinned_held(tw, w, "bfp8", n) for tw, w in zip(tws, wts)]
    return k, n, tws, held


@pytest.mark.parametrize("m", [1, 2])
def test_ns_gemv(device, ns_weights, m):
    """NS on the wide (32-column) GEMV the bench times, against the oracle; repeated calls bit-identical."""
    k, n, tws, held = ns_weights
    x, tx = x_input(device, m, k, 110 + m)
    assert_plan(linear.launch_plan(tx, tws[0], None), kernel="gemv", rows_per_pass=m, tile_cols=32)
    y = linear.matmul(tx, tws[0], None)
    check(f"NS bfp8 rows {m} K {k} N {n}", host(y, m, n), ref64(x, held[0]).float())
    same(f"NS rows {m}: repeated call", host(linear.matmul(tx, tws[0], None), m, n), host(y, m, n))


def test_ns_graph_replay(device, ns_weights):
    """NS as the bench runs it: the matmuls over rotating weights captured in one HIP graph, replayed three times with
    eager launches between the replays; every replay's outputs equal the eager ones bit for bit."""
    k, n, tws, held = ns_weights
    x, tx = x_input(device, 1, k, 120)
    ys = [torch.empty(1, 1, 1, n, dtype=torch.bfloat16, device=device.torch) for _ in tws]
    eager = [host(linear.matmul(tx, tw, None), 1, n) for tw in tws]
    for i, e in enumerate(eager):
        check(f"NS eager weight {i}", e, ref64(x, held[i]).float())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for tw, y in zip(tws, ys):
            linear.matmul(tx, tw, None, out=y)
    for rep in range(3):
        for y in ys:
            y.fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        for i, y in enumerate(ys):
            same(f"NS graph replay {rep} weight {i} against eager", host(y, 1, n), eager[i])
        linear.matmul(tx, tws[rep % len(tws)], None)  # eager work between the replays
        torch.cuda.synchronize()


# --- C1: bfloat8_b M=1 K=2048 N=4096, no fused stage ---------------------------------------------------------------


def test_c1_gemv(device):
    """C1 as the bench times it: x [1, 2048] against bfloat8_b W [4096, 2048], no scale, bf16 out, on dr_gemv_g1 (256-k
    chunks) with 16-column tiles (256 workgroups), against the oracle; repeated calls bit-identical, and the same bits
    as a launch of 32-column tiles (the weight as the first block of a list wide enough for them)."""
    k, n, m = 2048, 4096, 1
    wt = O.matrix(n, k, 130)
    tw = linear.native_weight(device, wt, linear.bfloat8_b)[0]
    held = pinned_held(tw, wt, "bfp8", n)
    x, tx = x_input(device, m, k, 131)
    p = linear.launch_plan(tx, tw, None)
    assert_plan(p, kernel="gemv", rows_per_pass=1, tile_cols=16, tiles=256, kch=256, splits=1)
    y = linear.matmul(tx, tw, None)
    check(f"C1 bfp8 rows {m} K {k} N {n}", host(y, m, n), ref64(x, held).float())
    same("C1: repeated call", host(linear.matmul(tx, tw, None), m, n), host(y, m, n))
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    wide_tiles = 7 * cus // 4  # (448 on 256 CUs: a launch of 32-column tiles)
    big = linear.native_weight(device, O.matrix(32 * wide_tiles - n, k, 132), linear.bfloat8_b)[0]
    blocks = [(tw, 0), (big, n // 32)]
    pb = linear.launch_plan(tx, blocks, None)
    assert_plan(pb, kernel="gemv", tile_cols=32, kch=256, tiles=wide_tiles)
    yb = host(linear.matmul(tx, blocks, None), m, n)
    same("C1: 16-column tiles against 32-column tiles (the weight inside a wider block list)", yb, host(y, m, n))


@pytest.mark.parametrize("m", [1, 2])
def test_int4_wide(device, m):
    """int4 W4A16 at the bench's K=4096 N=14336 (the wide GEMV), against the oracle's x @ (q * s).T."""
    from int4 import w4a16

    k, n = 4096, 14336
    g = torch.Generator().manual_seed(130)
    codes = torch.randint(-7, 8, (n, k), generator=g).to(torch.int8)
    scales = (torch.rand(n, k // 32, generator=g) * 0.01 + 0.001).to(torch.bfloat16)
    wq = w4a16.int4_weight(device, codes)
    ts = w4a16.group_scales(device, scales)
    x, tx = x_input(device, m, k, 131 + m)
    x2 = tx.reshape(m, k)
    assert_plan(w4a16.launch_plan(x2, wq, ts), kernel="gemv", rows_per_pass=m, tile_cols=32)
    y = w4a16.rows_matmul(x2, wq, ts).float().cpu()
    check(f"int4 rows {m} K {k} N {n}", y, O.int4_ref(x, codes, scales))


# --- C2: bfloat4_b gate/up with fp32 column scales on both, SwiGLU / GeGLU --------------------------------------------


@pytest.fixture(scope="module")
def c2_weights(device):
    k, n = 4096, 14336
    gate, up = O.matrix(n, k, 140), O.matrix(n, k, 141)
    tg = linear.native_weight(device, gate, linear.bfloat4_b)[0]
    tu = linear.native_weight(device, up, linear.bfloat4_b)[0]
    ti = linear.native_weight(device, linear.interleave_glu(gate, up), linear.bfloat4_b)[0]
    hg, hu = pinned_held(tg, gate, "bfp4", n), pinned_held(tu, up, "bfp4", n)
    hi = linear.held(ti, 2 * n).cpu()
    inter = torch.stack([hg.reshape(k, -1, 32), hu.reshape(k, -1, 32)], dim=2).reshape(k, 2 * n)
    same("C2 interleaved weight: held values are the gate's and up's tiles, alternating", hi, inter)
    sg, su = uniform_scales(n, 142), uniform_scales(n, 143)
    return k, n, tg, tu, ti, hg, hu, sg, su


@pytest.mark.parametrize("m", [1, 2])
@pytest.mark.parametrize("act", ["swiglu", "geglu"])
def test_c2_glu_scales(device, c2_weights, m, act):
    """act((x Wg) * sg) * ((x Wu) * su), two weights and interleave_glu's one, on the GLU GEMV (four panels a tile)."""
    k, n, tg, tu, ti, hg, hu, sg, su = c2_weights
    x, tx = x_input(device, m, k, 150 + m)
    tsg = linear.scale_tensor(device, sg, dtype=linear.float32)
    tsu = linear.scale_tensor(device, su, dtype=linear.float32)
    # interleave_glu's scales: the weight's columns, gate tile j then up tile j
    tsi = linear.scale_tensor(device, torch.stack([sg.reshape(-1, 32), su.reshape(-1, 32)], 1).reshape(-1),
                              dtype=linear.float32)
    g, u = ref64(x, hg, sg), ref64(x, hu, su)
    want = O.glu_ref(g, u, act)
    glu_act = {"swiglu": 0, "geglu": 1}[act]
    p = linear.launch_plan(tx, tg, tsg, glu=True, w_up=tu, scale_up=tsu, glu_act=glu_act)
    assert_plan(p, kernel="gemv", rows_per_pass=m, tile_cols=32, tiles=n // 32)
    y2 = linear.matmul(tx, tg, tsg, glu=True, w_up=tu, scale_up=tsu, glu_act=glu_act)
    check(f"C2 {act} two weights rows {m}", host(y2, m, n), want)
    yi = linear.matmul(tx, ti, tsi, glu=True, glu_act=glu_act)
    check(f"C2 {act} interleaved rows {m}", host(yi, m, n), want)
    same(f"C2 {act} rows {m}: interleaved against two weights", host(yi, m, n), host(y2, m, n))


# --- C3: bfloat8_b M=8 K=14336 N=4096, residual and fp32 output ---------------------------------------------------------


@pytest.fixture(scope="module")
def c3_weights(device):
    k, n = 14336, 4096
    wt = O.matrix(n, k, 160)
    tw = linear.native_weight(device, wt, linear.bfloat8_b)[0]
    return k, n, tw, pinned_held(tw, wt, "bfp8", n)


@pytest.mark.parametrize("mode", ["epilogue", "preload"])
def test_c3_residual_out32(device, c3_weights, mode):
    """y = x W + residual in fp32 (split K over two workgroups a tile), both residual modes; bf16 in place."""
    k, n, tw, h = c3_weights
    m = 8
    x, tx = x_input(device, m, k, 161)
    res = torch.randn(m, n, generator=torch.Generator().manual_seed(162)).to(torch.bfloat16)
    tr = res.reshape(1, 1, m, n).to(device.torch)
    want = ref64(x, h) + res.double()
    p = linear.launch_plan(tx, tw, None, residual=tr, residual_mode=mode, out32=True)
    assert_plan(p, kernel="mfma", rows_per_pass=16, splits=2)
    y = linear.matmul(tx, tw, None, residual=tr, residual_mode=mode, out32=True)
    assert y.dtype == torch.float32
    check(f"C3 residual ({mode}) + fp32 out rows {m}", host(y, m, n), want.float(), rel=1e-3, pcc=0.999999)
    same(f"C3 {mode}: repeated call", host(linear.matmul(tx, tw, None, residual=tr, residual_mode=mode, out32=True),
                                            m, n), host(y, m, n))
    # bf16 in place: out is the residual
    tr2 = tr.clone()
    y2 = linear.matmul(tx, tw, None, residual=tr2, residual_mode=mode, out=tr2)
    assert y2 is tr2
    check(f"C3 residual ({mode}) in place rows {m}", host(y2, m, n), want.float())


# --- C4: a block list of mixed dtypes with per-block scales at 32 rows ---------------------------------------------------


def test_c4_block_list(device):
    """Q [4096] K [1024] V [1024] bfloat8_b with fp32 column scales and O [4096] bf16, K = 4096, 32 rows, one launch:
    each block against the oracle and the whole output bit for bit against one call per block."""
    k, m = 4096, 32
    spec = [(4096, "bfp8", True), (1024, "bfp8", True), (1024, "bfp8", True), (4096, "bf16", False)]
    x, tx = x_input(device, m, k, 170)
    blocks, wants, c0 = [], [], 0
    for i, (n, fmt, scaled) in enumerate(spec):
        wt = O.matrix(n, k, 171 + i)
        tw = linear.native_weight(device, wt, FMT[fmt])[0]
        h = pinned_held(tw, wt, fmt, n)
        sc = uniform_scales(n, 181 + i) if scaled else None
        ts = linear.scale_tensor(device, sc, dtype=linear.float32) if scaled else None
        blocks.append((tw, c0 // 32, ts) if scaled else (tw, c0 // 32))
        wants.append((c0, n, ref64(x, h, sc)))
        c0 += n
    width = c0
    p = linear.launch_plan(tx, blocks, None)
    assert_plan(p, kernel="mfma", rows_per_pass=32, tiles=width // 32)
    y = host(linear.matmul(tx, blocks, None), m, width)
    for (b0, n, want), (_, fmt, scaled) in zip(wants, spec):
        check(f"C4 block at column {b0} ({fmt}, scales {scaled}) rows {m}", y[:, b0 : b0 + n], want.float())
    two = torch.zeros(1, 1, m, width, dtype=torch.bfloat16, device=device.torch)
    for blk in blocks:
        linear.matmul(tx, blk[0], blk[2] if len(blk) == 3 else None, out=two, col0=blk[1])
    same("C4 block list against one call per block", y, host(two, m, width))


# --- C5: fp32 top-8 records over an LM-head-sized weight, and the global top-32 -----------------------------------------


def _sorted_desc(a, axis):
    return -np.sort(-a, axis=axis)


def ids_match_with_ties(name, got_scores, want_scores, rel=1e-3):
    """got / want: float64 scores [..., k] of the chosen ids and of the best k, each sorted descending: the ids are
    exact except where a chosen id's score ties the one it displaced within rel."""
    tol = rel * np.maximum(np.abs(want_scores), 1e-30)
    bad = np.abs(got_scores - want_scores) > tol
    print(f"{'ok  ' if not bad.any() else 'FAIL'} {name}: {int(bad.sum())} of {bad.size} ranks off beyond ties",
          flush=True)
    assert not bad.any(), name


@pytest.fixture(scope="module")
def c5_case(device):
    """C5's weight (bfloat8_b [128256, 4096], its held tiles pinned against the oracle), x [4, 4096], and the float64
    logits x @ held [4, 128256]."""
    k, n, m = 4096, 128256, 4
    wt = O.matrix(n, k, 190)
    tw = linear.native_weight(device, wt, linear.bfloat8_b)[0]
    h = pinned_held(tw, wt, "bfp8", n)
    del wt
    x, tx = x_input(device, m, k, 191)
    xb = x.to(torch.bfloat16).double()
    s64 = torch.cat([xb @ h[:, c : c + 16384].double() for c in range(0, n, 16384)], dim=1).numpy()  # [m, n]
    del h
    return k, n, m, tw, tx, s64


@pytest.mark.parametrize("layout", ["per_tile", "grouped"])
def test_c5_topk_records(device, c5_case, layout):
    """x [4, 4096] against bfloat8_b W [128256, 4096]: fp32 top-8 records of every row, then the global top-32.
    "per_tile" is the bench's c5 call exactly ("slots": 0, write_y off): one record a 32-column tile, 4008 records, and
    the merge over all 4008; "grouped" the default slots (grid_slots()), tiles ranked together in groups. Record ids
    against the float64 logits of their columns (exact except ties within 1e-3 rel), record scores against the float64
    logits (rel 1e-3), the records bit for bit those of the same call with write_y on, record values rounded to bf16
    equal y at their ids, the merge against the oracle's merge of the records and its ids against the float64 global
    top-32."""
    k, n, m, tw, tx, s64 = c5_case
    kk = 8
    tiles = -(-n // 32)
    slots = 0 if layout == "per_tile" else None
    nrec = linear.topk_slots(n, slots)
    r = linear.topk_result(device, nrec, m, kk)
    spec = {"r": r, "k": kk, "rows": m, "slot0": 0, "base": 0, "n": n, "write_y": False, "fp32": True}
    if slots is not None:
        spec["slots"] = slots
    p = linear.launch_plan(tx, tw, None, topk=spec)
    assert_plan(p, kernel="mfma", rows_per_pass=16)
    per = p["tiles_per_record"]
    if layout == "per_tile":
        assert nrec == tiles == 4008 and p["records"] == 4008 and per == 1, p
    else:
        assert per > 1 and p["records"] == nrec == -(-tiles // per) and nrec <= linear.grid_slots(), p
    linear.matmul(tx, tw, None, topk=spec)
    rw = r.clone()
    r.zero_()
    y = host(linear.matmul(tx, tw, None, topk={**spec, "write_y": True}), m, n)
    same(f"C5 {layout}: records with write_y off equal those with it on", rw.cpu(), r.cpu())
    check(f"C5 y rows {m} N {n}", y, torch.from_numpy(s64).float())
    vals, ids = linear.topk_records(rw, m, kk, fp32=True)
    vals, ids = vals.numpy().reshape(m, nrec, kk), ids.numpy().reshape(m, nrec, kk)
    assert (ids >= 0).all(), "C5: every record slot is filled (each record spans at least 32 columns)"
    span = 32 * per
    lo = np.arange(nrec)[None, :, None] * span
    assert ((ids >= lo) & (ids < lo + span)).all(), "C5: a record's ids lie in its own columns"
    assert (np.diff(vals, axis=2) <= 0).all(), "C5: a record's values are ordered, highest first"
    got = np.take_along_axis(s64, ids.reshape(m, -1), axis=1).reshape(m, nrec, kk)
    pad = nrec * span - n
    sp = np.concatenate([s64, np.full((m, pad), -np.inf)], axis=1).reshape(m, nrec, span)
    want = _sorted_desc(sp, 2)[:, :, :kk]
    ids_match_with_ties(f"C5 {layout}: record ids against the float64 logits", _sorted_desc(got, 2), want)
    check(f"C5 {layout}: record scores against the float64 logits", torch.from_numpy(vals.reshape(-1)),
          torch.from_numpy(got.reshape(-1)).float(), rel=1e-3, pcc=0.999999)
    yb = y.numpy()
    at = np.take_along_axis(yb, ids.reshape(m, -1), axis=1).reshape(m, nrec, kk)
    same(f"C5 {layout}: record values rounded to bf16 equal y at their ids",
         torch.from_numpy(vals).to(torch.bfloat16).float(), torch.from_numpy(at))
    gv, gi = linear.topk_merge(rw, m, kk, k_out=32, fp32=True)
    wv, wi = O.global_topk(vals.reshape(m, -1), ids.reshape(m, -1), 32)
    same(f"C5 {layout}: global top-32 values against the oracle's merge of the records", gv.cpu(), torch.from_numpy(wv))
    same(f"C5 {layout}: global top-32 ids against the oracle's merge of the records", gi.cpu().long(),
         torch.from_numpy(wi))
    g64 = np.take_along_axis(s64, gi.cpu().numpy().astype(np.int64), axis=1)
    ids_match_with_ties(f"C5 {layout}: global top-32 ids against the float64 logits", g64, _sorted_desc(s64, 1)[:, :32])
