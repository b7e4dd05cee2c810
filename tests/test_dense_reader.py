"""The dense_reader op on the GPU against the CPU oracle (after XylolabsInc/tensix-kernels
dense_reader/tests/test_dense_reader.py, whose nine tests are mirrored here test for test, plus the packing checks the
MI355X layout needs).

Reference: x rounded to bf16 times the weight's own held values, in float64 (oracle.ref). Bars (the reference's):
relative Frobenius error below 1 % and PCC above 0.9999 for bf16 outputs, 0.1 % for the fp32 output; bit for bit where
two configurations of the op must agree (work-split knobs, repeated calls, a block list against one call per block,
the top-k records against the op's own output) and for the packing (codes, exponents, held values).
"""

import numpy as np
import pytest
import torch

from common import device as cdev
from common.testing import check, raises, same
from dense_reader import linear
from oracle import dense_oracle as O

pytestmark = pytest.mark.gpu

DTYPES = {"bfp8": linear.bfloat8_b, "bfp4": linear.bfloat4_b, "bf16": linear.bfloat16}


def x_input(device, m, k, seed):
    x = O.x_input(m, k, seed)  # randn with outlier channels 0..3 (test_dense_reader.py:28-39)
    return x, x.to(torch.bfloat16).reshape(1, 1, m, k).to(device.torch)


matrix = O.matrix


def held(tw, n):
    return linear.held(tw, n).cpu()


def host(y, m, n):
    return y.float().cpu().reshape(-1, y.shape[-1])[:m, :n]


ref = O.ref


def _special(n, k, seed):
    """[out, in] weights with zeros, a denormal, tiny values, ties and columns of very different size."""
    w = matrix(n, k, seed)
    w[::5, ::7] *= 50
    w[5, 3] = 0.0
    w[9, 7] = -1e-30
    w[1, 1] = 1e-40
    w[:16, 2] = 0.0
    w[16:24, 4] = torch.tensor([1.0, 0.5, 0.25, 0.125, 0.875, 1.875, -0.4375, 0.0625])
    return w


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4", "bf16"])
def test_pack_bitexact(device, fmt):
    n, k = 200, 160  # N padded to 256 (8 banks x 32), K to 256
    wt = _special(n, k, 30)
    tw, _ = linear.native_weight(device, wt, DTYPES[fmt])
    codes, exps = O.to_layout(wt.T.contiguous(), fmt, n_pad=tw.n_pad)
    same(f"{fmt} codes against the reference-format conversion", tw.codes.cpu(), torch.from_numpy(codes))
    if exps is not None:
        same(f"{fmt} exponents", tw.exps.cpu(), torch.from_numpy(exps))
    same(f"{fmt} held values", held(tw, n), torch.from_numpy(O.held(wt.T.contiguous(), fmt)))


def test_col_scale_pack(device):
    n, k = 96, 128
    wt = matrix(n, k, 31)
    wt[: n // 2] *= 40
    tw, ts = linear.native_weight(device, wt, linear.bfloat8_b, col_scale=True)
    c = O.bf16_ceil(wt.abs().amax(dim=1).clamp(min=1e-8))
    same("column scales", ts.float().cpu().reshape(-1), c)
    same("held values of w / c", held(tw, n), torch.from_numpy(O.held((wt / c[:, None]).T.contiguous(), "bfp8")))


def test_formats(device):
    k, n = 1024, 2048
    wt = matrix(n, k, 2)
    for fmt, dtype in DTYPES.items():
        tw, _ = linear.native_weight(device, wt, dtype)
        wk = held(tw, n)
        for m in (1, 7, 32):
            x, tx = x_input(device, m, k, 1 + m)
            check(f"{fmt} rows {m} K {k} N {n}", host(linear.matmul(tx, tw, None), m, n), ref(x, wk))


def test_scales_interleaved_prefill(device):
    k, n = 1024, 1536
    wt = matrix(n, k, 3)
    wt[: n // 2] *= 40  # columns of very different size
    tw, ts = linear.native_weight(device, wt, linear.bfloat8_b, col_scale=True)
    c = ts.float().cpu().reshape(-1)[:n]
    wk = held(tw, n)
    for m in (1, 100, 200):  # decode; prefill rows in passes
        x, tx = x_input(device, m, k, 4 + m)
        check(f"bfp8 column scales rows {m}", host(linear.matmul(tx, tw, ts), m, n), ref(x, wk, c))
    ti, _ = linear.native_weight(device, wt, linear.bfloat8_b, sharded=False)
    x, tx = x_input(device, 3, k, 5)
    check("bfp8 interleaved weight rows 3", host(linear.matmul(tx, ti, None), 3, n), ref(x, held(ti, n)))


def test_split_shares_bitwise(device):
    """The reference's work-split knobs change nothing; repeated calls are bit-identical."""
    k, n, m = 2048, 2048, 3
    x, tx = x_input(device, m, k, 6)
    tw, _ = linear.native_weight(device, matrix(n, k, 7), linear.bfloat4_b)
    base = host(linear.matmul(tx, tw, None), m, n)
    try:
        for share in (0.6, 2 / 3, 0.75):
            linear.SPLIT_SHARE = share
            same(f"split share {share:.3f} against 0.5", host(linear.matmul(tx, tw, None), m, n), base)
        linear.SPLIT_SHARE = 0.5
        same("one loader against two", host(linear.matmul(tx, tw, None, split=False), m, n), base)
        linear.REQ_TILES = 3
        same("requests of 3 tiles against one a row", host(linear.matmul(tx, tw, None), m, n), base)
    finally:
        linear.SPLIT_SHARE, linear.REQ_TILES = 0.5, 0
    for i in range(3):
        same(f"repeat {i}", host(linear.matmul(tx, tw, None), m, n), base)


def test_glu(device):
    k, n = 1024, 1024
    gate, up = matrix(n, k, 8), matrix(n, k, 9)
    tw, _ = linear.native_weight(device, linear.interleave_glu(gate, up), linear.bfloat8_b)
    tg, _ = linear.native_weight(device, gate, linear.bfloat8_b)
    tu, _ = linear.native_weight(device, up, linear.bfloat8_b)
    gk, uk = held(tg, n), held(tu, n)
    for m in (3, 20):
        x, tx = x_input(device, m, k, 10 + m)
        g, u = ref(x, gk).double(), ref(x, uk).double()
        swi = (torch.nn.functional.silu(g) * u).float()
        gel = (torch.nn.functional.gelu(g, approximate="tanh") * u).float()
        check(f"swiglu interleaved rows {m}", host(linear.linear(tx, tw, None, activation="swiglu"), m, n), swi)
        check(f"swiglu two weights rows {m}", host(linear.linear(tx, (tg, tu), None, activation="swiglu"), m, n), swi)
        check(f"geglu interleaved rows {m}", host(linear.linear(tx, tw, None, activation="geglu"), m, n), gel)
        check(f"geglu two weights rows {m}", host(linear.linear(tx, (tg, tu), None, activation="geglu"), m, n), gel)


def test_residual_out32(device):
    k, n, m = 1024, 2048, 5
    x, tx = x_input(device, m, k, 12)
    wt = matrix(n, k, 13)
    tw, _ = linear.native_weight(device, wt, linear.bfloat8_b)
    wk = held(tw, n)
    res = torch.randn(32, n, generator=torch.Generator().manual_seed(27))
    resb = res.to(torch.bfloat16)
    tr = resb.reshape(1, 1, 32, n).to(device.torch)
    want = ref(x, wk) + resb[:m].float()
    for mode in ("epilogue", "preload"):
        y = linear.matmul(tx, tw, None, residual=tr, residual_mode=mode)
        check(f"residual {mode} rows {m}", host(y, m, n), want)
    y = linear.linear(tx, tw, None, out_dtype=linear.float32, fidelity="hifi4")
    check(f"fp32 output rows {m}", host(y, m, n), ref(x, wk), rel=1e-3, pcc=0.999999)
    # in place: out is the residual itself
    tr2 = tr[:, :, :m].contiguous()
    y = linear.matmul(tx, tw, None, residual=tr2, out=tr2)
    assert y is tr2
    check(f"residual in place rows {m}", host(y, m, n), want)


def test_topk_records(device):
    k, n, rows, kk = 1024, 2048, 3, 8
    x, tx = x_input(device, 32, k, 14)
    tw, _ = linear.native_weight(device, matrix(n, k, 15), linear.bfloat4_b)
    for n_valid, base in ((n, 0), (n - 37, 1000)):
        r = linear.topk_result(device, linear.topk_slots(n), rows, kk)
        spec = {"r": r, "k": kk, "rows": rows, "slot0": 0, "base": base, "n": n_valid, "write_y": True}
        y = host(linear.matmul(tx, tw, None, topk=spec), rows, n)
        vals, idx = linear.topk_records(r, rows, kk)
        for t in range(rows):
            ok = idx[t] >= 0
            got = vals[t][ok]
            col = idx[t][ok] - base
            assert int(col.min()) >= 0 and int(col.max()) < n_valid, (col.min(), col.max())
            same(f"top-k records row {t} (n {n_valid}, base {base}): values at their ids", y[t][col], got)
            top = torch.sort(got, descending=True).values[:kk]
            same(f"top-k records row {t}: the best {kk} of the row", top, torch.topk(y[t][:n_valid], kk).values)
        # the records exactly as the oracle writes them from this output (per 32-column tile, ties to the lower id)
        words = O.tile_topk(y.numpy(), rows, kk, n_valid, base)
        same("records against the oracle's", r.cpu().reshape(-1, 2 * rows * kk), torch.from_numpy(words.view(np.int32)))


@pytest.mark.parametrize("fp32", [False, True])
def test_topk_records_grouped(device, fp32):
    """Blocks wider than the grid's records, their result sized as the reference's callers size it (a block's records
    are the grid's cores, lm_head_topk/lmhead.py:102-103): two blocks of 16384 columns into one result of
    2 x grid_slots() records at slot0 = b x grid_slots(). Each launch writes at most its slots (tiles in groups), the
    other block's slots stay untouched, every record equals the best k of the per-tile records it covers (the same
    launch with no limit) bit for bit, and bf16 records equal the oracle's ranking of the op's own output."""
    k, n, rows, kk = 1024, 16384, 3, 8
    S = linear.grid_slots()
    x, tx = x_input(device, 4, k, 90)
    r = linear.topk_result(device, 2 * S, rows, kk)
    for b in range(2):
        tw, _ = linear.native_weight(device, matrix(n, k, 91 + b), linear.bfloat8_b)
        spec = {"r": r, "k": kk, "rows": rows, "slot0": b * S, "base": b * n, "n": n, "write_y": True, "fp32": fp32}
        p = linear.launch_plan(tx, tw, None, topk=spec)
        G = p["tiles_per_record"]
        assert p["records"] == linear.topk_slots(n) <= S and G == -(-(n // 32) // S), p
        y = host(linear.matmul(tx, tw, None, topk=spec), rows, n)
        words = r.cpu().reshape(2 * S, -1)
        if b == 0:
            assert not words[S:].any(), "block 0 wrote into block 1's slots"
        one = linear.topk_result(device, n // 32, rows, kk)
        linear.matmul(tx, tw, None, topk={**spec, "r": one, "slot0": 0, "slots": 0})
        tv, ti = (t.numpy() for t in linear.topk_records(one, rows, kk, fp32=fp32))
        gv, gi = (t.numpy() for t in linear.records_host(words[b * S : b * S + p["records"]], rows, kk, fp32=fp32))
        for g in range(p["records"]):
            mv, mi = O.global_topk(tv[:, g * G * kk : (g + 1) * G * kk], ti[:, g * G * kk : (g + 1) * G * kk], kk)
            assert np.array_equal(mv, gv[:, g * kk : (g + 1) * kk]) and np.array_equal(mi, gi[:, g * kk : (g + 1) * kk]), (
                b, g, mv, gv[:, g * kk : (g + 1) * kk], mi, gi[:, g * kk : (g + 1) * kk])
        print(f"ok   block {b} (fp32 {fp32}): {p['records']} records of {G} tiles each equal the per-tile records' best "
              f"{kk}", flush=True)
        if not fp32:
            want = O.tile_topk(y.numpy(), rows, kk, n, b * n, width=32 * G)
            same(f"block {b}: grouped records against the oracle's", words[b * S : b * S + p["records"]],
                 torch.from_numpy(want.view(np.int32)))


def test_block_list_bitwise(device):
    k, m = 1024, 3
    x, tx = x_input(device, m, k, 16)
    a, _ = linear.native_weight(device, matrix(1024, k, 17), linear.bfloat8_b)
    b, _ = linear.native_weight(device, matrix(1024, k, 18), linear.bfloat8_b)
    width = 2048 + 64  # a gap of two tiles between the blocks
    one = linear.matmul(tx, [(a, 0), (b, 34)], None)
    two = torch.zeros(1, 1, m, width, dtype=torch.bfloat16, device=device.torch)
    linear.matmul(tx, a, None, out=two, col0=0)
    linear.matmul(tx, b, None, out=two, col0=34)
    ho, ht = host(one, m, width), host(two, m, width)
    same(
        "block list against one call per block",
        torch.cat([ho[:, :1024], ho[:, 1088:]], 1),
        torch.cat([ht[:, :1024], ht[:, 1088:]], 1),
    )
    g1, _ = linear.native_weight(device, matrix(512, k, 19), linear.bfloat8_b)
    u1, _ = linear.native_weight(device, matrix(512, k, 20), linear.bfloat8_b)
    g2, _ = linear.native_weight(device, matrix(512, k, 21), linear.bfloat8_b)
    u2, _ = linear.native_weight(device, matrix(512, k, 22), linear.bfloat8_b)
    for act in ("swiglu", "geglu"):
        one = linear.linear(tx, [((g1, u1), 0), ((g2, u2), 16)], None, activation=act)
        p1 = linear.linear(tx, (g1, u1), None, activation=act)
        p2 = linear.linear(tx, (g2, u2), None, activation=act)
        same(
            f"{act} block list against one call per pair",
            host(one, m, 1024),
            torch.cat([host(p1, m, 512), host(p2, m, 512)], 1),
        )


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4", "bf16"])
def test_narrow_tiles_bitwise(device, fmt):
    """A launch of few 32-column tiles runs 16-column tiles (one panel a workgroup, so that every CU streams); the same
    columns inside a launch of enough tiles for 32-column tiles (a block list whose second block brings the launch to
    1.75 tiles a CU) are the same bit for bit, with fp32 scales and a split K. launch_plan names the width each runs."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    wide_tiles = 7 * cus // 4  # 448 on 256 CUs: two 32-column tiles a CU at most, the same as four halves
    for k in (2048, 9216):
        n = 1000
        tw, _ = linear.native_weight(device, matrix(n, k, 80), DTYPES[fmt])
        big, _ = linear.native_weight(device, matrix(32 * (wide_tiles - 32), k, 81), DTYPES[fmt])
        sc = linear.scale_tensor(device, torch.rand(n, generator=torch.Generator().manual_seed(82)) + 0.5,
                                 dtype=linear.float32)
        for m in (1, 2):
            x, tx = x_input(device, m, k, 83 + m)
            narrow = linear.launch_plan(tx, tw, sc)
            wide = linear.launch_plan(tx, [(tw, 0, sc), (big, 32)], None)
            assert narrow["tile_cols"] == 16 and wide["tile_cols"] == 32, (narrow, wide)
            assert narrow["kernel"] == wide["kernel"] == "gemv" and wide["tiles"] == wide_tiles, (narrow, wide)
            alone = host(linear.matmul(tx, tw, sc), m, n)
            check(f"{fmt} K {k} rows {m} narrow tiles", alone, ref(x, held(tw, n)) * sc.float().cpu().reshape(1, -1))
            both = linear.matmul(tx, [(tw, 0, sc), (big, 32)], None)
            same(f"{fmt} K {k} rows {m} 16-column tiles against 32-column tiles", host(both, m, n), alone)


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4", "bf16"])
def test_rows32_staged_x(device, fmt):
    """Launches of 17 to 32 rows read x through LDS (buffer loads straight to LDS, a swizzled layout, rows past x
    outside the buffer). Every output row is its own MFMA row, accumulated in an order that depends on K and the rows a
    pass only, so permuting x's rows permutes y's bit for bit: the rows staged in each half of the tile and in each
    swizzle position land where they belong. At a ragged K (the last step's columns past K masked, the last row's past
    the buffer), a row count that leaves rows past x, and a K of 256-K chunks (16 wavefronts); against the oracle."""
    n = 320
    for k in (800, 4096, 4352):
        wt = _special(n, k, 90)
        tw, _ = linear.native_weight(device, wt, DTYPES[fmt])
        wk = held(tw, n)
        for m in (19, 32):
            x, tx = x_input(device, m, k, 91 + m)
            assert linear.launch_plan(tx, tw, None)["rows_per_pass"] == 32
            y = host(linear.matmul(tx, tw, None), m, n)
            check(f"{fmt} K {k} rows {m}", y, ref(x, wk))
            perm = torch.cat([torch.arange(m - 1, 15, -1), torch.arange(16)[torch.randperm(16, generator=torch.Generator().manual_seed(m))]])
            yp = host(linear.matmul(tx[..., perm.to(tx.device), :].contiguous(), tw, None), m, n)
            same(f"{fmt} K {k} rows {m}: rows permuted", yp, y[perm])


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4", "bf16"])
def test_mfma_narrow_tiles_bitwise(device, fmt):
    """An unsplit MFMA launch of few tiles runs 16-column tiles (`launch_plan` says which): a weight of 96 tiles alone
    (16-column) against the same weight in a block list of 256 tiles (32-column), bit for bit, at 8 and 32 rows."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    k = 2048
    wa, wb = matrix(96 * 32, k, 150), matrix(max(160, cus - 96 + 1) * 32, k, 151)
    ta, _ = linear.native_weight(device, wa, DTYPES[fmt])
    tb, _ = linear.native_weight(device, wb, DTYPES[fmt])
    na, nb = wa.shape[0], wb.shape[0]
    for m in (8, 32):
        x, tx = x_input(device, m, k, 152 + m)
        assert linear.launch_plan(tx, ta, None)["tile_cols"] == (16 if 2 * 96 <= cus else 32)
        assert linear.launch_plan(tx, [(ta, 0), (tb, 96)], None)["tile_cols"] == 32
        one = host(linear.matmul(tx, ta, None), m, na)
        check(f"{fmt} rows {m}: 96 tiles alone", one, ref(x, held(ta, na)))
        both = host(linear.matmul(tx, [(ta, 0), (tb, 96)], None), m, na + nb)
        same(f"{fmt} rows {m}: 16-column tiles against the 32-column block list", both[:, :na], one)


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4", "bf16"])
def test_rows_in_passes_bitwise(device, fmt):
    """Past 32 rows the launch runs passes of 32 (a last pass of at most 16 rows on the 16-row kernel): each pass's rows
    equal bit for bit those of a call on those rows alone. A row's sums do not depend on the call's other rows within
    one kernel: 32 rows against calls of 20 (17-32 rows: the 32-row kernel), 16 against calls of 5 (3-16 rows: the
    16-row kernel). (The two kernels visit a chunk's k in different orders, so across them a row agrees to rounding.)
    At 300 tiles (the 32-row passes take tile pairs) and at a K split over workgroups."""
    for k, n in ((1024, 9600), (9216, 320)):
        wt = matrix(n, k, 130)
        tw, _ = linear.native_weight(device, wt, DTYPES[fmt])
        wk = held(tw, n)
        for m in (40, 45, 70):
            x, tx = x_input(device, m, k, 131 + m)
            y = host(linear.matmul(tx, tw, None), m, n)
            check(f"{fmt} K {k} N {n} rows {m}", y, ref(x, wk))
            for r0 in range(0, m, 32):
                r1 = min(r0 + 32, m)
                one = host(linear.matmul(tx[..., r0:r1, :].contiguous(), tw, None), r1 - r0, n)
                same(f"{fmt} K {k} N {n} rows {m}: rows {r0}-{r1 - 1} against a call on them alone", y[r0:r1], one)
        x, tx = x_input(device, 32, k, 140)
        y32 = host(linear.matmul(tx, tw, None), 32, n)
        for r0, r1 in ((0, 20), (12, 32)):
            yr = host(linear.matmul(tx[..., r0:r1, :].contiguous(), tw, None), r1 - r0, n)
            same(f"{fmt} K {k} N {n}: 32 rows against a call of rows {r0}-{r1 - 1}", y32[r0:r1], yr)
        y16 = host(linear.matmul(tx[..., :16, :].contiguous(), tw, None), 16, n)
        check(f"{fmt} K {k} N {n}: 16 rows (the 16-row kernel) against the oracle", y16, ref(x[:16], wk))
        for r0, r1 in ((0, 5), (11, 16)):
            yr = host(linear.matmul(tx[..., r0:r1, :].contiguous(), tw, None), r1 - r0, n)
            same(f"{fmt} K {k} N {n}: 16 rows against a call of rows {r0}-{r1 - 1}", y16[r0:r1], yr)


@pytest.mark.parametrize("k", [768, 800, 3328])
def test_rows32_tile_pairs(device, k):
    """A 32-row launch of more tiles than CUs runs its block-float segments' tiles in pairs, a workgroup each (the
    last of an odd count alone), and its bf16 segments' one a workgroup: a block list of bfloat8_b (129 tiles, odd),
    bf16 (64) and bfloat4_b (65, odd), 258 tiles, equals one call per block bit for bit (each alone has fewer tiles
    than CUs: no pairs), with scales on the first block and 19 rows (rows past x), and the oracle; K a whole number of
    the pairs' 64-k steps, and not (800: the last step half past K); 3328: 512-k chunks visited rotated, the last
    one a single 256-k exponent group."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    m = 19
    spec = [("bfp8", 129), ("bf16", 64), ("bfp4", 65)]
    extra = max(0, cus + 2 - sum(t for _, t in spec))  # (more tiles than this box's CUs)
    spec[1] = ("bf16", spec[1][1] + extra)
    x, tx = x_input(device, m, k, 120)
    blocks, col0, parts = [], 0, []
    sc = linear.scale_tensor(device, torch.rand(32 * spec[0][1], generator=torch.Generator().manual_seed(121)) + 0.5,
                             dtype=linear.float32)
    for i, (fmt, tiles) in enumerate(spec):
        n = 32 * tiles
        wt = matrix(n, k, 122 + i)
        tw, _ = linear.native_weight(device, wt, DTYPES[fmt])
        blocks.append((tw, col0 // 32, sc) if i == 0 else (tw, col0 // 32))
        parts.append((tw, n, col0, sc if i == 0 else None))
        col0 += n
    p = linear.launch_plan(tx, blocks, None)
    assert (p["kernel"], p["rows_per_pass"], p["tiles_per_workgroup"]) == ("mfma", 32, 2), p
    assert p["workgroups"] == 65 + spec[1][1] + 33, p
    y = host(linear.matmul(tx, blocks, None), m, col0)
    for tw, n, c0, s in parts:
        assert linear.launch_plan(tx, tw, s)["tiles_per_workgroup"] == 1
        alone = host(linear.matmul(tx, tw, s), m, n)
        same(f"{tw.dtype} block of {n} columns against its own call", y[:, c0 : c0 + n], alone)
        want = ref(x, held(tw, n))
        if s is not None:
            want = want * s.float().cpu().reshape(1, -1)
        check(f"{tw.dtype} block of {n} columns", alone, want)


def _edge_weights(k, exps, seed, every=1):
    """[16 len(exps), k] weights at the ends of the shared-exponent range: in panel p (16 columns), at every `every`-th
    k, the face row's 16 values are (1 + u) 2^(E - 127), u in [0, 1), random signs, E = exps[p] (the face row's shared
    exponent); the other k hold N(0, 0.02). Column 3 at k = 1 is a denormal input (it rounds to zero)."""
    n = 16 * len(exps)
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(n, k, generator=g) * 0.02
    sel = torch.arange(0, k, every)
    e = torch.tensor(exps, dtype=torch.float64).repeat_interleave(16)
    mag = (1 + torch.rand(n, len(sel), generator=g, dtype=torch.float64)) * torch.exp2(e - 127)[:, None]
    sign = torch.where(torch.rand(n, len(sel), generator=g) < 0.5, -1.0, 1.0).double()
    w[:, sel] = (mag * sign).float()
    w[3, 1] = 1e-40
    return w, sel


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4"])
@pytest.mark.parametrize("edge,k", [("low", 1024), ("low", 4096), ("high", 1024), ("mixed", 4096)])
def test_exponent_edges(device, fmt, edge, k):
    """The exponent folding at the ends of the exponent range (moe8.py:147-149's zero / denormal rule): panels whose
    face rows all have shared exponent E = 1 .. 10 (x 2^(E - bias) would be an fp32 / bf16 denormal for the smallest),
    or E = 245 .. 250 at every 128th k (x there +-1.5, so that the float64 result stays finite in fp32), or ("mixed")
    E = 1 .. 10 at every k but the 64th, which holds N(0, 0.02) face rows (normal exponents in every chunk), through the
    GEMV (rows 1, 2; 256-k chunks at K = 1024, 512-k chunks at K = 4096) and the MFMA decode (rows 3, 32), panel by
    panel against x @ held in float64, every panel at the 1 % / PCC 0.9999 bar."""
    if edge == "low":
        exps = [1, 2, 3, 4, 5, 6, 8, 10]
        wt, sel = _edge_weights(k, exps, 300)
    elif edge == "mixed":
        exps = [1, 2, 3, 4, 5, 6, 8, 10]
        wt, sel = _edge_weights(k, exps, 303)
        normal = torch.arange(0, k, 64)
        wt[:, normal] = torch.randn(wt.shape[0], len(normal), generator=torch.Generator().manual_seed(304)) * 0.02
    else:
        exps = [245, 246, 247, 248, 249, 250]
        wt, sel = _edge_weights(k, exps, 301, every=128)
    n = wt.shape[0]
    tw, _ = linear.native_weight(device, wt, DTYPES[fmt])
    wk = held(tw, n)
    same(f"{fmt} {edge} exponents: held values against the oracle", wk, torch.from_numpy(O.held(wt.T.contiguous(), fmt)))
    assert bool(torch.isfinite(wk).all())
    for m in (1, 2, 3, 32):
        x = O.x_input(m, k, 302 + m)
        if edge == "high":
            x[:, sel] = torch.where(x[:, sel] < 0, -1.5, 1.5)
        tx = x.to(torch.bfloat16).reshape(1, 1, m, k).to(device.torch)
        y = host(linear.matmul(tx, tw, None), m, n)
        want = ref(x, wk)
        for p, e in enumerate(exps):
            c = slice(16 * p, 16 * p + 16)
            check(f"{fmt} K {k} rows {m} panel {p} shared exponent {e}", y[:, c], want[:, c])


def test_max_banks(device):
    k, n, m = 1024, 1024, 2
    banks = cdev.dram_banks(device)
    fewer = max(1, banks // 2)
    x, tx = x_input(device, m, k, 23)
    wt = matrix(n, k, 24)
    tw, _ = linear.native_weight(device, wt, linear.bfloat8_b, max_banks=fewer)
    assert tw.memory_config().banks == fewer
    check(f"weight over {fewer} of {banks} banks", host(linear.matmul(tx, tw, None), m, n), ref(x, held(tw, n)))
    full, _ = linear.native_weight(device, wt, linear.bfloat8_b)
    if banks > fewer:
        raises(
            f"a weight over {banks} banks with max_banks {fewer}",
            ValueError,
            lambda: linear.matmul(tx, full, None, max_banks=fewer),
        )


def test_linear_rank3(device):
    k, n, m = 1024, 1024, 4
    x, tx = x_input(device, m, k, 25)
    wt = matrix(n, k, 26)
    tw, _ = linear.native_weight(device, wt, linear.bfloat8_b)
    x3 = tx.reshape(1, m, k)
    y = linear.linear(x3, tw, None, activation="silu")
    assert list(y.shape) == [1, m, n], y.shape
    want = torch.nn.functional.silu(ref(x, held(tw, n)).double()).float()
    check(f"linear rank 3 with silu rows {m}", y.float().cpu().reshape(m, n), want)


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4", "bf16"])
def test_rows_each_pass_width(device, fmt):
    """Every rows-per-pass width (1, 2, 4, 8 and passes of 8) of every format, on a K that is not a multiple of the
    k-block (the padded values must not enter)."""
    k, n = 800, 320
    wt = _special(n, k, 40)
    tw, _ = linear.native_weight(device, wt, DTYPES[fmt])
    wk = held(tw, n)
    for m in (1, 2, 3, 5, 8, 13):
        x, tx = x_input(device, m, k, 50 + m)
        check(f"{fmt} K {k} rows {m}", host(linear.matmul(tx, tw, None), m, n), ref(x, wk))


def test_topk_merge(device):
    k, n, rows, kk = 512, 4096, 4, 8
    x, tx = x_input(device, 4, k, 60)
    tw, _ = linear.native_weight(device, matrix(n, k, 61), linear.bfloat8_b)
    for fp32 in (False, True):
        r = linear.topk_result(device, linear.topk_slots(n), rows, kk)
        spec = {"r": r, "k": kk, "rows": rows, "slot0": 0, "base": 0, "n": n, "write_y": True, "fp32": fp32}
        y = linear.matmul(tx, tw, None, topk=spec)
        vals, ids = linear.topk_merge(r, rows, kk, k_out=32, fp32=fp32)
        hv, hi = linear.topk_records(r, rows, kk, fp32=fp32)
        wv, wi = O.global_topk(hv.numpy(), hi.numpy(), 32)
        same(f"global top-32 values (fp32 {fp32})", vals.cpu(), torch.from_numpy(wv))
        same(f"global top-32 ids (fp32 {fp32})", ids.cpu().long(), torch.from_numpy(wi))
        if not fp32:
            yv = host(y, rows, n)
            same("global top-32 against torch.topk of y", vals.cpu(), torch.topk(yv, 32, dim=1).values)


def _records(nrec, rows, k, fp32, seed, values):
    """Synthetic top-k records [nrec, 2 * rows * k] int32: per record and row, k slots drawn from `values` (many
    ties), some empty; ids unique."""
    rng = np.random.default_rng(seed)
    v = rng.choice(values, size=(nrec, rows, k)).astype(np.float32)
    ids = (np.arange(nrec * rows * k, dtype=np.int64).reshape(nrec, rows, k) * 7919) % (1 << 30)
    empty = rng.random((nrec, rows, k)) < 0.2
    if fp32:
        keys = v.view(np.uint32).astype(np.int64)
        keys[empty] = 0xFF800000
    else:
        keys = O.key_bf16(O.bf16_bits(torch.from_numpy(v)))
        keys[empty] = 0
    ids = np.where(empty, 0xFFFFFFFF, ids)
    words = np.concatenate([keys.reshape(nrec, rows * k), ids.reshape(nrec, rows * k)], axis=1)
    return torch.from_numpy((words & 0xFFFFFFFF).astype(np.uint32).view(np.int32))


@pytest.mark.parametrize("fp32", [False, True])
def test_topk_merge_synthetic(device, fp32):
    """dr_topk_merge against the oracle's host merge on records with heavy ties, empty slots, negative values, rows
    with fewer valid candidates than k_out, k_out 64, and an LM-head-sized record count."""
    ties = np.array([-3.0, -1.0, -0.5, 0.0, 0.25, 0.5, 1.0, 2.0, 2.5, 3.0], np.float32)
    for nrec, rows, k, k_out, values in (
        (4008, 4, 8, 32, ties),
        (4008, 4, 8, 64, np.random.default_rng(5).standard_normal(4000).astype(np.float32)),
        (3, 2, 4, 32, ties),  # at most 24 valid of 32 asked
        (517, 32, 1, 16, ties),
        (300, 3, 5, 32, ties),  # k not a multiple of 4: the element-wise loads
        (700, 2, 16, 64, np.random.default_rng(7).standard_normal(3000).astype(np.float32)),
        (1, 1, 32, 64, ties),
        (16384, 1, 4, 64, np.random.default_rng(6).standard_normal(9000).astype(np.float32)),  # the most records
        (4100, 1, 5, 32, ties),  # 21 slices (an odd count: a pair register half empty)
        (2600, 2, 8, 33, np.random.default_rng(8).standard_normal(5000).astype(np.float32)),  # 33: the 64-wide lists
        (5000, 1, 9, 1, ties),  # 44 slices, the single best
        (1200, 3, 7, 31, ties),  # 9 slices
    ):
        t = _records(nrec, rows, k, fp32, nrec + rows, values)
        hv, hi = linear.records_host(t, rows, k, fp32=fp32)
        wv, wi = O.global_topk(hv.numpy(), hi.numpy(), k_out)
        r = t.reshape(1, 1, nrec, -1).to(device.torch)
        vals, ids = linear.topk_merge(r, rows, k, k_out=k_out, fp32=fp32)
        same(f"merge values nrec {nrec} rows {rows} k {k} k_out {k_out}", vals.cpu(), torch.from_numpy(wv))
        same(f"merge ids nrec {nrec} rows {rows} k {k} k_out {k_out}", ids.cpu().long(), torch.from_numpy(wi))


def test_topk_merge_ordered(device):
    """Records whose values rise or fall with the slot (the best all in the first or last loads of a slice, or in a
    few lanes of a load), so a wavefront's early threshold comes from the fewest lanes possible: against the oracle's
    host merge."""
    nrec, rows, k = 4008, 2, 8
    base = np.arange(nrec * k, dtype=np.float32) / 64.0
    for name, v in (("rising", base), ("falling", base[::-1].copy()),
                    ("a few lanes", np.where(np.arange(nrec * k) % 64 < 3, base, -base))):
        vals = np.stack([v, v[::-1]], axis=1).reshape(nrec, k, rows).transpose(0, 2, 1)  # [nrec, rows, k]
        ids = (np.arange(nrec * rows * k, dtype=np.int64).reshape(nrec, rows, k) * 7919) % (1 << 30)
        for fp32 in (False, True):
            if fp32:
                keys = vals.astype(np.float32).view(np.uint32).astype(np.int64)
            else:
                keys = O.key_bf16(O.bf16_bits(torch.from_numpy(np.ascontiguousarray(vals, np.float32))))
            words = np.concatenate([keys.reshape(nrec, rows * k), ids.reshape(nrec, rows * k)], axis=1)
            t = torch.from_numpy((words & 0xFFFFFFFF).astype(np.uint32).view(np.int32))
            hv, hi = linear.records_host(t, rows, k, fp32=fp32)
            r = t.reshape(1, 1, nrec, -1).to(device.torch)
            for k_out in (32, 64):
                wv, wi = O.global_topk(hv.numpy(), hi.numpy(), k_out)
                gv, gi = linear.topk_merge(r, rows, k, k_out=k_out, fp32=fp32)
                same(f"merge values {name} fp32 {fp32} k_out {k_out}", gv.cpu(), torch.from_numpy(wv))
                same(f"merge ids {name} fp32 {fp32} k_out {k_out}", gi.cpu().long(), torch.from_numpy(wi))


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4", "bf16"])
def test_split_k(device, fmt):
    """A K long enough to be split over several workgroups a tile (they meet in the workspace): against the oracle,
    repeated calls bit-identical, a block list bit-identical to one call per block."""
    n = 320
    for k in (9216, 14336):
        wt = matrix(n, k, 70)
        tw, _ = linear.native_weight(device, wt, DTYPES[fmt])
        tb, _ = linear.native_weight(device, matrix(256, k, 71), DTYPES[fmt])
        wk = held(tw, n)
        for m in (1, 3, 8):
            x, tx = x_input(device, m, k, 72 + m)
            y = linear.matmul(tx, tw, None)
            check(f"{fmt} K {k} rows {m} (split K)", host(y, m, n), ref(x, wk))
            same(f"{fmt} K {k} rows {m} repeated", host(linear.matmul(tx, tw, None), m, n), host(y, m, n))
            one = linear.matmul(tx, [(tw, 0), (tb, 12)], None)
            two = torch.zeros(1, 1, m, 12 * 32 + 256, dtype=torch.bfloat16, device=device.torch)
            linear.matmul(tx, tw, None, out=two, col0=0)
            linear.matmul(tx, tb, None, out=two, col0=12)
            same(f"{fmt} K {k} rows {m} block list (split K)", host(one, m, 12 * 32 + 256)[:, :n],
                 host(two, m, 12 * 32 + 256)[:, :n])
            same(f"{fmt} K {k} rows {m} block list second block", host(one, m, 640)[:, 384:], host(two, m, 640)[:, 384:])


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4", "bf16"])
def test_long_k(device, fmt):
    """K far past the configs' (a 70B-class FFN down's 28672, and 53280, ragged, split over seven workgroups a tile),
    every kernel that serves it (GEMV 1-2 rows, MFMA 8 and 32 rows, 40 rows in two passes): against the oracle, repeated
    calls bit-identical, a block list (up to 32 rows) bit-identical to one call per block."""
    n = 96
    for k in (28672, 53280):
        wt = matrix(n, k, 95)
        tw, _ = linear.native_weight(device, wt, DTYPES[fmt])
        tb, _ = linear.native_weight(device, matrix(64, k, 96), DTYPES[fmt])
        wk = held(tw, n)
        for m in (1, 2, 8, 32, 40):
            x, tx = x_input(device, m, k, 97 + m)
            p = linear.launch_plan(tx, tw, None)
            assert p["splits"] > 1, p
            y = linear.matmul(tx, tw, None)
            check(f"{fmt} K {k} rows {m} ({p['splits']} splits)", host(y, m, n), ref(x, wk))
            same(f"{fmt} K {k} rows {m} repeated", host(linear.matmul(tx, tw, None), m, n), host(y, m, n))
            if m > 32:
                continue  # (a block list is a decode call: up to 32 rows)
            one = linear.matmul(tx, [(tw, 0), (tb, 3)], None)
            two = torch.zeros(1, 1, m, n + 64, dtype=torch.bfloat16, device=device.torch)
            linear.matmul(tx, tw, None, out=two, col0=0)
            linear.matmul(tx, tb, None, out=two, col0=3)
            same(f"{fmt} K {k} rows {m} block list", host(one, m, n + 64), host(two, m, n + 64))


def test_split_k_shapes_share_workspace(device):
    """Split-K launches of any shape share one workspace: many tiles after few (with counters placed by the tile count,
    the second launch's would lie where the first one's partial sums were), and back, each against the oracle."""
    k = 9216
    for n in (320, 4096, 320):
        wt = matrix(n, k, 90 + n % 7)
        tw, _ = linear.native_weight(device, wt, linear.bfloat8_b)
        for m in (1, 3):
            x, tx = x_input(device, m, k, 91 + m)
            y = linear.matmul(tx, tw, None)
            check(f"split K N {n} rows {m} after other shapes", host(y, m, n), ref(x, held(tw, n)))


def test_pack_cache(device, tmp_path):
    """native_weight_cached: the first call packs and writes the cache, the second reads it back; the weights are
    byte for byte the same and the matmul bit for bit; another weight's call is refused until rebuild."""
    from dense_reader import pack_cache as pc

    k, n = 512, 320
    for fmt, cs in (("bfp8", False), ("bfp4", True), ("bf16", False)):
        wt = matrix(n, k, 80)
        path = tmp_path / f"w_{fmt}"
        w1, s1 = pc.native_weight_cached(device, wt, DTYPES[fmt], path, col_scale=cs)
        w2, s2 = pc.native_weight_cached(device, wt, DTYPES[fmt], path, col_scale=cs)
        same(f"pack cache {fmt}: codes", w2.codes.cpu(), w1.codes.cpu())
        if w1.exps is not None:
            same(f"pack cache {fmt}: exponents", w2.exps.cpu(), w1.exps.cpu())
        same(f"pack cache {fmt}: scales", s2.cpu(), s1.cpu())
        x, tx = x_input(device, 2, k, 81)
        same(f"pack cache {fmt}: matmul", linear.matmul(tx, w2, s2).cpu(), linear.matmul(tx, w1, s1).cpu())
        with pytest.raises(pc.PackCacheMismatch):
            pc.native_weight_cached(device, matrix(n, k, 82), DTYPES[fmt], path, col_scale=cs)
        w3, _ = pc.native_weight_cached(device, matrix(n, k, 82), DTYPES[fmt], path, col_scale=cs, rebuild=True)
        w4, _ = pc.native_weight_cached(device, matrix(n, k, 82), DTYPES[fmt], path, col_scale=cs)
        same(f"pack cache {fmt}: rebuilt", w4.codes.cpu(), w3.codes.cpu())
