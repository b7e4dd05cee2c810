"""The CPU oracle pinned before it is trusted (CPU only).

- bfp_round against hand-derived face rows (tests/golden/bfp_face_rows.json): ties to even, no sticky bit, the
  magnitude clamp, zero and denormal inputs, the dropped sign of a zero magnitude.
- held (bfp_tiles -> tile_values) against held_exact, an exact-rational restatement (Fractions, Python's round half to
  even on the block grid), on random and special inputs, for bfloat4_b and bfloat8_b.
- held is idempotent (values on the grid pack to themselves), odd (held(-w) = -held(w)) and scales by powers of two.
- the top-k key codec is monotone over every non-NaN bf16 pattern and its decode is its inverse.
- to_layout (the GPU layout built from the reference tiles) decodes element by element, with the per-element address
  of the layout, back to held.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import dense_oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"


def _row(case):
    return np.array([int(h, 16) for h in case["row"]], np.uint32).view(np.float32)


@pytest.mark.parametrize("i", range(len(O.load_golden(GOLDEN / "bfp_face_rows.json")["cases"])))
def test_golden_face_rows(i):
    case = O.load_golden(GOLDEN / "bfp_face_rows.json")["cases"][i]
    shared, sm = O.bfp_round(_row(case)[None, :], O.MANT_BITS[case["fmt"]])
    assert int(shared[0, 0]) == case["shared"], (case["why"], shared)
    assert sm[0].tolist() == case["m"], (case["why"], sm[0].tolist())


def _special(k, n, seed):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(k, n, generator=g) * 0.02
    w[::7, ::5] *= 50  # rows of very different size
    w[3, 5] = 0.0
    w[7, 9] = -1e-30
    w[1, 1] = 1e-40  # denormal
    w[2, :16] = 0.0  # an all-zero face row
    a = w.numpy()
    a[4, 16:32] = np.array([1.0, 0.5, 0.25, 0.125, 0.875, 1.875, -0.4375, 0.0625] * 2, np.float32)  # ties and clamp
    a[5, 0:16] = np.array([1.0, 2**-7, 3 * 2**-8, -(2**-7), 255 / 128] + [0.0] * 11, np.float32)
    return torch.from_numpy(a)


@pytest.mark.parametrize("fmt", ["bfp4", "bfp8"])
@pytest.mark.parametrize("seed", [0, 1])
def test_held_against_exact_rationals(fmt, seed):
    w = _special(32, 64, seed)
    got = O.held(w, fmt).astype(np.float64)
    want = O.held_exact(w.numpy(), fmt)
    assert np.array_equal(got, want), np.argwhere(got != want)[:5]


@pytest.mark.parametrize("fmt", ["bfp4", "bfp8", "bf16"])
def test_held_properties(fmt):
    w = _special(64, 96, 3)
    h = O.held(w, fmt)
    assert np.array_equal(O.held(h, fmt), h), "values on the grid pack to themselves"
    assert np.array_equal(O.held(-w, fmt), -h + 0.0), "odd"
    wn = w.clone()
    wn[1, 1] = 0.0  # (a bf16 denormal sits on a fixed grid: scaling is exact for normal values only)
    assert np.array_equal(O.held(wn * 8, fmt), O.held(wn, fmt) * 8), "a power of two moves the exponents only"
    if fmt != "bf16":
        # every value is within half a grid step of its face row's grid (or clamped at the top)
        f = O._face_rows(w.numpy())
        shared, _ = O.bfp_round(f, O.MANT_BITS[fmt])
        step = np.ldexp(1.0, shared.astype(np.int64) - O.BIAS[fmt])
        hv = O._face_rows(h)
        err = np.abs(hv - f) / step
        top = (1 << O.MANT_BITS[fmt]) - 1
        ok = (err <= 0.5 + 1e-9) | (np.abs(hv) / step == top) | (f == 0)
        assert ok.all()


def test_bf16_matches_torch():
    w = _special(32, 32, 4)
    assert np.array_equal(O.held(w, "bf16"), w.to(torch.bfloat16).float().numpy())


def test_key_codec_exhaustive():
    bits = np.arange(65536, dtype=np.uint32)
    vals = O.bf16_values(bits)
    ok = ~np.isnan(vals)
    keys = O.key_bf16(bits)
    # monotone: sorting by value sorts by key (both zeros map to adjacent keys, -0 below +0)
    order = np.lexsort((np.signbit(vals[ok]) == 0, vals[ok]))
    assert np.all(np.diff(keys[ok][order]) > 0)
    assert np.array_equal(O.key_value(keys[ok]), vals[ok])
    assert O.key_bf16(0x0000) == 0x8000 and O.key_bf16(0x8000) == 0x7FFF and O.key_bf16(0x7F80) == 0xFF80
    assert np.all(keys[ok] != 0), "0 is the empty key"


def test_tile_topk_round_trip():
    g = torch.Generator().manual_seed(5)
    y = torch.randn(3, 80, generator=g).to(torch.bfloat16).float().numpy()
    y[0, 3] = y[0, 9]  # a tie inside a tile
    words = O.tile_topk(y, rows=3, k=4, n_valid=75, base=1000)
    vals, ids = O.records_decode(words, 3, 4)
    for r in range(3):
        ok = ids[r] >= 0
        cols = ids[r][ok] - 1000
        assert np.array_equal(vals[r][ok], y[r, cols])
        assert cols.max() < 75
        top = np.sort(vals[r][ok])[::-1][:4]
        assert np.array_equal(top, np.sort(y[r, :75])[::-1][:4])
    # the tie: both columns 3 and 9 of row 0 share a value; the lower column ranks first
    gv, gi = O.global_topk(vals, ids, 8)
    assert np.all(np.diff(gv, axis=1) <= 0)


def test_tile_topk_groups():
    """A record of a group of tiles (width 96: three tiles) is the best k of the group's columns by brute force, and
    the best k of the three tile records it covers (the selection decomposes: highest first, ties to the lower id)."""
    g = torch.Generator().manual_seed(6)
    y = torch.randn(2, 200, generator=g).to(torch.bfloat16).float().numpy()
    y[1, 10] = y[1, 40] = y[1, 70] = 5.0  # a three-way tie across the three tiles of group 0
    n_valid = 190
    grouped = O.tile_topk(y, rows=2, k=5, n_valid=n_valid, base=7, width=96)
    tiles = O.tile_topk(y, rows=2, k=5, n_valid=n_valid, base=7)
    gv, gi = O.records_decode(grouped, 2, 5)
    tv, ti = O.records_decode(tiles, 2, 5)
    assert grouped.shape[0] == 3 and tiles.shape[0] == 7
    for rec in range(3):
        for r in range(2):
            cols = [c for c in range(96 * rec, min(96 * rec + 96, 200)) if c < n_valid]
            want = sorted(cols, key=lambda c: (-float(y[r, c]), c))[:5]
            got = gi[r, 5 * rec : 5 * rec + 5]
            assert [int(i) - 7 for i in got[got >= 0]] == want, (rec, r)
        lo, hi = 5 * 3 * rec, 5 * min(3 * rec + 3, 7)
        mv, mi = O.global_topk(tv[:, lo:hi], ti[:, lo:hi], 5)
        assert np.array_equal(mv, gv[:, 5 * rec : 5 * rec + 5]) and np.array_equal(mi, gi[:, 5 * rec : 5 * rec + 5])
    assert list(gi[1, :3]) == [7 + 10, 7 + 40, 7 + 70]  # the tie: lower ids first


def _eo(fmt, k):
    """Exponent byte of k within a panel, from the layout's statement: groups of 256 k, lane l's four exponents at
    bytes 4 l .. 4 l + 3, lane l making x' for (bfp8) k = 64 j + l, (bfp4) the pair 128 j' + 32 kq + 2 i (+1)."""
    g, r = divmod(k, 256)
    if fmt == "bfp8":
        j, lane = divmod(r, 64)
        return g * 256 + 4 * lane + j
    jp, r = divmod(r, 128)
    kq, r = divmod(r, 32)
    i, h = divmod(r, 2)
    return g * 256 + 4 * (16 * kq + i) + 2 * jp + h


def test_exponent_layout_is_a_permutation():
    for fmt in ("bfp8", "bfp4"):
        offs = sorted(O.exp_off(fmt, k) for k in range(512))
        assert offs == list(range(512))
        assert all(O.exp_off(fmt, k) == _eo(fmt, k) for k in range(512))


def _unlayout(codes, exps, fmt, k, n, n_pad):
    """Decode the library layout element by element with its address formula (independent of to_layout's
    reshapes)."""
    k_pad = -(-k // O.KALIGN) * O.KALIGN
    nkb = k_pad // O.KBLK[fmt]
    out = np.zeros((k, n), np.float32)
    for kk in range(k):
        for c in range(n):
            p, cc = divmod(c, 16)
            base = p * nkb * 1024
            if fmt == "bfp8":
                b, r = divmod(kk, 64)
                kq, i = divmod(r, 16)
                m = int(np.int8(codes[base + b * 1024 + (kq * 16 + cc) * 16 + i]))
                out[kk, c] = np.ldexp(np.float32(m), int(exps[p * k_pad + _eo('bfp8', kk)]) - 133)
            elif fmt == "bfp4":
                b, r = divmod(kk, 128)
                kq, r2 = divmod(r, 32)
                d, j = divmod(r2, 8)
                byte = int(codes[base + b * 1024 + (kq * 16 + cc) * 16 + d * 4 + (j & 3)])
                u = (byte if j < 4 else byte >> 4) & 15
                out[kk, c] = np.ldexp(np.float32(u - 8), int(exps[p * k_pad + _eo('bfp4', kk)]) - 129)
            else:
                b, r = divmod(kk, 32)
                kq, i = divmod(r, 8)
                o = base + b * 1024 + (kq * 16 + cc) * 16 + 2 * i
                h = int(codes[o]) | (int(codes[o + 1]) << 8)
                out[kk, c] = O.bf16_values(np.array([h], np.uint32))[0]
    return out


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4", "bf16"])
def test_layout_decodes_to_held(fmt):
    k, n = 288, 48  # K padded to 512, N to 64
    w = _special(k, n, 6)
    codes, exps = O.to_layout(w, fmt, n_pad=64)
    assert codes.size * {"bfp8": 1, "bfp4": 2, "bf16": 0.5}[fmt] == 512 * 64
    got = _unlayout(codes, exps, fmt, k, n, 64)
    assert np.array_equal(got, O.held(w, fmt))


def test_ref_closed_forms():
    x = torch.tensor([[1.0, 2.0, -3.0]])
    w = torch.eye(3, dtype=torch.float32) * 2
    assert torch.equal(O.ref(x, w), torch.tensor([[2.0, 4.0, -6.0]]))
    g = torch.linspace(-6, 6, 97, dtype=torch.float64)
    # the kernels' gelu form equals torch's tanh GELU: 1.5957691216 = 2 sqrt(2/pi), 0.0713548162 = 2 sqrt(2/pi) 0.044715
    assert abs(1.5957691216 - 2 * np.sqrt(2 / np.pi)) < 1e-10 and abs(0.0713548162 - 2 * np.sqrt(2 / np.pi) * 0.044715) < 1e-10
    assert torch.allclose(O.gelu_tanh(g), torch.nn.functional.gelu(g, approximate="tanh"), rtol=1e-7, atol=1e-12)
    assert torch.allclose(torch.nn.functional.silu(g), g / (1 + torch.exp(-g)), rtol=1e-12)
    # ref_f32 (the reference's float32 check path): x is rounded to bf16 first (1 + 2^-9 is not a bf16), the scale
    # multiplies columns, and on random data it stays within float32 rounding of the float64 ref
    x = torch.tensor([[1.0 + 2.0**-9, 2.0, -3.0]])
    s = torch.tensor([1.0, 0.5, 4.0])
    assert torch.equal(O.ref_f32(x, w, s), torch.tensor([[2.0, 2.0, -24.0]]))
    xr, wr = O.x_input(3, 512, 9), O.matrix(256, 512, 10).T.contiguous()
    y64, y32 = O.ref(xr, wr).double(), O.ref_f32(xr, wr).double()
    assert (y32 - y64).norm() / y64.norm() < 1e-6 and not torch.equal(y32, y64)


def test_bf16_ceil_and_interleave():
    s = torch.tensor([1.0, 1.0001, 0.3, 3.0e-5], dtype=torch.float32)
    c = O.bf16_ceil(s)
    assert torch.all(c >= s)
    assert torch.all(c.to(torch.bfloat16).float() == c)
    below = (c.view(torch.int32) - 0x10000).view(torch.float32)
    assert torch.all(below < s)
    g = torch.arange(64 * 2, dtype=torch.float32).reshape(64, 2)
    u = -g
    iv = O.interleave_glu(g, u)
    assert torch.equal(iv[:32], g[:32]) and torch.equal(iv[32:64], u[:32]) and torch.equal(iv[64:96], g[32:])


def test_int4_layout_decodes_to_codes():
    """The oracle's int4 layout, decoded with the bfloat4_b address formula above at exponent 129 (m * 2^0 = q), gives
    the codes back; zeros past N and K; the scale order puts column 16 p + c, group 4 b + kq at [p][b][kq][c]."""
    g = torch.Generator().manual_seed(21)
    n, k, n_pad = 40, 96, 64
    codes = torch.randint(-7, 8, (n, k), generator=g).numpy()
    lay = O.int4_layout(codes, n_pad, 256)
    exps = np.full(n_pad // 16 * 256, 129, np.uint8)
    got = _unlayout(lay, exps, "bfp4", k, n, n_pad)
    assert np.array_equal(got, codes.T.astype(np.float32))
    s = (torch.arange(n * (k // 32), dtype=torch.int64).reshape(n, k // 32) + 1).numpy().astype(np.uint16)
    sl = O.int4_scales_layout(s, n_pad, 256).reshape(n_pad // 16, 2, 4, 16)
    for col in (0, 17, 39):
        for grp in range(k // 32):
            p, c = divmod(col, 16)
            b, kq = divmod(grp, 4)
            assert sl[p, b, kq, c] == s[col, grp]
    assert sl[2, 0, 0, 9] == 0 and sl[0, 0, 3, 0] == 0  # column 41 (past N), group 3 (past K)


def test_int4_nibbles_matches_reference_format():
    """w4a16.nibbles (the reference's tile bytes, reshape form) against the oracle's element-by-element restatement."""
    from int4 import w4a16

    g = torch.Generator().manual_seed(22)
    codes = torch.randint(-7, 8, (64, 96), generator=g).to(torch.int8)  # [K, N]
    assert np.array_equal(w4a16.nibbles(codes).numpy(), O.int4_nibbles(codes.numpy()))


def test_int4_ref_hand_case():
    """int4_dequantized and int4_ref on a hand-worked case: the scale 0.1 held as the bf16 0.10009765625, q * s per
    group of 32 inputs, x rounded to bf16 first (1 + 2^-10 is 1 in bf16)."""
    codes = np.zeros((2, 64), np.int8)
    codes[0, :32], codes[0, 32:] = 1, -7
    codes[1, 0::2], codes[1, 1::2] = 3, -2
    scales = torch.tensor([[0.1, 2.0], [0.5, 0.25]])
    w = O.int4_dequantized(codes, scales)
    assert float(w[0, 0]) == 0.10009765625 and float(w[0, 40]) == -14.0
    assert float(w[1, 1]) == -1.0 and float(w[1, 33]) == -0.5 and float(w[1, 32]) == 0.75
    x = torch.ones(1, 64)
    x[0, 0] = 1.0009765625
    y = O.int4_ref(x, codes, scales)
    # row 0: 32 * 0.10009765625 - 32 * 7 * 2; row 1: 16 * (3 - 2) * 0.5 + 16 * (3 - 2) * 0.25
    assert y.tolist() == [[-444.796875, 12.0]]
