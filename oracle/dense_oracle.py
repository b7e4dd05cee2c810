"""CPU oracle of the dense_reader decode matmul -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only as the checker
(or, in the bench, as the timed CPU baseline); the product (tensix-kernels_amd/) never does.

It restates, in numpy / torch on the CPU, what XylolabsInc/tensix-kernels computes on this path (paths relative to
the reference's root):

- bfp_tiles / tile_values: the block-float tile format and its host conversion, moe/moe8.py:117-172 (bfloat4_b,
  three mantissa bits) and the same algorithm with seven mantissa bits for bfloat8_b (1088-byte tiles,
  dense_reader/linear.py:49-50); bfloat16 tiles are torch's round-to-nearest-even bf16 in face order.
- held: the values a weight of a format holds (dense_reader/tests/test_dense_reader.py:47-49).
- bf16_ceil, interleave_glu: dense_reader/linear.py:110-114, 122-130.
- ref: the tests' float64 check path, test_dense_reader.py:56-58; ref_f32: linear.py:166-169; glu_ref: test_dense_reader.py:113-115;
  gelu_tanh in the kernels' own form, common/kernels/dense_ops.h:44-59.
- key_bf16 / records_decode: the top-k key codec and record decode, dense_writer.cpp:215, 243-255 and
  dense_reader/linear.py:753-768; tile_topk: the records this build writes (one per 32-column tile) from an output.
- to_layout: the reference tile bytes rearranged into the MI355X library's HBM layout (codes and exponents), so a
  pack on the GPU can be compared byte for byte with the reference-format conversion above.

What pins each function (tests/test_oracle.py):
- bfp_tiles (bfloat4_b and bfloat8_b rounding): hand-derived golden vectors (tests/golden/bfp_face_rows.json) and an
  independent exact-rational restatement of the rule (round half to even of the truncated value on the block grid);
  ttnn's own BFP8 conversion is compiled code in a wheel that is not in the reference and cannot run here, so
  "the same bytes as ttnn for bfloat8_b" is parity unpinned; the B = 7 instance of the pinned BFP4 algorithm is what
  is restated.
- tile_values: closed form m * 2^(E - bias), checked against exact Fraction arithmetic; idempotence of held.
- key_bf16 / records_decode: exhaustive over all 65536 bf16 patterns (monotone order, inverse).
- ref, glu_ref: float64 closed forms.
"""

import json
from fractions import Fraction

import numpy as np
import torch

TILE = 32
FMTS = ("bfp8", "bfp4", "bf16")
TILE_BYTES = {"bfp8": 1088, "bfp4": 576, "bf16": 2048}  # dense_reader/linear.py:49-50
MANT_BITS = {"bfp8": 7, "bfp4": 3}
BIAS = {"bfp8": 133, "bfp4": 129}  # decode (-1)^s m 2^(E - 127 - (MB - 1)); moe/moe8.py:167 for bfp4


def bf16_bits(a):
    """float32 array -> bf16 bit patterns (uint16), round to nearest even, NaN -> 0x7FC0 (torch's conversion)."""
    t = torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def bf16_values(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)


def bf16_round(a):
    return bf16_values(bf16_bits(a))


def _face_rows(w):
    """float32 [K, N] -> [KT, NT, 64, 16]: each 32 x 32 tile in face order (face f = (r / 16) * 2 + c / 16, element
    (r, c) at f * 256 + (r % 16) * 16 + c % 16; moe/moe8.py:128-133, dense_writer.cpp:186-188)."""
    k, n = w.shape
    t = w.reshape(k // 32, 32, n // 32, 32).transpose(0, 2, 1, 3)
    f = t.reshape(k // 32, n // 32, 2, 16, 2, 16).transpose(0, 1, 2, 4, 3, 5)
    return np.ascontiguousarray(f).reshape(k // 32, n // 32, 64, 16)


def _unface(v):
    """[..., 64, 16] face rows of tiles -> [..., 32, 32] row-major tile values."""
    lead = v.shape[:-2]
    return v.reshape(*lead, 2, 2, 16, 16).swapaxes(-3, -2).reshape(*lead, 32, 32)


def bfp_round(rows, mb):
    """Face rows float32 [..., 16] -> (shared exponent [..., 1] uint32, signed magnitudes [..., 16] int64), the
    reference's host conversion (moe/moe8.py:134-150): shared = the largest biased exponent of the row; each value's
    24-bit mantissa (hidden bit) shifted down by its exponent's distance from it (0 past 31), rounded to mb bits, ties
    to even (shifted-out bits not sticky), at most 2^mb - 1; a zero or denormal value is 0; the sign only on a
    non-zero magnitude."""
    bits = np.ascontiguousarray(rows, np.float32).view(np.uint32)
    exp = (bits >> 23) & 0xFF
    sign = bits >> 31
    man = (bits & 0x7FFFFF) | (1 << 23)
    shared = exp.max(axis=-1, keepdims=True)
    diff = (shared - exp).astype(np.int64)
    m = np.where(diff > 31, 0, man.astype(np.int64) >> np.minimum(diff, 31))
    shift = 24 - mb
    rnd = m & ((1 << shift) - 1)
    m = m >> shift
    guard = m & 1
    tie = 1 << (shift - 1)
    m = m + ((rnd > tie) | ((rnd == tie) & (guard == 1)))
    m = np.minimum(m, (1 << mb) - 1)
    m = np.where(exp == 0, 0, m)
    s = np.where(m == 0, 0, sign)
    return shared.astype(np.uint32), np.where(s == 1, -m, m)


def bfp_tiles(w, fmt):
    """float [K, N] (K, N multiples of 32) -> uint8 [KT, NT, TILE_BYTES[fmt]]: each 32 x 32 tile in the reference's
    format. bfp: 64 exponent bytes (one a face row, face by face, row by row), then the codes face by face row-major:
    bfp8 one byte s<<7 | m, bfp4 one nibble s<<3 | m, two a byte, the first in the low nibble (moe/moe8.py:117-154).
    bf16: the 1024 bf16 values in face order."""
    w = np.ascontiguousarray(w.float().numpy() if isinstance(w, torch.Tensor) else w, np.float32)
    k, n = w.shape
    assert k % TILE == 0 and n % TILE == 0, w.shape
    f = _face_rows(w)
    kt, nt = k // 32, n // 32
    if fmt == "bf16":
        return bf16_bits(f).reshape(kt, nt, 1024).view(np.uint8).reshape(kt, nt, 2048)
    mb = MANT_BITS[fmt]
    shared, sm = bfp_round(f, mb)
    mag = np.abs(sm)
    s = (sm < 0).astype(np.int64)
    head = shared.reshape(kt, nt, 64).astype(np.uint8)
    if fmt == "bfp8":
        body = (s << 7 | mag).astype(np.uint8).reshape(kt, nt, 1024)
    else:
        code = (s << 3 | mag).astype(np.uint8).reshape(kt, nt, 1024)
        body = code[..., 0::2] | (code[..., 1::2] << 4)
    return np.concatenate([head, body], axis=-1)


def tile_values(tiles, fmt):
    """uint8 [..., TILE_BYTES[fmt]] tiles -> float32 [..., 32, 32] row-major tile values: (-1)^s m 2^(E - bias)
    (moe/moe8.py:157-172 for bfp4; bias 133 for bfp8), bf16 as it is."""
    tiles = np.asarray(tiles, np.uint8)
    lead = tiles.shape[:-1]
    if fmt == "bf16":
        v = bf16_values(tiles.reshape(*lead, 1024, 2).view(np.uint16).reshape(*lead, 1024))
        return _unface(v.reshape(*lead, 64, 16))
    head = tiles[..., :64].astype(np.int32)
    body = tiles[..., 64:]
    if fmt == "bfp8":
        code = body.astype(np.int32).reshape(*lead, 64, 16)
        mag = (code & 127).astype(np.float32)
        sgn = np.where(code & 128, -1.0, 1.0).astype(np.float32)
    else:
        code = np.stack([body & 15, body >> 4], axis=-1).reshape(*lead, 64, 16).astype(np.int32)
        mag = (code & 7).astype(np.float32)
        sgn = np.where(code & 8, -1.0, 1.0).astype(np.float32)
    scale = np.ldexp(np.float32(1.0), (head - BIAS[fmt])).astype(np.float32)
    val = (sgn * mag * scale[..., None]).astype(np.float32)
    return _unface(val)


def untile(v):
    """[KT, NT, 32, 32] -> [K, N]."""
    kt, nt = v.shape[:2]
    return v.transpose(0, 2, 1, 3).reshape(kt * 32, nt * 32)


def held(w, fmt):
    """The values a weight of fmt holds for the float [K, N] matrix w (K multiple of 32; N padded with zeros to 32)."""
    w = np.asarray(w.float().numpy() if isinstance(w, torch.Tensor) else w, np.float32)
    k, n = w.shape
    npad = -(-n // 32) * 32
    if npad != n:
        w = np.concatenate([w, np.zeros((k, npad - n), np.float32)], axis=1)
    return untile(tile_values(bfp_tiles(w, fmt), fmt))[:, :n]


def held_exact(w, fmt):
    """held computed a second way, exactly, one face row at a time with Python integers and Fractions: the block grid
    of a row is 2^(E - 127 - mb) with E its largest exponent; each value is truncated to the bits it keeps after the
    shift (the reference's shift drops them without a sticky bit) and then rounded half to even on that grid by
    Python's round(). For small inputs; pins bfp_round without sharing its arithmetic."""
    w = np.asarray(w, np.float32)
    k, n = w.shape
    out = np.zeros((k, n), np.float64)
    mb = MANT_BITS[fmt]
    for kk in range(k):
        for g in range(0, n, 16):
            row = w[kk, g : g + 16]
            bits = row.view(np.uint32).astype(np.int64)
            exps = (bits >> 23) & 0xFF
            E = int(exps.max())
            for c in range(len(row)):
                e = int(exps[c])
                if e == 0:
                    continue  # zero or denormal: 0
                man = int(bits[c] & 0x7FFFFF) | (1 << 23)
                d = E - e
                kept = 0 if d > 31 else man >> d  # the value is kept * 2^(E - 127 - 23)
                q = Fraction(kept, 1 << (24 - mb))  # on the grid of 2^(E - 127 - (mb - 1))
                m = min(round(q), (1 << mb) - 1)  # round(): half to even
                v = Fraction(m) * Fraction(2) ** (E - 127 - (mb - 1))
                out[kk, g + c] = float(-v if (bits[c] >> 31) and m else v)
    return out


# --- the MI355X library's HBM layout (the packing the GPU kernels read) ------------------------------------------------

KBLK = {"bfp8": 64, "bfp4": 128, "bf16": 32}


def exp_off(fmt, k):
    """The byte of a panel's exponents that holds k: groups of 256 k, byte 4 l + j of group g the j-th exponent lane l
    of a wavefront reads (bfp8: k = 256 g + 64 j + l; bfp4: k = 256 g + 128 (j >> 1) + 32 kq + 2 i + (j & 1), with
    l = 16 kq + i)."""
    g, r = divmod(k, 256)
    if fmt == "bfp8":
        return g * 256 + 4 * (r & 63) + (r >> 6)
    jb, r2 = divmod(r, 128)
    kq, r3 = divmod(r2, 32)
    i, h = divmod(r3, 2)
    return g * 256 + 4 * (16 * kq + i) + 2 * jb + h
KALIGN = 256


def to_layout(w, fmt, n_pad=None):
    """The library's packed (codes, exps) for the float [K, N] matrix w, built from the reference-format tiles
    (bfp_tiles): panels of 16 columns, k-blocks of 1 KiB, lane l = 16 kq + c holding column c's values of the kq-th
    quarter; bfp8 int8 m, bfp4 nibbles u = m + 8 (byte j of dword d: k 8d + j low, 8d + 4 + j high), bf16 as is;
    exponents one byte per (panel, k), placed by exp_off."""
    w = np.asarray(w.float().numpy() if isinstance(w, torch.Tensor) else w, np.float32)
    k, n = w.shape
    n_pad = n_pad or -(-n // 32) * 32
    k_pad = -(-k // KALIGN) * KALIGN
    wp = np.zeros((k_pad, n_pad), np.float32)
    wp[:k, :n] = w
    tiles = bfp_tiles(wp, fmt)  # [KT, NT, TB]
    kt, nt = k_pad // 32, n_pad // 32
    npan = n_pad // 16
    kb = KBLK[fmt]
    nkb = k_pad // kb
    if fmt == "bf16":
        vals = bf16_bits(untile(tile_values(tiles, fmt)))  # [K, N] bits (exact round trip)
        v = vals.reshape(nkb, 4, 8, npan, 16)  # k = b*32 + kq*8 + i ; n = p*16 + c
        codes = v.transpose(3, 0, 1, 4, 2).reshape(-1).view(np.uint8)
        return np.ascontiguousarray(codes), None
    # signed magnitudes and exponents per (k, n) from the tile bytes
    head = tiles[..., :64].reshape(kt, nt, 2, 2, 16)  # face (fr, fc), row r%16 -> [KT, NT, fr, fc, r]
    body = tiles[..., 64:]
    if fmt == "bfp8":
        code = body.astype(np.int64).reshape(kt, nt, 1024)
        mag, sgn = code & 127, (code >> 7) & 1
    else:
        code = np.stack([body & 15, body >> 4], axis=-1).reshape(kt, nt, 1024).astype(np.int64)
        mag, sgn = code & 7, (code >> 3) & 1
    sm = np.where(sgn == 1, -mag, mag).reshape(kt, nt, 2, 2, 16, 16)  # [KT, NT, fr, fc, r, c]
    sm = sm.transpose(0, 2, 4, 1, 3, 5).reshape(k_pad, n_pad)  # k = kt*32 + fr*16 + r, n = nt*32 + fc*16 + c
    ex = head.transpose(0, 2, 4, 1, 3).reshape(k_pad, nt * 2)  # [k, panel]
    # panel-major; within a panel, groups of 256 k with byte 4 l + j the j-th exponent lane l reads (exp_off)
    perm = np.array([exp_off(fmt, kk) for kk in range(k_pad)], np.int64)
    exps = np.zeros((npan, k_pad), np.uint8)
    exps[:, perm] = ex.T
    exps = exps.reshape(-1)
    if fmt == "bfp8":
        v = (sm & 0xFF).astype(np.uint8).reshape(nkb, 4, 16, npan, 16)  # k = b*64 + kq*16 + i
        codes = v.transpose(3, 0, 1, 4, 2).reshape(-1)
    else:
        u = (sm + 8).astype(np.uint8).reshape(nkb, 4, 4, 2, 4, npan, 16)  # k = b*128 + kq*32 + d*8 + h*4 + j
        lo, hi = u[:, :, :, 0], u[:, :, :, 1]  # [nkb, kq, d, j, p, c]
        byte = lo | (hi << 4)
        codes = byte.transpose(4, 0, 1, 5, 2, 3).reshape(-1)  # [p, b, kq, c, d, j]
    return np.ascontiguousarray(codes), exps


# --- host helpers restated -------------------------------------------------------------------------------------------


def bf16_ceil(s):
    """The smallest bf16 value >= s (s > 0, float32 tensor) (dense_reader/linear.py:110-114)."""
    b = s.to(torch.bfloat16).float()
    up = (b.view(torch.int32) + 0x10000).view(torch.float32)
    return torch.where(b >= s, b, up)


def interleave_glu(gate, up):
    """[2 out, in] with output tiles alternating gate, up (dense_reader/linear.py:122-130)."""
    o, i = gate.shape
    return torch.stack([gate.reshape(o // 32, 32, i), up.reshape(o // 32, 32, i)], dim=1).reshape(2 * o, i)


# --- the float64 check path ------------------------------------------------------------------------------------------


def x_input(m, k, seed):
    """The reference tests' activations (test_dense_reader.py:28-39): randn seeded, columns 0..3 times 8, as bf16."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g)
    x[:, :4] *= 8
    return x


def matrix(n, k, seed):
    """test_dense_reader.py:42-44: randn(n, k) * 0.02."""
    g = torch.Generator().manual_seed(seed)
    return torch.randn(n, k, generator=g) * 0.02


def ref(x, wk, scale=None):
    """x rounded to bf16 times the held weight, float64, times the scales (test_dense_reader.py:56-58)."""
    y = x.to(torch.bfloat16).double() @ torch.as_tensor(wk).double()
    return (y * torch.as_tensor(scale).double()[None, :] if scale is not None else y).float()


def ref_f32(x, wk, scale=None):
    """The reference's own CPU check path, float32 (dense_reader/linear.py:166-169): x rounded to bf16, as float32,
    times the held weight in float32, times the scales. The bench times it as the CPU baseline."""
    y = x.to(torch.bfloat16).float() @ torch.as_tensor(wk).float()
    return y * torch.as_tensor(scale).float()[None, :] if scale is not None else y


def gelu_tanh(g):
    """g * sigmoid(1.5957691216 g + 0.0713548162 g^3) (common/kernels/dense_ops.h:44-59): torch's gelu(tanh)."""
    return g * torch.sigmoid(1.5957691216 * g + 0.0713548162 * g**3)


def glu_ref(g, u, act):
    """act(g) * u in float64 (test_dense_reader.py:113-115): silu or gelu(approximate="tanh")."""
    g, u = g.double(), u.double()
    a = torch.nn.functional.silu(g) if act == "swiglu" else torch.nn.functional.gelu(g, approximate="tanh")
    return (a * u).float()


# --- top-k ------------------------------------------------------------------------------------------------------------


def key_bf16(bits):
    """The writer's key of bf16 bit patterns (dense_writer.cpp:215): b ^ (0x8000 | (0x7FFF & -(b >> 15)))."""
    b = np.asarray(bits, np.int64) & 0xFFFF
    return b ^ (0x8000 | (0x7FFF & (-(b >> 15))))


def key_value(keys):
    """Key -> float32 value (dense_reader/linear.py:762-765)."""
    keys = np.asarray(keys, np.int64)
    bits = np.where(keys >= 0x8000, keys & 0x7FFF, ~keys & 0xFFFF)
    return bf16_values(bits.astype(np.uint32))


def tile_topk(y, rows, k, n_valid, base, fp32=False, yf=None, width=32):
    """The records this build writes for output y [M, N] (bf16 values as float32; yf: the fp32 scores when fp32):
    per `width` columns (a 32-column tile, or a group of tiles; the reference's writer ranks each core's columns
    together, dense_writer.cpp:185-232), per row r < rows, the best k of columns [width t, width t + width) below
    n_valid, highest first, ties to the lower column. Returns uint32 words [records, 2 * rows * k]: keys then ids (bf16
    keys 0 / ids 0xFFFFFFFF empty; fp32: score bits, -inf / 0xFFFFFFFF empty)."""
    y = np.asarray(y, np.float32)
    M, N = y.shape
    tiles = -(-N // width)
    out = np.zeros((tiles, 2, rows, k), np.uint64)
    for t in range(tiles):
        for r in range(rows):
            cand = []
            for c in range(width * t, min(width * t + width, N)):
                if c >= n_valid:
                    continue
                if fp32:
                    v = np.float32(yf[r, c])
                    u = int(np.array(v, np.float32).view(np.uint32))
                    key = u ^ (0xFFFFFFFF if u >> 31 else 0x80000000)
                    word = u
                else:
                    b = int(bf16_bits(np.array([y[r, c]], np.float32))[0])
                    key = int(key_bf16(b))
                    word = key
                cand.append((-key, c, word))
            cand.sort()
            for q in range(k):
                if q < len(cand):
                    out[t, 0, r, q] = cand[q][2]
                    out[t, 1, r, q] = base + cand[q][1]
                else:
                    out[t, 0, r, q] = 0xFF800000 if fp32 else 0
                    out[t, 1, r, q] = 0xFFFFFFFF
    return out.reshape(tiles, -1).astype(np.uint32)


def records_decode(words, rows, k):
    """uint32 record words [records, 2 * rows * k] -> (values [rows, records * k] float32 with -inf empty, ids int64
    with -1 empty) (dense_reader/linear.py:753-768)."""
    t = np.asarray(words, np.int64).reshape(-1, 2, rows, k) & 0xFFFFFFFF
    keys = t[:, 0].transpose(1, 0, 2).reshape(rows, -1)
    idx = t[:, 1].transpose(1, 0, 2).reshape(rows, -1)
    vals = key_value(keys)
    empty = keys == 0
    vals = np.where(empty, -np.inf, vals).astype(np.float32)
    idx = np.where(empty | (idx == 0xFFFFFFFF), -1, idx)
    return vals, idx


def global_topk(vals, ids, k_out):
    """The best k_out (value, id) pairs per row, highest first, ties to the lower id; -inf / -1 padding."""
    rows = vals.shape[0]
    ov = np.full((rows, k_out), -np.inf, np.float32)
    oi = np.full((rows, k_out), -1, np.int64)
    for r in range(rows):
        ok = ids[r] >= 0
        v, i = vals[r][ok], ids[r][ok]
        order = sorted(range(len(v)), key=lambda j: (-float(v[j]), int(i[j])))[:k_out]
        ov[r, : len(order)] = v[order]
        oi[r, : len(order)] = i[order]
    return ov, oi


def load_golden(path):
    with open(path) as f:
        return json.load(f)


# --- the LM head's pick -----------------------------------------------------------------------------------------------


def pick_token(exact, ids, vocab):
    """The pick over rescored candidates, one row at a time (lm_head_topk/lmhead.py:40-46): the lowest id among the
    largest values, a NaN counting as the largest; -inf marks an empty slot; vocab when nothing is there."""
    exact = np.asarray(exact, np.float64)
    ids = np.asarray(ids, np.int64)
    out = np.empty(exact.shape[0], np.int64)
    for r in range(exact.shape[0]):
        v, i = exact[r], ids[r]
        if np.isnan(v).any():
            out[r] = int(i[np.isnan(v)].min())
            continue
        top = v.max()
        out[r] = int(i[v == top].min()) if top > -np.inf or (v == top).any() else vocab
    return out


def head_logits(x, w, logits="bf16"):
    """A bf16 host head's logits: x (bf16) times the bf16 rows w [vocab, dim] in float64, rounded to float32, then to
    bf16 unless logits is "float32" (lm_head_topk/tests/test_lm_head.py:50-54)."""
    z = (torch.as_tensor(x).to(torch.bfloat16).double() @ torch.as_tensor(w).to(torch.bfloat16).double().T).float()
    return z.to(torch.bfloat16).float() if logits == "bf16" else z


def pick_from_records(words, rows, k, top, x, w, logits="bf16", vocab=None):
    """The device pick restated (lm_head_topk/kernels/head_pick_reader.cpp:66-90, head_pick_writer.cpp:44-66): per
    row the best `top` valid slots by bf16 key (the earlier slot, record by record and slot by slot, first among
    equal keys; a slot is valid when its key is not 0 and its id is below vocab), their logits from the bf16 rows
    (head_logits), and pick_token over them. words: [records, 2 * rows * k] uint32. Returns (tokens, first
    candidate ids, counts)."""
    words = np.asarray(words, np.int64) & 0xFFFFFFFF
    vocab = w.shape[0] if vocab is None else vocab
    toks, firsts, counts = [], [], []
    for r in range(rows):
        keys = (words[:, r * k : (r + 1) * k] & 0xFFFF).reshape(-1)
        ids = words[:, rows * k + r * k : rows * k + (r + 1) * k].reshape(-1)
        order = [j for j in range(keys.size) if keys[j] != 0 and ids[j] < vocab]
        order.sort(key=lambda j: (-int(keys[j]), j))
        cand = [int(ids[j]) for j in order[:top]]
        counts.append(len(cand))
        firsts.append(cand[0] if cand else 0xFFFFFFFF)
        if not cand:
            toks.append(0)
            continue
        z = head_logits(torch.as_tensor(x)[r : r + 1], torch.as_tensor(w)[cand], logits).numpy()
        toks.append(int(pick_token(z, np.array([cand]), vocab)[0]))
    return np.array(toks), np.array(firsts), np.array(counts)


# --- int4 W4A16 -------------------------------------------------------------------------------------------------------


def int4_dequantized(codes, scales):
    """The float [N_out, K] weight q * s with s rounded to bf16 (int4/w4a16.py:100-102)."""
    codes = torch.as_tensor(codes)
    s = torch.as_tensor(scales).to(torch.bfloat16).double()
    return codes.double() * s.repeat_interleave(32, dim=1)


def int4_ref(x, codes, scales):
    """x rounded to bf16 times (q * s).T in float64 (int4/w4a16.py:105-107, in float64 here)."""
    return (torch.as_tensor(x).to(torch.bfloat16).double() @ int4_dequantized(codes, scales).T).float()


def int4_nibbles(codes):
    """The reference's int4 tile bytes of codes [K, N] (int4/w4a16.py:59-66), one value at a time: tile (kt, nt), face
    f = 2 (r // 16) + c // 16 of element (r, c), position 256 f + 16 (r % 16) + c % 16 in the tile, value sign << 3 |
    |q|, element 2i in the low nibble of byte i."""
    codes = np.asarray(codes, np.int64)
    k, n = codes.shape
    out = np.zeros((k // 32, n // 32, 512), np.uint8)
    for kk in range(k):
        for nn in range(n):
            q = int(codes[kk, nn])
            v = (8 if q < 0 else 0) | abs(q)
            r, c = kk % 32, nn % 32
            pos = 256 * (2 * (r // 16) + c // 16) + 16 * (r % 16) + c % 16
            out[kk // 32, nn // 32, pos // 2] |= v << (4 * (pos % 2))
    return out


def int4_layout(codes, n_pad, k_pad):
    """codes [N, K] (-7..7) in this build's int4 layout: bfloat4_b's codes (panel of 16 columns, k-block of 128, lane
    16 kq + c its 16 bytes, dword d holding k 8 d + j in the low nibble of byte j and 8 d + 4 + j in the high one, each
    u = q + 8); zeros (u = 8) past N and K. Returns uint8 [n_pad * k_pad / 2]."""
    codes = np.asarray(codes, np.int64)
    n, k = codes.shape
    q = np.zeros((n_pad, k_pad), np.int64)
    q[:n, :k] = codes
    u = (q + 8).reshape(n_pad // 16, 16, k_pad // 128, 4, 4, 2, 4)  # panel, c, block, kq, d, h, j
    u = u.transpose(0, 2, 3, 1, 4, 6, 5)  # panel, block, kq, c, d, j, h
    return (u[..., 0] | (u[..., 1] << 4)).astype(np.uint8).reshape(-1)


def int4_scales_layout(scales, n_pad, k_pad):
    """Group scales [N, K / 32] (bf16 bits as uint16) in this build's order [panel, k-block, kq, c]; zeros past N and
    K. Returns uint16 [n_pad / 16 * k_pad / 128 * 64]."""
    s = np.asarray(scales, np.uint16)
    n, g = s.shape
    full = np.zeros((n_pad, k_pad // 32), np.uint16)
    full[:n, :g] = s
    return full.reshape(n_pad // 16, 16, k_pad // 128, 4).transpose(0, 2, 3, 1).reshape(-1)
