"""linear.py: the dense_reader weight-streaming matmul for decode, on MI355X (gfx950).

y = x @ w (* scale): x bf16 activations, w a block-float (bfloat8_b, bfloat4_b) or bfloat16 weight, fp32
accumulation, bf16 output (or float32). Fused output stages: per-column scales, act(gate) * up (SwiGLU, GeGLU), a
residual add, the fp32 accumulator as it is, and top-k records of each output row. Block lists run two to four weights
as one launch into one output.

This module keeps the Python surface of XylolabsInc/tensix-kernels' dense_reader/linear.py (its file:line cited per
function) so callers switch by changing the import; the device work is the HIP library libdense_reader.so (csrc/,
C ABI include/dense_reader.h), called through ctypes with torch tensors on the GPU as the device memory. Device
tensors: x, y, scales, residuals and records are torch tensors on a ROCm device; a weight is a `Weight` (packed
codes and exponents in HBM).

Entry points:
- matmul(x, w, scale, ...): the op; x [1, 1, M, K] bf16 on the GPU (any leading dims of size 1 are taken).
- linear(x, w, scale, activation=...): the same for x of any rank, with "swiglu" / "geglu" / "silu".
- native_weight(device, t, dtype): a float [out, in] matrix as a weight [1, 1, in, out] and its scale tensor.
- interleave_glu(gate, up): [gate | up] with output tiles alternating, for the fused GLU stage.
- topk_result, topk_records, records_host: the top-k records' tensor and their decode on the host; topk_merge: the
  best k over all records on the device.
"""

import itertools
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
from common import device as dev  # noqa: E402
from common.device import (  # noqa: E402,F401  (re-exported, as the reference's module does)
    FIDELITY,
    TILE,
    DataType,
    MemoryConfig,
    bfloat4_b,
    bfloat8_b,
    bfloat16,
    check_banks,
    dram_banks,
    float32,
    is_dram_sharded,
    sharded_memcfg,
    uint32,
)

from . import _lib  # noqa: E402

BFP8_TILE = 1088
NATIVE_TILES = {bfloat8_b: BFP8_TILE, bfloat4_b: 576, bfloat16: 2048}
KALIGN = 256  # the packed layout pads K to this
XCDS = 8  # MI355X's XCDs (each with its own L2): a launch's workgroups go to them in turn

# --- settings (module attributes of the reference, linear.py:52-94) ---------------------------------------------------
# The Tensix work-split knobs have no meaning on MI355X; they are kept so that code setting them runs, and, as in the
# reference, they never change a result.
L1_BUDGET = None
L1_MARGIN = 32 * 1024
X_BUDGET = 600_000
XS_DEPTH = 3
MIN_CHUNKS = 0
MIN_CHUNKS_SHAPES = None
NARROW_N = 0
SPLIT_SHARE = 0.5
REQ_TILES = 0
GLU_ROWS = True
# the top-k result tensor as bfloat16 (the same bytes as the uint32 words the kernel writes; False: int32 words)
RECORDS_BF16 = False
CACHE = True
LOG = False
CONFIGS = ({},)


# --- host side --------------------------------------------------------------------------------------------------------


def bf16_ceil(s):
    """The smallest bf16 value >= s (s > 0, float32) (reference linear.py:110-114)."""
    b = s.to(torch.bfloat16).float()
    up = (b.view(torch.int32) + 0x10000).view(torch.float32)
    return torch.where(b >= s, b, up)


def native_tile(w):
    """Tile bytes of a weight this matmul reads (bfloat8_b, bfloat4_b, bfloat16), else 0 (reference linear.py:117-119)."""
    return NATIVE_TILES.get(getattr(w, "dtype", None), 0)


def interleave_glu(gate, up):
    """[gate | up] for the fused GLU stage: two float [out, in] matrices as one [2 * out, in] whose output tiles
    alternate, tile 2j the gate's rows 32j..32j+31 and tile 2j + 1 the up's (reference linear.py:122-130). Whole tiles
    move, so values already on a block-float grid keep their exponent groups."""
    assert gate.shape == up.shape and gate.shape[0] % TILE == 0, (gate.shape, up.shape)
    o, i = gate.shape
    g = gate.reshape(o // TILE, TILE, i)
    u = up.reshape(o // TILE, TILE, i)
    return torch.stack([g, u], dim=1).reshape(2 * o, i)


def scale_tensor(device, s, dtype=bfloat16):
    """Per-output-column scales s [N] as [1, 1, 1, N] on the device, bf16 as the reference stores them (reference
    linear.py:133-141), or float32 with dtype=float32."""
    d = dev.as_device(device)
    td = torch.float32 if dev.as_dtype(dtype) == float32 else torch.bfloat16
    return s.reshape(1, 1, 1, -1).to(device=d.torch, dtype=td).contiguous()


class Weight:
    """A packed weight [1, 1, K, N] in HBM: codes and (block-float) exponents in the library's layout, N padded to
    n_pad (banks * 32 when sharded), K to k_pad. shape, padded_shape, dtype and memory_config() answer as the
    reference's device weight does."""

    def __init__(self, device, k, n, dtype, codes, exps, n_pad, k_pad, memcfg):
        self.device_ = device
        self.k, self.n = k, n
        self.dtype = dtype
        self.codes, self.exps = codes, exps
        self.n_pad, self.k_pad = n_pad, k_pad
        self._mc = memcfg

    @property
    def shape(self):
        return torch.Size([1, 1, self.k, self.n])

    @property
    def padded_shape(self):
        return torch.Size([1, 1, self.k, self.n_pad])

    @property
    def fmt(self):
        return dev.FMT[self.dtype]

    def memory_config(self):
        return self._mc

    def device(self):
        return self.device_

    def nbytes(self):
        """Bytes of codes and exponents stored (padding included)."""
        return self.codes.numel() + (self.exps.numel() if self.exps is not None else 0)

    def algorithmic_bytes(self, n=None):
        """The reference's tile bytes of the first n columns (default N): 1088 / 576 / 2048 per 32 x 32 tile."""
        n = self.n if n is None else n
        return (self.k // TILE) * -(-n // TILE) * NATIVE_TILES[self.dtype]

    def exps_ptr(self):
        return self.exps.data_ptr() if self.exps is not None else None

    def __repr__(self):
        return f"Weight({self.dtype.name}, K {self.k}, N {self.n}, padded {self.n_pad}, banks {self._mc.banks})"


def _packed(device, k, n, dtype, n_pad):
    """Empty codes / exponents for a weight of k x n (n_pad columns)."""
    L = _lib.lib()
    k_pad = -(-k // KALIGN) * KALIGN
    f = dev.FMT[dtype]
    codes = torch.empty(L.dr_codes_bytes(f, k_pad, n_pad), dtype=torch.uint8, device=device.torch)
    eb = L.dr_exps_bytes(f, k_pad, n_pad)
    exps = torch.empty(eb, dtype=torch.uint8, device=device.torch) if eb else None
    return codes, exps, k_pad


def pack(device, t, dtype, col_div=None, n_pad=None, memcfg=None):
    """A float [out, in] matrix packed as the weight [1, 1, in, out] of dtype; col_div [out]: each row divided by it
    first. No padding beyond n_pad (default: out rounded to 32)."""
    d = dev.as_device(device)
    dtype = dev.as_dtype(dtype)
    assert dtype in NATIVE_TILES, f"dense_reader: weights are bfloat8_b, bfloat4_b or bfloat16, not {dtype}"
    t = t.to(device=d.torch, dtype=torch.float32).contiguous()
    assert t.dim() == 2, t.shape
    n, k = t.shape
    assert k % TILE == 0, f"dense_reader: K {k} is not a multiple of {TILE}"
    n_pad = n_pad or -(-n // TILE) * TILE
    codes, exps, k_pad = _packed(d, k, n, dtype, n_pad)
    cd = None
    if col_div is not None:
        cd = col_div.to(device=d.torch, dtype=torch.float32).contiguous()
    st = _lib.lib().dr_pack(
        t.data_ptr(), k, n, k, dev.FMT[dtype], cd.data_ptr() if cd is not None else None, codes.data_ptr(),
        exps.data_ptr() if exps is not None else None, n_pad, k_pad, d.stream(),
    )
    _lib.check(st, "dr_pack")
    return Weight(d, k, n, dtype, codes, exps, n_pad, k_pad, memcfg or MemoryConfig(0))


def native_weight(device, t, dtype, col_scale=False, sharded=True, max_banks=None):
    """A float [out, in] matrix as a weight [1, 1, in, out] of dtype (bfloat8_b, bfloat4_b or bfloat16), "sharded"
    over the device's banks (at most max_banks; N padded to banks * 32) or interleaved, and its [1, 1, 1, out] scales:
    ones, or with col_scale each output column divided by c = max |w| (rounded up to bf16) before the block-float
    rounding and multiplied back after the matmul (reference linear.py:144-156). The packing runs on the GPU."""
    d = dev.as_device(device)
    t = t.float()
    c = bf16_ceil(t.abs().amax(dim=1).clamp(min=1e-8)) if col_scale else torch.ones(t.shape[0])
    n, k = t.shape
    mc = sharded_memcfg(d, k, n, max_banks=max_banks) if sharded else MemoryConfig(0)
    n_pad = mc.banks * mc.shard_width if sharded else -(-n // TILE) * TILE
    w = pack(d, t, dtype, col_div=c if col_scale else None, n_pad=n_pad, memcfg=mc)
    return w, scale_tensor(d, c)


def to_torch(w):
    """The values a weight holds, [1, 1, K, n_pad] float32 on its device (the reference's ttnn.to_torch of a weight)."""
    if not isinstance(w, Weight):
        return w
    out = torch.empty(w.k, w.n_pad, dtype=torch.float32, device=w.device_.torch)
    st = _lib.lib().dr_unpack(
        w.codes.data_ptr(), w.exps_ptr(), w.fmt, w.n_pad, w.k, w.n_pad, w.k_pad, out.data_ptr(), w.n_pad,
        w.device_.stream(),
    )
    _lib.check(st, "dr_unpack")
    return out.reshape(1, 1, w.k, w.n_pad)


def held(w, n=None):
    """[K, N] values the weight holds, its first n columns (the reference test's held(), test_dense_reader.py:47-49)."""
    n = w.n if n is None else n
    return to_torch(w).reshape(w.k, -1)[:, :n]


def _bfp_host(t2, mb):
    """float32 [R, C] (C a multiple of 16) on the host, rounded to a block float of mb magnitude bits whose exponent is
    shared by each 16 consecutive values of a row (a face row of the 32 x 32 tile): the conversion the reference's
    host makes (moe/moe8.py:134-150) and dr_pack makes on the GPU. The shared exponent is the row's largest; each
    value's 24-bit significand is shifted down by its exponent's distance from it (nothing past 31), rounded to mb
    bits half to even on the bits shifted out, at most 2^mb - 1; zeros and denormals give 0, and a zero keeps no sign.
    Returns the values: magnitude * 2^(shared - 127 - (mb - 1)) with the value's sign."""
    r, c = t2.shape
    bits = t2.contiguous().view(torch.int32).to(torch.int64).reshape(r, c // 16, 16) & 0xFFFFFFFF
    exp = (bits >> 23) & 0xFF
    man = (bits & 0x7FFFFF) | (1 << 23)
    shared = exp.amax(dim=-1, keepdim=True)
    diff = shared - exp
    m = torch.where(diff > 31, torch.zeros_like(man), man >> diff.clamp(max=31))
    shift = 24 - mb
    low = m & ((1 << shift) - 1)
    m = m >> shift
    half = 1 << (shift - 1)
    m = m + ((low > half) | ((low == half) & ((m & 1) == 1))).to(torch.int64)
    m = torch.where(exp == 0, torch.zeros_like(m), m.clamp(max=(1 << mb) - 1))
    v = torch.ldexp(m.to(torch.float64), (shared - 127 - (mb - 1)).to(torch.float64))
    v = torch.where(((bits >> 31) == 1) & (m != 0), -v, v)
    return v.to(torch.float32).reshape(r, c)


def block_float(t, dtype, device=None):
    """t (float [..., rows, cols]) rounded to dtype's grid (the exponent shared along cols, 16 values a face row), as
    float32 on t's device: the values a weight of that dtype holds (reference linear.py:159-163, a host conversion).
    Runs on the host (finite inputs); with a device, by packing on that GPU instead (rows a multiple of 32), which
    gives the same values."""
    dtype = dev.as_dtype(dtype)
    assert dtype in NATIVE_TILES, f"dense_reader: weights are bfloat8_b, bfloat4_b or bfloat16, not {dtype}"
    shape = t.shape
    t2 = t.detach().float().reshape(-1, shape[-1])
    if device is not None:
        d = dev.as_device(device)
        w = pack(d, t2.T.contiguous(), dtype)  # the matrix [cols, rows] packs as [rows, cols]: face rows along cols
        return held(w).reshape(shape).to(t.device)
    h = t2.cpu()
    if dtype == bfloat16:
        out = h.to(torch.bfloat16).float()
    else:
        c = shape[-1]
        cp = -(-c // 16) * 16
        if cp != c:
            h = torch.nn.functional.pad(h, (0, cp - c))
        out = _bfp_host(h, 7 if dtype == bfloat8_b else 3)[:, :c]
    return out.reshape(shape).to(t.device)


def reference(x, w, scale=None):
    """x @ w (* scale) in float32, x as the device sees it (bf16); w [K, N] as the weight holds it (block_float)
    (reference linear.py:166-169)."""
    y = x.to(torch.bfloat16).float() @ w.float()
    return y * scale.float()[None, :] if scale is not None else y


# --- the plan ---------------------------------------------------------------------------------------------------------


def row_slices(x, full_sync=False):
    """[(first tile row, tile rows)] of x's rows, at most 4 tile rows each (8 with full_sync) (reference linear.py:
    179-184, where each slice is one program that reads all the weights). matmul needs no slicing: one launch takes
    all of x's rows, in passes of plan()["rows_per_pass"] inside it. A caller that slices x this way gets each slice's
    rows from its own matmul (the rows a call takes pick its kernel, so the sums of a slice's rows can differ in their
    last bits from those of one call over all rows)."""
    mt = -(-x.shape[-2] // TILE)
    cap = 8 if full_sync else 4
    return [(m0, min(cap, mt - m0)) for m0 in range(0, mt, cap)]


def plan(
    device,
    x,
    w,
    cores_per_bank=3,
    full_sync=False,
    kb=None,
    kw=None,
    sbw=None,
    split=False,
    mt=None,
    rows=False,
    budget=None,
    xs=False,
    noscale=False,
    glu=False,
    glu2=False,
    out32=False,
    blocks=None,
    max_banks=None,
):
    """The work split of one launch over x's rows (mt tile rows of them, default all), with the reference plan's keys
    (linear.py:187-382) given their MI355X meaning, and the launch's own (launch_plan's) beside them:

    MT, KT, NT: the tile rows, K tiles and output tiles (32 each). KB: the K tiles of x a workgroup reads (all: x is
    not cut into blocks). KW: the K tiles of one wavefront's chunk (its unit of work; a workgroup's wavefronts take the
    chunks in turn). SBW: the 16-column panels one wavefront sums at once (1, 2, or 4 for a GLU's gate and up tiles).
    NC: the 32-column output tiles a workgroup computes (0.5 for a 16-column tile, 2 for a pair). W_PAGES: the 1 KiB
    weight blocks of one chunk of one panel (bfloat8_b 64 K, bfloat4_b 128 K, bf16 32 K a block). l1: the LDS bytes a
    workgroup of the first pass's kernel holds (0 where no device answers). work: [(workgroup, (XCD, block, split,
    col0, ncols, n0))] for one pass: the XCD whose L2 serves it (workgroups go to the 8 XCDs in turn), the caller's
    block, the K split it sums, its first column in the block, its columns and its first output column. SEGS: the
    blocks of a block list (blocks: [(w | (gate, up), col0_tiles[, scale]), ...] as matmul takes it), seg_work: each
    block's workgroups. sharded: the weight's layout; native: a 32 x 32 tile's bytes in the reference's format.
    split, rows, xs, noscale, glu, glu2 and the Tensix knobs (cores_per_bank, kb, kw, sbw, budget, max_banks) are
    kept as given and change nothing; out32 plans an fp32 output. Nothing is launched."""
    first, target, opts = w, w, {"glu": glu, "out32": out32}
    if blocks:
        target = list(blocks)
        assert is_block_list(target), "dense_reader: blocks is matmul's block list"
        first, opts = block_entries(target)[0][0], {}
    L, _, keep = _launch(x, target, None, **opts)
    info = _lib.launch_info(L)
    placed = _lib.launch_work(L, info["workgroups"])
    del keep
    tc = info["tile_cols"]
    work = [(i, (i % XCDS, b, sp, t0 * tc, nt * tc, n0)) for i, (b, t0, nt, sp, n0) in enumerate(placed)]
    segs = L.nseg
    kblk = {bfloat8_b: 64, bfloat4_b: 128}.get(first.dtype, 32)
    K, N = first.shape[-2], first.shape[-1]
    return {
        "K": K,
        "M": x.shape[-2],
        "MT": mt or -(-x.shape[-2] // TILE),
        "KT": K // TILE,
        "NT": -(-N // TILE),
        "KB": K // TILE,
        "KW": info["kch"] // TILE,
        "SBW": 4 if glu else tc // 16,
        "NC": tc * info["tiles_per_workgroup"] / TILE,
        "W_PAGES": info["kch"] // kblk,
        "sharded": is_dram_sharded(first),
        "split": split,
        "rows": rows,
        "native": native_tile(first),
        "xs": xs,
        "noscale": noscale,
        "glu": glu,
        "glu2": glu2,
        "out32": out32,
        "SEGS": segs,
        "seg_work": tuple(tuple(i for i, wk in work if wk[1] == b) for b in range(segs)) if segs > 1 else (),
        "work": work,
        "l1": info["lds_bytes"],
        **info,
    }


def choose(device, x, w, full_sync=False, **forced):
    """[(first tile row, plan)] for x's rows (reference linear.py:455-495): one slice (passes run inside a launch)."""
    return [(0, plan(device, x, w, **forced))]


class BlockListMismatch(ValueError):
    """A block list refused before its launch because its output would not equal one call per block bit for bit
    (reference linear.py:498-501). The MI355X split depends on K and the rows (which kernel runs) alone, which a block
    list's weights share, so the output always equals one call per block; the class is kept for callers that catch
    it."""


def is_block_list(w):
    """True for matmul's block list [(w | (gate, up), col0_tiles[, scale]), ...]: a list or tuple of 2 to 4 entries
    (reference linear.py:520-530; the optional third item, a block's scales, goes beyond the reference)."""
    return (
        isinstance(w, (list, tuple))
        and 2 <= len(w) <= 4
        and all(
            isinstance(e, (list, tuple))
            and len(e) in (2, 3)
            and isinstance(e[1], int)
            and not isinstance(e[1], bool)
            for e in w
        )
    )


def block_entries(w):
    """A block list as [(gate, up or None, col0_tiles, scale or None)], checked: two to four entries, all plain
    weights or all pairs, of one K (reference linear.py:533-556). Unlike the reference, blocks may differ in dtype and
    carry their own scales."""
    out = []
    for item in w:
        assert isinstance(item, (tuple, list)) and len(item) in (2, 3), (
            f"dense_reader: a block is (weight, col0_tiles[, scale]): {item!r}"
        )
        wt, c0 = item[0], item[1]
        sc = item[2] if len(item) == 3 else None
        gate, up = (wt[0], wt[1]) if isinstance(wt, (tuple, list)) else (wt, None)
        assert isinstance(c0, int) and c0 >= 0, f"dense_reader: col0_tiles {c0!r}"
        if up is not None:
            assert up.dtype == gate.dtype and tuple(up.padded_shape) == tuple(gate.padded_shape), "gate and up differ"
            assert up.memory_config() == gate.memory_config(), "dense_reader: gate and up differ"
            assert sc is None, "dense_reader: a (gate, up) block takes no scale"
        out.append((gate, up, c0, sc))
    assert 2 <= len(out) <= 4, f"dense_reader: {len(out)} blocks (2 to 4; one weight goes in on its own)"
    assert len({up is None for _, up, _, _ in out}) == 1, "dense_reader: blocks all plain or all (gate, up) pairs"
    assert len({g.shape[-2] for g, _, _, _ in out}) == 1, "dense_reader: blocks of one K"
    return out


def choose_blocks(device, x, w, full_sync=False, **forced):
    """choose for a block list: the plan of its one call (reference linear.py:559-562)."""
    entries = block_entries(w)
    return choose(device, x, entries[0][0], full_sync, **forced)


# --- the op -----------------------------------------------------------------------------------------------------------


def _x2d(x):
    """x [..., M, K] with leading dims of 1 (or any rank <= 4 that flattens to rows) as a contiguous [M, K] bf16 whose
    rows start 16-byte aligned (a copy when x's do not)."""
    assert isinstance(x, torch.Tensor) and x.is_cuda, "dense_reader: x is a bf16 torch tensor on the GPU"
    assert x.dtype == torch.bfloat16, (x.dtype, "dense_reader: x is bf16")
    x2 = x.reshape(-1, x.shape[-1])
    if not x2.is_contiguous() or x2.data_ptr() % 16:  # (the kernels read x rows 16 bytes at a time)
        x2 = x2.contiguous() if not x2.is_contiguous() else x2.clone()
    return x2


def _scale_ptr(s, n):
    if s is None:
        return None, 0
    assert isinstance(s, torch.Tensor) and s.is_cuda, "dense_reader: scale is a torch tensor on the GPU"
    assert s.dtype in (torch.bfloat16, torch.float32), s.dtype
    assert s.numel() >= n, (s.shape, n)
    assert s.is_contiguous()
    return s.data_ptr(), int(s.dtype == torch.float32)


def _segment(seg, w, up, col0_tiles, scale, glu, scale_up=None):
    seg.fmt = w.fmt
    seg.n = w.n
    seg.n_pad = w.n_pad
    seg.glu = 0 if not glu else (2 if up is not None else 1)
    seg.codes = w.codes.data_ptr()
    seg.exps = w.exps_ptr()
    if up is not None:
        seg.codes_up = up.codes.data_ptr()
        seg.exps_up = up.exps_ptr()
    p, f32 = _scale_ptr(scale, w.n)
    seg.scale = p
    pu, f32u = _scale_ptr(scale_up, w.n)
    seg.scale_up = pu
    if p is not None and pu is not None:
        assert f32 == f32u, "dense_reader: gate and up scales of one dtype"
    seg.scale_f32 = f32 or f32u
    seg.col0 = TILE * col0_tiles


def matmul(
    x,
    w,
    scale,
    *,
    memory_config=None,
    fidelity="hifi2",
    full_sync=False,
    topk=None,
    out=None,
    col0=0,
    w_up=None,
    max_banks=None,
    **opts,
):
    """y = x @ w (* scale) on the GPU (reference linear.py:568-744): x [1, 1, M, K] bf16, w a [1, 1, K, N] weight
    (native_weight), scale [1, 1, 1, N] bf16 (scale_tensor) or None (unit scales). Returns [1, 1, M, N] bf16.
    max_banks: refuse a weight sharded over more banks (default common.device.MAX_BANKS; None: no limit).

    topk (M <= 32): {"r": result tensor (topk_result), "k": K <= 32, "rows": T <= 32, "slot0": first record, "base":
    index of output element 0, "n": valid output elements, "write_y": bool, "fp32": bool, "slots": records at most}:
    every 32-column output tile writes one record, slot0 + its tile index, of each of the first T rows' best K values
    (keys, then ids; topk_records decodes them); a launch of more tiles than "slots" (default grid_slots(), the
    reference's records per block; 0: no limit) writes one record a group of consecutive tiles instead, so that it
    writes at most "slots" (topk_slots gives the count). fp32 False (default): the reference's bf16 keys of the bf16
    output; True: fp32 scores (beyond the reference). y is still written with write_y. out: a [1, 1, M, N] tensor to write into instead of a new
    one. col0 (with out, no topk): out is wider, [1, 1, M, W], and output column tile c goes to its tile c + col0.

    Options (opts): glu (the weight is interleave_glu's [gate | up], output act(gate) * up, N / 2 wide), glu_act (0
    silu, 1 gelu_tanh), w_up (with glu: the up weight apart, w the gate's; output N wide), residual ([1, 1, M, N]
    bf16: y = bf16(x @ w + residual)), residual_mode ("epilogue" or "preload"), out32 (y float32, the fp32 accumulator
    as it is). The reference's Tensix work-split options (cores_per_bank, split, rows, xs, kb, kw, sbw) are accepted
    and change nothing. Beyond the reference: scales with GLU (w_up's own scales as opts["scale_up"]), residual with
    out32, block lists of mixed dtypes with per-block scales.

    A block list in place of w: matmul(x, [(w_or_(gate, up), col0_tiles[, scale]), ...], None, out=None, **opts) is
    one launch, one output, over two to four column blocks of one K; each block's columns go to its col0_tiles. The
    output equals one call per block (out=, col0=) bit for bit. Block output spans must not overlap."""
    L, y, keep = _launch(x, w, scale, topk=topk, out=out, col0=col0, w_up=w_up, max_banks=max_banks, **opts)
    d = x.device
    st = torch.cuda.current_stream(d)
    L.stream = st.cuda_stream
    need = _lib.lib().dr_workspace_bytes(L)
    _lib.check(_lib.DR_EINVAL if need < 0 else _lib.DR_OK, "dr_workspace_bytes")
    if need > 0:
        ws = _workspace(d, st, need)
        L.workspace, L.workspace_bytes = ws.data_ptr(), ws.numel()
    _lib.check(_lib.lib().dr_matmul(L), "dr_matmul")
    del keep
    return y


def launch_plan(x, w, scale, **kw):
    """What matmul(x, w, scale, **kw) launches, without launching it: {"kernel": "gemv" | "mfma", "rows_per_pass",
    "tile_cols" (16 or 32), "tiles", "chunks", "kch", "splits", "workgroups", "passes", "records",
    "tiles_per_record"} (the reference's choose/plan answer the same question for its Tensix split, linear.py:
    455-495)."""
    kw = dict(kw)
    for knob in ("memory_config", "fidelity", "full_sync"):
        kw.pop(knob, None)
    L, _, keep = _launch(x, w, scale, **kw)
    info = _lib.launch_info(L)
    del keep
    return info


def _launch(x, w, scale, *, topk=None, out=None, col0=0, w_up=None, max_banks=None, **opts):
    """matmul's checks (the reference's assertions), its dr_launch, y (allocated unless out is given), and the tensors
    the launch points into that the caller does not hold (keep them alive until the launch is enqueued)."""
    d = x.device
    # weights sharded over more banks than allowed are refused before anything else (reference linear.py:627-633)
    if not isinstance(w, (list, tuple)):
        check_banks(w, max_banks)
    elif is_block_list(w):
        for e in w:
            wt = e[0]
            for u in wt if isinstance(wt, (list, tuple)) else (wt,):
                check_banks(u, max_banks)
    check_banks(w_up, max_banks)
    entries = None
    if isinstance(w, (list, tuple)):
        assert is_block_list(w), "dense_reader: w is one weight or a block list [(w | (gate, up), col0_tiles), ...]"
        entries = block_entries(w)
        assert scale is None and topk is None and col0 == 0 and w_up is None, (
            "dense_reader: a block list takes no scale, topk, col0 or w_up (each block carries its own col0_tiles)"
        )
        assert "residual" not in opts and not opts.get("out32"), "dense_reader: a block list: no residual or out32"
        assert x.shape[-2] <= 32, "dense_reader: a block list is a decode call: up to 32 rows"
        if entries[0][1] is not None:
            opts = {**opts, "glu": True}
    res_mode = {"epilogue": 1, "preload": 2}[opts.pop("residual_mode", "epilogue")]
    residual = opts.pop("residual", None)
    scale_up = opts.pop("scale_up", None)
    out32 = bool(opts.get("out32"))
    assert not (out32 and topk is not None), "dense_reader: out32 without top-k"
    assert not (out32 and out is not None and out.dtype != torch.float32), out.dtype
    x2 = _x2d(x)
    M, K = x2.shape
    glu = bool(opts.get("glu", False))
    act = opts.pop("glu_act", 0)  # the GLU's activation: 0 silu, 1 gelu_tanh
    assert act in (0, 1) and (act == 0 or glu), "dense_reader: glu_act (0 silu, 1 gelu_tanh) needs glu"
    first = entries[0][0] if entries else w
    assert native_tile(first), f"dense_reader: weights are bfloat8_b, bfloat4_b or bfloat16, not {getattr(first, 'dtype', first)}"
    assert first.shape[-2] == K, (x.shape, first.shape)
    if w_up is not None:
        assert glu, "dense_reader: w_up is the GLU's up weight (glu=True)"
        assert w_up.dtype == w.dtype and tuple(w_up.padded_shape) == tuple(w.padded_shape)
        assert w_up.memory_config() == w.memory_config(), "dense_reader: gate and up differ"
    if glu and not entries and w_up is None:
        assert w.n % (2 * TILE) == 0, f"dense_reader: glu needs whole gate/up tile pairs ({w.n} columns)"
    if entries:
        n_out = max(TILE * c0 + (g.n // 2 if (glu and u is None) else g.n) for g, u, c0, _ in entries)
    else:
        n_out = w.n if (w_up is not None or not glu) else w.n // 2
    if residual is not None:
        assert not glu and topk is None and not entries, "dense_reader: residual: plain matmul, no GLU or top-k"
        assert scale is None, "dense_reader: residual: unit-scale matmul only"
        assert residual.dtype == torch.bfloat16 and residual.is_cuda, residual.dtype
        r2 = residual.reshape(-1, residual.shape[-1])
        assert r2.shape[0] >= M and r2.shape[1] >= n_out, (residual.shape, M, n_out)
        assert r2.is_contiguous()
        assert col0 == 0 and (out is None or out is residual), "dense_reader: residual with a fresh output or in place"
    y = out
    if y is None:
        y = torch.empty(1, 1, M, n_out, dtype=torch.float32 if out32 else torch.bfloat16, device=d)
    assert entries or col0 == 0 or (out is not None and topk is None), "dense_reader: col0 needs out, no top-k"
    y2 = y.reshape(-1, y.shape[-1])
    assert y2.shape[0] >= M and y.is_contiguous(), (y.shape, M)
    assert y.dtype == (torch.float32 if out32 else torch.bfloat16), (y.dtype, out32)
    blocks = entries or [(w, w_up, col0, scale)]
    ends = []
    for g, u, c0, _ in blocks:
        nb = g.n // 2 if (glu and u is None) else g.n
        ends.append((c0, -(-nb // TILE)))
        assert TILE * c0 + nb <= y2.shape[1], (c0, nb, y.shape)
    if entries:
        spans = sorted(ends)
        assert all(a0 + an <= b0 for (a0, an), (b0, _) in itertools.pairwise(spans)), (
            f"dense_reader: block output spans overlap (col0_tiles, tiles): {spans}"
        )
    L = _lib.Launch()
    L.x = x2.data_ptr()
    L.m, L.k, L.ldx = M, K, K
    L.y = y2.data_ptr()
    L.ldy = y2.shape[1]
    L.y_f32 = int(out32)
    if residual is not None:
        L.residual = r2.data_ptr()
        L.ldr = r2.shape[1]
        L.residual_mode = res_mode
    L.act = act
    L.nseg = len(blocks)
    for i, (g, u, c0, sc) in enumerate(blocks):
        _segment(L.seg[i], g, u, c0, sc, glu, scale_up if i == 0 else None)
    if topk is not None:
        assert M <= 32, "dense_reader: top-k needs one row slice (up to 32 rows)"
        r = topk["r"]
        rows, kk = topk["rows"], topk["k"]
        assert 1 <= kk <= 32 and 1 <= rows <= min(32, M), (kk, rows, M)
        words = r.reshape(r.shape[-2], -1)
        if words.dtype == torch.bfloat16:
            words = words.view(torch.int32)
        assert words.dtype == torch.int32 and words.shape[1] == 2 * rows * kk, (r.dtype, r.shape, rows, kk)
        L.topk.records = words.data_ptr()
        L.topk.k, L.topk.rows = kk, rows
        L.topk.slot0 = topk.get("slot0", 0)
        L.topk.records_cap = words.shape[0]
        L.topk.n_valid = topk.get("n", n_out)
        L.topk.base = topk.get("base", 0)
        L.topk.write_y = int(bool(topk.get("write_y", False)))
        L.topk.fp32 = int(bool(topk.get("fp32", False)))
        slots = topk.get("slots")
        L.topk.max_records = grid_slots() if slots is None else int(slots)
        records = topk_slots(n_out, L.topk.max_records)
        assert L.topk.slot0 + records <= L.topk.records_cap, (
            f"dense_reader: {records} records from slot {L.topk.slot0} do not fit {L.topk.records_cap}"
        )
    return L, y, (x2,)


_WORKSPACE = {}


def _workspace(device, stream, nbytes, kind="matmul"):
    """The workspace of one kind of launch (the matmul's split K, or the top-k merge and head pick) on a device and
    stream: zeroed once when allocated (or grown); every launch leaves its counters at zero, each kind's counters lie
    at one place whatever the launch's shape, and launches on one stream never overlap. The two kinds keep apart: each
    lays its counters out its own way."""
    key = (device, stream.cuda_stream, kind)
    ws = _WORKSPACE.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _WORKSPACE[key] = ws
    return ws


def linear(x, w, scale, memory_config=None, activation=None, out_dtype=None, **opts):
    """matmul for x of any rank (reference linear.py:1073-1124): x [..., rows, K] bf16, the [1, 1, K, N] weight and
    its [1, 1, 1, N] scales or None, the input's rank back. activation: None, "silu" (after the matmul), "swiglu" or
    "geglu" (w is interleave_glu's [gate | up] weight, the output act(gate) * up N / 2 wide; or w is (gate, up), two
    weights [1, 1, K, N], the output N wide). out_dtype float32: the output in float32 (out32). A block list for w:
    matmul's one call over column blocks, scale None; plain weights with activation None, (gate, up) pairs with
    "swiglu" or "geglu". opts go to matmul."""
    shape = list(x.shape)
    if out_dtype is not None and dev.as_dtype(out_dtype) != bfloat16:
        assert dev.as_dtype(out_dtype) == float32, f"dense_reader.linear: out_dtype {out_dtype}"
        opts = {**opts, "out32": True}
    blocks = is_block_list(w)
    if blocks:
        pairs = isinstance(w[0][0], (tuple, list))
        assert activation != "silu", "dense_reader.linear: no silu after a block list"
        takes = ("swiglu", "geglu") if pairs else (None,)
        assert activation in takes, (
            f"dense_reader.linear: a block list of {'(gate, up) pairs' if pairs else 'plain weights'} takes activation"
            f" {' or '.join(map(repr, takes))}, not {activation!r}"
        )
        if activation == "geglu":
            opts = {**opts, "glu_act": 1}
        n = max(TILE * e[1] + (e[0][0] if pairs else e[0]).shape[-1] for e in w)
    elif isinstance(w, (tuple, list)):
        assert activation in ("swiglu", "geglu"), "dense_reader.linear: two weights are the GLU's gate and up"
        w, w_up = w
        opts = {**opts, "w_up": w_up}
    rows, kd = shape[-2], shape[-1]
    if not blocks:
        n = w.shape[-1]
    if activation in ("swiglu", "geglu") and not blocks:
        opts = {**opts, "glu": True}
        if activation == "geglu":
            opts["glu_act"] = 1
        if opts.get("w_up") is None:
            n //= 2
    x4 = x.reshape(1, 1, rows, kd) if len(shape) != 4 else x
    y = matmul(x4, w, scale, memory_config=memory_config, **opts)
    if activation is not None and activation not in ("swiglu", "geglu"):
        assert activation == "silu", f"dense_reader.linear: activation {activation!r}"
        y = torch.nn.functional.silu(y.float()).to(y.dtype)
    if len(shape) != 4 and opts.get("out") is None:  # (a given out is returned as it is)
        y = y.reshape(*shape[:-1], n)
    return y


# --- top-k records ----------------------------------------------------------------------------------------------------


def grid_slots():
    """Records a top-k launch writes at most by default: the cores of the device's grid
    (compute_with_storage_grid_size), as the reference writes one a core of its plan and its callers size a block's
    records by the grid (lm_head_topk/lmhead.py:102-103)."""
    return dev.CU_GRID[0] * dev.CU_GRID[1]


def topk_slots(n, slots=None):
    """Records a top-k call over n output columns writes: one a 32-column tile, or for more tiles than `slots`
    (default grid_slots(); 0: no limit) one a group of ceil(tiles / slots) consecutive tiles, ranked together."""
    tiles = -(-n // TILE)
    slots = grid_slots() if slots is None else slots
    if slots <= 0 or tiles <= slots:
        return tiles
    g = -(-tiles // slots)
    return -(-tiles // g)


def topk_result(device, records, rows, k):
    """A result tensor for records top-k records of rows x k, zeroed (every slot empty): [1, 1, records, 2 * rows * k]
    int32 words (the reference's uint32), or with RECORDS_BF16 the same bytes as [1, 1, records, 4 * rows * k]
    bfloat16 (reference linear.py:771-785)."""
    d = dev.as_device(device)
    if RECORDS_BF16:
        return torch.zeros(1, 1, records, 4 * rows * k, dtype=torch.bfloat16, device=d.torch)
    return torch.zeros(1, 1, records, 2 * rows * k, dtype=torch.int32, device=d.torch)


def topk_records(r, rows, k, fp32=False):
    """The records of a top-k result tensor on the host: (values [rows, records * k] float32, indices [rows,
    records * k] int64); empty slots hold -inf and -1 (reference linear.py:747-750)."""
    return records_host(r.cpu(), rows, k, fp32=fp32)


def records_host(t, rows, k, fp32=False):
    """topk_records on a host copy of the result tensor (int32/uint32 words, or the same bytes as bfloat16)
    (reference linear.py:753-768; fp32 records: the scores' bits and int32 ids)."""
    if t.dtype == torch.bfloat16:
        t = t.contiguous().view(torch.int32)  # the bits, two bf16 per 32-bit word
    t = t.to(torch.int64).reshape(-1, 2, rows, k) & 0xFFFFFFFF
    keys, idx = (
        t[:, 0].permute(1, 0, 2).reshape(rows, -1),
        t[:, 1].permute(1, 0, 2).reshape(rows, -1),
    )
    if fp32:
        vals = torch.where(keys >= 1 << 31, keys - (1 << 32), keys).to(torch.int32).view(torch.float32)
        empty = idx == 0xFFFFFFFF
        vals = torch.where(empty, torch.full_like(vals, float("-inf")), vals)
        idx = torch.where(empty, torch.full_like(idx, -1), idx)
        return vals, idx
    bits = torch.where(keys >= 0x8000, keys & 0x7FFF, ~keys & 0xFFFF)
    v = bits << 16
    vals = torch.where(v >= 1 << 31, v - (1 << 32), v).to(torch.int32).view(torch.float32)
    empty = keys == 0
    vals = torch.where(empty, torch.full_like(vals, float("-inf")), vals)
    idx = torch.where(empty | (idx == 0xFFFFFFFF), torch.full_like(idx, -1), idx)
    return vals, idx


def topk_merge(r, rows, k, k_out=32, fp32=False, records=None):
    """The best k_out of all records per row, on the device: (values [rows, k_out] float32, ids [rows, k_out] int32),
    highest first, ties to the lower id, -inf / -1 where fewer exist. records: the first records to read (default
    all)."""
    words = r.reshape(r.shape[-2], -1)
    if words.dtype == torch.bfloat16:
        words = words.view(torch.int32)
    n = words.shape[0] if records is None else records
    vals = torch.empty(rows, k_out, dtype=torch.float32, device=r.device)
    ids = torch.empty(rows, k_out, dtype=torch.int32, device=r.device)
    st = torch.cuda.current_stream(r.device)
    need = _lib.lib().dr_topk_merge_workspace_bytes(n, rows, k)
    _lib.check(_lib.DR_EINVAL if need < 0 else _lib.DR_OK, "dr_topk_merge_workspace_bytes")
    wp, wn = None, 0
    if need > 0:
        ws = _workspace(r.device, st, need, "merge")
        wp, wn = ws.data_ptr(), ws.numel()
    st = _lib.lib().dr_topk_merge(
        words.data_ptr(), n, rows, k, int(fp32), k_out, vals.data_ptr(), ids.data_ptr(), wp, wn, st.cuda_stream
    )
    _lib.check(st, "dr_topk_merge")
    return vals, ids
