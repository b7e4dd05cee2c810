"""Host-side checks that need no GPU: the C ABI library loads and exports every symbol include/dense_reader.h
declares, its structs have the C layout, the planner and argument checks answer without touching a device, and the
Python surface refuses what the reference refuses with the same exception types."""

import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from dense_reader import _lib, linear

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))


def _declared():
    text = "".join(h.read_text() for h in HEADERS)
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(dr_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = _declared()
    assert set(names) == set(_lib.SYMBOLS), (names, _lib.SYMBOLS)
    for s in names:
        assert hasattr(lib, s), s
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True).stdout
    for s in names:
        assert re.search(rf"\bT {s}\b", out), s


def test_constants_match_the_headers():
    """The numbers the Python bindings pass (status codes, MoE modes and activations, the expert packs' formats) are
    the ones include/*.h defines."""
    from moe import moe8

    text = "".join(h.read_text() for h in HEADERS)
    defs = {k: int(v) for k, v in re.findall(r"^#define\s+(DR_\w+)\s+(\d+)\b", text, re.M)}
    want = {"DR_OK": _lib.DR_OK, "DR_EINVAL": _lib.DR_EINVAL, "DR_EHIP": _lib.DR_EHIP, "DR_ERANGE": _lib.DR_ERANGE,
            "DR_MOE_GATE_UP": _lib.DR_MOE_GATE_UP, "DR_MOE_DOWN": _lib.DR_MOE_DOWN,
            "DR_MOE_GATE_UP_ROWS": _lib.DR_MOE_GATE_UP_ROWS, "DR_MOE_DOWN_ROWS": _lib.DR_MOE_DOWN_ROWS,
            "DR_BFP4": moe8.DR_BFP4, "DR_BFP4_KB": moe8.DR_BFP4_KB, "DR_ACT_SILU": moe8.ACTS["silu"],
            "DR_ACT_GELU_TANH": moe8.ACTS["gelu_tanh"], "DR_ACT_SWIGLU_OAI": moe8.ACTS["swiglu_oai"]}
    for name, v in want.items():
        assert defs.get(name) == v, (name, defs.get(name), v)


def test_struct_layout_matches_c(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "dense_reader.h"\n'
        "int main(void){printf(\"%zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu\\n\", sizeof(dr_segment), sizeof(dr_topk),"
        " sizeof(dr_launch), offsetof(dr_launch, seg), offsetof(dr_launch, topk), offsetof(dr_launch, stream),"
        " offsetof(dr_topk, base), offsetof(dr_segment, col0), offsetof(dr_launch, workspace_bytes),"
        " sizeof(dr_launch_info), offsetof(dr_launch_info, tiles_per_record), offsetof(dr_launch_info, waves),"
        " offsetof(dr_launch_info, lds_bytes));return 0;}\n"
    )
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    want = [
        ctypes.sizeof(_lib.Segment),
        ctypes.sizeof(_lib.TopK),
        ctypes.sizeof(_lib.Launch),
        _lib.Launch.seg.offset,
        _lib.Launch.topk.offset,
        _lib.Launch.stream.offset,
        _lib.TopK.base.offset,
        _lib.Segment.col0.offset,
        _lib.Launch.workspace_bytes.offset,
        ctypes.sizeof(_lib.LaunchInfo),
        _lib.LaunchInfo.tiles_per_record.offset,
        _lib.LaunchInfo.waves.offset,
        _lib.LaunchInfo.lds_bytes.offset,
    ]
    assert got == want


def test_plan_depends_on_k_and_kernel():
    """The chunking is a function of K and the kernel (the GEMV for 1-2 rows, the MFMA kernel from 3): 512-k chunks past
    K = 2048 on the GEMV, past K = 3072 on the MFMA kernel, else 256."""
    lib = _lib.lib()
    assert lib.dr_version() >= 1
    for k in (32, 1024, 2048, 2080, 3072, 3584, 4096, 14336):
        k_pad = -(-k // 256) * 256
        for ms, last in (((1, 2), 2048), ((3, 8, 16, 17, 32, 100), 3072)):
            c, kch, _ = _lib.plan(k, ms[0])
            assert kch == (512 if k_pad > last else 256) and c == -(-k_pad // kch), (k, ms, kch)
            for m in ms[1:]:
                assert _lib.plan(k, m)[:2] == (c, kch), (k, m)
    assert [_lib.plan(4096, m)[2] for m in (1, 2, 3, 16, 17, 32, 100)] == [1, 2, 16, 16, 32, 32, 32]


def test_sizes():
    lib = _lib.lib()
    assert lib.dr_codes_bytes(0, 256, 64) == 256 * 64
    assert lib.dr_codes_bytes(1, 256, 64) == 256 * 32
    assert lib.dr_codes_bytes(2, 256, 64) == 256 * 128
    assert lib.dr_exps_bytes(0, 256, 64) == 256 * 4 and lib.dr_exps_bytes(2, 256, 64) == 0


def test_invalid_arguments_refused_on_the_host():
    lib = _lib.lib()
    L = _lib.Launch()  # every pointer NULL
    assert lib.dr_matmul(ctypes.byref(L)) == _lib.DR_EINVAL
    L.x, L.y, L.m, L.k, L.ldx, L.nseg = 8, 8, 1, 48, 48, 1  # K not a multiple of 32
    assert lib.dr_matmul(ctypes.byref(L)) == _lib.DR_EINVAL
    L.k = L.ldx = 64
    L.seg[0].fmt = 7  # no such format
    assert lib.dr_matmul(ctypes.byref(L)) == _lib.DR_EINVAL
    assert lib.dr_pack(None, 0, 0, 0, 0, None, None, None, 0, 0, None) == _lib.DR_EINVAL
    assert lib.dr_topk_merge(None, 1, 1, 1, 0, 65, None, None, None, 0, None) == _lib.DR_EINVAL
    assert lib.dr_topk_merge_workspace_bytes(4, 1, 8) == 0  # one workgroup a row: no workspace
    need = lib.dr_topk_merge_workspace_bytes(4008, 4, 8)
    assert need >= 4 * 64 * 8 * 2
    assert lib.dr_topk_merge(8, 4008, 4, 8, 0, 32, 8, 8, None, 0, None) == _lib.DR_EINVAL  # workspace missing
    assert lib.dr_topk_merge(8, 4008, 4, 8, 0, 32, 8, 8, 8, need - 1, None) == _lib.DR_EINVAL  # too small
    # more rows than a record holds (32): refused, so the rows' counters keep their places in a shared workspace
    assert lib.dr_topk_merge_workspace_bytes(4008, 33, 8) == -1
    assert lib.dr_topk_merge(8, 4008, 33, 8, 0, 32, 8, 8, 8, 1 << 30, None) == _lib.DR_EINVAL
    assert lib.dr_topk_merge_workspace_bytes(4008, 32, 8) > lib.dr_topk_merge_workspace_bytes(4008, 1, 8) > 0
    with pytest.raises(ValueError):
        _lib.check(_lib.DR_EINVAL, "x")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.DR_EHIP, "x")


def _ns_launch(m=1, k=4096, n=14336, fmt=0):
    L = _lib.Launch()  # device pointers that are never read: the plan only reads the launch's sizes
    L.x, L.y, L.m, L.k, L.ldx, L.ldy, L.nseg = 16, 16, m, k, k, n, 1
    s = L.seg[0]
    s.fmt, s.n, s.n_pad, s.codes, s.exps = fmt, n, -(-n // 32) * 32, 16, 16
    return L


def test_launch_plan_on_the_host():
    """dr_launch_plan answers without a device (as if it had 256 CUs): the north star on the wide GEMV, 32 rows on the
    MFMA kernel, a long K split, top-k records one a tile; an invalid launch is refused."""
    p = _lib.launch_info(_ns_launch())
    assert (p["kernel"], p["rows_per_pass"], p["tile_cols"], p["tiles"], p["splits"]) == ("gemv", 1, 32, 448, 1), p
    assert p["waves"] == 8 and p["chunks"] == 8, p
    p = _lib.launch_info(_ns_launch(m=32))
    assert (p["kernel"], p["rows_per_pass"], p["passes"], p["chunks"], p["kch"], p["waves"]) == ("mfma", 32, 1, 8, 512, 8), p
    p = _lib.launch_info(_ns_launch(m=8, k=14336, n=4096))
    assert (p["kernel"], p["rows_per_pass"], p["splits"], p["chunks"], p["kch"], p["waves"]) == ("mfma", 16, 2, 28, 512, 8), p
    p = _lib.launch_info(_ns_launch(n=1000))
    assert (p["tile_cols"], p["tiles"]) == (16, 63), p  # few tiles: 16-column tiles
    # the split-K workspace has counters for 16384 tiles: a launch of more runs unsplit (its workgroups walk all 28
    # chunks), one at the limit still splits
    p = _lib.launch_info(_ns_launch(m=8, k=14336, n=32 * 16384))
    assert (p["tiles"], p["splits"], p["chunks"]) == (16384, 2, 28), p
    p = _lib.launch_info(_ns_launch(m=8, k=14336, n=32 * 16385))
    assert (p["tiles"], p["splits"], p["chunks"], p["waves"]) == (16385, 1, 28, 8), p
    info = _lib.LaunchInfo()
    assert _lib.lib().dr_launch_plan(ctypes.byref(_lib.Launch()), ctypes.byref(info)) == _lib.DR_EINVAL
    # empty shapes and a K that is not a multiple of 32 are refused; more than 32 rows run in passes of 32
    for bad in ({"m": 0}, {"k": 0}, {"n": 0}, {"k": 8}, {"k": 33}):
        assert _lib.lib().dr_launch_plan(ctypes.byref(_ns_launch(**bad)), ctypes.byref(info)) == _lib.DR_EINVAL, bad
    p = _lib.launch_info(_ns_launch(m=100))
    assert (p["rows_per_pass"], p["passes"]) == (32, 4), p


def test_launch_work_on_the_host():
    """dr_launch_work lists the workgroups as the kernels map blockIdx.x: the north star one 32-column tile each, in
    column order; a split K launch every tile once a split, the splits after each other; 16-column tiles."""
    L = _ns_launch()
    work = _lib.launch_work(L, 448)
    assert work == [(0, i, 1, 0, 32 * i) for i in range(448)]
    assert _lib.lib().dr_launch_work(ctypes.byref(L), (ctypes.c_int32 * (5 * 447))(), 447) == _lib.DR_ERANGE
    work = _lib.launch_work(_ns_launch(m=8, k=14336, n=4096), 256)
    assert work == [(0, i % 128, 1, i // 128, 32 * (i % 128)) for i in range(256)]
    work = _lib.launch_work(_ns_launch(n=1000), 63)
    assert work == [(0, i, 1, 0, 16 * i) for i in range(63)]


class _FakeWeight:
    def __init__(self, k, n, dtype=linear.bfloat8_b, banks=8):
        self.dtype = dtype
        self.shape = (1, 1, k, n)
        self.padded_shape = (1, 1, k, n)
        self._mc = linear.MemoryConfig(banks, n // banks)

    def memory_config(self):
        return self._mc


def test_block_list_rules():
    a, b = _FakeWeight(1024, 256), _FakeWeight(1024, 512)
    assert linear.is_block_list([(a, 0), (b, 8)])
    assert not linear.is_block_list((a, b))  # linear's (gate, up) pair
    assert not linear.is_block_list([(a, 0)])
    assert not linear.is_block_list([(a, True), (b, 8)])
    assert linear.is_block_list([(a, 0, None), (b, 8)])  # a per-block scale (beyond the reference)
    with pytest.raises(AssertionError):
        linear.block_entries([(a, 0), ((a, b), 8)])  # mixed plain and pairs
    with pytest.raises(AssertionError):
        linear.block_entries([(a, 0), (_FakeWeight(2048, 256), 8)])  # two K
    assert len(linear.block_entries([(a, 0), (b, 8), (a, 24)])) == 3


def test_check_banks_refuses_oversharded():
    w = _FakeWeight(1024, 1024, banks=8)
    linear.check_banks(w, 8)
    with pytest.raises(ValueError):
        linear.check_banks(w, 4)


def test_records_host_decodes_the_reference_codec():
    import torch

    # two records of rows 1, k 2: keys of 1.0 (0x3F80 -> 0xBF80) and -2.0 (0xC000 -> 0x3FFF), an empty slot
    t = torch.tensor([[0xBF80, 0x3FFF, 5, 7], [0, 0xBF80, -1, 9]], dtype=torch.int64).to(torch.int32)
    vals, idx = linear.records_host(t, 1, 2)
    assert vals.tolist() == [[1.0, -2.0, float("-inf"), 1.0]]
    assert idx.tolist() == [[5, 7, -1, 9]]


def test_interleave_and_bf16_ceil_match_oracle():
    import torch

    from oracle import dense_oracle as O

    g = torch.randn(64, 32, generator=torch.Generator().manual_seed(1))
    u = torch.randn(64, 32, generator=torch.Generator().manual_seed(2))
    assert torch.equal(linear.interleave_glu(g, u), O.interleave_glu(g, u))
    s = torch.rand(100, generator=torch.Generator().manual_seed(3)) + 1e-3
    assert torch.equal(linear.bf16_ceil(s), O.bf16_ceil(s))


def test_pick_token_matches_oracle():
    """lmhead.pick_token (host logic) against the oracle's row-by-row restatement: NaN largest, lowest id on ties,
    -inf empty slots."""
    import numpy as np
    import torch

    from lm_head_topk import lmhead
    from oracle import dense_oracle as O

    g = torch.Generator().manual_seed(4)
    z = torch.randint(-3, 4, (64, 12), generator=g).float()  # many ties
    z[z == -3] = float("-inf")
    z[5, 3] = float("nan")
    z[9, :] = float("-inf")
    ids = torch.stack([torch.randperm(1000, generator=g)[:12] for _ in range(64)])
    want = O.pick_token(z.numpy(), ids.numpy(), 1000)
    assert np.array_equal(lmhead.pick_token(z, ids, 1000).numpy(), want)
    assert want[5] == int(ids[5, 3])


def test_pick_from_records_hand_case():
    """The oracle's device-pick restatement on a hand-built record set: the best `top` by key (the earlier slot first
    among equal keys), ids at or past vocab and empty keys skipped, then the largest logit, the lower id on a tie."""
    import numpy as np
    import torch

    from oracle import dense_oracle as O

    w = torch.zeros(8, 32)
    w[:, 0] = torch.tensor([1.0, 5.0, 5.0, 2.0, 9.0, 3.0, 4.0, 7.0])  # logits = row 0 of w times x[0] = 1
    x = torch.zeros(1, 32)
    x[0, 0] = 1.0
    key = lambda v: int(O.key_bf16(O.bf16_bits(torch.tensor([v]))[0]))  # noqa: E731
    # one row, k 2, three records: (key, id) slots
    rec = [[(key(5.0), 1), (key(4.0), 6)], [(key(5.0), 2), (0, 4)], [(key(9.0), 7), (key(1.0), 0)]]
    words = np.zeros((3, 4), np.int64)
    for p, slots in enumerate(rec):
        for s, (kk, i) in enumerate(slots):
            words[p, s], words[p, 2 + s] = kk, i
    tok, first, n = O.pick_from_records(words, 1, 2, 3, x, w, "float32", vocab=8)
    # best 3 by key: id 7 (key of 9), id 1 and id 2 (key of 5, record 0 first); logits 7, 5, 5 -> token 7
    assert (tok[0], first[0], n[0]) == (7, 7, 3)
    tok, first, n = O.pick_from_records(words, 1, 2, 3, x, w, "float32", vocab=7)  # id 7 past vocab
    # best 3: ids 1, 2 (key 5), 6 (key 4); logits 5, 5, 4 -> the lower id of the tie, 1
    assert (tok[0], first[0], n[0]) == (1, 1, 3)


def test_pack_cache_files(tmp_path):
    """The pack cache's file logic, with arrays of a made-up pack (no GPU): written whole then taken; a different
    meta refused and left as it is; a damaged array refused; rebuild hands the call back to be packed again."""
    import json

    import numpy as np

    from dense_reader import pack_cache as pc

    path = tmp_path / "w"
    meta = {"version": pc.PACK_VERSION, "format": "bfloat8_b", "k": 64, "n": 32, "weight": "x"}
    arrays = {"codes": np.arange(256, dtype=np.uint8), "scale": np.ones(32, np.float32)}
    assert pc.cache_read(path, meta) is None  # none yet
    pc.cache_write(path, meta, arrays)
    assert not (tmp_path / "w.tmp").exists()
    got = pc.cache_read(path, meta)
    assert set(got) == {"codes", "scale"} and np.array_equal(got["codes"], arrays["codes"])
    other = dict(meta, weight="y")
    with pytest.raises(pc.PackCacheMismatch, match="weight"):
        pc.cache_read(path, other)
    assert json.loads((path / "meta.json").read_text()) == meta  # not overwritten
    assert pc.cache_read(path, other, rebuild=True) is None
    np.save(path / "codes.npy", np.zeros(256, np.uint8))  # damaged
    with pytest.raises(pc.PackCacheMismatch, match="damaged"):
        pc.cache_read(path, meta)
    assert pc.cache_read(path, meta, verify=False) is not None
    a = torch.arange(10000, dtype=torch.float32).reshape(100, 100)
    assert pc.fingerprint(a) == pc.fingerprint(a.clone()) and pc.fingerprint(a) != pc.fingerprint(a + 1)


def test_row_slices_match_the_reference_rule():
    """row_slices cuts x's tile rows into slices of 4 (8 with full_sync), the last one short (reference linear.py:
    179-184): 1 row is one tile row, 200 rows seven, 257 rows nine."""
    x = torch.zeros(1, 1, 200, 64)
    assert linear.row_slices(x) == [(0, 4), (4, 3)]
    assert linear.row_slices(x, full_sync=True) == [(0, 7)]
    assert linear.row_slices(torch.zeros(1, 64)) == [(0, 1)]
    assert linear.row_slices(torch.zeros(257, 64), True) == [(0, 8), (8, 1)]


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4", "bf16"])
def test_block_float_on_the_host(fmt):
    """block_float with no device rounds on the host, bit for bit as the oracle's restatement of the reference's host
    conversion (and, at a small size, as its Fraction-exact form): ragged columns (a face row cut short is padded with
    zeros), rows not a multiple of 32, rank 3, values spanning the exponent range (both ends of a row's exponents,
    zeros, denormals, rounding ties, 2^mb - 1 overflow to the cap)."""
    from oracle import dense_oracle as O

    g = torch.Generator().manual_seed(5)
    t = torch.randn(3, 37, 70, generator=g) * torch.exp2(torch.randint(-100, 100, (3, 37, 70), generator=g).float())
    t[0, 0, :16] = torch.tensor([1.0, -1.0, 2.0**-127, -(2.0**-130), 0.0, -0.0, 1.5, 1.75, 1.875, 1.9375, 1.96875,
                                 1.984375, 1.9921875, 3.0, 2.0**-30, 2.0**-31])
    t[1, 5, 32:48] = 2.0**-125 * torch.arange(1, 17).float()
    t[2, 9, 48:64] = torch.tensor([2.0**127] * 8 + [-(2.0**126)] * 8)
    dt = {"bfp8": linear.bfloat8_b, "bfp4": linear.bfloat4_b, "bf16": linear.bfloat16}[fmt]
    got = linear.block_float(t, dt)
    assert got.shape == t.shape and got.dtype == torch.float32
    if fmt == "bf16":
        assert torch.equal(got, t.to(torch.bfloat16).float())
        return
    for i in range(3):
        rows = np.zeros((64, 70), np.float32)  # (the oracle takes whole tiles: the rows round apart)
        rows[:37] = t[i].numpy()
        want = O.held(rows, fmt)[:37]
        assert np.array_equal(got[i].numpy().view(np.uint32), want.astype(np.float32).view(np.uint32)), i
    small = t[0, :4, :32].numpy()
    assert np.array_equal(got[0, :4, :32].numpy().astype(np.float64), O.held_exact(small, fmt))
