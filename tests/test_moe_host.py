"""MoE checks that need no GPU: the C ABI structs of include/moe.h against their ctypes mirrors, the host BFP4_b tile
conversion (moe8.bfp4_tiles / bfp4_values) against the oracle's block-float restatement, the oracle's MoE
restatement pinned by closed forms, invariants and brute force, and moe8's host references against the oracle."""

import ctypes
import math
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from dense_reader import _lib
from moe import moe8
from oracle import dense_oracle as O
from oracle import moe_oracle as MO

ROOT = Path(__file__).resolve().parents[1]


def test_moe_structs_match_c(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "moe.h"\n'
        "int main(void){printf(\"%zu %zu %zu %zu %zu %zu %zu %zu\\n\", sizeof(dr_moe), offsetof(dr_moe, w),"
        " offsetof(dr_moe, codes_stride), offsetof(dr_moe, bias), sizeof(dr_route), offsetof(dr_route, scale),"
        " offsetof(dr_route, slot), offsetof(dr_route, stream));return 0;}\n"
    )
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    want = [
        ctypes.sizeof(_lib.Moe),
        _lib.Moe.w.offset,
        _lib.Moe.codes_stride.offset,
        _lib.Moe.bias.offset,
        ctypes.sizeof(_lib.Route),
        _lib.Route.scale.offset,
        _lib.Route.slot.offset,
        _lib.Route.stream.offset,
    ]
    assert got == want


def _weights(seed, k=96, n=128):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(k, n, generator=g) * 0.02
    w[3, 5], w[7, 9], w[10, 11] = 0.0, -1e-30, 2.0**-126 * 0.5  # a zero and denormals
    w[40:42, 64:80] = torch.tensor([0.09375, 0.078125]).reshape(2, 1)  # exact ties of the 3-bit grid
    return w


def test_bfp4_tiles_match_oracle():
    w = _weights(1)
    assert np.array_equal(moe8.bfp4_tiles(w), O.bfp_tiles(w, "bfp4"))
    v = moe8.bfp4_values(moe8.bfp4_tiles(w))
    assert np.array_equal(v, O.tile_values(O.bfp_tiles(w, "bfp4"), "bfp4"))


def test_bfp4_tiles_kblock_is_the_transposed_blocks():
    """kblock: each 32 x 32 block transposed in its tile, so its face rows run along K: the tiles of the matrix whose
    blocks are transposed, and the values come back in [K, N] order."""
    w = _weights(2)
    k, n = w.shape
    wt = w.reshape(k // 32, 32, n // 32, 32).transpose(1, 3).reshape(k, n)  # every block transposed in place
    assert np.array_equal(moe8.bfp4_tiles(w, kblock=True), O.bfp_tiles(wt, "bfp4"))
    vals = moe8.bfp4_values(moe8.bfp4_tiles(w, kblock=True), kblock=True)
    held_t = O.held(wt, "bfp4").reshape(k // 32, 32, n // 32, 32).transpose(0, 2, 3, 1)  # blocks turned back
    assert np.array_equal(vals, held_t)
    # the oracle's kblock values: the same tiles' values in [K, N] order
    assert np.array_equal(MO.held_kblock(w), vals.transpose(0, 2, 1, 3).reshape(k, n))


def test_held_kblock_groups_run_along_k():
    """A hand-made matrix: each 16-K group at one N holds one value 1.0 and fifteen 2^-3 + 2^-5; along K those round to
    the group's grid of 2^-2 steps (3-bit magnitudes under the exponent of 1.0): 0.15625 is 0.625 of a step, so 0.25;
    along N (the plain pack) their face rows hold no 1.0 and keep 2^-3 + 2^-5 (magnitude 101b) exactly."""
    w = np.full((64, 32), 2.0**-3 + 2.0**-5, np.float32)
    w[0::16, :] = 1.0
    h = MO.held_kblock(w)
    assert np.all(h[0::16] == 1.0)
    rest = np.ones(64, bool)
    rest[0::16] = False
    assert np.all(h[rest] == 0.25), np.unique(h[rest])
    assert np.all(O.held(w, "bfp4")[rest] == w[rest])


def test_moe_oracle_glu_closed_forms():
    g = np.array([-3.0, -0.5, 0.0, 0.5, 3.0, 7.0, 9.0, np.nan])
    u = np.array([1.0, 2.0, 3.0, -1.0, 10.0, -10.0, 0.5, 1.0])
    assert MO.glu(np.array([0.0]), np.array([5.0]), "silu")[0] == 0.0
    torch_gelu = torch.nn.functional.gelu(torch.tensor(g[:-1]), approximate="tanh").numpy() * u[:-1]
    assert np.allclose(MO.glu(g[:-1], u[:-1], "gelu_tanh"), torch_gelu, rtol=1e-15, atol=1e-15)
    silu = g[:-1] / (1 + np.exp(-g[:-1])) * u[:-1]
    assert np.allclose(MO.glu(g[:-1], u[:-1], "silu"), silu, rtol=1e-15, atol=0)
    oai = MO.glu(g, u, "swiglu_oai")
    # g = 9 is capped at 7; u = 10 and -10 clamp to 7 and -7 before the + 1
    assert oai[6] == pytest.approx(7.0 / (1 + math.exp(-1.702 * 7.0)) * 1.5, rel=1e-15)
    assert oai[4] == pytest.approx(3.0 / (1 + math.exp(-1.702 * 3.0)) * 8.0, rel=1e-15)
    assert oai[5] == pytest.approx(7.0 / (1 + math.exp(-1.702 * 7.0)) * -6.0, rel=1e-15)
    assert math.isnan(oai[7])


def _small_layer(seed, E=4, H=64, I=32):
    g = torch.Generator().manual_seed(seed)
    gu = (torch.randn(E, H, 2 * I, generator=g) * 0.1).double()
    dn = (torch.randn(E, I, H, generator=g) * 0.1).double()
    x = torch.randn(H, generator=g).double()
    return gu, dn, x


def test_moe_oracle_layer_invariants():
    gu, dn, x = _small_layer(3)
    E, H, I2 = gu.shape
    I = I2 // 2
    for act in ("silu", "gelu_tanh", "swiglu_oai"):
        y2, h2 = MO.layer(x, gu, dn, [1, 3], [0.25, 0.75], act)
        ya, ha = MO.layer(x, gu, dn, [1], [0.25], act)
        yb, hb = MO.layer(x, gu, dn, [3], [0.75], act)
        assert np.allclose(y2, ya + yb, rtol=1e-12, atol=1e-14)  # y: the sum of the slots alone
        assert np.array_equal(h2, np.concatenate([ha, hb]))  # h: the slots side by side
        y4, h4 = MO.layer(x, gu, dn, [1, 3], [0.5, 1.5], act)
        assert np.allclose(h4, 2 * h2, rtol=1e-15) and np.allclose(y4, 2 * y2, rtol=1e-12)  # linear in w
    # the gate half (columns I..2I-1) driven to -1e4 with x > 0: silu's gate is 0, so h = 0; the up half does not
    xp = np.abs(x.numpy()) + 0.1
    gz = gu.clone()
    gz[:, :, I:] = -1e4 / H
    assert np.allclose(MO.layer(xp, gz, dn, [0, 2], [1.0, 1.0], "silu")[1], 0.0, atol=1e-30)
    uz = gu.clone()
    uz[:, :, :I] = -1e4 / H
    assert np.abs(MO.layer(xp, uz, dn, [0], [1.0], "silu")[1]).max() > 1.0
    # a bias of minus x U (on the bf16 grid) cancels the up half exactly when x U is itself on the grid
    gb = gu.clone()
    gb[:, :, :I] = 0.0
    gb[:, 0, :I] = 0.5  # x U = x[0] * 0.5
    xb = np.zeros(H)
    xb[0] = 2.0  # x U = 1.0 on every up column
    bias = np.zeros((E, 2 * I), np.float32)
    bias[:, :I] = -1.0
    assert np.abs(MO.layer(xb, gb, dn, [2], [1.0], "silu", bias)[1]).max() == 0.0


def test_moe_oracle_layer_hand_case():
    """Two experts of H = 2, I = 1: x = (1, 2); expert 0 up (1, 0) gate (0, 1), down (2, -1); expert 1 up (0, 1) gate
    (1, 0), down (1, 1). Slots (0 at 0.5, 1 at 2): h = (0.5 silu(2) * 1, 2 silu(1) * 2), y = h0 (2, -1) + h1 (1, 1)."""
    gu = np.zeros((2, 2, 2))
    gu[0, :, 0], gu[0, :, 1] = (1, 0), (0, 1)  # [up | gate]
    gu[1, :, 0], gu[1, :, 1] = (0, 1), (1, 0)
    dn = np.array([[[2.0, -1.0]], [[1.0, 1.0]]])
    y, h = MO.layer(np.array([1.0, 2.0]), gu, dn, [0, 1], [0.5, 2.0], "silu")
    s2, s1 = 2 / (1 + math.exp(-2)), 1 / (1 + math.exp(-1))
    assert np.allclose(h, [0.5 * s2, 2 * s1 * 2], rtol=1e-15)
    assert np.allclose(y, [h[0] * 2 + h[1], -h[0] + h[1]], rtol=1e-15)


def test_moe_oracle_union_brute_force():
    ids = np.array([[5, 3, 9, 3], [0, 17, 5, 2]])
    assert MO.union(ids, 16) == [0, 2, 3, 5, 9]
    assert MO.union(ids, 4) == [0, 2, 3]
    assert moe8.union(torch.tensor(ids), 16) == MO.union(ids, 16)


def test_moe_oracle_route_brute_force():
    lg = np.array([[0.5, 2.0, 2.0, -1.0, 2.0, 0.0, 1.0, 2.0]])
    ids, w = MO.route(lg, 3)
    assert ids == [[1, 2, 4]]  # four logits tie at 2.0: the three lowest ids
    assert sum(w[0]) == pytest.approx(1.0, abs=1e-15) and w[0][0] == w[0][2]
    ids, w = MO.route(lg, 3, scale=2.5)
    assert sum(w[0]) == pytest.approx(2.5, abs=1e-14)
    ids, w = MO.route(lg, 2, kind="sigmoid", norm=False, slot=7)
    assert ids == [[1, 2, 7]] and w[0][2] == 1.0 and w[0][0] == pytest.approx(1 / (1 + math.exp(-2.0)))


def test_moe_oracle_route_groups_hand_case():
    """Four groups of two experts, keys 0.9 and -0.5 (group 0: score 0.4), 0.6 and 0.6 (1.2), 0.3 and 0.3 (0.6), 0.1
    and 0.1 (0.2). With two groups kept (1 and 2) the best single expert, 0, is dropped with its group."""
    lg = np.zeros((1, 8))
    bias = np.array([0.9, -0.5, 0.6, 0.6, 0.3, 0.3, 0.1, 0.1]) - 0.5  # keys = sigmoid(0) + bias = bias + 0.5
    ids, _ = MO.route(lg, 2, kind="sigmoid", bias=bias, groups=(4, 2))
    assert ids == [[2, 3]]
    ids, _ = MO.route(lg, 3, kind="sigmoid", bias=bias, groups=(4, 2))
    assert ids == [[2, 3, 4]]
    ids, _ = MO.route(lg, 1, kind="sigmoid", bias=bias)
    assert ids == [[0]]


def test_moe8_references_match_oracle():
    gu, dn, x = _small_layer(4, E=6)
    bias = (torch.randn(6, 64, generator=torch.Generator().manual_seed(5)) * 0.3).float()
    for act in ("silu", "gelu_tanh", "swiglu_oai"):
        for b in (None, bias):
            wt = torch.tensor([0.2, 0.3, 0.5])
            y, h = moe8.reference(x.float(), gu.float(), dn.float(), [4, 1, 5], wt, act, b)
            yo, ho = MO.layer(x.float().numpy(), gu.float().numpy(), dn.float().numpy(), [4, 1, 5], wt.numpy(),
                              act, None if b is None else b.numpy())
            assert np.allclose(h.numpy().reshape(-1), ho, rtol=1e-12, atol=1e-15), act
            assert np.allclose(y.numpy().reshape(-1), yo, rtol=1e-12, atol=1e-15), act


def test_moe8_route_reference_matches_oracle():
    g = torch.Generator().manual_seed(6)
    lg = torch.randn(6, 64, generator=g) * 3
    lg[::2] = lg[::2].to(torch.bfloat16).float()  # ties
    bias = torch.randn(64, generator=g) * 0.1
    cases = [
        dict(kind="softmax", k=8),
        dict(kind="softmax", k=4, scale=2.5),
        dict(kind="sigmoid", k=6, bias=bias),
        dict(kind="sigmoid", k=6),
        dict(kind="sigmoid", k=8, norm=False),
        dict(kind="sigmoid", k=8, bias=bias, groups=(8, 4), scale=2.5, slot=70),
    ]
    for c in cases:
        c = dict(c)
        k = c.pop("k")
        ids, w = moe8.route_reference(lg, k, **c)
        oi, ow = MO.route(lg.numpy(), k, bias=None if c.get("bias") is None else c["bias"].numpy(),
                          **{a: v for a, v in c.items() if a != "bias"})
        assert ids.tolist() == oi, c
        assert np.allclose(w.numpy(), np.array(ow), rtol=1e-12, atol=0), c


def test_gu_pairs_rotate_by_expert():
    """gu_pairs (reference moe8.py:199-201): every bank's parts of an expert's pairs tile them exactly once, in bank
    order from the part the rotation starts at; the larger parts (16 pairs on 3 banks: 6, 5, 5) move one bank on per
    expert; 2880 / 32 = 90 pairs on 8 banks give parts of 12 and 11."""
    assert [moe8.gu_pairs(0, b, 3) for b in range(3)] == [(0, 6), (6, 5), (11, 5)]
    assert [moe8.gu_pairs(1, b, 3) for b in range(3)] == [(11, 5), (0, 6), (6, 5)]
    assert [moe8.gu_pairs(2, b, 3) for b in range(3)] == [(6, 5), (11, 5), (0, 6)]
    for e in range(10):
        for banks, pairs in ((8, 90), (3, 16), (5, 4), (1, 7)):
            got = sorted(moe8.gu_pairs(e, b, banks, pairs) for b in range(banks))
            assert sum(c for _, c in got) == pairs
            assert all(s0 + c == s1 for (s0, c), (s1, _) in zip(got, got[1:])) and got[0][0] == 0
            assert {c for _, c in got} <= {pairs // banks, -(-pairs // banks)}
