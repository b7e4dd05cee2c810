"""The reference's example and the planner's answers on the GPU.

- The port of the reference's `examples/dense_reader_example.py` that the repository's integration guide gives, run
  as it is written there (the guide's example code block, with the repository's path filled in), then checked as the
  reference's example checks itself (examples/dense_reader_example.py:24-27): y against the float64 product of x
  (bf16) and the weight's own held values, relative Frobenius error below 1 %.
- plan(): the reference plan's keys (dense_reader/linear.py:187-382) for launches of each kernel, its `work` list
  covering every output column once a K split, and its LDS figure the kernel's own.
- block_float on the host gives the GPU packing's values bit for bit.
"""

import re
from pathlib import Path

import numpy as np
import pytest
import torch

from dense_reader import linear
from oracle import dense_oracle as O

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]


def _example_code():
    text = (ROOT / "INTEGRATION.md").read_text()
    sec = text[text.index("## 2. The reference's example") : text.index("## 3.")]
    code = re.search(r"```python\n(.*?)```", sec, re.S).group(1)
    return code.replace("<repo>", str(ROOT))


def test_reference_example_as_ported(device):
    code = _example_code()
    assert "linear.matmul(tx, tw, None" in code and "linear.native_weight(device, w, linear.bfloat8_b)" in code
    ns = {}
    exec(compile(code, "INTEGRATION.md#2", "exec"), ns)  # noqa: S102 (the repository's own document)
    x, y, wk = ns["x"], ns["y"], ns["wk"]
    assert y.shape == (1, 2048) and wk.shape == (1024, 2048)
    ref = x.double() @ wk.double()
    rel = ((y.double() - ref).norm() / ref.norm()).item()
    print(f"dense_reader example: y = x @ w for one token, relative error {100 * rel:.3f} % against torch")
    assert rel < 0.01, rel
    # the held values are the oracle's bfloat8_b of the same matrix, bit for bit
    want = O.held(ns["w"].T.contiguous().numpy(), "bfp8")
    assert np.array_equal(wk.numpy().view(np.uint32), want.astype(np.float32).view(np.uint32))


def _covers(p, n_out):
    """Every output column of [0, n_out) once a K split in p's work list."""
    splits = p["splits"]
    seen = np.zeros((splits, -(-n_out // 16) * 16), np.int32)
    for i, (xcd, block, split, c0, nc, n0) in p["work"]:
        assert xcd == i % 8
        seen[split, n0 : n0 + nc] += 1
    assert (seen[:, :n_out] == 1).all(), np.argwhere(seen[:, :n_out] != 1)[:4]


@pytest.mark.parametrize(
    "m, k, n, fmt, kernel, tile_cols, splits",
    [
        (1, 4096, 14336, "bfp8", "gemv", 32, 1),  # the north star
        (1, 2048, 1000, "bfp4", "gemv", 16, 1),  # few tiles: 16-column tiles
        (8, 14336, 4096, "bfp8", "mfma", 32, 2),  # C3's shape: K split in two
        (32, 1024, 16384, "bfp8", "mfma", 32, 1),  # 32 rows over more tiles than CUs: tile pairs
    ],
)
def test_plan_keys_and_work(device, m, k, n, fmt, kernel, tile_cols, splits):
    wt = O.matrix(n, k, 3)
    tw, _ = linear.native_weight(device, wt, {"bfp8": linear.bfloat8_b, "bfp4": linear.bfloat4_b}[fmt])
    tx = torch.zeros(1, 1, m, k, dtype=torch.bfloat16, device=device.torch)
    p = linear.plan(device, tx, tw)
    for key in ("MT", "KT", "NT", "KB", "KW", "SBW", "NC", "W_PAGES", "sharded", "split", "rows", "native", "xs",
                "noscale", "glu", "glu2", "out32", "SEGS", "seg_work", "work", "l1"):
        assert key in p, key
    assert (p["kernel"], p["tile_cols"], p["splits"]) == (kernel, tile_cols, splits), p
    assert (p["MT"], p["KT"], p["NT"], p["KB"], p["SEGS"]) == (-(-m // 32), k // 32, -(-n // 32), k // 32, 1)
    assert p["KW"] * 32 == p["kch"] and p["native"] == linear.native_tile(tw)
    assert len(p["work"]) == p["workgroups"] and p["l1"] > 0
    if m == 32:
        assert p["tiles_per_workgroup"] == 2 and p["NC"] == 2
    _covers(p, n)
    assert linear.choose(device, tx, tw)[0][1]["work"] == p["work"]


def test_plan_of_a_block_list(device):
    """A block list's plan: each block's workgroups (seg_work), together covering the blocks' output columns once."""
    k = 1024
    a, _ = linear.native_weight(device, O.matrix(512, k, 4), linear.bfloat8_b)
    b, _ = linear.native_weight(device, O.matrix(256, k, 5), linear.bfloat16)
    tx = torch.zeros(1, 1, 1, k, dtype=torch.bfloat16, device=device.torch)
    p = linear.plan(device, tx, a, blocks=[(a, 0), (b, 16)])
    assert p["SEGS"] == 2 and len(p["seg_work"]) == 2
    assert sorted(i for s in p["seg_work"] for i in s) == list(range(len(p["work"])))
    for blk, ids in enumerate(p["seg_work"]):
        assert all(p["work"][i][1][1] == blk for i in ids)
    _covers(p, 16 * 32 + 256)


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4"])
def test_block_float_host_equals_device(device, fmt):
    g = torch.Generator().manual_seed(9)
    t = torch.randn(64, 200, generator=g) * torch.exp2(torch.randint(-60, 60, (64, 200), generator=g).float())
    dt = {"bfp8": linear.bfloat8_b, "bfp4": linear.bfloat4_b}[fmt]
    h = linear.block_float(t, dt)
    d = linear.block_float(t, dt, device=device)
    assert torch.equal(h.view(torch.int32), d.cpu().view(torch.int32))
