"""The top-k LM head (lm_head_topk/lmhead.py, head_pick.py) on the GPU against the CPU oracle, after
XylolabsInc/tensix-kernels lm_head_topk/tests/test_lm_head.py, test for test.

A random bf16 head [vocab, dim] on a bfloat4_b device head and random x rows:
- the records: every kept (value, id) is the bf16 logit the block matmul computes at that id, and each row's best k
  over the records equal its best k over all logits (the same op's y, written), bit for bit;
- the host rescore's tokens against the oracle's bf16 head (x times the bf16 rows, rounded to bf16, the lowest id among
  the largest), token for token;
- the device pick (head_pick.pick) against the oracle's restatement of it on the same records and against the host
  rescore, in bf16 and float32 logits, on a head whose rows repeat in pairs (exact ties: the lowest id must win) and on
  a padded head (valid=), its table also given as the valid rows only;
- the records-only pick (pick_records) with and without a token map against the host's argmax over the same records;
- both picks with k 4 at 1 and 3 rows.
A token may differ from the oracle's only where the two logits tie within float32 rounding of the sum (the device sums
in its own order, as the reference's does); every such case is named in the output.
"""

import numpy as np
import pytest
import torch

from common.testing import same
from dense_reader import _lib, linear
from lm_head_topk import head_pick, lmhead
from oracle import dense_oracle as O

pytestmark = pytest.mark.gpu

VOCAB, DIM, CHUNKS = 8192, 1024, 4


def head(seed, pairs=False):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(VOCAB, DIM, generator=g) * 0.05).to(torch.bfloat16)
    if pairs:
        w[1::2] = w[0::2]  # rows 2i and 2i + 1 equal: every logit ties with its pair
    return w


def x_rows(device, rows, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, DIM, generator=g).to(torch.bfloat16)
    return x, x.reshape(1, 1, rows, DIM).to(device.torch)


def oracle_tokens(x, w, logits="bf16"):
    z = O.head_logits(x, w, logits).numpy()
    return O.pick_token(z, np.broadcast_to(np.arange(VOCAB), z.shape), VOCAB), z


def same_tokens(name, got, want, z=None):
    """Token for token; where they differ, the two logits must tie within float32 rounding of the sum (z: the
    oracle's logits [rows, vocab])."""
    got, want = np.asarray(got, np.int64), np.asarray(want, np.int64)
    bad = np.nonzero(got != want)[0]
    for r in bad:
        assert z is not None, (name, r, got[r], want[r])
        a, b = float(z[r, got[r]]), float(z[r, want[r]])
        assert abs(a - b) <= 2e-6 * max(abs(a), abs(b), 1.0), (name, r, got[r], want[r], a, b)
        print(f"note {name}: row {r} token {got[r]} vs {want[r]}, a float32 tie ({a} vs {b})", flush=True)
    print(f"ok   {name}: {len(got) - len(bad)} of {len(got)} tokens equal, the rest float32 ties", flush=True)


def test_records(device):
    w = head(1)
    rows, k = 3, 8
    x, tx = x_rows(device, rows, 2)
    dh = lmhead.DeviceHead(device, w, fmt="bfp4", chunks=CHUNKS, k=k, rescore=False)
    vals, ids = dh.candidates(tx, rows)
    ys = [linear.matmul(tx, tw, None).float().cpu().reshape(-1, dh.step)[:rows] for tw, _ in dh.blocks]
    y = torch.cat(ys, 1)
    for t in range(rows):
        ok = ids[t] >= 0
        same(f"records row {t}: values at their ids", y[t][ids[t][ok]], vals[t][ok])
        top = torch.sort(vals[t][ok], descending=True).values[:k]
        same(f"records row {t}: the best {k} of all logits", top, torch.topk(y[t], k).values)
    dh.deallocate()


def test_host_rescore(device):
    w = head(3)
    dh = lmhead.DeviceHead(device, w, fmt="bfp4", chunks=CHUNKS)
    for rows in (1, 5):
        x, tx = x_rows(device, rows, 4 + rows)
        want, z = oracle_tokens(x, w)
        same_tokens(f"host rescore rows {rows}: tokens against the bf16 head", dh(tx, rows).numpy(), want, z)
    dh.deallocate()


def _device_vs_oracle(name, dev, tx, x, w, rows, logits, valid=None):
    got = dev(tx, rows).numpy()
    words = dev.results[rows].reshape(dev.results[rows].shape[-2], -1).cpu().numpy()
    want, first, count = O.pick_from_records(words, rows, dev.k, dev.top, x, w, logits, valid)
    z = O.head_logits(x, w, logits).numpy()
    same_tokens(f"{name}: tokens against the oracle's pick of the same records", got, want, z)
    _, best, n = head_pick.tokens(dev.picks[rows], rows)
    assert np.array_equal(best.numpy(), first) and np.array_equal(n.numpy(), count), (name, best, first, n, count)
    return got, z


def test_device_pick(device):
    for kind, w in (("random", head(5)), ("ties", head(6, pairs=True))):
        for logits in ("bf16", "float32"):
            host = lmhead.DeviceHead(device, w, fmt="bfp4", chunks=CHUNKS, logits=logits)
            dev = lmhead.DeviceHead(device, w, fmt="bfp4", chunks=CHUNKS, logits=logits, device_pick=True)
            for rows in (1, 4):
                x, tx = x_rows(device, rows, 7 + rows)
                got, z = _device_vs_oracle(f"device pick ({kind}, {logits}) rows {rows}", dev, tx, x, w, rows, logits)
                same_tokens(f"device pick ({kind}, {logits}) rows {rows}: against the host rescore",
                            got, host(tx, rows).numpy(), z)
                if kind == "random" and logits == "bf16":
                    want, zz = oracle_tokens(x, w)
                    same_tokens(f"device pick rows {rows}: against the bf16 head", got, want, zz)
            dev.deallocate()
            host.deallocate()


def test_small_records(device):
    w = head(14)
    for rows in (1, 3):
        x, tx = x_rows(device, rows, 15 + rows)
        host = lmhead.DeviceHead(device, w, fmt="bfp4", chunks=CHUNKS, k=4)
        dev = lmhead.DeviceHead(device, w, fmt="bfp4", chunks=CHUNKS, k=4, device_pick=True)
        got, z = _device_vs_oracle(f"device pick, k 4, rows {rows}", dev, tx, x, w, rows, "bf16")
        same_tokens(f"device pick, k 4, rows {rows}: against the host rescore", got, host(tx, rows).numpy(), z)
        plain = lmhead.DeviceHead(device, w, fmt="bfp4", chunks=CHUNKS, k=4, rescore=False)
        vals, ids = plain.candidates(tx, rows)
        picked = lmhead.DeviceHead(device, w, fmt="bfp4", chunks=CHUNKS, k=4, rescore=False, device_pick=True)
        best = ids[torch.arange(rows), vals.argmax(dim=1)]
        same(f"records pick, k 4, rows {rows}: against the host's argmax over the records", picked(tx, rows), best)
        for h in (host, dev, plain, picked):
            h.deallocate()


def test_padded_head(device):
    w = head(9)
    valid = VOCAB - 3 * 32 - 5  # the last rows are padding: never candidates
    rows, k = 2, 8
    x, tx = x_rows(device, rows, 10)
    dh = lmhead.DeviceHead(device, w, fmt="bfp4", chunks=CHUNKS, k=k, rescore=False)
    r = dh.logits_topk(tx, rows)
    rows_t = head_pick.head_rows(device, w)
    out = head_pick.pick(r, tx, rows_t, rows, k, valid=valid)
    tok, _, _ = head_pick.tokens(out, rows)
    words = r.reshape(r.shape[-2], -1).cpu().numpy()
    want, _, _ = O.pick_from_records(words, rows, k, 16, x, w, "bf16", valid)
    z = O.head_logits(x, w).numpy()
    same_tokens(f"padded head (valid {valid}): tokens against the oracle's pick", tok.numpy(), want, z)
    assert int(tok.max()) < valid
    short = head_pick.head_rows(device, w[:valid])
    dv = lmhead.DeviceHead(device, w, fmt="bfp4", chunks=CHUNKS, k=k, device_pick=True, valid=valid, rows=short)
    same_tokens(f"padded head (valid {valid}), a table of the valid rows only", dv(tx, rows).numpy(), want, z)
    dv.deallocate()
    dh.deallocate()


def test_pick_ids_from_records(device):
    """Where the slots or the vocabulary pass 2**24, dr_head_pick reads each candidate's id from the records instead of
    carrying it in the candidate's key: the same records with a validity bound past 2**24 (every id in them is still
    below the table's rows, so the same rows are read) must give the same page, word for word, and the oracle's
    tokens."""
    w = head(17)
    rows, k, top = 3, 8, 16
    x, tx = x_rows(device, rows, 18)
    dh = lmhead.DeviceHead(device, w, fmt="bfp4", chunks=CHUNKS, k=k, rescore=False)
    r = dh.logits_topk(tx, rows)
    rows_t = head_pick.head_rows(device, w)
    packed = head_pick.pick(r, tx, rows_t, rows, k, top=top).clone()
    words = head_pick._words(r, rows, k)
    out = torch.zeros_like(packed)
    stream = torch.cuda.current_stream(tx.device)
    wp, wn = head_pick._select_workspace(tx.device, stream, words.shape[0], rows, k)
    x2 = tx.reshape(-1, DIM)
    st = _lib.lib().dr_head_pick(words.data_ptr(), words.shape[0], rows, k, top, 1, x2.data_ptr(), DIM, DIM,
                                 rows_t.data_ptr(), DIM, (1 << 24) + 1, out.data_ptr(), None, wp, wn,
                                 stream.cuda_stream)
    _lib.check(st, "dr_head_pick")
    assert torch.equal(out.cpu(), packed.cpu()), (out.reshape(32, 32)[:rows, :3], packed.reshape(32, 32)[:rows, :3])
    tok, _, _ = head_pick.tokens(out, rows)
    want, _, _ = O.pick_from_records(words.cpu().numpy(), rows, k, top, x, w, "bf16", VOCAB)
    same_tokens("ids read from the records: tokens against the oracle's pick", tok.numpy(), want,
                O.head_logits(x, w).numpy())
    dh.deallocate()


def test_records_pick(device):
    w = head(11)
    rows, k = 3, 8
    g = torch.Generator().manual_seed(12)
    tmap = torch.randperm(1 << 20, generator=g)[:VOCAB]  # row i of the sub-head is token tmap[i]
    x, tx = x_rows(device, rows, 13)
    plain = lmhead.DeviceHead(device, w, fmt="bfp4", chunks=CHUNKS, k=k, rescore=False)
    vals, ids = plain.candidates(tx, rows)
    best = ids[torch.arange(rows), vals.argmax(dim=1)]  # the host's argmax over the same records
    picked = lmhead.DeviceHead(device, w, fmt="bfp4", chunks=CHUNKS, k=k, rescore=False, device_pick=True)
    same("records pick: rows against the host's argmax over the records", picked(tx, rows), best)
    mapped = lmhead.DeviceHead(
        device, w, fmt="bfp4", chunks=CHUNKS, k=k, rescore=False, device_pick=True, token_map=tmap.tolist()
    )
    same("records pick with a token map: tokens", mapped(tx, rows), tmap[best])
    ids_out = torch.zeros(1, dtype=torch.int32, device=device.torch)
    mapped.logits_topk(tx, rows, ids_out=ids_out)
    assert int(ids_out.cpu()[0]) == int(tmap[best[0]])
    for h in (plain, picked, mapped):
        h.deallocate()


def test_wide_blocks(device):
    """The reference's head sizing with blocks wider than the grid's records (lm_head_topk/lmhead.py:102-103: a
    block's records are the grid's cores, block b's from slot b * cores): two blocks of 16384 columns (512 tiles)
    into 2 x grid_slots() records. Every launch stays within its block's slots (tile pairs share a record), and the
    device pick over those records gives the oracle's pick of them and the bf16 head's tokens."""
    vocab, dim, chunks, k, rows = 32768, 512, 2, 8, 3
    step, S = vocab // chunks, linear.grid_slots()
    g = torch.Generator().manual_seed(21)
    w = (torch.randn(vocab, dim, generator=g) * 0.05).to(torch.bfloat16)
    x = torch.randn(rows, dim, generator=g).to(torch.bfloat16)
    tx = x.reshape(1, 1, rows, dim).to(device.torch)
    assert step // 32 > S, (step, S)
    r = linear.topk_result(device, chunks * S, rows, k)
    y = torch.empty(1, 1, rows, step, dtype=torch.bfloat16, device=device.torch)
    for b in range(chunks):
        tw, _ = linear.native_weight(device, w[b * step : (b + 1) * step].float(), linear.bfloat8_b)
        spec = {"r": r, "k": k, "rows": rows, "slot0": b * S, "base": b * step, "n": step, "write_y": False}
        linear.matmul(tx, tw, None, topk=spec, out=y)
    vals, ids = linear.topk_records(r, rows, k)
    ids = ids.reshape(rows, chunks, -1)
    for b in range(chunks):
        ok = ids[:, b] >= 0
        assert bool(((ids[:, b] // step == b) | ~ok).all()), f"block {b}'s slots hold another block's ids"
        assert bool(ok.all()), f"block {b}: every slot filled (each record spans 64 columns)"
    rows_t = head_pick.head_rows(device, w)
    tok, _, _ = head_pick.tokens(head_pick.pick(r, tx, rows_t, rows, k, top=16), rows)
    words = r.reshape(r.shape[-2], -1).cpu().numpy()
    want, _, _ = O.pick_from_records(words, rows, k, 16, x, w, "bf16", vocab)
    z = O.head_logits(x, w).numpy()
    same_tokens("wide blocks sized by the grid: device pick against the oracle's pick of the records", tok.numpy(),
                want, z)
    true = O.pick_token(z, np.broadcast_to(np.arange(vocab), z.shape), vocab)
    same_tokens("wide blocks sized by the grid: device pick against the bf16 head", tok.numpy(), true, z)
