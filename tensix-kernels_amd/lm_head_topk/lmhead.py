"""lmhead.py: an LM head on the device that returns token ids, not logits (MI355X), after XylolabsInc/tensix-kernels'
lm_head_topk/lmhead.py (file:line cited per function).

The vocabulary is cut into `chunks` column blocks of the [dim, vocab] weight. Each block runs through the dense
reader's matmul (dense_reader.linear.matmul) with block-float weights, for up to 16 rows (tokens) at a time. No logits
are written: every 32-column tile of a block keeps the top-`k` of each row (linear.matmul's topk) as one small record,
so one small tensor holds every block's candidates.

With `rescore` (the default) the candidates' logits are recomputed exactly from the bf16 weight rows (x in bf16,
products summed in float32, rounded to bf16 unless logits="float32") and the largest is picked, the lowest token id
first on ties and a NaN counting as the largest (pick_token). The rescore and the pick run on the host (collect), or
with device_pick=True on the device (head_pick.py), which then returns only the token ids.

  head = DeviceHead(device, lm_head_weight, fmt="bfp4")                     # [vocab, dim] torch
  ids = head(x, rows)                                                       # x [1, 1, >= rows, dim] bf16 on the GPU
  head = DeviceHead(device, lm_head_weight, device_pick=True)               # rescore and pick on the device
  head = DeviceHead(device, sub_weight, rescore=False, device_pick=True, token_map=ids)   # a draft's sub-head
"""

import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
from common import device as dev  # noqa: E402
from dense_reader import linear  # noqa: E402
from lm_head_topk import head_pick  # noqa: E402

FORMATS = {"bfp8": linear.bfloat8_b, "bfp4": linear.bfloat4_b, "bf16": linear.bfloat16}


def pick_token(exact, ids, vocab):
    """The argmax over the rescored candidates: per row the lowest token id among the largest exact logits, a NaN
    counting as the largest (torch.argmax's rule). exact: [rows, c] float with -inf for empty slots, ids: [rows, c]
    token ids (reference lmhead.py:40-46)."""
    top = exact.max(dim=1, keepdim=True).values  # NaN where the row has one
    hit = (exact == top) | (exact.isnan() & top.isnan())
    return torch.where(hit, ids, torch.full_like(ids, vocab)).min(dim=1).values


class DeviceHead:
    """The LM head as `chunks` device matmuls with top-k records (reference lmhead.py:49-263)."""

    def __init__(
        self,
        device,
        weight,
        fmt="bfp4",
        chunks=16,
        k=8,
        rescore=True,
        top=16,
        blocks=None,
        logits="bf16",
        device_pick=False,
        rows=None,
        valid=None,
        token_map=None,
        l1x=True,
        **opts,
    ):
        """weight: the head [vocab, dim] (torch; kept on the host in bf16 for a host rescore). chunks: vocabulary
        blocks, one matmul each (vocab / chunks a multiple of 32). blocks: device weights already made, [(w [1, 1, dim,
        vocab / chunks], scale or None)] in vocabulary order; else made here in fmt ("bfp8", "bfp4" or "bf16"). k:
        candidates per 32-column tile and row; top: of all candidates, the best `top` by device logit are rescored.
        logits: the rescore's logits, "bf16" (rounded) or "float32". device_pick: the rescore and the pick on the
        device (head_pick.py) with a bf16 copy of the head on the device instead of the host's; `top` at most 32. rows:
        that bf16 copy when it is already on the device (head_pick.check_rows), used instead of a second one. valid: a
        padded head's real vocabulary for the device pick (pad rows never candidates). Without a rescore, device_pick
        is the records-only pick (head_pick.pick_records) and token_map maps the head's rows to token ids (a list or
        tensor of ids, or head_pick.token_map's device tensor). l1x is accepted and changes nothing (x is read where it
        lies). opts go to linear.matmul (reference lmhead.py:52-133)."""
        vocab, dim = weight.shape
        chunks = len(blocks) if blocks is not None else chunks
        step = vocab // chunks
        assert step * chunks == vocab and step % 32 == 0, (vocab, chunks)
        assert fmt in FORMATS, fmt
        assert logits in ("bf16", "float32"), logits
        self.round = logits == "bf16"
        self.logits = logits
        self.device_pick = bool(device_pick)
        self.l1x = l1x
        self.rows_t = None  # the bf16 head on the device (device_pick)
        self.own_rows = False
        self.valid = valid
        self.picks = {}  # rows -> the pick's output tensor (device_pick)
        self.records_pick = not rescore and self.device_pick
        self.tmap, self.own_tmap = None, False
        assert token_map is None or self.records_pick, "lmhead: token_map is for rescore=False, device_pick=True"
        self.device = dev.as_device(device)
        self.slots = linear.topk_slots(step)  # records per block: one a 32-column tile
        self.fmt, self.step, self.k, self.opts = fmt, step, k, opts
        self.vocab, self.dim, self.top = vocab, dim, top
        self.results = {}  # rows -> the top-k result tensor
        self.y = None  # the matmuls' placeholder output (never written)
        self.host = None
        if self.records_pick and token_map is not None:
            if isinstance(token_map, torch.Tensor) and token_map.is_cuda:
                self.tmap = token_map
            else:
                assert len(token_map) == vocab, (len(token_map), vocab)
                self.tmap, self.own_tmap = head_pick.token_map(self.device, token_map), True
        if rescore and self.device_pick:
            assert 1 <= top <= 32, f"lmhead: the device pick rescores at most 32 candidates, top {top}"
            if rows is not None:
                head_pick.check_rows(rows, dim, vocab if valid is None else valid)
                self.rows_t = rows
            else:
                self.rows_t = head_pick.head_rows(self.device, weight)
                self.own_rows = True
        elif rescore:
            self.host = weight.to(torch.bfloat16)
        self.miss = 0  # rows whose device-best candidate was not the rescored best
        if blocks is not None:
            self.blocks = list(blocks)
            return
        self.blocks = []
        for a in range(0, vocab, step):
            tw, _ = linear.native_weight(self.device, weight[a : a + step].float(), FORMATS[fmt])
            self.blocks.append((tw, None))  # unit scales: no scale tensor, no multiply

    def logits_topk(self, x, rows=1, ids_out=None):
        """The device part: per block the matmul keeping each tile's top-k of the first `rows` rows (no logits are
        written), then with device_pick the rescore and the pick. Returns the result tensor (block b's records at b *
        slots ..). ids_out (a device pick only): row 0's token also into this one-element int32 tensor. Nothing is
        read back and the tensors are kept from call to call, so a HIP graph can capture it (reference
        lmhead.py:135-193)."""
        assert 1 <= rows <= 16 and rows <= x.shape[-2], f"lmhead: 1 to 16 rows, at most x's ({rows})"
        r = self.results.get(rows)
        if r is None:
            r = self.results[rows] = linear.topk_result(self.device, len(self.blocks) * self.slots, rows, self.k)
        if self.y is None or self.y.shape[-2] != x.shape[-2]:
            self.y = torch.empty(1, 1, x.shape[-2], self.step, dtype=torch.bfloat16, device=self.device.torch)
        for b, (tw, ts) in enumerate(self.blocks):
            spec = {"r": r, "k": self.k, "rows": rows, "slot0": b * self.slots}
            spec |= {"base": b * self.step, "n": self.step, "write_y": False}
            linear.matmul(x, tw, ts, topk=spec, out=self.y, **self.opts)
        if self.rows_t is not None:
            self.picks[rows] = head_pick.pick(
                r,
                x,
                self.rows_t,
                rows,
                self.k,
                top=self.top,
                logits=self.logits,
                out=self.picks.get(rows),
                valid=self.valid,
                ids_out=ids_out,
            )
        elif self.records_pick:
            self.picks[rows] = head_pick.pick_records(
                r,
                rows,
                self.k,
                self.vocab if self.valid is None else self.valid,
                tmap=self.tmap,
                out=self.picks.get(rows),
                ids_out=ids_out,
            )
        assert ids_out is None or rows in self.picks, "lmhead: ids_out needs the device pick"
        return r

    def candidates(self, x, rows):
        """(values [rows, c] float, global ids [rows, c] long) of the device's candidates (reference
        lmhead.py:195-198)."""
        r = self.logits_topk(x, rows)
        return linear.topk_records(r, rows, self.k)

    def rescore(self, xh, ids):
        """Exact logits of the candidates: x (bf16) times the bf16 weight rows, float32 sums on the host, rounded to
        bf16 (unless logits="float32") (reference lmhead.py:200-205)."""
        w = self.host[ids.reshape(-1)].float().reshape(*ids.shape, self.dim)
        z = torch.einsum("rd,rcd->rc", xh.float(), w)
        return z.to(torch.bfloat16).float() if self.round else z

    def __call__(self, x, rows=1):
        """Token ids [rows] (long) for the first `rows` rows of x [1, 1, >= rows, dim] bf16 (reference
        lmhead.py:207-210)."""
        self.logits_topk(x, rows)
        return self.collect(x, rows)

    def collect(self, x, rows=1, xh=None):
        """The host part, after logits_topk ran (directly, or in a graph being replayed): with a device pick the token
        ids read back; else the records' readback, x's readback (or xh, a host copy of x's first rows) and the
        rescore. Token ids [rows] (long) (reference lmhead.py:212-239)."""
        if self.rows_t is not None:
            tok, best, _ = head_pick.tokens(self.picks[rows], rows)
            self.miss += int((best != tok).sum())
            return tok
        if self.records_pick:
            return head_pick.tokens(self.picks[rows], rows)[0]
        vh, ids = linear.topk_records(self.results[rows], rows, self.k)
        best = vh.argmax(dim=1)
        if self.host is None:
            return ids[torch.arange(rows), best]
        if xh is None:
            xh = x.reshape(-1, self.dim)[:rows].cpu()
        xh = xh.reshape(-1, self.dim)[:rows].to(torch.bfloat16)
        if self.top and self.top < ids.shape[1]:
            pick = vh.topk(self.top, dim=1).indices
            vh, ids = vh.gather(1, pick), ids.gather(1, pick)
            best = vh.argmax(dim=1)
        valid = ids >= 0  # (empty records: -1)
        ids = ids.clamp(min=0)
        exact = self.rescore(xh, ids)
        exact = torch.where(valid, exact, torch.full_like(exact, float("-inf")))
        tok = pick_token(exact, ids, self.vocab)
        self.miss += int((ids[torch.arange(rows), best] != tok).sum())
        return tok

    def deallocate(self):
        """Drops the device tensors this head made (the caller's rows table and token map stay) (reference
        lmhead.py:241-263)."""
        self.picks = {}
        if self.tmap is not None and self.own_tmap:
            self.tmap = None
        if self.rows_t is not None and self.own_rows:
            self.rows_t = None
        self.results = {}
        self.y = None
        self.blocks = []
