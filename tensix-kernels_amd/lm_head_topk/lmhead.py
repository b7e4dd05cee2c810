"""lmhead.py: an LM head that hands back token ids instead of logits, on MI355X. The surface is XylolabsInc/
tensix-kernels' lm_head_topk/lmhead.py (DeviceHead, pick_token; file:line cited per function); the work is this
build's:

1. the vocabulary [vocab, dim] is cut into `chunks` column blocks, each packed once as a dense_reader weight
   [dim, vocab / chunks] (block-float or bf16);
2. per step, one dense_reader matmul a block with top-k records and no logits written: each launch ranks its columns
   on the device and leaves one record of the best `k` (value, id) of each row for every 32-column tile, block b's
   from slot b * slots (slots: the block's tiles);
3. the choice among the candidates:
   - rescore (default): the best `top` candidates by device value get their logits recomputed from the bf16 rows of
     the head (x as bf16, float32 sums, rounded to bf16 unless logits="float32"), and the largest wins, the lowest id
     among equals, NaN above everything (pick_token); on the host (collect), or with device_pick=True on the device
     (head_pick.pick), which leaves only the token ids to read;
   - rescore=False: the best record slot (head_pick.pick_records on the device, or the host's argmax), mapped through
     `token_map` when the head is a sub-head.

  head = DeviceHead(device, lm_head_weight, fmt="bfp4")                     # weight [vocab, dim] torch
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
    """Per row of exact [rows, c] (float, -inf in empty slots) the token of ids [rows, c] with the largest logit, the
    lowest id among equal ones, a NaN above every number (the rule of reference lmhead.py:40-46, torch.argmax's):
    rows holding a NaN choose among their NaNs, the others among their maxima."""
    nan = exact.isnan()
    inf = float("inf")
    numeric_max = exact.nan_to_num(nan=-inf, posinf=inf, neginf=-inf).amax(dim=1, keepdim=True)
    best = torch.where(nan.any(dim=1, keepdim=True), nan, exact == numeric_max)
    return torch.where(best, ids, torch.full_like(ids, vocab)).amin(dim=1)


class _Step:
    """The device tensors of one row count: the records every block's launch writes into, and the pick's page."""

    def __init__(self, head, rows):
        self.records = linear.topk_result(head.device, len(head.blocks) * head.slots, rows, head.k)
        self.page = None


class DeviceHead:
    """The LM head as one top-k matmul a vocabulary block and a pick over their records (reference
    lmhead.py:49-263)."""

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
        """weight: the head [vocab, dim] (torch). chunks: vocabulary blocks, one matmul each (vocab / chunks a multiple
        of 32), packed here in fmt ("bfp8", "bfp4" or "bf16"), or blocks: such weights already packed, [(w [1, 1, dim,
        vocab / chunks], scale or None)] in vocabulary order. k: candidates a record keeps for each row. top: how many
        of the best candidates are rescored (the device pick: at most 32). logits: "bf16" (the rescore's logits
        rounded to bf16) or "float32". device_pick: rescore and pick (or, without rescore, the records-only pick) on
        the device; rows: the head's bf16 table already on the device for it (head_pick.check_rows), else one is made
        here; valid: a padded head's real vocabulary (the pad rows never win); token_map: a sub-head's row -> token ids
        for the records-only pick (ids, or head_pick.token_map's device tensor). l1x changes nothing (x is read where
        it lies). opts go to linear.matmul (reference lmhead.py:52-133)."""
        vocab, dim = weight.shape
        nblk = len(blocks) if blocks is not None else chunks
        step = vocab // nblk
        assert step * nblk == vocab and step % 32 == 0, f"lmhead: {vocab} tokens in {nblk} blocks of 32-column tiles"
        assert fmt in FORMATS, fmt
        assert logits in ("bf16", "float32"), logits
        self.device = dev.as_device(device)
        self.vocab, self.dim, self.step, self.k, self.top = vocab, dim, step, k, top
        self.fmt, self.logits, self.opts, self.l1x = fmt, logits, opts, l1x
        self.round = logits == "bf16"
        self.device_pick = bool(device_pick)
        self.records_pick = self.device_pick and not rescore
        self.valid = valid
        # records a block's launch writes, the slot stride between blocks: one a 32-column tile (this head sizes its own
        # result, so it takes the per-tile records the device pick ranks fastest)
        self.slots = linear.topk_slots(step, 0)
        self.steps = {}  # rows -> _Step
        self.y = None  # the launches' output tensor: never written (write_y False), shared by the blocks
        self.miss = 0  # rows where the device's best candidate was not the rescored winner
        # the choice: host rescore (host rows), device rescore (rows_t), or the records-only pick (tmap)
        self.host, self.rows_t, self.own_rows = None, None, False
        self.tmap, self.own_tmap = None, False
        assert token_map is None or self.records_pick, "lmhead: token_map is for rescore=False, device_pick=True"
        if rescore and self.device_pick:
            assert 1 <= top <= 32, f"lmhead: the device pick rescores 1 to 32 candidates, not {top}"
            if rows is None:
                self.rows_t, self.own_rows = head_pick.head_rows(self.device, weight), True
            else:
                head_pick.check_rows(rows, dim, vocab if valid is None else valid)
                self.rows_t = rows
        elif rescore:
            self.host = weight.to(torch.bfloat16)
        elif token_map is not None:
            if isinstance(token_map, torch.Tensor) and token_map.is_cuda:
                self.tmap = token_map
            else:
                assert len(token_map) == vocab, (len(token_map), vocab)
                self.tmap, self.own_tmap = head_pick.token_map(self.device, token_map), True
        if blocks is not None:
            self.blocks = list(blocks)
        else:
            wf = weight.float()
            self.blocks = [(linear.native_weight(self.device, wf[b * step : (b + 1) * step], FORMATS[fmt])[0], None)
                           for b in range(nblk)]

    @property
    def results(self):
        """rows -> the records tensor of that row count (block b's records from slot b * slots)."""
        return {rows: s.records for rows, s in self.steps.items()}

    @property
    def picks(self):
        """rows -> the device pick's output page of that row count."""
        return {rows: s.page for rows, s in self.steps.items() if s.page is not None}

    def _step(self, rows, x):
        s = self.steps.get(rows)
        if s is None:
            s = self.steps[rows] = _Step(self, rows)
        m = x.shape[-2]
        if self.y is None or self.y.shape[-2] != m:
            self.y = torch.empty(1, 1, m, self.step, dtype=torch.bfloat16, device=self.device.torch)
        return s

    def logits_topk(self, x, rows=1, ids_out=None):
        """Enqueue the device part for the first `rows` rows of x [1, 1, >= rows, dim] bf16: every block's top-k
        matmul, then with device_pick the pick. Returns the records tensor. ids_out (a device pick): row 0's token also
        into this one-element int32 tensor. Nothing is allocated after the first call for a row count and nothing is
        read back, so a HIP graph can hold it (reference lmhead.py:135-193)."""
        assert 1 <= rows <= 16 and rows <= x.shape[-2], f"lmhead: 1 to 16 rows, at most x's ({rows})"
        s = self._step(rows, x)
        for b, (w, scale) in enumerate(self.blocks):
            spec = {"r": s.records, "k": self.k, "rows": rows, "slot0": b * self.slots, "base": b * self.step,
                    "n": self.step, "write_y": False, "slots": self.slots}
            linear.matmul(x, w, scale, topk=spec, out=self.y, **self.opts)
        if self.rows_t is not None:
            s.page = head_pick.pick(s.records, x, self.rows_t, rows, self.k, top=self.top, logits=self.logits,
                                    out=s.page, valid=self.valid, ids_out=ids_out)
        elif self.records_pick:
            s.page = head_pick.pick_records(s.records, rows, self.k, self.vocab if self.valid is None else self.valid,
                                            tmap=self.tmap, out=s.page, ids_out=ids_out)
        else:
            assert ids_out is None, "lmhead: ids_out needs the device pick"
        return s.records

    def candidates(self, x, rows):
        """Run the device part and read its candidates back: (values [rows, c] float, token ids [rows, c] long, -inf
        and -1 in empty slots) (reference lmhead.py:195-198)."""
        return linear.topk_records(self.logits_topk(x, rows), rows, self.k)

    def rescore(self, xh, ids):
        """The candidates' logits from the bf16 head on the host: x [rows, dim] as bf16 times the rows ids [rows, c],
        float32, rounded to bf16 unless logits="float32" (reference lmhead.py:200-205)."""
        w = self.host[ids.reshape(-1)].float().reshape(*ids.shape, self.dim)  # [rows, c, dim]
        z = torch.bmm(w, xh.to(torch.bfloat16).float().unsqueeze(-1)).squeeze(-1)
        return z.to(torch.bfloat16).float() if self.round else z

    def __call__(self, x, rows=1):
        """Token ids [rows] (long) for the first `rows` rows of x (reference lmhead.py:207-210)."""
        self.logits_topk(x, rows)
        return self.collect(x, rows)

    def collect(self, x, rows=1, xh=None):
        """The host's part once logits_topk has run (directly or in a replayed graph): the device pick's token ids, or
        the records read back and chosen from (rescored with x, or xh, a host copy of x's first rows). Token ids
        [rows] (long) (reference lmhead.py:212-239)."""
        s = self.steps[rows]
        if s.page is not None:
            tok, best, _ = head_pick.tokens(s.page, rows)
            if self.rows_t is not None:
                self.miss += int((best != tok).sum())
            return tok
        vals, ids = linear.topk_records(s.records, rows, self.k)
        order = vals.argsort(dim=1, descending=True, stable=True)
        if self.host is None:  # no rescore: the best record slot
            return ids.gather(1, order[:, :1]).squeeze(1)
        keep = order[:, : self.top] if self.top else order
        vals, ids = vals.gather(1, keep), ids.gather(1, keep)
        xh = (x.reshape(-1, self.dim)[:rows].cpu() if xh is None else xh.reshape(-1, self.dim)[:rows])
        exact = self.rescore(xh, ids.clamp(min=0))
        exact = exact.masked_fill(ids < 0, float("-inf"))
        tok = pick_token(exact, ids.clamp(min=0), self.vocab)
        self.miss += int((ids[:, 0] != tok).sum())  # (column 0: the device's best)
        return tok

    def deallocate(self):
        """Drop the device tensors made here (a caller's rows table and token map stay theirs) (reference
        lmhead.py:241-263)."""
        self.steps = {}
        self.y = None
        self.blocks = []
        if self.own_rows:
            self.rows_t = None
        if self.own_tmap:
            self.tmap = None
