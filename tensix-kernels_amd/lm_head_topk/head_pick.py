"""head_pick.py: the top-k LM head's exact rescore and pick on the device (MI355X), after XylolabsInc/tensix-kernels'
lm_head_topk/head_pick.py (file:line cited per function).

lmhead.DeviceHead's device part leaves, per row, the best candidates of every 32-column tile of the vocabulary in a
top-k result tensor (linear.matmul's topk records). pick() takes the best `top` of them by the device's logit,
recomputes their logits from the bf16 head rows (bf16 x times bf16 rows, summed in float32, rounded to bf16 unless
logits="float32") and picks the largest (the lowest id on ties, a NaN counting as the largest: lmhead.pick_token's
rule), in one launch with no host reads (graph-capturable; several workgroups a row meet in the top-k merge's
workspace):

  rows = head_rows(device, weight)                    # the bf16 head [vocab, dim] on the device, one row a token
  out = pick(records, x, rows, nrows, k, top=16)      # [1, 1, 32, 32] int32; row r: token, device best, count

pick_records takes each row's best record by the device's own logit, with no rescore, through a token map:

  tmap = token_map(device, ids)                       # row i of the sub-head is token ids[i]
  out = pick_records(records, nrows, k, len(ids), tmap)

The kernels are dr_head_pick and dr_head_pick_records of libdense_reader.so (include/lm_head.h).
"""

import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
from common import device as dev  # noqa: E402
from dense_reader import _lib, linear  # noqa: E402

TILE = 32


def head_rows(device, weight):
    """The bf16 head [vocab, dim] (torch) on the device as [1, 1, vocab, dim], one row a token
    (reference head_pick.py:43-52)."""
    vocab, dim = weight.shape
    d = dev.as_device(device)
    return weight.to(torch.bfloat16).reshape(1, 1, vocab, dim).contiguous().to(d.torch)


def check_rows(rows_t, dim, vocab=None):
    """A bf16 head table pick can gather from: [rows, dim] or [1, 1, rows, dim], bf16, contiguous, on the GPU, with at
    least vocab rows when vocab is given (reference head_pick.py:55-70)."""
    shape = tuple(rows_t.shape)
    assert (
        isinstance(rows_t, torch.Tensor)
        and rows_t.is_cuda
        and rows_t.dtype == torch.bfloat16
        and rows_t.is_contiguous()
        and all(s == 1 for s in shape[:-2])
        and shape[-1] == dim
        and (vocab is None or shape[-2] >= vocab)
    ), (shape, rows_t.dtype, dim, vocab)


def check_ids_out(t):
    """ids_out: a one-element int32 tensor on the GPU (an embedding's index for a draft's next step;
    reference head_pick.py:73-87)."""
    assert isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == torch.int32 and t.numel() == 1, (t.shape, t.dtype)


def _out_page(device):
    return torch.zeros(1, 1, TILE, TILE, dtype=torch.int32, device=device)


def _select_workspace(device, stream, n_records, rows, k):
    """(pointer, bytes) of the selection's workspace (the top-k merge's), or (None, 0) when one workgroup a row does."""
    need = _lib.lib().dr_topk_merge_workspace_bytes(n_records, rows, k)
    _lib.check(_lib.DR_EINVAL if need < 0 else _lib.DR_OK, "dr_topk_merge_workspace_bytes")
    if need == 0:
        return None, 0
    ws = linear._workspace(device, stream, need, "merge")
    return ws.data_ptr(), ws.numel()


def _words(records, nrows, k):
    w = records.reshape(records.shape[-2], -1)
    if w.dtype == torch.bfloat16:
        w = w.view(torch.int32)
    assert w.dtype == torch.int32 and w.shape[1] == 2 * nrows * k and w.is_contiguous(), (records.shape, nrows, k)
    return w


def pick(records, x, rows_t, nrows, k, top=16, logits="bf16", out=None, valid=None, ids_out=None):
    """Token ids for the first nrows rows of x [..., >= nrows, dim] bf16: per row the best `top` candidates of the
    top-k result `records` (linear.topk_result's, made for nrows rows and k), rescored with the bf16 rows of rows_t
    (head_rows') and picked (lmhead.pick_token's rule). out: [1, 1, 32, 32] int32 (made here unless given; a graph
    passes the same one each step); row r = [token, the device's own best candidate, the valid count, 0, ...].
    valid: a padded head's real vocabulary (ids at or past it are empty slots; default the table's rows). A row with
    no valid candidate gets token 0 and count 0. ids_out: also row 0's token into this one-element int32 tensor
    (reference head_pick.py:101-220)."""
    assert logits in ("bf16", "float32"), logits
    assert 1 <= top <= 32 and 1 <= nrows <= TILE, (top, nrows)
    dim = x.shape[-1]
    check_rows(rows_t, dim)
    vocab = rows_t.shape[-2] if valid is None else int(valid)
    assert 1 <= vocab <= rows_t.shape[-2], (valid, rows_t.shape)
    words = _words(records, nrows, k)
    assert x.dtype == torch.bfloat16 and x.is_cuda, x.dtype
    x2 = x.reshape(-1, dim)
    assert x2.shape[0] >= nrows, (x.shape, nrows)
    x2 = x2 if x2.is_contiguous() else x2.contiguous()
    if out is None:
        out = _out_page(x.device)
    assert out.dtype == torch.int32 and out.numel() >= TILE * TILE and out.is_contiguous(), (out.shape, out.dtype)
    if ids_out is not None:
        check_ids_out(ids_out)
    stream = torch.cuda.current_stream(x.device)
    wp, wn = _select_workspace(x.device, stream, words.shape[0], nrows, k)
    st = _lib.lib().dr_head_pick(
        words.data_ptr(), words.shape[0], nrows, k, top, int(logits == "bf16"), x2.data_ptr(), x2.shape[1], dim,
        rows_t.data_ptr(), dim, vocab, out.data_ptr(), None if ids_out is None else ids_out.data_ptr(), wp, wn,
        stream.cuda_stream,
    )
    _lib.check(st, "dr_head_pick")
    return out


def token_map(device, ids):
    """A sub-head's token map for pick_records: row i of the sub-head is token ids[i] (below 2**31); [1, 1, ceil(n /
    32), 32] int32 on the device, the tail past n zero (reference head_pick.py:223-238)."""
    ids = torch.as_tensor(ids, dtype=torch.int64).reshape(-1)
    n = ids.numel()
    assert n >= 1 and int(ids.min()) >= 0 and int(ids.max()) < 1 << 31, (n, ids.min(), ids.max())
    pages = -(-n // TILE)
    t = torch.zeros(pages * TILE, dtype=torch.int32)
    t[:n] = ids.to(torch.int32)
    return t.reshape(1, 1, pages, TILE).to(dev.as_device(device).torch)


def pick_records(records, nrows, k, vocab, tmap=None, out=None, ids_out=None):
    """Token ids for the first nrows rows of a top-k result, with no rescore: per row the best record slot by the
    device's logit (the first of equal keys, record by record and slot by slot; a NaN counts as the largest), its id
    mapped through tmap (token_map's, at least vocab ids; None: the id itself). vocab: the head's rows that count.
    out: [1, 1, 32, 32] int32; row r = [token, the best id, the valid slots' count, 0, ...]; a row with no valid slot
    gets [0, 0xFFFFFFFF, 0]. ids_out: as pick's (reference head_pick.py:241-329)."""
    assert 1 <= nrows <= TILE and k >= 1, (nrows, k)
    words = _words(records, nrows, k)
    vocab = int(vocab)
    assert 1 <= vocab < 1 << 32, vocab
    if tmap is not None:
        assert tmap.dtype == torch.int32 and tmap.is_cuda and tmap.is_contiguous() and tmap.numel() >= vocab, (
            tmap.shape,
            tmap.dtype,
            vocab,
        )
    if out is None:
        out = _out_page(records.device)
    if ids_out is not None:
        check_ids_out(ids_out)
    stream = torch.cuda.current_stream(records.device)
    wp, wn = _select_workspace(records.device, stream, words.shape[0], nrows, k)
    st = _lib.lib().dr_head_pick_records(
        words.data_ptr(), words.shape[0], nrows, k, vocab, None if tmap is None else tmap.data_ptr(), out.data_ptr(),
        None if ids_out is None else ids_out.data_ptr(), wp, wn, stream.cuda_stream,
    )
    _lib.check(st, "dr_head_pick_records")
    return out


def tokens(out, nrows):
    """The host's read of a pick's output: (tokens [nrows], the device's own best [nrows], valid counts [nrows]), long
    (reference head_pick.py:332-335)."""
    t = out.reshape(TILE, TILE)[:nrows].cpu().to(torch.int64) & 0xFFFFFFFF
    return t[:, 0], t[:, 1], t[:, 2]
