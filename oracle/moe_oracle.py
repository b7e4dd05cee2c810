"""CPU oracle of the MoE layer -- TEST INFRASTRUCTURE ONLY.

Only tests/ (and __graft_entry__.smoke() / bench.py's cpu_baseline leg) may import this module, and only as the
checker; the product (tensix-kernels_amd/) never does.

It restates, in numpy float64 on the CPU, what XylolabsInc/tensix-kernels' moe/moe8.py computes (paths relative to the
reference's root):

- glu: the experts' activation times the up half, moe8.py:607-616 and moe_gu_compute.cpp (silu, gelu_tanh as
  HF's gelu_pytorch_tanh, swiglu_oai as gpt-oss's clamped SwiGLU, common/kernels/dense_ops.h:90-118);
- layer / layer_rows: one row's h and y (moe8.py:619-644): per slot s, w_s * glu(x G_e + b_g, x U_e + b_u), gate_up
  [E, H, 2I] as [up | gate] columns, then y = sum_s h_s @ D_e;
- union: the rows' distinct ids below E in increasing order (moe8.py:647-649, kernels/moe8_rows.h);
- route: the router, one row at a time in plain Python (moe8.py:1139-1286): keys, optional group-limited routing,
  the top k by key with the lower id first among equal keys, the softmax or sigmoid weights, the scale, a fixed slot;
- held_kblock: the values a kblock pack holds (moe8.py:117-154 with kblock, 507-527): BFP4_b's rounding with each
  face row 16 consecutive K at one N.

What pins each function (tests/test_oracle.py, test_moe_oracle_*):
- glu: closed forms (silu(0) = 0, the gelu_tanh constants against torch's gelu(approximate="tanh"), the clamps of
  swiglu_oai at and beyond 7);
- layer: invariants a slip would break -- a gate half driven to large negative values gives h = 0 (so the [up | gate]
  order is pinned), h and y linear in the routing weights, y of two slots the sum of the slots alone, a bias equal to
  minus x U zeroing h -- and a hand-worked two-expert case;
- union: brute force on small id sets (duplicates, ids past E);
- route: brute-force sort on small rows with ties (the lower id first), the softmax weights summing to the scale,
  a hand-built group case where the best single expert sits in a dropped group;
- held_kblock: against the BFP4_b tiles of the matrix with every 32 x 32 block transposed in place (the reference's
  kblock conversion), their values turned back, bit for bit, and against a hand-made matrix whose 16-K groups each
  hold one large value (the rest of the group rounds to its grid, the 16-N rounding would not).
"""

import math

import numpy as np

OAI_ALPHA, OAI_LIMIT = 1.702, 7.0


def _sigmoid(z):
    with np.errstate(over="ignore"):  # (exp overflows to inf for very negative z: the sigmoid is then 0)
        return 1.0 / (1.0 + np.exp(-z))


def glu(g, u, act):
    """act(g) * u in float64 (numpy arrays): silu g * sigmoid(g); gelu_tanh 0.5 g (1 + tanh(sqrt(2 / pi) (g +
    0.044715 g^3))); swiglu_oai min(g, 7) * sigmoid(1.702 min(g, 7)) * (clip(u, -7, 7) + 1) (moe8.py:607-616)."""
    g, u = np.asarray(g, np.float64), np.asarray(u, np.float64)
    if act == "silu":
        return g * _sigmoid(g) * u
    if act == "gelu_tanh":
        return 0.5 * g * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (g + 0.044715 * g**3))) * u
    if act == "swiglu_oai":
        gc = np.minimum(g, OAI_LIMIT)
        return gc * _sigmoid(OAI_ALPHA * gc) * (np.clip(u, -OAI_LIMIT, OAI_LIMIT) + 1.0)
    raise ValueError(act)


def held_kblock(w):
    """The values a kblock BFP4_b pack holds for the float [K, N] matrix w (K, N multiples of 32): each shared
    exponent covers 16 consecutive K at one N (reference moe8.py:117-154, the tile's block transposed before the
    rounding), so it is dense_oracle.held of w transposed, transposed back."""
    from oracle import dense_oracle as O

    w = np.asarray(w, np.float32)
    return np.ascontiguousarray(O.held(np.ascontiguousarray(w.T), "bfp4").T)


def _bf16(a):
    """float -> the nearest bf16 value (ties to even), as float64."""
    b = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    b = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    return b.astype(np.uint32).view(np.float32).astype(np.float64)


def layer(x, gate_up, down, ids, w, act="silu", gu_bias=None):
    """(y [H], h [k * I]) in float64 for one row x [H]: slot s of h = w[s] * glu(x G_e + b_g, x U_e + b_u) with e =
    ids[s], G_e = gate_up[e][:, I:], U_e = gate_up[e][:, :I], b = gu_bias[e] rounded to bf16 ([up | gate]); y = the
    sum over the slots of h_s @ down[e] (moe8.py:619-636)."""
    x = np.asarray(x, np.float64).reshape(-1)
    gu = np.asarray(gate_up, np.float64)
    dn = np.asarray(down, np.float64)
    I = gu.shape[-1] // 2
    hs, y = [], np.zeros(dn.shape[-1])
    for s, e in enumerate(ids):
        e = int(e)
        up = x @ gu[e][:, :I]
        gate = x @ gu[e][:, I:]
        if gu_bias is not None:
            b = _bf16(np.asarray(gu_bias, np.float32)[e])
            up, gate = up + b[:I], gate + b[I:]
        h = float(w[s]) * glu(gate, up, act)
        hs.append(h)
        y = y + h @ dn[e]
    return y, np.concatenate(hs)


def layer_rows(x, gate_up, down, ids, w, act="silu", gu_bias=None):
    """y [R, H]: layer() of each row with its own ids and weights."""
    return np.stack([layer(x[r], gate_up, down, ids[r], w[r], act, gu_bias)[0] for r in range(len(ids))])


def union(ids, E):
    """The distinct ids below E, in increasing order."""
    seen = set()
    for e in np.asarray(ids).reshape(-1).tolist():
        if 0 <= int(e) < E:
            seen.add(int(e))
    return sorted(seen)


def route(logits, k, kind="softmax", bias=None, scale=1.0, norm=True, groups=None, slot=None):
    """(ids [R][k'], w [R][k']) as Python lists, one row at a time: keys (the logit; sigmoid + bias for the sigmoid kind
    with a bias); groups (n_group, topk_group): a group's score the sum of its two largest keys, the groups ranked by
    score then index, those past topk_group dropped; the top k by key then id; weights the softmax over the picked
    logits or the picks' sigmoids (over their sum when norm), times scale; slot: one more id at weight 1.0."""
    lg = np.asarray(logits, np.float64)
    out_ids, out_w = [], []
    for row in lg:
        E = len(row)
        sg = [0.0 if v < -709.0 else 1.0 / (1.0 + math.exp(-v)) for v in row]  # (exp(-v) past the double range)
        if kind == "sigmoid" and bias is not None:
            key = [sg[e] + float(bias[e]) for e in range(E)]
        else:
            key = [float(v) for v in row]
        if groups is not None:
            ng, tg = groups
            gs = E // ng
            score = []
            for gi in range(ng):
                top = sorted(key[gi * gs : (gi + 1) * gs], reverse=True)
                score.append(top[0] + top[1])
            kept = sorted(range(ng), key=lambda gi: (-score[gi], gi))[:tg]
            key = [key[e] if e // gs in kept else -math.inf for e in range(E)]
        picks = sorted(range(E), key=lambda e: (-key[e], e))[:k]
        if kind == "softmax":
            m = max(row[e] for e in picks)
            ex = [math.exp(row[e] - m) for e in picks]
            wts = [v / sum(ex) for v in ex]
        else:
            v = [sg[e] for e in picks]
            wts = [a / sum(v) for a in v] if norm else v
        wts = [a * scale for a in wts]
        if slot is not None:
            picks, wts = picks + [int(slot)], wts + [1.0]
        out_ids.append(picks)
        out_w.append(wts)
    return out_ids, out_w
