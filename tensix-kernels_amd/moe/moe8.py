"""moe8.py: a mixture-of-experts layer that reads only the chosen experts, on MI355X, after XylolabsInc/tensix-kernels'
moe/moe8.py (file:line cited per function). The expert ids are read on the device, so nothing goes to the host and a
HIP graph can capture every op.

Ops per MoE layer (the reference's names and arguments):
- route(logits, ids, w, k): the router's top k and their weights (softmax or sigmoid scoring, an optional score bias,
  group-limited routing, a scaling factor, a fixed shared-expert slot, a shared expert's gate), one wavefront a row;
- gate_up(x, P, ids, w, k) -> h [1, 1, 1, k * I]: per slot s, w_s * act(x G_e + b_g) * (x U_e + b_u) of expert
  ids[s], act "silu", "gelu_tanh" or "swiglu_oai";
- down(h, P, ids, k) -> y [1, 1, 1, H]: the sum over the slots of h_s @ D_e;
- gate_up_rows / down_rows: up to 32 rows, each with its own k experts, by expert of the rows' union (every expert
  of the union read once for all rows).

The packed layer (pack): each expert's gate and up [K = H, N = I] and down [K = I, N = H] are dense_reader bfloat4_b
weights (16-column panels, 1 KiB k-blocks, exponents apart), packed on the GPU by dr_pack with the reference's
block-float rounding (moe8.py:117-154), one expert after another, so an op reaches expert e's weights at e times a
stride. The ops are dense_reader's GEMV (one row, two rows) or MFMA kernel (more rows) with an expert gather: the
workgroup's expert (gate/up) or each K chunk's (down) comes from the ids on the device (include/moe.h). gate and up
run as one GLU launch; the routing weight, the bias and the activation are its epilogue.

The Tensix work split (cores per bank, loaders, the split share, chunk depths, fidelity) is accepted and changes
nothing, as in the reference where it never changes a result. The `banks` of a pack are kept in its meta (and its
column groups checked as the reference checks them) but do not change the layout.

Entry points: bfp4_tiles, bfp4_values, pack, pack_host, pack_upload, prepack, pack_cached, repack_down, route,
gate_up, down, gate_up_rows, down_rows, reference, reference_rows, route_reference, union, u_max, sigmoid_table,
gu_groups, PackCacheMismatch.
"""

import ctypes
import json
import math
import shutil
import sys
from pathlib import Path

import numpy as np
import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
from common import device as dev  # noqa: E402
from dense_reader import _lib, linear  # noqa: E402
from dense_reader import pack_cache as pc  # noqa: E402

TILE = 32
TB = 576  # a BFP4_b tile of the reference: 64 exponent bytes, 512 bytes of sign + 3-bit magnitudes
DR_BFP4 = 1
DR_BFP4_KB = 4  # bfloat4_b's rounding with the shared exponent over 16 consecutive K at one N (kblock packs)
ACTS = {"silu": 0, "gelu_tanh": 1, "swiglu_oai": 2}
OAI_ALPHA, OAI_LIMIT = 1.702, 7.0

# --- settings (module attributes of the reference, moe8.py:73-91): the Tensix work split; they change nothing here
ROWS_SFPU = True
GU_CPB = 0
GU_ROWS_CPB = 0
LOADERS = 2
ROWS_LOADERS = 1
SPLIT_SHARE = 0.5
L1_MARGIN = 32 * 1024
GW_MAX = 8
PACK_VERSION = 1  # the layout below; a cache of another version is refused
LAYOUT = "moe-bfp4-panels16-kblock1k-exp256"
ARRAYS = ("gu", "gu_exps", "dn", "dn_exps", "bias")

PackCacheMismatch = pc.PackCacheMismatch


def sigmoid_table():
    """The reference route kernel's bounds table: sigmoid(i / 16 - 16), i = 0 .. 512, in Q2.30, rounded (reference
    moe8.py:108-114). The router here computes in double and does not need it; it is kept for code that reads it."""
    return [round((1.0 / (1.0 + math.exp(-(i / 16 - 16)))) * (1 << 30)) for i in range(513)]


# --- the reference's BFP4_b tile bytes on the host --------------------------------------------------------------------


def _face_rows(w, kblock):
    """float32 [K, N] -> [KT, NT, 64, 16]: each tile's 64 face rows of 16 values (kblock: of the tile transposed)."""
    k, n = w.shape
    t = w.reshape(k // 32, 32, n // 32, 32).transpose(0, 2, 1, 3)
    if kblock:
        t = t.transpose(0, 1, 3, 2)
    f = t.reshape(k // 32, n // 32, 2, 16, 2, 16).transpose(0, 1, 2, 4, 3, 5)
    return np.ascontiguousarray(f).reshape(k // 32, n // 32, 64, 16)


def bfp4_tiles(w, kblock=False):
    """float [K, N] (multiples of 32) -> uint8 [KT, NT, 576]: each 32 x 32 tile as BFP4_b, as tt-metal's host
    conversion makes it. Per face row of 16 the shared exponent is the largest biased float32 exponent; each mantissa
    (hidden bit set) is shifted down by its distance from it (to 0 past 31 places), rounded to 3 bits half to even
    (shifted-out bits not sticky), at most 7; zero and denormal inputs give 0 and the sign stays only on a non-zero
    magnitude. 64 exponent bytes (face by face, row by row), then two codes a byte (the first in the low nibble).
    kblock: each tile holds its block transposed, so a face row is 16 consecutive K at one N (reference
    moe8.py:117-154)."""
    w = np.ascontiguousarray(w.float().numpy() if isinstance(w, torch.Tensor) else w, np.float32)
    k, n = w.shape
    assert k % TILE == 0 and n % TILE == 0, w.shape
    bits = _face_rows(w, kblock).view(np.uint32)
    ex = ((bits >> 23) & 0xFF).astype(np.int64)
    top = ex.max(axis=-1, keepdims=True)
    man = ((bits & 0x7FFFFF) | 0x800000).astype(np.int64)
    dist = top - ex
    kept = np.where(dist > 31, 0, man >> np.minimum(dist, 31))
    q, low = kept >> 21, kept & ((1 << 21) - 1)
    up = (low > (1 << 20)) | ((low == (1 << 20)) & ((q & 1) == 1))
    mag = np.minimum(q + up, 7)
    mag = np.where(ex == 0, 0, mag)
    neg = ((bits >> 31) == 1) & (mag != 0)
    code = (np.where(neg, 8, 0) | mag).astype(np.uint8).reshape(k // 32, n // 32, 1024)
    head = top.astype(np.uint8).reshape(k // 32, n // 32, 64)
    return np.concatenate([head, code[..., 0::2] | (code[..., 1::2] << 4)], axis=-1)


def bfp4_values(tiles, kblock=False):
    """uint8 [..., 576] BFP4_b tiles -> float32 [..., 32, 32] row-major tile values, (-1)^s m 2^(E - 129) (kblock: the
    block turned back to [K, N] order) (reference moe8.py:157-172)."""
    tiles = np.asarray(tiles)
    lead = tiles.shape[:-1]
    head = tiles[..., :64].astype(np.int32)
    body = tiles[..., 64:]
    code = np.stack([body & 15, body >> 4], axis=-1).reshape(*lead, 64, 16).astype(np.int32)
    val = np.where(code & 8, -1.0, 1.0) * (code & 7) * np.exp2(head - 129.0)[..., None]
    val = val.astype(np.float32).reshape(*lead, 2, 2, 16, 16).swapaxes(-3, -2).reshape(*lead, 32, 32)
    return val.swapaxes(-1, -2) if kblock else val


# --- the reference's Tensix layout helpers (kept: tests and callers read them) ----------------------------------------


def _split(total, parts):
    """[(start, count)]: total in parts as even as they go, the first total % parts parts one larger (reference
    moe8.py:175-183)."""
    q, r = divmod(total, parts)
    starts = [i * q + min(i, r) for i in range(parts)]
    return [(s0, q + (i < r)) for i, s0 in enumerate(starts)]


def gu_pairs(e, bank, banks, pairs=16):
    """(first pair, pairs) of expert e's gate/up tile pairs that the reference's bank holds: the pairs split over the
    banks as _split does, the split's parts handed to banks rotated by the expert, so that the larger parts fall on
    different banks from one expert to the next (reference moe8.py:199-201). Here a layout helper only: the packed
    experts keep each expert's panels in one place, read by every CU."""
    return _split(pairs, banks)[(bank - e) % banks]


def gu_groups(it, banks):
    """(G, GW): the reference's gate_up column groups per expert and bank, and their width in tiles (reference
    moe8.py:204-212). Here a Tensix dest-size rule only: the layout does not depend on it, but gate_up refuses column
    groups with one loader as the reference does."""
    ncmax = 2 * -(-it // banks)
    if ncmax <= GW_MAX:
        return 1, ncmax
    return -(-ncmax // GW_MAX), GW_MAX


def _clamp_cpb(device, banks, cores_per_bank):
    """cores_per_bank capped at the grid's share of a bank (reference moe8.py:502-504)."""
    g = dev.as_device(device).compute_with_storage_grid_size()
    return max(1, min(cores_per_bank, (g.x * g.y) // banks))


# --- the packed layer --------------------------------------------------------------------------------------------------


def _geometry(E, H, I):
    """Bytes of one expert's packed gate (or up) and down weights: (gu_codes, gu_exps, dn_codes, dn_exps) and the
    padding (gu_kpad, gu_npad, dn_kpad, dn_npad)."""
    lib = _lib.lib()
    gk, gn = -(-H // linear.KALIGN) * linear.KALIGN, -(-I // TILE) * TILE
    dk, dn = -(-I // linear.KALIGN) * linear.KALIGN, -(-H // TILE) * TILE
    sizes = (lib.dr_codes_bytes(DR_BFP4, gk, gn), lib.dr_exps_bytes(DR_BFP4, gk, gn),
             lib.dr_codes_bytes(DR_BFP4, dk, dn), lib.dr_exps_bytes(DR_BFP4, dk, dn))
    return sizes, (gk, gn, dk, dn)


def _pack_one(d, w_nk, n, k, codes, exps, n_pad, k_pad, fmt):
    """dr_pack of a float32 [N][K] device matrix into codes / exps (device uint8 views) as bfloat4_b (fmt DR_BFP4) or
    its kblock packs (DR_BFP4_KB)."""
    st = _lib.lib().dr_pack(w_nk.data_ptr(), k, n, k, fmt, None, codes.data_ptr(), exps.data_ptr(), n_pad, k_pad,
                            d.stream())
    _lib.check(st, "dr_pack (moe8)")


def _bias_rows(gu_bias, I):
    """[E, 2I] as [up | gate] -> bf16 [E, 2, I] as (gate, up), the kernels' order."""
    b = torch.as_tensor(gu_bias).to(torch.bfloat16)
    return torch.stack([b[:, I:], b[:, :I]], dim=1).contiguous()


def _pack_device(d, gate_up, down, gu_bias=None, kblock=False):
    """The packed arrays on the device: gu [E, 2, codes] (gate, up), gu_exps [E, 2, exps], dn [E, codes], dn_exps
    [E, exps], bias [E, 2, I] bf16 or None. One expert at a time goes to the device in float32. kblock: each shared
    exponent covers 16 consecutive K at one N (the codes keep bfloat4_b's layout; the exponents their own order)."""
    fmt = DR_BFP4_KB if kblock else DR_BFP4
    E, H, I2 = gate_up.shape
    I = I2 // 2
    (gc, ge, dc, de), (gk, gn, dk, dn) = _geometry(E, H, I)
    t = d.torch
    gu = torch.zeros(E, 2, gc, dtype=torch.uint8, device=t)
    gu_e = torch.zeros(E, 2, ge, dtype=torch.uint8, device=t)
    dn_c = torch.zeros(E, dc, dtype=torch.uint8, device=t)
    dn_e = torch.zeros(E, de, dtype=torch.uint8, device=t)
    for e in range(E):
        w = torch.as_tensor(gate_up[e]).to(device=t, dtype=torch.float32)  # [H, 2I] as [up | gate]
        gate = w[:, I:].t().contiguous()  # [I][H]
        up = w[:, :I].t().contiguous()
        _pack_one(d, gate, I, H, gu[e, 0], gu_e[e, 0], gn, gk, fmt)
        _pack_one(d, up, I, H, gu[e, 1], gu_e[e, 1], gn, gk, fmt)
        dw = torch.as_tensor(down[e]).to(device=t, dtype=torch.float32).t().contiguous()  # [H][I]
        _pack_one(d, dw, H, I, dn_c[e], dn_e[e], dn, dk, fmt)
    bias = _bias_rows(gu_bias, I).to(t) if gu_bias is not None else None
    return {"gu": gu, "gu_exps": gu_e, "dn": dn_c, "dn_exps": dn_e, "bias": bias}


def _meta(E, H, I, banks, cpb, gate_up, down, gu_bias, kblock):
    """The pack cache's meta: what the packed arrays depend on (reference moe8.py:349-376)."""
    meta = {
        "version": PACK_VERSION,
        "layout": LAYOUT,
        "banks": banks,
        "cpb": cpb,
        "E": E,
        "H": H,
        "I": I,
        "gate_up": pc.fingerprint(gate_up),
        "down": pc.fingerprint(down),
    }
    G = gu_groups(I // TILE, banks)[0]
    if G > 1:
        meta["gu_groups"] = G
    if gu_bias is not None:
        meta["gu_bias"] = pc.fingerprint(gu_bias)
    if kblock:
        meta["kblock"] = True
    return meta


def _short(v):
    v = repr(v)
    return v if len(v) <= 48 else v[:45] + "..."


def _split_hint(old, diff):
    if set(diff) <= {"cpb", "banks"}:
        return f" Only the split differs: call with cores_per_bank={old.get('cpb')}, banks={old.get('banks')} to use it."
    return ""


def _check_weights(gate_up, down, gu_bias, kblock):
    E, H, I2 = gate_up.shape
    I = I2 // 2
    assert tuple(down.shape) == (E, I, H), (tuple(down.shape), (E, I, H))
    assert H % TILE == 0 and I % TILE == 0, (H, I)
    assert E <= 1024, "moe8: at most 1024 experts"
    if gu_bias is not None:
        assert tuple(gu_bias.shape) == (E, 2 * I), (tuple(gu_bias.shape), (E, 2 * I))
    return E, H, I


def pack_host(gate_up, down, banks, cores_per_bank=3, cache=None, gu_bias=None, rebuild=False, kblock=False):
    """pack()'s arrays on the host: a dict of numpy arrays and numbers that pack_upload puts on a device. The packing
    itself runs on the current GPU. Keys: version, E, H, I, banks, cpb, gu, gu_exps, dn, dn_exps, bias (or absent),
    gu_bias (bool), kblock (bool). cache, gu_bias, rebuild: as pack()'s (reference moe8.py:435-465)."""
    E, H, I = _check_weights(gate_up, down, gu_bias, kblock)
    meta = _meta(E, H, I, banks, cores_per_bank, gate_up, down, gu_bias, kblock)
    arrays = None
    if cache is not None:
        arrays = pc.cache_read(cache, meta, rebuild, True, ARRAYS, "moe8", _split_hint)
    if arrays is None:
        dv = _pack_device(dev.as_device(None), gate_up, down, gu_bias, kblock)
        arrays = {n: v.cpu().view(torch.int16).numpy() if v.dtype == torch.bfloat16 else v.cpu().numpy()
                  for n, v in dv.items() if v is not None}
        if cache is not None:
            pc.cache_write(cache, meta, arrays)
    out = {"version": PACK_VERSION, "E": E, "H": H, "I": I, "banks": banks, "cpb": cores_per_bank,
           "gu_bias": "bias" in arrays, "kblock": bool(kblock)}
    out.update(arrays)
    return out


def pack_upload(device, host):
    """pack_host's dict on the device: the dict the ops take (reference moe8.py:468-499)."""
    assert host["version"] == PACK_VERSION, (host["version"], PACK_VERSION)
    d = dev.as_device(device)
    banks, cpb = host["banks"], host["cpb"]
    assert banks <= dev.dram_banks(d), (banks, dev.dram_banks(d))
    g = d.compute_with_storage_grid_size()
    assert cpb == max(1, min(cpb, (g.x * g.y) // banks)), (cpb, g)
    arrays = {}
    for n in ARRAYS:
        if n in host and host[n] is not None:
            t = torch.from_numpy(np.array(host[n]))
            arrays[n] = t.view(torch.bfloat16).to(d.torch) if n == "bias" else t.to(d.torch)
    return _device_dict(d, host["E"], host["H"], host["I"], banks, cpb, arrays, bool(host.get("kblock", False)))


def _device_dict(d, E, H, I, banks, cpb, arrays, kblock):
    sizes, pads = _geometry(E, H, I)
    nbytes = sum(v.numel() * v.element_size() for v in arrays.values() if v is not None)
    return {
        "E": E,
        "H": H,
        "I": I,
        "banks": banks,
        "cpb": cpb,
        "gu": arrays["gu"],
        "gu_exps": arrays["gu_exps"],
        "dn": arrays["dn"],
        "dn_exps": arrays["dn_exps"],
        "bias": arrays.get("bias"),
        "gu_bias": arrays.get("bias") is not None,
        "kblock": kblock,
        "sizes": sizes,
        "pads": pads,
        "bytes": nbytes,
        "device": d,
    }


def pack(device, gate_up, down, cores_per_bank=3, banks=None, cache=None, gu_bias=None, rebuild=False, kblock=False):
    """One MoE layer's experts as moe8's packed weights. gate_up: [E, H, 2I] float with up in columns 0..I-1 and gate
    in I..2I-1 ([up | gate]); down: [E, I, H]. Returns the dict the ops take. banks (default the device's) and
    cores_per_bank (capped at the grid's share) are kept for the cache's meta and change nothing else.

    cache: a directory for this layer's packed arrays (their .npy, meta.json, sums.json). Taken when its meta matches
    (the layout version, the banks and cores, the shapes and a fingerprint of the weights); made and written when the
    directory is absent or empty. A cache that differs or cannot be read raises PackCacheMismatch and is left as it
    is; rebuild=True packs again and writes over it.

    gu_bias: [E, 2I] as [up | gate], added to x U and x G before the activation, held in bf16. kblock: each shared
    exponent covers 16 consecutive K at one N instead of 16 N at one K (reference moe8.py:507-527, the tiles
    transposed before the block-float rounding); the same ops take either pack."""
    d = dev.as_device(device)
    banks = banks or dev.dram_banks(d)
    cpb = _clamp_cpb(d, banks, cores_per_bank)
    E, H, I = _check_weights(gate_up, down, gu_bias, kblock)
    if cache is not None:
        return pack_upload(d, pack_host(gate_up, down, banks, cpb, cache, gu_bias, rebuild, kblock))
    arrays = _pack_device(d, gate_up, down, gu_bias, kblock)
    return _device_dict(d, E, H, I, banks, cpb, arrays, bool(kblock))


def prepack(gate_up, down, cache, banks, cores_per_bank=3, gu_bias=None, rebuild=False, kblock=False):
    """pack()'s arrays into its cache: the cache pack(..., cache=) or pack_cached then takes on a device. True when it
    was made, False when the cache already held these weights. A cache that differs raises PackCacheMismatch unless
    rebuild=True (reference moe8.py:423-432)."""
    E, H, I = _check_weights(gate_up, down, gu_bias, kblock)
    before = (Path(cache) / "meta.json").read_text() if (Path(cache) / "meta.json").exists() else None
    pack_host(gate_up, down, banks, cores_per_bank, cache, gu_bias, rebuild, kblock)
    return (Path(cache) / "meta.json").read_text() != before


def pack_cached(device, cache, cores_per_bank=3, banks=None, kblock=False, gu_bias=None, verify=True):
    """pack()'s result from a pack cache alone, without the weights. The call must match the cache's meta: the layout
    version, the banks and cores per bank (clamped to the device as pack() does), kblock, and the bias (gu_bias None:
    the cache has none; True: it has one; a tensor: its fingerprint must equal the cache's). verify: every array's
    sha256 against sums.json (a cache without one is refused unless verify=False). Anything that differs raises
    PackCacheMismatch and nothing is changed (reference moe8.py:530-604)."""
    path = Path(cache)
    try:
        meta = json.loads((path / "meta.json").read_text())
    except (OSError, ValueError) as e:
        raise PackCacheMismatch(f"moe8 pack cache {path}: no readable meta.json ({type(e).__name__})") from e
    d = dev.as_device(device)
    banks = banks or dev.dram_banks(d)
    cpb = _clamp_cpb(d, banks, cores_per_bank)
    checks = [  # (what, the cache's, the call's)
        ("version", meta.get("version"), PACK_VERSION),
        ("layout", meta.get("layout"), LAYOUT),
        ("banks", meta.get("banks"), banks),
        ("cpb", meta.get("cpb"), cpb),
        ("kblock", bool(meta.get("kblock", False)), bool(kblock)),
        ("a bias", "gu_bias" in meta, gu_bias is not None),
    ]
    if isinstance(gu_bias, torch.Tensor) and "gu_bias" in meta:
        checks.append(("the bias's fingerprint", meta["gu_bias"], pc.fingerprint(gu_bias)))
    diff = [f"{what}: cache {_short(c)}, call {_short(v)}" for what, c, v in checks if c != v]
    if diff:
        raise PackCacheMismatch(f"moe8 pack cache {path} does not match this call ({'; '.join(diff)}). It was not taken.")
    try:
        arrays = {n: np.load(path / f"{n}.npy", mmap_mode="r") for n in ARRAYS if (path / f"{n}.npy").exists()}
    except (OSError, ValueError) as e:
        raise PackCacheMismatch(f"moe8 pack cache {path}: its arrays cannot be read ({type(e).__name__})") from e
    if verify:
        try:
            sums = json.loads((path / "sums.json").read_text())
        except (OSError, ValueError) as e:
            raise PackCacheMismatch(
                f"moe8 pack cache {path} has no readable sums.json; pack it again, or pass verify=False to take it"
                " unchecked"
            ) from e
        got = pc.array_sums(arrays)
        bad = sorted(n for n in set(got) | set(sums) if got.get(n) != sums.get(n))
        if bad:
            raise PackCacheMismatch(f"moe8 pack cache {path}: {', '.join(bad)} differ from sums.json. It was not taken.")
    host = {"version": PACK_VERSION, "E": meta["E"], "H": meta["H"], "I": meta["I"], "banks": banks, "cpb": cpb,
            "kblock": bool(kblock)}
    host.update(arrays)
    return pack_upload(d, host)


def repack_down(cache, cores_per_bank=2):
    """A pack cache moved to another split of down's columns per core, without the weights (reference
    moe8.py:379-420). The layout here does not depend on the cores, so only the meta's cpb changes, written beside the
    cache and swapped in as cache_write does; the result equals a fresh pack at cores_per_bank bit for bit, its meta
    too. True when it was changed, False when the cache already has that split."""
    cache = Path(cache)
    meta = json.loads((cache / "meta.json").read_text())
    assert meta["version"] == PACK_VERSION, (cache, meta["version"], PACK_VERSION)
    if meta["cpb"] == cores_per_bank:
        return False
    meta["cpb"] = cores_per_bank
    tmp = cache.with_name(cache.name + ".tmp")
    shutil.rmtree(tmp, ignore_errors=True)
    shutil.copytree(cache, tmp)
    (tmp / "meta.json").write_text(json.dumps(meta, indent=1))
    shutil.rmtree(cache)
    tmp.rename(cache)
    return True


# --- references (host, float64) ----------------------------------------------------------------------------------------


def _glu(g, u, act):
    """The GLU of the pre-activations (float64 tensors): act(g) * u, act silu, gelu_tanh (HF's gelu_pytorch_tanh), or
    the clamped SwiGLU of gpt-oss, where g is capped at 7 and u clamped to +-7 then shifted by 1 (reference
    moe8.py:607-616)."""
    assert act in ACTS, f"moe8: act {act!r}"
    if act == "swiglu_oai":
        gc = torch.clamp(g, max=OAI_LIMIT)
        return gc * torch.sigmoid(gc * OAI_ALPHA) * (torch.clamp(u, -OAI_LIMIT, OAI_LIMIT) + 1.0)
    a = torch.nn.functional.gelu(g, approximate="tanh") if act == "gelu_tanh" else g * torch.sigmoid(g)
    return a * u


def reference(x, gate_up, down, ids, w, act="silu", gu_bias=None):
    """(y [1, H], h [1, k * I]) in float64 for one row: h's slot s = w_s * GLU(x G_e + b_g, x U_e + b_u) of expert
    e = ids[s], y = sum over the slots of h_s @ D_e. gate_up [E, H, 2I] as [up | gate], down [E, I, H], used as given;
    gu_bias [E, 2I] as [up | gate], rounded to bf16 as packed (reference moe8.py:619-636)."""
    I = gate_up.shape[-1] // 2
    chosen = [int(e) for e in ids]
    xd = x.reshape(-1).double()
    pre = torch.stack([xd @ gate_up[e].double() for e in chosen])  # [k, 2I] as [up | gate]
    if gu_bias is not None:
        pre = pre + torch.as_tensor(gu_bias)[chosen].to(torch.bfloat16).double()
    wd = torch.as_tensor(w).double().reshape(-1, 1)
    h = _glu(pre[:, I:], pre[:, :I], act) * wd  # [k, I]
    y = sum(h[s] @ down[e].double() for s, e in enumerate(chosen))
    return y.reshape(1, -1), h.reshape(1, -1)


def reference_rows(x, gate_up, down, ids, w, act="silu", gu_bias=None):
    """y [R, H] in float64: row r's reference() with its own ids[r] and w[r] (reference moe8.py:639-644)."""
    rows = [reference(x[r], gate_up, down, ids[r], w[r], act, gu_bias)[0] for r in range(len(ids))]
    return torch.cat(rows, dim=0)


def union(ids, E):
    """The ids' distinct experts below E in increasing order (the kernels' union; reference moe8.py:647-649)."""
    return sorted({int(e) for e in torch.as_tensor(ids).reshape(-1).tolist() if 0 <= int(e) < E})


def u_max(P, rows, k):
    """The most experts the union of rows x k ids can hold: h's width is u_max(...) * I (reference moe8.py:923-925)."""
    return min(P["E"], rows * k)


# --- the ops -------------------------------------------------------------------------------------------------------------


def _loaders(loaders, default):
    loaders = default if loaders is None else loaders
    assert loaders in (1, 2), loaders
    return loaders == 2


def _gu_cpb(P, cpb, default=0):
    """gate_up's cores per bank (reference moe8.py:693-701): a work split only; checked as there."""
    g = P["device"].compute_with_storage_grid_size()
    most = (g.x * g.y) // P["banks"]
    if not cpb:
        return max(1, min(default, most)) if default else P["cpb"]
    assert 1 <= cpb <= most, (cpb, g, P["banks"])
    return cpb


def _ids_ptr(ids, ids32, rows, k):
    """(pointer, row stride) of the ids tensor: uint16 / int16 (ids32 False) or uint32 / int32, on the GPU, its last
    dim the row (at least k values), at least `rows` rows."""
    want = (torch.int32, torch.uint32) if ids32 else (torch.int16, torch.uint16)
    assert ids.dtype in want, f"moe8: ids are {ids.dtype}, ids32={ids32} wants {want[0]} or {want[1]}"
    assert ids.is_cuda and ids.is_contiguous(), (ids.device, ids.is_contiguous())
    ld = ids.shape[-1]
    assert ld >= k and ids.numel() // ld >= rows, (tuple(ids.shape), rows, k)
    return ids.data_ptr(), ld


def _w_ptr(w, rows, k):
    assert w.dtype == torch.bfloat16 and w.is_cuda and w.is_contiguous(), (w.dtype, w.device)
    ld = w.shape[-1]
    assert ld >= k and w.numel() // ld >= rows, (tuple(w.shape), rows, k)
    return w.data_ptr(), ld


def _run(P, x2, m, k_launch, ldx, y, ldy, gate_up_mode, mode, ids, ids32, w, slots, id_rows, act, route=None):
    """One dr_moe_matmul: the launch of expert 0's weight and the gather (include/moe.h); with route (a dr_route),
    dr_moe_route_gate_up: the token routed into ids and w by the same launch."""
    (gc, ge, dc, de), (gk, gn, dk, dn) = P["sizes"], P["pads"]
    L = _lib.Launch()
    L.x, L.m, L.k, L.ldx = x2.data_ptr(), m, k_launch, ldx
    L.y, L.ldy = y.data_ptr(), ldy
    L.act = ACTS[act]
    L.nseg = 1
    s0 = L.seg[0]
    s0.fmt = DR_BFP4_KB if P["kblock"] else DR_BFP4
    M = _lib.Moe()
    M.mode = mode
    M.ids, M.ld_ids = _ids_ptr(ids, ids32, id_rows, slots)
    M.ids32 = int(bool(ids32))
    M.slots, M.id_rows, M.experts = slots, id_rows, P["E"]
    if gate_up_mode:
        s0.glu, s0.n, s0.n_pad = 2, P["I"], gn
        s0.codes, s0.exps = P["gu"][0, 0].data_ptr(), P["gu_exps"][0, 0].data_ptr()
        s0.codes_up, s0.exps_up = P["gu"][0, 1].data_ptr(), P["gu_exps"][0, 1].data_ptr()
        M.w, M.ld_w = _w_ptr(w, id_rows, slots)
        M.expert_n = P["I"]
        M.codes_stride, M.exps_stride = 2 * gc, 2 * ge
        M.bias = P["bias"].data_ptr() if P["bias"] is not None else None
    else:
        s0.glu, s0.n, s0.n_pad = 0, P["H"], dn
        s0.codes, s0.exps = P["dn"][0].data_ptr(), P["dn_exps"][0].data_ptr()
        M.expert_k = P["I"]
        M.codes_stride, M.exps_stride = dc, de
    stream = torch.cuda.current_stream(x2.device)
    L.stream = stream.cuda_stream
    lib = _lib.lib()
    need = lib.dr_moe_workspace_bytes(ctypes.byref(L), ctypes.byref(M))
    _lib.check(_lib.DR_EINVAL if need < 0 else _lib.DR_OK, "dr_moe_workspace_bytes")
    if need > 0:
        ws = linear._workspace(x2.device, stream, need)
        L.workspace, L.workspace_bytes = ws.data_ptr(), ws.numel()
    if route is not None:
        _lib.check(lib.dr_moe_route_gate_up(ctypes.byref(L), ctypes.byref(M), ctypes.byref(route)), "dr_moe_route_gate_up")
    else:
        _lib.check(lib.dr_moe_matmul(ctypes.byref(L), ctypes.byref(M)), "dr_moe_matmul")
    return y


def _x_rows(x, rows, H):
    assert x.dtype == torch.bfloat16 and x.is_cuda, (x.dtype, x.device)
    assert x.shape[-1] == H and x.numel() // H >= rows, (tuple(x.shape), rows, H)
    return x.reshape(-1, H).contiguous()


def gate_up(x, P, ids, w, k, *, ids32=False, kw=8, fidelity="hifi2", memory_config=None, cpb=None, loaders=None,
            act="silu"):
    """h [1, 1, 1, k * I] bf16: per slot s the routing weight w[s] times act(x G + b_g) * (x U + b_u) of expert
    ids[s] (a slot whose id is not below E: zeros). x [1, 1, 1, H] bf16; ids [..., k] uint16 (uint32 with ids32) and
    w [..., k] bf16 on the GPU, their first row used. cpb, loaders, kw, fidelity: the reference's work split,
    checked as there and changing nothing; column groups and a bias need loaders=2 as there. act: "silu", "gelu_tanh"
    or "swiglu_oai" (reference moe8.py:710-817)."""
    assert act in ACTS, f"moe8: act {act!r}"
    assert 1 <= k <= 16, k
    H, I = P["H"], P["I"]
    _gu_cpb(P, cpb, GU_CPB)
    split = _loaders(loaders, LOADERS)
    G, _ = gu_groups(I // TILE, P["banks"])
    assert G == 1 or split, "moe8: gate_up's column groups need two loaders (loaders=2)"
    assert not P["gu_bias"] or split, "moe8: gate_up's bias needs two loaders (loaders=2)"
    x2 = _x_rows(x, 1, H)[:1]
    h = torch.empty(1, 1, 1, k * I, dtype=torch.bfloat16, device=x2.device)
    return _run(P, x2, 1, H, H, h, k * I, True, _lib.DR_MOE_GATE_UP, ids, ids32, w, k, 1, act)


def down(h, P, ids, k, *, ids32=False, kw=8, fidelity="hifi2", memory_config=None, loaders=None):
    """y [1, 1, 1, H] bf16 = h @ the chosen experts' down rows (slot s's I values of h times expert ids[s]'s I rows;
    a slot whose id is not below E adds nothing). h [1, 1, 1, k * I] bf16 (gate_up's) (reference moe8.py:820-910)."""
    assert 1 <= k <= 16, k
    _loaders(loaders, LOADERS)
    H, I = P["H"], P["I"]
    assert h.dtype == torch.bfloat16 and h.is_cuda and h.shape[-1] == k * I, (tuple(h.shape), h.dtype, k * I)
    h2 = h.reshape(-1, k * I)[:1].contiguous()
    y = torch.empty(1, 1, 1, H, dtype=torch.bfloat16, device=h2.device)
    return _run(P, h2, 1, k * I, k * I, y, H, False, _lib.DR_MOE_DOWN, ids, ids32, None, k, 1, "silu")


def _rows_args(rows, k):
    assert 1 <= rows <= TILE and 1 <= k <= 16, (rows, k)


def gate_up_rows(x, P, ids, w, k, rows, *, ids32=False, kw=8, fidelity="hifi2", memory_config=None, cpb=None,
                 act="silu", loaders=None):
    """h [1, 1, 32, u_max * I] bf16 for x's first `rows` rows: union index q's I columns hold row r's routing weight
    for expert union(ids)[q] times act(x_r G + b_g) * (x_r U + b_u) (0 where row r did not choose it); rows past
    `rows` and columns past the union are 0. ids [1, 1, >= rows, k] uint16 (uint32 with ids32) and w [1, 1, >= rows,
    k] bf16, their first `rows` rows (reference moe8.py:928-1037)."""
    assert act in ACTS, f"moe8: act {act!r}"
    _rows_args(rows, k)
    _loaders(loaders, ROWS_LOADERS)
    _gu_cpb(P, cpb, GU_ROWS_CPB)
    H, I = P["H"], P["I"]
    um = u_max(P, rows, k)
    x2 = _x_rows(x, rows, H)[:rows]
    h = torch.zeros(1, 1, TILE, um * I, dtype=torch.bfloat16, device=x2.device)
    return _run(P, x2, rows, H, H, h, um * I, True, _lib.DR_MOE_GATE_UP_ROWS, ids, ids32, w, k, rows, act)


def down_rows(h, P, ids, k, rows, *, ids32=False, kw=8, fidelity="hifi2", memory_config=None, loaders=None):
    """y [1, 1, 32, H] bf16: row r = the sum over the union of the rows x k ids of h's row r (union index q's I
    columns) times expert union(ids)[q]'s down rows; rows past `rows` are 0. h is gate_up_rows' (the same ids, rows
    and k) (reference moe8.py:1040-1136)."""
    _rows_args(rows, k)
    _loaders(loaders, ROWS_LOADERS)
    H, I = P["H"], P["I"]
    um = u_max(P, rows, k)
    assert h.dtype == torch.bfloat16 and h.is_cuda and h.shape[-1] == um * I, (tuple(h.shape), rows, k)
    h2 = h.reshape(-1, um * I)[:rows].contiguous()
    y = torch.zeros(1, 1, TILE, H, dtype=torch.bfloat16, device=h2.device)
    return _run(P, h2, rows, um * I, um * I, y, H, False, _lib.DR_MOE_DOWN_ROWS, ids, ids32, None, k, rows, "silu")


# --- the router ------------------------------------------------------------------------------------------------------


def _route_args(logits, ids, w, k, kind, bias, ids32, experts, shared, scale, norm, groups, slot):
    """route's arguments checked as route takes them, as a dr_route."""
    assert kind in ("softmax", "sigmoid"), f"moe8.route: kind {kind!r}"
    R, W = logits.shape[-2], logits.shape[-1]
    E = experts or W
    assert E <= W and (shared is None or E + 1 <= W), (E, W)
    assert logits.dtype == torch.float32 and logits.is_cuda and logits.is_contiguous(), logits.dtype
    assert R <= 32 and E % TILE == 0 and 1 <= k <= 16, (R, E, k)
    assert 0 < scale < 4, scale
    assert norm or kind == "sigmoid", "moe8.route: norm=False is for the sigmoid kind"
    assert slot is None or (k + 1 <= 16 and 0 <= int(slot) < (1 << 32 if ids32 else 1 << 16)), (k, slot)
    ng, tg = (0, 0) if groups is None else (int(groups[0]), int(groups[1]))
    if groups is not None:
        assert kind == "sigmoid" and bias is not None, "moe8.route: groups need the sigmoid kind with a bias"
        assert ng <= 32 and E % ng == 0 and E // ng >= 2 and 1 <= tg <= ng and tg * (E // ng) >= k, (E, groups, k)
    kk = k + (slot is not None)
    ids_p, ld_ids = _ids_ptr(ids, ids32, R, kk)
    w_p, ld_w = _w_ptr(w, R, kk)
    sig = kind == "sigmoid" and bias is not None
    if sig:
        assert bias.dtype == torch.float32 and bias.is_cuda and bias.shape[-1] == E and bias.is_contiguous(), bias.dtype
    if shared is not None:
        assert shared.dtype == torch.bfloat16 and shared.is_cuda and shared.numel() >= R, shared.dtype
    A = _lib.Route()
    A.logits, A.rows, A.ld_logits, A.experts, A.k = logits.data_ptr(), R, W, E, k
    A.kind = 0 if kind == "softmax" else 1
    A.bias = bias.data_ptr() if sig else None
    A.ids, A.ids32, A.ld_ids = ids_p, int(bool(ids32)), ld_ids
    A.w, A.ld_w = w_p, ld_w
    A.shared = shared.data_ptr() if shared is not None else None
    A.ld_shared = shared.shape[-1] if shared is not None else 0
    A.scale, A.norm = float(scale), int(bool(norm))
    A.n_group, A.topk_group = ng, tg
    A.slot = -1 if slot is None else int(slot)
    A.stream = torch.cuda.current_stream(logits.device).cuda_stream
    return A




def route(logits, ids, w, k, *, kind="softmax", bias=None, ids32=False, experts=None, shared=None, scale=1.0,
          norm=True, groups=None, slot=None):
    """The router's top k and their weights, written into ids [1, 1, R, k] (uint16, or uint32 with ids32) and w [1, 1,
    R, k] bf16 (k + 1 slots with `slot`), slots in decreasing order of the pick's key, the lower id first among equal
    keys. logits [1, 1, R, W] float32 on the GPU, R <= 32; experts (default W): its columns 0 .. E - 1, E a multiple of
    32.
    - kind "softmax": the top k by logit; the weights the softmax over the k.
    - kind "sigmoid": the top k by sigmoid(logit) + bias (bias [E] float32, or None: by logit); the weights the picks'
      sigmoids over their sum (norm=False: not divided).
    shared: [1, 1, R, 1] bf16 that gets sigmoid(logits[:, E]). scale: every weight times it (0 < scale < 4). groups=
    (n_group, topk_group) (sigmoid with a bias): a group's score the sum of its two largest keys, the topk_group best
    groups kept (the lower group first among equal scores). slot: an id written as slot k of every row at weight 1.0.
    Keys and weights in double, rounded to bf16 at the end. Returns w (reference moe8.py:1139-1253)."""
    A = _route_args(logits, ids, w, k, kind, bias, ids32, experts, shared, scale, norm, groups, slot)
    _lib.check(_lib.lib().dr_moe_route(ctypes.byref(A)), "dr_moe_route")
    return w


ROUTE_GATE_UP_MAX_E = 256  # (dr_moe_route_gate_up routes at most this many experts in the gather's launch)


def route_gate_up(logits, x, P, ids, w, k, *, act="silu", kind="softmax", bias=None, ids32=False, shared=None,
                  scale=1.0, norm=True, groups=None, slot=None, loaders=None, cpb=None):
    """route(logits, ids, w, k, ...) of one token, then gate_up(x, P, ids, w, k + (slot given), act=act), in one
    launch (dr_moe_route_gate_up): every workgroup of the gather routes the token itself, with the router's code, so
    ids, w and h are route's and gate_up's bit for bit, with no kernel boundary between them. logits [1, 1, 1, W]
    float32 (one row, E = P's experts); the other arguments as route's and gate_up's. More than 256 experts: route,
    then gate_up (two launches, the same results). Returns h."""
    assert logits.shape[-2] == 1 and logits.numel() == logits.shape[-1], tuple(logits.shape)
    if P["E"] > ROUTE_GATE_UP_MAX_E:
        route(logits, ids, w, k, kind=kind, bias=bias, ids32=ids32, experts=P["E"], shared=shared, scale=scale,
              norm=norm, groups=groups, slot=slot)
        return gate_up(x, P, ids, w, k + (slot is not None), ids32=ids32, loaders=loaders, cpb=cpb, act=act)
    A = _route_args(logits, ids, w, k, kind, bias, ids32, P["E"], shared, scale, norm, groups, slot)
    kk = k + (slot is not None)
    assert act in ACTS, f"moe8: act {act!r}"
    H, I = P["H"], P["I"]
    _gu_cpb(P, cpb, GU_CPB)
    split = _loaders(loaders, LOADERS)
    G, _ = gu_groups(I // TILE, P["banks"])
    assert G == 1 or split, "moe8: gate_up's column groups need two loaders (loaders=2)"
    assert not P["gu_bias"] or split, "moe8: gate_up's bias needs two loaders (loaders=2)"
    x2 = _x_rows(x, 1, H)[:1]
    h = torch.empty(1, 1, 1, kk * I, dtype=torch.bfloat16, device=x2.device)
    return _run(P, x2, 1, H, H, h, kk * I, True, _lib.DR_MOE_GATE_UP, ids, ids32, w, kk, 1, act, route=A)


def route_reference(logits, k, kind="softmax", bias=None, scale=1.0, norm=True, groups=None, slot=None):
    """route's result on the host: (ids [R, k] long, w [R, k] float64) for float32 logits [R, E], in float64 with the
    lower id first among equal keys (a stable sort). Keys: the logits (softmax, or sigmoid without a bias), else
    sigmoid + bias; groups: a group's score the sum of its two largest keys, the topk_group best groups (the lower
    first among equal scores) keeping their keys, the rest -inf. slot: one more column of that id at weight 1.0
    (reference moe8.py:1256-1286)."""
    lg = logits.double()
    R, E = lg.shape
    sg = torch.sigmoid(lg)
    key = sg + bias.double().reshape(1, -1) if (kind == "sigmoid" and bias is not None) else lg
    if groups is not None:
        ng, tg = groups
        score = key.reshape(R, ng, E // ng).topk(2, dim=-1).values.sum(-1)
        rank = torch.argsort(torch.argsort(-score, dim=-1, stable=True), dim=-1)  # each group's place
        keep = (rank < tg).repeat_interleave(E // ng, dim=1)
        key = torch.where(keep, key, torch.full_like(key, float("-inf")))
    ids = torch.argsort(-key, dim=-1, stable=True)[:, :k]
    if kind == "softmax":
        w = torch.softmax(lg.gather(1, ids), dim=-1)
    else:
        v = sg.gather(1, ids)
        w = v / v.sum(dim=-1, keepdim=True) if norm else v
    w = w * scale
    if slot is not None:
        ids = torch.cat([ids, torch.full((R, 1), int(slot), dtype=ids.dtype)], dim=1)
        w = torch.cat([w, torch.ones(R, 1, dtype=w.dtype)], dim=1)
    return ids, w
