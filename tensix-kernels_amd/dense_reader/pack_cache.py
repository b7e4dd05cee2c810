"""pack_cache.py: a versioned on-disk cache of packed dense_reader weights, so a large weight (an LM head of 558 MB)
is packed once and then only read back and uploaded.

It follows the pack cache of XylolabsInc/tensix-kernels' moe/moe8.py (file:line cited per function): a directory per
weight holding the packed arrays (.npy), meta.json (what was packed: the format, the shape and padding, the layout
version, a fingerprint of the source weight) and sums.json (the sha256 of every array), written whole into PATH.tmp
and renamed, so a cache is either complete or absent. A cache whose meta differs from the call is neither taken nor
overwritten (PackCacheMismatch) unless the caller asks to rebuild it; one whose arrays do not match their sums (a
damaged file) is refused the same way.

  w, scale = native_weight_cached(device, lm_head, bfloat8_b, cache="/data/packs/lm_head_bfp8")
"""

import hashlib
import json
import shutil
from pathlib import Path

import numpy as np
import torch

from . import linear

# the packed layout's version: a cache made by another layout (panel width, k-block, exponent order) is refused
PACK_VERSION = 1
LAYOUT = "panels16-kblock1k-exp256"
ARRAYS = ("codes", "exps", "scale")


class PackCacheMismatch(RuntimeError):
    """A pack cache that does not match the call (its meta differs, or its arrays do not match their sums). It is
    neither taken nor overwritten: pass rebuild=True to pack again from the weights and write it over
    (reference moe/moe8.py:278-283)."""


def fingerprint(t):
    """A cheap identity of a weight tensor: its shape, dtype and the sha256 of every 4093rd value as float32
    (reference moe/moe8.py:215-222)."""
    t = torch.as_tensor(t)
    sample = t.reshape(-1)[::4093].float().contiguous().cpu().numpy()
    h = hashlib.sha256(sample.tobytes()).hexdigest()[:32]
    return f"{tuple(t.shape)}:{t.dtype}:{h}"


def _short(v):
    v = repr(v)
    return v if len(v) <= 48 else v[:45] + "..."


def array_sums(arrays):
    """{name: the sha256 of the array's bytes in C order} (reference moe/moe8.py:324-332)."""
    out = {}
    for name, a in arrays.items():
        h = hashlib.sha256()
        h.update(memoryview(np.ascontiguousarray(a)).cast("B"))
        out[name] = h.hexdigest()
    return out


def cache_read(path, meta, rebuild=False, verify=True, names=ARRAYS, what="dense_reader", hint=None):
    """{name: array} of `names` from a cache made with the same meta (memory-mapped); None when there is none (no
    directory or an empty one). A cache that differs from meta, cannot be read or (verify) does not match its sums
    raises PackCacheMismatch and nothing is written; with rebuild it is None and the caller makes it again over it
    (reference moe/moe8.py:289-321). hint(old meta, the keys that differ): a sentence for the message, or ""."""
    path = Path(path)
    if not path.exists() or (path.is_dir() and not any(path.iterdir())):
        return None
    why = None
    try:
        old = json.loads((path / "meta.json").read_text())
    except (OSError, ValueError) as e:
        old, why = None, f"its meta.json cannot be read ({type(e).__name__})"
    if old is not None and not isinstance(old, dict):
        old, why = None, "its meta.json is not a pack's"
    if old == meta:
        try:
            arrays = {n: np.load(path / f"{n}.npy", mmap_mode="r") for n in names if (path / f"{n}.npy").exists()}
            if verify:
                sums = json.loads((path / "sums.json").read_text())
                got = array_sums(arrays)
                if got != sums:
                    bad = sorted(n for n in set(got) | set(sums) if got.get(n) != sums.get(n))
                    raise ValueError(f"arrays {bad} do not match sums.json")
            return arrays
        except (OSError, ValueError) as e:
            why = f"its arrays cannot be read or are damaged ({type(e).__name__}: {e})"
    extra = ""
    if old is not None and old != meta:
        keys = sorted(set(old) | set(meta), key=str)
        diff = [k for k in keys if old.get(k) != meta.get(k)]
        why = "; ".join(f"{k}: cache {_short(old.get(k))}, call {_short(meta.get(k))}" for k in diff)
        extra = hint(old, diff) if hint is not None else ""
    if rebuild:
        return None
    raise PackCacheMismatch(
        f"{what} pack cache {path} does not match this call ({why}). It was neither taken nor overwritten.{extra} "
        "To pack again from these weights over it, pass rebuild=True."
    )


def cache_write(path, meta, arrays):
    """The cache, whole or absent: written into PATH.tmp, then renamed over PATH (reference moe/moe8.py:335-346)."""
    path = Path(path)
    tmp = path.with_name(path.name + ".tmp")
    shutil.rmtree(tmp, ignore_errors=True)
    tmp.mkdir(parents=True)
    for name, a in arrays.items():
        np.save(tmp / f"{name}.npy", np.ascontiguousarray(a))
    (tmp / "sums.json").write_text(json.dumps(array_sums(arrays), indent=1))
    (tmp / "meta.json").write_text(json.dumps(meta, indent=1))
    shutil.rmtree(path, ignore_errors=True)
    tmp.rename(path)


def weight_meta(t, dtype, col_scale, mc, n_pad, k_pad):
    """What a packed weight depends on: the cache's meta.json."""
    n, k = t.shape
    return {
        "version": PACK_VERSION,
        "layout": LAYOUT,
        "format": linear.dev.as_dtype(dtype).name,
        "k": k,
        "n": n,
        "k_pad": k_pad,
        "n_pad": n_pad,
        "banks": mc.banks,
        "shard_width": mc.shard_width,
        "col_scale": bool(col_scale),
        "weight": fingerprint(t),
    }


def native_weight_cached(device, t, dtype, cache, col_scale=False, sharded=True, max_banks=None, rebuild=False,
                         verify=True):
    """linear.native_weight(device, t, dtype, col_scale, sharded, max_banks), taken from the cache directory when its
    meta matches the call (the arrays read back and uploaded), else packed on the GPU and written there. A cache that
    differs raises PackCacheMismatch unless rebuild (then it is packed again and written over). verify: check the
    arrays against their sha256 sums when reading. Returns (weight, scale) as native_weight does (after the reference's
    moe/moe8.py:349-376, which caches its MoE packs the same way)."""
    d = linear.dev.as_device(device)
    t = torch.as_tensor(t)
    n, k = t.shape
    mc = linear.sharded_memcfg(d, k, n, max_banks=max_banks) if sharded else linear.MemoryConfig(0)
    n_pad = mc.banks * mc.shard_width if sharded else -(-n // linear.TILE) * linear.TILE
    k_pad = -(-k // linear.KALIGN) * linear.KALIGN
    dtype = linear.dev.as_dtype(dtype)
    meta = weight_meta(t, dtype, col_scale, mc, n_pad, k_pad)
    arrays = cache_read(cache, meta, rebuild, verify)
    if arrays is None:
        w, scale = linear.native_weight(d, t, dtype, col_scale=col_scale, sharded=sharded, max_banks=max_banks)
        arrays = {"codes": w.codes.cpu().numpy(), "scale": scale.reshape(-1).float().cpu().numpy()}
        if w.exps is not None:
            arrays["exps"] = w.exps.cpu().numpy()
        cache_write(cache, meta, arrays)
        return w, scale
    codes = torch.from_numpy(np.array(arrays["codes"])).to(d.torch)
    exps = torch.from_numpy(np.array(arrays["exps"])).to(d.torch) if "exps" in arrays else None
    w = linear.Weight(d, k, n, dtype, codes, exps, n_pad, k_pad, mc)
    return w, linear.scale_tensor(d, torch.from_numpy(np.array(arrays["scale"])))
