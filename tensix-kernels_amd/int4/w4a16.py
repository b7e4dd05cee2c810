"""w4a16.py: an int4-weight matmul with group scales along K (G = 32) for one token, on MI355X, after
XylolabsInc/tensix-kernels' int4/w4a16.py (file:line cited per function).

The weight: symmetric int4 codes q in -7..7 with one bf16 scale per output channel and 32 inputs, the weight being
q * s exactly. int4_weight packs the codes in the bfloat4_b code layout of dense_reader (16-column panels, 1 KiB
k-blocks, a nibble u = q + 8 per value) with no exponents; group_scales lays the scales out so that each lane of a
k-block reads its one scale in a 128-byte run. The matmul is dense_reader's GEMV with a DR_INT4 segment: a lane's 32
values of a k-block are one scale group, so each group sum is scaled once (dr_matmul, include/dense_reader.h).

Entry points: w4a16_linear(x, w, scale), int4_weight(device, codes), group_scales(device, scales), dequantize(w,
scale) (the weight as bfloat8_b for an ordinary matmul over many rows), reference(x, codes, scales).
"""

import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
from common import device as dev  # noqa: E402
from dense_reader import _lib, linear  # noqa: E402

TILE = 32
Q4_TILE = 512
BFP4_TILE = 576
EXP = 129  # the bfloat4_b exponent that reads a 3-bit magnitude m as m (2^(129 - 129))
DR_INT4 = 3
# accepted for code that sets them (the reference's Tensix L1 budget); they change nothing here
L1_BUDGET = None
L1_MARGIN = 32 * 1024
PACK_PRECISE = True


def nibbles(codes):
    """int codes [K, N] (-7..7) -> uint8 [KT, NT, 512]: the reference's tile bytes, per tile the 1024 values in face
    order, sign << 3 | magnitude, two per byte (element 2i in the low nibble) (reference w4a16.py:59-66)."""
    k, n = codes.shape
    q = codes.to(torch.int16).reshape(k // 32, 32, n // 32, 32).permute(0, 2, 1, 3)
    q = q.reshape(k // 32, n // 32, 2, 16, 2, 16).permute(0, 1, 2, 4, 3, 5).reshape(k // 32, n // 32, 1024)
    v = ((q < 0).to(torch.int16) * 8 + q.abs()).to(torch.uint8)
    return v[..., 0::2] | (v[..., 1::2] << 4)


def int4_weight(device, codes, banks=None, max_banks=None):
    """codes [N_out, K] int8 in -7..7 (a linear layer's [out, in] weight) as the kernel's weight: the packed codes "t"
    (uint8, N padded to banks * 32, K to 256) and its layout (reference w4a16.py:69-86)."""
    assert int(codes.abs().max()) <= 7, "w4a16: codes are -7..7"
    n, k = codes.shape
    assert k % TILE == 0, f"w4a16: K = {k} must be a multiple of 32"
    d = dev.as_device(device)
    banks = banks or dev.dram_banks(d, max_banks)
    n_pad = -(-n // (TILE * banks)) * TILE * banks
    k_pad = -(-k // linear.KALIGN) * linear.KALIGN
    q = codes.to(device=d.torch, dtype=torch.int8).contiguous()
    t = torch.empty(_lib.lib().dr_codes_bytes(DR_INT4, k_pad, n_pad), dtype=torch.uint8, device=d.torch)
    _lib.check(_lib.lib().dr_pack_int4(q.data_ptr(), k, n, k, t.data_ptr(), n_pad, k_pad, d.stream()), "dr_pack_int4")
    ns = n_pad // TILE // banks
    return {"t": t, "k": k, "n": n, "banks": banks, "ns": ns, "pitch": ns * Q4_TILE, "n_pad": n_pad, "k_pad": k_pad,
            "device": d}


def group_scales(device, scales):
    """scales [N_out, K/32] (one per output channel and 32 inputs) as bf16 on the device in the kernel's order,
    [panels, k-blocks, 4, 16] (reference w4a16.py:89-97)."""
    d = dev.as_device(device)
    n, g = scales.shape
    k = 32 * g
    n_pad = -(-n // TILE) * TILE
    k_pad = -(-k // linear.KALIGN) * linear.KALIGN
    s = scales.to(device=d.torch, dtype=torch.bfloat16).contiguous()
    out = torch.empty(n_pad // 16, k_pad // 128, 4, 16, dtype=torch.bfloat16, device=d.torch)
    st = _lib.lib().dr_pack_int4_scales(s.data_ptr(), g, n, k, out.data_ptr(), n_pad, k_pad, d.stream())
    _lib.check(st, "dr_pack_int4_scales")
    return out


def dequantized(codes, scales):
    """The float [N_out, K] weight q * s (s rounded to bf16, as the device holds it) (reference w4a16.py:100-102)."""
    return codes.float() * scales.to(torch.bfloat16).float().repeat_interleave(32, dim=1)


def reference(x, codes, scales):
    """x @ (q * s).T in float32 (x as the device sees it: bf16) (reference w4a16.py:105-107)."""
    return x.to(torch.bfloat16).float() @ dequantized(codes, scales).T


def plan(device, wq, cores_per_bank=3, kb=None, kw=None, sbw=None, full_sync=True, split=True, budget=None):
    """The work split, for inspection: the Tensix options are accepted and change nothing (reference
    w4a16.py:110-167)."""
    chunks, kch, rows = _lib.plan(wq["k"], 1)
    return {"chunks": chunks, "kch": kch, "tiles": -(-wq["n"] // TILE), "rows_per_pass": rows}


def algorithmic_bytes(wq):
    """The reference's bytes of an int4 weight: a 512-byte tile of codes per 32 x 32 values and their bf16 group
    scales, 64 bytes a tile (its [K / 32, N] scale tensor)."""
    return (wq["k"] // TILE) * -(-wq["n"] // TILE) * (Q4_TILE + 2 * TILE)


def w4a16_linear(x, wq, scale, *, memory_config=None, fidelity="hifi2", **opts):
    """y = x @ (q * s).T for one token: x [1, 1, 1, K] bf16 on the GPU, wq from int4_weight, scale from group_scales.
    Returns [1, 1, 1, N] bf16. opts (the reference's Tensix work split) change nothing (reference
    w4a16.py:170-253)."""
    assert x.shape[-2] == 1, f"w4a16: one token, got {x.shape[-2]} rows"
    assert x.dtype == torch.bfloat16 and x.is_cuda, (x.dtype, x.device)
    assert x.shape[-1] == wq["k"], (x.shape, wq["k"])
    return rows_matmul(x.reshape(1, wq["k"]), wq, scale).reshape(1, 1, 1, wq["n"])


def rows_matmul(x2, wq, scale):
    """y [M, N] bf16 = x2 [M, K] (bf16, GPU) @ (q * s).T: dr_matmul with a DR_INT4 segment, any M (the library runs
    its GEMV two rows a pass)."""
    L, y, x2 = _launch(x2, wq, scale)
    need = _lib.lib().dr_workspace_bytes(L)
    _lib.check(_lib.DR_EINVAL if need < 0 else _lib.DR_OK, "dr_workspace_bytes")
    if need > 0:
        ws = linear._workspace(x2.device, torch.cuda.current_stream(x2.device), need)
        L.workspace, L.workspace_bytes = ws.data_ptr(), ws.numel()
    _lib.check(_lib.lib().dr_matmul(L), "dr_matmul (int4)")
    return y


def launch_plan(x2, wq, scale):
    """What rows_matmul(x2, wq, scale) launches (linear.launch_plan's dict), without launching it."""
    L, _, x2 = _launch(x2, wq, scale)
    return _lib.launch_info(L)


def _launch(x2, wq, scale):
    """rows_matmul's checks, its dr_launch (one DR_INT4 segment), y, and the contiguous x the launch reads (the
    caller holds it until the launch is enqueued)."""
    n, k = wq["n"], wq["k"]
    assert x2.dim() == 2 and x2.shape[1] == k and x2.dtype == torch.bfloat16 and x2.is_cuda, (x2.shape, x2.dtype, k)
    assert (
        scale.dtype == torch.bfloat16
        and scale.is_cuda
        and scale.dim() == 4
        and scale.shape[0] * 16 >= -(-n // TILE) * TILE
        and scale.shape[1] * 128 == wq["k_pad"]
    ), (scale.shape, n, k)
    m = x2.shape[0]
    x2 = x2.contiguous()
    y = torch.empty(m, n, dtype=torch.bfloat16, device=x2.device)
    L = _lib.Launch()
    L.x, L.m, L.k, L.ldx = x2.data_ptr(), m, k, k
    L.y, L.ldy = y.data_ptr(), n
    L.nseg = 1
    s0 = L.seg[0]
    s0.fmt, s0.n, s0.n_pad = DR_INT4, n, wq["n_pad"]
    s0.codes, s0.exps = wq["t"].data_ptr(), None
    s0.scale = scale.data_ptr()
    L.stream = torch.cuda.current_stream(x2.device).cuda_stream
    return L, y, x2


def _codes_q(wq):
    """The int4 codes [n_pad, k_pad] (int8) of a packed weight, decoded on the device."""
    n_pad, k_pad = wq["n_pad"], wq["k_pad"]
    b = wq["t"].reshape(n_pad // 16, k_pad // 128, 4, 16, 4, 4)  # panel, block, kq, c, dword d, byte j
    u = torch.stack([b & 15, b >> 4], dim=5)  # panel, block, kq, c, d, h (low, high), j: k = 32 kq + 8 d + 4 h + j
    q = u.to(torch.int8) - 8
    return q.permute(0, 3, 1, 2, 4, 5, 6).reshape(n_pad, k_pad)


def dequantize(wq, scale, out=None, cores_per_bank=3):
    """The int4 weight times its group scales as a bfloat8_b weight [1, 1, K, N] over the same banks, for an ordinary
    block-float matmul over many rows (prefill). out: a weight of that shape to write into (reference
    w4a16.py:255-337)."""
    n, k, n_pad, k_pad = wq["n"], wq["k"], wq["n_pad"], wq["k_pad"]
    q = _codes_q(wq)[:n, :k].float()
    s = scale.permute(0, 3, 1, 2).reshape(scale.shape[0] * 16, -1)[:n, : k // 32].float()  # [n, K / 32]
    w = q * s.repeat_interleave(32, dim=1)
    mb = wq["banks"]
    fresh, _ = linear.native_weight(wq["device"], w, linear.bfloat8_b, max_banks=mb)
    if out is None:
        return fresh
    assert tuple(out.shape) == tuple(fresh.shape) and out.dtype == fresh.dtype and out.n_pad == fresh.n_pad, out
    out.codes.copy_(fresh.codes)
    out.exps.copy_(fresh.exps)
    return out
