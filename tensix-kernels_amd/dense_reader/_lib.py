"""ctypes binding of libdense_reader.so (the C ABI declared in include/dense_reader.h, include/lm_head.h and
include/moe.h).

The library is built in-tree (`python -c "import __graft_entry__; __graft_entry__.build()"` at the repository root,
or `make -C tensix-kernels_amd/dense_reader/csrc`). There is no fallback: without the library every op raises.
"""

import ctypes
import os
from pathlib import Path

LIB_NAME = "libdense_reader.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

DR_OK, DR_EINVAL, DR_EHIP, DR_ERANGE = 0, 1, 2, 3

# every symbol include/dense_reader.h, include/lm_head.h and include/moe.h declare
SYMBOLS = (
    "dr_codes_bytes",
    "dr_exps_bytes",
    "dr_pack",
    "dr_pack_int4",
    "dr_int4_scales_bytes",
    "dr_pack_int4_scales",
    "dr_unpack",
    "dr_matmul",
    "dr_matmul_noalloc",
    "dr_scratch_bytes",
    "dr_workspace_bytes",
    "dr_topk_merge",
    "dr_topk_merge_workspace_bytes",
    "dr_plan",
    "dr_launch_plan",
    "dr_launch_work",
    "dr_stream_read",
    "dr_status_string",
    "dr_version",
    "dr_head_pick",
    "dr_head_pick_records",
    "dr_moe_workspace_bytes",
    "dr_moe_matmul",
    "dr_moe_route",
    "dr_moe_route_gate_up",
)

DR_MOE_GATE_UP, DR_MOE_DOWN, DR_MOE_GATE_UP_ROWS, DR_MOE_DOWN_ROWS = 1, 2, 3, 4

c_int, c_int32, c_int64, c_void_p = ctypes.c_int, ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p


class Segment(ctypes.Structure):
    _fields_ = [
        ("fmt", c_int32),
        ("n", c_int32),
        ("n_pad", c_int32),
        ("glu", c_int32),
        ("codes", c_void_p),
        ("exps", c_void_p),
        ("codes_up", c_void_p),
        ("exps_up", c_void_p),
        ("scale", c_void_p),
        ("scale_up", c_void_p),
        ("scale_f32", c_int32),
        ("col0", c_int32),
    ]


class TopK(ctypes.Structure):
    _fields_ = [
        ("records", c_void_p),
        ("k", c_int32),
        ("rows", c_int32),
        ("slot0", c_int32),
        ("records_cap", c_int32),
        ("n_valid", c_int32),
        ("base", c_int64),
        ("write_y", c_int32),
        ("fp32", c_int32),
        ("max_records", c_int32),
    ]


class Launch(ctypes.Structure):
    _fields_ = [
        ("x", c_void_p),
        ("m", c_int32),
        ("k", c_int32),
        ("ldx", c_int32),
        ("y", c_void_p),
        ("ldy", c_int32),
        ("y_f32", c_int32),
        ("residual", c_void_p),
        ("ldr", c_int32),
        ("residual_mode", c_int32),
        ("act", c_int32),
        ("nseg", c_int32),
        ("seg", Segment * 4),
        ("topk", TopK),
        ("workspace", c_void_p),
        ("workspace_bytes", c_int64),
        ("stream", c_void_p),
    ]


class LaunchInfo(ctypes.Structure):
    _fields_ = [
        ("kernel", c_int32),
        ("rows_per_pass", c_int32),
        ("tile_cols", c_int32),
        ("tiles", c_int32),
        ("chunks", c_int32),
        ("kch", c_int32),
        ("splits", c_int32),
        ("workgroups", c_int32),
        ("passes", c_int32),
        ("records", c_int32),
        ("tiles_per_record", c_int32),
        ("waves", c_int32),
        ("tiles_per_workgroup", c_int32),
        ("lds_bytes", c_int32),
        ("reserved", c_int32 * 2),
    ]


class Moe(ctypes.Structure):
    _fields_ = [
        ("mode", c_int32),
        ("ids", c_void_p),
        ("ids32", c_int32),
        ("ld_ids", c_int32),
        ("slots", c_int32),
        ("id_rows", c_int32),
        ("experts", c_int32),
        ("w", c_void_p),
        ("ld_w", c_int32),
        ("expert_n", c_int32),
        ("expert_k", c_int32),
        ("codes_stride", c_int64),
        ("exps_stride", c_int64),
        ("bias", c_void_p),
    ]


class Route(ctypes.Structure):
    _fields_ = [
        ("logits", c_void_p),
        ("rows", c_int32),
        ("ld_logits", c_int32),
        ("experts", c_int32),
        ("k", c_int32),
        ("kind", c_int32),
        ("bias", c_void_p),
        ("ids", c_void_p),
        ("ids32", c_int32),
        ("ld_ids", c_int32),
        ("w", c_void_p),
        ("ld_w", c_int32),
        ("shared", c_void_p),
        ("ld_shared", c_int32),
        ("scale", ctypes.c_double),
        ("norm", c_int32),
        ("n_group", c_int32),
        ("topk_group", c_int32),
        ("slot", c_int64),
        ("stream", c_void_p),
    ]


_lib = None


def lib():
    """The loaded library (RuntimeError when it is not built)."""
    global _lib
    if _lib is None:
        path = os.environ.get("DENSE_READER_LIB", str(LIB_PATH))
        if not Path(path).exists():
            raise RuntimeError(
                f"dense_reader: {path} is not built (run __graft_entry__.build() or make in dense_reader/csrc); "
                "there is no fallback path"
            )
        L = ctypes.CDLL(path)
        L.dr_codes_bytes.restype = c_int64
        L.dr_codes_bytes.argtypes = [c_int, c_int, c_int]
        L.dr_exps_bytes.restype = c_int64
        L.dr_exps_bytes.argtypes = [c_int, c_int, c_int]
        L.dr_pack.restype = c_int
        L.dr_pack.argtypes = [c_void_p, c_int64, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p]
        L.dr_pack_int4.restype = c_int
        L.dr_pack_int4.argtypes = [c_void_p, c_int64, c_int, c_int, c_void_p, c_int, c_int, c_void_p]
        L.dr_int4_scales_bytes.restype = c_int64
        L.dr_int4_scales_bytes.argtypes = [c_int, c_int]
        L.dr_pack_int4_scales.restype = c_int
        L.dr_pack_int4_scales.argtypes = [c_void_p, c_int64, c_int, c_int, c_void_p, c_int, c_int, c_void_p]
        L.dr_unpack.restype = c_int
        L.dr_unpack.argtypes = [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p, c_int64, c_void_p]
        L.dr_matmul.restype = c_int
        L.dr_matmul.argtypes = [ctypes.POINTER(Launch)]
        L.dr_matmul_noalloc.restype = c_int
        L.dr_matmul_noalloc.argtypes = [ctypes.POINTER(Launch)]
        L.dr_scratch_bytes.restype = c_int64
        L.dr_scratch_bytes.argtypes = []
        L.dr_workspace_bytes.restype = c_int64
        L.dr_workspace_bytes.argtypes = [ctypes.POINTER(Launch)]
        L.dr_topk_merge.restype = c_int
        L.dr_topk_merge.argtypes = [c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p, c_int64,
                                    c_void_p]
        L.dr_topk_merge_workspace_bytes.restype = c_int64
        L.dr_topk_merge_workspace_bytes.argtypes = [c_int, c_int, c_int]
        L.dr_plan.restype = c_int
        L.dr_plan.argtypes = [c_int, c_int, ctypes.POINTER(c_int32), ctypes.POINTER(c_int32), ctypes.POINTER(c_int32)]
        L.dr_launch_plan.restype = c_int
        L.dr_launch_plan.argtypes = [ctypes.POINTER(Launch), ctypes.POINTER(LaunchInfo)]
        L.dr_launch_work.restype = c_int
        L.dr_launch_work.argtypes = [ctypes.POINTER(Launch), ctypes.POINTER(c_int32), c_int]
        L.dr_stream_read.restype = c_int
        L.dr_stream_read.argtypes = [c_void_p, c_int64, c_void_p, c_void_p]
        L.dr_status_string.restype = ctypes.c_char_p
        L.dr_status_string.argtypes = [c_int]
        L.dr_version.restype = c_int
        L.dr_version.argtypes = []
        L.dr_head_pick.restype = c_int
        L.dr_head_pick.argtypes = [c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p, c_int, c_int, c_void_p, c_int64,
                                   c_int64, c_void_p, c_void_p, c_void_p, c_int64, c_void_p]
        L.dr_head_pick_records.restype = c_int
        L.dr_head_pick_records.argtypes = [c_void_p, c_int, c_int, c_int, c_int64, c_void_p, c_void_p, c_void_p,
                                           c_void_p, c_int64, c_void_p]
        L.dr_moe_workspace_bytes.restype = c_int64
        L.dr_moe_workspace_bytes.argtypes = [ctypes.POINTER(Launch), ctypes.POINTER(Moe)]
        L.dr_moe_matmul.restype = c_int
        L.dr_moe_matmul.argtypes = [ctypes.POINTER(Launch), ctypes.POINTER(Moe)]
        L.dr_moe_route.restype = c_int
        L.dr_moe_route.argtypes = [ctypes.POINTER(Route)]
        L.dr_moe_route_gate_up.restype = c_int
        L.dr_moe_route_gate_up.argtypes = [ctypes.POINTER(Launch), ctypes.POINTER(Moe), ctypes.POINTER(Route)]
        _lib = L
    return _lib


def check(status, what):
    """Raise for a non-zero status: ValueError for an argument the op does not take, else RuntimeError."""
    if status == DR_OK:
        return
    msg = f"{what}: {lib().dr_status_string(status).decode()} (status {status})"
    if status in (DR_EINVAL, DR_ERANGE):
        raise ValueError(msg)
    raise RuntimeError(msg)


def launch_info(L):
    """dr_launch_plan of a filled dr_launch: what dr_matmul would launch, as a dict ("kernel": "gemv" or "mfma")."""
    info = LaunchInfo()
    check(lib().dr_launch_plan(L, info), "dr_launch_plan")
    out = {f: getattr(info, f) for f, _ in LaunchInfo._fields_ if f != "reserved"}
    out["kernel"] = ("gemv", "mfma")[info.kernel]
    return out


def launch_work(L, workgroups):
    """dr_launch_work of a filled dr_launch: [(block, first tile, tiles, split, first output column)] a workgroup."""
    buf = (c_int32 * (5 * max(1, workgroups)))()
    check(lib().dr_launch_work(L, buf, workgroups), "dr_launch_work")
    return [tuple(buf[5 * i : 5 * i + 5]) for i in range(workgroups)]


def plan(k, m):
    """(chunks, kch, rows_per_pass) of the library's work split for K and M."""
    c, ch, r = c_int32(), c_int32(), c_int32()
    check(lib().dr_plan(k, m, ctypes.byref(c), ctypes.byref(ch), ctypes.byref(r)), "dr_plan")
    return c.value, ch.value, r.value
