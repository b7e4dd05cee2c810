"""The gfx950 code of the HIP library, scanned for one hazard the compiler cannot see (CPU only: hipcc emits the device
assembly here, no GPU runs).

The bfloat4_b and int4 loops issue v_dot2c_f32_bf16 (with DPP) from inline asm. A DOT result needs 3 wait states before
another VALU instruction reads it (a v_dot2c reading it as its own accumulator needs none); the compiler schedules
around asm it cannot see into, so the source fences every accumulator behind the last dot and its s_nop 2. This test
reads the emitted assembly of every kernel: after each v_dot2c, no instruction may read its destination register
within 3 wait states (each instruction counts one, s_nop N counts N + 1). A read that comes too early takes the value
from before the dot: one lost product, which a relative-error check can miss.
"""

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _vregs(op):
    m = re.match(r"v\[(\d+):(\d+)\]", op)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", op.split()[0]) if op else None
    return {int(m.group(1))} if m else set()


def dot_hazards(asm):
    """[(function, dot line, reading line)] for every read of a v_dot2c destination within 3 wait states."""
    found, func, pending = [], None, []  # pending: (register, wait states left, line of the dot)
    lines = asm.split("\n")
    for ln, raw in enumerate(lines):
        s = raw.strip()
        m = re.match(r"^(_Z\S+):", s)
        if m:
            func, pending = m.group(1), []
            continue
        if not s or s.startswith((";", ".")) or s.endswith(":"):
            continue
        op = s.split()[0]
        if op == "s_nop":
            n = int(s.split()[1], 0) + 1
            pending = [(r, w - n, d) for r, w, d in pending if w - n > 0]
            continue
        if op.startswith(("v_", "global_", "ds_", "buffer_", "flat_")):
            ops = [o.strip() for o in (s.split(None, 1)[1] if " " in s else "").split(",")]
            stores = op.startswith(("global_store", "ds_write", "buffer_store", "flat_store"))
            srcs = ops if stores or not op.startswith("v_") else ops[1:]
            read = set().union(*(_vregs(o) for o in srcs)) if srcs else set()
            dot = op.startswith("v_dot2c")
            if dot:
                read -= _vregs(ops[0])  # (a dot2c accumulating into its own destination)
            found += [(func, lines[d].strip(), s) for r, _, d in pending if r in read]
            pending = [(r, w - 1, d) for r, w, d in pending if w > 1]
            if dot:
                dst = _vregs(ops[0])
                pending = [(r, w, d) for r, w, d in pending if r not in dst] + [(r, 3, ln) for r in dst]
        elif op.startswith("s_"):
            pending = [(r, w - 1, d) for r, w, d in pending if w > 1]
    return found


def test_scanner_finds_a_planted_hazard():
    """The scanner itself: a VALU read one instruction after a dot is found; after s_nop 2 it is not."""
    head = "_Zkernel:\n\tv_dot2c_f32_bf16_dpp v4, v1, v2 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
    assert dot_hazards(head + "\tv_sub_f32_e32 v5, v4, v3\n")
    assert not dot_hazards(head + "\ts_nop 2\n\tv_sub_f32_e32 v5, v4, v3\n")
    assert not dot_hazards(head + "\tv_dot2c_f32_bf16_dpp v4, v1, v6 row_newbcast:1 row_mask:0xf bank_mask:0xf\n")
    assert dot_hazards(head + "\tv_mov_b32_e32 v7, v0\n\tv_add_f32_e32 v5, v3, v4\n")


@pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(), reason="no hipcc")
def test_no_dot_result_read_early(tmp_path):
    import __graft_entry__ as G

    hipcc = G.HIPCC if Path(G.HIPCC).exists() else shutil.which("hipcc")
    flags = [f for f in G.FLAGS if f not in ("-shared", "-fPIC")]
    ndots = 0
    for src in G.SOURCES:
        out = tmp_path / (src.stem + ".s")
        r = subprocess.run([hipcc, *flags, "--cuda-device-only", "-S", str(src), "-o", str(out)], capture_output=True,
                           text=True)
        assert r.returncode == 0, r.stderr[-2000:]
        asm = out.read_text()
        ndots += asm.count("v_dot2c_f32_bf16")
        bad = dot_hazards(asm)
        assert not bad, f"{src.name}: {len(bad)} reads of a dot result inside its wait states, e.g. {bad[:3]}"
    assert ndots > 0, "no v_dot2c found: the scanner is not looking at the loops it guards"
