"""The gfx950 code of the HIP library, scanned for orders the source depends on but cannot state (CPU only: hipcc emits
the device assembly here, no GPU runs).

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


@pytest.fixture(scope="module")
def library_asm(tmp_path_factory):
    """{source file name: its gfx950 assembly}, compiled once for the module's tests."""
    import __graft_entry__ as G

    if shutil.which("hipcc") is None and not Path(G.HIPCC).exists():
        pytest.skip("no hipcc")
    hipcc = G.HIPCC if Path(G.HIPCC).exists() else shutil.which("hipcc")
    flags = [f for f in G.FLAGS if f not in ("-shared", "-fPIC")]
    tmp = tmp_path_factory.mktemp("asm")
    out = {}
    for src in G.SOURCES:
        dst = tmp / (src.stem + ".s")
        r = subprocess.run([hipcc, *flags, "--cuda-device-only", "-S", str(src), "-o", str(dst)], capture_output=True,
                           text=True)
        assert r.returncode == 0, r.stderr[-2000:]
        out[src.name] = dst.read_text()
    return out


def test_no_dot_result_read_early(library_asm):
    ndots = 0
    for name, asm in library_asm.items():
        ndots += asm.count("v_dot2c_f32_bf16")
        bad = dot_hazards(asm)
        assert not bad, f"{name}: {len(bad)} reads of a dot result inside its wait states, e.g. {bad[:3]}"
    assert ndots > 0, "no v_dot2c found: the scanner is not looking at the loops it guards"

def _func_bodies(asm):
    """[(function name, [instruction lines])] of the assembly."""
    out, name, body = [], None, []
    for raw in asm.split("\n"):
        s = raw.strip()
        m = re.match(r"^(_Z\S+):", s)
        if m:
            if name:
                out.append((name, body))
            name, body = m.group(1), []
            continue
        if name and s and not s.startswith((";", ".")) and not s.endswith(":"):
            body.append(s)
    if name:
        out.append((name, body))
    return out


def meeting_order_faults(asm, names=("dr_gemv", "dr_mfma")):
    """[(function, what)] for every kernel whose name holds one of `names` and that has the split-K meeting (one
    returning global_atomic_add, device-scope sc1 stores and loads) where the emitted order breaks the handoff:
    a partial-sum store not followed by an s_waitcnt vmcnt(0) and an s_barrier before the atomic; or a partial-sum load
    before the atomic's result is waited for (s_waitcnt vmcnt(0) after it) and a barrier after that."""
    faults = []
    for func, body in _func_bodies(asm):
        if not any(n in func for n in names):
            continue
        atomics = [i for i, s in enumerate(body) if s.startswith("global_atomic_add") and re.search(r"\bsc0\b", s)]
        if not atomics:
            continue
        if len(atomics) != 1:
            faults.append((func, f"{len(atomics)} returning atomics"))
            continue
        a = atomics[0]
        stores = [i for i, s in enumerate(body) if s.startswith("global_store") and re.search(r"\bsc1\b", s)]
        loads = [i for i, s in enumerate(body) if s.startswith("global_load") and re.search(r"\bsc1\b", s)]
        before = [i for i in stores if i < a]
        if not before or not loads:
            faults.append((func, "no partial-sum stores before the atomic, or no loads"))
            continue
        last = max(before)
        waits = [i for i in range(last + 1, a) if body[i].startswith("s_waitcnt") and "vmcnt(0)" in body[i]]
        if not waits or not any(body[i] == "s_barrier" for i in range(min(waits) + 1, a)):
            faults.append((func, "partial-sum stores not waited for (vmcnt(0), then a barrier) before the atomic"))
        got = [i for i in range(a + 1, len(body)) if body[i].startswith("s_waitcnt") and "vmcnt(0)" in body[i]]
        bar = [i for i in range(got[0] + 1, len(body)) if body[i] == "s_barrier"] if got else []
        if not bar or any(i < bar[0] for i in loads):
            faults.append((func, "a partial-sum load before the atomic's result and the barrier after it"))
    return faults


_MEETING = """_ZN12_GLOBAL__N_17dr_gemvILi1ELi2ELi0ELb1EEEvNS_4ArgsE:
\tv_add_f32_e32 v7, v7, v8
\tglobal_store_dword v[8:9], v7, off sc1
\ts_waitcnt vmcnt(0) expcnt(0) lgkmcnt(0)
\ts_barrier
\tglobal_atomic_add v4, v4, v5, s[18:19] sc0
\ts_waitcnt vmcnt(0)
\tds_write_b32 v4, v3 offset:6400
\ts_waitcnt lgkmcnt(0)
\ts_barrier
\tglobal_load_dword v7, v[4:5], off sc1
\tglobal_store_dword v[0:1], v3, off sc1
"""


def test_meeting_scanner_finds_planted_reorders():
    """The scanner itself: the order above passes; a wait taken out, a store sunk past the atomic or a load hoisted
    above the barrier (or above the atomic) is flagged."""
    assert meeting_order_faults(_MEETING) == []
    no_wait = _MEETING.replace("\ts_waitcnt vmcnt(0) expcnt(0) lgkmcnt(0)\n", "", 1)
    assert meeting_order_faults(no_wait)
    sunk = _MEETING.replace("\tglobal_store_dword v[8:9], v7, off sc1\n", "", 1).replace(
        "\tglobal_atomic_add v4, v4, v5, s[18:19] sc0\n",
        "\tglobal_atomic_add v4, v4, v5, s[18:19] sc0\n\tglobal_store_dword v[8:9], v7, off sc1\n")
    assert meeting_order_faults(sunk)
    hoisted = _MEETING.replace("\tglobal_load_dword v7, v[4:5], off sc1\n", "", 1).replace(
        "\ts_waitcnt lgkmcnt(0)\n\ts_barrier\n", "\tglobal_load_dword v7, v[4:5], off sc1\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier\n")
    assert meeting_order_faults(hoisted)
    early = _MEETING.replace("\tglobal_load_dword v7, v[4:5], off sc1\n", "", 1).replace(
        "\tglobal_atomic_add", "\tglobal_load_dword v7, v[4:5], off sc1\n\tglobal_atomic_add")
    assert meeting_order_faults(early)


def test_split_k_meeting_order(library_asm):
    """Every dense kernel with the split-K meeting (dr_gemv, dr_gemv_g1, dr_mfma, the expert gathers) keeps the
    handoff's order in its gfx950 code."""
    asm = library_asm["dense_reader.hip"]
    met = [f for f, body in _func_bodies(asm) if any(n in f for n in ("dr_gemv", "dr_mfma"))
           and any(s.startswith("global_atomic_add") for s in body)]
    assert len(met) >= 20, f"only {len(met)} kernels with the meeting found: the scanner is not looking at them"
    bad = meeting_order_faults(asm)
    assert not bad, f"{len(bad)} kernels break the split-K handoff's order, e.g. {bad[:3]}"
