"""Benchmark of the dense_reader decode matmul on one MI355X.

  python bench.py [--steps K] [--warmup W] [--config ns|c1|c2|c3|c4|c5|int4|moe|moe_rows|lm] [--no-cpu] [--cpu-seconds S]
  python bench.py --copy-probe      (a plain 256 MiB copy kernel: the byte counters' calibration under rocprofv3)
  python bench.py --read-probe BYTES  (the read ceiling: dr_stream_read of BYTES, timed as a config is)
  --no-eager: skip the eager timing loop (rocprofv3 traces then hold the graph-replayed launches but the warm-up's)

Default workload: the north-star decode matmul, bfloat8_b M=1, x [1, 4096] bf16 @ W [4096 in, 14336 out] (W ~
N(0, 0.02)), no fused stage, bf16 output. A step is one call of the op (c5: the matmul with top-k records, then the
merge of the records). Weights rotate over enough distinct copies (>= 512 MB) that the 256 MB Infinity Cache cannot
serve them. The K timed steps are captured once in a HIP graph (the analogue of the reference's ttnn trace) and
replayed between synchronisations; events on the replay stream bracket the timed region. One JSON line on stdout:

  value             algorithmic weight bytes per step (the reference's 1088 / 576 / 2048 B per 32x32 tile of
                    bfloat8_b / bfloat4_b / bfloat16; int4: 512 B of codes and 64 B of bf16 group scales) x steps /
                    timed seconds, GB/s, inputs resident in HBM;
  roofline.achieved the same bytes per matmul launch / that kernel's mean duration (a graph of K launches of the
                    matmul alone, timed the same way; the step itself when it is one launch);
  roofline.traffic  HBM bytes per launch from rocprofv3 FETCH_SIZE / WRITE_SIZE runs (profiles/traffic.md), scaled by
                    what the counters read for a copy kernel of known size, or null when no such row exists;
  cpu_baseline      the reference's own float32 CPU check path (dense_reader/linear.py:166-169, restated in
                    oracle.dense_oracle.ref_f32) with the config's epilogue, on this host's cores, on the same shapes.
"""

import argparse
import json
import math
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "tensix-kernels_amd"))
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MALL_BYTES = 512 * 2**20
TRAFFIC_TABLE = ROOT / "profiles" / "traffic.md"
METRIC = "weight GB/s and % HBM peak, bfp8_b M=1 decode matmul; µs/call"

# name: (workload, m, k, weights [(n, fmt, scaled)], options)
CONFIGS = {
    "ns": ("bfp8 M=1 K=4096 N=14336 decode matmul (north star)", 1, 4096, [(14336, "bfp8", False)], {}),
    "c1": ("bfp8 M=1 K=2048 N=4096, no fused stage", 1, 2048, [(4096, "bfp8", False)], {}),
    "c2": (
        "bfp4 M=1 K=4096 gate+up 2x14336, fp32 column scales, SwiGLU",
        1,
        4096,
        [(14336, "bfp4", True), (14336, "bfp4", True)],
        {"glu2": True},
    ),
    "c3": ("bfp8 M=8 K=14336 N=4096, residual, fp32 out", 8, 14336, [(4096, "bfp8", False)], {"residual": True}),
    "c4": (
        "block list M=32 K=4096: Q 4096 + K 1024 + V 1024 bfp8 with column scales, O 4096 bf16, one launch",
        32,
        4096,
        [(4096, "bfp8", True), (1024, "bfp8", True), (1024, "bfp8", True), (4096, "bf16", False)],
        {"blocks": True},
    ),
    "c5": (
        "bfp8 M=4 K=4096 N=128256 LM head, fp32 top-8 records per 32-column tile + global top-32 merge",
        4,
        4096,
        [(128256, "bfp8", False)],
        {"topk": True},
    ),
    "int4": (
        "int4 W4A16 M=1 K=4096 N=14336: codes -7..7 with a bf16 scale per column and 32 inputs (int4 w4a16_linear)",
        1,
        4096,
        [(14336, "int4", True)],
        {"int4": True},
    ),
    "moe": (
        "MoE layer decode, gpt-oss-20b shape: E=32 experts, top-4, H=2880, I=2880, swiglu_oai with gate/up bias, "
        "bfp4 experts; a step is route (softmax top-4 of the router logits) + gate_up, in one launch "
        "(moe8.route_gate_up), then down",
        1,
        2880,
        [(2880, "bfp4", False)],
        {"moe": (32, 4, 2880, 2880)},
    ),
    "moe_rows": (
        "MoE layer at 32 rows (verify / prefill), gpt-oss-20b shape: E=32, top-4 per row of random distinct experts, "
        "H=I=2880, swiglu_oai with gate/up bias, bfp4 experts; a step is gate_up over the rows' union of experts "
        "(moe8.gate_up_rows), then down (moe8.down_rows)",
        32,
        2880,
        [(2880, "bfp4", False)],
        {"moe": (32, 4, 2880, 2880), "rows": 32},
    ),
    "lm": (
        "LM head to token ids, M=4 K=4096 vocab=128256 bfp8: bf16 top-8 records, the best 16 rescored from the bf16 "
        "rows and picked on the device (lm_head_topk DeviceHead, device_pick)",
        4,
        4096,
        [(128256, "bfp8", False)],
        {"lmhead": True},
    ),
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=2000)
    ap.add_argument("--config", default="ns", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--copy-probe", action="store_true")
    ap.add_argument("--read-probe", type=int, default=0, metavar="BYTES")
    ap.add_argument("--no-eager", action="store_true")
    ap.add_argument("--kblock", action="store_true",
                    help="config moe: the experts packed with their shared exponents along K (moe8.pack(kblock=True))")
    return ap.parse_args()


def copy_probe():
    """Five launches of one elementwise kernel that reads 256 MiB and writes 256 MiB (torch.neg, float32)."""
    import torch

    n = 64 * 2**20
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe": "torch.neg float32", "read_bytes": 4 * n, "write_bytes": 4 * n}), flush=True)


def read_probe(torch, nbytes, steps, warmup):
    """The read ceiling: `steps` launches of dr_stream_read over nbytes each, rotating over enough buffers (>= 512 MB)
    that the Infinity Cache cannot serve them, captured in a HIP graph and timed as a config's steps are."""
    from dense_reader import _lib

    lib = _lib.lib()
    nbytes = nbytes // 16 * 16
    copies = max(2, math.ceil(MALL_BYTES / nbytes) + 1)
    bufs = [torch.ones(nbytes, dtype=torch.uint8, device="cuda") for _ in range(copies)]
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")

    def step(i):
        st = torch.cuda.current_stream()
        _lib.check(lib.dr_stream_read(bufs[i % copies].data_ptr(), nbytes, sink.data_ptr(), st.cuda_stream),
                   "dr_stream_read")

    for i in range(min(warmup, 20)):
        step(i)
    torch.cuda.synchronize()
    ms = timed_graph(torch, step, steps, warm_replays(warmup, steps))
    us = ms * 1e3 / steps
    print(json.dumps({"read_probe": "dr_stream_read", "bytes": nbytes, "steps": steps, "buffers_rotated": copies,
                      "us_per_launch": round(us, 3), "GB/s": round(nbytes / (us * 1e-6) / 1e9, 2),
                      "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}), flush=True)


MFMA_TABLE = ROOT / "profiles" / "mfma_l2.md"
MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense bf16


def mfma_row(name):
    """The counter figures of config `name` from profiles/mfma_l2.md (a row `| name | kernel | rows | TFLOP/s | % of
    peak | busy % | L1 -> L2 MB | x weight bytes | L2 hit % |`), or None."""
    if not MFMA_TABLE.exists():
        return None
    for line in MFMA_TABLE.read_text().splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) == 9 and cells[0] == name:
            try:
                return {"counter_tflops": float(cells[3]), "counter_pct_of_peak": float(cells[4]),
                        "busy_pct": float(cells[5]), "l1_to_l2_read_mb": float(cells[6]), "l2_hit_pct": float(cells[8])}
            except ValueError:
                return None
    return None


def traffic_row(name):
    """HBM bytes per matmul launch for config `name` from the table of profiles/traffic.md (a row
    `| name | kernel | ... | bytes |` whose last cell is the scaled traffic), or None."""
    if not TRAFFIC_TABLE.exists():
        return None
    for line in TRAFFIC_TABLE.read_text().splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 3 and cells[0] == name and re.fullmatch(r"\d+", cells[-1]):
            return int(cells[-1])
    return None


class Workload:
    """The inputs of one config on the GPU and its two launch sequences: step(i) (the op as a user calls it) and
    kernel(i) (the matmul launch alone)."""

    def __init__(self, name, linear, torch, kblock=False):
        self.name = name
        self.kblock = kblock
        desc, m, k, ws, o = CONFIGS[name]
        self.desc, self.m, self.k, self.spec, self.o = desc, m, k, ws, o
        self.linear = linear
        dev = linear.dev.open_device(0)
        g = torch.Generator(device="cuda").manual_seed(0)
        fmts = {"bfp8": linear.bfloat8_b, "bfp4": linear.bfloat4_b, "bf16": linear.bfloat16}
        self.x = torch.randn(m, k, generator=g, device="cuda").to(torch.bfloat16).reshape(1, 1, m, k)

        self.heads = None
        self.kbytes = None  # bytes of the dominant kernel a launch (default: the step's weight bytes)
        if o.get("moe"):
            self._init_moe(dev, g, torch)
            return
        if o.get("int4"):
            from int4 import w4a16

            def make():
                n = ws[0][0]
                codes = torch.randint(-7, 8, (n, k), generator=g, device="cuda", dtype=torch.int8)
                scales = (torch.rand(n, k // 32, generator=g, device="cuda") * 0.01 + 0.001).to(torch.bfloat16)
                return [Int4Set(w4a16, dev, codes, scales)]

        elif o.get("lmhead"):
            from lm_head_topk import lmhead

            def make():
                w = torch.randn(ws[0][0], k, generator=g, device="cuda") * 0.02
                h = lmhead.DeviceHead(dev, w, fmt=ws[0][1], chunks=1, k=8, top=16, device_pick=True)
                return h

            self.heads = [make()]
        else:

            def make():
                return [
                    linear.native_weight(dev, torch.randn(n, k, generator=g, device="cuda") * 0.02, fmts[f])[0]
                    for n, f, _ in ws
                ]

        first = make() if self.heads is None else [self.heads[0].blocks[0][0]]
        self.wbytes = sum(w.algorithmic_bytes() for w in first)
        self.copies = max(2, math.ceil(MALL_BYTES / sum(w.nbytes() for w in first)) + 1)
        if self.heads is not None:
            self.heads += [make() for _ in range(self.copies - 1)]
            self.sets = [[h.blocks[0][0]] for h in self.heads]
        else:
            self.sets = [first] + [make() for _ in range(self.copies - 1)]
        self.scales = [
            linear.scale_tensor(dev, torch.rand(n, generator=g, device="cuda") + 0.5, dtype=linear.float32)
            if sc and not o.get("int4") else None
            for n, _, sc in ws
        ]
        self.n = ws[0][0] if (o.get("glu2")) else sum(n for n, _, _ in ws)
        n = self.n
        self.res = torch.randn(m, n, generator=g, device="cuda").to(torch.bfloat16).reshape(1, 1, m, n) if o.get("residual") else None
        self.y = torch.empty(1, 1, m, n, dtype=torch.bfloat16, device="cuda")
        # (c5: a record per 32-column block, as the config asks: no limit on the records)
        self.rec = linear.topk_result(dev, linear.topk_slots(n, 0), m, 8) if o.get("topk") else None
        self.col0 = []
        c = 0
        for nb, _, _ in ws:
            self.col0.append(c // 32)
            c += nb

    def _init_moe(self, dev, g, torch):
        """The MoE layer: E experts packed once (their fp32 weights made on the GPU and dropped), E / k disjoint sets
        of k experts that steps cycle through (each set's router logits favour it; the ids and weights of each set are
        routed once for the kernel-alone timing), and one token x."""
        from moe import moe8

        E, k, H, I = self.o["moe"]
        self.moe8, self.moe_shape = moe8, (E, k, H, I)
        gate_up = torch.randn(E, H, 2 * I, generator=g, device="cuda") * 0.02
        down = torch.randn(E, I, H, generator=g, device="cuda") * 0.02
        bias = torch.randn(E, 2 * I, generator=g, device="cuda") * 0.1
        self.P = moe8.pack(dev, gate_up, down, gu_bias=bias, kblock=self.kblock)
        self.host_w = (gate_up[:k].cpu(), down[:k].cpu(), bias[:k].cpu())  # (the CPU baseline's experts)
        del gate_up, down
        nsets = E // k
        self.logits = []
        for s_ in range(nsets):
            lg = torch.randn(1, 1, 1, E, generator=g, device="cuda") * 0.5
            lg[..., s_ * k : (s_ + 1) * k] += 10.0
            self.logits.append(lg)
        self.ids = torch.zeros(1, 1, 1, k, dtype=torch.int16, device="cuda")
        self.wts = torch.zeros(1, 1, 1, k, dtype=torch.bfloat16, device="cuda")
        self.set_ids, self.set_wts = [], []
        for lg in self.logits:
            ti = torch.zeros(1, 1, 1, k, dtype=torch.int16, device="cuda")
            tw = torch.zeros(1, 1, 1, k, dtype=torch.bfloat16, device="cuda")
            moe8.route(lg, ti, tw, k)
            self.set_ids.append(ti)
            self.set_wts.append(tw)
        self.x = (torch.randn(1, 1, 1, H, generator=g, device="cuda")).to(torch.bfloat16)
        tile = 576  # the reference's bytes of a BFP4_b tile
        units = k
        self.copies = nsets
        R = self.o.get("rows")
        if R:  # R rows of random distinct experts each: the launches read the rows' union of experts once
            gc = torch.Generator().manual_seed(1)
            rid = torch.stack([torch.randperm(E, generator=gc)[:k] for _ in range(R)])
            self.rows_ids = rid.to(torch.int16).reshape(1, 1, R, k).to("cuda")
            self.rows_wts = torch.softmax(torch.randn(R, k, generator=gc), -1).to(torch.bfloat16).reshape(1, 1, R, k).to("cuda")
            self.x = torch.randn(1, 1, R, H, generator=g, device="cuda").to(torch.bfloat16)
            units = len(set(rid.flatten().tolist()))
            self.copies = 1  # (the union's weights, units x 14 MB, are already past the 256 MB Infinity Cache)
        self.kbytes = units * (H // 32) * (2 * I // 32) * tile  # gate_up
        self.wbytes = self.kbytes + units * (I // 32) * (H // 32) * tile  # + down
        self.scales, self.res, self.rec, self.n = [None], None, None, H

    def kernel(self, i):
        if self.o.get("rows"):
            _, k, _, _ = self.moe_shape
            self.moe8.gate_up_rows(self.x, self.P, self.rows_ids, self.rows_wts, k, self.o["rows"], act="swiglu_oai",
                                   loaders=2)
            return
        if self.o.get("moe"):
            _, k, _, _ = self.moe_shape
            s_ = i % self.copies
            self.moe8.route_gate_up(self.logits[s_], self.x, self.P, self.set_ids[s_], self.set_wts[s_], k,
                                    act="swiglu_oai", loaders=2)
            return
        L, o, ws = self.linear, self.o, self.sets[i % self.copies]
        if o.get("glu2"):
            L.matmul(self.x, ws[0], self.scales[0], out=self.y, glu=True, w_up=ws[1], scale_up=self.scales[1])
        elif o.get("blocks"):
            blocks = [(w, c0, s) if s is not None else (w, c0) for w, c0, s in zip(ws, self.col0, self.scales)]
            L.matmul(self.x, blocks, None, out=self.y)
        elif o.get("topk"):
            spec = {"r": self.rec, "k": 8, "rows": self.m, "slot0": 0, "base": 0, "n": self.n, "write_y": False,
                    "fp32": True, "slots": 0}
            L.matmul(self.x, ws[0], None, out=self.y, topk=spec)
        elif o.get("lmhead"):
            h = self.heads[i % self.copies]
            if self.m not in h.results:
                h.logits_topk(self.x, self.m)  # (the result tensor, made once outside any graph)
            spec = {"r": h.results[self.m], "k": h.k, "rows": self.m, "slot0": 0, "base": 0, "n": h.step, "write_y": False,
                    "slots": h.slots}
            L.matmul(self.x, ws[0], None, out=h.y, topk=spec)
        elif o.get("int4"):
            ws[0].w4a16.w4a16_linear(self.x, ws[0].wq, ws[0].ts)
        elif self.res is not None:
            L.matmul(self.x, ws[0], None, residual=self.res, out32=True)  # (fp32 out: a fresh output each call)
        else:
            L.matmul(self.x, ws[0], None, out=self.y)

    def step(self, i):
        if self.o.get("rows"):
            m8, (_, k, _, _), R = self.moe8, self.moe_shape, self.o["rows"]
            h = m8.gate_up_rows(self.x, self.P, self.rows_ids, self.rows_wts, k, R, act="swiglu_oai", loaders=2)
            m8.down_rows(h, self.P, self.rows_ids, k, R, loaders=2)
            return
        if self.o.get("moe"):
            m8, (_, k, _, _) = self.moe8, self.moe_shape
            h = m8.route_gate_up(self.logits[i % self.copies], self.x, self.P, self.ids, self.wts, k,
                                 act="swiglu_oai", loaders=2)
            m8.down(h, self.P, self.ids, k)
            return
        if self.o.get("lmhead"):
            self.heads[i % self.copies].logits_topk(self.x, self.m)
            return
        self.kernel(i)
        if self.o.get("topk"):
            self.linear.topk_merge(self.rec, self.m, 8, k_out=32, fp32=True)


class Int4Set:
    """An int4 weight and its group scales on the GPU (int4.w4a16), with the byte counts the bench reports."""

    def __init__(self, w4a16, dev, codes, scales):
        self.w4a16, self.codes, self.scales = w4a16, codes, scales
        self.wq = w4a16.int4_weight(dev, codes)
        self.ts = w4a16.group_scales(dev, scales)

    def algorithmic_bytes(self):
        return self.w4a16.algorithmic_bytes(self.wq)

    def nbytes(self):
        return self.wq["t"].numel() + 2 * self.ts.numel()


def warm_replays(warmup, steps):
    """Untimed replays of the K-step graph that make up the W warm-up steps (at least one)."""
    return max(1, math.ceil(warmup / steps))


def timed_graph(torch, fn, steps, warm=1):
    """ms for `steps` calls of fn captured in one HIP graph and replayed once after `warm` untimed replays back to
    back, events on the replay stream. The untimed replays are the warm-up: from idle, this MI355X streams 5-8 % slower
    for its first ~10 ms of work (the north star's launch 12.3 -> 11.3 us over its first five 200-launch replays, and
    back to 11.6-11.9 after a second idle), so the timed replay follows tens of ms of the same work."""
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(steps):
            fn(i)
    for _ in range(warm):
        graph.replay()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(st)
    graph.replay()
    t1.record(st)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1)


def main():
    a = parse()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(
            "bench.py: this build measures one GPU only; the decode matmul would shard its output columns over GPUs "
            "and no figure at several GPUs is produced",
            file=sys.stderr,
        )
        sys.exit(2)
    import torch

    if a.copy_probe:
        copy_probe()
        return
    if a.read_probe:
        read_probe(torch, a.read_probe, a.steps, a.warmup)
        return

    from dense_reader import linear

    if a.kblock and not CONFIGS[a.config][4].get("moe"):
        print("bench.py: --kblock applies to the moe config only", file=sys.stderr)
        sys.exit(2)
    wl = Workload(a.config, linear, torch, a.kblock)
    # warm-up: a few eager steps (first calls: workspaces, result tensors), the rest as untimed replays of the captured
    # graph right before the timed one
    eager_warm = min(a.warmup, 20)
    for i in range(eager_warm):
        wl.step(i)
    torch.cuda.synchronize()
    warm = warm_replays(a.warmup - eager_warm, a.steps)

    # eager: each call bracketed by events on its stream (host launch cost included)
    st = torch.cuda.current_stream()
    nev = 0 if a.no_eager else min(a.steps, 100)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(nev)]
    for i in range(nev):
        ev[i][0].record(st)
        wl.step(i)
        ev[i][1].record(st)
    torch.cuda.synchronize()
    eager = sorted(e0.elapsed_time(e1) * 1e3 for e0, e1 in ev)

    total_ms = timed_graph(torch, wl.step, a.steps, warm)
    ms_per_step = total_ms / a.steps
    value = wl.wbytes * a.steps / (total_ms * 1e-3) / 1e9
    several = wl.o.get("topk") or wl.o.get("lmhead") or wl.o.get("moe")  # (steps of more than the one launch)
    kern_ms = timed_graph(torch, wl.kernel, a.steps, warm) if several else total_ms
    launch_us = kern_ms * 1e3 / a.steps
    kbytes = wl.kbytes or wl.wbytes
    achieved = kbytes / (launch_us * 1e-6) / 1e9

    cpu = None if a.no_cpu else cpu_baseline(wl, a.cpu_seconds)
    # the MFMA configs (more than 2 rows): the matrix cores' rate over the launch (rows padded to the 16- or 32-row
    # MFMA tile), live, and the counter figures of profiles/mfma_l2.md
    mfma = None
    if wl.m > 2 and not wl.o.get("moe") and not wl.o.get("int4"):
        mpad = 16 if wl.m <= 16 else 32
        nsum = wl.spec[0][0] * 2 if wl.o.get("glu2") else sum(n for n, _, _ in wl.spec)
        tflops = 2 * mpad * wl.k * nsum / (launch_us * 1e-6) / 1e12
        mfma = {"rows_in_tiles": mpad, "tflops": round(tflops, 2), "peak_tflops": MFMA_PEAK_TFLOPS,
                "frac": round(tflops / MFMA_PEAK_TFLOPS, 4), **(mfma_row(a.config) or {})}
    fmts = sorted({f for _, f, _ in wl.spec})
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": eager_warm + warm * a.steps,
        "ms_per_step": round(ms_per_step, 5),
        "us_per_call": round(ms_per_step * 1e3, 3),
        "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "+".join(fmts) + " weights x bf16 -> f32 accumulate",
        "data": "synthetic (seeded N(0,0.02) weights, N(0,1) x, U(0.5,1.5) scales)",
        "config": {
            "workload": wl.desc,
            "name": a.config,
            "m": wl.m,
            "k": wl.k,
            "n": [n for n, _, _ in wl.spec],
            "weight_bytes_per_call": wl.wbytes,
            "weight_copies_rotated": wl.copies,
            **({"experts": wl.moe_shape[0], "top_k": wl.moe_shape[1], "hidden": wl.moe_shape[2],
                "intermediate": wl.moe_shape[3], "pack": "kblock" if wl.kblock else "bfloat4_b",
                **({"rows": wl.o["rows"], "union_experts": wl.kbytes // (wl.moe_shape[2] // 32 * (2 * wl.moe_shape[3] // 32) * 576),
                    "kernel": "gate_up_rows (the step's larger launch)"} if wl.o.get("rows") else
                   {"kernel": "route_gate_up (the routing and gate_up in one launch, the step's larger)"})}
               if wl.o.get("moe") else {}),
            "timing": "HIP graph of the timed steps, replayed; events on the replay stream",
        },
        "eager_us_per_call": {"median": round(eager[len(eager) // 2], 3), "min": round(eager[0], 3)} if eager else None,
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_row(a.config),
            "launch_us": round(launch_us, 3),
            "algorithmic_bytes": kbytes,
            "mfma": mfma,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def cpu_baseline(wl, seconds):
    """The oracle's restatement of the reference's float32 CPU check path on the config's shapes (the held weights
    copied from the GPU), with the config's epilogue in torch, timed on this host's cores for about `seconds`."""
    import torch

    from oracle import dense_oracle as O

    threads = os.cpu_count()
    torch.set_num_threads(threads)
    m, o = wl.m, wl.o
    xc = wl.x.reshape(m, -1).cpu()
    if o.get("moe"):  # the reference's host check of the layer (moe8.py:642-660), float32, the k experts of a step
        gu, dn, bias = wl.host_w
        E, k, H, I = wl.moe_shape
        xm = wl.x.reshape(-1, H).cpu().float()
        wr = torch.full((k,), 1.0 / k)

        def moe_token(xr):
            pre = torch.stack([xr @ gu[e] for e in range(k)]) + bias.to(torch.bfloat16).float()
            gc = pre[:, I:].clamp(max=7.0)
            h = gc * torch.sigmoid(1.702 * gc) * (pre[:, :I].clamp(-7.0, 7.0) + 1.0) * wr[:, None]
            return sum(h[e] @ dn[e] for e in range(k))

        R = o.get("rows")
        if R:  # (every row through k experts, the first k of the pack's: the same work a row as the rows' own k)
            return _time_cpu(wl, lambda: [moe_token(xm[r]) for r in range(R)], seconds, threads,
                             f"a float32 port of the reference's layer check, {R} rows each through k experts "
                             "(gate_up, the clamped SwiGLU, the routing weights and down)")
        return _time_cpu(wl, lambda: moe_token(xm[0]), seconds, threads, "a float32 port of the reference's layer "
                         "check (the k experts' gate_up, the clamped SwiGLU, the routing weights and down)")
    if o.get("int4"):  # the reference's host check: x (bf16) @ (q * s).T in float32 (int4/w4a16.py:100-107)
        hw = [O.int4_dequantized(w.codes.cpu(), w.scales.cpu()).float().T.contiguous() for w in wl.sets[0]]
    else:
        hw = [wl.linear.held(w).cpu().contiguous() for w in wl.sets[0]]
    sc = [s.float().cpu().reshape(-1) if s is not None else None for s in wl.scales]
    rc = wl.res.reshape(m, -1).float().cpu() if wl.res is not None else None

    def step():
        if o.get("glu2"):
            return torch.nn.functional.silu(O.ref_f32(xc, hw[0], sc[0])) * O.ref_f32(xc, hw[1], sc[1])
        if o.get("blocks"):
            return torch.cat([O.ref_f32(xc, h, s) for h, s in zip(hw, sc)], dim=1)
        y = O.ref_f32(xc, hw[0], sc[0])
        if rc is not None:
            y = y + rc
        if o.get("topk") or o.get("lmhead"):
            t = y.reshape(m, -1, 32)
            torch.topk(t, 8, dim=2)
            torch.topk(y, 32 if o.get("topk") else 16, dim=1)
        return y

    return _time_cpu(wl, step, seconds, threads, "oracle.ref_f32 (x bf16->f32 @ held W f32; int4: W = q * s) plus the "
                     "epilogue")


def _time_cpu(wl, step, seconds, threads, what):
    """The median time of step() over about `seconds` (two untimed calls first), as the bench's cpu_baseline."""
    for _ in range(2):
        step()
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 5:
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return {
        "value": round(wl.wbytes / med / 1e9, 3),
        "unit": "GB/s",
        "us_per_call": round(med * 1e6, 1),
        "cores": threads,
        "kind": "port",
        "sample": f"{len(times)} calls (median) of {what}, the full config shapes, {threads} threads, ~{seconds:.0f} s",
    }


if __name__ == "__main__":
    main()
