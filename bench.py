"""Benchmark of the dense_reader decode matmul on one MI355X.

  python bench.py [--steps K] [--warmup W] [--config ns|c1|c2|c3|c4|c5] [--no-cpu]

Default workload: the north-star decode matmul, bfloat8_b M=1, x [1, 4096] bf16 @ W [4096 in, 14336 out] (W ~
N(0, 0.02)), no fused stage, bf16 output. A step is one call. Weights rotate over enough distinct copies (>= 512 MB)
that the 256 MB Infinity Cache cannot serve them; the K timed steps are captured once in a HIP graph and replayed
(the analogue of the reference's ttnn trace), bracketed by synchronisation; each launch's own duration is also measured
with HIP events around it on the stream it runs on (eager calls). One JSON line on stdout:

  value = algorithmic weight bytes (the reference's 1088 B per bfloat8_b 32x32 tile) x steps / timed seconds, GB/s;
  roofline.achieved = the same bytes per launch / the mean launch duration; cpu_baseline = the reference's torch CPU
  check path (x in bf16 times the held weight in float32, dense_reader/linear.py:166-169) on this host's cores.
"""

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "tensix-kernels_amd"))
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MALL_BYTES = 512 * 2**20

CONFIGS = {
    # name: (description, m, k, n, fmt, options)
    "ns": ("bfp8 M=1 K=4096 N=14336 decode matmul (north star)", 1, 4096, 14336, "bfp8", {}),
    "c1": ("bfp8 M=1 K=2048 N=4096, no fused stage", 1, 2048, 4096, "bfp8", {}),
    "c2": ("bfp4 M=1 K=4096 gate+up 2x14336, column scales, SwiGLU", 1, 4096, 14336, "bfp4", {"glu2": True, "scales": True}),
    "c3": ("bfp8 M=8 K=14336 N=4096, residual, fp32 out", 8, 14336, 4096, "bfp8", {"residual": True, "out32": True}),
    "c5": ("bfp8 M=4 K=4096 N=128256 LM head, top-8 per 32-column tile + global top-32", 4, 4096, 128256, "bfp8", {"topk": True}),
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="ns", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    return ap.parse_args()


def main():
    a = parse()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(
            "bench.py: this build measures one GPU; the decode matmul would shard its output columns over GPUs "
            "(see DESIGN.md) and no multi-GPU figure is produced",
            file=sys.stderr,
        )
        sys.exit(2)
    import torch

    from dense_reader import linear

    name = a.config
    desc, m, k, n, fmt, o = CONFIGS[name]
    dtype = {"bfp8": linear.bfloat8_b, "bfp4": linear.bfloat4_b, "bf16": linear.bfloat16}[fmt]
    dev = linear.dev.open_device(0)
    g = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(m, k, generator=g, device="cuda").to(torch.bfloat16).reshape(1, 1, m, k)
    nw = 2 if o.get("glu2") else 1

    def make():
        ws = [linear.native_weight(dev, torch.randn(n, k, generator=g, device="cuda") * 0.02, dtype)[0] for _ in range(nw)]
        return ws

    one = make()
    wbytes = sum(w.algorithmic_bytes() for w in one)
    copies = max(2, math.ceil(MALL_BYTES / sum(w.nbytes() for w in one)) + 1)
    sets = [one] + [make() for _ in range(copies - 1)]
    scales = None
    if o.get("scales"):
        scales = [linear.scale_tensor(dev, torch.rand(n, generator=g, device="cuda") + 0.5, dtype=linear.float32) for _ in range(nw)]
    res = torch.randn(m, n, generator=g, device="cuda").to(torch.bfloat16).reshape(1, 1, m, n) if o.get("residual") else None
    out32 = bool(o.get("out32"))
    n_out = n
    y = torch.empty(1, 1, m, n_out, dtype=torch.float32 if out32 else torch.bfloat16, device="cuda")
    rec = None
    if o.get("topk"):
        rec = linear.topk_result(dev, linear.topk_slots(n), m, 8)
        gv = torch.empty(m, 32, dtype=torch.float32, device="cuda")

    def call(i):
        ws = sets[i % copies]
        if o.get("glu2"):
            linear.matmul(x, ws[0], scales[0], out=y, glu=True, w_up=ws[1], scale_up=scales[1])
        elif o.get("topk"):
            spec = {"r": rec, "k": 8, "rows": m, "slot0": 0, "base": 0, "n": n, "write_y": False, "fp32": True}
            linear.matmul(x, ws[0], None, out=y, topk=spec)
            linear.topk_merge(rec, m, 8, k_out=32, fp32=True)
        elif res is not None:
            linear.matmul(x, ws[0], None, residual=res, out32=out32)  # (a residual takes a fresh output)
        else:
            linear.matmul(x, ws[0], None, out=y, out32=out32)

    for i in range(a.warmup):
        call(i)
    torch.cuda.synchronize()

    # each launch's own duration, eager, events on the launch stream
    st = torch.cuda.current_stream()
    nev = min(a.steps, 100)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(nev)]
    for i in range(nev):
        ev[i][0].record(st)
        call(i)
        ev[i][1].record(st)
    torch.cuda.synchronize()
    durs = sorted(e0.elapsed_time(e1) * 1e3 for e0, e1 in ev)  # us
    mean_us = sum(durs) / len(durs)
    med_us = durs[len(durs) // 2]

    # the timed region: K steps captured in one graph, replayed between synchronisations
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(a.steps):
            call(i)
    graph.replay()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record()
    graph.replay()
    t1.record()
    torch.cuda.synchronize()
    total_ms = t0.elapsed_time(t1)
    ms_per_step = total_ms / a.steps
    value = wbytes * a.steps / (total_ms * 1e-3) / 1e9
    achieved = wbytes / (mean_us * 1e-6) / 1e9

    cpu = None
    if not a.no_cpu:
        cpu = cpu_baseline(linear, x, one, scales, res, o, m, n, wbytes, a.cpu_seconds)

    line = {
        "metric": "weight GB/s and % HBM peak, bfp8_b M=1 decode matmul; us/call",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "us_per_call": round(ms_per_step * 1e3, 3),
        "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": fmt,
        "data": "synthetic (seeded N(0,0.02) weights, N(0,1) x)",
        "config": {
            "workload": desc,
            "m": m,
            "k": k,
            "n": n,
            "format": fmt,
            "weight_bytes_per_call": wbytes,
            "weight_copies_rotated": copies,
            "timing": "HIP graph of the timed steps, replayed",
        },
        "launch_us": {"mean": round(mean_us, 3), "median": round(med_us, 3), "min": round(durs[0], 3)},
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def cpu_baseline(linear, x, ws, scales, res, o, m, n, wbytes, seconds):
    """The reference's CPU check path on the same inputs: x (bf16) as float32 times the held weight(s) in float32, plus
    the config's epilogue, timed on this host's cores for about `seconds`."""
    import torch

    threads = os.cpu_count()
    torch.set_num_threads(threads)
    xc = x.reshape(m, -1).float().cpu()
    hw = [linear.held(w).cpu().contiguous() for w in ws]
    sc = [s.float().cpu().reshape(-1) for s in scales] if scales else None
    rc = res.reshape(m, -1).float().cpu() if res is not None else None

    def step():
        if o.get("glu2"):
            gt = (xc @ hw[0]) * sc[0]
            up = (xc @ hw[1]) * sc[1]
            return torch.nn.functional.silu(gt) * up
        y = xc @ hw[0]
        if rc is not None:
            y = y + rc
        if o.get("topk"):
            t = y.reshape(m, -1, 32)[:, : n // 32]
            torch.topk(t, 8, dim=2)
            torch.topk(y, 32, dim=1)
        return y

    for _ in range(3):
        step()
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 20:
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
        if len(times) >= 2000:
            break
    times.sort()
    med = times[len(times) // 2]
    return {
        "value": round(wbytes / med / 1e9, 3),
        "unit": "GB/s",
        "us_per_call": round(med * 1e6, 1),
        "cores": threads,
        "kind": "port",
        "sample": f"{len(times)} calls of torch float32 x @ held W on the CPU (median), the same shapes",
    }


if __name__ == "__main__":
    main()
