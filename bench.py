"""Benchmark: sampled rows/s at V = 248,320, batch 64, one MI355X.

One step = one xs_sample launch over the batch-64 configuration (64 rows x
248,320 f32 logits, N(0, 2.5^2) + 8 spikes U(8, 14) per row, T 0.7 / top_k 20 /
top_p 0.80, one uniform per row).  Inputs are resident in HBM before the timed
region; consecutive steps cycle through NBUF copies of the batch whose total
exceeds the 256 MiB Infinity Cache, so every step streams its rows from HBM.

Prints one JSON line (rank 0, N = 1):
  value      rows/s over the timed region (whole job, one GPU)
  roofline   algorithmic bytes per launch (64 x 993,280 B) / mean launch time,
             against MI355X's 8 TB/s HBM peak; `traffic` is the HBM bytes per
             launch that rocprofv3's FETCH_SIZE + WRITE_SIZE counters measured
             (profiles/sample_kernel_c2_traffic.md)
  cpu_baseline  the CPU oracle's restatement of the reference sampler (serial
             f32 softmax with libm expf, streaming top-k, top-p, WeightedIndex),
             one thread, on a bounded sample of the same rows
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
ROW_BYTES = 4 * 248_320


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_baseline(wl, seconds: float) -> dict:
    """Time the oracle (libm expf, serial f32 sums: the reference's control-path
    arithmetic) on the workload's rows, one thread, for about `seconds`."""
    import numpy as np

    from oracle import oracle as o
    o.build()
    o.set_exp_mode(1)
    rows = wl.logits.shape[0]
    done, reps = 0, 0
    t0 = time.perf_counter()
    while True:
        o.sample_rows(wl.logits, wl.logits.shape[1], wl.temperature, wl.top_k, wl.top_p, wl.u,
                      sum_mode=o.SUM_SEQ_F32, nthreads=1)
        done += rows
        reps += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt = time.perf_counter() - t0
    o.set_exp_mode(0)
    del np
    return {"value": round(done / dt, 2), "unit": "rows/s", "cores": 1, "kind": "port",
            "sample": f"{reps} passes over the {rows} batch rows (V=248,320), 1 thread, "
                      f"oracle control path with libm expf, {dt:.1f} s"}


def measured_traffic() -> int | None:
    """HBM bytes per sampler launch from the committed rocprofv3 FETCH_SIZE +
    WRITE_SIZE passes (scaled by a plain copy of known size), or None."""
    path = os.path.join(ROOT, "profiles", "sample_kernel_c2_traffic.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def calibrate_copy(nbytes: int, reps: int) -> None:
    """A plain device copy of known size, for scaling rocprof FETCH/WRITE_SIZE."""
    import torch
    a = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").uniform_()
    b = torch.empty_like(a)
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "copy", "bytes_read": nbytes, "bytes_written": nbytes,
                      "launches": reps}), flush=True)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--nbuf", type=int, default=5, help="rotating input copies (>256 MiB total)")
    ap.add_argument("--no-graph", action="store_true", help="launch eagerly instead of a hipGraph")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="BYTES")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested); rows shard across GPUs with no exchange, "
              f"so N GPUs would run N independent copies of this step.", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    if args.calibrate_copy:
        calibrate_copy(args.calibrate_copy, max(args.steps, 1))
        return 0

    from tests import workloads
    from xwen_amd import _lib
    from xwen_amd import sampler as xsm

    log("generating the batch-64 workload")
    wl = workloads.c2_batch()
    rows, V = wl.logits.shape
    dev = torch.device("cuda:0")
    ctx = xsm.Context(max_rows=rows, vocab=V)
    bufs = []
    base = torch.as_tensor(wl.logits).to(dev)
    for i in range(args.nbuf):
        bufs.append(base if i == 0 else base.clone())
    params = xsm.params_tensor(wl.temperature, wl.top_k, wl.top_p, rows, dev)
    u = torch.as_tensor(wl.u).to(dev)
    outs = [xsm.Draws(token=torch.empty(rows, dtype=torch.int32, device=dev),
                      status=torch.empty(rows, dtype=torch.int32, device=dev))
            for _ in range(args.nbuf)]
    lib = _lib.load()

    def make_args(i):
        a = _lib.SampleArgs()
        a.logits = bufs[i].data_ptr()
        a.rows, a.ld, a.width, a.enc = rows, V, V, V
        a.params = params.data_ptr()
        a.uniforms = u.data_ptr()
        a.token = outs[i].token.data_ptr()
        a.status = outs[i].status.data_ptr()
        return a

    argv = [make_args(i) for i in range(args.nbuf)]
    refs = [C.byref(a) for a in argv]
    h = ctx.h

    def step(i):
        rc = lib.xs_sample(h, refs[i % args.nbuf])
        if rc:
            raise RuntimeError(f"xs_sample failed: {rc}")

    stream = torch.cuda.current_stream(dev)
    ctx.bind_current_stream()
    log("warmup")
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    st = outs[0].status.cpu().numpy()
    if st.any():
        raise RuntimeError(f"row errors in the warm-up batch: {st}")

    use_graph = not args.no_graph
    graph = None
    per_graph = args.nbuf * 20
    if use_graph:
        try:
            g = torch.cuda.CUDAGraph()
            side = torch.cuda.Stream(dev)
            side.wait_stream(stream)
            with torch.cuda.stream(side):
                ctx.bind_current_stream()
                with torch.cuda.graph(g, stream=side):
                    ctx.bind_current_stream()
                    for i in range(per_graph):
                        step(i)
            ctx.bind_current_stream()
            torch.cuda.synchronize()
            for _ in range(3):
                g.replay()
            torch.cuda.synchronize()
            graph = g
        except Exception as e:  # graph capture unavailable: fall back to eager launches
            log(f"graph capture failed ({e}); launching eagerly")
            graph = None
            stream = torch.cuda.current_stream(dev)
            ctx.bind_current_stream()
            torch.cuda.synchronize()

    steps = args.steps
    if graph is not None:
        steps = max(per_graph, (steps + per_graph - 1) // per_graph * per_graph)
    log(f"timing {steps} steps ({'hipGraph' if graph is not None else 'eager'})")
    torch.cuda.synchronize()
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    cur = torch.cuda.current_stream(dev)
    t_start.record(cur)
    if graph is not None:
        for _ in range(steps // per_graph):
            graph.replay()
    else:
        for i in range(steps):
            step(i)
    t_end.record(cur)
    torch.cuda.synchronize()
    ms_total = t_start.elapsed_time(t_end)
    ms_step = ms_total / steps
    rows_per_s = rows / (ms_step / 1e3)
    alg_bytes = rows * ROW_BYTES
    achieved = alg_bytes / (ms_step / 1e3) / 1e9
    log(f"{ms_step * 1e3:.2f} us/step, {rows_per_s / 1e6:.3f} M rows/s, {achieved:.0f} GB/s")

    # parity spot check of the timed outputs against the first warm-up batch
    tok0 = outs[0].token.cpu().numpy()
    for o in outs[1:]:
        assert (o.token.cpu().numpy() == tok0).all(), "rotating buffers disagree"

    result = {
        "metric": "sampled rows/sec at V=248,320 batch 64 (1 GPU); achieved HBM GB/s vs peak",
        "value": round(rows_per_s, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded numpy PCG64: N(0,2.5^2) + 8 spikes U(8,14) per row)",
        "config": {"workload": "C2 batched sampling: 64 rows x V=248,320 fp32, T 0.7 / "
                               "top_k 20 / top_p 0.80, one uniform per row",
                   "rows": rows, "vocab": V, "temperature": 0.7, "top_k": 20, "top_p": 0.8,
                   "launch": "hipGraph" if graph is not None else "eager",
                   "rotating_buffers": args.nbuf,
                   "buffer_bytes_total": args.nbuf * alg_bytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic()},
    }
    if not args.no_cpu_baseline:
        log(f"CPU baseline (~{args.cpu_seconds:.0f} s)")
        result["cpu_baseline"] = cpu_baseline(wl, args.cpu_seconds)
    else:
        result["cpu_baseline"] = None
    ctx.close()
    print(json.dumps(result), flush=True)
    del np
    return 0


if __name__ == "__main__":
    sys.exit(main())
