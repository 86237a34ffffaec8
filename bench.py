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
             f32 softmax with libm expf, streaming top-k, top-p, WeightedIndex)
             on a bounded sample of the same rows: `value` on the host cores of
             the box's share (one row per thread), `single_thread` one row at a
             time, as the reference samples, both timed in this run

Exactly `--steps` launches are timed, as one hipGraph replay (or eagerly with
--no-graph), after `--warmup` untimed launches.
`--workload c3|c4|c5` times the other measured configurations the same way
(masked rows, a speculative verify block through xs_verify, a heterogeneous
256-row batch with held_row statistics); their lines carry no traffic figure.
The default (c2) is the headline line.  `--cpu-threads N` runs the CPU
baseline N rows at a time (its `cores`).
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


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def host_threads() -> int:
    """Host cores this process may use, capped at the 16 a one-GPU share holds."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def cpu_baseline(name: str, wl, seconds: float, threads: int) -> dict:
    """Time the oracle (libm expf, serial f32 sums: the reference's control-path
    arithmetic) on the workload's rows for about `seconds`, `threads` rows at a
    time: the mask for c3, the accept_drafts walks for c4, held_row for c5."""
    import numpy as np

    from oracle import oracle as o
    o.build()
    o.set_exp_mode(1)
    rows, V = wl.logits.shape
    mask = wl.mask if name in ("c3", "c3p1") else None
    done, reps = 0, 0
    t0 = time.perf_counter()
    while True:
        d = o.sample_rows(wl.logits, V, wl.temperature, wl.top_k, wl.top_p, wl.u, mask=mask,
                          sum_mode=o.SUM_SEQ_F32, nthreads=threads)
        if name == "c4":
            tok = d["token"]
            for q in range(wl.seqs):
                t = tok[q * wl.span:(q + 1) * wl.span]
                o.accept_drafts(list(wl.drafts[q]), 1 << 62, list(t), [False] * wl.span)
        if name == "c5":
            for r in range(rows):
                o.held_row(wl.logits[r], V)
        done += rows
        reps += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt = time.perf_counter() - t0
    o.set_exp_mode(0)
    del np
    extra = {"c3": " + allow-masks", "c3p1": " + allow-masks", "c4": " + the accept_drafts walks",
             "c5": " + held_row (serial)"}.get(name, "")
    return {"value": round(done / dt, 2), "unit": "rows/s", "cores": threads, "kind": "port",
            "sample": f"{reps} passes over the {rows} rows of {name.upper()} (V=248,320){extra}, "
                      f"{threads} thread{'s' if threads > 1 else ''} of {os.cpu_count()} "
                      f"({cpu_model()}), oracle control path with libm expf, {dt:.1f} s"}


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


def setup(name, nbuf, dev, torch, workloads, xsm, _lib, lib, k_max=None, call_k_max=0,
          tokens_only=False) -> dict:
    """Build one workload's inputs (resident in HBM, `nbuf` rotating copies)
    and its launch.  c2 is the headline configuration; c3-c5 are the other
    measured configurations of the path."""
    import ctypes as C
    import numpy as np

    log(f"generating the {name} workload")
    wl = {"c1": workloads.c1_single, "c1g": lambda: workloads.c1_single(greedy=True),
          "c2": workloads.c2_batch, "c2w": workloads.c2_batch, "c3": workloads.c3_masked,
          "c3p1": workloads.c3_masked,
          "c4": workloads.c4_verify, "c5": workloads.c5_heterogeneous}[name]()
    if name == "c3p1":  # C3 at top_p = 1: the serial denominator reaches the weights
        wl.top_p = np.ones_like(wl.top_p)
    if name == "c2w":  # C2 with top_k >= V: the whole-row (top-p-only) path
        wl.top_k = np.full_like(wl.top_k, 2**31 - 1)
    if name in ("c1", "c1g"):  # one 1 MB row: rotate enough copies to leave the Infinity Cache
        nbuf = max(nbuf, 300)
    rows, V = wl.logits.shape
    if k_max is None and name == "c2w":
        k_max = 2**31 - 1
    ctx = xsm.Context(max_rows=rows, vocab=V, **({} if k_max is None else {"k_max": k_max}))
    base = torch.as_tensor(wl.logits).to(dev)
    bufs = [base if i == 0 else base.clone() for i in range(nbuf)]
    params = xsm.params_tensor(wl.temperature, wl.top_k, wl.top_p, rows, dev)
    u = torch.as_tensor(wl.u).to(dev)
    i32 = dict(dtype=torch.int32, device=dev)
    row_bytes = ROW_BYTES
    if name == "c4":
        drafts = torch.as_tensor(wl.drafts).to(dev)
        outs = [xsm.Verdict(row_token=torch.empty(rows, **i32), row_status=torch.empty(rows, **i32),
                            accepted=torch.empty(wl.seqs, **i32),
                            committed=torch.empty((wl.seqs, wl.span), **i32),
                            n_committed=torch.empty(wl.seqs, **i32),
                            seq_status=torch.empty(wl.seqs, **i32)) for _ in range(nbuf)]
        argv = []
        for i in range(nbuf):
            a = _lib.VerifyArgs()
            a.logits = bufs[i].data_ptr()
            a.seqs, a.span, a.ld, a.width, a.enc = wl.seqs, wl.span, V, V, V
            a.k_max = call_k_max
            a.params, a.uniforms, a.drafts = params.data_ptr(), u.data_ptr(), drafts.data_ptr()
            a.row_token, a.row_status = outs[i].row_token.data_ptr(), outs[i].row_status.data_ptr()
            a.accepted, a.committed = outs[i].accepted.data_ptr(), outs[i].committed.data_ptr()
            a.n_committed, a.seq_status = outs[i].n_committed.data_ptr(), outs[i].seq_status.data_ptr()
            argv.append(a)
        call = lib.xs_verify
        token_of = lambda o: o.row_token
    else:
        outs = [xsm.Draws(token=torch.empty(rows, **i32), status=torch.empty(rows, **i32))
                for _ in range(nbuf)]
        extra = {}
        # a heterogeneous batch starts its costliest rows first (xs_sample's
        # row_order hint); the others run in their natural order
        order = xsm.cost_order(wl.temperature, wl.top_k) if name == "c5" else None
        if name in ("c3", "c3p1"):
            extra["mask"] = torch.as_tensor(wl.mask.view(np.int32)).to(dev)
            row_bytes += 4 * wl.mask.shape[1]
        # the outputs each configuration names: C1 the renormalised top-k
        # probabilities, C2 the top-20 (id, prob) per row, C3 at top_p 1 the
        # top-20 list with the softmax denominator
        if name in ("c1", "c2", "c3p1") and not tokens_only:
            for o in outs:
                o.cand_id = torch.empty((rows, 20), **i32)
                o.cand_w = torch.empty((rows, 20), dtype=torch.float32, device=dev)
                o.n_cand = torch.empty(rows, **i32)
        if name == "c3p1":
            for o in outs:
                o.soft_sum = torch.empty(rows, dtype=torch.float32, device=dev)
        if name == "c5":
            for o in outs:
                o.row_max = torch.empty(rows, dtype=torch.float32, device=dev)
                o.row_lse = torch.empty(rows, dtype=torch.float64, device=dev)
                o.top_id = torch.empty((rows, wl.n_top), **i32)
                o.top_logprob = torch.empty((rows, wl.n_top), dtype=torch.float32, device=dev)
        argv = []
        for i in range(nbuf):
            a = _lib.SampleArgs()
            a.logits = bufs[i].data_ptr()
            a.rows, a.ld, a.width, a.enc = rows, V, V, V
            a.k_max = call_k_max
            a.params, a.uniforms = params.data_ptr(), u.data_ptr()
            a.token, a.status = outs[i].token.data_ptr(), outs[i].status.data_ptr()
            if "mask" in extra:
                a.allowed = extra["mask"].data_ptr()
                a.allowed_words = a.allowed_ld = wl.mask.shape[1]
            if outs[i].cand_id is not None:
                a.cand_id, a.cand_w = outs[i].cand_id.data_ptr(), outs[i].cand_w.data_ptr()
                a.n_cand, a.cand_ld = outs[i].n_cand.data_ptr(), 20
            if outs[i].soft_sum is not None:
                a.soft_sum = outs[i].soft_sum.data_ptr()
            if outs[i].top_id is not None:
                a.row_max, a.row_lse = outs[i].row_max.data_ptr(), outs[i].row_lse.data_ptr()
                a.n_top, a.top_ld = wl.n_top, wl.n_top
                a.top_id, a.top_logprob = outs[i].top_id.data_ptr(), outs[i].top_logprob.data_ptr()
            if order is not None:
                a.row_order = order.ctypes.data
            argv.append(a)
        call = lib.xs_sample
        token_of = lambda o: o.token
    refs = [C.byref(a) for a in argv]
    h = ctx.h

    def step(i):
        rc = call(h, refs[i % nbuf])
        if rc:
            raise RuntimeError(f"launch failed: {rc}")

    status_of = (lambda o: o.row_status) if name == "c4" else (lambda o: o.status)
    S = dict(wl=wl, rows=rows, ctx=ctx, step=step, outs=outs, alg_bytes=rows * row_bytes,
             token_of=token_of, status_of=status_of, bufs=bufs, keep=(params, u, argv), nbuf=nbuf)
    if name == "c4":
        S["keep"] += (drafts,)
    elif name in ("c3", "c3p1"):
        S["keep"] += (extra["mask"],)
    elif name == "c5":
        S["keep"] += (order,)  # the launches read it on the host at each call
    return S


WORKLOAD_TEXT = {
    "c1": "C1 single-row decode: 1 row x V=248,320 fp32, T 1.0 / top_k 20 / top_p 0.95, "
          "outputs the token and the renormalised top-20 probabilities (latency per row; 300 "
          "rotating copies)",
    "c1g": "C1 single-row greedy decode: 1 row x V=248,320 fp32, T 0 (latency per row; "
           "300 rotating copies)",
    "c2": "C2 batched sampling: 64 rows x V=248,320 fp32, T 0.7 / top_k 20 / top_p 0.80, "
          "one uniform per row; outputs 64 token ids plus the top-20 (id, prob) per row",
    "c2w": "C2 rows with top_k >= V, the whole-row (top-p-only) path: 64 rows x V=248,320 fp32, "
           "T 0.7 / top_p 0.80, tokens only: the row sorted by (p desc, id asc) but for the ids "
           "at p < 1.75 * 2^-26, whose additions to the serial sums all round back",
    "c3": "C3 grammar-constrained sampling: 32 rows x V=248,320 fp32 + packed u32 allow-masks "
          "(1% / 10% / 50% dense, one one-hot), T 1.0 / top_k 20 / top_p 0.95",
    "c3p1": "C3 at top_p 1.0 with the top-20 candidate list and the softmax denominator: the "
            "controlled rows' serial f32 denominator (sample_kernel + serial_kernel)",
    "c4": "C4 speculative verify: 16 sequences x 16 positions x V=248,320 fp32, 15 drafts each, "
          "top_k 20 / top_p 0.95 / T 1.0, accept_drafts on the device",
    "c5": "C5 heterogeneous batch: 256 rows x V=248,320 fp32 Student-t(3)x2, per-row T/k/p, "
          "held_row max / logsumexp / top-20 log-probs; rows started costliest first (row_order)",
}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--nbuf", type=int, default=5, help="rotating input copies (>256 MiB total)")
    ap.add_argument("--no-graph", action="store_true", help="launch eagerly instead of a hipGraph")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="rows the CPU baseline samples at once (one per thread); 0 = the "
                         "host cores of this process's share (at most 16)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="BYTES")
    ap.add_argument("--workload", choices=["c1", "c1g", "c2", "c2w", "c3", "c3p1", "c4", "c5"], default="c2",
                    help="c2 (default) is the headline configuration; c1/c1g one row (latency)")
    ap.add_argument("--k-max", type=int, default=None,
                    help="the context's k_max (default: 127, or INT32_MAX for c2w); above 127 every "
                         "call also launches the whole-row kernels")
    ap.add_argument("--call-k-max", type=int, default=0,
                    help="the calls' own bound on min(top_k, enc) (xs_sample_args.k_max; 0 = the "
                         "context's): 127 or less leaves the whole-row kernels out")
    ap.add_argument("--tokens-only", action="store_true",
                    help="take only tokens and statuses from c1 / c2 (their configurations also "
                         "name the top-20 candidates), to price those outputs")
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

    dev = torch.device("cuda:0")
    lib = _lib.load()
    S = setup(args.workload, args.nbuf, dev, torch, workloads, xsm, _lib, lib, args.k_max, args.call_k_max,
              args.tokens_only)
    wl, rows, ctx, step, outs, alg_bytes = S["wl"], S["rows"], S["ctx"], S["step"], S["outs"], S["alg_bytes"]
    V = wl.logits.shape[1]

    stream = torch.cuda.current_stream(dev)
    ctx.bind_current_stream()
    log("warmup")
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    st = S["status_of"](outs[0]).cpu().numpy()
    if st.any():
        raise RuntimeError(f"row errors in the warm-up batch: {st}")

    # Exactly `steps` launches are timed: one hipGraph holding `steps` launches
    # (cycling the rotating copies), replayed once after an untimed replay.
    steps = max(1, args.steps)
    nbuf = S["nbuf"]
    use_graph = not args.no_graph
    graph = None
    if use_graph:
        try:
            g = torch.cuda.CUDAGraph()
            side = torch.cuda.Stream(dev)
            side.wait_stream(stream)
            with torch.cuda.stream(side):
                ctx.bind_current_stream()
                with torch.cuda.graph(g, stream=side):
                    ctx.bind_current_stream()
                    for i in range(steps):
                        step(i)
            ctx.bind_current_stream()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            graph = g
        except Exception as e:  # graph capture unavailable: fall back to eager launches
            log(f"graph capture failed ({e}); launching eagerly")
            graph = None
            stream = torch.cuda.current_stream(dev)
            ctx.bind_current_stream()
            torch.cuda.synchronize()

    log(f"timing {steps} steps ({'hipGraph' if graph is not None else 'eager'})")
    torch.cuda.synchronize()
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    cur = torch.cuda.current_stream(dev)
    # keep the GPU busy while the host enqueues the timed launches, so the
    # region between the two events holds the launches and nothing else
    torch.cuda._sleep(2_000_000)
    t_start.record(cur)
    if graph is not None:
        graph.replay()
    else:
        for i in range(steps):
            step(i)
    t_end.record(cur)
    torch.cuda.synchronize()
    ms_total = t_start.elapsed_time(t_end)
    ms_step = ms_total / steps
    rows_per_s = rows / (ms_step / 1e3)
    achieved = alg_bytes / (ms_step / 1e3) / 1e9
    log(f"{ms_step * 1e3:.2f} us/step, {rows_per_s / 1e6:.3f} M rows/s, {achieved:.0f} GB/s")

    # parity spot check: every rotating copy written so far drew the same tokens
    tok0 = S["token_of"](outs[0]).cpu().numpy()
    for o in outs[1:min(len(outs), max(steps, args.warmup))]:
        assert (S["token_of"](o).cpu().numpy() == tok0).all(), "rotating buffers disagree"

    headline = args.workload == "c2"
    config = {"workload": WORKLOAD_TEXT[args.workload], "rows": rows, "vocab": V}
    if args.k_max is not None:
        config["k_max"] = args.k_max
    if args.call_k_max:
        config["call_k_max"] = args.call_k_max
    if args.tokens_only:
        config["outputs"] = "token ids only (--tokens-only)"
    if headline:
        config.update({"temperature": 0.7, "top_k": 20, "top_p": 0.8})
        config.setdefault("outputs", "token ids + top-20 (id, prob) per row (cand_id, cand_w)")
    config.update({"launch": "hipGraph" if graph is not None else "eager",
                   "rotating_buffers": nbuf, "buffer_bytes_total": nbuf * alg_bytes})
    result = {
        "metric": ("sampled rows/sec at V=248,320 batch 64 (1 GPU); achieved HBM GB/s vs peak"
                   if headline else f"sampled rows/sec at V=248,320, {args.workload.upper()} (1 GPU)"),
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
        "data": ("synthetic (seeded numpy PCG64: N(0,2.5^2) + 8 spikes U(8,14) per row)"
                 if headline else "synthetic (seeded numpy PCG64, tests/workloads.py)"),
        "config": config,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic() if headline else None},
    }
    if not args.no_cpu_baseline:
        # all host cores of the box's share (one row per thread), and one thread
        # (rows one after another, as the reference samples), in the same run
        threads = args.cpu_threads or host_threads()
        log(f"CPU baseline (~{args.cpu_seconds:.0f} s on {threads} threads, then 1 thread)")
        cb = cpu_baseline(args.workload, wl, args.cpu_seconds, threads)
        if threads > 1:
            one = cpu_baseline(args.workload, wl, args.cpu_seconds, 1)
            cb["single_thread"] = {"value": one["value"], "unit": one["unit"], "cores": 1,
                                   "sample": one["sample"]}
        result["cpu_baseline"] = cb
    else:
        result["cpu_baseline"] = None
    del S
    ctx.close()
    print(json.dumps(result), flush=True)
    del np
    return 0


if __name__ == "__main__":
    sys.exit(main())
