#!/usr/bin/env python3
"""Headline benchmark: batched token sampling on one MI355X.

Workload (configuration 5, the headline metric's shape): 128 rows x 248,320 bf16 logits,
near-flat N(0, 0.1), top_k off, top_p 0.95, repetition / presence / frequency
penalties over 32,768-token int32 histories, an independent Philox stream per row.
Five distinct input sets (~402 MB of logits) rotate across steps so the 256 MB
Infinity Cache cannot serve repeats.

One step is one decode step of all 128 lanes, one call (every row takes the
full-vocabulary route: the slice kernel, then the merge kernel):

* ``--route state`` (default): ``vi_sample_rows_state`` with record = 1.  Each
  lane's penalties come from its device penalty state (presence bitmap, count
  hash, repeat list), built from the lane's 32,768-token history before timing,
  as the histories themselves are; every step also records the sampled token in
  the state, so the lane's history grows by one token per step as in decoding.
* ``--route history``: ``vi_sample_rows`` over the int32 histories.

With the state route, the history route is also timed (``--compare-steps``) and
reported beside it.  Prints ONE JSON line: rows/s (whole job), achieved HBM GB/s
of the call (both kernels) against MI355X's 8 TB/s peak (per-call HIP events on
the launch stream), the oracle's CPU rate on the same inputs, and a GPU-vs-oracle
parity count for one step.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "sampled rows/sec + achieved HBM GB/s (% peak) at 128×248,320 bf16 logits"
PEAK_GBPS = 8000.0
ROWS, VOCAB, HISTORY, SETS = 128, 248_320, 32_768, 5
SLOTS = 65_536   # penalty-state hash slots per lane (>= 2 x distinct tokens)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--rows", type=int, default=ROWS)
    ap.add_argument("--route", choices=("state", "history"), default="state")
    ap.add_argument("--compare-steps", type=int, default=200,
                    help="steps of the history route timed beside the state route (0: none)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample length")
    ap.add_argument("--workload", choices=("config5", "config1", "config2", "config3", "config4", "config4-full",
                                           "wide"),
                    default="config5",
                    help="config5 (the headline); config1 / config2 report decode-step latency; config3 / config4 "
                         "time the top-k and verification kernels; wide times the fp32 full-vocabulary route")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run the copy kernel over 256 MiB x 10 (HBM-counter calibration) and exit")
    return ap.parse_args()


def calibrate_copy():
    """Known-traffic launches for scaling rocprofv3's FETCH_SIZE / WRITE_SIZE:
    5 x vi_probe_read over a 2 GiB buffer (2,147,483,648 bytes read per launch,
    8x the 256 MB Infinity Cache, evicted first by a 512 MiB fill) and
    5 x vi_probe_copy of 256 MiB (268,435,456 bytes written per launch)."""
    import torch

    import voidinfer_amd as vi
    from voidinfer_amd import ops
    dev = torch.device("cuda:0")
    assert vi.load().vi_init() == 0, "device is not gfx950"
    big = torch.ones(1 << 31, dtype=torch.uint8, device=dev)
    evict = torch.empty(1 << 29, dtype=torch.uint8, device=dev)
    evict.fill_(2)
    sink = torch.empty(2048, dtype=torch.int32, device=dev)
    for _ in range(5):
        ops.probe_read(big, sink)
    src, dst = big[: 1 << 28], evict[: 1 << 28]
    for _ in range(5):
        ops.probe_copy(dst, src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": {"vi_probe_read": {"bytes_read_per_launch": 1 << 31, "launches": 5},
                                      "vi_probe_copy": {"bytes_written_per_launch": 1 << 28, "launches": 5}}}))


def _timed(fn, stream, K: int, warmup: int):
    """HIP events around every launch on `stream`: (mean ms per step, per-launch ms)."""
    import numpy as np
    import torch
    for i in range(warmup):
        st = fn(i)
        assert st == 0, st
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(K)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(K)]
    for i in range(K):
        starts[i].record(stream)
        fn(i)
        ends[i].record(stream)
    torch.cuda.synchronize()
    return starts[0].elapsed_time(ends[-1]) / K, np.array([a.elapsed_time(b) for a, b in zip(starts, ends)])


def cpu_record(value: float, unit: str, cores: int, sample: str, flags: str) -> dict:
    import oracle
    return {"value": value, "unit": unit, "cores": cores, "kind": "port", "sample": sample,
            "cpu_model": oracle.cpu_model(), "build": flags}


def latency(args):
    """Configurations 1 and 2: one decode step of 1 lane (fp32, V=151,936) or 8
    lanes (bf16, V=248,320, mixed per-lane parameters, 4,096-token histories),
    launch-latency bound.  Per call: the GPU time (HIP events on the launch
    stream around each call, calls back to back) and the host round trip (call,
    then hipStreamSynchronize, wall clock), medians over the timed calls; for
    config 1 also the greedy call (vi_greedy_rows).  value = the sampled call's
    GPU-time median in microseconds (lower is better)."""
    import numpy as np
    import torch

    import voidinfer_amd as vi
    from voidinfer_amd import ops
    from voidinfer_amd import workloads as W
    dev = torch.device("cuda:0")
    lib = vi.load()
    assert lib.vi_init() == 0, "device is not gfx950"
    stream = torch.cuda.current_stream()
    sptr = stream.cuda_stream
    if args.workload == "config1":
        x, h, off, p = W.config1()
        host_logits, dtype, elem = x, vi.F32, 4
        logits = torch.from_numpy(x).to(dev)
        max_h = 256
        workload = ("config1: 1 lane x 151,936 fp32 N(0,2)+Zipf; greedy, then T .7 / top_k 20 / top_p .8 / "
                    "repetition 1.05 over a 256-token history")
        metric = "decode-step latency, 1 x 151,936 fp32 (sampled call; greedy call beside it)"
    else:
        bits, h, off, p = W.config2()
        host_logits, dtype, elem = bits, vi.BF16, 2
        logits = torch.from_numpy(bits.view(np.int16)).to(dev).view(torch.bfloat16)
        max_h = 4096
        workload = ("config2: 8 lanes x 248,320 bf16 N(0,2)+Zipf, mixed per-lane T / top_k {0,20,50} / top_p / "
                    "min_p and repetition / presence / frequency penalties over 4,096-token histories")
        metric = "decode-step latency, 8 lanes x 248,320 bf16, mixed per-lane parameters"
    rows, V = logits.shape
    hist = torch.from_numpy(h).to(dev)
    offs = torch.from_numpy(off).to(dev)
    pdev = vi.to_device_bytes(p, dev)
    routes = ops.route_mask(p)
    tokens = torch.empty(rows, dtype=torch.int32, device=dev)
    stats = torch.empty(rows * 32, dtype=torch.uint8, device=dev)
    nb = lib.vi_sample_workspace_bytes(rows, V, max_h)
    ws = torch.zeros(nb, dtype=torch.uint8, device=dev)
    grows = torch.empty(rows * 16, dtype=torch.uint8, device=dev)
    nbg = lib.vi_greedy_workspace_bytes(rows, V)
    wsg = torch.zeros(max(nbg, 1), dtype=torch.uint8, device=dev)

    def sample(i):
        return lib.vi_sample_rows(logits.data_ptr(), dtype, rows, V, V, pdev.data_ptr(), hist.data_ptr(),
                                  offs.data_ptr(), max_h, tokens.data_ptr(), None, None, V, stats.data_ptr(), routes,
                                  ws.data_ptr(), nb, sptr)

    def greedy(i):
        return lib.vi_greedy_rows(logits.data_ptr(), dtype, rows, V, V, i + 1, grows.data_ptr(), wsg.data_ptr(), nbg,
                                  sptr)

    K = min(args.steps, 500)

    def measure(fn):
        _, gpu_ms = _timed(fn, stream, K, args.warmup)
        host = []
        for i in range(K):
            t0 = time.perf_counter()
            assert fn(i) == 0
            stream.synchronize()
            host.append((time.perf_counter() - t0) * 1e6)
        us = gpu_ms * 1e3
        return {"gpu_us_p50": float(np.median(us)), "gpu_us_p10": float(np.percentile(us, 10)),
                "gpu_us_p90": float(np.percentile(us, 90)), "host_round_trip_us_p50": float(np.median(host)),
                "calls": K}
    assert sample(0) == 0
    torch.cuda.synchronize()
    gpu_tok = tokens.cpu().numpy().copy()
    s_lat = measure(sample)
    g_lat = measure(greedy) if args.workload == "config1" else None
    bytes_per_call = rows * V * elem + int(off[-1]) * 4
    kernel_s = s_lat["gpu_us_p50"] / 1e6
    achieved = bytes_per_call / kernel_s / 1e9
    cpu = parity = None
    if not args.no_cpu:
        import oracle
        flags = oracle.use_native()
        threads = min(rows, args.cpu_threads or len(os.sched_getaffinity(0)))
        w_tok, _, _, _, margins = oracle.sample_rows(host_logits, dtype, p, h, off, threads=threads)
        t0 = time.perf_counter()
        reps = 0
        while time.perf_counter() - t0 < args.cpu_seconds and reps < 100000:
            oracle.sample_rows(host_logits, dtype, p, h, off, threads=threads)
            reps += 1
        cpu_s = time.perf_counter() - t0
        mism = [r for r in range(rows) if w_tok[r] != gpu_tok[r]]
        parity = {"rows": rows, "mismatches": len(mism),
                  "unexplained": len([r for r in mism if not (margins[r, 0] < 1e-6 or margins[r, 1] < 1e-6)])}
        cpu = cpu_record(cpu_s / reps * 1e6, "us per call", threads,
                         f"{reps} calls of the same step through the oracle ({threads} thread(s)), {cpu_s:.1f} s", flags)
    print(json.dumps({
        "metric": metric, "value": s_lat["gpu_us_p50"], "unit": "us", "n_gpus": 1, "steps": K,
        "warmup": args.warmup, "ms_per_step": s_lat["gpu_us_p50"] / 1e3, "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp32" if dtype == vi.F32 else "bf16", "data": "synthetic",
        "config": {"workload": workload, "rows": int(rows), "vocabulary": int(V), "history": max_h,
                   "routes": int(routes), "kernel": "vi_sample_rows (topk.hip / sample_slices.hip routes)"},
        "latency": {"sampled": s_lat, "greedy": g_lat},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / PEAK_GBPS, "traffic": None, "bytes_per_launch": bytes_per_call,
                     "kernel_ms": s_lat["gpu_us_p50"] / 1e3,
                     "note": "latency-bound: one call reads a few hundred KB to 4 MB; frac is not the target"},
        "cpu_baseline": cpu, "parity": parity}))


def secondary(args):
    """Configuration 3 (DFlash2 draft top-8 + log-probs over 128 fp16 rows) or 4
    (verification of 8 lanes x 16 drafted positions: sampled rejection with the
    target softmax fused, and greedy prefix) on five rotating input sets; one JSON
    line in the headline's schema.  Not the headline metric."""
    import numpy as np
    import torch

    import voidinfer_amd as vi
    from voidinfer_amd import workloads as W
    dev = torch.device("cuda:0")
    lib = vi.load()
    assert lib.vi_init() == 0, "device is not gfx950"
    stream = torch.cuda.current_stream()
    sptr = stream.cuda_stream
    K, V = args.steps, VOCAB
    t16 = lambda bits, dt: torch.from_numpy(bits.view(np.int16)).to(dev).view(dt)   # noqa: E731
    extra = {}
    if args.workload == "wide":
        # the full-vocabulary route on fp32 logits (sample_wide.hip): 128 rows x
        # 248,320 fp32 N(0,2)+Zipf, T .7 / top_k off / top_p .95, no penalties
        rows = 128
        sets_w = []
        for s in range(SETS):
            bits_w = W.encode(W.gaussian_zipf(rows, V, 2.0, 700 + s), "f32")
            p_w = W.lane_params(rows, 7000 + s, top_k_choices=(0,), top_p_choices=(0.95,), min_p_choices=(0.0,))
            p_w["temperature"] = 0.7
            p_w["repetition_penalty"] = 1.0
            p_w["presence_penalty"] = 0.0
            p_w["frequency_penalty"] = 0.0
            sets_w.append((bits_w, p_w))
        logits = [torch.from_numpy(b.view(np.float32)).to(dev) for b, _ in sets_w]
        pdev = [vi.to_device_bytes(p_, dev) for _, p_ in sets_w]
        tok = torch.empty(rows, dtype=torch.int32, device=dev)
        nb = lib.vi_sample_workspace_bytes(rows, V, 0)
        ws = torch.zeros(nb, dtype=torch.uint8, device=dev)

        def fn(i):
            j = i % SETS
            return lib.vi_sample_rows(logits[j].data_ptr(), vi.F32, rows, V, V, pdev[j].data_ptr(), None, None, 0,
                                      tok.data_ptr(), None, None, V, None, vi.ROUTE_FULL, ws.data_ptr(), nb, sptr)
        bytes_per_launch = rows * V * 4
        metric, kernel = "sampled rows/sec at 128x248,320 fp32 (full-vocabulary route)", "wide_* (sample_wide.hip)"
        workload = "wide: 128 rows x 248,320 fp32 N(0,2)+Zipf, T .7 / top_k off / top_p .95, no penalties"
        assert fn(0) == 0
        torch.cuda.synchronize()
        gpu = tok.cpu().numpy()
    elif args.workload == "config3":
        rows, k = 128, 8
        bits = [W.config3(seed=300 + s, rows=rows) for s in range(SETS)]
        logits = [t16(b, torch.float16) for b in bits]
        ids = torch.empty(rows, k, dtype=torch.int64, device=dev)
        vals = torch.empty(rows, k, dtype=torch.float32, device=dev)
        lp = torch.empty(rows, k, dtype=torch.float32, device=dev)
        nb = lib.vi_topk_workspace_bytes(rows, V, k)
        ws = torch.zeros(nb, dtype=torch.uint8, device=dev)

        def fn(i):
            return lib.vi_topk_rows(logits[i % SETS].data_ptr(), vi.F16, rows, V, V, k, ids.data_ptr(),
                                    vals.data_ptr(), lp.data_ptr(), None, ws.data_ptr(), nb, sptr)
        bytes_per_launch = rows * V * 2 + rows * k * (8 + 4 + 4)
        metric, kernel = "draft top-8 + log-probs rows/sec at 128x248,320 fp16", "topk_kernel (topk.hip)"
        workload = "config3: 128 rows x 248,320 fp16 N(0,1.5) with 8 planted peaks +6..+10; exact top-8 ids + log-probs"
        assert fn(0) == 0
        torch.cuda.synchronize()
        gpu = ids.cpu().numpy()
    else:
        lanes, drafts = 8, 16
        rows = lanes * drafts
        full = args.workload == "config4-full"   # top_k off, top_p .8: the full-vocabulary path
        sets = []
        for s in range(SETS):
            t_, d_, x_, p_ = W.config4(seed=400 + s, lanes=lanes, drafts=drafts)
            if full:
                p_["top_k"] = 0
            sets.append((t_, d_, x_, p_))
        sampled = vi.VERIFY_SAMPLED if full else vi.VERIFY_SAMPLED_TOPK
        tgt = [t16(t, torch.bfloat16) for t, _, _, _ in sets]
        dft = [t16(d, torch.float16) for _, d, _, _ in sets]
        drafted = [torch.from_numpy(np.ascontiguousarray(x, dtype=np.int32)).to(dev) for _, _, x, _ in sets]
        params = [vi.to_device_bytes(p, dev) for _, _, _, p in sets]
        acc = torch.empty(lanes, dtype=torch.int32, device=dev)
        com = torch.empty(lanes, drafts + 1, dtype=torch.int32, device=dev)
        cnt = torch.empty(lanes, dtype=torch.int32, device=dev)
        flg = torch.empty(lanes, dtype=torch.int32, device=dev)
        nb = lib.vi_verify_workspace_bytes(lanes, drafts, V)
        ws = torch.zeros(nb, dtype=torch.uint8, device=dev)

        def call(i, mode):
            j = i % SETS
            smp = mode != vi.VERIFY_GREEDY
            return lib.vi_verify_rows(mode, tgt[j].data_ptr(), vi.BF16, V, drafts,
                                      dft[j].data_ptr() if smp else None, vi.F16 if smp else 0, V if smp else 0,
                                      lanes, drafts, V, drafted[j].data_ptr(),
                                      params[j].data_ptr() if smp else None, None, 0,
                                      acc.data_ptr(), com.data_ptr(), cnt.data_ptr(), flg.data_ptr(), ws.data_ptr(),
                                      nb, sptr)

        def fn(i):
            return call(i, sampled)
        g_ms, g_launch = _timed(lambda i: call(i, vi.VERIFY_GREEDY), stream, max(K // 2, 50), 10)
        extra["greedy_mode"] = {"ms_per_step": g_ms, "kernel_ms": float(g_launch.mean()),
                                "bytes_per_launch": rows * V * 2,
                                "achieved_gbps": rows * V * 2 / (float(g_launch.mean()) / 1e3) / 1e9}
        bytes_per_launch = rows * V * 2 * 2
        metric, kernel = "verified drafted rows/sec (8 lanes x 16, sampled rejection)", "verify_* (verify.hip)"
        workload = ("config4: 8 lanes x 16 drafted positions, target bf16 = draft fp16 + N(0,0.5), V=248,320, "
                    + ("T .7 / top_p .8 / top_k off (full-vocabulary p and q)" if full else "T .7 / top_p .8 / top_k 20")
                    + "; sampled rejection with the target softmax fused")
        assert fn(0) == 0
        torch.cuda.synchronize()
        gpu = (acc.cpu().numpy().copy(), com.cpu().numpy().copy())
    ms, launch = _timed(fn, stream, K, args.warmup)
    kernel_ms = float(launch.mean())
    achieved = bytes_per_launch / (kernel_ms / 1e3) / 1e9
    cpu = parity = None
    if not args.no_cpu:
        import oracle
        flags = oracle.use_native()
        threads = args.cpu_threads or min(len(os.sched_getaffinity(0)), 64)
        t0 = time.perf_counter()
        reps = 0
        while True:
            if args.workload == "config3":
                w_ids = oracle.topk_rows(bits[0], oracle.F16, 8, threads=threads)[0]
            elif args.workload == "wide":
                w_tok, _, _, _, w_m = oracle.sample_rows(sets_w[0][0], oracle.F32, sets_w[0][1], threads=threads)
            else:
                t, d, x, p = sets[0]
                w = oracle.verify_rows(vi.VERIFY_SAMPLED, t, oracle.BF16, d, oracle.F16, 8, 16, x, p, threads=threads)
            reps += 1
            if time.perf_counter() - t0 >= args.cpu_seconds or reps >= 1000:
                break
        cpu_s = time.perf_counter() - t0
        if args.workload == "config3":
            parity = {"rows": rows, "mismatched_rows": int((w_ids != gpu).any(axis=1).sum())}
            cores = threads
        elif args.workload == "wide":
            mism = [r for r in range(rows) if int(w_tok[r]) != int(gpu[r])]
            parity = {"rows": rows, "mismatches": len(mism),
                      "unexplained": len([r for r in mism if not (w_m[r, 0] < 1e-6 or w_m[r, 1] < 1e-6)])}
            cores = threads
        else:
            near = w[4] < 1e-6
            parity = {"lanes": 8, "accepted_mismatches": int((w[0] != gpu[0]).sum()),
                      "committed_mismatches": int(sum((w[1][l] != gpu[1][l]).any() for l in range(8)
                                                      if not near[l].any()))}
            cores = threads
        cpu = cpu_record(rows * reps / cpu_s, "rows/s", cores,
                         f"{reps} steps of input set 0 through the oracle ({cores} thread(s)), {cpu_s:.1f} s", flags)
    print(json.dumps({
        "metric": metric, "value": rows / (ms / 1e3), "unit": "rows/s", "n_gpus": 1, "steps": K,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"config3": "fp16", "wide": "fp32"}.get(args.workload, "bf16+fp16"), "data": "synthetic",
        "config": {"workload": workload, "rows": rows, "vocabulary": V, "input_sets": SETS, "kernel": kernel},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / PEAK_GBPS, "traffic": None, "bytes_per_launch": bytes_per_launch,
                     "kernel_ms": kernel_ms, "kernel_ms_p50": float(np.median(launch))},
        **extra, "cpu_baseline": cpu, "parity": parity}))


def traffic_from_profiles(route: str) -> float | None:
    """HBM bytes per call of the full-vocabulary route (slice and merge kernels) on
    `route`, from the rocprofv3 FETCH_SIZE / WRITE_SIZE passes recorded in profiles/
    (None if absent)."""
    f = ROOT / "profiles" / f"full_route_config5_{route}_traffic.md"
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1].strip())
    return None


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus > 1 or world > 1:
        print(f"bench.py runs on one GPU only (asked for {max(args.gpus, world)}); rows are independent, "
              "so N GPUs would run N independent copies of this step.", file=sys.stderr)
        sys.exit(2)

    if args.calibrate_copy:
        calibrate_copy()
        return
    if args.workload in ("config1", "config2"):
        latency(args)
        return
    if args.workload != "config5":
        secondary(args)
        return

    import numpy as np
    import torch

    import voidinfer_amd as vi
    from voidinfer_amd import ops, workloads

    dev = torch.device("cuda:0")
    assert vi.load().vi_init() == 0, "device is not gfx950"
    rows = args.rows
    print(f"[bench] generating {SETS} input sets of {rows}x{VOCAB} bf16 + {HISTORY}-token histories",
          file=sys.stderr, flush=True)
    sets = []
    for s in range(SETS):
        g = torch.Generator(device=dev)
        g.manual_seed(1000 + s)
        logits = (torch.randn(rows, VOCAB, generator=g, device=dev) * 0.1).to(torch.bfloat16)
        hist = torch.randint(0, VOCAB, (rows * HISTORY,), generator=g, device=dev, dtype=torch.int32)
        offs = torch.arange(rows + 1, device=dev, dtype=torch.int64) * HISTORY
        p = workloads.lane_params(rows, 5000 + s, top_k_choices=(0,), top_p_choices=(0.95,),
                                  min_p_choices=(0.0,))
        sets.append((logits, hist, offs, p, vi.to_device_bytes(p, dev)))
    routes = ops.route_mask(sets[0][3])
    assert routes == vi.ROUTE_FULL, routes

    lib = vi.load()
    tokens = torch.empty(rows, dtype=torch.int32, device=dev)
    stats = torch.empty(rows * 32, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()
    sptr = stream.cuda_stream
    nb_h = lib.vi_sample_workspace_bytes(rows, VOCAB, HISTORY)
    ws_h = torch.zeros(nb_h, dtype=torch.uint8, device=dev)
    hist_calls = [(lg.data_ptr(), 0, rows, VOCAB, VOCAB, pd.data_ptr(), h.data_ptr(), o.data_ptr(), HISTORY,
                   tokens.data_ptr(), None, None, VOCAB, stats.data_ptr(), routes, ws_h.data_ptr(), nb_h, sptr)
                  for lg, h, o, _, pd in sets]

    def hist_step(i):
        return lib.vi_sample_rows(*hist_calls[i % SETS])

    state_info = None
    if args.route == "state":
        print("[bench] building the lanes' penalty states from the histories", file=sys.stderr, flush=True)
        states = []
        for _, h, o, _, _ in sets:
            st = vi.PenaltyState(rows, VOCAB, SLOTS, device=dev)
            st.update(h, o)
            states.append(st)
        hdr = states[0].header()
        assert (hdr[:, 0] == 0).all() and (hdr[:, 2] == HISTORY).all(), hdr[:4]
        nrep = int(np.frombuffer(states[0].buf.view(rows, states[0].lane_bytes)[:, 16:20].cpu().numpy().tobytes(),
                                 dtype=np.uint32).mean())
        nb_s = lib.vi_sample_workspace_bytes(rows, VOCAB, 0)
        ws_s = torch.zeros(nb_s, dtype=torch.uint8, device=dev)

        def state_args(i, record):
            lg, _, _, _, pd = sets[i % SETS]
            return (lg.data_ptr(), 0, rows, VOCAB, VOCAB, pd.data_ptr(), states[i % SETS].buf.data_ptr(), SLOTS,
                    record, tokens.data_ptr(), None, None, VOCAB, stats.data_ptr(), routes, ws_s.data_ptr(), nb_s,
                    sptr)
        state_calls = [state_args(i, 1) for i in range(SETS)]

        def step(i):
            return lib.vi_sample_rows_state(*state_calls[i % SETS])
        # bytes per launch: the logits, the presence bitmap and the repeat list (8 B per entry)
        bytes_per_row = VOCAB * 2 + (VOCAB + 31) // 32 * 4 + 8 * nrep
        state_info = {"slots": SLOTS, "lane_bytes": states[0].lane_bytes, "repeat_list_mean": nrep,
                      "record": "each step records its sampled tokens in the lanes' states (same launch)"}
        # parity input: set 0's states before anything is recorded
        assert lib.vi_sample_rows_state(*state_args(0, 0)) == 0
    else:
        step = hist_step
        bytes_per_row = VOCAB * 2 + HISTORY * 4
        assert hist_step(0) == 0
    torch.cuda.synchronize()
    gpu_tok = tokens.cpu().numpy().copy()

    def timed(fn, K, warmup):
        """K steps back to back, HIP events on the launch stream at both ends of
        the timed region only (an event between steps would add its own packet
        to every step): per-step GPU time and host wall time."""
        for i in range(warmup):
            st = fn(i)
            assert st == 0, st
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        start.record(stream)
        for i in range(K):
            fn(i)
        end.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        return start.elapsed_time(end) / K, wall

    K = args.steps
    print(f"[bench] timing {K} steps ({args.route} route)", file=sys.stderr, flush=True)
    ms_per_step, wall = timed(step, K, args.warmup)
    rows_per_s = rows / (ms_per_step / 1e3)
    # the steps run back to back on one stream, so the GPU time per step is the
    # call's kernel time (its two launches and the gap between them)
    kernel_ms = ms_per_step
    bytes_per_launch = rows * bytes_per_row
    achieved = bytes_per_launch / (kernel_ms / 1e3) / 1e9
    history_route = None
    if args.route == "state" and args.compare_steps > 0:
        print(f"[bench] timing {args.compare_steps} steps of the history route", file=sys.stderr, flush=True)
        h_ms, _ = timed(hist_step, args.compare_steps, 20)
        history_route = {"ms_per_step": h_ms, "rows_per_s": rows / (h_ms / 1e3),
                         "kernel_ms": h_ms,
                         "bytes_per_launch": rows * (VOCAB * 2 + HISTORY * 4), "steps": args.compare_steps}

    # stream-read probe (measured HBM read rate) over a 1 GiB buffer
    probe = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    probe.fill_(1)
    sink = torch.empty(2048, dtype=torch.int32, device=dev)
    for _ in range(3):
        ops.probe_read(probe, sink)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(10):
        ops.probe_read(probe, sink)
    e1.record(stream)
    torch.cuda.synchronize()
    probe_gbps = (1 << 30) * 10 / (e0.elapsed_time(e1) / 1e3) / 1e9
    del probe

    # parity of the first step (set 0, before any recording) against the CPU
    # oracle, and the CPU baseline on the same inputs
    logits0, hist0, offs0, p0, p0_dev = sets[0]
    cpu = None
    parity = None
    if not args.no_cpu:
        import oracle
        bits = logits0.view(torch.int16).cpu().numpy().view(np.uint16)
        h = hist0.cpu().numpy()
        o = offs0.cpu().numpy()
        threads = args.cpu_threads or min(len(os.sched_getaffinity(0)), 64)
        flags = oracle.use_native()
        t = time.perf_counter()
        w_tok, _, _, _, margins = oracle.sample_rows(bits, oracle.BF16, p0, h, o, threads=threads)
        reps = 1
        while time.perf_counter() - t < args.cpu_seconds and reps < 1000:
            oracle.sample_rows(bits, oracle.BF16, p0, h, o, threads=threads)
            reps += 1
        cpu_s = time.perf_counter() - t
        mism = [r for r in range(rows) if w_tok[r] != gpu_tok[r]]
        unexplained = [r for r in mism if not (margins[r, 0] < 1e-6 or margins[r, 1] < 1e-6)]
        parity = {"rows": rows, "mismatches": len(mism), "unexplained": len(unexplained)}
        cpu = cpu_record(rows * reps / cpu_s, "rows/s", threads,
                         f"{reps} full steps of the workload ({rows} rows x {VOCAB} bf16, {HISTORY}-token "
                         f"histories, input set 0) through the oracle (C++ restatement, {threads} threads), "
                         f"{cpu_s:.1f} s", flags)

    out = {
        "metric": METRIC,
        "value": rows_per_s,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "config5: 128 lanes x 248,320 bf16 logits N(0,0.1), top_k off, top_p 0.95, "
                               "rep/presence/frequency penalties over 32,768-token histories, Philox per row",
                   "rows": rows, "vocabulary": VOCAB, "history": HISTORY, "input_sets": SETS,
                   "route": args.route, "penalty_state": state_info,
                   "kernel": "stream_kernel<bf16> + merge_kernel<bf16> (voidinfer_amd/csrc/sample_stream.hip)"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / PEAK_GBPS, "traffic": traffic_from_profiles(args.route),
                     "bytes_per_launch": bytes_per_launch, "kernel_ms": kernel_ms,
                     "probe_read_gbps": probe_gbps, "frac_of_probe": achieved / probe_gbps},
        "history_route": history_route,
        "cpu_baseline": cpu,
        "parity": parity,
        "host_wall_s": wall,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
