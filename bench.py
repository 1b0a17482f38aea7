#!/usr/bin/env python3
"""Benchmark of the decode-time sampler on one MI355X.

A step is one tgs_sample call over one B=64, V=128256 fp32 batch (the
headline configuration: penalties from a 512-id history, temperature,
top-k 50, top-p 0.9, one host uniform per row).  Inputs are resident in HBM before timing; 16
distinct logits buffers (525 MB) rotate so the 256 MB Infinity Cache cannot
serve repeats.  Launches are captured in a HIP graph (16 launches, one per
buffer) and replayed; the timed region is bracketed by synchronisations and
HIP events on the launch stream.

Prints one JSON line with the roofline of the sampling kernel and the CPU
oracle timed on this host.

`--calibrate-copy MIB` instead runs a plain device-to-device copy of MIB MiB
a few times: profiling it with the FETCH_SIZE / WRITE_SIZE counters gives the
scale between those counters and bytes actually moved, which converts the
sampling kernel's counter readings into HBM bytes per launch.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

METRIC = "sampled rows/sec @B=64,V=128256 full chain; HBM GB/s as % of peak"
HBM_PEAK_GBS = 8000.0
ROT = 16


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--eager", action="store_true", help="time eager launches instead of graph replay")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="run only a plain copy of MIB MiB (counter calibration)")
    return ap.parse_args()


def make_sets(n, B, V, H):
    from tinygpt_amd import workloads as W

    sets = []
    for i in range(n):
        sets.append(W.config2(B=B, V=V, H=H, seed_offset=i * 1000))
    return sets


def cpu_baseline(sets, seconds):
    """Oracle (C restatement of the reference sampler) on this host: rows/s
    with all host threads (up to 16) and with one thread."""
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "oracle"))
    import pyoracle

    pyoracle.build()
    nthr = max(1, min(16, os.cpu_count() or 1))

    def run(nthreads, budget):
        rows = 0
        t0 = time.perf_counter()
        i = 0
        ids = {}
        while time.perf_counter() - t0 < budget or rows == 0:
            s = sets[i % len(sets)]
            r = pyoracle.sample_batch(s["logits"], s["params"], s["u"], hist=s["hist"],
                                      hist_len=s["hist_len"], nthreads=nthreads)
            ids[i % len(sets)] = r["ids"]
            rows += s["logits"].shape[0]
            i += 1
        return rows / (time.perf_counter() - t0), rows, ids

    rate_n, rows_n, ids = run(nthr, seconds * 0.6)
    rate_1, rows_1, _ = run(1, seconds * 0.4)
    return dict(
        value=round(rate_n, 2), unit="rows/s", cores=nthr, kind="port",
        sample=f"{rows_n} C2 rows (B=64 batches cycling over {len(sets)} seeded sets) on {nthr} threads; "
               f"1 thread: {round(rate_1, 2)} rows/s over {rows_1} rows",
        single_thread_value=round(rate_1, 2),
    ), ids


def calibrate_copy(torch, mib, reps=8):
    """Plain copy of a known size, for scaling HBM byte counters."""
    n = mib << 20
    src = torch.empty(n // 4, dtype=torch.float32, device="cuda:0").fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(reps):
        dst.copy_(src)
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / reps
    print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "reps": reps,
                      "ms_per_copy": round(ms, 4), "GBps": round(2 * n / (ms * 1e-3) / 1e9, 1)}), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}): this build runs on a "
              "single GPU; the sampler is row-parallel and would shard by batch rows with "
              "no exchange between GPUs", file=sys.stderr)
        sys.exit(2)
    import torch

    if args.calibrate_copy:
        calibrate_copy(torch, args.calibrate_copy)
        return

    import tinygpt_amd as tg
    from tinygpt_amd import workloads as W

    dev = "cuda:0"
    B, V, H = 64, 128256, 512
    sets = make_sets(ROT, B, V, H)
    sampler = tg.Sampler(device=0, max_batch=B, max_vocab=V, max_hist=H)
    sampler.set_mask_table(np.zeros((0, 1), np.uint32), 1)
    d = []
    for s in sets:
        d.append(dict(
            logits=torch.from_numpy(s["logits"]).to(dev),
            params=tg.params_to_device(s["params"], dev),
            u=torch.from_numpy(s["u"]).to(dev),
            hist=torch.from_numpy(s["hist"]).to(dev),
            hist_len=torch.from_numpy(s["hist_len"]).to(dev),
            out=torch.empty(B, dtype=torch.int32, device=dev),
        ))
    torch.cuda.synchronize()

    stream = torch.cuda.Stream(device=dev)  # default priority

    hints = [tg.batch_hint(s["params"], V) for s in sets]

    def launch(i):
        x = d[i % ROT]
        sampler.sample(x["logits"], x["params"], x["u"], hist=x["hist"], hist_len=x["hist_len"],
                       out=x["out"], stream=stream.cuda_stream, hint=hints[i % ROT])

    with torch.cuda.stream(stream):
        for i in range(args.warmup):
            launch(i)
    torch.cuda.synchronize()

    graph = None
    if not args.eager:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream, capture_error_mode="thread_local"):
            for i in range(ROT):
                launch(i)
        torch.cuda.synchronize()
        for _ in range(3):
            graph.replay()
        torch.cuda.synchronize()

    reps = max(1, (args.steps + ROT - 1) // ROT)
    steps = reps * ROT if graph is not None else args.steps
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        ev0.record(stream)
        if graph is not None:
            for _ in range(reps):
                graph.replay()
        else:
            for i in range(steps):
                launch(i)
        ev1.record(stream)
    torch.cuda.synchronize()
    ms_total = ev0.elapsed_time(ev1)
    ms_per_step = ms_total / steps

    # parity of the timed outputs against the oracle (same inputs)
    gpu_ids = {i: d[i]["out"].cpu().numpy() for i in range(ROT)}
    cpu = None
    agreement = None
    if not args.no_cpu:
        cpu, cpu_ids = cpu_baseline(sets, args.cpu_seconds)
        match = [np.array_equal(gpu_ids[i], cpu_ids[i]) for i in cpu_ids]
        agreement = float(np.mean([np.mean(gpu_ids[i] == cpu_ids[i]) for i in cpu_ids]))
        if not all(match):
            print("WARNING: GPU ids differ from the oracle", file=sys.stderr)

    alg_bytes = W.algorithmic_bytes_per_row("c2", V, H) * B  # 4V + 4H per row
    achieved = alg_bytes / (ms_per_step * 1e-3) / 1e9
    rows_per_s = B / (ms_per_step * 1e-3)
    traffic = None
    tfile = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "k64_kernel_c2_traffic.json")
    if os.path.exists(tfile):
        try:
            traffic = json.load(open(tfile)).get("hbm_bytes_per_launch")
        except Exception:
            traffic = None
    line = {
        "metric": METRIC,
        "value": round(rows_per_s, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "c2_llama3_bpe", "B": B, "V": V, "history": H, "top_k": 50,
                   "top_p": 0.9, "temperature": 0.7, "presence": 0.5, "frequency": 0.3,
                   "rotating_buffers": ROT, "timing": "graph replay" if graph is not None else "eager"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "alg_bytes_per_launch": alg_bytes, "kernel": "k64_kernel<float>"},
        "cpu_baseline": cpu,
        "id_agreement": agreement,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
