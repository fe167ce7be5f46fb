#!/usr/bin/env python3
"""Throughput of the fused token-selection pass on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c3]

A step is one gse_sample call (main pass, split-row finish of the deep rows, exact fallback) over one batch of the
selected workload with every input already resident in HBM: logits, packed grammar masks, token histories, per-row
parameters and shared uniforms. The inputs rotate over enough copies to exceed the 256 MB Infinity Cache, so every step
reads HBM.

Two timed regions of K steps each, both bracketed by torch.cuda.synchronize():
  1. plain steps: whole-job rows/s (wall clock) -> "value";
  2. profiled steps: the library records HIP events on the launch stream around each of its kernels (gse_profile);
     the dominant kernel's average duration gives the roofline (algorithmic bytes per launch / duration). The events
     add a few microseconds between kernels, which is why region 1 carries none.
The roofline's "traffic" (HBM bytes the kernel moves per launch) is read from the committed rocprofv3 counter summary
profiles/main_kernel_c3_traffic.txt when it exists (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by a plain copy's
reading). The CPU baseline is the numpy oracle timed on this host (1 core) on a bounded sample of the same workload.
"""
import argparse
import ctypes as C
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "rows/sec & % HBM roofline, B=256 V=151936 fused penalties+top-k/p+mask"
PEAK_HBM = 8.0e12
MALL = 256 << 20

WORKLOADS = {
    "c3": "full penalty stack + top-k/top-p/min-p + grammar mask, heterogeneous rows (B=256, V=151936, fp32, H=2048)",
    "c2": "grammar-masked greedy (B=64, V=128256, fp32, 4008-word masks)",
    "c5": "nucleus top-p 0.9 + top-20 logprobs (B=1024, V=262144, bf16)",
    "c1": "CPU-sampler workload (B=8, V=32000, fp32, T 0.8, top-k 40, top-p 0.95, rep 1.1, H=64)",
}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def cpu_model():
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def read_traffic(config):
    """HBM bytes per launch of the main kernel from the committed counter summary (a line "traffic_bytes: N"), or
    None when there is none for this workload."""
    path = os.path.join(ROOT, "profiles", f"main_kernel_{config}_traffic.txt")
    try:
        for ln in open(path):
            if ln.startswith("traffic_bytes:"):
                return int(ln.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c3", choices=sorted(WORKLOADS))
    ap.add_argument("--copies", type=int, default=0, help="input copies to rotate over (0: enough to exceed the MALL)")
    ap.add_argument("--cpu-passes", type=int, default=5, help="passes of the CPU oracle over the sample rows")
    ap.add_argument("--cpu-rows", type=int, default=0, help="rows of the CPU sample (0: the whole batch)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="before the steps, copy a MIB-MiB device buffer 5 times (a plain copy kernel of known size, "
                         "the reference point for rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py runs on one GPU only: --gpus {args.gpus} / WORLD_SIZE {world} is not supported "
              "(row-parallel sharding over several GPUs is designed, not built)", file=sys.stderr)
        sys.exit(2)

    import importlib

    import torch
    ge = importlib.import_module("goethe-engine_amd")
    lib = ge._lib
    if not torch.cuda.is_available():
        raise RuntimeError("bench.py needs a HIP device")
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)

    if args.calibrate_copy:
        n = args.calibrate_copy << 20
        src = torch.ones(n // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] calibration: 5 device copies of {n} bytes ({args.calibrate_copy} MiB)")
        del src, dst

    t0 = time.perf_counter()
    batch = getattr(ge.workloads, args.config)()
    log(f"[bench] generated {args.config}: {batch.rows} x {batch.vocab} in {time.perf_counter() - t0:.1f}s")
    rows, vocab = batch.rows, batch.vocab
    a_bytes = batch.bytes_per_row() * rows
    copies = args.copies or max(2, -(-2 * MALL // (batch.logits.nbytes + 1)) + 1)

    # resident inputs, one set per copy
    x0 = torch.from_numpy(batch.logits).to(dev)
    if batch.bf16:
        x0 = x0.view(torch.bfloat16)
    masks0 = None if batch.masks is None else [torch.from_numpy(m) for m in batch.masks]
    h, x, code, _, b0, keep0 = ge.sampling._prepare(x0, batch.params, None, None, masks0, batch.history,
                                                     batch.uniforms)
    nlp = max([p.logprobs or 0 for p in batch.params] + [0])
    sets = []
    for c in range(copies):
        xc = x0.clone()
        mk = keep0[2].clone() if keep0[2] is not None else None
        hs = keep0[3].clone() if keep0[3] is not None else None
        un = keep0[4].clone() if keep0[4] is not None else None
        b = ge.sampling._batch(xc, code, keep0[1], mk, b0.mask_ld, hs, un, dev)
        toks = torch.empty(rows, dtype=torch.int32, device=dev)
        o = lib.Out()
        o.size = C.sizeof(lib.Out)
        o.tokens = toks.data_ptr()
        lp = None
        if nlp:
            lp = (torch.empty((rows, nlp), dtype=torch.int32, device=dev),
                  torch.empty((rows, nlp), dtype=torch.float32, device=dev))
            o.logprob_ids, o.logprobs, o.logprobs_ld = lp[0].data_ptr(), lp[1].data_ptr(), nlp
        sets.append(dict(b=b, o=o, toks=toks, keep=(xc, mk, hs, un, lp)))
    torch.cuda.synchronize()
    log(f"[bench] {copies} input copies resident ({copies * batch.logits.nbytes / 2**20:.0f} MiB of logits)")

    def step(k, profile=False):
        s = sets[k % copies]
        s["b"].flags = lib.BATCH_PROFILE if profile else 0
        rc = h.L.gse_sample(h.h, C.byref(s["b"]), C.byref(s["o"]))
        if rc:
            h.ck(rc, "gse_sample")

    for k in range(args.warmup):
        step(k)
    torch.cuda.synchronize()
    gpu_tokens = sets[0]["toks"].cpu().tolist()

    # timed region 1: K plain steps -> whole-job throughput
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    ev0.record()
    for k in range(args.steps):
        step(k)
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    ev_ms = ev0.elapsed_time(ev1)
    # timed region 2: K profiled steps -> per-kernel durations from HIP events on the launch stream
    h.profile()
    torch.cuda.synchronize()
    for k in range(args.steps):
        step(k, profile=True)
    torch.cuda.synchronize()
    calls, kms = h.profile()
    kern = ["main_kernel", "deep_kernel", "exact_kernel"]
    per = {kern[i]: kms[i] / calls * 1e3 for i in range(min(len(kern), len(kms)))}
    ms_per_step = wall * 1e3 / args.steps
    value = rows * args.steps / wall
    main_us = per["main_kernel"]
    log(f"[bench] {args.steps} steps: wall {wall * 1e3:.2f} ms, events {ev_ms:.2f} ms; per call (profiled) " +
        ", ".join(f"{k} {v:.2f} us" for k, v in per.items()))
    traffic = read_traffic(args.config)

    result = {
        "metric": METRIC if args.config == "c3" else f"rows/sec, {args.config}",
        "value": round(value, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if batch.bf16 else "f32",
        "data": "synthetic (seeded splitmix64 workload generator, goethe-engine_amd/workloads.py)",
        "config": {"workload": f"{args.config}: {WORKLOADS[args.config]}", "rows": rows, "vocab": vocab,
                   "input_copies": copies, "algorithmic_bytes_per_step": a_bytes},
        "roofline": {"bound": "hbm", "achieved": round(a_bytes / (main_us * 1e-6) / 1e9, 1), "peak": PEAK_HBM / 1e9,
                     "unit": "GB/s", "frac": round(a_bytes / (main_us * 1e-6) / PEAK_HBM, 4), "traffic": traffic,
                     "kernel": "main_kernel", "kernel_us": round(main_us, 3)},
        "kernels_us": {k: round(v, 3) for k, v in per.items()},
        "end_to_end": {"step_us_wall": round(ms_per_step * 1e3, 3), "step_us_events": round(ev_ms * 1e3 / args.steps, 3),
                       "hbm_frac": round(a_bytes / (ms_per_step * 1e-3) / PEAK_HBM, 4)},
    }

    if not args.no_cpu:
        from oracle import sampling_ref as ora
        masks = None if batch.masks is None else [ora.unpack_mask(m, vocab) for m in batch.masks]
        lf = batch.logits_f32()
        n = min(rows, args.cpu_rows) if args.cpu_rows > 0 else rows
        sub = lambda v: None if v is None else v[:n]
        ora.sample(lf[:1], batch.params[:1], None, None, None if masks is None else masks[:1],
                   None if batch.history is None else batch.history[:1], batch.uniforms[:1])
        t = time.perf_counter()
        cpu_tokens = None
        for _ in range(args.cpu_passes):
            cpu_tokens = ora.sample(lf[:n], batch.params[:n], None, None, sub(masks), sub(batch.history),
                                    batch.uniforms[:n])
        dt = time.perf_counter() - t
        what = f"the full {rows}-row batch" if n == rows else f"the first {n} of the {rows} rows"
        result["cpu_baseline"] = {"value": round(n * args.cpu_passes / dt, 2), "unit": "rows/s", "cores": 1,
                                  "kind": "port",
                                  "sample": f"{what} of the same workload, {args.cpu_passes} pass(es) in {dt:.1f} s "
                                            f"(numpy oracle on one core, {cpu_model()}, {os.cpu_count()} host cores)"}
        result["parity"] = {"rows": n, "tokens_equal": gpu_tokens[:n] == cpu_tokens,
                            "mismatches": int(sum(a != b for a, b in zip(gpu_tokens[:n], cpu_tokens)))}
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
