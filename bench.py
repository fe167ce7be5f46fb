#!/usr/bin/env python3
"""Throughput of the fused token-selection pass on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c3]

A step is one gse_sample call (scan + exact kernels) over one batch of the selected workload with every input already
resident in HBM: logits, packed grammar masks, token histories, per-row parameters and shared uniforms. The inputs
rotate over enough copies to exceed the 256 MB Infinity Cache, so every step reads HBM. The JSON line reports
whole-job rows/s (wall clock over the K timed steps), the dominant kernel's roofline (algorithmic bytes per launch
divided by its average duration from HIP events recorded on the launch stream over the timed steps) and the CPU
oracle timed on this host (1 core) on a bounded sample of the same workload.
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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c3", choices=sorted(WORKLOADS))
    ap.add_argument("--copies", type=int, default=0, help="input copies to rotate over (0: enough to exceed the MALL)")
    ap.add_argument("--cpu-passes", type=int, default=2, help="passes of the CPU oracle over the sample rows")
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

    # timed region: K steps with per-kernel HIP events on the launch stream
    h.profile()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    ev0.record()
    for k in range(args.steps):
        step(k, profile=True)
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    calls, kms = h.profile()
    ev_ms = ev0.elapsed_time(ev1)
    ms_per_step = wall * 1e3 / args.steps
    value = rows * args.steps / wall
    scan_ms = kms[0] / calls
    exact_ms = kms[1] / calls
    log(f"[bench] {args.steps} steps: wall {wall * 1e3:.2f} ms, events {ev_ms:.2f} ms; per call scan {scan_ms * 1e3:.2f} us,"
        f" exact {exact_ms * 1e3:.2f} us")

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
        "roofline": {"bound": "hbm", "achieved": round(a_bytes / (scan_ms * 1e-3) / 1e9, 1), "peak": PEAK_HBM / 1e9,
                     "unit": "GB/s", "frac": round(a_bytes / (scan_ms * 1e-3) / PEAK_HBM, 4), "traffic": None,
                     "kernel": "scan_kernel", "kernel_us": round(scan_ms * 1e3, 3)},
        "end_to_end": {"step_us_wall": round(ms_per_step * 1e3, 3), "step_us_events": round(ev_ms * 1e3 / args.steps, 3),
                       "exact_kernel_us": round(exact_ms * 1e3, 3),
                       "hbm_frac": round(a_bytes / (ms_per_step * 1e-3) / PEAK_HBM, 4)},
    }

    if not args.no_cpu:
        from oracle import sampling_ref as ora
        masks = None if batch.masks is None else [ora.unpack_mask(m, vocab) for m in batch.masks]
        lf = batch.logits_f32()
        ora.sample(lf[:1], batch.params[:1], None, None, None if masks is None else masks[:1],
                   None if batch.history is None else batch.history[:1], batch.uniforms[:1])
        t = time.perf_counter()
        cpu_tokens = None
        for _ in range(args.cpu_passes):
            cpu_tokens = ora.sample(lf, batch.params, None, None, masks, batch.history, batch.uniforms)
        dt = time.perf_counter() - t
        result["cpu_baseline"] = {"value": round(rows * args.cpu_passes / dt, 2), "unit": "rows/s", "cores": 1,
                                  "kind": "port",
                                  "sample": f"the full {rows}-row batch of the same workload, {args.cpu_passes} passes "
                                            f"({dt:.1f} s, numpy oracle, {cpu_model()}, {os.cpu_count()} host cores)"}
        result["parity"] = {"rows": rows, "tokens_equal": gpu_tokens == cpu_tokens,
                            "mismatches": int(sum(a != b for a, b in zip(gpu_tokens, cpu_tokens)))}
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
