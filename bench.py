#!/usr/bin/env python3
"""Throughput of the fused token-selection path on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c3|c1|c2|c4|c5|all] [--no-cpu] [--no-through-sample]

A step is one call of the selection path over one batch of the chosen workload, with every input already resident in
HBM (logits, packed grammar masks, token histories, per-row parameters, shared uniforms, draft trees):
  c1, c2, c3, c5  one gse_sample call (main pass, split-row finish of the deep rows, exact fallback) over B rows;
  c4              one gse_verify_tree call over 32 requests' draft trees (every node decided, the walk, on the device).
The inputs rotate over enough copies to exceed the 256 MB Infinity Cache, so every step reads HBM.

Timed regions, each bracketed by torch.cuda.synchronize():
  1. K plain steps: whole-job throughput from the wall clock -> "value" (rows/s; requests/s for c4);
  2. K steps with a HIP event on the launch stream between steps -> per-step median, P10 and P90;
  3. (c1, c2, c3, c5) K profiled steps: the library records HIP events around each of its kernels (gse_profile) -> the
     dominant kernel's average duration, which gives the roofline (algorithmic bytes per launch / duration). Those
     events add a few microseconds between kernels, which is why regions 1 and 2 carry none.
  4. the read-only ceiling: a plain streaming read (libgse_probe.so) over the same logits, best of a few launch shapes.
  5. (c1, c2, c3, c5) the drop-in's Python surface, sampling.sample() called as the engine calls it, each call returning
     its tokens: microseconds per call and the host time per call ("through_sample"; never "value").
The roofline's "traffic" (HBM bytes per launch of the main kernel) is read from the committed rocprofv3 counter
summary profiles/main_kernel_<config>_traffic.txt when one exists (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by a
plain copy's reading).

The CPU baseline is the numpy oracle on this host, on a bounded sample of the same workload, measured before the GPU is
touched: on one core (one BLAS/OpenMP thread, set before numpy is imported), and on every usable core (up to 16) with
rows split over processes.
"""
import os

for _v in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS", "MKL_NUM_THREADS"):  # (read when numpy is imported)
    os.environ[_v] = "1"

import argparse  # noqa: E402
import ctypes as C  # noqa: E402
import importlib  # noqa: E402
import json  # noqa: E402
import multiprocessing as mp  # noqa: E402
import platform  # noqa: E402
import sys  # noqa: E402
import time  # noqa: E402

import numpy as np  # noqa: E402

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "rows/sec & % HBM roofline, B=256 V=151936 fused penalties+top-k/p+mask"
PEAK_HBM = 8.0e12
MALL = 256 << 20
CPU_SECONDS = 10.0  # CPU work per baseline figure

WORKLOADS = {
    "c1": "CPU-sampler workload (B=8, V=32000, fp32, T 0.8, top-k 40, top-p 0.95, rep 1.1, H=64)",
    "c2": "grammar-masked greedy (B=64, V=128256, fp32, 4008-word masks)",
    "c3": "full penalty stack + top-k/top-p/min-p + grammar mask, heterogeneous rows (B=256, V=151936, fp32, H=2048)",
    "c4": "speculative tree verification (32 requests x 8-node draft trees, V=128256, fp32 target + drafter logits, "
          "rejection sampling)",
    "c5": "nucleus top-p 0.9 + top-20 logprobs (B=1024, V=262144, bf16)",
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


def usable_cores():
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


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


def pkg():
    return importlib.import_module("goethe-engine_amd")


# ---- CPU baseline (the numpy oracle) -----------------------------------------------------------------------------

def _c4_q(r):
    """The draft distributions of one request's nodes with kids: softmax(draft row) in fp64 (what the kids were drawn
    from)."""
    from oracle import spec_ref as spo
    q = {}
    for u, ks in enumerate(spo.kids_of(r["parents"])):
        if ks:
            z = r["draft"][u].astype(np.float64)
            e = np.exp(z - z.max())
            q[u] = e / e.sum()
    return q


class CpuWork:
    """The oracle's work on a subset of a workload's rows (requests for c4), with the inputs prepared beforehand."""

    def __init__(self, config, rows):
        ge = pkg()
        self.config = config
        if config == "c4":
            self.reqs = ge.workloads.c4(requests=rows)
            self.n = len(self.reqs)
            return
        b = getattr(ge.workloads, config)(rows=rows)
        from oracle import sampling_ref as ora
        self.ora = ora
        self.masks = None if b.masks is None else [ora.unpack_mask(m, b.vocab) for m in b.masks]
        self.x, self.params, self.hist, self.uni = b.logits_f32(), b.params, b.history, b.uniforms
        self.n = b.rows

    def run(self):
        if self.config == "c4":
            from oracle import spec_ref as spo
            return [spo.verify_tree(r["target"], _c4_q(r), r["tokens"], r["parents"], r["params"], r["seed"])
                    for r in self.reqs]
        return self.ora.sample(self.x, self.params, None, None, self.masks, self.hist, self.uni)


def _cpu_worker(config, rows, passes, barrier, q):
    try:
        w = CpuWork(config, rows)
        barrier.wait(timeout=600)
        t = time.perf_counter()
        for _ in range(passes):
            w.run()
        q.put((len(rows) * passes, time.perf_counter() - t))
    except Exception as e:  # noqa: BLE001 (reported by the parent)
        barrier.abort()
        q.put(e)


def cpu_baseline(config, total):
    """1-core and all-cores rows/s (requests/s for c4) of the oracle on bounded samples of the workload."""
    unit = "requests/s" if config == "c4" else "rows/s"
    one = CpuWork(config, range(1))
    t = time.perf_counter()
    one.run()
    per = max(time.perf_counter() - t, 1e-4)  # seconds per row, from one row
    n = max(1, min(total, int(CPU_SECONDS / per)))
    w = CpuWork(config, range(n))
    passes = max(1, min(10000, int(CPU_SECONDS / (n * per))))
    t = time.perf_counter()
    toks = None
    for _ in range(passes):
        toks = w.run()
    dt = time.perf_counter() - t
    what = f"the full {total}-row batch" if n == total else f"the first {n} of the {total} rows"
    if config == "c4":
        what = what.replace("row", "request")
    res = {"value": round(n * passes / dt, 2), "unit": unit, "cores": 1, "kind": "port",
           "sample": f"{what} of the same workload, {passes} pass(es) in {dt:.1f} s (numpy oracle, one process, "
                     f"OMP_NUM_THREADS=1, {cpu_model()}, {os.cpu_count()} host cores)"}
    # all usable cores: the rows split over processes, each with one thread
    k = usable_cores()
    if k > 1:
        rows_all = min(total, max(k, n * k))
        chunks = [r for r in np.array_split(np.arange(rows_all), k) if len(r)]
        p_all = max(1, min(10000, int(CPU_SECONDS / (len(chunks[0]) * per))))
        ctx = mp.get_context("spawn")
        barrier, q = ctx.Barrier(len(chunks)), ctx.Queue()
        procs = [ctx.Process(target=_cpu_worker, args=(config, [int(i) for i in c], p_all, barrier, q))
                 for c in chunks]
        for p in procs:
            p.start()
        out = []
        while len(out) < len(procs):
            try:
                out.append(q.get(timeout=5))
            except Exception:  # noqa: BLE001 (queue.Empty: check that no worker died without an answer)
                dead = [p.exitcode for p in procs if p.exitcode not in (None, 0)]
                if dead:
                    for p in procs:
                        p.kill()
                    raise RuntimeError(f"CPU baseline worker exited with {dead[0]}")
        for p in procs:
            p.join()
        errs = [o for o in out if isinstance(o, Exception)]
        if errs:
            raise errs[0]
        done, secs = sum(o[0] for o in out), max(o[1] for o in out)
        res["all_cores"] = {"value": round(done / secs, 2), "unit": unit, "cores": len(chunks),
                            "sample": f"{rows_all} {'requests' if config == 'c4' else 'rows'} split over "
                                      f"{len(chunks)} processes (one thread each), {p_all} pass(es), slowest "
                                      f"process {secs:.1f} s"}
    return res, w, toks


# ---- GPU -------------------------------------------------------------------------------------------------------------

def percentiles(ts):
    a = np.sort(np.asarray(ts))
    return {"median_us": round(float(np.median(a)), 3), "p10_us": round(float(np.percentile(a, 10)), 3),
            "p90_us": round(float(np.percentile(a, 90)), 3)}


def timed(step, steps, torch):
    """Region 1 (wall clock, no events between steps) and region 2 (an event between steps) -> (seconds, step times
    in microseconds)."""
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    for k in range(steps):
        step(k)
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    torch.cuda.synchronize()
    evs[0].record()
    for k in range(steps):
        step(k)
        evs[k + 1].record()
    torch.cuda.synchronize()
    return wall, [evs[k].elapsed_time(evs[k + 1]) * 1e3 for k in range(steps)]


def read_ceiling(bufs, torch):
    """Best GB/s of a plain read of one buffer (rotating over bufs) over a few launch shapes."""
    path = os.path.join(ROOT, "goethe-engine_amd", "libgse_probe.so")
    if not os.path.exists(path):
        return None
    L = C.CDLL(path)
    L.gse_probe_read.restype = C.c_int
    L.gse_probe_read.argtypes = [C.c_void_p, C.c_uint64, C.c_void_p, C.c_int, C.c_int, C.c_void_p]
    dev = bufs[0].device
    sink = torch.zeros(16384, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    nbytes = bufs[0].numel() * bufs[0].element_size() // 16 * 16
    best = None
    for grid in (1024, 2048, 4096, 8192):
        for unroll in (4, 8):
            def go(k):
                rc = L.gse_probe_read(bufs[k % len(bufs)].data_ptr(), nbytes, sink.data_ptr(), grid, unroll, stream)
                if rc:
                    raise RuntimeError(f"gse_probe_read failed ({rc})")
            for k in range(3):
                go(k)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record()
            for k in range(30):
                go(k)
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / 30
            gbs = nbytes / (us * 1e-6) / 1e9
            if best is None or gbs > best["read_GBps"]:
                best = {"read_GBps": round(gbs, 1), "us": round(us, 3), "bytes": nbytes, "grid": grid,
                        "unroll": unroll}
    return best


def run_sample(args, ge, torch, batch):
    lib = ge._lib
    dev = torch.device("cuda", 0)
    rows, vocab = batch.rows, batch.vocab
    copies = args.copies or max(2, -(-2 * MALL // (batch.logits.nbytes + 1)) + 1)
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
        sets.append(dict(b=b, o=o, toks=toks, x=xc, keep=(mk, hs, un, lp)))
    del x0, x
    torch.cuda.synchronize()
    log(f"[bench] {copies} input copies resident ({copies * batch.logits.nbytes / 2**20:.0f} MiB of logits)")

    base_flags = ge.sampling._sample_flags(batch.params)  # (what the drop-in adds: sample_ex)

    def step(k, profile=False):
        s = sets[k % copies]
        s["b"].flags = base_flags | (lib.BATCH_PROFILE if profile else 0)
        rc = h.L.gse_sample(h.h, C.byref(s["b"]), C.byref(s["o"]))
        if rc:
            h.ck(rc, "gse_sample")

    for k in range(args.warmup):
        step(k)
    torch.cuda.synchronize()
    step(0)  # (copy 0 last: the tokens and the finishing path of each of its rows)
    torch.cuda.synchronize()
    gpu_tokens = sets[0]["toks"].cpu().tolist()
    paths = np.bincount(h.row_paths(rows), minlength=3)
    log(f"[bench] rows finished by the main pass / split-row finish / exact path: {paths.tolist()}")
    wall, ts = timed(step, args.steps, torch)
    log(f"[bench] region 1: {args.steps} steps in {wall * 1e3:.2f} ms; region 2: median {np.median(ts):.2f} us")
    # region 3: per-kernel durations from HIP events on the launch stream
    h.profile()
    torch.cuda.synchronize()
    for k in range(args.steps):
        step(k, profile=True)
    torch.cuda.synchronize()
    calls, kms = h.profile()
    # (the profile's interval per kernel slot: main, split-row, exact; a call launches the split-row kernel, which
    # finishes every hard row itself, or, without it, the exact kernel)
    slot = {"main_kernel": 0, "deep_kernel": 1, "exact_kernel": 2}
    kern = ["main_kernel", "exact_kernel" if base_flags & lib.BATCH_NO_SPLIT else "deep_kernel"]
    per = {k: kms[slot[k]] / calls * 1e3 for k in kern}
    log("[bench] per call (profiled) " + ", ".join(f"{k} {v:.2f} us" for k, v in per.items()))
    ceil = read_ceiling([s["x"] for s in sets], torch)
    thr = through_sample(args, ge, torch, batch, [s["x"] for s in sets], gpu_tokens) if args.through_sample else None
    return dict(wall=wall, ts=ts, per=per, dom=("main_kernel", per["main_kernel"]), copies=copies,
                a_bytes=batch.bytes_per_row() * rows, units=rows, gpu_out=gpu_tokens, ceiling=ceil, through=thr,
                paths={"main": int(paths[0]), "split_row": int(paths[1]), "exact": int(paths[2])})


def through_sample(args, ge, torch, batch, xs, want):
    """The drop-in's Python surface timed as the engine calls it (engine.py:271-273: sample(logits, params, seeds,
    idxs, masks) -> list of ints, one host round trip per call), with the extensions' keywords: the step's SamplingParams
    objects, per-row seeds and idxs as Python lists, the uniforms as a device tensor, and
      resident: the grammar masks in a grammar.MaskBatch (packed words in one pinned buffer, one copy) and the penalty
                histories in a sampling.History (device-resident, read in place);
      lists:    per-row mask tensors (packed int32, the words xgrammar fills) and per-row history arrays, as a caller
                that keeps them per request passes them.
    Per variant: microseconds per sample() call (wall clock over K calls, each returning its tokens), and the host
    microseconds per call spent before the library call returns (sample_ex over K calls, no synchronisation)."""
    dev = xs[0].device
    rows, v = batch.rows, batch.vocab
    params = list(batch.params)
    seeds, idxs = list(range(1000, 1000 + rows)), [7] * rows
    uni = torch.from_numpy(batch.uniforms).to(dev)
    hist_res = mb = None
    if batch.history is not None:
        hist_res = ge.sampling.History(rows, max(len(h) for h in batch.history), dev)
        for r, hh in enumerate(batch.history):
            hist_res.set(r, hh)
    if batch.masks is not None:
        mb = ge.grammar.MaskBatch(rows, v)
        for r in range(rows):
            mb.set(r, batch.masks[r])
    variants = {"resident": (mb, hist_res),
                "lists": (None if batch.masks is None else [torch.from_numpy(m) for m in batch.masks],
                          batch.history)}
    out = {}
    steps = max(20, args.steps // 2)
    for name, (masks, hist) in variants.items():
        got = ge.sampling.sample(xs[0], params, seeds, idxs, masks, history=hist, uniforms=uni)
        if got != want:
            raise RuntimeError(f"through-sample ({name}) tokens differ from gse_sample's")
        for k in range(3):
            ge.sampling.sample(xs[k % len(xs)], params, seeds, idxs, masks, history=hist, uniforms=uni)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for k in range(steps):
            ge.sampling.sample(xs[k % len(xs)], params, seeds, idxs, masks, history=hist, uniforms=uni)
        wall = time.perf_counter() - t0
        host = 0.0
        torch.cuda.synchronize()
        for k in range(steps):
            t1 = time.perf_counter()
            ge.sampling.sample_ex(xs[k % len(xs)], params, seeds, idxs, masks, history=hist, uniforms=uni)
            host += time.perf_counter() - t1
            if k % 8 == 7:
                torch.cuda.synchronize()  # (the host keeps at most 8 calls ahead)
        torch.cuda.synchronize()
        out[name] = {"us_per_call": round(wall * 1e6 / steps, 2), "rows_per_s": round(rows * steps / wall, 1),
                     "host_us_per_call": round(host * 1e6 / steps, 2), "calls": steps}
        log(f"[bench] through sample() ({name}): {out[name]['us_per_call']} us per call, host "
            f"{out[name]['host_us_per_call']} us")
    return out


def run_verify(args, ge, torch):
    dev = torch.device("cuda", 0)
    reqs = ge.workloads.c4()
    v = reqs[0]["target"].shape[1]
    n_req = len(reqs)
    a_bytes = sum((r["target"].shape[0] + sum(1 for k in ge.spec.kids_of(list(r["parents"])) if k)) * v * 4
                  for r in reqs)
    per_copy = sum(r["target"].nbytes + r["draft"].nbytes for r in reqs)
    copies = args.copies or max(2, -(-2 * MALL // per_copy) + 1)
    calls = []
    for c in range(copies):
        tgt = torch.from_numpy(np.concatenate([r["target"] for r in reqs])).to(dev)
        drf = torch.from_numpy(np.stack([r["draft"] for r in reqs])).to(dev)
        off = 0
        creq = []
        for a, r in enumerate(reqs):
            n = r["target"].shape[0]
            creq.append(dict(target=tgt[off:off + n], tokens=r["tokens"], parents=r["parents"], params=r["params"],
                             seed=r["seed"], draft=drf[a], draft_t=1.0))
            off += n
        call = ge.spec.VerifyCall(creq)
        call.keep_inputs = (tgt, drf)
        calls.append(call)
    torch.cuda.synchronize()
    log(f"[bench] {copies} input copies resident ({copies * per_copy / 2**20:.0f} MiB of target + drafter logits)")

    def step(k):
        calls[k % copies].launch()

    for k in range(args.warmup):
        step(k)
    torch.cuda.synchronize()
    gpu_out = calls[0].result()
    wall, ts = timed(step, args.steps, torch)
    log(f"[bench] region 1: {args.steps} steps in {wall * 1e3:.2f} ms; region 2: median {np.median(ts):.2f} us")
    med = float(np.median(ts))
    ceil = read_ceiling([c.keep_inputs[0] for c in calls], torch)
    return dict(wall=wall, ts=ts, per={}, dom=("verify call (all its kernels, per-step median)", med), copies=copies,
                a_bytes=a_bytes, units=n_req, gpu_out=gpu_out, ceiling=ceil)


def bench_one(args, config):
    ge = pkg()
    t0 = time.perf_counter()
    batch = None if config == "c4" else getattr(ge.workloads, config)()
    log(f"[bench] {config}: inputs generated in {time.perf_counter() - t0:.1f}s")
    total = 32 if config == "c4" else batch.rows
    cpu = None
    if not args.no_cpu:  # before the GPU is touched (the all-cores figure starts processes)
        cpu, cpu_work, cpu_out = cpu_baseline(config, total)
        log(f"[bench] {config}: CPU baseline {cpu['value']} {cpu['unit']} (1 core)" +
            (f", {cpu['all_cores']['value']} ({cpu['all_cores']['cores']} cores)" if "all_cores" in cpu else ""))

    import torch
    if not torch.cuda.is_available():
        raise RuntimeError("bench.py needs a HIP device")
    torch.cuda.set_device(0)
    if args.calibrate_copy:
        dev = torch.device("cuda", 0)
        nb = args.calibrate_copy << 20
        src = torch.ones(nb // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] calibration: 5 device copies of {nb} bytes ({args.calibrate_copy} MiB)")
        del src, dst
        args.calibrate_copy = 0
    r = run_verify(args, ge, torch) if config == "c4" else run_sample(args, ge, torch, batch)
    steps = args.steps
    value = r["units"] * steps / r["wall"]
    dom_name, dom_us = r["dom"]
    a = r["a_bytes"]
    unit = "requests/s" if config == "c4" else "rows/s"
    cfg = {"workload": f"{config}: {WORKLOADS[config]}", "algorithmic_bytes_per_step": a, "input_copies": r["copies"]}
    if config == "c4":
        cfg.update(requests=32, vocab=128256, nodes_per_request=9)
    else:
        cfg.update(rows=batch.rows, vocab=batch.vocab, input_dtype="bf16" if batch.bf16 else "f32")
    result = {
        "metric": METRIC if config == "c3" else f"{unit.split('/')[0]}/sec & % HBM roofline, {config}",
        "value": round(value, 1),
        "unit": unit,
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["wall"] * 1e3 / steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded splitmix64 workload generator, goethe-engine_amd/workloads.py)",
        "config": cfg,
        "roofline": {"bound": "hbm", "achieved": round(a / (dom_us * 1e-6) / 1e9, 1), "peak": PEAK_HBM / 1e9,
                     "unit": "GB/s", "frac": round(a / (dom_us * 1e-6) / PEAK_HBM, 4),
                     "traffic": read_traffic(config) if config != "c4" else None,
                     "kernel": dom_name, "kernel_us": round(dom_us, 3)},
        "step_us": percentiles(r["ts"]),
        "kernels_us": {k: round(v, 3) for k, v in r["per"].items()},
        "end_to_end": {"step_us_wall": round(r["wall"] * 1e6 / steps, 3),
                       "hbm_frac": round(a / (r["wall"] / steps) / PEAK_HBM, 4)},
    }
    if r.get("paths"):
        result["row_paths"] = r["paths"]
    if r.get("through"):
        result["through_sample"] = r["through"]
    if r["ceiling"]:
        c = r["ceiling"]
        result["read_ceiling"] = dict(c, frac_of_peak=round(c["read_GBps"] * 1e9 / PEAK_HBM, 4),
                                      kernel_frac_of_ceiling=round(a / (dom_us * 1e-6) / 1e9 / c["read_GBps"], 4))
    if cpu is not None:
        result["cpu_baseline"] = cpu
        n = cpu_work.n
        if config == "c4":
            want = cpu_out
            got = r["gpu_out"][:n]
        else:
            want, got = cpu_out, r["gpu_out"][:n]
        result["parity"] = {"units": n, "equal": got == want,
                            "mismatches": int(sum(x != y for x, y in zip(got, want)))}
    print(json.dumps(result), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c3", choices=sorted(WORKLOADS) + ["all"])
    ap.add_argument("--copies", type=int, default=0, help="input copies to rotate over (0: enough to exceed the MALL)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-through-sample", dest="through_sample", action="store_false",
                    help="skip timing the drop-in's sample() surface (done for c1, c2, c3, c5 by default)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="before the steps, copy a MIB-MiB device buffer 5 times (a plain copy kernel of known size, "
                         "the reference point for rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py runs on one GPU only: --gpus {args.gpus} / WORLD_SIZE {world} is not supported "
              "(row-parallel sharding over several GPUs is designed, not built)", file=sys.stderr)
        sys.exit(2)
    for config in (["c1", "c2", "c3", "c4", "c5"] if args.config == "all" else [args.config]):
        bench_one(args, config)


if __name__ == "__main__":
    main()
