#!/usr/bin/env python3
"""Headline benchmark of the MI355X HIP backend for zlm's quantized GEMV path.

A step is one pass of the configs[1] workload -- the Qwen3-8B FFN GEMVs in
Q8_0 at batch 1: gate 12288x4096, up 12288x4096, down 4096x12288 -- over
weights already resident in HBM and activations already on the device.  Every
step reads a different copy of the three weights (>= 512 MiB in rotation), so
the 256 MiB Infinity Cache cannot serve them and the rate is an HBM rate.

Timing: W warm-up steps, then untimed steps until at least 50 ms of GPU work
has run (the clocks ramp over the first milliseconds after the host-side weight
synthesis; a short warm-up alone read ~4.5% low), then exactly K steps between
two HIP events on the backend's stream (the stream every launch goes to).
`value` = algorithmic bytes of a step (weights + x + y) / (elapsed / K).  The
roofline object reports the dominant kernel (the k=4096 Q8_0 GEMV of gate/up),
timed on its own after ~50 ms of untimed launches, median of three runs; the
other configs likewise.  The CPU baseline is the oracle's restatement of zlm's
production sweep on the same gate weight, on one thread per physical core (at
most 16, the CPU share of one GPU) and on one thread; configs[4] and [2] get
CPU figures of their own in `extra`.

Prints one JSON line.  --gpus N with N > 1 is refused: this backend runs on one
GPU.
"""
import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from zlm_amd import device as zd  # noqa: E402
from zlm_amd import synth  # noqa: E402

PEAK_GBPS = 8000.0
MALL_DEFEAT_BYTES = 512 * 1024 * 1024
# The kernel the host picks for the 12288 x 4096 Q8_0 gate/up GEMV (the roofline kernel).
ROOFLINE_KERNEL = "zlm_gemv_q8_0_r1_s4"
METRIC = "quant GEMV HBM GB/s (% of 8 TB/s peak); decode tok/s, Qwen3-8B-shape Q4_0 bs=1"
# Untimed GPU work before each timed measurement (the headline's whatever
# --warmup is), and a scale on the launches per measurement; --counters sets
# both low so a rocprofv3 counter pass (which serialises every dispatch) stays
# short.  Figures from a --counters run are not timings.
WARM = {"ms": 50.0, "launch_scale": 1.0}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class Gemv:
    """One GEMV shape with its resident weight copies and device vectors."""

    def __init__(self, dev, name, qt, rows, k, seed, copies=None):
        self.dev, self.name, self.qt, self.rows, self.k = dev, name, qt, rows, k
        self.w = synth.weights(qt, rows, k, seed)
        self.wbytes = self.w.size
        if copies is None:
            copies = max(1, math.ceil(MALL_DEFEAT_BYTES / self.wbytes))
        self.copies = copies
        self.res = []
        for _ in range(copies):
            r = dev.upload_resident(self.w)
            if r is None:
                raise RuntimeError(dev.last_error())
            self.res.append(r)
        self.x = synth.activation(seed + 1, k)
        self.x_dev = dev.dev_malloc(k * 4)
        dev.dev_upload(self.x_dev, self.x)
        self.y_dev = dev.dev_malloc(rows * 4)

    @property
    def algo_bytes(self) -> int:
        return self.wbytes + 4 * self.k + 4 * self.rows

    def desc(self, c):
        return (self.res[c % self.copies], zd.quant(self.qt), self.rows, self.k, self.x_dev, self.y_dev)

    def free(self):
        for r in self.res:
            self.dev.free_resident(r)
        self.dev.dev_free(self.x_dev)
        self.dev.dev_free(self.y_dev)
        self.res = []


def time_launches(dev, descs, launches_target):
    """Average ms per pass over `descs` (a pass = every desc once): untimed
    passes until ~50 ms of GPU work has run (the clocks ramp over the first
    milliseconds after an idle host phase), then the median of three timed
    runs of launches_target launches."""
    passes = max(1, int(launches_target * WARM["launch_scale"]) // len(descs))
    spent = 0.0
    while spent < WARM["ms"]:
        spent += dev.time_gemv_sequence(descs, passes)
    runs = sorted(dev.time_gemv_sequence(descs, passes) / passes for _ in range(3))
    return runs[1]


def cpu_threads() -> tuple:
    """(threads, physical cores): one thread per physical core among the cores
    this process may run on (the reference pins one worker per physical core),
    capped at the process's CPU share when OMP_NUM_THREADS states one (the
    benchmark box gives each GPU 16 CPUs and sets OMP_NUM_THREADS=16 for it)."""
    import oracle

    cores = len(oracle.physical_cores()) or len(os.sched_getaffinity(0))
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return max(1, min(cores, share) if share > 0 else cores), cores


def host_copies(w: np.ndarray) -> list:
    """Distinct host copies of a weight whose total is past the CPU's last
    level cache (>= 1 GiB and >= 4x the cache), so a timed CPU call streams
    its weights from DRAM as the GPU side's rotation over HBM copies does."""
    import oracle

    target = max(1 << 30, 4 * oracle.last_level_cache_bytes())
    n = max(2, math.ceil(target / max(1, w.nbytes)))
    return [w] + [w.copy() for _ in range(n - 1)]


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _min_time(fn, budget_s: float, max_reps: int = 50000) -> tuple:
    """(best seconds, reps) of fn(reps) -> min-of-reps seconds, sized to ~budget_s."""
    t1 = fn(2)
    reps = max(3, min(max_reps, int(budget_s / max(t1, 1e-6))))
    return min(t1, fn(reps)), reps + 2


def cpu_baseline(g: Gemv, budget_s: float):
    """zlm's production sweep on the headline gate weight, on the CPU: the
    speed-faithful restatement (oracle/zlm_cpu_sweep.c: compile-time lanes at
    zlm's native width, per-type row loops, vector dequant; bit-identical to
    the oracle) over the persistent pinned pool split by rangeOf, plus one
    thread, plus the single-thread [4096, 8192] q8_0 / q4_0 GEMVs zlm publishes."""
    import oracle

    threads, cores = cpu_threads()
    lanes = oracle.fast_native_lanes()
    t0 = time.perf_counter()
    copies = host_copies(g.w)
    best, reps = _min_time(lambda r: oracle.fast_time_matvec_copies(g.qt, copies, g.k, g.rows, g.x, threads, r),
                           0.5 * budget_s)
    best1, reps1 = _min_time(lambda r: oracle.fast_time_matvec_copies(g.qt, copies, g.k, g.rows, g.x, 1, r),
                             0.2 * budget_s, max_reps=200)
    n_copies = len(copies)
    del copies
    published = {}
    # zlm's own single-thread figures: [4096, 8192] (8192 rows of 4096) on a
    # Ryzen 7 5700X (sdd/tasks/kernels/12-instruction-audit.md:81-82)
    for qt, name, ref in ((synth.Q8_0, "q8_0", 17.93), (synth.Q4_0, "q4_0", 7.23)):
        w = synth.weights(qt, 8192, 4096, 0x5A4C4DA0 + qt)
        x = synth.activation(0x5A4C4DA8 + qt, 4096)
        wc = host_copies(w)
        t1 = _min_time(lambda r: oracle.fast_time_matvec_copies(qt, wc, 4096, 8192, x, 1, r), 0.15 * budget_s,
                       100)[0]
        published[name] = {"GBps_1_thread": round(w.nbytes / t1 / 1e9, 2), "ms": round(t1 * 1e3, 3),
                           "zlm_published_GBps_1_thread": ref, "zlm_host": "Ryzen 7 5700X (AVX2, 8 lanes)"}
        del wc
    spent = time.perf_counter() - t0
    return {
        "value": round(g.algo_bytes / best / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"zlm's production sweep restated at zlm's speed (oracle/zlm_cpu_sweep.c, {lanes} lanes as "
                  f"simd.native on this host; bit-identical to the oracle), {g.name} {g.rows}x{g.k} Q8_0 GEMV, "
                  f"{threads} threads pinned one per physical core ({cores} in the affinity mask) split by "
                  f"rangeOf, min of {reps} reps rotating over {n_copies} host copies of the weight (past the "
                  f"{oracle.last_level_cache_bytes() >> 20} MiB last level cache); 1 thread: min of {reps1} reps "
                  f"({spent:.1f} s in all)",
        "ms_per_gemv": round(best * 1e3, 4),
        "cpu": cpu_model(),
        "lanes": lanes,
        "one_thread": {"value": round(g.algo_bytes / best1 / 1e9, 3), "unit": "GB/s",
                       "ms_per_gemv": round(best1 * 1e3, 4)},
        "published_shapes_1_thread": published,
    }


def cpu_prefill_sample(w: np.ndarray, rows: int, k: int, budget_s: float):
    """configs[4] on the CPU: zlm's int path (q8 activations, Q4_0 intBlock)
    at zlm's speed over a 64-token sample of the 512-token workload, all
    threads of the pool; rates scale per token."""
    import oracle

    threads, _ = cpu_threads()
    m = 64
    x = synth.activation(0x5A4C4D0D, m * k)
    best, reps = _min_time(lambda r: oracle.fast_time_matmul_int(synth.Q4_0, w, k, rows, m, x, threads, r),
                           budget_s, 20)
    ops = 2.0 * rows * k * m
    return {"tok_per_s": round(m / best, 1), "TOPS_int8": round(ops / best / 1e12, 4), "cores": threads,
            "kind": "port", "sample": f"zlm's int sweep (Q4_0 intBlock, {oracle.fast_native_lanes()} lanes) "
                                      f"{rows}x{k}, {m} of the 512 tokens, {threads} pinned threads split by "
                                      f"rangeOf, min of {reps} reps"}


def upload_rate(dev) -> dict:
    """uploadResident's rate (reference runtime/session.zig:452-474 uploads
    each planned tensor from the mmap'd image): a 256 MiB Q4_0 weight from
    ordinary (pageable) host memory, as an mmap'd file page is, uploaded 8
    times into fresh residents (2 GiB); host wall time per upload, median of
    the 8, and the configs[2] model's 4.57 GB at that rate."""
    from zlm_amd import decode as zdec

    nb = (256 << 20) // 18
    w = np.frombuffer(np.random.default_rng(7).bytes(nb * 18), np.uint8).copy()
    times = []
    for _ in range(8):
        t0 = time.perf_counter()
        r = dev.upload_resident(w)
        times.append(time.perf_counter() - t0)
        if r is None:
            raise RuntimeError(dev.last_error())
        dev.free_resident(r)
    t = sorted(times)[len(times) // 2]
    gbps = w.nbytes / t / 1e9
    model = zdec.weight_bytes(zdec.QWEN3_8B)
    return {"GBps": round(gbps, 2), "bytes_per_upload": int(w.nbytes), "ms_per_upload": round(t * 1e3, 2),
            "configs2_model_bytes": model, "configs2_upload_s": round(model / gbps / 1e9, 3),
            "note": "uploadResident from pageable host memory into a new resident (synchronous), median of 8"}


def split_efficiency(dev, threads: int) -> dict:
    """measureSplitEfficiency (reference tuner/calibrate.zig:778-834) on this
    device: a 32768 x 4096 Q4_0 resident GEMV through matVecResident alone,
    then split -- matVecResidentAsync over rows [0, m/2) while `threads` CPU
    workers run zlm's production sweep over [m/2, m), then waitResident --
    min of 5 each after 32 warm-up calls; the ratio split rate / GPU rate is
    the tuner's split coefficient (< 1: a split loses to the whole-GPU op)."""
    import oracle

    n, m = 4096, 32768
    q = zd.quant(zd.Q4_0)
    w = synth.weights(synth.Q4_0, m, n, 0x5A4C4DB0)
    x = np.array([((i * 7 + 3) % 17 - 8) * 0.125 for i in range(n)], np.float32)
    res = dev.upload_resident(w)
    if res is None:
        raise RuntimeError(dev.last_error())
    out = np.zeros(m, np.float32)
    for _ in range(32):
        dev.mat_vec_resident(res, q, m, n, x, out)
    dev.sync()
    g = m // 2
    rb = synth.row_bytes(synth.Q4_0, n)
    w_cpu = w[g * rb:]
    gpu_best = split_best = float("inf")
    split_out = np.zeros(m, np.float32)
    for _ in range(5):
        t0 = time.perf_counter()
        dev.mat_vec_resident(res, q, m, n, x, out)
        dev.sync()
        gpu_best = min(gpu_best, time.perf_counter() - t0)
        t0 = time.perf_counter()
        h = dev.mat_vec_resident_async(res, q, g, n, x)
        if h is None:
            raise RuntimeError(dev.last_error())
        oracle.fast_time_matvec(synth.Q4_0, w_cpu, n, m - g, x, threads, 1, out=split_out[g:])
        if not dev.wait_resident(h, split_out, g):
            raise RuntimeError(dev.last_error())
        split_best = min(split_best, time.perf_counter() - t0)
    dev.free_resident(res)
    # the split's rows agree with the whole-GPU op's (fp32 summation order aside)
    err = float(np.linalg.norm(split_out.astype(np.float64) - out) / np.linalg.norm(out))
    if not err <= 1e-3:
        raise AssertionError(f"split GEMV rel-L2 {err:.2e} against the whole-GPU GEMV")
    return {"ratio": round(gpu_best / split_best, 4), "gpu_us": round(gpu_best * 1e6, 1),
            "split_us": round(split_best * 1e6, 1), "gpu_GBps": round(w.nbytes / gpu_best / 1e9, 1),
            "split_GBps": round(w.nbytes / split_best / 1e9, 1), "cpu_threads": threads,
            "rel_l2_split_vs_gpu": err,
            "note": "measureSplitEfficiency: Q4_0 32768x4096 through matVecResident (host x and y) vs "
                    "matVecResidentAsync rows [0, m/2) + CPU production sweep rows [m/2, m) + waitResident, "
                    "min of 5 host wall times each"}


def cpu_decode_sample(cfg, budget_s: float):
    """configs[2] on the CPU: one token's projection GEMVs (q;k;v, o, gate, up,
    down per layer, times the layer count, plus the Q8_0 lm_head) with zlm's
    production sweep at zlm's speed on the pool's threads.  Attention and the
    elementwise glue are not included (on the GPU they are ~20% of a token)."""
    import oracle

    threads, _ = cpu_threads()
    per = max(0.5, budget_s / 6.0)
    h, f = cfg.hidden, cfg.ffn
    shapes = [("qkv", cfg.qkv_rows, h, synth.Q4_0), ("o", h, cfg.n_heads * cfg.head_dim, synth.Q4_0),
              ("gate", f, h, synth.Q4_0), ("up", f, h, synth.Q4_0), ("down", h, f, synth.Q4_0)]
    layer_s = 0.0
    for i, (name, rows, k, qt) in enumerate(shapes):
        wc = host_copies(synth.weights(qt, rows, k, 0x5A4C4D70 + i))
        x = synth.activation(0x5A4C4D78 + i, k)
        layer_s += _min_time(lambda r: oracle.fast_time_matvec_copies(qt, wc, k, rows, x, threads, r), per, 200)[0]
        del wc
    wc = host_copies(synth.weights(cfg.lm_type, cfg.vocab, h, 0x5A4C4D7F))
    x = synth.activation(0x5A4C4D7E, h)
    lm_s = _min_time(lambda r: oracle.fast_time_matvec_copies(cfg.lm_type, wc, h, cfg.vocab, x, threads, r), per,
                     50)[0]
    del wc
    tok_s = cfg.n_layers * layer_s + lm_s
    return {"tok_per_s": round(1.0 / tok_s, 2), "ms_per_token": round(tok_s * 1e3, 2), "cores": threads,
            "kind": "port", "sample": f"production-sweep GEMVs of one layer (x{cfg.n_layers}) and the lm_head, "
                                      f"{threads} threads, min of reps each over host copies past the last level "
                                      f"cache; attention and glue not timed"}


def sections(dev, args, want, extra):
    """The reported sections after the headline: the other configs' GEMVs, the
    configs[4] GEMM, the small-M sweep and the configs[2] decode step (each
    runs when want(section) says so); results go into `extra`."""
    only = args.only
    # ---- the other GEMV configs (reported, not the headline) --------------------
    if want("gemvs"):
        others = [
            ("c0_q4_0_4096x4096", synth.Q4_0, 4096, 4096),
            ("c3_q4_k_15360x3840", synth.Q4_K, 15360, 3840),
            ("c3_q4_k_3840x15360", synth.Q4_K, 3840, 15360),
            ("c3_q6_k_15360x3840", synth.Q6_K, 15360, 3840),
            ("c3_q6_k_3840x15360", synth.Q6_K, 3840, 15360),
            ("c3_q6_k_lm_head_262144x3840", synth.Q6_K, 262144, 3840),
            ("c2_lm_head_q8_0_151936x4096", synth.Q8_0, 151936, 4096),
        ]
        for name, qt, rows, k in others:
            g = Gemv(dev, name, qt, rows, k, 0x5A4C4D40 + rows)
            descs = [g.desc(c) for c in range(g.copies)]
            target = max(len(descs), min(400, int(2e9 / g.wbytes)))
            ms = time_launches(dev, descs, target) / len(descs)
            gbps = g.algo_bytes / (ms * 1e-3) / 1e9
            extra[name] = {"us": round(ms * 1e3, 3), "GBps": round(gbps, 1), "pct_peak": round(100 * gbps / PEAK_GBPS, 1),
                           "copies": g.copies}
            log(f"{name}: {ms * 1e3:.2f} us, {gbps:.1f} GB/s ({100 * gbps / PEAK_GBPS:.1f}%)")
            if name.startswith("c0_"):
                # n GEMVs of this shape over one x in one matVecResidentBatch launch
                batched = {}
                for nb in (2, 4, 8):
                    bd = [g.desc(c)[:6] + (1 if c % nb != nb - 1 else 0,) for c in range(g.copies - g.copies % nb)]
                    msb = time_launches(dev, bd, max(len(bd), 400)) / len(bd)
                    batched[f"x{nb}"] = {"us_per_gemv": round(msb * 1e3, 3),
                                         "GBps": round(g.algo_bytes / (msb * 1e-3) / 1e9, 1)}
                extra[name]["batched"] = batched
                log(f"{name} batched: " + ", ".join(f"{key} {v['us_per_gemv']} us/GEMV ({v['GBps']} GB/s)"
                                                    for key, v in batched.items()))
            g.free()
        # lm_heads of other models (hidden 4096-8192, vocab 128256-152064): the
        # prefetching lm_head instances beyond the configs' row lengths
        lm = {}
        for name, qt, rows, k in (("q4_0_151936x4096", synth.Q4_0, 151936, 4096),
                                  ("q8_0_152064x5120", synth.Q8_0, 152064, 5120),
                                  ("q6_k_152064x5120", synth.Q6_K, 152064, 5120),
                                  ("q4_k_128256x8192", synth.Q4_K, 128256, 8192)):
            g = Gemv(dev, name, qt, rows, k, 0x5A4C4D60 + rows)
            descs = [g.desc(c) for c in range(g.copies)]
            ms = time_launches(dev, descs, max(len(descs), min(400, int(2e9 / g.wbytes)))) / len(descs)
            gbps = g.algo_bytes / (ms * 1e-3) / 1e9
            lm[name] = {"us": round(ms * 1e3, 3), "GBps": round(gbps, 1), "pct_peak": round(100 * gbps / PEAK_GBPS, 1)}
            log(f"lm_head {name}: {ms * 1e3:.2f} us, {gbps:.1f} GB/s ({100 * gbps / PEAK_GBPS:.1f}%)")
            g.free()
        extra["other_models_lm_heads"] = lm

    # ---- prefill GEMM, Q4_0 12288x4096 x 512 tokens, int8 MFMA ---------
    if want("gemm"):
        rows, k, m = 12288, 4096, 512
        w = synth.weights(synth.Q4_0, rows, k, 0x5A4C4D04)
        ncopy = max(1, math.ceil(MALL_DEFEAT_BYTES / w.size))
        ress = [dev.upload_resident(w) for _ in range(ncopy)]
        xg = synth.activation(0x5A4C4D0D, m * k)
        x_dev = dev.dev_malloc(xg.nbytes)
        dev.dev_upload(x_dev, xg)
        o_dev = dev.dev_malloc(m * rows * 4)
        iters = max(2, int(4 * ncopy * WARM["launch_scale"]))
        spent = 0.0
        while spent < WARM["ms"]:  # untimed: clocks up, as for the GEMVs
            spent += dev.time_mat_mul(ress, zd.quant(zd.Q4_0), rows, k, m, x_dev, o_dev, iters)
        ms = sorted(dev.time_mat_mul(ress, zd.quant(zd.Q4_0), rows, k, m, x_dev, o_dev, iters) / iters
                    for _ in range(3))[1]
        ops = 2.0 * rows * k * m
        extra["c4_prefill_q4_0_12288x4096_m512"] = {
            "us": round(ms * 1e3, 2), "TOPS_int8": round(ops / (ms * 1e-3) / 1e12, 2),
            "pct_int8_peak_5000": round(100 * ops / (ms * 1e-3) / 5e15, 2),
            "tok_per_s": round(m / (ms * 1e-3), 1),
            "note": "activation quantizer + int8-MFMA GEMM per iteration; dense int8 peak taken as 5.0 POP/s"}
        log(f"c4 prefill GEMM: {ms * 1e3:.1f} us, {ops / (ms * 1e-3) / 1e12:.1f} TOP/s")
        if not args.no_cpu:
            c4cpu = cpu_prefill_sample(w, rows, k, 0.25 * args.cpu_seconds)
            extra["c4_prefill_q4_0_12288x4096_m512"]["cpu_baseline"] = c4cpu
            log(f"c4 CPU: {c4cpu['tok_per_s']} tok/s on {c4cpu['cores']} threads")
        for r in ress:
            dev.free_resident(r)
        dev.dev_free(x_dev)
        dev.dev_free(o_dev)

    # ---- small token counts (verify / microbatch), as reference gpu/root_test.zig:651-696 ----
    if (only is None and not args.quick and not args.no_small_m) or only == "smallm":
        sweep = {}
        few = (1, 2, 3, 4, 5, 8, 9)
        for sname, qt, rows, k, ms in (("q4_0_4096x4096", synth.Q4_0, 4096, 4096, few + (33, 64, 128, 256)),
                                       ("q4_k_4096x4096", synth.Q4_K, 4096, 4096, few + (33, 64, 128, 256)),
                                       ("q4_k_lm_head_262144x3840", synth.Q4_K, 262144, 3840, few)):
            w = synth.weights(qt, rows, k, 0x5A4C4D05)
            ncopy = max(1, math.ceil(MALL_DEFEAT_BYTES / w.size))
            ress = [dev.upload_resident(w) for _ in range(ncopy)]
            xs = synth.activation(0x5A4C4D0E, max(ms) * k)
            x_dev = dev.dev_malloc(xs.nbytes)
            dev.dev_upload(x_dev, xs)
            o_dev = dev.dev_malloc(max(ms) * rows * 4)
            it = max(2, int(4 * ncopy * WARM["launch_scale"]))
            spent = 0.0
            while spent < WARM["ms"]:
                spent += dev.time_mat_vec(ress, zd.quant(qt), rows, k, x_dev, o_dev, it)
            gemv_us = sorted(dev.time_mat_vec(ress, zd.quant(qt), rows, k, x_dev, o_dev, it) / it
                             for _ in range(3))[1] * 1e3
            row = {"gemv_us": round(gemv_us, 2)}
            for m in ms:
                dev.time_mat_mul(ress, zd.quant(qt), rows, k, m, x_dev, o_dev, ncopy)
                us = sorted(dev.time_mat_mul(ress, zd.quant(qt), rows, k, m, x_dev, o_dev, it) / it
                            for _ in range(3))[1] * 1e3
                row[f"m{m}_us"] = round(us, 2)
            sweep[sname] = row
            log(f"small-m {sname}: GEMV {gemv_us:.1f} us; " +
                ", ".join(f"M{m} {row[f'm{m}_us']:.1f}" for m in ms))
            for r in ress:
                dev.free_resident(r)
            dev.dev_free(x_dev)
            dev.dev_free(o_dev)
        sweep["note"] = ("device-level matMul at m tokens vs one GEMV (weights rotated over >= 512 MiB): m = 1 the fp "
                         "GEMV, m = 2 the two-token fp GEMV (one pass over the weights), 3..4 the int-path token GEMV "
                         "(activations quantized in its prologue), 5..32 the split-K int8-MFMA GEMM (activation "
                         "quantizer included), past 32 that kernel over several 32-token tiles or the tiled int8-MFMA "
                         "GEMM, whichever the host's cost model predicts faster")
        extra["small_m_matmul"] = sweep

    # ---- decode step of a Qwen3-8B-shaped Q4_0 model, batch 1 ----------
    cfg = None
    if want("decode"):
        from zlm_amd import decode as zdec

        cfg = zdec.QWEN3_8B
        log("c2 decode: synthesising the Qwen3-8B-shaped model in HBM")
        model = zdec.DecodeModel(dev, cfg)
        x = synth.activation(0x5A4C4D02, cfg.hidden)
        model.step(x, cfg.max_seq - 1)  # eager: converts layouts, sizes scratch
        tok_bytes = zdec.weight_bytes(cfg) + zdec.kv_bytes(cfg, cfg.max_seq)
        if args.decode_eager:
            # profiled runs: the step's kernels launched eagerly, no graph (a
            # graph replayed under rocprofv3's kernel trace aborted the queue)
            model.set_input(x, cfg.max_seq - 1)
            for _ in range(args.decode_eager):
                model.enqueue_step()
            dev.sync()
            extra["c2_decode_qwen3_8b_q4_0"] = {
                "eager_steps": args.decode_eager, "bytes_per_token": tok_bytes,
                "note": "--decode-eager: kernels launched eagerly for a profiler; no tok/s measured"}
            log(f"c2 decode: {args.decode_eager} eager steps (profiling run, not timed)")
            model.free()
            cfg = None
    if want("decode") and cfg is not None:
        if zd.profiler_loaded():
            # the library refuses graph replays under a profiler (replays of
            # this step under rocprofv3's kernel trace aborted the process)
            raise SystemExit("bench.py: a rocprofiler library is loaded in this process, and the decode step is "
                             "timed from graph replays, which the library refuses under a profiler; profile the "
                             "decode kernels with --decode-eager N instead")
        graph = model.capture()
        model.set_input(x, cfg.max_seq - 1)
        reps = max(1, args.decode_replays)
        dev.graph_launch(graph, reps)  # ~50 ms untimed (30 replays): clocks up after the host-side synthesis
        ms = sorted(dev.graph_launch(graph, reps) / reps for _ in range(3))[1]
        gbps = tok_bytes / (ms * 1e-3) / 1e9
        extra["c2_decode_qwen3_8b_q4_0"] = {
            "tok_per_s": round(1e3 / ms, 1), "ms_per_token": round(ms, 4), "bytes_per_token": tok_bytes,
            "GBps": round(gbps, 1), "pct_peak": round(100 * gbps / PEAK_GBPS, 1), "context": cfg.max_seq,
            "launches_per_token": 1 + 6 * cfg.n_layers + 1,
            "note": "36 layers, Q4_0 projections (q;k;v fused rows), Q8_0 lm_head, fp16 KV at 2048; one step "
                    "captured in a HIP graph and replayed; weights synthesised in HBM"}
        log(f"c2 decode: {ms:.3f} ms/token = {1e3 / ms:.1f} tok/s, {gbps:.1f} GB/s ({100 * gbps / PEAK_GBPS:.1f}%)")
        dev.graph_destroy(graph)
        model.free()
        # the same step at longer caches (the last position of each): attention's
        # share grows with the KV bytes
        if not args.no_long_context:
            import dataclasses

            longer = {}
            for ctx in (8192, 32768):
                lcfg = dataclasses.replace(cfg, max_seq=ctx)
                lmodel = zdec.DecodeModel(dev, lcfg)
                lmodel.step(x, ctx - 1)
                lgraph = lmodel.capture()
                lmodel.set_input(x, ctx - 1)
                dev.graph_launch(lgraph, reps)
                lms = sorted(dev.graph_launch(lgraph, reps) / reps for _ in range(3))[1]
                lbytes = zdec.weight_bytes(lcfg) + zdec.kv_bytes(lcfg, ctx)
                longer[str(ctx)] = {"tok_per_s": round(1e3 / lms, 1), "ms_per_token": round(lms, 4),
                                    "bytes_per_token": lbytes, "GBps": round(lbytes / (lms * 1e-3) / 1e9, 1)}
                log(f"c2 decode at context {ctx}: {lms:.3f} ms/token = {1e3 / lms:.1f} tok/s, "
                    f"{longer[str(ctx)]['GBps']} GB/s")
                if ctx == 32768:
                    # a step early in that cache (position 511): the full-cache
                    # graph reads every position's K/V, the graph captured for
                    # the position's window bucket (512) only the first 512
                    short = {}
                    for name, window in (("full_cache_graph", None), ("window_graph", lmodel.window_for(511))):
                        g_ = lmodel.capture(window)
                        lmodel.set_input(x, 511)
                        dev.graph_launch(g_, reps)
                        short[name] = round(sorted(dev.graph_launch(g_, reps) / reps for _ in range(3))[1], 4)
                        dev.graph_destroy(g_)
                    short["note"] = ("ms/token at position 511 of a 32768-position cache: the full-cache graph "
                                     "against the graph for the position's attention window (512)")
                    longer[str(ctx)]["position_511"] = short
                    log(f"c2 decode at position 511 of a 32768 cache: {short['full_cache_graph']:.3f} ms/token "
                        f"(full-cache graph), {short['window_graph']:.3f} ms/token (window-512 graph)")
                dev.graph_destroy(lgraph)
                lmodel.free()
            extra["c2_decode_qwen3_8b_q4_0"]["longer_contexts"] = longer
        # the same token's projections through the contract ops only, as zlm's
        # executor submits them (separate q/k/v residents, bursts and drains,
        # host activations); the CPU glue between them is not run
        log("c2 decode via the contract ops: synthesising separate q/k/v/o/gate/up/down residents")
        h_, f_ = cfg.hidden, cfg.ffn
        qr, kvr = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
        shapes = [(qr, h_), (kvr, h_), (kvr, h_), (h_, qr), (f_, h_), (f_, h_), (h_, f_)]
        layers, allres = [], []
        for li in range(cfg.n_layers):
            layer = []
            for j, (rr, kk) in enumerate(shapes):
                r_ = dev.synth_resident(zd.Q4_0, rr * kk // 32, 0x5A4C4D90 + 16 * li + j, 0.02)
                if r_ is None:
                    raise RuntimeError(dev.last_error())
                layer.append(r_)
            layers.append(layer)
            allres += layer
        lm = dev.synth_resident(zd.Q8_0, cfg.vocab * h_ // 32, 0x5A4C4D9F, 0.01)
        allres.append(lm)
        ms_c = sorted(dev.time_contract_decode(layers, zd.quant(zd.Q4_0), h_, qr, kvr, f_, lm, zd.quant(zd.Q8_0),
                                               cfg.vocab, 3) for _ in range(3))[1]
        extra["c2_decode_qwen3_8b_q4_0"]["contract_path"] = {
            "ms_per_token": round(ms_c, 3), "tok_per_s": round(1e3 / ms_c, 1),
            "note": "projections only, through matVecResidentBurstAsync / matVecMlpPairResidentBurstAsync / "
                    "waitResident / matVecResident with host activations, in the executor's burst pattern; "
                    "CPU attention and glue not included"}
        log(f"c2 decode via the contract ops: {ms_c:.3f} ms/token (GPU ops only)")
        for r_ in allres:
            dev.free_resident(r_)
        if not args.no_cpu:
            c2cpu = cpu_decode_sample(cfg, 0.25 * args.cpu_seconds)
            extra["c2_decode_qwen3_8b_q4_0"]["cpu_baseline"] = c2cpu
            log(f"c2 CPU: {c2cpu['tok_per_s']} tok/s (projection GEMVs) on {c2cpu['cores']} threads")

    return extra


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--quick", action="store_true", help="headline workload only")
    ap.add_argument("--cpu-seconds", type=float, default=16.0,
                    help="CPU-baseline budget: half on the headline GEMV, a quarter each on configs[4] and [2]")
    ap.add_argument("--decode-eager", type=int, default=0, metavar="N",
                    help="run N eager decode steps instead of timing graph replays (for kernel-trace profiling)")
    ap.add_argument("--decode-replays", type=int, default=30, metavar="N",
                    help="graph replays per timed decode run (warm-up run + 3 timed runs of N)")
    ap.add_argument("--no-long-context", action="store_true",
                    help="skip the decode step at 8192 and 32768 cached positions")
    ap.add_argument("--no-small-m", action="store_true",
                    help="skip the small-token-count matMul sweep (its GEMVs share kernels with configs[0]/[3])")
    ap.add_argument("--counters", action="store_true",
                    help="short warm-ups and few launches per shape, for rocprofv3 --pmc passes (not a timing run)")
    ap.add_argument("--only", choices=("roofline", "gemvs", "gemm", "smallm", "decode"), default=None,
                    help="run one section for a profiler: the roofline kernel's timing (configs[1] gate/up), the "
                         "other configs' GEMVs, the configs[4] GEMM, the small-token-count matMul sweep or the "
                         "decode step; no JSON line")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="BYTES",
                    help="also run the library copy kernel 5x over BYTES (for HBM traffic counter calibration)")
    args = ap.parse_args()
    if args.counters:
        WARM["ms"], WARM["launch_scale"] = 0.0, 0.05
    if args.gpus != 1:
        print(f"bench.py: this backend runs on one GPU; --gpus {args.gpus} is not supported "
              "(the multi-GPU sharding is a design note, not a measured path)", file=sys.stderr)
        sys.exit(2)

    dev = zd.Device()
    if not dev.available():
        raise SystemExit(f"HIP backend unavailable: {dev.last_error()}")
    log(f"device: {dev.device_name()}, {dev.cu_count()} CUs")
    if args.calibrate_copy:
        nbytes = (args.calibrate_copy // 16) * 16
        a, b = dev.dev_malloc(nbytes), dev.dev_malloc(nbytes)
        for _ in range(5):
            dev.dev_copy(b, a, nbytes)
        dev.dev_free(a)
        dev.dev_free(b)
        log(f"copy calibration: 5 x {nbytes} bytes")

    only = args.only

    def want(section: str) -> bool:
        return (only is None and not args.quick) or only == section

    if only in ("gemvs", "gemm", "smallm", "decode"):
        return sections(dev, args, want, {})

    # ---- headline: configs[1], Q8_0 Qwen3-8B FFN GEMVs ------------------------------
    step_w = 2 * synth.weight_bytes(synth.Q8_0, 12288, 4096) + synth.weight_bytes(synth.Q8_0, 4096, 12288)
    copies = max(1, math.ceil(MALL_DEFEAT_BYTES / step_w))
    log(f"C1: generating Q8_0 gate/up/down, {copies} resident copies each")
    gate = Gemv(dev, "gate", synth.Q8_0, 12288, 4096, 0x5A4C4D01, copies)
    up = Gemv(dev, "up", synth.Q8_0, 12288, 4096, 0x5A4C4D11, copies)
    down = Gemv(dev, "down", synth.Q8_0, 4096, 12288, 0x5A4C4D21, copies)
    step_descs = []
    for c in range(copies):
        step_descs += [gate.desc(c), up.desc(c), down.desc(c)]
    step_bytes = gate.algo_bytes + up.algo_bytes + down.algo_bytes

    def steps_of(n):  # n consecutive steps, step i on weight copy i % copies
        out = []
        for i in range(n):
            out += [gate.desc(i), up.desc(i), down.desc(i)]
        return out

    # W warm-up steps, then untimed steps until >= 50 ms of GPU time have run
    # since the host-side synthesis (the clocks ramp over the first
    # milliseconds; a short warm-up alone reads several percent low), then
    # exactly K timed steps.
    steps = max(1, args.steps)
    warmup = max(0, args.warmup)
    clock_ms = dev.time_gemv_sequence(steps_of(warmup), 1) if warmup else 0.0
    while clock_ms < WARM["ms"]:
        clock_ms += dev.time_gemv_sequence(step_descs, max(1, 200 // copies))
    ms_total = dev.time_gemv_sequence(steps_of(steps), 1)
    ms_step = ms_total / steps
    value = step_bytes / (ms_step * 1e-3) / 1e9
    log(f"C1 step: {ms_step * 1e3:.2f} us -> {value:.1f} GB/s ({100 * value / PEAK_GBPS:.1f}% of peak) over "
        f"{steps} steps after {warmup} warm-up steps ({clock_ms:.1f} ms of untimed GPU work)")

    # dominant kernel: the k=4096 gate/up GEMV, alone, same rotation
    gu_descs = []
    for c in range(copies):
        gu_descs += [gate.desc(c), up.desc(c)]
    gu_target = 4 * len(gu_descs) * 25
    ms_gu = time_launches(dev, gu_descs, gu_target) / len(gu_descs)
    gu_gbps = gate.algo_bytes / (ms_gu * 1e-3) / 1e9
    if only == "roofline":
        # the timed launches are the last 3 x timed_launches dispatches of the kernel
        timed = max(1, int(gu_target * WARM["launch_scale"]) // len(gu_descs)) * len(gu_descs)
        log(f"roofline kernel {ROOFLINE_KERNEL}: {ms_gu * 1e3:.3f} us per launch (HIP events, median of 3 runs of "
            f"{timed} launches: the last {3 * timed} dispatches of the kernel) -> {gu_gbps:.1f} GB/s; "
            f"profiler loaded: {zd.profiler_loaded()}")
        print(json.dumps({"roofline_only": {"kernel": ROOFLINE_KERNEL, "avg_launch_us": round(ms_gu * 1e3, 4),
                                            "timed_dispatches": 3 * timed, "GBps": round(gu_gbps, 1),
                                            "profiler_loaded": zd.profiler_loaded()}}), flush=True)
        for g in (gate, up, down):
            g.free()
        dev.deinit()
        return
    ms_dn = time_launches(dev, [down.desc(c) for c in range(copies)], 100 * copies) / copies
    dn_gbps = down.algo_bytes / (ms_dn * 1e-3) / 1e9
    log(f"gate/up GEMV {ms_gu * 1e3:.2f} us ({gu_gbps:.1f} GB/s); down GEMV {ms_dn * 1e3:.2f} us ({dn_gbps:.1f} GB/s)")

    extra = {
        "c1_gate_up_q8_0_12288x4096": {"us": round(ms_gu * 1e3, 3), "GBps": round(gu_gbps, 1)},
        "c1_down_q8_0_4096x12288": {"us": round(ms_dn * 1e3, 3), "GBps": round(dn_gbps, 1)},
    }
    # gate and up over the same x as one matVecResidentBatch launch
    pair = []
    for c in range(copies):
        pair += [gate.desc(c)[:4] + (gate.x_dev, gate.y_dev, 1), up.desc(c)[:4] + (gate.x_dev, up.y_dev, 0)]
    ms_pair = time_launches(dev, pair, 4 * len(pair) * 25) / len(pair)
    extra["c1_gate_up_batched"] = {
        "us_per_gemv": round(ms_pair * 1e3, 3), "GBps": round(gate.algo_bytes / (ms_pair * 1e-3) / 1e9, 1),
        "note": "gate and up over one x as one matVecResidentBatch launch (the batch kernel, both ops' rows)"}
    log(f"gate + up as one batch launch: {ms_pair * 1e3:.2f} us per GEMV "
        f"({extra['c1_gate_up_batched']['GBps']} GB/s)")

    # the same GEMVs through the contract ops zlm's executor calls: a burst of
    # one (host x staged) + waitResident (host y read back), host wall time
    cit = max(20, int(400 * WARM["launch_scale"]))
    for g_, key in ((gate, "c1_gate_up_q8_0_12288x4096"), (down, "c1_down_q8_0_4096x12288")):
        dev.time_contract_gemv(g_.res, zd.quant(g_.qt), g_.rows, g_.k, cit)
        us = sorted(dev.time_contract_gemv(g_.res, zd.quant(g_.qt), g_.rows, g_.k, cit) for _ in range(3))[1]
        extra[key]["contract_us"] = round(us, 2)
        extra[key]["contract_GBps"] = round(g_.algo_bytes / (us * 1e-6) / 1e9, 1)
    log(f"contract path (burst + waitResident, host x/y): gate/up {extra['c1_gate_up_q8_0_12288x4096']['contract_us']}"
        f" us, down {extra['c1_down_q8_0_4096x12288']['contract_us']} us")
    # where a contract GEMV's host wall time goes: the submit call, the
    # waitResident call, and the GPU's time between events around the submission
    split = [dev.time_contract_gemv_split(gate.res, zd.quant(gate.qt), gate.rows, gate.k, cit) for _ in range(3)]
    split = sorted(split, key=lambda v: v["total_us"])[1]
    extra["c1_gate_up_q8_0_12288x4096"]["contract_split_us"] = {
        key: round(v, 2) for key, v in split.items()}
    extra["c1_gate_up_q8_0_12288x4096"]["contract_split_us"]["note"] = (
        "per op: total host wall time = submit (x into the slot's pinned buffer, copy kernel and GEMV enqueued) + "
        "wait (waitResident: the rest of the GPU's run, wake-up, y copied out); gpu = HIP events around the "
        "submission (copy kernel + GEMV); the two extra events add ~2-5 us to the total")
    log(f"contract split (gate/up): {split}")

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            t = json.load(f)
        traffic = t.get(ROOFLINE_KERNEL, {}).get("bytes_per_launch")
    # the same kernel's average duration in the committed kernel trace of its
    # timed launches: algorithmic bytes / that duration / peak
    frac_profile, trace_ns = None, None
    rpath = os.path.join(ROOT, "profiles", "roofline_trace.json")
    if os.path.exists(rpath):
        with open(rpath) as f:
            trace_ns = json.load(f).get(ROOFLINE_KERNEL, {}).get("trace_avg_ns")
        if trace_ns:
            frac_profile = round(gate.algo_bytes / (trace_ns * 1e-9) / 1e9 / PEAK_GBPS, 4)

    cpu = None
    if not args.no_cpu:
        log(f"CPU baseline (~{0.5 * args.cpu_seconds:.0f} s)")
        cpu = cpu_baseline(gate, 0.5 * args.cpu_seconds)
        log(f"CPU ({cpu['cpu']}, {cpu['lanes']} lanes): {cpu['value']} GB/s on {cpu['cores']} threads, "
            f"{cpu['one_thread']['value']} GB/s on 1; [4096, 8192] on 1 thread: " +
            ", ".join(f"{n} {v['GBps_1_thread']} GB/s (zlm {v['zlm_published_GBps_1_thread']})"
                      for n, v in cpu["published_shapes_1_thread"].items()))
        extra["upload_resident"] = upload_rate(dev)
        log(f"uploadResident: {extra['upload_resident']['GBps']} GB/s from pageable host memory "
            f"(configs[2] weights in {extra['upload_resident']['configs2_upload_s']} s)")
        extra["split_efficiency"] = split_efficiency(dev, cpu["cores"])
        log(f"split probe (GPU rows [0, m/2) + {cpu['cores']} CPU threads [m/2, m)): "
            f"{extra['split_efficiency']['split_us']} us against {extra['split_efficiency']['gpu_us']} us "
            f"whole-GPU, ratio {extra['split_efficiency']['ratio']}")
    for g in (gate, up, down):
        g.free()

    sections(dev, args, want, extra)

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "warmup_gpu_ms": round(clock_ms, 2),
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded splitmix64: f16 scales |N(0,1)|*0.01, int8 quants U[-127,127], x N(0,1))",
        "config": {
            "workload": "configs[1]: Q8_0 Qwen3-8B FFN GEMVs at batch 1, gate+up 12288x4096 and down 4096x12288 "
                        "per step, weights resident in HBM",
            "weight_copies_rotated": copies,
            "bytes_per_step": step_bytes,
        },
        "pct_of_peak": round(100 * value / PEAK_GBPS, 2),
        "roofline": {
            "bound": "hbm",
            "kernel": f"{ROOFLINE_KERNEL} (gate/up 12288x4096)",
            "achieved": round(gu_gbps, 1),
            "peak": PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(gu_gbps / PEAK_GBPS, 4),
            "frac_profile": frac_profile,
            "profile_avg_ns": trace_ns,
            "traffic": traffic,
            "algorithmic_bytes_per_launch": gate.algo_bytes,
            "avg_launch_us": round(ms_gu * 1e3, 3),
        },
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    dev.deinit()


if __name__ == "__main__":
    main()
