#!/usr/bin/env python3
"""Benchmark of the gfx950 e-means hot path on one MI355X.

Headline workload (the metric "train s & assign Mrows/s at 200k x 768 k=1024
FP32; % of FP32 MFMA peak"): 200,000 x 768 rows from a 1024-component Gaussian
mixture (means ~N(0, I), per-component diagonal std ~U(0.2, 1), Zipf(1.1)
weights, seed 0), exact FP32, L2. One step = one full training run (5 epochs,
the throughput-law recipe: 13 batches of 16,384 per epoch) followed by the
assignment of all 200,000 rows, with the data resident in HBM.

value = top-1 rows processed per second over the whole step (5 training passes
plus the final assignment: 1.2 M rows per step), in Mrows/s. The line also
reports train seconds, assignment Mrows/s, the rooflines and the CPU baseline:

  roofline         the dominant kernel, the MFMA screen (the dense x.C^T
                   contraction ahead of the exact f32 check): algorithmic
                   2 rows k d FLOP per launch over the HIP-event-timed
                   duration of every 8th launch in the timed steps, against
                   the 2.5 PFLOP/s dense bf16 peak of the unit it runs on (its
                   three bf16 passes, x.c ~ xh.ch + xh.cl + xl.ch, are
                   reported apart as the issued rate);
  update_rooflines scatter_add and ema_update, algorithmic HBM bytes per
                   call over their HIP-event time in two more steps with every
                   call timed, against 8 TB/s;
  cpu_baseline     the oracle's C++ restatement of the reference CPU backend
                   (cpu-fused float order) running the same training and
                   assignment on this host, median of three runs, with a
                   bit-exact parity check;
  other_workloads  assign-only 2M x 1024 vs k = 16,384 (IP) and knn_self k = 10
                   on 500k x 384, data resident, with the oracle on a sample
                   of queries; C5, auto_cluster of 900,000 x 768 nested rows
                   then the add of 100,000 (stage times, fits per second, the
                   oracle's fit rate, and a reduced C5 sequence compared with
                   the oracle whole).

`f32_screen` repeats the step with the screen on v_mfma_f32_32x32x2_f32
(same bits, checked).
"""

import argparse
import json
import os
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

FP32_MFMA_PEAK = 157.3  # TFLOP/s, MI355X dense
BF16_MFMA_PEAK = 2500.0  # TFLOP/s, MI355X dense
HBM_PEAK = 8000.0       # GB/s
METRIC = "train s & assign Mrows/s at 200k×768 k=1024 FP32; % of FP32 MFMA peak"
# HBM bytes per screen launch over this workload's launch mix (calibrated
# FETCH_SIZE + WRITE_SIZE from two rocprofv3 --pmc passes of this script, with
# a plain copy kernel of known size as the scale;
# profiles/k_screen_train_assign_200kx768_k1024_hbm_traffic.md): 89.2 MB per
# 16,384-row batch launch (50.3 MB of split rows, the centroids once per XCD),
# 335 MB per 65,536-row assignment chunk, 40 MB per epoch-tail batch (the
# 128 x 128 screen). Measured at commit 2b8405f; the run does not count it
# again (counters need a profiler pass of their own), so the line names where
# the figure comes from.
SCREEN_TRAFFIC_BYTES = 95.6e6
SCREEN_TRAFFIC_SOURCE = ("profiles/k_screen_train_assign_200kx768_k1024_hbm_traffic.md, "
                         "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE at commit 2b8405f")
# The screen's roofline times every PROFILE_EVERY-th launch of the timed steps
# with HIP events (an event pair between two kernels costs the stream a few
# microseconds; on every launch that was ~5 % of the headline step).
PROFILE_EVERY = 8


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def screen_roofline(ms, launches, flop, kernel, traffic=None, traffic_source=None):
    """The screen's roofline: algorithmic FLOP (2 rows k d per launch) over its
    HIP-event time against the dense bf16 MFMA peak of the unit it runs on.
    Beside it: the bf16 MFMA work it issues (three products per multiply-add)
    and the ratio of the algorithmic rate to the f32 MFMA peak (above 1 when
    the exact f32 results come faster than f32 MFMA arithmetic could give)."""
    alg = flop / (ms * 1e-3) / 1e12 if ms > 0 else 0.0
    return {"bound": "mfma", "kernel": kernel, "achieved": alg, "peak": BF16_MFMA_PEAK,
            "unit": "TFLOP/s", "frac": alg / BF16_MFMA_PEAK, "traffic": traffic,
            "traffic_source": traffic_source,
            "launches": launches, "avg_launch_ms": ms / max(launches, 1),
            "flop_per_launch": flop / max(launches, 1),
            "issued_bf16": {"achieved": 3.0 * alg, "frac": 3.0 * alg / BF16_MFMA_PEAK},
            "vs_fp32_mfma_peak": {"peak": FP32_MFMA_PEAK, "ratio": alg / FP32_MFMA_PEAK}}


def hbm_roofline(ms, instances, nbytes, kernels):
    """An update op's roofline: algorithmic bytes per call over its
    HIP-event time against the 8 TB/s HBM peak."""
    gbs = nbytes / (ms * 1e-3) / 1e9 if ms > 0 else 0.0
    return {"bound": "hbm", "kernels": kernels, "achieved": gbs, "peak": HBM_PEAK, "unit": "GB/s",
            "frac": gbs / HBM_PEAK, "calls": instances, "avg_call_ms": ms / max(instances, 1),
            "bytes_per_call": nbytes / max(instances, 1)}


def host_cpu():
    """The host CPU as lscpu reports it (model, sockets, physical cores, clock)."""
    info = {"nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0))}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        kv = {}
        for line in out.splitlines():
            if ":" in line:
                a, v = line.split(":", 1)
                kv[a.strip()] = v.strip()
        sockets = int(kv.get("Socket(s)", "1") or 1)
        cps = int(kv.get("Core(s) per socket", "0") or 0)
        info.update({"model": kv.get("Model name"), "sockets": sockets,
                     "physical_cores": sockets * cps,
                     "threads_per_core": int(kv.get("Thread(s) per core", "1") or 1),
                     "max_mhz": float(kv["CPU max MHz"]) if "CPU max MHz" in kv else None})
        with open("/proc/cpuinfo") as f:
            mhz = [float(l.split(":")[1]) for l in f if l.startswith("cpu MHz")]
        if mhz:
            info["cpuinfo_mhz"] = max(mhz)
    except Exception as e:  # lscpu missing: report what Python sees
        info["lscpu_error"] = str(e)
    return info


def headline(args):
    from emeans_amd import Config, HipDevice, synth

    n, d, k = 200_000, 768, 1024
    t = time.time()
    x, _ = synth.gmm_zipf(n=n, d=d, comps=1024, s=1.1, seed=0)
    log(f"data: {n} x {d} generated in {time.time() - t:.1f} s")
    dev = HipDevice()
    xb = dev.bind(x)
    labels = dev.zeros_u32(n)
    scores = dev.zeros_f32(n)
    cfg = Config(d=d, k=k, seed=0)
    cb = dev.zeros_f32(k * d)  # the trained centroids stay on the device for the assignment

    def step():
        t0 = time.perf_counter()
        cent, info = dev.train_dev(xb, n, cfg, centroids_out=cb)
        t1 = time.perf_counter()
        dev.assign_dev(xb, n, d, cb, k, "l2", labels, scores)
        dev.sync()
        t2 = time.perf_counter()
        return t1 - t0, t2 - t1, cent, info

    def timed(mode, steps, warmup):
        """Warmup, then `steps` timed steps with the screen in `mode`
        (1: bf16 three-pass, 2: f32), the screen's launches profiled."""
        dev.set_screen(mode)
        for i in range(warmup):
            tr, asg, _, info = step()
            log(f"warmup {i} (screen {mode}): train {tr * 1e3:.1f} ms, assign {asg * 1e3:.1f} ms, "
                f"fallback rows {info['fallback_rows']}")
        dev.sync()
        dev.profile(PROFILE_EVERY, "screen")
        trains, assigns = [], []
        t0 = time.perf_counter()
        for i in range(steps):
            tr, asg, cent, info = step()
            trains.append(tr)
            assigns.append(asg)
        dev.sync()
        t1 = time.perf_counter()
        dev.profile(False)
        ms, launches, flop = dev.profile_read("screen")
        # The update ops' rooflines come from two more steps with every call
        # timed, after the timed region (their event pairs stay out of the value).
        dev.profile(1)
        for _ in range(2):
            step()
        dev.sync()
        dev.profile(False)
        dev.profile_read("screen")
        upd = {op: dev.profile_read(op) for op in ("scatter_add", "ema_update")}
        r = {"step_s": (t1 - t0) / steps, "train_s": float(np.median(trains)),
             "assign_s": float(np.median(assigns)), "ms": ms, "launches": launches, "flop": flop,
             "update": upd,
             "cent": cent, "info": info, "labels": dev.read_u32(labels),
             "scores": dev.read_f32(scores)}
        dev.set_screen(1)
        return r

    main = timed(1, args.steps, args.warmup)
    step_s, info, cent = main["step_s"], main["info"], main["cent"]
    ms, launches, flop = main["ms"], main["launches"], main["flop"]
    epochs = len(info["stats"])
    rows_per_step = epochs * n + n
    gpu_labels, gpu_scores = main["labels"], main["scores"]
    out = {
        "metric": METRIC,
        "value": rows_per_step / step_s / 1e6,
        "unit": "Mrows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_s * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "train+assign 200000x768 k=1024 L2, GMM 1024 comps Zipf(1.1), seed 0",
                   "n": n, "d": d, "k": k, "epochs": epochs,
                   "batch": info["batch_size"], "steps_per_run": info["total_steps"]},
        "train_s": main["train_s"],
        "assign_s": main["assign_s"],
        "assign_mrows_s": n / main["assign_s"] / 1e6,
        "train_mrows_s": epochs * n / main["train_s"] / 1e6,
        "fallback_rows_per_run": info["fallback_rows"],
        "roofline": screen_roofline(
            ms, launches, flop,
            "k_screen4 (bf16 MFMA, three passes xh.ch + xh.cl + xl.ch on operands split "
            "ahead of time, f32 accumulation, LDS-DMA ring; per-row candidate lists within "
            "the bound of each lane's best); the epoch tails' 3,392-row batches on the "
            "128 x 128 k_screen", SCREEN_TRAFFIC_BYTES, SCREEN_TRAFFIC_SOURCE),
        "update_rooflines": {
            "scatter_add": hbm_roofline(*main["update"]["scatter_add"],
                                        "k_place_scan + k_sums (labels tallied by the "
                                        "check and the queued-row scan, chunked counting-sort "
                                        "placement, ordered per-cluster sums)"),
            "ema_update": hbm_roofline(*main["update"]["ema_update"], "k_ema"),
        },
    }
    if not args.no_f32:
        f = timed(2, max(2, args.steps // 2), 1)
        fa = f["flop"] / (f["ms"] * 1e-3) / 1e12 if f["ms"] > 0 else 0.0
        out["f32_screen"] = {
            "value": rows_per_step / f["step_s"] / 1e6, "train_s": f["train_s"],
            "assign_s": f["assign_s"],
            "roofline": {"bound": "mfma", "kernel": "k_screen (f32 MFMA, v_mfma_f32_32x32x2_f32)",
                         "achieved": fa, "peak": FP32_MFMA_PEAK, "unit": "TFLOP/s",
                         "frac": fa / FP32_MFMA_PEAK, "launches": f["launches"],
                         "avg_launch_ms": f["ms"] / max(f["launches"], 1)},
            "equal_to_bf16_screen": bool(np.array_equal(f["labels"], gpu_labels)
                                         and f["scores"].tobytes() == gpu_scores.tobytes()
                                         and f["cent"].tobytes() == cent.tobytes()),
        }
    if not args.no_host:
        out["from_host"] = from_host(dev, x, cfg, gpu_labels, gpu_scores)
    if not args.no_cpu:
        out["cpu_baseline"], out["parity"] = cpu_baseline(x, cfg, cent, info, gpu_labels,
                                                          gpu_scores, args)
    if not args.no_others:
        del xb, labels, scores, cb
        dev.close()
        out["ops_bench"] = ops_bench()
        out["other_workloads"] = other_workloads(args)
    return out


def from_host(dev, x, cfg, gpu_labels, gpu_scores):
    """The same training and assignment with x handed over in host memory
    (emh_train: staged upload of the 614 MB, then the device loop; emh_assign:
    chunks staged and copied in while the previous chunk runs). Not the value:
    the PCIe-inclusive times, best of two, after the timed steps."""
    from emeans_amd import Emeans

    n = x.shape[0]
    best_t = best_a = float("inf")
    same = True
    for _ in range(2):
        m = Emeans(cfg, dev)
        t0 = time.perf_counter()
        m.train(x)
        t1 = time.perf_counter()
        a = m.assign(x)
        t2 = time.perf_counter()
        best_t, best_a = min(best_t, t1 - t0), min(best_a, t2 - t1)
        same &= bool(np.array_equal(a.labels, gpu_labels)) and a.scores.tobytes() == gpu_scores.tobytes()
    return {"train_s": best_t, "assign_s": best_a, "assign_mrows_s": n / best_a / 1e6,
            "bytes_in": int(x.nbytes), "equal_to_device_path": same}


def cpu_baseline(x, cfg, gpu_cent, info, gpu_labels, gpu_scores, args):
    """The oracle (the C++ restatement of the reference CPU backend, OpenMP)
    on the same training and assignment: the median of `--cpu-runs` runs."""
    from oracle import oracle as O

    if args.cpu_threads:
        O.set_threads(args.cpu_threads)
    threads = O.get_threads()
    n, d, k = x.shape[0], cfg.d, cfg.k
    runs = []
    for _ in range(max(1, args.cpu_runs)):
        t0 = time.perf_counter()
        o = O.train(x, d, k, seed=cfg.seed)
        t1 = time.perf_counter()
        ol, osc = O.assign(x, d, o["centroids"], "l2")
        t2 = time.perf_counter()
        runs.append((t2 - t0, t1 - t0, t2 - t1))
    runs.sort()
    cpu_s, train_s, assign_s = runs[len(runs) // 2]
    epochs = len(o["obj"])
    base = {
        "value": (epochs * n + n) / cpu_s / 1e6,
        "unit": "Mrows/s",
        "cores": threads,
        "kind": "port",
        "sample": "the full workload: training (5 epochs) + assignment of all 200,000 rows; "
                  f"median of {len(runs)} runs",
        "train_s": train_s,
        "assign_s": assign_s,
        "runs_s": [r[0] for r in runs],
        "threads": threads,
        "host": host_cpu(),
    }
    parity = {
        "centroids_bit_equal": bool(gpu_cent.tobytes() == o["centroids"].tobytes()),
        "positions_bit_equal": bool(info["positions"].tobytes() == o["positions"].tobytes()),
        "last_pass_labels_equal": bool(np.array_equal(info["labels"], o["labels"])),
        "objectives_equal": [s.obj for s in info["stats"]] == o["obj"].tolist(),
        "nsplit": [s.nsplit for s in info["stats"]],
        "assign_labels_equal": bool(np.array_equal(gpu_labels, ol)),
        "assign_scores_bit_equal": bool(gpu_scores.tobytes() == osc.tobytes()),
        "final_objective": O.mean_objective(osc, False),
    }
    return base, parity


def other_workloads(args):
    """Assign-only at scale (2,000,000 x 1024 unit queries vs 16,384 unit
    centroids, IP, seed 1) and exact kNN (knn_self k = 10 on 500,000 x 384 unit
    rows with 5% near-duplicates, seed 2), both at full size on data drawn on
    the host (emeans_amd.synth) and resident: `--other-steps` timed runs
    each after one warmup, the screen timed with HIP events on every launch,
    and the oracle on a sample of the queries (bit-exact labels, scores, ids
    and sims) as the CPU baseline."""
    from emeans_amd import HipDevice, synth
    from oracle import oracle as O

    dev = HipDevice()
    res = {}
    # --- assign 2M x 1024 vs 16,384, IP
    n, d, k = 2_000_000, 1024, 16_384
    t = time.time()
    q, c = synth.assign_at_scale(n, d, k, seed=1)
    log(f"assign data: {n} x {d} and {k} centroids generated in {time.time() - t:.1f} s")
    qb, cb = dev.bind(q), dev.upload_f32(c)
    labels, scores = dev.zeros_u32(n), dev.zeros_f32(n)
    dev.assign_dev(qb, n, d, cb, k, "ip", labels, scores)
    dev.sync()
    dev.profile(1)
    t0 = time.perf_counter()
    for _ in range(args.other_steps):
        dev.assign_dev(qb, n, d, cb, k, "ip", labels, scores)
    dev.sync()
    step_s = (time.perf_counter() - t0) / args.other_steps
    dev.profile(0)
    ms, launches, flop = dev.profile_read("screen")
    gl, gs = dev.read_u32(labels), dev.read_f32(scores)
    g = np.random.default_rng(0)
    sample = np.sort(g.choice(n, size=args.assign_sample, replace=False))
    t0 = time.perf_counter()
    ol, osc = O.assign(q[sample], d, c, "ip")
    cpu_s = time.perf_counter() - t0
    res["assign_2Mx1024_k16384_ip"] = {
        "value": n / step_s / 1e6, "unit": "Mrows/s", "ms_per_run": step_s * 1e3,
        "steps": args.other_steps,
        "roofline": screen_roofline(ms, launches, flop, "k_screen3 (sorted-insert lists)"),
        "cpu_baseline": {"value": len(sample) / cpu_s / 1e6, "unit": "Mrows/s",
                         "cores": O.get_threads(), "kind": "port",
                         "sample": f"{len(sample)} of the {n} queries against all {k} centroids"},
        "parity": {"labels_equal": bool(np.array_equal(gl[sample], ol)),
                   "scores_bit_equal": gs[sample].tobytes() == osc.tobytes()}}
    log(f"assign 2M: {step_s * 1e3:.1f} ms per run")
    del qb, cb, labels, scores, q, c
    # --- knn_self k = 10 on 500k x 384
    n, d, kk = 500_000, 384, 10
    t = time.time()
    xh, dst, src = synth.knn_near_duplicates(n, d, seed=2)
    log(f"knn data: {n} x {d} generated in {time.time() - t:.1f} s")
    xb = dev.bind(xh)
    ids, sims = dev.zeros_u32(n * kk), dev.zeros_f32(n * kk)
    dev.topk_dev(xb, n, xb, n, d, kk, True, ids, sims)
    dev.sync()
    dev.profile(1)
    t0 = time.perf_counter()
    for _ in range(args.other_steps):
        dev.topk_dev(xb, n, xb, n, d, kk, True, ids, sims)
    dev.sync()
    step_s = (time.perf_counter() - t0) / args.other_steps
    dev.profile(0)
    ms, launches, flop = dev.profile_read("screen")
    gi, gsm = dev.read_u32(ids).reshape(n, kk), dev.read_f32(sims).reshape(n, kk)
    sample = np.sort(g.choice(n, size=args.knn_sample, replace=False))
    t0 = time.perf_counter()
    oi, osm = O.knn(xh[sample], xh, d, kk + 1, False)
    cpu_s = time.perf_counter() - t0
    oi, osm = oi.reshape(-1, kk + 1), osm.reshape(-1, kk + 1)
    # exclude_self on the sample: the oracle searched kk + 1 among all rows; drop the query itself
    wi, ws = np.empty((len(sample), kk), np.uint32), np.empty((len(sample), kk), np.float32)
    for r, qi in enumerate(sample):
        keep = oi[r] != qi
        wi[r], ws[r] = oi[r][keep][:kk], osm[r][keep][:kk]
    recall = float(np.mean((gi[dst] == src[:, None]).any(axis=1)))
    res["knn_self_500kx384_k10"] = {
        "value": 2.0 * n * n * d / step_s / 1e12, "unit": "TFLOP/s", "ms_per_run": step_s * 1e3,
        "steps": args.other_steps,
        "roofline": screen_roofline(ms, launches, flop,
                                    "k_screen4kn (kNN over rows split once, 24-entry lists)"),
        "cpu_baseline": {"value": 2.0 * len(sample) * n * d / cpu_s / 1e12, "unit": "TFLOP/s",
                         "cores": O.get_threads(), "kind": "port",
                         "sample": f"{len(sample)} queries against all {n} rows"},
        "parity": {"ids_equal": bool(np.array_equal(gi[sample], wi)),
                   "sims_bit_equal": gsm[sample].tobytes() == ws.tobytes()},
        "duplicates_found_as_a_neighbour": recall}
    log(f"knn 500k: {step_s * 1e3:.1f} ms per run")
    dev.close()
    if not args.no_autok:
        res["auto_cluster_900k_add_100k"] = autok_run(args)
    return res


def knn_workload(args):
    """Exact kNN (knn_self, k = 10) on 500,000 x 384 unit rows with 5% injected
    near-duplicates (seed 2): one step = the whole all-pairs top-10, data
    resident. The CPU baseline and parity run on a sample of the queries."""
    from emeans_amd import HipDevice, synth

    n, d, kk = args.knn_n, 384, 10
    t = time.time()
    x, _, _ = synth.knn_near_duplicates(n=n, d=d, seed=2)
    log(f"data: {n} x {d} generated in {time.time() - t:.1f} s")
    dev = HipDevice()
    xb = dev.bind(x)
    ids, sims = dev.zeros_u32(n * kk), dev.zeros_f32(n * kk)
    for _ in range(args.warmup):
        dev.topk_dev(xb, n, xb, n, d, kk, True, ids, sims)
    dev.sync()
    dev.profile(True)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        dev.topk_dev(xb, n, xb, n, d, kk, True, ids, sims)
    dev.sync()
    step_s = (time.perf_counter() - t0) / args.steps
    dev.profile(False)
    ms, launches, flop = dev.profile_read()
    gi, gs = dev.read_u32(ids).reshape(n, kk), dev.read_f32(sims).reshape(n, kk)
    out = {"metric": "knn_self top-10 TFLOP/s at 500k x 384 FP32", "value": 2.0 * n * n * d / step_s / 1e12,
           "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": step_s * 1e3, "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "f32", "data": "synthetic",
           "config": {"workload": f"knn_self k=10 {n}x{d} unit rows, 5% near-duplicates, seed 2"},
           "roofline": screen_roofline(ms, launches, flop,
                                       "k_screen4kn (kNN over rows split once, bf16 three-pass "
                                       "MFMA, 24-entry lists)")}
    if not args.no_cpu:
        from oracle import oracle as O
        g = np.random.default_rng(0)
        sample = np.sort(g.choice(n, size=args.sample, replace=False))
        t0 = time.perf_counter()
        oi, osm = O.knn(x[sample], x, d, kk, False)
        cpu_s = time.perf_counter() - t0
        oi, osm = oi.reshape(-1, kk).copy(), osm.reshape(-1, kk).copy()
        for r, q in enumerate(sample):  # exclude_self on the sample: drop q itself
            keep = oi[r] != q
            oi[r, :keep.sum()], osm[r, :keep.sum()] = oi[r][keep], osm[r][keep]
        # the oracle ran with kk neighbours including self; compare the first kk-1
        m = kk - 1
        out["cpu_baseline"] = {"value": 2.0 * len(sample) * n * d / cpu_s / 1e12, "unit": "TFLOP/s",
                               "cores": O.get_threads(), "kind": "port",
                               "sample": f"{len(sample)} queries against all {n} rows"}
        out["parity"] = {"ids_equal_first_9": bool(np.array_equal(gi[sample, :m], oi[:, :m])),
                         "sims_bit_equal_first_9": gs[sample, :m].tobytes() == osm[:, :m].tobytes()}
    return out


def assign_workload(args):
    """Assign-only at scale: 2,000,000 x 1024 unit queries against 16,384 unit
    centroids, inner product (seed 1); data resident, labels and scores per row."""
    from emeans_amd import HipDevice, synth

    n, d, k = args.assign_n, 1024, 16384
    t = time.time()
    q, c = synth.assign_at_scale(n=n, d=d, k=k, seed=1)
    log(f"data: {n} x {d} and {k} centroids generated in {time.time() - t:.1f} s")
    dev = HipDevice()
    qb, cb = dev.bind(q), dev.upload_f32(c)
    labels, scores = dev.zeros_u32(n), dev.zeros_f32(n)
    for _ in range(args.warmup):
        dev.assign_dev(qb, n, d, cb, k, "ip", labels, scores)
    dev.sync()
    dev.profile(True)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        dev.assign_dev(qb, n, d, cb, k, "ip", labels, scores)
    dev.sync()
    step_s = (time.perf_counter() - t0) / args.steps
    dev.profile(False)
    ms, launches, flop = dev.profile_read()
    out = {"metric": "assign Mrows/s at 2M x 1024 vs k=16384 IP FP32", "value": n / step_s / 1e6,
           "unit": "Mrows/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": step_s * 1e3, "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "f32", "data": "synthetic",
           "config": {"workload": f"assign {n}x{d} vs {k} centroids, IP, unit rows, seed 1"},
           "tflops": 2.0 * n * k * d / step_s / 1e12,
           "roofline": screen_roofline(ms, launches, flop, "k_screen (bf16 three-pass MFMA x.C^T + per-row 5-entry candidate lists)")}
    if not args.no_host:
        # The same assignment from host arrays (8.2 GB of queries staged in
        # while earlier chunks run): the PCIe-inclusive rate, not the value.
        t0 = time.perf_counter()
        hl, hs = dev.assign(q, d, c, "ip")
        host_s = time.perf_counter() - t0
        out["from_host"] = {"assign_s": host_s, "assign_mrows_s": n / host_s / 1e6,
                            "bytes_in": int(q.nbytes + c.nbytes),
                            "equal_to_device_path": bool(np.array_equal(hl, dev.read_u32(labels)))
                            and hs.tobytes() == dev.read_f32(scores).tobytes()}
    if not args.no_cpu:
        from oracle import oracle as O
        gl, gsc = dev.read_u32(labels), dev.read_f32(scores)
        g = np.random.default_rng(0)
        sample = np.sort(g.choice(n, size=args.sample, replace=False))
        t0 = time.perf_counter()
        ol, osc = O.assign(q[sample], d, c, "ip")
        cpu_s = time.perf_counter() - t0
        out["cpu_baseline"] = {"value": len(sample) / cpu_s / 1e6, "unit": "Mrows/s",
                               "cores": O.get_threads(), "kind": "port",
                               "sample": f"{len(sample)} of the {n} queries against all {k} centroids"}
        out["parity"] = {"labels_equal": bool(np.array_equal(gl[sample], ol)),
                         "scores_bit_equal": gsc[sample].tobytes() == osc.tobytes()}
    return out


def ops_bench(reps=5, n=200_000, d=768, k=1024, b=16_384):
    """Each Device op on one training batch, the reference's ops_bench pattern
    (bench/src/bin/ops_bench.rs:23-167): unit rows from 500 blobs (sigma 0.5,
    seed 5), one warm-up, then the median of `reps` calls, each followed by a
    one-element read that waits for the device (so a time includes one round
    trip, which "sync" alone measures). Milliseconds per call."""
    from emeans_amd import EmaStep, HipDevice, Mat, Select, synth

    x, _ = synth.blobs_spherical(n=n, d=d, k=500, sigma=0.5, seed=5)
    dev = HipDevice()
    xb = dev.bind(x)
    perm = ((np.arange(n, dtype=np.uint64) * 7919 + 1) % n).astype(np.uint32)
    ids = dev.upload_u32(perm)
    c = dev.upload_f32(x[:k])
    unit, cn = dev.zeros_f32(k * d), dev.zeros_f32(k)
    lab, sco = dev.zeros_u32(n), dev.zeros_f32(n)
    sums, counts, pas = dev.zeros_f32(k * d), dev.zeros_u32(k), dev.zeros_f32(k * d)
    pos, usage = dev.upload_f32(x[:k]), dev.upload_f32(np.ones(k, np.float32))
    probe = dev.zeros_u32(1)
    kq, kk = 2048, 10
    knn_ids, knn_sims = dev.zeros_u32(kq * kk), dev.zeros_f32(kq * kk)
    plan = [(j, k - 1 - j) for j in range(16)]
    out = {}

    def time_op(name, f):
        f()
        dev.read_u32(probe, (0, 1))
        t = []
        for _ in range(reps):
            s = time.perf_counter()
            f()
            dev.read_u32(probe, (0, 1))
            t.append((time.perf_counter() - s) * 1e3)
        out[name] = float(np.median(t))

    time_op("sync", lambda: None)
    time_op("normalize_rows", lambda: dev.normalize_rows(c, k, d, unit))
    time_op("row_norms", lambda: dev.row_norms(c, k, d, cn))
    time_op("top1", lambda: dev.top1(Mat(xb, d), Select(ids, (0, b)), unit, None, k, "ip", lab,
                                     sco))
    time_op("top1_dense", lambda: dev.top1(Mat(xb, d), Select(None, (0, b)), unit, None, k, "ip",
                                           lab, sco))
    time_op("top1_l2", lambda: dev.top1(Mat(xb, d), Select(ids, (0, b)), c, cn, k, "l2", lab,
                                        sco))
    time_op("scatter_add", lambda: dev.scatter_add(Mat(xb, d), Select(ids, (0, b)), lab, k, sums,
                                                   counts, pas))
    time_op("ema_update", lambda: dev.ema_update(pos, usage, sums, counts, k, d,
                                                 EmaStep.new(0.3)))
    time_op("split", lambda: dev.split(pos, usage, plan, d))
    time_op(f"topk_{kq}x{n}_k{kk}", lambda: dev.topk_dev(xb, kq, xb, n, d, kk, False, knn_ids,
                                                         knn_sims))
    time_op("read_usage", lambda: dev.read_f32(usage, (0, k)))
    time_op("read_pos", lambda: dev.read_f32(pos, (0, k * d)))
    dev.close()
    log("ops_bench (ms, median of %d, synced): " % reps
        + ", ".join(f"{kk_} {v:.3f}" for kk_, v in out.items()))
    return {"unit": "ms per call (median, one device round trip included)", "reps": reps,
            "n": n, "d": d, "k": k, "batch": b, "ops": out}


def ops_workload(args):
    """The per-op table alone (`--workload ops`)."""
    return ops_bench(reps=max(args.steps, 5))


def autok_workload(args):
    """C5 alone (`--workload autok`): the autok leg of the headline run."""
    return autok_run(args)


def autok_run(args):
    """C5 (two-level auto_cluster plus incremental add on 1,000,000 x 768
    nested unit rows, 64 Zipf(1.3) top groups of 16 sub-groups, seed 3):
    auto_cluster of the first 900,000 rows with the reference's defaults
    (auto.rs:1001-1101: the level-1 sweep k = 2..40 with four k-means++
    restarts each, a level-2 sweep per group, resplits, refine, average
    linkage and the cut, the hierarchy's labels and floors), then
    Hierarchy::add of the last 100,000 rows (incremental.rs:306-596: 11 % new
    rows call for the EMA update). The sweeps' trainings, assignments,
    seedings and internal scores run on the device, the data bound on one
    context (each sweep's restarts at once on four). `value`: spherical
    e-means fits per second of auto_cluster's wall time. CPU baseline: the
    oracle's fit at k = 21 on the same rows. Parity: the same sequence on a
    reduced C5 set (8,000 rows of the same generator with 8 x 4 groups;
    k1 in 2..4, k2 <= 4, leaves above 100 rows split again, so that every
    stage runs) over the device and over the oracle, compared whole."""
    from emeans_amd import HipDevice, auto, autocluster, synth
    from emeans_amd import hierarchy as H
    from oracle import oracle as O

    n_all, n, d = args.autok_n, args.autok_n * 9 // 10, 768
    t = time.time()
    x_all, _ = synth.nested(n=n_all, d=d, seed=3)
    x = x_all[:n]
    log(f"autok data: {n_all} x {d} generated in {time.time() - t:.1f} s")
    dev = HipDevice()
    cfg = auto.AutoConfig(restarts=args.autok_restarts, seed=3, verbose=True)
    dev.contexts(min(cfg.restarts, auto.MAX_CONTEXTS))  # before the warm-up fit's copy stream
    xb = dev.bind(x)
    auto.fit(dev, x, xb, 8, 1.0, 1, None)  # warm the kernels up
    dev.sync()
    tm = {}
    t0 = time.perf_counter()
    h, labels = autocluster.auto_cluster(dev, x, cfg, H.IncrementalConfig(grow_min_size=0),
                                         timing=tm)
    dev.sync()
    ac_s = time.perf_counter() - t0
    k1, k2 = h.chosen_k()
    dg = h.diagnostics
    log(f"autok: auto_cluster {ac_s:.1f} s ({tm['fits']} sweep fits), k1 = {k1}, "
        f"{sum(k2)} leaves, {dg.resplits} resplits; stages "
        + ", ".join(f"{kk[:-2]} {v:.1f} s" for kk, v in tm.items() if kk.endswith("_s")))
    t0 = time.perf_counter()
    rep = h.add(x_all, n)
    add_s = time.perf_counter() - t0
    log(f"autok: add of {n_all - n} rows: {rep.action}, {add_s:.2f} s, "
        f"{rep.new_outliers} new outliers")
    # CPU baseline: the oracle's fit (train_from k-means++ rows + assign) at k = 21.
    kc = 21
    init = x[dev.kmeans_pp(xb, n, d, kc, 7)]
    c0 = time.perf_counter()
    o = O.train(x, d, kc, spherical=True, seed=7, init=init)
    O.assign(x, d, o["centroids"], "ip")
    cpu_fit_s = time.perf_counter() - c0
    rep_action, rep_outliers = rep.action, rep.new_outliers
    best1 = max(dg.level1, key=lambda s: s.silhouette) if dg.level1 else None
    del h, labels, rep, xb, x, x_all
    parity = autok_parity(dev)
    dev.close()
    return {"value": tm["fits"] / ac_s, "unit": "fits/s", "rows": n, "added_rows": n_all - n,
            "auto_cluster_s": ac_s,
            "sweep_fits": tm["fits"], "ms_per_fit": tm["fit_s"] / max(tm["fits"], 1) * 1e3,
            "kmeans_pp_s": tm["kmeans_pp_s"], "internal_scores_s": tm["scores_s"],
            "stages_s": {kk[:-2]: v for kk, v in tm.items()
                         if kk.endswith("_s") and kk not in ("fit_s", "kmeans_pp_s", "scores_s")},
            "k1": k1, "leaves": sum(k2), "resplits": dg.resplits, "flat": dg.flat,
            "level1_cuts_scored": len(dg.level1),
            "level1_best_silhouette": None if best1 is None else
            {"k": best1.k, "silhouette": best1.silhouette},
            "add": {"rows": n_all - n, "action": rep_action, "seconds": add_s,
                    "new_outliers": rep_outliers},
            "cpu_baseline": {"value": 1.0 / cpu_fit_s, "unit": "fits/s", "cores": O.get_threads(),
                             "kind": "port", "fit_s": cpu_fit_s,
                             "sample": f"one fit (k = {kc}: train_from k-means++ rows, 5 epochs, "
                                       f"then assign) on the same {n} rows"},
            "parity": parity}


def autok_parity(dev):
    """auto_cluster then Hierarchy::add on a reduced C5 set, on the device and
    over the oracle (tests/oracle_device.py): sweeps, resplits, leaves, the
    cut, labels, the hierarchy and its file, the add's labels."""
    from emeans_amd import auto, autocluster, synth
    from tests.oracle_device import OracleDevice

    x, _ = synth.nested(n=8000, d=768, top=8, sub=4, seed=3)
    cfg = auto.AutoConfig(k1_range=(2, 4), k2_max=4, max_cluster_size=100, restarts=2)
    out = {}
    hs = []
    for name, dv in (("device", dev), ("oracle", OracleDevice(dev.name()))):
        t = time.perf_counter()
        h, lab = autocluster.auto_cluster(dv, x[:7200], cfg)
        rep = h.add(x, 7200)
        out[f"{name}_s"] = time.perf_counter() - t
        hs.append((h, lab, rep))
    (hg, lg, rg), (ho, lo, ro) = hs
    same = lambda a, b: all(np.asarray(getattr(a, f)).tobytes() == np.asarray(getattr(b, f)).tobytes()
                            for f in ("l1", "l2", "sim1", "sim", "outlier", "slot1", "slot2"))
    ho.diagnostics = hg.diagnostics  # wall-clock seconds aside, compared below
    for a, b in zip([hg.level1] + [g.model for g in hg.groups],
                    [ho.level1] + [g.model for g in ho.groups]):
        if a is not None and b is not None:
            b.stats = [(s[0], t[1], s[2], s[3]) for s, t in zip(b.stats, a.stats)]
    out.update({"rows": 7200, "added": 800, "resplits": hg.diagnostics.resplits,
                "leaves": sum(hg.chosen_k()[1]), "chosen_k_equal": hg.chosen_k() == ho.chosen_k(),
                "add_action_equal": rg.action == ro.action,
                "labels_equal": same(rg.labels, ro.labels),
                "hierarchy_file_equal": hg.to_bytes() == ho.to_bytes()})
    log(f"autok parity (reduced C5, device vs oracle): {out}")
    return out


def copy_probe(mib):
    """A plain device-to-device copy of `mib` MiB, three times: the known-size
    kernel that calibrates the HBM byte counters (FETCH_SIZE, WRITE_SIZE)."""
    import torch

    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copy probe: 3 copies of {mib} MiB ({n * 4} bytes each)")


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline and parity")
    ap.add_argument("--no-f32", action="store_true",
                    help="skip the headline's comparison run with the f32 MFMA screen")
    ap.add_argument("--no-host", action="store_true",
                    help="skip the runs from host arrays (PCIe-inclusive times)")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--cpu-runs", type=int, default=3, help="CPU baseline runs (median)")
    ap.add_argument("--no-others", action="store_true",
                    help="skip the assign-at-scale and kNN lines of the headline run")
    ap.add_argument("--other-steps", type=int, default=3)
    ap.add_argument("--assign-sample", type=int, default=2000,
                    help="queries the oracle checks at 2M x 1024 (the CPU baseline sample)")
    ap.add_argument("--knn-sample", type=int, default=200,
                    help="queries the oracle checks at 500k x 384 (the CPU baseline sample)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="first run a plain device copy of MIB MiB (HBM counter calibration)")
    ap.add_argument("--autok-restarts", type=int, default=4)
    ap.add_argument("--autok-n", type=int, default=1_000_000,
                    help="C5 rows (auto_cluster on 90 %%, then the add of the rest)")
    ap.add_argument("--no-autok", action="store_true",
                    help="skip the C5 leg of the headline run's other workloads")
    ap.add_argument("--workload", choices=["headline", "knn", "assign", "autok", "ops"],
                    default="headline",
                    help="headline: train + assign 200k x 768 (the metric); knn: knn_self "
                         "500k x 384; assign: 2M x 1024 vs k = 16384")
    ap.add_argument("--knn-n", type=int, default=500_000)
    ap.add_argument("--assign-n", type=int, default=2_000_000)
    ap.add_argument("--sample", type=int, default=200, help="queries in the CPU baseline sample")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this backend runs on one GPU; --gpus {args.gpus} "
              f"(WORLD_SIZE {world}) is not supported", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1:
        sys.exit("--steps must be >= 1")
    if args.copy_probe:
        copy_probe(args.copy_probe)
    out = {"headline": headline, "knn": knn_workload, "assign": assign_workload,
           "autok": autok_workload, "ops": ops_workload}[args.workload](args)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
