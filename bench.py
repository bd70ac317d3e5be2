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
reports train seconds, assignment Mrows/s, the MFMA screen kernel's roofline
and the CPU baseline. The screen (the dense x.C^T contraction ahead of the
exact f32 check) runs on the bf16 MFMA in three passes (x.c ~ xh.ch + xh.cl +
xl.ch); its roofline is the bf16 MFMA work it issues (3 x 2 rows k d FLOP per
launch over the HIP-event-timed duration of every 8th launch in the timed
steps) against the 2.5 PFLOP/s dense bf16 peak, with the f32-equivalent rate (2 rows k d FLOP per launch) against the
157.3 TFLOP/s dense f32 MFMA peak beside it. `f32_screen` repeats the step
with the screen on v_mfma_f32_32x32x2_f32 (same bits, checked). The CPU
baseline is the oracle's C++ restatement of the reference CPU backend
(cpu-fused float order) running the same training and assignment on this
host, with a bit-exact parity check.
"""

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

FP32_MFMA_PEAK = 157.3  # TFLOP/s, MI355X dense
BF16_MFMA_PEAK = 2500.0  # TFLOP/s, MI355X dense
HBM_PEAK = 8000.0       # GB/s
METRIC = "train s & assign Mrows/s at 200k×768 k=1024 FP32; % of FP32 MFMA peak"
# HBM bytes per k_screen launch over this workload's launch mix (calibrated
# FETCH_SIZE + WRITE_SIZE from two rocprofv3 --pmc passes of this script, with
# a plain copy kernel of known size as the scale;
# profiles/k_screen_train_assign_200kx768_k1024_hbm_traffic.md).
SCREEN_TRAFFIC_BYTES = 108.4e6
# The screen's roofline times every PROFILE_EVERY-th launch of the timed steps
# with HIP events (an event pair between two kernels costs the stream a few
# microseconds; on every launch that was ~5 % of the headline step).
PROFILE_EVERY = 8


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def screen_roofline(ms, launches, flop, kernel, traffic=None):
    """The bf16 screen's roofline: the MFMA work it issues (three bf16 products
    per multiply-add of the algorithmic 2 rows k d FLOP) over its HIP-event
    time, against the dense bf16 peak; the f32-equivalent rate beside it."""
    alg = flop / (ms * 1e-3) / 1e12 if ms > 0 else 0.0
    return {"bound": "mfma", "kernel": kernel, "achieved": 3.0 * alg, "peak": BF16_MFMA_PEAK,
            "unit": "TFLOP/s", "frac": 3.0 * alg / BF16_MFMA_PEAK, "traffic": traffic,
            "launches": launches, "avg_launch_ms": ms / max(launches, 1),
            "flop_per_launch": 3.0 * flop / max(launches, 1),
            "fp32_equivalent": {"achieved": alg, "peak": FP32_MFMA_PEAK, "frac": alg / FP32_MFMA_PEAK,
                                "flop_per_launch": flop / max(launches, 1)}}


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
        dev.profile(PROFILE_EVERY)
        trains, assigns = [], []
        t0 = time.perf_counter()
        for i in range(steps):
            tr, asg, cent, info = step()
            trains.append(tr)
            assigns.append(asg)
        dev.sync()
        t1 = time.perf_counter()
        dev.profile(False)
        ms, launches, flop = dev.profile_read()
        r = {"step_s": (t1 - t0) / steps, "train_s": float(np.median(trains)),
             "assign_s": float(np.median(assigns)), "ms": ms, "launches": launches, "flop": flop,
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
            "k_screen (bf16 MFMA, three passes xh.ch + xh.cl + xl.ch, f32 accumulation, "
            "+ per-row 5-entry candidate lists per centroid part)", SCREEN_TRAFFIC_BYTES),
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
    from oracle import oracle as O

    if args.cpu_threads:
        O.set_threads(args.cpu_threads)
    threads = O.get_threads()
    n, d, k = x.shape[0], cfg.d, cfg.k
    t0 = time.perf_counter()
    o = O.train(x, d, k, seed=cfg.seed)
    t1 = time.perf_counter()
    ol, osc = O.assign(x, d, o["centroids"], "l2")
    t2 = time.perf_counter()
    epochs = len(o["obj"])
    cpu_s = t2 - t0
    base = {
        "value": (epochs * n + n) / cpu_s / 1e6,
        "unit": "Mrows/s",
        "cores": threads,
        "kind": "port",
        "sample": "the full workload once: training (5 epochs) + assignment of all rows",
        "train_s": t1 - t0,
        "assign_s": t2 - t1,
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
           "roofline": screen_roofline(ms, launches, flop, "k_screen (kNN, bf16 three-pass MFMA, 24-entry lists)")}
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
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="first run a plain device copy of MIB MiB (HBM counter calibration)")
    ap.add_argument("--workload", choices=["headline", "knn", "assign"], default="headline",
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
    out = {"headline": headline, "knn": knn_workload, "assign": assign_workload}[args.workload](args)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
