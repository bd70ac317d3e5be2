"""ctypes face of the oracle library (liboracle.so).

TEST INFRASTRUCTURE ONLY: the CPU restatement of the reference's float order
that the HIP backend is checked against, and the CPU baseline the benchmark
reports beside it. The product package never imports this module.
"""

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(_HERE, "liboracle.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _load():
    if not os.path.exists(_LIB):
        build()
    lib = C.CDLL(_LIB)
    u64, i32, u32, f64, vp = C.c_uint64, C.c_int, C.c_uint32, C.c_double, C.c_void_p
    sig = {
        "orc_rng_new": (vp, [u32]),
        "orc_rng_free": (None, [vp]),
        "orc_rng_random_sample": (f64, [vp]),
        "orc_rng_permutation": (None, [vp, u64, _u32p]),
        "orc_resolve_batch_and_step": (None, [u64, u64, f64, i32, u64, i32, f64,
                                              C.POINTER(u64), C.POINTER(f64)]),
        "orc_resolve_law": (i32, [i32, u64]),
        "orc_epoch_rows": (u64, [u64, f64, np.ctypeslib.ndpointer(np.uint64), u64]),
        "orc_scheduled_alpha": (f64, [f64, u64, u64]),
        "orc_epoch_seed": (u32, [u32, u64]),
        "orc_unused_threshold": (f64, [u64]),
        "orc_numpy_sum_f32": (C.c_float, [_f32p, u64]),
        "orc_top1": (None, [_f32p, u64, vp, u64, u64, _f32p, u64, i32, _u32p, _f32p]),
        "orc_row_norms": (None, [_f32p, u64, u64, _f32p]),
        "orc_normalize_rows": (None, [_f32p, u64, u64, _f32p]),
        "orc_scatter_add": (None, [_f32p, u64, vp, u64, u64, _u32p, u64, _f32p, _u32p, vp]),
        "orc_ema_update": (None, [_f32p, _f32p, _f32p, _u32p, u64, u64, f64]),
        "orc_apply_splits": (None, [_f32p, _f32p, u64, _u32p, u64]),
        "orc_plan_revival": (u64, [_f32p, u64, f64, vp, _u32p]),
        "orc_closing_means": (None, [_f32p, _f32p, _f64p, u64, u64, i32, _f32p]),
        "orc_knn": (None, [_f32p, u64, _f32p, u64, u64, u64, i32, _u32p, _f32p]),
        "orc_set_threads": (None, [i32]),
        "orc_get_threads": (i32, []),
        "orc_train": (i32, [_f32p, u64, vp, vp]),
        "orc_train_from": (i32, [_f32p, u64, vp, vp, vp, vp, vp]),
        "orc_kmeans_pp": (u64, [_f32p, u64, u64, u64, u32, _u32p]),
        "orc_dots": (None, [_f32p, u64, _f32p, u64, u64, _f32p]),
        "orc_internal_scores": (i32, [_f32p, u64, u64, _u32p, u64, _f64p,
                                      np.ctypeslib.ndpointer(np.uint64), C.POINTER(u64)]),
        "orc_dedup": (u64, [_f32p, u64, u64, _u32p, _f32p, u64, C.c_float, C.c_float, i32, f64,
                            vp, vp, vp, _u32p, _u32p, _u32p, _u32p, C.POINTER(u64),
                            C.POINTER(u64)]),
        "orc_contract_mixture": (None, [u64, u64, u64, f64, i32, u32, _f32p]),
        "orc_common_mixture": (None, [u64, u64, u64, C.c_float, i32, u32, _f32p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ------------------------------------------------------------------ MT19937
class RandomState:
    """numpy legacy RandomState (reference rng.rs)."""

    def __init__(self, seed):
        self._h = lib.orc_rng_new(seed & 0xFFFFFFFF)

    def __del__(self):
        if getattr(self, "_h", None):
            lib.orc_rng_free(self._h)
            self._h = None

    def random_sample(self):
        return lib.orc_rng_random_sample(self._h)

    def permutation(self, n):
        out = np.empty(n, np.uint32)
        lib.orc_rng_permutation(self._h, n, out)
        return out


# ------------------------------------------------------------------- recipe
LAWS = {"auto": 0, "throughput": 1, "quality": 2}
LAW_NAMES = {v: k for k, v in LAWS.items()}


def resolve_law(law, d):
    return LAW_NAMES[lib.orc_resolve_law(LAWS[law], d)]


def resolve_batch_and_step(n, k, nepochs, law, batch_size=None, alpha0=None):
    b, a = C.c_uint64(), C.c_double()
    lib.orc_resolve_batch_and_step(n, k, float(nepochs), LAWS[law], batch_size or 0,
                                   int(alpha0 is not None), float(alpha0 or 0.0),
                                   C.byref(b), C.byref(a))
    return b.value, a.value


def epoch_rows(n, nepochs):
    out = np.zeros(64, np.uint64)
    m = lib.orc_epoch_rows(n, float(nepochs), out, 64)
    return [int(v) for v in out[:m]]


def scheduled_alpha(alpha0, step, total):
    return lib.orc_scheduled_alpha(alpha0, step, total)


def epoch_seed(seed, epoch):
    return lib.orc_epoch_seed(seed, epoch)


def unused_threshold(d):
    return lib.orc_unused_threshold(d)


def numpy_sum_f32(a):
    a = np.ascontiguousarray(a, np.float32)
    return np.float32(lib.orc_numpy_sum_f32(a, a.size))


# ------------------------------------------------------------------ layer 1
def top1(x, d, centroids, metric, ids=None, rows=None, labels=None, scores=None):
    """Fused top-1 in the cpu-fused order. Outputs written at selection positions."""
    x = np.ascontiguousarray(x, np.float32)
    c = np.ascontiguousarray(centroids, np.float32)
    n_sel = len(ids) if ids is not None else x.size // d
    lo, hi = rows if rows is not None else (0, n_sel)
    if labels is None:
        labels = np.zeros(n_sel, np.uint32)
    if scores is None:
        scores = np.zeros(n_sel, np.float32)
    ids_a = None if ids is None else np.ascontiguousarray(ids, np.uint32)
    lib.orc_top1(x, d, _ptr(ids_a), lo, hi, c, c.size // d, int(metric == "ip"), labels, scores)
    return labels, scores


def row_norms(m, rows, d):
    m = np.ascontiguousarray(m, np.float32)
    out = np.zeros(rows, np.float32)
    lib.orc_row_norms(m, rows, d, out)
    return out


def normalize_rows(m, rows, d):
    m = np.ascontiguousarray(m, np.float32)
    out = np.zeros(rows * d, np.float32)
    lib.orc_normalize_rows(m, rows, d, out)
    return out


def scatter_add(x, d, labels, k, ids=None, rows=None, acc=None):
    x = np.ascontiguousarray(x, np.float32)
    n_sel = len(ids) if ids is not None else x.size // d
    lo, hi = rows if rows is not None else (0, n_sel)
    sums = np.zeros(k * d, np.float32)
    counts = np.zeros(k, np.uint32)
    ids_a = None if ids is None else np.ascontiguousarray(ids, np.uint32)
    lab = np.ascontiguousarray(labels, np.uint32)
    lib.orc_scatter_add(x, d, _ptr(ids_a), lo, hi, lab, k, sums, counts, _ptr(acc))
    return sums, counts


def ema_update(pos, usage, sums, counts, k, d, alpha):
    """In place on pos/usage (float32 arrays); EmaStep::new(alpha) semantics."""
    lib.orc_ema_update(pos, usage, np.ascontiguousarray(sums, np.float32),
                       np.ascontiguousarray(counts, np.uint32), k, d, float(alpha))


def apply_splits(pos, usage, d, plan):
    pairs = np.ascontiguousarray(np.asarray(plan, np.uint32).reshape(-1))
    lib.orc_apply_splits(pos, usage, d, pairs, len(plan))


def plan_revival(usage, tau, rng):
    usage = np.ascontiguousarray(usage, np.float32)
    out = np.zeros(2 * usage.size, np.uint32)
    m = lib.orc_plan_revival(usage, usage.size, float(tau), rng._h, out)
    return [(int(out[2 * i]), int(out[2 * i + 1])) for i in range(m)]


def closing_means(positions, sums, counts, k, d, spherical):
    out = np.zeros(k * d, np.float32)
    lib.orc_closing_means(np.ascontiguousarray(positions, np.float32),
                          np.ascontiguousarray(sums, np.float32),
                          np.ascontiguousarray(counts, np.float64), k, d, int(spherical), out)
    return out


def knn(queries, data, d, kk, exclude_self):
    q = np.ascontiguousarray(queries, np.float32)
    x = np.ascontiguousarray(data, np.float32)
    m, n = q.size // d, x.size // d
    ids = np.zeros(m * kk, np.uint32)
    sims = np.zeros(m * kk, np.float32)
    lib.orc_knn(q, m, x, n, d, kk, int(exclude_self), ids, sims)
    return ids, sims


def set_threads(t):
    lib.orc_set_threads(int(t))


def get_threads():
    return lib.orc_get_threads()


# -------------------------------------------------------------------- train
class _Cfg(C.Structure):
    _fields_ = [("k", C.c_uint64), ("d", C.c_uint64), ("nepochs", C.c_double),
                ("batch_size", C.c_uint64), ("has_alpha0", C.c_int), ("alpha0", C.c_double),
                ("batch_law", C.c_int), ("seed", C.c_uint32), ("spherical", C.c_int),
                ("has_unused_threshold", C.c_int), ("unused_threshold", C.c_double),
                ("assignment_chunk_size", C.c_uint64)]


class _Out(C.Structure):
    _fields_ = [("centroids", C.c_void_p), ("positions", C.c_void_p), ("usage", C.c_void_p),
                ("labels", C.c_void_p), ("obj", C.c_void_p), ("imbalance", C.c_void_p),
                ("nsplit", C.c_void_p), ("n_epochs", C.c_uint64), ("n_splits", C.c_uint64),
                ("batch_size", C.c_uint64), ("alpha0", C.c_double), ("total_steps", C.c_uint64)]


def train(x, d, k, nepochs=5.0, batch_size=None, alpha0=None, batch_law="auto", seed=1234,
          spherical=False, unused_threshold=None, assignment_chunk_size=None, init=None,
          positions=None, usage=None):
    """Emeans::train on the CPU device loop (model.rs:700-811, core/train.rs:60-303);
    with init, train_from (model.rs:705-736); with positions and usage,
    train_resume (model.rs:739-749)."""
    x = np.ascontiguousarray(x, np.float32)
    n = x.size // d
    cfg = _Cfg(k, d, float(nepochs), batch_size or 0, int(alpha0 is not None),
               float(alpha0 or 0.0), LAWS[batch_law], seed & 0xFFFFFFFF, int(spherical),
               int(unused_threshold is not None), float(unused_threshold or 0.0),
               assignment_chunk_size or 0)
    cent = np.zeros(k * d, np.float32)
    pos = np.zeros(k * d, np.float32)
    us = np.zeros(k, np.float32)
    labels = np.zeros(n, np.int32)
    obj = np.zeros(64, np.float64)
    imb = np.zeros(64, np.float64)
    nsp = np.zeros(64, np.uint64)
    out = _Out(_ptr(cent), _ptr(pos), _ptr(us), _ptr(labels), _ptr(obj), _ptr(imb),
               _ptr(nsp), 0, 0, 0, 0.0, 0)
    keep = [None if v is None else np.ascontiguousarray(v, np.float32).reshape(-1)
            for v in (init, positions, usage)]
    rc = lib.orc_train_from(x, n, C.addressof(cfg), *[_ptr(v) for v in keep], C.addressof(out))
    if rc == 2:
        raise ValueError("oracle train: initial state not finite, or masses not finite and >= 0")
    if rc != 0:
        raise ValueError("oracle train: bad arguments")
    e = out.n_epochs
    return {
        "centroids": cent, "positions": pos, "usage": us, "labels": labels,
        "obj": obj[:e].copy(), "imbalance": imb[:e].copy(), "nsplit": nsp[:e].astype(int),
        "n_splits": out.n_splits, "batch_size": out.batch_size, "alpha0": out.alpha0,
        "total_steps": out.total_steps,
    }


def assign(x, d, centroids, metric):
    labels, scores = top1(x, d, centroids, metric)
    return labels, scores


def mean_objective(scores, spherical):
    """Assignment::mean_objective (model.rs:127-141), in f64."""
    s = np.asarray(scores, np.float32).astype(np.float64)
    v = 2.0 - 2.0 * s if spherical else s
    tot = 0.0
    for a in v:  # sequential f64 sum, the reference's iterator order
        tot += a
    return tot / max(len(v), 1)


# -------------------------------------------------------------------- dedup
def dedup(x, d, nb_ids, nb_sims, kk, sim_threshold, rep_threshold=None, priority=None,
          created_unix=None, max_gap_secs=None, burst=None):
    """dedup_with_neighbors (dedup.rs:186-358). burst: one id per row, negative
    (or None entries) for rows without one; created_unix: NaN = unknown."""
    x = np.ascontiguousarray(x, np.float32)
    n = x.size // d
    group_of = np.zeros(n, np.uint32)
    reps = np.zeros(n, np.uint32)
    anchors = np.zeros(n, np.uint32)
    sizes = np.zeros(n, np.uint32)
    lp, sc = C.c_uint64(), C.c_uint64()
    pr = None if priority is None else np.ascontiguousarray(priority, np.float32)
    tm = None if created_unix is None else np.ascontiguousarray(created_unix, np.float64)
    bu = None if burst is None else np.array([-1 if b is None else b for b in burst], np.int64)
    g = lib.orc_dedup(x, n, d, np.ascontiguousarray(nb_ids, np.uint32),
                      np.ascontiguousarray(nb_sims, np.float32), kk, float(sim_threshold),
                      float(sim_threshold if rep_threshold is None else rep_threshold),
                      int(max_gap_secs is not None), float(max_gap_secs or 0.0), _ptr(tm),
                      _ptr(bu), _ptr(pr), group_of, reps, anchors, sizes, C.byref(lp),
                      C.byref(sc))
    return {"group_of": group_of, "representatives": reps[:g], "anchors": anchors[:g],
            "sizes": sizes[:g], "linked_pairs": lp.value, "split_components": sc.value}


# ----------------------------------------------------------------- auto-k
def kmeans_pp(x, d, kmax, seed):
    """kmeans_pp (emeans-cluster/src/auto.rs:401-455): kmax row ids in pick order."""
    x = np.ascontiguousarray(x, np.float32)
    n = x.size // d
    picks = np.zeros(max(min(kmax, n), 1), np.uint32)
    m = lib.orc_kmeans_pp(x, n, d, kmax, seed & 0xFFFFFFFF, picks)
    return picks[:m]


def dots(a, b):
    """gemm_nt (emeans-core/src/assign.rs:813-825) as fma chains: (m x nb)."""
    a, b = np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32)
    m, nb, d = a.shape[0], b.shape[0], a.shape[1]
    out = np.zeros((m, nb), np.float32)
    if m and nb:
        lib.orc_dots(a, m, b, nb, d, out)
    return out


def internal_scores(x, d, labels, k):
    """internal_scores (emeans-cluster/src/metrics.rs:113-268), fma-chain dots."""
    x = np.ascontiguousarray(x, np.float32)
    n = x.size // d
    out = np.zeros(4, np.float64)
    sizes = np.zeros(k, np.uint64)
    ke = C.c_uint64()
    rc = lib.orc_internal_scores(x, n, d, np.ascontiguousarray(labels, np.uint32), k, out, sizes,
                                 C.byref(ke))
    if rc != 0:
        raise ValueError("label out of range")
    return {"k_eff": ke.value, "silhouette": out[0], "calinski_harabasz": out[1],
            "davies_bouldin": out[2], "objective": out[3], "sizes": sizes.astype(np.int64)}


# --------------------------------------------------------------- generators
def contract_mixture(n, d, centers, sigma, unit, seed):
    """core/contract.rs:40-60 test data (MT19937 Box-Muller)."""
    out = np.zeros(n * d, np.float32)
    lib.orc_contract_mixture(n, d, centers, float(sigma), int(unit), seed & 0xFFFFFFFF, out)
    return out


def common_mixture(n, d, centers, spread, spherical, seed):
    """tests/common/mod.rs:7-35 test data."""
    out = np.zeros(n * d, np.float32)
    lib.orc_common_mixture(n, d, centers, float(spread), int(spherical), seed & 0xFFFFFFFF, out)
    return out
