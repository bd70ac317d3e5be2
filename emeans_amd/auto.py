"""The sweep pattern of automatic k (emeans-cluster/src/auto.rs) on the gfx950
backend: many spherical e-means models trained and scored on one context with
the data bound once.

  seed_for   auto.rs:343-349  the seed of each (salt, k, restart)
  fit        auto.rs:351-375  train_from k-means++ rows (or train), then assign
  sweep      auto.rs:457-510  every k of a list, best of `restarts`, scored by
                              internal_scores (on the device)
  select     auto.rs:513-542  the chosen k of a sweep
  kmeans_pp  auto.rs:401-455  on the device (HipDevice.kmeans_pp)

Two-level auto_cluster (emeans_amd.autocluster) and the hierarchy
(emeans_amd.hierarchy) are callers of these.
"""

import time
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass, field
from typing import Callable, List, Optional, Tuple

import numpy as np

from . import Config, HipDevice


@dataclass
class AutoConfig:
    """The AutoConfig fields the sweeps read (auto.rs:99-175), with its defaults."""
    k1_range: Tuple[int, int] = (2, 40)
    k2_max: int = 20
    criterion1: str = "silhouette"
    criterion2: str = "davies_bouldin"
    level1_tolerance: float = 0.0
    level2_tolerance: float = 0.05
    min_cluster_size: int = 20
    max_cluster_size: int = 200
    min_split_size: int = 60
    split_min_silhouette: float = 0.05
    restarts: int = 4
    nepochs: float = 5.0
    init: str = "k_means_plus_plus"  # or "random_rows"
    level1_method: str = "bottom_up"  # or "top_down"
    resplit_passes: int = 2
    level1_max_share: float = 0.5
    seed: int = 1234
    verbose: bool = False


@dataclass
class KScore:
    """Scores of one k in a sweep (auto.rs:178-192)."""
    k: int
    k_eff: int
    silhouette: float
    calinski_harabasz: float
    davies_bouldin: float
    objective: float
    browsable: float
    seconds: float


@dataclass
class Diagnostics:
    """Sweep results (auto.rs:209-238): the level-1 candidates, each group's
    level-2 sweep, seconds, the stage-A level-1 sweep, resplits, leaves, the
    gap cut, flatness and the rejected cuts."""
    level1: list = field(default_factory=list)
    level2: list = field(default_factory=list)
    seconds: float = 0.0
    stage_a_level1: list = field(default_factory=list)
    resplits: int = 0
    leaves: int = 0
    gap_k: int = 0
    flat: bool = False
    level1_rejected: list = field(default_factory=list)


@dataclass
class Fitted:
    """One fitted model of a sweep: its centroids and assignment (device buffers)."""
    k: int
    seed: int
    centroids: np.ndarray
    labels: object  # DevBuf, u32 n
    scores: object  # DevBuf, f32 n
    objective: float
    positions: np.ndarray = None  # EMA state, for a later resume
    usage: np.ndarray = None


def criterion_value(crit: str, s: KScore) -> float:
    """Criterion::value (auto.rs:53-60): the criterion as higher-is-better."""
    if crit == "silhouette":
        return s.silhouette
    if crit == "calinski_harabasz":
        return s.calinski_harabasz
    if crit == "davies_bouldin":
        return -s.davies_bouldin
    raise ValueError(f"unknown criterion {crit!r}")


def seed_for(cfg: AutoConfig, salt: int, k: int, restart: int) -> int:
    """u32 wrapping arithmetic of auto.rs:343-349."""
    m = 0xFFFFFFFF
    return (cfg.seed + ((salt * 7919) & m) + ((k * 131) & m) + ((restart * 1_000_003) & m)) & m


def fit(dev: HipDevice, x: np.ndarray, xb, k: int, nepochs: float, seed: int,
        init_rows: Optional[np.ndarray]) -> Fitted:
    """auto.rs:351-375: one spherical e-means model (capture off) from the
    first k k-means++ rows (or k sampled rows), then the assignment of every row."""
    n, d = x.shape
    c = Config(d=d, k=k, spherical=True, nepochs=nepochs, seed=seed, capture_assignments=False)
    if init_rows is not None:
        if len(init_rows) < k:
            raise ValueError("need k init rows")
        init = x[np.asarray(init_rows[:k], np.int64)]
    else:
        init = None
    cb = dev.zeros_f32(k * d)
    cent, info = dev.train_dev(xb, n, c, centroids_out=cb, init=init)
    labels, scores = dev.zeros_u32(n), dev.zeros_f32(n)
    dev.assign_dev(xb, n, d, cb, k, "ip", labels, scores)
    s = dev.read_f32(scores).astype(np.float64)
    obj = float(np.cumsum(2.0 - 2.0 * s)[-1] / n)  # Assignment::mean_objective(true)
    return Fitted(k, seed, cent, labels, scores, obj, info["positions"], info["usage"])


def browsable(sizes, cfg: AutoConfig) -> float:
    """auto.rs:377-384: the fraction of rows in clusters of browsable size."""
    sizes = np.asarray(sizes, np.int64)
    ok = sizes[(sizes >= cfg.min_cluster_size) & (sizes <= cfg.max_cluster_size)].sum()
    return float(ok) / float(max(int(sizes.sum()), 1))


def score(k: int, i: dict, cfg: AutoConfig, seconds: float) -> KScore:
    """auto.rs:386-397: a k's KScore from its internal_scores."""
    return KScore(k, i["k_eff"], i["silhouette"], i["calinski_harabasz"], i["davies_bouldin"],
                  i["objective"], browsable(i["sizes"], cfg), seconds)


# Independent fits at once: one thread per context, at most four contexts (a
# process gets four hardware queues on the GPU; measured on 8 small fits, four
# contexts ran them 2.6-3x faster than one, six slower than four).
MAX_CONTEXTS = 4


def _contexts(dev, n: int) -> list:
    """dev and up to n - 1 more contexts on its GPU (HipDevice.contexts); a
    device without them (the tests' oracle) runs the work in turn."""
    more = getattr(dev, "contexts", None)
    return more(max(min(n, MAX_CONTEXTS), 1)) if more is not None else [dev]


def _each(devs: list, pool: Optional[ThreadPoolExecutor], tasks: List[Callable]) -> list:
    """tasks[i](device) for every i, results in task order: waves of len(devs)
    tasks, each on its own context, so no context runs two at once."""
    if pool is None:
        return [t(devs[0]) for t in tasks]
    out = []
    for w in range(0, len(tasks), len(devs)):
        futs = [pool.submit(t, devs[j]) for j, t in enumerate(tasks[w:w + len(devs)])]
        out += [f.result() for f in futs]
    return out


def sweep(dev: HipDevice, x: np.ndarray, xb, ks: List[int], cfg: AutoConfig, salt: int,
          verbose: bool = False, timing: Optional[dict] = None):
    """auto.rs:457-510: for every k, the best (lowest objective) of
    cfg.restarts fits, each seeded by its restart's k-means++ rows (one
    seeding per restart, up to the largest k); scored by internal_scores.
    Returns [(KScore, Fitted)] and the k-means++ picks of each restart.
    The restarts' seedings, and each k's restarts, run at once on up to four
    contexts; each is deterministic, and the best is taken in restart order,
    so the results are those of running them in turn."""
    n, d = x.shape
    tm = timing if timing is not None else {}
    for key in ("kmeans_pp_s", "fit_s", "scores_s"):
        tm.setdefault(key, 0.0)
    tm.setdefault("fits", 0)
    kmax = max(ks) if ks else 1
    restarts = max(cfg.restarts, 1)
    devs = _contexts(dev, restarts)
    pool = ThreadPoolExecutor(len(devs)) if len(devs) > 1 else None
    if pool is not None:
        # The other contexts read xb: wait for dev's stream, which the upload
        # of a fresh binding (dev.bind) orders, before they start.
        dev.sync()
    try:
        return _sweep(dev, devs, pool, x, xb, ks, cfg, salt, kmax, restarts, verbose, tm)
    finally:
        if pool is not None:
            pool.shutdown()


def _sweep(dev, devs, pool, x, xb, ks, cfg, salt, kmax, restarts, verbose, tm):
    n, d = x.shape
    t0 = time.perf_counter()
    if cfg.init == "k_means_plus_plus":
        inits = _each(devs, pool, [
            (lambda dv, r=r: dv.kmeans_pp(xb, n, d, kmax, seed_for(cfg, salt, 0, r)))
            for r in range(restarts)])
    else:
        inits = [None] * restarts
    tm["kmeans_pp_s"] += time.perf_counter() - t0
    out = []
    for k in ks:
        t = time.perf_counter()
        fits = _each(devs, pool, [
            (lambda dv, r=r: fit(dv, x, xb, k, cfg.nepochs, seed_for(cfg, salt, k, r), inits[r]))
            for r in range(restarts)])
        tm["fits"] += len(fits)
        best = None
        for f in fits:
            if best is None or f.objective < best.objective:
                best = f
        t1 = time.perf_counter()
        tm["fit_s"] += t1 - t
        i = dev.internal_scores(xb, n, d, best.labels, k)
        tm["scores_s"] += time.perf_counter() - t1
        s = score(k, i, cfg, time.perf_counter() - t)
        if verbose:
            print(f"  k={k:3} k_eff={s.k_eff:3} sil={s.silhouette:.4f} "
                  f"ch={s.calinski_harabasz:.1f} db={s.davies_bouldin:.3f} "
                  f"obj={s.objective:.4f} browsable={s.browsable:.2f} ({s.seconds:.2f}s)")
        out.append((s, best))
    return out, inits


def select(scores: List[KScore], cfg: AutoConfig, prefer_browsable: bool) -> int:
    """auto.rs:513-542: among the k within the tolerance of the best criterion,
    the smallest k (level 1), or the most browsable then the smaller k (level 2)."""
    crit = cfg.criterion2 if prefer_browsable else cfg.criterion1
    v = [criterion_value(crit, s) for s in scores]
    best = max(v) if v else float("-inf")
    tol = cfg.level2_tolerance if prefer_browsable else cfg.level1_tolerance
    floor = best - tol * abs(best)
    cands = [i for i in range(len(scores)) if v[i] >= floor]
    if prefer_browsable:
        # max_by: browsable (total order), then the smaller k; the last of equal maxima
        top = cands[0]
        for i in cands[1:]:
            a, b = scores[i], scores[top]
            if (a.browsable, -a.k) >= (b.browsable, -b.k):
                top = i
        return top
    return min(cands, key=lambda i: scores[i].k)
