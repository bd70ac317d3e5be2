"""auto_cluster (emeans-cluster/src/auto.rs:544-1101) on the gfx950 backend:
two-level clustering of unit rows with automatic k, its sweeps' trainings,
assignments, k-means++ seedings and internal scores on the device, and the
rest on the host as in the reference:

  fit_group        auto.rs:544-590    a group's level-2 sweep and decision
  stage_a          auto.rs:603-660    level-1 sweep, then a sweep per group
  resplit          auto.rs:666-748    leaves above max_cluster_size split
                                      again when a k <= 4 screen finds structure
  refine           auto.rs:768-797    two passes of every row to its nearest
                                      leaf mean (the assignment on the device)
  average_linkage  auto.rs:799-858    leaves merged by exact mean row cosine
  cut              auto.rs:860-878
  group_bottom_up  auto.rs:880-953    the cut scored best on criterion1
  auto_cluster     auto.rs:1001-1101  the hierarchy assembled from the leaves
  full_retrain     incremental.rs:598-650  auto_cluster on all rows, stable
                                      ids carried by matching

Float sums follow Rust's Sum (a left fold from -0.0: a sum is its first term
plus the rest in order); f64 row sums are sequential, as unit_means'.
"""

import sys
import time
from dataclasses import dataclass
from typing import List, Optional

import numpy as np

from . import HipDevice
from . import auto
from . import hierarchy as H
from .auto import Diagnostics

SCREEN_K = 4  # auto.rs:663


@dataclass
class Leaves:
    """auto.rs:592-600: rows per leaf, the level-1 group each came from, and
    the best silhouette of the last split sweep inside it."""
    rows: List[np.ndarray]
    parent: List[int]
    sweep: List[Optional[float]]


def _fmax_fold(vals) -> float:
    """fold(-inf, f64::max): the largest, NaN skipped."""
    b = -np.inf
    for v in vals:
        if not (v <= b) and v == v:
            b = v
    return b


def _total_key64(v: float) -> int:
    """f64::total_cmp as an integer key."""
    b = int(np.array([v], np.float64).view(np.int64)[0])
    return b ^ 0x7FFFFFFFFFFFFFFF if b < 0 else b


def fit_group(dev: HipDevice, xg: np.ndarray, cfg, salt: int, tm: Optional[dict] = None):
    """auto.rs:544-590: (Fitted or None, decision, sweep scores)."""
    n, d = xg.shape
    if n == 0:
        return None, ("Empty", None), []
    xgb = dev.bind(xg)

    def one():
        return auto.fit(dev, xg, xgb, 1, cfg.nepochs, auto.seed_for(cfg, salt, 1, 0), None)

    kmax = min(cfg.k2_max, n // max(cfg.min_cluster_size, 1))
    if n < cfg.min_split_size or kmax < 2:
        return one(), ("TooSmall", None), []
    runs, _ = auto.sweep(dev, xg, xgb, list(range(2, kmax + 1)), cfg, salt, timing=tm)
    scores = [s for s, _ in runs]
    best_sil = _fmax_fold(s.silhouette for s in scores)
    if best_sil < cfg.split_min_silhouette:
        return one(), ("NoStructure", best_sil), scores
    pick = auto.select(scores, cfg, True)
    return runs[pick][1], ("Split", scores[pick].k), scores


def _split_rows(r: np.ndarray, labels: np.ndarray, k: int) -> List[np.ndarray]:
    """The rows r grouped by their labels 0..k, each group in row order (a
    stable sort by label keeps the order within a label)."""
    labels = np.asarray(labels, np.int64)
    order = np.argsort(labels, kind="stable")
    counts = np.bincount(labels, minlength=k)[:k]
    return np.split(np.asarray(r)[order[:int(counts.sum())]], np.cumsum(counts)[:-1])


def stage_a(dev: HipDevice, x: np.ndarray, xb, cfg, diag: Diagnostics,
            tm: Optional[dict] = None) -> Leaves:
    """auto.rs:603-660."""
    n, d = x.shape
    k1_hi = min(cfg.k1_range[1], n)
    k1_lo = min(cfg.k1_range[0], k1_hi)
    runs, _ = auto.sweep(dev, x, xb, list(range(k1_lo, k1_hi + 1)), cfg, 0, timing=tm)
    scores = [s for s, _ in runs]
    pick = auto.select(scores, cfg, False)
    level1 = runs[pick][1]
    diag.stage_a_level1 = scores
    a1 = dev.read_u32(level1.labels)
    leaves = Leaves([], [], [])
    for g in range(level1.k):
        r = np.flatnonzero(a1 == g)
        if len(r) == 0:
            diag.level2.append([])
            continue
        xg = np.ascontiguousarray(x[r])
        model, decision, sc = fit_group(dev, xg, cfg, 1 + g, tm)
        if cfg.verbose:
            print(f"  group {g}: {len(r)} rows, {decision[0]} {decision[1]}", file=sys.stderr,
                  flush=True)
        best = _fmax_fold(s.silhouette for s in sc)
        diag.level2.append(sc)
        sub = _split_rows(r, dev.read_u32(model.labels), model.k)
        for s in sub:
            if len(s) == 0:
                continue
            leaves.rows.append(s)
            leaves.parent.append(g)
            leaves.sweep.append(None if decision[0] == "Split" else
                                (best if np.isfinite(best) else None))
    return leaves


def resplit(dev: HipDevice, x: np.ndarray, cfg, leaves: Leaves, tm: Optional[dict] = None):
    """auto.rs:666-748: (leaves, number of splits)."""
    cur, splits = leaves, 0
    for pas in range(cfg.resplit_passes):
        nxt = Leaves([], [], [])
        changed = False
        for li, (r, p, sw) in enumerate(zip(cur.rows, cur.parent, cur.sweep)):
            swept_flat = sw is not None and sw < cfg.split_min_silhouette
            if len(r) <= cfg.max_cluster_size or len(r) < cfg.min_split_size or swept_flat:
                nxt.rows.append(r)
                nxt.parent.append(p)
                nxt.sweep.append(sw)
                continue
            xg = np.ascontiguousarray(x[r])
            salt = (50_000 + 1000 * pas + li) & 0xFFFFFFFF
            kmax = min(cfg.k2_max, len(r) // max(cfg.min_cluster_size, 1))
            screen = list(range(2, min(kmax, SCREEN_K) + 1))
            screen_best = -np.inf
            if screen:
                runs, _ = auto.sweep(dev, xg, dev.bind(xg), screen, cfg, salt, timing=tm)
                screen_best = _fmax_fold(s.silhouette for s, _ in runs)
            if not screen or screen_best < cfg.split_min_silhouette:
                if cfg.verbose:
                    print(f"  resplit pass {pas} leaf {li}: {len(r)} rows, screen {screen_best:.3f}",
                          file=sys.stderr, flush=True)
                nxt.rows.append(r)
                nxt.parent.append(p)
                nxt.sweep.append(screen_best if np.isfinite(screen_best) else None)
                continue
            model, decision, sc = fit_group(dev, xg, cfg, salt, tm)
            best = _fmax_fold(s.silhouette for s in sc)
            if cfg.verbose:
                print(f"  resplit pass {pas} leaf {li}: {len(r)} rows, {decision[0]} {decision[1]}",
                      file=sys.stderr, flush=True)
            if decision[0] == "Split" and model is not None:
                for s in _split_rows(r, dev.read_u32(model.labels), decision[1]):
                    if len(s) == 0:
                        continue
                    nxt.rows.append(s)
                    nxt.parent.append(p)
                    nxt.sweep.append(None)
                splits += 1
                changed = True
            else:
                nxt.rows.append(r)
                nxt.parent.append(p)
                nxt.sweep.append(best if np.isfinite(best) else None)
        cur = nxt
        if not changed:
            break
    return cur, splits


def refine(dev: HipDevice, x: np.ndarray, leaves: Leaves) -> Leaves:
    """auto.rs:768-797: twice, every row to its nearest leaf mean (cosine,
    the top-1 on the device, bit-equal to the reference's CPU assigner);
    emptied leaves dropped."""
    d = x.shape[1]
    cur = leaves
    for _ in range(2):
        c = H.unit_means(x, cur.rows)
        lab, _ = dev.assign(x, d, c, "ip", 1 << 16)
        rows = _split_rows(np.arange(x.shape[0]), lab.astype(np.int64), len(cur.rows))
        keep = [j for j in range(len(rows)) if len(rows[j])]
        cur = Leaves([rows[j] for j in keep], [cur.parent[j] for j in keep],
                     [cur.sweep[j] for j in keep])
    return cur


def _seq_dot64(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Σ_t a_t b_t per row pair (rows of a against the row b), f64 in order."""
    return np.add.accumulate(a * b[None, :], axis=1)[:, -1]


def average_linkage(x: np.ndarray, rows: List[np.ndarray]):
    """auto.rs:799-858: merges (a, b, similarity) by the exact mean row cosine
    s_A . s_B / (|A| |B|); the merged cluster keeps id a."""
    l = len(rows)
    sums = H.row_sums_f64(x, rows)
    size = np.array([float(len(r)) for r in rows], np.float64)
    dots = np.zeros((l, l), np.float64)
    for a in range(l):
        v = _seq_dot64(sums[a:], sums[a])
        dots[a, a:] = v
        dots[a:, a] = v
    alive = np.ones(l, bool)
    neg = -np.inf
    # The pair merged next is the first (a < b, both alive) in row-major order
    # of the largest s = dots[a, b] / (size[a] size[b]) above -inf (NaN never
    # wins), as a scan with a strict > finds it. Each row keeps its own first
    # best column (bv, bb); a merge changes row a, column a and kills b, so
    # only rows whose best was a or b are scanned again, and the others
    # compare their new column a with their best.
    bv = np.full(l, neg)
    bb = np.full(l, -1, np.int64)

    def scan(a):
        if a >= l - 1 or not alive[a]:
            bv[a], bb[a] = neg, -1
            return
        s = dots[a, a + 1:] / (size[a] * size[a + 1:])
        v = np.where(alive[a + 1:] & (s > neg), s, neg)
        j = int(np.argmax(v))
        bv[a], bb[a] = (float(v[j]), a + 1 + j) if v[j] > neg else (neg, -1)

    for a in range(l):
        scan(a)
    merges = []
    for _ in range(1, l):
        cand = np.where(alive & (bb >= 0), bv, neg)
        a = int(np.argmax(cand))
        if cand[a] > neg:
            b, best = int(bb[a]), float(bv[a])
        else:
            best, a, b = neg, 0, 0
        alive[b] = False
        size[a] += size[b]
        sums[a] = sums[a] + sums[b]
        merged = dots[a] + dots[b]
        dots[:, a] = merged
        dots[a] = merged
        dots[a, a] = float(np.add.accumulate(sums[a] * sums[a])[-1])
        merges.append((a, b, best))
        scan(b)
        scan(a)
        rows = np.flatnonzero(alive[:a])
        if len(rows):
            v = dots[rows, a] / (size[rows] * size[a])
            redo = (bb[rows] == a) | (bb[rows] == b)
            up = ~redo & (v > neg) & ((v > bv[rows]) | ((v == bv[rows]) & (a < bb[rows])))
            bv[rows[up]], bb[rows[up]] = v[up], a
            for r in rows[redo]:
                scan(int(r))
        for r in np.flatnonzero(alive[a + 1:b] & (bb[a + 1:b] == b)) + a + 1:
            scan(int(r))
    return merges


def cut(l: int, merges, k: int) -> np.ndarray:
    """auto.rs:860-878: each leaf's group after the first l - k merges,
    numbered 0.. by lowest leaf."""
    owner = np.arange(l)
    for a, b, _ in merges[:l - k]:
        owner[owner == b] = a
    ids = {}
    for o in owner.tolist():
        ids.setdefault(o, len(ids))
    return np.array([ids[o] for o in owner.tolist()], np.int64)


def group_bottom_up(dev: HipDevice, x: np.ndarray, xb, cfg, leaves: Leaves,
                    diag: Diagnostics) -> np.ndarray:
    """auto.rs:880-953."""
    n, d = x.shape
    l = len(leaves.rows)
    if l <= 2:
        return np.arange(l)
    merges = average_linkage(x, leaves.rows)
    leaf_of = np.zeros(n, np.int64)
    for j, r in enumerate(leaves.rows):
        leaf_of[r] = j
    hi = min(cfg.k1_range[1], l - 1)
    lo = min(max(cfg.k1_range[0], 2), hi)
    ks = list(range(lo, hi + 1)) + [l]
    scores, eligible = [], []
    for k in ks:
        t = time.perf_counter()
        labels = cut(l, merges, k)[leaf_of].astype(np.uint32)
        sizes = np.bincount(labels, minlength=k)
        largest = float(sizes.max()) / max(n, 1)
        eligible.append(k == l or largest <= cfg.level1_max_share)
        lb = dev.upload_u32(labels)
        i = dev.internal_scores(xb, n, d, lb, k)
        scores.append(auto.score(k, i, cfg, time.perf_counter() - t))
    gaps = [merges[t][2] - merges[t + 1][2] for t in range(len(merges) - 1)]
    if gaps:  # max_by with total_cmp: the last of equal maxima
        keys = [_total_key64(g) for g in gaps]
        t = max(range(len(gaps)), key=lambda i: (keys[i], i))
        diag.gap_k = l - 1 - t
    else:
        diag.gap_k = 1
    v = [auto.criterion_value(cfg.criterion1, s) if ok else -np.inf
         for s, ok in zip(scores, eligible)]
    # max_by(v total order, then the smaller k): the last of equal maxima
    best = max(range(len(ks)), key=lambda i: (_total_key64(v[i]), -ks[i], i))
    diag.flat = ks[best] == l
    diag.level1_rejected = [k for k, ok in zip(ks, eligible) if not ok]
    diag.level1 = scores
    return cut(l, merges, ks[best])


def _decision(members: List[int], leaves: Leaves, size: int, cfg):
    """auto.rs:1058-1072: why a group has its level-2 k."""
    if len(members) >= 2:
        return H.decision_split(len(members))
    b = leaves.sweep[members[0]]
    if b is not None and b < cfg.split_min_silhouette:
        return H.decision_no_structure(b)
    if size < cfg.min_split_size or size <= cfg.max_cluster_size:
        return H.DECISION_TOO_SMALL
    if b is not None:
        return H.decision_no_structure(b)
    return H.DECISION_TOO_SMALL


def auto_cluster(dev: HipDevice, x: np.ndarray, cfg, inc: Optional[H.IncrementalConfig] = None,
                 timing: Optional[dict] = None):
    """auto.rs:1001-1101: (Hierarchy, Labels) of the unit rows of x. With
    timing, the sweeps' counters (auto.sweep) and each stage's seconds
    accumulate in it."""
    tm = timing if timing is not None else {}
    x = np.ascontiguousarray(x, np.float32)
    if x.ndim != 2:
        raise ValueError("x must be n x d")
    n, d = x.shape
    if n < 2:
        raise ValueError("need at least 2 rows")
    if not (1 <= cfg.k1_range[0] <= cfg.k1_range[1]):
        raise ValueError("bad k1_range")
    t = time.perf_counter()
    # The sweeps' contexts, made now: the runtime gives each new stream the
    # least-used hardware queue, so their kernel streams, made one after
    # another before any copy stream, land on different queues (two sharing
    # one ran the fits up to 1.5x slower).
    auto._contexts(dev, cfg.restarts)
    xb = dev.bind(x)
    diag = Diagnostics()
    lap = time.perf_counter()

    def stage(name):  # the reference's verbose laps (auto.rs:1015-1020)
        nonlocal lap
        now = time.perf_counter()
        tm[name + "_s"] = tm.get(name + "_s", 0.0) + now - lap
        lap = now
        if cfg.verbose:
            print(f"[{now - t:.1f}s] {name}", file=sys.stderr, flush=True)

    leaves = stage_a(dev, x, xb, cfg, diag, tm)
    stage("stage_a")
    leaves, resplits = resplit(dev, x, cfg, leaves, tm)
    stage("resplit")
    leaves = refine(dev, x, leaves)
    stage("refine")
    diag.resplits = resplits
    diag.leaves = len(leaves.rows)
    if cfg.level1_method == "bottom_up":
        group_of_leaf = group_bottom_up(dev, x, xb, cfg, leaves, diag)
    else:
        ids = {}
        for p in leaves.parent:
            ids.setdefault(p, len(ids))
        diag.level1 = list(diag.stage_a_level1)
        group_of_leaf = np.array([ids[p] for p in leaves.parent], np.int64)
    stage("level1")
    k1 = int(group_of_leaf.max()) + 1 if len(group_of_leaf) else 0
    groups, group_rows = [], []
    for g in range(k1):
        members = [j for j in range(len(leaves.rows)) if group_of_leaf[j] == g]
        rows = [leaves.rows[j] for j in members]
        counts = [len(r) for r in rows]
        model = H.model_from(H.unit_means(x, rows), counts, d, cfg.nepochs, cfg.seed)
        group_rows.append(np.concatenate(rows) if rows else np.zeros(0, np.int64))
        k2 = len(members)
        groups.append(H.Group(model, list(range(k2)), np.full(k2, np.nan, np.float32), k2,
                              _decision(members, leaves, sum(counts), cfg)))
    counts1 = [len(r) for r in group_rows]
    level1 = H.model_from(H.unit_means(x, group_rows), counts1, d, cfg.nepochs, cfg.seed)
    h = H.Hierarchy(d, level1, groups, list(range(k1)), H.State.new(n, k1),
                    H.HipBackend(dev), inc or H.IncrementalConfig(), config=cfg)
    h.diagnostics = diag
    labels = h.assign(x)
    h.set_floors(labels)
    labels = h.assign(x)
    stage("assemble")
    diag.seconds = time.perf_counter() - t
    return h, labels


def full_retrain(dev: HipDevice, h: "H.Hierarchy", x_all: np.ndarray, cfg):
    """incremental.rs:598-650: auto_cluster on all rows (seed + rows seen),
    then the old level-1 and leaf ids carried over to matching centroids."""
    d, n = h.d, x_all.shape[0]
    min_sim = h.inc.match_min_sim
    c2 = auto.AutoConfig(**{**cfg.__dict__, "seed": (cfg.seed + h.state.n_seen) & 0xFFFFFFFF})
    nh, _ = auto_cluster(dev, x_all, c2, h.inc)
    matched = H.match_centroids(h.level1_centroids(), nh.level1_centroids(), d, min_sim)
    nh.ids1, next1 = H.carry_ids(matched, h.ids1, h.state.next_id1)
    for slot, o in enumerate(matched):
        if o is None:
            continue
        m2 = H.match_centroids(h.leaf_centroids(o), nh.leaf_centroids(slot), d, min_sim)
        og = h.groups[o]
        nxt = max(og.next_id, 1)
        if og.model is not None:
            ids, nxt = H.carry_ids(m2, og.ids, nxt)
        else:
            ids, nxt = H.carry_ids([None] * len(m2), [], nxt)
        g = nh.groups[slot]
        if g.model is not None:
            g.ids = ids
        g.next_id = nxt
    h.level1, h.groups, h.ids1 = nh.level1, nh.groups, nh.ids1
    h.state = H.State.new(n, next1)
    h.diagnostics = nh.diagnostics
