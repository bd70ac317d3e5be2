"""Hierarchy labelling and its incremental update on the gfx950 backend
(emeans-cluster/src/auto.rs:1103-1300, incremental.rs:52-600).

A hierarchy holds a level-1 model (one centroid per group) and a level-2
model per group (its leaves). What runs on the device:

  Hierarchy.assign   auto.rs:1135-1189  the nearest leaf of every row over all
                                        leaves (top-1, inner product, on the
                                        device in chunks of 65,536 rows)
  Hierarchy.add      incremental.rs:306-360   label new rows, then by the
                                        policy: nothing, the EMA update, or a
                                        full retrain
  ema_update         incremental.rs:546-596   each group's leaves resume from
                                        their EMA state on the group's rows
                                        (the training loop on the device); the
                                        level 1 follows its groups' means

and on the host, as in the reference: the outlier floors (auto.rs:1194-1292),
the policy, the centroid matching that keeps stable ids (incremental.rs:
176-290), unit means (auto.rs:750-765) and model_from (auto.rs:955-987).

The full retrain runs auto_cluster (emeans_amd.autocluster) on all rows.
Not built here: the grow step's leaf formation from pending outliers
(incremental.rs:376-540); its early exits are kept, and a call that would
form leaves raises NotImplementedError rather than returning other results.

The device work goes through a backend object with two methods, so that the
same host logic runs over any device:
  leaf_top1(x, cents) -> (labels u32, sims f32)   top-1 by inner product
  resume(config, x, positions, usage) -> (centroids, positions, usage)
HipBackend is the gfx950 one.
"""

import math
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

from . import Config, HipDevice, recipe_batch

MAD_SIGMA = np.float32(1.4826)  # auto.rs:1220
OWN_SPREAD_MIN = 20             # auto.rs:1217


@dataclass
class IncrementalConfig:
    """incremental.rs:52-105, with its defaults."""
    outlier_mad_k: float = 3.0
    outlier_min_sim: Optional[float] = None
    grow_min_size: int = 20
    update_min_outliers: int = 50
    update_added_fraction: float = 0.10
    update_epochs: float = 1.0
    retrain_added_fraction: float = 0.5
    retrain_outlier_fraction: float = 0.25
    match_min_sim: float = 0.8


@dataclass
class State:
    """The counters behind the update policy (incremental.rs:108-135)."""
    n_seen: int
    n_full: int
    n_update: int
    added_since_full: int = 0
    outliers_since_full: int = 0
    added_since_update: int = 0
    pending: List[int] = field(default_factory=list)
    next_id1: int = 0

    @staticmethod
    def new(n: int, next_id1: int) -> "State":
        return State(n, n, n, next_id1=next_id1)


@dataclass
class Model:
    """An e-means model's state: its config, centroids and EMA state (k x d)."""
    config: Config
    centroids: np.ndarray
    positions: np.ndarray
    usage: np.ndarray

    @property
    def k(self) -> int:
        return self.config.k


@dataclass
class Group:
    """A level-1 slot (auto.rs Group): its leaves' model, their stable ids and outlier floors."""
    model: Optional[Model]
    ids: List[int]
    floors: np.ndarray
    next_id: int


@dataclass
class Labels:
    """auto.rs Labels: stable ids, cosines, outlier flags and slots of every row."""
    l1: np.ndarray
    l2: np.ndarray
    sim1: np.ndarray
    sim: np.ndarray
    outlier: np.ndarray
    slot1: np.ndarray
    slot2: np.ndarray


@dataclass
class AddReport:
    """incremental.rs:144-158."""
    action: str
    labels: Labels
    new_outliers: int
    pending: int
    outlier_fraction: float
    new_leaves: list


class HipBackend:
    """The device work of a hierarchy on a gfx950 context."""

    def __init__(self, dev: HipDevice):
        self.dev = dev

    def leaf_top1(self, x: np.ndarray, cents: np.ndarray):
        return self.dev.assign(x, x.shape[1], cents, "ip", 1 << 16)

    def resume(self, config: Config, x: np.ndarray, positions, usage):
        n, d = x.shape
        cent, info = self.dev.train_dev(self.dev.bind(x), n, config, state=(positions, usage))
        return cent, info["positions"], info["usage"]


# ---------------------------------------------------------------- host rules
def _total_key(v: np.ndarray) -> np.ndarray:
    """An integer key that orders f32 values as f32::total_cmp does."""
    b = np.ascontiguousarray(v, np.float32).view(np.int32).astype(np.int64)
    return np.where(b < 0, b ^ 0x7FFFFFFF, b)


def quantile(v, q: float) -> np.float32:
    """metrics.rs:271-279: the sorted (total order) value at round(q (n - 1))."""
    v = np.asarray(v, np.float32)
    if v.size == 0:
        return np.float32(np.nan)
    s = v[np.argsort(_total_key(v), kind="stable")]
    i = int(math.floor(min(max(q, 0.0), 1.0) * (v.size - 1) + 0.5))  # f64::round, x >= 0
    return s[i]


@dataclass
class Spread:
    median: List[np.float32]
    mad: List[np.float32]
    pooled_mad: np.float32
    global_median: np.float32


def spread(sims: List[np.ndarray]) -> Spread:
    """auto.rs:1228-1246."""
    median = [quantile(v, 0.5) for v in sims]
    res, mad = [], []
    for v, m in zip(sims, median):
        r = np.abs(np.asarray(v, np.float32) - m)
        mad.append(quantile(r, 0.5))
        res.append(r)
    allv = np.concatenate([np.asarray(v, np.float32) for v in sims]) if sims else np.zeros(0, np.float32)
    allr = np.concatenate(res) if res else np.zeros(0, np.float32)
    return Spread(median, mad, quantile(allr, 0.5), quantile(allv, 0.5))


def leaf_floors(sims: List[np.ndarray], inc: IncrementalConfig) -> List[np.float32]:
    """auto.rs:1266-1292: median - outlier_mad_k 1.4826 MAD (own spread from
    OWN_SPREAD_MIN rows, else pooled), f32 arithmetic left to right."""
    if inc.outlier_min_sim is not None:
        return [np.float32(inc.outlier_min_sim)] * len(sims)
    sp = spread(sims)
    k = np.float32(inc.outlier_mad_k)
    out = []
    for j, v in enumerate(sims):
        v = np.asarray(v, np.float32)
        if v.size == 0:
            out.append(np.float32(sp.global_median - k * MAD_SIGMA * sp.pooled_mad))
            continue
        own = sp.mad[j]
        s = own if v.size >= OWN_SPREAD_MIN and own > 0 else sp.pooled_mad
        if s > 0:
            out.append(np.float32(sp.median[j] - k * MAD_SIGMA * s))
        else:
            out.append(np.float32(np.fmin.reduce(v, initial=np.inf)))  # fold(inf, f32::min)
    return out


def hungarian(cost: List[List[float]]) -> List[int]:
    """incremental.rs:176-240: the column of every row of a minimum-cost
    assignment (rows <= cols), the same steps in f64."""
    n = len(cost)
    if n == 0:
        return []
    m = len(cost[0])
    assert n <= m
    inf = math.inf
    u, v = [0.0] * (n + 1), [0.0] * (m + 1)
    p, way = [0] * (m + 1), [0] * (m + 1)
    for i in range(1, n + 1):
        p[0] = i
        j0 = 0
        minv = [inf] * (m + 1)
        used = [False] * (m + 1)
        while True:
            used[j0] = True
            i0 = p[j0]
            delta, j1 = inf, 0
            for j in range(1, m + 1):
                if not used[j]:
                    cur = cost[i0 - 1][j - 1] - u[i0] - v[j]
                    if cur < minv[j]:
                        minv[j] = cur
                        way[j] = j0
                    if minv[j] < delta:
                        delta = minv[j]
                        j1 = j
            for j in range(m + 1):
                if used[j]:
                    u[p[j]] += delta
                    v[j] -= delta
                else:
                    minv[j] -= delta
            j0 = j1
            if p[j0] == 0:
                break
        while True:
            j1 = way[j0]
            p[j0] = p[j1]
            j0 = j1
            if j0 == 0:
                break
    ans = [0] * n
    for j in range(1, m + 1):
        if p[j] != 0:
            ans[p[j] - 1] = j - 1
    return ans


def _sims64(old: np.ndarray, new: np.ndarray) -> np.ndarray:
    """sim[a][b] = Σ_t old_a,t new_b,t in f64, added in order (incremental.rs:
    244-250; the f64 products of f32 values are exact)."""
    p = old.astype(np.float64)[:, None, :] * new.astype(np.float64)[None, :, :]
    return np.add.accumulate(p, axis=2)[:, :, -1]


def match_centroids(old: np.ndarray, new: np.ndarray, d: int, min_sim: float):
    """incremental.rs:241-275: for each new centroid the old one it continues,
    by a maximum-similarity matching; pairs below min_sim dropped."""
    old = np.asarray(old, np.float32).reshape(-1, d)
    new = np.asarray(new, np.float32).reshape(-1, d)
    ko, kn = old.shape[0], new.shape[0]
    out: List[Optional[int]] = [None] * kn
    if ko == 0 or kn == 0:
        return out
    sim = _sims64(old, new).tolist()
    ms = float(np.float32(min_sim))
    if kn <= ko:
        for b, a in enumerate(hungarian([[-sim[a][b] for a in range(ko)] for b in range(kn)])):
            if sim[a][b] >= ms:
                out[b] = a
    else:
        for a, b in enumerate(hungarian([[-sim[a][b] for b in range(kn)] for a in range(ko)])):
            if sim[a][b] >= ms:
                out[b] = a
    return out


def carry_ids(matched, old_ids: List[int], next_id: int):
    """incremental.rs:277-289: matched slots keep the old id, others take fresh ones."""
    ids = []
    for m in matched:
        if m is not None:
            ids.append(old_ids[m])
        else:
            ids.append(next_id)
            next_id += 1
    return ids, next_id


# Float sums below follow Rust's f32/f64 Sum (the toolchain the reference
# pins, 1.99): a left fold from -0.0, so a sum is its first term plus the
# rest in order.


def normalize_rows(m: np.ndarray) -> np.ndarray:
    """model.rs:952-967 (faiss normalize_into): divide by the largest
    magnitude, then by the f32 norm summed in order; zero rows stay zero."""
    m = np.array(m, np.float32, copy=True)
    mx = np.max(np.abs(m), axis=1, initial=np.float32(0))
    s = np.where(mx > 0, mx, np.float32(1)).astype(np.float32)
    m = (m / s[:, None]).astype(np.float32)
    sq = (m * m).astype(np.float32)
    norm = np.sqrt(np.add.accumulate(sq, axis=1, dtype=np.float32)[:, -1]).astype(np.float32)
    s = np.where(norm > 0, norm, np.float32(1)).astype(np.float32)
    return (m / s[:, None]).astype(np.float32)


def row_sums_f64(x: np.ndarray, rows: List[np.ndarray]) -> np.ndarray:
    """Each group's f64 sum of its rows, added row by row in order (from 0)."""
    d = x.shape[1]
    out = np.zeros((len(rows), d), np.float64)
    for g, r in enumerate(rows):
        acc = np.zeros(d, np.float64)
        for lo in range(0, len(r), 4096):
            blk = x[np.asarray(r[lo:lo + 4096], np.int64)].astype(np.float64)
            blk[0] += acc
            acc = np.add.accumulate(blk, axis=0)[-1]
        out[g] = acc
    return out


def unit_means(x: np.ndarray, rows: List[np.ndarray]) -> np.ndarray:
    """auto.rs:750-765: each group's f64 sum of its rows in order, cast to f32,
    then normalize_rows."""
    return normalize_rows(row_sums_f64(x, rows).astype(np.float32))


def model_from(centroids: np.ndarray, counts: List[int], d: int, nepochs: float, seed: int) -> Model:
    """auto.rs:955-987: a spherical model at the given centroids (positions
    too), masses count b / n (at least 1e-3) with b the recipe's batch size."""
    k = len(counts)
    n = max(sum(counts), 1)
    c = Config(d=d, k=k, spherical=True, nepochs=nepochs, seed=seed, capture_assignments=False,
               unused_threshold=0.0)
    b = recipe_batch(n, c)
    usage = np.array([np.float32(max(m * float(b) / float(n), 1e-3)) for m in counts], np.float32)
    cent = np.asarray(centroids, np.float32).reshape(k, d).copy()
    return Model(c, cent, cent.copy(), usage)


# ---------------------------------------------------------------- hierarchy
class Hierarchy:
    """auto.rs Hierarchy over a device backend: level 1, the groups' leaves,
    stable ids, outlier floors and the update counters."""

    def __init__(self, d: int, level1: Model, groups: List[Group], ids1: List[int],
                 state: State, backend, inc: Optional[IncrementalConfig] = None,
                 nepochs: float = 5.0, seed: int = 1234):
        self.d, self.level1, self.groups, self.ids1 = d, level1, groups, ids1
        self.state, self.backend = state, backend
        self.inc = inc or IncrementalConfig()
        self.nepochs, self.seed = nepochs, seed
        self.retrain = None  # full retrain (x_all) -> None, set by auto_cluster
        self.diagnostics = None

    @staticmethod
    def from_models(x: np.ndarray, level1: Model, leaves: List[Optional[Model]], backend,
                    inc: Optional[IncrementalConfig] = None, nepochs: float = 5.0,
                    seed: int = 1234) -> "Hierarchy":
        """A hierarchy from trained models, assembled as auto_cluster ends
        (auto.rs:1064-1100): ids 0.., state at n rows, floors from the labels
        of x, then x labelled again."""
        groups = [Group(m, list(range(m.k if m else 0)), np.full(m.k if m else 0, np.nan, np.float32),
                        m.k if m else 0) for m in leaves]
        h = Hierarchy(x.shape[1], level1, groups, list(range(level1.k)),
                      State.new(x.shape[0], level1.k), backend, inc, nepochs, seed)
        h.set_floors(h.assign(x))
        return h

    def level1_centroids(self) -> np.ndarray:
        return self.level1.centroids

    def leaf_centroids(self, g: int) -> np.ndarray:
        """auto.rs:1123-1128: group g's leaf centroids; its level-1 centroid
        when it has no model."""
        m = self.groups[g].model
        if m is not None:
            return m.centroids.reshape(-1, self.d)
        return self.level1_centroids().reshape(-1, self.d)[g:g + 1]

    def chosen_k(self):
        """auto.rs:1104-1113: (k1, [k2 of each group])."""
        return self.level1.k, [g.model.k if g.model is not None else 0 for g in self.groups]

    def assign(self, x: np.ndarray) -> Labels:
        """auto.rs:1135-1189: the nearest leaf over all leaves (cosine); level 1
        is that leaf's group; sim1 the f32 dot with the group's level-1
        centroid (rounded products added in order)."""
        x = np.ascontiguousarray(x, np.float32)
        d = self.d
        if x.ndim != 2 or x.shape[1] != d:
            raise ValueError("x must be n x d")
        cents, slot = [], []
        for g, grp in enumerate(self.groups):
            if grp.model is not None:
                cents.append(grp.model.centroids.reshape(-1, d))
                slot.extend((g, j) for j in range(grp.model.k))
        if not slot:
            raise ValueError("hierarchy has no leaves")
        leaf, sims = self.backend.leaf_top1(x, np.concatenate(cents))
        sl = np.asarray(slot, np.int64)[leaf.astype(np.int64)]
        slot1, slot2 = sl[:, 0].astype(np.uint32), sl[:, 1].astype(np.uint32)
        ids1 = np.asarray(self.ids1, np.uint32)
        c1 = self.level1_centroids().reshape(-1, d)
        l2 = np.zeros(x.shape[0], np.uint32)
        floor = np.full(x.shape[0], np.nan, np.float32)
        for g, grp in enumerate(self.groups):
            sel = slot1 == g
            if not sel.any():
                continue
            j = slot2[sel].astype(np.int64)
            ids = np.asarray(grp.ids + [0], np.uint32)
            l2[sel] = ids[np.minimum(j, len(grp.ids))]
            fl = np.concatenate([grp.floors.astype(np.float32), [np.float32(np.nan)]])
            floor[sel] = fl[np.minimum(j, len(grp.floors))]
        sim1 = np.empty(x.shape[0], np.float32)
        for lo in range(0, x.shape[0], 16384):
            p = (x[lo:lo + 16384] * c1[slot1[lo:lo + 16384]]).astype(np.float32)
            sim1[lo:lo + 16384] = np.add.accumulate(p, axis=1, dtype=np.float32)[:, -1]
        out = Labels(ids1[slot1], l2, sim1, sims.astype(np.float32),
                     np.isfinite(floor) & (sims < floor), slot1, slot2)
        return out

    def leaf_sims(self, labels: Labels):
        """auto.rs:1191-1205: every leaf's member cosines (in row order), group
        then leaf order."""
        at, first = [], []
        for g, grp in enumerate(self.groups):
            first.append(len(at))
            at.extend((g, j) for j in range(len(grp.ids)))
        nids = np.asarray([len(g.ids) for g in self.groups] + [0], np.int64)
        s1, s2 = labels.slot1.astype(np.int64), labels.slot2.astype(np.int64)
        keep = s2 < nids[s1]
        flat = np.asarray(first + [0], np.int64)[s1[keep]] + s2[keep]
        order = np.argsort(flat, kind="stable")
        cuts = np.searchsorted(flat[order], np.arange(len(at) + 1))
        sv = labels.sim[keep][order].astype(np.float32)
        return at, [sv[cuts[i]:cuts[i + 1]] for i in range(len(at))]

    def set_floors(self, labels: Labels):
        """auto.rs:1207-1215."""
        at, sims = self.leaf_sims(labels)
        floors = leaf_floors(sims, self.inc)
        for grp in self.groups:
            grp.floors = np.full(len(grp.ids), np.nan, np.float32)
        for (g, j), f in zip(at, floors):
            self.groups[g].floors[j] = f

    def add(self, x_all: np.ndarray, n_old: int) -> AddReport:
        """incremental.rs:306-360: label rows n_old.. and act by the policy."""
        x_all = np.ascontiguousarray(x_all, np.float32)
        n = x_all.shape[0]
        if n_old != self.state.n_seen:
            raise ValueError(f"the model has seen {self.state.n_seen} rows but n_old is {n_old}")
        if n < n_old:
            raise ValueError("x_all has fewer rows than n_old")
        fresh = self.assign(x_all[n_old:])
        new_outliers = int(fresh.outlier.sum())
        inc, st = self.inc, self.state
        st.pending.extend(int(n_old + i) for i in np.flatnonzero(fresh.outlier))
        m = n - n_old
        st.n_seen = n
        st.added_since_full += m
        st.added_since_update += m
        st.outliers_since_full += new_outliers
        outlier_fraction = st.outliers_since_full / max(st.added_since_full, 1)
        added_full = st.added_since_full / max(st.n_full, 1)
        added_update = st.added_since_update / max(st.n_update, 1)
        bucket_full = len(st.pending) >= inc.update_min_outliers
        if added_full >= inc.retrain_added_fraction or (
                bucket_full and outlier_fraction >= inc.retrain_outlier_fraction):
            action = "FullRetrain"
        elif bucket_full or added_update >= inc.update_added_fraction:
            action = "EmaUpdate"
        else:
            action = "AssignOnly"
        new_leaves = []
        if action == "EmaUpdate":
            new_leaves = self.ema_update(x_all)
        elif action == "FullRetrain":
            if self.retrain is None:
                raise NotImplementedError("a full retrain needs a hierarchy from auto_cluster")
            self.retrain(x_all)
        return AddReport(action, self.assign(x_all), new_outliers, len(self.state.pending),
                         outlier_fraction, new_leaves)

    def _grow(self, x_all: np.ndarray):
        """incremental.rs:376-395: the grow step's early exits; forming leaves
        from coherent pending outliers is not built here."""
        min_size = self.inc.grow_min_size
        if min_size == 0 or len(self.state.pending) < min_size:
            return []
        labels = self.assign(x_all)
        pend = [i for i in self.state.pending if labels.outlier[i]]
        if len(pend) < min_size:
            return []
        raise NotImplementedError("forming leaves from pending outliers (grow) is not built here")

    def ema_update(self, x_all: np.ndarray):
        """incremental.rs:546-596: leaves resume on their groups' rows for
        update_epochs, keeping stable ids by matching; level 1 follows."""
        d, n = self.d, x_all.shape[0]
        new_leaves = self._grow(x_all)
        labels = self.assign(x_all)
        rows = [np.flatnonzero(labels.slot1 == g) for g in range(len(self.groups))]
        for g, grp in enumerate(self.groups):
            mdl = grp.model
            if mdl is None or len(rows[g]) < mdl.k:
                continue
            old2 = mdl.centroids.copy()
            c = Config(**{**mdl.config.__dict__, "nepochs": self.inc.update_epochs})
            cent, pos, usage = self.backend.resume(c, x_all[rows[g]], mdl.positions, mdl.usage)
            mdl.centroids = np.asarray(cent, np.float32).reshape(mdl.k, d)
            mdl.positions, mdl.usage = pos, usage
            m2 = match_centroids(old2, mdl.centroids, d, self.inc.match_min_sim)
            grp.ids, grp.next_id = carry_ids(m2, grp.ids, grp.next_id)
        labels = self.assign(x_all)
        k1 = len(self.groups)
        grp_rows = [np.flatnonzero(labels.slot1 == g) for g in range(k1)]
        c1 = unit_means(x_all, grp_rows)
        old1 = self.level1_centroids().reshape(-1, d)
        for g, r in enumerate(grp_rows):
            if len(r) == 0:
                c1[g] = old1[g]
        counts = [max(len(r), 1) for r in grp_rows]
        self.level1 = model_from(c1, counts, d, self.nepochs, self.seed)
        self.set_floors(self.assign(x_all))
        st = self.state
        st.pending.clear()
        st.added_since_update = 0
        st.n_update = n
        return new_leaves
