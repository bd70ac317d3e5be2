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
  add_photos         incremental.rs:615-860   new photos against the dedup
                                        groups of the old ones (neighbours and
                                        the new groups' dedup on the device),
                                        then add of the representatives
  grow               incremental.rs:376-458   new leaves from coherent pending
                                        outliers: the candidates' pairwise dots
                                        and their dots with each trial mean on
                                        the device (fma chains)
  ema_update         incremental.rs:546-596   each group's leaves resume from
                                        their EMA state on the group's rows
                                        (the training loop on the device); the
                                        level 1 follows its groups' means

and on the host, as in the reference: the outlier floors (auto.rs:1194-1300),
the policy, the centroid matching that keeps stable ids (incremental.rs:
176-290), unit means (auto.rs:750-765), model_from (auto.rs:955-987), the
new leaf's placement (incremental.rs:460-538) and the hierarchy files
(incremental.rs:862-1073: a directory or one blob, each model in the model
file layout).

The full retrain runs auto_cluster (emeans_amd.autocluster) on all rows.

The device work goes through a backend object, so that the same host logic
runs over any device:
  leaf_top1(x, cents) -> (labels u32, sims f32)   top-1 by inner product
  resume(config, x, positions, usage) -> (centroids, positions, usage[, run])
  dots(a, b) -> a b^T                             f32 dots (grow)
HipBackend is the gfx950 one; it also returns each resumed run's record
(recipe, splits, epoch statistics) for the model files.
"""

import math
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

from . import Config, HipDevice, _epoch_rows, model_file, recipe_batch
from .auto import AutoConfig, Diagnostics, KScore

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
    """An e-means model's state: its config, centroids and EMA state (k x d),
    and what its last run recorded (recipe, splits, per-epoch statistics as
    (obj, time, imbalance_factor, nsplit)); a model made by model_from has
    run nothing (io.rs Snapshot with recipe None)."""
    config: Config
    centroids: np.ndarray
    positions: np.ndarray
    usage: np.ndarray
    recipe: Optional[dict] = None
    n_splits: int = 0
    stats: list = field(default_factory=list)

    @property
    def k(self) -> int:
        return self.config.k

    def to_bytes(self) -> bytes:
        """The model file's bytes (io.rs:92-121)."""
        return model_file.to_bytes(self.config, self.recipe, self.n_splits, self.stats,
                                   self.centroids, self.positions,
                                   self.usage if self.usage is not None else [])

    @staticmethod
    def from_bytes(b) -> "Model":
        """A model from a model file's bytes (io.rs:137-186)."""
        header, cent, pos, usage = model_file.from_bytes(b)
        cfg = Config(**header["config"])
        if cent is None:
            raise ValueError("model has no centroids")
        stats = [(s["obj"], s["time"], s["imbalance_factor"], int(s["nsplit"]))
                 for s in header["iteration_stats"]]
        return Model(cfg, cent.reshape(cfg.k, cfg.d), pos, usage, header["recipe"],
                     int(header["n_splits"]), stats)


def decision_split(k: int):
    """GroupDecision::Split (auto.rs:195-206) as serde writes it."""
    return {"split": {"k": int(k)}}


def decision_no_structure(best: float):
    """GroupDecision::NoStructure (auto.rs:195-206) as serde writes it."""
    return {"no_structure": {"best_silhouette": float(best)}}


DECISION_EMPTY, DECISION_TOO_SMALL = "empty", "too_small"


@dataclass
class Group:
    """A level-1 slot (auto.rs Group): its leaves' model, their stable ids,
    outlier floors, the next unused id and why it has the level-2 k it has
    (GroupDecision, held as its serde value)."""
    model: Optional[Model]
    ids: List[int]
    floors: np.ndarray
    next_id: int
    decision: object = DECISION_TOO_SMALL


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
        """train_resume on x: (centroids, positions, usage, the run's record)."""
        n, d = x.shape
        cent, info = self.dev.train_dev(self.dev.bind(x), n, config, state=(positions, usage))
        run = {"recipe": model_file.recipe_dict(config, n, info["batch_size"], info["alpha0"],
                                                _epoch_rows(n, config), self.dev.name()),
               "n_splits": info["n_splits"],
               "stats": [(s.obj, s.time, s.imbalance_factor, s.nsplit) for s in info["stats"]]}
        return cent, info["positions"], info["usage"], run

    def dots(self, a: np.ndarray, b: np.ndarray) -> np.ndarray:
        return self.dev.dots(a, b)


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


def pooled_floor(median, sp: Spread, inc: IncrementalConfig) -> np.float32:
    """auto.rs:1294-1300: the floor of a leaf whose median member cosine is
    median, with the pooled spread (f32, left to right)."""
    if inc.outlier_min_sim is not None:
        return np.float32(inc.outlier_min_sim)
    return np.float32(np.float32(median) - np.float32(inc.outlier_mad_k) * MAD_SIGMA *
                      sp.pooled_mad)


def _dot_sum(a: np.ndarray, b: np.ndarray) -> np.float32:
    """The f32 sum, in order, of the rounded products a_t b_t
    (incremental.rs:462, iterator sum)."""
    p = (np.asarray(a, np.float32) * np.asarray(b, np.float32)).astype(np.float32)
    return np.float32(np.add.accumulate(p, dtype=np.float32)[-1]) if p.size else np.float32(0)


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
    """Each group's f64 sum of its rows, added row by row in order (from 0).
    numpy reduces axis 0 of a C-contiguous block one row after another into
    the accumulator (the pairwise scheme is for the contiguous axis), so the
    reduce is that chain; tests/test_hierarchy_host.py holds it bit-equal to
    the running sums of np.add.accumulate."""
    d = x.shape[1]
    out = np.zeros((len(rows), d), np.float64)
    for g, r in enumerate(rows):
        acc = np.zeros(d, np.float64)
        for lo in range(0, len(r), 4096):
            blk = x[np.asarray(r[lo:lo + 4096], np.int64)].astype(np.float64)
            blk[0] += acc
            acc = np.add.reduce(blk, axis=0)
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
                 nepochs: float = 5.0, seed: int = 1234, config: Optional[AutoConfig] = None,
                 dedup=None):
        self.d, self.level1, self.groups, self.ids1 = d, level1, groups, ids1
        self.state, self.backend = state, backend
        self.inc = inc or IncrementalConfig()
        # The AutoConfig the hierarchy was built with (its policy is self.inc).
        self.config = config if config is not None else AutoConfig(nepochs=nepochs, seed=seed)
        self.nepochs, self.seed = self.config.nepochs, self.config.seed
        self.dedup = dedup  # DedupConfig used upstream, or None
        self.diagnostics = Diagnostics()

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

    # -- files (incremental.rs:862-1047); the functions are below the class
    def to_bytes(self) -> bytes:
        """The hierarchy as one blob (incremental.rs:898-915)."""
        return _hierarchy_to_bytes(self)

    @staticmethod
    def from_bytes(b, backend) -> "Hierarchy":
        """A hierarchy from the bytes of to_bytes (incremental.rs:917-946)."""
        return _hierarchy_from_bytes(b, backend)

    def save(self, path):
        """Write the hierarchy to directory path, replaced as a whole (incremental.rs:864-894)."""
        _hierarchy_save(self, path)

    @staticmethod
    def load(path, backend) -> "Hierarchy":
        """A hierarchy written by save (incremental.rs:978-988)."""
        return _hierarchy_load(path, backend)

    def add_photos(self, photos, n_old: int, dd, input=None, dev=None) -> "PhotoAddReport":
        """New photos when the hierarchy clusters dedup representatives
        (incremental.rs:615-860); the function below the class."""
        return add_photos(self, photos, n_old, dd, input, dev)

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
        # Per leaf of the concatenation: its stable id (0 past the group's
        # ids) and its floor (NaN past the group's floors).
        l2_of, floor_of = [], []
        for g, grp in enumerate(self.groups):
            if grp.model is None:
                continue
            j = np.arange(grp.model.k)
            ids = np.asarray(grp.ids + [0], np.uint32)
            fl = np.concatenate([grp.floors.astype(np.float32), [np.float32(np.nan)]])
            l2_of.append(ids[np.minimum(j, len(grp.ids))])
            floor_of.append(fl[np.minimum(j, len(grp.floors))])
        li = leaf.astype(np.int64)
        l2 = np.concatenate(l2_of)[li]
        floor = np.concatenate(floor_of).astype(np.float32)[li]
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
            self.full_retrain(x_all)
        return AddReport(action, self.assign(x_all), new_outliers, len(self.state.pending),
                         outlier_fraction, new_leaves)

    def full_retrain(self, x_all: np.ndarray):
        """incremental.rs:598-633: auto_cluster on all rows on the device,
        old ids carried over (emeans_amd.autocluster.full_retrain)."""
        dev = getattr(self.backend, "dev", None)
        if dev is None:
            raise NotImplementedError("a full retrain runs auto_cluster on a device backend")
        from . import autocluster
        autocluster.full_retrain(dev, self, x_all, self.config)

    def grow(self, x_all: np.ndarray):
        """incremental.rs:376-458: new leaves from the pending rows that are
        still outliers and form coherent groups. The row with the most
        candidates within `pair` seeds a group; four rounds of mean and
        members (within the pooled floor of the leaves' 10 % median cosine,
        and nearer than their current leaf); a group of grow_min_size rows
        whose median cosine to its mean reaches that cohesion becomes a leaf
        (add_leaf); three failed seeds end the search. The dots (gemm_nt in
        the reference) run on the backend: the device's fma chains."""
        d, inc = self.d, self.inc
        min_size = inc.grow_min_size
        made = []
        if min_size == 0 or len(self.state.pending) < min_size:
            return made
        labels = self.assign(x_all)
        pend = np.asarray([i for i in self.state.pending if labels.outlier[i]], np.int64)
        p = len(pend)
        if p < min_size:
            return made
        _, sims = self.leaf_sims(labels)
        sp = spread(sims)
        medians = [m for m in sp.median if np.isfinite(m)]
        cohesion = quantile(np.asarray(medians, np.float32), 0.10)
        floor = pooled_floor(cohesion, sp, inc)
        if not np.isfinite(floor):
            raise ValueError("no leaf statistics to grow from")
        f0 = np.float32(max(floor, np.float32(0.0)))
        pair = np.float32(f0 * f0)
        xp = np.ascontiguousarray(x_all[pend], np.float32)
        cur = labels.sim[pend].astype(np.float32)
        degree = np.zeros(p, np.int64)
        for b0 in range(0, p, 1024):
            out = self.backend.dots(xp[b0:b0 + 1024], xp)
            degree[b0:b0 + len(out)] = ((out >= pair).sum(axis=1) - 1) & 0xFFFFFFFF

        def to(c):
            return self.backend.dots(xp, np.asarray(c, np.float32).reshape(1, d))[:, 0]

        def mean_of(mem):
            return unit_means(xp, [np.asarray(mem, np.int64)])[0]

        free = np.ones(p, bool)
        tried = np.zeros(p, bool)
        fails = 0
        while fails < 3 and int(free.sum()) >= min_size:
            cand = np.flatnonzero(free & ~tried)
            if len(cand) == 0:
                break
            # max_by_key((degree, Reverse(t))): the highest degree, then the lowest t
            seed = int(cand[np.lexsort((cand, -degree[cand]))[0]])
            tried[seed] = True
            s0 = to(xp[seed])
            mem = np.flatnonzero(free & (s0 >= pair))
            for _ in range(4):
                if len(mem) < min_size:
                    break
                s = to(mean_of(mem))
                mem = np.flatnonzero(free & (s >= floor) & (s > cur))
            if len(mem) < min_size:
                fails += 1
                continue
            center = mean_of(mem)
            s = to(center)
            if quantile(s[mem], 0.5) < cohesion:
                fails += 1
                continue
            free[mem] = False
            made.append(self.add_leaf(center, len(mem), labels))
        return made

    def add_leaf(self, center: np.ndarray, rows: int, labels: Labels):
        """incremental.rs:460-538: the new leaf joins the level-1 group (of two
        or more leaves) whose centroid it is as close to as that group's own
        leaves are, the closest such group; otherwise it becomes a new level-1
        group. Slots are appended; models are rebuilt by model_from with the
        current labels' counts. Returns the leaf's stable (level-1, leaf) ids."""
        d = self.d
        center = np.asarray(center, np.float32).reshape(d)
        c1 = self.level1_centroids().reshape(-1, d)
        home = None
        for g, grp in enumerate(self.groups):
            m = grp.model
            if m is None or m.k < 2:
                continue
            cg = c1[g]
            reach = np.float32(np.inf)
            for leaf in m.centroids.reshape(-1, d):
                v = _dot_sum(leaf, cg)
                if not np.isnan(v):
                    reach = min(reach, v)  # fold(inf, f32::min)
            s = _dot_sum(center, cg)
            if s >= reach and (home is None or s > home[0]):
                home = (s, g)
        ng = len(self.groups)
        count1 = np.bincount(labels.slot1.astype(np.int64), minlength=ng)[:ng]
        if home is not None:
            g = home[1]
            grp = self.groups[g]
            k = grp.model.k
            cents = np.concatenate([grp.model.centroids.reshape(k, d), center[None, :]])
            sel = labels.slot1 == g
            counts = np.bincount(labels.slot2[sel].astype(np.int64), minlength=k)[:k]
            counts = [max(int(c), 1) for c in counts] + [rows]
            grp.model = model_from(cents, counts, d, self.nepochs, self.seed)
            nid = grp.next_id
            grp.next_id += 1
            grp.ids.append(nid)
            grp.floors = np.append(grp.floors.astype(np.float32), np.float32(np.nan))
            grp.decision = decision_split(k + 1)
            return (self.ids1[g], nid)
        model = model_from(center[None, :], [rows], d, self.nepochs, self.seed)
        self.groups.append(Group(model, [0], np.full(1, np.nan, np.float32), 1,
                                 DECISION_TOO_SMALL))
        id1 = self.state.next_id1
        self.state.next_id1 += 1
        self.ids1.append(id1)
        cents1 = np.concatenate([c1, center[None, :]])
        counts1 = [max(int(c), 1) for c in count1] + [rows]
        self.level1 = model_from(cents1, counts1, d, self.nepochs, self.seed)
        return (id1, 0)

    def ema_update(self, x_all: np.ndarray):
        """incremental.rs:546-596: leaves resume on their groups' rows for
        update_epochs, keeping stable ids by matching; level 1 follows."""
        d, n = self.d, x_all.shape[0]
        new_leaves = self.grow(x_all)
        labels = self.assign(x_all)
        rows = [np.flatnonzero(labels.slot1 == g) for g in range(len(self.groups))]
        for g, grp in enumerate(self.groups):
            mdl = grp.model
            if mdl is None or len(rows[g]) < mdl.k:
                continue
            old2 = mdl.centroids.copy()
            c = Config(**{**mdl.config.__dict__, "nepochs": self.inc.update_epochs})
            r = self.backend.resume(c, x_all[rows[g]], mdl.positions, mdl.usage)
            cent, pos, usage = r[:3]
            mdl.centroids = np.asarray(cent, np.float32).reshape(mdl.k, d)
            mdl.positions, mdl.usage = pos, usage
            if len(r) > 3:  # the run's record, kept for the model file
                mdl.recipe, mdl.n_splits, mdl.stats = r[3]["recipe"], r[3]["n_splits"], \
                    r[3]["stats"]
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


# ---------------------------------------------------------------- hierarchy files
# incremental.rs:862-1070. A directory holds hierarchy.json (the manifest,
# serde_json's pretty form), level1.emeans and group-<g>.emeans for every
# group with a model. The blob is EMHIER\0\x01, u64 manifest length, the
# manifest (compact), then each model as u64 length + model file bytes (level
# 1, then the groups with a model, in group order); little-endian.
MANIFEST_VERSION = 1
BLOB_MAGIC = b"EMHIER\x00\x01"


def _opt_f32(v):
    return None if v is None else model_file.F32(float(np.float32(v)))


def _kscore_dict(s: KScore):
    """KScore (auto.rs:178-192), fields in declaration order."""
    return {"k": int(s.k), "k_eff": int(s.k_eff), "silhouette": float(s.silhouette),
            "calinski_harabasz": float(s.calinski_harabasz),
            "davies_bouldin": float(s.davies_bouldin), "objective": float(s.objective),
            "browsable": float(s.browsable), "seconds": float(s.seconds)}


def _f64(v, what):
    """An f64 field: serde reads null (a non-finite value it wrote) as an error."""
    if isinstance(v, bool) or not isinstance(v, (int, float)):
        raise ValueError(f"invalid type for {what}: expected f64, found {json_type(v)}")
    return float(v)


def json_type(v):
    return "null" if v is None else type(v).__name__


def _kscore(d) -> KScore:
    return KScore(int(d["k"]), int(d["k_eff"]),
                  *[_f64(d[f], f) for f in ("silhouette", "calinski_harabasz", "davies_bouldin",
                                             "objective", "browsable", "seconds")])


def _auto_config_dict(c: AutoConfig, inc: IncrementalConfig):
    """AutoConfig (auto.rs:99-147) without the backend (serde skip), with
    IncrementalConfig (incremental.rs:52-83) in its place before verbose."""
    return {"k1_range": [int(c.k1_range[0]), int(c.k1_range[1])], "k2_max": int(c.k2_max),
            "criterion1": c.criterion1, "criterion2": c.criterion2,
            "level1_tolerance": float(c.level1_tolerance),
            "level2_tolerance": float(c.level2_tolerance),
            "min_cluster_size": int(c.min_cluster_size),
            "max_cluster_size": int(c.max_cluster_size), "min_split_size": int(c.min_split_size),
            "split_min_silhouette": float(c.split_min_silhouette), "restarts": int(c.restarts),
            "nepochs": float(c.nepochs), "init": c.init, "level1_method": c.level1_method,
            "resplit_passes": int(c.resplit_passes),
            "level1_max_share": float(c.level1_max_share), "seed": int(c.seed) & 0xFFFFFFFF,
            "incremental": {
                "outlier_mad_k": float(inc.outlier_mad_k),
                "outlier_min_sim": _opt_f32(inc.outlier_min_sim),
                "grow_min_size": int(inc.grow_min_size),
                "update_min_outliers": int(inc.update_min_outliers),
                "update_added_fraction": float(inc.update_added_fraction),
                "update_epochs": float(inc.update_epochs),
                "retrain_added_fraction": float(inc.retrain_added_fraction),
                "retrain_outlier_fraction": float(inc.retrain_outlier_fraction),
                "match_min_sim": _opt_f32(inc.match_min_sim)},
            "verbose": bool(c.verbose)}


def _auto_config(d):
    """AutoConfig and IncrementalConfig from the manifest, serde's defaults
    for the fields marked #[serde(default)]."""
    i = d["incremental"]
    inc = IncrementalConfig(
        outlier_mad_k=_f64(i.get("outlier_mad_k", 3.0), "outlier_mad_k"),
        outlier_min_sim=None if i["outlier_min_sim"] is None else float(np.float32(
            i["outlier_min_sim"])),
        grow_min_size=int(i.get("grow_min_size", 20)),
        update_min_outliers=int(i["update_min_outliers"]),
        update_added_fraction=_f64(i["update_added_fraction"], "update_added_fraction"),
        update_epochs=_f64(i["update_epochs"], "update_epochs"),
        retrain_added_fraction=_f64(i["retrain_added_fraction"], "retrain_added_fraction"),
        retrain_outlier_fraction=_f64(i["retrain_outlier_fraction"], "retrain_outlier_fraction"),
        match_min_sim=float(np.float32(_f64(i["match_min_sim"], "match_min_sim"))))
    for key, allowed in (("criterion1", CRITERIA), ("criterion2", CRITERIA),
                         ("init", ("k_means_plus_plus", "random_rows")),
                         ("level1_method", ("bottom_up", "top_down"))):
        if d.get(key, "bottom_up") not in allowed:
            raise ValueError(f"unknown variant {d.get(key)!r} for {key}")
    c = AutoConfig(
        k1_range=(int(d["k1_range"][0]), int(d["k1_range"][1])), k2_max=int(d["k2_max"]),
        criterion1=d["criterion1"], criterion2=d["criterion2"],
        level1_tolerance=_f64(d["level1_tolerance"], "level1_tolerance"),
        level2_tolerance=_f64(d["level2_tolerance"], "level2_tolerance"),
        min_cluster_size=int(d["min_cluster_size"]), max_cluster_size=int(d["max_cluster_size"]),
        min_split_size=int(d["min_split_size"]),
        split_min_silhouette=_f64(d["split_min_silhouette"], "split_min_silhouette"),
        restarts=int(d["restarts"]), nepochs=_f64(d["nepochs"], "nepochs"), init=d["init"],
        level1_method=d.get("level1_method", "bottom_up"),
        resplit_passes=int(d.get("resplit_passes", 2)),
        level1_max_share=_f64(d.get("level1_max_share", 0.5), "level1_max_share"),
        seed=int(d["seed"]), verbose=bool(d["verbose"]))
    return c, inc


CRITERIA = ("silhouette", "calinski_harabasz", "davies_bouldin")


def _dedup_dict(c):
    """DedupConfig (dedup.rs:39-51)."""
    if c is None:
        return None
    return {"k": int(c.k), "sim_threshold": model_file.F32(float(np.float32(c.sim_threshold))),
            "rep_threshold": _opt_f32(c.rep_threshold),
            "max_gap_secs": None if c.max_gap_secs is None else float(c.max_gap_secs)}


def _dedup(d):
    if d is None:
        return None
    from . import DedupConfig
    return DedupConfig(int(d["k"]), float(np.float32(_f64(d["sim_threshold"], "sim_threshold"))),
                       None if d["rep_threshold"] is None else float(np.float32(
                           d["rep_threshold"])),
                       None if d["max_gap_secs"] is None else float(d["max_gap_secs"]))


def _decision(v):
    """GroupDecision from its serde value (externally tagged, snake_case)."""
    if v in (DECISION_EMPTY, DECISION_TOO_SMALL):
        return v
    if isinstance(v, dict) and len(v) == 1:
        if "split" in v:
            return decision_split(int(v["split"]["k"]))
        if "no_structure" in v:
            return decision_no_structure(_f64(v["no_structure"]["best_silhouette"],
                                              "best_silhouette"))
    raise ValueError(f"unknown group decision {v!r}")


def _diag_dict(g: Diagnostics):
    """Diagnostics (auto.rs:209-238), fields in declaration order."""
    return {"level1": [_kscore_dict(s) for s in g.level1],
            "level2": [[_kscore_dict(s) for s in sw] for sw in g.level2],
            "seconds": float(g.seconds),
            "stage_a_level1": [_kscore_dict(s) for s in g.stage_a_level1],
            "resplits": int(g.resplits), "leaves": int(g.leaves), "gap_k": int(g.gap_k),
            "flat": bool(g.flat), "level1_rejected": [int(k) for k in g.level1_rejected]}


def _diag(d) -> Diagnostics:
    return Diagnostics(level1=[_kscore(s) for s in d["level1"]],
                       level2=[[_kscore(s) for s in sw] for sw in d["level2"]],
                       seconds=_f64(d["seconds"], "seconds"),
                       stage_a_level1=[_kscore(s) for s in d.get("stage_a_level1", [])],
                       resplits=int(d.get("resplits", 0)), leaves=int(d.get("leaves", 0)),
                       gap_k=int(d.get("gap_k", 0)), flat=bool(d.get("flat", False)),
                       level1_rejected=[int(k) for k in d.get("level1_rejected", [])])


def _state_dict(st: State):
    """State (incremental.rs:105-122)."""
    return {"n_seen": int(st.n_seen), "n_full": int(st.n_full), "n_update": int(st.n_update),
            "added_since_full": int(st.added_since_full),
            "outliers_since_full": int(st.outliers_since_full),
            "added_since_update": int(st.added_since_update),
            "pending": [int(i) for i in st.pending], "next_id1": int(st.next_id1)}


def manifest(h: "Hierarchy"):
    """Manifest (incremental.rs:1052-1073, built at 949-975): floors that are
    not finite are written as null."""
    return {"version": MANIFEST_VERSION, "d": int(h.d),
            "config": _auto_config_dict(h.config, h.inc), "dedup": _dedup_dict(h.dedup),
            "ids1": [int(i) for i in h.ids1],
            "groups": [{"has_model": g.model is not None, "ids": [int(i) for i in g.ids],
                        "floors": [model_file.F32(float(f)) if np.isfinite(f) else None
                                   for f in np.asarray(g.floors, np.float32)],
                        "decision": g.decision, "next_id": int(g.next_id)}
                       for g in h.groups],
            "diagnostics": _diag_dict(h.diagnostics), "state": _state_dict(h.state)}


def _assemble(mf, backend, model) -> "Hierarchy":
    """incremental.rs:990-1047: the hierarchy of a manifest; model(None)
    reads the level-1 model, model(g) group g's, in that order."""
    if mf["version"] != MANIFEST_VERSION:
        raise ValueError(f"unsupported hierarchy version {mf['version']}")
    d = int(mf["d"])
    cfg, inc = _auto_config(mf["config"])
    level1 = model(None)
    if level1.config.d != d:
        raise ValueError("level-1 model d differs from the manifest")
    ids1 = [int(i) for i in mf["ids1"]]
    if level1.k != len(ids1) or len(mf["groups"]) != len(ids1):
        raise ValueError("level-1 k, ids and groups disagree")
    groups = []
    for g, gf in enumerate(mf["groups"]):
        m = None
        ids = [int(i) for i in gf["ids"]]
        if gf["has_model"]:
            m = model(g)
            if m.k != len(ids) or m.config.d != d:
                raise ValueError(f"group {g}: model and ids disagree")
        floors = np.array([np.nan if f is None else f for f in gf["floors"]], np.float32)
        groups.append(Group(m, ids, floors, int(gf["next_id"]), _decision(gf["decision"])))
    st = mf["state"]
    state = State(int(st["n_seen"]), int(st["n_full"]), int(st["n_update"]),
                  int(st["added_since_full"]), int(st["outliers_since_full"]),
                  int(st["added_since_update"]), [int(i) for i in st["pending"]],
                  int(st["next_id1"]))
    h = Hierarchy(d, level1, groups, ids1, state, backend, inc, config=cfg,
                  dedup=_dedup(mf["dedup"]))
    h.diagnostics = _diag(mf["diagnostics"])
    return h


def _hierarchy_to_bytes(h: "Hierarchy") -> bytes:
    """Hierarchy::to_bytes (incremental.rs:898-915)."""
    import struct
    js = model_file.to_json(manifest(h)).encode()
    parts = [BLOB_MAGIC, struct.pack("<Q", len(js)), js]
    for m in [h.level1] + [g.model for g in h.groups if g.model is not None]:
        b = m.to_bytes()
        parts += [struct.pack("<Q", len(b)), b]
    return b"".join(parts)


def _hierarchy_from_bytes(b, backend) -> "Hierarchy":
    """Hierarchy::from_bytes (incremental.rs:917-946): the same checks and errors."""
    import json
    import struct
    b = bytes(b)
    if len(b) < 8 or b[:8] != BLOB_MAGIC:
        raise ValueError("not an emeans hierarchy")
    off = 8

    def take(what):
        nonlocal off
        if len(b) - off < 8:
            raise ValueError(f"truncated {what}")
        n = struct.unpack("<Q", b[off:off + 8])[0]
        if n > len(b) - off - 8:
            raise ValueError(f"truncated {what}")
        part = b[off + 8:off + 8 + n]
        off += 8 + n
        return part

    mf = json.loads(take("manifest"))

    def model(g):
        what = "level-1 model" if g is None else f"group {g} model"
        part = take(what)
        try:
            return Model.from_bytes(part)
        except ValueError as e:
            raise ValueError(f"{what}: {e}") from e

    h = _assemble(mf, backend, model)
    if off != len(b):
        raise ValueError(f"{len(b) - off} bytes after the last model")
    return h


def _hierarchy_save(h: "Hierarchy", path):
    """Hierarchy::save (incremental.rs:864-894): the directory is written as
    <dir>.tmp, then renamed over <dir> (the old one moved to <dir>.old and
    removed)."""
    import os
    import shutil
    path = os.fspath(path).rstrip("/") or "/"
    base = os.path.splitext(path)[0]
    tmp, old = base + ".tmp", base + ".old"
    if os.path.exists(tmp):
        shutil.rmtree(tmp)
    os.makedirs(tmp)
    model_file.save_bytes(os.path.join(tmp, "level1.emeans"), h.level1.to_bytes())
    for g, grp in enumerate(h.groups):
        if grp.model is not None:
            model_file.save_bytes(os.path.join(tmp, f"group-{g}.emeans"), grp.model.to_bytes())
    with open(os.path.join(tmp, "hierarchy.json"), "wb") as f:
        f.write(model_file.to_json_pretty(manifest(h)).encode())
    if os.path.exists(old):
        shutil.rmtree(old)
    if os.path.exists(path):
        os.rename(path, old)
    os.rename(tmp, path)
    if os.path.exists(old):
        shutil.rmtree(old)


def _hierarchy_load(path, backend) -> "Hierarchy":
    """Hierarchy::load (incremental.rs:978-988)."""
    import json
    import os
    path = os.fspath(path)
    try:
        with open(os.path.join(path, "hierarchy.json"), "rb") as f:
            mf = json.loads(f.read())
    except OSError as e:
        raise ValueError(f"read {path}/hierarchy.json: {e}") from e

    def model(g):
        name = "level1.emeans" if g is None else f"group-{g}.emeans"
        with open(os.path.join(path, name), "rb") as f:
            return Model.from_bytes(f.read())

    return _assemble(mf, backend, model)



# ---------------------------------------------------------------- photos
@dataclass
class PhotoAddReport:
    """incremental.rs PhotoAddReport: new photos that joined existing dedup
    groups, new groups formed, every photo's stable leaf and outlier flag (via
    its group's representative), and the representatives' AddReport."""
    joined_existing: int
    new_groups: int
    leaf: list
    outlier: np.ndarray
    reps: AddReport


def add_photos(h: "Hierarchy", photos, n_old: int, dd, input=None, dev=None) -> PhotoAddReport:
    """Hierarchy::add_photos (incremental.rs:615-860) when the hierarchy
    clusters dedup representatives. Each new photo joins an existing group when
    it shares a burst id with one of the group's photos, or when one of its k
    neighbours among all photos is an old photo with cos >= sim_threshold (and
    the time rule) and the photo is within rep_threshold of that group's anchor
    (and the time rule to it); the closest such anchor wins, and a new burst
    joins only when every one of its photos fits. The rest are grouped among
    themselves by dedup, each new group appending one representative, which
    then go through Hierarchy.add. dd (a DedupResult of the old photos) is
    updated in place. The neighbours and the new groups' dedup run on the
    device; the star rule's dots are f32 sums in order, as the reference's."""
    from . import NONE, DedupConfig, DedupInput, dedup, knn
    d = h.d
    photos = np.ascontiguousarray(photos, np.float32)
    if photos.size % d:
        raise ValueError("photos must be n x d")
    photos = photos.reshape(-1, d)
    n = photos.shape[0]
    if n < n_old:
        raise ValueError("photos has fewer rows than n_old")
    if len(dd.group_of) != n_old:
        raise ValueError(f"dedup result covers {len(dd.group_of)} photos but n_old is {n_old}")
    n_reps_old = len(dd.representatives)
    if n_reps_old != h.state.n_seen:
        raise ValueError(f"the hierarchy has seen {h.state.n_seen} rows but the dedup result "
                         f"has {n_reps_old} groups")
    inp = input or DedupInput()
    t_all = None if inp.created_unix is None else np.asarray(inp.created_unix, np.float64)
    if t_all is not None and len(t_all) != n:
        raise ValueError("one timestamp per photo")
    if inp.burst is not None and len(inp.burst) != n:
        raise ValueError("one burst id per photo")
    if inp.priority is not None and len(inp.priority) != n:
        raise ValueError("one priority per photo")
    if dev is None:
        dev = getattr(h.backend, "dev", None)
        if dev is None:
            raise ValueError("add_photos needs a device for its neighbours and dedup")
    cfg = h.dedup if h.dedup is not None else DedupConfig()
    sim_t = np.float32(cfg.sim_threshold)
    rep_t = np.float32(cfg.rep_threshold if cfg.rep_threshold is not None else cfg.sim_threshold)

    def time_ok(i, j):
        if cfg.max_gap_secs is None or t_all is None:
            return True
        a, b = t_all[i], t_all[j]
        if not (np.isfinite(a) and np.isfinite(b)):
            return True
        return abs(a - b) <= cfg.max_gap_secs

    m = n - n_old
    # Neighbours of the new photos among all photos (self excluded below).
    k = max(min(cfg.k, max(n - 1, 0)), 1)
    nb = knn(photos[n_old:], photos, d, k + 1, dev) if m > 0 and n > 1 else None
    # Results written before anchors were stored tested against the representative.
    if len(dd.anchors) != n_reps_old:
        dd.anchors = np.asarray(dd.representatives, np.uint32).copy()
    burst = inp.burst
    burst_group = {}
    if burst is not None:
        for i in range(n_old):
            if burst[i] is not None and burst[i] not in burst_group:
                burst_group[burst[i]] = int(dd.group_of[i])
    # Units of new photos: a burst is one unit and always stays together.
    units, unit_of_burst = [], {}
    for t in range(m):
        bid = burst[n_old + t] if burst is not None else None
        if bid is None:
            units.append([t])
        else:
            if bid not in unit_of_burst:
                unit_of_burst[bid] = len(units)
                units.append([])
            units[unit_of_burst[bid]].append(t)

    def fits(i, g):
        """The star rule of dedup: within the threshold of the group's anchor."""
        a = dd.anchor(g)
        s = _dot_sum(photos[i], photos[a])
        return s if (s >= rep_t and time_ok(i, a)) else None

    joined = [None] * m
    nn_new = np.full(m, -np.inf, np.float32)
    for unit in units:
        linked, forced = set(), None
        for t in unit:
            i = n_old + t
            if forced is None and burst is not None and burst[i] is not None:
                forced = burst_group.get(burst[i])
            if nb is None:
                continue
            ids, sims = nb.row(t)
            for j, s in zip(ids.tolist(), sims):
                if j == NONE or j == i:
                    continue
                if s > nn_new[t]:
                    nn_new[t] = s
                if j < n_old and s >= sim_t and time_ok(i, j):
                    linked.add(int(dd.group_of[j]))
        # Every row of the unit must fit the anchor; the closest anchor wins.
        best = None
        for g in sorted(linked):
            worst = np.float32(np.inf)
            for t in unit:
                s = fits(n_old + t, g)
                if s is None:
                    worst = None
                    break
                worst = min(worst, s)
            if worst is not None and (best is None or worst > best[0]):
                best = (worst, g)
        group = forced if forced is not None else (best[1] if best is not None else None)
        for t in unit:
            joined[t] = group

    # Group the remaining new photos among themselves.
    rest = [t for t in range(m) if joined[t] is None]
    group_of_new = np.array([0xFFFFFFFF if g is None else g for g in joined], np.uint32)
    new_groups = sub_split = sub_pairs = 0
    reps, anchors, sizes = list(dd.representatives), list(dd.anchors), list(dd.sizes)
    if rest:
        idx = np.array([n_old + t for t in rest], np.int64)
        sub_in = DedupInput(
            None if t_all is None else t_all[idx],
            None if burst is None else [burst[i] for i in idx],
            None if inp.priority is None else np.asarray(inp.priority, np.float32)[idx])
        r = dedup(photos[idx], d, sub_in, cfg, dev)
        base = len(reps)
        for t, g in zip(rest, r.group_of.tolist()):
            group_of_new[t] = base + g
        for g, (rep, size) in enumerate(zip(r.representatives.tolist(), r.sizes.tolist())):
            reps.append(int(idx[rep]))
            anchors.append(int(idx[r.anchor(g)]))
            sizes.append(size)
        new_groups = r.n_groups()
        sub_split, sub_pairs = r.split_components, r.linked_pairs
    for g in group_of_new.tolist():
        if g < n_reps_old:
            sizes[g] += 1
    dd.representatives = np.array(reps, np.uint32)
    dd.anchors = np.array(anchors, np.uint32)
    dd.sizes = np.array(sizes, np.uint32)
    dd.group_of = np.concatenate([np.asarray(dd.group_of, np.uint32), group_of_new])
    dd.nn_sim = np.concatenate([np.asarray(dd.nn_sim, np.float32), nn_new])
    dd.split_components += sub_split
    dd.linked_pairs += sub_pairs

    report = h.add(photos[dd.representatives.astype(np.int64)], n_reps_old)
    g_of = dd.group_of.astype(np.int64)
    leaf = list(zip(report.labels.l1[g_of].tolist(), report.labels.l2[g_of].tolist()))
    return PhotoAddReport(sum(g is not None for g in joined), new_groups, leaf,
                          report.labels.outlier[g_of], report)
