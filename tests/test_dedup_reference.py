"""The reference's near-duplicate known-answer tests
(crates/emeans-cluster/tests/dedup.rs:112-300), restated on the same data
(tests/ref_synth.py restates its generators), for the oracle's dedup and for
the backend's host grouping (emh_dedup_neighbors through the C ABI; no GPU).

Both run on the same neighbours: the oracle's exact kNN with the query itself
excluded (knn_self), k = min(DedupConfig.k, n - 1) as dedup does
(dedup.rs:172). Each test first asserts that the two agree to the last field,
then the reference's own assertions. These pin the grouping rules
independently of either restatement: the star cover's bounded diameter, the
time gap, unknown times, burst units, priority, and "a burst joins a star only
when every row fits".
"""

import numpy as np
import pytest

from emeans_amd import DedupConfig, DedupInput, Neighbors, dedup_with_neighbors
from oracle import oracle as O

from .ref_synth import add_scaled, nested, normalize_rows, random_unit, unit, with_bursts, Normal

NONE = 0xFFFFFFFF


def _dot(x, a, b):
    """dedup.rs's dot: sequential f32 sum of the products."""
    return np.cumsum(x[a] * x[b], dtype=np.float32)[-1]


def _dedup(x, d, inp=DedupInput(), cfg=DedupConfig()):
    x = np.ascontiguousarray(x, np.float32).reshape(-1, d)
    n = x.shape[0]
    k = max(min(cfg.k, n - 1), 1)
    if n > 1:
        ids, sims = O.knn(x, x, d, k, True)
    else:
        ids, sims = np.full(n, NONE, np.uint32), np.full(n, -np.inf, np.float32)
    want = O.dedup(x, d, ids, sims, k, cfg.sim_threshold, cfg.rep_threshold,
                   priority=inp.priority, created_unix=inp.created_unix,
                   max_gap_secs=cfg.max_gap_secs, burst=inp.burst)
    got = dedup_with_neighbors(x, d, Neighbors(k, ids, sims), inp, cfg)
    assert np.array_equal(got.group_of, want["group_of"])
    assert np.array_equal(got.representatives, want["representatives"])
    assert np.array_equal(got.anchors, want["anchors"])
    assert np.array_equal(got.sizes, want["sizes"])
    assert (got.linked_pairs, got.split_components) == (want["linked_pairs"],
                                                        want["split_components"])
    assert np.array_equal(got.nn_sim, sims.reshape(n, k)[:, 0])
    return got


def _same_partition(a, b):
    """ARI == 1 exactly when the two labelings split the rows the same way."""
    a, b = np.asarray(a), np.asarray(b)
    pairs = set(zip(a.tolist(), b.tolist()))
    return len(pairs) == len(set(a.tolist())) == len(set(b.tolist()))


def test_dedup_recovers_injected_bursts():
    """tests/dedup.rs:112-153: 800 nested rows plus 40 bursts of perturbed copies."""
    d = 128
    x, _, _ = nested(n=800, d=d, n_broad=4, sub_range=(2, 3), seed=21)
    wx, truth, _ = with_bursts(x, d, 40, (1, 6), 0.143, 5)
    r = _dedup(wx, d)
    assert _same_partition(truth, r.group_of), "groups differ from the injected bursts"
    assert r.n_groups() == 800
    for g, rep in enumerate(r.representatives):
        assert r.group_of[rep] == g
    labels = np.arange(r.n_groups(), dtype=np.uint32) * 10
    assert np.array_equal(r.expand(labels), r.group_of * 10)
    assert r.gather(wx, d).size == r.n_groups() * d


def test_dedup_cuts_chains():
    """tests/dedup.rs:155-193: a random walk, cosine ~0.976 per step, ends far apart."""
    d = 256
    rng = Normal(8)
    rows = [random_unit(1, d, 1)[0]]
    for _ in range(1, 40):
        rows.append(unit(add_scaled(rows[-1], rng.direction(d), 0.22), d))
    x = np.stack(rows).astype(np.float32)
    cfg = DedupConfig()
    r = _dedup(x, d, cfg=cfg)
    ends = _dot(x, 0, 39)
    assert ends < 0.8, f"the walk should drift (ends cos {ends})"
    assert r.n_groups() > 1, "the chain was not cut"
    assert r.split_components >= 1
    t = np.float32(cfg.sim_threshold)
    min_pair = 2.0 * t * t - 1.0 - 1e-4
    for g in range(r.n_groups()):
        m = np.nonzero(r.group_of == g)[0]
        for a in m:
            for b in m:
                assert _dot(x, a, b) >= min_pair, f"group {g}: cos({a},{b})"


def test_bursts_time_gap_and_priority():
    """tests/dedup.rs:195-255."""
    d = 64
    x = random_unit(4, d, 77)
    c = (x[0] + np.float32(0.001)).astype(np.float32)
    normalize_rows(c.reshape(1, d), d)
    x = np.vstack([x, c])  # row 4: a near copy of row 0
    t = np.array([0.0, 10.0, 20.0, 30.0, 86_400.0])
    cfg = DedupConfig()
    r = _dedup(x, d)
    assert r.group_of[0] == r.group_of[4]
    assert r.n_groups() == 4
    # A one-minute gap keeps a copy taken a day later apart.
    gap = DedupConfig(max_gap_secs=60.0)
    r = _dedup(x, d, DedupInput(created_unix=t), gap)
    assert r.group_of[0] != r.group_of[4]
    # Unknown time: the rule does not apply.
    t_nan = np.array([0.0, 10.0, 20.0, 30.0, np.nan])
    r = _dedup(x, d, DedupInput(created_unix=t_nan), gap)
    assert r.group_of[0] == r.group_of[4]
    # Burst ids group unrelated rows 1 and 2.
    r = _dedup(x, d, DedupInput(burst=[None, 7, 7, None, None]), cfg)
    assert r.group_of[1] == r.group_of[2]
    assert r.n_groups() == 3
    # Priority picks the representative.
    for fav in (0, 4):
        p = np.zeros(5, np.float32)
        p[fav] = 1.0
        r = _dedup(x, d, DedupInput(priority=p), cfg)
        assert r.representatives[r.group_of[0]] == fav


def _crafted(d, parts):
    v = np.zeros(d, np.float32)
    for a, w in parts:
        v[a] = w
    normalize_rows(v.reshape(1, d), d)
    return v


def test_burst_joins_a_star_only_when_every_row_fits():
    """tests/dedup.rs:269-300: anchor A with three rim rows at cosine 0.96, and
    a burst of two rows: b1 on the rim, b2 unrelated to A."""
    d = 32
    rows = [_crafted(d, [(0, 1.0)])]
    for a in range(1, 4):
        rows.append(_crafted(d, [(0, 0.96), (a, 0.28)]))
    rows.append(_crafted(d, [(0, 0.96), (4, 0.28)]))  # b1 = row 4
    rows.append(_crafted(d, [(9, 1.0)]))  # b2 = row 5
    x = np.stack(rows)
    burst = [None, None, None, None, 1, 1]
    cfg = DedupConfig()
    r = _dedup(x, d, DedupInput(burst=burst), cfg)
    assert r.group_of[4] == r.group_of[5], "a burst stays together"
    assert r.group_of[5] != r.group_of[0], "a burst row unrelated to the anchor joined its group"
    assert len(r.anchors) == r.n_groups()
    assert r.anchors[r.group_of[0]] == 0
    for i in range(6):
        a = r.anchors[r.group_of[i]]
        assert r.group_of[a] == r.group_of[i], "anchor outside its group"
        same_burst = burst[i] is not None and burst[i] == burst[a]
        assert same_burst or _dot(x, i, a) >= np.float32(cfg.sim_threshold) - np.float32(1e-6)


def test_generators_restate_the_reference():
    """Invariants of the restated synth.rs draws: unit rows, the nested
    spec's sizes (noise rows, minimum sub-group), with_bursts' layout."""
    d = 64
    x, broad, sub = nested(n=400, d=d, n_broad=3, sub_range=(2, 2), min_sub=15, seed=4)
    assert x.shape == (400, d)
    assert np.allclose(np.linalg.norm(x.astype(np.float64), axis=1), 1.0, atol=1e-6)
    assert np.sum(broad == -1) == 12  # round(400 * 0.03)
    counts = np.bincount(sub[sub >= 0])
    assert counts.size == 6 and counts.min() >= 15
    wx, truth, created = with_bursts(x, d, 10, (2, 2), 0.1, 3)
    assert wx.shape == (420, d) and np.array_equal(truth[:400], np.arange(400))
    copies = np.arange(400, 420)
    assert np.all(created[copies] - created[truth[copies]] >= 1.0)
    assert np.all(np.diff(created[copies].reshape(10, 2), axis=1) == 1.0)
