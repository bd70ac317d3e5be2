"""The oracle's auto-k pieces: kmeans_pp (emeans-cluster/src/auto.rs:401-455)
and internal_scores (emeans-cluster/src/metrics.rs:113-268).

Pins: the reference's own tests. internal_scores against scikit-learn on the
reference's three fixture cases (tests/metrics.rs:10-52, relative 1e-5: the
reference's dots come from the un-vendored gemm crate, so its bits are not
pinned; the oracle's fma-chain dots must land within the same tolerance of
scikit-learn). kmeans_pp on the reference's nested data
(tests/hierarchy.rs:143-162): 12 distinct picks, every broad group within the
first 8, the same picks again for the same seed, and never more picks than
rows; plus the first pick, which is numpy's legacy random_interval(n - 1) of
the seed's stream (RandomState.randint), and a brute-force restatement of the
D^2 draws on a small input (sequential f32 dots, f64 weights, the same uniform).
"""

import json
import os

import numpy as np
import pytest

from oracle import oracle as O

from .ref_synth import nested

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _close(a, b, rel):
    return abs(a - b) <= rel * max(abs(b), 1e-12)


def test_internal_scores_match_scikit_learn():
    j = json.load(open(os.path.join(GOLD, "metrics.json")))
    for c in j["cases"]:
        d, k = c["d"], c["k"]
        x = np.fromfile(os.path.join(GOLD, f"metrics_{c['name']}.f32"), "<f4").reshape(-1, d)
        s = O.internal_scores(x, d, np.array(c["labels"], np.uint32), k)
        assert _close(s["silhouette"], c["silhouette"], 1e-5), (c["name"], s)
        assert _close(s["calinski_harabasz"], c["calinski_harabasz"], 1e-5), (c["name"], s)
        assert _close(s["davies_bouldin"], c["davies_bouldin"], 1e-5), (c["name"], s)
        assert int(s["sizes"].sum()) == x.shape[0]


def _kmeans_pp_brute(x, kmax, seed):
    """D^2 seeding as auto.rs states it, in numpy (row dots as sequential f32 sums)."""
    n = x.shape[0]
    rs = np.random.RandomState(seed)
    first = int(rs.randint(n))  # random_interval(n - 1)
    picks = [first]
    best = np.full(n, -np.inf, np.float32)
    last = first
    while len(picks) < min(kmax, n):
        s = np.array([np.cumsum(r * x[last], dtype=np.float32)[-1] for r in x], np.float32)
        best = np.where(s > best, s, best)
        w = np.maximum(1.0 - best.astype(np.float64), 0.0) ** 2
        total = 0.0
        for v in w:
            total += v
        u = rs.random_sample() * total
        j = n - 1
        for i, v in enumerate(w):
            if u < v:
                j = i
                break
            u -= v
        if w[j] == 0.0:
            j = int(n - 1 - np.argmax(w[::-1]))
        picks.append(j)
        last = j
    return picks


def test_kmeans_pp_matches_a_brute_force_restatement():
    g = np.random.default_rng(4)
    x = g.standard_normal((300, 16)).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    for seed in (1, 5, 77):
        assert O.kmeans_pp(x, 16, 20, seed).tolist() == _kmeans_pp_brute(x, 20, seed)


def test_kmeans_pp_on_the_reference_nested_data():
    """tests/hierarchy.rs:143-162."""
    x, broad, _ = nested(n=3000, d=96, n_broad=4, sub_range=(2, 4), min_sub=60, noise_frac=0.0,
                         seed=31)
    picks = O.kmeans_pp(x, 96, 12, 5)
    assert len(picks) == 12 and len(set(picks.tolist())) == 12, "duplicate picks"
    assert len(set(broad[picks[:8]].tolist())) == 4, "D^2 sampling missed a broad group"
    assert np.array_equal(O.kmeans_pp(x, 96, 12, 5), picks)
    assert len(O.kmeans_pp(x[:3], 96, 12, 5)) == 3
    assert picks[0] == np.random.RandomState(5).randint(3000)
