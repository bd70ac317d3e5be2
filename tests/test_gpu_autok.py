"""The automatic-k callers on the GPU (emeans-cluster/src/auto.rs, metrics.rs)
against the oracle.

- kmeans_pp: the same picks as the oracle's restatement (which follows the
  reference's order: sequential f32 dots, f64 weights, the seed's stream), on
  the reference's own nested test data with its assertions
  (tests/hierarchy.rs:143-162), and on a reduced C5-shaped set.
- internal_scores: bit-equal to the oracle (same fma-chain dots, same f64
  order) on the reference's scikit-learn fixtures, and within 1e-5 of
  scikit-learn as the reference's own test asks (tests/metrics.rs:10-52).
- sweep: a reduced C5 level-1 sweep (30,000 x 768 nested unit rows, Zipf
  weights, seed 3; k = 2 .. 10, two k-means++ restarts) on one context with
  the data bound once, equal to the oracle doing the same sequence: picks,
  every fit's centroids and assignment, the best restart, every score, and
  the selected k.
"""

import json
import os

import numpy as np
import pytest

from oracle import oracle as O

from .ref_synth import nested as ref_nested

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def dev():
    from emeans_amd import HipDevice
    d = HipDevice()
    yield d
    d.close()


def test_kmeans_pp_reference_data(dev):
    x, broad, _ = ref_nested(n=3000, d=96, n_broad=4, sub_range=(2, 4), min_sub=60,
                             noise_frac=0.0, seed=31)
    xb = dev.bind(x)
    picks = dev.kmeans_pp(xb, 3000, 96, 12, 5)
    assert np.array_equal(picks, O.kmeans_pp(x, 96, 12, 5))
    assert len(set(picks.tolist())) == 12
    assert len(set(broad[picks[:8]].tolist())) == 4
    assert len(dev.kmeans_pp(dev.bind(x[:3]), 3, 96, 12, 5)) == 3


def test_kmeans_pp_c5_shape(dev):
    from emeans_amd import synth
    x, _ = synth.nested(n=40_000, d=768, seed=3)
    xb = dev.bind(x)
    for seed in (1234, 99):
        assert np.array_equal(dev.kmeans_pp(xb, 40_000, 768, 16, seed),
                              O.kmeans_pp(x, 768, 16, seed))


def _scores_equal(g, o):
    assert g["k_eff"] == o["k_eff"]
    for key in ("silhouette", "calinski_harabasz", "davies_bouldin", "objective"):
        assert g[key] == o[key], (key, g[key], o[key])
    assert np.array_equal(g["sizes"], o["sizes"])


def test_internal_scores_fixtures_and_scale(dev):
    j = json.load(open(os.path.join(GOLD, "metrics.json")))
    for c in j["cases"]:
        d, k = c["d"], c["k"]
        x = np.fromfile(os.path.join(GOLD, f"metrics_{c['name']}.f32"), "<f4").reshape(-1, d)
        lab = np.array(c["labels"], np.uint32)
        g = dev.internal_scores(dev.bind(x), x.shape[0], d, dev.upload_u32(lab), k)
        _scores_equal(g, O.internal_scores(x, d, lab, k))
        for key in ("silhouette", "calinski_harabasz", "davies_bouldin"):
            assert abs(g[key] - c[key]) <= 1e-5 * max(abs(c[key]), 1e-12), (c["name"], key)
    # 100 clusters (two passes of the 64-sum kernel), one empty label, skewed sizes.
    from emeans_amd import synth
    x, lab = synth.nested(n=20_000, d=128, top=8, sub=16, seed=5)
    lab = (lab % 100).astype(np.uint32)
    lab[lab == 7] = 8
    g = dev.internal_scores(dev.bind(x), 20_000, 128, dev.upload_u32(lab), 101)
    _scores_equal(g, O.internal_scores(x, 128, lab, 101))
    assert g["k_eff"] > 64  # two launches of the 64-sum kernel


def test_level1_sweep_reduced_c5(dev):
    from emeans_amd import auto, synth
    x, _ = synth.nested(n=30_000, d=768, seed=3)
    n, d = x.shape
    cfg = auto.AutoConfig(restarts=2, seed=3)
    ks = list(range(2, 11))
    xb = dev.bind(x)
    got, picks = auto.sweep(dev, x, xb, ks, cfg, salt=0)
    # The oracle, step by step.
    want_picks = [O.kmeans_pp(x, d, max(ks), auto.seed_for(cfg, 0, 0, r)) for r in range(2)]
    for a, b in zip(picks, want_picks):
        assert np.array_equal(a, b)
    scores = []
    for (s, f), k in zip(got, ks):
        best = None
        for r in range(2):
            seed = auto.seed_for(cfg, 0, k, r)
            o = O.train(x, d, k, spherical=True, seed=seed, init=x[want_picks[r][:k]])
            lab, sc = O.assign(x, d, o["centroids"], "ip")
            obj = O.mean_objective(sc, True)
            if best is None or obj < best[0]:
                best = (obj, seed, o["centroids"], lab, sc)
        assert f.seed == best[1] and f.objective == best[0], k
        assert f.centroids.tobytes() == best[2].tobytes(), k
        assert np.array_equal(dev.read_u32(f.labels), best[3]), k
        assert dev.read_f32(f.scores).tobytes() == best[4].tobytes(), k
        i = O.internal_scores(x, d, best[3], k)
        assert (s.k_eff, s.silhouette, s.calinski_harabasz, s.davies_bouldin, s.objective) == \
            (i["k_eff"], i["silhouette"], i["calinski_harabasz"], i["davies_bouldin"],
             i["objective"]), k
        scores.append(s)
    assert auto.select(scores, cfg, False) == auto.select([s for s, _ in got], cfg, False)
