"""C5's sequence end to end on its own generator: auto_cluster
(emeans-cluster/src/auto.rs:1001-1101) of the first 90 % of the rows, then
Hierarchy::add (incremental.rs:306-360) of the rest, on the gfx950 backend
and, step for step, over the oracle (tests/oracle_device.py answers the same
device calls: training, assignment, kmeans_pp, internal_scores, dots).

Data: synth.nested, C5's generator (nested unit rows: top-level centers with
Zipf(1.3) weights, sub-centers at N(0, 0.3^2), row noise 0.05, seed 3) at
8,000 x 768 with 8 x 4 sub-centers; auto_cluster on 7,200 rows, add 800.
Three configurations:

  defaults        the reference's AutoConfig (k1 in 2..40, four k-means++
                  restarts, davies_bouldin at level 2, bottom-up level 1)
  resplit         k1 in 2..4, k2 <= 4, max_cluster_size 100: stage A leaves
                  large leaves, which the resplit stage splits again
  other branches  the same with random_rows starts, top_down level 1,
                  calinski_harabasz and silhouette criteria (auto.rs:64-83,
                  344-375, 457-542)

Everything must be equal: every sweep's scores, resplits, leaves, the cut,
the chosen k, the labels of every row, the hierarchy (centroids, EMA state,
ids, floors) and its file, then the add's action, labels, outliers and the
updated hierarchy. The reference's own assertions about a clustering
(tests/hierarchy.rs:49-69) are stated on the result too: the labels the
hierarchy reproduces by assigning the rows again, one leaf per level-2
centroid, and the leaves recovering the generator's sub-centers (ARI)."""

import numpy as np
import pytest
from sklearn.metrics import adjusted_rand_score as ari

from .oracle_device import OracleDevice
from .test_gpu_hierarchy import _same_files, _same_hierarchy, _same_labels

pytestmark = pytest.mark.gpu

N, N_FIT, TOP, SUB = 8000, 7200, 8, 4
CONFIGS = {
    "defaults": {},
    "resplit": dict(k1_range=(2, 4), k2_max=4, max_cluster_size=100, restarts=2),
    "other_branches": dict(k1_range=(2, 4), k2_max=4, max_cluster_size=100, restarts=2,
                           init="random_rows", level1_method="top_down",
                           criterion1="calinski_harabasz", criterion2="silhouette"),
}


@pytest.fixture(scope="module")
def dev():
    from emeans_amd import HipDevice
    d = HipDevice()
    yield d
    d.close()


@pytest.fixture(scope="module")
def data():
    from emeans_amd import synth
    return synth.nested(n=N, d=768, top=TOP, sub=SUB, seed=3)


def _scores(lst):
    return [(s.k, s.k_eff, s.silhouette, s.calinski_harabasz, s.davies_bouldin, s.objective,
             s.browsable) for s in lst]


def _same_diagnostics(a, b):
    assert _scores(a.stage_a_level1) == _scores(b.stage_a_level1), "stage A level-1 sweep"
    assert [_scores(g) for g in a.level2] == [_scores(g) for g in b.level2], "level-2 sweeps"
    assert _scores(a.level1) == _scores(b.level1), "level-1 candidates"
    for f in ("resplits", "leaves", "gap_k", "flat", "level1_rejected"):
        assert getattr(a, f) == getattr(b, f), f


@pytest.mark.parametrize("name", list(CONFIGS))
def test_auto_cluster_then_add_equals_oracle(dev, data, name):
    from emeans_amd import auto, autocluster as A
    x, truth = data
    cfg = auto.AutoConfig(**CONFIGS[name])
    od = OracleDevice(dev.name())
    hg, lg = A.auto_cluster(dev, x[:N_FIT], cfg)
    ho, lo = A.auto_cluster(od, x[:N_FIT], cfg)
    _same_diagnostics(hg.diagnostics, ho.diagnostics)
    if name != "defaults":
        assert hg.diagnostics.resplits > 0, "precondition: the resplit stage splits leaves"
    assert hg.chosen_k() == ho.chosen_k()
    _same_labels(lg, lo)
    _same_hierarchy(hg, ho)
    _same_files(hg, ho)
    # tests/hierarchy.rs:49-69 on this data.
    again = hg.assign(x[:N_FIT])
    _same_labels(again, lg)
    k1, k2 = hg.chosen_k()
    codes = (lg.l1.astype(np.int64) << 32) | lg.l2.astype(np.int64)
    assert len(set(codes.tolist())) <= sum(k2) and k1 == len(k2)
    assert ari(truth[:N_FIT], codes) > 0.95, "leaves vs the generator's sub-centers"
    # Hierarchy::add of the remaining rows.
    rg = hg.add(x, N_FIT)
    ro = ho.add(x, N_FIT)
    assert rg.action == ro.action
    assert rg.new_outliers == ro.new_outliers and rg.pending == ro.pending
    assert rg.new_leaves == ro.new_leaves
    _same_labels(rg.labels, ro.labels)
    _same_hierarchy(hg, ho)
    _same_files(hg, ho)
    codes = (rg.labels.l1.astype(np.int64) << 32) | rg.labels.l2.astype(np.int64)
    assert ari(truth, codes) > 0.95
