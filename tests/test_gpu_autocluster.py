"""auto_cluster on the gfx950 backend (emeans_amd.autocluster) against the
reference's own tests of it (emeans-cluster/tests/hierarchy.rs:48-67
auto_cluster_finds_both_levels, 276-295 flat_data_stays_flat) on the same
data: the reference's nested generator (synth.rs, restated in
tests/ref_synth.py) with the tests' specs and AutoConfig (k1 in 2..10,
k2 <= 8). The assertions are the reference's: chosen k, sweep lengths, ARI
of both levels against the generating groups, leaf count, and labels that
the hierarchy reproduces. Then a full retrain through Hierarchy::add
(incremental.rs:598-650) on the same rows keeps the level-1 ids."""

import numpy as np
import pytest
from sklearn.metrics import adjusted_rand_score as ari

from .ref_synth import nested

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    from emeans_amd import HipDevice
    d = HipDevice()
    yield d
    d.close()


def _cfg():
    from emeans_amd import auto
    return auto.AutoConfig(k1_range=(2, 10), k2_max=8)


def _leaf_codes(l):
    return (l.l1.astype(np.int64) << 32) | l.l2.astype(np.int64)


def test_auto_cluster_finds_both_levels(dev):
    from emeans_amd import autocluster as A
    d = 96
    x, broad, sub = nested(n=3000, d=d, n_broad=4, sub_range=(2, 4), min_sub=60,
                           noise_frac=0.0, seed=31)
    x = np.asarray(x, np.float32).reshape(-1, d)
    h, l = A.auto_cluster(dev, x, _cfg())
    k1, k2 = h.chosen_k()
    assert k1 == 4, "k1"
    assert len(h.diagnostics.stage_a_level1) == 9
    assert h.diagnostics.level1 and not h.diagnostics.flat
    assert ari(broad, l.l1) > 0.98, "level-1 ARI"
    truth = len(set(np.asarray(sub).tolist()))
    assert abs(sum(k2) - truth) <= 2, f"{sum(k2)} leaves vs {truth} true sub groups"
    assert ari(sub, _leaf_codes(l)) > 0.85, "leaf ARI"
    again = h.assign(x)
    for f in ("l1", "l2", "sim1", "sim", "outlier", "slot1", "slot2"):
        assert np.array_equal(getattr(again, f), getattr(l, f)), f
    # A full retrain on the same rows carries the level-1 ids over.
    from emeans_amd import hierarchy as H
    h.inc = H.IncrementalConfig(retrain_added_fraction=0.0, grow_min_size=0)
    rep = h.add(x, x.shape[0])
    assert rep.action == "FullRetrain"
    assert sorted(h.ids1) == list(range(4)) and h.state.n_full == 3000
    assert ari(broad, rep.labels.l1) > 0.98


def test_flat_data_stays_flat(dev):
    from emeans_amd import autocluster as A
    d = 96
    x, broad, _ = nested(n=2400, d=d, n_broad=6, sub_range=(1, 1), min_sub=100,
                         noise_frac=0.0, seed=41)
    x = np.asarray(x, np.float32).reshape(-1, d)
    h, l = A.auto_cluster(dev, x, _cfg())
    k1, k2 = h.chosen_k()
    assert h.diagnostics.flat, f"grouped flat data: k1 {k1}"
    assert k1 == 6
    assert all(k == 1 for k in k2), k2
    assert ari(broad, l.l1) > 0.98
