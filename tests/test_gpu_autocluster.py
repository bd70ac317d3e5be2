"""auto_cluster and Hierarchy::add on the gfx950 backend
(emeans_amd.autocluster, emeans_amd.hierarchy) against the reference's own
tests of them (emeans-cluster/tests/hierarchy.rs) on the same data: the
reference's nested generator (synth.rs, restated in tests/ref_synth.py) with
the tests' specs and AutoConfig (k1 in 2..10, k2 <= 8). The assertions are
the reference's:

  auto_cluster_finds_both_levels (48-67)     chosen k, sweep lengths, ARI of
                                             both levels, leaf count, labels
                                             the hierarchy reproduces
  incremental_adds_keep_ids_and_survive_save_load (69-119)
                                             directory and blob round trips,
                                             append-only rows, adds in four
                                             chunks: an EMA update, no
                                             retrain, stable leaf ids
  full_retrain_carries_ids (121-140)         a retrain keeps level-1 ids
  flat_data_stays_flat (276-295)
  outlier_flag_carries_information (505-536)
  update_grows_a_leaf_for_a_new_group (538-600)
                                             one new leaf for a new group,
                                             kept by the files; none for
                                             scattered rows
  add_photos_joins_near_duplicate_groups (164-245), add_photos_follows_burst_ids
  (247-274), add_photos_agrees_with_a_fresh_dedup (392-477)
                                             Hierarchy::add_photos over
                                             dedup representatives"""

import numpy as np
import pytest
from sklearn.metrics import adjusted_rand_score as ari

from .ref_synth import nested, new_group, scattered_rows

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


def _data():
    d = 96
    x, broad, sub = nested(n=3000, d=d, n_broad=4, sub_range=(2, 4), min_sub=60,
                           noise_frac=0.0, seed=31)
    return np.asarray(x, np.float32).reshape(-1, d), np.asarray(broad), np.asarray(sub)


def _same(a, b):
    for f in ("l1", "l2", "sim1", "sim", "outlier", "slot1", "slot2"):
        assert np.asarray(getattr(a, f)).tobytes() == np.asarray(getattr(b, f)).tobytes(), f


def _stability(a, b):
    """label_stability (auto.rs:1303-1307): rows whose stable leaf id is the same."""
    n = min(len(a.l1), len(b.l1))
    same = (a.l1[:n] == b.l1[:n]) & (a.l2[:n] == b.l2[:n])
    return float(same.sum()) / max(n, 1)


def test_incremental_adds_keep_ids_and_survive_save_load(dev, tmp_path):
    from emeans_amd import autocluster as A, hierarchy as H
    x, broad, sub = _data()
    d, n = x.shape[1], x.shape[0]
    n0 = n * 8 // 10
    h, l0 = A.auto_cluster(dev, x[:n0], _cfg())
    path = tmp_path / "hier"
    h.save(path)
    h2 = H.Hierarchy.load(path, H.HipBackend(dev))
    _same(h2.assign(x[:n0]), l0)
    assert h2.chosen_k() == h.chosen_k()
    blob = h.to_bytes()
    h3 = H.Hierarchy.from_bytes(blob, H.HipBackend(dev))
    _same(h3.assign(x[:n0]), l0)
    assert h3.chosen_k() == h.chosen_k()
    assert h3.to_bytes() == blob
    with pytest.raises(ValueError):
        H.Hierarchy.from_bytes(blob[:-1], H.HipBackend(dev))
    with pytest.raises(ValueError):
        H.Hierarchy.from_bytes(blob + b"\x00", H.HipBackend(dev))
    with pytest.raises(ValueError):
        h.add(x, n0 + 1)  # rows are append-only
    chunk = (n - n0) // 4
    seen, actions, last = n0, [], None
    while seen < n:
        end = min(seen + chunk, n)
        r = h.add(x[:end], seen)
        assert len(r.labels.l1) == end
        actions.append(r.action)
        seen, last = end, r.labels
    assert h.state.n_seen == n
    assert "EmaUpdate" in actions and "FullRetrain" not in actions, actions
    assert _stability(l0, last) > 0.97
    assert ari(sub, _leaf_codes(last)) > 0.85
    # The updated hierarchy (resumed leaves with their run records) survives the blob.
    h4 = H.Hierarchy.from_bytes(h.to_bytes(), H.HipBackend(dev))
    assert h4.to_bytes() == h.to_bytes()
    _same(h4.assign(x), h.assign(x))


def test_full_retrain_carries_ids(dev):
    from emeans_amd import autocluster as A, hierarchy as H
    x, broad, sub = _data()
    n = x.shape[0]
    n0 = n // 2
    h, l0 = A.auto_cluster(dev, x[:n0], _cfg(), H.IncrementalConfig(retrain_added_fraction=0.5))
    r = h.add(x, n0)
    assert r.action == "FullRetrain"
    stable1 = float(np.mean(l0.l1 == r.labels.l1[:n0]))
    assert stable1 > 0.98, f"level-1 id stability {stable1}"
    assert _stability(l0, r.labels) > 0.9


def test_outlier_flag_carries_information(dev):
    from emeans_amd import autocluster as A
    x, broad, sub = _data()
    d, n = x.shape[1], x.shape[0]
    n0 = n * 8 // 10
    h, l0 = A.auto_cluster(dev, x[:n0], _cfg())
    assert l0.outlier.mean() < 0.01, "clean training rows flagged"
    assert h.assign(x[n0:]).outlier.mean() < 0.02, "held-out rows of the same groups flagged"
    assert h.assign(new_group(d, 50, 77)).outlier.all(), "rows of an unseen group must be flagged"


def test_update_grows_a_leaf_for_a_new_group(dev, tmp_path):
    from emeans_amd import autocluster as A, hierarchy as H
    x, broad, sub = _data()
    d, n = x.shape[1], x.shape[0]
    n0 = n * 8 // 10
    inc = H.IncrementalConfig(update_min_outliers=20, retrain_outlier_fraction=0.9)
    h, l0 = A.auto_cluster(dev, x[:n0], _cfg(), inc)
    old_ids = set(zip(l0.l1.tolist(), l0.l2.tolist()))
    leaves0 = sum(h.chosen_k()[1])
    xa = np.concatenate([x[:n0 + 340], new_group(d, 60, 99)])
    first_new = n0 + 340
    r = h.add(xa, n0)
    assert r.action == "EmaUpdate", "precondition"
    assert len(r.new_leaves) == 1, r.new_leaves
    leaf = r.new_leaves[0]
    assert leaf not in old_ids, "the new leaf reuses an old id"
    in_leaf = (r.labels.l1 == leaf[0]) & (r.labels.l2 == leaf[1])
    assert in_leaf[first_new:].sum() >= 60 * 95 // 100
    assert in_leaf[:first_new].sum() <= 3
    assert sum(h.chosen_k()[1]) == leaves0 + 1
    assert _stability(l0, r.labels) > 0.97
    path = tmp_path / "grown"
    h.save(path)
    _same(H.Hierarchy.load(path, H.HipBackend(dev)).assign(xa), r.labels)
    r2 = h.add(np.concatenate([xa, scattered_rows(d, 30, 5)]), xa.shape[0])
    assert r2.action == "EmaUpdate", "precondition"
    assert r2.new_leaves == []


# ---------------------------------------------------------------- add_photos
def _reps(x, dd):
    return np.ascontiguousarray(x[np.asarray(dd.representatives, np.int64)])


def _crafted(d, parts):
    """tests/hierarchy.rs:382-390: a unit row with the given (axis, weight) parts."""
    from .ref_synth import normalize_rows
    v = np.zeros((1, d), np.float32)
    for a, w in parts:
        v[0, a] = np.float32(w)
    return normalize_rows(v, d)[0]


def test_add_photos_joins_near_duplicate_groups(dev):
    """tests/hierarchy.rs:164-245: near copies of old photos join their
    groups, new pairs and fresh photos form new groups, sizes add up, and a
    wrong offset fails."""
    from emeans_amd import DedupConfig, DedupInput, autocluster as A, dedup
    from .ref_synth import Normal, normalize_rows, with_bursts
    x, _, _ = _data()
    d = x.shape[1]
    old, _, _ = with_bursts(x[:1500], d, 60, (1, 4), 0.1, 3)
    n_old = old.shape[0]
    dd = dedup(old, d, DedupInput(), DedupConfig(), dev)
    h, _ = A.auto_cluster(dev, _reps(old, dd), _cfg())
    h.dedup = DedupConfig()
    n_reps_old = dd.n_groups()
    rng = Normal(11)

    def near(src):
        v = (src + np.float32(0.05) * rng.direction(d)).astype(np.float32)
        return normalize_rows(v.reshape(1, d).copy(), d)[0]

    rows = [old, np.stack([near(old[i]) for i in range(20)])]
    pairs = []
    for i in range(10):
        pairs += [x[2000 + i], near(x[2000 + i])]
    rows += [np.stack(pairs), x[2010:2040]]
    photos = np.concatenate(rows).astype(np.float32)
    n = photos.shape[0]
    r = h.add_photos(photos, n_old, dd, DedupInput(), dev)
    assert r.joined_existing == 20 and r.new_groups == 40
    assert len(r.leaf) == n and len(dd.group_of) == n
    assert dd.n_groups() == n_reps_old + 40 and h.state.n_seen == dd.n_groups()
    for i in range(20):
        assert dd.group_of[n_old + i] == dd.group_of[i], f"copy {i} did not join its source"
        assert r.leaf[n_old + i] == r.leaf[i]
    for p in range(10):
        a, b = n_old + 20 + 2 * p, n_old + 21 + 2 * p
        assert dd.group_of[a] == dd.group_of[b] and dd.group_of[a] >= n_reps_old
        assert r.leaf[a] == r.leaf[b]
    fresh = {int(dd.group_of[i]) for i in range(n_old + 40, n)}
    assert len(fresh) == 30 and all(g >= n_reps_old for g in fresh)
    assert int(np.sum(dd.sizes, dtype=np.int64)) == n
    with pytest.raises(ValueError):
        h.add_photos(photos, n_old, dd, DedupInput(), dev)


def test_add_photos_follows_burst_ids(dev):
    """tests/hierarchy.rs:247-274: a new photo sharing an old photo's burst id
    joins that photo's group; an unrelated one does not."""
    from emeans_amd import DedupConfig, DedupInput, autocluster as A, dedup
    x, _, _ = _data()
    d, n_old = x.shape[1], 800
    old = x[:n_old]
    burst = [None] * (n_old + 2)
    burst[5] = 9
    dd = dedup(old, d, DedupInput(burst=burst[:n_old]), DedupConfig(), dev)
    h, _ = A.auto_cluster(dev, _reps(old, dd), _cfg())
    burst[n_old] = 9
    r = h.add_photos(x[:n_old + 2], n_old, dd, DedupInput(burst=burst), dev)
    assert r.joined_existing == 1
    assert dd.group_of[n_old] == dd.group_of[5] and dd.group_of[n_old + 1] != dd.group_of[5]
    assert r.leaf[n_old] == r.leaf[5]


def test_add_photos_agrees_with_a_fresh_dedup(dev):
    """tests/hierarchy.rs:392-477: add_photos and a fresh dedup of the same
    photos apply one rule (within the threshold of the group's anchor, the star
    center, whatever the representative), and give the same partition,
    sizes, anchors and representatives."""
    from emeans_amd import DedupConfig, DedupInput, auto, autocluster as A, dedup
    from .ref_synth import normalize_rows
    x, _, _ = _data()
    d, n_bg = x.shape[1], 800
    old = []
    for i in range(n_bg):
        r = x[i].copy()
        r[80:] = 0.0
        old.append(normalize_rows(r.reshape(1, d), d)[0])
    old.append(_crafted(d, [(80, 1.0)]))
    for a in range(81, 87):
        old.append(_crafted(d, [(80, 0.96), (a, 0.28)]))
    old = np.stack(old).astype(np.float32)
    n_old = old.shape[0]
    a_row, r1 = n_bg, n_bg + 1
    n2 = (np.float32(0.96) * old[r1]).astype(np.float32)
    n2[88] = np.float32(0.28)
    photos = np.concatenate([old, np.stack([_crafted(d, [(80, 0.96), (87, 0.28)]), n2,
                                            _crafted(d, [(80, 0.96), (89, 0.28)]),
                                            _crafted(d, [(90, 1.0)])])]).astype(np.float32)
    n = photos.shape[0]
    n1, n2i, n3, n4 = n_old, n_old + 1, n_old + 2, n_old + 3
    priority = np.zeros(n, np.float32)
    priority[r1] = 1.0
    burst = [None] * n
    burst[n3] = burst[n4] = 4
    cfg = DedupConfig()
    dd = dedup(old, d, DedupInput(priority=priority[:n_old], burst=burst[:n_old]), cfg, dev)
    ga = int(dd.group_of[a_row])
    assert dd.sizes[ga] == 7, "precondition: A and its rim are one group"
    assert dd.representatives[ga] == r1 and dd.anchors[ga] == a_row, "precondition"
    h, _ = A.auto_cluster(dev, _reps(old, dd), auto.AutoConfig(k1_range=(2, 6), k2_max=4,
                                                              restarts=1))
    h.dedup = cfg
    inp = DedupInput(priority=priority, burst=burst)
    h.add_photos(photos, n_old, dd, inp, dev)
    fresh = dedup(photos, d, inp, cfg, dev)
    assert dd.group_of[n1] == dd.group_of[a_row], "N1 is within the threshold of the anchor"
    assert dd.group_of[n2i] != dd.group_of[a_row], "N2 is outside the threshold of the anchor"
    assert dd.group_of[n3] == dd.group_of[n4], "a new burst stays together"
    assert dd.group_of[n4] != dd.group_of[a_row]
    for f in ("group_of", "sizes", "anchors", "representatives"):
        assert np.array_equal(np.asarray(getattr(dd, f)), np.asarray(getattr(fresh, f))), f
