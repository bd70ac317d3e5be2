"""A hierarchy on the gfx950 backend against the same hierarchy run over the
oracle (emeans_amd.hierarchy; auto.rs:1103-1300, incremental.rs:306-596).

A reduced C5 (22,000 x 768 nested unit rows, seed 3: 20,000 to build on and
2,000 to add): a level-1 model and one level-2 model per group, fitted on the
device, are assembled into two hierarchies that differ only in their backend
(the device, or the oracle's top-1 and training loop). Their labels, cosines,
outlier floors and flags must be equal bit for bit, and so must everything
the add of the last 10 % of the rows changes: the EMA update resumes each
group's leaves on the group's rows, carries the leaves' stable ids by the
Hungarian matching, and rebuilds level 1 from the groups' unit means (grow
off, grow_min_size = 0, as its leaf formation is not built)."""

import copy

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    from emeans_amd import HipDevice
    d = HipDevice()
    yield d
    d.close()


class OracleBackend:
    """The hierarchy's device work by the oracle; resumed runs carry the
    record a model file keeps (recipe under the device's backend name, epoch
    times zero: wall-clock time is not part of the trajectory)."""

    def __init__(self, name="hip"):
        self.name = name

    def leaf_top1(self, x, cents):
        return O.assign(x, x.shape[1], cents, "ip")

    def resume(self, config, x, positions, usage):
        from emeans_amd import _epoch_rows, model_file as MF
        o = O.train(x, config.d, config.k, nepochs=config.nepochs, seed=config.seed,
                    spherical=config.spherical, unused_threshold=config.unused_threshold,
                    positions=positions, usage=usage)
        n = x.shape[0]
        run = {"recipe": MF.recipe_dict(config, n, o["batch_size"], o["alpha0"],
                                        _epoch_rows(n, config), self.name),
               "n_splits": o["n_splits"],
               "stats": [(ob, 0.0, im, int(ns)) for ob, im, ns in zip(o["obj"], o["imbalance"],
                                                                     o["nsplit"])]}
        return o["centroids"], o["positions"], o["usage"], run

    def dots(self, a, b):
        return O.dots(a, b)


def _same_files(hg, ho):
    """The two hierarchies' blobs are equal once the oracle side takes the
    device runs' epoch times."""
    for a, b in zip([hg.level1] + [g.model for g in hg.groups],
                    [ho.level1] + [g.model for g in ho.groups]):
        if a is not None and b is not None:
            assert len(a.stats) == len(b.stats)
            b.stats = [(s[0], t[1], s[2], s[3]) for s, t in zip(b.stats, a.stats)]
    ho.diagnostics = hg.diagnostics
    assert hg.to_bytes() == ho.to_bytes(), "hierarchy files differ"


def _same_labels(a, b):
    for f in ("l1", "l2", "sim1", "sim", "outlier", "slot1", "slot2"):
        va, vb = np.asarray(getattr(a, f)), np.asarray(getattr(b, f))
        assert va.shape == vb.shape and va.tobytes() == vb.tobytes(), f


def _same_hierarchy(hg, ho):
    assert hg.level1.centroids.tobytes() == ho.level1.centroids.tobytes()
    assert hg.level1.usage.tobytes() == ho.level1.usage.tobytes()
    assert hg.ids1 == ho.ids1
    for g, (a, b) in enumerate(zip(hg.groups, ho.groups)):
        assert a.ids == b.ids and a.next_id == b.next_id, g
        assert a.floors.tobytes() == b.floors.tobytes(), g
        if a.model is None:
            assert b.model is None
            continue
        for f in ("centroids", "positions", "usage"):
            assert np.asarray(getattr(a.model, f), np.float32).tobytes() == \
                np.asarray(getattr(b.model, f), np.float32).tobytes(), (g, f)


def test_hierarchy_assign_and_ema_update_reduced_c5(dev):
    from emeans_amd import Config, auto, synth, hierarchy as H
    d, n, k1, k2 = 768, 20_000, 6, 4
    x_all, _ = synth.nested(n=22_000, d=d, seed=3)
    x = x_all[:n]
    xb = dev.bind(x)
    f1 = auto.fit(dev, x, xb, k1, 5.0, 11, dev.kmeans_pp(xb, n, d, k1, 11))
    lab1 = dev.read_u32(f1.labels)
    cfg = lambda k, s: Config(d=d, k=k, spherical=True, nepochs=5.0, seed=s,
                              capture_assignments=False)
    level1 = H.Model(cfg(k1, 11), f1.centroids.reshape(k1, d), f1.positions, f1.usage)
    leaves = []
    for g in range(k1):
        rows = np.flatnonzero(lab1 == g)
        if len(rows) < 2 * k2:
            leaves.append(None)
            continue
        xg = np.ascontiguousarray(x[rows])
        xgb = dev.bind(xg)
        fg = auto.fit(dev, xg, xgb, k2, 5.0, 100 + g, dev.kmeans_pp(xgb, len(rows), d, k2, 100 + g))
        leaves.append(H.Model(cfg(k2, 100 + g), fg.centroids.reshape(k2, d), fg.positions,
                              fg.usage))
    assert sum(m is not None for m in leaves) >= 3
    inc = H.IncrementalConfig(grow_min_size=0)
    build = lambda be: H.Hierarchy.from_models(x, copy.deepcopy(level1), copy.deepcopy(leaves),
                                               be, inc)
    hg, ho = build(H.HipBackend(dev)), build(OracleBackend(dev.name()))
    _same_hierarchy(hg, ho)
    lg, lo = hg.assign(x), ho.assign(x)
    _same_labels(lg, lo)
    assert np.isfinite(np.concatenate([g.floors for g in hg.groups])).all()
    rg, ro = hg.add(x_all, n), ho.add(x_all, n)
    assert rg.action == ro.action == "EmaUpdate", (rg.action, ro.action)
    assert rg.new_outliers == ro.new_outliers and rg.pending == ro.pending == 0
    _same_labels(rg.labels, ro.labels)
    _same_hierarchy(hg, ho)
    assert hg.state == ho.state and hg.state.n_seen == 22_000
    moved = sum(not np.array_equal(a.model.centroids, m.centroids)
                for a, m in zip(hg.groups, leaves) if m is not None)
    assert moved >= 1, "the update resumed no group"
    _same_files(hg, ho)


def test_grow_on_the_device_equals_the_oracle(dev):
    """Hierarchy::add with the grow step (incremental.rs:376-538) on the
    reference's update_grows_a_leaf_for_a_new_group data (tests/hierarchy.rs:
    538-575): a hierarchy from auto_cluster on the device, then the same
    hierarchy read from its blob over the oracle; both add 340 known rows and
    60 rows of a new group. Labels, the new leaf, every model and the files
    must be equal bit for bit."""
    from emeans_amd import autocluster as A, auto, hierarchy as H
    from .ref_synth import nested, new_group
    d = 96
    x, _, _ = nested(n=3000, d=d, n_broad=4, sub_range=(2, 4), min_sub=60, noise_frac=0.0,
                     seed=31)
    x = np.asarray(x, np.float32).reshape(-1, d)
    n0 = 2400
    inc = H.IncrementalConfig(update_min_outliers=20, retrain_outlier_fraction=0.9)
    hg, _ = A.auto_cluster(dev, x[:n0], auto.AutoConfig(k1_range=(2, 10), k2_max=8), inc)
    ho = H.Hierarchy.from_bytes(hg.to_bytes(), OracleBackend(dev.name()))
    xa = np.concatenate([x[:n0 + 340], new_group(d, 60, 99)])
    rg, ro = hg.add(xa, n0), ho.add(xa, n0)
    assert rg.action == ro.action == "EmaUpdate"
    assert rg.new_leaves == ro.new_leaves and len(rg.new_leaves) == 1, (rg.new_leaves,
                                                                       ro.new_leaves)
    _same_labels(rg.labels, ro.labels)
    _same_hierarchy(hg, ho)
    assert hg.state == ho.state
    _same_files(hg, ho)
