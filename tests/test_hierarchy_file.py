"""Hierarchy files (emeans_amd.hierarchy; incremental.rs:862-1073) and the
grow step of Hierarchy::add (incremental.rs:376-538) on the CPU.

No fixture of a hierarchy file exists in the reference, so the layout is
pinned piece by piece: the blob's framing (magic, u64 lengths, level 1 then
the groups with a model) and its errors as incremental.rs:898-946 states
them; the manifest's keys in the declaration order of the serde structs
(incremental.rs:1052-1073 Manifest/GroupFile, auto.rs:99-147 AutoConfig,
auto.rs:178-192 KScore, auto.rs:195-238 GroupDecision/Diagnostics,
incremental.rs:52-83 IncrementalConfig and 105-122 State, dedup.rs:39-51
DedupConfig); serde_json's pretty layout against text it writes; and each
model inside as a model file (pinned by tests/test_model_file.py).

The grow step runs here over the oracle (top-1, training loop and dots), on
the reference's own hierarchy test data (tests/hierarchy.rs:16-27, 489-503,
538-600): a hierarchy whose leaves are the generator's sub groups, then an
update with 60 rows of a new group forms exactly one new leaf holding them,
and 30 scattered rows form none."""

import json
import struct

import numpy as np
import pytest

from emeans_amd import DedupConfig, auto, hierarchy as H, model_file as MF
from oracle import oracle as O

from .ref_synth import nested, new_group, normalize_rows, scattered_rows


class OracleBackend:
    """The hierarchy's device work done by the oracle."""

    def leaf_top1(self, x, cents):
        return O.assign(x, x.shape[1], cents, "ip")

    def resume(self, config, x, positions, usage):
        o = O.train(x, config.d, config.k, nepochs=config.nepochs, seed=config.seed,
                    spherical=config.spherical, unused_threshold=config.unused_threshold,
                    positions=positions, usage=usage)
        return o["centroids"], o["positions"], o["usage"]

    def dots(self, a, b):
        return O.dots(a, b)


def _ks(k, seconds=0.25):
    return auto.KScore(k, k, 0.125 * k, 10.5, 0.75, 1.0 / 3.0, 0.5, seconds)


def _small_hierarchy():
    """Three groups (one without a model), NaN floors, pending rows, a dedup
    config and sweep diagnostics; models by model_from (no run)."""
    d = 8
    rs = np.random.RandomState(5)
    c = normalize_rows(rs.standard_normal((6, d)).astype(np.float32), d)
    level1 = H.model_from(c[:3], [40, 25, 1], d, 5.0, 1234)
    g0 = H.model_from(c[:2], [30, 10], d, 5.0, 1234)
    g1 = H.model_from(c[2:3], [25], d, 5.0, 1234)
    groups = [H.Group(g0, [0, 3], np.array([0.5, np.nan], np.float32), 4, H.decision_split(2)),
              H.Group(g1, [0], np.array([0.8125], np.float32), 1,
                      H.decision_no_structure(0.03125)),
              H.Group(None, [], np.zeros(0, np.float32), 0, H.DECISION_EMPTY)]
    st = H.State(66, 60, 62, 6, 2, 4, [61, 64], 3)
    h = H.Hierarchy(d, level1, groups, [0, 2, 1], st, OracleBackend(), H.IncrementalConfig(),
                    config=auto.AutoConfig(k1_range=(2, 10), k2_max=8),
                    dedup=DedupConfig(10, 0.97, None, 3600.0))
    h.diagnostics = auto.Diagnostics(level1=[_ks(2), _ks(3)], level2=[[_ks(2)], [], []],
                                     seconds=1.5, stage_a_level1=[_ks(2)], resplits=1, leaves=3,
                                     gap_k=2, flat=False, level1_rejected=[1])
    return h


def _manifest_of(blob):
    n = struct.unpack("<Q", blob[8:16])[0]
    return blob[16:16 + n], 16 + n


def test_blob_framing_and_round_trip():
    h = _small_hierarchy()
    b = h.to_bytes()
    assert b[:8] == b"EMHIER\x00\x01"
    js, off = _manifest_of(b)
    models = [h.level1, h.groups[0].model, h.groups[1].model]  # level 1, then groups with one
    for m in models:
        n = struct.unpack("<Q", b[off:off + 8])[0]
        assert b[off + 8:off + 8 + n] == m.to_bytes()
        assert b[off + 8:off + 16] == b"EMEANS\x00\x01"
        off += 8 + n
    assert off == len(b)
    assert b" " not in js.replace(b'"d <= 16"', b"")  # compact
    h2 = H.Hierarchy.from_bytes(b, OracleBackend())
    assert h2.to_bytes() == b
    assert h2.chosen_k() == h.chosen_k() == (3, [2, 1, 0])
    assert h2.groups[0].floors.tobytes() == h.groups[0].floors.tobytes()
    assert h2.state == h.state and h2.ids1 == [0, 2, 1]
    assert h2.groups[1].decision == {"no_structure": {"best_silhouette": 0.03125}}
    assert h2.groups[2].decision == "empty" and h2.groups[2].model is None
    assert h2.config == h.config
    f32_fields = ("match_min_sim", "outlier_min_sim")
    assert {k: v for k, v in vars(h2.inc).items() if k not in f32_fields} == \
        {k: v for k, v in vars(h.inc).items() if k not in f32_fields}
    assert np.float32(h2.inc.match_min_sim) == np.float32(h.inc.match_min_sim)
    assert np.float32(h2.dedup.sim_threshold) == np.float32(h.dedup.sim_threshold)
    assert (h2.dedup.k, h2.dedup.rep_threshold, h2.dedup.max_gap_secs) == (10, None, 3600.0)
    assert h2.diagnostics == h.diagnostics


def test_blob_errors_follow_the_reference():
    """tests/hierarchy.rs:85-94 and incremental.rs:917-946, 996-1021."""
    h = _small_hierarchy()
    b = h.to_bytes()
    for cut in (len(b) - 1, 20, 9):
        with pytest.raises(ValueError, match="truncated"):
            H.Hierarchy.from_bytes(b[:cut], OracleBackend())
    with pytest.raises(ValueError, match="1 bytes after the last model"):
        H.Hierarchy.from_bytes(b + b"\x00", OracleBackend())
    with pytest.raises(ValueError, match="not an emeans hierarchy"):
        H.Hierarchy.from_bytes(b"EMHIEX\x00\x01" + b[8:], OracleBackend())
    js, off = _manifest_of(b)

    def with_manifest(mf):
        j = MF.to_json(mf).encode()
        return b[:8] + struct.pack("<Q", len(j)) + j + b[off:]

    mf = json.loads(js)
    mf["version"] = 2
    with pytest.raises(ValueError, match="unsupported hierarchy version 2"):
        H.Hierarchy.from_bytes(with_manifest(mf), OracleBackend())
    mf = json.loads(js)
    mf["groups"][0]["ids"] = [0]
    with pytest.raises(ValueError, match="group 0: model and ids disagree"):
        H.Hierarchy.from_bytes(with_manifest(mf), OracleBackend())
    mf = json.loads(js)
    mf["ids1"] = [0, 1]
    with pytest.raises(ValueError, match="level-1 k, ids and groups disagree"):
        H.Hierarchy.from_bytes(with_manifest(mf), OracleBackend())
    mf = json.loads(js)
    mf["d"] = 9
    with pytest.raises(ValueError, match="level-1 model d differs"):
        H.Hierarchy.from_bytes(with_manifest(mf), OracleBackend())


def test_manifest_keys_in_declaration_order():
    """The serde structs' field order (serde writes fields as declared)."""
    h = _small_hierarchy()
    mf = json.loads(_manifest_of(h.to_bytes())[0])
    assert list(mf) == ["version", "d", "config", "dedup", "ids1", "groups", "diagnostics",
                        "state"]  # incremental.rs:1063-1072
    assert list(mf["config"]) == [  # auto.rs:101-147, backend skipped
        "k1_range", "k2_max", "criterion1", "criterion2", "level1_tolerance",
        "level2_tolerance", "min_cluster_size", "max_cluster_size", "min_split_size",
        "split_min_silhouette", "restarts", "nepochs", "init", "level1_method",
        "resplit_passes", "level1_max_share", "seed", "incremental", "verbose"]
    assert list(mf["config"]["incremental"]) == [  # incremental.rs:52-83
        "outlier_mad_k", "outlier_min_sim", "grow_min_size", "update_min_outliers",
        "update_added_fraction", "update_epochs", "retrain_added_fraction",
        "retrain_outlier_fraction", "match_min_sim"]
    assert list(mf["dedup"]) == ["k", "sim_threshold", "rep_threshold", "max_gap_secs"]
    assert list(mf["groups"][0]) == ["has_model", "ids", "floors", "decision", "next_id"]
    assert list(mf["diagnostics"]) == [  # auto.rs:209-238
        "level1", "level2", "seconds", "stage_a_level1", "resplits", "leaves", "gap_k", "flat",
        "level1_rejected"]
    assert list(mf["diagnostics"]["level1"][0]) == [  # auto.rs:178-192
        "k", "k_eff", "silhouette", "calinski_harabasz", "davies_bouldin", "objective",
        "browsable", "seconds"]
    assert list(mf["state"]) == [  # incremental.rs:105-122
        "n_seen", "n_full", "n_update", "added_since_full", "outliers_since_full",
        "added_since_update", "pending", "next_id1"]
    js = _manifest_of(h.to_bytes())[0].decode()
    # Enums in snake_case (auto.rs:42-83, 193-206); a NaN floor as null; f32
    # fields in f32 digits; the tuple k1_range as an array.
    assert '"criterion1":"silhouette","criterion2":"davies_bouldin"' in js
    assert '"init":"k_means_plus_plus","level1_method":"bottom_up"' in js
    assert '"decision":{"split":{"k":2}}' in js and '"decision":"empty"' in js
    assert '"decision":{"no_structure":{"best_silhouette":0.03125}}' in js
    assert '"floors":[0.5,null]' in js and '"k1_range":[2,10]' in js
    assert '"match_min_sim":0.8},' in js and '"outlier_min_sim":null,' in js
    assert '"sim_threshold":0.97,' in js and '"max_gap_secs":3600.0}' in js


def test_pretty_layout_is_serde_json_pretty():
    """serde_json::to_vec_pretty's layout: two-space indents, "key": value,
    one element per line, [] and {} when empty."""
    v = {"a": [1, 2], "b": {}, "c": [], "d": {"e": None, "f": [[], [0.5]]}, "g": "x"}
    want = ('{\n  "a": [\n    1,\n    2\n  ],\n  "b": {},\n  "c": [],\n  "d": {\n'
            '    "e": null,\n    "f": [\n      [],\n      [\n        0.5\n      ]\n    ]\n'
            '  },\n  "g": "x"\n}')
    assert MF.to_json_pretty(v) == want
    h = _small_hierarchy()
    mf = H.manifest(h)
    assert json.loads(MF.to_json_pretty(mf)) == json.loads(MF.to_json(mf))


def test_directory_save_and_load(tmp_path):
    """Hierarchy::save / load (incremental.rs:864-894, 978-988)."""
    h = _small_hierarchy()
    path = tmp_path / "hier"
    h.save(path)
    names = sorted(p.name for p in path.iterdir())
    assert names == ["group-0.emeans", "group-1.emeans", "hierarchy.json", "level1.emeans"]
    assert (path / "level1.emeans").read_bytes() == h.level1.to_bytes()
    text = (path / "hierarchy.json").read_text()
    assert text == MF.to_json_pretty(H.manifest(h))
    h2 = H.Hierarchy.load(path, OracleBackend())
    assert h2.to_bytes() == h.to_bytes()
    h2.state.n_seen += 1
    h2.save(path)  # replaced as a whole
    assert H.Hierarchy.load(path, OracleBackend()).state.n_seen == 67
    assert sorted(p.name for p in tmp_path.iterdir()) == ["hier"]
    with pytest.raises(ValueError, match="hierarchy.json"):
        H.Hierarchy.load(tmp_path / "missing", OracleBackend())


def test_oracle_dots_are_the_top1_chains():
    """orc_dots restates gemm_nt as fma chains: each row's largest dot and its
    column are the inner-product top-1's score and label (the same chains,
    pinned by the faiss runs), and every dot is within 1e-5 of f64."""
    rs = np.random.RandomState(3)
    a = rs.standard_normal((300, 37)).astype(np.float32)
    b = rs.standard_normal((50, 37)).astype(np.float32)
    g = O.dots(a, b)
    lab, sco = O.top1(a, 37, b, "ip")
    assert np.array_equal(np.argmax(g, axis=1), lab)
    assert g[np.arange(300), lab].tobytes() == sco.tobytes()
    ref = a.astype(np.float64) @ b.astype(np.float64).T
    assert np.max(np.abs(g - ref)) < 1e-5 * np.max(np.abs(ref)) * 37


# ------------------------------------------------------------------ grow
def test_grow_forms_a_leaf_for_a_new_group_over_the_oracle():
    """update_grows_a_leaf_for_a_new_group (tests/hierarchy.rs:538-600) on a
    hierarchy whose leaves are the generator's sub groups: 340 rows of the
    known groups and 60 of a new group give one new leaf holding >= 95 % of
    them and <= 3 strays; the files keep it; 30 scattered rows give none."""
    d = 96
    x, broad, sub = nested(n=3000, d=d, n_broad=4, sub_range=(2, 4), min_sub=60,
                           noise_frac=0.0, seed=31)
    x = np.asarray(x, np.float32).reshape(-1, d)
    n0 = 2400
    subs = sorted(set(sub[:n0].tolist()))
    leaves_of = {b: [s for s in subs if broad[np.flatnonzero(sub == s)[0]] == b]
                 for b in sorted(set(broad.tolist()))}
    groups, grp_rows = [], []
    for b, ss in leaves_of.items():
        rows = [np.flatnonzero(sub[:n0] == s) for s in ss]
        m = H.model_from(H.unit_means(x[:n0], rows), [len(r) for r in rows], d, 5.0, 1234)
        groups.append(H.Group(m, list(range(len(ss))), np.full(len(ss), np.nan, np.float32),
                              len(ss), H.decision_split(len(ss))))
        grp_rows.append(np.concatenate(rows))
    level1 = H.model_from(H.unit_means(x[:n0], grp_rows), [len(r) for r in grp_rows], d, 5.0,
                          1234)
    inc = H.IncrementalConfig(update_min_outliers=20, retrain_outlier_fraction=0.9)
    h = H.Hierarchy(d, level1, groups, list(range(len(groups))),
                    H.State.new(n0, len(groups)), OracleBackend(), inc)
    l0 = h.assign(x[:n0])
    h.set_floors(l0)
    l0 = h.assign(x[:n0])
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
    same = (r.labels.l1[:n0] == l0.l1) & (r.labels.l2[:n0] == l0.l2)
    assert same.mean() > 0.97, "label stability"
    h2 = H.Hierarchy.from_bytes(h.to_bytes(), OracleBackend())
    again = h2.assign(xa)
    for f in ("l1", "l2", "sim1", "sim", "outlier", "slot1", "slot2"):
        assert getattr(again, f).tobytes() == getattr(r.labels, f).tobytes(), f
    scattered = scattered_rows(d, 30, 5)
    r2 = h.add(np.concatenate([xa, scattered]), xa.shape[0])
    assert r2.action == "EmaUpdate", "precondition"
    assert r2.new_leaves == []


def test_assign_lookup_equals_the_per_group_loop():
    """Hierarchy.assign's leaf tables (stable id, floor) give what a loop over
    the groups gives (auto.rs:1135-1189): groups without a model, NaN floors,
    and a group with fewer ids and floors than leaves (0 and NaN past them)."""
    h = _small_hierarchy()
    h.groups[0].ids = [7]
    h.groups[0].floors = np.array([0.25], np.float32)
    d = h.d
    x = normalize_rows(np.random.RandomState(8).standard_normal((500, d)).astype(np.float32), d)
    got = h.assign(x)
    cents, slot = [], []
    for g, grp in enumerate(h.groups):
        if grp.model is not None:
            cents.append(grp.model.centroids.reshape(-1, d))
            slot.extend((g, j) for j in range(grp.model.k))
    leaf, sims = OracleBackend().leaf_top1(x, np.concatenate(cents))
    sl = np.asarray(slot, np.int64)[leaf.astype(np.int64)]
    l2 = np.zeros(len(x), np.uint32)
    floor = np.full(len(x), np.nan, np.float32)
    for g, grp in enumerate(h.groups):
        sel = sl[:, 0] == g
        if not sel.any():
            continue
        j = sl[sel, 1]
        ids = np.asarray(grp.ids + [0], np.uint32)
        l2[sel] = ids[np.minimum(j, len(grp.ids))]
        fl = np.concatenate([grp.floors.astype(np.float32), [np.float32(np.nan)]])
        floor[sel] = fl[np.minimum(j, len(grp.floors))]
    assert np.array_equal(got.l2, l2)
    assert np.array_equal(got.outlier, np.isfinite(floor) & (sims.astype(np.float32) < floor))
    assert set(got.l2[got.slot1 == 0].tolist()) <= {7, 0} and 0 in got.l2[got.slot1 == 0]
