"""Layer 2 and its callers on the GPU against the oracle.

Training is chaotic (one flipped near-tie label moves a later revival draw,
.okf/design/core.md:77-80 in the reference), so the bar is the reference's
whole trajectory: per-epoch objectives equal as f64, split counts, last-pass
labels, positions, masses and closing centroids bit-equal to the oracle's CPU
device loop on the same seeded input; and, for the faiss fixtures, within the
reference test's tolerances of faiss itself (tests/reference.rs:136-209).
"""

import json
import os

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def dev():
    from emeans_amd import HipDevice
    d = HipDevice()
    yield d
    d.close()


def _train_both(dev, x, cfg, init=None):
    from emeans_amd import Emeans
    m = Emeans(cfg, dev)
    t = m.train_from(x, init)
    o = _oracle_train(x, cfg, init=init)
    return m, t, o


def _oracle_train(x, cfg, **start):
    return O.train(x, cfg.d, cfg.k, nepochs=cfg.nepochs, batch_size=cfg.batch_size,
                   alpha0=cfg.alpha0, batch_law=cfg.batch_law, seed=cfg.seed,
                   spherical=cfg.spherical, unused_threshold=cfg.unused_threshold, **start)


def _assert_same_run(m, t, o, tag):
    assert m.recipe()["batch_size"] == o["batch_size"], tag
    assert m.recipe()["alpha0"] == o["alpha0"], tag
    st = m.iteration_stats()
    assert [s.nsplit for s in st] == o["nsplit"].tolist(), tag
    assert [s.obj for s in st] == o["obj"].tolist(), f"{tag}: objectives"
    assert [s.imbalance_factor for s in st] == o["imbalance"].tolist(), tag
    assert np.array_equal(t.labels, o["labels"]), f"{tag}: last-pass labels"
    pos, usage = m.ema_state()
    assert pos.tobytes() == o["positions"].tobytes(), f"{tag}: positions"
    assert usage.tobytes() == o["usage"].tobytes(), f"{tag}: masses"
    assert t.centroids.tobytes() == o["centroids"].tobytes(), f"{tag}: centroids"


def _assert_same_model_file(dev, m, o, cfg, x):
    """The HIP-trained model's file (io.rs:72-186) equals the one the oracle's
    run makes, byte for byte. Two header fields are not the trajectory's and
    come from the HIP run on both sides: the backend name (recipe.backend, the
    assigner's name) and each epoch's wall-clock time. Then the file loads
    back to the same model and the same assignment."""
    from emeans_amd import Emeans, _epoch_rows, model_file as MF
    hb = m.to_bytes()
    n = x.shape[0]
    rec = MF.recipe_dict(cfg, n, o["batch_size"], o["alpha0"], _epoch_rows(n, cfg), dev.name())
    times = [s.time for s in m.iteration_stats()]
    stats = [(ob, t, im, int(ns)) for ob, t, im, ns in zip(o["obj"], times, o["imbalance"],
                                                           o["nsplit"])]
    ob = MF.to_bytes(cfg, rec, o["n_splits"], stats, o["centroids"], o["positions"], o["usage"])
    assert hb == ob, "model file differs from the oracle-trained one"
    back = Emeans.from_bytes_with(hb, dev)
    assert back.to_bytes() == hb
    a, b = m.assign(x), back.assign(x)
    assert np.array_equal(a.labels, b.labels) and a.scores.tobytes() == b.scores.tobytes()


def test_faiss_fixture_runs(dev):
    """The five faiss NumpyEmeans runs: GPU == oracle bit for bit, and faiss within tolerance."""
    from emeans_amd import Config
    ref = json.load(open(os.path.join(GOLD, "reference.json")))
    for c in ref["runs"]:
        d, k = c["d"], c["k"]
        x = np.fromfile(os.path.join(GOLD, c["data"] + ".f32"), dtype="<f4").reshape(-1, d)
        cfg = Config(d=d, k=k, nepochs=c["nepochs"], batch_law=c["batch_law"], seed=c["seed"],
                     spherical=c["spherical"])
        m, t, o = _train_both(dev, x, cfg)
        _assert_same_run(m, t, o, c["data"])
        assert t.labels.tolist() == c["labels"]
        assert [s.nsplit for s in m.iteration_stats()] == c["nsplit"]
        for s, ob in zip(m.obj(), c["obj"]):
            assert abs(s - ob) <= 1e-5 * abs(ob)
        want = np.asarray(c["centroids"], np.float32)
        assert np.all(np.abs(t.centroids - want) <= 1e-4 * np.maximum(np.abs(want), 1.0))
        a = m.assign(x)
        assert a.labels.tolist() == c["assign_labels"]


def test_spherical_blobs_config(dev):
    """20,000 x 64, k = 32, spherical, seed 7 (the CPU-runnable plumbing case)."""
    from emeans_amd import Config, synth
    x, _ = synth.blobs_spherical(20_000, 64, 32, 0.1, seed=7)
    cfg = Config(d=64, k=32, spherical=True, seed=7)
    m, t, o = _train_both(dev, x, cfg)
    _assert_same_run(m, t, o, "blobs")
    _assert_same_model_file(dev, m, o, cfg, x)
    a = m.assign(x)
    ol, osc = O.assign(x, 64, t.centroids, "ip")
    assert np.array_equal(a.labels, ol) and a.scores.tobytes() == osc.tobytes()
    assert a.mean_objective(True) == O.mean_objective(osc, True)


@pytest.mark.parametrize("mode", [1, 3], ids=["bf16x3", "f16x2"])
def test_l2_gmm_mid_size(dev, mode):
    """A 40,000 x 256, k = 512 L2 run through the MFMA screen, with revival,
    in either arithmetic of the split-operand screen."""
    from emeans_amd import Config, synth
    x, _ = synth.gmm_zipf(n=40_000, d=256, comps=512, s=1.1, seed=5)
    cfg = Config(d=256, k=512, seed=11)
    dev.set_screen(mode)
    try:
        m, t, o = _train_both(dev, x, cfg)
    finally:
        dev.set_screen(1)
    _assert_same_run(m, t, o, "gmm-mid")
    assert sum(s.nsplit for s in m.iteration_stats()) > 0


@pytest.mark.parametrize("mode", [1, 3], ids=["bf16x3", "f16x2"])
def test_headline_config_bit_exact(dev, mode):
    """200,000 x 768, k = 1024, exact FP32, L2, seed 0: the whole training run and
    the final assignment equal the oracle's CPU run bit for bit (with either
    arithmetic of the split-operand screen)."""
    from emeans_amd import Config, synth
    x, _ = synth.gmm_zipf(n=200_000, d=768, comps=1024, s=1.1, seed=0)
    cfg = Config(d=768, k=1024, seed=0)
    dev.set_screen(mode)
    try:
        m, t, o = _train_both(dev, x, cfg)
        _assert_same_run(m, t, o, "headline")
        _assert_same_model_file(dev, m, o, cfg, x)
        a = m.assign(x)
    finally:
        dev.set_screen(1)
    ol, osc = O.assign(x, 768, t.centroids, "l2")
    assert np.array_equal(a.labels, ol) and a.scores.tobytes() == osc.tobytes()
    assert a.mean_objective(False) == O.mean_objective(osc, False)


def test_assign_after_training_reuses_split_rows_only_while_unchanged(dev):
    """A training run on bound rows leaves them split in bf16 halves, and an
    assignment of the same buffer takes those halves instead of splitting
    again. The results must be those of the rows as they are: right after the
    run, after a write into the bound rows (the halves are stale then), and
    after the buffer's address was handed out (writes may come from outside)."""
    from emeans_amd import Config, synth
    n, d, k = 40_000, 256, 512
    x, _ = synth.gmm_zipf(n=n, d=d, comps=k, s=1.1, seed=7)
    xb = dev.bind(x)
    cfg = Config(d=d, k=k, seed=3)
    cb = dev.zeros_f32(k * d)
    cent, _ = dev.train_dev(xb, n, cfg, centroids_out=cb)
    lab, sco = dev.zeros_u32(n), dev.zeros_f32(n)

    def check(rows, tag):
        dev.assign_dev(xb, n, d, cb, k, "l2", lab, sco)
        ol, osc = O.assign(rows, d, cent, "l2")
        assert np.array_equal(dev.read_u32(lab), ol), tag
        assert dev.read_f32(sco).tobytes() == osc.tobytes(), tag

    check(x, "right after training")
    y = x.copy()
    y[1000:1500] = x[30_000:30_500] * np.float32(1.5)  # moved rows: other labels and scores
    dev.write_f32(xb, 1000 * d, y[1000:1500].reshape(-1))
    check(y, "after a write into the bound rows")
    dev.train_dev(xb, n, cfg, centroids_out=cb)  # split again, at the new contents
    cent = dev.read_f32(cb).reshape(k, d)
    _ = xb.ptr  # the address is out: no reuse from here on
    check(y, "after the address was handed out")


def test_knn_self_and_dedup(dev):
    """knn_self k = 10 and dedup at 0.97 on unit rows with injected near-duplicates."""
    from emeans_amd import DedupConfig, dedup, knn_self, synth
    x, dst, src = synth.knn_near_duplicates(n=6000, d=96, frac=0.05, noise=0.01, seed=2)
    nb = knn_self(x, 96, 10, dev)
    oi, osims = O.knn(x, x, 96, 10, True)
    assert np.array_equal(nb.ids, oi) and nb.sims.tobytes() == osims.tobytes()
    r = dedup(x, 96, cfg=DedupConfig(k=10, sim_threshold=0.97), dev=dev)
    want = O.dedup(x, 96, oi, osims, 10, 0.97)
    assert np.array_equal(r.group_of, want["group_of"])
    assert np.array_equal(r.representatives, want["representatives"])
    assert np.array_equal(r.anchors, want["anchors"])
    assert np.array_equal(r.sizes, want["sizes"])
    assert r.linked_pairs == want["linked_pairs"]
    assert r.split_components == want["split_components"]
    # Every injected duplicate lands in its source row's group.
    assert np.mean(r.group_of[dst] == r.group_of[src]) > 0.99


def test_assign_at_scale_sample(dev):
    """Inner-product assignment against many centroids (k-tiling of the fused
    GEMM + argmin): 40,000 unit queries x 16,384 unit centroids, d = 1024."""
    from emeans_amd import synth
    q, c = synth.assign_at_scale(n=40_000, d=1024, k=16_384, seed=1)
    gl, gs = dev.assign(q, 1024, c, "ip")
    sub = slice(0, 4000)  # the oracle on a tenth of the queries
    ol, osc = O.assign(q[sub], 1024, c, "ip")
    assert np.array_equal(gl[sub], ol) and gs[sub].tobytes() == osc.tobytes()


@pytest.mark.parametrize("metric", ["l2", "ip"])
def test_assign_host_buffers_in_chunks(dev, metric):
    """The host-buffer assignment pipelines its chunks (the next chunk's rows are
    staged and copied in while the current chunk's kernels run, results go out
    through alternating pinned buffers): six chunks of 1,000 rows, the last one
    partial, bit-equal to the oracle."""
    n, d, k = 5_500, 96, 300
    x = O.contract_mixture(n, d, 40, 0.3, metric == "ip", 17).reshape(n, d)
    c = x[(np.arange(k) * 11) % n] * np.float32(0.97)
    gl, gs = dev.assign(x, d, c, metric, chunk=1000)
    ol, osc = O.assign(x, d, c, metric)
    assert np.array_equal(gl, ol)
    assert gs.tobytes() == osc.tobytes()


def test_dedup_bursts_time_gap_priority(dev):
    """dedup with every side input on the GPU's kNN: the reference's nested
    data (6,000 x 128) plus 300 bursts of perturbed copies one second apart
    (synth.rs:215-248), burst ids on each source and its copies, creation times
    (5% unknown) under a one-minute gap, and random priorities. The whole result
    equals the oracle's grouping of the same neighbours, and the groups are the
    injected bursts."""
    from emeans_amd import DedupConfig, DedupInput, dedup

    from .ref_synth import nested, with_bursts
    d = 128
    x, _, _ = nested(n=6000, d=d, n_broad=8, sub_range=(2, 4), seed=21)
    wx, truth, created = with_bursts(x, d, 300, (1, 6), 0.143, 5)
    n = wx.shape[0]
    g = np.random.default_rng(3)
    created[g.choice(n, n // 20, replace=False)] = np.nan
    counts = np.bincount(truth, minlength=n)
    burst = [int(truth[i]) if counts[truth[i]] > 1 else None for i in range(n)]
    pr = g.random(n).astype(np.float32)
    inp = DedupInput(created_unix=created, burst=burst, priority=pr)
    cfg = DedupConfig(k=10, sim_threshold=0.95, max_gap_secs=60.0)
    r = dedup(wx, d, inp, cfg, dev=dev)
    ids, sims = O.knn(wx, wx, d, 10, True)
    assert np.array_equal(r.nn_sim, sims.reshape(n, 10)[:, 0])
    want = O.dedup(wx, d, ids, sims, 10, 0.95, priority=pr, created_unix=created,
                   max_gap_secs=60.0, burst=burst)
    assert np.array_equal(r.group_of, want["group_of"])
    assert np.array_equal(r.representatives, want["representatives"])
    assert np.array_equal(r.anchors, want["anchors"])
    assert np.array_equal(r.sizes, want["sizes"])
    assert r.linked_pairs == want["linked_pairs"]
    assert r.split_components == want["split_components"]
    assert r.n_groups() == x.shape[0]
    pairs = set(zip(truth.tolist(), r.group_of.tolist()))
    assert len(pairs) == r.n_groups(), "groups differ from the injected bursts"


@pytest.mark.parametrize("spherical", [False, True])
def test_train_from_given_centroids(dev, spherical):
    """train_from (model.rs:705-736): given initial centroids, normalized when
    spherical; a quarter of them far from every row, so revival splits run."""
    from emeans_amd import Config, synth
    n, d, k = 30_000, 128, 256
    if spherical:
        x, _ = synth.blobs_spherical(n, d, 200, 0.2, seed=13)
    else:
        x, _ = synth.gmm_zipf(n=n, d=d, comps=300, s=1.1, seed=13)
    g = np.random.default_rng(2)
    init = (x[g.choice(n, k, replace=False)] * np.float32(1.7)).astype(np.float32)
    init[k - k // 4:] += np.float32(50.0)
    cfg = Config(d=d, k=k, seed=21, spherical=spherical)
    m, t, o = _train_both(dev, x, cfg, init=init)
    _assert_same_run(m, t, o, f"train_from sph={spherical}")
    assert sum(s.nsplit for s in m.iteration_stats()) >= k // 4


def test_train_resume_on_grown_data(dev):
    """train_resume (model.rs:739-749): train, then continue two epochs from the
    EMA state on the data grown by a fifth; both runs bit-equal to the oracle's,
    and the same resume through train_dev with the state given explicitly and
    the initial centroids from a device buffer."""
    from emeans_amd import Config, Emeans, synth
    x, _ = synth.gmm_zipf(n=60_000, d=192, comps=600, s=1.1, seed=17)
    x1 = x[:50_000]
    cfg = Config(d=192, k=512, seed=5)
    m, t, o = _train_both(dev, x1, cfg)
    _assert_same_run(m, t, o, "first run")
    cfg.nepochs = 2.0
    t2 = m.train_resume(x)
    o2 = _oracle_train(x, cfg, positions=o["positions"], usage=o["usage"])
    _assert_same_run(m, t2, o2, "resume on grown data")
    assert len(m.iteration_stats()) == 2
    # The same on the device entry point, state given explicitly.
    xb = dev.bind(x)
    cent, info = dev.train_dev(xb, x.shape[0], cfg, state=(o["positions"], o["usage"]))
    assert cent.tobytes() == o2["centroids"].tobytes()
    assert info["positions"].tobytes() == o2["positions"].tobytes()
    # train_from with the initial centroids in a device buffer.
    init = x[::117][:512].copy()
    cb = dev.upload_f32(init)
    cent, info = dev.train_dev(xb, x.shape[0], cfg, init=cb)
    o3 = _oracle_train(x, cfg, init=init)
    assert cent.tobytes() == o3["centroids"].tobytes()
    assert [s.obj for s in info["stats"]] == o3["obj"].tolist()


def test_train_start_refuses_bad_state(dev):
    from emeans_amd import Config, EmeansHipInvalid
    x = O.common_mixture(2000, 16, 8, 0.5, False, 1).reshape(2000, 16)
    xb = dev.bind(x)
    cfg = Config(d=16, k=8)
    pos = x[:8].copy()
    with pytest.raises(EmeansHipInvalid, match="usage must be finite"):
        dev.train_dev(xb, 2000, cfg, state=(pos, np.full(8, -1.0, np.float32)))
    bad = pos.copy()
    bad[3, 2] = np.nan
    with pytest.raises(EmeansHipInvalid, match="finite"):
        dev.train_dev(xb, 2000, cfg, init=bad)
    # the context still works afterwards
    cent, _ = dev.train_dev(xb, 2000, cfg, init=pos)
    assert cent.tobytes() == _oracle_train(x, cfg, init=pos)["centroids"].tobytes()
