"""Top-k beyond the screen's 16 neighbours on the gfx950 backend.

The reference's knn (emeans-cluster/src/knn.rs:42) sends k > GPU_KMAX = 16 to
its CPU search (core/src/knn.rs:53-107): keep a row's k best data rows by
replacing the worst kept entry only on a strictly larger score while ids
increase, then sort by score (IEEE total order) descending, id ascending;
NaN and -inf scores are never kept; missing entries are id 0xFFFFFFFF, score
-inf. Here that search runs on the GPU (emh_topk_long.hip) and its ids and
similarities must equal the oracle's (the same rule over fma-chain dots) bit
for bit: at k = 17 (what Hierarchy::add_photos asks for with
DedupConfig.k = 16, incremental.rs:700-710), up to the 4,096 the device
keeps, with ties from duplicated rows, rows of zeros, NaN and infinite
scores, and fewer candidates than k. dedup with k = 20 and add_photos with
DedupConfig(k = 16) run on it too."""

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


def _mix(n, d, centers, sigma, unit, seed):
    return O.contract_mixture(n, d, centers, sigma, unit, seed).reshape(n, d)


def _same(g, o, what=""):
    gi, gs = g
    oi, os_ = o
    bad = np.nonzero(gi != oi)[0]
    assert bad.size == 0, f"{what}: {bad.size} ids differ, first at {bad[:4]}"
    assert gs.tobytes() == os_.tobytes(), f"{what}: sims differ"


@pytest.mark.parametrize("m,n,d,kk", [
    (300, 300, 768, 17),     # knn_self at the smallest k past the screen
    (200, 900, 20, 40),      # d < 32, d % 4 != 0 below
    (130, 7, 33, 20),        # fewer data rows than k: padding
    (64, 5000, 100, 300),    # the 256 .. 4096 sort
    (40, 6000, 96, 4096),    # the largest k, with more rows than k
    (33, 3000, 64, 4096),    # the largest k, fewer rows than k
])
def test_topk_long_equals_oracle(dev, m, n, d, kk):
    data = _mix(n, d, 9, 0.3, True, m + n)
    q = _mix(m, d, 9, 0.3, True, 7 * m + n)
    _same(dev.topk(q, data, d, kk, False), O.knn(q, data, d, kk, False), "knn")
    if m == n:
        _same(dev.topk(data, data, d, kk, True), O.knn(data, data, d, kk, True), "knn_self")


def test_topk_long_ties_zeros_nan_inf(dev):
    """Duplicated data rows (equal scores: the lower id first), a query of
    zeros (every score +0: the lowest ids), a NaN row (never kept), a row of
    +inf (kept first for positive queries, -inf scores never kept), and
    exclude_self over duplicates."""
    n, d, kk = 1500, 48, 50
    data = _mix(n, d, 6, 0.2, True, 5)
    data[700:760] = data[100:160]          # exact duplicates: equal scores, ids apart
    data[900] = np.nan
    data[901] = np.inf
    data[902] = -np.inf
    q = np.concatenate([data[100:140], np.zeros((1, d), np.float32), -data[5:8],
                        np.abs(data[10:12])]).astype(np.float32)
    _same(dev.topk(q, data, d, kk, False), O.knn(q, data, d, kk, False), "ties")
    _same(dev.topk(data, data, d, kk, True), O.knn(data, data, d, kk, True), "self ties")


def test_topk_long_on_device_buffers_and_limit(dev):
    from emeans_amd import EmeansHipInvalid
    m, n, d, kk = 500, 2500, 384, 64
    data = _mix(n, d, 12, 0.25, True, 11)
    q = _mix(m, d, 12, 0.25, True, 12)
    qb, xb = dev.upload_f32(q), dev.upload_f32(data)
    ib, sb = dev.zeros_u32(m * kk), dev.zeros_f32(m * kk)
    dev.topk_dev(qb, m, xb, n, d, kk, False, ib, sb)
    _same((dev.read_u32(ib), dev.read_f32(sb)), O.knn(q, data, d, kk, False), "device buffers")
    with pytest.raises(EmeansHipInvalid):
        dev.topk(q[:4], data, d, 4097, False)


def test_knn_api_and_dedup_past_sixteen(dev):
    """knn / knn_self at k = 17 through the user API, and dedup with k = 20:
    the same groups as the oracle's dedup over the oracle's neighbours."""
    from emeans_amd import DedupConfig, knn, knn_self, dedup
    n, d = 4000, 128
    base = _mix(n, d, 40, 0.05, True, 21)
    base[3000:3200] = base[:200] + np.float32(1e-3)  # near-duplicates
    base /= np.linalg.norm(base, axis=1, keepdims=True)
    base = base.astype(np.float32)
    nb = knn_self(base, d, 17, dev)
    _same((nb.ids, nb.sims), O.knn(base, base, d, 17, True), "knn_self")
    nb2 = knn(base[:300], base, d, 17, dev)
    _same((nb2.ids, nb2.sims), O.knn(base[:300], base, d, 17, False), "knn")
    cfg = DedupConfig(k=20, sim_threshold=0.9)
    g = dedup(base, d, None, cfg, dev)
    oi, osims = O.knn(base, base, d, 20, True)
    o = O.dedup(base, d, oi, osims, 20, 0.9)
    assert np.array_equal(g.group_of, o["group_of"])
    assert np.array_equal(g.representatives, o["representatives"])
    assert np.array_equal(g.sizes, o["sizes"])
    assert g.linked_pairs == o["linked_pairs"]


def test_add_photos_with_sixteen_neighbours(dev):
    """tests/hierarchy.rs:164-245 with DedupConfig(k = 16), so that
    Hierarchy::add_photos asks for 17 neighbours (incremental.rs:700-710):
    near copies of old photos join their groups, new pairs and fresh photos
    form new groups, sizes add up; the neighbours equal the oracle's."""
    from emeans_amd import DedupConfig, DedupInput, autocluster as A, dedup, knn
    from .ref_synth import Normal, normalize_rows, with_bursts
    from .test_gpu_autocluster import _cfg, _data, _reps
    x, _, _ = _data()
    d = x.shape[1]
    old, _, _ = with_bursts(x[:1500], d, 60, (1, 4), 0.1, 3)
    n_old = old.shape[0]
    cfg = DedupConfig(k=16)
    dd = dedup(old, d, DedupInput(), cfg, dev)
    h, _ = A.auto_cluster(dev, _reps(old, dd), _cfg())
    h.dedup = cfg
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
    nb = knn(photos[n_old:], photos, d, 17, dev)
    _same((nb.ids, nb.sims), O.knn(photos[n_old:], photos, d, 17, False), "add_photos' knn")
    r = h.add_photos(photos, n_old, dd, DedupInput(), dev)
    assert r.joined_existing == 20 and r.new_groups == 40
    assert len(r.leaf) == n and len(dd.group_of) == n
    assert dd.n_groups() == n_reps_old + 40 and h.state.n_seen == dd.n_groups()
    for i in range(20):
        assert dd.group_of[n_old + i] == dd.group_of[i], f"copy {i} did not join its source"
    fresh = {int(dd.group_of[i]) for i in range(n_old + 40, n)}
    assert len(fresh) == 30 and all(g >= n_reps_old for g in fresh)
    assert int(np.sum(dd.sizes, dtype=np.int64)) == n
