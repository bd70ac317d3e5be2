"""The two largest configurations at their full shapes on the GPU.

- Assign-only at scale: 2,000,000 x 1024 unit queries against 16,384 unit
  centroids, inner product (seed 1). Every query runs through the k-tiled
  screen (64 centroid tiles per part) and the check; the oracle re-scores a
  fixed sample of 4,000 queries, labels and scores bit-equal.
- Exact kNN and dedup: knn_self k = 10 on 500,000 x 384 unit rows with 5%
  injected near-duplicates (a base row plus N(0, 0.01^2) noise, renormalised:
  cosine about 0.981 to its source at d = 384, close to the 0.97 threshold),
  then dedup at 0.97 (seed 2). kNN ids and sims of a fixed 2,000-query sample
  equal the oracle's (the reference's exclude_self rule,
  emeans-cluster/src/knn.rs:17-19); the whole dedup result equals the
  oracle's grouping of the GPU's neighbours (dedup.rs:186-358); and the
  injected duplicates land in their source row's group.

The data come from the seeded generators of emeans_amd.synth (chunked PCG64
streams filled on a thread pool) and are bound to the device once.
"""

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


def test_assign_2m_x_1024_k16384_full_size(dev):
    from emeans_amd import synth
    n, d, k = 2_000_000, 1024, 16_384
    q, c = synth.assign_at_scale(n, d, k, seed=1)
    qb, cb = dev.bind(q), dev.upload_f32(c)
    labels, scores = dev.zeros_u32(n), dev.zeros_f32(n)
    dev.assign_dev(qb, n, d, cb, k, "ip", labels, scores)
    gl, gs = dev.read_u32(labels), dev.read_f32(scores)
    del qb
    assert np.all(gl < k), "every query gets a label"
    sample = np.sort(np.random.default_rng(0).choice(n, size=4000, replace=False))
    ol, osc = O.assign(q[sample], d, c, "ip")
    bad = np.nonzero(gl[sample] != ol)[0]
    assert bad.size == 0, f"{bad.size} labels differ, first at query {sample[bad[0]]}"
    assert gs[sample].tobytes() == osc.tobytes(), "scores not bit-equal"


def _knn_sample_oracle(x, sample, d, kk):
    """The oracle's kNN of rows `sample` among all rows with the query itself
    skipped (exclude_self): the kk + 1 best over all rows, query dropped."""
    oi, osm = O.knn(x[sample], x, d, kk + 1, False)
    oi, osm = oi.reshape(-1, kk + 1), osm.reshape(-1, kk + 1)
    wi = np.empty((len(sample), kk), np.uint32)
    ws = np.empty((len(sample), kk), np.float32)
    for r, qi in enumerate(sample):
        keep = oi[r] != qi
        wi[r], ws[r] = oi[r][keep][:kk], osm[r][keep][:kk]
    return wi, ws


def test_knn_self_and_dedup_500k_x_384(dev):
    from emeans_amd import DedupConfig, dedup, synth
    n, d, kk = 500_000, 384, 10
    xh, dst, src = synth.knn_near_duplicates(n, d, seed=2)
    xb = dev.bind(xh)
    ids, sims = dev.zeros_u32(n * kk), dev.zeros_f32(n * kk)
    dev.topk_dev(xb, n, xb, n, d, kk, True, ids, sims)
    gi, gsm = dev.read_u32(ids).reshape(n, kk), dev.read_f32(sims).reshape(n, kk)
    del xb
    # kNN: a fixed sample of 2,000 queries against the oracle.
    sample = np.sort(np.random.default_rng(1).choice(n, size=2000, replace=False))
    wi, ws = _knn_sample_oracle(xh, sample, d, kk)
    bad = np.nonzero((gi[sample] != wi).any(axis=1))[0]
    assert bad.size == 0, f"{bad.size} sampled rows' ids differ, first query {sample[bad[0]]}"
    assert gsm[sample].tobytes() == ws.tobytes(), "sampled sims not bit-equal"
    # The injected duplicates sit above the threshold: each one's source is a neighbour.
    assert np.mean((gi[dst] == src[:, None]).any(axis=1)) > 0.999
    # dedup through the full path (kNN on the GPU from host rows, groups on the host).
    r = dedup(xh, d, cfg=DedupConfig(k=kk, sim_threshold=0.97), dev=dev)
    assert np.array_equal(r.nn_sim, gsm[:, 0]), "dedup's kNN differs from topk_dev's"
    want = O.dedup(xh, d, gi.reshape(-1), gsm.reshape(-1), kk, 0.97)
    assert np.array_equal(r.group_of, want["group_of"])
    assert np.array_equal(r.representatives, want["representatives"])
    assert np.array_equal(r.anchors, want["anchors"])
    assert np.array_equal(r.sizes, want["sizes"])
    assert r.linked_pairs == want["linked_pairs"]
    assert r.split_components == want["split_components"]
    # At least 99% of the duplicates share their source's group.
    assert np.mean(r.group_of[dst] == r.group_of[src]) >= 0.99
