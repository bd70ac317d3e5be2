"""The oracle's training starts (model.rs:772-797): train_from (given
centroids, begin) and train_resume (saved EMA state, begin_with_state).

Pins: two exact identities, then the reference's own behaviour tests of
these paths (crates/emeans-core/tests/model.rs:107-124 and 140-172) on their
own data (tests/common/mod.rs:7-35 mixtures).
  - train_from with the very rows train samples (permutation(n)[..k] of
    RandomState(seed)) is train, bit for bit;
  - train_resume from (c, 2^-16 for every mass) is train_from(c), bit for bit
    (L2: begin's only other step is the spherical normalisation);
  - dead clusters revived by splitting after a far-away train_from;
  - resuming on new data does not worsen its objective by more than 5%.
"""

import numpy as np
import pytest

from oracle import oracle as O

INIT_USAGE = np.float32(1.0 / 65536.0)


def _same(a, b):
    for key in ("centroids", "positions", "usage", "labels", "obj", "nsplit"):
        assert np.asarray(a[key]).tobytes() == np.asarray(b[key]).tobytes(), key


@pytest.mark.parametrize("spherical", [False, True])
def test_train_from_the_sampled_rows_is_train(spherical):
    n, d, k, seed = 3000, 12, 20, 9
    x = O.common_mixture(n, d, 15, 0.6, spherical, 3).reshape(n, d)
    a = O.train(x, d, k, nepochs=3.0, seed=seed, spherical=spherical)
    init = x[O.RandomState(seed).permutation(n)[:k]]
    b = O.train(x, d, k, nepochs=3.0, seed=seed, spherical=spherical, init=init)
    _same(a, b)


def test_resume_from_fresh_state_is_train_from():
    n, d, k = 4000, 10, 24
    x = O.common_mixture(n, d, 20, 0.5, False, 5).reshape(n, d)
    c = (x[:: n // k][:k] * np.float32(0.97)).astype(np.float32)
    a = O.train(x, d, k, seed=4, init=c)
    b = O.train(x, d, k, seed=4, positions=c, usage=np.full(k, INIT_USAGE, np.float32))
    _same(a, b)
    assert a["n_splits"] == b["n_splits"]


def test_dead_clusters_are_revived_by_splitting():
    """tests/model.rs:107-124: 15 centroids far from every row must be revived."""
    n, d, k = 4000, 4, 16
    x = O.common_mixture(n, d, 16, 0.3, False, 11).reshape(n, d)
    init = np.zeros((k, d), np.float32)
    for j in range(1, k):
        init[j] = np.float32(1e3 + j)
    init[0] = x[0]
    o = O.train(x, d, k, init=init)
    assert o["n_splits"] >= 15
    labels, _ = O.assign(x, d, o["centroids"], "l2")
    assert len(set(labels.tolist())) >= 12


def test_resume_on_new_data_does_not_get_worse():
    """tests/model.rs:140-172 (the resume part): train spherical, then continue
    for 2 epochs from the EMA state on new rows."""
    n, d, k = 3000, 16, 12
    x = O.common_mixture(n, d, 12, 0.5, True, 4).reshape(n, d)
    m = O.train(x, d, k, spherical=True)
    more = O.common_mixture(1500, d, 12, 0.5, True, 40).reshape(1500, d)
    _, s0 = O.assign(more, d, m["centroids"], "ip")
    before = O.mean_objective(s0, True)
    r = O.train(more, d, k, nepochs=2.0, spherical=True, positions=m["positions"],
                usage=m["usage"])
    _, s1 = O.assign(more, d, r["centroids"], "ip")
    after = O.mean_objective(s1, True)
    assert after <= before * 1.05, (before, after)
    assert len(r["obj"]) == 2


def test_resume_refuses_bad_state():
    n, d, k = 500, 4, 8
    x = O.common_mixture(n, d, 8, 0.5, False, 1).reshape(n, d)
    pos = x[:k].copy()
    with pytest.raises(ValueError, match="finite"):
        O.train(x, d, k, positions=pos, usage=np.full(k, -1.0, np.float32))
    bad = pos.copy()
    bad[2, 1] = np.inf
    with pytest.raises(ValueError, match="finite"):
        O.train(x, d, k, init=bad)
