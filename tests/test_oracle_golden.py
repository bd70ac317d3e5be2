"""The oracle against the reference's own golden vectors and independent checks.

Each check is chosen so that a plausible slip in the oracle (a dropped term, a
wrong index, a different float order) fails: bit-exact fixtures from faiss
(`tests/golden/reference.json`, written by the reference's bench/py/fixtures.py),
numpy's own MT19937 and pairwise sum, glibc's correctly rounded `fmaf`, numpy's
sequential `cumsum` / `add.at` for the f32 orders, and f64 brute force.
"""

import ctypes
import json
import math
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
_libm = ctypes.CDLL("libm.so.6")
_libm.fmaf.restype = ctypes.c_float
_libm.fmaf.argtypes = [ctypes.c_float] * 3


@pytest.fixture(scope="module")
def ref():
    with open(os.path.join(GOLD, "reference.json")) as f:
        return json.load(f)


def fma_chain(a, b):
    """One sequential f32 fma chain from +0 (glibc fmaf, correctly rounded)."""
    acc = 0.0
    for p, q in zip(a.tolist(), b.tolist()):
        acc = _libm.fmaf(p, q, acc)
    return np.float32(acc)


# --------------------------------------------------------------- golden vectors
def test_recipes_bit_exact(ref):
    """reference.json recipes: batch, alpha0 bits, epoch plan (tests/reference.rs:33-84)."""
    checked = 0
    for c in ref["recipes"]:
        n, k, d, ne = c["n"], c["k"], c["d"], c["nepochs"]
        if c["batch_law"] == "given":
            b, a0 = O.resolve_batch_and_step(n, k, ne, "throughput", c["given_batch_size"],
                                             c.get("given_alpha0"))
        else:
            law = O.resolve_law(c["batch_law"], d)
            assert law == c["resolved_law"], c
            b, a0 = O.resolve_batch_and_step(n, k, ne, law)
            rows = O.epoch_rows(n, ne)
            assert rows == c["epoch_rows"], c
            steps = [-(-r // b) for r in rows]
            assert steps == c["epoch_steps"], c
            assert sum(steps) == c["total_steps"]
            assert -(-n // b) == c["steps_per_pass"]
            assert O.unused_threshold(d) == c["unused_threshold"]
        assert b == c["batch_size"], c
        assert a0 == c["alpha0"], ("alpha0 bits", c)
        checked += 1
    assert checked > 1400


def test_cosine_schedule_bit_exact(ref):
    for c in ref["alphas"]:
        assert O.scheduled_alpha(c["alpha0"], c["step"], c["total"]) == c["alpha"], c


def test_mt19937_matches_fixture_and_numpy(ref):
    for c in ref["mt19937"]:
        seed = c["seed"]
        if "random_sample" in c:
            r = O.RandomState(seed)
            got = [r.random_sample() for _ in c["random_sample"]]
            assert got == c["random_sample"], seed
            np_r = np.random.RandomState(seed)
            assert got == np_r.random_sample(len(got)).tolist()
            continue
        n = c["n"]
        perm = O.RandomState(seed).permutation(n)
        assert perm[:64].tolist() == c["head"], (seed, n)
        m = min(n, 5000)
        assert int(np.dot(np.arange(m, dtype=np.int64), perm[:m].astype(np.int64))) == c["sum"]
        assert np.array_equal(perm, np.random.RandomState(seed).permutation(n))


def test_epoch_seed_and_interval_draws():
    assert O.epoch_seed(1234, 0) == (1234 * 1000003) % 2**32
    assert O.epoch_seed(0xFFFFFFFF, 3) == (0xFFFFFFFF * 1000003 + 3) % 2**32
    # Permutations past 2^16 exercise the masked rejection with large masks.
    for seed, n in [(5, 70001), (99, 3)]:
        assert np.array_equal(O.RandomState(seed).permutation(n),
                              np.random.RandomState(seed).permutation(n))


def _fixture(name, d):
    return np.fromfile(os.path.join(GOLD, name + ".f32"), dtype="<f4").reshape(-1, d)


def test_training_matches_faiss_runs(ref):
    """The whole loop vs faiss NumpyEmeans (tests/reference.rs:136-209 tolerances)."""
    for c in ref["runs"]:
        d, k = c["d"], c["k"]
        x = _fixture(c["data"], d)
        t = O.train(x, d, k, nepochs=c["nepochs"], batch_law=c["batch_law"], seed=c["seed"],
                    spherical=c["spherical"])
        assert t["batch_size"] == c["batch_size"]
        assert t["alpha0"] == c["alpha0"]
        assert t["nsplit"].tolist() == c["nsplit"], c["data"]
        for s, o in zip(t["obj"], c["obj"]):
            assert abs(s - o) <= 1e-5 * abs(o), (s, o)
        for s, o in zip(t["imbalance"], c["imbalance"]):
            assert abs(s - o) < 1e-9
        assert t["labels"].tolist() == c["labels"], "last-pass labels"
        want = np.asarray(c["centroids"], np.float32)
        assert np.all(np.abs(t["centroids"] - want) <= 1e-4 * np.maximum(np.abs(want), 1.0))
        metric = "ip" if c["spherical"] else "l2"
        lab, sco = O.assign(x, d, t["centroids"], metric)
        assert lab.tolist() == c["assign_labels"]
        ws = np.asarray(c["assign_scores"], np.float32)
        assert np.all(np.abs(sco - ws) <= 1e-4 * np.maximum(np.abs(ws), 1.0))


# ----------------------------------------------------------------- float orders
def test_top1_is_the_fma_chain_with_lowest_id_ties():
    """fused.rs:383-420: each dot is one fma chain; strict scan keeps the lowest id."""
    rng = np.random.RandomState(3)
    n, d, k = 13, 37, 21
    x = (rng.rand(n, d) - 0.5).astype(np.float32)
    c = (rng.rand(k, d) - 0.5).astype(np.float32)
    c[9] = c[4]  # exact duplicate: the lower id must win
    x[2] = c[4] * np.float32(1.5)
    for metric in ("ip", "l2"):
        lab, sco = O.top1(x, d, c, metric)
        for i in range(n):
            dots = [fma_chain(x[i], c[j]) for j in range(k)]
            if metric == "ip":
                keys = dots
                better = lambda a, b: a > b
            else:
                cn = [np.cumsum(c[j] * c[j], dtype=np.float32)[-1] for j in range(k)]
                keys = [np.float32(cn[j] - np.float32(2.0) * dots[j]) for j in range(k)]
                better = lambda a, b: a < b
            bj, bv = 0, keys[0]
            for j in range(1, k):
                if better(keys[j], bv):
                    bj, bv = j, keys[j]
            assert lab[i] == bj
            if metric == "ip":
                assert sco[i].tobytes() == np.float32(bv).tobytes()
            else:
                xn = np.cumsum(x[i] * x[i], dtype=np.float32)[-1]
                assert sco[i].tobytes() == np.float32(max(np.float32(xn + bv), 0.0)).tobytes()
    lab, _ = O.top1(np.ones((3, 8), np.float32), 8,
                    np.where(np.isin(np.arange(40), [5, 17, 33])[:, None], 1.0, 0.0)
                    .repeat(8, 1).astype(np.float32), "ip")
    assert lab.tolist() == [5, 5, 5]


def test_top1_matches_f64_brute_force_except_ties():
    """core/contract.rs:177-274 on the contract's own mixtures (stride 1)."""
    for n, d, k in [(513, 13, 70), (300, 64, 1), (600, 96, 100)]:
        for metric in ("ip", "l2"):
            x = O.contract_mixture(n, d, 11, 0.6, metric == "ip", 3 * n + k).reshape(n, d)
            c = (np.resize(x[: min(k, n)].reshape(-1), k * d) * np.float32(0.95)).reshape(k, d)
            perm = ((np.arange(n, dtype=np.uint64) * 7919 + 13) % n).astype(np.uint32)
            lo, hi = n // 7, n - n // 9
            lab = np.full(n, 0xFFFFFFFF, np.uint32)
            sco = np.full(n, np.nan, np.float32)
            O.top1(x, d, c, metric, ids=perm, rows=(lo, hi), labels=lab, scores=sco)
            assert np.all(lab[:lo] == 0xFFFFFFFF) and np.all(np.isnan(sco[hi:]))
            xs = x[perm[lo:hi]].astype(np.float64)
            c64 = c.astype(np.float64)
            if metric == "ip":
                s64 = xs @ c64.T
                want = np.argmax(s64, 1)
                mag = np.maximum(np.sqrt((xs**2).sum(1)[:, None] * (c64**2).sum(1)[None]), 1.0)
            else:
                s64 = ((xs[:, None, :] - c64[None]) ** 2).sum(2)
                want = np.argmin(s64, 1)
                mag = np.maximum((xs**2).sum(1)[:, None] + (c64**2).sum(1)[None], 1.0)
            got = lab[lo:hi].astype(np.int64)
            r = np.arange(hi - lo)
            sg, sw = s64[r, got], s64[r, want]
            ties = got != want
            assert np.all(np.abs(sg - sw)[ties] <= 1e-5 * mag[r, got][ties])
            assert np.all(np.abs(sco[lo:hi] - sg) <= 1e-5 * mag[r, got])


def test_norms_and_normalize_float_order():
    """assign.rs:150-155, cpu.rs:219-230; contract.rs:500-554 incl. the zero and 1e30 rows."""
    d = 768
    m = O.contract_mixture(300, d, 7, 0.5, False, 1000 + d).reshape(300, d)
    m[0] = 0.0
    m[1] *= np.float32(1e30)
    got = O.row_norms(m, 300, d)
    seq = np.array([np.cumsum(r * r, dtype=np.float32)[-1] for r in m], np.float32)
    assert got.tobytes() == seq.tobytes()
    w = (m.astype(np.float64) ** 2).sum(1)
    ok = np.arange(300) != 1
    assert np.all(np.abs(got[ok] - w[ok]) <= 1e-5 * np.maximum(w[ok], 1e-30))
    u = O.normalize_rows(m, 300, d).reshape(300, d)
    for i in range(300):
        r = m[i].copy()
        mx = np.float32(np.max(np.abs(r)))
        r = r / (mx if mx > 0 else np.float32(1.0))
        nr = np.sqrt(np.cumsum(r * r, dtype=np.float32)[-1])
        r = r / (nr if nr > 0 else np.float32(1.0))
        assert u[i].tobytes() == r.astype(np.float32).tobytes(), i
    m64 = m.astype(np.float64)
    nr = np.sqrt((m64**2).sum(1, keepdims=True))
    want = m64 / np.where(nr > 0, nr, 1.0)
    assert np.all(np.abs(u - want) <= 1e-5 * np.maximum(np.abs(want), 1.0 / math.sqrt(d)))
    assert np.all(u[0] == 0.0)


def test_numpy_pairwise_sum():
    rng = np.random.RandomState(0)
    for n in [0, 1, 7, 8, 9, 100, 128, 129, 1000, 1024, 4097]:
        a = (rng.rand(n) * 1000).astype(np.float32)
        assert O.numpy_sum_f32(a).tobytes() == np.sum(a, dtype=np.float32).tobytes(), n


def test_scatter_row_order_and_acc():
    """contract.rs:355-437: skewed labels with empty clusters, a sub-range selection."""
    n, d, k = 2000, 20, 300
    x = O.contract_mixture(n, d, 7, 0.5, False, n + d).reshape(n, d)
    live = max(k - k // 5, 1)
    labels = (((np.arange(n, dtype=np.uint64) * 2654435761) % 2**32 >> 7) % live).astype(np.uint32)
    perm = ((np.arange(n, dtype=np.uint64) * 31 + 5) % n).astype(np.uint32)
    lo, hi = n // 5, n
    acc0 = ((np.arange(k * d) % 13) * 0.25).astype(np.float32)
    acc = acc0.copy()
    sums, counts = O.scatter_add(x, d, labels, k, ids=perm, rows=(lo, hi), acc=acc)
    ws = np.zeros((k, d), np.float32)
    np.add.at(ws, labels[lo:hi], x[perm[lo:hi]])  # unbuffered, in index order
    assert sums.tobytes() == ws.reshape(-1).tobytes()
    assert counts.tolist() == np.bincount(labels[lo:hi], minlength=k).tolist()
    assert acc.tobytes() == (acc0 + ws.reshape(-1)).tobytes()
    r64 = np.zeros((k, d))
    np.add.at(r64, labels[lo:hi], x[perm[lo:hi]].astype(np.float64))
    tol = 1e-5 * (1 + np.abs(r64)) * np.sqrt(np.maximum(counts, 1))[:, None]
    assert np.all(np.abs(sums.reshape(k, d) - r64) <= tol)


def test_ema_closed_form():
    """cpu.rs:389-432 vs plain f32 numpy, and reference.rs:117-152 (f64) within 1e-5."""
    k, d = 70, 13
    rng = np.random.RandomState(1)
    sums = rng.randn(k * d).astype(np.float32)
    counts = rng.randint(0, 5, k).astype(np.uint32)
    pos0 = rng.randn(k * d).astype(np.float32)
    for alpha, u0 in [(0.37, 0.8), (1.0, 0.5), (0.9, 0.0)]:
        usage0 = (u0 + (np.arange(k) % 5) * 0.125).astype(np.float32)
        p, u = pos0.copy(), usage0.copy()
        O.ema_update(p, u, sums, counts, k, d, alpha)
        a32, decay, replace = np.float32(alpha), np.float32(1.0 - alpha), alpha == 1.0
        wp, wu = pos0.reshape(k, d).copy(), usage0.copy()
        if not replace:
            wu = wu * decay
        for j in range(k):
            if counts[j] == 0:
                continue
            cnt = np.float32(counts[j])
            step = a32 * cnt
            mass = (np.float32(0) if replace else wu[j]) + step
            w = step / mass
            mean = sums.reshape(k, d)[j] / cnt
            wp[j] = mean if w == np.float32(1) else wp[j] + w * (mean - wp[j])
            wu[j] = mass
        assert p.tobytes() == wp.reshape(-1).tobytes() and u.tobytes() == wu.tobytes()
        # f64 reference (reference.rs:117-152)
        p64, u64 = pos0.astype(np.float64).reshape(k, d), usage0.astype(np.float64)
        if not replace:
            u64 = u64 * (1 - alpha)
        for j in range(k):
            if counts[j] == 0:
                continue
            c = float(counts[j])
            mass = (0.0 if replace else u64[j]) + alpha * c
            p64[j] += alpha * c / mass * (sums.reshape(k, d)[j] / c - p64[j])
            u64[j] = mass
        assert np.all(np.abs(p - p64.reshape(-1)) <= 1e-5 * (1 + np.abs(p64.reshape(-1))))
        assert np.all(np.abs(u - u64) <= 1e-5 * (1 + np.abs(u64)))


def test_split_with_zero_row_nudge():
    """contract.rs:468-496 and core/mod.rs:374-399."""
    k, d = 40, 9
    pos = O.contract_mixture(k, d, 7, 0.5, False, 5).copy()
    pos[d:2 * d] = 0.0
    usage = (1.0 + np.arange(k) * 0.37).astype(np.float32)
    plan = [(j, k - 1 - j) for j in range(k // 2) if j % 3 != 2 and j != k - 1 - j]
    p, u = pos.copy(), usage.copy()
    O.apply_splits(p, u, d, plan)
    eps = np.float32(1e-4)
    off = np.where(np.arange(d) % 2 == 0, eps, -eps).astype(np.float32)
    wp, wu = pos.reshape(k, d).copy(), usage.copy()
    for s, t in plan:
        c = wp[s].copy()
        donor = c * (np.float32(1) - off)
        child = c * (np.float32(1) + off)
        if np.array_equal(donor, child):
            child[0] = np.nextafter(child[0], np.float32(np.inf))
        half = wu[s] / np.float32(2)
        wu[s] = half
        wp[s] = donor
        wu[t] = half
        wp[t] = child
    assert p.tobytes() == wp.reshape(-1).tobytes() and u.tobytes() == wu.tobytes()
    assert p[(k - 2) * d] == np.float32(1e-45) and np.all(p[(k - 2) * d + 1:(k - 1) * d] == 0)


def test_plan_revival_gumbel_topk():
    """core/mod.rs:339-370 against a restatement on numpy's own RandomState."""
    rng = np.random.RandomState(11)
    for seed in (1, 7, 1234):
        usage = (rng.rand(64) ** 4).astype(np.float32)
        usage[:5] = 0.0
        plan = O.plan_revival(usage, 0.1, O.RandomState(seed))
        total = np.sum(usage, dtype=np.float32)
        thr = (total * np.float32(0.1)) / np.float32(64)
        unused = usage < thr
        donors = ~unused & (usage > 0)
        nsplit = min(unused.sum(), donors.sum())
        assert len(plan) == nsplit
        uni = np.maximum(np.random.RandomState(seed).random_sample(64), 2.2250738585072014e-308)
        keys = [(float(np.log(usage[j])) - math.log(-math.log(uni[j])), j)
                for j in range(64) if donors[j]]
        keys.sort(key=lambda kv: (-kv[0], -kv[1]))
        want = list(zip([j for _, j in keys[:nsplit]], np.nonzero(unused)[0].tolist()))
        assert plan == want


def test_closing_means():
    k, d = 6, 5
    pos = np.arange(k * d, dtype=np.float32)
    sums = (np.arange(k * d, dtype=np.float32) * 3 + 1)
    counts = np.array([0, 1, 2, 3, 0, 7], np.float64)
    out = O.closing_means(pos, sums, counts, k, d, False).reshape(k, d)
    for j in range(k):
        want = pos.reshape(k, d)[j] if counts[j] == 0 else sums.reshape(k, d)[j] / np.float32(counts[j])
        assert out[j].tobytes() == want.tobytes()
    out = O.closing_means(pos, sums, counts, k, d, True).reshape(k, d)
    assert np.allclose(np.linalg.norm(out, axis=1), 1.0, atol=1e-6)


def test_knn_fma_chain_ties_and_padding():
    """reference.rs:48-84 ordering; knn.rs padding; contract.rs:276-353 tie rule."""
    rng = np.random.RandomState(4)
    n, d = 50, 16
    x = rng.randn(n, d).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    x[30] = x[7]  # duplicate row: 7 ranks before 30 for every query
    for excl in (False, True):
        ids, sims = O.knn(x, x, d, 6, excl)
        ids, sims = ids.reshape(n, 6), sims.reshape(n, 6)
        for i in range(n):
            dots = [(fma_chain(x[i], x[j]), j) for j in range(n) if not (excl and j == i)]
            dots.sort(key=lambda t: (-float(t[0]), t[1]))
            assert ids[i].tolist() == [j for _, j in dots[:6]], i
            assert sims[i].tobytes() == np.array([s for s, _ in dots[:6]], np.float32).tobytes()
    ids, sims = O.knn(x[:3], x[:4], d, 6, False)
    ids, sims = ids.reshape(3, 6), sims.reshape(3, 6)
    assert np.all(ids[:, 4:] == 0xFFFFFFFF) and np.all(sims[:, 4:] == -np.inf)
    ids, sims = O.knn(x[:4], x[:4], d, 6, True)
    assert np.all(ids.reshape(4, 6)[:, 3:] == 0xFFFFFFFF)


def test_knn_matches_f64_brute_force():
    d = 33
    data = O.contract_mixture(900, d, 9, 0.3, True, 1100).reshape(900, d)
    q = O.contract_mixture(200, d, 9, 0.3, True, 200 * 7 + 900).reshape(200, d)
    ids, sims = O.knn(q, data, d, 5, False)
    s64 = q.astype(np.float64) @ data.astype(np.float64).T
    want = np.argsort(-s64, axis=1, kind="stable")[:, :5]
    ids = ids.reshape(200, 5)
    r = np.arange(200)[:, None]
    ties = ids != want
    assert np.all(np.abs(s64[r, ids] - s64[r, want])[ties] <= 1e-5)
    assert np.all(np.abs(sims.reshape(200, 5) - s64[r, ids]) <= 1e-5)


def test_dedup_groups():
    """dedup.rs:186-358 on a hand-built set: two near-duplicate pairs, one chain cut by the star cover."""
    d = 4
    x = np.array([[1, 0, 0, 0], [0.999, 0.0447, 0, 0], [0, 1, 0, 0], [0, 0, 1, 0],
                  [0, 0, 0.999, 0.0447], [0, 0, 0, 1]], np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    ids, sims = O.knn(x, x, d, 2, True)
    r = O.dedup(x, d, ids, sims, 2, 0.97)
    assert r["group_of"].tolist() == [0, 0, 1, 2, 2, 3]
    assert r["sizes"].tolist() == [2, 1, 2, 1]
    assert r["linked_pairs"] == 2 and r["split_components"] == 0
    assert r["representatives"].tolist() == [0, 2, 3, 5]
    # Chain a-b-c-d (0.2 rad steps, cos 0.98 per link): the star around b keeps a, b, c;
    # d is cos(0.4) from b and starts its own group.
    ang = np.array([0.0, 0.2, 0.4, 0.6])
    y = np.stack([np.cos(ang), np.sin(ang), np.zeros(4), np.zeros(4)], 1).astype(np.float32)
    ids, sims = O.knn(y, y, d, 2, True)
    r = O.dedup(y, d, ids, sims, 2, 0.97)
    assert r["split_components"] == 1 and r["group_of"].tolist() == [0, 0, 0, 1]
    assert r["anchors"].tolist() == [1, 3] and r["linked_pairs"] == 3
    # Priority wins the representative.
    r = O.dedup(x, d, *O.knn(x, x, d, 2, True), 2, 0.97,
                priority=np.array([0, 1, 0, 0, 0, 0], np.float32))
    assert r["representatives"].tolist()[0] == 1
