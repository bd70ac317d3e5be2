"""The hierarchy's host rules (emeans_amd.hierarchy) against the reference's
own known-answer tests: leaf_floors (auto.rs:1313-1336,
floors_flag_stragglers_not_a_fixed_share), the Hungarian matching and stable
ids (incremental.rs:1079-1130, hungarian_finds_the_optimum,
matching_keeps_ids_under_permutation); plus quantile against its definition
(metrics.rs:271-279) and unit means against f64 brute force."""

import itertools

import numpy as np

from emeans_amd import hierarchy as H


def test_floors_flag_stragglers_not_a_fixed_share():
    inc = H.IncrementalConfig()
    clean = np.array([np.float32(0.88) + np.float32(0.0002) * np.float32(i) for i in range(200)],
                     np.float32)
    small = [np.float32(0.90) + np.float32(0.002) * np.float32(i) for i in range(9)]
    small = np.array(small + [np.float32(0.55)], np.float32)
    sims = [clean, small, np.zeros(0, np.float32)]
    f = H.leaf_floors(sims, inc)
    flagged = lambda v, fl: int(np.sum(v < fl))
    assert flagged(clean, f[0]) == 0, "a clean leaf flags no row"
    assert flagged(small, f[1]) == 1, "a small leaf flags its straggler"
    assert 0.55 < f[1] < 0.90
    assert np.isfinite(f[2]), "an empty leaf still has a floor"
    absf = H.IncrementalConfig(outlier_min_sim=0.5)
    assert [float(v) for v in H.leaf_floors(sims, absf)] == [0.5] * 3
    same = [np.full(30, np.float32(0.9), np.float32)]
    assert flagged(same[0], H.leaf_floors(same, inc)[0]) == 0


def test_hungarian_finds_the_optimum():
    c = [[7.0, 3.0, 9.0, 1.0, 4.0],
         [2.0, 8.0, 6.0, 5.0, 3.0],
         [4.0, 4.0, 2.0, 7.0, 9.0],
         [6.0, 1.0, 3.0, 8.0, 2.0],
         [5.0, 7.0, 4.0, 2.0, 6.0]]
    a = H.hungarian(c)
    total = sum(c[i][j] for i, j in enumerate(a))
    best = min(sum(c[i][p[i]] for i in range(5)) for p in itertools.permutations(range(5)))
    assert total == best
    assert sorted(a) == list(range(5))


def test_hungarian_rectangular_matches_brute_force():
    rng = np.random.default_rng(4)
    for _ in range(20):
        n, m = 3, 5
        c = rng.integers(0, 20, size=(n, m)).astype(float).tolist()
        a = H.hungarian(c)
        assert len(set(a)) == n
        total = sum(c[i][j] for i, j in enumerate(a))
        best = min(sum(c[i][p[i]] for i in range(n)) for p in itertools.permutations(range(m), n))
        assert total == best


def test_matching_keeps_ids_under_permutation():
    d = 4
    old = np.array([1, 0, 0, 0, 0, 1, 0, 0, 0, 0, 1, 0], np.float32)
    new = np.array([0, 0, 1, 0, 1, 0, 0, 0, 0, 0, 0, 1], np.float32)
    m = H.match_centroids(old, new, d, 0.8)
    assert m == [2, 0, None]
    ids, nxt = H.carry_ids(m, [10, 11, 12], 3)
    assert ids == [12, 10, 3] and nxt == 4


def test_quantile_rounds_half_away_and_orders_totally():
    v = np.array([3.0, -0.0, 0.0, 1.0, -2.0, 5.0], np.float32)
    # sorted (total order): -2, -0, 0, 1, 3, 5; q (n - 1) = 2.5 rounds to 3
    assert H.quantile(v, 0.5) == np.float32(1.0)
    assert H.quantile(v, 0.0) == np.float32(-2.0)
    assert H.quantile(v, 1.0) == np.float32(5.0)
    assert np.isnan(H.quantile(np.zeros(0, np.float32), 0.5))
    z = H.quantile(np.array([0.0, -0.0], np.float32), 0.0)
    assert z == 0 and np.signbit(z), "-0 sorts before +0"


def test_unit_means_against_f64_brute_force():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((500, 24)).astype(np.float32)
    rows = [np.arange(0, 500, 3), np.arange(1, 200), np.zeros(0, np.int64)]
    c = H.unit_means(x, rows)
    for g, r in enumerate(rows):
        acc = np.zeros(24, np.float64)
        for i in r:
            acc += x[i].astype(np.float64)
        want = acc.astype(np.float32)
        mx = np.float32(np.max(np.abs(want))) if len(r) else np.float32(0)
        want = want / (mx if mx > 0 else np.float32(1))
        nrm = np.float32(0)
        for v in want:
            nrm = np.float32(nrm + np.float32(v * v))
        want = (want / (np.float32(np.sqrt(nrm)) if nrm > 0 else np.float32(1))).astype(np.float32)
        assert c[g].tobytes() == want.astype(np.float32).tobytes(), g


def test_average_linkage_merges_the_closest_mean_cosine():
    """Each merge joins the pair of live clusters with the largest mean
    pairwise row cosine (brute force over the rows), the lower id kept."""
    from emeans_amd import autocluster as A
    rng = np.random.default_rng(11)
    x = rng.standard_normal((60, 8)).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    rows = [np.arange(i, 60, 7) for i in range(7)]
    merges = A.average_linkage(x, rows)
    assert len(merges) == 6
    members = {j: list(rows[j]) for j in range(7)}
    x64 = x.astype(np.float64)
    for a, b, s in merges:
        assert a < b and a in members and b in members
        best = max(((p, q) for p in members for q in members if p < q),
                   key=lambda pq: np.mean(x64[members[pq[0]]] @ x64[members[pq[1]]].T))
        want = np.mean(x64[members[a]] @ x64[members[b]].T)
        assert (a, b) == best
        assert abs(s - want) < 1e-12
        members[a] += members.pop(b)


def test_cut_numbers_groups_by_lowest_leaf():
    from emeans_amd import autocluster as A
    merges = [(2, 4, 0.9), (0, 3, 0.8), (0, 2, 0.7)]
    assert A.cut(5, merges, 5).tolist() == [0, 1, 2, 3, 4]
    assert A.cut(5, merges, 4).tolist() == [0, 1, 2, 3, 2]
    assert A.cut(5, merges, 3).tolist() == [0, 1, 2, 0, 2]
    assert A.cut(5, merges, 2).tolist() == [0, 1, 0, 0, 0]


def _linkage_full_scan(x, rows):
    """auto.rs:799-858 as a full scan per merge: the first pair (row-major,
    a < b, both alive) of the largest s = dots / (|A| |B|) above -inf."""
    from emeans_amd import autocluster as A
    from emeans_amd import hierarchy as H
    l = len(rows)
    sums = H.row_sums_f64(x, rows)
    size = np.array([float(len(r)) for r in rows], np.float64)
    dots = np.zeros((l, l), np.float64)
    for a in range(l):
        v = A._seq_dot64(sums[a:], sums[a])
        dots[a, a:] = v
        dots[a:, a] = v
    alive = np.ones(l, bool)
    merges = []
    for _ in range(1, l):
        best, a, b = -np.inf, 0, 0
        for p in range(l):
            for q in range(p + 1, l):
                if alive[p] and alive[q]:
                    s = dots[p, q] / (size[p] * size[q])
                    if s > best:
                        best, a, b = float(s), p, q
        alive[b] = False
        size[a] += size[b]
        sums[a] = sums[a] + sums[b]
        merged = dots[a] + dots[b]
        dots[:, a] = merged
        dots[a] = merged
        dots[a, a] = float(np.add.accumulate(sums[a] * sums[a])[-1])
        merges.append((a, b, best))
    return merges


def test_average_linkage_equals_a_full_scan_per_merge():
    """The incremental search (each row's best partner, rescanned only when a
    merge touches it) makes the merges a strict-> full scan makes: exact ties
    (rows of -1/0/1, all-equal rows), NaN sums, random data."""
    from emeans_amd import autocluster as A
    g = np.random.default_rng(5)
    for trial in range(24):
        n, d, l = int(g.integers(30, 800)), int(g.integers(2, 12)), int(g.integers(2, 40))
        kind = trial % 4
        if kind == 0:
            x = g.standard_normal((n, d)).astype(np.float32)
        elif kind == 1:
            x = g.integers(-1, 2, (n, d)).astype(np.float32)
        elif kind == 2:
            x = g.standard_normal((n, d)).astype(np.float32)
            x[g.integers(0, n, 2)] = np.nan
        else:
            x = np.zeros((n, d), np.float32)
            x[:, 0] = 1.0
        lab = g.integers(0, l, n)
        rows = [np.flatnonzero(lab == j) for j in range(l)]
        rows = [r if len(r) else np.array([0]) for r in rows]
        want, got = _linkage_full_scan(x, rows), A.average_linkage(x, rows)
        assert [(a, b) for a, b, _ in got] == [(a, b) for a, b, _ in want], trial
        assert np.array([s for _, _, s in got]).tobytes() == \
            np.array([s for _, _, s in want]).tobytes(), trial


def test_row_sums_are_the_running_sum_and_splits_keep_row_order():
    """row_sums_f64 equals np.add.accumulate's last running sum bit for bit
    (values over 16 orders of magnitude, groups above the 4,096-row block),
    and _split_rows groups rows by label in row order."""
    from emeans_amd import autocluster as A
    from emeans_amd import hierarchy as H
    g = np.random.default_rng(9)
    n, d, l = 20_000, 24, 5
    x = (g.standard_normal((n, d)) * 10.0 ** g.integers(-8, 8, (n, 1))).astype(np.float32)
    lab = g.integers(0, l, n)
    rows = [np.flatnonzero(lab == j) for j in range(l)]
    got = H.row_sums_f64(x, rows)
    for j, r in enumerate(rows):
        want = np.add.accumulate(x[r].astype(np.float64), axis=0)[-1]
        assert got[j].tobytes() == want.tobytes(), j
    r = g.permutation(n)[:9000]
    lr = g.integers(0, 7, 9000)
    for j, part in enumerate(A._split_rows(r, lr, 7)):
        assert np.array_equal(part, r[lr == j]), j
