"""The C ABI without a GPU: the library loads, exports every function that
include/emeans_hip.h declares, refuses to run without a gfx950 device, and its
host-side replay (MT19937, recipe, schedule, revival plan, pairwise sum, dedup
grouping) matches the reference's golden vectors and the oracle."""

import ctypes as C
import json
import os
import re

import numpy as np
import pytest

from emeans_amd import _lib
from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "emeans_hip.h")
GOLD = os.path.join(ROOT, "tests", "golden")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(emh_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return _lib.lib()


@pytest.fixture(scope="module")
def ref():
    with open(os.path.join(GOLD, "reference.json")) as f:
        return json.load(f)


def test_every_declared_function_is_exported_and_typed(lib):
    names = declared_functions()
    assert len(names) >= 45, names
    raw = C.CDLL(_lib.LIB_PATH)
    for name in names:
        assert hasattr(raw, name), f"{name} declared in the header but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    # and the loader types nothing the header does not declare
    assert set(_lib.SIGNATURES) <= set(names)


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is present on this host")
def test_create_fails_without_a_device(lib):
    ctx = C.c_void_p()
    rc = lib.emh_create(0, C.byref(ctx))
    assert rc == _lib.EMH_ERROR
    assert not ctx.value, "no context is written on failure"
    assert lib.emh_last_error()


def test_null_context_is_an_invalid_argument(lib):
    assert lib.emh_sync(None) == _lib.EMH_INVALID
    assert lib.emh_top1(None, None, 8, None, 0, 1, None, None, 4, 0, None, None) == _lib.EMH_INVALID
    assert b"" != lib.emh_last_error()
    out = C.c_void_p()
    assert lib.emh_zeros_f32(None, 4, C.byref(out)) == _lib.EMH_INVALID
    assert not out.value


def test_host_permutation_and_samples_match_the_fixture(lib, ref):
    for c in ref["mt19937"]:
        seed = c["seed"]
        if "random_sample" in c:
            got = [lib.emh_host_random_sample(seed, i) for i in range(len(c["random_sample"]))]
            assert got == c["random_sample"], seed
            continue
        n = c["n"]
        p = np.empty(n, np.uint32)
        lib.emh_host_permutation(seed, n, p.ctypes.data)
        assert p[:64].tolist() == c["head"], (seed, n)
        m = min(n, 5000)
        assert int(np.dot(np.arange(m, dtype=np.int64), p[:m].astype(np.int64))) == c["sum"]


def test_host_permutation_equals_numpy_across_sizes(lib):
    """Whole permutations against numpy's legacy RandomState, on both sides of
    the size where the swaps move to a second thread (2^15) and of the masks'
    power-of-two boundaries."""
    for seed, n in [(0, 1), (1, 2), (2, 3), (3, 624), (4, 625), (5, 32767), (6, 32768),
                    (7, 65536), (8, 65537), (9, 200000), (10, 262145)]:
        p = np.empty(n, np.uint32)
        lib.emh_host_permutation(seed, n, p.ctypes.data)
        assert np.array_equal(p, np.random.RandomState(seed).permutation(n)), (seed, n)


def _cfg(c):
    cfg = _lib.Config()
    cfg.k, cfg.d, cfg.nepochs, cfg.seed = c["k"], c["d"], float(c["nepochs"]), 1234
    law = c["batch_law"]
    cfg.batch_law = {"auto": 0, "throughput": 1, "quality": 2, "given": 1}[law]
    if law == "given":
        cfg.batch_size = c["given_batch_size"]
        if c.get("given_alpha0") is not None:
            cfg.has_alpha0, cfg.alpha0 = 1, c["given_alpha0"]
    return cfg


def test_host_recipe_matches_the_fixture(lib, ref):
    rows = (C.c_uint64 * 64)()
    for c in ref["recipes"]:
        b, a0, ne, tot = C.c_uint64(), C.c_double(), C.c_uint64(), C.c_uint64()
        cfg = _cfg(c)
        rc = lib.emh_host_recipe(c["n"], C.byref(cfg), C.byref(b), C.byref(a0), rows, 64,
                                 C.byref(ne), C.byref(tot))
        assert rc == _lib.EMH_OK
        assert b.value == c["batch_size"], c
        assert a0.value == c["alpha0"], ("alpha0 bits", c)
        if "epoch_rows" in c:
            assert list(rows[: ne.value]) == c["epoch_rows"], c
            assert tot.value == c["total_steps"], c


def test_host_schedule_matches_the_fixture(lib, ref):
    for c in ref["alphas"]:
        assert lib.emh_host_scheduled_alpha(c["alpha0"], c["step"], c["total"]) == c["alpha"], c


def test_host_revival_plan_and_pairwise_sum_match_the_oracle(lib):
    g = np.random.default_rng(5)
    for k in (7, 64, 1024):
        usage = g.gamma(0.3, 1.0, k).astype(np.float32)
        usage[g.choice(k, k // 4, replace=False)] = 0.0
        pairs = np.empty(2 * k, np.uint32)
        npairs = lib.emh_host_plan_revival(usage.ctypes.data, k, 0.1, 1234, pairs.ctypes.data)
        want = O.plan_revival(usage, 0.1, O.RandomState(1234))
        assert pairs[: 2 * npairs].tolist() == np.asarray(want).reshape(-1).tolist(), k
        s = lib.emh_host_numpy_sum_f32(usage.ctypes.data, k)
        assert np.float32(s) == np.sum(usage, dtype=np.float32), k


def test_host_revival_plan_over_many_masses_matches_the_oracle(lib):
    """The plan computes exact keys only for donors an approximate key cannot
    rule out: the pairs equal the oracle's over mass distributions with few
    and many dead clusters, ties, subnormal and huge masses, and k = 1024."""
    g = np.random.default_rng(21)
    cases = 0
    for k in (16, 257, 1024):
        for it in range(12):
            kind = it % 4
            if kind == 0:
                usage = g.gamma(0.3, 1.0, k)
            elif kind == 1:
                usage = g.pareto(1.1, k) * 1e-3
            elif kind == 2:
                usage = np.repeat(g.random(k // 8 + 1), 8)[:k]  # many ties
            else:
                usage = np.exp(g.uniform(-100, 80, k))  # subnormal to huge
            usage = usage.astype(np.float32)
            usage[g.choice(k, int(k * g.uniform(0.02, 0.5)), replace=False)] = 0.0
            tau = float(g.choice([0.05, 0.1, 0.5, 2.0]))
            seed = int(g.integers(0, 2**32))
            pairs = np.empty(2 * k, np.uint32)
            npairs = lib.emh_host_plan_revival(usage.ctypes.data, k, tau, seed, pairs.ctypes.data)
            want = O.plan_revival(usage, tau, O.RandomState(seed))
            assert pairs[: 2 * npairs].tolist() == np.asarray(want).reshape(-1).tolist(), (k, it)
            cases += npairs > 0
    assert cases > 20


def test_dedup_neighbors_matches_the_oracle(lib):
    """The host grouping with every side input: priorities, creation times
    (some unknown) under a time gap, and burst ids, against the oracle."""
    from emeans_amd import DedupConfig, DedupInput, Neighbors, dedup_with_neighbors
    g = np.random.default_rng(11)
    n, d, kk = 400, 16, 5
    x = g.standard_normal((n, d)).astype(np.float32)
    dst = g.choice(n, 60, replace=False)
    src = g.choice(np.setdiff1d(np.arange(n), dst), 60)
    x[dst] = x[src] + 0.02 * g.standard_normal((60, d)).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    ids, sims = O.knn(x, x, d, kk, True)
    pr = g.random(n).astype(np.float32)
    t = g.uniform(0, 600, n)
    t[g.choice(n, 40, replace=False)] = np.nan
    burst = [None] * n
    for b, rows in enumerate(np.array_split(g.choice(n, 90, replace=False), 30)):
        for r in rows:
            burst[r] = b
    cases = [(DedupInput(), DedupConfig(sim_threshold=0.97)),
             (DedupInput(priority=pr), DedupConfig(sim_threshold=0.97)),
             (DedupInput(created_unix=t), DedupConfig(sim_threshold=0.97, max_gap_secs=120.0)),
             (DedupInput(burst=burst, priority=pr),
              DedupConfig(sim_threshold=0.97, rep_threshold=0.98)),
             (DedupInput(created_unix=t, burst=burst),
              DedupConfig(sim_threshold=0.96, max_gap_secs=200.0))]
    for inp, cfg in cases:
        want = O.dedup(x, d, ids, sims, kk, cfg.sim_threshold, cfg.rep_threshold,
                       priority=inp.priority, created_unix=inp.created_unix,
                       max_gap_secs=cfg.max_gap_secs, burst=inp.burst)
        r = dedup_with_neighbors(x, d, Neighbors(kk, ids, sims), inp, cfg)
        assert r.group_of.tolist() == want["group_of"].tolist()
        assert r.representatives.tolist() == want["representatives"].tolist()
        assert r.anchors.tolist() == want["anchors"].tolist()
        assert r.sizes.tolist() == want["sizes"].tolist()
        assert (r.linked_pairs, r.split_components) == (want["linked_pairs"],
                                                        want["split_components"])
        assert r.n_groups() < n  # the injected duplicates merged
        if inp.burst is not None:  # rows of one burst share a group
            for b in range(30):
                rows = [i for i in range(n) if burst[i] == b]
                assert len(set(r.group_of[rows].tolist())) == 1


def test_dedup_neighbors_rejects_bad_arguments(lib):
    from emeans_amd import DedupConfig, DedupInput, EmeansHipInvalid, Neighbors, \
        dedup_with_neighbors
    from emeans_amd._lib import DedupConfig as CCfg, DedupInput as CIn, DedupResult as COut
    x = np.zeros((2, 4), np.float32)
    ids = np.zeros(2, np.uint32)
    sims = np.zeros(2, np.float32)
    out = [np.zeros(2, np.uint32) for _ in range(4)]
    res = COut(*[o.ctypes.data for o in out], None, 7, 0, 0)
    cfg = CCfg(10, 1.5, 0, 0.0, 0, 0.0)
    rc = lib.emh_dedup_neighbors(x.ctypes.data, 2, 4, ids.ctypes.data, sims.ctypes.data, 1,
                                 C.byref(CIn()), C.byref(cfg), C.byref(res))
    assert rc == _lib.EMH_INVALID
    assert b"sim_threshold" in lib.emh_last_error()
    assert res.n_groups == 7, "no out-parameter is written on failure"
    nb = Neighbors(1, ids, sims)
    with pytest.raises(EmeansHipInvalid, match="priority"):
        dedup_with_neighbors(x, 4, nb, DedupInput(priority=np.array([0, np.nan], np.float32)))
    with pytest.raises(ValueError, match="one timestamp per row"):
        dedup_with_neighbors(x, 4, nb, DedupInput(created_unix=np.zeros(3)), DedupConfig())


def test_backend_names_and_availability():
    """The "hip" name as emeans_cluster::Backend would list it (backend.rs:41-102)
    and available_backends (bindings/common/src/lib.rs:131-137): names whose
    make_assigner succeeds; none on a machine without a gfx950 device."""
    from emeans_amd import Backend, EmeansHipError, available_backends, make_assigner
    assert Backend.NAMES == ("hip",)
    assert Backend.from_str("hip") == Backend.from_str("hip-gfx950")
    assert Backend.from_str("hip-gfx950").name() == "hip"
    with pytest.raises(ValueError, match=r"unknown backend 'cuda' \(hip\)"):
        Backend.from_str("cuda")
    if not os.path.exists("/dev/kfd"):
        assert available_backends() == []
        with pytest.raises(EmeansHipError):
            make_assigner(Backend.from_str("hip"))
