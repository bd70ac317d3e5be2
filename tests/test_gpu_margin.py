"""How much margin the screen's error bound has, measured.

Every top-1 and top-k result is exact only if the screen's key of each listed
candidate is within the per-row bound E (screen_bound) of the exact fma-chain
key the check computes. emh_screen_margin runs the screen on a call's
arguments and re-scores every list entry with that chain; these tests assert
that no entry is beyond E, and that the dot error stays within half of the
bound's dot term (the split and the MFMA rounding model, the part that rests
on probes of the hardware) once the allowances for the keys' own IEEE
rounding and the column tag are taken off. (Two correctly rounded L2 keys may
lie an ulp apart whatever the dot error, so |screen key - exact key| / E alone
can reach 1/1.125 on rows where that allowance dominates E.) Inputs are
adversarial: crowds of centroids within 1e-6,
exact duplicates, rows at scales 1e3 .. 1e-15, rows in the bf16 subnormal
range, centroids up to 5e17 (1e34 overflows the bound's |c|^2 and sends every
row to the exact scan), d from 36 to 2500 (d < 32 runs no screen), both
screen arithmetics, the split-operand screen's filtered single-tile lists
(k <= 2048), the sorted many-tile lists of larger k, the 128 x 128 screen of
small k, and the kNN screen's 24-entry lists. They
also pin which screen variant ran, whatever the CU count. With
EMEANS_MARGIN_OUT set, each case's report is appended to that file (JSON lines).
"""

import json
import os

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    from emeans_amd import HipDevice
    d = HipDevice()
    d.set_exact_below(0)  # The screens run at every size here
    yield d
    d.close()


def _mix(n, d, centers, sigma, unit, seed):
    return O.contract_mixture(n, d, centers, sigma, unit, seed).reshape(n, d)


def _noise(i):
    i = np.asarray(i, np.uint64)
    with np.errstate(over="ignore"):
        h = i * np.uint64(0x9E3779B97F4A7C15)
        h = ((h << np.uint64(29)) | (h >> np.uint64(35))) ^ np.uint64(0xD1B54A32D192ED03)
        h = h * np.uint64(0x94D049BB133111EB)
    return (h >> np.uint64(11)).astype(np.float64) / float(1 << 52) - 1.0


def _record(tag, r):
    path = os.environ.get("EMEANS_MARGIN_OUT")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps({"case": tag, **r}) + "\n")


def _margin(dev, x, c, metric, tag, variant=None, ids=None):
    from emeans_amd import Mat, Select
    n, d = x.shape
    k = c.shape[0]
    xb, cb = dev.bind(x), dev.upload_f32(c)
    cn = None
    if metric == "l2":
        cn = dev.zeros_f32(k)
        dev.row_norms(cb, k, d, cn)
    idb = dev.upload_u32(ids) if ids is not None else None
    r = dev.screen_margin(Mat(xb, d), Select(idb, (0, n if ids is None else len(ids))), cb, cn,
                          k, metric)
    _record(tag, r)
    if variant is not None:
        assert r["variant"] == variant, (tag, r)
    if r["variant"] != "none":
        assert r["pairs"] > 0 or "beyond range" in tag, (tag, r)
        assert r["over"] == 0 and r["max_ratio"] <= 1.0, (tag, r)
        assert r["max_dot_ratio"] <= 0.5, (tag, r)
    return r


def _crowds(k, d, seed):
    """Half the centroids in crowds of 32 within 1e-6 (one exact duplicate
    each), the other half in pairs within 1e-6 (every other pair duplicated)."""
    crowds, pairs = k // 2 // 32, k // 2 // 2
    groups = crowds + pairs
    bases = _mix(groups, d, groups, 0.0, True, seed)
    c = np.zeros((k, d), np.float32)
    t = np.arange(d)
    for j in range(k):
        if j < k // 2:
            g, first, dup = j // 32, j % 32 == 0, j % 32 == 31
        else:
            q = (j - k // 2) // 2
            g, first, dup = crowds + q, j % 2 == 0, j % 2 == 1 and q % 2 == 1
        if dup:
            c[j] = c[j - 31 if j < k // 2 else j - 1]
        elif first:
            c[j] = bases[g]
        else:
            c[j] = (bases[g].astype(np.float64) * (1.0 + 1e-6 * _noise(j * d + t))).astype(np.float32)
    return c, groups


@pytest.mark.parametrize("mode", [1, 2, 3], ids=["bf16x3", "f32", "f16x2"])
@pytest.mark.parametrize("metric", ["ip", "l2"])
@pytest.mark.parametrize("d", [36, 99, 768, 2500])
def test_margin_near_tie_crowds(dev, mode, metric, d):
    n, k = 16384, 512  # 64 row tiles x 2 parts: enough blocks for the split-operand screen
    c, groups = _crowds(k, d, 21)
    rows = _mix(n, d, groups, 0.05, True, 21)
    scale = np.array([1.0, 1e3, 1e-3, 1e-15], np.float32)[np.arange(n) % 4]
    x = (rows * scale[:, None]).astype(np.float32)
    dev.set_screen(mode)
    try:
        want = {1: "big_tagged", 2: "small_f32", 3: "big_f16"}[mode]
        _margin(dev, x, c, metric, f"crowds d={d} {metric} screen={mode}", want)
    finally:
        dev.set_screen(1)


@pytest.mark.parametrize("metric", ["ip", "l2"])
def test_margin_extreme_scales(dev, metric):
    """Rows in the bf16 subnormal range (1e-40 .. 1e-36) up to 1e18 against
    centroids up to 5e17, the largest scale whose squared norm (the bound's
    input) stays finite at d = 768 (IP); for L2, scales whose squared norms
    stay finite. Centroids at 1e34 overflow |c|^2: the bound is infinite and
    every row goes to the exact scan, so no list entry is measured."""
    n, d, k = 2048, 768, 256
    base = _mix(n, d, 16, 0.2, True, 31)
    cb = _mix(k, d, 16, 0.2, True, 32)
    if metric == "ip":
        xs = np.array([1e-40, 1e-38, 1e-36, 1e-20, 1.0, 1e18], np.float64)
        cs = np.array([5e17, 1e-38, 1.0], np.float64)
    else:
        xs = np.array([1e-30, 1e-18, 1.0, 1e15], np.float64)
        cs = np.array([1e-18, 1.0, 1e15], np.float64)
    x = (base * xs[np.arange(n) % len(xs)][:, None]).astype(np.float32)
    c = (cb * cs[np.arange(k) % len(cs)][:, None]).astype(np.float32)
    for mode in (1, 2, 3):
        dev.set_screen(mode)
        try:
            _margin(dev, x, c, metric, f"extreme scales {metric} screen={mode}")
            if metric == "ip":
                huge = (cb * np.float32(1e34)).astype(np.float32)
                r = dev.screen_margin(*_args(dev, x, huge), "ip")
                assert r["pairs"] == 0 and r["variant"] != "none", r
        finally:
            dev.set_screen(1)


@pytest.mark.parametrize("metric", ["ip", "l2"])
def test_margin_f16_ranges(dev, metric):
    """The fp16 two-pass screen (mode 3) on rows from 1e-6 to 1e3 and
    centroids from 1e-3 to 1e2 (32,768 rows x 512 centroids: the
    split-operand screen): every entry within the bound. Centroids beyond
    |c| = 32768 make the bound NaN, so no entry is measured and every row
    takes the exact scan: the labels and scores still equal the exact
    kernels' bits."""
    n, d, k = 32768, 256, 512
    base = _mix(n, d, 32, 0.3, True, 61)
    cb = _mix(k, d, 32, 0.3, True, 62)
    xs = np.array([1e-6, 1e-3, 1.0, 1e3], np.float64)
    cs = np.array([1e-3, 1.0, 1e2], np.float64)
    x = (base * xs[np.arange(n) % len(xs)][:, None]).astype(np.float32)
    c = (cb * cs[np.arange(k) % len(cs)][:, None]).astype(np.float32)
    dev.set_screen(3)
    try:
        _margin(dev, x, c, metric, f"f16 ranges {metric}", "big_f16")
        big = (cb * np.float32(1e5)).astype(np.float32)
        r = _margin(dev, x, big, metric, f"f16 beyond range {metric}", "big_f16")
        assert r["pairs"] == 0, r
        got = _top1(dev, x, big, metric)
    finally:
        dev.set_screen(1)
    dev.set_screen(0)
    try:
        want = _top1(dev, x, big, metric)
    finally:
        dev.set_screen(1)
    assert np.array_equal(got[0], want[0]) and got[1].tobytes() == want[1].tobytes()


def _top1(dev, x, c, metric):
    from emeans_amd import Mat, Select
    n, d = x.shape
    k = c.shape[0]
    cb = dev.upload_f32(c)
    cn = None
    if metric == "l2":
        cn = dev.zeros_f32(k)
        dev.row_norms(cb, k, d, cn)
    lab, sco = dev.zeros_u32(n), dev.zeros_f32(n)
    dev.top1(Mat(dev.bind(x), d), Select(None, (0, n)), cb, cn, k, metric, lab, sco)
    return dev.read_u32(lab), dev.read_f32(sco)


def _args(dev, x, c):
    from emeans_amd import Mat, Select
    n, d = x.shape
    return Mat(dev.bind(x), d), Select(None, (0, n)), dev.upload_f32(c), None, c.shape[0]


@pytest.mark.parametrize("metric", ["ip", "l2"])
def test_margin_tagged_and_sorted_lists(dev, metric):
    """16,384 rows: k = 1024 takes the split-operand screen (parts of one
    256-centroid tile, tagged keys), k = 4096 the screen that splits its own
    slabs with parts of several tiles (sorted insert): both measured, and the
    variant each ran is the one expected."""
    from emeans_amd import HipDevice
    n, d = 16384, 256
    x = _mix(n, d, 64, 0.6, metric == "ip", 9 * n)
    for k, want in ((1024, "big_tagged"), (4096, "big_sorted")):
        c = (x[(np.arange(k) * 37) % n] * np.float32(0.95)).astype(np.float32)
        r = _margin(dev, x, c, metric, f"lists k={k} {metric}", want)
        assert (r["tiles_per_part"] == 1) == (want == "big_tagged")


@pytest.mark.parametrize("mode", [1, 2], ids=["bf16x3", "f32"])
@pytest.mark.parametrize("k", [2, 21, 63])
def test_margin_small_k(dev, mode, k):
    """Small k on the 128 x 128 screen (one partly filled tile) at d = 768,
    crowded near ties included."""
    n, d = 4096, 768
    c = _mix(k, d, k, 0.0, True, 40 + k)
    if k > 2:
        c[1] = (c[0].astype(np.float64) * (1.0 + 1e-6 * _noise(np.arange(d)))).astype(np.float32)
    x = _mix(n, d, k, 0.3, True, 50 + k)
    dev.set_screen(mode)
    try:
        for metric in ("ip", "l2"):
            want = "small_f32" if mode == 2 else "small_bf16"
            _margin(dev, x, c, metric, f"small k={k} {metric} screen={mode}", want)
    finally:
        dev.set_screen(1)


def test_margin_no_screen_below_32_dims(dev):
    x = _mix(1000, 13, 8, 0.5, False, 3)
    r = _margin(dev, x, x[:100].copy(), "l2", "d=13", "none")
    assert r["pairs"] == 0


def test_margin_headline_batch(dev):
    """A 16,384-row batch of the 200k x 768 L2 mixture against 1024 of its rows."""
    from emeans_amd import synth
    x, _ = synth.gmm_zipf(n=40_000, d=768, comps=1024, s=1.1, seed=0)
    c = x[(np.arange(1024) * 37) % x.shape[0]].copy()
    ids = ((np.arange(16384, dtype=np.uint64) * 7919 + 11) % x.shape[0]).astype(np.uint32)
    _margin(dev, x, c, "l2", "headline batch", "big_tagged", ids=ids)
    # An epoch's tail batch (3,392 rows: 56 large-tile blocks) takes the 128 x 128 screen.
    _margin(dev, x, c, "l2", "headline tail batch", "small_bf16", ids=ids[:3392].copy())
    # The training run's arithmetic on the same batch: fp16 two-pass.
    dev.set_screen(3)
    try:
        r = _margin(dev, x, c, "l2", "headline batch fp16", "big_f16", ids=ids)
        assert r["pairs"] > 0, r
    finally:
        dev.set_screen(1)


@pytest.mark.parametrize("mode", [1, 2], ids=["bf16x3", "f32"])
def test_margin_knn_lists(dev, mode):
    """The kNN screen's merged lists on unit rows with near-duplicates (d = 384)."""
    from emeans_amd import synth
    n, d = 20_000, 384
    x, _, _ = synth.knn_near_duplicates(n=n, d=d, seed=2)
    xb = dev.bind(x)
    dev.set_screen(mode)
    try:
        r = dev.screen_margin_topk(xb, n, xb, n, d, True)
    finally:
        dev.set_screen(1)
    _record(f"knn 20000x384 screen={mode}", r)
    assert r["variant"] == ("small_f32" if mode == 2 else "big_knn")
    assert r["pairs"] > 0 and r["over"] == 0 and r["max_dot_ratio"] <= 0.5, r


def test_margin_knn_lists_small_screen(dev):
    """The 128 x 128 kNN screen, which calls of fewer than 256 queries take."""
    from emeans_amd import synth
    n, d = 8_000, 384
    x, _, _ = synth.knn_near_duplicates(n=n, d=d, seed=4)
    r = dev.screen_margin_topk(dev.bind(x[:200]), 200, dev.bind(x), n, d, False)
    _record("knn 200x8000x384 small screen", r)
    assert r["variant"] == "small_bf16"
    assert r["pairs"] > 0 and r["over"] == 0 and r["max_dot_ratio"] <= 0.5, r
