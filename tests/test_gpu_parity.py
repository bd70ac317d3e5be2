"""Layer-1 parity on the GPU: every Device op against the oracle, bit for bit.

The shapes and inputs are the reference contract's (core/contract.rs:75-161,
355-554) and the CUDA backend's adversarial near-tie set
(emeans-cuda/tests/contract.rs:44-152). The bar is the reference CPU
backend's exact output: labels, scores, sums, EMA, splits and norms
bit-equal; kNN ids and sims bit-equal to the oracle's fma-chain order.
"""

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    from emeans_amd import HipDevice
    d = HipDevice()
    d.set_exact_below(0)  # These tests exercise the screens at small sizes too
    yield d
    d.close()


@pytest.fixture(params=[1, 2, 3], ids=["bf16x3", "f32", "f16x2"])
def screen(request, dev):
    """The MFMA screen's arithmetic: bf16 three-pass (default) or f32."""
    dev.set_screen(request.param)
    yield request.param
    dev.set_screen(1)


def _mix(n, d, centers, sigma, unit, seed):
    return O.contract_mixture(n, d, centers, sigma, unit, seed).reshape(n, d)


def _gpu_top1(dev, x, c, metric, ids=None, rows=None, fill=True):
    from emeans_amd import Mat, Select
    n, d = x.shape
    k = c.shape[0]
    xb = dev.bind(x)
    cb = dev.upload_f32(c)
    cn = None
    if metric == "l2":
        cn = dev.zeros_f32(k)
        dev.row_norms(cb, k, d, cn)
    n_sel = len(ids) if ids is not None else n
    lo, hi = rows if rows is not None else (0, n_sel)
    lab = dev.upload_u32(np.full(n_sel, 0xFFFFFFFF, np.uint32))
    sco = dev.upload_f32(np.full(n_sel, np.nan, np.float32))
    idb = dev.upload_u32(ids) if ids is not None else None
    dev.top1(Mat(xb, d), Select(idb, (lo, hi)), cb, cn, k, metric, lab, sco)
    return dev.read_u32(lab), dev.read_f32(sco)


def _check_top1(dev, x, c, metric, tag):
    n, d = x.shape
    perm = ((np.arange(n, dtype=np.uint64) * 7919 + 13) % n).astype(np.uint32)
    lo, hi = n // 7, n - n // 9
    for ids in (perm, None):
        gl, gs = _gpu_top1(dev, x, c, metric, ids=ids, rows=(lo, hi))
        ol = np.full(n, 0xFFFFFFFF, np.uint32)
        osc = np.full(n, np.nan, np.float32)
        O.top1(x, d, c, metric, ids=ids, rows=(lo, hi), labels=ol, scores=osc)
        # Only the selection is written (contract.rs:225-231).
        assert np.all(gl[:lo] == 0xFFFFFFFF) and np.all(gl[hi:] == 0xFFFFFFFF), tag
        assert np.all(np.isnan(gs[:lo])) and np.all(np.isnan(gs[hi:])), tag
        bad = np.nonzero(gl[lo:hi] != ol[lo:hi])[0]
        assert bad.size == 0, f"{tag}: {bad.size} labels differ, first at {lo + bad[0]}"
        assert gs[lo:hi].tobytes() == osc[lo:hi].tobytes(), f"{tag}: scores not bit-equal"


CONTRACT_SHAPES = [(1000, 768, 64), (777, 768, 100), (513, 13, 70), (2000, 20, 300),
                   (300, 64, 1), (600, 768, 1024)]


@pytest.mark.parametrize("n,d,k", CONTRACT_SHAPES)
@pytest.mark.parametrize("metric", ["ip", "l2"])
def test_top1_contract_shapes(dev, screen, n, d, k, metric):
    x = _mix(n, d, 11, 0.6, metric == "ip", 3 * n + k)
    c = (np.resize(x[: min(k, n)].reshape(-1), k * d) * np.float32(0.95)).reshape(k, d)
    _check_top1(dev, x, c, metric, f"n={n} d={d} k={k} {metric}")


@pytest.mark.parametrize("k", [1024, 1000])
@pytest.mark.parametrize("metric", ["ip", "l2"])
def test_top1_production_shape_with_duplicates(dev, screen, k, metric):
    """contract.rs:120-146: 16,384 x 768; the last 256 centroids copy earlier ones."""
    n, d = 16384, 768
    x = _mix(n, d, 64, 0.6, metric == "ip", 5 * n + k)
    base = k - 256
    c = np.zeros((k, d), np.float32)
    for j in range(k):
        c[j] = x[(j * 37) % n] * np.float32(0.95) if j < base else c[(j * 7) % base]
    gl, gs = _gpu_top1(dev, x, c, metric)
    ol, osc = O.top1(x, d, c, metric)
    assert np.array_equal(gl, ol)
    assert gs.tobytes() == osc.tobytes()
    # Exact duplicates: the lower id wins (contract.rs:237-243).
    assert np.all(gl < base)


@pytest.mark.parametrize("n,k", [(16384, 2048), (8192, 4096)])
@pytest.mark.parametrize("metric", ["ip", "l2"])
def test_top1_parts_of_several_tiles(dev, screen, n, k, metric):
    """2,048 centroids: the split-operand screen's eight single-tile parts
    (tagged keys); 4,096 centroids (16 tiles, more than eight parts): the
    large-tile screen that splits its own slabs, on 256 CUs eight parts of two
    tiles each, so its lists take the sorted insert across tiles. Bit-equal to
    the oracle; with the bf16 screen, the variant that ran is the intended one
    (the parts follow the device's CU count)."""
    from emeans_amd import Mat, Select
    d = 256
    x = _mix(n, d, 64, 0.6, metric == "ip", 7 * n + k)
    c = (x[(np.arange(k) * 37) % n] * np.float32(0.95)).astype(np.float32)
    gl, gs = _gpu_top1(dev, x, c, metric)
    ol, osc = O.top1(x, d, c, metric)
    assert np.array_equal(gl, ol)
    assert gs.tobytes() == osc.tobytes()
    if screen == 1:
        cb = dev.upload_f32(c)
        cn = None
        if metric == "l2":
            cn = dev.zeros_f32(k)
            dev.row_norms(cb, k, d, cn)
        r = dev.screen_margin(Mat(dev.bind(x), d), Select(None, (0, n)), cb, cn, k, metric)
        want = "big_tagged" if k <= 2048 else "big_sorted"
        assert r["variant"] == want, r
        assert (r["tiles_per_part"] == 1) == (want == "big_tagged"), r


@pytest.mark.parametrize("k", [2, 3, 21, 40, 63])
@pytest.mark.parametrize("d", [768, 99, 32])
@pytest.mark.parametrize("metric", ["ip", "l2"])
def test_top1_small_k(dev, screen, k, d, metric):
    """Small k (the automatic-k sweeps' k = 2 .. 40) on the 128 x 128 screen
    with one partly filled centroid tile: an exact duplicate pair, a near pair
    within 1e-6 and rows on the bisector of two centroids."""
    n = 6000
    x = _mix(n, d, 9, 0.4, metric == "ip", 11 * k + d)
    c = (x[(np.arange(k) * 101) % n] * np.float32(0.97)).astype(np.float32)
    if k >= 3:
        c[k - 1] = c[0]  # the lower id wins
        c[1] = (c[0].astype(np.float64) * (1.0 + 1e-6 * _noise(np.arange(d)))).astype(np.float32)
    mid = (0.5 * (c[0].astype(np.float64) + c[k // 2])).astype(np.float32)
    x[::7] = mid
    _check_top1(dev, x, c, metric, f"small k={k} d={d} {metric}")


@pytest.mark.parametrize("metric", ["ip", "l2"])
def test_small_calls_take_the_exact_scan(dev, metric):
    """By default, calls of at most 4096 exact items (rows x max(ceil(k / 64), 2)),
    or of at most 1024 items of the latency-bound scan (4 rows x 16 centroids,
    d % 4 == 0), run the exact kernels alone instead of the screen: a choice of
    speed only. On both sides of each boundary the bits equal the screened
    call's and the oracle's."""
    d = 768
    for n, k in ((2048, 64), (2049, 64), (2048, 65), (2049, 65), (64, 4), (300, 2),
                 (4096, 2), (4097, 2), (1024, 256), (1025, 256)):
        x = _mix(n, d, 9, 0.4, metric == "ip", n + k)
        c = (x[(np.arange(k) * 101) % n] * np.float32(0.97)).astype(np.float32)
        c[k - 1] = c[0]  # the lower id wins
        dev.set_exact_below(dev.EXACT_BELOW)
        try:
            dl, ds = _gpu_top1(dev, x, c, metric)
        finally:
            dev.set_exact_below(0)
        sl, ss = _gpu_top1(dev, x, c, metric)
        ol, osc = O.top1(x, d, c, metric)
        assert np.array_equal(dl, ol) and ds.tobytes() == osc.tobytes(), f"n={n} k={k} default"
        assert np.array_equal(sl, ol) and ss.tobytes() == osc.tobytes(), f"n={n} k={k} screened"


def _noise(i):
    i = np.asarray(i, np.uint64)
    with np.errstate(over="ignore"):
        h = i * np.uint64(0x9E3779B97F4A7C15)
        h = ((h << np.uint64(29)) | (h >> np.uint64(35))) ^ np.uint64(0xD1B54A32D192ED03)
        h = h * np.uint64(0x94D049BB133111EB)
    return (h >> np.uint64(11)).astype(np.float64) / float(1 << 52) - 1.0


@pytest.mark.parametrize("n,d,k", [(4000, 768, 512), (3000, 72, 256)])
@pytest.mark.parametrize("metric", ["ip", "l2"])
def test_screen_bit_equal_on_near_ties(dev, n, d, k, metric):
    """emeans-cuda/tests/contract.rs:44-152: crowds of 32 centroids within 1e-6,
    pairs within 1e-6, exact duplicates, rows scaled 1, 1e3, 1e-3, 1e-15."""
    crowds, pairs = k // 2 // 32, k // 2 // 2
    groups = crowds + pairs
    bases = _mix(groups, d, groups, 0.0, True, 21)
    c = np.zeros((k, d), np.float32)
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
            t = np.arange(d)
            c[j] = (bases[g].astype(np.float64) * (1.0 + 1e-6 * _noise(j * d + t))).astype(np.float32)
    rows = _mix(n, d, groups, 0.05, True, 21)
    scale = np.array([1.0, 1e3, 1e-3, 1e-15], np.float32)[np.arange(n) % 4]
    x = (rows * scale[:, None]).astype(np.float32)
    perm = ((np.arange(n, dtype=np.uint64) * 7919 + 5) % n).astype(np.uint32)
    outs = []
    for mode in (1, 2, 0):  # bf16 screen, f32 screen, exact kernel alone
        dev.set_screen(mode)
        outs.append(_gpu_top1(dev, x, c, metric, ids=perm))
    dev.set_screen(1)
    ol, osc = O.top1(x, d, c, metric, ids=perm)
    for mode, (gl, gs) in zip((1, 2, 0), outs):
        assert np.array_equal(gl, ol), f"mode {mode} labels"
        assert gs.tobytes() == osc.tobytes(), f"mode {mode} scores"


@pytest.mark.parametrize("layout", ["spread", "together"])
@pytest.mark.parametrize("metric", ["ip", "l2"])
def test_check_several_candidates_per_row(dev, screen, metric, layout):
    """Centroids in groups within a relative 1e-7 of each other, rows near the
    groups: every row keeps all of its group's members inside the screen bound.
    spread: groups of four, fewer than a part's list keeps, so each 32-row block
    of the check holds 128 (row, candidate) pairs and takes several passes over
    its staged chunks, and the check settles the rows. together: groups of six
    consecutive ids in one part, whose list overflows, so the rows go to the
    exact scan. Labels and scores bit-equal to the oracle, and to the exact
    kernel, either way."""
    n, d, k = 2048, 256, 192
    g = 4 if layout == "spread" else 6
    groups = k // g
    bases = _mix(groups, d, groups, 0.0, True, 7)
    t = np.arange(d)
    group_of = (np.arange(k) % groups) if layout == "spread" else (np.arange(k) // g)
    c = np.stack([(bases[group_of[j]].astype(np.float64) * (1.0 + 1e-7 * _noise(j * d + t)))
                  .astype(np.float32) for j in range(k)])
    x = _mix(n, d, groups, 0.05, True, 7)
    perm = ((np.arange(n, dtype=np.uint64) * 7919 + 3) % n).astype(np.uint32)
    before = dev.fallback_rows()
    gl, gs = _gpu_top1(dev, x, c, metric, ids=perm)
    rescanned = dev.fallback_rows() - before
    ol, osc = O.top1(x, d, c, metric, ids=perm)
    assert np.array_equal(gl, ol)
    assert gs.tobytes() == osc.tobytes()
    if layout == "spread":
        assert rescanned < n // 10, rescanned  # the check settled them, not the exact scan
    else:
        assert rescanned > n // 2, rescanned  # a full list that cannot certify its part
    dev.set_screen(0)
    el, es = _gpu_top1(dev, x, c, metric, ids=perm)
    dev.set_screen(screen)
    assert np.array_equal(gl, el) and gs.tobytes() == es.tobytes()


@pytest.mark.parametrize("d", [1000, 100])
@pytest.mark.parametrize("metric", ["ip", "l2"])
def test_queued_rows_across_phases(dev, metric, d):
    """Groups of six near-identical consecutive centroids overflow their part's
    list, so every row is queued for the exact scan: d = 1000 takes the scan's
    copies in two phases (768 + 232 dimensions), d = 100 in one partial phase,
    and k = 200 leaves the last 16-centroid item part-empty. Bit-equal to the
    oracle."""
    n, k, g = 700, 200, 6
    groups = (k + g - 1) // g
    bases = _mix(groups, d, groups, 0.0, True, 17)
    t = np.arange(d)
    c = np.stack([(bases[j // g].astype(np.float64) * (1.0 + 1e-7 * _noise(j * d + t)))
                  .astype(np.float32) for j in range(k)])
    x = _mix(n, d, groups, 0.05, True, 17)
    before = dev.fallback_rows()
    gl, gs = _gpu_top1(dev, x, c, metric)
    assert dev.fallback_rows() - before > n // 2
    ol, osc = O.top1(x, d, c, metric)
    assert np.array_equal(gl, ol)
    assert gs.tobytes() == osc.tobytes()


def test_screen_fallback_is_rare_on_separated_data(dev, screen):
    """On data without near-ties the exact kernel rescans few rows."""
    n, d, k = 16384, 768, 1024
    x = _mix(n, d, 64, 0.6, False, 99)
    c = x[(np.arange(k) * 13) % n] * np.float32(0.95)
    before = dev.fallback_rows()
    gl, gs = _gpu_top1(dev, x, c, "l2")
    rescanned = dev.fallback_rows() - before
    ol, osc = O.top1(x, d, c, "l2")
    assert np.array_equal(gl, ol) and gs.tobytes() == osc.tobytes()
    assert rescanned <= n // 20, rescanned


@pytest.mark.parametrize("metric", ["ip", "l2"])
def test_screen_extreme_scales(dev, screen, metric):
    """Rows and centroids far from unit scale: rows whose bf16 halves fall in
    the subnormal range (1e-40 .. 1e-36) against centroids up to 1e34 (IP), a
    row near FLT_MAX whose bf16 half rounds to infinity, and, for L2, scales
    whose squared norms stay finite. Every row bit-equal to the oracle."""
    n, d, k = 1024, 768, 256
    base = _mix(n, d, 16, 0.2, True, 31)
    cb = _mix(k, d, 16, 0.2, True, 32)
    if metric == "ip":
        xs = np.array([1e-40, 1e-38, 1e-36, 1e-20, 1.0, 1e30], np.float64)
        cs = np.array([1e30, 1e34, 1e-38, 1.0], np.float64)
    else:
        xs = np.array([1e-30, 1e-18, 1.0, 1e15], np.float64)
        cs = np.array([1e-18, 1.0, 1e15], np.float64)
    x = (base * xs[np.arange(n) % len(xs)][:, None]).astype(np.float32)
    c = (cb * cs[np.arange(k) % len(cs)][:, None]).astype(np.float32)
    if metric == "ip":
        x[5, 0] = np.float32(3.4e38)  # bf16(3.4e38) = inf
    gl, gs = _gpu_top1(dev, x, c, metric)
    ol, osc = O.top1(x, d, c, metric)
    assert np.array_equal(gl, ol)
    assert gs.tobytes() == osc.tobytes()


@pytest.mark.parametrize("n,d,k", CONTRACT_SHAPES)
def test_scatter_ema_split(dev, n, d, k):
    """contract.rs:355-497 on the contract's shapes, bit-equal to the CPU order."""
    from emeans_amd import EmaStep, Mat, Select
    k = min(k, n)
    x = _mix(n, d, 7, 0.5, False, n + d)
    live = max(k - k // 5, 1)
    labels = (((np.arange(n, dtype=np.uint64) * 2654435761) % 2**32 >> 7) % live).astype(np.uint32)
    perm = ((np.arange(n, dtype=np.uint64) * 31 + 5) % n).astype(np.uint32)
    lo, hi = n // 5, n
    acc0 = ((np.arange(k * d) % 13) * 0.25).astype(np.float32)
    xb, idb, lb = dev.bind(x), dev.upload_u32(perm), dev.upload_u32(labels)
    sums = dev.upload_f32(np.full(k * d, 7.0, np.float32))
    counts = dev.upload_u32(np.full(k, 3, np.uint32))
    acc = dev.upload_f32(acc0)
    dev.scatter_add(Mat(xb, d), Select(idb, (lo, hi)), lb, k, sums, counts, acc)
    gs, gc, ga = dev.read_f32(sums), dev.read_u32(counts), dev.read_f32(acc)
    oacc = acc0.copy()
    os_, oc = O.scatter_add(x, d, labels, k, ids=perm, rows=(lo, hi), acc=oacc)
    assert np.array_equal(gc, oc)
    assert gs.tobytes() == os_.tobytes()
    assert ga.tobytes() == oacc.tobytes()
    pos0 = x.reshape(-1)[: k * d].copy()
    for alpha, u0 in [(0.37, 0.8), (1.0, 0.5), (0.9, 0.0)]:
        usage0 = (u0 + (np.arange(k) % 5) * 0.125).astype(np.float32)
        p, u = dev.upload_f32(pos0), dev.upload_f32(usage0)
        dev.ema_update(p, u, sums, counts, k, d, EmaStep.new(alpha))
        wp, wu = pos0.copy(), usage0.copy()
        O.ema_update(wp, wu, gs, gc, k, d, alpha)
        assert dev.read_f32(p).tobytes() == wp.tobytes(), alpha
        assert dev.read_f32(u).tobytes() == wu.tobytes(), alpha
    pos1 = pos0.copy()
    if k >= 4:
        pos1[d:2 * d] = 0.0
    usage1 = (1.0 + np.arange(k) * 0.37).astype(np.float32)
    plan = [(j, k - 1 - j) for j in range(k // 2) if j % 3 != 2 and j != k - 1 - j]
    p, u = dev.upload_f32(pos1), dev.upload_f32(usage1)
    dev.split(p, u, plan, d)
    wp, wu = pos1.copy(), usage1.copy()
    O.apply_splits(wp, wu, d, plan)
    assert dev.read_f32(p).tobytes() == wp.tobytes()
    assert dev.read_f32(u).tobytes() == wu.tobytes()


@pytest.mark.parametrize("d,k", [(200, 96), (768, 96), (64, 4096), (64, 9000)])
def test_scatter_skewed_clusters(dev, d, k):
    """Skewed cluster sizes (the Zipf case of training): clusters of several
    thousand rows, sizes at the edges of the per-column path (127..129, 256,
    257 rows), a single row and empty clusters; rows gathered by id; with acc.
    k = 96 and 4096 take the counting sort with chunk histograms; k = 9000
    the placement path for more clusters than the chunk histograms hold."""
    from emeans_amd import Mat, Select
    n = 20000
    g = np.random.default_rng(d)
    sizes = [5000, 2049, 257, 256, 129, 128, 127, 1, 0]
    rest = n - sum(sizes)
    labels = np.concatenate([np.full(s, j, np.uint32) for j, s in enumerate(sizes)] +
                            [g.integers(len(sizes), k, rest).astype(np.uint32)])
    g.shuffle(labels)
    nx = n + 37
    x = g.standard_normal((nx, d)).astype(np.float32)
    perm = g.permutation(nx)[:n].astype(np.uint32)
    acc0 = g.standard_normal(k * d).astype(np.float32)
    xb, idb, lb = dev.bind(x), dev.upload_u32(perm), dev.upload_u32(labels)
    sums, counts, acc = dev.zeros_f32(k * d), dev.zeros_u32(k), dev.upload_f32(acc0)
    for lo, hi in [(0, n), (3, n - 5)]:
        dev.scatter_add(Mat(xb, d), Select(idb, (lo, hi)), lb, k, sums, counts, acc)
        oacc = acc0.copy()
        os_, oc = O.scatter_add(x, d, labels, k, ids=perm, rows=(lo, hi), acc=oacc)
        assert np.array_equal(dev.read_u32(counts), oc), (lo, hi)
        assert dev.read_f32(sums).tobytes() == os_.tobytes(), (lo, hi)
        assert dev.read_f32(acc).tobytes() == oacc.tobytes(), (lo, hi)
        acc = dev.upload_f32(acc0)
    # Without ids (rows are positions) and without acc.
    dev.scatter_add(Mat(xb, d), Select(None, (0, n)), lb, k, sums, counts, None)
    os_, oc = O.scatter_add(x[:n], d, labels, k)
    assert np.array_equal(dev.read_u32(counts), oc)
    assert dev.read_f32(sums).tobytes() == os_.tobytes()


@pytest.mark.parametrize("k", [96, 4096])
def test_scatter_label_out_of_range_fails(dev, k):
    """A label >= k (an index out of the sums in core/cpu.rs:118-143, which
    panics) fails at the next wait, as every error the kernels record, with
    few clusters (k = 96) and many (k = 4096); the next call runs as usual."""
    from emeans_amd import Mat, Select
    n, d = 20000, 64
    g = np.random.default_rng(k)
    x = g.standard_normal((n, d)).astype(np.float32)
    labels = g.integers(0, k, n).astype(np.uint32)
    bad = labels.copy()
    bad[n // 2] = k + 3
    xb = dev.bind(x)
    sums, counts = dev.zeros_f32(k * d), dev.zeros_u32(k)
    with pytest.raises(Exception, match="label out of range"):
        dev.scatter_add(Mat(xb, d), Select(None, (0, n)), dev.upload_u32(bad), k, sums, counts, None)
        dev.read_u32(counts)
    dev.scatter_add(Mat(xb, d), Select(None, (0, n)), dev.upload_u32(labels), k, sums, counts, None)
    os_, oc = O.scatter_add(x, d, labels, k)
    assert np.array_equal(dev.read_u32(counts), oc)
    assert dev.read_f32(sums).tobytes() == os_.tobytes()


@pytest.mark.parametrize("d", [768, 20, 13, 33, 64, 96, 1000, 1024, 1056, 2500])
def test_norms_and_normalize(dev, d):
    """contract.rs:500-554: a zero row and a 1e30-scaled row (the max-prescale path)."""
    rows = 300
    m = _mix(rows, d, 7, 0.5, False, 1000 + d)
    m[0] = 0.0
    m[1] *= np.float32(1e30)
    mb = dev.upload_f32(m)
    nb = dev.zeros_f32(rows)
    dev.row_norms(mb, rows, d, nb)
    with np.errstate(over="ignore"):
        assert dev.read_f32(nb).tobytes() == O.row_norms(m, rows, d).tobytes()
    ub = dev.zeros_f32(rows * d)
    dev.normalize_rows(mb, rows, d, ub)
    assert dev.read_f32(ub).tobytes() == O.normalize_rows(m, rows, d).tobytes()


def test_split_zero_row_nudge_and_sequential_plan(dev):
    """The child-nudge path on an all-zero donor, and a plan that reuses a centroid."""
    k, d = 8, 5
    pos = np.arange(k * d, dtype=np.float32) * 0.5
    pos[:d] = 0.0
    usage = np.arange(1, k + 1, dtype=np.float32)
    for plan in ([(0, 7), (1, 6)], [(1, 2), (2, 3), (3, 1)]):
        p, u = dev.upload_f32(pos), dev.upload_f32(usage)
        dev.split(p, u, plan, d)
        wp, wu = pos.copy(), usage.copy()
        O.apply_splits(wp, wu, d, plan)
        assert dev.read_f32(p).tobytes() == wp.tobytes(), plan
        assert dev.read_f32(u).tobytes() == wu.tobytes(), plan


@pytest.mark.parametrize("m,n,d,kk", [(300, 300, 768, 16), (200, 900, 20, 5), (130, 7, 33, 10)])
def test_topk_contract_shapes(dev, screen, m, n, d, kk):
    """contract.rs:103-110 shapes: ids and sims bit-equal to the oracle (fma-chain dots)."""
    data = _mix(n, d, 9, 0.3, True, m + n)
    q = _mix(m, d, 9, 0.3, True, m * 7 + n)
    gi, gs = dev.topk(q, data, d, kk, False)
    oi, osims = O.knn(q, data, d, kk, False)
    assert np.array_equal(gi, oi) and gs.tobytes() == osims.tobytes()
    if m == n:
        gi, gs = dev.topk(data, data, d, kk, True)
        oi, osims = O.knn(data, data, d, kk, True)
        assert np.array_equal(gi, oi) and gs.tobytes() == osims.tobytes()


def test_topk_production_duplicates(dev, screen):
    """contract.rs:147-159: 64 queries vs 16,384 rows with 512 duplicated rows, k = 16."""
    n, d = 16384, 768
    data = _mix(n, d, 9, 0.3, True, 77)
    for j in range(8192, 8192 + 512):
        data[j] = data[j - 8000]
    q = np.stack([data[192 + i] if i % 2 == 0 else data[(i * 61) % n] for i in range(64)])
    gi, gs = dev.topk(q, data, d, 16, False)
    oi, osims = O.knn(q, data, d, 16, False)
    assert np.array_equal(gi, oi) and gs.tobytes() == osims.tobytes()


@pytest.mark.parametrize("m,n,d,kk,self_", [
    (256, 20_000, 384, 10, False),   # two query tiles: eight parts of ten data tiles
    (1000, 3000, 100, 16, False),    # a partial last slab (100 = 3 x 32 + 4)
    (777, 5000, 99, 7, False),       # d % 4 != 0 (the split's scalar loads)
    (3000, 3000, 64, 16, True),      # exclude_self
    (2048, 2048, 768, 1, True),      # k = 1
])
def test_topk_split_screen(dev, screen, m, n, d, kk, self_):
    """Calls of at least 256 queries against at least 512 rows take the kNN
    screen over operands split once (k_screen4kn): ids and sims bit-equal to
    the oracle, with exact duplicates among the data rows."""
    data = _mix(n, d, 12, 0.25, True, m + n + d)
    data[n // 2:n // 2 + 64] = data[:64]  # exact duplicates: equal scores, lower id first
    q = data[:m].copy() if self_ else _mix(m, d, 12, 0.25, True, 3 * m + d)
    if not self_:
        q[:32] = data[n // 2:n // 2 + 32]
    gi, gs = dev.topk(q if not self_ else data, data, d, kk, self_)
    oi, osims = O.knn(q if not self_ else data, data, d, kk, self_)
    bad = np.nonzero(gi != oi)[0]
    assert bad.size == 0, f"{bad.size} ids differ, first {bad[:4]}"
    assert gs.tobytes() == osims.tobytes()


def test_backend_is_available_by_name():
    """available_backends lists "hip" on a gfx950 machine; make_assigner builds
    it from either name (backend.rs:84-114)."""
    from emeans_amd import Backend, available_backends, make_assigner
    assert available_backends() == ["hip"]
    d = make_assigner(Backend.from_str("hip-gfx950"))
    assert d.name() == "hip-gfx950"
    d.close()


@pytest.mark.parametrize("metric", ["ip", "l2"])
def test_screen_tiny_rows_finite_bound(dev, screen, metric):
    """Rows whose squared norm underflows f32 (scales 1e-40 .. 1e-20, elements
    in the f32 and bf16 subnormal ranges) against centroids up to 5e17, the
    largest scale whose |c|^2 is finite at d = 768, so the screen's bound stays
    finite and the check decides these rows: bit-equal to the oracle in both
    screen arithmetics."""
    n, d, k = 2048, 768, 256
    base = _mix(n, d, 16, 0.2, True, 41)
    cb = _mix(k, d, 16, 0.2, True, 42)
    if metric == "ip":
        xs = np.array([1e-40, 1e-38, 1e-36, 1e-30, 1e-20, 1.0], np.float64)
        cs = np.array([5e17, 1e3, 1.0], np.float64)
    else:
        xs = np.array([1e-40, 1e-38, 1e-30, 1e-20, 1.0], np.float64)
        cs = np.array([1e-18, 1.0, 1e12], np.float64)
    x = (base * xs[np.arange(n) % len(xs)][:, None]).astype(np.float32)
    c = (cb * cs[np.arange(k) % len(cs)][:, None]).astype(np.float32)
    gl, gs = _gpu_top1(dev, x, c, metric)
    ol, osc = O.top1(x, d, c, metric)
    bad = np.nonzero(gl != ol)[0]
    assert bad.size == 0, f"{bad.size} labels differ, rows {bad[:8]} (scales {xs[bad[:8] % len(xs)]})"
    assert gs.tobytes() == osc.tobytes()
