"""emh_top1_noalloc (top-1 with its scratch in a fixed device block, no
allocation) against emh_top1 through the C ABI: labels and scores bit-equal,
on two calls in a row where the second has fewer rows (the block keeps the
first call's contents), on each top-1 path (the large-tile bf16 screen with
queued near-tie rows, the 128 x 128 screen with d % 4 != 0 and the exact scan
alone); and a call whose scratch exceeds the block is refused before anything
runs."""

import ctypes as C

import numpy as np
import pytest

from emeans_amd import _lib
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    from emeans_amd import HipDevice
    d = HipDevice()
    d.set_exact_below(0)  # The screen's lists live in the fixed block: screen every call
    yield d
    d.close()


def _call(dev, fn, x, d, ids, lo, hi, cb, cn, k, metric):
    n_out = len(ids) if ids is not None else x.shape[0]
    lab = dev.upload_u32(np.full(n_out, 0xFFFFFFFF, np.uint32))
    sco = dev.upload_f32(np.full(n_out, np.nan, np.float32))
    xb = dev.bind(x)
    idb = dev.upload_u32(ids) if ids is not None else None
    rc = fn(dev._ctx, xb.h, d, idb.h if idb else None, lo, hi, cb.h, cn.h if cn else None, k,
            _lib.EMH_L2 if metric == "l2" else _lib.EMH_IP, lab.h, sco.h)
    _lib.check(rc)
    return dev.read_u32(lab), dev.read_f32(sco)


CASES = [
    # (n first call, n second call, d, k, metric): large-tile screen, 128 x 128
    # screen (d % 4 != 0), 128 x 128 screen at small k, exact scan alone (d < 32)
    (20_000, 3_000, 768, 1024, "l2"),
    (5_000, 1_000, 99, 300, "ip"),
    (4_000, 500, 64, 32, "l2"),
    (4_000, 500, 24, 40, "ip"),
]


@pytest.mark.parametrize("n1,n2,d,k,metric", CASES)
def test_noalloc_equals_top1_on_two_calls(dev, n1, n2, d, k, metric):
    lib = _lib.lib()
    x = O.contract_mixture(n1, d, 60, 0.3, metric == "ip", 29).reshape(n1, d)
    c = x[(np.arange(k) * 13) % n1].copy()
    c[k // 2:k // 2 + 16] = c[:16]  # exact duplicates in other tiles: queued rows
    cb = dev.upload_f32(c)
    cn = None
    if metric == "l2":
        cn = dev.zeros_f32(k)
        dev.row_norms(cb, k, d, cn)
    for n in (n1, n2):  # the second call has fewer rows
        xs = x[:n]
        ids = ((np.arange(n, dtype=np.uint64) * 7919 + 5) % n).astype(np.uint32)
        lo, hi = n // 10, n - n // 8
        ga, gs = _call(dev, lib.emh_top1_noalloc, xs, d, ids, lo, hi, cb, cn, k, metric)
        wa, ws = _call(dev, lib.emh_top1, xs, d, ids, lo, hi, cb, cn, k, metric)
        assert np.array_equal(ga, wa), f"n = {n}: labels differ from emh_top1"
        assert ga[lo:hi].max() < k and np.all(ga[:lo] == 0xFFFFFFFF) and np.all(ga[hi:] == 0xFFFFFFFF)
        assert gs.tobytes() == ws.tobytes(), f"n = {n}: scores differ from emh_top1"
        ol = np.full(n, 0xFFFFFFFF, np.uint32)
        osc = np.full(n, np.nan, np.float32)
        O.top1(xs, d, c, metric, ids=ids, rows=(lo, hi), labels=ol, scores=osc)
        assert np.array_equal(ga, ol) and gs.tobytes() == osc.tobytes(), f"n = {n}: oracle"


def test_noalloc_refuses_a_call_beyond_its_block(dev):
    """2,000,000 selected rows against 16,384 centroids at d = 4 (no screen):
    the exact scan's partials alone would take 4 GB."""
    lib = _lib.lib()
    d, k, n = 4, 16_384, 2_000_000
    x = np.ones((64, d), np.float32)
    xb, cb = dev.bind(x), dev.upload_f32(np.ones((k, d), np.float32))
    ids = dev.zeros_u32(n)
    lab, sco = dev.zeros_u32(n), dev.zeros_f32(n)
    rc = lib.emh_top1_noalloc(dev._ctx, xb.h, d, ids.h, 0, n, cb.h, None, k, _lib.EMH_IP, lab.h,
                              sco.h)
    assert rc == _lib.EMH_INVALID
    assert b"scratch" in lib.emh_last_error()
    assert np.all(dev.read_u32(lab, (0, 16)) == 0), "nothing ran"


def test_noalloc_two_contexts_back_to_back(dev):
    """Two contexts (two streams) call emh_top1_noalloc one right after the
    other with no wait between them: the block is the GPU's, so the second
    call's stream must wait for the first call's work. Both results equal
    emh_top1's."""
    from emeans_amd import HipDevice
    lib = _lib.lib()
    d, k, metric = 768, 1024, "l2"
    n1, n2 = 30_000, 7_000
    x = O.contract_mixture(n1, d, 60, 0.3, False, 31).reshape(n1, d)
    c = x[(np.arange(k) * 11) % n1].copy()
    c[k // 2:k // 2 + 16] = c[:16]
    other = HipDevice()
    other.set_exact_below(0)
    try:
        calls = []
        for dv, n in ((dev, n1), (other, n2)):
            cb = dv.upload_f32(c)
            cn = dv.zeros_f32(k)
            dv.row_norms(cb, k, d, cn)
            xb = dv.bind(x[:n])
            lab = dv.upload_u32(np.full(n, 0xFFFFFFFF, np.uint32))
            sco = dv.upload_f32(np.full(n, np.nan, np.float32))
            dv.sync()
            calls.append((dv, n, xb, cb, cn, lab, sco))
        for dv, n, xb, cb, cn, lab, sco in calls:  # queued back to back, no wait between
            _lib.check(lib.emh_top1_noalloc(dv._ctx, xb.h, d, None, 0, n, cb.h, cn.h, k,
                                            _lib.EMH_L2, lab.h, sco.h))
        for dv, n, xb, cb, cn, lab, sco in calls:
            got_l, got_s = dv.read_u32(lab), dv.read_f32(sco)
            wl, ws = dv.zeros_u32(n), dv.zeros_f32(n)
            _lib.check(lib.emh_top1(dv._ctx, xb.h, d, None, 0, n, cb.h, cn.h, k, _lib.EMH_L2,
                                    wl.h, ws.h))
            assert np.array_equal(got_l, dv.read_u32(wl)), f"n = {n}: labels differ"
            assert got_s.tobytes() == dv.read_f32(ws).tobytes(), f"n = {n}: scores differ"
    finally:
        other.close()
