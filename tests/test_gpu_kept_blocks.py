"""Freed buffers' device blocks are kept per device for the next buffer of the
same size (emh_free: blocks of up to 64 MB, hipFree waiting for the whole
device otherwise). A buffer that takes a kept block holds what it was made
with (zeros or the upload), and when another context had work queued on the
freed block, the new owner's writes wait for that work."""

import numpy as np
import pytest

from emeans_amd import HipDevice, Mat, Select
from emeans_amd._lib import lib

pytestmark = pytest.mark.gpu


def _unit(rng, n, d):
    x = rng.standard_normal((n, d)).astype(np.float32)
    return x / np.linalg.norm(x, axis=1, keepdims=True).astype(np.float32)


def test_reused_blocks_hold_their_new_contents():
    a, b = HipDevice(), HipDevice()
    try:
        rng = np.random.default_rng(0)
        n = 300_000
        for _ in range(3):
            for first, second in ((a, b), (b, a)):
                v = rng.standard_normal(n).astype(np.float32)
                buf = first.upload_f32(v)
                assert np.array_equal(first.read_f32(buf), v)
                del buf  # freed on `first`: the block is kept
                z = second.zeros_f32(n)  # the same size: the kept block
                assert not second.read_f32(z).any()
                del z
                w = rng.standard_normal(n).astype(np.float32)
                u = first.upload_f32(w)
                assert np.array_equal(first.read_f32(u), w)
                del u
                iz = second.zeros_u32(n)
                assert not second.read_u32(iz).any()
    finally:
        a.close()
        b.close()


def test_a_kept_block_waits_for_the_other_contexts_work():
    """Context a queues top-1 calls over rows in buffer xq (no wait); context b
    frees xq and takes its block for a zero fill. a's results must be those of
    the rows, not of zeros."""
    a, b = HipDevice(), HipDevice()
    try:
        rng = np.random.default_rng(1)
        n, d, k = 20_000, 768, 1024  # 61.4 MB of rows: a kept size
        x = _unit(rng, n, d)
        c = _unit(rng, k, d)
        xa = a.bind(x)
        cb = a.upload_f32(c)
        lab, sco = a.zeros_u32(n), a.zeros_f32(n)
        a.top1(Mat(xa, d), Select(None, (0, n)), cb, None, k, "ip", lab, sco)
        ref_l, ref_s = a.read_u32(lab), a.read_f32(sco)
        for _ in range(3):
            xq = a.bind(x)
            outs = []
            for _ in range(4):  # queued on a's stream, not waited for
                l2, s2 = a.zeros_u32(n), a.zeros_f32(n)
                a.top1(Mat(xq, d), Select(None, (0, n)), cb, None, k, "ip", l2, s2)
                outs.append((l2, s2))
            assert lib().emh_free(b._ctx, xq.h) == 0  # freed through the other context
            xq.h = None
            z = b.zeros_f32(n * d)  # takes xq's block
            assert not b.read_f32(z, (0, 1024)).any()
            for l2, s2 in outs:
                assert np.array_equal(a.read_u32(l2), ref_l)
                assert a.read_f32(s2).tobytes() == ref_s.tobytes()
            del z
    finally:
        a.close()
        b.close()
