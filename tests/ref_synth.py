"""The reference's test-data generators, restated for the known-answer tests
of its dedup (crates/emeans-cluster/tests/dedup.rs).

crates/emeans-cluster/src/synth.rs draws everything from one numpy-legacy
MT19937 stream (rng.rs): Box-Muller normals in f64 with libm's ln, sqrt and
cos (Python's math module is the same glibc libm, so each draw has the same
bits), cast to f32, and RandomState::permutation (numpy's legacy shuffle).
Row normalisation is faiss normalize_into (model.rs:954-967): divide by the
largest magnitude, then by the square root of the sequential f32 sum of
squares.
"""

import math

import numpy as np


def normalize_rows(x, d):
    """model.rs:954-967, in place on an (n, d) f32 array."""
    x = x.reshape(-1, d)
    for r in x:
        mx = np.float32(np.max(np.abs(r))) if r.size else np.float32(0)
        if mx > 0:
            r /= mx
        q = np.cumsum(r * r, dtype=np.float32)[-1]  # sequential f32 sum
        nr = np.sqrt(np.float32(q))
        if nr > 0:
            r /= nr
    return x


class Normal:
    """synth.rs:69-100: normal draws from MT19937 (Box-Muller)."""

    def __init__(self, seed):
        self.rs = np.random.RandomState(seed & 0xFFFFFFFF)

    def sample(self):
        u1 = max(self.rs.random_sample(), 1e-300)
        u2 = self.rs.random_sample()
        return np.float32(math.sqrt(-2.0 * math.log(u1)) * math.cos(2.0 * math.pi * u2))

    def samples(self, m):
        u = self.rs.random_sample(2 * m)
        return np.array([math.sqrt(-2.0 * math.log(max(u[2 * i], 1e-300))) *
                         math.cos(2.0 * math.pi * u[2 * i + 1]) for i in range(m)],
                        np.float64).astype(np.float32)

    def uniform(self):
        return self.rs.random_sample()

    def direction(self, d):
        """d normal draws times 1 / sqrt(d) (both f32)."""
        s = np.float32(1.0) / np.sqrt(np.float32(d))
        return self.samples(d) * s

    def permutation(self, n):
        return self.rs.permutation(n).astype(np.uint32)


def unit(v, d):
    v = np.array(v, np.float32)
    normalize_rows(v.reshape(-1, d), d)
    return v


def add_scaled(a, b, s):
    """a + s b elementwise in f32 (two roundings: Rust does not fuse)."""
    return (np.asarray(a, np.float32) + np.float32(s) * np.asarray(b, np.float32)).astype(np.float32)


def random_unit(n, d, seed):
    """tests/dedup.rs:17-22."""
    r = Normal(seed)
    x = r.samples(n * d).reshape(n, d)
    normalize_rows(x, d)
    return x


def _allocate(total, w, mn):
    """synth.rs:109-124."""
    s = 0.0
    for v in w:
        s += v
    free = max(total - mn * len(w), 0)
    out = [mn + int(math.floor(free * v / s)) for v in w]
    left = max(total - sum(out), 0)
    i = 0
    while left > 0:
        out[i % len(w)] += 1
        left -= 1
        i += 1
    return out


def nested(n=16_000, d=768, n_broad=8, sub_range=(3, 12), noise_frac=0.03, global_weight=0.82,
           sub_spread=0.6, point_spread=0.577, size_sigma=0.7, min_sub=15, seed=7):
    """synth.rs:127-200 (NestedSpec defaults): returns (x, broad, sub)."""
    rng = Normal(seed)
    g = unit(rng.direction(d), d)
    n_noise = int(math.floor(n * noise_frac + 0.5))  # f64::round, half away from zero
    n_groups = n - n_noise

    def lognormal(s):
        return math.exp(s * float(rng.sample()))

    bw = [lognormal(size_sigma) for _ in range(n_broad)]
    subs_per_broad, sub_w = [], []
    for _ in range(n_broad):
        lo, hi = sub_range
        m = min(lo + int(math.floor(rng.uniform() * (hi - lo + 1))), hi)
        subs_per_broad.append(m)
        sub_w.append([lognormal(size_sigma) for _ in range(m)])
    flat_w = []
    for b, ws in zip(bw, sub_w):
        s = 0.0
        for w in ws:
            s += w
        flat_w += [b * w / s for w in ws]
    sizes = _allocate(n_groups, flat_w, min_sub)
    rows = []
    sid = 0
    for b, m in enumerate(subs_per_broad):
        bc = unit(add_scaled(rng.direction(d), g, global_weight), d)
        for _ in range(m):
            sc = unit(add_scaled(bc, rng.direction(d), sub_spread), d)
            for _ in range(sizes[sid]):
                rows.append((unit(add_scaled(sc, rng.direction(d), point_spread), d), b, sid))
            sid += 1
    for _ in range(n_noise):
        c = unit(add_scaled(rng.direction(d), g, global_weight), d)
        rows.append((unit(add_scaled(c, rng.direction(d), point_spread), d), -1, -1))
    perm = rng.permutation(len(rows))
    x = np.stack([rows[i][0] for i in perm]).astype(np.float32)
    broad = np.array([rows[i][1] for i in perm], np.int32)
    sub = np.array([rows[i][2] for i in perm], np.int32)
    return x, broad, sub


def with_bursts(x, d, n_bursts, size_range, eps, seed):
    """synth.rs:215-248: x plus n_bursts bursts of perturbed copies one second
    apart; returns (rows, truth, created_unix)."""
    x = np.asarray(x, np.float32).reshape(-1, d)
    n = x.shape[0]
    rng = Normal(seed)
    out = [r for r in x]
    truth = list(range(n))
    created = [rng.uniform() * 5.0 * 365.0 * 86400.0 for _ in range(n)]
    picks = rng.permutation(n)
    for base in picks[:n_bursts]:
        b = int(base)
        lo, hi = size_range
        m = min(lo + int(math.floor(rng.uniform() * (hi - lo + 1))), hi)
        for t in range(m):
            out.append(unit(add_scaled(x[b], rng.direction(d), eps), d))
            truth.append(b)
            created.append(created[b] + 1.0 + float(t))
    return np.stack(out).astype(np.float32), np.array(truth, np.uint32), np.array(created)


def new_group(d, rows, seed):
    """tests/hierarchy.rs:489-503: rows of one tight group around a random
    direction (center + 0.5 z, renormalised)."""
    rng = Normal(seed)
    center = normalize_rows(rng.direction(d).reshape(1, d).copy(), d)[0]
    out = []
    for _ in range(rows):
        v = (center + np.float32(0.5) * rng.direction(d)).astype(np.float32)
        out.append(normalize_rows(v.reshape(1, d), d)[0])
    return np.stack(out).astype(np.float32)


def scattered_rows(d, rows, seed):
    """tests/hierarchy.rs:587-592: unrelated random unit rows."""
    rng = Normal(seed)
    return np.stack([normalize_rows(rng.direction(d).reshape(1, d).copy(), d)[0]
                     for _ in range(rows)]).astype(np.float32)
