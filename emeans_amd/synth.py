"""Seeded synthetic data sets of the benchmark workloads (numpy PCG64).

Each generator returns float32 row-major data; the same seed gives the same
bytes on every machine, so the GPU run and the CPU baseline read identical
inputs. (The reference's own generator is crates/emeans-cluster/src/synth.rs;
these follow the workload definitions instead.)
"""

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np


def _unit(x):
    n = np.sqrt(np.einsum("ij,ij->i", x, x, dtype=np.float64)).astype(np.float32)
    n[n == 0] = 1.0
    x /= n[:, None]
    return x


def blobs_spherical(n=20_000, d=64, k=32, sigma=0.1, seed=7):
    """Unit rows from k Gaussian blobs: centers ~N(0, I) normalised, equal blob
    sizes, row noise sigma, rows renormalised; rows shuffled."""
    g = np.random.default_rng(seed)
    centers = _unit(g.standard_normal((k, d), dtype=np.float32))
    lab = np.repeat(np.arange(k), -(-n // k))[:n]
    lab = lab[g.permutation(n)]
    x = centers[lab] + np.float32(sigma) * g.standard_normal((n, d), dtype=np.float32)
    return _unit(x), lab


def zipf_weights(m, s):
    w = 1.0 / np.arange(1, m + 1, dtype=np.float64) ** s
    return w / w.sum()


def gmm_zipf(n=200_000, d=768, comps=1024, s=1.1, seed=0, chunk=50_000):
    """Gaussian mixture: means ~N(0, I), per-component diagonal std ~U(0.2, 1.0),
    Zipf(s) component weights."""
    g = np.random.default_rng(seed)
    means = g.standard_normal((comps, d), dtype=np.float32)
    std = g.uniform(0.2, 1.0, size=(comps, d)).astype(np.float32)
    lab = g.choice(comps, size=n, p=zipf_weights(comps, s))
    x = np.empty((n, d), np.float32)
    for a in range(0, n, chunk):
        b = min(a + chunk, n)
        z = g.standard_normal((b - a, d), dtype=np.float32)
        x[a:b] = means[lab[a:b]] + std[lab[a:b]] * z
    return x, lab


def unit_gaussian(n, d, seed, chunk=65_536, threads=None):
    """Rows i.i.d. ~N(0, I) normalised. Chunk i of `chunk` rows comes from its
    own PCG64 stream (SeedSequence(seed).spawn), so the bytes do not depend on
    how many threads fill the chunks."""
    x = np.empty((n, d), np.float32)
    starts = list(range(0, n, chunk))
    seqs = np.random.SeedSequence(seed).spawn(len(starts))

    def fill(i):
        a = starts[i]
        b = min(a + chunk, n)
        g = np.random.Generator(np.random.PCG64(seqs[i]))
        x[a:b] = _unit(g.standard_normal((b - a, d), dtype=np.float32))

    nt = threads or min(16, os.cpu_count() or 1)
    with ThreadPoolExecutor(max_workers=nt) as ex:
        list(ex.map(fill, range(len(starts))))
    return x


def assign_at_scale(n=2_000_000, d=1024, k=16_384, seed=1):
    """Queries and centroids, both unit rows ~N(0, I) normalised."""
    g = np.random.default_rng(seed)
    c = _unit(g.standard_normal((k, d), dtype=np.float32))
    q = unit_gaussian(n, d, int(g.integers(1 << 31)))
    return q, c


def knn_near_duplicates(n=500_000, d=384, frac=0.05, noise=0.01, seed=2):
    """Unit rows ~N(0, I); a fraction replaced by a random base row plus
    N(0, noise^2) noise, renormalised."""
    g = np.random.default_rng(seed)
    x = unit_gaussian(n, d, int(g.integers(1 << 31)))
    m = int(round(frac * n))
    dst = g.choice(n, size=m, replace=False)
    base = np.setdiff1d(np.arange(n), dst)  # copy only rows that stay base rows
    src = base[g.integers(0, base.size, size=m)]
    x[dst] = _unit(x[src] + np.float32(noise) * g.standard_normal((m, d), dtype=np.float32))
    return x, dst, src


def nested(n=1_000_000, d=768, top=64, sub=16, s=1.3, sub_sigma=0.3, row_sigma=0.05, seed=3,
           chunk=65_536, threads=None):
    """Two-level mixture: top centers (Zipf(s) weights), sub-centers = center +
    N(0, sub_sigma^2) renormalised, rows = sub-center + N(0, row_sigma^2)
    renormalised. Returns the rows and each row's sub-center (top * sub + j).
    Row chunks draw their noise from their own PCG64 streams."""
    g = np.random.default_rng(seed)
    centers = _unit(g.standard_normal((top, d), dtype=np.float32))
    subs = centers[:, None, :] + np.float32(sub_sigma) * g.standard_normal((top, sub, d),
                                                                            dtype=np.float32)
    subs = _unit(subs.reshape(top * sub, d))
    t = g.choice(top, size=n, p=zipf_weights(top, s))
    lab = t * sub + g.integers(0, sub, size=n)
    x = np.empty((n, d), np.float32)
    starts = list(range(0, n, chunk))
    seqs = np.random.SeedSequence(int(g.integers(1 << 31))).spawn(len(starts))

    def fill(i):
        a = starts[i]
        b = min(a + chunk, n)
        gc = np.random.Generator(np.random.PCG64(seqs[i]))
        x[a:b] = _unit(subs[lab[a:b]] + np.float32(row_sigma) *
                       gc.standard_normal((b - a, d), dtype=np.float32))

    with ThreadPoolExecutor(max_workers=threads or min(16, os.cpu_count() or 1)) as ex:
        list(ex.map(fill, range(len(starts))))
    return x, lab
