"""A device that answers the calls the automatic-k sweeps and the hierarchy
make of a HipDevice (bind, buffers, train_dev, assign_dev, kmeans_pp,
internal_scores, assign, dots, topk) with the oracle, so that
emeans_amd.autocluster.auto_cluster and Hierarchy.add run end to end over the
oracle, the way the reference runs auto_cluster over whatever Backend it is
handed (emeans-cluster/src/auto.rs:1001). Buffers are numpy arrays; epoch
times are zero (wall-clock time is not part of a trajectory).

Test infrastructure only: the product never imports this file."""

import numpy as np

from emeans_amd import EpochStats
from oracle import oracle as O


class OracleDevice:
    def __init__(self, name="hip-gfx950"):
        self._name = name
        self.fits = 0

    def name(self):
        return self._name

    # -- buffers: host arrays standing in for device memory
    def bind(self, x):
        return np.ascontiguousarray(x, np.float32).reshape(-1).copy()

    def upload_f32(self, v):
        return np.ascontiguousarray(v, np.float32).reshape(-1).copy()

    def upload_u32(self, v):
        return np.ascontiguousarray(v, np.uint32).reshape(-1).copy()

    def zeros_f32(self, n):
        return np.zeros(n, np.float32)

    def zeros_u32(self, n):
        return np.zeros(n, np.uint32)

    def read_f32(self, b, rng=None):
        lo, hi = rng if rng is not None else (0, len(b))
        return np.asarray(b[lo:hi], np.float32).copy()

    def read_u32(self, b, rng=None):
        lo, hi = rng if rng is not None else (0, len(b))
        return np.asarray(b[lo:hi], np.uint32).copy()

    def sync(self):
        pass

    # -- the device work
    def train_dev(self, x, n, config, centroids_out=None, init=None, state=None):
        d, k = config.d, config.k
        pos, usage = state if state is not None else (None, None)
        o = O.train(np.asarray(x[:n * d]).reshape(n, d), d, k, nepochs=config.nepochs,
                    seed=config.seed, spherical=config.spherical,
                    unused_threshold=config.unused_threshold,
                    init=None if init is None else np.asarray(init, np.float32),
                    positions=pos, usage=usage)
        self.fits += 1
        if centroids_out is not None:
            centroids_out[:k * d] = o["centroids"]
        info = {"stats": [EpochStats(ob, 0.0, im, int(ns))
                          for ob, im, ns in zip(o["obj"], o["imbalance"], o["nsplit"])],
                "n_splits": int(o["n_splits"]), "batch_size": int(o["batch_size"]),
                "alpha0": o["alpha0"], "total_steps": int(o["total_steps"]),
                "fallback_rows": 0, "positions": o["positions"], "usage": o["usage"],
                "labels": o["labels"]}
        return o["centroids"], info

    def assign(self, x, d, centroids, metric, chunk=65536):
        return O.assign(np.asarray(x, np.float32), d, np.asarray(centroids, np.float32), metric)

    def assign_dev(self, x, n, d, centroids, k, metric, labels, scores, chunk=65536):
        lab, sco = O.assign(np.asarray(x[:n * d]), d, np.asarray(centroids[:k * d]), metric)
        labels[:n] = lab
        scores[:n] = sco

    def kmeans_pp(self, x, n, d, kmax, seed):
        return O.kmeans_pp(np.asarray(x[:n * d]), d, kmax, seed)

    def internal_scores(self, x, n, d, labels, k):
        return O.internal_scores(np.asarray(x[:n * d]), d, np.asarray(labels[:n], np.uint32), k)

    def dots(self, a, b):
        return O.dots(a, b)

    def topk(self, queries, data, d, kk, exclude_self):
        return O.knn(np.asarray(queries, np.float32), np.asarray(data, np.float32), d, kk,
                     exclude_self)
