"""emeans on AMD Instinct MI355X (gfx950): the reference's Device / Assigner /
Emeans / knn / dedup interfaces over hand-written HIP kernels.

Mirrors, name for name, the Rust reference (samhvw8/emeans):
  HipDevice            core::Device + Assigner   (crates/emeans-core/src/core/mod.rs:71-178,
                                                   assign.rs:71-117)
  EmaStep, Mat, Select core::EmaStep / Mat / Select (core/mod.rs:27-56, 180-197)
  Config, Emeans       model.rs:24-76, 165-919 (train, assign, iteration_stats, ...)
  knn_self, knn        emeans-cluster/src/knn.rs:17-64
  dedup                emeans-cluster/src/dedup.rs:163-358
  make_assigner        emeans-cluster/src/backend.rs:170-178 for the backend name "hip"

Every computation runs on the GPU through libemeans_hip.so; nothing here
falls back to a CPU path.
"""

import ctypes as C
from dataclasses import dataclass, field
from typing import List, Optional, Tuple

import numpy as np

from . import model_file
from ._lib import (EMH_IP, EMH_L2, EMH_PROF_EMA, EMH_PROF_SCATTER, EMH_PROF_SCREEN,
                   Config as _CConfig, DedupConfig as _CDedupConfig,
                   DedupInput as _CDedupInput, DedupResult as _CDedupResult, EmeansHipError,
                   EmeansHipInvalid, EpochStats as _CEpoch, TrainInit as _CTrainInit,
                   TrainOut as _CTrainOut, check, lib)

__all__ = [
    "HipDevice", "DevBuf", "EmaStep", "Mat", "Select", "Config", "Emeans", "Trained",
    "Assignment", "EpochStats", "Neighbors", "DedupConfig", "DedupInput", "DedupResult",
    "knn_self", "knn", "dedup", "dedup_with_neighbors", "make_assigner", "available_backends",
    "Backend", "BACKEND_NAME", "EmeansHipError", "EmeansHipInvalid",
    "GPU_KMAX", "KLONG", "NONE",
]

BACKEND_NAME = "hip"
GPU_KMAX = 16          # emeans-core/src/knn.rs:16: the screened top-k's largest k
KLONG = 4096           # the exact top-k's largest k beyond GPU_KMAX (no CPU fallback)
NONE = 0xFFFFFFFF      # emeans-core/src/knn.rs:19


def _metric(m) -> int:
    if m in ("l2", "L2", EMH_L2):
        return EMH_L2
    if m in ("ip", "inner_product", "InnerProduct", EMH_IP):
        return EMH_IP
    raise ValueError(f"unknown metric {m!r}")


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u32(a):
    return np.ascontiguousarray(a, dtype=np.uint32)


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class DevBuf:
    """A backend-owned device buffer (Device::F / Device::U)."""

    __slots__ = ("_dev", "h", "kind")

    def __init__(self, dev, h, kind):
        self._dev, self.h, self.kind = dev, h, kind

    def __len__(self):
        return lib().emh_buf_len(self.h)

    @property
    def ptr(self):
        return lib().emh_buf_ptr(self.h)

    def __del__(self):
        if getattr(self, "h", None) and self._dev is not None and self._dev._ctx:
            lib().emh_free(self._dev._ctx, self.h)
            self.h = None


@dataclass
class EmaStep:
    """Scalars of one EMA step (core/mod.rs:182-197)."""
    alpha: float
    decay: float
    replace: bool

    @staticmethod
    def new(alpha: float) -> "EmaStep":
        return EmaStep(float(np.float32(alpha)), float(np.float32(1.0 - alpha)), alpha == 1.0)


@dataclass
class Mat:
    """An n x d matrix on the device (core/mod.rs:30-34)."""
    dev: DevBuf
    d: int


@dataclass
class Select:
    """Rows `rows` of a selection: x[ids[r]] when ids is given, else x[r] (core/mod.rs:44-47)."""
    ids: Optional[DevBuf]
    rows: Tuple[int, int]


class HipDevice:
    """The gfx950 backend: core::Device + Assigner over the C ABI."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        check(lib().emh_create(device, C.byref(h)))
        self._ctx = h
        self._device = device
        self._more: List["HipDevice"] = []

    def contexts(self, n: int) -> List["HipDevice"]:
        """This context and n - 1 more on the same GPU (made once, closed with
        this one): independent work, one thread per context, runs at once on
        their streams. Buffers of any of them serve the others, but each
        context orders only its own stream: a buffer another context writes is
        ready once that context's read (or sync) has returned."""
        while len(self._more) < n - 1:
            self._more.append(HipDevice(self._device))
        return [self] + self._more[:max(n - 1, 0)]

    def close(self):
        for m in getattr(self, "_more", []):
            m.close()
        self._more = []
        if self._ctx:
            lib().emh_destroy(self._ctx)
            self._ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- Device::name, bind, upload, zeros, write, read, flush
    def name(self) -> str:
        return lib().emh_name(self._ctx).decode()

    def _new(self, fn, *args, kind):
        h = C.c_void_p()
        check(fn(self._ctx, *args, C.byref(h)))
        return DevBuf(self, h, kind)

    def bind(self, x) -> DevBuf:
        x = _f32(x)
        return self._new(lib().emh_bind, _p(x), x.size, kind=0)

    def upload_f32(self, v) -> DevBuf:
        v = _f32(v)
        return self._new(lib().emh_upload_f32, _p(v), v.size, kind=0)

    def upload_u32(self, v) -> DevBuf:
        v = _u32(v)
        return self._new(lib().emh_upload_u32, _p(v), v.size, kind=1)

    def zeros_f32(self, n: int) -> DevBuf:
        return self._new(lib().emh_zeros_f32, n, kind=0)

    def zeros_u32(self, n: int) -> DevBuf:
        return self._new(lib().emh_zeros_u32, n, kind=1)

    def write_f32(self, b: DevBuf, offset: int, v):
        v = _f32(v)
        check(lib().emh_write_f32(self._ctx, b.h, offset, _p(v), v.size))

    def write_u32(self, b: DevBuf, offset: int, v):
        v = _u32(v)
        check(lib().emh_write_u32(self._ctx, b.h, offset, _p(v), v.size))

    def read_f32(self, b: DevBuf, rng=None) -> np.ndarray:
        lo, hi = rng if rng is not None else (0, len(b))
        out = np.empty(max(hi - lo, 0), np.float32)
        check(lib().emh_read_f32(self._ctx, b.h, lo, hi, _p(out)))
        return out

    def read_u32(self, b: DevBuf, rng=None) -> np.ndarray:
        lo, hi = rng if rng is not None else (0, len(b))
        out = np.empty(max(hi - lo, 0), np.uint32)
        check(lib().emh_read_u32(self._ctx, b.h, lo, hi, _p(out)))
        return out

    def flush(self):
        check(lib().emh_flush(self._ctx))

    def sync(self):
        check(lib().emh_sync(self._ctx))

    def wrap(self, ptr: int, length: int, kind: int) -> DevBuf:
        """A non-owning view of device memory (e.g. a torch tensor's data_ptr())."""
        h = C.c_void_p()
        check(lib().emh_wrap(self._ctx, C.c_void_p(ptr), length, kind, C.byref(h)))
        return DevBuf(self, h, kind)

    # -- Device ops
    def top1(self, x: Mat, sel: Select, centroids: DevBuf, cnorm: Optional[DevBuf], k: int,
             metric, labels: DevBuf, scores: DevBuf):
        check(lib().emh_top1(self._ctx, x.dev.h, x.d, sel.ids.h if sel.ids else None,
                             sel.rows[0], sel.rows[1], centroids.h, cnorm.h if cnorm else None,
                             k, _metric(metric), labels.h, scores.h))

    def topk(self, queries, data, d: int, kk: int, exclude_self: bool):
        q, x = _f32(queries), _f32(data)
        m, n = q.size // d, x.size // d
        ids = np.empty(m * kk, np.uint32)
        sims = np.empty(m * kk, np.float32)
        same = queries is data
        check(lib().emh_topk(self._ctx, _p(q), m, _p(q) if same else _p(x), n, d, kk,
                             int(exclude_self), _p(ids), _p(sims)))
        return ids, sims

    def topk_dev(self, q: DevBuf, m: int, data: DevBuf, n: int, d: int, kk: int,
                 exclude_self: bool, ids: DevBuf, sims: DevBuf):
        check(lib().emh_topk_dev(self._ctx, q.h, m, data.h, n, d, kk, int(exclude_self),
                                 ids.h, sims.h))

    def scatter_add(self, x: Mat, sel: Select, labels: DevBuf, k: int, sums: DevBuf,
                    counts: DevBuf, acc: Optional[DevBuf] = None):
        check(lib().emh_scatter_add(self._ctx, x.dev.h, x.d, sel.ids.h if sel.ids else None,
                                    sel.rows[0], sel.rows[1], labels.h, k, sums.h, counts.h,
                                    acc.h if acc else None))

    def row_norms(self, m: DevBuf, rows: int, d: int, out: DevBuf):
        check(lib().emh_row_norms(self._ctx, m.h, rows, d, out.h))

    def normalize_rows(self, src: DevBuf, rows: int, d: int, dst: DevBuf):
        check(lib().emh_normalize_rows(self._ctx, src.h, rows, d, dst.h))

    def split(self, positions: DevBuf, usage: DevBuf, plan: List[Tuple[int, int]], d: int):
        pairs = _u32(np.asarray(plan, dtype=np.uint32).reshape(-1))
        check(lib().emh_split(self._ctx, positions.h, usage.h, _p(pairs), len(plan), d))

    def ema_update(self, positions: DevBuf, usage: DevBuf, sums: DevBuf, counts: DevBuf, k: int,
                   d: int, step: EmaStep):
        check(lib().emh_ema_update(self._ctx, positions.h, usage.h, sums.h, counts.h, k, d,
                                   step.alpha, step.decay, int(step.replace)))

    # -- Assigner::assign (assign_all over assign_on)
    def assign(self, x, d: int, centroids, metric, chunk: int = 65536):
        x, c = _f32(x), _f32(centroids)
        n, k = x.size // d, c.size // d
        labels = np.empty(n, np.uint32)
        scores = np.empty(n, np.float32)
        check(lib().emh_assign(self._ctx, _p(x), n, d, _p(c), k, _metric(metric), chunk,
                               _p(labels), _p(scores)))
        return labels, scores

    def assign_dev(self, x: DevBuf, n: int, d: int, centroids: DevBuf, k: int, metric,
                   labels: DevBuf, scores: DevBuf, chunk: int = 65536):
        """assign_on with rows, centroids and outputs resident on the device."""
        check(lib().emh_assign_dev(self._ctx, x.h, n, d, centroids.h, k, _metric(metric), chunk,
                                   labels.h, scores.h))

    def train_dev(self, x: DevBuf, n: int, config: "Config", centroids_out: Optional[DevBuf] = None,
                  init=None, state=None):
        """Emeans::train on data already bound to the device; returns (centroids, info).
        init: initial centroids (k*d host array or DevBuf; train_from); state:
        (positions, usage) EMA state (train_resume). With centroids_out (a k*d
        f32 buffer) the centroids also stay on the device."""
        k, d = config.k, config.d
        cent = np.empty(k * d, np.float32)
        pos = np.empty(k * d, np.float32)
        usage = np.empty(k, np.float32)
        labels = np.empty(n, np.int32)
        stats = (_CEpoch * 64)()
        out = _CTrainOut(_p(cent), _p(pos), _p(usage), _p(labels), C.addressof(stats), 64)
        out.centroids_dev = centroids_out.h if centroids_out is not None else None
        ccfg = config._c()
        cin, keep = _train_init(k, d, init, state)
        check(lib().emh_train_dev(self._ctx, x.h, n, C.byref(ccfg), cin, C.byref(out)))
        del keep
        info = {"stats": [EpochStats(stats[e].obj, stats[e].time, stats[e].imbalance_factor,
                                     int(stats[e].nsplit)) for e in range(out.n_epochs)],
                "n_splits": int(out.n_splits), "batch_size": int(out.batch_size),
                "alpha0": out.alpha0, "total_steps": int(out.total_steps),
                "fallback_rows": int(out.fallback_rows), "positions": pos, "usage": usage,
                "labels": labels}
        return cent, info

    _PROF_OPS = {"screen": EMH_PROF_SCREEN, "scatter_add": EMH_PROF_SCATTER,
                 "ema_update": EMH_PROF_EMA}

    def profile(self, every, op: Optional[str] = None):
        """Time every `every`-th instance of the MFMA screen, scatter_add and
        ema_update (or of `op` alone) with HIP events on the context's stream
        (0 or False: off; 1 or True: every instance)."""
        if op is None:
            check(lib().emh_profile(self._ctx, int(every)))
        else:
            check(lib().emh_profile_op(self._ctx, self._PROF_OPS[op], int(every)))

    def profile_read(self, op: str = "screen"):
        """(total ms, instances timed, algorithmic units) of op ("screen": FLOP,
        "scatter_add" or "ema_update": HBM bytes); resets op's totals."""
        code = self._PROF_OPS[op]
        ms, n, u = C.c_double(), C.c_uint64(), C.c_double()
        check(lib().emh_profile_read_op(self._ctx, code, C.byref(ms), C.byref(n), C.byref(u)))
        return ms.value, n.value, u.value

    def kmeans_pp(self, x: DevBuf, n: int, d: int, kmax: int, seed: int) -> np.ndarray:
        """kmeans_pp (emeans-cluster/src/auto.rs:401-455) on rows resident on the device."""
        picks = np.zeros(max(kmax, 1), np.uint32)
        m = C.c_size_t()
        check(lib().emh_kmeans_pp(self._ctx, x.h, n, d, kmax, seed & 0xFFFFFFFF, _p(picks),
                                  C.byref(m)))
        return picks[:m.value].copy()

    def internal_scores(self, x: DevBuf, n: int, d: int, labels: DevBuf, k: int) -> dict:
        """internal_scores (emeans-cluster/src/metrics.rs:113-268) on the device."""
        from ._lib import Internal
        r = Internal()
        sizes = np.zeros(k, np.uint64)
        check(lib().emh_internal_scores(self._ctx, x.h, n, d, labels.h, k, C.byref(r),
                                        _p(sizes)))
        return {"k_eff": int(r.k_eff), "silhouette": r.silhouette,
                "calinski_harabasz": r.calinski_harabasz, "davies_bouldin": r.davies_bouldin,
                "objective": r.objective, "sizes": sizes.astype(np.int64)}

    def dots(self, a: np.ndarray, b: np.ndarray) -> np.ndarray:
        """gemm_nt (emeans-core/src/assign.rs:813-825) on the device: the
        (m x nb) dots of the rows of a (m x d) with the rows of b (nb x d),
        each one fma chain over the columns in order."""
        a, b = np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32)
        if a.ndim != 2 or b.ndim != 2 or a.shape[1] != b.shape[1]:
            raise ValueError("a and b must be m x d and nb x d")
        m, nb, d = a.shape[0], b.shape[0], a.shape[1]
        if m == 0 or nb == 0:
            return np.zeros((m, nb), np.float32)
        ab, bb = self.upload_f32(a), self.upload_f32(b)
        out = self.zeros_f32(m * nb)
        check(lib().emh_dots(self._ctx, ab.h, m, bb.h, nb, d, out.h))
        return self.read_f32(out).reshape(m, nb)

    SCREEN_VARIANTS = {0: "none", 1: "big_tagged", 2: "big_sorted", 3: "small_bf16",
                       4: "small_f32", 5: "big_knn", 6: "big_f16"}

    def screen_margin(self, x: Mat, sel: Select, centroids: DevBuf, cnorm: Optional[DevBuf],
                      k: int, metric) -> dict:
        """The screen of top1 on these arguments, measured instead of checked:
        which screen ran, and max |screen key - exact key| / E over its lists."""
        from ._lib import ScreenReport
        r = ScreenReport()
        check(lib().emh_screen_margin(self._ctx, x.dev.h, x.d, sel.ids.h if sel.ids else None,
                                      sel.rows[0], sel.rows[1], centroids.h,
                                      cnorm.h if cnorm else None, k, _metric(metric),
                                      C.byref(r)))
        return self._report(r)

    def screen_margin_topk(self, q: DevBuf, m: int, data: DevBuf, n: int, d: int,
                           exclude_self: bool) -> dict:
        """The same for the kNN screen (16-neighbour lists) of topk_dev."""
        from ._lib import ScreenReport
        r = ScreenReport()
        check(lib().emh_screen_margin_topk(self._ctx, q.h, m, data.h, n, d, int(exclude_self),
                                           C.byref(r)))
        return self._report(r)

    def _report(self, r):
        return {"variant": self.SCREEN_VARIANTS[r.variant], "parts": r.parts,
                "tiles_per_part": r.tiles_per_part, "pairs": int(r.pairs), "over": int(r.over),
                "max_ratio": r.max_ratio, "max_dot_ratio": r.max_dot_ratio}

    def fallback_rows(self) -> int:
        return lib().emh_fallback_rows(self._ctx)

    def set_screen(self, mode):
        """Top-1 / top-k path: 1 or True = bf16 three-pass MFMA screen + exact
        check (default), 3 = the same with the split-operand top-1 screen in
        fp16 two-pass arithmetic, 2 = f32 MFMA screen + exact check, 0 or
        False = the exact kernels alone. Every mode gives the same bits."""
        check(lib().emh_set_screen(self._ctx, int(mode)))

    EXACT_BELOW = 4096

    def set_exact_below(self, items: int):
        """Top-1 calls of at most `items` exact items (rows x max(ceil(k / 64),
        2)) take the exact kernels alone even when the mode screens (default
        EXACT_BELOW); 0 screens every call the mode screens. Same bits."""
        check(lib().emh_set_exact_below(self._ctx, int(items)))


def _train_init(k, d, init, state):
    """The emh_train_init of a run (or None) and the arrays it points into."""
    if init is None and state is None:
        return None, []
    if init is not None and state is not None:
        raise ValueError("give initial centroids or EMA state, not both")
    if isinstance(init, DevBuf):
        return C.byref(_CTrainInit(None, init.h, None, None)), [init]
    if init is not None:
        c = _f32(init).reshape(-1)
        if c.size != k * d:
            raise ValueError("init centroids must be k x d")
        return C.byref(_CTrainInit(_p(c), None, None, None)), [c]
    pos, usage = (_f32(v).reshape(-1) for v in state)
    if pos.size != k * d:
        raise ValueError("positions must be k x d")
    if usage.size != k:
        raise ValueError("usage must have k entries")
    return C.byref(_CTrainInit(None, None, _p(pos), _p(usage))), [pos, usage]


def _epoch_rows(n, cfg):
    """Recipe::resolve's epoch rows for n rows (emh_host_recipe, no device)."""
    b, a0, ne, tot = C.c_uint64(), C.c_double(), C.c_uint64(), C.c_uint64()
    rows = np.zeros(64, np.uint64)
    ccfg = cfg._c()
    check(lib().emh_host_recipe(n, C.byref(ccfg), C.byref(b), C.byref(a0), _p(rows), 64,
                                C.byref(ne), C.byref(tot)))
    return [int(r) for r in rows[:ne.value]]


def recipe_batch(n, cfg) -> int:
    """Recipe::resolve's batch size for n rows (emh_host_recipe, no device)."""
    b, a0, ne, tot = C.c_uint64(), C.c_double(), C.c_uint64(), C.c_uint64()
    rows = np.zeros(64, np.uint64)
    ccfg = cfg._c()
    check(lib().emh_host_recipe(n, C.byref(ccfg), C.byref(b), C.byref(a0), _p(rows), 64,
                                C.byref(ne), C.byref(tot)))
    return int(b.value)


class Backend:
    """The backend names of this package, as emeans_cluster::Backend gives
    them (backend.rs:41-102): NAMES lists what from_str accepts for help
    texts; "hip-gfx950" is an alias of "hip"."""
    NAMES = (BACKEND_NAME,)
    _ALIASES = {"hip": BACKEND_NAME, "hip-gfx950": BACKEND_NAME}

    def __init__(self, name: str = BACKEND_NAME):
        self._name = Backend.from_str(name)._name if name != BACKEND_NAME else name

    @staticmethod
    def from_str(s: str) -> "Backend":
        if s not in Backend._ALIASES:
            raise ValueError(f"unknown backend {s!r} ({', '.join(Backend.NAMES)})")
        b = Backend.__new__(Backend)
        b._name = Backend._ALIASES[s]
        return b

    def name(self) -> str:
        return self._name

    def __eq__(self, other):
        return isinstance(other, Backend) and other._name == self._name

    def __repr__(self):
        return f"Backend({self._name!r})"


def make_assigner(backend=BACKEND_NAME, device: int = 0) -> HipDevice:
    """make_assigner (backend.rs:106-114) for the "hip" backend: builds the
    gfx950 engine; fails when the library or a gfx950 device is missing."""
    b = backend if isinstance(backend, Backend) else Backend.from_str(backend)
    assert b.name() == BACKEND_NAME
    return HipDevice(device)


def available_backends():
    """available_backends (bindings/common/src/lib.rs:131-137): the names of
    Backend.NAMES whose make_assigner succeeds on this machine."""
    out = []
    for n in Backend.NAMES:
        try:
            make_assigner(n).close()
            out.append(n)
        except (EmeansHipError, EmeansHipInvalid, OSError):
            pass
    return out


# ---------------------------------------------------------------------- model
@dataclass
class Config:
    """Emeans constructor options (model.rs:24-76); faiss defaults."""
    d: int
    k: int
    nepochs: float = 5.0
    batch_size: Optional[int] = None
    alpha0: Optional[float] = None
    batch_law: str = "auto"
    seed: int = 1234
    spherical: bool = False
    unused_threshold: Optional[float] = None
    max_points_per_centroid: Optional[int] = None
    assignment_chunk_size: Optional[int] = None
    capture_assignments: bool = True
    verbose: bool = False

    def metric(self):
        return "ip" if self.spherical else "l2"

    def _c(self):
        laws = {"auto": 0, "throughput": 1, "quality": 2}
        if self.batch_law not in laws:
            raise ValueError(f"unknown batch law {self.batch_law!r} (auto, throughput, quality)")
        return _CConfig(self.k, self.d, float(self.nepochs), self.batch_size or 0,
                        int(self.alpha0 is not None), float(self.alpha0 or 0.0),
                        laws[self.batch_law], self.seed & 0xFFFFFFFF, int(self.spherical),
                        int(self.unused_threshold is not None),
                        float(self.unused_threshold or 0.0), self.assignment_chunk_size or 0,
                        int(self.capture_assignments), int(self.verbose))


@dataclass
class EpochStats:
    obj: float
    time: float
    imbalance_factor: float
    nsplit: int


@dataclass
class Trained:
    centroids: np.ndarray
    labels: Optional[np.ndarray]


@dataclass
class Assignment:
    labels: np.ndarray
    scores: np.ndarray

    def mean_objective(self, spherical: bool) -> float:
        """Mean squared distance, or mean of 2 - 2 cos (model.rs:127-141): an
        f64 sum in row order."""
        s = self.scores.astype(np.float64)
        v = 2.0 - 2.0 * s if spherical else s
        return float(np.cumsum(v)[-1] / len(v)) if len(v) else 0.0


class Emeans:
    """faiss NumpyEmeans (model.rs) with the device loop on the gfx950 backend."""

    def __init__(self, config: Config, assigner: Optional[HipDevice] = None):
        if config.d <= 0 or config.k <= 0:
            raise ValueError("d and k must be positive")
        if not (np.isfinite(config.nepochs) and config.nepochs > 0):
            raise ValueError("nepochs must be positive")
        if config.max_points_per_centroid is not None and config.max_points_per_centroid < 1:
            raise ValueError("max_points_per_centroid must be >= 1 or None")
        if config.unused_threshold is not None and config.unused_threshold < 0:
            raise ValueError("unused_threshold must be >= 0 (0 disables revival)")
        self.config = config
        self._dev = assigner  # made on first use when not given
        self._centroids = None
        self._positions = None
        self._usage = None
        self._stats: List[EpochStats] = []
        self._n_splits = 0
        self._recipe = {}
        self.failed = False
        self.fallback_rows = 0

    @property
    def dev(self) -> HipDevice:
        if self._dev is None:
            self._dev = make_assigner()
        return self._dev

    def _require_ok(self):
        if self.failed:
            raise RuntimeError("create a new object after execution failure")

    def training_subset(self, n: int):
        """Sorted rows kept by max_points_per_centroid (model.rs:752-770)."""
        m = self.config.max_points_per_centroid
        if m is None or n <= m * self.config.k:
            return None
        keep = np.empty(n, np.uint32)
        lib().emh_host_permutation((self.config.seed ^ 0x9E3779B9) & 0xFFFFFFFF, n, _p(keep))
        return np.sort(keep[: m * self.config.k])

    def train(self, x) -> Trained:
        """Sample k initial centroids, train, close with exact means (model.rs:700-703)."""
        return self.train_from(x, None)

    def train_from(self, x, init=None) -> Trained:
        """train with given initial centroids (k x d; model.rs:705-736)."""
        self._require_ok()
        try:
            return self._train(x, init=init)
        except Exception:
            self.failed = True
            raise

    def train_resume(self, x) -> Trained:
        """Continue from the saved EMA state on x, new or grown data (model.rs:739-749)."""
        self._require_ok()
        if self._usage is None:
            raise RuntimeError("no EMA state to resume from")
        try:
            return self._train(x, state=(self._positions, self._usage))
        except Exception:
            self.failed = True
            raise

    def _train(self, x, init=None, state=None) -> Trained:
        cfg = self.config
        x = _f32(x).reshape(-1)
        if x.size % cfg.d:
            raise ValueError("x must be n x d")
        n = x.size // cfg.d
        keep = self.training_subset(n) if state is None else None  # resume: all rows
        xs = x if keep is None else x.reshape(n, cfg.d)[keep].reshape(-1)
        m = xs.size // cfg.d
        k, d = cfg.k, cfg.d
        cent = np.empty(k * d, np.float32)
        pos = np.empty(k * d, np.float32)
        usage = np.empty(k, np.float32)
        labels = np.empty(m, np.int32)
        stats = (_CEpoch * 64)()
        out = _CTrainOut(_p(cent), _p(pos), _p(usage), _p(labels), C.addressof(stats), 64)
        ccfg = cfg._c()
        cin, hold = _train_init(k, d, init, state)
        check(lib().emh_train(self.dev._ctx, _p(xs), m, C.byref(ccfg), cin, C.byref(out)))
        del hold
        self._centroids, self._positions, self._usage = cent, pos, usage
        self._stats = [EpochStats(stats[e].obj, stats[e].time, stats[e].imbalance_factor,
                                  int(stats[e].nsplit)) for e in range(out.n_epochs)]
        self._n_splits = int(out.n_splits)
        self._recipe = model_file.recipe_dict(cfg, m, int(out.batch_size), out.alpha0,
                                              _epoch_rows(m, cfg), self.dev.name())
        self.fallback_rows = int(out.fallback_rows)
        lab = labels if cfg.capture_assignments else None
        if lab is not None and keep is not None:
            full = np.full(n, -1, np.int32)
            full[keep] = lab
            lab = full
        return Trained(cent.copy(), lab)

    def assign(self, x) -> Assignment:
        self._require_ok()
        if self._centroids is None:
            raise RuntimeError("model is not trained")
        labels, scores = self.dev.assign(x, self.config.d, self._centroids, self.config.metric(),
                                         self.config.assignment_chunk_size or 65536)
        return Assignment(labels, scores)

    def centroids(self):
        return self._centroids

    def ema_state(self):
        return (self._positions, self._usage) if self._usage is not None else None

    def iteration_stats(self):
        return list(self._stats)

    def obj(self):
        return [s.obj for s in self._stats]

    def n_splits(self):
        return self._n_splits

    def recipe(self):
        return dict(self._recipe)

    # -- model files (io.rs:72-186)
    def to_bytes(self) -> bytes:
        """The model file's bytes (io.rs:92-121)."""
        self._require_ok()
        st = [(s.obj, s.time, s.imbalance_factor, s.nsplit) for s in self._stats]
        return model_file.to_bytes(self.config, self._recipe or None, self._n_splits, st,
                                   self._centroids, self._positions,
                                   self._usage if self._usage is not None else [])

    def save(self, path):
        """Write the model file to a temporary file, then rename it over path (io.rs:74-88)."""
        model_file.save_bytes(path, self.to_bytes())

    @classmethod
    def from_bytes_with(cls, b, assigner: Optional[HipDevice] = None) -> "Emeans":
        """A model from the bytes of to_bytes or a model file (io.rs:137-186)."""
        header, cent, pos, usage = model_file.from_bytes(b)
        c = header["config"]
        cfg = Config(**c)
        m = cls(cfg, assigner)
        m._recipe = header["recipe"] or {}
        m._n_splits = int(header["n_splits"])
        m._stats = [EpochStats(s["obj"], s["time"], s["imbalance_factor"], int(s["nsplit"]))
                    for s in header["iteration_stats"]]
        m._centroids, m._positions, m._usage = cent, pos, usage
        return m

    @classmethod
    def load_with(cls, path, assigner: Optional[HipDevice] = None) -> "Emeans":
        with open(path, "rb") as f:
            return cls.from_bytes_with(f.read(), assigner)


# ------------------------------------------------------------------------ kNN
@dataclass
class Neighbors:
    """k nearest rows per query, best first (emeans-core/src/knn.rs:21-45)."""
    k: int
    ids: np.ndarray
    sims: np.ndarray

    def __len__(self):
        return self.ids.size // max(self.k, 1)

    def row(self, i: int):
        return self.ids[i * self.k:(i + 1) * self.k], self.sims[i * self.k:(i + 1) * self.k]


def _search(queries, data, d, k, exclude_self, dev):
    q, x = _f32(queries).reshape(-1), _f32(data).reshape(-1)
    if d <= 0 or q.size % d or x.size % d:
        raise ValueError("queries and data must be n x d")
    if k <= 0:
        raise ValueError("k must be positive")
    if k > KLONG:
        raise ValueError(f"the gfx950 top-k keeps at most {KLONG} neighbours")
    # k <= GPU_KMAX: the MFMA screen; above it (the reference's CPU search,
    # knn.rs:42) the exact top-k on the GPU, with the same results.
    dev = dev or make_assigner()
    ids, sims = dev.topk(q, q if exclude_self else x, d, k, exclude_self)
    return Neighbors(k, ids, sims)


def knn_self(data, d: int, k: int, dev: Optional[HipDevice] = None) -> Neighbors:
    """Neighbours of every row among the other rows (knn.rs:17-19)."""
    return _search(data, data, d, k, True, dev)


def knn(queries, data, d: int, k: int, dev: Optional[HipDevice] = None) -> Neighbors:
    """Neighbours of every query among the data rows (knn.rs:22-30)."""
    return _search(queries, data, d, k, False, dev)


# ---------------------------------------------------------------------- dedup
@dataclass
class DedupConfig:
    """dedup.rs:39-62: neighbours per row, link threshold, star threshold
    (None = sim_threshold) and the largest time gap of a link (None: similarity
    alone decides)."""
    k: int = 10
    sim_threshold: float = 0.95
    rep_threshold: Optional[float] = None
    max_gap_secs: Optional[float] = None

    def _c(self):
        return _CDedupConfig(self.k, self.sim_threshold, int(self.rep_threshold is not None),
                             float(self.rep_threshold or 0.0), int(self.max_gap_secs is not None),
                             float(self.max_gap_secs or 0.0))


@dataclass
class DedupInput:
    """dedup.rs:65-76: optional per-row creation times (NaN = unknown), burst
    ids (None = no burst; rows of one id always share a group) and
    representative priorities (higher wins)."""
    created_unix: Optional[np.ndarray] = None
    burst: Optional[list] = None
    priority: Optional[np.ndarray] = None


@dataclass
class DedupResult:
    group_of: np.ndarray
    representatives: np.ndarray
    anchors: np.ndarray
    sizes: np.ndarray
    nn_sim: np.ndarray
    linked_pairs: int
    split_components: int

    def n_groups(self):
        return len(self.representatives)

    def anchor(self, g: int) -> int:
        return int(self.anchors[g]) if len(self.anchors) == len(self.representatives) \
            else int(self.representatives[g])

    def expand(self, rep_labels):
        rep_labels = np.asarray(rep_labels)
        assert len(rep_labels) == len(self.representatives)
        return rep_labels[self.group_of]

    def gather(self, x, d: int):
        return np.asarray(x, np.float32).reshape(-1, d)[self.representatives].reshape(-1)


def _dedup_call(fn, n, input, cfg, *lead):
    if not (-1.0 <= cfg.sim_threshold <= 1.0):
        raise ValueError("sim_threshold must be in [-1, 1]")
    keep = []

    def arr(v, dt, what):
        if v is None:
            return None
        a = np.ascontiguousarray(v, dt)
        if a.size != n:
            raise ValueError(f"one {what} per row")
        keep.append(a)
        return a.ctypes.data

    inp = input or DedupInput()
    burst = None if inp.burst is None else [-1 if b is None else int(b) for b in inp.burst]
    cin = _CDedupInput(arr(inp.created_unix, np.float64, "timestamp"),
                       arr(burst, np.int64, "burst id"), arr(inp.priority, np.float32, "priority"))
    g = np.zeros(n, np.uint32)
    reps, anchors, sizes = (np.zeros(max(n, 1), np.uint32) for _ in range(3))
    nn = np.zeros(n, np.float32)
    out = _CDedupResult(_p(g), _p(reps), _p(anchors), _p(sizes), _p(nn), 0, 0, 0)
    ccfg = cfg._c()
    check(fn(*lead, C.byref(cin), C.byref(ccfg), C.byref(out)))
    m = out.n_groups
    return DedupResult(g, reps[:m].copy(), anchors[:m].copy(), sizes[:m].copy(), nn,
                       int(out.linked_pairs), int(out.split_components))


def dedup(x, d: int, input: Optional[DedupInput] = None, cfg: DedupConfig = DedupConfig(),
          dev: Optional[HipDevice] = None, priority=None) -> DedupResult:
    """Near-duplicate groups of unit rows (dedup.rs:163-183): kNN on the GPU,
    groups on the host. `priority` is a shorthand for DedupInput(priority=...)."""
    if input is not None and not isinstance(input, DedupInput):
        raise TypeError("dedup(x, d, input, cfg, ...): input must be a DedupInput")
    x = _f32(x).reshape(-1)
    if d <= 0 or x.size % d:
        raise ValueError("x must be n x d")
    n = x.size // d
    if priority is not None:
        input = DedupInput(*(input.created_unix, input.burst) if input else (None, None), priority)
    dev = dev or make_assigner()
    return _dedup_call(lib().emh_dedup, n, input, cfg, dev._ctx, _p(x), n, d)


def dedup_with_neighbors(x, d: int, nb: Neighbors, input: Optional[DedupInput] = None,
                         cfg: DedupConfig = DedupConfig()) -> DedupResult:
    """dedup with neighbours the caller computed (dedup.rs:186-358); host only."""
    x = _f32(x).reshape(-1)
    if d <= 0 or x.size % d:
        raise ValueError("x must be n x d")
    n = x.size // d
    if len(nb) != n:
        raise ValueError("neighbours must have one row per row of x")
    ids, sims = _u32(nb.ids), _f32(nb.sims)
    return _dedup_call(lib().emh_dedup_neighbors, n, input, cfg, _p(x), n, d, _p(ids), _p(sims),
                       nb.k)
