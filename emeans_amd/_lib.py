"""Loader of libemeans_hip.so: ctypes signatures of include/emeans_hip.h.

The product has no CPU fallback: when the library is missing or no gfx950
device is present, every entry point raises.
"""

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libemeans_hip.so")

EMH_OK, EMH_INVALID, EMH_ERROR = 0, 1, 2
EMH_L2, EMH_IP = 0, 1
EMH_PROF_SCREEN, EMH_PROF_SCATTER, EMH_PROF_EMA = 0, 1, 2


class EmeansHipError(RuntimeError):
    """A failed call of the gfx950 backend (EMH_ERROR)."""


class EmeansHipInvalid(ValueError):
    """A call rejected for its arguments (EMH_INVALID)."""


class Config(C.Structure):
    _fields_ = [("k", C.c_uint64), ("d", C.c_uint64), ("nepochs", C.c_double),
                ("batch_size", C.c_uint64), ("has_alpha0", C.c_int), ("alpha0", C.c_double),
                ("batch_law", C.c_int), ("seed", C.c_uint32), ("spherical", C.c_int),
                ("has_unused_threshold", C.c_int), ("unused_threshold", C.c_double),
                ("assignment_chunk_size", C.c_uint64), ("capture_assignments", C.c_int),
                ("verbose", C.c_int)]


class EpochStats(C.Structure):
    _fields_ = [("obj", C.c_double), ("time", C.c_double), ("imbalance_factor", C.c_double),
                ("nsplit", C.c_uint64)]


class TrainOut(C.Structure):
    _fields_ = [("centroids", C.c_void_p), ("positions", C.c_void_p), ("usage", C.c_void_p),
                ("labels", C.c_void_p), ("stats", C.c_void_p), ("max_epochs", C.c_uint64),
                ("n_epochs", C.c_uint64), ("n_splits", C.c_uint64), ("batch_size", C.c_uint64),
                ("alpha0", C.c_double), ("total_steps", C.c_uint64),
                ("fallback_rows", C.c_uint64), ("centroids_dev", C.c_void_p)]


class ScreenReport(C.Structure):
    _fields_ = [("variant", C.c_int), ("parts", C.c_int), ("tiles_per_part", C.c_int),
                ("pairs", C.c_uint64), ("over", C.c_uint64), ("max_ratio", C.c_double),
                ("max_dot_ratio", C.c_double)]


class Internal(C.Structure):
    _fields_ = [("k_eff", C.c_uint64), ("silhouette", C.c_double),
                ("calinski_harabasz", C.c_double), ("davies_bouldin", C.c_double),
                ("objective", C.c_double)]


class TrainInit(C.Structure):
    _fields_ = [("centroids", C.c_void_p), ("centroids_dev", C.c_void_p),
                ("positions", C.c_void_p), ("usage", C.c_void_p)]


class DedupConfig(C.Structure):
    _fields_ = [("k", C.c_uint64), ("sim_threshold", C.c_float), ("has_rep_threshold", C.c_int),
                ("rep_threshold", C.c_float), ("has_max_gap_secs", C.c_int),
                ("max_gap_secs", C.c_double)]


class DedupInput(C.Structure):
    _fields_ = [("created_unix", C.c_void_p), ("burst", C.c_void_p), ("priority", C.c_void_p)]


class DedupResult(C.Structure):
    _fields_ = [("group_of", C.c_void_p), ("representatives", C.c_void_p),
                ("anchors", C.c_void_p), ("sizes", C.c_void_p), ("nn_sim", C.c_void_p),
                ("n_groups", C.c_uint64), ("linked_pairs", C.c_uint64),
                ("split_components", C.c_uint64)]


# name: (restype, argtypes). Every function is declared in include/emeans_hip.h.
_vp, _sz, _i, _u32, _u64, _f, _d = (C.c_void_p, C.c_size_t, C.c_int, C.c_uint32, C.c_uint64,
                                     C.c_float, C.c_double)
_pp = C.POINTER(C.c_void_p)
SIGNATURES = {
    "emh_last_error": (C.c_char_p, []),
    "emh_create": (_i, [_i, _pp]),
    "emh_destroy": (_i, [_vp]),
    "emh_name": (C.c_char_p, [_vp]),
    "emh_flush": (_i, [_vp]),
    "emh_sync": (_i, [_vp]),
    "emh_stream": (_vp, [_vp]),
    "emh_bind": (_i, [_vp, _vp, _sz, _pp]),
    "emh_upload_f32": (_i, [_vp, _vp, _sz, _pp]),
    "emh_upload_u32": (_i, [_vp, _vp, _sz, _pp]),
    "emh_zeros_f32": (_i, [_vp, _sz, _pp]),
    "emh_zeros_u32": (_i, [_vp, _sz, _pp]),
    "emh_write_f32": (_i, [_vp, _vp, _sz, _vp, _sz]),
    "emh_write_u32": (_i, [_vp, _vp, _sz, _vp, _sz]),
    "emh_read_f32": (_i, [_vp, _vp, _sz, _sz, _vp]),
    "emh_read_u32": (_i, [_vp, _vp, _sz, _sz, _vp]),
    "emh_free": (_i, [_vp, _vp]),
    "emh_wrap": (_i, [_vp, _vp, _sz, _i, _pp]),
    "emh_buf_ptr": (_vp, [_vp]),
    "emh_buf_len": (_sz, [_vp]),
    "emh_top1": (_i, [_vp, _vp, _sz, _vp, _sz, _sz, _vp, _vp, _sz, _i, _vp, _vp]),
    "emh_top1_noalloc": (_i, [_vp, _vp, _sz, _vp, _sz, _sz, _vp, _vp, _sz, _i, _vp, _vp]),
    "emh_topk": (_i, [_vp, _vp, _sz, _vp, _sz, _sz, _sz, _i, _vp, _vp]),
    "emh_topk_dev": (_i, [_vp, _vp, _sz, _vp, _sz, _sz, _sz, _i, _vp, _vp]),
    "emh_scatter_add": (_i, [_vp, _vp, _sz, _vp, _sz, _sz, _vp, _sz, _vp, _vp, _vp]),
    "emh_row_norms": (_i, [_vp, _vp, _sz, _sz, _vp]),
    "emh_normalize_rows": (_i, [_vp, _vp, _sz, _sz, _vp]),
    "emh_split": (_i, [_vp, _vp, _vp, _vp, _sz, _sz]),
    "emh_ema_update": (_i, [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _f, _f, _i]),
    "emh_train": (_i, [_vp, _vp, _sz, _vp, _vp, _vp]),
    "emh_train_dev": (_i, [_vp, _vp, _sz, _vp, _vp, _vp]),
    "emh_assign": (_i, [_vp, _vp, _sz, _sz, _vp, _sz, _i, _sz, _vp, _vp]),
    "emh_assign_dev": (_i, [_vp, _vp, _sz, _sz, _vp, _sz, _i, _sz, _vp, _vp]),
    "emh_profile": (_i, [_vp, _i]),
    "emh_profile_op": (_i, [_vp, _i, _i]),
    "emh_profile_read": (_i, [_vp, C.POINTER(_d), C.POINTER(_u64), C.POINTER(_d)]),
    "emh_profile_read_op": (_i, [_vp, _i, C.POINTER(_d), C.POINTER(_u64), C.POINTER(_d)]),
    "emh_knn": (_i, [_vp, _vp, _sz, _vp, _sz, _sz, _sz, _i, _vp, _vp]),
    "emh_dedup_neighbors": (_i, [_vp, _sz, _sz, _vp, _vp, _sz, _vp, _vp, _vp]),
    "emh_dedup": (_i, [_vp, _vp, _sz, _sz, _vp, _vp, _vp]),
    "emh_fallback_rows": (_u64, [_vp]),
    "emh_kmeans_pp": (_i, [_vp, _vp, _sz, _sz, _sz, _u32, _vp, C.POINTER(_sz)]),
    "emh_internal_scores": (_i, [_vp, _vp, _sz, _sz, _vp, _sz, _vp, _vp]),
    "emh_dots": (_i, [_vp, _vp, _sz, _vp, _sz, _sz, _vp]),
    "emh_screen_margin": (_i, [_vp, _vp, _sz, _vp, _sz, _sz, _vp, _vp, _sz, _i, _vp]),
    "emh_screen_margin_topk": (_i, [_vp, _vp, _sz, _vp, _sz, _sz, _i, _vp]),
    "emh_set_screen": (_i, [_vp, _i]),
    "emh_set_exact_below": (_i, [_vp, _u64]),
    "emh_host_permutation": (None, [_u32, _u64, _vp]),
    "emh_host_random_sample": (_d, [_u32, _u64]),
    "emh_host_recipe": (_i, [_u64, _vp, C.POINTER(_u64), C.POINTER(_d), _vp, _u64,
                             C.POINTER(_u64), C.POINTER(_u64)]),
    "emh_host_scheduled_alpha": (_d, [_d, _u64, _u64]),
    "emh_host_plan_revival": (_u64, [_vp, _u64, _d, _u32, _vp]),
    "emh_host_numpy_sum_f32": (_f, [_vp, _u64]),
}

_lib = None


def lib():
    """The loaded library; raises if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise EmeansHipError(
                f"{LIB_PATH} is not built; run `python -m emeans_amd.build` (hipcc, gfx950)")
        h = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def check(rc):
    """Raise the library's error for a non-zero status."""
    if rc == EMH_OK:
        return
    msg = (lib().emh_last_error() or b"").decode(errors="replace")
    if rc == EMH_INVALID:
        raise EmeansHipInvalid(msg)
    raise EmeansHipError(msg)
