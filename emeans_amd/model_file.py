"""Model files (crates/emeans-core/src/io.rs:72-186) for models trained on
this backend: the reference's layout, so a file written here loads in the
reference and the other way round.

Layout (little-endian): 8-byte magic EMEANS\\0\\x01 | u64 header length h |
h bytes of JSON header {version, k, d, config, recipe, n_splits,
iteration_stats, has_centroids, has_ema} | centroids k*d f32 (if
has_centroids) | EMA positions k*d f32 and masses k f32 (if has_ema). Loading
checks the exact length.

The header is what the reference's serde_json writes for its Header struct
(io.rs:39-50 with Config model.rs:24-52, Recipe recipe.rs:167-196 and
EpochStats model.rs:80-89): keys in declaration order, no whitespace, None as
null, the batch law in lower case, and floats in ryu's shortest round-trip
form laid out as ryu's pretty printer does (json_float below).
"""

import json
import math
import struct
from decimal import Decimal

import numpy as np

MAGIC = b"EMEANS\x00\x01"
VERSION = 1
# recipe.rs:10-24
ALPHA_MIN_FACTOR = 0.1
CHECK_UNUSED_EVERY = 5
INIT_USAGE = 1.0 / 65536.0
SPLIT_EPSILON = 1e-4
UNUSED_THRESHOLD = 0.1
NO_REVIVAL_MAX_D = 2
AUTO_QUALITY_MAX_D = 16
DEFAULT_ASSIGNMENT_CHUNK = 65536


class F32(float):
    """A value the reference stores as f32 (serialized with f32 digits)."""


def _digits(s):
    """(decimal digits, exponent) of a shortest round-trip repr: value = digits 10^exp."""
    t = Decimal(s).as_tuple()
    digits = "".join(map(str, t.digits)).lstrip("0") or "0"
    stripped = digits.rstrip("0") or "0"  # trailing zeros move into the exponent
    return stripped, t.exponent + (len(digits) - len(stripped))


def json_float(v, f32=False):
    """ryu's pretty layout of the shortest round-trip digits of v (f64, or
    f32 when f32): with n digits and the decimal point kk places after the
    first, plain notation when the point falls within the first 16 places (13
    for f32) or at most 5 zeros (6 for f32) follow "0.", else d.ddde<exp>;
    whole numbers end in ".0"."""
    if not math.isfinite(v):
        return "null"  # serde_json writes non-finite floats as null
    if v == 0.0:
        return "-0.0" if math.copysign(1.0, v) < 0 else "0.0"
    sign = "-" if v < 0 else ""
    if f32:
        s = np.format_float_scientific(np.float32(abs(v)), unique=True, trim="-")
    else:
        s = repr(abs(float(v)))
    digits, k = _digits(s)
    n = len(digits)
    kk = n + k
    hi, lo = (13, -6) if f32 else (16, -5)
    if 0 <= k and kk <= hi:
        out = digits + "0" * k + ".0"
    elif 0 < kk <= hi:
        out = digits[:kk] + "." + digits[kk:]
    elif lo < kk <= 0:
        out = "0." + "0" * (-kk) + digits
    elif n == 1:
        out = digits + "e" + str(kk - 1)
    else:
        out = digits[0] + "." + digits[1:] + "e" + str(kk - 1)
    return sign + out


def to_json(v):
    """serde_json's compact form of an ordered structure of dicts, lists,
    strings, bools, None, ints, floats and F32s."""
    if v is None:
        return "null"
    if isinstance(v, bool):
        return "true" if v else "false"
    if isinstance(v, F32):
        return json_float(float(v), f32=True)
    if isinstance(v, float):
        return json_float(v)
    if isinstance(v, (int, np.integer)):
        return str(int(v))
    if isinstance(v, str):
        return json.dumps(v, ensure_ascii=False)
    if isinstance(v, dict):
        return "{" + ",".join(json.dumps(k) + ":" + to_json(x) for k, x in v.items()) + "}"
    if isinstance(v, (list, tuple)):
        return "[" + ",".join(to_json(x) for x in v) + "]"
    raise TypeError(f"cannot serialize {type(v).__name__}")


def to_json_pretty(v, indent=""):
    """serde_json's pretty form (to_vec_pretty): two-space indents, one
    element or key per line, "key": value, and [] / {} when empty."""
    inner = indent + "  "
    if isinstance(v, dict):
        if not v:
            return "{}"
        items = (inner + json.dumps(k) + ": " + to_json_pretty(x, inner) for k, x in v.items())
        return "{\n" + ",\n".join(items) + "\n" + indent + "}"
    if isinstance(v, (list, tuple)):
        if not v:
            return "[]"
        return "[\n" + ",\n".join(inner + to_json_pretty(x, inner) for x in v) + "\n" + \
            indent + "]"
    return to_json(v)


def save_bytes(path, b):
    """Write b to path's .tmp sibling, flush it to disk, then rename it over
    path (io.rs:74-88)."""
    import os
    tmp = os.path.splitext(str(path))[0] + ".tmp"
    with open(tmp, "wb") as f:
        f.write(b)
        f.flush()
        os.fsync(f.fileno())
    os.replace(tmp, path)


def config_dict(c):
    """model.rs:24-52, field order kept."""
    return {"d": int(c.d), "k": int(c.k), "nepochs": float(c.nepochs),
            "batch_size": None if c.batch_size is None else int(c.batch_size),
            "alpha0": None if c.alpha0 is None else float(c.alpha0),
            "batch_law": c.batch_law, "seed": int(c.seed) & 0xFFFFFFFF,
            "spherical": bool(c.spherical),
            "unused_threshold": None if c.unused_threshold is None else float(c.unused_threshold),
            "max_points_per_centroid": None if c.max_points_per_centroid is None
            else int(c.max_points_per_centroid),
            "assignment_chunk_size": None if c.assignment_chunk_size is None
            else int(c.assignment_chunk_size),
            "capture_assignments": bool(c.capture_assignments), "verbose": bool(c.verbose)}


def resolve_law(batch_law, d):
    """BatchLaw::resolve (recipe.rs:44-53): (law, reason)."""
    if batch_law == "auto":
        return ("quality", f"d <= {AUTO_QUALITY_MAX_D}") if d <= AUTO_QUALITY_MAX_D \
            else ("throughput", f"d > {AUTO_QUALITY_MAX_D}")
    return batch_law, "requested"


def recipe_dict(c, n, batch_size, alpha0, epoch_rows, backend):
    """Recipe::resolve (recipe.rs:198-254) around the resolved batch size,
    alpha0 and epoch rows: every field in declaration order."""
    law, reason = resolve_law(c.batch_law, c.d)
    given = c.batch_size is not None
    name = ("manual" if c.alpha0 is not None else "manual_batch") if given else "canonical_v1"
    epoch_steps = [-(-int(r) // int(batch_size)) for r in epoch_rows]
    tau = c.unused_threshold if c.unused_threshold is not None else \
        (0.0 if c.d <= NO_REVIVAL_MAX_D else UNUSED_THRESHOLD)
    return {"name": name,
            "batch_law": None if given else law,
            "batch_law_requested": None if given else c.batch_law,
            "batch_law_reason": None if given else reason,
            "batch_size": int(batch_size),
            "batch_size_requested": None if c.batch_size is None else int(c.batch_size),
            "alpha0": float(alpha0),
            "alpha0_source": "given" if c.alpha0 is not None else "step_law",
            "nepochs": float(c.nepochs),
            "steps_per_pass": -(-int(n) // int(batch_size)),
            "total_steps": int(sum(epoch_steps)),
            "epoch_rows": [int(r) for r in epoch_rows],
            "epoch_steps": epoch_steps,
            "alpha_min_factor": ALPHA_MIN_FACTOR,
            "check_unused_every": CHECK_UNUSED_EVERY,
            "unused_threshold": float(tau),
            "split_epsilon": SPLIT_EPSILON,
            "init_usage": F32(INIT_USAGE),
            "seed": int(c.seed) & 0xFFFFFFFF,
            "backend": backend,
            "assignment_chunk_size": int(c.assignment_chunk_size or DEFAULT_ASSIGNMENT_CHUNK),
            "spherical": bool(c.spherical),
            "n": int(n)}


def _f32le(a):
    return np.ascontiguousarray(a, dtype="<f4").tobytes()


def to_bytes(config, recipe, n_splits, stats, centroids, positions, usage):
    """Emeans::to_bytes (io.rs:92-121). stats: (obj, time, imbalance_factor,
    nsplit) per epoch; centroids None when untrained; usage empty without EMA state."""
    k, d = int(config.k), int(config.d)
    has_ema = usage is not None and len(usage) > 0
    if recipe is not None:
        recipe = dict(recipe)
        recipe["init_usage"] = F32(recipe["init_usage"])
    header = {"version": VERSION, "k": k, "d": d, "config": config_dict(config),
              "recipe": recipe, "n_splits": int(n_splits),
              "iteration_stats": [{"obj": float(s[0]), "time": float(s[1]),
                                   "imbalance_factor": float(s[2]), "nsplit": int(s[3])}
                                  for s in stats],
              "has_centroids": centroids is not None, "has_ema": has_ema}
    js = to_json(header).encode()
    parts = [MAGIC, struct.pack("<Q", len(js)), js]
    if centroids is not None:
        parts.append(_f32le(centroids))
    if has_ema:
        parts += [_f32le(positions), _f32le(usage)]
    return b"".join(parts)


def from_bytes(b):
    """Emeans::from_bytes_with (io.rs:137-186) without the assigner: the
    header (a dict) and the arrays; the same checks and errors."""
    b = bytes(b)
    if len(b) < 16 or b[:8] != MAGIC:
        raise ValueError("not an emeans model")
    h = struct.unpack("<Q", b[8:16])[0]
    if h > len(b) - 16:
        raise ValueError("truncated header")
    header = json.loads(b[16:16 + h])
    if header["version"] != VERSION:
        raise ValueError(f"unsupported model version {header['version']}")
    k, d = header["k"], header["d"]
    if header["config"]["k"] != k or header["config"]["d"] != d:
        raise ValueError("header k/d disagree with config")
    want = 16 + h + (k * d * 4 if header["has_centroids"] else 0) + \
        ((k * d + k) * 4 if header["has_ema"] else 0)
    if len(b) != want:
        raise ValueError(f"model file has {len(b)} bytes, expected {want}")
    off = 16 + h
    cent = pos = usage = None
    if header["has_centroids"]:
        cent = np.frombuffer(b, "<f4", k * d, off).astype(np.float32)
        off += k * d * 4
    if header["has_ema"]:
        pos = np.frombuffer(b, "<f4", k * d, off).astype(np.float32)
        usage = np.frombuffer(b, "<f4", k, off + k * d * 4).astype(np.float32)
    return header, cent, pos, usage
