"""Model files (crates/emeans-core/src/io.rs:72-186) without a GPU.

Pins: the recipe's numeric fields against the 1443 faiss recipes of the
reference's fixture (tests/reference.rs:210-271); ryu's float layout on
values whose serde_json text is fixed by ryu's pretty printer (plain within
16 integer places, at most five zeros after "0.", exponent form otherwise;
13 and six for f32); the layout's exact length, magic and little-endian
header length; and the reference's own failure cases (tests/model.rs:173-186:
a file one byte short, a header length of u64::MAX, a truncated file).
"""

import json
import os
import struct

import numpy as np
import pytest

from emeans_amd import Config, Emeans, model_file as MF
from oracle import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("v,text", [
    (1.0, "1.0"), (0.1, "0.1"), (5.0, "5.0"), (-2.5, "-2.5"), (0.0, "0.0"), (-0.0, "-0.0"),
    (1e-4, "0.0001"), (1e-5, "0.00001"), (1.5e-5, "0.000015"), (1e-6, "1e-6"),
    (4.5e-6, "4.5e-6"), (123.456, "123.456"), (1e15, "1000000000000000.0"), (1e16, "1e16"),
    (1.5e300, "1.5e300"), (123456789012345680.0, "1.2345678901234568e17"),
    (12541.318635046482, "12541.318635046482"), (float("nan"), "null"),
])
def test_f64_layout(v, text):
    assert MF.json_float(v) == text


@pytest.mark.parametrize("v,text", [
    (1.0 / 65536.0, "0.000015258789"), (0.1, "0.1"), (1e10, "10000000000.0"), (1e13, "1e13"),
    (1e-6, "0.000001"), (1e-7, "1e-7"), (3.4028235e38, "3.4028235e38"),
])
def test_f32_layout(v, text):
    assert MF.json_float(v, f32=True) == text


def test_recipe_fields_match_the_faiss_recipes():
    from emeans_amd import _epoch_rows, _lib
    import ctypes as C
    ref = json.load(open(os.path.join(GOLD, "reference.json")))
    for r in ref["recipes"]:
        if r["batch_law"] == "given":  # batch size (and maybe alpha0) given (reference.rs:42-50)
            cfg = Config(d=r["d"], k=r["k"], nepochs=float(r["nepochs"]),
                         batch_size=r["given_batch_size"], alpha0=r["given_alpha0"])
        else:
            cfg = Config(d=r["d"], k=r["k"], nepochs=float(r["nepochs"]),
                         batch_law=r["batch_law"])
        b, a0, ne, tot = C.c_uint64(), C.c_double(), C.c_uint64(), C.c_uint64()
        rows = np.zeros(64, np.uint64)
        cc = cfg._c()
        _lib.check(_lib.lib().emh_host_recipe(r["n"], C.byref(cc), C.byref(b), C.byref(a0),
                                              rows.ctypes.data, 64, C.byref(ne), C.byref(tot)))
        got = MF.recipe_dict(cfg, r["n"], b.value, a0.value, _epoch_rows(r["n"], cfg), "cpu")
        assert got["batch_size"] == r["batch_size"]
        assert got["alpha0"] == r["alpha0"]
        if r["batch_law"] == "given":
            assert got["batch_law"] is None and got["batch_size_requested"] == r["given_batch_size"]
            assert got["name"] == ("manual" if r["given_alpha0"] is not None else "manual_batch")
            continue
        assert got["batch_law"] == r["resolved_law"]
        assert got["steps_per_pass"] == r["steps_per_pass"]
        assert got["epoch_rows"] == r["epoch_rows"]
        assert got["epoch_steps"] == r["epoch_steps"]
        assert got["total_steps"] == r["total_steps"]
        assert got["unused_threshold"] == r["unused_threshold"]
        assert got["name"] == "canonical_v1" and got["alpha0_source"] == "step_law"


def _oracle_model_bytes(x, cfg, backend="cpu-fused"):
    n = x.shape[0]
    o = O.train(x, cfg.d, cfg.k, nepochs=cfg.nepochs, seed=cfg.seed, spherical=cfg.spherical)
    from emeans_amd import _epoch_rows
    rec = MF.recipe_dict(cfg, n, o["batch_size"], o["alpha0"], _epoch_rows(n, cfg), backend)
    stats = [(ob, 0.0, im, int(ns)) for ob, im, ns in zip(o["obj"], o["imbalance"], o["nsplit"])]
    return MF.to_bytes(cfg, rec, o["n_splits"], stats, o["centroids"], o["positions"],
                       o["usage"]), o


def test_layout_and_round_trip():
    n, d, k = 1500, 8, 12
    x = O.common_mixture(n, d, 12, 0.5, False, 4).reshape(n, d)
    cfg = Config(d=d, k=k, nepochs=3.0)
    b, o = _oracle_model_bytes(x, cfg)
    assert b[:8] == b"EMEANS\x00\x01"
    h = struct.unpack("<Q", b[8:16])[0]
    assert len(b) == 16 + h + (2 * k * d + k) * 4
    head = b[16:16 + h].decode()
    assert head.startswith('{"version":1,"k":12,"d":8,"config":{"d":8,"k":12,"nepochs":3.0,'
                           '"batch_size":null,"alpha0":null,"batch_law":"auto","seed":1234,')
    assert '"init_usage":0.000015258789,' in head and '"check_unused_every":5,' in head
    assert ' ' not in head.replace('"d <= 16"', '')
    assert np.frombuffer(b, "<f4", k * d, 16 + h).tobytes() == o["centroids"].tobytes()
    m = Emeans.from_bytes_with(b)  # no device is needed to read a model
    assert m.centroids().tobytes() == o["centroids"].tobytes()
    pos, usage = m.ema_state()
    assert pos.tobytes() == o["positions"].tobytes() and usage.tobytes() == o["usage"].tobytes()
    assert m.obj() == o["obj"].tolist() and m.n_splits() == o["n_splits"]
    assert m.to_bytes() == b


def test_bad_files_fail_loudly(tmp_path):
    """tests/model.rs:173-186."""
    x = O.common_mixture(800, 8, 8, 0.5, False, 2).reshape(800, 8)
    b, _ = _oracle_model_bytes(x, Config(d=8, k=8, nepochs=2.0))
    with pytest.raises(ValueError, match="expected"):
        Emeans.from_bytes_with(b[:-1])
    huge = bytearray(b)
    huge[8:16] = struct.pack("<Q", 2 ** 64 - 1)
    with pytest.raises(ValueError, match="truncated header"):
        Emeans.from_bytes_with(bytes(huge))
    with pytest.raises(ValueError, match="not an emeans model"):
        Emeans.from_bytes_with(b"EMEANZ\x00\x01" + b[8:])
    p = tmp_path / "model.emeans"
    p.write_bytes(b[:-4])
    with pytest.raises(ValueError):
        Emeans.load_with(p)
    p.write_bytes(b)
    assert Emeans.load_with(p).to_bytes() == b
