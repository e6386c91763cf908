"""The mojotrees C ABI without a GPU: the library loads and exports every
declared symbol, argument and parameter validation, error objects, and the
host-side model surface (v4 text load/save, prediction, inspection) on a
model file written by hand.

Mirrors the reference's capi/test_capi.c checks for the calls that need no
training (ajhendel/mojoboost capi/test_capi.c).
"""
import ctypes as C
import json
import re
from pathlib import Path

import numpy as np
import pytest

from mojoboost_amd import _lib
from mojoboost_amd._lib import lib, ptr

ROOT = Path(__file__).resolve().parent.parent


def declared(header):
    text = (ROOT / "include" / header).read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b((?:mojotrees|mbh)_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    L = lib()
    names = declared("mojotrees.h") + declared("mojoboost_hip.h")
    assert len(declared("mojotrees.h")) == 21
    for name in names:
        assert hasattr(L, name), name
    assert sorted(_lib.MOJOTREES_SYMBOLS) == declared("mojotrees.h")
    assert sorted(_lib.MBH_SYMBOLS) == declared("mojoboost_hip.h")


def test_versions_and_constants():
    L = lib()
    assert L.mojotrees_abi_version() == 3
    a, b, c = C.c_int32(-1), C.c_int32(-1), C.c_int32(-1)
    L.mojotrees_library_version(C.byref(a), C.byref(b), C.byref(c))
    assert min(a.value, b.value, c.value) >= 0
    L.mojotrees_library_version(None, None, None)
    assert L.mojotrees_gpu_available() in (0, 1)


def test_error_object_lifecycle():
    L = lib()
    e = L.mojotrees_error_create()
    assert L.mojotrees_error_message(e) == b""
    assert L.mojotrees_error_message(None) is None
    L.mojotrees_error_free(e)
    L.mojotrees_error_free(None)
    L.mojotrees_model_free(None)
    L.mojotrees_string_free(None)


def _train(params, data=None, labels=None, n=10, f=2, weights=None):
    L = lib()
    e = L.mojotrees_error_create()
    x = np.zeros(n * f) if data is None else data
    y = np.zeros(n) if labels is None else labels
    h = C.c_void_p()
    rc = L.mojotrees_train_dense(ptr(x), n, f, ptr(y), ptr(weights),
                                 None if params is None else params.encode(), C.byref(h), e)
    msg = L.mojotrees_error_message(e).decode()
    L.mojotrees_error_free(e)
    return rc, msg, h


def test_train_argument_errors():
    L = lib()
    e = L.mojotrees_error_create()
    h = C.c_void_p()
    rc = L.mojotrees_train_dense(None, 10, 2, None, None, None, C.byref(h), e)
    assert rc == _lib.ERROR_INVALID_ARGUMENT and h.value is None
    assert L.mojotrees_error_message(e) != b""
    L.mojotrees_error_free(e)
    assert _train("num_leaves=31", n=0)[0] == _lib.ERROR_INVALID_ARGUMENT


@pytest.mark.parametrize("params,code", [
    ("no_such_key=1", _lib.ERROR_INVALID_ARGUMENT),
    ("num_leaves", _lib.ERROR_INVALID_ARGUMENT),
    ("num_leaves=abc", _lib.ERROR_INVALID_ARGUMENT),
    ("num_class=3", _lib.ERROR_INVALID_ARGUMENT),
    ("objective=nonsense", _lib.ERROR_INVALID_ARGUMENT),
    ("device=cpu", _lib.ERROR_UNSUPPORTED),
    ("boosting=dart", _lib.ERROR_UNSUPPORTED),
    ("objective=poisson", _lib.ERROR_UNSUPPORTED),
    # GossParams.validate (goss.mojo:129-145), the cases of test_goss.mojo:217-241
    ("boosting=goss top_rate=1.5", _lib.ERROR_INVALID_ARGUMENT),
    ("boosting=goss top_rate=-0.1", _lib.ERROR_INVALID_ARGUMENT),
    ("boosting=goss other_rate=1.5", _lib.ERROR_INVALID_ARGUMENT),
    ("boosting=goss other_rate=-0.1", _lib.ERROR_INVALID_ARGUMENT),
    ("boosting=goss top_rate=0.7 other_rate=0.4", _lib.ERROR_INVALID_ARGUMENT),
    ("boosting=goss top_rate=0 other_rate=0", _lib.ERROR_INVALID_ARGUMENT),
    ("boosting=goss bagging_seed=-1", _lib.ERROR_INVALID_ARGUMENT),
    ("boosting=goss top_rate=0.9 other_rate=0.2", _lib.ERROR_INVALID_ARGUMENT),
    # lambdarank needs query groups, which only mbh_train_ranker_dense takes
    ("objective=lambdarank", _lib.ERROR_INVALID_ARGUMENT),
    ("sigmoid=abc", _lib.ERROR_INVALID_ARGUMENT),
    # _check_goss (boosting.mojo:346-355): GOSS and row bagging both own the row list
    ("boosting=goss bagging_fraction=0.5 bagging_freq=1", _lib.ERROR_INVALID_ARGUMENT),
])
def test_parameter_string_errors(params, code):
    rc, msg, h = _train(params)
    assert rc == code, (rc, msg)
    assert msg and h.value is None


def test_gpu_request_without_gpu_is_unsupported():
    if lib().mojotrees_gpu_available():
        pytest.skip("a GPU is present on this host")
    rc, msg, h = _train("device=gpu objective=binary")
    assert rc == _lib.ERROR_UNSUPPORTED and "gfx950" in msg and h.value is None


def test_gpu_predict_without_gpu_is_unsupported(tmp_path):
    if lib().mojotrees_gpu_available():
        pytest.skip("a GPU is present on this host")
    L = lib()
    path = tmp_path / "m.txt"
    write_model(path)
    rc, msg, h = _load(path)
    assert rc == 0
    x = np.zeros(12)
    out = np.zeros(6)
    e = L.mojotrees_error_create()
    assert L.mojotrees_predict_ex(h, ptr(x), 6, 2, 0, 0, 1, _lib.DEVICE_GPU, ptr(out), 6, e) == \
        _lib.ERROR_UNSUPPORTED
    assert b"gfx950" in L.mojotrees_error_message(e)
    # AUTO without a GPU predicts on the CPU
    assert L.mojotrees_predict_ex(h, ptr(x), 6, 2, 0, 0, 1, _lib.DEVICE_AUTO, ptr(out), 6, e) == 0
    L.mojotrees_error_free(e)
    L.mojotrees_model_free(h)


def test_parameter_keys():
    L = lib()
    out = C.c_char_p()
    e = L.mojotrees_error_create()
    assert L.mojotrees_parameter_keys(C.byref(out), e) == 0
    keys = out.value.decode().split(",")
    L.mojotrees_string_free(out)
    L.mojotrees_error_free(e)
    for k in ("objective", "num_leaves", "learning_rate", "use_quantized_grad",
              "num_grad_quant_bins", "device", "lambdarank_truncation_level", "sigmoid",
              "lambdarank_norm"):
        assert k in keys


def _bits(x):
    return str(np.float64(x).view(np.uint64))


def write_model(path, objective=1):
    """A two-tree v4 model over 2 features, in the reference's token format
    (serialize.mojo:485-545, :999-1037)."""
    edges = [-1.0, 0.0, 1.0, 0.5]          # feature 0: 3 edges, feature 1: 1 edge
    lines = ["mojotrees v4", f"objective {objective}", f"learning_rate {_bits(0.5)}",
             f"base_score {_bits(0.25)}", f"mapper 2 255 {len(edges)}",
             " ".join(_bits(e) for e in edges), "0 3 4", "-1 2", "trees 2",
             "tree 3 2", "0 -1 -1", "1 -1 -1", "1 -1 -1", "2 -1 -1",
             f"{_bits(0.0)} {_bits(-1.0)} {_bits(2.0)}", "1 0 0", "-1 -1 -1",
             "counts 1", f"{_bits(10.0)} {_bits(4.0)} {_bits(6.0)}",
             "gains 1", f"{_bits(3.5)} {_bits(0.0)} {_bits(0.0)}",
             "tree 1 1", "-1", "-1", "-1", "-1", _bits(0.125), "0", "-1",
             "counts 1", _bits(10.0), "gains 0"]
    Path(path).write_text("\n".join(lines) + "\n")


def _load(path):
    L = lib()
    e = L.mojotrees_error_create()
    h = C.c_void_p()
    rc = L.mojotrees_load_model(str(path).encode(), C.byref(h), e)
    msg = L.mojotrees_error_message(e).decode()
    L.mojotrees_error_free(e)
    return rc, msg, h


def test_model_file_predict_and_roundtrip(tmp_path):
    L = lib()
    p = tmp_path / "m.txt"
    write_model(p)
    rc, msg, h = _load(p)
    assert rc == 0, msg
    e = L.mojotrees_error_create()
    v = C.c_int64()
    assert L.mojotrees_model_num_features(h, C.byref(v), e) == 0 and v.value == 2
    assert L.mojotrees_model_num_trees(h, C.byref(v), e) == 0 and v.value == 2
    assert L.mojotrees_model_num_classes(h, C.byref(v), e) == 0 and v.value == 1
    assert L.mojotrees_model_num_iterations(h, C.byref(v), e) == 0 and v.value == 2
    # rows: feature 0 values; feature 1 irrelevant. NaN on f0 -> bin of 0.0
    x0 = np.array([-2.0, -0.5, 0.0, 0.3, 5.0, np.nan])
    x = np.concatenate([x0, np.zeros(6)])
    raw = np.zeros(6)
    assert L.mojotrees_predict_raw(h, ptr(x), 6, 2, ptr(raw), 6, e) == 0
    bins0 = np.array([0, 1, 1, 2, 3, 1])     # v <= edge -> first such edge
    leaf = np.where(bins0 <= 1, -1.0, 2.0)
    want = np.array([np.fma(0.5, 0.125, np.fma(0.5, l, 0.25)) if hasattr(np, "fma") else 0.0
                     for l in leaf])
    exact = [float(np.float64(0.25) + np.float64(0.5) * l + np.float64(0.5) * 0.125) for l in leaf]
    assert np.allclose(raw, exact, rtol=0, atol=1e-15)
    resp = np.zeros(6)
    assert L.mojotrees_predict(h, ptr(x), 6, 2, ptr(resp), 6, e) == 0
    assert np.allclose(resp, 1 / (1 + np.exp(-raw)), rtol=1e-12)
    # iteration ranges: [0,1) + [1,2) == full raw (base belongs to iteration 0)
    r0, r1 = np.zeros(6), np.zeros(6)
    assert L.mojotrees_predict_ex(h, ptr(x), 6, 2, 0, 1, 1, 0, ptr(r0), 6, e) == 0
    assert L.mojotrees_predict_ex(h, ptr(x), 6, 2, 1, 0, 1, 0, ptr(r1), 6, e) == 0
    assert np.allclose(r0 + r1, raw, atol=1e-15)
    # validation
    assert L.mojotrees_predict(h, ptr(x), 6, 3, ptr(resp), 6, e) == _lib.ERROR_INVALID_ARGUMENT
    assert L.mojotrees_predict(h, ptr(x), 6, 2, ptr(resp), 5, e) == _lib.ERROR_INVALID_ARGUMENT
    assert L.mojotrees_predict_ex(h, ptr(x), 6, 2, 0, 0, 7, 0, ptr(r0), 6, e) == _lib.ERROR_INVALID_ARGUMENT
    # importance
    imp = np.zeros(2)
    assert L.mojotrees_feature_importance(h, 0, ptr(imp), 2, e) == 0 and list(imp) == [1.0, 0.0]
    assert L.mojotrees_feature_importance(h, 1, ptr(imp), 2, e) == 0 and list(imp) == [3.5, 0.0]
    assert L.mojotrees_feature_importance(h, 9, ptr(imp), 2, e) == _lib.ERROR_INVALID_ARGUMENT
    # json
    out = C.c_char_p()
    assert L.mojotrees_model_dump_json(h, C.byref(out), e) == 0
    doc = json.loads(out.value.decode())
    L.mojotrees_string_free(out)
    assert doc["num_trees"] == 2 and doc["has_split_gain"] is True
    assert doc["trees"][0]["nodes"][0]["split_feature"] == 0
    # save -> load -> byte-identical file and predictions
    q = tmp_path / "sub" / "m2.txt"
    q.parent.mkdir()
    assert L.mojotrees_save_model(h, str(q).encode(), e) == 0
    rc, msg, h2 = _load(q)
    assert rc == 0, msg
    q2 = tmp_path / "m3.txt"
    assert L.mojotrees_save_model(h2, str(q2).encode(), e) == 0
    assert q.read_text() == q2.read_text()
    raw2 = np.zeros(6)
    assert L.mojotrees_predict_raw(h2, ptr(x), 6, 2, ptr(raw2), 6, e) == 0
    assert np.array_equal(raw, raw2)
    assert L.mojotrees_save_model(h, b"/dev/null/x/y", e) == _lib.ERROR_IO
    L.mojotrees_model_free(h)
    L.mojotrees_model_free(h2)
    L.mojotrees_error_free(e)


def test_load_errors(tmp_path):
    assert _load(tmp_path / "missing.txt")[0] == _lib.ERROR_IO
    bad = tmp_path / "bad.txt"
    bad.write_text("mojotrees v9\nobjective 1\n")
    rc, msg, h = _load(bad)
    assert rc == _lib.ERROR_IO and h.value is None
    trunc = tmp_path / "trunc.txt"
    write_model(trunc)
    trunc.write_text(trunc.read_text()[:-40])
    assert _load(trunc)[0] == _lib.ERROR_IO


def test_c_program_against_the_header(tmp_path):
    """tests/c/capi_program.c, compiled as C99 with -Werror against
    include/mojotrees.h and linked to the shared library, calls all 21
    functions on the CPU (the reference's capi/test_capi.c calls)."""
    import shutil
    import subprocess

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    exe = tmp_path / "capi_program"
    libdir = ROOT / "mojoboost_amd"
    subprocess.run([cc, "-std=c99", "-Wall", "-Wextra", "-Werror", "-pedantic",
                    "-I", str(ROOT / "include"), str(ROOT / "tests" / "c" / "capi_program.c"),
                    "-o", str(exe), "-L", str(libdir), "-lmojoboost_hip",
                    "-Wl,-rpath," + str(libdir), "-lm"], check=True)
    r = subprocess.run([str(exe), str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip() == "ok"
