"""Model files the reference writes, read by this library on the CPU.

The reference's reader accepts v1 through v4 (serialize._read_version,
src/mojotrees/serialize.mojo:1372-1398) and its writer emits an optional v4
`feature_names` section right after the version token (serialize.mojo:
389-415) whenever its estimators know the column names. The cases below are
the reference's own: the literal v1 file of tests/test_serialize.mojo:246-270
with its expected predictions (1.0 + 0.5 * 10 and 1.0 + 0.5 * 20), and
hand-written v2, v3 and v4 files laid out as serialize.mojo's readers read
them (v3 covers without a presence flag, v4 flags for covers and gains, the
name escapes of _escape_name :276-319).
"""
import ctypes as C
import struct

import numpy as np
import pytest

from mojoboost_amd import _lib
from mojoboost_amd._lib import lib, ptr
from mojoboost_amd.sklearn import MojoTreesRegressor, _Booster


def _bits(x):
    return str(struct.unpack("<Q", struct.pack("<d", float(x)))[0])


def _load(path):
    L = lib()
    e = L.mojotrees_error_create()
    h = C.c_void_p()
    rc = L.mojotrees_load_model(str(path).encode(), C.byref(h), e)
    msg = L.mojotrees_error_message(e).decode()
    L.mojotrees_error_free(e)
    return rc, msg, h


def _predict(h, x, n, f):
    L = lib()
    e = L.mojotrees_error_create()
    out = np.zeros(n)
    x = np.ascontiguousarray(x, np.float64)
    rc = L.mojotrees_predict(h, ptr(x), n, f, ptr(out), n, e)
    L.mojotrees_error_free(e)
    assert rc == 0
    return out


def _v1_text():
    """tests/test_serialize.mojo:246-270, token for token."""
    s = "mojotrees v1\nobjective 0\n"
    s += "learning_rate " + _bits(0.5) + "\n"
    s += "base_score " + _bits(1.0) + "\n"
    s += "mapper 1 4 1\n"
    s += _bits(2.0) + "\n"
    s += "0 1\n"
    s += "trees 1\n"
    s += "tree 3 2\n"
    s += "0 -1 -1\n"
    s += "0 -1 -1\n"
    s += "1 -1 -1\n"
    s += "2 -1 -1\n"
    s += _bits(0.0) + " " + _bits(10.0) + " " + _bits(20.0) + "\n"
    return s


def test_loads_the_reference_v1_file(tmp_path):
    p = tmp_path / "v1.txt"
    p.write_text(_v1_text())
    rc, msg, h = _load(p)
    assert rc == 0, msg
    # values <= 2.0 take the left leaf, above it the right one, each scaled by
    # the learning rate on top of the base score
    out = _predict(h, [1.0, 3.0], 2, 1)
    assert out[0] == 1.0 + 0.5 * 10.0
    assert out[1] == 1.0 + 0.5 * 20.0
    # v1 reserves no missing bin: NaN lands in the bin of 0.0 (the left leaf)
    assert _predict(h, [np.nan], 1, 1)[0] == 1.0 + 0.5 * 10.0
    lib().mojotrees_model_free(h)


def _v4_named_text(names_tokens, n_features=2):
    s = "mojotrees v4\n"
    if names_tokens is not None:
        s += f"feature_names {len(names_tokens)}\n" + " ".join(names_tokens) + " \n"
    s += "objective 0\n"
    s += "learning_rate " + _bits(0.5) + "\nbase_score " + _bits(1.0) + "\n"
    s += f"mapper {n_features} 4 {n_features}\n"
    s += " ".join(_bits(2.0) for _ in range(n_features)) + "\n"
    s += " ".join(str(i) for i in range(n_features + 1)) + "\n"
    s += " ".join("-1" for _ in range(n_features)) + "\n"
    s += "trees 1\ntree 3 2\n"
    s += "1 -1 -1\n0 -1 -1\n1 -1 -1\n2 -1 -1\n"
    s += _bits(0.0) + " " + _bits(10.0) + " " + _bits(20.0) + "\n"
    s += "0 0 0\n-1 -1 -1\n"
    s += "counts 1\n" + " ".join(_bits(c) for c in (7.0, 3.0, 4.0)) + "\n"
    s += "gains 1\n" + " ".join(_bits(g) for g in (1.5, 0.0, 0.0)) + "\n"
    return s


def test_loads_a_v4_file_with_feature_names(tmp_path):
    # escapes of serialize._escape_name: space, backslash, empty name
    tokens = ["my\\sfeature", "back\\\\slash"]
    p = tmp_path / "named.txt"
    p.write_text(_v4_named_text(tokens))
    rc, msg, h = _load(p)
    assert rc == 0, msg
    # the split is on feature 1
    out = _predict(h, np.array([0.0, 0.0, 1.0, 3.0]), 2, 2)
    assert list(out) == [1.0 + 0.5 * 10.0, 1.0 + 0.5 * 20.0]
    assert _Booster.feature_names(p) == ["my feature", "back\\slash"]
    # the C ABI's model carries no names (serialize.load_model drops them),
    # so its save writes none
    q = tmp_path / "resaved.txt"
    e = lib().mojotrees_error_create()
    assert lib().mojotrees_save_model(h, str(q).encode(), e) == 0
    lib().mojotrees_error_free(e)
    assert _Booster.feature_names(q) == []
    assert q.read_text().splitlines()[1].startswith("objective")
    lib().mojotrees_model_free(h)


def test_named_save_round_trip(tmp_path):
    p = tmp_path / "plain.txt"
    p.write_text(_v4_named_text(None))
    b = _Booster.load(p)
    names = ["", "tab\there", "nl\nx", "cr\rx", "üñí cödé"]
    q = tmp_path / "n.txt"
    with pytest.raises(_lib.MojoTreesError):   # 5 names for 2 features
        b.save(q, names)
    b.save(q, names[3:])
    assert _Booster.feature_names(q) == names[3:]
    b.save(q, names[:2])
    assert _Booster.feature_names(q) == names[:2]
    assert q.read_text().splitlines()[1:3] == ["feature_names 2", "\\e tab\\there "]
    # a control byte other than the escaped whitespace is refused
    with pytest.raises(_lib.MojoTreesError):
        b.save(q, ["a\x01", "b"])
    # loads and predicts as the unnamed file does
    b2 = _Booster.load(q)
    x = np.array([[0.0, 1.0], [0.0, 3.0]])
    assert np.array_equal(b.predict(x), b2.predict(x))


def test_estimator_load_restores_feature_names(tmp_path):
    p = tmp_path / "named.txt"
    p.write_text(_v4_named_text(["a", "b"]))
    est = MojoTreesRegressor.load(p)
    assert list(est.feature_names_in_) == ["a", "b"]
    q = tmp_path / "again.txt"
    est.save(q)
    assert _Booster.feature_names(q) == ["a", "b"]
    p2 = tmp_path / "plain.txt"
    p2.write_text(_v4_named_text(None))
    assert not hasattr(MojoTreesRegressor.load(p2), "feature_names_in_")


def test_feature_names_count_must_match_the_mapper(tmp_path):
    p = tmp_path / "bad.txt"
    p.write_text(_v4_named_text(["a", "b", "c"]))
    rc, msg, _ = _load(p)
    assert rc == _lib.ERROR_IO and "feature_names" in msg
    p.write_text(_v4_named_text(["a\\qb", "c"]))   # unknown escape
    assert _load(p)[0] == _lib.ERROR_IO


def _v2_v3_text(version):
    """A v2 file (missing routing, no covers) and a v3 file (covers with no
    presence flag, serialize._read_trees :1300-1320), with a monotone
    section between the mapper and the trees."""
    s = f"mojotrees {version}\nobjective 0\n"
    s += "learning_rate " + _bits(0.5) + "\nbase_score " + _bits(1.0) + "\n"
    s += "mapper 1 5 1\n" + _bits(2.0) + "\n0 1\n2\n"   # missing bin 2
    s += "monotone 1 1\n"
    s += "trees 1\ntree 3 2\n0 -1 -1\n0 -1 -1\n1 -1 -1\n2 -1 -1\n"
    s += _bits(0.0) + " " + _bits(10.0) + " " + _bits(20.0) + "\n"
    s += "0 0 0\n2 -1 -1\n"        # default_left false: NaN goes right
    if version == "v3":
        s += " ".join(_bits(c) for c in (9.0, 4.0, 5.0)) + "\n"
    return s


@pytest.mark.parametrize("version", ["v2", "v3"])
def test_loads_v2_and_v3_files(tmp_path, version):
    p = tmp_path / "m.txt"
    p.write_text(_v2_v3_text(version))
    rc, msg, h = _load(p)
    assert rc == 0, msg
    out = _predict(h, [1.0, 3.0, np.nan], 3, 1)
    assert list(out) == [6.0, 11.0, 11.0]
    # re-saved as v4: covers flagged (v3) or absent (v2), monotone kept
    q = tmp_path / "v4.txt"
    e = lib().mojotrees_error_create()
    assert lib().mojotrees_save_model(h, str(q).encode(), e) == 0
    lib().mojotrees_error_free(e)
    text = q.read_text()
    assert text.startswith("mojotrees v4\n")
    assert "monotone 1 1\n" in text
    assert ("counts 1\n" in text) == (version == "v3")
    rc, msg, h2 = _load(q)
    assert rc == 0, msg
    assert np.array_equal(_predict(h2, [1.0, 3.0, np.nan], 3, 1), out)
    lib().mojotrees_model_free(h)
    lib().mojotrees_model_free(h2)


def test_version_and_section_errors(tmp_path):
    p = tmp_path / "m.txt"
    p.write_text(_v1_text().replace("v1", "v5", 1))
    rc, msg, _ = _load(p)
    assert rc == _lib.ERROR_IO and "v5" in msg
    p.write_text(_v1_text().replace("v1", "v99", 1))
    assert _load(p)[0] == _lib.ERROR_IO
    # a v2 file must carry the missing bins that v1 lacks
    p.write_text(_v1_text().replace("v1", "v2", 1))
    assert _load(p)[0] == _lib.ERROR_IO
    # more nodes than a binary tree with that many leaves can hold
    p.write_text(_v1_text().replace("tree 3 2", "tree 3 1"))
    assert _load(p)[0] == _lib.ERROR_IO
    # v4 covers: all zero means none, a mix of zero and positive is corrupt
    p.write_text(_v4_named_text(None).replace(
        "counts 1\n" + " ".join(_bits(c) for c in (7.0, 3.0, 4.0)),
        "counts 1\n" + " ".join(_bits(c) for c in (7.0, 0.0, 4.0))))
    assert _load(p)[0] == _lib.ERROR_IO
    p.write_text(_v4_named_text(None).replace(
        "counts 1\n" + " ".join(_bits(c) for c in (7.0, 3.0, 4.0)),
        "counts 1\n" + " ".join(_bits(c) for c in (0.0, 0.0, 0.0))))
    assert _load(p)[0] == 0


@pytest.mark.gpu
def test_estimator_fit_on_named_columns_saves_the_names(tmp_path):
    """A DataFrame's column names become feature_names_in_ at fit, travel in
    the v4 file's feature_names section, and come back on load, as the
    reference's estimators do (python/mojotrees/sklearn.py:6140-6170)."""
    pd = pytest.importorskip("pandas")
    from mojoboost_amd import device

    if device.device_count() < 1:
        pytest.skip("no gfx950 GPU")
    rng = np.random.default_rng(5)
    X = pd.DataFrame(rng.normal(size=(3000, 3)), columns=["alpha", "beta gamma", "δ"])
    y = X["alpha"].to_numpy() * 2.0 + rng.normal(size=3000) * 0.1
    est = MojoTreesRegressor(n_estimators=5, num_leaves=7, device="gpu").fit(X, y)
    assert list(est.feature_names_in_) == ["alpha", "beta gamma", "δ"]
    p = tmp_path / "m.txt"
    est.save(p)
    back = MojoTreesRegressor.load(p)
    assert list(back.feature_names_in_) == ["alpha", "beta gamma", "δ"]
    assert np.array_equal(back.predict(X.to_numpy()), est.predict(X.to_numpy()))
    # a plain array leaves no names behind
    est.fit(X.to_numpy(), y)
    assert not hasattr(est, "feature_names_in_")
