"""Categorical features on the host side, without a GPU: the library's
category-table binning (mbh_bin_dense_cat) on the reference's binning cases
(tests/test_categorical.mojo:109-194), and the model file's `categorical` and
`cat` sections (src/mojotrees/serialize.mojo:533-566, :1196-1232) through the
C ABI: load, set routing in the host predictor, save byte for byte.
"""
import ctypes as C

import numpy as np
import pytest

from mojoboost_amd import _lib, device
from mojoboost_amd._lib import lib, ptr


def cat_bins(x_cm, n, f, categorical, max_bins=255):
    return device.bin_dense(np.asarray(x_cm, float), n, f, max_bins=max_bins, categorical=categorical)


def test_category_codes_map_to_bins_from_one():
    # test_categorical.mojo:109-118: bins follow ascending code order
    bins, mb, nc = cat_bins([7.0, 2.0, 5.0, 2.0, 7.0, 5.0], 6, 1, [0])
    assert nc.tolist() == [3] and mb.tolist() == [-1]
    assert bins.tolist() == [3, 1, 2, 1, 3, 2]


def test_missing_unseen_and_out_of_range_land_in_bin_zero():
    # test_categorical.mojo:121-133: fit on 0, 1, 2; then a second column
    # carries values the table never saw (transform is the same bin_of)
    x = np.array([0.0, 1.0, 2.0, 0.0, 1.0, 2.0, 9.0, -1.0, np.nan, 2.9], float)
    bins, _, nc = cat_bins(x, 10, 1, [0])
    assert nc.tolist() == [4]  # 0, 1, 2, 9 seen; 2.9 truncates to 2
    assert bins.tolist() == [1, 2, 3, 1, 2, 3, 4, 0, 0, 3]


def test_high_cardinality_keeps_the_most_frequent_categories():
    # test_categorical.mojo:136-151: code c appears 40 - c times; max_bins=11
    x = np.concatenate([np.full(40 - c, float(c)) for c in range(40)])
    bins, _, nc = cat_bins(x, len(x), 1, [0], max_bins=11)
    assert nc.tolist() == [10]
    want = np.where(x < 10, x + 1, 0).astype(np.uint8)
    assert np.array_equal(bins, want)


def test_categorical_binning_leaves_numerical_edges_untouched():
    # test_categorical.mojo:154-178
    n = 300
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.uniform(size=n), (np.arange(n) % 6).astype(float)])
    plain, _ = device.bin_dense(x, n, 2, max_bins=32)
    mixed, mb, nc = cat_bins(x, n, 2, [1], max_bins=32)
    assert np.array_equal(mixed[:n], plain[:n])
    assert np.array_equal(mixed[n:], (np.arange(n) % 6 + 1).astype(np.uint8))
    assert nc.tolist() == [0, 6]


@pytest.mark.parametrize("cats,values", [([2], None), ([-1], None), ([0, 0], None),
                                         ([0], [0.0, 5.0e9])])
def test_categorical_marking_is_validated(cats, values):
    # test_categorical.mojo:181-193
    x = np.array(values if values is not None else [0.0, 1.0, 0.0, 1.0])
    f = 1 if values is not None else 2
    with pytest.raises(_lib.MojoTreesError):
        cat_bins(x, len(x) // f, f, cats)


MODEL = """mojotrees v4
objective 0
learning_rate {lr}
base_score {base}
mapper 2 255 1
{edge}
0 1 1
-1 -1
categorical 2 3
0 1
10 20 30
0 0 3
trees 1
tree 5 3
1 -1 0 -1 -1
-1 -1 0 -1 -1
1 -1 3 -1 -1
2 -1 4 -1 -1
0 {v1} 0 {v3} {v4}
0 0 0 0 0
-1 -1 -1 -1 -1
counts 0
gains 0
cat 4
0 -1 -1 -1 -1
{bits} 0 0 0
"""


def bits(x):
    return str(np.float64(x).view(np.uint64))


def test_model_file_with_category_sets_loads_routes_and_saves(tmp_path):
    # node 0 splits feature 1 by the set {bin 1, bin 3} (codes 10 and 30);
    # everything else, missing and unseen codes included, goes right
    text = MODEL.format(lr=bits(0.5), base=bits(1.0), edge=bits(0.25), v1=bits(2.0),
                        v3=bits(-4.0), v4=bits(8.0), bits=(1 << 1) | (1 << 3))
    src = tmp_path / "cat.model"
    src.write_text(text)
    L = lib()
    e = L.mojotrees_error_create()
    h = C.c_void_p()
    assert L.mojotrees_load_model(str(src).encode(), C.byref(h), e) == 0, L.mojotrees_error_message(e)
    # rows: (f0, f1) -- code 10 left, 20 right, 30 left, 99 unseen right,
    # NaN right, -3 right; then node 2 splits f0 at 0.25
    f0 = np.array([0.0, 0.0, 1.0, 0.0, 1.0, 0.0])
    f1 = np.array([10.0, 20.0, 30.0, 99.0, np.nan, -3.0])
    x = np.concatenate([f0, f1])
    out = np.zeros(6)
    rc = L.mojotrees_predict_ex(h, ptr(x), 6, 2, 0, 0, _lib.PREDICT_RAW, _lib.DEVICE_CPU, ptr(out), 6, e)
    assert rc == 0, L.mojotrees_error_message(e)
    right = np.where(f0 <= 0.25, -4.0, 8.0)
    want = 1.0 + 0.5 * np.where(np.isin(f1, [10.0, 30.0]), 2.0, right)
    assert np.array_equal(out, want)
    dst = tmp_path / "again.model"
    assert L.mojotrees_save_model(h, str(dst).encode(), e) == 0
    assert dst.read_text().split() == text.split()
    s = C.c_void_p()
    assert L.mojotrees_model_dump_json(h, C.byref(s), e) == 0
    dump = C.cast(s, C.c_char_p).value.decode()
    assert '"categories_left":[10,30]' in dump
    L.mojotrees_string_free(s)
    L.mojotrees_model_free(h)
    L.mojotrees_error_free(e)


def test_corrupt_categorical_sections_are_refused(tmp_path):
    text = MODEL.format(lr=bits(0.5), base=bits(1.0), edge=bits(0.25), v1=bits(2.0),
                        v3=bits(-4.0), v4=bits(8.0), bits=2)
    L = lib()
    e = L.mojotrees_error_create()
    for bad in (text.replace("10 20 30", "10 30 20"),           # codes not ascending
                text.replace("0 1\n10", "1 0\n10"),              # table on a numerical feature
                text.replace("0 -1 -1 -1 -1\n", "8 -1 -1 -1 -1\n")):  # set offset past the pool
        p = tmp_path / "bad.model"
        p.write_text(bad)
        h = C.c_void_p()
        assert L.mojotrees_load_model(str(p).encode(), C.byref(h), e) != 0
        assert h.value is None
    L.mojotrees_error_free(e)


def test_categorical_parameters_are_accepted_and_checked():
    L = lib()
    e = L.mojotrees_error_create()
    keys = C.c_void_p()
    assert L.mojotrees_parameter_keys(C.byref(keys), e) == 0
    names = C.cast(keys, C.c_char_p).value.decode()
    for k in ("categorical_feature", "max_cat_to_onehot", "max_cat_threshold", "cat_smooth",
              "cat_l2", "min_data_per_group", "one_hot_max_size"):
        assert k in names
    L.mojotrees_string_free(keys)
    x = np.zeros(20)
    y = np.zeros(10)
    h = C.c_void_p()
    rc = L.mojotrees_train_dense(ptr(x), 10, 2, ptr(y), None, b"categorical_feature=5", C.byref(h), e)
    assert rc == _lib.ERROR_INVALID_ARGUMENT and h.value is None
    L.mojotrees_error_free(e)
