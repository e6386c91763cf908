"""ctypes binding to libmojoboost_hip.so (the HIP library in this package).

The library is built in-tree by `__graft_entry__.build()` (or
`make -C mojoboost_amd/csrc`). Loading fails loudly when it is missing:
there is no fallback implementation behind these calls.
"""
import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libmojoboost_hip.so"

OK = 0
ERROR_INVALID_ARGUMENT = -1
ERROR_TRAINING = -2
ERROR_IO = -3
ERROR_UNSUPPORTED = -4
DEVICE_CPU, DEVICE_GPU, DEVICE_AUTO = 0, 1, 2
PREDICT_RESPONSE, PREDICT_RAW = 0, 1
IMPORTANCE_SPLIT, IMPORTANCE_GAIN = 0, 1
OBJ_REGRESSION, OBJ_BINARY, OBJ_MULTICLASS, OBJ_LAMBDARANK = 0, 1, 2, 3

# Every symbol include/mojotrees.h and include/mojoboost_hip.h declare.
MOJOTREES_SYMBOLS = [
    "mojotrees_abi_version", "mojotrees_library_version", "mojotrees_gpu_available",
    "mojotrees_error_create", "mojotrees_error_free", "mojotrees_error_message",
    "mojotrees_train_dense", "mojotrees_predict", "mojotrees_predict_raw",
    "mojotrees_predict_ex", "mojotrees_save_model", "mojotrees_load_model",
    "mojotrees_model_num_features", "mojotrees_model_num_classes",
    "mojotrees_model_num_trees", "mojotrees_model_num_iterations",
    "mojotrees_model_dump_json", "mojotrees_feature_importance",
    "mojotrees_parameter_keys", "mojotrees_string_free", "mojotrees_model_free",
]
MBH_SYMBOLS = [
    "mbh_bin_dense", "mbh_device_count", "mbh_dataset_create", "mbh_dataset_free", "mbh_train",
    "mbh_fit_free", "mbh_fit_num_trees", "mbh_fit_num_class", "mbh_fit_total_nodes",
    "mbh_fit_arrays", "mbh_fit_train_raw", "mbh_fit_stats", "mbh_exp_sigmoid",
    "mbh_objective_quantize", "mbh_histogram", "mbh_histogram_fp32", "mbh_bench_root_histogram",
    "mbh_predict_binned", "mbh_dataset_set_groups", "mbh_lambdarank", "mbh_train_ranker_dense",
    "mbh_bin_dense_cat", "mbh_dataset_set_categorical", "mbh_fit_cat_bits", "mbh_dataset_set_weights",
    "mbh_histogram_noalloc", "mbh_save_model_named", "mbh_model_feature_names",
    "mbh_objective_quantize32", "mbh_histogram32", "mbh_bin_dense_device", "mbh_fit_launch_log",
]


class MbhParams(C.Structure):
    _fields_ = [
        ("objective", C.c_int32),
        ("num_class", C.c_int32),
        ("num_iterations", C.c_int32),
        ("learning_rate", C.c_double),
        ("num_leaves", C.c_int32),
        ("min_data_in_leaf", C.c_int32),
        ("lambda_l1", C.c_double),
        ("lambda_l2", C.c_double),
        ("min_sum_hessian", C.c_double),
        ("max_depth", C.c_int32),
        ("feature_fraction", C.c_double),
        ("feature_fraction_seed", C.c_int32),
        ("bagging_fraction", C.c_double),
        ("bagging_freq", C.c_int32),
        ("bagging_seed", C.c_int32),
        ("num_grad_quant_bins", C.c_int32),
        ("stochastic_rounding", C.c_int32),
        ("quant_seed", C.c_int32),
        ("time_histograms", C.c_int32),
        ("use_quantized_grad", C.c_int32),
        ("goss", C.c_int32),
        ("top_rate", C.c_double),
        ("other_rate", C.c_double),
        ("goss_band", C.c_double),
        ("goss_exact_walk", C.c_int32),
        ("lambdarank_truncation_level", C.c_int32),
        ("lambdarank_norm", C.c_int32),
        ("lambdarank_sigmoid", C.c_double),
        ("max_cat_to_onehot", C.c_int32),
        ("max_cat_threshold", C.c_int32),
        ("cat_smooth", C.c_double),
        ("cat_l2", C.c_double),
        ("min_data_per_group", C.c_int32),
        ("one_hot_max_size", C.c_int32),
        ("quant_scale_rule", C.c_int32),
        ("quant_staging", C.c_int32),
        ("partition_mode", C.c_int32),
    ]


def mbh_params(**kw) -> MbhParams:
    p = MbhParams(objective=OBJ_REGRESSION, num_class=1, num_iterations=100,
                  learning_rate=0.1, num_leaves=31, min_data_in_leaf=20, lambda_l1=0.0,
                  lambda_l2=1.0, min_sum_hessian=1e-3, max_depth=-1, feature_fraction=1.0,
                  feature_fraction_seed=2, bagging_fraction=1.0, bagging_freq=0,
                  bagging_seed=3, num_grad_quant_bins=4, stochastic_rounding=1,
                  quant_seed=11, time_histograms=0, use_quantized_grad=1, goss=0,
                  top_rate=0.2, other_rate=0.1, goss_band=6.0, goss_exact_walk=0,
                  lambdarank_truncation_level=30, lambdarank_norm=1, lambdarank_sigmoid=1.0,
                  max_cat_to_onehot=4, max_cat_threshold=32, cat_smooth=10.0, cat_l2=10.0,
                  min_data_per_group=100, one_hot_max_size=-1, quant_scale_rule=0,
                  quant_staging=0, partition_mode=0)
    for k, v in kw.items():
        setattr(p, k, v)
    return p


class MojoTreesError(Exception):
    def __init__(self, code, message):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


_lib = None


def lib():
    """Load the HIP library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
            "(hipcc --offload-arch=gfx950); there is no CPU fallback")
    L = C.CDLL(str(LIB_PATH))
    P, V, I32, I64, D = C.POINTER, C.c_void_p, C.c_int32, C.c_int64, C.c_double
    sig = {
        "mojotrees_abi_version": (I32, []),
        "mojotrees_library_version": (None, [V, V, V]),
        "mojotrees_gpu_available": (I32, []),
        "mojotrees_error_create": (V, []),
        "mojotrees_error_free": (None, [V]),
        "mojotrees_error_message": (C.c_char_p, [V]),
        "mojotrees_train_dense": (I32, [V, I64, I64, V, V, C.c_char_p, V, V]),
        "mojotrees_predict": (I32, [V, V, I64, I64, V, I64, V]),
        "mojotrees_predict_raw": (I32, [V, V, I64, I64, V, I64, V]),
        "mojotrees_predict_ex": (I32, [V, V, I64, I64, I64, I64, I32, I32, V, I64, V]),
        "mojotrees_save_model": (I32, [V, C.c_char_p, V]),
        "mojotrees_load_model": (I32, [C.c_char_p, V, V]),
        "mojotrees_model_num_features": (I32, [V, V, V]),
        "mojotrees_model_num_classes": (I32, [V, V, V]),
        "mojotrees_model_num_trees": (I32, [V, V, V]),
        "mojotrees_model_num_iterations": (I32, [V, V, V]),
        "mojotrees_model_dump_json": (I32, [V, V, V]),
        "mojotrees_feature_importance": (I32, [V, I32, V, I64, V]),
        "mojotrees_parameter_keys": (I32, [V, V]),
        "mojotrees_string_free": (None, [V]),
        "mojotrees_model_free": (None, [V]),
        "mbh_bin_dense": (I32, [V, I64, I32, I32, I32, I32, I64, I64, V, V, C.c_char_p, I32]),
        "mbh_device_count": (I32, []),
        "mbh_dataset_create": (I32, [V, I64, I32, I32, V, V, V, C.c_char_p, I32]),
        "mbh_dataset_free": (None, [V]),
        "mbh_train": (I32, [V, P(MbhParams), V, C.c_char_p, I32]),
        "mbh_fit_free": (None, [V]),
        "mbh_fit_num_trees": (I32, [V]),
        "mbh_fit_num_class": (I32, [V]),
        "mbh_fit_total_nodes": (I64, [V]),
        "mbh_fit_arrays": (None, [V] * 12),
        "mbh_fit_train_raw": (I32, [V, V, C.c_char_p, I32]),
        "mbh_fit_stats": (I32, [V, V, I32]),
        "mbh_fit_launch_log": (I64, [V, V, I64]),
        "mbh_exp_sigmoid": (I32, [V, I64, V, V, C.c_char_p, I32]),
        "mbh_objective_quantize": (I32, [V, P(MbhParams), V, I64, V, V, V, V, V, C.c_char_p, I32]),
        "mbh_histogram": (I32, [V, V, V, V, I64, I32, V, C.c_char_p, I32]),
        "mbh_objective_quantize32": (I32, [V, P(MbhParams), V, I64, V, V, V, V, V, C.c_char_p, I32]),
        "mbh_histogram32": (I32, [V, V, V, V, I64, V, C.c_char_p, I32]),
        "mbh_histogram_fp32": (I32, [V, V, V, V, I64, V, V, C.c_char_p, I32]),
        "mbh_histogram_noalloc": (I32, [V, I64, I32, I32, V, V, V, I64, I32, V, V, V, C.c_char_p, I32]),
        "mbh_bench_root_histogram": (I32, [V, I32, V, C.c_char_p, I32]),
        "mbh_predict_binned": (I32, [V, I64, I32, I32, C.c_double, V, V, I64, I64, V, V, V, V, V, V, V,
                                     V, V, C.c_char_p, I32]),
        "mbh_bin_dense_cat": (I32, [V, I64, I32, I32, I32, I32, I64, I64, V, I32, V, V, V,
                                    C.c_char_p, I32]),
        "mbh_bin_dense_device": (I32, [V, I64, I32, I32, I32, I32, I64, I64, V, I32, V, V, V, V,
                                       C.c_char_p, I32]),
        "mbh_dataset_set_categorical": (I32, [V, V, C.c_char_p, I32]),
        "mbh_fit_cat_bits": (None, [V, V]),
        "mbh_dataset_set_groups": (I32, [V, V, I64, C.c_char_p, I32]),
        "mbh_dataset_set_weights": (I32, [V, V, I64, C.c_char_p, I32]),
        "mbh_lambdarank": (I32, [V, P(MbhParams), V, V, V, C.c_char_p, I32]),
        "mbh_train_ranker_dense": (I32, [V, I64, I64, V, V, V, I64, C.c_char_p, V, V]),
        "mbh_save_model_named": (I32, [V, C.c_char_p, V, I64, V]),
        "mbh_model_feature_names": (I32, [C.c_char_p, V, V, V]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def check(rc, errbuf):
    if rc != OK:
        raise MojoTreesError(rc, errbuf.value.decode(errors="replace"))
