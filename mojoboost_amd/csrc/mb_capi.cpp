// The mojotrees C ABI (include/mojotrees.h) over the device trainer.
//
// Follows the reference implementation's contract
// (capi/mojotrees_capi.mojo:325-895, capi/README.md): parameter strings with
// LightGBM names and aliases, an unknown key is INVALID_ARGUMENT, a known
// feature the path does not serve is UNSUPPORTED, errors are cleared on
// entry, `out_*` arguments are written only on success.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <new>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/mojoboost_hip.h"
#include "../../include/mojotrees.h"
#include "mb_host.h"

struct MojoTreesError {
    std::string message;
};

struct MojoTreesModel {
    mb::Model m;
};

namespace {

struct ApiError {
    int32_t code;
    std::string msg;
};

void clear(MojoTreesError *e) {
    if (e) e->message.clear();
}

int32_t fail(MojoTreesError *e, int32_t code, const std::string &msg) {
    if (e) e->message = msg;
    return code;
}

// Canonical key for every accepted name (capi/README.md:83-103, plus the
// LightGBM keys of the quantized-gradient and bagging paths,
// src/mojotrees/params.mojo:1388-1401).
const std::map<std::string, std::string> &aliases() {
    static const std::map<std::string, std::string> a = {
        {"objective", "objective"},
        {"application", "objective"},
        {"num_class", "num_class"},
        {"num_classes", "num_class"},
        {"num_iterations", "num_iterations"},
        {"n_estimators", "num_iterations"},
        {"num_round", "num_iterations"},
        {"num_boost_round", "num_iterations"},
        {"learning_rate", "learning_rate"},
        {"eta", "learning_rate"},
        {"shrinkage_rate", "learning_rate"},
        {"num_leaves", "num_leaves"},
        {"num_leaf", "num_leaves"},
        {"min_data_in_leaf", "min_data_in_leaf"},
        {"min_data", "min_data_in_leaf"},
        {"min_child_samples", "min_data_in_leaf"},
        {"min_sum_hessian_in_leaf", "min_sum_hessian_in_leaf"},
        {"min_child_weight", "min_sum_hessian_in_leaf"},
        {"min_sum_hessian", "min_sum_hessian_in_leaf"},
        {"lambda_l1", "lambda_l1"},
        {"reg_alpha", "lambda_l1"},
        {"lambda_l2", "lambda_l2"},
        {"reg_lambda", "lambda_l2"},
        {"lambda", "lambda_l2"},
        {"max_depth", "max_depth"},
        {"feature_fraction", "feature_fraction"},
        {"sub_feature", "feature_fraction"},
        {"colsample_bytree", "feature_fraction"},
        {"feature_fraction_bynode", "feature_fraction_bynode"},
        {"colsample_bynode", "feature_fraction_bynode"},
        {"feature_fraction_seed", "feature_fraction_seed"},
        {"max_bin", "max_bin"},
        {"alpha", "alpha"},
        {"device", "device"},
        {"device_type", "device"},
        {"use_missing", "use_missing"},
        {"use_quantized_grad", "use_quantized_grad"},
        {"num_grad_quant_bins", "num_grad_quant_bins"},
        {"stochastic_rounding", "stochastic_rounding"},
        {"quant_scale_rule", "quant_scale_rule"},
        {"quant_staging", "quant_staging"},
        {"bagging_fraction", "bagging_fraction"},
        {"subsample", "bagging_fraction"},
        {"bagging_freq", "bagging_freq"},
        {"subsample_freq", "bagging_freq"},
        {"bagging_seed", "bagging_seed"},
        {"boosting", "boosting"},
        {"boosting_type", "boosting"},
        {"top_rate", "top_rate"},
        {"other_rate", "other_rate"},
        {"min_data_in_bin", "min_data_in_bin"},
        {"bin_construct_sample_cnt", "bin_construct_sample_cnt"},
        {"data_random_seed", "data_random_seed"},
        {"lambdarank_truncation_level", "lambdarank_truncation_level"},
        {"sigmoid", "sigmoid"},
        {"lambdarank_norm", "lambdarank_norm"},
        // categorical features (LightGBM names; categorical.mojo:164-240)
        {"categorical_feature", "categorical_feature"},
        {"categorical_features", "categorical_feature"},
        {"cat_features", "categorical_feature"},
        {"categorical_column", "categorical_feature"},
        {"cat_feature", "categorical_feature"},
        {"max_cat_to_onehot", "max_cat_to_onehot"},
        {"max_cat_threshold", "max_cat_threshold"},
        {"cat_smooth", "cat_smooth"},
        {"cat_l2", "cat_l2"},
        {"min_data_per_group", "min_data_per_group"},
        {"one_hot_max_size", "one_hot_max_size"},
    };
    return a;
}

const char *kPrimaryKeys =
    "objective,num_class,num_iterations,learning_rate,num_leaves,min_data_in_leaf,"
    "min_sum_hessian_in_leaf,lambda_l1,lambda_l2,max_depth,feature_fraction,"
    "feature_fraction_bynode,feature_fraction_seed,max_bin,alpha,device,use_missing,"
    "use_quantized_grad,num_grad_quant_bins,stochastic_rounding,bagging_fraction,"
    "bagging_freq,bagging_seed,boosting,top_rate,other_rate,min_data_in_bin,"
    "bin_construct_sample_cnt,data_random_seed,lambdarank_truncation_level,sigmoid,lambdarank_norm,"
    "categorical_feature,max_cat_to_onehot,max_cat_threshold,cat_smooth,cat_l2,min_data_per_group,"
    "one_hot_max_size,quant_scale_rule,quant_staging";

struct Config {
    mbh_params p{};
    int device = MOJOTREES_DEVICE_AUTO;
    int max_bin = 255;
    int min_data_in_bin = 3;
    int64_t bin_sample = 200000;
    int64_t data_seed = 1;
    bool use_missing = true;
    bool quantized = false;  // LightGBM's default; the reference trains unquantized
    int num_class = 1;
    bool saw_num_class = false;
    std::vector<int> categorical;  // categorical_feature: column indices
};

double to_double(const std::string &k, const std::string &v) {
    char *end = nullptr;
    double d = std::strtod(v.c_str(), &end);
    if (v.empty() || *end) throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "parameter " + k + ": '" + v + "' is not a number"};
    return d;
}

int64_t to_int(const std::string &k, const std::string &v) {
    char *end = nullptr;
    long long d = std::strtoll(v.c_str(), &end, 10);
    if (v.empty() || *end) throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "parameter " + k + ": '" + v + "' is not an integer"};
    return d;
}

bool to_bool(const std::string &k, const std::string &v) {
    std::string s = v;
    std::transform(s.begin(), s.end(), s.begin(), ::tolower);
    if (s == "true" || s == "1") return true;
    if (s == "false" || s == "0") return false;
    throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "parameter " + k + ": '" + v + "' is not a boolean"};
}

Config parse(const char *spec) {
    Config c;
    mbh_params &p = c.p;
    // defaults: BoosterParams.default() / TreeParams.default()
    // (src/mojotrees/boosting.mojo:1611, src/mojotrees/tree.mojo:284)
    p.objective = MBH_OBJ_REGRESSION;
    p.num_class = 1;
    p.goss = 0;
    p.goss_band = 6.0;
    p.goss_exact_walk = 0;
    p.top_rate = 0.2;    // LightGBM / GossParams defaults
    p.other_rate = 0.1;
    p.num_iterations = 100;
    p.learning_rate = 0.1;
    p.num_leaves = 31;
    p.min_data_in_leaf = 20;
    p.lambda_l1 = 0.0;
    p.lambda_l2 = 1.0;
    p.min_sum_hessian = 1e-3;
    p.max_depth = -1;
    p.feature_fraction = 1.0;
    p.feature_fraction_seed = 2;
    p.bagging_fraction = 1.0;
    p.bagging_freq = 0;
    p.bagging_seed = 3;
    p.num_grad_quant_bins = 4;
    p.stochastic_rounding = 1;
    p.quant_seed = 11;
    p.time_histograms = 0;
    p.lambdarank_truncation_level = 30;  // RankerParams.default (ranking.mojo:478-490)
    p.lambdarank_norm = 1;
    p.lambdarank_sigmoid = 1.0;
    p.max_cat_to_onehot = 4;  // CategoricalParams.default (categorical.mojo:205-207)
    p.max_cat_threshold = 32;
    p.cat_smooth = 10.0;
    p.cat_l2 = 10.0;
    p.min_data_per_group = 100;
    p.one_hot_max_size = -1;
    if (!spec) return c;
    std::istringstream in(spec);
    std::string item;
    while (in >> item) {
        const size_t eq = item.find('=');
        if (eq == std::string::npos || eq == 0)
            throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "parameter '" + item + "' is not key=value"};
        std::string key = item.substr(0, eq), val = item.substr(eq + 1);
        auto it = aliases().find(key);
        if (it == aliases().end())
            throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "unknown parameter '" + key + "'"};
        const std::string &k = it->second;
        if (k == "objective") {
            if (val == "regression" || val == "regression_l2" || val == "l2" || val == "mse")
                p.objective = MBH_OBJ_REGRESSION;
            else if (val == "binary")
                p.objective = MBH_OBJ_BINARY;
            else if (val == "multiclass" || val == "softmax")
                p.objective = MBH_OBJ_MULTICLASS;
            else if (val == "lambdarank")
                p.objective = MBH_OBJ_LAMBDARANK;
            else if (val == "poisson" || val == "huber" || val == "quantile" || val == "mae" ||
                     val == "regression_l1" || val == "l1")
                throw ApiError{MOJOTREES_ERROR_UNSUPPORTED,
                               "objective=" + val + " is not served by the MI355X training path (regression, binary)"};
            else
                throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "unknown objective '" + val + "'"};
        } else if (k == "num_class") {
            c.num_class = (int)to_int(k, val);
            c.saw_num_class = true;
        } else if (k == "num_iterations") {
            p.num_iterations = (int)to_int(k, val);
        } else if (k == "learning_rate") {
            p.learning_rate = to_double(k, val);
        } else if (k == "num_leaves") {
            p.num_leaves = (int)to_int(k, val);
        } else if (k == "min_data_in_leaf") {
            p.min_data_in_leaf = (int)to_int(k, val);
        } else if (k == "min_sum_hessian_in_leaf") {
            p.min_sum_hessian = to_double(k, val);
        } else if (k == "lambda_l1") {
            p.lambda_l1 = to_double(k, val);
        } else if (k == "lambda_l2") {
            p.lambda_l2 = to_double(k, val);
        } else if (k == "max_depth") {
            p.max_depth = (int)to_int(k, val);
        } else if (k == "feature_fraction") {
            p.feature_fraction = to_double(k, val);
        } else if (k == "feature_fraction_bynode") {
            if (to_double(k, val) != 1.0)
                throw ApiError{MOJOTREES_ERROR_UNSUPPORTED, "feature_fraction_bynode < 1 is not served by the device path"};
        } else if (k == "feature_fraction_seed") {
            p.feature_fraction_seed = (int)to_int(k, val);
        } else if (k == "max_bin") {
            c.max_bin = (int)to_int(k, val);
        } else if (k == "alpha") {
            (void)to_double(k, val);
        } else if (k == "device") {
            if (val == "cpu") c.device = MOJOTREES_DEVICE_CPU;
            else if (val == "gpu" || val == "cuda" || val == "rocm" || val == "hip") c.device = MOJOTREES_DEVICE_GPU;
            else if (val == "auto") c.device = MOJOTREES_DEVICE_AUTO;
            else throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "unknown device '" + val + "'"};
        } else if (k == "use_missing") {
            c.use_missing = to_bool(k, val);
        } else if (k == "use_quantized_grad") {
            c.quantized = to_bool(k, val);
        } else if (k == "num_grad_quant_bins") {
            p.num_grad_quant_bins = (int)to_int(k, val);
        } else if (k == "stochastic_rounding") {
            p.stochastic_rounding = to_bool(k, val) ? 1 : 0;
        } else if (k == "quant_scale_rule") {
            // derive_scales' two rules (quantized_gradient.mojo:1343-1453):
            // LightGBM's max-abs lattice, or the reference's magnitude-sum
            // power-of-two lattice (its MOJOTREES_CPU_QUANT_SCALE switch)
            if (val == "max_abs" || val == "0") p.quant_scale_rule = 0;
            else if (val == "magnitude_sum" || val == "1") p.quant_scale_rule = 1;
            else throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "quant_scale_rule must be max_abs or magnitude_sum"};
        } else if (k == "quant_staging") {
            // the magnitude-sum lattice's staged pair width
            // (GpuActiveRows.set_packed_gradients, gpu_active_rows.mojo:2257-2395)
            if (val == "int32" || val == "0") p.quant_staging = 0;
            else if (val == "int16" || val == "1") p.quant_staging = 1;
            else throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "quant_staging must be int32 or int16"};
        } else if (k == "bagging_fraction") {
            p.bagging_fraction = to_double(k, val);
        } else if (k == "bagging_freq") {
            p.bagging_freq = (int)to_int(k, val);
        } else if (k == "bagging_seed") {
            p.bagging_seed = (int)to_int(k, val);
        } else if (k == "boosting") {
            if (val == "goss")
                p.goss = 1;
            else if (val != "gbdt" && val != "gbrt")
                throw ApiError{MOJOTREES_ERROR_UNSUPPORTED, "boosting=" + val + " is not served by this library"};
        } else if (k == "top_rate") {
            p.top_rate = to_double(k, val);
        } else if (k == "other_rate") {
            p.other_rate = to_double(k, val);
        } else if (k == "min_data_in_bin") {
            c.min_data_in_bin = (int)to_int(k, val);
        } else if (k == "bin_construct_sample_cnt") {
            c.bin_sample = to_int(k, val);
        } else if (k == "data_random_seed") {
            c.data_seed = to_int(k, val);
        } else if (k == "lambdarank_truncation_level") {
            p.lambdarank_truncation_level = (int)to_int(k, val);
        } else if (k == "sigmoid") {
            p.lambdarank_sigmoid = to_double(k, val);
        } else if (k == "lambdarank_norm") {
            p.lambdarank_norm = to_bool(k, val) ? 1 : 0;
        } else if (k == "categorical_feature") {
            // comma-separated column indices (LightGBM's form)
            c.categorical.clear();
            std::istringstream cs(val);
            for (std::string tok; std::getline(cs, tok, ',');) {
                if (tok.empty()) continue;
                const int64_t f = to_int(k, tok);
                if (f < 0) throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "categorical_feature indices must be non-negative"};
                c.categorical.push_back((int)f);
            }
        } else if (k == "max_cat_to_onehot") {
            p.max_cat_to_onehot = (int)to_int(k, val);
        } else if (k == "max_cat_threshold") {
            p.max_cat_threshold = (int)to_int(k, val);
        } else if (k == "cat_smooth") {
            p.cat_smooth = to_double(k, val);
        } else if (k == "cat_l2") {
            p.cat_l2 = to_double(k, val);
        } else if (k == "min_data_per_group") {
            p.min_data_per_group = (int)to_int(k, val);
        } else if (k == "one_hot_max_size") {
            p.one_hot_max_size = (int)to_int(k, val);
        }
    }
    if (c.saw_num_class && p.objective != MBH_OBJ_MULTICLASS)
        throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "num_class is only valid with objective=multiclass"};
    if (p.objective == MBH_OBJ_MULTICLASS) {
        if (!c.saw_num_class) throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "objective=multiclass needs num_class"};
        p.num_class = c.num_class;
    }
    p.use_quantized_grad = c.quantized ? 1 : 0;
    if (p.goss) {
        // GossParams.validate (goss.mojo:129-145) and _check_goss (boosting.mojo:346-355)
        const double tr = p.top_rate, orr = p.other_rate;
        if (!(tr >= 0.0 && tr <= 1.0)) throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "goss top_rate must be in [0, 1]"};
        if (!(orr >= 0.0 && orr <= 1.0))
            throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "goss other_rate must be in [0, 1]"};
        if (!(tr + orr <= 1.0))
            throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "goss top_rate + other_rate must not exceed 1"};
        if (!(tr + orr > 0.0))
            throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "goss top_rate + other_rate must be positive"};
        if (p.bagging_seed < 0) throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "goss seed must be nonnegative"};
        if (p.bagging_freq > 0 && p.bagging_fraction < 1.0)
            throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "goss and bagging cannot both be enabled"};
    }
    if (c.max_bin < 2 || c.max_bin > 256) throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "max_bin must be in [2, 256]"};
    return c;
}

template <class Fn>
int32_t guarded(MojoTreesError *err, Fn fn) {
    clear(err);
    try {
        return fn();
    } catch (const ApiError &e) {
        return fail(err, e.code, e.msg);
    } catch (const std::bad_alloc &) {
        return fail(err, MOJOTREES_ERROR_TRAINING, "out of host memory");
    } catch (const std::invalid_argument &e) {
        return fail(err, MOJOTREES_ERROR_INVALID_ARGUMENT, e.what());
    } catch (const std::exception &e) {
        return fail(err, MOJOTREES_ERROR_TRAINING, e.what());
    }
}

void check_model(const MojoTreesModel *m) {
    if (!m) throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "model is NULL"};
}

// Row x tree visits from which device=auto predicts on the GPU.
constexpr int64_t kAutoGpuRowTrees = (int64_t)1 << 24;

int32_t predict_common(const MojoTreesModel *model, const double *data, int64_t n_rows, int64_t n_features,
                       int64_t start_it, int64_t num_it, int32_t flags, int32_t device, double *out,
                       int64_t out_len, MojoTreesError *error) {
    return guarded(error, [&]() -> int32_t {
        check_model(model);
        if (!data || !out) throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "data and out_values must not be NULL"};
        if (n_rows <= 0) throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "n_rows must be positive"};
        const mb::Model &m = model->m;
        if (n_features != m.mapper.n_features)
            throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT,
                           "n_features " + std::to_string(n_features) + " does not match the model's " +
                               std::to_string(m.mapper.n_features)};
        if (flags != MOJOTREES_PREDICT_RESPONSE && flags != MOJOTREES_PREDICT_RAW)
            throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "unknown prediction flags"};
        if (device != MOJOTREES_DEVICE_CPU && device != MOJOTREES_DEVICE_GPU && device != MOJOTREES_DEVICE_AUTO)
            throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "unknown device"};
        const bool have_gpu = mbh_device_count() > 0;
        if (device == MOJOTREES_DEVICE_GPU && !have_gpu)
            throw ApiError{MOJOTREES_ERROR_UNSUPPORTED,
                           "no gfx950 (MI355X) GPU is available; device=gpu never falls back to the CPU"};
        const int64_t k = m.num_class;
        if (out_len < n_rows * k) throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "out_len is smaller than n_rows * num_classes"};
        const int64_t total = m.num_iterations();
        int64_t s0 = start_it < 0 ? 0 : std::min(start_it, total);
        int64_t s1 = num_it <= 0 ? total : std::min(total, s0 + num_it);
        std::vector<double> tmp((size_t)(n_rows * k));
        // AUTO takes the device for batches large enough to pay for the upload
        // (both paths give the same bits)
        const bool on_gpu = device == MOJOTREES_DEVICE_GPU ||
                            (device == MOJOTREES_DEVICE_AUTO && have_gpu && n_rows * (s1 - s0) * k >= kAutoGpuRowTrees);
        if (on_gpu) {
            std::vector<uint8_t> bins((size_t)n_rows * n_features);
            m.mapper.transform(data, n_rows, bins.data());
            char msg[512] = {0};
            const int32_t rc = mbh_predict_binned(
                bins.data(), n_rows, (int32_t)n_features, (int32_t)k, m.learning_rate, s0 == 0 ? m.base.data() : nullptr,
                m.offsets.data(), s0 * k, s1 * k, m.feature.data(), m.threshold.data(), m.left.data(), m.right.data(),
                m.value.data(), m.default_left.data(), m.missing_bin.data(),
                m.mapper.any_cat() ? m.cat_bits.data() : nullptr, tmp.data(), msg, sizeof(msg));
            if (rc != MOJOTREES_OK) throw ApiError{rc, msg};
        } else {
            m.predict_raw(data, n_rows, s0, s1, tmp.data());
        }
        if (flags == MOJOTREES_PREDICT_RESPONSE) m.response(tmp.data(), n_rows);
        std::memcpy(out, tmp.data(), tmp.size() * sizeof(double));
        return MOJOTREES_OK;
    });
}

// categorical_feature indices name columns of the matrix, each once
// (fit_categorical_spec's checks, categorical.mojo:434-444)
void check_categorical(const Config &c, int64_t n_features) {
    std::vector<int> seen;
    for (int f : c.categorical) {
        if (f >= n_features)
            throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT,
                           "categorical_feature index " + std::to_string(f) + " is out of range"};
        if (std::find(seen.begin(), seen.end(), f) != seen.end())
            throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "duplicate categorical feature index"};
        seen.push_back(f);
    }
}

// boosting._check_sample_weight (boosting.mojo:334-343), before any device
// work so a bad vector is named on any host; null means unweighted
void check_weights(const double *weights, int64_t n_rows) {
    if (!weights) return;
    double total = 0.0;
    for (int64_t r = 0; r < n_rows; ++r) {
        if (!std::isfinite(weights[r]) || weights[r] < 0.0)
            throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "sample_weight must be finite and nonnegative"};
        total += weights[r];
    }
    if (!(total > 0.0)) throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "sample_weight must have a positive sum"};
}

// Host binning, the resident dataset, device training and the model: the
// common body of the training entry points. groups: per-query row counts
// (lambdarank), or null.
MojoTreesModel *train_model(const double *data, int64_t n_rows, int64_t n_features, const double *labels,
                            const double *weights, const int32_t *groups, int64_t n_groups, Config &c) {
    check_categorical(c, n_features);
    mb::BinMapper mapper = mb::fit_bins(data, n_rows, (int)n_features, c.max_bin, c.min_data_in_bin,
                                        c.use_missing, c.bin_sample, c.data_seed, c.categorical);
    std::vector<uint8_t> bins((size_t)n_rows * n_features);
    mapper.transform(data, n_rows, bins.data());
    char msg[512] = {0};
    mbh_dataset *ds = nullptr;
    int32_t rc = mbh_dataset_create(bins.data(), n_rows, (int32_t)n_features, c.max_bin,
                                    mapper.missing_bin.data(), labels, &ds, msg, sizeof(msg));
    if (rc != MOJOTREES_OK) throw ApiError{rc, msg};
    if (mapper.any_cat()) {
        std::vector<int32_t> ncat(n_features);
        for (int f = 0; f < (int)n_features; ++f) ncat[f] = mapper.n_categories(f);
        rc = mbh_dataset_set_categorical(ds, ncat.data(), msg, sizeof(msg));
        if (rc != MOJOTREES_OK) {
            mbh_dataset_free(ds);
            throw ApiError{rc, msg};
        }
    }
    if (weights) {
        rc = mbh_dataset_set_weights(ds, weights, n_rows, msg, sizeof(msg));
        if (rc != MOJOTREES_OK) {
            mbh_dataset_free(ds);
            throw ApiError{rc, msg};
        }
    }
    if (groups) {
        rc = mbh_dataset_set_groups(ds, groups, n_groups, msg, sizeof(msg));
        if (rc != MOJOTREES_OK) {
            mbh_dataset_free(ds);
            throw ApiError{rc, msg};
        }
    }
    mbh_fit *fit = nullptr;
    rc = mbh_train(ds, &c.p, &fit, msg, sizeof(msg));
    mbh_dataset_free(ds);
    if (rc != MOJOTREES_OK) throw ApiError{rc, msg};
    auto *model = new MojoTreesModel();
    mb::Model &m = model->m;
    // model objective codes: 0 regression, 1 binary, -1 multiclass, 7
    // lambdarank (objective_registry.mojo:289)
    m.objective = c.p.objective == MBH_OBJ_MULTICLASS ? -1
                  : c.p.objective == MBH_OBJ_LAMBDARANK ? 7
                                                         : c.p.objective;
    m.num_class = mbh_fit_num_class(fit);
    m.learning_rate = c.p.learning_rate;
    m.mapper = mapper;
    const int nt = mbh_fit_num_trees(fit);
    const int64_t nn = mbh_fit_total_nodes(fit);
    m.base.resize(m.num_class);
    m.offsets.resize(nt + 1);
    m.feature.resize(nn);
    m.threshold.resize(nn);
    m.left.resize(nn);
    m.right.resize(nn);
    m.value.resize(nn);
    m.default_left.resize(nn);
    m.missing_bin.resize(nn);
    m.gain.resize(nn);
    m.count.resize(nn);
    mbh_fit_arrays(fit, m.base.data(), m.offsets.data(), m.feature.data(), m.threshold.data(), m.left.data(),
                   m.right.data(), m.value.data(), m.default_left.data(), m.missing_bin.data(), m.gain.data(),
                   m.count.data());
    m.cat_bits.resize((size_t)nn * 4);
    mbh_fit_cat_bits(fit, m.cat_bits.data());
    m.is_cat_node.resize(nn);
    for (int64_t i = 0; i < nn; ++i) m.is_cat_node[i] = (m.feature[i] >= 0 && m.threshold[i] < 0) ? 1 : 0;
    mbh_fit_free(fit);
    m.n_leaves.resize(nt);
    for (int t = 0; t < nt; ++t) {
        int leaves = 0;
        for (int64_t i = m.offsets[t]; i < m.offsets[t + 1]; ++i) leaves += m.feature[i] < 0;
        m.n_leaves[t] = leaves;
    }
    return model;
}

}  // namespace

extern "C" {

int32_t mojotrees_abi_version(void) { return MOJOTREES_ABI_VERSION; }

void mojotrees_library_version(int32_t *major, int32_t *minor, int32_t *patch) {
    if (major) *major = 0;
    if (minor) *minor = 1;
    if (patch) *patch = 0;
}

int32_t mojotrees_gpu_available(void) { return mbh_device_count() > 0 ? 1 : 0; }

MojoTreesError *mojotrees_error_create(void) { return new (std::nothrow) MojoTreesError(); }
void mojotrees_error_free(MojoTreesError *e) { delete e; }
const char *mojotrees_error_message(const MojoTreesError *e) { return e ? e->message.c_str() : nullptr; }

int32_t mojotrees_train_dense(const double *data, int64_t n_rows, int64_t n_features, const double *labels,
                              const double *weights, const char *parameters, MojoTreesModel **out_model,
                              MojoTreesError *error) {
    return guarded(error, [&]() -> int32_t {
        if (!data || !labels || !out_model)
            throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "data, labels and out_model must not be NULL"};
        if (n_rows <= 0 || n_features <= 0)
            throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "n_rows and n_features must be positive"};
        Config c = parse(parameters);
        check_categorical(c, n_features);
        if (c.p.objective == MBH_OBJ_LAMBDARANK)
            throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT,
                           "objective=lambdarank needs query groups: train it with mbh_train_ranker_dense"};
        check_weights(weights, n_rows);
        if (c.device == MOJOTREES_DEVICE_CPU)
            throw ApiError{MOJOTREES_ERROR_UNSUPPORTED,
                           "device=cpu: this library is the MI355X training path and has no CPU trainer"};
        if (mbh_device_count() == 0)
            throw ApiError{MOJOTREES_ERROR_UNSUPPORTED,
                           "no gfx950 (MI355X) GPU is available; device=gpu never falls back to the CPU"};
        if (c.p.objective == MBH_OBJ_BINARY)
            for (int64_t r = 0; r < n_rows; ++r)
                if (labels[r] != 0.0 && labels[r] != 1.0)
                    throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "binary labels must be 0 or 1"};
        MojoTreesModel *model = train_model(data, n_rows, n_features, labels, weights, nullptr, 0, c);
        *out_model = model;
        return MOJOTREES_OK;
    });
}

int32_t mojotrees_predict(const MojoTreesModel *model, const double *data, int64_t n_rows, int64_t n_features,
                          double *out_values, int64_t out_len, MojoTreesError *error) {
    return predict_common(model, data, n_rows, n_features, 0, 0, MOJOTREES_PREDICT_RESPONSE, MOJOTREES_DEVICE_CPU,
                          out_values, out_len, error);
}

int32_t mojotrees_predict_raw(const MojoTreesModel *model, const double *data, int64_t n_rows, int64_t n_features,
                              double *out_values, int64_t out_len, MojoTreesError *error) {
    return predict_common(model, data, n_rows, n_features, 0, 0, MOJOTREES_PREDICT_RAW, MOJOTREES_DEVICE_CPU,
                          out_values, out_len, error);
}

int32_t mojotrees_predict_ex(const MojoTreesModel *model, const double *data, int64_t n_rows, int64_t n_features,
                             int64_t start_iteration, int64_t num_iteration, int32_t flags, int32_t device,
                             double *out_values, int64_t out_len, MojoTreesError *error) {
    return predict_common(model, data, n_rows, n_features, start_iteration, num_iteration, flags, device,
                          out_values, out_len, error);
}

int32_t mojotrees_save_model(const MojoTreesModel *model, const char *path, MojoTreesError *error) {
    return guarded(error, [&]() -> int32_t {
        check_model(model);
        if (!path) throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "path is NULL"};
        try {
            model->m.save(path);
        } catch (const std::runtime_error &e) {
            throw ApiError{MOJOTREES_ERROR_IO, e.what()};
        }
        return MOJOTREES_OK;
    });
}

int32_t mojotrees_load_model(const char *path, MojoTreesModel **out_model, MojoTreesError *error) {
    return guarded(error, [&]() -> int32_t {
        if (!path || !out_model) throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "path and out_model must not be NULL"};
        mb::Model m;
        try {
            m = mb::Model::load(path);
        } catch (const std::exception &e) {
            throw ApiError{MOJOTREES_ERROR_IO, e.what()};
        }
        // serialize.load_model checks a names section and leaves the names
        // out of the model (serialize.mojo:1463-1475): a C ABI model carries
        // none, and mbh_model_feature_names reads them from the file
        m.feature_names.clear();
        auto *model = new MojoTreesModel();
        model->m = std::move(m);
        *out_model = model;
        return MOJOTREES_OK;
    });
}

int32_t mojotrees_model_num_features(const MojoTreesModel *model, int64_t *out, MojoTreesError *error) {
    return guarded(error, [&]() -> int32_t {
        check_model(model);
        if (!out) throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "out_value is NULL"};
        *out = model->m.mapper.n_features;
        return MOJOTREES_OK;
    });
}

int32_t mojotrees_model_num_classes(const MojoTreesModel *model, int64_t *out, MojoTreesError *error) {
    return guarded(error, [&]() -> int32_t {
        check_model(model);
        if (!out) throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "out_value is NULL"};
        *out = model->m.num_class;
        return MOJOTREES_OK;
    });
}

int32_t mojotrees_model_num_trees(const MojoTreesModel *model, int64_t *out, MojoTreesError *error) {
    return guarded(error, [&]() -> int32_t {
        check_model(model);
        if (!out) throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "out_value is NULL"};
        *out = model->m.num_trees();
        return MOJOTREES_OK;
    });
}

int32_t mojotrees_model_num_iterations(const MojoTreesModel *model, int64_t *out, MojoTreesError *error) {
    return guarded(error, [&]() -> int32_t {
        check_model(model);
        if (!out) throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "out_value is NULL"};
        *out = model->m.num_iterations();
        return MOJOTREES_OK;
    });
}

int32_t mojotrees_model_dump_json(const MojoTreesModel *model, char **out_text, MojoTreesError *error) {
    return guarded(error, [&]() -> int32_t {
        check_model(model);
        if (!out_text) throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "out_text is NULL"};
        std::string s = model->m.dump_json();
        char *buf = (char *)std::malloc(s.size() + 1);
        if (!buf) throw std::bad_alloc();
        std::memcpy(buf, s.c_str(), s.size() + 1);
        *out_text = buf;
        return MOJOTREES_OK;
    });
}

int32_t mojotrees_feature_importance(const MojoTreesModel *model, int32_t type, double *out_values, int64_t out_len,
                                     MojoTreesError *error) {
    return guarded(error, [&]() -> int32_t {
        check_model(model);
        if (!out_values) throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "out_values is NULL"};
        if (type != MOJOTREES_IMPORTANCE_SPLIT && type != MOJOTREES_IMPORTANCE_GAIN)
            throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "unknown importance type"};
        const mb::Model &m = model->m;
        if (out_len < m.mapper.n_features) throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "out_len is too small"};
        std::vector<double> imp(m.mapper.n_features, 0.0);
        for (size_t i = 0; i < m.feature.size(); ++i)
            if (m.feature[i] >= 0) imp[m.feature[i]] += type == MOJOTREES_IMPORTANCE_SPLIT ? 1.0 : m.gain[i];
        std::memcpy(out_values, imp.data(), imp.size() * sizeof(double));
        return MOJOTREES_OK;
    });
}

int32_t mojotrees_parameter_keys(char **out_text, MojoTreesError *error) {
    return guarded(error, [&]() -> int32_t {
        if (!out_text) throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "out_text is NULL"};
        const size_t n = std::strlen(kPrimaryKeys);
        char *buf = (char *)std::malloc(n + 1);
        if (!buf) throw std::bad_alloc();
        std::memcpy(buf, kPrimaryKeys, n + 1);
        *out_text = buf;
        return MOJOTREES_OK;
    });
}

void mojotrees_string_free(char *text) { std::free(text); }

int32_t mbh_save_model_named(const MojoTreesModel *model, const char *path, const char *const *names,
                             int64_t n_names, MojoTreesError *error) {
    return guarded(error, [&]() -> int32_t {
        check_model(model);
        if (!path) throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "path is NULL"};
        if (n_names < 0 || (n_names > 0 && !names))
            throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "names must hold n_names strings"};
        if (n_names > 0 && n_names != model->m.mapper.n_features)
            throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT,
                           "feature_names has " + std::to_string(n_names) + " entries for " +
                               std::to_string(model->m.mapper.n_features) + " features"};
        mb::Model m = model->m;
        m.feature_names.clear();
        for (int64_t f = 0; f < n_names; ++f) {
            if (!names[f]) throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "a feature name is NULL"};
            m.feature_names.emplace_back(names[f]);
        }
        try {
            m.save(path);
        } catch (const std::runtime_error &e) {
            throw ApiError{MOJOTREES_ERROR_IO, e.what()};
        }
        return MOJOTREES_OK;
    });
}

int32_t mbh_model_feature_names(const char *path, char **out_names, int64_t *out_count, MojoTreesError *error) {
    return guarded(error, [&]() -> int32_t {
        if (!path || !out_names || !out_count)
            throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "path, out_names and out_count must not be NULL"};
        std::vector<std::string> names;
        try {
            names = mb::Model::load_feature_names(path);
        } catch (const std::exception &e) {
            throw ApiError{MOJOTREES_ERROR_IO, e.what()};
        }
        *out_names = nullptr;
        *out_count = (int64_t)names.size();
        if (names.empty()) return MOJOTREES_OK;
        size_t total = 0;
        for (const std::string &nm : names) total += nm.size() + 1;
        char *buf = (char *)std::malloc(total);
        if (!buf) throw std::bad_alloc();
        size_t at = 0;
        for (const std::string &nm : names) {
            std::memcpy(buf + at, nm.c_str(), nm.size() + 1);
            at += nm.size() + 1;
        }
        *out_names = buf;
        return MOJOTREES_OK;
    });
}
void mojotrees_model_free(MojoTreesModel *model) { delete model; }

int32_t mbh_train_ranker_dense(const double *data, int64_t n_rows, int64_t n_features, const double *labels,
                               const double *weights, const int32_t *group_counts, int64_t n_groups, const char *parameters,
                               MojoTreesModel **out_model, MojoTreesError *error) {
    return guarded(error, [&]() -> int32_t {
        if (!data || !labels || !group_counts || !out_model)
            throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "data, labels, group_counts and out_model must not be NULL"};
        if (n_rows <= 0 || n_features <= 0 || n_groups <= 0)
            throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "n_rows, n_features and n_groups must be positive"};
        Config c = parse(parameters);
        check_categorical(c, n_features);
        c.p.objective = MBH_OBJ_LAMBDARANK;
        check_weights(weights, n_rows);
        if (c.device == MOJOTREES_DEVICE_CPU)
            throw ApiError{MOJOTREES_ERROR_UNSUPPORTED,
                           "device=cpu: this library is the MI355X training path and has no CPU trainer"};
        if (mbh_device_count() == 0)
            throw ApiError{MOJOTREES_ERROR_UNSUPPORTED,
                           "no gfx950 (MI355X) GPU is available; device=gpu never falls back to the CPU"};
        // check_labels (ranking.mojo:221-232)
        for (int64_t r = 0; r < n_rows; ++r)
            if (!(labels[r] >= 0.0 && labels[r] <= 30.0) || labels[r] != std::floor(labels[r]))
                throw ApiError{MOJOTREES_ERROR_INVALID_ARGUMENT, "relevance labels must be integers in [0, 30]"};
        *out_model = train_model(data, n_rows, n_features, labels, weights, group_counts, n_groups, c);
        return MOJOTREES_OK;
    });
}

}  // extern "C"
