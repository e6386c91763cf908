/* CPU oracle for the mojoboost-amd GBDT training path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is a plain C++ restatement of the
 * reference (ajhendel/mojoboost, package `mojotrees`) CPU training algorithm,
 * used as the parity checker for the HIP path and as the CPU baseline timed by
 * bench.py. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it. The product library (mojoboost_amd/) never links or calls
 * it.
 *
 * Every function names the reference file:line it follows in oracle.cpp.
 * Pinning (what checks each part) is listed at the top of oracle.cpp.
 */
#ifndef MOJOBOOST_ORACLE_H
#define MOJOBOOST_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_OBJ_L2 0
#define ORC_OBJ_BINARY 1
#define ORC_OBJ_MULTICLASS 2
#define ORC_OBJ_LAMBDARANK 3

typedef struct {
    int32_t objective;          /* ORC_OBJ_* */
    int32_t num_class;          /* multiclass only */
    int32_t num_iterations;
    double learning_rate;
    int32_t num_leaves;
    int32_t min_data_in_leaf;
    double lambda_l2;
    double lambda_l1;
    double min_sum_hessian;
    int32_t max_depth;          /* <= 0: unlimited */
    double feature_fraction;
    int32_t feature_fraction_seed;
    double bagging_fraction;
    int32_t bagging_freq;
    int32_t bagging_seed;
    int32_t use_quantized_grad;
    int32_t num_grad_quant_bins;
    int32_t stochastic_rounding;
    int32_t quant_seed;
    int32_t goss;
    double top_rate;
    double other_rate;
    int32_t goss_seed;
    int32_t n_threads;          /* <= 0: hardware concurrency */
    int32_t fused_score_update; /* 1: raw = fma(lr, v, raw) (reference default) */
    int32_t fused_predict;      /* 1: prediction sums with fma */
    int32_t totals_tree_reduce; /* 1: SIMD totals reduced pairwise (Mojo reduce) */
    int32_t use_init_base;      /* 1: start every row at init_base (single output) */
    double init_base;
    /* lambdarank: query q owns rows [query_starts[q], query_starts[q + 1]) */
    const int64_t *query_starts;
    int64_t n_queries;
    int32_t lambdarank_truncation_level;
    int32_t lambdarank_norm;
    double lambdarank_sigmoid;
    /* categorical features (categorical.mojo): n_categories[f] > 0 marks
     * feature f categorical, its categories in bins 1..n_categories[f] and
     * bin 0 holding missing, unseen and dropped codes; NULL: all numerical */
    const int32_t *n_categories;
    int32_t max_cat_to_onehot;  /* LightGBM default 4 */
    int32_t max_cat_threshold;  /* 32 */
    double cat_smooth;          /* 10 */
    double cat_l2;              /* 10 */
    int32_t min_data_per_group; /* 100 */
    int32_t one_hot_max_size;   /* -1: off (CatBoost's one-hot rule when >= 0) */
    /* per-row sample weights (n_rows), or NULL for unweighted: they scale
     * each row's gradient and hessian and weight the base score / class
     * priors (boosting._fill_grad_hess_into, _base_score, train_multiclass) */
    const double *weights;
    /* quantized-gradient lattice (derive_scales, quantized_gradient.mojo:
     * 1343-1453): 0 LightGBM's max-abs rule (num_grad_quant_bins units), 1
     * the reference's magnitude-sum power-of-two rule (2^30 lattice) */
    int32_t quant_scale_rule;
} orc_params;

/* A trained model in flat arrays. Trees are laid out one after another;
 * tree t owns nodes [node_offset[t], node_offset[t + 1]). */
typedef struct orc_model orc_model;

/* -------------------------------------------------------------- arithmetic */
uint64_t orc_splitmix64(uint64_t state);
double orc_uniform(uint64_t counter);
double orc_exp(double x);
double orc_log(double x);
double orc_sigmoid(double x);
uint64_t orc_quant_stream(int64_t seed, int64_t round_index,
                          int64_t class_index, int64_t plane);

/* ---------------------------------------------------------------- binning */
int32_t orc_bin_equal_width(const double *x, int64_t n_rows,
                            int32_t n_features, int32_t n_bins,
                            uint8_t *out_bins);
/* fit_bins + transform. out_edges is n_features * max_bins doubles,
 * out_n_edges and out_missing_bin n_features each. Returns 0 on success. */
int32_t orc_fit_bins(const double *x, int64_t n_rows, int32_t n_features,
                     int32_t max_bins, int32_t min_data_in_bin,
                     int32_t use_missing, int64_t sample_cnt, int64_t seed,
                     double *out_edges, int32_t *out_n_edges,
                     int32_t *out_missing_bin);
/* bin_construct_sample_rows: the ascending rows a sampled fit reads
 * (written to out when not NULL); returns their count, 0 meaning every row. */
int64_t orc_bin_sample_rows(int64_t n_rows, int64_t sample_cnt, int64_t seed, int64_t *out);
int32_t orc_transform(const double *x, int64_t n_rows, int32_t n_features,
                      int32_t max_bins, const double *edges,
                      const int32_t *n_edges, const int32_t *missing_bin,
                      uint8_t *out_bins);

/* ------------------------------------------------------------- objectives */
/* Per-row narrowed derivatives. labels are class ids for multiclass. */
int32_t orc_grad_hess(int32_t objective, const double *raw,
                      const double *labels, int64_t n_rows,
                      int32_t num_class, int32_t class_k, double *grad,
                      double *hess);
/* The same with per-row weights (NULL: unweighted). */
int32_t orc_grad_hess_w(int32_t objective, const double *raw,
                        const double *labels, const double *weights,
                        int64_t n_rows, int32_t num_class, int32_t class_k,
                        double *grad, double *hess);

/* ----------------------------------------------------------- quantization */
/* gradient_stats + derive_scales (max-abs rule) + per-row rounding.
 * rows may be NULL (every row). Writes q_grad/q_hess (all n rows) and
 * out_scales[0..1] = grad_units, hess_units; out_limits = max units. */
int32_t orc_quantize(const double *grad, const double *hess, int64_t n_rows,
                     const int32_t *rows, int64_t n_sel, int32_t quant_bins,
                     int32_t stochastic, int64_t seed, int64_t round_index,
                     int64_t class_index, int32_t const_hessian,
                     int8_t *q_grad, int8_t *q_hess, double *out_scales);

/* The same for either lattice (rule 0 max-abs, 1 magnitude sum), with
 * int32 outputs; returns -1 when the magnitudes are out of range. */
int32_t orc_quantize_rule(const double *grad, const double *hess, int64_t n_rows,
                          const int32_t *rows, int64_t n_sel, int32_t quant_bins,
                          int32_t stochastic, int64_t seed, int64_t round_index,
                          int64_t class_index, int32_t const_hessian, int32_t rule,
                          int32_t *q_grad, int32_t *q_hess, double *out_scales);
/* The device magnitude reduction's sums (sum |g|, sum |h|) in its fixed
 * order; in_sample NULL or n_rows flags (0: the row adds nothing). */
int32_t orc_magnitude_sums(const double *grad, const double *hess, int64_t n_rows,
                           const uint8_t *in_sample, double *out_sums);
/* largest_power_of_two_at_most / fixed_point_scale_pow2; -1 when refused. */
double orc_largest_power_of_two_at_most(double x);
double orc_fixed_point_scale_pow2(double total);

/* ------------------------------------------------------------ histograms */
int32_t orc_hist_quantized32(const uint8_t *bins, int64_t n_rows, int32_t n_features,
                             int32_t n_bins, const int32_t *q_grad, const int32_t *q_hess,
                             const int32_t *rows, int64_t n_sel, int64_t *out);
/* Integer histogram over `rows` (or all rows when rows == NULL):
 * out is n_features * n_bins cells of int64 {grad, hess, count}. */
int32_t orc_hist_quantized(const uint8_t *bins, int64_t n_rows,
                           int32_t n_features, int32_t n_bins,
                           const int8_t *q_grad, const int8_t *q_hess,
                           const int32_t *rows, int64_t n_sel,
                           int64_t *out);
/* Float64 histogram (reference order), cells {grad, hess} + counts. */
int32_t orc_hist_float(const uint8_t *bins, int64_t n_rows,
                       int32_t n_features, int32_t n_bins,
                       const double *grad, const double *hess,
                       const int32_t *rows, int64_t n_sel,
                       int32_t row_blocks, double *out_gh,
                       int64_t *out_count);

/* ---------------------------------------------------------------- ranking */
/* LambdaRank gradients and hessians of every query (binary64), and the log2
 * the discounts use. */
int32_t orc_lambdarank(const double *scores, const double *labels, const int64_t *starts,
                       int64_t n_queries, int32_t truncation, double sigma, int32_t norm,
                       double *grad, double *hess);
double orc_log2(double x);

/* ------------------------------------------------------------------ GOSS */
/* One GOSS selection of round `round_index` (no warmup): ascending kept rows,
 * each row's scale (1 for the top set, the multiplier for sampled rows), and
 * grad/hess scaled in place. rows_out and scale_out hold n entries. */
int32_t orc_goss_select(double *grad, double *hess, int64_t n, double top_rate,
                        double other_rate, int32_t seed, int64_t round_index,
                        int32_t *rows_out, double *scale_out, int64_t *n_out);
/* One multiclass round's GOSS sample (boosting._multiclass_goss_select):
 * prob row-major n x K, weights may be NULL; see oracle.cpp. */
int32_t orc_goss_select_multiclass(const double *prob, const double *labels, int64_t n, int32_t K,
                                   const double *weights, double top_rate, double other_rate,
                                   int32_t seed, int64_t round_index, int32_t *rows_out,
                                   uint8_t *other_out, double *mult_out, int64_t *n_out);

/* ----------------------------------------------------------- split search */
/* Best split of one node from an integer histogram. Returns found (0/1);
 * out_feature, out_bin, out_default_left, out_gain. */
int32_t orc_split_quantized(const int64_t *hist, int32_t n_features,
                            int32_t n_bins, const int32_t *missing_bin,
                            const int32_t *widths, double grad_units,
                            double hess_units, double lambda_l1,
                            double lambda_l2, double min_sum_hessian,
                            int32_t min_data_in_leaf, int32_t *out_feature,
                            int32_t *out_bin, int32_t *out_default_left,
                            double *out_gain);

/* Best category partition of one categorical feature from a Float64
 * histogram plane (categorical.find_best_categorical_split): gh holds
 * n_categories + 1 interleaved (grad, hess) cells (bin 0 first), count the
 * matching counts. Returns found (0/1); out_bits is the 256-bit set of bins
 * routed left. */
int32_t orc_cat_split(const double *gh, const int64_t *count, int32_t n_categories,
                      double total_g, double total_h, int64_t total_c,
                      double lambda_l2, double lambda_l1, double min_child_hess,
                      int32_t min_data_in_leaf, int32_t max_cat_to_onehot,
                      int32_t max_cat_threshold, double cat_smooth, double cat_l2,
                      int32_t min_data_per_group, int32_t one_hot_max_size,
                      double *out_gain, uint64_t *out_bits);

/* --------------------------------------------------------------- training */
orc_model *orc_train(const uint8_t *bins, int64_t n_rows, int32_t n_features,
                     int32_t n_bins, const int32_t *missing_bin,
                     const double *labels, const orc_params *params,
                     char *err, int32_t err_len);
void orc_model_free(orc_model *model);
int32_t orc_model_num_trees(const orc_model *model);
int32_t orc_model_num_class(const orc_model *model);
int64_t orc_model_total_nodes(const orc_model *model);
/* base has num_class entries. node_offset has num_trees + 1 entries. */
void orc_model_arrays(const orc_model *model, double *base,
                      int64_t *node_offset, int32_t *feature,
                      int32_t *threshold_bin, int32_t *left, int32_t *right,
                      double *value, int32_t *default_left,
                      int32_t *missing_bin, double *split_gain,
                      double *count);
/* Category sets, 4 words per node (all zero on numerical nodes and leaves);
 * a categorical node has threshold_bin -1 and a non-empty set. */
void orc_model_cat_bits(const orc_model *model, uint64_t *out);
/* Training-time raw scores after the last round, row-major n * num_class. */
void orc_model_train_raw(const orc_model *model, double *out);
/* Per-round wall seconds, num_iterations entries (0 for rounds not run). */
void orc_model_round_seconds(const orc_model *model, double *out);

/* Prediction over a binned matrix: raw (row-major n * k) and response. */
int32_t orc_predict_binned(const orc_model *model, const uint8_t *bins,
                           int64_t n_rows, int32_t n_features, double *raw,
                           double *response);

#ifdef __cplusplus
}
#endif

#endif /* MOJOBOOST_ORACLE_H */
