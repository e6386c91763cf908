/* mojoboost-amd device-level C ABI.
 *
 * The training hot path of the `mojotrees` GPU trainer, re-built for one
 * AMD Instinct MI355X (gfx950): the binned matrix stays resident in HBM and
 * each boosting round runs as a sequence of HIP kernels that grow the tree
 * on the device. `mojotrees.h` (the reference's public ABI) is implemented on
 * top of these calls; they are exported separately so benchmarks and parity
 * tests can keep inputs resident and call individual stages.
 *
 * Reference interfaces these replace (ajhendel/mojoboost):
 *   mbh_dataset_create    GpuHistogramBuilder(data) bin upload
 *                         (src/mojotrees/histogram_gpu.mojo:591-606)
 *   mbh_train             train_gpu / _train_gpu_rounds
 *                         (src/mojotrees/train_gpu.mojo:5098-5168, :4235-5095)
 *   mbh_objective_quantize  fill_gradients_device + the quantizer
 *                         (histogram_gpu.mojo:1697-1712,
 *                          quantized_gradient.mojo:2487-2565)
 *   mbh_histogram         GpuActiveRows.enqueue_range_histogram
 *                         (src/mojotrees/gpu_active_rows.mojo:8586)
 *   mbh_exp_sigmoid       the device objective's sigmoid
 *                         (src/mojotrees/gpu_objectives_native.mojo:417-436)
 *
 * Conventions: every fallible call returns 0 on success or a negative
 * MOJOTREES_ERROR_* code and writes a NUL-terminated message into `err`
 * (err_len bytes, may be NULL). Host buffers are the caller's and are not
 * retained. Binned matrices are column-major uint8, bins[f * n_rows + r].
 */
#ifndef MOJOBOOST_HIP_H
#define MOJOBOOST_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MBH_OBJ_REGRESSION 0
#define MBH_OBJ_BINARY 1
#define MBH_OBJ_MULTICLASS 2
#define MBH_OBJ_LAMBDARANK 3  /* needs query groups (mbh_dataset_set_groups) */

typedef struct mbh_dataset mbh_dataset;
typedef struct mbh_fit mbh_fit;

typedef struct {
    int32_t objective;
    int32_t num_class;
    int32_t num_iterations;
    double learning_rate;
    int32_t num_leaves;
    int32_t min_data_in_leaf;
    double lambda_l1;
    double lambda_l2;
    double min_sum_hessian;
    int32_t max_depth;
    double feature_fraction;
    int32_t feature_fraction_seed;
    double bagging_fraction;
    int32_t bagging_freq;
    int32_t bagging_seed;
    int32_t num_grad_quant_bins;
    int32_t stochastic_rounding;
    int32_t quant_seed;
    int32_t time_histograms; /* 1: bracket each histogram launch with events */
    int32_t use_quantized_grad; /* 1: int8 gradients, integer histograms;
                                   0: fp32 gradients, fp64 histogram sums */
    int32_t goss;               /* 1: gradient-based one-side sampling after
                                   floor(1 / learning_rate) rounds, stream
                                   keyed by bagging_seed */
    double top_rate, other_rate;
    /* GOSS count: decisions outside a band of goss_band standard deviations
     * (+64) around the count's expectation are taken in parallel and checked
     * exactly; goss_exact_walk = 1 always runs the full sequential count.
     * Both give the reference's sample. Defaults 6 and 0 (at 6 the
     * check fails in well under one round in 10^5; C3 ran 0.5 % faster per
     * 500 trees than at 10). */
    double goss_band;
    int32_t goss_exact_walk;
    /* lambdarank (LightGBM names): pairs whose better-ranked member sits
     * within the truncation level, the pairwise logistic's scale, per-pair
     * and per-query normalization. Defaults 30, 1.0, 1. */
    int32_t lambdarank_truncation_level;
    int32_t lambdarank_norm;
    double lambdarank_sigmoid;
    /* categorical features (categorical.CategoricalParams,
     * src/mojotrees/categorical.mojo:164-240, LightGBM names and defaults
     * 4, 32, 10, 10, 100; one_hot_max_size -1 = off). Used only when the
     * dataset marks features categorical (mbh_dataset_set_categorical). */
    int32_t max_cat_to_onehot;
    int32_t max_cat_threshold;
    double cat_smooth;
    double cat_l2;
    int32_t min_data_per_group;
    int32_t one_hot_max_size;
    /* quantized-gradient lattice (derive_scales,
     * src/mojotrees/quantized_gradient.mojo:1343-1453): 0 LightGBM's
     * max-abs rule, num_grad_quant_bins units, int8 pairs (default); 1 the
     * reference's magnitude-sum power-of-two rule (the lattice its GPU
     * histogram ships and its CPU quantized path defaults to): scales
     * 2^k <= 2^30 / sum|g| (sum|h|), int32 pairs, int32 histogram sums;
     * num_grad_quant_bins is then unused. n_rows < 2^30; not with
     * lambdarank. */
    int32_t quant_scale_rule;
    /* magnitude-sum lattice staging (GpuActiveRows.set_packed_gradients,
     * src/mojotrees/gpu_active_rows.mojo:2257-2395): 0 int32 pairs (the
     * reference's default), 1 the packed int16 arm -- each row's pair
     * narrowed to int16 in its record, exact while every value fits; a fit
     * in which any value does not is refused (MOJOTREES_ERROR_TRAINING,
     * naming the count per plane). */
    int32_t quant_staging;
    /* how a leaf holds its rows during growth: 0 automatic (default), 1 as
     * their records, 2 as row ids. As records (int8 pairs of the max-abs
     * lattice, one feature tile of at most 64-byte records), the partition
     * moves each row's whole record into the child's contiguous range and
     * the histogram streams it; as row ids, the partition moves 4-byte ids
     * and the histogram gathers each record by id. Automatic takes row ids
     * (measured faster end to end). The trees are the same either way. */
    int32_t partition_mode;
} mbh_params;

/* Host binning of a column-major double matrix (NaN = missing) with the
 * reference's quantile rule (binning.fit_bins + BinMapper.transform,
 * src/mojotrees/binning.mojo:3565-4047, :3264): out_bins is n_features *
 * n_rows uint8, out_missing_bin n_features (-1: none reserved). */
int32_t mbh_bin_dense(const double *data, int64_t n_rows, int32_t n_features,
                      int32_t max_bins, int32_t min_data_in_bin,
                      int32_t use_missing, int64_t sample_cnt, int64_t seed,
                      uint8_t *out_bins, int32_t *out_missing_bin, char *err,
                      int32_t err_len);
/* The same with categorical features (categorical.fit_categorical_spec,
 * src/mojotrees/categorical.mojo:419-464): the n_categorical features listed
 * in `categorical` are fitted as category tables over all rows -- code c of
 * the feature's kept codes (at most max_bins - 1, the most frequent) in bin
 * 1 + its rank, missing (negative, NaN), unseen and dropped codes in bin 0 --
 * and out_n_categories[f] receives each feature's category count (0 for a
 * numerical feature). */
int32_t mbh_bin_dense_cat(const double *data, int64_t n_rows, int32_t n_features,
                          int32_t max_bins, int32_t min_data_in_bin,
                          int32_t use_missing, int64_t sample_cnt, int64_t seed,
                          const int32_t *categorical, int32_t n_categorical,
                          uint8_t *out_bins, int32_t *out_missing_bin,
                          int32_t *out_n_categories, char *err, int32_t err_len);

/* mbh_bin_dense_cat with the per-value transform on the GPU: the fit runs
 * on the host as above, the column-major doubles are copied to the device and
 * mapped there (BinMapper.transform, src/mojotrees/binning.mojo:3264-3330,
 * bin_value :3242-3262; categorical codes by CategoricalSpec.bin_of,
 * src/mojotrees/categorical.mojo:296-322), and the bins copied back; the
 * result is byte-identical to mbh_bin_dense_cat's. n_categorical may be 0
 * (categorical NULL); out_n_categories may be NULL. out_times_ms, when not
 * NULL, receives 4 values: the host fit, the host-to-device copy, the
 * transform kernel and the device-to-host copy, in milliseconds. */
int32_t mbh_bin_dense_device(const double *data, int64_t n_rows, int32_t n_features,
                             int32_t max_bins, int32_t min_data_in_bin,
                             int32_t use_missing, int64_t sample_cnt, int64_t seed,
                             const int32_t *categorical, int32_t n_categorical,
                             uint8_t *out_bins, int32_t *out_missing_bin,
                             int32_t *out_n_categories, double *out_times_ms,
                             char *err, int32_t err_len);

/* Number of usable gfx950 devices (0 without a GPU or runtime). */
int32_t mbh_device_count(void);

/* Upload a binned matrix and its labels; builds the per-row records
 * (F bin bytes + 2 gradient bytes, padded to a power of two). */
int32_t mbh_dataset_create(const uint8_t *bins_cm, int64_t n_rows,
                           int32_t n_features, int32_t n_bins,
                           const int32_t *missing_bin, const double *labels,
                           mbh_dataset **out, char *err, int32_t err_len);
void mbh_dataset_free(mbh_dataset *ds);
/* Marks categorical features of a resident dataset: n_categories[f] > 0
 * makes feature f categorical with its categories in bins 1..n_categories[f]
 * (bin 0: missing, unseen, dropped); 0 keeps it numerical. Training then
 * searches that feature as category sets (categorical.
 * find_best_categorical_split, src/mojotrees/categorical.mojo:684-782) and a
 * categorical node routes its set left and every other bin right. Served on
 * the quantized-gradient path. */
int32_t mbh_dataset_set_categorical(mbh_dataset *ds, const int32_t *n_categories,
                                    char *err, int32_t err_len);

/* Train on a resident dataset: quantized gradients with integer histograms,
 * or fp32 gradients with fp64 histogram sums (use_quantized_grad = 0). */
int32_t mbh_train(mbh_dataset *ds, const mbh_params *params, mbh_fit **out,
                  char *err, int32_t err_len);
void mbh_fit_free(mbh_fit *fit);
int32_t mbh_fit_num_trees(const mbh_fit *fit);
int32_t mbh_fit_num_class(const mbh_fit *fit);
int64_t mbh_fit_total_nodes(const mbh_fit *fit);
void mbh_fit_arrays(const mbh_fit *fit, double *base, int64_t *node_offset,
                    int32_t *feature, int32_t *threshold_bin, int32_t *left,
                    int32_t *right, double *value, int32_t *default_left,
                    int32_t *missing_bin, double *split_gain, double *count);
/* Category sets, 4 words per node in mbh_fit_arrays' order: the bins a
 * categorical node (threshold_bin -1) routes left; zero elsewhere. */
void mbh_fit_cat_bits(const mbh_fit *fit, uint64_t *out);
/* Final raw scores of the training rows, row-major n_rows * num_class. */
int32_t mbh_fit_train_raw(const mbh_fit *fit, double *out, char *err,
                          int32_t err_len);
/* Training statistics. Writes min(n_out, count) values and returns count
 * (22). Milliseconds are summed HIP-event times and are filled only with
 * time_histograms=1.
 *   [0] wall seconds of the training loop (enqueue to final sync)
 *   [1] ms of the histogram-accumulating kernels (root build + expansions)
 *   [2] histogram algorithmic bytes of the committed trees: (root rows + the
 *       smaller child of every split) * (n_features + gh), gh = 2 for int8
 *       g/h (use_quantized_grad=1), 8 for fp32 g/h
 *   [3] the same rows * n_features    [4] builds of the committed trees
 *   [5] root-build algorithmic bytes  [6] root-build ms   [7] trees grown
 *   [8] ms of every growth kernel (accumulation + merge/scan/plan)
 *   [9] the same for the root build
 *   [10] expansion launches that did work   [11] leaves expanded (including
 *        speculative expansions the best-first replay discarded)
 *   [12] rows accumulated by expansions     [13] parent rows partitioned
 *   [14] expansion iterations enqueued
 *   [15] ms of their partition and accumulation launches
 *   [16] their algorithmic bytes: [13] * 9 (row id in, bin, row id out)
 *        + [12] * (n_features + gh)
 *   [17] ms of the partition launches   [18] ms of the accumulation launches
 *   [19] the accumulations' algorithmic bytes: [12] * (n_features + gh)
 *   [20] bytes of the quantizer fused into the root build, not in [2] or
 *        [5]: root rows * 10 (binary32 g, h read, int8 pair written) when
 *        the root build quantizes (max-abs lattice), else 0
 *   [21] the partitions' algorithmic bytes: [13] * 9 with row ids; with
 *        records [13] * 2 * record bytes + root rows * 2 (the root's pairs) */
int32_t mbh_fit_stats(const mbh_fit *fit, double *out, int32_t n_out);

/* Per expansion launch of a time_histograms=1 fit, six values each: tree,
 * expansion iteration, rows partitioned, rows accumulated (from the
 * planner's batch; 0 for the empty launches after a tree is done), and the
 * partition and accumulation kernels' durations in ms. Writes min(n_out,
 * count) values and returns count (6 per launch; 0 for untimed fits). */
int64_t mbh_fit_launch_log(const mbh_fit *fit, double *out, int64_t n_out);

/* Query groups of a resident dataset, for objective lambdarank: counts[q]
 * rows per query, in row order (LightGBM's `group`,
 * ranking.groups_from_counts, src/mojotrees/ranking.mojo:152-169); counts must
 * be positive and sum to n_rows, and a query holds at most 2^30 rows
 * (queries above 2048 rows are sorted in global memory rather than LDS). */
int32_t mbh_dataset_set_groups(mbh_dataset *ds, const int32_t *counts, int64_t n_queries,
                               char *err, int32_t err_len);

/* Per-row sample weights of a resident dataset (the `sample_weight` of
 * mojotrees_train_dense, include/capi/mojotrees.h; checked as
 * boosting._check_sample_weight, src/mojotrees/boosting.mojo:334-343: one
 * finite, nonnegative weight per row, positive sum). Every later mbh_train
 * scales each row's gradient and hessian by its weight after the hessian
 * floor (boosting._fill_grad_hess_into, boosting.mojo:676-811) and boosts
 * from the weighted mean or weighted class shares. weights == NULL clears
 * them. Not served with objective lambdarank (MOJOTREES_ERROR_UNSUPPORTED). */
int32_t mbh_dataset_set_weights(mbh_dataset *ds, const double *weights, int64_t n_weights,
                                char *err, int32_t err_len);

/* LambdaRank gradients and hessians (binary64) of one set of raw scores on
 * the device (ranking.lambdarank_gradients, src/mojotrees/ranking.mojo:
 * 603-654), with the dataset's labels and groups, scaled by its sample
 * weights when mbh_dataset_set_weights gave it some. */
int32_t mbh_lambdarank(mbh_dataset *ds, const mbh_params *params, const double *raw,
                       double *grad, double *hess, char *err, int32_t err_len);

/* A ranker through the C ABI's model type: bins the column-major matrix with
 * the parameters' max_bin (as mojotrees_train_dense does), trains objective
 * lambdarank on the device over query groups (group_counts, one row count
 * per query) and returns a MojoTreesModel that every mojotrees_* function
 * takes (raw-score predictions, v4 save/load with objective 7). The
 * reference serves its ranker only from Python (MojoTreesRanker,
 * python/mojotrees/sklearn.py:6951); this entry is what an estimator or a C
 * caller uses here. Parameters as for mojotrees_train_dense plus
 * lambdarank_truncation_level, sigmoid, lambdarank_norm. weights: per-row
 * sample weights scaling each finished lambda and hessian (train_ranker's
 * sample_weight, ranking.mojo:613-616), or NULL. bagging_fraction /
 * bagging_freq bag whole queries (ranking._refresh_query_bag,
 * ranking.mojo:667-686). */
struct MojoTreesModel;
struct MojoTreesError;
int32_t mbh_train_ranker_dense(const double *data, int64_t n_rows, int64_t n_features,
                               const double *labels, const double *weights,
                               const int32_t *group_counts,
                               int64_t n_groups, const char *parameters,
                               struct MojoTreesModel **out_model, struct MojoTreesError *error);

/* Save with feature names, as the reference's estimators do
 * (bindings/_mojotrees.mojo:4931 `save(model, path, names, n)` over
 * serialize.save_model(model, path, feature_names),
 * src/mojotrees/serialize.mojo:999-1030): the v4 file gains the optional
 * `feature_names` section. n_names 0 writes none; otherwise it must equal the
 * model's feature count. Names may hold any bytes but other control bytes
 * than tab, newline and carriage return (MOJOTREES_ERROR_IO). */
int32_t mbh_save_model_named(const struct MojoTreesModel *model, const char *path,
                             const char *const *names, int64_t n_names,
                             struct MojoTreesError *error);
/* The feature names a model file carries (serialize.load_feature_names,
 * src/mojotrees/serialize.mojo:1448-1460; bindings/_mojotrees.mojo:4968):
 * *out_count names, back to back as NUL-terminated strings in *out_names
 * (free with mojotrees_string_free); 0 and NULL when the file has none. */
int32_t mbh_model_feature_names(const char *path, char **out_names, int64_t *out_count,
                                struct MojoTreesError *error);

/* Raw scores on the device (Booster.predict_raw_row,
 * src/mojotrees/boosting.mojo:1722-1760; the reference's device counterpart is
 * _predict_kernel, src/mojotrees/gpu_predict.mojo:206, in Float32). bins_cm is
 * the column-major uint8 matrix (n_rows x n_features) the model's bin mapper
 * produced; trees [tree_begin, tree_end) of a flat ensemble laid out as
 * mbh_fit_arrays does (tree_begin a multiple of num_class). base: num_class
 * scores added first, or NULL for a range that starts after iteration 0. out:
 * row-major n_rows x num_class, bit-identical to the host predictor (fused
 * multiply-adds in ascending tree order). cat_bits: 4 words per node, the
 * left set of a categorical node (threshold -1), or NULL without any. */
int32_t mbh_predict_binned(const uint8_t *bins_cm, int64_t n_rows, int32_t n_features,
                           int32_t num_class, double learning_rate, const double *base,
                           const int64_t *node_offset, int64_t tree_begin, int64_t tree_end,
                           const int32_t *feature, const int32_t *threshold,
                           const int32_t *left, const int32_t *right, const double *value,
                           const int32_t *default_left, const int32_t *missing_bin,
                           const uint64_t *cat_bits, double *out, char *err, int32_t err_len);

/* ------------------------------------------- stage-level (parity, bench) */
/* Device exp and sigmoid of x[0..n). */
int32_t mbh_exp_sigmoid(const double *x, int64_t n, double *out_exp,
                        double *out_sigmoid, char *err, int32_t err_len);

/* One round's gradient pass and quantizer on a resident dataset, from the
 * given raw scores (n_rows): writes narrowed grad/hess, int8 q_grad/q_hess and
 * scales[0..1] = grad units, hess units. */
int32_t mbh_objective_quantize(mbh_dataset *ds, const mbh_params *params,
                               const double *raw, int64_t round_index,
                               float *grad, float *hess, int8_t *q_grad,
                               int8_t *q_hess, double *scales, char *err,
                               int32_t err_len);

/* The same for either lattice with int32 outputs: with quant_scale_rule 1
 * (the magnitude-sum lattice) q_grad/q_hess receive the 2^30-lattice values
 * (with quant_staging 1, the staged int16 values) and scales[2..3] the
 * device magnitude sums (sum |g|, sum |h|) the scales came from, and with
 * quant_staging 1 scales[4..5] the counts of grad and hess values that did
 * not fit int16; scales holds 6 doubles. */
int32_t mbh_objective_quantize32(mbh_dataset *ds, const mbh_params *params,
                                 const double *raw, int64_t round_index, float *grad,
                                 float *hess, int32_t *q_grad, int32_t *q_hess,
                                 double *scales, char *err, int32_t err_len);

/* Histogram of the magnitude-sum lattice (int32 values per row, hessians
 * nonnegative, the selection's sums of |q| below 2^31) over `rows[0..n_sel)`
 * (all rows when rows is NULL): out is n_features * n_bins * 3 int32
 * {grad, hess, count}. */
int32_t mbh_histogram32(mbh_dataset *ds, const int32_t *q_grad, const int32_t *q_hess,
                        const int32_t *rows, int64_t n_sel, int32_t *out, char *err,
                        int32_t err_len);

/* Histogram of the rows `rows[0..n_sel)` (all rows when rows is NULL) with the
 * given int8 q_grad/q_hess: out is n_features * n_bins * 3 int32
 * {grad, hess, count}. */
int32_t mbh_histogram(mbh_dataset *ds, const int8_t *q_grad,
                      const int8_t *q_hess, const int32_t *rows,
                      int64_t n_sel, int32_t num_grad_quant_bins,
                      int32_t *out, char *err, int32_t err_len);

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): the histogram of mbh_histogram, computed from the
 * caller's DEVICE buffers without any allocation. bins_cm: n_rows x
 * n_features column-major uint8 bins (< n_bins); q_grad, q_hess: n_rows
 * int8 each (|q_grad| <= B/2 + 1, 0 <= q_hess <= B + 1, B =
 * num_grad_quant_bins); rows: n_sel row ids, or NULL for every row; out:
 * n_features * n_bins * 3 int32 {grad, hess, count}, fully written; status:
 * NULL or one int32 set to 0, then to 1 when an entry was out of range (a
 * row id, a quantized pair, a bin id), which is then left out. Enqueued on
 * `stream` (a hipStream_t, NULL for the default stream); returns without
 * waiting. Block partials live in a static device array of
 * MBH_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends: one
 * partial of n_features * n_bins * 8 bytes must fit it, and sizes beyond it
 * are refused (MOJOTREES_ERROR_INVALID_ARGUMENT). Calls that overlap on one
 * GPU share that array and race. */
#define MBH_NOALLOC_SCRATCH_BYTES (16u << 20)
int32_t mbh_histogram_noalloc(const uint8_t *bins_cm, int64_t n_rows, int32_t n_features,
                              int32_t n_bins, const int8_t *q_grad, const int8_t *q_hess,
                              const int32_t *rows, int64_t n_sel, int32_t num_grad_quant_bins,
                              int32_t *out, int32_t *status, void *stream, char *err,
                              int32_t err_len);

/* fp32-gradient histogram of the rows `rows[0..n_sel)` (all rows when rows
 * is NULL) with the given fp32 grad/hess (n_rows each), summed in fp64 on the
 * device: out_gh is n_features * n_bins * 2 doubles {grad, hess} per cell,
 * out_count n_features * n_bins counts. The reference's Float64 histogram
 * (histogram.mojo:1002, build_histogram_subset_into :2038). */
int32_t mbh_histogram_fp32(mbh_dataset *ds, const float *grad, const float *hess,
                           const int32_t *rows, int64_t n_sel, double *out_gh,
                           int64_t *out_count, char *err, int32_t err_len);

/* Root histogram of all rows, `reps` times back to back on resident data
 * (HIP events): out_ms[0] mean histogram-kernel milliseconds, out_ms[1] its
 * min, out_ms[2] mean milliseconds of histogram + the scan kernel that
 * merges its partials. out_ms has 3 entries. */
int32_t mbh_bench_root_histogram(mbh_dataset *ds, int32_t reps,
                                 double *out_ms, char *err, int32_t err_len);

#ifdef __cplusplus
}
#endif

#endif /* MOJOBOOST_HIP_H */
