// Host-side pieces of the library: binning, the model container, prediction
// and the model file format. Everything here runs on the CPU around the GPU
// training path (the reference does the same: binning and the tree walk are
// host work, docs/ARCHITECTURE.md:167-195).
#pragma once

#include <stdint.h>

#include <string>
#include <vector>

namespace mb {

// A fitted bin mapper (binning.BinMapper, src/mojotrees/binning.mojo:2974):
// per feature, ascending upper edges; a value v lands in the first bin whose
// edge is >= v; NaN lands in the feature's reserved missing bin, or in the bin
// of 0.0 when it has none.
struct BinMapper {
    int n_features = 0;
    int n_bins = 255;
    std::vector<double> edges;         // concatenated
    std::vector<int64_t> edge_offsets; // n_features + 1
    std::vector<int32_t> missing_bin;  // -1: none
    // categorical.CategoricalSpec (src/mojotrees/categorical.mojo:242-323):
    // feature f's kept category codes are cat_codes[cat_offsets[f],
    // cat_offsets[f + 1]), ascending, the i-th in bin i + 1; bin 0 holds
    // missing (negative or NaN), unseen and dropped codes. Empty when no
    // feature is categorical.
    std::vector<uint8_t> is_cat;
    std::vector<int64_t> cat_codes;
    std::vector<int64_t> cat_offsets;

    bool any_cat() const;
    int n_categories(int f) const;
    int bin_of(int f, double v) const;
    // Column-major doubles -> column-major uint8 bins (threads over columns).
    void transform(const double *x, int64_t n_rows, uint8_t *out) const;
};

// binning.fit_bins with the quantile border type
// (src/mojotrees/binning.mojo:3565-4047).
// `categorical` lists the features fitted as category tables
// (fit_categorical_spec, categorical.mojo:419-464, over all rows): no edges,
// no missing bin, the max_bins - 1 most frequent codes kept.
BinMapper fit_bins(const double *x, int64_t n_rows, int n_features, int max_bins,
                   int min_data_in_bin, bool use_missing, int64_t sample_cnt, int64_t seed,
                   const std::vector<int> &categorical = {});

struct Model {
    int objective = 0;  // 0 regression (squared error), 1 binary, -1 multiclass, 7 lambdarank (raw scores)
    int num_class = 1;
    double learning_rate = 0.1;
    std::vector<double> base;  // num_class
    BinMapper mapper;
    // trees, one after another; tree t owns nodes [offsets[t], offsets[t+1])
    std::vector<int64_t> offsets{0};
    std::vector<int32_t> n_leaves;
    std::vector<int32_t> feature, threshold, left, right, default_left, missing_bin;
    std::vector<double> value, gain, count;
    // 4 words per node: the bins a categorical node routes left (tree.mojo:
    // 300-306); is_cat_node marks those nodes (threshold -1, no missing bin)
    std::vector<uint64_t> cat_bits;
    std::vector<uint8_t> is_cat_node;
    // optional file sections carried through load and save: the v4
    // `feature_names` section (serialize.mojo:389-430) and the `monotone`
    // constraint vector (serialize.mojo:964-995); empty when absent
    std::vector<std::string> feature_names;
    std::vector<int32_t> monotone;

    int64_t num_trees() const { return (int64_t)offsets.size() - 1; }
    int64_t num_iterations() const { return num_trees() / num_class; }
    // raw scores for rows of a column-major matrix, iterations [it0, it1)
    void predict_raw(const double *x, int64_t n_rows, int64_t it0, int64_t it1, double *out) const;
    // tree.goes_left (src/mojotrees/tree.mojo:483-495) for node k (model-wide index)
    bool goes_left(int64_t k, int bin) const {
        if (is_cat_node[k]) return (cat_bits[4 * (size_t)k + (bin >> 6)] >> (bin & 63)) & 1ULL;
        if (bin == missing_bin[k]) return default_left[k] != 0;
        return bin <= threshold[k];
    }
    void response(double *raw, int64_t n_rows) const;

    // v4 text file; feature_names (when not empty) and monotone are written
    // as their optional sections. Throws std::runtime_error.
    void save(const std::string &path) const;
    // v1..v4 files (serialize.mojo:1372-1500); throws std::runtime_error
    static Model load(const std::string &path);
    // the feature_names section of a model file, empty when it has none
    static std::vector<std::string> load_feature_names(const std::string &path);
    std::string dump_json() const;
};

}  // namespace mb
