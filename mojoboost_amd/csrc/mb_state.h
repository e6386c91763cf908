// Device-resident state of one training run on one GPU.
//
// The tree grows entirely on the device: every kernel reads what it needs
// (which leaf to split, its row range, the split) from a step descriptor that
// the previous split kernel wrote, so the host enqueues a whole tree without
// reading anything back. The host downloads the finished trees once, at the
// end of training.
#pragma once

#include <stdint.h>

namespace mb {

constexpr int kObjL2 = 0;
constexpr int kObjBinary = 1;
constexpr int kObjMulticlass = 2;

// One split of the leaf-wise growth loop. Written by the last block of the
// split kernel (the "pick"), read by the partition, histogram and split
// kernels of the next step.
struct Step {
    int32_t active;        // 0: the tree is finished, every kernel returns
    int32_t parent_slot;   // frontier slot being split; the left child keeps it
    int32_t new_slot;      // frontier slot of the right child (= leaves so far)
    int32_t feature;
    int32_t bin;           // inclusive left threshold
    int32_t default_left;  // direction of the feature's missing bin
    int32_t missing_bin;   // -1: none
    int32_t src_buf;       // row buffer holding the parent's range
    int64_t begin, end;    // parent's range in the row buffers
    int64_t n_left;        // rows routed left, from the parent's histogram
    int32_t builds_left;   // the smaller child (left on ties) is built
    int32_t parent_hist;   // histogram buffer of the parent (sibling lands here)
    int32_t child_hist;    // histogram buffer the built child accumulates into
    int32_t depth;         // parent depth
    int32_t parent_node;
    int32_t node_left, node_right;
    int32_t pad_;
    double gain;
};

// One leaf of the frontier.
struct Slot {
    int64_t begin, end;
    int32_t node, buf, hist, depth;
    int32_t found, feature, bin, default_left;
    double gain;
};

// Best candidate of one (child, feature) scan.
struct ScanResult {
    double gain;
    int32_t bin, default_left, found, pad_;
    int64_t tot_g, tot_h, tot_c;
};

// Per-round values shared by the kernels of one tree, advanced on the device
// by the score-update kernel so a captured tree graph is the same every round.
struct Round {
    int64_t round;       // boosting iteration
    int32_t class_k;     // class of this tree (0 for single output)
    int32_t tree_index;  // position in the ensemble
    int32_t parity;      // which magnitude-stats pair this tree uses
    int32_t pad_;
    int64_t n_root;      // rows in the root range (bag size, or n)
    double grad_units, hess_units;
};

struct HyperParams {
    int32_t objective;
    int32_t num_class;
    int32_t num_leaves;
    int32_t min_data_in_leaf;
    int32_t max_depth;
    int32_t quant_bins;
    int32_t stochastic;
    int32_t quant_seed;
    int32_t const_hessian;
    int32_t bagging;        // 1: rows sampled per bag
    int32_t bagging_freq;
    int32_t bagging_seed;
    double bagging_fraction;
    double learning_rate;
    double lambda_l1, lambda_l2, min_sum_hessian;
};

// Everything the kernels touch, passed by value.
struct DevState {
    // data (resident for the whole fit)
    const uint8_t *records;  // n x rec_bytes: F bin bytes, pad, then q_grad, q_hess
    const uint8_t *bins_cm;  // F x n, column-major (partition, score update)
    const double *labels;    // n
    const int32_t *missing_bin;  // F
    const int32_t *widths;       // F: realized bin count bound
    const uint8_t *feature_mask; // num_trees x F (1: the tree may split it)
    uint8_t *records_w;          // same buffer as records, writable view
    int64_t n;
    int32_t n_features;
    int32_t n_bins;        // histogram stride per feature
    int32_t rec_bytes;
    int32_t lds_stride;    // per-feature LDS stride (odd, >= n_bins)
    // per round
    double *raw;           // n x num_class
    float *grad, *hess;    // n
    uint32_t *stats;       // [2 parities][2]: max |g|, max |h| as float bits
    Round *round;
    // rows and histograms
    int32_t *rows0, *rows1;
    int32_t *hist;         // num_leaves x F x n_bins x 3 (grad, hess, count)
    unsigned long long *part;  // hist_grid x F x n_bins packed per-block partials
    int32_t hist_grid;         // blocks of a histogram launch
    int32_t part_stride;       // per-feature stride of a partial (even, >= n_bins)
    int64_t hist_chunk_min;    // fewest rows a histogram block takes
    int64_t hist_chunk_limit;  // most rows a block may pack (field bounds)
    // growth
    Step *step;
    Slot *slots;
    ScanResult *scan;      // 2 x F
    uint32_t *ticket;      // last-block counter of the split kernel
    int64_t *cursor;       // [2]: partition output cursors
    int32_t *error;        // sticky error flag (partition overflow)
    // tree being grown (max 2 * num_leaves - 1 nodes)
    int32_t *t_feature, *t_threshold, *t_left, *t_right, *t_default_left, *t_missing_bin;
    double *t_value, *t_gain, *t_count;
    int32_t *t_meta;       // [0] n_nodes, [1] n_leaves
    // archive of finished trees (downloaded at the end)
    int32_t *arc_int;      // per tree: max_nodes x 6 ints + 2 meta
    double *arc_dbl;       // per tree: max_nodes x 3 doubles
    int64_t *arc_rows;     // per tree: rows of every histogram build (max num_leaves)
    int32_t max_nodes;
    HyperParams hp;
};

}  // namespace mb
