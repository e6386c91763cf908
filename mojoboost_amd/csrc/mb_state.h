// Device-resident state of one training run on one GPU.
//
// The tree grows entirely on the device: every kernel reads what it needs
// (the leaves to expand, their row ranges and splits) from the per-item
// tables the planning kernel wrote, so the host enqueues a
// tree without reading anything back except a done flag between groups of
// launches. The host downloads the finished trees once, at the end of
// training.
#pragma once

#include <stdint.h>

namespace mb {

constexpr int kObjL2 = 0;
constexpr int kObjBinary = 1;
constexpr int kObjMulticlass = 2;
constexpr int kObjLambdarank = 3;
constexpr int kMaxQueryRows = 2048;  // the largest query the LDS sort takes (larger: k_lambdarank_big)

// Leaf-wise growth, batched. The reference grows a tree best-first: split the
// frontier leaf of largest gain, score both children, repeat. A leaf's best
// split depends only on its own rows and depth, so the tree it produces is
// fixed by the set of leaves' best splits alone; the order only decides which
// splits make the num_leaves cut and how nodes are numbered. Here several
// frontier leaves are expanded per launch (the highest-gain ones, some of
// them speculatively), and a single-block replay of the best-first order over
// the expanded leaves commits splits in the reference's order, assigning its
// node ids and frontier slots. Expansions the replay never reaches are
// discarded; the tree is the reference's.

// A node of the explored tree (every leaf ever created in this tree).
struct ENode {
    int64_t begin, end;          // row range in row buffer `buf`
    int64_t n_left;              // rows on the left side of the best split
    int64_t tot_g, tot_h, tot_c; // integer sums of the node's rows
    double gain;                 // best split gain (valid when found)
    double value;                // leaf output
    int32_t buf, hist, depth;
    int32_t found, feature, bin, default_left;
    int32_t left_e, right_e;     // explored children, -1 until expanded
    int32_t cat;                 // 1: the best split is a category set (e_cat holds it)
};

// One leaf expanded by a launch of the partition+histogram and scan kernels.
struct Item {
    int64_t begin, end;     // the parent's range in row buffer src_buf
    int64_t n_left;         // rows routed left (exact, from the parent's scan)
    int32_t parent_e, left_e;   // right child = left_e + 1
    int32_t src_buf;        // children land in the other buffer, same range
    int32_t builds_left;    // the smaller child (left on ties) is accumulated
    int32_t hist_built;     // histogram buffer of the accumulated child (new)
    int32_t hist_sib;       // the parent's buffer; the sibling is written over it
    int32_t depth_child;
    int32_t part_off, part_cnt;  // block partials of the accumulated child
    int32_t pad_;
};

// A batch item's partition work: its parent range [begin, begin + m) of
// row buffer src_buf, split into tasks of the batch's chunk_p rows numbered
// from qoff (task t of the batch belongs to the last item with qoff <= t).
struct PartItem {
    int64_t begin, n_left, m;
    int32_t qoff, src_buf, feature, bin, default_left, missing_bin;
    int32_t cat_e;  // categorical split: the explored node whose e_cat set routes left; -1 numerical
    int32_t direct; // 1: the parent is the root over every row in order (row id = position, no list read)
    int32_t root;   // 1: the parent is the round's root (record partition: read the dataset's records)
    int32_t pad_;
};

// A batch item's accumulation work: its accumulated child, rows [lo, hi) of
// row buffer `buf`, in tasks of the batch's chunk_a rows numbered from poff
// (one block partial each).
struct AccItem {
    int64_t lo, hi;
    int32_t poff, buf;
};

// Written by the planner; the host reads it back between launch groups.
struct Batch {
    int32_t n_items;   // 0: nothing to do this iteration
    int32_t n_blocks;  // partition tasks in use
    int32_t done;      // the tree is complete
    int32_t iters;     // expansion iterations planned so far in this tree
    int32_t n_acc;     // accumulation tasks (block partials) in use
    int32_t chunk_p;   // parent rows per partition task
    int32_t chunk_a;   // accumulated rows per accumulation task
    int32_t pad_;
};

// Replay state of the best-first order (touched by the planning block only).
struct Grow {
    int32_t n_leaves, n_nodes;  // of the committed (reference) tree
    int32_t n_explored;         // ENode entries in use
    int32_t n_hist;             // histogram buffers in use
    int32_t expansions;
    int32_t iterations;
    int64_t rows_built;         // rows accumulated by this tree's expansions
    int64_t rows_parted;        // parent rows routed by this tree's expansions
};

// Best candidate of one (child, feature) scan.
struct ScanResult {
    double gain;
    int32_t bin, default_left, found;
    int32_t cat;  // 1: a category set (scan_cat holds it), bin -1
    int64_t tot_g, tot_h, tot_c;  // integer sums (quantized path; tot_c on both)
    int64_t n_left;  // rows left of the candidate
    double fg, fh;   // fp64 serial sums over the feature's bins (fp32 path's leaf value)
};

// One cell of an fp64 histogram (fp32 gradient path).
struct HistF {
    double g, h;
    int64_t c;
};

// Per-round values shared by the kernels of one tree, advanced on the device
// by the score-update kernel so a captured tree graph is the same every round.
struct Round {
    int64_t round;       // boosting iteration
    int32_t class_k;     // class of this tree (0 for single output)
    int32_t tree_index;  // position in the ensemble
    int32_t parity;      // which magnitude-stats pair this tree uses
    int32_t stopped;     // training stopped (boosting._boost_rounds' stop rule): later trees do nothing
    int32_t progress;    // a tree of the current multiclass round split or moved
    int32_t sampled;     // the root range is the row list rows0[0 .. cursor[0]) (bag or GOSS sample)
    double grad_units, hess_units;
    double goss_mult;    // GOSS weight of the sampled small-gradient rows (1 when off)
};

// Parent rows of a partition task: at most kPartChunk (one task per block
// pass), at least kPartChunkMin (the host bounds a batch's task count by
// it). The planner spreads a batch over about part_target tasks in between,
// in multiples of kPartChunkStep rows.
#ifndef MB_PART_CHUNK
#define MB_PART_CHUNK 4096
#endif
constexpr int kPartChunk = MB_PART_CHUNK;
#ifndef MB_PART_CHUNK_MIN
#define MB_PART_CHUNK_MIN 512
#endif
constexpr int kPartChunkMin = MB_PART_CHUNK_MIN;
constexpr int kPartChunkStep = 256;
// Rows one fp32-path histogram block may add: its counts are 16-bit halves
// of 32-bit LDS cells.
constexpr int64_t kFAccChunk = 65535;
// Threads of a record-partition block (leaves holding records); its tasks
// take at most kPartRecChunk rows (kPartRows per thread).
#ifndef MB_PART_REC_THREADS
#define MB_PART_REC_THREADS 512
#endif
constexpr int kPartRecThreads = MB_PART_REC_THREADS;
constexpr int kPartChunkRoot = 16384;  // at most, per task of the root's batch (its own launch)
// Root build launch: kHistThreads per block, kHistBlocksPerCU blocks per CU
// (each with its own LDS histogram).
#ifndef MB_HIST_THREADS
#define MB_HIST_THREADS 1024
#endif
#ifndef MB_HIST_BPC
#define MB_HIST_BPC 1
#endif
constexpr int kHistThreads = MB_HIST_THREADS;
constexpr int kHistBlocksPerCU = MB_HIST_BPC;

// Rows per tile of the GOSS count; the kappa buffer is padded to whole tiles.
constexpr int kGossTileRows = 16384;
constexpr int kGossHistSlots = 8;  // partial digit histograms per radix pass
constexpr int kStatSlots = 64;  // slots of each max |g|, |h| (parity x grad/hess x slot)
// blocks of a radix-select pass, each a contiguous row range (C3: 2048 ran
// 0.5 % faster per 500 trees than 1024 or 4096)
constexpr int kGossDigitBlocks = 2048;

// The state of a run before its first tree: no sampling, unit GOSS weight.
inline Round initial_round() {
    Round r{};
    r.goss_mult = 1.0;
    return r;
}

// The Round of each state growing a multiclass round's class trees side by
// side (at most kMaxClassStates; measured on C5's 10 classes, one MI355X:
// 2 states 0.90, 3 states 0.79, 4 states 0.90, 5 states 0.82 s per 100
// rounds, against 1.32 s for the classes in turn).
#ifndef MB_CLASS_STATES
#define MB_CLASS_STATES 3
#endif
constexpr int kMaxClassStates = MB_CLASS_STATES;
struct RoundStates {
    Round *r[kMaxClassStates];
    int32_t n;
};

// GOSS selection of one round (goss.mojo:294-396).
struct GossState {
    unsigned long long prefix;  // radix select: high bits of the threshold found so far
    int64_t rank;               // remaining rank (0-based, descending) inside the prefix
    int64_t top_k, other_k;
    double threshold;           // top_k-th largest |g h|
    int64_t kept_other;         // rows kept by the selection sampling
    int64_t bag_n;              // top + kept rows
    int64_t n_uncertain;        // rows whose keep decision the predicted count band left open
    int32_t fallback;           // 1: the band's decisions failed the check (or were not used)
    int32_t pad_;
};

struct HyperParams {
    int32_t objective;
    int32_t num_class;
    // class trees a state grows per round: 1, every class in turn; S > 1,
    // one of S states grown side by side on its own stream, this state's
    // classes c, c + S, c + 2 S, ... (its first class c, its Round's
    // class_k at the start of a round)
    int32_t class_stride;
    int32_t pad_cs_;
    int32_t num_leaves;
    int32_t min_data_in_leaf;
    int32_t max_depth;
    int32_t quant_bins;
    int32_t stochastic;
    int32_t quant_seed;
    int32_t const_hessian;
    int32_t bagging;        // 1: rows sampled per bag
    int32_t quantized;      // 1: quantized gradients, integer histograms; 0: fp32 gradients, fp64 sums
    // quantized lattice: 0 LightGBM's max-abs rule (int8 pair in each record,
    // packed 64-bit LDS counters), 1 the reference's magnitude-sum
    // power-of-two rule (int32 pair per row in `gq`, 2^30 lattice, int32 LDS
    // sums: derive_scales with SCALE_MAGNITUDE_SUM, quantized_gradient.mojo:
    // 1343-1453, and _quantize_grad_hess_kernel, gpu_active_rows.mojo:
    // 2211-2255)
    int32_t wide;
    // magnitude-sum lattice, the reference's packed Int16 staging arm
    // (QUANT_SOURCE_PACKED16, gpu_active_rows.mojo:2257-2395): each row's
    // pair narrowed to int16 in its record's last four bytes, with per-plane
    // counts of the values that did not fit
    int32_t stage16;
    int32_t goss;           // 1: GOSS from round goss_warm on
    int32_t goss_warm;
    int32_t goss_seed;
    int32_t goss_exact;     // 1: always the full sequential count (no predicted band)
    double goss_band;       // band half-width in standard deviations of the count
    int32_t grad64;         // 1: derivatives kept in binary64 (lambdarank), else narrowed to fp32
    int32_t rank_trunc;     // lambdarank_truncation_level
    int32_t rank_norm;      // lambdarank_norm
    int32_t pad_rank_;
    double rank_sigma;      // lambdarank sigmoid
    double top_rate, other_rate;
    int32_t bagging_freq;
    int32_t bagging_seed;
    double bagging_fraction;
    double learning_rate;
    double lambda_l1, lambda_l2, min_sum_hessian;
    // categorical splits (categorical.CategoricalParams, LightGBM names)
    int32_t max_cat_to_onehot, max_cat_threshold, min_data_per_group, one_hot_max_size;
    double cat_smooth, cat_l2;
};

// Everything the kernels touch, passed by value.
struct DevState {
    // data (resident for the whole fit)
    // n_tiles x n x rec_bytes, tile-major: tile t holds features
    // [t * tile_f, t * tile_f + tile_f) of a row, zero pad, then q_grad,
    // q_hess in its last two bytes (every tile carries the pair)
    const uint8_t *records;
    const uint8_t *bins_cm;  // F x n, column-major (partition, score update)
    const double *labels;    // n
    const uint8_t *labels8;  // n, when every label is an integer in [0, 255] (else null)
    const double *weights;   // n sample weights, or null (unweighted)
    const int32_t *qid;      // n: each row's query when lambdarank bags by query, else null
    const int64_t *bag_fallback;  // per bag index: the unit an empty bag takes, or -1 (null: none)
    int64_t n_bags;               // entries of bag_fallback
    const int32_t *missing_bin;  // F
    const int32_t *widths;       // F: realized bin count bound
    const int32_t *ncat;         // F: categories of a categorical feature (bins 1..ncat), 0 numerical; null: none
    const int32_t *scan_order;  // F, with ncat: scan task order of the features (category-set ones first)
    const uint8_t *feature_mask; // num_trees x F (1: the tree may split it)
    uint8_t *records_w;          // same buffer as records, writable view
    // Record partition (rcp = 1): a leaf's rows are held as their records,
    // contiguous in the leaf's range [begin, end) of crec0 / crec1 (the
    // leaf's buf), each with the round's int8 pair in its last two bytes; the
    // partition moves whole records to the children's ranges and the
    // accumulation streams them, so no row id is read below the root. The
    // root build writes each root row's pair to `pairs` (2 bytes per row)
    // instead of into the dataset's records, and the root's partition reads
    // the dataset's records (by position or through the root list) with
    // their pairs. rcp = 0: leaves hold row ids in rows0 / rows1 and every
    // record is gathered by id.
    uint8_t *crec0, *crec1;      // n x rec_bytes each (rcp)
    uint16_t *pairs;             // n: the root rows' int8 (grad, hess) pairs (rcp)
    int32_t rcp;
    int32_t pad_rcp_;
    int64_t n;
    int32_t n_features;
    int32_t n_bins;        // histogram stride per feature
    int32_t rec_bytes;     // bytes of one row's record in one tile (16..128)
    int32_t tile_f;        // features per tile (the last tile may hold fewer)
    int32_t n_tiles;
    int32_t lds_stride;    // per-feature LDS stride (odd, >= n_bins)
    // per round
    double *raw;           // n x num_class
    double *prob;          // n x num_class softmax of raw at the start of a round (multiclass)
    float *grad, *hess;    // n (not written when gh2 is set)
    // the fp32 path's binary32 derivatives, (g, h) interleaved per row (one
    // gather per accumulated row); h's sign bit is set when the round's GOSS
    // sample took the row with the GOSS weight (hessians are >= 0)
    float *gh2;            // 2n: g at 2r, h at 2r + 1
    double *grad64, *hess64;        // n, when hp.grad64
    unsigned long long *stats64;    // [2 parities][2]: max |g|, |h| as double bits, when hp.grad64
    // lambdarank: query q owns rows [qstart[q], qstart[q + 1])
    const int64_t *qstart;
    const double *inv_max_dcg;      // per query: 1 / maxDCG at the truncation level (0: none)
    const double *rank_disc;        // 1 / log2(rank + 2) for ranks below the largest query
    int32_t n_queries;
    int32_t rank_pad;               // largest query of at most kMaxQueryRows rows, rounded up to a power of two
    // queries of more than kMaxQueryRows rows (k_lambdarank_big): their
    // indices, and per block slot the query's keys, G, H (binary64) and
    // positions, labels (int32), each rank_big_pad long
    const int32_t *rank_big;
    int32_t n_big;
    int32_t rank_big_pad;
    int32_t rank_big_slots;         // blocks of k_lambdarank_big (one slot each)
    int32_t pad_big_;
    double *rank_scratch;           // slots x 3 x rank_big_pad
    int32_t *rank_scratch_i;        // slots x 2 x rank_big_pad
    uint32_t *stats;       // [2 parities][2][kStatSlots]: max |g|, max |h| as float bits, per slot
    // magnitude-sum lattice (hp.wide): each row's quantized (grad, hess)
    // interleaved, and the magnitude reduction's 256 + 256 binary32
    // workgroup sums (|g| then |h|)
    int32_t *gq;
    float *magpart;
    unsigned long long *stage16_over;  // [2]: grad and hess values outside int16 (stage16)
    Round *round;
    // rows and histograms
    int32_t *rows0, *rows1;
    int32_t *hist;         // (1 + max_exp) x F x n_bins x 3 (grad, hess, count)
    unsigned long long *part;  // max(hist_grid, pb_grid) x F x part_stride packed partials
    uint32_t *part_c;          // magnitude-sum lattice: the partials' counts (part holds grad | hess)
    HistF *histf;              // fp32 path: (1 + max_exp) x F x n_bins cells
    double *fpart_g, *fpart_h; // fp32 path partials, same shape as part
    uint32_t *fpart_c;
    int32_t hist_grid;         // blocks of a histogram launch
    int32_t part_stride;       // per-feature stride of a partial (even, >= n_bins)
    int64_t hist_chunk_min;    // fewest rows a histogram block takes
    int64_t hist_chunk_limit;  // most rows a block may pack (field bounds)
    // GOSS (fp32 path)
    GossState *gst;
    uint32_t *goss_hist;        // 8 passes x kGossHistSlots x 256 digit counts
    unsigned long long *goss_sel;   // 8 x (prefix, rank): the radix select's state after each pick
    unsigned long long *goss_cand;  // n: per select block, the keys that match the 16-bit prefix
    int32_t *goss_ccnt;         // kGossDigitBlocks: their counts
    int32_t *goss_kappa;        // n: top row -> INT_MIN, else the count bound of the sampling
    unsigned long long *goss_mask;  // ceil(n / 64): rows kept by the sampling
    unsigned long long *goss_topmask;  // ceil(n / 64): top rows (importance at or above the threshold)
    int32_t *goss_blk;          // per 1024-row block counts, then their exclusive prefix
    int32_t *goss_blk_u;        // per block: rows the band leaves open, then their prefix
    int32_t *goss_ukappa;       // the open rows in row order: kappa - certain keeps before it
    int32_t *goss_urow;         // their row ids
    unsigned long long *goss_umask; // the open rows' decisions, one bit per list position
    uint8_t *goss_other;        // n: 1 when the row was kept by the sampling (weighted)
    int32_t *goss_rows;         // n: the round's sample, ascending (copied to the root list per tree)
    double *goss_imp;           // n (multiclass): the round's importance, summed over the classes
    unsigned long long *goss_max;  // 2 x 2: max |g|, |h| of the weighted sample (binary64 bits), by parity
    int32_t goss_nblk;
    int32_t pad_goss_;
    // growth
    ENode *enodes;         // e_cap
    double *e_gain;        // e_cap: best gain when > 0 and found, else -1 (planner's view)
    int32_t *e_left;       // e_cap: left child (right = left + 1), -1 while unexpanded
    int32_t *e_parent;     // e_cap: parent, -1 for the root
    int32_t *e_rows;       // e_cap: rows of the node (n < 2^31)
    Item *items;           // kmax
    PartItem *part_items;  // kmax: the batch's partition work per item
    AccItem *acc_items;    // kmax: the batch's accumulation work per item
    Batch *batch;
    Grow *grow;
    int32_t *slot_e;       // num_leaves: explored node of each frontier slot
    int32_t *slot_fid;     // num_leaves: its node id in the committed tree
    ScanResult *scan;      // kmax x 2 x F
    double *scan_gain;     // kmax x 2 x F: a result's gain when found, else -1 (all the planner's fold reads)
    // more than 64 features: each pair's best gain (0: none) and its feature
    // (0x7FFFFFFF: none), folded by k_fold for the planner
    double *pair_gain;     // 2 x kmax
    int32_t *pair_feat;    // 2 x kmax
    unsigned long long *scan_cat;  // kmax x 2 x F x 4: a categorical result's left set
    unsigned long long *e_cat;     // e_cap x 4: an explored node's categorical left set
    int64_t *cursor;       // [0] root bag size; [2 + 2j], [3 + 2j]: item j's output cursors
    int32_t *error;        // sticky error flag (partition overflow)
    int32_t kmax;          // most leaves expanded per launch
    int32_t max_exp;       // most expansions per tree (2 num_leaves - 1)
    int32_t e_cap;         // ENode capacity (1 + 2 max_exp)
    int32_t pb_grid;       // most accumulation tasks (block partials) of a batch
    int32_t part_grid;     // most partition tasks of a batch
    int32_t scan_grid;     // blocks of a scan launch
    int32_t pb_launch;     // blocks of an accumulation launch (grid-strided)
    int32_t part_launch;   // blocks of a partition launch (grid-strided)
    int32_t part_target;   // partition tasks a batch is spread over
    int32_t part_root;     // 1: the root's batch takes its own launch of kPartChunkRoot-row tasks
    // tree being grown (max 2 * num_leaves - 1 nodes)
    int32_t *t_feature, *t_threshold, *t_left, *t_right, *t_default_left, *t_missing_bin;
    double *t_value, *t_gain, *t_count;
    unsigned long long *t_cat;  // max_nodes x 4: left set of a categorical node, zero elsewhere
    int32_t *t_meta;       // [0] n_nodes, [1] n_leaves
    // archive of finished trees (downloaded at the end)
    int32_t *arc_int;      // per tree: max_nodes x 6 ints + 2 meta
    double *arc_dbl;       // per tree: max_nodes x 3 doubles
    int64_t *arc_aux;      // per tree: rows accumulated, iterations, expansions, 0
    // per (tree, expansion iteration): the rows the iteration's batch
    // partitions and accumulates, written by the planner when it plans the
    // batch (time_histograms runs only; null otherwise)
    int64_t *iter_log;
    int32_t iter_stride;   // iterations per tree in iter_log
    int32_t pad_log_;
    unsigned long long *arc_cat;  // per tree: max_nodes x 4 (when a feature is categorical)
    int32_t max_nodes;
    HyperParams hp;
};

}  // namespace mb
