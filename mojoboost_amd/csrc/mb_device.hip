// Host control plane of the device-resident trainer: dataset residency, the
// per-round kernel sequence, tree download, and the stage-level entry points
// of include/mojoboost_hip.h.
//
// A round enqueues, per tree: objective, quantize, root histogram, root scan
// and plan (which plans the first batch), then groups of [partition +
// histogram, scan, plan] iterations until the device reports the tree done,
// then the score update and round end. The host reads back only the batch
// header (done flag, iteration count), one group behind: it enqueues group
// k + 1 before waiting for group k's header, so the device does not idle
// while the host decides; launches after the tree is done find an empty
// batch and return at once.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/mojoboost_hip.h"
#include "../../include/mojotrees.h"
#include "mb_host.h"
#include "mb_kernels.h"
#include "mb_math.h"
#include "mb_state.h"

namespace {

struct Error {
    int32_t code;
    std::string msg;
};

void set_err(char *err, int32_t len, const std::string &m) {
    if (err && len > 0) std::snprintf(err, (size_t)len, "%s", m.c_str());
}

#define HIPX(expr)                                                                        \
    do {                                                                                  \
        hipError_t e_ = (expr);                                                           \
        if (e_ != hipSuccess)                                                             \
            throw Error{MOJOTREES_ERROR_TRAINING,                                         \
                        std::string("HIP error in ") + #expr + ": " + hipGetErrorString(e_)}; \
    } while (0)

template <class T>
T *dalloc(size_t count, std::vector<void *> &owned) {
    void *p = nullptr;
    size_t bytes = count * sizeof(T);
    if (bytes == 0) bytes = sizeof(T);
    HIPX(hipMalloc(&p, bytes));
    owned.push_back(p);
    return (T *)p;
}

int device_count_gfx950() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    int good = 0;
    for (int i = 0; i < n; ++i) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, i) != hipSuccess) continue;
        if (std::strncmp(prop.gcnArchName, "gfx950", 6) == 0) ++good;
    }
    return good;
}

// sampling.select_tree_features (src/mojotrees/sampling.mojo:319-465):
// selection sampling of round(F * fraction + 0.5) features (at least 2),
// keyed by (seed, tree index).
std::vector<uint8_t> tree_feature_mask(int F, double fraction, int64_t seed, int64_t tree_index) {
    std::vector<uint8_t> mask(F, 1);
    if (fraction >= 1.0) return mask;
    int count = (int)((double)F * fraction + 0.5);
    int floor_count = F >= 2 ? 2 : F;
    if (count < floor_count) count = floor_count;
    if (count > F) count = F;
    uint64_t h = mb::splitmix64((uint64_t)(seed & 0x7FFFFFFFFFFFFFFFLL));
    h = mb::splitmix64(h ^ (uint64_t)(tree_index & 0x7FFFFFFFFFFFFFFFLL));
    uint64_t stream = mb::splitmix64(h ^ 0ULL);
    std::fill(mask.begin(), mask.end(), 0);
    int chosen = 0;
    for (int i = 0; i < F && chosen < count; ++i) {
        double prob = (double)(count - chosen) / (double)(F - i);
        if (mb::uniform53(stream + (uint64_t)i) < prob) {
            mask[i] = 1;
            ++chosen;
        }
    }
    return mask;
}

}  // namespace

struct mbh_dataset {
    int64_t n = 0;
    int F = 0, nb = 0, lds_stride = 0;
    // the records' current layout (built for the last training's histogram
    // kind; rebuilt from d_bins_cm when another kind needs other tiles)
    int rec = 0, tile_f = 0, n_tiles = 0;
    int device = 0;
    int n_cu = 0;
    uint8_t *d_records = nullptr, *d_bins_cm = nullptr;
    double *d_labels = nullptr;
    uint8_t *d_labels8 = nullptr;  // the labels as bytes, when integers in [0, 255]
    int32_t *d_missing = nullptr, *d_widths = nullptr;
    std::vector<int32_t> missing, widths;
    // categories per feature (0: numerical), set by mbh_dataset_set_categorical
    std::vector<int32_t> ncat;
    int32_t *d_ncat = nullptr;
    // the scan's feature order when some feature is categorical: the
    // category-set features first (their tasks run longest), then the others
    int32_t *d_scan_order = nullptr;
    bool any_cat = false;
    double label_sum = 0.0;  // sequential sum, for the base score
    std::vector<double> class_count;  // when labels are integers in [0, 1024)
    // sample weights (mbh_dataset_set_weights): the weighted label sum, the
    // weight total and per-class weight, each a sequential sum in row order
    std::vector<double> weights;
    double *d_weights = nullptr, *d_weights_buf = nullptr;
    double wlabel_sum = 0.0, weight_sum = 0.0;
    std::vector<double> class_weight;
    bool labels_integral = false;
    double label_min = 0.0, label_max = 0.0;
    // lambdarank: labels as relevance grades (when integers in [0, 30]) and
    // the query boundaries set by mbh_dataset_set_groups
    std::vector<int8_t> grades;
    std::vector<int64_t> qstart;
    int64_t *d_qstart = nullptr;
    int max_query = 0;
    std::vector<void *> owned;
    ~mbh_dataset() {
        for (void *p : owned) (void)hipFree(p);
    }
};

constexpr int kNumStats = 22;

struct mbh_fit {
    int num_class = 1;
    int objective = 0;
    int n_features = 0;
    double learning_rate = 0.1;
    std::vector<double> base;
    std::vector<int64_t> offsets{0};
    std::vector<int32_t> feature, threshold, left, right, default_left, missing_bin;
    std::vector<double> value, gain, count;
    std::vector<uint64_t> cat_bits;  // 4 words per node
    std::vector<double> train_raw;
    double stats[kNumStats] = {0};
    // time_histograms runs: per expansion launch, (tree, iteration, rows
    // partitioned, rows accumulated, partition ms, accumulation ms)
    std::vector<double> launch_log;
};

namespace {

struct Run {
    std::vector<void *> owned;
    ~Run() {
        for (void *p : owned) (void)hipFree(p);
    }
};

struct PinnedFlags {
    mb::Batch *p = nullptr;
    ~PinnedFlags() {
        if (p) (void)hipHostFree(p);
    }
};

// A state growing its share of a multiclass round's class trees on its own
// stream (mbh_train with several states side by side): the device state, the
// two pinned batch headers and group markers of its iteration groups, and
// where the tree it grows stands.
struct ClassState {
    mb::DevState s{};
    hipStream_t st = nullptr;
    PinnedFlags flags;
    hipEvent_t ev[2] = {nullptr, nullptr};
    hipEvent_t done = nullptr;
    int est = 0;          // expansion iterations its previous tree needed
    int cls = 0;          // class of the tree it grows next
    bool growing = false; // a tree is in flight
    int pending = 0;      // slot of the iteration group whose header is read next
    int iters = 0;        // iterations enqueued for the tree in flight
    ClassState() = default;
    ClassState(const ClassState &) = delete;
    ClassState &operator=(const ClassState &) = delete;
    ~ClassState() {
        for (hipEvent_t e : {ev[0], ev[1], done})
            if (e) (void)hipEventDestroy(e);
        if (st) (void)hipStreamDestroy(st);
    }
};

// LDS a histogram block leaves free beside its histogram (scheduling slack).
constexpr size_t kPbStaticLds = 2048;
// Leaves expanded per launch, at most (the best-first replay of C2-shaped
// trees reaches the tree's depth in iterations with 32).
#ifndef MB_MAX_BATCH
#define MB_MAX_BATCH 32
#endif
constexpr int kMaxBatch = MB_MAX_BATCH;  // at most 64 (the planner's one-wave batch steps)
static_assert(kMaxBatch >= 1 && kMaxBatch <= 64, "batch of 1..64 leaves");
// Expansion iterations ([partition, accumulation, scan, plan]) per group of
// launches between done-flag reads: the first group of a tree is as long as
// the previous tree needed (kFirstGroup for the first tree), later ones
// kNextGroup.
constexpr int kFirstGroup = 8;
// Most classes of a multiclass objective.
constexpr int kMaxClass = 1024;
constexpr int kNextGroup = 1;
#ifndef MB_STATE_NEXT_GROUP
#define MB_STATE_NEXT_GROUP 1
#endif
constexpr int kStateNextGroup = MB_STATE_NEXT_GROUP;  // later groups of a side-by-side class state
constexpr int kMaxGroup = 64;

int64_t chunk_limit_for(int B) {
    // rows per LDS accumulation so no packed field overflows:
    // count < 2^20, hess sum < 2^22 (|h| <= B + 1), |grad sum| < 2^21
    // (|g| <= B/2 + 1; +1 covers the rounding edge at the clamp).
    int64_t lim = (1 << 20) - 1;
    lim = std::min<int64_t>(lim, ((1 << 22) - 1) / (B + 1));
    lim = std::min<int64_t>(lim, ((1 << 21) - 1) / (B / 2 + 1));
    return lim;
}

void check_params(const mbh_dataset *ds, const mbh_params *p) {
    auto bad = [](const std::string &m) { throw Error{MOJOTREES_ERROR_INVALID_ARGUMENT, m}; };
    auto unsup = [](const std::string &m) { throw Error{MOJOTREES_ERROR_UNSUPPORTED, m}; };
    if (p->objective != MBH_OBJ_REGRESSION && p->objective != MBH_OBJ_BINARY &&
        p->objective != MBH_OBJ_MULTICLASS && p->objective != MBH_OBJ_LAMBDARANK)
        bad("unknown objective");
    if (p->objective == MBH_OBJ_LAMBDARANK) {
        // train_ranker's checks (ranking.mojo:205-232, :492-497, :713-737)
        if (ds->qstart.empty()) bad("objective lambdarank needs query groups");
        if (ds->grades.empty()) bad("relevance labels must be integers in [0, 30]");
        if (p->lambdarank_truncation_level < 1) bad("lambdarank_truncation_level must be positive");
        if (!(p->lambdarank_sigmoid > 0.0)) bad("sigmoid must be positive");
        if (p->goss) unsup("GOSS with lambdarank is not built on the device path");
    }
    if (ds->any_cat) {
        // CategoricalParams.check_one_hot (categorical.mojo:216-240) and
        // the search's own bounds
        if (!(p->cat_smooth > 0.0)) bad("cat_smooth must be positive");
        if (!(p->cat_l2 >= 0.0)) bad("cat_l2 must be non-negative");
        if (p->max_cat_threshold < 1) bad("max_cat_threshold must be positive");
        if (p->min_data_per_group < 1) bad("min_data_per_group must be positive");
        if (p->max_cat_to_onehot < 1) bad("max_cat_to_onehot must be positive");
        if (p->one_hot_max_size < -1 || p->one_hot_max_size > 256)
            bad("one_hot_max_size must be -1 (off) or in [0, 256]");
    }
    if (p->objective == MBH_OBJ_MULTICLASS) {
        if (p->num_class < 2 || p->num_class > kMaxClass) bad("num_class must be in [2, 1024]");
        if (!ds->labels_integral || ds->label_min < 0.0 || ds->label_max >= (double)p->num_class)
            bad("multiclass labels must be integers in [0, num_class)");
    }
    if (p->num_iterations < 0) bad("num_iterations must be nonnegative");
    if (p->num_leaves < 1) bad("num_leaves must be positive");
    if (p->num_leaves > 1024)
        unsup("num_leaves above 1024: the planner keeps the explored tree in LDS");
    if (ds->F >= 0xFFFF) unsup("65535 or more features: the score update packs a node's feature in 16 bits");
    if (p->min_data_in_leaf < 0) bad("min_data_in_leaf must be nonnegative");
    if (!(p->learning_rate > 0.0)) bad("learning_rate must be positive");
    if (!(p->lambda_l2 >= 0.0) || !(p->lambda_l1 >= 0.0)) bad("lambda_l1 and lambda_l2 must be nonnegative");
    if (!(p->min_sum_hessian >= 0.0)) bad("min_sum_hessian_in_leaf must be nonnegative");
    if (!(p->feature_fraction > 0.0 && p->feature_fraction <= 1.0)) bad("feature_fraction must be in (0, 1]");
    if (!(p->bagging_fraction > 0.0 && p->bagging_fraction <= 1.0)) bad("bagging_fraction must be in (0, 1]");
    if (p->bagging_freq < 0) bad("bagging_freq must be nonnegative");
    const int B = p->num_grad_quant_bins;
    if (p->quant_scale_rule != 0 && p->quant_scale_rule != 1)
        bad("quant_scale_rule must be 0 (max_abs) or 1 (magnitude_sum)");
    if (p->quant_staging != 0 && p->quant_staging != 1) bad("quant_staging must be 0 (int32) or 1 (int16)");
    if (p->quant_staging == 1 && !(p->use_quantized_grad && p->quant_scale_rule == 1))
        bad("quant_staging=int16 stages the magnitude-sum lattice (quant_scale_rule=magnitude_sum)");
    if (p->use_quantized_grad && p->quant_scale_rule == 1) {
        // the headroom argument of fixed_point_scale_pow2
        // (quantized_gradient.mojo:908-1117): a node's int32 sum stays
        // within 2^30 + n_rows
        if (ds->n >= ((int64_t)1 << 30))
            unsup("quant_scale_rule=magnitude_sum needs n_rows below 2^30 (int32 histogram sums)");
        if (p->objective == MBH_OBJ_LAMBDARANK)
            unsup("quant_scale_rule=magnitude_sum with lambdarank is not built on the device path");
    } else if (p->use_quantized_grad) {
        if (B < 2 || B > 126 || B % 2 != 0)
            unsup("num_grad_quant_bins must be even and in [2, 126] (int8 gradient storage)");
        if ((double)ds->n * (double)(B + 1) >= 2147483647.0)
            unsup("n_rows * (num_grad_quant_bins + 1) must stay below 2^31 for int32 histogram cells");
    }
    if (p->goss) {
        // GossParams.validate (goss.mojo:129-145), _check_goss (boosting.mojo:346-355)
        if (p->bagging_freq > 0 && p->bagging_fraction < 1.0) bad("goss and bagging cannot both be enabled");
        if (!(p->top_rate >= 0.0 && p->top_rate <= 1.0) || !(p->other_rate >= 0.0 && p->other_rate <= 1.0) ||
            !(p->top_rate + p->other_rate <= 1.0) || !(p->top_rate + p->other_rate > 0.0))
            bad("goss needs top_rate and other_rate in [0, 1] with 0 < top_rate + other_rate <= 1");
        if (p->bagging_seed < 0) bad("goss seed (bagging_seed) must be nonnegative");
    }
    if (p->objective == MBH_OBJ_BINARY && (ds->label_min < 0.0 || ds->label_max > 1.0))
        bad("binary labels must be in [0, 1]");
}

// Feature tiles of the row records. A tile holds as many features as one
// workgroup's LDS histogram takes for the histogram kind in use (8 bytes per
// cell quantized, 20 fp32, plus the partition's row list) and a 128-byte
// record allows (126 features and the g/h pair); the features are then
// spread evenly over the tiles. Narrow data is one tile: each row's bins in
// one 16..128-byte record.
struct RecLayout {
    int rec = 0, tile_f = 0, n_tiles = 0;
};

// pair_bytes: the g/h pair at the end of each record (2: an int8 pair, 4: the
// int16 staging pair).
RecLayout record_layout(int F, int lds_stride, int kind, int pair_bytes = 2) {
    int ft_max = 126;
    while (ft_max > 0 && mb::pb_lds_bytes_for(ft_max, lds_stride, kind) + kPbStaticLds > 160 * 1024)
        --ft_max;
    if (ft_max < 1)
        throw Error{MOJOTREES_ERROR_UNSUPPORTED, "one feature's histogram exceeds a workgroup's LDS"};
    RecLayout l;
    l.n_tiles = (F + ft_max - 1) / ft_max;
    l.tile_f = (F + l.n_tiles - 1) / l.n_tiles;
    l.rec = 16;
    while (l.rec < l.tile_f + pair_bytes) l.rec *= 2;
    return l;
}

// (Re)build the dataset's records for a layout; the g/h pairs start at zero.
void ensure_records(mbh_dataset *ds, const RecLayout &l) {
    if (ds->d_records && ds->rec == l.rec && ds->tile_f == l.tile_f && ds->n_tiles == l.n_tiles) return;
    if (ds->d_records) {
        HIPX(hipDeviceSynchronize());
        for (void *&q : ds->owned)
            if (q == ds->d_records) {
                (void)hipFree(q);
                q = ds->owned.back();
                ds->owned.pop_back();
                break;
            }
        ds->d_records = nullptr;
    }
    ds->d_records = dalloc<uint8_t>((size_t)l.rec * l.n_tiles * ds->n, ds->owned);
    ds->rec = l.rec;
    ds->tile_f = l.tile_f;
    ds->n_tiles = l.n_tiles;
    HIPX(mb::launch_build_records(ds->d_bins_cm, ds->d_records, ds->n, ds->F, l.rec, l.tile_f, l.n_tiles,
                                  4 * ds->n_cu, nullptr));
    HIPX(hipDeviceSynchronize());
}

// Histogram launch geometry and the partial buffer. The root build of m rows
// runs ceil(m / chunk) blocks with chunk = clamp(ceil(m / grid), chunk_min,
// chunk_limit); the grid is widened when needed so grid * chunk_limit covers
// every row. An expansion's accumulation gives each accumulated child of m
// rows ceil(m / chunk) tasks (block partials) with chunk = clamp(ceil(batch
// rows / (2 n_cu)), chunk_min, chunk_limit); the leaves of a batch are disjoint,
// so n / chunk_min + (batch size) tasks always suffice. Its partition tasks
// take at least kPartChunkMin parent rows each (but the last of a leaf),
// n / kPartChunkMin + (batch size) of them at most, spread over about two
// tasks per CU.
constexpr int64_t kHistChunkMin = 2048;
constexpr int64_t kHistChunkMinF = 1536;  // fp32 cells

void configure_hist(mb::DevState &s, const mbh_dataset *ds, int B, int kind, Run &run) {
    const bool quantized = kind != mb::kAccFloat;
    // the packed int8-lattice counters bound a block's rows; the other
    // accumulators hold whole-round sums in every field
    // the fp32 cells' 16-bit count halves bound a block's rows too
    const int64_t limit = kind == mb::kAccQuant   ? chunk_limit_for(B)
                          : kind == mb::kAccFloat ? mb::kFAccChunk
                                                  : (int64_t)1 << 30;
    // resident root-build blocks, shared by the feature tiles (a launch runs
    // grid x tiles blocks): every block then takes more rows, and zeroes,
    // stores and leaves to the scan's merge one partial per tile and block
    int64_t grid = std::max<int64_t>(1, (int64_t)ds->n_cu * mb::kHistBlocksPerCU / std::max(1, s.n_tiles));
    const int64_t need = (ds->n + limit - 1) / limit;
    if (grid < need) grid = need;
    s.hist_grid = (int32_t)grid;
    s.part_stride = (ds->nb + 1) & ~1;
    // the fp32 cells' per-row LDS work is three times the quantized one's:
    // smaller launches are spread over more blocks
    s.hist_chunk_min = std::min<int64_t>(kind == mb::kAccFloat ? kHistChunkMinF : kHistChunkMin, limit);
    s.hist_chunk_limit = limit;
    s.kmax = kMaxBatch;
    // one accumulation task per resident block: two per CU where two LDS
    // histograms fit (quantized), one for the fp32 cells, whose histogram
    // fills a CU's LDS (half the partials to merge; measured 0.3 % faster on
    // C3 than two tasks per CU run one after the other)
    // (no more blocks than a batch can have tasks: n / hist_chunk_min + one
    // per item; every block of a launch, empty or not, is dispatched -- times
    // the feature tiles)
    s.pb_launch = (int32_t)std::min<int64_t>((kind == mb::kAccFloat ? 1 : 2) * ds->n_cu,
                                             (ds->n + s.hist_chunk_min - 1) / s.hist_chunk_min + s.kmax);
    // a batch's accumulation tasks: with chunk >= its rows / pb_launch (or
    // = limit) an item of m rows takes at most m / chunk + 1 of them
    s.pb_grid = (int32_t)(s.pb_launch + s.kmax + (ds->n + limit - 1) / limit);
    s.part_grid = (int32_t)((ds->n + mb::kPartChunkMin - 1) / mb::kPartChunkMin + s.kmax);
    s.scan_grid = std::min(s.kmax * ds->F, 4 * ds->n_cu);
    s.part_launch = std::min<int32_t>(s.part_grid, 8 * ds->n_cu);
    s.part_target = 2 * ds->n_cu;
    // the root's batch gets the launch of larger tasks only where its rows
    // fill them (C2's 10.5M: 16K-row tasks; C5's 2M rows would leave three
    // quarters of each task's slots empty)
    s.part_root = (int64_t)ds->n >= (int64_t)mb::kPartChunkRoot * s.part_target ? 1 : 0;
    // a root build uses at most ceil(n / chunk_min) chunks
    const int64_t parts = std::max<int64_t>(std::min<int64_t>(grid, (ds->n + s.hist_chunk_min - 1) / s.hist_chunk_min),
                                            s.pb_grid);
    const size_t cells = (size_t)parts * ds->F * s.part_stride;
    if (quantized) {
        s.part = dalloc<unsigned long long>(cells, run.owned);
        if (kind == mb::kAccWide) s.part_c = dalloc<uint32_t>(cells, run.owned);
    } else {
        s.fpart_g = dalloc<double>(cells, run.owned);
        s.fpart_h = dalloc<double>(cells, run.owned);
        s.fpart_c = dalloc<uint32_t>(cells, run.owned);
    }
    s.part_items = dalloc<mb::PartItem>(s.kmax, run.owned);
    s.acc_items = dalloc<mb::AccItem>(s.kmax, run.owned);
}

double base_score_for(const mbh_dataset *ds, int objective) {
    // boosting._base_score (src/mojotrees/boosting.mojo:521-568): the
    // sequential label mean; binary takes the clamped log-odds.
    double mean = ds->d_weights ? ds->wlabel_sum / ds->weight_sum : ds->label_sum / (double)ds->n;
    if (objective == MBH_OBJ_BINARY) {
        double p = mean;
        if (p < 1e-15) p = 1e-15;
        if (p > 1.0 - 1e-15) p = 1.0 - 1e-15;
        return mb::ref_log(p / (1.0 - p));
    }
    return mean;
}

// Per-class base scores. boosting.train_multiclass
// (src/mojotrees/boosting.mojo:4167-4250): log of each class's clamped share.
std::vector<double> base_scores_for(const mbh_dataset *ds, int objective, int K) {
    // train_ranker boosts from 0 (ranking.mojo:700-712)
    if (objective == MBH_OBJ_LAMBDARANK) return {0.0};
    if (objective != MBH_OBJ_MULTICLASS) return {base_score_for(ds, objective)};
    std::vector<double> b(K);
    for (int k = 0; k < K; ++k) {
        const std::vector<double> &cc = ds->d_weights ? ds->class_weight : ds->class_count;
        const double cnt = (size_t)k < cc.size() ? cc[k] : 0.0;
        double p = cnt / (ds->d_weights ? ds->weight_sum : (double)ds->n);
        if (p < 1e-15) p = 1e-15;
        if (p > 1.0 - 1e-15) p = 1.0 - 1e-15;
        b[k] = mb::ref_log(p);
    }
    return b;
}


struct TrainBuffers {
    mb::DevState s{};
    int T = 0, L = 0, max_nodes = 0;
};

TrainBuffers setup_state(mbh_dataset *ds, const mbh_params *p, Run &run, int64_t last_round = 0) {
    TrainBuffers tb;
    const int K = p->objective == MBH_OBJ_MULTICLASS ? p->num_class : 1;
    const int L = p->num_leaves;
    const int T = std::max(1, p->num_iterations * K);
    const int max_nodes = 2 * L - 1;
    const int F = ds->F;
    mb::DevState &s = tb.s;
    const bool quantized = p->use_quantized_grad != 0;
    const bool wide = quantized && p->quant_scale_rule == 1;
    const bool stage16 = wide && p->quant_staging == 1;
    const int kind = wide ? mb::kAccWide : quantized ? mb::kAccQuant : mb::kAccFloat;
    ensure_records(ds, record_layout(F, ds->lds_stride, kind, stage16 ? 4 : 2));
    s.records = ds->d_records;
    s.records_w = ds->d_records;
    s.bins_cm = ds->d_bins_cm;
    s.labels = ds->d_labels;
    s.labels8 = ds->d_labels8;
    s.weights = ds->d_weights;
    s.missing_bin = ds->d_missing;
    s.widths = ds->d_widths;
    s.ncat = ds->any_cat ? ds->d_ncat : nullptr;
    s.scan_order = ds->any_cat ? ds->d_scan_order : nullptr;
    s.n = ds->n;
    s.n_features = F;
    s.n_bins = ds->nb;
    s.rec_bytes = ds->rec;
    s.tile_f = ds->tile_f;
    s.n_tiles = ds->n_tiles;
    s.lds_stride = ds->lds_stride;
    s.raw = dalloc<double>((size_t)ds->n * K, run.owned);
    s.prob = K > 1 ? dalloc<double>((size_t)ds->n * K, run.owned) : nullptr;
    s.grad = dalloc<float>(ds->n, run.owned);
    s.hess = dalloc<float>(ds->n, run.owned);
    s.stats = dalloc<uint32_t>(4 * mb::kStatSlots, run.owned);
    s.round = dalloc<mb::Round>(1, run.owned);
    s.rows0 = dalloc<int32_t>(ds->n, run.owned);
    s.rows1 = dalloc<int32_t>(ds->n, run.owned);
    const int max_exp = std::min(4 * L - 1, 2047);
    s.max_exp = max_exp;
    s.e_cap = 1 + 2 * max_exp;
    if (quantized) s.hist = dalloc<int32_t>((size_t)(1 + max_exp) * F * ds->nb * 3, run.owned);
    else s.histf = dalloc<mb::HistF>((size_t)(1 + max_exp) * F * ds->nb, run.owned);
    configure_hist(s, ds, quantized ? p->num_grad_quant_bins : 4, kind, run);
    if (wide) {
        if (!stage16) s.gq = dalloc<int32_t>(2 * (size_t)ds->n, run.owned);
        s.magpart = dalloc<float>(2 * 256, run.owned);
        s.stage16_over = dalloc<unsigned long long>(2, run.owned);
        HIPX(hipMemset(s.stage16_over, 0, 2 * sizeof(unsigned long long)));
    }
    s.enodes = dalloc<mb::ENode>(s.e_cap, run.owned);
    s.items = dalloc<mb::Item>(s.kmax, run.owned);
    s.batch = dalloc<mb::Batch>(1, run.owned);
    s.grow = dalloc<mb::Grow>(1, run.owned);
    s.slot_e = dalloc<int32_t>(L, run.owned);
    s.slot_fid = dalloc<int32_t>(L, run.owned);
    s.scan = dalloc<mb::ScanResult>((size_t)s.kmax * 2 * F, run.owned);
    s.scan_gain = dalloc<double>((size_t)s.kmax * 2 * F, run.owned);
    s.pair_gain = dalloc<double>((size_t)s.kmax * 2, run.owned);
    s.pair_feat = dalloc<int32_t>((size_t)s.kmax * 2, run.owned);
    s.e_gain = dalloc<double>(s.e_cap, run.owned);
    s.e_left = dalloc<int32_t>(s.e_cap, run.owned);
    s.e_rows = dalloc<int32_t>(s.e_cap, run.owned);
    s.e_parent = dalloc<int32_t>(s.e_cap, run.owned);
    s.cursor = dalloc<int64_t>(2 + 2 * (size_t)s.kmax, run.owned);
    s.error = dalloc<int32_t>(1, run.owned);
    s.t_feature = dalloc<int32_t>(max_nodes, run.owned);
    s.t_threshold = dalloc<int32_t>(max_nodes, run.owned);
    s.t_left = dalloc<int32_t>(max_nodes, run.owned);
    s.t_right = dalloc<int32_t>(max_nodes, run.owned);
    s.t_default_left = dalloc<int32_t>(max_nodes, run.owned);
    s.t_missing_bin = dalloc<int32_t>(max_nodes, run.owned);
    s.t_value = dalloc<double>(max_nodes, run.owned);
    s.t_gain = dalloc<double>(max_nodes, run.owned);
    s.t_count = dalloc<double>(max_nodes, run.owned);
    s.t_meta = dalloc<int32_t>(2, run.owned);
    s.arc_int = dalloc<int32_t>((size_t)T * (6 * max_nodes + 2), run.owned);
    s.arc_dbl = dalloc<double>((size_t)T * 3 * max_nodes, run.owned);
    s.arc_aux = dalloc<int64_t>((size_t)T * 4, run.owned);
    if (ds->any_cat) {
        s.scan_cat = dalloc<unsigned long long>((size_t)s.kmax * 2 * F * 4, run.owned);
        s.e_cat = dalloc<unsigned long long>((size_t)s.e_cap * 4, run.owned);
        s.t_cat = dalloc<unsigned long long>((size_t)max_nodes * 4, run.owned);
        s.arc_cat = dalloc<unsigned long long>((size_t)T * max_nodes * 4, run.owned);
        HIPX(hipMemset(s.t_cat, 0, (size_t)max_nodes * 4 * sizeof(unsigned long long)));
        HIPX(hipMemset(s.arc_cat, 0, (size_t)T * max_nodes * 4 * sizeof(unsigned long long)));
    }
    s.max_nodes = max_nodes;
    uint8_t *fmask = dalloc<uint8_t>((size_t)T * F, run.owned);
    s.feature_mask = fmask;
    mb::HyperParams &hp = s.hp;
    hp.objective = p->objective;
    hp.num_class = K;
    hp.class_stride = 1;
    hp.num_leaves = L;
    hp.min_data_in_leaf = p->min_data_in_leaf;
    hp.max_depth = p->max_depth;
    hp.quant_bins = p->num_grad_quant_bins;
    hp.stochastic = p->stochastic_rounding;
    hp.quant_seed = p->quant_seed;
    // boosting.round_has_constant_hessian: squared error without weights.
    // a GOSS round weights some rows' hessians: not constant
    hp.const_hessian = p->objective == MBH_OBJ_REGRESSION && !ds->d_weights && !p->goss ? 1 : 0;
    if (p->objective == MBH_OBJ_LAMBDARANK) {
        // binary64 lambdas (the reference's ranker does not narrow them), the
        // queries, 1 / maxDCG per query at the truncation level and the
        // position discounts (ranking.mojo:240-245, :306-338), on the host
        hp.grad64 = 1;
        hp.rank_trunc = p->lambdarank_truncation_level;
        hp.rank_norm = p->lambdarank_norm ? 1 : 0;
        hp.rank_sigma = p->lambdarank_sigmoid;
        s.grad64 = dalloc<double>(ds->n, run.owned);
        s.hess64 = dalloc<double>(ds->n, run.owned);
        s.stats64 = dalloc<unsigned long long>(4, run.owned);
        HIPX(hipMemset(s.stats64, 0, 4 * sizeof(unsigned long long)));
        const int64_t nq = (int64_t)ds->qstart.size() - 1;
        std::vector<double> disc(ds->max_query), inv(nq);
        for (int i = 0; i < ds->max_query; ++i) disc[i] = 1.0 / mb::ref_log2((double)i + 2.0);
        for (int64_t q = 0; q < nq; ++q) {
            const int64_t a = ds->qstart[q], c = ds->qstart[q + 1] - a;
            std::vector<int> g(ds->grades.begin() + a, ds->grades.begin() + a + c);
            std::sort(g.begin(), g.end(), [](int x, int y) { return x > y; });
            const int64_t m = std::min<int64_t>(c, hp.rank_trunc);
            double md = 0.0;
            for (int64_t j = 0; j < m; ++j) md += mb::label_gain(g[j]) * disc[j];
            inv[q] = md > 0.0 ? 1.0 / md : 0.0;
        }
        double *d_disc = dalloc<double>(std::max(1, ds->max_query), run.owned);
        double *d_inv = dalloc<double>(nq, run.owned);
        HIPX(hipMemcpy(d_disc, disc.data(), disc.size() * sizeof(double), hipMemcpyHostToDevice));
        HIPX(hipMemcpy(d_inv, inv.data(), inv.size() * sizeof(double), hipMemcpyHostToDevice));
        s.rank_disc = d_disc;
        s.inv_max_dcg = d_inv;
        s.qstart = ds->d_qstart;
        s.n_queries = (int32_t)nq;
        // queries the LDS sort holds go to k_lambdarank; larger ones to
        // k_lambdarank_big, which sorts in a global slot per block
        int max_small = 1, max_big = 0;
        std::vector<int32_t> big;
        for (int64_t q = 0; q < nq; ++q) {
            const int c = (int)(ds->qstart[q + 1] - ds->qstart[q]);
            if (c > mb::kMaxQueryRows) {
                big.push_back((int32_t)q);
                max_big = std::max(max_big, c);
            } else {
                max_small = std::max(max_small, c);
            }
        }
        int pad = 1;
        while (pad < max_small) pad <<= 1;
        s.rank_pad = pad;
        if (!big.empty()) {
            int bp = 1;
            while (bp < max_big) bp <<= 1;
            const size_t slot_bytes = (size_t)bp * (3 * sizeof(double) + 2 * sizeof(int32_t));
            int slots = (int)std::min<size_t>(big.size(), (size_t)ds->n_cu);
            slots = (int)std::max<size_t>(1, std::min<size_t>(slots, ((size_t)4 << 30) / slot_bytes));
            s.n_big = (int32_t)big.size();
            s.rank_big_pad = bp;
            s.rank_big_slots = slots;
            s.rank_scratch = dalloc<double>((size_t)slots * 3 * bp, run.owned);
            s.rank_scratch_i = dalloc<int32_t>((size_t)slots * 2 * bp, run.owned);
            int32_t *d_big = dalloc<int32_t>(big.size(), run.owned);
            HIPX(hipMemcpy(d_big, big.data(), big.size() * sizeof(int32_t), hipMemcpyHostToDevice));
            s.rank_big = d_big;
        }
    }
    hp.quantized = p->use_quantized_grad ? 1 : 0;
    hp.wide = wide ? 1 : 0;
    hp.stage16 = stage16 ? 1 : 0;
    hp.goss = p->goss ? 1 : 0;
    // GossParams.warmup (goss.mojo:102-157): floor(1 / learning_rate) rounds
    hp.goss_warm = p->learning_rate > 0.0 ? (int32_t)(1.0 / p->learning_rate) : 0;
    hp.goss_seed = p->bagging_seed;
    hp.top_rate = p->top_rate;
    hp.other_rate = p->other_rate;
    hp.goss_band = p->goss_band;
    hp.goss_exact = p->goss_exact_walk ? 1 : 0;
    if (hp.goss) {
        s.goss_nblk = (int32_t)((ds->n + 1023) / 1024);
        s.gst = dalloc<mb::GossState>(1, run.owned);
        s.goss_hist = dalloc<uint32_t>(8 * mb::kGossHistSlots * 256, run.owned);
        s.goss_sel = dalloc<unsigned long long>(16, run.owned);
        s.goss_cand = dalloc<unsigned long long>(ds->n, run.owned);
        s.goss_ccnt = dalloc<int32_t>(mb::kGossDigitBlocks, run.owned);
        // padded to whole count tiles; the pad holds INT_MIN (never kept) and
        // no kernel writes it
        const int64_t padded = (ds->n + mb::kGossTileRows - 1) / mb::kGossTileRows * mb::kGossTileRows;
        s.goss_kappa = dalloc<int32_t>(padded, run.owned);
        if (padded > ds->n) {
            std::vector<int32_t> pad(padded - ds->n, INT32_MIN);
            HIPX(hipMemcpy(s.goss_kappa + ds->n, pad.data(), pad.size() * sizeof(int32_t), hipMemcpyHostToDevice));
        }
        s.goss_mask = dalloc<unsigned long long>((ds->n + 63) / 64, run.owned);
        s.goss_topmask = dalloc<unsigned long long>((ds->n + 63) / 64, run.owned);
        s.goss_blk = dalloc<int32_t>(s.goss_nblk, run.owned);
        s.goss_blk_u = dalloc<int32_t>(s.goss_nblk, run.owned);
        s.goss_ukappa = dalloc<int32_t>(padded, run.owned);  // whole count tiles
        s.goss_urow = dalloc<int32_t>(ds->n, run.owned);
        s.goss_umask = dalloc<unsigned long long>((ds->n + 63) / 64, run.owned);
        s.goss_other = dalloc<uint8_t>(ds->n, run.owned);
        HIPX(hipMemset(s.goss_other, 0, ds->n));
        s.goss_rows = dalloc<int32_t>(ds->n, run.owned);
        s.goss_max = dalloc<unsigned long long>(4, run.owned);
        HIPX(hipMemset(s.goss_max, 0, 4 * sizeof(unsigned long long)));
        if (p->objective == MBH_OBJ_MULTICLASS) s.goss_imp = dalloc<double>(ds->n, run.owned);
    }
    hp.bagging = (p->bagging_freq > 0 && p->bagging_fraction < 1.0) ? 1 : 0;
    hp.bagging_freq = p->bagging_freq;
    hp.bagging_seed = p->bagging_seed;
    hp.bagging_fraction = p->bagging_fraction;
    if (hp.bagging) {
        // bagging.sample_rows (bagging.mojo:101-129) never returns an empty
        // bag: it then takes the unit of the least draw. Per bag index (the
        // score kernel draws the next round's bag, so one past the last
        // round), -1, or that unit when no unit is drawn; the scan stops at
        // the first drawn unit, after ~1 / fraction draws.
        const bool by_query = p->objective == MBH_OBJ_LAMBDARANK;
        const int64_t units = by_query ? (int64_t)ds->qstart.size() - 1 : ds->n;
        const int64_t n_bags = std::max<int64_t>(p->num_iterations, last_round + 1) / p->bagging_freq + 2;
        std::vector<int64_t> fb((size_t)n_bags, -1);
        for (int64_t b = 0; b < n_bags; ++b) {
            const uint64_t stream = mb::splitmix64((uint64_t)(p->bagging_seed & 0x7FFFFFFFFFFFFFFFLL) ^
                                                   ((uint64_t)b * mb::kGolden));
            double min_draw = 2.0;
            int64_t min_unit = 0;
            bool any = false;
            for (int64_t u = 0; u < units && !any; ++u) {
                const double d = mb::uniform53(stream + (uint64_t)u);
                any = d < p->bagging_fraction;
                if (d < min_draw) {
                    min_draw = d;
                    min_unit = u;
                }
            }
            if (!any) fb[(size_t)b] = min_unit;
        }
        int64_t *d_fb = dalloc<int64_t>(n_bags, run.owned);
        HIPX(hipMemcpy(d_fb, fb.data(), n_bags * sizeof(int64_t), hipMemcpyHostToDevice));
        s.bag_fallback = d_fb;
        s.n_bags = n_bags;
        if (by_query) {
            // ranking._refresh_query_bag (ranking.mojo:667-686): the draw is
            // per query, so each row carries its query's index
            std::vector<int32_t> qid((size_t)ds->n);
            for (size_t q = 0; q + 1 < ds->qstart.size(); ++q)
                for (int64_t r = ds->qstart[q]; r < ds->qstart[q + 1]; ++r) qid[(size_t)r] = (int32_t)q;
            int32_t *d_qid = dalloc<int32_t>(ds->n, run.owned);
            HIPX(hipMemcpy(d_qid, qid.data(), (size_t)ds->n * sizeof(int32_t), hipMemcpyHostToDevice));
            s.qid = d_qid;
        }
    }
    hp.learning_rate = p->learning_rate;
    hp.lambda_l1 = p->lambda_l1;
    hp.lambda_l2 = p->lambda_l2;
    hp.min_sum_hessian = p->min_sum_hessian;
    hp.max_cat_to_onehot = p->max_cat_to_onehot;
    hp.max_cat_threshold = p->max_cat_threshold;
    hp.min_data_per_group = p->min_data_per_group;
    hp.one_hot_max_size = p->one_hot_max_size;
    hp.cat_smooth = p->cat_smooth;
    hp.cat_l2 = p->cat_l2;

    // the fp32 path's binary32 derivatives, interleaved per row
    if (!quantized && !hp.grad64) s.gh2 = dalloc<float>(2 * (size_t)ds->n, run.owned);
    if (mb::plan_lds_bytes(s) > 160 * 1024)
        throw Error{MOJOTREES_ERROR_UNSUPPORTED,
                    "num_leaves * n_features too large for the planner's LDS (160 KiB)"};
    if (mb::hist_lds_bytes(s) + kPbStaticLds > 160 * 1024)
        throw Error{MOJOTREES_ERROR_TRAINING, "internal: the feature tile exceeds one workgroup's LDS"};
    HIPX(hipMemset(s.rows0, 0, (size_t)ds->n * sizeof(int32_t)));
    HIPX(hipMemset(s.rows1, 0, (size_t)ds->n * sizeof(int32_t)));
    HIPX(hipMemset(s.stats, 0, 4 * mb::kStatSlots * sizeof(uint32_t)));
    HIPX(hipMemset(s.batch, 0, sizeof(mb::Batch)));
    HIPX(hipMemset(s.grow, 0, sizeof(mb::Grow)));
    HIPX(hipMemset(s.part_items, 0, (size_t)s.kmax * sizeof(mb::PartItem)));
    HIPX(hipMemset(s.acc_items, 0, (size_t)s.kmax * sizeof(mb::AccItem)));
    HIPX(hipMemset(s.cursor, 0, (2 + 2 * (size_t)s.kmax) * sizeof(int64_t)));
    HIPX(hipMemset(s.error, 0, sizeof(int32_t)));
    HIPX(hipMemset(s.t_meta, 0, 2 * sizeof(int32_t)));
    HIPX(hipMemset(s.arc_aux, 0, (size_t)T * 4 * sizeof(int64_t)));
    HIPX(hipMemset(s.arc_int, 0, (size_t)T * (6 * max_nodes + 2) * sizeof(int32_t)));
    mb::Round r0 = mb::initial_round();
    HIPX(hipMemcpy(s.round, &r0, sizeof(r0), hipMemcpyHostToDevice));
    std::vector<uint8_t> masks((size_t)T * F);
    for (int t = 0; t < T; ++t) {
        std::vector<uint8_t> m = tree_feature_mask(F, p->feature_fraction, p->feature_fraction_seed, t);
        std::memcpy(masks.data() + (size_t)t * F, m.data(), F);
    }
    HIPX(hipMemcpy(fmask, masks.data(), masks.size(), hipMemcpyHostToDevice));
    tb.T = T;
    tb.L = L;
    tb.max_nodes = max_nodes;
    return tb;
}

// The round's binary32 derivatives to the host: the planes, or the fp32
// path's interleaved pairs.
void download_derivatives(const mb::DevState &s, int64_t n, float *grad, float *hess) {
    if (s.gh2) {
        HIPX(hipMemcpy2D(grad, sizeof(float), s.gh2, 2 * sizeof(float), sizeof(float), n, hipMemcpyDeviceToHost));
        HIPX(hipMemcpy2D(hess, sizeof(float), s.gh2 + 1, 2 * sizeof(float), sizeof(float), n, hipMemcpyDeviceToHost));
    } else {
        HIPX(hipMemcpy(grad, s.grad, n * sizeof(float), hipMemcpyDeviceToHost));
        HIPX(hipMemcpy(hess, s.hess, n * sizeof(float), hipMemcpyDeviceToHost));
    }
}

// The leaf row representation of a training run (mbh_params.partition_mode):
// records (s.rcp = 1) where the layout allows it -- the max-abs lattice's
// int8 pairs, whose root build quantizes (a pair per row to the pair plane),
// one feature tile, records of at most 64 bytes -- and the mode asks for it;
// row ids otherwise. Automatic takes row ids: on C2 (32-byte records) the
// records' histograms stream (k_accum 15.6 -> 10.8 us per launch) but
// moving 64 bytes per partitioned row instead of 9 costs more than that
// saves (0.99 -> 1.09 s per 500 trees).
void setup_record_partition(mb::DevState &s, const mbh_dataset *ds, const mbh_params *p, Run &run) {
    const bool eligible = mb::acc_kind(s.hp) == mb::kAccQuant && !s.hp.grad64 && s.n_tiles == 1 &&
                          s.rec_bytes <= 64;
    const int mode = p->partition_mode;
    if (mode < 0 || mode > 2) throw Error{MOJOTREES_ERROR_INVALID_ARGUMENT, "partition_mode must be 0, 1 or 2"};
    s.rcp = eligible && mode == 1 ? 1 : 0;
    if (!s.rcp) return;
    s.crec0 = dalloc<uint8_t>((size_t)ds->n * s.rec_bytes, run.owned);
    s.crec1 = dalloc<uint8_t>((size_t)ds->n * s.rec_bytes, run.owned);
    s.pairs = dalloc<uint16_t>(ds->n, run.owned);
    // the root's batch shares the record partition's kPartChunk-row tasks
    // (16K-row tasks would hold 16 records per thread)
    s.part_root = 0;
}

// One more state for a multiclass round's class trees grown side by side:
// a copy of s0 sharing the dataset, the scores and probabilities, the
// archive, the feature masks, the bag tables, the error word and the
// round-level GOSS sample, with its own copy of everything one tree's growth
// writes -- the records (each tree's quantized pairs land in them), the
// derivatives and their magnitude statistics, the round state, the row
// lists, histograms, partials, explored nodes, batch, frontier, scan
// results and the tree being grown. Its first class is `first`; it grows
// classes first, first + stride, ... of every round.
mb::DevState clone_class_state(const mb::DevState &s0, const mbh_dataset *ds, int first, int stride,
                               int L, int max_nodes, Run &run) {
    mb::DevState s = s0;
    const int64_t n = ds->n;
    const int F = ds->F;
    s.hp.class_stride = stride;
    const size_t rec_total = (size_t)s0.n_tiles * (size_t)n * (size_t)s0.rec_bytes;
    uint8_t *rec = dalloc<uint8_t>(rec_total, run.owned);
    HIPX(hipMemcpy(rec, s0.records, rec_total, hipMemcpyDeviceToDevice));
    s.records = rec;
    s.records_w = rec;
    s.grad = dalloc<float>(n, run.owned);
    s.hess = dalloc<float>(n, run.owned);
    if (s0.gh2) s.gh2 = dalloc<float>(2 * (size_t)n, run.owned);
    s.stats = dalloc<uint32_t>(4 * mb::kStatSlots, run.owned);
    s.round = dalloc<mb::Round>(1, run.owned);
    s.rows0 = dalloc<int32_t>(n, run.owned);
    s.rows1 = dalloc<int32_t>(n, run.owned);
    if (s0.hist) s.hist = dalloc<int32_t>((size_t)(1 + s0.max_exp) * F * ds->nb * 3, run.owned);
    if (s0.histf) s.histf = dalloc<mb::HistF>((size_t)(1 + s0.max_exp) * F * ds->nb, run.owned);
    const int kind = s0.hp.wide ? mb::kAccWide : s0.hp.quantized ? mb::kAccQuant : mb::kAccFloat;
    s.part = nullptr;
    s.part_c = nullptr;
    s.fpart_g = s.fpart_h = nullptr;
    s.fpart_c = nullptr;
    configure_hist(s, ds, s0.hp.quantized ? s0.hp.quant_bins : 4, kind, run);
    if (s0.gq) s.gq = dalloc<int32_t>(2 * (size_t)n, run.owned);
    if (s0.magpart) s.magpart = dalloc<float>(2 * 256, run.owned);
    if (s0.stage16_over) {
        s.stage16_over = dalloc<unsigned long long>(2, run.owned);
        HIPX(hipMemset(s.stage16_over, 0, 2 * sizeof(unsigned long long)));
    }
    if (s0.goss_max) {
        s.goss_max = dalloc<unsigned long long>(4, run.owned);
        HIPX(hipMemset(s.goss_max, 0, 4 * sizeof(unsigned long long)));
    }
    s.enodes = dalloc<mb::ENode>(s.e_cap, run.owned);
    s.items = dalloc<mb::Item>(s.kmax, run.owned);
    s.batch = dalloc<mb::Batch>(1, run.owned);
    s.grow = dalloc<mb::Grow>(1, run.owned);
    s.slot_e = dalloc<int32_t>(L, run.owned);
    s.slot_fid = dalloc<int32_t>(L, run.owned);
    s.scan = dalloc<mb::ScanResult>((size_t)s.kmax * 2 * F, run.owned);
    s.scan_gain = dalloc<double>((size_t)s.kmax * 2 * F, run.owned);
    s.pair_gain = dalloc<double>((size_t)s.kmax * 2, run.owned);
    s.pair_feat = dalloc<int32_t>((size_t)s.kmax * 2, run.owned);
    s.e_gain = dalloc<double>(s.e_cap, run.owned);
    s.e_left = dalloc<int32_t>(s.e_cap, run.owned);
    s.e_rows = dalloc<int32_t>(s.e_cap, run.owned);
    s.e_parent = dalloc<int32_t>(s.e_cap, run.owned);
    s.cursor = dalloc<int64_t>(2 + 2 * (size_t)s.kmax, run.owned);
    s.t_feature = dalloc<int32_t>(max_nodes, run.owned);
    s.t_threshold = dalloc<int32_t>(max_nodes, run.owned);
    s.t_left = dalloc<int32_t>(max_nodes, run.owned);
    s.t_right = dalloc<int32_t>(max_nodes, run.owned);
    s.t_default_left = dalloc<int32_t>(max_nodes, run.owned);
    s.t_missing_bin = dalloc<int32_t>(max_nodes, run.owned);
    s.t_value = dalloc<double>(max_nodes, run.owned);
    s.t_gain = dalloc<double>(max_nodes, run.owned);
    s.t_count = dalloc<double>(max_nodes, run.owned);
    s.t_meta = dalloc<int32_t>(2, run.owned);
    if (s0.scan_cat) {
        s.scan_cat = dalloc<unsigned long long>((size_t)s.kmax * 2 * F * 4, run.owned);
        s.e_cat = dalloc<unsigned long long>((size_t)s.e_cap * 4, run.owned);
        s.t_cat = dalloc<unsigned long long>((size_t)max_nodes * 4, run.owned);
        HIPX(hipMemset(s.t_cat, 0, (size_t)max_nodes * 4 * sizeof(unsigned long long)));
    }
    HIPX(hipMemset(s.rows0, 0, (size_t)n * sizeof(int32_t)));
    HIPX(hipMemset(s.rows1, 0, (size_t)n * sizeof(int32_t)));
    HIPX(hipMemset(s.stats, 0, 4 * mb::kStatSlots * sizeof(uint32_t)));
    HIPX(hipMemset(s.batch, 0, sizeof(mb::Batch)));
    HIPX(hipMemset(s.grow, 0, sizeof(mb::Grow)));
    HIPX(hipMemset(s.part_items, 0, (size_t)s.kmax * sizeof(mb::PartItem)));
    HIPX(hipMemset(s.acc_items, 0, (size_t)s.kmax * sizeof(mb::AccItem)));
    HIPX(hipMemset(s.cursor, 0, (2 + 2 * (size_t)s.kmax) * sizeof(int64_t)));
    HIPX(hipMemset(s.t_meta, 0, 2 * sizeof(int32_t)));
    mb::Round r0 = mb::initial_round();
    r0.class_k = first;
    r0.tree_index = first;
    HIPX(hipMemcpy(s.round, &r0, sizeof(r0), hipMemcpyHostToDevice));
    return s;
}

// The packed int16 arm's refusal (gpu_active_rows._raise_stage16): values
// that did not fit a signed 16-bit word were counted per plane by the
// quantizer; any such value (the hessian plane only when it is read, not
// under a constant hessian) refuses the fit and names the counts. The
// remedy is the int32 staging, not a smaller scale.
void check_stage16(const mb::DevState &s, int64_t n) {
    if (!s.hp.stage16) return;
    unsigned long long over[2] = {0ULL, 0ULL};
    HIPX(hipMemcpy(over, s.stage16_over, sizeof(over), hipMemcpyDeviceToHost));
    if (s.hp.const_hessian) over[1] = 0ULL;
    if (over[0] || over[1])
        throw Error{MOJOTREES_ERROR_TRAINING,
                    "the packed int16 gradient staging lost " + std::to_string(over[0]) + " gradient and " +
                        std::to_string(over[1]) + " hessian values (over all rounds, " + std::to_string(n) +
                        " rows each) that do not fit a signed 16-bit word at the round's scale; this bound is "
                        "per row and tightens as the row count falls, so the remedy is the int32 staging "
                        "(quant_staging=0, the default), not a smaller scale"};
}

}  // namespace

extern "C" {

int32_t mbh_device_count(void) { return device_count_gfx950(); }

int32_t mbh_bin_dense(const double *data, int64_t n, int32_t F, int32_t max_bins, int32_t min_data_in_bin,
                      int32_t use_missing, int64_t sample_cnt, int64_t seed, uint8_t *out_bins,
                      int32_t *out_missing, char *err, int32_t err_len) {
    if (!data || !out_bins || !out_missing || n <= 0 || F <= 0) {
        set_err(err, err_len, "invalid arguments");
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    try {
        mb::BinMapper m = mb::fit_bins(data, n, F, max_bins, min_data_in_bin, use_missing != 0, sample_cnt, seed);
        m.transform(data, n, out_bins);
        for (int f = 0; f < F; ++f) out_missing[f] = m.missing_bin[f];
    } catch (const std::exception &e) {
        set_err(err, err_len, e.what());
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    return MOJOTREES_OK;
}

int32_t mbh_bin_dense_cat(const double *data, int64_t n, int32_t F, int32_t max_bins, int32_t min_data_in_bin,
                          int32_t use_missing, int64_t sample_cnt, int64_t seed, const int32_t *categorical,
                          int32_t n_categorical, uint8_t *out_bins, int32_t *out_missing, int32_t *out_ncat,
                          char *err, int32_t err_len) {
    if (!data || !out_bins || !out_missing || !out_ncat || n <= 0 || F <= 0 || n_categorical < 0 ||
        (n_categorical > 0 && !categorical)) {
        set_err(err, err_len, "invalid arguments");
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    try {
        const std::vector<int> cats(categorical, categorical + n_categorical);
        mb::BinMapper m = mb::fit_bins(data, n, F, max_bins, min_data_in_bin, use_missing != 0, sample_cnt, seed, cats);
        m.transform(data, n, out_bins);
        for (int f = 0; f < F; ++f) {
            out_missing[f] = m.missing_bin[f];
            out_ncat[f] = m.n_categories(f);
        }
    } catch (const std::exception &e) {
        set_err(err, err_len, e.what());
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    return MOJOTREES_OK;
}

int32_t mbh_dataset_set_categorical(mbh_dataset *ds, const int32_t *ncat, char *err, int32_t err_len) {
    if (!ds || !ncat) {
        set_err(err, err_len, "null argument");
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    try {
        for (int f = 0; f < ds->F; ++f) {
            if (ncat[f] < 0) throw Error{MOJOTREES_ERROR_INVALID_ARGUMENT, "n_categories must be non-negative"};
            // a split search past the histogram's bins would read another
            // feature's cells (split.mojo:1028-1033)
            if (ncat[f] >= ds->nb)
                throw Error{MOJOTREES_ERROR_INVALID_ARGUMENT, "categorical feature has more categories than bins"};
        }
        ds->ncat.assign(ncat, ncat + ds->F);
        ds->any_cat = false;
        for (int f = 0; f < ds->F; ++f) ds->any_cat = ds->any_cat || ncat[f] > 0;
        if (!ds->d_ncat) ds->d_ncat = dalloc<int32_t>(ds->F, ds->owned);
        HIPX(hipMemcpy(ds->d_ncat, ds->ncat.data(), ds->F * sizeof(int32_t), hipMemcpyHostToDevice));
        std::vector<int32_t> order;
        for (int f = 0; f < ds->F; ++f)
            if (ncat[f] > 0) order.push_back(f);
        for (int f = 0; f < ds->F; ++f)
            if (ncat[f] <= 0) order.push_back(f);
        if (!ds->d_scan_order) ds->d_scan_order = dalloc<int32_t>(ds->F, ds->owned);
        HIPX(hipMemcpy(ds->d_scan_order, order.data(), ds->F * sizeof(int32_t), hipMemcpyHostToDevice));
    } catch (const Error &e) {
        set_err(err, err_len, e.msg);
        return e.code;
    }
    return MOJOTREES_OK;
}

int32_t mbh_dataset_create(const uint8_t *bins_cm, int64_t n, int32_t F, int32_t nb,
                           const int32_t *missing_bin, const double *labels, mbh_dataset **out,
                           char *err, int32_t err_len) {
    if (!bins_cm || !labels || !out || n <= 0 || F <= 0 || nb < 2 || nb > 256) {
        set_err(err, err_len, "invalid dataset arguments");
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    if (n >= (int64_t)1 << 31) {
        set_err(err, err_len, "n_rows must be below 2^31 (int32 row ids)");
        return MOJOTREES_ERROR_UNSUPPORTED;
    }
    if (device_count_gfx950() == 0) {
        set_err(err, err_len, "no gfx950 (MI355X) device is available to this process");
        return MOJOTREES_ERROR_UNSUPPORTED;
    }
    auto *ds = new mbh_dataset();
    try {
        ds->n = n;
        ds->F = F;
        ds->nb = nb;
        ds->lds_stride = nb | 1;
        // validate bins and derive the realized widths (binning.histogram_widths)
        ds->missing.assign(F, -1);
        if (missing_bin)
            for (int f = 0; f < F; ++f) ds->missing[f] = missing_bin[f];
        ds->widths.assign(F, 1);
        for (int f = 0; f < F; ++f) {
            const uint8_t *col = bins_cm + (size_t)f * n;
            int mx = 0;
            for (int64_t r = 0; r < n; ++r) mx = std::max(mx, (int)col[r]);
            if (mx >= nb) throw Error{MOJOTREES_ERROR_INVALID_ARGUMENT, "a bin id is >= n_bins"};
            if (ds->missing[f] >= nb) throw Error{MOJOTREES_ERROR_INVALID_ARGUMENT, "missing bin out of range"};
            int w = std::max(1, mx + 1);
            w = std::max(w, ds->missing[f] + 1);
            ds->widths[f] = std::min(w, nb);
        }
        double sum = 0.0, lo = labels[0], hi = labels[0];
        for (int64_t r = 0; r < n; ++r) {
            const double y = labels[r];
            if (!std::isfinite(y)) throw Error{MOJOTREES_ERROR_INVALID_ARGUMENT, "labels must be finite"};
            sum += 1.0 * y;
            lo = std::min(lo, y);
            hi = std::max(hi, y);
        }
        ds->label_sum = sum;
        ds->label_min = lo;
        ds->label_max = hi;
        // class counts, for a multiclass base score
        ds->labels_integral = lo >= 0.0 && hi < (double)kMaxClass;
        for (int64_t r = 0; r < n && ds->labels_integral; ++r)
            if (labels[r] != std::floor(labels[r])) ds->labels_integral = false;
        if (ds->labels_integral && hi <= 30.0) {
            ds->grades.resize(n);
            for (int64_t r = 0; r < n; ++r) ds->grades[r] = (int8_t)labels[r];
        }
        if (ds->labels_integral) {
            ds->class_count.assign((size_t)hi + 1, 0.0);
            for (int64_t r = 0; r < n; ++r) ds->class_count[(size_t)labels[r]] += 1.0;
        }
        HIPX(hipGetDevice(&ds->device));
        hipDeviceProp_t prop;
        HIPX(hipGetDeviceProperties(&prop, ds->device));
        ds->n_cu = prop.multiProcessorCount;
        ds->d_bins_cm = dalloc<uint8_t>((size_t)F * n, ds->owned);
        ds->d_labels = dalloc<double>(n, ds->owned);
        ds->d_missing = dalloc<int32_t>(F, ds->owned);
        ds->d_widths = dalloc<int32_t>(F, ds->owned);
        HIPX(hipMemcpy(ds->d_bins_cm, bins_cm, (size_t)F * n, hipMemcpyHostToDevice));
        HIPX(hipMemcpy(ds->d_labels, labels, (size_t)n * sizeof(double), hipMemcpyHostToDevice));
        if (ds->labels_integral && hi <= 255.0) {
            std::vector<uint8_t> l8((size_t)n);
            for (int64_t r = 0; r < n; ++r) l8[(size_t)r] = (uint8_t)labels[r];
            ds->d_labels8 = dalloc<uint8_t>(n, ds->owned);
            HIPX(hipMemcpy(ds->d_labels8, l8.data(), (size_t)n, hipMemcpyHostToDevice));
        }
        HIPX(hipMemcpy(ds->d_missing, ds->missing.data(), F * sizeof(int32_t), hipMemcpyHostToDevice));
        HIPX(hipMemcpy(ds->d_widths, ds->widths.data(), F * sizeof(int32_t), hipMemcpyHostToDevice));
        HIPX(hipDeviceSynchronize());
    } catch (const Error &e) {
        set_err(err, err_len, e.msg);
        delete ds;
        return e.code;
    }
    *out = ds;
    return MOJOTREES_OK;
}

void mbh_dataset_free(mbh_dataset *ds) { delete ds; }

int32_t mbh_train(mbh_dataset *ds, const mbh_params *p, mbh_fit **out, char *err, int32_t err_len) {
    if (!ds || !p || !out) {
        set_err(err, err_len, "null argument");
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    auto *fit = new mbh_fit();
    std::vector<hipEvent_t> events;
    try {
        check_params(ds, p);
        Run run;
        TrainBuffers tb = setup_state(ds, p, run);
        mb::DevState &s = tb.s;
        setup_record_partition(s, ds, p, run);
        const int K = s.hp.num_class;
        fit->num_class = K;
        fit->objective = p->objective;
        fit->n_features = ds->F;
        fit->learning_rate = p->learning_rate;
        fit->base = base_scores_for(ds, p->objective, K);
        double *d_base = dalloc<double>(K, run.owned);
        HIPX(hipMemcpy(d_base, fit->base.data(), K * sizeof(double), hipMemcpyHostToDevice));
        const int grid_rows = 8 * ds->n_cu;
        HIPX(mb::launch_fill_f64(s.raw, ds->n, K, d_base, grid_rows, nullptr));
        HIPX(mb::prepare_kernels(s));
        const int grid_score = mb::rows_grid(s, mb::kRowsScore, ds->n_cu);
        const int grid_score_obj = mb::rows_grid(s, mb::kRowsScoreObjective, ds->n_cu);
        const int grid_softmax = mb::rows_grid(s, mb::kRowsSoftmax, ds->n_cu);
        HIPX(hipDeviceSynchronize());
        const int L = tb.L;
        const int T = p->num_iterations * K;
        const bool timed = p->time_histograms != 0;
        hipStream_t st = nullptr;
        PinnedFlags flags;
        HIPX(hipHostMalloc((void **)&flags.p, 2 * sizeof(mb::Batch), hipHostMallocDefault));
        // events: [0..1] flag markers of the two in-flight groups; when
        // timed, [2..4] the root build (kernel start, kernel end, after its
        // scan + plan) and per group slot kMaxGroup x 6: the partition and
        // the accumulation kernels' own start and end (recorded by the
        // launch itself, so no queue gap is counted) and stream events
        // around scan + plan
        constexpr int kEvPer = 6;
        const int n_ev = 2 + (timed ? 3 + 2 * kMaxGroup * kEvPer : 0);
        events.resize(n_ev);
        for (int i = 0; i < n_ev; ++i)
            HIPX(hipEventCreateWithFlags(&events[i], i < 2 ? hipEventDisableTiming : hipEventDefault));
        auto ev_group = [&](int slot, int c, int k) {
            return events[5 + (slot * kMaxGroup + c) * kEvPer + k];
        };
        double t_acc = 0.0, t_root = 0.0, t_root_scan = 0.0, t_pb = 0.0, t_scan = 0.0;
        double t_part = 0.0, t_accum = 0.0;
        double pb_launches = 0.0;
        // per launch of a group slot: its tree and iteration index
        int group_tree[2] = {0, 0}, group_iter0[2] = {0, 0};
        std::vector<double> launch_ms;  // tree, iteration, partition ms, accumulation ms
        auto add_group = [&](int slot, int n) {
            for (int c = 0; c < n; ++c) {
                float a = 0.f, b = 0.f, d = 0.f;
                HIPX(hipEventElapsedTime(&a, ev_group(slot, c, 0), ev_group(slot, c, 1)));
                HIPX(hipEventElapsedTime(&b, ev_group(slot, c, 2), ev_group(slot, c, 3)));
                HIPX(hipEventElapsedTime(&d, ev_group(slot, c, 4), ev_group(slot, c, 5)));
                t_part += a;
                t_accum += b;
                t_pb += a + b;
                t_scan += d;
                launch_ms.insert(launch_ms.end(), {(double)group_tree[slot], (double)(group_iter0[slot] + c),
                                                   (double)a, (double)b});
            }
        };
        if (timed) {
            s.iter_stride = L + kMaxGroup + 4;
            s.iter_log = dalloc<int64_t>((size_t)T * s.iter_stride * 2, run.owned);
            HIPX(hipMemset(s.iter_log, 0, (size_t)T * s.iter_stride * 2 * sizeof(int64_t)));
        }
        // expansion launches the previous tree needed: the first group of a
        // tree is that long, later groups kNextGroup
        int est = kFirstGroup;
        // single-output L2 / binary: the score update of tree t computes the
        // objective of tree t + 1 in the same pass
        const bool fuse_objective =
            K == 1 && (p->objective == MBH_OBJ_BINARY || p->objective == MBH_OBJ_REGRESSION);
        // Multiclass: the K trees of a round are independent (each reads the
        // round's probabilities and writes only its class's scores), so S
        // states grow them side by side, each on its own stream, and the
        // latency-bound launches of several trees overlap on the chip. A
        // state grows classes j, j + S, ...; every round starts with the
        // softmax (and the GOSS sample) on state 0's stream, and state 0
        // joins the others' streams before the round's stop rule. Timed
        // runs and the record partition keep the single stream.
        const int S = (K > 1 && !timed && !s.rcp) ? std::min(K, mb::kMaxClassStates) : 1;
        std::vector<ClassState> cs(S > 1 ? S : 0);
        if (S > 1) {
            s.hp.class_stride = S;
            for (int j = 0; j < S; ++j) {
                ClassState &c = cs[j];
                c.s = j == 0 ? s : clone_class_state(s, ds, j, S, L, tb.max_nodes, run);
                c.est = kFirstGroup;
                HIPX(hipStreamCreateWithFlags(&c.st, hipStreamNonBlocking));
                HIPX(hipHostMalloc((void **)&c.flags.p, 2 * sizeof(mb::Batch), hipHostMallocDefault));
                for (int e = 0; e < 2; ++e) HIPX(hipEventCreateWithFlags(&c.ev[e], hipEventDisableTiming));
                HIPX(hipEventCreateWithFlags(&c.done, hipEventDisableTiming));
            }
            HIPX(hipDeviceSynchronize());
        }
        auto t0 = std::chrono::steady_clock::now();
        if (S > 1) {
            // one iteration group of state c in header slot `slot`: its last
            // planning launch writes the batch header there
            auto enqueue_group = [&](ClassState &c, int slot, int n, bool first) {
                for (int i = 0; i < n; ++i) {
                    HIPX(mb::launch_partition(c.s, c.st, nullptr, nullptr, c.s.part_root && first && i == 0));
                    HIPX(mb::launch_accum(c.s, c.st));
                    HIPX(mb::launch_scan(c.s, 0, c.st));
                    HIPX(mb::launch_plan(c.s, 0, c.st, i == n - 1 ? &c.flags.p[slot] : nullptr));
                }
                pb_launches += n;
                HIPX(hipEventRecord(c.ev[slot], c.st));
            };
            // a class tree's objective, quantizer and root, then two
            // iteration groups in flight (as the single-stream loop)
            auto start_tree = [&](ClassState &c) {
                mb::DevState &z = c.s;
                HIPX(mb::launch_objective(z, grid_rows, c.st));
                if (z.hp.goss && z.hp.quantized) HIPX(mb::launch_goss_stats(z, grid_rows, c.st));
                if (z.hp.wide) HIPX(mb::launch_magnitude(z, c.st));
                const bool fuse_q = mb::acc_kind(z.hp) == mb::kAccQuant && !z.hp.grad64;
                const bool q_rows = !fuse_q || z.hp.bagging || z.hp.goss;
                HIPX(mb::launch_quantize(z, q_rows ? grid_rows : 1, c.st, !fuse_q));
                HIPX(mb::launch_hist(z, c.st, nullptr, nullptr, fuse_q));
                HIPX(mb::launch_scan(z, 1, c.st));
                HIPX(mb::launch_plan(z, 1, c.st));
                const int n0 = std::max(1, std::min(c.est - 2, kMaxGroup));
                enqueue_group(c, 0, n0, true);
                enqueue_group(c, 1, kStateNextGroup, false);
                c.pending = 0;
                c.iters = n0 + kStateNextGroup;
                c.growing = true;
            };
            // reads the header of the group in flight longest once its
            // marker completed: the tree is finished (score update, round
            // end) or one more group is enqueued in the freed slot
            auto poll = [&](ClassState &c) {
                const hipError_t q = hipEventQuery(c.ev[c.pending]);
                if (q == hipErrorNotReady) return;
                HIPX(q);
                if (c.flags.p[c.pending].done) {
                    c.est = c.flags.p[c.pending].iters;
                    HIPX(mb::launch_score(c.s, grid_score, c.st));
                    HIPX(mb::launch_round_end(c.s, c.st));
                    c.growing = false;
                    c.cls += S;
                    return;
                }
                if (c.iters > L + kMaxGroup + 2)
                    throw Error{MOJOTREES_ERROR_TRAINING, "tree growth did not finish (internal error)"};
                enqueue_group(c, c.pending, kStateNextGroup, false);
                c.iters += kStateNextGroup;
                c.pending = 1 - c.pending;
            };
            mb::RoundStates rs{};
            rs.n = S;
            for (int j = 0; j < S; ++j) rs.r[j] = cs[j].s.round;
            const int sampling = (s.hp.bagging || s.hp.goss) ? 1 : 0;
            for (int rr = 0; rr < T / K; ++rr) {
                ClassState &c0 = cs[0];
                HIPX(mb::launch_softmax(c0.s, grid_softmax, c0.st));
                if (c0.s.hp.goss) HIPX(mb::launch_goss(c0.s, grid_rows, c0.st));
                HIPX(hipEventRecord(c0.done, c0.st));
                for (int j = 1; j < S; ++j) HIPX(hipStreamWaitEvent(cs[j].st, c0.done, 0));
                for (int j = 0; j < S; ++j) cs[j].cls = j;
                for (;;) {
                    bool active = false;
                    for (ClassState &c : cs) {
                        if (!c.growing && c.cls < K) start_tree(c);
                        if (c.growing) {
                            active = true;
                            poll(c);
                        }
                    }
                    if (!active) break;
                }
                for (int j = 1; j < S; ++j) {
                    HIPX(hipEventRecord(cs[j].done, cs[j].st));
                    HIPX(hipStreamWaitEvent(c0.st, cs[j].done, 0));
                }
                HIPX(mb::launch_round_combine(rs, sampling, c0.st));
            }
            HIPX(hipDeviceSynchronize());
            for (int j = 1; j < S; ++j) check_stage16(cs[j].s, ds->n);
        }
        for (int t = 0; S == 1 && t < T; ++t) {
            // GOSS draws its sample after the derivatives it ranks rows by
            // and before the quantizer, which sees the weighted derivatives
            // (goss_round, then the grower's quantizer): per tree for a
            // single output, once per round from the softmax probabilities
            // for multiclass (every class tree of the round on that sample)
            if (K > 1 && t % K == 0) {
                HIPX(mb::launch_softmax(s, grid_softmax, st));
                if (s.hp.goss) HIPX(mb::launch_goss(s, grid_rows, st));
            }
            if (!(fuse_objective && t > 0)) HIPX(mb::launch_objective(s, grid_rows, st));
            if (s.hp.goss && K == 1) HIPX(mb::launch_goss(s, grid_rows, st));
            if (s.hp.goss && s.hp.quantized) HIPX(mb::launch_goss_stats(s, grid_rows, st));
            if (s.hp.wide) HIPX(mb::launch_magnitude(s, st));
            // the max-abs lattice quantizes in the root build, which reads
            // every record of the round's rows anyway
            const bool fuse_q = mb::acc_kind(s.hp) == mb::kAccQuant && !s.hp.grad64;
            // with the pairs written by the root build and no row list to
            // gather (no bag, no GOSS), one block publishes the scales
            const bool q_rows = !fuse_q || s.hp.bagging || s.hp.goss;
            // ... in the previous tree's round-end launch when nothing is
            // launched between the two
            const bool merge_rq = K == 1 && fuse_objective && !s.hp.goss && !s.hp.wide && !q_rows;
            if (!(merge_rq && t > 0)) HIPX(mb::launch_quantize(s, q_rows ? grid_rows : 1, st, !fuse_q));
            if (timed) HIPX(mb::launch_hist(s, st, events[2], events[3], fuse_q));
            else HIPX(mb::launch_hist(s, st, nullptr, nullptr, fuse_q));
            HIPX(mb::launch_scan(s, 1, st));
            HIPX(mb::launch_plan(s, 1, st));
            if (timed) HIPX(hipEventRecord(events[4], st));
            int iters = 0;
            int group_size[2] = {0, 0};
            for (int k = 0;; ++k) {
                const int slot = k & 1;
                // a little short of the previous tree: a tree that needs more
                // costs one more group read, one that needs fewer costs empty
                // launches
                const int n = k == 0 ? std::max(1, std::min(est - 2, kMaxGroup)) : kNextGroup;
                group_size[slot] = n;
                group_tree[slot] = t;
                group_iter0[slot] = iters;
                for (int c = 0; c < n; ++c) {
                    if (timed) {
                        HIPX(mb::launch_partition(s, st, ev_group(slot, c, 0), ev_group(slot, c, 1),
                                                  s.part_root && k == 0 && c == 0));
                        HIPX(mb::launch_accum(s, st, ev_group(slot, c, 2), ev_group(slot, c, 3)));
                        HIPX(hipEventRecord(ev_group(slot, c, 4), st));
                    } else {
                        HIPX(mb::launch_partition(s, st, nullptr, nullptr, s.part_root && k == 0 && c == 0));
                        HIPX(mb::launch_accum(s, st));
                    }
                    HIPX(mb::launch_scan(s, 0, st));
                    // the group's last planning launch also writes the header
                    // into the pinned slot the host reads after the event
                    HIPX(mb::launch_plan(s, 0, st, c == n - 1 ? &flags.p[slot] : nullptr));
                    if (timed) HIPX(hipEventRecord(ev_group(slot, c, 5), st));
                }
                pb_launches += n;
                iters += n;
                HIPX(hipEventRecord(events[slot], st));
                if (k == 0) continue;
                HIPX(hipEventSynchronize(events[1 - slot]));
                if (timed) add_group(1 - slot, group_size[1 - slot]);
                if (flags.p[1 - slot].done) {
                    est = flags.p[1 - slot].iters;
                    if (timed) {
                        HIPX(hipEventSynchronize(events[slot]));
                        add_group(slot, n);
                    }
                    break;
                }
                // every iteration commits at least one split once the first
                // batch is planned, so a tree ends within num_leaves + 1
                if (iters > L + kMaxGroup + 2)
                    throw Error{MOJOTREES_ERROR_TRAINING, "tree growth did not finish (internal error)"};
            }
            if (timed) {
                float a = 0.f, b = 0.f;
                HIPX(hipEventElapsedTime(&a, events[2], events[3]));
                HIPX(hipEventElapsedTime(&b, events[3], events[4]));
                t_root += a;
                t_root_scan += b;
            }
            if (fuse_objective && t + 1 < T) HIPX(mb::launch_score_objective(s, grid_score_obj, st));
            else HIPX(mb::launch_score(s, grid_score, st));
            if (merge_rq && t + 1 < T) HIPX(mb::launch_round_end_quantize(s, st));
            else HIPX(mb::launch_round_end(s, st));
        }
        HIPX(hipStreamSynchronize(st));
        auto t1 = std::chrono::steady_clock::now();
        t_acc = t_root + t_pb;
        int32_t h_error = 0;
        HIPX(hipMemcpy(&h_error, s.error, sizeof(int32_t), hipMemcpyDeviceToHost));
        if (h_error & 4)
            throw Error{MOJOTREES_ERROR_TRAINING,
                        "gradient/hessian magnitudes are out of range for the fixed-point histogram "
                        "(quant_scale_rule=magnitude_sum)"};
        if (h_error)
            throw Error{MOJOTREES_ERROR_TRAINING,
                        std::string("device growth check failed (internal error, code ") +
                            std::to_string(h_error) + ")"};
        check_stage16(s, ds->n);
        const int mn = tb.max_nodes;
        std::vector<int32_t> ai((size_t)tb.T * (6 * mn + 2));
        std::vector<double> ad((size_t)tb.T * 3 * mn);
        std::vector<int64_t> ax((size_t)tb.T * 4);
        HIPX(hipMemcpy(ai.data(), s.arc_int, ai.size() * sizeof(int32_t), hipMemcpyDeviceToHost));
        HIPX(hipMemcpy(ad.data(), s.arc_dbl, ad.size() * sizeof(double), hipMemcpyDeviceToHost));
        HIPX(hipMemcpy(ax.data(), s.arc_aux, ax.size() * sizeof(int64_t), hipMemcpyDeviceToHost));
        if (timed) {
            // each launch's rows from the planner's log (zero for the empty
            // launches after a tree is done)
            std::vector<int64_t> lg((size_t)T * s.iter_stride * 2);
            HIPX(hipMemcpy(lg.data(), s.iter_log, lg.size() * sizeof(int64_t), hipMemcpyDeviceToHost));
            for (size_t i = 0; i + 3 < launch_ms.size(); i += 4) {
                const int t = (int)launch_ms[i], it = (int)launch_ms[i + 1];
                const bool in = it < s.iter_stride;
                const size_t o = 2 * ((size_t)t * s.iter_stride + (in ? it : 0));
                fit->launch_log.insert(fit->launch_log.end(),
                                       {(double)t, (double)it, in ? (double)lg[o] : 0.0, in ? (double)lg[o + 1] : 0.0,
                                        launch_ms[i + 2], launch_ms[i + 3]});
            }
        }
        std::vector<unsigned long long> acat;
        if (s.arc_cat) {
            acat.resize((size_t)tb.T * mn * 4);
            HIPX(hipMemcpy(acat.data(), s.arc_cat, acat.size() * sizeof(unsigned long long), hipMemcpyDeviceToHost));
        }
        fit->train_raw.resize((size_t)ds->n * K);
        HIPX(hipMemcpy(fit->train_raw.data(), s.raw, fit->train_raw.size() * sizeof(double),
                       hipMemcpyDeviceToHost));
        if (K > 1) {  // the device's class-major scores to the row-major layout of the API
            std::vector<double> cm(fit->train_raw);
            for (int64_t r = 0; r < ds->n; ++r)
                for (int k = 0; k < K; ++k) fit->train_raw[(size_t)r * K + k] = cm[(size_t)k * ds->n + r];
        }
        const bool bagging = s.hp.bagging != 0 || s.hp.goss != 0;  // sampled rounds are skipped, not stops
        // algorithmic bytes per accumulated row: its bins plus its g/h pair
        // (int8 x 2 quantized, fp32 x 2 otherwise)
        const double rb = ds->F + (s.hp.wide ? 8 : s.hp.quantized ? 2 : 8);
        // a root build that quantizes (max-abs lattice) also reads each root
        // row's binary32 g, h and writes its int8 pair: the quantizer's
        // algorithmic bytes are the root kernel's too
        const double rq = mb::acc_kind(s.hp) == mb::kAccQuant && !s.hp.grad64 ? 10.0 : 0.0;
        double useful_rows = 0.0, builds = 0.0, root_rows = 0.0;
        double iters_total = 0.0, exps = 0.0, rows_built = 0.0, rows_parted = 0.0;
        int grown = 0;
        auto tree_int = [&](int t) { return ai.data() + (size_t)t * (6 * mn + 2); };
        auto tree_dbl = [&](int t) { return ad.data() + (size_t)t * 3 * mn; };
        auto degenerate = [&](int t) {
            return tree_int(t)[6 * mn + 1] == 1 && std::fabs(tree_dbl(t)[0]) < 1e-12;
        };
        const int R = T / K;
        for (int rr = 0; rr < R; ++rr) {
            bool progress = false;
            for (int k = 0; k < K; ++k) {
                const int t = rr * K + k;
                const int32_t *ti = tree_int(t);
                const double *td = tree_dbl(t);
                const int nn = ti[6 * mn];
                // builds of the committed tree: the root, then the smaller
                // child of every split
                root_rows += td[2];
                useful_rows += td[2];
                builds += 1;
                for (int i = 0; i < nn; ++i) {
                    if (ti[6 * i] < 0) continue;
                    const double cl = td[3 * ti[6 * i + 2] + 2], cr = td[3 * ti[6 * i + 3] + 2];
                    useful_rows += std::min(cl, cr);
                    builds += 1;
                }
                rows_built += (double)ax[(size_t)t * 4 + 0];
                iters_total += (double)ax[(size_t)t * 4 + 1];
                exps += (double)ax[(size_t)t * 4 + 2];
                rows_parted += (double)ax[(size_t)t * 4 + 3];
                progress |= !degenerate(t);
            }
            // boosting._boost_rounds' stop rule (boosting.mojo:2898-2907):
            // a round that does not move ends training, or is skipped when
            // rows are sampled; multiclass judges the round's K trees
            // together (:3876-4165)
            if (!progress) {
                if (bagging) continue;
                break;
            }
            for (int k = 0; k < K; ++k) {
                const int t = rr * K + k;
                const int32_t *ti = tree_int(t);
                const double *td = tree_dbl(t);
                const int nn = ti[6 * mn];
                for (int i = 0; i < nn; ++i) {
                    fit->feature.push_back(ti[6 * i + 0]);
                    fit->threshold.push_back(ti[6 * i + 1]);
                    fit->left.push_back(ti[6 * i + 2]);
                    fit->right.push_back(ti[6 * i + 3]);
                    fit->default_left.push_back(ti[6 * i + 4]);
                    fit->missing_bin.push_back(ti[6 * i + 5]);
                    fit->value.push_back(td[3 * i + 0]);
                    fit->gain.push_back(td[3 * i + 1]);
                    fit->count.push_back(td[3 * i + 2]);
                    for (int w = 0; w < 4; ++w)
                        fit->cat_bits.push_back(acat.empty() ? 0ULL : acat[((size_t)t * mn + i) * 4 + w]);
                }
                fit->offsets.push_back((int64_t)fit->feature.size());
                ++grown;
            }
        }
        double *o = fit->stats;
        o[0] = std::chrono::duration<double>(t1 - t0).count();
        o[1] = t_acc;
        o[2] = useful_rows * rb;
        o[3] = useful_rows * ds->F;
        o[4] = builds;
        o[5] = root_rows * rb;
        o[6] = t_root;
        o[7] = grown;
        o[8] = t_root + t_root_scan + t_pb + t_scan;
        o[9] = t_root + t_root_scan;
        o[10] = iters_total;
        o[11] = exps;
        o[12] = rows_built;
        o[13] = rows_parted;
        o[14] = pb_launches;
        o[15] = t_pb;
        o[16] = rows_parted * 9.0 + rows_built * rb;
        o[17] = t_part;
        o[18] = t_accum;
        o[19] = rows_built * rb;
        o[20] = root_rows * rq;
        // the partitions' algorithmic bytes: row ids in and out and the
        // split column's byte, or each row's record in and out (the root's
        // pair read from the pair plane)
        o[21] = s.rcp ? rows_parted * 2.0 * s.rec_bytes + root_rows * 2.0 : rows_parted * 9.0;
        for (auto &e : events) (void)hipEventDestroy(e);
        events.clear();
    } catch (const Error &e) {
        for (auto &ev : events) (void)hipEventDestroy(ev);
        set_err(err, err_len, e.msg);
        delete fit;
        return e.code;
    }
    *out = fit;
    return MOJOTREES_OK;
}

void mbh_fit_free(mbh_fit *fit) { delete fit; }
int32_t mbh_fit_num_trees(const mbh_fit *fit) { return (int32_t)fit->offsets.size() - 1; }
int32_t mbh_fit_num_class(const mbh_fit *fit) { return fit->num_class; }
int64_t mbh_fit_total_nodes(const mbh_fit *fit) { return (int64_t)fit->feature.size(); }
void mbh_fit_arrays(const mbh_fit *fit, double *base, int64_t *off, int32_t *feature, int32_t *thr,
                    int32_t *left, int32_t *right, double *value, int32_t *dl, int32_t *mb_,
                    double *gain, double *count) {
    for (int k = 0; k < fit->num_class; ++k) base[k] = fit->base[k];
    std::memcpy(off, fit->offsets.data(), fit->offsets.size() * sizeof(int64_t));
    const size_t nn = fit->feature.size();
    std::memcpy(feature, fit->feature.data(), nn * sizeof(int32_t));
    std::memcpy(thr, fit->threshold.data(), nn * sizeof(int32_t));
    std::memcpy(left, fit->left.data(), nn * sizeof(int32_t));
    std::memcpy(right, fit->right.data(), nn * sizeof(int32_t));
    std::memcpy(value, fit->value.data(), nn * sizeof(double));
    std::memcpy(dl, fit->default_left.data(), nn * sizeof(int32_t));
    std::memcpy(mb_, fit->missing_bin.data(), nn * sizeof(int32_t));
    std::memcpy(gain, fit->gain.data(), nn * sizeof(double));
    std::memcpy(count, fit->count.data(), nn * sizeof(double));
}
void mbh_fit_cat_bits(const mbh_fit *fit, uint64_t *out) {
    if (fit && out) std::memcpy(out, fit->cat_bits.data(), fit->cat_bits.size() * sizeof(uint64_t));
}
int32_t mbh_fit_train_raw(const mbh_fit *fit, double *out, char *err, int32_t err_len) {
    if (!fit || !out) {
        set_err(err, err_len, "null argument");
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    std::memcpy(out, fit->train_raw.data(), fit->train_raw.size() * sizeof(double));
    return MOJOTREES_OK;
}
int64_t mbh_fit_launch_log(const mbh_fit *fit, double *out, int64_t n_out) {
    if (!fit) return 0;
    const int64_t n = (int64_t)fit->launch_log.size();
    if (out)
        for (int64_t i = 0; i < n && i < n_out; ++i) out[i] = fit->launch_log[(size_t)i];
    return n;
}
int32_t mbh_fit_stats(const mbh_fit *fit, double *out, int32_t n_out) {
    if (fit && out)
        for (int i = 0; i < kNumStats && i < n_out; ++i) out[i] = fit->stats[i];
    return kNumStats;
}

int32_t mbh_exp_sigmoid(const double *x, int64_t n, double *out_exp, double *out_sig, char *err,
                        int32_t err_len) {
    if (!x || !out_exp || !out_sig || n <= 0) {
        set_err(err, err_len, "invalid arguments");
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    if (device_count_gfx950() == 0) {
        set_err(err, err_len, "no gfx950 device");
        return MOJOTREES_ERROR_UNSUPPORTED;
    }
    Run run;
    try {
        double *dx = dalloc<double>(n, run.owned), *de = dalloc<double>(n, run.owned),
               *dsg = dalloc<double>(n, run.owned);
        HIPX(hipMemcpy(dx, x, n * sizeof(double), hipMemcpyHostToDevice));
        HIPX(mb::launch_exp_sigmoid(dx, de, dsg, n, nullptr));
        HIPX(hipMemcpy(out_exp, de, n * sizeof(double), hipMemcpyDeviceToHost));
        HIPX(hipMemcpy(out_sig, dsg, n * sizeof(double), hipMemcpyDeviceToHost));
    } catch (const Error &e) {
        set_err(err, err_len, e.msg);
        return e.code;
    }
    return MOJOTREES_OK;
}

int32_t mbh_dataset_set_weights(mbh_dataset *ds, const double *weights, int64_t n_weights, char *err,
                                int32_t err_len) {
    // boosting._check_sample_weight (src/mojotrees/boosting.mojo:334-343):
    // one finite, nonnegative weight per row with a positive sum; null clears
    if (!ds) {
        set_err(err, err_len, "null dataset");
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    try {
        if (!weights) {
            ds->weights.clear();
            ds->class_weight.clear();
            ds->d_weights = nullptr;  // the buffer stays owned until the dataset is freed
            return MOJOTREES_OK;
        }
        if (n_weights != ds->n) throw Error{MOJOTREES_ERROR_INVALID_ARGUMENT, "sample_weight length must equal n_rows"};
        double total = 0.0, wy = 0.0;
        for (int64_t r = 0; r < ds->n; ++r) {
            const double w = weights[r];
            if (!std::isfinite(w) || w < 0.0)
                throw Error{MOJOTREES_ERROR_INVALID_ARGUMENT, "sample_weight must be finite and nonnegative"};
            total += w;
        }
        if (!(total > 0.0)) throw Error{MOJOTREES_ERROR_INVALID_ARGUMENT, "sample_weight must have a positive sum"};
        // the labels are on the device only; the base score needs Σ w·y
        std::vector<double> y((size_t)ds->n);
        HIPX(hipMemcpy(y.data(), ds->d_labels, (size_t)ds->n * sizeof(double), hipMemcpyDeviceToHost));
        for (int64_t r = 0; r < ds->n; ++r) wy += weights[r] * y[r];
        ds->class_weight.clear();
        if (ds->labels_integral) {
            ds->class_weight.assign(ds->class_count.size(), 0.0);
            for (int64_t r = 0; r < ds->n; ++r) ds->class_weight[(size_t)y[r]] += weights[r];
        }
        ds->weights.assign(weights, weights + ds->n);
        if (!ds->d_weights_buf) ds->d_weights_buf = dalloc<double>(ds->n, ds->owned);
        HIPX(hipMemcpy(ds->d_weights_buf, weights, (size_t)ds->n * sizeof(double), hipMemcpyHostToDevice));
        ds->d_weights = ds->d_weights_buf;
        ds->weight_sum = total;
        ds->wlabel_sum = wy;
    } catch (const Error &e) {
        set_err(err, err_len, e.msg);
        return e.code;
    }
    return MOJOTREES_OK;
}

int32_t mbh_dataset_set_groups(mbh_dataset *ds, const int32_t *counts, int64_t nq, char *err, int32_t err_len) {
    if (!ds || !counts || nq < 1) {
        set_err(err, err_len, "group must contain at least one query");
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    try {
        // groups_from_counts + check_groups (ranking.mojo:152-169, :205-218)
        std::vector<int64_t> st(nq + 1, 0);
        int max_q = 0;
        for (int64_t q = 0; q < nq; ++q) {
            if (counts[q] <= 0) throw Error{MOJOTREES_ERROR_INVALID_ARGUMENT, "group counts must be positive"};
            st[q + 1] = st[q] + counts[q];
            max_q = std::max(max_q, counts[q]);
        }
        if (st[nq] != ds->n) throw Error{MOJOTREES_ERROR_INVALID_ARGUMENT, "group counts must sum to n_rows"};
        if (max_q > (1 << 30))
            throw Error{MOJOTREES_ERROR_UNSUPPORTED, "a query holds more than 2^30 rows"};
        int64_t *d = dalloc<int64_t>(nq + 1, ds->owned);
        HIPX(hipMemcpy(d, st.data(), st.size() * sizeof(int64_t), hipMemcpyHostToDevice));
        ds->qstart = std::move(st);
        ds->d_qstart = d;
        ds->max_query = max_q;
    } catch (const Error &e) {
        set_err(err, err_len, e.msg);
        return e.code;
    }
    return MOJOTREES_OK;
}

int32_t mbh_lambdarank(mbh_dataset *ds, const mbh_params *p, const double *raw, double *grad, double *hess,
                       char *err, int32_t err_len) {
    if (!ds || !p || !raw || !grad || !hess) {
        set_err(err, err_len, "null argument");
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    try {
        mbh_params p1 = *p;
        p1.objective = MBH_OBJ_LAMBDARANK;
        p1.num_iterations = 1;
        check_params(ds, &p1);
        Run run;
        TrainBuffers tb = setup_state(ds, &p1, run);
        mb::DevState &s = tb.s;
        HIPX(hipMemcpy(s.raw, raw, ds->n * sizeof(double), hipMemcpyHostToDevice));
        HIPX(mb::prepare_kernels(s));
        HIPX(mb::launch_objective(s, 8 * ds->n_cu, nullptr));
        HIPX(hipDeviceSynchronize());
        HIPX(hipMemcpy(grad, s.grad64, ds->n * sizeof(double), hipMemcpyDeviceToHost));
        HIPX(hipMemcpy(hess, s.hess64, ds->n * sizeof(double), hipMemcpyDeviceToHost));
    } catch (const Error &e) {
        set_err(err, err_len, e.msg);
        return e.code;
    }
    return MOJOTREES_OK;
}

int32_t mbh_predict_binned(const uint8_t *bins_cm, int64_t n, int32_t F, int32_t num_class,
                           double learning_rate, const double *base, const int64_t *node_offset,
                           int64_t tree_begin, int64_t tree_end, const int32_t *feature,
                           const int32_t *threshold, const int32_t *left, const int32_t *right,
                           const double *value, const int32_t *default_left, const int32_t *missing_bin,
                           const uint64_t *cat_bits, double *out, char *err, int32_t err_len) {
    if (!bins_cm || !node_offset || !feature || !threshold || !left || !right || !value || !default_left ||
        !missing_bin || !out || n <= 0 || F <= 0 || num_class <= 0 || tree_begin < 0 || tree_end < tree_begin ||
        tree_begin % num_class != 0) {
        set_err(err, err_len, "invalid prediction arguments");
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    if (device_count_gfx950() == 0) {
        set_err(err, err_len, "no gfx950 (MI355X) device is available to this process");
        return MOJOTREES_ERROR_UNSUPPORTED;
    }
    Run run;
    try {
        const int K = num_class;
        // the trees in range, rebased: absolute child indices, validated so
        // that every walk moves to a larger index and ends at a leaf
        const int64_t o0 = node_offset[tree_begin], o1 = node_offset[tree_end];
        const int64_t nn = o1 - o0;
        if (nn < 0 || nn >= ((int64_t)1 << 31))
            throw Error{MOJOTREES_ERROR_INVALID_ARGUMENT, "invalid node offsets"};
        std::vector<int4> nodes((size_t)std::max<int64_t>(nn, 1));
        std::vector<int32_t> md((size_t)std::max<int64_t>(nn, 1)), root((size_t)std::max<int64_t>(tree_end - tree_begin, 1));
        int32_t max_steps = 1;
        for (int64_t t = tree_begin; t < tree_end; ++t) {
            const int64_t a = node_offset[t], b = node_offset[t + 1];
            if (b <= a || a < o0 || b > o1) throw Error{MOJOTREES_ERROR_INVALID_ARGUMENT, "invalid node offsets"};
            max_steps = std::max<int32_t>(max_steps, (int32_t)(b - a));
            root[t - tree_begin] = (int32_t)(a - o0);
            for (int64_t i = a; i < b; ++i) {
                const int64_t loc = i - a;
                int4 v;
                v.x = feature[i] >= 0 ? feature[i] : -1;
                v.y = threshold[i];
                v.z = (int32_t)(a - o0 + left[i]);
                v.w = (int32_t)(a - o0 + right[i]);
                if (feature[i] >= 0 && (feature[i] >= F || left[i] <= loc || right[i] <= loc ||
                                        left[i] >= b - a || right[i] >= b - a))
                    throw Error{MOJOTREES_ERROR_INVALID_ARGUMENT, "malformed tree: a child index must exceed its parent's"};
                // a node without a threshold is categorical and routes by its set
                if (feature[i] >= 0 && threshold[i] < 0 && !cat_bits)
                    throw Error{MOJOTREES_ERROR_INVALID_ARGUMENT, "a categorical node needs its category set (cat_bits)"};
                nodes[i - o0] = v;
                md[i - o0] = missing_bin[i] * 2 + (default_left[i] ? 1 : 0);
            }
        }
        std::vector<double> vals(value + o0, value + o0 + std::max<int64_t>(nn, 0));
        if (vals.empty()) vals.push_back(0.0);
        int dev = 0;
        HIPX(hipGetDevice(&dev));
        hipDeviceProp_t prop;
        HIPX(hipGetDeviceProperties(&prop, dev));
        int4 *d_nodes = dalloc<int4>(nodes.size(), run.owned);
        int32_t *d_md = dalloc<int32_t>(md.size(), run.owned);
        int32_t *d_root = dalloc<int32_t>(root.size(), run.owned);
        double *d_val = dalloc<double>(vals.size(), run.owned);
        double *d_base = base ? dalloc<double>(K, run.owned) : nullptr;
        unsigned long long *d_cat = nullptr;
        if (cat_bits) {
            d_cat = dalloc<unsigned long long>((size_t)std::max<int64_t>(nn, 1) * 4, run.owned);
            HIPX(hipMemcpy(d_cat, cat_bits + (size_t)o0 * 4, (size_t)std::max<int64_t>(nn, 0) * 4 * sizeof(uint64_t),
                           hipMemcpyHostToDevice));
        }
        HIPX(hipMemcpy(d_nodes, nodes.data(), nodes.size() * sizeof(int4), hipMemcpyHostToDevice));
        HIPX(hipMemcpy(d_md, md.data(), md.size() * sizeof(int32_t), hipMemcpyHostToDevice));
        HIPX(hipMemcpy(d_root, root.data(), root.size() * sizeof(int32_t), hipMemcpyHostToDevice));
        HIPX(hipMemcpy(d_val, vals.data(), vals.size() * sizeof(double), hipMemcpyHostToDevice));
        if (base) HIPX(hipMemcpy(d_base, base, K * sizeof(double), hipMemcpyHostToDevice));
        // row batches bound the device copy of the matrix (bins + records)
        RecLayout l;
        l.n_tiles = (F + 125) / 126;
        l.tile_f = (F + l.n_tiles - 1) / l.n_tiles;
        l.rec = 16;
        while (l.rec < l.tile_f + 2) l.rec *= 2;
        const int64_t per_row = (int64_t)F + (int64_t)l.rec * l.n_tiles + 8 * K;
        const int64_t batch = std::max<int64_t>(4096, std::min<int64_t>(n, ((int64_t)1 << 31) / per_row));
        uint8_t *d_bins = dalloc<uint8_t>((size_t)F * batch, run.owned);
        uint8_t *d_rec = dalloc<uint8_t>((size_t)l.rec * l.n_tiles * batch, run.owned);
        double *d_out = dalloc<double>((size_t)batch * K, run.owned);
        std::vector<uint8_t> stage((size_t)F * batch);
        for (int64_t r0 = 0; r0 < n; r0 += batch) {
            const int64_t m = std::min(batch, n - r0);
            for (int f = 0; f < F; ++f)
                std::memcpy(stage.data() + (size_t)f * m, bins_cm + (size_t)f * n + r0, (size_t)m);
            HIPX(hipMemcpy(d_bins, stage.data(), (size_t)F * m, hipMemcpyHostToDevice));
            HIPX(mb::launch_build_records(d_bins, d_rec, m, F, l.rec, l.tile_f, l.n_tiles, 4 * prop.multiProcessorCount,
                                          nullptr));
            mb::PredictArgs a{};
            a.records = d_rec;
            a.n = m;
            a.rec_bytes = l.rec;
            a.tile_f = l.tile_f;
            a.n_tiles = l.n_tiles;
            a.num_class = K;
            a.nodes = d_nodes;
            a.md = d_md;
            a.cat = d_cat;
            a.value = d_val;
            a.root = d_root;
            a.max_steps = max_steps;
            a.t0 = 0;
            a.t1 = tree_end - tree_begin;
            a.learning_rate = learning_rate;
            a.base = d_base;
            a.out = d_out;
            const int grid = (int)std::min<int64_t>((m + 255) / 256, 16 * (int64_t)prop.multiProcessorCount);
            HIPX(mb::launch_predict(a, grid, nullptr));
            HIPX(hipMemcpy(out + r0 * K, d_out, (size_t)m * K * sizeof(double), hipMemcpyDeviceToHost));
        }
    } catch (const Error &e) {
        set_err(err, err_len, e.msg);
        return e.code;
    }
    return MOJOTREES_OK;
}

int32_t mbh_objective_quantize(mbh_dataset *ds, const mbh_params *p, const double *raw,
                               int64_t round_index, float *grad, float *hess, int8_t *q_grad,
                               int8_t *q_hess, double *scales, char *err, int32_t err_len) {
    if (!ds || !p || !raw || !grad || !hess || !q_grad || !q_hess || !scales) {
        set_err(err, err_len, "null argument");
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    try {
        check_params(ds, p);
        Run run;
        mbh_params p1 = *p;
        p1.num_iterations = 1;
        if (round_index < 0) throw Error{MOJOTREES_ERROR_INVALID_ARGUMENT, "round_index must be nonnegative"};
        TrainBuffers tb = setup_state(ds, &p1, run, round_index);
        mb::DevState &s = tb.s;
        mb::Round r0 = mb::initial_round();
        r0.round = round_index;
        HIPX(hipMemcpy(s.round, &r0, sizeof(r0), hipMemcpyHostToDevice));
        HIPX(hipMemcpy(s.raw, raw, ds->n * sizeof(double), hipMemcpyHostToDevice));
        const int grid = 8 * ds->n_cu;
        HIPX(mb::launch_objective(s, grid, nullptr));
        HIPX(mb::launch_quantize(s, grid, nullptr));
        HIPX(hipDeviceSynchronize());
        download_derivatives(s, ds->n, grad, hess);
        // the pairs of tile 0 (every tile holds the same pair)
        std::vector<uint8_t> rec((size_t)ds->n * ds->rec);
        HIPX(hipMemcpy(rec.data(), ds->d_records, rec.size(), hipMemcpyDeviceToHost));
        for (int64_t r = 0; r < ds->n; ++r) {
            q_grad[r] = (int8_t)rec[(size_t)r * ds->rec + ds->rec - 2];
            q_hess[r] = (int8_t)rec[(size_t)r * ds->rec + ds->rec - 1];
        }
        mb::Round rr;
        HIPX(hipMemcpy(&rr, s.round, sizeof(rr), hipMemcpyDeviceToHost));
        scales[0] = rr.grad_units;
        scales[1] = rr.hess_units;
    } catch (const Error &e) {
        set_err(err, err_len, e.msg);
        return e.code;
    }
    return MOJOTREES_OK;
}

int32_t mbh_objective_quantize32(mbh_dataset *ds, const mbh_params *p, const double *raw, int64_t round_index,
                                 float *grad, float *hess, int32_t *q_grad, int32_t *q_hess, double *scales,
                                 char *err, int32_t err_len) {
    if (!ds || !p || !raw || !grad || !hess || !q_grad || !q_hess || !scales) {
        set_err(err, err_len, "null argument");
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    try {
        if (!p->use_quantized_grad) throw Error{MOJOTREES_ERROR_INVALID_ARGUMENT, "use_quantized_grad must be 1"};
        check_params(ds, p);
        Run run;
        mbh_params p1 = *p;
        p1.num_iterations = 1;
        if (round_index < 0) throw Error{MOJOTREES_ERROR_INVALID_ARGUMENT, "round_index must be nonnegative"};
        TrainBuffers tb = setup_state(ds, &p1, run, round_index);
        mb::DevState &s = tb.s;
        mb::Round r0 = mb::initial_round();
        r0.round = round_index;
        HIPX(hipMemcpy(s.round, &r0, sizeof(r0), hipMemcpyHostToDevice));
        HIPX(hipMemcpy(s.raw, raw, ds->n * sizeof(double), hipMemcpyHostToDevice));
        const int grid = 8 * ds->n_cu;
        HIPX(mb::launch_objective(s, grid, nullptr));
        if (s.hp.wide) HIPX(mb::launch_magnitude(s, nullptr));
        HIPX(mb::launch_quantize(s, grid, nullptr));
        HIPX(hipDeviceSynchronize());
        int32_t h_error = 0;
        HIPX(hipMemcpy(&h_error, s.error, sizeof(int32_t), hipMemcpyDeviceToHost));
        if (h_error & 4)
            throw Error{MOJOTREES_ERROR_TRAINING, "gradient/hessian magnitudes are out of range for the fixed-point histogram"};
        download_derivatives(s, ds->n, grad, hess);
        scales[4] = 0.0;
        scales[5] = 0.0;
        if (s.hp.stage16) {
            std::vector<uint8_t> rec((size_t)ds->n * ds->rec);
            HIPX(hipMemcpy(rec.data(), ds->d_records, rec.size(), hipMemcpyDeviceToHost));
            for (int64_t r = 0; r < ds->n; ++r) {
                int16_t g16, h16;
                std::memcpy(&g16, rec.data() + (size_t)r * ds->rec + ds->rec - 4, 2);
                std::memcpy(&h16, rec.data() + (size_t)r * ds->rec + ds->rec - 2, 2);
                q_grad[r] = g16;
                q_hess[r] = h16;
            }
            unsigned long long over[2];
            HIPX(hipMemcpy(over, s.stage16_over, sizeof(over), hipMemcpyDeviceToHost));
            scales[4] = (double)over[0];
            scales[5] = (double)over[1];
        } else if (s.hp.wide) {
            std::vector<int32_t> q(2 * (size_t)ds->n);
            HIPX(hipMemcpy(q.data(), s.gq, q.size() * sizeof(int32_t), hipMemcpyDeviceToHost));
            for (int64_t r = 0; r < ds->n; ++r) {
                q_grad[r] = q[2 * (size_t)r];
                q_hess[r] = q[2 * (size_t)r + 1];
            }
            float part[512];
            HIPX(hipMemcpy(part, s.magpart, sizeof(part), hipMemcpyDeviceToHost));
            double tg = 0.0, th = 0.0;
            for (int b = 0; b < 256; ++b) {
                tg += (double)part[b];
                th += (double)part[256 + b];
            }
            scales[2] = tg;
            scales[3] = th;
        } else {
            std::vector<uint8_t> rec((size_t)ds->n * ds->rec);
            HIPX(hipMemcpy(rec.data(), ds->d_records, rec.size(), hipMemcpyDeviceToHost));
            for (int64_t r = 0; r < ds->n; ++r) {
                q_grad[r] = (int8_t)rec[(size_t)r * ds->rec + ds->rec - 2];
                q_hess[r] = (int8_t)rec[(size_t)r * ds->rec + ds->rec - 1];
            }
            scales[2] = 0.0;
            scales[3] = 0.0;
        }
        mb::Round rr;
        HIPX(hipMemcpy(&rr, s.round, sizeof(rr), hipMemcpyDeviceToHost));
        scales[0] = rr.grad_units;
        scales[1] = rr.hess_units;
    } catch (const Error &e) {
        set_err(err, err_len, e.msg);
        return e.code;
    }
    return MOJOTREES_OK;
}

int32_t mbh_histogram32(mbh_dataset *ds, const int32_t *q_grad, const int32_t *q_hess, const int32_t *rows,
                        int64_t n_sel, int32_t *out, char *err, int32_t err_len) {
    if (!ds || !q_grad || !q_hess || !out || (rows && n_sel <= 0)) {
        set_err(err, err_len, "invalid arguments");
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    try {
        if (ds->n >= ((int64_t)1 << 30)) throw Error{MOJOTREES_ERROR_UNSUPPORTED, "n_rows must be below 2^30"};
        // every subset of the selection must sum within int32: the lattice's
        // headroom (|q| <= 2^30, sums of |q| below 2^31), checked here
        const int64_t m = rows ? n_sel : ds->n;
        int64_t sg = 0, sh = 0;
        for (int64_t i = 0; i < m; ++i) {
            const int64_t r = rows ? rows[i] : i;
            if (r < 0 || r >= ds->n) throw Error{MOJOTREES_ERROR_INVALID_ARGUMENT, "row id out of range"};
            if (q_hess[r] < 0) throw Error{MOJOTREES_ERROR_INVALID_ARGUMENT, "quantized hessians must be nonnegative"};
            sg += q_grad[r] < 0 ? -(int64_t)q_grad[r] : (int64_t)q_grad[r];
            sh += q_hess[r];
        }
        if (sg >= ((int64_t)1 << 31) || sh >= ((int64_t)1 << 31))
            throw Error{MOJOTREES_ERROR_INVALID_ARGUMENT, "the selection's quantized magnitudes exceed int32 cells"};
        Run run;
        mbh_params p{};
        p.objective = MBH_OBJ_BINARY;
        p.num_iterations = 1;
        p.num_leaves = 2;
        p.learning_rate = 0.1;
        p.feature_fraction = 1.0;
        p.bagging_fraction = 1.0;
        p.num_grad_quant_bins = 4;
        p.use_quantized_grad = 1;
        p.quant_scale_rule = 1;
        TrainBuffers tb = setup_state(ds, &p, run);
        mb::DevState &s = tb.s;
        std::vector<int32_t> q(2 * (size_t)ds->n);
        for (int64_t r = 0; r < ds->n; ++r) {
            q[2 * (size_t)r] = q_grad[r];
            q[2 * (size_t)r + 1] = q_hess[r];
        }
        HIPX(hipMemcpy(s.gq, q.data(), q.size() * sizeof(int32_t), hipMemcpyHostToDevice));
        const size_t cells = (size_t)ds->F * ds->nb * 3;
        mb::Round r0 = mb::initial_round();
        r0.grad_units = 1.0;
        r0.hess_units = 1.0;
        r0.sampled = rows ? 1 : 0;
        HIPX(hipMemcpy(s.round, &r0, sizeof(r0), hipMemcpyHostToDevice));
        if (rows) {
            HIPX(hipMemcpy(s.rows0, rows, n_sel * sizeof(int32_t), hipMemcpyHostToDevice));
            int64_t c[2] = {n_sel, 0};
            HIPX(hipMemcpy(s.cursor, c, sizeof(c), hipMemcpyHostToDevice));
        }
        HIPX(mb::prepare_kernels(s));
        HIPX(mb::launch_hist(s, nullptr));
        HIPX(mb::launch_scan(s, 1, nullptr));
        HIPX(hipDeviceSynchronize());
        HIPX(hipMemcpy(out, s.hist, cells * sizeof(int32_t), hipMemcpyDeviceToHost));
    } catch (const Error &e) {
        set_err(err, err_len, e.msg);
        return e.code;
    }
    return MOJOTREES_OK;
}

int32_t mbh_histogram(mbh_dataset *ds, const int8_t *q_grad, const int8_t *q_hess,
                      const int32_t *rows, int64_t n_sel, int32_t B, int32_t *out, char *err,
                      int32_t err_len) {
    if (!ds || !q_grad || !q_hess || !out || (rows && n_sel <= 0)) {
        set_err(err, err_len, "invalid arguments");
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    try {
        if (rows)
            for (int64_t i = 0; i < n_sel; ++i)
                if (rows[i] < 0 || rows[i] >= ds->n)
                    throw Error{MOJOTREES_ERROR_INVALID_ARGUMENT, "row id out of range"};
        for (int64_t r = 0; r < ds->n; ++r)
            if (q_grad[r] < -(B / 2 + 1) || q_grad[r] > B / 2 + 1 || q_hess[r] < 0 || q_hess[r] > B + 1)
                throw Error{MOJOTREES_ERROR_INVALID_ARGUMENT, "quantized value outside the lattice"};
        Run run;
        mbh_params p{};
        p.objective = MBH_OBJ_BINARY;
        p.num_iterations = 1;
        p.num_leaves = 2;
        p.learning_rate = 0.1;
        p.feature_fraction = 1.0;
        p.bagging_fraction = 1.0;
        p.num_grad_quant_bins = B;
        p.use_quantized_grad = 1;
        TrainBuffers tb = setup_state(ds, &p, run);
        mb::DevState &s = tb.s;
        // place the int8 pairs into every tile's records
        std::vector<uint8_t> rec((size_t)ds->n * ds->rec * ds->n_tiles);
        HIPX(hipMemcpy(rec.data(), ds->d_records, rec.size(), hipMemcpyDeviceToHost));
        for (int t = 0; t < ds->n_tiles; ++t)
            for (int64_t r = 0; r < ds->n; ++r) {
                const size_t at = ((size_t)t * ds->n + r) * ds->rec + ds->rec - 2;
                rec[at] = (uint8_t)q_grad[r];
                rec[at + 1] = (uint8_t)q_hess[r];
            }
        HIPX(hipMemcpy(ds->d_records, rec.data(), rec.size(), hipMemcpyHostToDevice));
        const size_t cells = (size_t)ds->F * ds->nb * 3;
        // unit lattice scales: the root split's gains are not read here, only
        // the histogram it merges into buffer 0
        mb::Round r0 = mb::initial_round();
        r0.grad_units = 1.0;
        r0.hess_units = 1.0;
        r0.sampled = rows ? 1 : 0;  // root range = rows0[0 .. cursor[0])
        HIPX(hipMemcpy(s.round, &r0, sizeof(r0), hipMemcpyHostToDevice));
        if (rows) {
            HIPX(hipMemcpy(s.rows0, rows, n_sel * sizeof(int32_t), hipMemcpyHostToDevice));
            int64_t c[2] = {n_sel, 0};
            HIPX(hipMemcpy(s.cursor, c, sizeof(c), hipMemcpyHostToDevice));
        }
        HIPX(mb::prepare_kernels(s));
        HIPX(mb::launch_hist(s, nullptr));
        HIPX(mb::launch_scan(s, 1, nullptr));
        HIPX(hipDeviceSynchronize());
        HIPX(hipMemcpy(out, s.hist, cells * sizeof(int32_t), hipMemcpyDeviceToHost));
    } catch (const Error &e) {
        set_err(err, err_len, e.msg);
        return e.code;
    }
    return MOJOTREES_OK;
}

int32_t mbh_histogram_fp32(mbh_dataset *ds, const float *grad, const float *hess, const int32_t *rows,
                           int64_t n_sel, double *out_gh, int64_t *out_count, char *err, int32_t err_len) {
    if (!ds || !grad || !hess || !out_gh || !out_count || (rows && n_sel <= 0)) {
        set_err(err, err_len, "invalid arguments");
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    try {
        if (rows)
            for (int64_t i = 0; i < n_sel; ++i)
                if (rows[i] < 0 || rows[i] >= ds->n)
                    throw Error{MOJOTREES_ERROR_INVALID_ARGUMENT, "row id out of range"};
        Run run;
        mbh_params p{};
        p.objective = MBH_OBJ_REGRESSION;
        p.num_iterations = 1;
        p.num_leaves = 2;
        p.learning_rate = 0.1;
        p.feature_fraction = 1.0;
        p.bagging_fraction = 1.0;
        p.num_grad_quant_bins = 4;
        p.use_quantized_grad = 0;
        TrainBuffers tb = setup_state(ds, &p, run);
        mb::DevState &s = tb.s;
        // the fp32 path reads the derivatives interleaved
        HIPX(hipMemcpy2D(s.gh2, 2 * sizeof(float), grad, sizeof(float), sizeof(float), ds->n, hipMemcpyHostToDevice));
        HIPX(hipMemcpy2D(s.gh2 + 1, 2 * sizeof(float), hess, sizeof(float), sizeof(float), ds->n,
                         hipMemcpyHostToDevice));
        mb::Round r0 = mb::initial_round();
        r0.sampled = rows ? 1 : 0;  // root range = rows0[0 .. cursor[0])
        HIPX(hipMemcpy(s.round, &r0, sizeof(r0), hipMemcpyHostToDevice));
        if (rows) {
            HIPX(hipMemcpy(s.rows0, rows, n_sel * sizeof(int32_t), hipMemcpyHostToDevice));
            int64_t c = n_sel;
            HIPX(hipMemcpy(s.cursor, &c, sizeof(c), hipMemcpyHostToDevice));
        }
        HIPX(mb::prepare_kernels(s));
        HIPX(mb::launch_hist(s, nullptr));
        HIPX(mb::launch_scan(s, 1, nullptr));
        HIPX(hipDeviceSynchronize());
        const size_t cells = (size_t)ds->F * ds->nb;
        std::vector<mb::HistF> h(cells);
        HIPX(hipMemcpy(h.data(), s.histf, cells * sizeof(mb::HistF), hipMemcpyDeviceToHost));
        for (size_t i = 0; i < cells; ++i) {
            out_gh[2 * i] = h[i].g;
            out_gh[2 * i + 1] = h[i].h;
            out_count[i] = h[i].c;
        }
    } catch (const Error &e) {
        set_err(err, err_len, e.msg);
        return e.code;
    }
    return MOJOTREES_OK;
}

int32_t mbh_bench_root_histogram(mbh_dataset *ds, int32_t reps, double *out_ms, char *err,
                                 int32_t err_len) {
    if (!ds || reps <= 0 || !out_ms) {
        set_err(err, err_len, "invalid arguments");
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    std::vector<hipEvent_t> ev((size_t)3 * reps);
    try {
        Run run;
        mbh_params p{};
        p.objective = MBH_OBJ_BINARY;
        p.num_iterations = 1;
        p.num_leaves = 2;
        p.learning_rate = 0.1;
        p.feature_fraction = 1.0;
        p.bagging_fraction = 1.0;
        p.num_grad_quant_bins = 4;
        p.use_quantized_grad = 1;
        TrainBuffers tb = setup_state(ds, &p, run);
        mb::DevState &s = tb.s;
        mb::Round r0 = mb::initial_round();
        r0.grad_units = 1.0;
        r0.hess_units = 1.0;
        HIPX(hipMemcpy(s.round, &r0, sizeof(r0), hipMemcpyHostToDevice));
        HIPX(mb::prepare_kernels(s));
        for (auto &e : ev) HIPX(hipEventCreate(&e));
        for (int i = 0; i < reps; ++i) {
            // the kernel's own start and end (no queue gap), then its merge
            HIPX(mb::launch_hist(s, nullptr, ev[3 * i], ev[3 * i + 1]));
            HIPX(mb::launch_scan(s, 1, nullptr));
            HIPX(mb::launch_plan(s, 1, nullptr));
            HIPX(hipEventRecord(ev[3 * i + 2], nullptr));
        }
        HIPX(hipDeviceSynchronize());
        double sum = 0.0, mn = 1e30, sum2 = 0.0;
        for (int i = 0; i < reps; ++i) {
            float ms = 0.f, ms2 = 0.f;
            HIPX(hipEventElapsedTime(&ms, ev[3 * i], ev[3 * i + 1]));
            HIPX(hipEventElapsedTime(&ms2, ev[3 * i], ev[3 * i + 2]));
            sum += ms;
            sum2 += ms2;
            mn = std::min(mn, (double)ms);
        }
        out_ms[0] = sum / reps;
        out_ms[1] = mn;
        out_ms[2] = sum2 / reps;
        for (auto &e : ev) (void)hipEventDestroy(e);
    } catch (const Error &e) {
        for (auto &x : ev)
            if (x) (void)hipEventDestroy(x);
        set_err(err, err_len, e.msg);
        return e.code;
    }
    return MOJOTREES_OK;
}

}  // extern "C"
