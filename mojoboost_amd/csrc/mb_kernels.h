// Launchers for the kernels in mb_kernels.hip.
#pragma once

#include <hip/hip_runtime.h>

#include "mb_state.h"

namespace mb {

hipError_t launch_objective(const DevState &s, int grid, hipStream_t st);
hipError_t launch_softmax(const DevState &s, int grid, hipStream_t st);
// The GOSS selection of the round (no-ops before the warmup ends).
hipError_t launch_goss(const DevState &s, int grid, hipStream_t st);
// max |g|, |h| of the round's weighted GOSS sample (quantized gradients,
// between launch_goss and launch_quantize).
hipError_t launch_goss_stats(const DevState &s, int grid, hipStream_t st);
// The magnitude-sum lattice's reduction and scales (before launch_quantize).
hipError_t launch_magnitude(const DevState &s, hipStream_t st);
// write_pairs = false leaves the max-abs int8 pairs to launch_hist(quantize).
hipError_t launch_quantize(const DevState &s, int grid, hipStream_t st, bool write_pairs = true);
// Raises the dynamic LDS limits of the kernels that need more than 64 KB.
hipError_t prepare_kernels(const DevState &s);
size_t hist_lds_bytes(const DevState &s);
// histogram accumulators: packed int8-lattice counters, fp64 sums of fp32
// gradients, int32 sums of the magnitude-sum lattice
enum AccKind { kAccQuant = 0, kAccFloat = 1, kAccWide = 2 };
inline int acc_kind(const HyperParams &hp) { return hp.wide ? kAccWide : hp.quantized ? kAccQuant : kAccFloat; }
// accumulation LDS of a tile of tile_f features
size_t pb_lds_bytes_for(int tile_f, int lds_stride, int kind);
size_t plan_lds_bytes(const DevState &s);
size_t score_lds_bytes(const DevState &s);
size_t rank_lds_bytes(const DevState &s);
// With both events given, the runtime records them at the kernel's own start
// and end (for timing without queue gaps).
// quantize: the root build quantizes the rows it reads and writes their
// pairs into the records (max-abs lattice only; other kinds ignore it).
hipError_t launch_hist(const DevState &s, hipStream_t st, hipEvent_t ev0 = nullptr, hipEvent_t ev1 = nullptr,
                       bool quantize = false);
hipError_t launch_partition(const DevState &s, hipStream_t st, hipEvent_t ev0 = nullptr, hipEvent_t ev1 = nullptr,
                            bool root = false);
hipError_t launch_accum(const DevState &s, hipStream_t st, hipEvent_t ev0 = nullptr, hipEvent_t ev1 = nullptr);
hipError_t launch_scan(const DevState &s, int root_mode, hipStream_t st);
hipError_t launch_plan(const DevState &s, int root_mode, hipStream_t st, Batch *host = nullptr);
hipError_t launch_score(const DevState &s, int grid, hipStream_t st);
// The score update fused with the next round's objective (single-output L2
// and binary): after it, the next tree skips launch_objective.
hipError_t launch_score_objective(const DevState &s, int grid, hipStream_t st);
hipError_t launch_round_end(const DevState &s, hipStream_t st);
hipError_t launch_round_end_quantize(const DevState &s, hipStream_t st);
hipError_t launch_round_combine(const RoundStates &rs, int sampling, hipStream_t st);
// Grid of a grid-stride rows kernel: as many blocks per CU as its registers
// and LDS let stay resident (at most 8), times n_cu, so that every block runs
// from the start instead of a partial second round of blocks following the
// first.
enum RowsKernel { kRowsScore = 0, kRowsScoreObjective = 1, kRowsSoftmax = 2 };
int rows_grid(const DevState &s, RowsKernel k, int n_cu);
hipError_t launch_build_records(const uint8_t *bins_cm, uint8_t *records, int64_t n, int F, int rec,
                                int tile_f, int n_tiles, int grid, hipStream_t st);
hipError_t launch_fill_f64(double *p, int64_t n, int K, const double *base, int grid, hipStream_t st);
hipError_t launch_exp_sigmoid(const double *x, double *e, double *sg, int64_t n, hipStream_t st);

// Batch prediction over row records (the training layout), one thread per
// (row, class): trees t0 + k, t0 + k + K, ... < t1 of a flat ensemble whose
// nodes hold absolute child indices.
struct PredictArgs {
    const uint8_t *records;
    int64_t n;
    int32_t rec_bytes, tile_f, n_tiles, num_class;
    const int4 *nodes;        // {feature (-1: leaf), threshold bin, left, right}
    const int32_t *md;        // missing_bin * 2 + default_left
    const unsigned long long *cat;  // 4 words per node, the left set of a categorical node (threshold -1)
    const double *value;      // per node
    const int32_t *root;      // per tree: index of its root node
    int32_t max_steps;        // nodes of the largest tree: no walk is longer
    int64_t t0, t1;           // trees [t0, t1); t0 a multiple of num_class
    double learning_rate;
    const double *base;       // num_class base scores, or null (a range after iteration 0)
    double *out;              // n x num_class
};
hipError_t launch_predict(const PredictArgs &a, int grid, hipStream_t st);

}  // namespace mb
