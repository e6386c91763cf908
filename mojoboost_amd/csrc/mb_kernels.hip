// gfx950 kernels of the GBDT training step (one boosting round = one tree per
// class):
//
//   k_objective   fused gradient/hessian of the round + max |g|, |h| of the
//                 sampled rows (one pass over raw scores and labels)
//   k_quantize    max-abs lattice + stochastic rounding to int8 g/h, written
//                 into each row's record; root row list and root histogram
//                 reset
//   k_hist        per-leaf histogram: LDS-privatized packed 64-bit counters
//                 (grad | hess | count in one ds_add_u64), merged into the
//                 global int32 histogram with integer atomics
//   k_partition   row partition of the chosen leaf's range: wave ballot +
//                 popcount ranks, one atomic cursor reservation per block
//   k_split       sibling subtraction + per-feature integer prefix scan with
//                 fp64 gains + argmax; the last block folds features, writes
//                 the tree nodes and frontier slots, and picks the next leaf
//   k_score       raw += lr * tree(row) by tree walk, fused multiply-add
//   k_round_end   archives the finished tree and advances the round state
//
// Reference behaviour these restate: boosting._fill_grad_hess_into and
// quantized_gradient.quantize_round_cpu (objective + quantizer), the range
// histogram kernels of gpu_active_rows.mojo:3903-4300, the partition of
// gpu_active_rows.mojo:1054-1707, split.find_best_split with
// quantized_split_gain, tree.grow_tree_leaves_profiled and
// growth_policy.GrowthSchedule.next_leaf (leaf choice), and
// boosting._add_by_leaf (score update).
#include <hip/hip_runtime.h>

#include "mb_kernels.h"
#include "mb_math.h"
#include "mb_state.h"

namespace mb {

namespace {

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

template <class T>
__device__ __forceinline__ T load_agent(const T *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ double load_agent_f64(const double *p) {
    unsigned long long v =
        __hip_atomic_load((const unsigned long long *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return __longlong_as_double((long long)v);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v = fmaxf(v, __shfl_xor(v, d, 64));
    return v;
}

__device__ __forceinline__ long long wave_sum_ll(long long v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
    return v;
}

// Inclusive prefix sum across the 64 lanes of a wave.
__device__ __forceinline__ long long wave_incl_scan(long long v) {
    const int lane = lane_id();
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        long long t = __shfl_up(v, d, 64);
        if (lane >= d) v += t;
    }
    return v;
}

// (gain, order) argmax across the wave: larger gain wins, equal gains go to
// the smaller order, so the result is the first maximum in scan order.
__device__ __forceinline__ void wave_argmax(double &gain, int &order) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        double og = __shfl_xor(gain, d, 64);
        int oo = __shfl_xor(order, d, 64);
        if (og > gain || (og == gain && oo < order)) {
            gain = og;
            order = oo;
        }
    }
}

__device__ __forceinline__ bool in_bag(const HyperParams &hp, uint64_t bag_stream, int64_t r) {
    return uniform53(bag_stream + (uint64_t)r) < hp.bagging_fraction;
}

// bagging.sample_rows stream of one bag (src/mojotrees/bagging.mojo).
__device__ __forceinline__ uint64_t bag_stream_of(const HyperParams &hp, int64_t round) {
    int64_t bag_index = hp.bagging_freq > 0 ? round / hp.bagging_freq : 0;
    return splitmix64((uint64_t)(hp.bagging_seed & 0x7FFFFFFFFFFFFFFFLL) ^
                      ((uint64_t)bag_index * kGolden));
}

}  // namespace

// --------------------------------------------------------------- objective
// boosting._fill_grad_hess_into (src/mojotrees/boosting.mojo:676-811):
// derivatives computed in binary64 and narrowed to binary32 (score_t), then
// gradient_stats' max |g|, max |h| over the round's rows
// (quantized_gradient.mojo:762-810) as binary32 bit patterns, which order
// like unsigned integers for non-negative values.
__global__ __launch_bounds__(256) void k_objective(DevState s) {
    __shared__ float red_g[4], red_h[4];
    const Round rd = *s.round;
    const HyperParams &hp = s.hp;
    if (blockIdx.x == 0 && threadIdx.x == 0) s.cursor[0] = 0;  // root row count
    const uint64_t bstream = hp.bagging ? bag_stream_of(hp, rd.round) : 0;
    float mg = 0.0f, mh = 0.0f;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < s.n; r += stride) {
        float g, h;
        if (hp.objective == kObjBinary) {
            double p = sigmoid(s.raw[r]);
            g = (float)(p - s.labels[r]);
            double hh = p * (1.0 - p);
            if (hh < 1e-16) hh = 1e-16;
            h = (float)hh;
        } else {
            g = (float)(s.raw[r] - s.labels[r]);
            h = 1.0f;
        }
        s.grad[r] = g;
        s.hess[r] = h;
        float ag = fabsf(g), ah = fabsf(h);
        bool sel = !hp.bagging || in_bag(hp, bstream, r);
        if (sel && isfinite(ag) && isfinite(ah)) {
            mg = fmaxf(mg, ag);
            mh = fmaxf(mh, ah);
        }
    }
    mg = wave_max(mg);
    mh = wave_max(mh);
    const int w = threadIdx.x >> 6;
    if (lane_id() == 0) {
        red_g[w] = mg;
        red_h[w] = mh;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < (int)(blockDim.x >> 6); ++i) {
            mg = fmaxf(mg, red_g[i]);
            mh = fmaxf(mh, red_h[i]);
        }
        atomicMax(&s.stats[rd.parity * 2 + 0], __float_as_uint(mg));
        atomicMax(&s.stats[rd.parity * 2 + 1], __float_as_uint(mh));
    }
}

// ---------------------------------------------------------------- quantize
// derive_scales (max-abs rule, quantized_gradient.mojo:1343-1453) and
// quantize_scalar per row (:1479-1545). Every row is quantized, sampled or
// not, with the row id as the stream counter. The int8 pair lands in the
// last two bytes of the row's record, next to its bins. The root row list
// (the bag) is gathered here; without bagging the root reads rows directly.
__global__ __launch_bounds__(256) void k_quantize(DevState s) {
    const Round rd = *s.round;
    const HyperParams &hp = s.hp;
    double max_g = (double)__uint_as_float(s.stats[rd.parity * 2 + 0]);
    double max_h = (double)__uint_as_float(s.stats[rd.parity * 2 + 1]);
    if (max_g < 1e-12) max_g = 1e-12;
    if (max_h < 1e-12) max_h = 1e-12;
    const int32_t gmax = hp.quant_bins / 2;
    const int32_t hmax = hp.const_hessian ? 1 : hp.quant_bins;
    const double gu = (double)gmax / max_g;
    const double hu = hp.const_hessian ? 1.0 / max_h : (double)hmax / max_h;
    const uint64_t gs = quant_stream(hp.quant_seed, rd.round, rd.class_k, 0);
    const uint64_t hs = quant_stream(hp.quant_seed, rd.round, rd.class_k, 1);
    const bool stoch = hp.stochastic != 0;
    const uint64_t bstream = hp.bagging ? bag_stream_of(hp, rd.round) : 0;
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        s.round->grad_units = gu;
        s.round->hess_units = hu;
        s.stats[(1 - rd.parity) * 2 + 0] = 0u;
        s.stats[(1 - rd.parity) * 2 + 1] = 0u;
    }
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int rec = s.rec_bytes;
    for (int64_t r0 = (int64_t)blockIdx.x * blockDim.x; r0 < s.n; r0 += stride) {
        const int64_t r = r0 + threadIdx.x;
        const bool valid = r < s.n;
        if (valid) {
            int32_t qg = quantize_scalar((double)s.grad[r], gu, gmax, stoch, gs + (uint64_t)r);
            int32_t qh = quantize_scalar((double)s.hess[r], hu, hmax, stoch, hs + (uint64_t)r);
            uint16_t v = (uint16_t)(uint8_t)(int8_t)qg | (uint16_t)((uint16_t)(uint8_t)(int8_t)qh << 8);
            *(uint16_t *)(s.records_w + r * rec + rec - 2) = v;
        }
        if (!hp.bagging) {
            if (valid) s.rows0[r] = (int32_t)r;
        } else {
            // Sampled rows appended with one atomic per wave; their order in
            // the root range does not matter (integer histograms).
            bool take = valid && in_bag(hp, bstream, r);
            unsigned long long m = __ballot(take);
            int cnt = __popcll(m);
            long long base = 0;
            if (lane_id() == 0 && cnt) base = atomicAdd((unsigned long long *)&s.cursor[0], (unsigned long long)cnt);
            base = __shfl(base, 0, 64);
            if (take) {
                int rank = __popcll(m & ((1ULL << lane_id()) - 1ULL));
                s.rows0[base + rank] = (int32_t)r;
            }
        }
    }
}

// --------------------------------------------------------------- histogram
// Rows of a node with m rows handled by each histogram block. The split
// kernel recomputes it to know how many block partials a build left.
__device__ __forceinline__ int64_t hist_chunk(const DevState &s, int64_t m) {
    const int64_t g = s.hist_grid;
    int64_t chunk = (m + g - 1) / g;
    if (chunk < s.hist_chunk_min) chunk = s.hist_chunk_min;
    if (chunk > s.hist_chunk_limit) chunk = s.hist_chunk_limit;
    return chunk;
}

// One leaf's histogram, accumulation pass. Rows are split into contiguous
// chunks, one per block; a block accumulates its rows into LDS-private
// packed counters and stores them, all cells, as its partial. The split
// kernel merges the partials. A row's record is LPR x 16 bytes: each of the
// LPR lanes of a row group loads 16 bytes (16 features) and the int8 g/h pair
// (the record's last two bytes) reaches the group by a lane shuffle. Each
// lane keeps kHistUnroll row loads in flight.
//
// Packed counter (64 bits): count in bits [0,20), hess sum in [20,42), grad
// sum (signed) in [42,64). Adding packed values adds the three fields while
// no field overflows, which hist_chunk_limit guarantees for the lattice in
// use (host-checked).
constexpr int kHistUnroll = 4;

template <int LPR>
__global__ __launch_bounds__(1024) void k_hist(DevState s, int root_mode) {
    extern __shared__ unsigned long long lds[];
    int64_t m;
    const int32_t *rows;
    bool direct;
    if (root_mode) {
        m = s.hp.bagging ? s.cursor[0] : s.n;
        rows = s.rows0;
        direct = !s.hp.bagging;
    } else {
        const Step st = *s.step;
        if (!st.active) return;
        int64_t beg;
        if (st.builds_left) {
            beg = st.begin;
            m = st.n_left;
        } else {
            beg = st.begin + st.n_left;
            m = st.end - beg;
        }
        rows = (st.src_buf ? s.rows0 : s.rows1) + beg;
        direct = false;
    }
    if (m <= 0) return;
    const int64_t chunk = hist_chunk(s, m);
    const int64_t c0 = (int64_t)blockIdx.x * chunk;
    if (c0 >= m) return;
    const int64_t c1 = c0 + chunk < m ? c0 + chunk : m;
    const int F = s.n_features, nb = s.n_bins, ls = s.lds_stride;
    for (int i = threadIdx.x; i < F * ls; i += blockDim.x) lds[i] = 0ULL;
    __syncthreads();
    const int lane = lane_id();
    const int sub = threadIdx.x % LPR;
    const int rr = threadIdx.x / LPR;
    const int rpp = blockDim.x / LPR;
    const int src_lane = (lane / LPR) * LPR + (LPR - 1);
    const uint4 *rec = (const uint4 *)s.records;
    for (int64_t i0 = c0; i0 < c1; i0 += (int64_t)kHistUnroll * rpp) {
        uint4 w[kHistUnroll];
        bool ok[kHistUnroll];
#pragma unroll
        for (int u = 0; u < kHistUnroll; ++u) {
            const int64_t i = i0 + (int64_t)u * rpp + rr;
            ok[u] = i < c1;
            int64_t row = 0;
            if (ok[u]) {
                row = direct ? i : (int64_t)rows[i];
                if ((uint64_t)row >= (uint64_t)s.n) row = 0;  // never taken: ids come from the row lists
            }
            w[u] = ok[u] ? rec[row * LPR + sub] : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < kHistUnroll; ++u) {
            const uint32_t gh = __shfl(w[u].w, src_lane, 64);
            if (!ok[u]) continue;
            const int g = (int)(int8_t)(gh >> 16);
            const int h = (int)(int8_t)(gh >> 24);
            const unsigned long long packed =
                (unsigned long long)(((long long)g << 42) + ((long long)h << 20) + 1LL);
            const uint32_t d[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int f = sub * 16 + q * 4 + j;
                    if (f < F) atomicAdd(&lds[f * ls + ((d[q] >> (8 * j)) & 255u)], packed);
                }
        }
    }
    __syncthreads();
    const int ps = s.part_stride;
    unsigned long long *out = s.part + (size_t)blockIdx.x * F * ps;
    for (int c = threadIdx.x; c < F * ps; c += blockDim.x) {
        const int f = c / ps;
        const int b = c - f * ps;
        out[c] = b < nb ? lds[f * ls + b] : 0ULL;
    }
}

// --------------------------------------------------------------- partition
// Routes the parent's rows (tree.partition_rows_into semantics: the missing
// bin follows default_left, otherwise bin <= threshold goes left) into the
// other row buffer: left rows fill [begin, begin + n_left), right rows the
// rest. Each block counts its chunk, reserves its output with one atomic per
// side, and scatters tile by tile with ballot ranks; each thread keeps
// kPartUnroll rows in flight. The order inside a child is not the
// reference's (blocks land in reservation order); every consumer is
// order-free because histograms are integer sums.
constexpr int kPartUnroll = 8;

__global__ __launch_bounds__(256) void k_partition(DevState s) {
    __shared__ int wave_l[kPartUnroll][4], wave_r[kPartUnroll][4];
    __shared__ int red[4];
    __shared__ long long base_l, base_r;
    const Step st = *s.step;
    if (!st.active) return;
    const int64_t m = st.end - st.begin;
    int64_t chunk = (m + gridDim.x - 1) / gridDim.x;
    if (chunk < 2048) chunk = 2048;
    chunk = (chunk + 255) / 256 * 256;
    const int64_t c0 = (int64_t)blockIdx.x * chunk;
    if (c0 >= m) return;
    const int64_t c1 = c0 + chunk < m ? c0 + chunk : m;
    const int32_t *src = (st.src_buf ? s.rows1 : s.rows0) + st.begin;
    int32_t *dst = (st.src_buf ? s.rows0 : s.rows1) + st.begin;
    const uint8_t *col = s.bins_cm + (size_t)st.feature * s.n;
    const int mb = st.missing_bin, thr = st.bin, dl = st.default_left;
    const int lane = lane_id(), w = threadIdx.x >> 6;
    const int64_t tile = (int64_t)blockDim.x * kPartUnroll;
    // pass 1: count rows going left
    int my_l = 0;
    for (int64_t t0 = c0; t0 < c1; t0 += tile) {
        int32_t r[kPartUnroll];
#pragma unroll
        for (int u = 0; u < kPartUnroll; ++u) {
            const int64_t i = t0 + (int64_t)u * blockDim.x + threadIdx.x;
            r[u] = i < c1 ? src[i] : -1;
        }
#pragma unroll
        for (int u = 0; u < kPartUnroll; ++u) {
            if (r[u] < 0) continue;
            const int32_t row = (uint64_t)r[u] < (uint64_t)s.n ? r[u] : 0;
            const int b = col[row];
            my_l += (b == mb) ? dl : (b <= thr);
        }
    }
    const long long tl = wave_sum_ll(my_l);
    if (lane == 0) red[w] = (int)tl;
    __syncthreads();
    if (threadIdx.x == 0) {
        long long nl = 0;
        for (int i = 0; i < (int)(blockDim.x >> 6); ++i) nl += red[i];
        const long long nr = (c1 - c0) - nl;
        base_l = nl ? (long long)atomicAdd((unsigned long long *)&s.cursor[0], (unsigned long long)nl) : 0;
        base_r = nr ? (long long)atomicAdd((unsigned long long *)&s.cursor[1], (unsigned long long)nr) : 0;
    }
    __syncthreads();
    long long run_l = base_l, run_r = base_r;
    const int64_t n_left = st.n_left;
    const unsigned long long below = (1ULL << lane) - 1ULL;
    // pass 2: scatter; a tile is kPartUnroll sub-tiles of blockDim rows
    for (int64_t t0 = c0; t0 < c1; t0 += tile) {
        int32_t r[kPartUnroll];
        bool left[kPartUnroll], right[kPartUnroll];
        unsigned long long lm[kPartUnroll], rm[kPartUnroll];
#pragma unroll
        for (int u = 0; u < kPartUnroll; ++u) {
            const int64_t i = t0 + (int64_t)u * blockDim.x + threadIdx.x;
            r[u] = i < c1 ? src[i] : -1;
        }
#pragma unroll
        for (int u = 0; u < kPartUnroll; ++u) {
            left[u] = right[u] = false;
            if (r[u] >= 0) {
                const int32_t row = (uint64_t)r[u] < (uint64_t)s.n ? r[u] : 0;
                const int b = col[row];
                left[u] = (b == mb) ? (dl != 0) : (b <= thr);
                right[u] = !left[u];
            }
            lm[u] = __ballot(left[u]);
            rm[u] = __ballot(right[u]);
            if (lane == 0) {
                wave_l[u][w] = __popcll(lm[u]);
                wave_r[u][w] = __popcll(rm[u]);
            }
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < kPartUnroll; ++u) {
            long long off_l = 0, off_r = 0, tot_l = 0, tot_r = 0;
            for (int k = 0; k < (int)(blockDim.x >> 6); ++k) {
                if (k < w) {
                    off_l += wave_l[u][k];
                    off_r += wave_r[u][k];
                }
                tot_l += wave_l[u][k];
                tot_r += wave_r[u][k];
            }
            if (left[u]) {
                const long long p = run_l + off_l + __popcll(lm[u] & below);
                if (p < n_left) dst[p] = r[u];
                else atomicOr(s.error, 1);
            } else if (right[u]) {
                const long long p = n_left + run_r + off_r + __popcll(rm[u] & below);
                if (p < m) dst[p] = r[u];
                else atomicOr(s.error, 1);
            }
            run_l += tot_l;
            run_r += tot_r;
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------------- split
// One block (8 waves) per feature. First the built child's histogram is
// merged from the block partials of its build and stored; the sibling is
// parent - built, written back over the parent's buffer. Then waves 0-3 scan
// the built child and waves 4-7 the sibling, one bin per thread. The scan
// follows split.find_best_split (src/mojotrees/split.mojo:601-1360) with the
// sums kept as integers and each candidate scored by quantized_split_gain
// (quantized_gradient.mojo:3283-3310): ascending bins, missing-left scored
// before missing-right, strict '>' keeps the first maximum; the hessian guard
// compares against hessian_units_at_least (:3336).
//
// The last block to finish folds the features of each child (strict '>',
// lowest feature on ties), computes the children's leaf values
// (quantized_leaf_output), records the nodes, replaces the parent's frontier
// slot with the left child and appends the right one, then picks the next
// leaf (max gain, lowest slot on ties; growth_policy.mojo:659-677) and writes
// the next step with the left count read from that leaf's histogram.
constexpr int kSplitThreads = 512;
constexpr int kMaxScan = 256;  // 2 x max features

__global__ __launch_bounds__(kSplitThreads) void k_split(DevState s, int root_mode) {
    __shared__ long long cgs[2][256], chs[2][256], ccs[2][256];
    __shared__ long long wtot[8][3];
    __shared__ double wgain[8];
    __shared__ int word_[8];
    __shared__ unsigned int s_ticket;
    __shared__ ScanResult sres[kMaxScan];
    __shared__ long long part_acc[3][256];
    const int tid = threadIdx.x, lane = lane_id(), wv = tid >> 6;
    const HyperParams &hp = s.hp;
    const int F = s.n_features, nb = s.n_bins;
    const size_t hsz = (size_t)F * nb * 3;
    Step st;
    if (!root_mode) {
        st = *s.step;
        if (!st.active) return;
    }
    const Round rd = *s.round;
    const double gu = rd.grad_units, hu = rd.hess_units;
    const int f = blockIdx.x;
    int64_t m_built, m_sib = 0;
    int built_buf, depth_child;
    if (root_mode) {
        m_built = hp.bagging ? s.cursor[0] : s.n;
        built_buf = 0;
        depth_child = 0;
    } else {
        const int64_t m = st.end - st.begin;
        m_built = st.builds_left ? st.n_left : m - st.n_left;
        m_sib = m - m_built;
        built_buf = st.child_hist;
        depth_child = st.depth + 1;
    }
    // ---- merge the built child's partials: thread -> (bin, half of the parts)
    const int64_t chunk = hist_chunk(s, m_built);
    const int64_t nparts = m_built > 0 ? (m_built + chunk - 1) / chunk : 0;
    {
        const int bin = tid & 255, half = tid >> 8;
        long long g = 0, h = 0, c = 0;
        if (bin < nb) {
            const size_t pstride = (size_t)F * s.part_stride;
            const unsigned long long *p = s.part + (size_t)f * s.part_stride + bin;
            int64_t b = half;
            for (; b + 14 < nparts; b += 16) {
                unsigned long long v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) v[u] = p[(size_t)(b + 2 * u) * pstride];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    c += (long long)(v[u] & 0xFFFFFULL);
                    h += (long long)((v[u] >> 20) & 0x3FFFFFULL);
                    g += (long long)v[u] >> 42;
                }
            }
            for (; b < nparts; b += 2) {
                const unsigned long long v = p[(size_t)b * pstride];
                c += (long long)(v & 0xFFFFFULL);
                h += (long long)((v >> 20) & 0x3FFFFFULL);
                g += (long long)v >> 42;
            }
        }
        if (half == 1) {
            part_acc[0][bin] = g;
            part_acc[1][bin] = h;
            part_acc[2][bin] = c;
        }
        __syncthreads();
        if (half == 0) {
            g += part_acc[0][bin];
            h += part_acc[1][bin];
            c += part_acc[2][bin];
            cgs[0][bin] = g;
            chs[0][bin] = h;
            ccs[0][bin] = c;
            long long sgv = 0, shv = 0, scv = 0;
            if (bin < nb) {
                int32_t *ob = s.hist + (size_t)built_buf * hsz + ((size_t)f * nb + bin) * 3;
                ob[0] = (int32_t)g;
                ob[1] = (int32_t)h;
                ob[2] = (int32_t)c;
                if (!root_mode) {
                    int32_t *pp = s.hist + (size_t)st.parent_hist * hsz + ((size_t)f * nb + bin) * 3;
                    sgv = (long long)pp[0] - g;
                    shv = (long long)pp[1] - h;
                    scv = (long long)pp[2] - c;
                    pp[0] = (int32_t)sgv;
                    pp[1] = (int32_t)shv;
                    pp[2] = (int32_t)scv;
                }
            }
            cgs[1][bin] = sgv;
            chs[1][bin] = shv;
            ccs[1][bin] = scv;
        }
        __syncthreads();
    }
    // ---- scan: waves 0-3 the built child, waves 4-7 the sibling; one bin each
    const int child = tid >> 8;
    const int bin = tid & 255;
    const int cw = wv & 3;  // wave within the child
    const long long vg = cgs[child][bin], vh = chs[child][bin], vc = ccs[child][bin];
    const long long ig = wave_incl_scan(vg), ih = wave_incl_scan(vh), ic = wave_incl_scan(vc);
    if (lane == 63) {
        wtot[wv][0] = ig;
        wtot[wv][1] = ih;
        wtot[wv][2] = ic;
    }
    __syncthreads();
    long long pg = 0, ph = 0, pc = 0, TG = 0, TH = 0, TC = 0;
    for (int k = 0; k < 4; ++k) {
        const int ww = (child << 2) + k;
        if (k < cw) {
            pg += wtot[ww][0];
            ph += wtot[ww][1];
            pc += wtot[ww][2];
        }
        TG += wtot[ww][0];
        TH += wtot[ww][1];
        TC += wtot[ww][2];
    }
    const long long lg = pg + ig, lh = ph + ih, lc = pc + ic;  // inclusive prefix at `bin`
    const int64_t n_child = child == 0 ? m_built : m_sib;
    const int mb = s.missing_bin[f];
    const bool gated = (root_mode && child == 1) || (hp.max_depth > 0 && depth_child >= hp.max_depth) ||
                       n_child < 2 * (int64_t)hp.min_data_in_leaf || n_child < 2 ||
                       !s.feature_mask[(size_t)rd.tree_index * F + f];
    double best_gain = 0.0;
    int best_order = 0x7FFFFFFF;
    if (!gated) {
        const long long mg = mb >= 0 ? cgs[child][mb] : 0, mh = mb >= 0 ? chs[child][mb] : 0,
                        mc = mb >= 0 ? ccs[child][mb] : 0;
        const double l1 = hp.lambda_l1, l2 = hp.lambda_l2;
        long long hmin = 0;  // hessian_units_at_least: min_sum_hessian in lattice units, rounded up
        if (hp.min_sum_hessian > 0.0) {
            const double u = hp.min_sum_hessian * hu;
            double fl = floor(u);
            if (fl < u) fl += 1.0;
            hmin = (long long)fl;
        }
        const long long min_c = hp.min_data_in_leaf;
        const int n_scan = mb >= 0 ? mb : nb;
        int lim = n_scan < s.widths[f] ? n_scan : s.widths[f];
        if (mc == 0 && lim > n_scan - 1) lim = n_scan - 1;
        if (bin < lim) {
            const double parent = qscore(TG, TH, gu, hu, l1, l2);
            if (mb >= 0) {
                const long long ag = lg + mg, ah = lh + mh, ac = lc + mc;
                const long long rg = TG - ag, rh = TH - ah, rc = TC - ac;
                if (!(ah < hmin || rh < hmin || ac < min_c || rc < min_c)) {
                    const double gain = qscore(ag, ah, gu, hu, l1, l2) + qscore(rg, rh, gu, hu, l1, l2) - parent;
                    if (gain > best_gain) {
                        best_gain = gain;
                        best_order = 2 * bin;
                    }
                }
            }
            if (mb < 0 || mc > 0) {
                const long long rg = TG - lg, rh = TH - lh, rc = TC - lc;
                if (!(lh < hmin || rh < hmin || lc < min_c || rc < min_c)) {
                    const double gain = qscore(lg, lh, gu, hu, l1, l2) + qscore(rg, rh, gu, hu, l1, l2) - parent;
                    if (gain > best_gain) {
                        best_gain = gain;
                        best_order = 2 * bin + 1;
                    }
                }
            }
        }
    }
    wave_argmax(best_gain, best_order);
    if (lane == 0) {
        wgain[wv] = best_gain;
        word_[wv] = best_order;
    }
    __syncthreads();
    if (tid == 0 || tid == 256) {
        double bg = wgain[child << 2];
        int bo = word_[child << 2];
        for (int k = 1; k < 4; ++k) {
            const double og = wgain[(child << 2) + k];
            const int oo = word_[(child << 2) + k];
            if (og > bg || (og == bg && oo < bo)) {
                bg = og;
                bo = oo;
            }
        }
        if (!(root_mode && child == 1)) {
            ScanResult r;
            r.gain = bg;
            r.found = bo != 0x7FFFFFFF;
            r.bin = r.found ? bo >> 1 : -1;
            r.default_left = r.found ? ((bo & 1) == 0) : 0;
            r.pad_ = 0;
            r.tot_g = TG;
            r.tot_h = TH;
            r.tot_c = TC;
            s.scan[child * F + f] = r;
        }
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) s_ticket = atomicAdd(s.ticket, 1u);
    __syncthreads();
    if (s_ticket != (unsigned int)(F - 1)) return;
    __threadfence();

    // ------------------------------------------------ last block: fold + pick
    const int nchild = root_mode ? 1 : 2;
    for (int i = tid; i < nchild * F; i += blockDim.x) {
        const ScanResult *p = &s.scan[i];
        ScanResult r;
        r.found = load_agent(&p->found);
        r.gain = load_agent_f64(&p->gain);
        r.bin = load_agent(&p->bin);
        r.default_left = load_agent(&p->default_left);
        r.pad_ = 0;
        r.tot_g = load_agent(&p->tot_g);
        r.tot_h = load_agent(&p->tot_h);
        r.tot_c = load_agent(&p->tot_c);
        sres[i] = r;
    }
    __syncthreads();
    if (wv < nchild) {
        double bg = 0.0;
        int bf = 0x7FFFFFFF;
        for (int ff = lane; ff < F; ff += 64) {
            const ScanResult &r = sres[wv * F + ff];
            if (r.found && r.gain > bg) {
                bg = r.gain;
                bf = ff;
            }
        }
        wave_argmax(bg, bf);
        if (lane == 0) {
            wgain[wv] = bg;
            word_[wv] = bf;
        }
    }
    __syncthreads();
    if (tid == 0) {
        int32_t *meta = s.t_meta;
        const double l1 = hp.lambda_l1, l2 = hp.lambda_l2;
        auto fill_slot = [&](Slot &sl, int ch) {
            const int bf = word_[ch];
            sl.found = bf != 0x7FFFFFFF;
            if (sl.found) {
                const ScanResult &r = sres[ch * F + bf];
                sl.feature = bf;
                sl.bin = r.bin;
                sl.default_left = r.default_left;
                sl.gain = wgain[ch];
            } else {
                sl.feature = -1;
                sl.bin = -1;
                sl.default_left = 0;
                sl.gain = 0.0;
            }
        };
        auto new_node = [&](int id, double v, double cnt) {
            s.t_feature[id] = -1;
            s.t_threshold[id] = -1;
            s.t_left[id] = -1;
            s.t_right[id] = -1;
            s.t_default_left[id] = 0;
            s.t_missing_bin[id] = -1;
            s.t_value[id] = v;
            s.t_gain[id] = 0.0;
            s.t_count[id] = cnt;
        };
        if (root_mode) {
            const ScanResult &r = sres[0];
            new_node(0, qleaf(r.tot_g, r.tot_h, gu, hu, l1, l2), (double)r.tot_c);
            meta[0] = 1;
            meta[1] = 1;
            Slot sl;
            sl.begin = 0;
            sl.end = r.tot_c;
            sl.node = 0;
            sl.buf = 0;
            sl.hist = 0;
            sl.depth = 0;
            fill_slot(sl, 0);
            s.slots[0] = sl;
            s.arc_rows[(size_t)rd.tree_index * hp.num_leaves + 0] = r.tot_c;
        } else {
            const ScanResult &b = sres[0];
            const ScanResult &sb = sres[F];
            const bool bl = st.builds_left != 0;
            const ScanResult &Lr = bl ? b : sb;
            const ScanResult &Rr = bl ? sb : b;
            new_node(st.node_left, qleaf(Lr.tot_g, Lr.tot_h, gu, hu, l1, l2), (double)Lr.tot_c);
            new_node(st.node_right, qleaf(Rr.tot_g, Rr.tot_h, gu, hu, l1, l2), (double)Rr.tot_c);
            const int pn = st.parent_node;
            s.t_feature[pn] = st.feature;
            s.t_threshold[pn] = st.bin;
            s.t_left[pn] = st.node_left;
            s.t_right[pn] = st.node_right;
            s.t_default_left[pn] = st.default_left;
            s.t_missing_bin[pn] = st.missing_bin;
            s.t_gain[pn] = st.gain;
            Slot L, R;
            L.begin = st.begin;
            L.end = st.begin + st.n_left;
            R.begin = L.end;
            R.end = st.end;
            L.node = st.node_left;
            R.node = st.node_right;
            L.buf = R.buf = 1 - st.src_buf;
            L.hist = bl ? st.child_hist : st.parent_hist;
            R.hist = bl ? st.parent_hist : st.child_hist;
            L.depth = R.depth = st.depth + 1;
            fill_slot(L, bl ? 0 : 1);
            fill_slot(R, bl ? 1 : 0);
            s.slots[st.parent_slot] = L;
            s.slots[st.new_slot] = R;
            meta[0] += 2;
            meta[1] += 1;
        }
    }
    __syncthreads();
    // pick the next leaf (wave 0)
    __shared__ int s_pick;
    __shared__ Slot s_slot;
    if (wv == 0) {
        const int n_leaves = s.t_meta[1];
        double bg = 0.0;
        int bi = 0x7FFFFFFF;
        if (n_leaves < hp.num_leaves) {
            for (int i = lane; i < n_leaves; i += 64) {
                const Slot &sl = s.slots[i];
                if (sl.found && sl.gain > 0.0 && sl.gain > bg) {
                    bg = sl.gain;
                    bi = i;
                }
            }
        }
        wave_argmax(bg, bi);
        if (lane == 0) {
            s_pick = bi;
            if (bi != 0x7FFFFFFF) s_slot = s.slots[bi];
        }
    }
    __syncthreads();
    const int bi = s_pick;
    if (bi == 0x7FFFFFFF) {
        if (tid == 0) {
            s.step->active = 0;
            *s.ticket = 0u;
        }
        return;
    }
    const Slot sl = s_slot;
    const int32_t *pick_h = s.hist + (size_t)sl.hist * hsz + (size_t)sl.feature * nb * 3;
    const int fmb = s.missing_bin[sl.feature];
    long long nl = 0;
    if (tid < nb) {
        const bool goes_left = (tid == fmb) ? (sl.default_left != 0) : (tid <= sl.bin);
        if (goes_left) nl = load_agent(&pick_h[3 * tid + 2]);
    }
    nl = wave_sum_ll(nl);
    if (lane == 0) wtot[wv][0] = nl;
    __syncthreads();
    if (tid == 0) {
        long long tot = 0;
        for (int k = 0; k < 8; ++k) tot += wtot[k][0];
        const int n_leaves = s.t_meta[1];
        const int n_nodes = s.t_meta[0];
        Step ns;
        ns.active = 1;
        ns.parent_slot = bi;
        ns.new_slot = n_leaves;
        ns.feature = sl.feature;
        ns.bin = sl.bin;
        ns.default_left = sl.default_left;
        ns.missing_bin = fmb;
        ns.src_buf = sl.buf;
        ns.begin = sl.begin;
        ns.end = sl.end;
        ns.n_left = tot;
        ns.builds_left = tot <= (sl.end - sl.begin) - tot;
        ns.parent_hist = sl.hist;
        ns.child_hist = n_leaves;
        ns.depth = sl.depth;
        ns.parent_node = sl.node;
        ns.node_left = n_nodes;
        ns.node_right = n_nodes + 1;
        ns.pad_ = 0;
        ns.gain = sl.gain;
        *s.step = ns;
        s.cursor[0] = 0;
        s.cursor[1] = 0;
        s.arc_rows[(size_t)rd.tree_index * hp.num_leaves + n_leaves] =
            ns.builds_left ? tot : (sl.end - sl.begin) - tot;
        *s.ticket = 0u;
    }
}

// ------------------------------------------------------------- score update
// raw[r] += lr * value(leaf of r), fused (boosting._add_by_leaf,
// src/mojotrees/boosting.mojo:1991-2112), by walking the tree for every row
// over the row's record (its bins are contiguous), so sampled-out rows are
// covered too (the traversal route, :1947). A single-leaf tree whose value is
// below 1e-12 is the reference's stopping condition (:2898-2907) and adds
// nothing.
__global__ __launch_bounds__(256) void k_score(DevState s) {
    extern __shared__ int32_t tnode[];  // 5 ints per node
    const int n_nodes = s.t_meta[0];
    const int n_leaves = s.t_meta[1];
    if (n_leaves == 1 && fabs(s.t_value[0]) < 1e-12) return;
    double *vals = (double *)(tnode + 5 * s.max_nodes + (s.max_nodes & 1));
    for (int i = threadIdx.x; i < n_nodes; i += blockDim.x) {
        tnode[5 * i + 0] = s.t_feature[i];
        tnode[5 * i + 1] = s.t_threshold[i];
        tnode[5 * i + 2] = s.t_left[i];
        tnode[5 * i + 3] = s.t_right[i];
        tnode[5 * i + 4] = s.t_missing_bin[i] * 2 + (s.t_default_left[i] ? 1 : 0);
        vals[i] = s.t_value[i];
    }
    __syncthreads();
    const double lr = s.hp.learning_rate;
    const int K = s.hp.num_class;
    const int k = s.round->class_k;
    const int rec = s.rec_bytes;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < s.n; r += stride) {
        const uint8_t *rb = s.records + r * rec;
        int node = 0;
        // children always have larger ids than their parent, so a walk ends
        // within n_nodes steps
        for (int d = 0; d < n_nodes && tnode[5 * node] >= 0; ++d) {
            const int f = tnode[5 * node];
            const int b = rb[f];
            const int md = tnode[5 * node + 4];
            const int mbin = md >> 1;  // arithmetic shift keeps -1
            const bool left = (b == mbin) ? (md & 1) : (b <= tnode[5 * node + 1]);
            node = left ? tnode[5 * node + 2] : tnode[5 * node + 3];
            if ((unsigned)node >= (unsigned)n_nodes) node = 0;
        }
        double *slot = s.raw + r * K + k;
        *slot = fma(lr, vals[node], *slot);
    }
}

// Archive the finished tree and advance the round state (one block).
__global__ __launch_bounds__(256) void k_round_end(DevState s) {
    const Round rd = *s.round;
    const int mn = s.max_nodes;
    int32_t *ai = s.arc_int + (size_t)rd.tree_index * (6 * mn + 2);
    double *ad = s.arc_dbl + (size_t)rd.tree_index * (3 * mn);
    const int n_nodes = s.t_meta[0];
    for (int i = threadIdx.x; i < n_nodes; i += blockDim.x) {
        ai[6 * i + 0] = s.t_feature[i];
        ai[6 * i + 1] = s.t_threshold[i];
        ai[6 * i + 2] = s.t_left[i];
        ai[6 * i + 3] = s.t_right[i];
        ai[6 * i + 4] = s.t_default_left[i];
        ai[6 * i + 5] = s.t_missing_bin[i];
        ad[3 * i + 0] = s.t_value[i];
        ad[3 * i + 1] = s.t_gain[i];
        ad[3 * i + 2] = s.t_count[i];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        ai[6 * mn + 0] = n_nodes;
        ai[6 * mn + 1] = s.t_meta[1];
        Round nr = rd;
        nr.tree_index = rd.tree_index + 1;
        nr.class_k = rd.class_k + 1;
        if (nr.class_k >= s.hp.num_class) {
            nr.class_k = 0;
            nr.round = rd.round + 1;
        }
        nr.parity = 1 - rd.parity;
        *s.round = nr;
    }
}

// Bins column-major -> per-row records (F bin bytes, zero pad).
__global__ __launch_bounds__(256) void k_build_records(const uint8_t *bins_cm, uint8_t *records,
                                                       int64_t n, int F, int rec) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < n; r += stride) {
        uint8_t *o = records + r * rec;
        for (int f = 0; f < rec; ++f) o[f] = f < F ? bins_cm[(size_t)f * n + r] : 0;
    }
}

__global__ __launch_bounds__(256) void k_fill_f64(double *p, int64_t n, int K, const double *base) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n * K; i += stride)
        p[i] = base[i % K];
}

__global__ void k_exp_sigmoid(const double *x, double *e, double *sg, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        e[i] = ref_exp(x[i]);
        sg[i] = sigmoid(x[i]);
    }
}

// ------------------------------------------------------------------ launch
hipError_t launch_objective(const DevState &s, int grid, hipStream_t st) {
    hipLaunchKernelGGL(k_objective, dim3(grid), dim3(256), 0, st, s);
    return hipGetLastError();
}
hipError_t launch_quantize(const DevState &s, int grid, hipStream_t st) {
    hipLaunchKernelGGL(k_quantize, dim3(grid), dim3(256), 0, st, s);
    return hipGetLastError();
}
size_t score_lds_bytes(const DevState &s) {
    return (size_t)(5 * s.max_nodes + (s.max_nodes & 1)) * 4 + (size_t)s.max_nodes * 8;
}
size_t hist_lds_bytes(const DevState &s) { return (size_t)s.n_features * s.lds_stride * 8; }
hipError_t prepare_hist(const DevState &s) {
    const int bytes = (int)hist_lds_bytes(s);
    hipError_t e = hipFuncSetAttribute((const void *)k_hist<1>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess) return e;
    e = hipFuncSetAttribute((const void *)k_hist<2>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess) return e;
    e = hipFuncSetAttribute((const void *)k_score, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)score_lds_bytes(s));
    if (e != hipSuccess) return e;
    e = hipFuncSetAttribute((const void *)k_hist<4>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess) return e;
    return hipFuncSetAttribute((const void *)k_hist<8>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}
hipError_t launch_hist(const DevState &s, int root_mode, hipStream_t st) {
    const size_t lds = hist_lds_bytes(s);
    const int lpr = s.rec_bytes / 16;
    const dim3 grid(s.hist_grid), block(1024);
    switch (lpr) {
    case 1: hipLaunchKernelGGL(k_hist<1>, grid, block, lds, st, s, root_mode); break;
    case 2: hipLaunchKernelGGL(k_hist<2>, grid, block, lds, st, s, root_mode); break;
    case 4: hipLaunchKernelGGL(k_hist<4>, grid, block, lds, st, s, root_mode); break;
    case 8: hipLaunchKernelGGL(k_hist<8>, grid, block, lds, st, s, root_mode); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
hipError_t launch_partition(const DevState &s, int grid, hipStream_t st) {
    hipLaunchKernelGGL(k_partition, dim3(grid), dim3(256), 0, st, s);
    return hipGetLastError();
}
hipError_t launch_split(const DevState &s, int root_mode, hipStream_t st) {
    hipLaunchKernelGGL(k_split, dim3(s.n_features), dim3(kSplitThreads), 0, st, s, root_mode);
    return hipGetLastError();
}
hipError_t launch_score(const DevState &s, int grid, hipStream_t st) {
    hipLaunchKernelGGL(k_score, dim3(grid), dim3(256), score_lds_bytes(s), st, s);
    return hipGetLastError();
}
hipError_t launch_round_end(const DevState &s, hipStream_t st) {
    hipLaunchKernelGGL(k_round_end, dim3(1), dim3(256), 0, st, s);
    return hipGetLastError();
}
hipError_t launch_build_records(const uint8_t *bins_cm, uint8_t *records, int64_t n, int F, int rec,
                                int grid, hipStream_t st) {
    hipLaunchKernelGGL(k_build_records, dim3(grid), dim3(256), 0, st, bins_cm, records, n, F, rec);
    return hipGetLastError();
}
hipError_t launch_fill_f64(double *p, int64_t n, int K, const double *base, int grid, hipStream_t st) {
    hipLaunchKernelGGL(k_fill_f64, dim3(grid), dim3(256), 0, st, p, n, K, base);
    return hipGetLastError();
}
hipError_t launch_exp_sigmoid(const double *x, double *e, double *sg, int64_t n, hipStream_t st) {
    const int grid = (int)((n + 255) / 256);
    hipLaunchKernelGGL(k_exp_sigmoid, dim3(grid), dim3(256), 0, st, x, e, sg, n);
    return hipGetLastError();
}

}  // namespace mb
