// gfx950 kernels of the GBDT training step (one boosting round = one tree per
// class):
//
//   k_objective   fused gradient/hessian of the round + max |g|, |h| of the
//                 sampled rows (one pass over raw scores and labels)
//   k_quantize    max-abs lattice + stochastic rounding to int8 g/h, written
//                 into each row's record; root row list
//   k_hist        root histogram: LDS-privatized packed 64-bit counters
//                 (grad | hess | count in one ds_add_u64) per block, stored
//                 as block partials
//   k_partition   expansion of a batch of leaves, step 1: row partition (wave
//                 ballot ranks, one atomic reservation per tile and side)
//   k_accum       step 2: the smaller child's histogram from its now
//                 contiguous rows (as k_hist), one block partial per task
//   k_scan        partial merge + sibling subtraction + per-feature integer
//                 prefix scan with fp64 gains + argmax, per (leaf, feature)
//   k_plan        one block: folds features into each new leaf's best split,
//                 replays the best-first order, commits the reference's
//                 splits and selects the next batch
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
#include <hip/hip_ext.h>
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

// Cross-lane moves through DPP (data-parallel primitives): a VALU operand
// modifier, so a reduction step costs a few cycles instead of an LDS
// crossbar round trip. Lanes a control does not cover keep their own value,
// which every reduction below treats as its identity.
// Lane l's 64-bit value on every lane (l wave-uniform).
__device__ __forceinline__ int64_t readlane_i64(int64_t v, int l) {
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(uint64_t)v, l);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)((uint64_t)v >> 32), l);
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ unsigned dpp_u32(unsigned x) {
    return (unsigned)__builtin_amdgcn_update_dpp((int)x, (int)x, CTRL, ROW_MASK, 0xF, false);
}

// Max / min of a 32-bit value over the 64 lanes (every lane active),
// returned wave-uniform: quad swaps, half-row and row mirrors fold each row
// of 16 lanes, then row broadcasts 15 and 31 fold the rows into lane 63.
// (The moved value of a lane a control leaves out is 0, the identity of an
// unsigned maximum, so each step compiles to one v_max_u32 with a DPP
// source.)
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ unsigned dpp_max0(unsigned x) {
    return (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, ROW_MASK, 0xF, false);
}
__device__ __forceinline__ unsigned wave_max_u32(unsigned x) {
    x = max(x, dpp_max0<0xB1, 0xF>(x));   // quad_perm [1,0,3,2]
    x = max(x, dpp_max0<0x4E, 0xF>(x));   // quad_perm [2,3,0,1]
    x = max(x, dpp_max0<0x141, 0xF>(x));  // row_half_mirror
    x = max(x, dpp_max0<0x140, 0xF>(x));  // row_mirror
    x = max(x, dpp_max0<0x142, 0xA>(x));  // row_bcast:15 into rows 1, 3
    x = max(x, dpp_max0<0x143, 0xC>(x));  // row_bcast:31 into rows 2, 3
    return (unsigned)__builtin_amdgcn_readlane((int)x, 63);
}

// max |g|, |h| of a tree's rows (binary32 bits: non-negative floats order
// like their bits), by parity: the blocks of the objective kernels fold
// their maxima into kStatSlots slots (block b into slot b mod kStatSlots),
// so no single address takes an atomic from every block; readers fold the
// slots.
__device__ __forceinline__ int stat_slot(int parity, int which, int b) {
    return (parity * 2 + which) * kStatSlots + (b & (kStatSlots - 1));
}
// Every lane of the wave calls it (one slot per lane).
__device__ __forceinline__ float stats_max_wave(const DevState &s, int parity, int which) {
    static_assert(kStatSlots == 64, "one slot per lane");
    return __uint_as_float(wave_max_u32(s.stats[stat_slot(parity, which, lane_id())]));
}

__device__ __forceinline__ unsigned wave_min_u32(unsigned x) {
    x = min(x, dpp_u32<0xB1, 0xF>(x));
    x = min(x, dpp_u32<0x4E, 0xF>(x));
    x = min(x, dpp_u32<0x141, 0xF>(x));
    x = min(x, dpp_u32<0x140, 0xF>(x));
    x = min(x, dpp_u32<0x142, 0xA>(x));
    x = min(x, dpp_u32<0x143, 0xC>(x));
    return (unsigned)__builtin_amdgcn_readlane((int)x, 63);
}

// Lane l's binary64 value on every lane (l wave-uniform).
__device__ __forceinline__ double rl_f64(double d, int l) {
    const unsigned long long b = (unsigned long long)__double_as_longlong(d);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(b >> 32), l);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)b, l);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

// Sum of a 32-bit value over the 64 lanes, the same DPP steps as
// wave_max_u32 but with lanes a control does not cover reading 0 (the
// identity of the sum), returned wave-uniform.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ unsigned dpp0_u32(unsigned x) {
    return (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, ROW_MASK, 0xF, false);
}
__device__ __forceinline__ unsigned wave_add_u32(unsigned x) {
    x += dpp0_u32<0xB1, 0xF>(x);
    x += dpp0_u32<0x4E, 0xF>(x);
    x += dpp0_u32<0x141, 0xF>(x);
    x += dpp0_u32<0x140, 0xF>(x);
    x += dpp0_u32<0x142, 0xA>(x);
    x += dpp0_u32<0x143, 0xC>(x);
    return (unsigned)__builtin_amdgcn_readlane((int)x, 63);
}

// Inclusive prefix sum of a 32-bit value across the 64 lanes, by DPP
// (GPUOpen's cross-lane scan): row shifts 1, 2, 3 sum each lane's four-lane
// window, shifts 4 and 8 (lanes of the upper banks only) complete each row
// of 16, and row broadcasts 15 and 31 carry the rows' totals upward. A lane
// a control leaves out adds 0. No LDS crossbar round trip.
template <int CTRL, int ROW_MASK, int BANK_MASK>
__device__ __forceinline__ int dpp_add0(int x) {
    return __builtin_amdgcn_update_dpp(0, x, CTRL, ROW_MASK, BANK_MASK, true);
}
__device__ __forceinline__ int wave_incl_scan_i(int v) {
    int t = v + dpp_add0<0x111, 0xF, 0xF>(v);  // row_shr:1
    t += dpp_add0<0x112, 0xF, 0xF>(v);         // row_shr:2
    t += dpp_add0<0x113, 0xF, 0xF>(v);         // row_shr:3
    t += dpp_add0<0x114, 0xF, 0xE>(t);         // row_shr:4, lanes 4-15 of each row
    t += dpp_add0<0x118, 0xF, 0xC>(t);         // row_shr:8, lanes 8-15 of each row
    t += dpp_add0<0x142, 0xA, 0xF>(t);         // row_bcast:15 into rows 1 and 3
    t += dpp_add0<0x143, 0xC, 0xF>(t);         // row_bcast:31 into rows 2 and 3
    return t;
}

// (gain, order) argmax across the wave, result on every lane: larger gain
// wins, equal gains go to the smaller order, so the result is the first
// maximum in scan order. Gains must be >= 0 (a lane with nothing to offer
// holds 0.0); non-negative binary64 values order like their bit patterns,
// so the maximum is found on the high word, then the low word among lanes
// tied on it, then the smallest order among lanes holding the maximum.
// Orders are non-negative.
// The same argmax in one pass: every DPP step carries (gain bits, order)
// and keeps the better pair (larger gain, then smaller order), so the
// reduction is one chain of 6 steps instead of three.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ void lex_step(unsigned &hi, unsigned &lo, unsigned &ord) {
    const unsigned ohi = dpp_u32<CTRL, ROW_MASK>(hi), olo = dpp_u32<CTRL, ROW_MASK>(lo),
                   oord = dpp_u32<CTRL, ROW_MASK>(ord);
    const bool better = ohi > hi || (ohi == hi && (olo > lo || (olo == lo && oord < ord)));
    hi = better ? ohi : hi;
    lo = better ? olo : lo;
    ord = better ? oord : ord;
}
__device__ __forceinline__ void wave_argmax_lex(double &gain, int &order) {
    const unsigned long long bits = gain > 0.0 ? (unsigned long long)__double_as_longlong(gain) : 0ULL;
    unsigned hi = (unsigned)(bits >> 32), lo = (unsigned)bits, ord = (unsigned)order;
    lex_step<0xB1, 0xF>(hi, lo, ord);
    lex_step<0x4E, 0xF>(hi, lo, ord);
    lex_step<0x141, 0xF>(hi, lo, ord);
    lex_step<0x140, 0xF>(hi, lo, ord);
    lex_step<0x142, 0xA>(hi, lo, ord);
    lex_step<0x143, 0xC>(hi, lo, ord);
    hi = (unsigned)__builtin_amdgcn_readlane((int)hi, 63);
    lo = (unsigned)__builtin_amdgcn_readlane((int)lo, 63);
    order = __builtin_amdgcn_readlane((int)ord, 63);
    gain = __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

__device__ __forceinline__ void wave_argmax(double &gain, int &order) {
    const unsigned long long bits = gain > 0.0 ? (unsigned long long)__double_as_longlong(gain) : 0ULL;
    const unsigned hi = (unsigned)(bits >> 32), lo = (unsigned)bits;
    const unsigned mhi = wave_max_u32(hi);
    const unsigned mlo = wave_max_u32(hi == mhi ? lo : 0u);
    const bool top = hi == mhi && lo == mlo;
    const unsigned mord = wave_min_u32(top ? (unsigned)order : 0xFFFFFFFFu);
    gain = __longlong_as_double((long long)(((unsigned long long)mhi << 32) | mlo));
    order = (int)mord;
}

// bagging.sample_rows (src/mojotrees/bagging.mojo:101-129): unit u is in
// the bag when uniform(stream + u) < fraction, and an empty bag takes the
// unit of the least draw (`fallback`, found on the host per bag; -1 when the
// bag is not empty). The unit is the row, or under lambdarank the row's query
// (ranking._refresh_query_bag, ranking.mojo:667-686: whole queries).
__device__ __forceinline__ bool in_bag(const DevState &s, uint64_t bag_stream, int64_t fallback, int64_t r) {
    const int64_t u = s.qid ? (int64_t)s.qid[r] : r;
    return uniform53(bag_stream + (uint64_t)u) < s.hp.bagging_fraction || u == fallback;
}

__device__ __forceinline__ int64_t bag_index_of(const HyperParams &hp, int64_t round) {
    return hp.bagging_freq > 0 ? round / hp.bagging_freq : 0;
}

// bagging.sample_rows stream of one bag (src/mojotrees/bagging.mojo).
__device__ __forceinline__ uint64_t bag_stream_of(const HyperParams &hp, int64_t round) {
    return splitmix64((uint64_t)(hp.bagging_seed & 0x7FFFFFFFFFFFFFFFLL) ^
                      ((uint64_t)bag_index_of(hp, round) * kGolden));
}

__device__ __forceinline__ int64_t bag_fallback_of(const DevState &s, int64_t round) {
    const int64_t b = bag_index_of(s.hp, round);
    return s.bag_fallback && b < s.n_bags ? s.bag_fallback[b] : -1;
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
    if (rd.stopped) return;
    const HyperParams &hp = s.hp;
    if (blockIdx.x == 0 && threadIdx.x == 0) s.cursor[0] = 0;  // root row count
    const uint64_t bstream = hp.bagging ? bag_stream_of(hp, rd.round) : 0;
    const int64_t bfall = hp.bagging ? bag_fallback_of(s, rd.round) : -1;
    const int K = hp.num_class, ck = rd.class_k;
    const double factor = K > 1 ? (double)K / (double)(K - 1) : 0.0;
    float mg = 0.0f, mh = 0.0f;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < s.n; r += stride) {
        float g, h;
        // boosting._fill_grad_hess_into (boosting.mojo:676-811): the weight
        // scales both, after the hessian floor
        const double w = s.weights ? s.weights[r] : 1.0;
        if (hp.objective == kObjMulticlass) {
            // _fill_softmax_grad_hess_at (boosting.mojo:3621-3678) on the
            // probabilities of the round's start
            const double p = s.prob[(size_t)ck * s.n + r];
            const double y = ((int)s.labels[r] == ck) ? 1.0 : 0.0;
            g = (float)(w * (p - y));
            double hh = factor * p * (1.0 - p);
            if (hh < 1e-16) hh = 1e-16;
            h = (float)(w * hh);
        } else if (hp.objective == kObjBinary) {
            double p = sigmoid(s.raw[r]);
            g = (float)(w * (p - s.labels[r]));
            double hh = p * (1.0 - p);
            if (hh < 1e-16) hh = 1e-16;
            h = (float)(w * hh);
        } else {
            g = (float)(w * (s.raw[r] - s.labels[r]));
            h = (float)(w * 1.0);
        }
        if (s.gh2) {
            ((float2 *)s.gh2)[r] = make_float2(g, h);
        } else {
            s.grad[r] = g;
            s.hess[r] = h;
        }
        float ag = fabsf(g), ah = fabsf(h);
        bool sel = !hp.bagging || in_bag(s, bstream, bfall, r);
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
        atomicMax(&s.stats[stat_slot(rd.parity, 0, blockIdx.x)], __float_as_uint(mg));
        atomicMax(&s.stats[stat_slot(rd.parity, 1, blockIdx.x)], __float_as_uint(mh));
    }
}

// --------------------------------------------------------------- lambdarank
// LambdaRank gradients (ranking._fill_query_lambdas,
// src/mojotrees/ranking.mojo:510-570, over every query, _fill_lambdas
// :573-600), one block per query, in binary64 as the reference's ranker
// keeps them. The query's documents are sorted by score in LDS (bitonic,
// descending, ties by position: the reference's stable order). The pairs
// (i, j), i below the truncation level, j > i, are then taken one rank i at
// a time: the block evaluates row i's pairs in parallel, each rank j > i
// adds its one contribution (it receives the pairs in i order, as in the
// reference's loop), and two threads add row i's values in j order into the
// running sum of |lambda| and into rank i's own gradient. Every sum thus has
// the reference's order and the lambdas its bits. Query LDS: 49 bytes per
// document of the largest query (rounded up to a power of two).
__device__ __forceinline__ bool rank_before(double ka, int ia, double kb, int ib) {
    return ka > kb || (ka == kb && ia < ib);
}

__global__ __launch_bounds__(256) void k_lambdarank(DevState s) {
    extern __shared__ unsigned char rank_lds[];
    __shared__ double s_factor;
    __shared__ double red_g[4], red_h[4];
    const Round rd = *s.round;
    if (rd.stopped) return;
    const HyperParams &hp = s.hp;
    if (blockIdx.x == 0 && threadIdx.x == 0) s.cursor[0] = 0;  // root row count
    const int P = s.rank_pad;
    double *key = (double *)rank_lds;
    double *G = key + P;
    double *H = G + P;
    double *PL = H + P;
    double *PH = PL + P;
    int32_t *idx = (int32_t *)(PH + P);
    int32_t *lab = idx + P;
    uint8_t *V = (uint8_t *)(lab + P);
    const int tid = threadIdx.x, nt = blockDim.x;
    const double sigma = hp.rank_sigma;
    const bool norm = hp.rank_norm != 0;
    const uint64_t bstream = hp.bagging ? bag_stream_of(hp, rd.round) : 0;
    const int64_t bfall = hp.bagging ? bag_fallback_of(s, rd.round) : -1;
    double mg = 0.0, mh = 0.0;
    for (int q = blockIdx.x; q < s.n_queries; q += gridDim.x) {
        const int64_t a = s.qstart[q];
        const int cnt = (int)(s.qstart[q + 1] - a);
        if (cnt > kMaxQueryRows) continue;  // k_lambdarank_big's (block-uniform)
        int p2 = 1;
        while (p2 < cnt) p2 <<= 1;
        for (int i = tid; i < p2; i += nt) {
            key[i] = i < cnt ? s.raw[a + i] : -INFINITY;
            idx[i] = i;
        }
        __syncthreads();
        for (int k = 2; k <= p2; k <<= 1)
            for (int j = k >> 1; j > 0; j >>= 1) {
                for (int i = tid; i < p2; i += nt) {
                    const int l = i ^ j;
                    if (l > i) {
                        const bool l_first = rank_before(key[l], idx[l], key[i], idx[i]);
                        if ((i & k) == 0 ? l_first : !l_first) {
                            const double tk = key[i];
                            key[i] = key[l];
                            key[l] = tk;
                            const int ti = idx[i];
                            idx[i] = idx[l];
                            idx[l] = ti;
                        }
                    }
                }
                __syncthreads();
            }
        for (int k = tid; k < cnt; k += nt) {
            lab[k] = (int)s.labels[a + idx[k]];
            G[k] = 0.0;
            H[k] = 0.0;
        }
        __syncthreads();
        const double best = key[0], worst = key[cnt - 1];
        const double inv = s.inv_max_dcg[q];
        const int top = cnt - 1 < hp.rank_trunc ? cnt - 1 : hp.rank_trunc;
        double sum = 0.0;  // thread 0's running sum of |lambda| (ranking.mojo:565)
        for (int i = 0; i < top; ++i) {
            const int li = lab[i];
            const double si = key[i];
            for (int j = i + 1 + tid; j < cnt; j += nt) {
                const int lj = lab[j];
                double pl = 0.0, ph = 0.0;
                uint8_t v = 0;
                if (li != lj) {
                    const bool ih = li > lj;  // rank i holds the more relevant document
                    const int hr = ih ? i : j, lr = ih ? j : i;
                    const double delta = ih ? si - key[j] : key[j] - si;
                    const double gap = label_gain(ih ? li : lj) - label_gain(ih ? lj : li);
                    const double paired = fabs(s.rank_disc[hr] - s.rank_disc[lr]);
                    double dn = gap * paired * inv;
                    if (norm && best != worst) dn /= 0.01 + fabs(delta);
                    double p = pair_sigmoid(delta, sigma);
                    double phh = p * (1.0 - p);
                    p *= -sigma * dn;
                    phh *= sigma * sigma * dn;
                    pl = p;
                    ph = phh;
                    v = ih ? 3 : 1;
                    G[j] = ih ? G[j] - p : G[j] + p;
                    H[j] = H[j] + phh;
                }
                PL[j] = pl;
                PH[j] = ph;
                V[j] = v;
            }
            __syncthreads();
            if (tid == 0) {
                for (int j = i + 1; j < cnt; ++j)
                    if (V[j]) sum -= 2.0 * PL[j];
            } else if (tid == 64) {
                double g = G[i], h = H[i];
                for (int j = i + 1; j < cnt; ++j) {
                    const uint8_t v = V[j];
                    if (!v) continue;
                    g = (v & 2) ? g + PL[j] : g - PL[j];
                    h = h + PH[j];
                }
                G[i] = g;
                H[i] = h;
            }
            __syncthreads();
        }
        // the query's normalizer log2(1 + S) / S (ranking.mojo:567-570); 0
        // marks "not applied"
        if (tid == 0) s_factor = (norm && sum > 0.0) ? ref_log2(1.0 + sum) / sum : 0.0;
        __syncthreads();
        const double factor = s_factor;
        // the magnitude stats are the bag's (whole queries)
        const bool sel = !hp.bagging || in_bag(s, bstream, bfall, a);
        for (int k = tid; k < cnt; k += nt) {
            double g = G[k], h = H[k];
            if (factor != 0.0) {
                g *= factor;
                h *= factor;
            }
            const int64_t r = a + idx[k];
            // lambdarank_gradients (ranking.mojo:613-616): sample weights
            // scale the finished lambda and hessian
            if (s.weights) {
                g *= s.weights[r];
                h *= s.weights[r];
            }
            s.grad64[r] = g;
            s.hess64[r] = h;
            if (sel && isfinite(g) && isfinite(h)) {
                mg = fmax(mg, fabs(g));
                mh = fmax(mh, fabs(h));
            }
        }
        __syncthreads();  // the LDS is the next query's
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        mg = fmax(mg, __shfl_xor(mg, d, 64));
        mh = fmax(mh, __shfl_xor(mh, d, 64));
    }
    const int w = tid >> 6;
    if (lane_id() == 0) {
        red_g[w] = mg;
        red_h[w] = mh;
    }
    __syncthreads();
    if (tid == 0) {
        for (int i = 1; i < (nt >> 6); ++i) {
            mg = fmax(mg, red_g[i]);
            mh = fmax(mh, red_h[i]);
        }
        // non-negative doubles order like their bit patterns
        atomicMax(&s.stats64[rd.parity * 2 + 0], (unsigned long long)__double_as_longlong(mg));
        atomicMax(&s.stats64[rd.parity * 2 + 1], (unsigned long long)__double_as_longlong(mh));
    }
}

// Queries of more than kMaxQueryRows documents, which the LDS sort cannot
// hold: one block per query at a time, with the query's sort keys,
// positions, labels and running lambdas in the block's slot of global
// memory. The same bitonic order and the same arithmetic as k_lambdarank;
// each rank i's pairs are evaluated kRankChunk documents at a time, their
// values staged in LDS, and the two sequential sums (the running |lambda|
// and rank i's own lambda and hessian) walk each chunk in document order,
// carried from chunk to chunk, so every sum keeps
// ranking._fill_query_lambdas' order (src/mojotrees/ranking.mojo:504-654).
constexpr int kRankChunk = 2048;
__global__ __launch_bounds__(256) void k_lambdarank_big(DevState s) {
    __shared__ double PL[kRankChunk], PH[kRankChunk];
    __shared__ uint8_t V[kRankChunk];
    __shared__ double s_factor;
    __shared__ double red_g[4], red_h[4];
    const Round rd = *s.round;
    if (rd.stopped) return;
    const HyperParams &hp = s.hp;
    const size_t P = (size_t)s.rank_big_pad;
    double *key = s.rank_scratch + (size_t)blockIdx.x * 3 * P;
    double *G = key + P;
    double *H = G + P;
    int32_t *idx = s.rank_scratch_i + (size_t)blockIdx.x * 2 * P;
    int32_t *lab = idx + P;
    const int tid = threadIdx.x, nt = blockDim.x;
    const double sigma = hp.rank_sigma;
    const bool norm = hp.rank_norm != 0;
    const uint64_t bstream = hp.bagging ? bag_stream_of(hp, rd.round) : 0;
    const int64_t bfall = hp.bagging ? bag_fallback_of(s, rd.round) : -1;
    double mg = 0.0, mh = 0.0;
    for (int bq = blockIdx.x; bq < s.n_big; bq += gridDim.x) {
        const int q = s.rank_big[bq];
        const int64_t a = s.qstart[q];
        const int cnt = (int)(s.qstart[q + 1] - a);
        int p2 = 1;
        while (p2 < cnt) p2 <<= 1;
        for (int i = tid; i < p2; i += nt) {
            key[i] = i < cnt ? s.raw[a + i] : -INFINITY;
            idx[i] = i;
        }
        __threadfence_block();
        __syncthreads();
        for (int k = 2; k <= p2; k <<= 1)
            for (int j = k >> 1; j > 0; j >>= 1) {
                for (int i = tid; i < p2; i += nt) {
                    const int l = i ^ j;
                    if (l > i) {
                        const double ki = key[i], kl = key[l];
                        const int ii = idx[i], il = idx[l];
                        const bool l_first = rank_before(kl, il, ki, ii);
                        if ((i & k) == 0 ? l_first : !l_first) {
                            key[i] = kl;
                            key[l] = ki;
                            idx[i] = il;
                            idx[l] = ii;
                        }
                    }
                }
                __threadfence_block();
                __syncthreads();
            }
        for (int k = tid; k < cnt; k += nt) {
            lab[k] = (int)s.labels[a + idx[k]];
            G[k] = 0.0;
            H[k] = 0.0;
        }
        __threadfence_block();
        __syncthreads();
        const double best = key[0], worst = key[cnt - 1];
        const double inv = s.inv_max_dcg[q];
        const int top = cnt - 1 < hp.rank_trunc ? cnt - 1 : hp.rank_trunc;
        double sum = 0.0;         // thread 0's running sum of |lambda| (ranking.mojo:565)
        double gi = 0.0, hi = 0.0;  // thread 64's rank-i lambda and hessian
        for (int i = 0; i < top; ++i) {
            const int li = lab[i];
            const double si = key[i];
            if (tid == 64) {
                gi = G[i];
                hi = H[i];
            }
            for (int c0 = i + 1; c0 < cnt; c0 += kRankChunk) {
                const int c1 = c0 + kRankChunk < cnt ? c0 + kRankChunk : cnt;
                for (int j = c0 + tid; j < c1; j += nt) {
                    const int lj = lab[j];
                    double pl = 0.0, ph = 0.0;
                    uint8_t v = 0;
                    if (li != lj) {
                        const bool ih = li > lj;  // rank i holds the more relevant document
                        const double kj = key[j];
                        const int hr = ih ? i : j, lr = ih ? j : i;
                        const double delta = ih ? si - kj : kj - si;
                        const double gap = label_gain(ih ? li : lj) - label_gain(ih ? lj : li);
                        const double paired = fabs(s.rank_disc[hr] - s.rank_disc[lr]);
                        double dn = gap * paired * inv;
                        if (norm && best != worst) dn /= 0.01 + fabs(delta);
                        double p = pair_sigmoid(delta, sigma);
                        double phh = p * (1.0 - p);
                        p *= -sigma * dn;
                        phh *= sigma * sigma * dn;
                        pl = p;
                        ph = phh;
                        v = ih ? 3 : 1;
                        G[j] = ih ? G[j] - p : G[j] + p;
                        H[j] = H[j] + phh;
                    }
                    PL[j - c0] = pl;
                    PH[j - c0] = ph;
                    V[j - c0] = v;
                }
                __syncthreads();
                if (tid == 0) {
                    for (int j = 0; j < c1 - c0; ++j)
                        if (V[j]) sum -= 2.0 * PL[j];
                } else if (tid == 64) {
                    for (int j = 0; j < c1 - c0; ++j) {
                        const uint8_t v = V[j];
                        if (!v) continue;
                        gi = (v & 2) ? gi + PL[j] : gi - PL[j];
                        hi = hi + PH[j];
                    }
                }
                __syncthreads();  // the staged chunk is rewritten next
            }
            if (tid == 64) {
                G[i] = gi;
                H[i] = hi;
            }
            __threadfence_block();
            __syncthreads();
        }
        if (tid == 0) s_factor = (norm && sum > 0.0) ? ref_log2(1.0 + sum) / sum : 0.0;
        __syncthreads();
        const double factor = s_factor;
        const bool sel = !hp.bagging || in_bag(s, bstream, bfall, a);
        for (int k = tid; k < cnt; k += nt) {
            double g = G[k], h = H[k];
            if (factor != 0.0) {
                g *= factor;
                h *= factor;
            }
            const int64_t r = a + idx[k];
            if (s.weights) {
                g *= s.weights[r];
                h *= s.weights[r];
            }
            s.grad64[r] = g;
            s.hess64[r] = h;
            if (sel && isfinite(g) && isfinite(h)) {
                mg = fmax(mg, fabs(g));
                mh = fmax(mh, fabs(h));
            }
        }
        __threadfence_block();
        __syncthreads();  // the slot is the next query's
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        mg = fmax(mg, __shfl_xor(mg, d, 64));
        mh = fmax(mh, __shfl_xor(mh, d, 64));
    }
    const int w = tid >> 6;
    if (lane_id() == 0) {
        red_g[w] = mg;
        red_h[w] = mh;
    }
    __syncthreads();
    if (tid == 0) {
        for (int i = 1; i < (nt >> 6); ++i) {
            mg = fmax(mg, red_g[i]);
            mh = fmax(mh, red_h[i]);
        }
        atomicMax(&s.stats64[rd.parity * 2 + 0], (unsigned long long)__double_as_longlong(mg));
        atomicMax(&s.stats64[rd.parity * 2 + 1], (unsigned long long)__double_as_longlong(mh));
    }
}

// ----------------------------------------------------------------- softmax
// boosting._softmax_rows (src/mojotrees/boosting.mojo:3529-3573): per row,
// shift by the maximum, exponentiate with the reference's exp, sum in class
// order, divide. Run once at the start of each multiclass round; every class
// tree of the round uses these probabilities. Raw scores and probabilities
// of a multiclass training are class-major (class k of row r at k n + r), so
// each class's pass reads and writes consecutive rows.
__global__ __launch_bounds__(256) void k_softmax(DevState s) {
    if (s.round->stopped) return;
    const int K = s.hp.num_class;
    const int64_t n = s.n;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    constexpr int kRegK = 16;  // up to this many classes, the exponentials stay in registers
    if (K <= kRegK) {
        for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < n; r += stride) {
            const double *x = s.raw + r;
            double *p = s.prob + r;
            double e[kRegK];
#pragma unroll
            for (int i = 0; i < kRegK; ++i) e[i] = i < K ? x[(size_t)i * n] : 0.0;
            double m = e[0];
#pragma unroll
            for (int i = 1; i < kRegK; ++i)
                if (i < K && e[i] > m) m = e[i];
            double total = 0.0;
#pragma unroll
            for (int i = 0; i < kRegK; ++i)
                if (i < K) {
                    e[i] = ref_exp(e[i] - m);
                    total += e[i];
                }
#pragma unroll
            for (int i = 0; i < kRegK; ++i)
                if (i < K) p[(size_t)i * n] = e[i] / total;
        }
        return;
    }
    for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < n; r += stride) {
        const double *x = s.raw + r;
        double *p = s.prob + r;
        double m = x[0];
        for (int i = 1; i < K; ++i)
            if (x[(size_t)i * n] > m) m = x[(size_t)i * n];
        double total = 0.0;
        for (int i = 0; i < K; ++i) {
            const double e = ref_exp(x[(size_t)i * n] - m);
            p[(size_t)i * n] = e;
            total += e;
        }
        for (int i = 0; i < K; ++i) p[(size_t)i * n] = p[(size_t)i * n] / total;
    }
}

// GOSS is on for this tree: enabled and past its warmup rounds
// (GossParams.active, goss.mojo:102-157).
__device__ __forceinline__ bool goss_on(const DevState &s) {
    const Round &rd = *s.round;
    return s.hp.goss && !rd.stopped && rd.round >= s.hp.goss_warm;
}

// The GOSS weight of the round's sampled small-importance rows.
__device__ __forceinline__ double goss_weight(const GossState &g, int64_t n) {
    return g.other_k > 0 ? (double)(n - g.top_k) / (double)g.other_k : 1.0;
}

// ---------------------------------------------------------------- quantize
// derive_scales (max-abs rule, quantized_gradient.mojo:1343-1453) and
// quantize_scalar per row (:1479-1545). Every row is quantized, sampled or
// not, with the row id as the stream counter. The int8 pair lands in the
// last two bytes of the row's record, next to its bins. The root row list
// (the bag) is gathered here; without bagging the root reads rows directly.
// The quantizer of one tree: its scales, lattice bounds and streams, and
// the tree's GOSS weight (rounds where GOSS samples: the quantizer sees the
// weighted derivatives, goss_round before the grower).
struct QCtx {
    double gu, hu, gmult;
    int32_t gmax, hmax;
    uint64_t gs, hs;
    bool stoch, gs_on;
};

__device__ __forceinline__ QCtx quant_ctx(const DevState &s, const Round &rd) {
    const HyperParams &hp = s.hp;
    QCtx c;
    c.gs_on = goss_on(s);
    c.gmult = c.gs_on ? goss_weight(*s.gst, s.n) : 1.0;
    const double sg = (double)stats_max_wave(s, rd.parity, 0), sh = (double)stats_max_wave(s, rd.parity, 1);
    double max_g = c.gs_on ? __longlong_as_double((long long)s.goss_max[rd.parity * 2 + 0])
                   : hp.grad64 ? __longlong_as_double((long long)s.stats64[rd.parity * 2 + 0])
                               : sg;
    double max_h = c.gs_on ? __longlong_as_double((long long)s.goss_max[rd.parity * 2 + 1])
                   : hp.grad64 ? __longlong_as_double((long long)s.stats64[rd.parity * 2 + 1])
                               : sh;
    if (max_g < 1e-12) max_g = 1e-12;
    if (max_h < 1e-12) max_h = 1e-12;
    // max-abs: (B / 2) / max|g| and B / max|h| with clamps B / 2, B; the
    // magnitude-sum lattice: the round's power-of-two scales (k_magfold)
    // with clamps 2^30; a constant hessian takes one unit over max|h| on both
    c.gmax = hp.wide ? (int32_t)kFixedOne : hp.quant_bins / 2;
    c.hmax = hp.const_hessian ? 1 : hp.wide ? (int32_t)kFixedOne : hp.quant_bins;
    c.gu = hp.wide ? rd.grad_units : (double)c.gmax / max_g;
    c.hu = hp.wide ? rd.hess_units : hp.const_hessian ? 1.0 / max_h : (double)c.hmax / max_h;
    c.gs = quant_stream(hp.quant_seed, rd.round, rd.class_k, 0);
    c.hs = quant_stream(hp.quant_seed, rd.round, rd.class_k, 1);
    c.stoch = hp.stochastic != 0;
    return c;
}

// Row r's quantized pair (quantize_scalar with the row id as the stream
// counter), weighted by the GOSS weight when the row was sampled with it.
__device__ __forceinline__ void quant_row(const DevState &s, const QCtx &c, int64_t r, int32_t &qg, int32_t &qh) {
    const double gw = c.gs_on && s.goss_other[r] ? c.gmult : 1.0;
    const double gv = (s.hp.grad64 ? s.grad64[r] : (double)s.grad[r]) * gw;
    const double hv = (s.hp.grad64 ? s.hess64[r] : (double)s.hess[r]) * gw;
    qg = quantize_scalar(gv, c.gu, c.gmax, c.stoch, c.gs + (uint64_t)r);
    qh = quantize_scalar(hv, c.hu, c.hmax, c.stoch, c.hs + (uint64_t)r);
}

// One of row r's two binary32 values, its gradient (isg) or hessian, with
// its GOSS weight applied in binary64 (w: the row was sampled with the
// weight), quantized as quant_row does: the loads (binary32 derivatives
// only) can be issued ahead of their use.
__device__ __forceinline__ int32_t quant_value(const QCtx &c, float v, bool w, int64_t r, bool isg) {
    return quantize_scalar((double)v * (w ? c.gmult : 1.0), isg ? c.gu : c.hu, isg ? c.gmax : c.hmax, c.stoch,
                           (isg ? c.gs : c.hs) + (uint64_t)r);
}

// write_pairs = 0: the max-abs int8 pairs are left to the root build
// (k_hist quantizes the rows it reads, k_hist<.., kQuant>); the scales and
// the root row list are still published here.
__device__ __forceinline__ void quantize_body(const DevState &s, int write_pairs) {
    const Round rd = *s.round;
    if (rd.stopped) return;
    const HyperParams &hp = s.hp;
    const QCtx c = quant_ctx(s, rd);
    const bool gs_on = c.gs_on;
    GossState gst{};
    if (gs_on) gst = *s.gst;
    const double gmult = c.gmult;
    const double gu = c.gu, hu = c.hu;
    const uint64_t bstream = hp.bagging ? bag_stream_of(hp, rd.round) : 0;
    const int64_t bfall = hp.bagging ? bag_fallback_of(s, rd.round) : -1;
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        s.round->sampled = hp.bagging || gs_on;
        s.round->goss_mult = gmult;
        if (gs_on) s.cursor[0] = gst.bag_n;
        if (hp.goss) {
            s.goss_max[(1 - rd.parity) * 2 + 0] = 0ULL;
            s.goss_max[(1 - rd.parity) * 2 + 1] = 0ULL;
        }
        if (!hp.wide) {
            s.round->grad_units = gu;
            s.round->hess_units = hu;
        }
        for (int i = 0; i < 2 * kStatSlots; ++i) s.stats[stat_slot(1 - rd.parity, 0, 0) + i] = 0u;
        if (hp.grad64) {
            s.stats64[(1 - rd.parity) * 2 + 0] = 0ULL;
            s.stats64[(1 - rd.parity) * 2 + 1] = 0ULL;
        }
    }
    // the round's GOSS sample is copied into the root list per class tree
    // (one tree per round: k_goss_scatter wrote it there)
    const bool copy_sample = gs_on && hp.num_class > 1;
    // no pairs to write and no list to fill: nothing per row
    if (!(hp.quantized && write_pairs) && !copy_sample && !(hp.bagging && !gs_on)) return;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int rec = s.rec_bytes;
    for (int64_t r0 = (int64_t)blockIdx.x * blockDim.x; r0 < s.n; r0 += stride) {
        const int64_t r = r0 + threadIdx.x;
        const bool valid = r < s.n;
        if (valid && hp.quantized && write_pairs) {
            int32_t qg, qh;
            quant_row(s, c, r, qg, qh);
            if (hp.stage16) {
                // _quantize_grad_hess_i16_kernel: the same integers narrowed,
                // each plane's misfits counted (a constant hessian's plane is
                // never read, and its values are 1)
                if (qg > 32767 || qg < -32768) atomicAdd(&s.stage16_over[0], 1ULL);
                if (qh > 32767 || qh < -32768) atomicAdd(&s.stage16_over[1], 1ULL);
                const uint32_t v = (uint32_t)(uint16_t)(int16_t)qg | ((uint32_t)(uint16_t)(int16_t)qh << 16);
                for (int t = 0; t < s.n_tiles; ++t)
                    *(uint32_t *)(s.records_w + ((size_t)t * s.n + r) * rec + rec - 4) = v;
            } else if (hp.wide) {
                *(int2 *)(s.gq + 2 * r) = make_int2(qg, qh);
            } else {
                uint16_t v = (uint16_t)(uint8_t)(int8_t)qg | (uint16_t)((uint16_t)(uint8_t)(int8_t)qh << 8);
                for (int t = 0; t < s.n_tiles; ++t)
                    *(uint16_t *)(s.records_w + ((size_t)t * s.n + r) * rec + rec - 2) = v;
            }
        }
        if (gs_on) {
            if (copy_sample && r < gst.bag_n) {
                const int32_t rr = s.goss_rows[r];
                s.rows0[r] = rr;
                // interleaved binary32 derivatives: the row's GOSS weight bit
                // goes into its hessian's sign bit (hessians are >= 0), which
                // the fp32 accumulation reads with the pair
                if (s.gh2 && s.goss_other[rr]) {
                    uint32_t *hw = (uint32_t *)(s.gh2 + 2 * (size_t)rr + 1);
                    *hw = *hw | 0x80000000u;
                }
            }
        } else if (!hp.bagging) {
            // every row in order: the root build and the root's partition
            // compute the ids, no list is written
        } else {
            // Sampled rows appended with one atomic per wave; their order in
            // the root range does not matter (integer histograms).
            bool take = valid && in_bag(s, bstream, bfall, r);
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

__global__ __launch_bounds__(256) void k_quantize(DevState s, int write_pairs) { quantize_body(s, write_pairs); }

// ------------------------------------------------ magnitude-sum lattice
// The magnitude reduction of the reference's device histogram, in its fixed
// order (gpu_objectives_native._abs_sum_kernel :982-1040): 256 workgroups of
// 256 threads; thread t of workgroup b adds |g| and |h| in binary32 for rows
// b * 256 + t + k * 65536 of the round's sample (gradient_stats' subset,
// quantized_gradient.mojo:762-810: rows outside it, and rows whose gradient
// or hessian is not finite, add nothing); each workgroup then halves its 256
// sums in LDS. The sums are the same bits on every run and every GPU.
constexpr int kMagBlocks = 256, kMagThreads = 256;

__global__ __launch_bounds__(kMagThreads) void k_magsum(DevState s) {
    __shared__ float sg[kMagThreads], sh[kMagThreads];
    const Round rd = *s.round;
    if (rd.stopped) return;
    const HyperParams &hp = s.hp;
    const uint64_t bstream = hp.bagging ? bag_stream_of(hp, rd.round) : 0;
    const int64_t bfall = hp.bagging ? bag_fallback_of(s, rd.round) : -1;
    // a GOSS round's sample: its top rows (kappa INT_MIN) and the rows the
    // sampling kept, whose derivatives carry the GOSS weight (applied in
    // binary64, then narrowed as gradient_stats' caller narrows them)
    const bool gs = goss_on(s);
    const double gmult = gs ? goss_weight(*s.gst, s.n) : 1.0;
    const int t = threadIdx.x;
    float ag = 0.0f, ah = 0.0f;
    for (int64_t r = (int64_t)blockIdx.x * kMagThreads + t; r < s.n; r += (int64_t)kMagBlocks * kMagThreads) {
        if (hp.bagging && !in_bag(s, bstream, bfall, r)) continue;
        float g = s.grad[r], h = s.hess[r];
        if (gs) {
            const bool other = s.goss_other[r] != 0;
            if (!other && s.goss_kappa[r] != INT_MIN) continue;  // not sampled
            if (other) {
                g = (float)((double)g * gmult);
                h = (float)((double)h * gmult);
            }
        }
        g = fabsf(g);
        h = fabsf(h);
        if (!(isfinite(g) && isfinite(h))) continue;
        ag += g;
        ah += h;
    }
    sg[t] = ag;
    sh[t] = ah;
    __syncthreads();
    for (int a = kMagThreads / 2; a > 0; a >>= 1) {
        if (t < a) {
            sg[t] = sg[t] + sg[t + a];
            sh[t] = sh[t] + sh[t + a];
        }
        __syncthreads();
    }
    if (t == 0) {
        s.magpart[blockIdx.x] = sg[0];
        s.magpart[kMagBlocks + blockIdx.x] = sh[0];
    }
}

// sum_abs_partials (gpu_objectives_native.mojo:1100-1125): the workgroup sums
// added in binary64 in ascending order, then derive_scales' magnitude-sum
// rule (quantized_gradient.mojo:1343-1420): the power-of-two scales
// fixed_point_scale_pow2(sum |g|) and (sum |h|), or one unit over max|h| for
// a constant hessian. A total out of the fixed-point range flags the sticky
// error (code 4) and leaves a unit scale.
__global__ void k_magfold(DevState s) {
    if (threadIdx.x != 0) return;
    Round *rp = s.round;
    if (rp->stopped) return;
    double tg = 0.0, th = 0.0;
    for (int b = 0; b < kMagBlocks; ++b) {
        tg += (double)s.magpart[b];
        th += (double)s.magpart[kMagBlocks + b];
    }
    bool okg = false, okh = true;
    const double gu = fixed_point_scale_pow2(tg, okg);
    double hu;
    if (s.hp.const_hessian) {
        unsigned mb = 0u;
        for (int i = 0; i < kStatSlots; ++i) mb = max(mb, s.stats[stat_slot(rp->parity, 1, i)]);
        double mh = (double)__uint_as_float(mb);
        if (mh < 1e-12) mh = 1e-12;
        hu = 1.0 / mh;
    } else {
        hu = fixed_point_scale_pow2(th, okh);
    }
    if (!okg || !okh) atomicOr(s.error, 4);
    rp->grad_units = gu;
    rp->hess_units = hu;
}

// -------------------------------------------------------------------- GOSS
// goss_round (src/mojotrees/goss.mojo:294-396), from round floor(1 / lr) on
// (GossParams.warmup, :102-157): importance |g h| of the fp32 derivatives in
// fp64, the top_k-th largest importance as threshold (every row at or above
// it is kept), then selection sampling of the other rows in row order --
// row r is kept with probability (other_k - kept) / rest with rest =
// (n - r) - (top_k - tops before r), drawn as uniform(stream + r) -- and
// the kept rows' g and h weighted by (n - top_k) / other_k.
//
// The selection sampling is a sequential count: row r is kept iff the
// number kept before it is below kappa_r, the least count at which the
// reference's comparison u_r < (other_k - count) / rest fails (found from
// the same double expression, so the decisions are the reference's). A
// single wave then runs the count over 64 rows at a time: a row whose kappa
// is at most the count is dropped and one whose kappa exceeds the count by
// 64 or more is kept whatever the rows before it do, so a step costs a
// ballot and a popcount; only steps with a kappa inside that window take the
// 64 rows one by one.

// A row's sampling importance: goss_importance's |g h| (goss.mojo:294-305)
// of a single-output round, the class sum of a multiclass round (goss_imp).
__device__ __forceinline__ unsigned long long goss_key(const DevState &s, int64_t r) {
    double imp;
    if (s.hp.num_class > 1) {
        imp = s.goss_imp[r];
    } else if (s.gh2) {
        const float2 gh = ((const float2 *)s.gh2)[r];
        imp = fabs((double)gh.x * (double)gh.y);
    } else {
        imp = fabs((double)s.grad[r] * (double)s.hess[r]);
    }
    return (unsigned long long)__double_as_longlong(imp);  // non-negative: ordered like its bits
}


// _multiclass_goss_select's importance (boosting.mojo:3680-3710): per row,
// the sum in class order of |g_k h_k| over every class k, each class's
// derivatives exactly as k_objective writes them for that class's tree
// (narrowed to binary32, weight applied), the products and the sum in
// binary64.
__global__ __launch_bounds__(256) void k_goss_importance(DevState s) {
    if (!goss_on(s)) return;
    const int K = s.hp.num_class;
    const double factor = (double)K / (double)(K - 1);
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < s.n; r += stride) {
        const double w = s.weights ? s.weights[r] : 1.0;
        const int y = (int)s.labels[r];
        double imp = 0.0;
        for (int k = 0; k < K; ++k) {
            const double p = s.prob[(size_t)k * s.n + r];
            const float g = (float)(w * (p - (y == k ? 1.0 : 0.0)));
            double hh = factor * p * (1.0 - p);
            if (hh < 1e-16) hh = 1e-16;
            const float h = (float)(w * hh);
            imp += fabs((double)g * (double)h);
        }
        s.goss_imp[r] = imp;
    }
}

__global__ __launch_bounds__(256) void k_goss_setup(DevState s) {
    if (!goss_on(s)) return;
    for (int i = threadIdx.x; i < 8 * kGossHistSlots * 256; i += blockDim.x) s.goss_hist[i] = 0u;
    if (threadIdx.x == 0) {
        GossState g;
        const int64_t n = s.n;
        int64_t top_k = (int64_t)((double)n * s.hp.top_rate);
        if (top_k < 1) top_k = 1;
        if (top_k > n) top_k = n;
        int64_t other_k = (int64_t)((double)n * s.hp.other_rate);
        if (other_k > n - top_k) other_k = n - top_k;
        g.prefix = 0ULL;
        g.rank = top_k - 1;
        s.goss_sel[0] = 0ULL;
        s.goss_sel[1] = (unsigned long long)(top_k - 1);
        g.top_k = top_k;
        g.other_k = other_k;
        g.threshold = 0.0;
        g.kept_other = 0;
        g.bag_n = 0;
        g.n_uncertain = 0;
        g.fallback = s.hp.goss_exact ? 1 : 0;
        g.pad_ = 0;
        *s.gst = g;
    }
}

// Radix select of the top_k-th largest key, 8 bits per pass from the top.
// The digit of the rank-th largest key (0-based, descending) in a 256-bin
// digit histogram, by one wave: the highest digit whose count from the top
// passes rank (digit 0 when none does); rank becomes the rank inside that
// digit. Lane l holds digits 4l .. 4l + 3; counts are below n < 2^31. h: the
// pass's kGossHistSlots partial histograms (a block adds its counts into
// slot blockIdx mod kGossHistSlots, so no counter takes an atomic from every
// block), summed here.
__device__ __forceinline__ int goss_pick_wave(const uint32_t *h, long long &rank) {
    const int lane = lane_id();
    uint4 c = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
    for (int k = 0; k < kGossHistSlots; ++k) {
        const uint4 v = ((const uint4 *)(h + k * 256))[lane];
        c.x += v.x;
        c.y += v.y;
        c.z += v.z;
        c.w += v.w;
    }
    const int t = (int)(c.x + c.y + c.z + c.w);
    const int incl = wave_incl_scan_i(t);
    const int total = __builtin_amdgcn_readlane(incl, 63);
    const int cc[4] = {(int)c.x, (int)c.y, (int)c.z, (int)c.w};
    int above = total - incl;  // the keys of the digits above this lane's four
    int hit = -1, hit_above = 0;
#pragma unroll
    for (int b = 3; b >= 0; --b) {
        if (hit < 0 && rank >= above && rank < (long long)above + cc[b]) {
            hit = b;
            hit_above = above;
        }
        above += cc[b];
    }
    const unsigned long long m = __ballot(hit >= 0);
    if (m) {
        const int l = __builtin_ctzll(m);
        rank -= __builtin_amdgcn_readlane(hit_above, l);
        return 4 * l + __builtin_amdgcn_readlane(hit, l);
    }
    rank -= total - __builtin_amdgcn_readlane(cc[0], 0);
    return 0;
}

// Radix select of the top_k-th largest key, 8 bits per pass from the top.
// The state after p picks (the prefix of the high 8p bits and the rank inside
// it) is goss_sel[2p], goss_sel[2p + 1]; pass p's kernel takes pick p - 1
// from pass p - 1's histogram in every block (block 0 stores it), so no
// launch runs between passes. Each of kGossDigitBlocks blocks owns a
// contiguous range of rows. Passes 0 to 2 read every row's key; pass 2 also
// lists, in the block's own segment of goss_cand, the keys that match the
// 16-bit prefix (they are the only keys later passes count), and passes 3 to
// 7 read those lists.
__global__ __launch_bounds__(256) void k_goss_digits(DevState s, int pass) {
    __shared__ uint32_t hist[256];
    __shared__ unsigned long long s_prefix;
    __shared__ long long s_rank;
    __shared__ int s_nc;
    if (!goss_on(s)) return;
    hist[threadIdx.x] = 0u;
    if (threadIdx.x == 0) s_nc = 0;
    if (threadIdx.x < 64) {
        unsigned long long prefix = 0ULL;
        long long rank;
        if (pass == 0) {
            rank = (long long)s.goss_sel[1];
        } else {
            prefix = s.goss_sel[2 * (pass - 1)];
            rank = (long long)s.goss_sel[2 * (pass - 1) + 1];
            const int d = goss_pick_wave(s.goss_hist + (pass - 1) * kGossHistSlots * 256, rank);
            prefix |= (unsigned long long)d << (56 - 8 * (pass - 1));
        }
        if (threadIdx.x == 0) {
            s_prefix = prefix;
            s_rank = rank;
            if (blockIdx.x == 0 && pass > 0) {
                s.goss_sel[2 * pass] = prefix;
                s.goss_sel[2 * pass + 1] = (unsigned long long)rank;
            }
        }
    }
    __syncthreads();
    const unsigned long long prefix = s_prefix;
    const int shift = 56 - 8 * pass;
    const int64_t n = s.n;
    const int64_t seg = (n + kGossDigitBlocks - 1) / kGossDigitBlocks;
    const int64_t lo = (int64_t)blockIdx.x * seg;
    if (pass < 3) {
        const int64_t hi = lo + seg < n ? lo + seg : n;
        unsigned long long *cand = s.goss_cand + lo;
        // four keys per thread in flight; the trip count is block-uniform
        // (the candidate list's ballots need every lane)
        for (int64_t b0 = lo; b0 < hi; b0 += 4 * 256) {
            const int64_t r0 = b0 + threadIdx.x;
            unsigned long long key[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int64_t r = r0 + u * 256;
                key[u] = r < hi ? goss_key(s, r) : 0ULL;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const bool in = r0 + u * 256 < hi && (pass == 0 || (key[u] >> (shift + 8)) == (prefix >> (shift + 8)));
                if (in) atomicAdd(&hist[(key[u] >> shift) & 255u], 1u);
                if (pass == 2) {
                    const unsigned long long m = __ballot(in);
                    int at = 0;
                    if (lane_id() == 0 && m) at = atomicAdd(&s_nc, __popcll(m));
                    at = __shfl(at, 0, 64);
                    if (in) cand[at + __popcll(m & ((1ULL << lane_id()) - 1ULL))] = key[u];
                }
            }
        }
    } else {
        const int nc = s.goss_ccnt[blockIdx.x];
        const unsigned long long *cand = s.goss_cand + lo;
        for (int j0 = threadIdx.x; j0 < nc; j0 += 4 * 256) {
            unsigned long long key[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) key[u] = j0 + u * 256 < nc ? cand[j0 + u * 256] : 0ULL;
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (j0 + u * 256 < nc && (key[u] >> (shift + 8)) == (prefix >> (shift + 8)))
                    atomicAdd(&hist[(key[u] >> shift) & 255u], 1u);
        }
    }
    __syncthreads();
    const uint32_t v = hist[threadIdx.x];
    if (v) atomicAdd(&s.goss_hist[(pass * kGossHistSlots + (blockIdx.x & (kGossHistSlots - 1))) * 256 + threadIdx.x], v);
    if (pass == 2 && threadIdx.x == 0) s.goss_ccnt[blockIdx.x] = s_nc;
}

// The last pick: the threshold's low byte from pass 7's histogram.
__global__ void k_goss_pick(DevState s) {
    if (!goss_on(s) || threadIdx.x >= 64) return;
    unsigned long long prefix = s.goss_sel[14];
    long long rank = (long long)s.goss_sel[15];
    const int d = goss_pick_wave(s.goss_hist + 7 * kGossHistSlots * 256, rank);
    prefix |= (unsigned long long)d;
    if (threadIdx.x == 0) {
        GossState g = *s.gst;
        g.prefix = prefix;
        g.rank = rank;
        g.threshold = __longlong_as_double((long long)prefix);
        *s.gst = g;
    }
}

// Rows of the GOSS kernels below come in blocks of 1024: a workgroup of 256
// threads takes one, thread t the rows t, t + 256, t + 512 and t + 768 (each
// load instruction reads consecutive rows; four rows per thread in flight).
// Row j * 256 + w * 64 + lane of the block is slot j of lane `lane` of wave w.
constexpr int kGossRowThreads = 256;

__device__ __forceinline__ bool goss_top(const DevState &s, int64_t r, unsigned long long thr_bits) {
    return goss_key(s, r) >= thr_bits;
}

// The sampling's kept bit of row r (the 64-row word is the same for the
// whole wave: one broadcast load).
__device__ __forceinline__ bool goss_kept_bit(const DevState &s, int64_t r) {
    return (s.goss_mask[r >> 6] >> (r & 63)) & 1ULL;
}

// In-block exclusive prefix, in row order, of four flags per thread; returns
// the block's total. wc: 4 x 4 ints of LDS.
__device__ __forceinline__ int goss_block_prefix(const bool (&f)[4], int (&pre)[4], int (*wc)[4]) {
    const int lane = lane_id(), w = threadIdx.x >> 6;
    unsigned long long b[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) b[j] = __ballot(f[j]);
    if (lane == 0)
#pragma unroll
        for (int j = 0; j < 4; ++j) wc[j][w] = __popcll(b[j]);
    __syncthreads();
    const unsigned long long lt = (1ULL << lane) - 1ULL;
    int base = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        int tj = 0, bw = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = wc[j][i];
            tj += c;
            bw += i < w ? c : 0;
        }
        pre[j] = base + bw + __popcll(b[j] & lt);
        base += tj;
    }
    return base;
}

// The block's count of four flags per thread (thread 0 gets it).
__device__ __forceinline__ int goss_block_count(const bool (&f)[4], int *wc) {
    int c = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) c += __popcll(__ballot(f[j]));
    if (lane_id() == 0) wc[threadIdx.x >> 6] = c;
    __syncthreads();
    return wc[0] + wc[1] + wc[2] + wc[3];
}

// Per block of 1024 rows: count of top rows (mode 0), of rows in the sample
// (mode 1) or of rows kept by the sampling (mode 2).
__global__ __launch_bounds__(kGossRowThreads) void k_goss_count(DevState s, int mode) {
    __shared__ int wc[4];
    if (!goss_on(s)) return;
    const int64_t n = s.n, r0 = (int64_t)blockIdx.x * 1024 + threadIdx.x;
    const unsigned long long thr = mode == 0 ? (unsigned long long)__double_as_longlong(s.gst->threshold) : 0ULL;
    bool in[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t r = r0 + j * 256;
        in[j] = false;
        if (r < n) {
            if (mode == 0) {
                in[j] = goss_top(s, r, thr);
            } else {
                const bool other = goss_kept_bit(s, r);
                // a top row: its bit of k_goss_count(0)'s words (its kappa is INT_MIN)
                in[j] = mode == 2 ? other : (((s.goss_topmask[r >> 6] >> (r & 63)) & 1ULL) != 0 || other);
            }
        }
    }
    if (mode == 0) {
        // the top rows' bits, for the kappa pass (it need not read the
        // derivatives again): slot j of the wave's lanes is one 64-row word
        const int lane = lane_id(), w = threadIdx.x >> 6;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const unsigned long long m = __ballot(in[j]);
            const int64_t rw = (int64_t)blockIdx.x * 1024 + j * 256 + w * 64;
            if (lane == 0 && rw < n) s.goss_topmask[rw >> 6] = m;
        }
    }
    const int t = goss_block_count(in, wc);
    if (threadIdx.x == 0) s.goss_blk[blockIdx.x] = t;
}

// Exclusive prefix of per-block counts, in place (one block); the total
// goes to *total when given.
// blk2, total2: a second array scanned by block 1 of a two-block launch.
__global__ __launch_bounds__(1024) void k_goss_scan(DevState s, int32_t *blk, int64_t *total, int32_t *blk2,
                                                    int64_t *total2) {
    __shared__ long long wtot[16];
    if (!goss_on(s)) return;
    if (blockIdx.x == 1) {
        blk = blk2;
        total = total2;
    }
    const int nb = s.goss_nblk;
    // a thread's run of `per` counts, kC loads in flight at a time (the
    // runs of up to 16M rows' blocks are one round of loads); the counts of
    // the first kC stay in registers for the write-back
    constexpr int kC = 16;
    const int per = (nb + 1023) / 1024;
    const int lo = threadIdx.x * per;
    const int hi = lo + per < nb ? lo + per : nb;
    long long sum = 0;
    int v0[kC];
#pragma unroll
    for (int u = 0; u < kC; ++u) v0[u] = lo + u < hi ? blk[lo + u] : 0;
#pragma unroll
    for (int u = 0; u < kC; ++u) sum += v0[u];
    for (int c = lo + kC; c < hi; c += kC) {
        int v[kC];
#pragma unroll
        for (int u = 0; u < kC; ++u) v[u] = c + u < hi ? blk[c + u] : 0;
#pragma unroll
        for (int u = 0; u < kC; ++u) sum += v[u];
    }
    const int lane = lane_id(), w = threadIdx.x >> 6;
    const long long inc = wave_incl_scan(sum);
    if (lane == 63) wtot[w] = inc;
    __syncthreads();
    long long before = 0;
    for (int i = 0; i < w; ++i) before += wtot[i];
    if (total != nullptr && threadIdx.x == 1023) *total = before + inc;
    long long acc = before + inc - sum;
#pragma unroll
    for (int u = 0; u < kC; ++u) {
        if (lo + u < hi) blk[lo + u] = (int32_t)acc;
        acc += v0[u];
    }
    for (int c = lo + kC; c < hi; c += kC) {
        int v[kC];
#pragma unroll
        for (int u = 0; u < kC; ++u) v[u] = c + u < hi ? blk[c + u] : 0;
#pragma unroll
        for (int u = 0; u < kC; ++u) {
            if (c + u < hi) blk[c + u] = (int32_t)acc;
            acc += v[u];
        }
    }
}

// u < a / rest in binary64 (a = K - count and rest exact integers), as the
// reference compares the draw with the keep probability: the sign of
// u rest - a is exact from one fma (u rest - a is a multiple of 2^-53), so
// the rounded quotient is computed only when u lies within a few of its ulps.
__device__ __forceinline__ bool goss_keep(double u, double a, double rest) {
    const double e = fma(u, rest, -a);
    if (e >= 0.0) return false;        // u >= a / rest: the rounded quotient is at most u
    if (e < -a * 0x1p-50) return true;  // below the quotient by more than its rounding
    return u < a / rest;
}

// kappa of every row, then its class against a predicted band of the count:
// before row r the count is expected at K (1 - rest_r / N) (selection
// sampling takes a uniform K-subset of the N = n - top_k other rows) with a
// hypergeometric standard deviation sigma_r; with D = band * sigma_r + 64, a
// row with kappa > expected + D is kept and one with kappa <= expected - D
// dropped if the count stays inside the band, which the check after the
// count verifies; the rows in between are left to the sequential count.
// Class (in goss_other): 0 dropped, 1 kept, 2 open. Kept rows' bits go to
// goss_mask; per block the kept (goss_blk) and open (goss_blk_u) counts.
__global__ __launch_bounds__(kGossRowThreads) void k_goss_kappa(DevState s) {
    __shared__ int wc[4][4], wk[4], wu[4];
    if (!goss_on(s)) return;
    const GossState g = *s.gst;
    const int64_t n = s.n;
    const int64_t r0 = (int64_t)blockIdx.x * 1024 + threadIdx.x;
    const int lane = lane_id(), w = threadIdx.x >> 6;
    const int64_t top_before_blk = s.goss_blk[blockIdx.x];
    bool top[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t r = r0 + j * 256;
        const int64_t rw = (int64_t)blockIdx.x * 1024 + j * 256 + w * 64;
        top[j] = r < n && ((s.goss_topmask[rw >> 6] >> lane) & 1ULL);  // k_goss_count(0)'s bits
    }
    int pre[4];
    goss_block_prefix(top, pre, wc);
    const uint64_t stream = splitmix64((uint64_t)(s.hp.goss_seed & 0x7FFFFFFFFFFFFFFFLL) ^
                                       ((uint64_t)s.round->round * kGolden));
    const int64_t K = g.other_k;
    const double N = (double)(n - g.top_k);
    const double inv_n = N > 0.0 ? 1.0 / N : 0.0;
    const double cvar = N > 1.0 ? (double)K * (N - (double)K) / (N - 1.0) : 0.0;
    int nk = 0, nu = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t r = r0 + j * 256;
        int cls = 0;
        if (r < n && !top[j]) {
            const int64_t n_top = top_before_blk + pre[j];
            const int64_t rest = (n - r) - (g.top_k - n_top);
            int64_t kappa;
            if (rest <= 0) {
                kappa = K;  // the reference keeps the row iff rows are still needed
            } else {
                const double u = uniform53(stream + (uint64_t)r);
                const double drest = (double)rest;
                auto keep = [&](int64_t cnt) { return goss_keep(u, (double)(K - cnt), drest); };
                int64_t c = (int64_t)floor((double)K - u * (double)rest);
                if (c < 0) c = 0;
                if (c > K) c = K;
                while (c > 0 && !keep(c - 1)) --c;
                while (c < K && keep(c)) ++c;
                kappa = c;
            }
            s.goss_kappa[r] = (int32_t)kappa;
            // the band needs no exact rounding (the check decides)
            double f = N > 0.0 ? 1.0 - (double)(rest > 0 ? rest : 0) * inv_n : 1.0;
            f = f < 0.0 ? 0.0 : (f > 1.0 ? 1.0 : f);
            const double expect = (double)K * f;
            const double var = cvar * f * (1.0 - f);
            const double d = s.hp.goss_band * (double)sqrtf((float)(var > 0.0 ? var : 0.0)) + 64.0;
            cls = (double)kappa > expect + d ? 1 : ((double)kappa <= expect - d ? 0 : 2);
        } else if (r < n) {
            s.goss_kappa[r] = INT_MIN;
        }
        if (r < n) s.goss_other[r] = (uint8_t)cls;
        const unsigned long long km = __ballot(cls == 1), um = __ballot(cls == 2);
        const int64_t rw = (int64_t)blockIdx.x * 1024 + j * 256 + w * 64;
        if (lane == 0 && rw < n) s.goss_mask[rw >> 6] = km;
        nk += __popcll(km);
        nu += __popcll(um);
    }
    if (lane == 0) {
        wk[w] = nk;
        wu[w] = nu;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        s.goss_blk[blockIdx.x] = wk[0] + wk[1] + wk[2] + wk[3];
        s.goss_blk_u[blockIdx.x] = wu[0] + wu[1] + wu[2] + wu[3];
    }
}

// The open rows in row order, each with its kappa less the kept rows before
// it, which turns their decisions into the same sequential count.
__global__ __launch_bounds__(kGossRowThreads) void k_goss_compact(DevState s) {
    __shared__ int wk[4][4], wu[4][4];
    if (!goss_on(s)) return;
    const int64_t n = s.n;
    const int64_t r0 = (int64_t)blockIdx.x * 1024 + threadIdx.x;
    int cls[4];
    bool fk[4], fu[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t r = r0 + j * 256;
        cls[j] = r < n ? (int)s.goss_other[r] : 0;
        fk[j] = cls[j] == 1;
        fu[j] = cls[j] == 2;
    }
    int pk[4], pu[4];
    goss_block_prefix(fk, pk, wk);
    goss_block_prefix(fu, pu, wu);
    const int64_t kb = s.goss_blk[blockIdx.x], ub = s.goss_blk_u[blockIdx.x];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (fu[j]) {
            const int64_t r = r0 + j * 256;
            const int64_t pos = ub + pu[j];
            s.goss_ukappa[pos] = (int32_t)((int64_t)s.goss_kappa[r] - (kb + pk[j]));
            s.goss_urow[pos] = (int32_t)r;
        }
}

// Decisions of the open rows into goss_mask.
__global__ __launch_bounds__(256) void k_goss_apply(DevState s) {
    if (!goss_on(s)) return;
    const int64_t u = s.gst->n_uncertain;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < u; j += stride)
        if ((s.goss_umask[j >> 6] >> (j & 63)) & 1ULL) {
            const int32_t r = s.goss_urow[j];
            atomicOr(&s.goss_mask[r >> 6], 1ULL << (r & 63));
        }
}

// The check: the sequential count keeps row r iff the rows it kept before r
// number less than kappa_r, so kept flags that satisfy this at every row are
// its result. goss_blk holds the exclusive prefix of kept rows per block.
__global__ __launch_bounds__(kGossRowThreads) void k_goss_verify(DevState s) {
    __shared__ int wc[4][4];
    if (!goss_on(s)) return;
    const int64_t n = s.n;
    const int64_t r0 = (int64_t)blockIdx.x * 1024 + threadIdx.x;
    bool kept[4];
    int32_t k[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t r = r0 + j * 256;
        kept[j] = r < n && goss_kept_bit(s, r);
        k[j] = r < n ? s.goss_kappa[r] : 0;
    }
    int pre[4];
    goss_block_prefix(kept, pre, wc);
    const int64_t kb = s.goss_blk[blockIdx.x];
    bool bad = false;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (r0 + j * 256 < n) bad |= (kb + pre[j] < (int64_t)k[j]) != kept[j];
    if (__ballot(bad) && lane_id() == 0) atomicOr(&s.gst->fallback, 1);
}

// One 64-row slice of the count: rows whose kappa exceeds the count by 64 or
// more are kept and rows whose kappa is at most the count dropped whatever
// the slice's other rows do; the rest are resolved in row order.
__device__ __forceinline__ unsigned long long goss_slice(int k, int &cnt) {
    const unsigned long long a = __ballot(k > cnt + 63);
    const unsigned long long z = __ballot(k <= cnt);
    unsigned long long kept = a, amb = ~(a | z);
    while (amb) {
        const int i = __builtin_ctzll(amb);
        amb &= amb - 1ULL;
        const int ki = __builtin_amdgcn_readlane(k, i);
        if (cnt + __popcll(kept & ((1ULL << i) - 1ULL)) < ki) kept |= 1ULL << i;
    }
    cnt += __popcll(kept);
    return kept;
}

constexpr int kGossTile = kGossTileRows;

// One block; wave 0 runs the count while the other 15 waves stage kappa
// tiles into LDS, one tile ahead through registers: in the iteration that
// wave 0 walks tile t, they store tile t + 1 (loaded during the previous
// iteration) and issue the loads of tile t + 2. The kappa buffer is padded to
// whole tiles with INT_MIN (never kept). The count advances 256 rows per
// step when every kappa of the step is above count + 255 or at most the
// count (always true but for rows whose draw falls within 256 of the
// boundary), else by 64-row slices.
constexpr int kGossStep = 256;
constexpr int kGossVec = kGossTile / 4;       // int4 per tile
constexpr int kGossStagers = 1024 - 64;
constexpr int kGossSlots = (kGossVec + kGossStagers - 1) / kGossStagers;

__device__ __forceinline__ int4 goss_clip(int4 v, int64_t e, int64_t len) {
    v.x = e < len ? v.x : INT_MIN;
    v.y = e + 1 < len ? v.y : INT_MIN;
    v.z = e + 2 < len ? v.z : INT_MIN;
    v.w = e + 3 < len ? v.w : INT_MIN;
    return v;
}

// list = 1: the count over the open rows (goss_ukappa -> goss_umask);
// list = 0: the full count over every row (goss_kappa -> goss_mask), run
// only when the band's decisions failed the check or were not used.
__global__ __launch_bounds__(1024) void k_goss_walk(DevState s, int list) {
    extern __shared__ int32_t gbuf[];  // 2 x kGossTile
    if (!goss_on(s)) return;
    if (!list && !s.gst->fallback) return;
    const int64_t n = list ? s.gst->n_uncertain : s.n;
    if (n <= 0) return;
    unsigned long long *out = list ? s.goss_umask : s.goss_mask;
    const int64_t n_words = (n + 63) / 64;
    const int lane = lane_id(), w = threadIdx.x >> 6;
    const int64_t tiles = (n + kGossTile - 1) / kGossTile;
    const int4 *kv = (const int4 *)(list ? s.goss_ukappa : s.goss_kappa);
    for (int i = threadIdx.x; i < kGossVec; i += blockDim.x) ((int4 *)gbuf)[i] = goss_clip(kv[i], 4 * i, n);
    // the stagers' registers: slot j holds int4 sid + j * kGossStagers of a tile
    static_assert(kGossSlots == 5, "staging slots are written out below");
    const int sid = (int)threadIdx.x - 64;
    const bool last_slot = sid + 4 * kGossStagers < kGossVec;
    int4 r0, r1, r2, r3, r4;
#define MB_GOSS_LOAD(tile)                                                       \
    do {                                                                         \
        const int64_t e_ = ((int64_t)(tile) * kGossVec + sid) * 4;               \
        const int4 *src_ = kv + (int64_t)(tile) * kGossVec + sid;                \
        r0 = goss_clip(src_[0], e_, n);                                          \
        r1 = goss_clip(src_[kGossStagers], e_ + 4 * kGossStagers, n);            \
        r2 = goss_clip(src_[2 * kGossStagers], e_ + 8 * kGossStagers, n);        \
        r3 = goss_clip(src_[3 * kGossStagers], e_ + 12 * kGossStagers, n);       \
        if (last_slot) r4 = goss_clip(src_[4 * kGossStagers], e_ + 16 * kGossStagers, n); \
    } while (0)
    if (w != 0 && tiles > 1) MB_GOSS_LOAD(1);
    __syncthreads();
    int cnt = 0;
    for (int64_t t = 0; t < tiles; ++t) {
        const int32_t *cur = gbuf + (t & 1) * kGossTile;
        if (w != 0) {
            if (t + 1 < tiles) {
                int4 *dst = (int4 *)(gbuf + ((t + 1) & 1) * kGossTile) + sid;
                dst[0] = r0;
                dst[kGossStagers] = r1;
                dst[2 * kGossStagers] = r2;
                dst[3 * kGossStagers] = r3;
                if (last_slot) dst[4 * kGossStagers] = r4;
            }
            if (t + 2 < tiles) MB_GOSS_LOAD(t + 2);
        }
        if (w == 0) {
            const int64_t base = t * kGossTile;
            int k0 = cur[lane], k1 = cur[64 + lane], k2 = cur[128 + lane], k3 = cur[192 + lane];
            for (int st = 0; st < kGossTile / kGossStep; ++st) {
                const int64_t row0 = base + (int64_t)st * kGossStep;
                if (row0 >= n) break;
                // the next step's kappas do not depend on the count
                const int o = st + 1 < kGossTile / kGossStep ? (st + 1) * kGossStep : 0;
                const int n0 = cur[o + lane], n1 = cur[o + 64 + lane], n2 = cur[o + 128 + lane],
                          n3 = cur[o + 192 + lane];
                unsigned long long m0, m1, m2, m3;
                bool whole = false;
                if (!list) {  // launch-uniform
                    // the whole step at once when no kappa lies within
                    // 256 above the count (the open rows' kappas, within
                    // the band around the count, almost never allow it)
                    const int hi = cnt + kGossStep - 1;
                    const unsigned long long a0 = __ballot(k0 > hi), a1 = __ballot(k1 > hi),
                                             a2 = __ballot(k2 > hi), a3 = __ballot(k3 > hi);
                    const unsigned long long z0 = __ballot(k0 <= cnt), z1 = __ballot(k1 <= cnt),
                                             z2 = __ballot(k2 <= cnt), z3 = __ballot(k3 <= cnt);
                    whole = ((a0 | z0) & (a1 | z1) & (a2 | z2) & (a3 | z3)) == ~0ULL;
                    m0 = a0;
                    m1 = a1;
                    m2 = a2;
                    m3 = a3;
                    if (whole) cnt += __popcll(a0) + __popcll(a1) + __popcll(a2) + __popcll(a3);
                }
                if (!whole) {
                    m0 = goss_slice(k0, cnt);
                    m1 = goss_slice(k1, cnt);
                    m2 = goss_slice(k2, cnt);
                    m3 = goss_slice(k3, cnt);
                }
                const int64_t wd = (row0 >> 6) + lane;
                if (lane < 4 && wd < n_words)
                    out[wd] = lane == 0 ? m0 : lane == 1 ? m1 : lane == 2 ? m2 : m3;
                k0 = n0;
                k1 = n1;
                k2 = n2;
                k3 = n3;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0 && !list) s.gst->kept_other = cnt;
}
#undef MB_GOSS_LOAD

__global__ __launch_bounds__(kGossRowThreads) void k_goss_scatter(DevState s) {
    __shared__ int wc[4][4];
    if (!goss_on(s)) return;
    const int64_t n = s.n;
    const int64_t r0 = (int64_t)blockIdx.x * 1024 + threadIdx.x;
    bool in[4], other[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t r = r0 + j * 256;
        bool top = false;
        other[j] = false;
        if (r < n) {
            top = ((s.goss_topmask[r >> 6] >> (r & 63)) & 1ULL) != 0;  // its kappa is INT_MIN
            other[j] = !top && goss_kept_bit(s, r);
        }
        in[j] = top || other[j];
    }
    int pre[4];
    goss_block_prefix(in, pre, wc);
    const int64_t base = s.goss_blk[blockIdx.x];
    // one tree per round: the sample goes straight into the root's row list
    // (several class trees each copy it from goss_rows instead), and a kept
    // small-gradient row's weight bit into its interleaved hessian's sign bit
    const bool direct = s.hp.num_class == 1;
    int32_t *dst = direct ? s.rows0 : s.goss_rows;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t r = r0 + j * 256;
        if (r < n) {
            if (in[j]) dst[base + pre[j]] = (int32_t)r;
            s.goss_other[r] = other[j] ? 1 : 0;
            if (direct && other[j] && s.gh2) {
                uint32_t *hw = (uint32_t *)(s.gh2 + 2 * (size_t)r + 1);
                *hw = *hw | 0x80000000u;
            }
        }
    }
}

// max |g w| and |h w| over the round's sample, w the row's GOSS weight
// (goss_weight for a sampled small-importance row, else 1), in binary64 as
// apply_goss_scaling leaves the derivatives (goss.mojo:360-373); rows whose
// weighted derivatives are not finite add nothing (gradient_stats,
// quantized_gradient.mojo:762-810). Accumulated into goss_max[parity]; the
// quantizer reads it and clears the other pair for the next tree.
__global__ __launch_bounds__(256) void k_goss_stats(DevState s) {
    __shared__ double red_g[4], red_h[4];
    if (!goss_on(s) || !s.hp.quantized) return;
    const GossState g = *s.gst;
    const double mult = goss_weight(g, s.n);
    const int parity = s.round->parity;
    double mg = 0.0, mh = 0.0;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < g.bag_n; j += stride) {
        const int32_t r = (s.hp.num_class == 1 ? s.rows0 : s.goss_rows)[j];
        const double m = s.goss_other[r] ? mult : 1.0;
        const double ag = fabs((double)s.grad[r] * m), ah = fabs((double)s.hess[r] * m);
        if (isfinite(ag) && isfinite(ah)) {
            mg = fmax(mg, ag);
            mh = fmax(mh, ah);
        }
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        mg = fmax(mg, __shfl_xor(mg, d, 64));
        mh = fmax(mh, __shfl_xor(mh, d, 64));
    }
    const int w = threadIdx.x >> 6;
    if (lane_id() == 0) {
        red_g[w] = mg;
        red_h[w] = mh;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < (int)(blockDim.x >> 6); ++i) {
            mg = fmax(mg, red_g[i]);
            mh = fmax(mh, red_h[i]);
        }
        // non-negative doubles order like their bit patterns
        atomicMax(&s.goss_max[parity * 2 + 0], (unsigned long long)__double_as_longlong(mg));
        atomicMax(&s.goss_max[parity * 2 + 1], (unsigned long long)__double_as_longlong(mh));
    }
}

// --------------------------------------------------------------- histogram
// Rows of the root build handled by each block. The scan kernel recomputes it
// to know how many block partials the build left.
__device__ __forceinline__ int64_t hist_chunk(const DevState &s, int64_t m) {
    const int64_t g = s.hist_grid;
    int64_t chunk = (m + g - 1) / g;
    if (chunk < s.hist_chunk_min) chunk = s.hist_chunk_min;
    if (chunk > s.hist_chunk_limit) chunk = s.hist_chunk_limit;
    return chunk;
}

__device__ __forceinline__ int64_t root_rows(const DevState &s) {
    return s.round->sampled ? load_agent(&s.cursor[0]) : s.n;
}

// Block-private LDS histograms, two kinds.
//
// QAcc (quantized gradients): one packed 64-bit counter per cell -- count in
// bits [0,20), hess sum in [20,42), grad sum (signed) in [42,64) -- so a row
// costs one ds_add_u64 per feature; the int8 pair travels in the record's
// last two bytes. Adding packed values adds the three fields while no field
// overflows, which hist_chunk_limit guarantees for the lattice in use
// (host-checked): a block never packs more rows than that.
//
// FAcc (fp32 gradients): fp64 grad and hess sums (ds_add_f64) and a uint32
// count per cell, summing the fp32 gradient values exactly as the
// reference's Float64 histograms do (histogram.mojo:1002); only the order of
// the additions differs.
// Bytes of a row's record in a tile of tf features: the tile's bins, zero
// pad, the g/h pair in the last two bytes, rounded up to a power of two.
__host__ __device__ constexpr int record_bytes_for(int tf) {
    int r = 16;
    while (r < tf + 2) r *= 2;
    return r;
}

// A lane's 16-byte record slice (dwords d0..d3) rotated right by rot bytes:
// byte k of the result is byte (k + rot) mod 16 of the slice. The histogram
// kinds with bin-major cells give each lane rot = (lane mod 16) xor (bit 4
// of lane), so at every step the lanes of a wave take different byte
// positions.
__device__ __forceinline__ void rotate_slice(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3, uint32_t rot,
                                             uint32_t (&r)[4]) {
    if (rot & 4u) {  // one dword
        const uint32_t t = d0;
        d0 = d1;
        d1 = d2;
        d2 = d3;
        d3 = t;
    }
    if (rot & 8u) {  // two dwords
        uint32_t t = d0;
        d0 = d2;
        d2 = t;
        t = d1;
        d1 = d3;
        d3 = t;
    }
    const uint32_t sh = rot & 3u;
    r[0] = __builtin_amdgcn_alignbyte(d1, d0, sh);
    r[1] = __builtin_amdgcn_alignbyte(d2, d1, sh);
    r[2] = __builtin_amdgcn_alignbyte(d3, d2, sh);
    r[3] = __builtin_amdgcn_alignbyte(d0, d3, sh);
}

struct QAcc {
    // LDS cells are bin-major: cell (byte position p of the record, bin) at
    // bin * FS + p, FS = max(32, record bytes). A 64-bit cell's banks then
    // depend on p alone, whatever the bin, and add() has the lanes of a wave
    // take different byte positions at each step, so a step's 64 atomics
    // meet no bank conflict (measured: random bins cost twice the LDS cycles
    // of this layout). Every byte of the record is
    // added, unconditionally: the pad and g/h positions land in bin-0 cells
    // that the store never reads.
    static __host__ __device__ constexpr int row_cells_for(int rec) { return rec < 32 ? 32 : rec; }
    static __host__ __device__ size_t lds_bytes(int tf, int ls) {
        return (size_t)row_cells_for(record_bytes_for(tf)) * ls * 8;
    }
    template <int LPR>
    __device__ static void zero(unsigned char *lds, int, int ls) {
        constexpr int FS = row_cells_for(LPR * 16);
        unsigned long long *a = (unsigned long long *)lds;
        for (int i = threadIdx.x; i < FS * ls; i += blockDim.x) a[i] = 0ULL;
    }
    // one record slice (this lane's 16 bytes: positions sub*16 ..). The slice
    // is rotated right by rot bytes, so step k adds position
    // sub*16 + (k + rot) mod 16, with rot = (lane mod 16) xor (bit 4 of
    // lane): the 16 lanes of a quarter-wave take 16 different positions
    // mod 16 (no conflict when the LDS serves a 64-bit op 16 lanes at a time
    // over 32 banks), and the 32 lanes of a half-wave 32 different positions
    // mod 32 (none when it serves 32 lanes over 64 banks), for LPR >= 2.
    template <int LPR>
    __device__ static void add(unsigned char *lds, const DevState &, const uint4 &w, int sub, int, int, int64_t,
                               uint32_t gh_word, double) {
        constexpr int FS = row_cells_for(LPR * 16);
        constexpr int kRowShift = FS == 32 ? 8 : FS == 64 ? 9 : 10;  // log2(FS * 8 bytes)
        static_assert(FS * 8 == (1 << kRowShift), "row of a power-of-two size");
        const int g = (int)(int8_t)(gh_word >> 16);
        const int h = (int)(int8_t)(gh_word >> 24);
        const unsigned long long packed =
            (unsigned long long)(((long long)g << 42) + ((long long)h << 20) + 1LL);
        const uint32_t rot = ((uint32_t)lane_id() & 15u) ^ (((uint32_t)lane_id() >> 4) & 1u);
        // the g/h bytes are added as bin 0 (any bin id must be below the LDS
        // rows, n_bins); pad bytes are zero
        uint32_t r[4];
        rotate_slice(w.x, w.y, w.z, sub == LPR - 1 ? w.w & 0xFFFFu : w.w, rot, r);
        const uint32_t pb = (uint32_t)sub * 128u;  // byte offset of position sub*16
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const uint32_t p8 = pb | ((((uint32_t)k + rot) & 15u) << 3);
            const uint32_t bin = (r[k >> 2] >> (8 * (k & 3))) & 255u;
            atomicAdd((unsigned long long *)(lds + ((bin << kRowShift) | p8)), packed);
        }
    }
    // every cell of the block's histogram as its partial (feature-major:
    // features [f0, f0 + Ft) of partial blk). A lane reads four bins of one
    // feature (the lanes of a wave spread over 32 positions, two per bank
    // pair) and writes them as 32 contiguous bytes.
    template <int LPR>
    __device__ static void store(const DevState &s, const unsigned char *lds, int blk, int f0, int Ft) {
        constexpr int FS = row_cells_for(LPR * 16);
        const unsigned long long *a = (const unsigned long long *)lds;
        const int F = s.n_features, nb = s.n_bins, ps = s.part_stride;
        unsigned long long *out = s.part + ((size_t)blk * F + f0) * ps;
        const int nq = (ps + 3) >> 2;
        for (int u = threadIdx.x; u < FS * nq; u += blockDim.x) {
            const int q = u / FS;
            const int f = u - q * FS;
            if (f >= Ft) continue;
            const int b = 4 * q;
            unsigned long long v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = b + i < nb ? a[(b + i) * FS + f] : 0ULL;
            ulonglong2 *o = (ulonglong2 *)(out + (size_t)f * ps + b);  // ps is even: 16-byte aligned
            o[0] = make_ulonglong2(v[0], v[1]);
            if (b + 2 < ps) o[1] = make_ulonglong2(v[2], v[3]);
        }
    }
};

struct FAcc {
    // grad and hess cells bin-major, as QAcc's: cell (byte position p, bin)
    // at bin * FS + p, FS = max(32, record bytes), so a binary64 cell's banks
    // depend on p alone and, with QAcc's lane rotation, a step's 64 adds
    // meet no bank conflict (feature-major cells lost a third of the LDS
    // cycles to conflicts); positions past the tile's features are skipped.
    // The counts of two neighbouring bins share a 32-bit cell (bin b in its
    // half b & 1, 16 bits each), bin-pair-major at (b >> 1) * FS + p: a
    // cell's bank is p plus 32 times one bit of the bin, so the 32 lanes of
    // a half-wave, at 32 different positions, meet no conflict either
    // (feature-major 32-bit counts, whose banks follow the random bins, cost
    // 43 % of the accumulation's LDS cycles in conflicts), and the pairs
    // fit beside the sums in one workgroup's LDS. A block adds at most
    // kFAccChunk rows, so no half overflows.
    static __host__ __device__ int count_rows(int ls) { return (ls + 1) / 2; }
    static __host__ __device__ size_t lds_bytes(int tf, int ls) {
        const int FS = QAcc::row_cells_for(record_bytes_for(tf));
        return (size_t)2 * FS * ls * 8 + (size_t)count_rows(ls) * FS * 4;
    }
    template <int LPR>
    __device__ static void zero(unsigned char *lds, int, int ls) {
        constexpr int FS = QAcc::row_cells_for(LPR * 16);
        double *g = (double *)lds;
        uint32_t *c = (uint32_t *)(g + 2 * (size_t)FS * ls);
        for (int i = threadIdx.x; i < 2 * FS * ls; i += blockDim.x) g[i] = 0.0;
        for (int i = threadIdx.x; i < count_rows(ls) * FS; i += blockDim.x) c[i] = 0u;
    }
    // gv, hv: the row's derivatives in binary64 with its GOSS weight applied
    // (accumulate_rows loads them with the record)
    template <int LPR>
    __device__ static void add(unsigned char *lds, const uint4 &w, int sub, int F, int ls, double gv, double hv) {
        constexpr int FS = QAcc::row_cells_for(LPR * 16);
        double *g = (double *)lds;
        double *h = g + (size_t)FS * ls;
        uint32_t *c = (uint32_t *)(h + (size_t)FS * ls);
        const uint32_t rot = ((uint32_t)lane_id() & 15u) ^ (((uint32_t)lane_id() >> 4) & 1u);
        uint32_t r[4];
        rotate_slice(w.x, w.y, w.z, w.w, rot, r);
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int p = sub * 16 + (int)(((uint32_t)k + rot) & 15u);
            const int bin = (int)((r[k >> 2] >> (8 * (k & 3))) & 255u);
            if (p < F) {
                atomicAdd(&g[bin * FS + p], gv);
                atomicAdd(&h[bin * FS + p], hv);
                atomicAdd(&c[(bin >> 1) * FS + p], (bin & 1) ? 0x10000u : 1u);
            }
        }
    }
    // every cell of the block's histogram as its partial (feature-major), as
    // QAcc::store: a lane takes four bins of one position, so the lanes of
    // a wave read 32 consecutive positions of a bin row (conflict-free; a
    // lane per bin of one feature read cells FS apart, all on one bank), and
    // writes them as contiguous runs.
    template <int LPR>
    __device__ static void store(const DevState &s, const unsigned char *lds, int blk, int f0, int Ft) {
        constexpr int FS = QAcc::row_cells_for(LPR * 16);
        const int F = s.n_features, nb = s.n_bins, ls = s.lds_stride, ps = s.part_stride;
        const double *g = (const double *)lds;
        const double *h = g + (size_t)FS * ls;
        const uint32_t *c = (const uint32_t *)(h + (size_t)FS * ls);
        const size_t base = ((size_t)blk * F + f0) * ps;
        const int nq = (ps + 3) >> 2;
        for (int u = threadIdx.x; u < FS * nq; u += blockDim.x) {
            const int q = u / FS;
            const int f = u - q * FS;
            if (f >= Ft) continue;
            const int b = 4 * q;
            double vg[4], vh[4];
            uint32_t vc[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bool in = b + i < nb;
                vg[i] = in ? g[(b + i) * FS + f] : 0.0;
                vh[i] = in ? h[(b + i) * FS + f] : 0.0;
                vc[i] = in ? (c[((b + i) >> 1) * FS + f] >> (16 * ((b + i) & 1))) & 0xFFFFu : 0u;
            }
            const size_t o = base + (size_t)f * ps + b;  // ps is even: 16-byte aligned pairs
            *(double2 *)(s.fpart_g + o) = make_double2(vg[0], vg[1]);
            *(double2 *)(s.fpart_h + o) = make_double2(vh[0], vh[1]);
            *(uint2 *)(s.fpart_c + o) = make_uint2(vc[0], vc[1]);
            if (b + 2 < ps) {
                *(double2 *)(s.fpart_g + o + 2) = make_double2(vg[2], vg[3]);
                *(double2 *)(s.fpart_h + o + 2) = make_double2(vh[2], vh[3]);
                *(uint2 *)(s.fpart_c + o + 2) = make_uint2(vc[2], vc[3]);
            }
        }
    }
};

// WAcc (the magnitude-sum lattice): each row's int32 (grad, hess) pair from
// `gq`, gathered by row id -- or, with int16 staging (K16), the int16 pair in
// the record's last four bytes, which the row's lanes already hold; per cell
// one 64-bit LDS add of the packed pair --
// hess in the low 32 bits (nonnegative, a cell's sum below 2^32), signed grad
// in the high 32 -- and one 32-bit count. Any subset of a round's rows sums
// to at most 2^30 + n in magnitude on this lattice (quantized_gradient.mojo:
// 908-1117, the headroom argument), so neither field overflows and no carry
// crosses from hess into grad, whatever the block's row count.
template <bool K16>
struct WAccT {
    static __host__ __device__ size_t lds_bytes(int F, int ls) { return (size_t)F * ls * 12; }
    template <int LPR>
    __device__ static void zero(unsigned char *lds, int F, int ls) {
        unsigned long long *gh = (unsigned long long *)lds;
        uint32_t *c = (uint32_t *)(gh + (size_t)F * ls);
        for (int i = threadIdx.x; i < F * ls; i += blockDim.x) {
            gh[i] = 0ULL;
            c[i] = 0u;
        }
    }
    template <int LPR>
    __device__ static void add(unsigned char *lds, const DevState &s, const uint4 &w, int sub, int F, int ls,
                               int64_t row, uint32_t gh_word, double) {
        unsigned long long *gh = (unsigned long long *)lds;
        uint32_t *c = (uint32_t *)(gh + (size_t)F * ls);
        int2 q;
        if constexpr (K16) q = make_int2((int)(int16_t)(gh_word & 0xFFFFu), (int)(int16_t)(gh_word >> 16));
        else q = *(const int2 *)(s.gq + 2 * row);
        const unsigned long long packed = ((unsigned long long)(uint32_t)q.x << 32) | (uint32_t)q.y;
        const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int f = sub * 16 + k * 4 + j;
                if (f < F) {
                    const int cell = f * ls + (int)((d[k] >> (8 * j)) & 255u);
                    atomicAdd(&gh[cell], packed);
                    atomicAdd(&c[cell], 1u);
                }
            }
    }
    template <int LPR>
    __device__ static void store(const DevState &s, const unsigned char *lds, int blk, int f0, int Ft) {
        const int F = s.n_features, nb = s.n_bins, ls = s.lds_stride, ps = s.part_stride;
        const unsigned long long *gh = (const unsigned long long *)lds;
        const uint32_t *c = (const uint32_t *)(gh + (size_t)Ft * ls);
        const size_t base = ((size_t)blk * F + f0) * ps;
        for (int i = threadIdx.x; i < Ft * ps; i += blockDim.x) {
            const int f = i / ps;
            const int b = i - f * ps;
            const bool in = b < nb;
            s.part[base + i] = in ? gh[f * ls + b] : 0ULL;
            s.part_c[base + i] = in ? c[f * ls + b] : 0u;
        }
    }
};

using WAcc = WAccT<false>;
using WAcc16 = WAccT<true>;

// Root histogram, accumulation pass. Rows are split into contiguous chunks,
// one per block; a block accumulates its rows into its LDS histogram and
// stores it as its partial; the scan kernel merges the partials. A row's
// record is LPR x 16 bytes: each of the LPR lanes of a row group loads 16
// bytes (16 features) and the int8 g/h pair (the record's last two bytes)
// reaches the group by a lane shuffle. Each lane takes U rows per step.
// The root build (one pass over every row, 1024-thread blocks, one per CU)
// keeps 4 rows per step in flight (3 while it also quantizes: its extra
// loads). An expansion's accumulation takes 1: with the software pipelining
// of accumulate_rows (ids two steps ahead, records one step ahead) that is
// three loads per lane in flight at 50 VGPRs, so two 16-wave blocks fit a CU
// (4 rows per step took 92 VGPRs, one block per CU, and accumulated 13 %
// slower on C2). blockIdx.y is the feature tile: the block reads that
// tile's records and stores that tile's features of its partial.
constexpr int kRootUnroll = 4;
constexpr int kAccUnroll = 1;
#ifndef MB_ACC_UNROLL_F
#define MB_ACC_UNROLL_F 1
#endif
constexpr int kAccUnrollF = MB_ACC_UNROLL_F;

// The value of the last lane of each LPR-lane group, on every lane of the
// group, by DPP (a VALU operand modifier): unlike a crossbar shuffle it does
// not go through the LDS queue, so reading it never waits for the LDS
// atomics issued before it. LPR 2: quad_perm [1,1,3,3]; LPR 4: quad_perm
// [3,3,3,3]; LPR 8: that, then row_shl:4 into lane banks 0 and 2 (lanes
// 0-3 and 8-11 of each row take lanes 4-7 and 12-15).
template <int LPR>
__device__ __forceinline__ uint32_t group_last_lane(uint32_t x) {
    if constexpr (LPR == 1) {
        return x;
    } else if constexpr (LPR == 2) {
        return (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0xF5, 0xF, 0xF, false);
    } else {
        static_assert(LPR == 4 || LPR == 8, "records of 16, 32, 64 or 128 bytes");
        const int y = __builtin_amdgcn_update_dpp((int)x, (int)x, 0xFF, 0xF, 0xF, false);
        if constexpr (LPR == 4) return (uint32_t)y;
        else return (uint32_t)__builtin_amdgcn_update_dpp(y, y, 0x104, 0xF, 0x5, false);
    }
}

// Accumulates the records of rows [lo, hi) of a row list (kList), or of the
// rows lo .. hi - 1 themselves, into the block's LDS histogram:
// LPR lanes per row, each loading 16 bytes of the record, the g/h pair
// reaching the row's lanes by a shuffle. Loads are software-pipelined: while
// the records of step i are added into LDS, the records of step i + 1 and
// the row ids of step i + 2 are in flight. (The memory counter completes in
// issue order, so a step's ids must be issued a step before its records or
// waiting for them would also wait for every record load issued earlier.)
// kQ (the root build of the max-abs lattice): each row's int8 pair is
// quantized here from its derivatives (quant_row, the quantizer k_quantize
// would apply) instead of read from the record, and the row's record is
// written back with the pair in place, for the expansions' accumulations;
// rec_w is the record tile being read.
struct NoPre {
    __device__ void operator()() const {}
};
// pre: run by every thread once the first step's loads are in flight (and
// on an empty range): the caller's zeroing of the LDS histogram and its
// barrier, so they overlap the first records' latency.
template <int LPR, class Acc, bool kList, bool kQ, int U, class Pre = NoPre>
__device__ __forceinline__ void accumulate_rows(const DevState &s, unsigned char *lds, const int32_t *rows,
                                                int64_t lo, int64_t hi, int Ft, const uint4 *rec,
                                                double goss_mult, const QCtx *qc = nullptr, uint4 *rec_w = nullptr,
                                                Pre pre = Pre()) {
    const int ls = s.lds_stride;
    const int sub = threadIdx.x % LPR;
    const int rr = threadIdx.x / LPR;
    const int rpp = blockDim.x / LPR;
    const int64_t step = (int64_t)U * rpp;
    const uint32_t n32 = (uint32_t)s.n;  // n < 2^31
    if (lo >= hi) {
        pre();
        return;
    }
    // Every load is unconditional (an entry past the range loads the last
    // row again and is masked off when added): branches around loads would
    // make the compiler wait for every load in flight at each of them.
    auto load_ids = [&](int64_t i0, int32_t *id) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            int64_t i = i0 + (int64_t)u * rpp + rr;
            i = i < hi ? i : hi - 1;
            id[u] = kList ? rows[i] : (int32_t)i;
        }
    };
    // kQ: the value this lane quantizes (lane 0 of a row its gradient, lane 1
    // its hessian; one lane per row takes both) and the rows' GOSS weight
    // bits, loaded with the records
    float qv[U], qv2[U], qv_nxt[U], qv2_nxt[U];
    uint32_t qw = 0u, qw_nxt = 0u;
    const bool q_goss = kQ && qc->gs_on;
    // fp32 cells (FAcc): each row's derivatives (binary32 bits, or binary64
    // with grad64) and GOSS weight bit, loaded with the record a step ahead;
    // binary32 derivatives come as one interleaved (g, h) pair whose h sign
    // bit carries the GOSS weight bit (one gather per row, not three)
    constexpr bool kF = std::is_same<Acc, FAcc>::value;
    const bool f64 = kF && s.hp.grad64;
    const bool f_goss = kF && goss_mult != 1.0 && (f64 ? s.goss_other != nullptr : true);
    unsigned long long fg[U], fh[U], fg_nxt[U], fh_nxt[U];
    uint32_t fw = 0u, fw_nxt = 0u;
    auto load_recs = [&](int64_t, const int32_t *id, uint4 *w, float *v, float *v2, uint32_t &wb,
                         unsigned long long *xg, unsigned long long *xh, uint32_t &xw) {
        wb = 0u;
        xw = 0u;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t r = (uint32_t)id[u] < n32 ? (uint32_t)id[u] : 0u;  // ids come from the row lists
            w[u] = rec[(size_t)r * LPR + sub];
            if constexpr (kQ) {
                v[u] = (LPR == 1 || (sub & 1) == 0) ? s.grad[r] : s.hess[r];
                if constexpr (LPR == 1) v2[u] = s.hess[r];
                if (q_goss) wb |= (s.goss_other[r] ? 1u : 0u) << u;
            }
            if constexpr (kF) {
                if (f64) {
                    xg[u] = ((const unsigned long long *)s.grad64)[r];
                    xh[u] = ((const unsigned long long *)s.hess64)[r];
                    if (f_goss) xw |= (s.goss_other[r] ? 1u : 0u) << u;
                } else {
                    const uint2 gh = ((const uint2 *)s.gh2)[r];
                    xg[u] = gh.x;
                    xh[u] = gh.y;  // sign bit: the GOSS weight bit
                }
            }
        }
    };
    auto accumulate = [&](int64_t i0, const int32_t *id, const uint4 *w, const float *v, const float *v2,
                          uint32_t wb, const unsigned long long *xg, const unsigned long long *xh, uint32_t xw) {
        uint32_t gh[U];
        if constexpr (kQ) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int64_t i = i0 + (int64_t)u * rpp + rr;
                const uint32_t r = (uint32_t)id[u] < n32 ? (uint32_t)id[u] : 0u;
                int32_t qg, qh;
                const bool wt = (wb >> u) & 1u;
                if constexpr (LPR == 1) {
                    qg = quant_value(*qc, v[u], wt, (int64_t)r, true);
                    qh = quant_value(*qc, v2[u], wt, (int64_t)r, false);
                } else {
                    // the row's lane 0 quantizes g, lane 1 h, then both are
                    // read across the row's lanes
                    const int q = quant_value(*qc, v[u], wt, (int64_t)r, (sub & 1) == 0);
                    if constexpr (LPR == 2) {  // DPP, off the LDS queue the histogram atomics use
                        qg = __builtin_amdgcn_update_dpp(q, q, 0xA0, 0xF, 0xF, false);  // quad_perm [0,0,2,2]
                        qh = __builtin_amdgcn_update_dpp(q, q, 0xF5, 0xF, 0xF, false);  // quad_perm [1,1,3,3]
                    } else if constexpr (LPR == 4) {
                        qg = __builtin_amdgcn_update_dpp(q, q, 0x00, 0xF, 0xF, false);  // quad_perm [0,0,0,0]
                        qh = __builtin_amdgcn_update_dpp(q, q, 0x55, 0xF, 0xF, false);  // quad_perm [1,1,1,1]
                    } else {
                        const int base = (int)lane_id() & ~(LPR - 1);
                        qg = __shfl(q, base, 64);
                        qh = __shfl(q, base + 1, 64);
                    }
                }
                const uint32_t pair = (uint32_t)(uint8_t)(int8_t)qg | ((uint32_t)(uint8_t)(int8_t)qh << 8);
                uint4 v = w[u];
                if (sub == LPR - 1) v.w = (v.w & 0xFFFFu) | (pair << 16);
                // record partition: the pair goes to the pair plane (the
                // root's partition patches it into each record it moves);
                // otherwise every lane writes its 16 bytes back, so
                // consecutive rows rewrite whole 128-byte lines (no
                // partial-line update)
                if (s.rcp) {
                    if (i < hi && sub == LPR - 1) s.pairs[r] = (uint16_t)pair;
                } else if (i < hi) {
                    rec_w[(size_t)r * LPR + sub] = v;
                }
                gh[u] = group_last_lane<LPR>(v.w);
            }
        } else {
#pragma unroll
            for (int u = 0; u < U; ++u) gh[u] = group_last_lane<LPR>(w[u].w);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = i0 + (int64_t)u * rpp + rr;
            if constexpr (kF) {
                // goss.apply_goss_scaling: the sampled small-gradient rows'
                // g and h times the GOSS weight, in binary64
                double gv = f64 ? __longlong_as_double((long long)xg[u]) : (double)__uint_as_float((uint32_t)xg[u]);
                double hv = f64 ? __longlong_as_double((long long)xh[u])
                                : (double)__uint_as_float((uint32_t)xh[u] & 0x7FFFFFFFu);
                const bool wbit = f64 ? ((xw >> u) & 1u) != 0 : (f_goss && ((uint32_t)xh[u] >> 31) != 0);
                if (wbit) {
                    gv *= goss_mult;
                    hv *= goss_mult;
                }
                if (i < hi) FAcc::template add<LPR>(lds, w[u], sub, Ft, ls, gv, hv);
            } else {
                if (i < hi)
                    Acc::template add<LPR>(lds, s, w[u], sub, Ft, ls, (int64_t)(uint32_t)id[u], gh[u], goss_mult);
            }
        }
    };
    int32_t id_cur[U], id_nxt[U], id_nn[U];
    uint4 w_cur[U], w_nxt[U];
    int64_t i0 = lo;
    load_ids(i0, id_cur);
    load_recs(i0, id_cur, w_cur, qv, qv2, qw, fg, fh, fw);
    load_ids(i0 + step, id_nxt);
    pre();
    // The next step's loads are issued unconditionally (past the range they
    // re-read the last row): under a branch, the compiler's wait for the
    // current records at the join would also wait for them, and loads would
    // no longer overlap the LDS atomics.
    for (;;) {
        const bool more = i0 + step < hi;
        load_recs(i0 + step, id_nxt, w_nxt, qv_nxt, qv2_nxt, qw_nxt, fg_nxt, fh_nxt, fw_nxt);
        load_ids(i0 + 2 * step, id_nn);
        accumulate(i0, id_cur, w_cur, qv, qv2, qw, fg, fh, fw);
        if (!more) break;
        i0 += step;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            id_cur[u] = id_nxt[u];
            id_nxt[u] = id_nn[u];
            w_cur[u] = w_nxt[u];
            if constexpr (kQ) {
                qv[u] = qv_nxt[u];
                if constexpr (LPR == 1) qv2[u] = qv2_nxt[u];
            }
            if constexpr (kF) {
                fg[u] = fg_nxt[u];
                fh[u] = fh_nxt[u];
            }
        }
        qw = qw_nxt;
        fw = fw_nxt;
    }
}

template <int LPR, class Acc, bool kQ = false>
__global__ __launch_bounds__(1024) void k_hist(DevState s) {
    extern __shared__ unsigned char lds[];
    if (s.round->stopped) return;
    const int64_t m = root_rows(s);
    const bool direct = !s.round->sampled;
    const double goss_mult = s.round->goss_mult;
    if (m <= 0) return;
    const int64_t chunk = hist_chunk(s, m);
    const int64_t c0 = (int64_t)blockIdx.x * chunk;
    if (c0 >= m) return;
    const int64_t c1 = c0 + chunk < m ? c0 + chunk : m;
    const int ls = s.lds_stride;
    const int f0 = (int)blockIdx.y * s.tile_f;
    const int Ft = min(s.tile_f, s.n_features - f0);
    Acc::template zero<LPR>(lds, Ft, ls);
    __syncthreads();
    const uint4 *rec = (const uint4 *)(s.records + (size_t)blockIdx.y * s.n * s.rec_bytes);
    if constexpr (kQ) {
        const QCtx qc = quant_ctx(s, *s.round);
        uint4 *rec_w = (uint4 *)(s.records_w + (size_t)blockIdx.y * s.n * s.rec_bytes);
        if (direct) accumulate_rows<LPR, Acc, false, true, 3>(s, lds, nullptr, c0, c1, Ft, rec, goss_mult, &qc, rec_w);
        else accumulate_rows<LPR, Acc, true, true, 3>(s, lds, s.rows0, c0, c1, Ft, rec, goss_mult, &qc, rec_w);
    } else {
        // fp32 cells: two rows per step (four need more than the 128 VGPRs
        // a 1024-thread block may hold)
        constexpr int U = std::is_same<Acc, FAcc>::value ? 2 : kRootUnroll;
        if (direct) accumulate_rows<LPR, Acc, false, false, U>(s, lds, nullptr, c0, c1, Ft, rec, goss_mult);
        else accumulate_rows<LPR, Acc, true, false, U>(s, lds, s.rows0, c0, c1, Ft, rec, goss_mult);
    }
    __syncthreads();
    Acc::template store<LPR>(s, lds, blockIdx.x, f0, Ft);
}

// A raw buffer resource over `bytes` bytes at p (gfx9 word 3): loads through
// it take 32-bit offsets, and offsets at or past `bytes` read 0.
// The arguments must be wave-uniform; they are moved to scalar registers so
// the loads need no per-lane descriptor.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *p, uint32_t bytes) {
    const uint64_t a = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    void *q = (void *)(((uint64_t)hi << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(q, (short)0, (int)__builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

// ------------------------------------------------------------- partition
// One launch routes the rows of every leaf of the batch to the children
// (tree.partition_rows_into semantics: the missing bin follows default_left,
// otherwise bin <= threshold goes left) in the other row buffer -- left rows
// fill [begin, begin + n_left), right rows the rest. Each task is a chunk
// of 512-4K rows of one leaf (the item whose first task number, in the
// planner's per-item table, is the last at or below the task's): each of
// the block's 1024 threads keeps its kPartRows (4) row ids and their sides in
// registers (slots past the chunk read nothing: buffer loads out of range
// return 0), wave ballots count the rows of each (row group u, wave) entry,
// one wave scans the entries in row order, the chunk's output is reserved
// with one atomic per side, and the rows are written in their input order
// within each side. Few rows per thread keep the kernel at 64 VGPRs or less
// and many gathers in flight per CU; measured on C2, 4K-row chunks of 1024
// threads partition 31 % faster than 8K-row chunks of 256 threads with 32
// rows each. The root's batch, one leaf over every row, is the exception
// (below: 16K-row chunks, a quarter of the same-address reservations on its
// two cursors, which the L2 serializes).
// The order of rows inside a child is not the reference's (chunks land in
// reservation order); integer histograms are order-free, fp64 sums differ
// only in their rounding.
#ifndef MB_PART_THREADS
#define MB_PART_THREADS 1024
#endif
constexpr int kPartThreads = MB_PART_THREADS;
constexpr int kPartRows = kPartChunk / kPartThreads;  // rows per thread of a task
static_assert(kPartRows * kPartThreads == kPartChunk && kPartRows <= 32, "a task's rows fit the thread bit masks");
// The root's batch (one leaf over every row of the round) is partitioned by
// its own launch with kPartRowsRoot rows per thread: a quarter of the tasks,
// so a quarter of the same-address reservations on the root's two cursors
// (one wave of tasks holds the chip; the occupancy lost to the registers
// costs less there).
constexpr int kPartRowsRoot = kPartChunkRoot / kPartThreads;
static_assert(kPartRowsRoot * kPartThreads == kPartChunkRoot && kPartRowsRoot <= 32, "root task rows fit the masks");

template <int R>
__global__ __launch_bounds__(kPartThreads) void k_partition(DevState s) {
    constexpr int NW = kPartThreads / 64;  // waves
    constexpr int E = R * NW;              // (row group, wave) entries of a task
    constexpr int SW = (E + 63) / 64;      // waves that scan one side's entries
    static_assert((E % 64 == 0 || E < 64) && 2 * SW <= NW, "one wave scans up to 64 entries");
    __shared__ int cnt_l[E], cnt_r[E];     // counts, then exclusive prefixes within a scan wave
    __shared__ int wtot[2][SW];            // scan-wave totals, then their exclusive prefixes
    __shared__ long long base[2];
    const Batch bh = *s.batch;
    const int n_blocks = bh.n_blocks;
    if ((int)blockIdx.x >= n_blocks) return;
    const int tid = threadIdx.x, lane = lane_id(), w = tid >> 6;
    const unsigned long long below = (1ULL << lane) - 1ULL;
    const uint32_t n32 = (uint32_t)s.n;  // n < 2^31
    // every wave holds the batch's items, lane i item i (n_items <= 64); a
    // task finds its item by a ballot over the items' first tasks
    PartItem pit{};
    if (lane < bh.n_items) pit = s.part_items[lane];
    for (int blk = blockIdx.x; blk < n_blocks; blk += gridDim.x) {
        const unsigned long long own = __ballot(lane < bh.n_items && pit.qoff <= blk);  // item 0 starts at 0
        const int q = 63 - (int)__builtin_clzll(own);
        struct {
            int64_t begin, n_left, m, c0, c1;
            int item, src_buf, feature, bin, default_left, missing_bin, cat_e, direct;
        } d;
        d.begin = readlane_i64(pit.begin, q);
        d.n_left = readlane_i64(pit.n_left, q);
        d.m = readlane_i64(pit.m, q);
        d.c0 = (int64_t)(blk - __builtin_amdgcn_readlane(pit.qoff, q)) * bh.chunk_p;
        d.c1 = d.c0 + bh.chunk_p < d.m ? d.c0 + bh.chunk_p : d.m;
        d.item = q;
        d.src_buf = __builtin_amdgcn_readlane(pit.src_buf, q);
        d.feature = __builtin_amdgcn_readlane(pit.feature, q);
        d.bin = __builtin_amdgcn_readlane(pit.bin, q);
        d.default_left = __builtin_amdgcn_readlane(pit.default_left, q);
        d.missing_bin = __builtin_amdgcn_readlane(pit.missing_bin, q);
        d.cat_e = __builtin_amdgcn_readlane(pit.cat_e, q);
        d.direct = __builtin_amdgcn_readlane(pit.direct, q);
        const int32_t *src = (d.src_buf ? s.rows1 : s.rows0) + d.begin;
        int32_t *dst = (d.src_buf ? s.rows0 : s.rows1) + d.begin;
        const int mb = d.missing_bin, thr = d.bin, dl = d.default_left;
        // a categorical split routes by its set (tree.goes_left): bins in it go left
        unsigned long long cset[4] = {0ULL, 0ULL, 0ULL, 0ULL};
        const bool is_cat = d.cat_e >= 0;
        if (is_cat)
#pragma unroll
            for (int w = 0; w < 4; ++w) cset[w] = s.e_cat[(size_t)d.cat_e * 4 + w];
        // buffer loads: 32-bit offsets (one VGPR per gather instead of a
        // 64-bit address), and any offset past the range reads 0
        const __amdgpu_buffer_rsrc_t ids = buffer_rsrc(src + d.c0, (uint32_t)(d.c1 - d.c0) * 4u);
        const __amdgpu_buffer_rsrc_t col = buffer_rsrc(s.bins_cm + (size_t)d.feature * s.n, (uint32_t)s.n);
        int32_t r[R];
        uint32_t vbits = 0, lbits = 0;
        // every load unconditional (a row past the task reads id 0 and is
        // masked off), so all of them are in flight together
        if (d.direct) {  // task-uniform: ids are positions (the root, begin 0)
#pragma unroll
            for (int u = 0; u < R; ++u) {
                const int64_t i = d.c0 + (int64_t)u * kPartThreads + tid;
                vbits |= (i < d.c1 ? 1u : 0u) << u;
                r[u] = i < d.c1 ? (int32_t)(d.begin + i) : 0;
            }
        } else {
#pragma unroll
            for (int u = 0; u < R; ++u) {
                const int64_t i = d.c0 + (int64_t)u * kPartThreads + tid;
                vbits |= (i < d.c1 ? 1u : 0u) << u;
                r[u] = __builtin_amdgcn_raw_buffer_load_b32(ids, (u * kPartThreads + tid) * 4, 0, 0);
                if ((uint32_t)r[u] >= n32) r[u] = 0;  // never taken: ids come from the row lists
            }
        }
        uint32_t bin[R];
#pragma unroll
        for (int u = 0; u < R; ++u) bin[u] = __builtin_amdgcn_raw_buffer_load_b8(col, r[u], 0, 0);
#pragma unroll
        for (int u = 0; u < R; ++u) {
            const bool valid = (vbits >> u) & 1u;
            const int b = (int)bin[u];
            const unsigned long long cw = b < 64 ? cset[0] : b < 128 ? cset[1] : b < 192 ? cset[2] : cset[3];
            const bool left = is_cat ? ((cw >> (b & 63)) & 1ULL) != 0 : (b == mb) ? (dl != 0) : (b <= thr);
            lbits |= (left ? 1u : 0u) << u;
            const unsigned long long lm = __ballot(valid && left);
            const unsigned long long rm = __ballot(valid && !left);
            if (lane == 0) {
                cnt_l[u * NW + w] = __popcll(lm);
                cnt_r[u * NW + w] = __popcll(rm);
            }
        }
        __syncthreads();
        // entry k = u * NW + wave is in row order; waves 0 .. SW-1 scan the
        // left counts, SW .. 2 SW - 1 the right ones
        if (w < 2 * SW) {
            int *c = w < SW ? cnt_l : cnt_r;
            const int k = (w % SW) * 64 + lane;
            const int v = k < E ? c[k] : 0;
            const int inc = wave_incl_scan_i(v);
            if (k < E) c[k] = inc - v;
            if (lane == 63) wtot[w / SW][w % SW] = inc;
        }
        __syncthreads();
        if (tid < 2) {
            int a = 0;
            for (int j = 0; j < SW; ++j) {
                const int t = wtot[tid][j];
                wtot[tid][j] = a;
                a += t;
            }
            unsigned long long *cur = (unsigned long long *)&s.cursor[2 + 2 * d.item + tid];
            base[tid] = a ? (long long)atomicAdd(cur, (unsigned long long)a) : 0;
        }
        __syncthreads();
        // positions relative to the leaf's begin (below m < 2^31); a store
        // past the leaf's range is dropped by the buffer and flagged
        const int bl = (int)base[0], br = (int)base[1];
        const int nl = (int)d.n_left, m = (int)d.m;
        const __amdgpu_buffer_rsrc_t out = buffer_rsrc(dst, (uint32_t)m * 4u);
        bool overflow = false;
        // opaque to the compiler, so the ballots below are not merged with
        // the counting ones (which would keep 64 wave masks live across the
        // barriers)
        asm volatile("" : "+v"(lbits), "+v"(vbits));
#pragma unroll
        for (int u = 0; u < R; ++u) {
            const bool valid = (vbits >> u) & 1u;
            const bool left = (lbits >> u) & 1u;
            const unsigned long long lm = __ballot(valid && left);
            const unsigned long long rm = __ballot(valid && !left);
            const int k = u * NW + w;
            const int pl = bl + wtot[0][k >> 6] + cnt_l[k] + (int)__popcll(lm & below);
            const int pr = nl + br + wtot[1][k >> 6] + cnt_r[k] + (int)__popcll(rm & below);
            const int p = left ? pl : pr;
            overflow |= valid && (left ? pl >= nl : pr >= m);
            if (valid) __builtin_amdgcn_raw_buffer_store_b32(r[u], out, p * 4, 0, 0);
        }
        if (overflow) atomicOr(s.error, 1);
        __syncthreads();  // counts and offsets are rewritten by the next task
    }
}

// ------------------------------------------------------ record partition
// kPartRecThreads x kPartRows rows per task at most (the planner caps a
// record partition's tasks at kPartRecChunk rows).
// The partition of the record layout (s.rcp): the same tasks, counts, scans
// and reservations as k_partition, but a row travels as its whole record
// (LPR x 16 bytes, with its int8 pair in the last two bytes) from the
// parent's range of one record buffer to the child's range of the other, so
// the split feature's bin is a byte of the record already loaded (no column
// gather) and the children's accumulations read their records as one
// contiguous stream. The root's batch reads the dataset's records instead
// -- row id = position, or from the root list -- with each row's pair from
// the plane the root build wrote. kPartRows (4) rows per thread.
template <int LPR>
__global__ __launch_bounds__(kPartRecThreads) void k_partition_rec(DevState s) {
    constexpr int R = kPartRows;
    constexpr int T = kPartRecThreads;
    constexpr int NW = T / 64;             // waves
    constexpr int E = R * NW;              // (row group, wave) entries of a task
    constexpr int SW = (E + 63) / 64;      // waves that scan one side's entries
    static_assert((E % 64 == 0 || E < 64) && 2 * SW <= NW, "one wave scans up to 64 entries");
    __shared__ int cnt_l[E], cnt_r[E];
    __shared__ int wtot[2][SW];
    __shared__ long long base[2];
    const Batch bh = *s.batch;
    const int n_blocks = bh.n_blocks;
    if ((int)blockIdx.x >= n_blocks) return;
    const int tid = threadIdx.x, lane = lane_id(), w = tid >> 6;
    const unsigned long long below = (1ULL << lane) - 1ULL;
    const uint32_t n32 = (uint32_t)s.n;  // n < 2^31
    PartItem pit{};
    if (lane < bh.n_items) pit = s.part_items[lane];
    for (int blk = blockIdx.x; blk < n_blocks; blk += gridDim.x) {
        const unsigned long long own = __ballot(lane < bh.n_items && pit.qoff <= blk);  // item 0 starts at 0
        const int q = 63 - (int)__builtin_clzll(own);
        const int64_t begin = readlane_i64(pit.begin, q);
        const int64_t n_left = readlane_i64(pit.n_left, q);
        const int64_t m = readlane_i64(pit.m, q);
        const int64_t c0 = (int64_t)(blk - __builtin_amdgcn_readlane(pit.qoff, q)) * bh.chunk_p;
        const int64_t c1 = c0 + bh.chunk_p < m ? c0 + bh.chunk_p : m;
        const int src_buf = __builtin_amdgcn_readlane(pit.src_buf, q);
        const int feature = __builtin_amdgcn_readlane(pit.feature, q);
        const int thr = __builtin_amdgcn_readlane(pit.bin, q);
        const int dl = __builtin_amdgcn_readlane(pit.default_left, q);
        const int mbin = __builtin_amdgcn_readlane(pit.missing_bin, q);
        const int cat_e = __builtin_amdgcn_readlane(pit.cat_e, q);
        const int direct = __builtin_amdgcn_readlane(pit.direct, q);
        const int root = __builtin_amdgcn_readlane(pit.root, q);
        unsigned long long cset[4] = {0ULL, 0ULL, 0ULL, 0ULL};
        const bool is_cat = cat_e >= 0;
        if (is_cat)
#pragma unroll
            for (int k = 0; k < 4; ++k) cset[k] = s.e_cat[(size_t)cat_e * 4 + k];
        uint4 rec[R][LPR];
        uint32_t vbits = 0, lbits = 0;
#pragma unroll
        for (int u = 0; u < R; ++u) {
            const int64_t i = c0 + (int64_t)u * T + tid;
            vbits |= (i < c1 ? 1u : 0u) << u;
        }
        // every load unconditional (a slot past the task re-reads its last
        // row and is masked off), so all of them are in flight together
        if (root) {
            int32_t r[R];
            uint32_t pr[R];
#pragma unroll
            for (int u = 0; u < R; ++u) {
                int64_t i = c0 + (int64_t)u * T + tid;
                i = i < c1 ? i : c1 - 1;
                r[u] = direct ? (int32_t)(begin + i) : s.rows0[begin + i];
                if ((uint32_t)r[u] >= n32) r[u] = 0;  // never taken: ids come from the root list
            }
            const uint4 *src = (const uint4 *)s.records;
#pragma unroll
            for (int u = 0; u < R; ++u) {
#pragma unroll
                for (int k = 0; k < LPR; ++k) rec[u][k] = src[(size_t)(uint32_t)r[u] * LPR + k];
                pr[u] = s.pairs[(uint32_t)r[u]];
            }
#pragma unroll
            for (int u = 0; u < R; ++u) rec[u][LPR - 1].w = (rec[u][LPR - 1].w & 0xFFFFu) | (pr[u] << 16);
        } else {
            const uint4 *src = (const uint4 *)(src_buf ? s.crec1 : s.crec0) + (size_t)begin * LPR;
#pragma unroll
            for (int u = 0; u < R; ++u) {
                int64_t i = c0 + (int64_t)u * T + tid;
                i = i < c1 ? i : c1 - 1;
#pragma unroll
                for (int k = 0; k < LPR; ++k) rec[u][k] = src[(size_t)i * LPR + k];
            }
        }
        // the split feature's byte of each record: the dword holding it is
        // picked by a task-uniform select (no indexing into registers)
        const int fw = feature >> 2, fsh = 8 * (feature & 3);
#pragma unroll
        for (int u = 0; u < R; ++u) {
            uint32_t word = 0u;
#pragma unroll
            for (int k = 0; k < LPR; ++k) {
                word = fw == 4 * k + 0 ? rec[u][k].x : word;
                word = fw == 4 * k + 1 ? rec[u][k].y : word;
                word = fw == 4 * k + 2 ? rec[u][k].z : word;
                word = fw == 4 * k + 3 ? rec[u][k].w : word;
            }
            const int b = (int)((word >> fsh) & 255u);
            const bool valid = (vbits >> u) & 1u;
            const unsigned long long cw = b < 64 ? cset[0] : b < 128 ? cset[1] : b < 192 ? cset[2] : cset[3];
            const bool left = is_cat ? ((cw >> (b & 63)) & 1ULL) != 0 : (b == mbin) ? (dl != 0) : (b <= thr);
            lbits |= (left ? 1u : 0u) << u;
            const unsigned long long lm = __ballot(valid && left);
            const unsigned long long rm = __ballot(valid && !left);
            if (lane == 0) {
                cnt_l[u * NW + w] = __popcll(lm);
                cnt_r[u * NW + w] = __popcll(rm);
            }
        }
        __syncthreads();
        if (w < 2 * SW) {
            int *c = w < SW ? cnt_l : cnt_r;
            const int k = (w % SW) * 64 + lane;
            const int v = k < E ? c[k] : 0;
            const int inc = wave_incl_scan_i(v);
            if (k < E) c[k] = inc - v;
            if (lane == 63) wtot[w / SW][w % SW] = inc;
        }
        __syncthreads();
        if (tid < 2) {
            int a = 0;
            for (int j = 0; j < SW; ++j) {
                const int t = wtot[tid][j];
                wtot[tid][j] = a;
                a += t;
            }
            unsigned long long *cur = (unsigned long long *)&s.cursor[2 + 2 * q + tid];
            base[tid] = a ? (long long)atomicAdd(cur, (unsigned long long)a) : 0;
        }
        __syncthreads();
        // positions relative to the leaf's begin (below m < 2^31); a record
        // that would land past its side of the range is not stored, and
        // flagged
        const int bl = (int)base[0], br = (int)base[1];
        const int nl = (int)n_left, mm = (int)m;
        uint4 *dst = (uint4 *)(src_buf ? s.crec0 : s.crec1) + (size_t)begin * LPR;
        bool overflow = false;
        asm volatile("" : "+v"(lbits), "+v"(vbits));
#pragma unroll
        for (int u = 0; u < R; ++u) {
            const bool valid = (vbits >> u) & 1u;
            const bool left = (lbits >> u) & 1u;
            const unsigned long long lm = __ballot(valid && left);
            const unsigned long long rm = __ballot(valid && !left);
            const int k = u * NW + w;
            const int pl = bl + wtot[0][k >> 6] + cnt_l[k] + (int)__popcll(lm & below);
            const int pr = nl + br + wtot[1][k >> 6] + cnt_r[k] + (int)__popcll(rm & below);
            const int pos = left ? pl : pr;
            const bool bad = left ? pl >= nl : pr >= mm;
            overflow |= valid && bad;
            if (valid && !bad) {
#pragma unroll
                for (int kk = 0; kk < LPR; ++kk) dst[(size_t)pos * LPR + kk] = rec[u][kk];
            }
        }
        if (overflow) atomicOr(s.error, 1);
        __syncthreads();  // counts and offsets are rewritten by the next task
    }
}

// ---------------------------------------------------------- accumulation
// One launch accumulates the smaller child of every leaf of the batch from
// its rows, now contiguous in the partitioned row buffer. Each task (found
// from the planner's per-item table as in the partition) is a chunk of one
// child's rows and yields one block partial; the scan kernel merges an
// item's partials.
// blockIdx.y is the feature tile: the block reads that tile's records and
// stores that tile's features of its partial.
constexpr int kAccThreads = 1024;  // two blocks per CU resident (launch grid 2 x CUs)
template <int LPR, class Acc>
__global__ __launch_bounds__(kAccThreads) void k_accum(DevState s) {
    extern __shared__ unsigned char lds[];
    const Batch bh = *s.batch;
    const int n_acc = bh.n_acc;
    if ((int)blockIdx.x >= n_acc) return;
    const double goss_mult = s.round->goss_mult;
    const int ls = s.lds_stride;
    const int f0 = (int)blockIdx.y * s.tile_f;
    const int Ft = min(s.tile_f, s.n_features - f0);
    const uint4 *rec = (const uint4 *)(s.records + (size_t)blockIdx.y * s.n * s.rec_bytes);
    const int lane = lane_id();
    // every wave holds the batch's items, lane i item i (n_items <= 64); a
    // task finds its item by a ballot over the items' first tasks
    AccItem ait{};
    if (lane < bh.n_items) ait = s.acc_items[lane];
    for (int blk = blockIdx.x; blk < n_acc; blk += gridDim.x) {
        const unsigned long long own = __ballot(lane < bh.n_items && ait.poff <= blk);  // item 0 starts at 0
        const int q = 63 - (int)__builtin_clzll(own);
        const int64_t lo = readlane_i64(ait.lo, q) + (int64_t)(blk - __builtin_amdgcn_readlane(ait.poff, q)) * bh.chunk_a;
        const int64_t hi_item = readlane_i64(ait.hi, q);
        const int64_t hi = lo + bh.chunk_a < hi_item ? lo + bh.chunk_a : hi_item;
        const int buf = __builtin_amdgcn_readlane(ait.buf, q);
        // the histogram is zeroed while the task's first records load
        accumulate_rows<LPR, Acc, true, false, std::is_same<Acc, FAcc>::value ? kAccUnrollF : kAccUnroll>(
            s, lds, buf ? s.rows1 : s.rows0, lo, hi, Ft, rec, goss_mult, nullptr, nullptr, [&]() {
                Acc::template zero<LPR>(lds, Ft, ls);
                __syncthreads();
            });
        __syncthreads();
        Acc::template store<LPR>(s, lds, blk, f0, Ft);
        __syncthreads();  // the LDS histogram is zeroed again for the next task
    }
}

// The accumulation of the record layout (s.rcp): an accumulated child's
// records are contiguous in its range of a record buffer, so a task streams
// them (no row id, no gather), kAccUnrollRec rows per lane and step.
#ifndef MB_ACC_UNROLL_REC
#define MB_ACC_UNROLL_REC 2
#endif
constexpr int kAccUnrollRec = MB_ACC_UNROLL_REC;
template <int LPR>
__global__ __launch_bounds__(kAccThreads) void k_accum_rec(DevState s) {
    extern __shared__ unsigned char lds[];
    const Batch bh = *s.batch;
    const int n_acc = bh.n_acc;
    if ((int)blockIdx.x >= n_acc) return;
    const int ls = s.lds_stride;
    const int Ft = s.n_features;  // one tile
    const int lane = lane_id();
    AccItem ait{};
    if (lane < bh.n_items) ait = s.acc_items[lane];
    for (int blk = blockIdx.x; blk < n_acc; blk += gridDim.x) {
        const unsigned long long own = __ballot(lane < bh.n_items && ait.poff <= blk);  // item 0 starts at 0
        const int q = 63 - (int)__builtin_clzll(own);
        const int64_t lo = readlane_i64(ait.lo, q) + (int64_t)(blk - __builtin_amdgcn_readlane(ait.poff, q)) * bh.chunk_a;
        const int64_t hi_item = readlane_i64(ait.hi, q);
        const int64_t hi = lo + bh.chunk_a < hi_item ? lo + bh.chunk_a : hi_item;
        const int buf = __builtin_amdgcn_readlane(ait.buf, q);
        const uint4 *rec = (const uint4 *)(buf ? s.crec1 : s.crec0);
        QAcc::template zero<LPR>(lds, Ft, ls);
        __syncthreads();
        accumulate_rows<LPR, QAcc, false, false, kAccUnrollRec>(s, lds, nullptr, lo, hi, Ft, rec, 1.0);
        __syncthreads();
        QAcc::template store<LPR>(s, lds, blk, 0, Ft);
        __syncthreads();  // the LDS histogram is zeroed again for the next task
    }
}

// ------------------------------------------------------------------- scan
// Tasks (item, feature), grid-strided, 512 threads each. The accumulated
// child's histogram is merged from its block partials (two threads per bin)
// and stored; the sibling is parent - accumulated, written over the parent's
// buffer. Threads 0-255 then scan the accumulated child and 256-511 the
// sibling, one bin per thread, with int32 sums (node totals stay below
// 2^31: n_rows * (num_grad_quant_bins + 1) < 2^31 is checked on the host).
// The scan follows split.find_best_split (src/mojotrees/split.mojo:601-1360)
// with each candidate scored by quantized_split_gain
// (quantized_gradient.mojo:3283-3310): ascending bins, missing-left scored
// before missing-right, strict '>' keeps the first maximum; the hessian
// guard compares against hessian_units_at_least (:3336). Each task writes one
// ScanResult per child; the planner folds them.
constexpr int kScanThreads = 512;


// Lane l's binary64 value on every lane (l wave-uniform).
__device__ __forceinline__ double readlane_f64_early(double d, int l) {
    return __longlong_as_double((long long)readlane_i64((int64_t)__double_as_longlong(d), l));
}

// kCat: the dataset has categorical features (the category-set search is
// compiled in). At most 128 VGPRs (4 waves per SIMD): two 512-thread blocks
// per CU, so a batch's (leaf, feature) tasks need half the block rounds.
template <bool kCat>
__global__ __launch_bounds__(kScanThreads, 4) void k_scan(DevState s, int root_mode) {
    __shared__ int cg[2][256], ch[2][256], cc[2][256];
    __shared__ int acc[3][256];
    __shared__ int wtot[8][3];
    __shared__ double wgain[8];
    __shared__ int word[8];
    __shared__ long long wleft[8];
    // categorical search (per child): sort keys, the sorted candidates, their
    // count, and each walk direction's best (gain, step, left rows)
    __shared__ double ckey[2][256];
    __shared__ int csort[2][256];
    __shared__ int rpart[2][4][64];  // rank counts of bins 0-63 per wave of a half (below 64 categories)
    __shared__ int cwcnt[8];
    __shared__ double cdg[2][2];
    __shared__ int cdi[2][2];
    __shared__ long long cdl[2][2];
    const int tid = threadIdx.x, lane = lane_id(), wv = tid >> 6;
    const HyperParams &hp = s.hp;
    const int F = s.n_features, nb = s.n_bins;
    const size_t hsz = (size_t)F * nb * 3;
    const int n_items = root_mode ? 1 : s.batch->n_items;
    const int n_tasks = n_items * F;
    if ((int)blockIdx.x >= n_tasks) return;
    const Round rd = *s.round;
    if (rd.stopped) return;
    const double gu = rd.grad_units, hu = rd.hess_units;
    const double l1 = hp.lambda_l1, l2 = hp.lambda_l2;
    long long hmin = 0;  // hessian_units_at_least: min_sum_hessian in lattice units, rounded up
    if (hp.min_sum_hessian > 0.0) {
        const double u = hp.min_sum_hessian * hu;
        double fl = floor(u);
        if (fl < u) fl += 1.0;
        hmin = (long long)fl;
    }
    for (int task = blockIdx.x; task < n_tasks; task += gridDim.x) {
        // with category-set features, tasks go feature-major in scan_order
        // (those features first: their searches run longest, so the
        // shorter numerical tasks fill in behind them)
        int j, f;
        if (kCat && s.scan_order != nullptr) {
            const int pos = task / n_items;
            j = task - pos * n_items;
            f = s.scan_order[pos];
        } else {
            j = task / F;
            f = task - j * F;
        }
        Item it;
        int64_t m_built, m_sib;
        if (root_mode) {
            m_built = root_rows(s);
            m_sib = 0;
            it.part_off = 0;
            const int64_t chk = hist_chunk(s, m_built);
            it.part_cnt = m_built > 0 ? (int)((m_built + chk - 1) / chk) : 0;
            it.hist_built = 0;
            it.hist_sib = 0;
            it.depth_child = 0;
        } else {
            it = s.items[j];
            const int64_t m = it.end - it.begin;
            m_built = it.builds_left ? it.n_left : m - it.n_left;
            m_sib = m - m_built;
        }
        // ---- merge the accumulated child's partials: thread -> (bin, half)
        {
            const int bin = tid & 255, half = tid >> 8;
            int g = 0, h = 0, c = 0;
            // the parent's cells (the sibling is parent - accumulated) are
            // loaded with the partials, one memory round trip for both
            int32_t *pp = nullptr;
            int pg0 = 0, ph0 = 0, pc0 = 0;
            if (half == 0 && !root_mode && bin < nb) {
                pp = s.hist + (size_t)it.hist_sib * hsz + ((size_t)f * nb + bin) * 3;
                pg0 = pp[0];
                ph0 = pp[1];
                pc0 = pp[2];
            }
            if (bin < nb) {
                const size_t pstride = (size_t)F * s.part_stride;
                const unsigned long long *p =
                    s.part + (size_t)it.part_off * pstride + (size_t)f * s.part_stride + bin;
                const int np = it.part_cnt;
                int b = half;
                if (hp.wide) {
                    // grad | hess halves and a separate count per partial
                    // (WAcc); the sums wrap as unsigned words, and every
                    // subset of the round's rows fits int32
                    const uint32_t *pc =
                        s.part_c + (size_t)it.part_off * pstride + (size_t)f * s.part_stride + bin;
                    uint32_t ug = 0u, uh = 0u, uc = 0u;
                    for (; b < np; b += 2) {
                        const unsigned long long vv = p[(size_t)b * pstride];
                        ug += (uint32_t)(vv >> 32);
                        uh += (uint32_t)vv;
                        uc += pc[(size_t)b * pstride];
                    }
                    g = (int)ug;
                    h = (int)uh;
                    c = (int)uc;
                } else {
                    for (; b + 14 < np; b += 16) {
                        unsigned long long vv[8];
#pragma unroll
                        for (int u = 0; u < 8; ++u) vv[u] = p[(size_t)(b + 2 * u) * pstride];
#pragma unroll
                        for (int u = 0; u < 8; ++u) {
                            c += (int)(vv[u] & 0xFFFFFULL);
                            h += (int)((vv[u] >> 20) & 0x3FFFFFULL);
                            g += (int)((long long)vv[u] >> 42);
                        }
                    }
                    for (; b < np; b += 2) {
                        const unsigned long long vv = p[(size_t)b * pstride];
                        c += (int)(vv & 0xFFFFFULL);
                        h += (int)((vv >> 20) & 0x3FFFFFULL);
                        g += (int)((long long)vv >> 42);
                    }
                }
            }
            if (half == 1) {
                acc[0][bin] = g;
                acc[1][bin] = h;
                acc[2][bin] = c;
            }
            __syncthreads();
            if (half == 0) {
                g += acc[0][bin];
                h += acc[1][bin];
                c += acc[2][bin];
                cg[0][bin] = g;
                ch[0][bin] = h;
                cc[0][bin] = c;
                int sgv = 0, shv = 0, scv = 0;
                if (bin < nb) {
                    int32_t *ob = s.hist + (size_t)it.hist_built * hsz + ((size_t)f * nb + bin) * 3;
                    ob[0] = g;
                    ob[1] = h;
                    ob[2] = c;
                    if (!root_mode) {
                        sgv = pg0 - g;
                        shv = ph0 - h;
                        scv = pc0 - c;
                        pp[0] = sgv;
                        pp[1] = shv;
                        pp[2] = scv;
                    }
                }
                cg[1][bin] = sgv;
                ch[1][bin] = shv;
                cc[1][bin] = scv;
            }
            __syncthreads();
        }
        // ---- scan: threads 0-255 the accumulated child, 256-511 the sibling
        const int child = tid >> 8;
        const int bin = tid & 255;
        const int cw = wv & 3;
        const int vg = cg[child][bin], vh = ch[child][bin], vc = cc[child][bin];
        const int ig = wave_incl_scan_i(vg), ih = wave_incl_scan_i(vh), ic = wave_incl_scan_i(vc);
        if (lane == 63) {
            wtot[wv][0] = ig;
            wtot[wv][1] = ih;
            wtot[wv][2] = ic;
        }
        __syncthreads();
        int pg = 0, ph = 0, pc = 0, TG = 0, TH = 0, TC = 0;
#pragma unroll
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
        const int lg = pg + ig, lh = ph + ih, lc = pc + ic;  // inclusive prefix at `bin`
        const int64_t n_child = child == 0 ? m_built : m_sib;
        const int mbf = s.missing_bin[f];
        const bool gated = (root_mode && child == 1) ||
                           (hp.max_depth > 0 && it.depth_child >= hp.max_depth) ||
                           n_child < 2 * (int64_t)hp.min_data_in_leaf || n_child < 2 ||
                           !s.feature_mask[(size_t)rd.tree_index * F + f];
        double best_gain = 0.0;
        int best_order = 0x7FFFFFFF;
        int best_left = 0;
        // a categorical feature is searched as category partitions
        // (categorical.find_best_categorical_split, categorical.mojo:684-782)
        const int ncf = kCat && s.ncat ? s.ncat[f] : 0;  // block-uniform
        const bool cat_onehot = ncf > 0 && (hp.one_hot_max_size >= 0 ? ncf <= hp.one_hot_max_size
                                                                      : ncf + 1 <= hp.max_cat_to_onehot);
        bool cat_sorted = false;
        if (ncf > 0) {
            const double parent = qscore(TG, TH, gu, hu, l1, l2);
            const long long min_c = hp.min_data_in_leaf;
            if (cat_onehot) {
                // _onehot_search (:478-525): each category alone goes left;
                // the argmax below keeps the lowest bin on equal gains
                if (!gated && ncf >= 2 && bin >= 1 && bin <= ncf && !(vc < min_c || vh < hmin) &&
                    !(TC - vc < min_c) && !(TH - vh < hmin)) {
                    const double gain = qscore(vg, vh, gu, hu, l1, l2) + qscore(TG - vg, TH - vh, gu, hu, l1, l2) - parent;
                    if (gain > best_gain) {
                        best_gain = gain;
                        best_order = bin;
                        best_left = vc;
                    }
                }
            } else {
                // _sorted_search (:527-623): categories holding at least
                // cat_smooth rows, ordered by G / (H + cat_smooth) (stable:
                // equal keys keep bin order, as metrics._argsort), prefixes
                // walked from both ends
                cat_sorted = true;
                const bool cand = !gated && ncf >= 2 && bin >= 1 && bin <= ncf && (double)vc >= hp.cat_smooth;
                const double key = ((double)vg / gu) / ((double)vh / hu + hp.cat_smooth);
                ckey[child][bin] = cand ? key : 0.0;
                const unsigned long long cm = __ballot(cand);
                if (lane == 0) cwcnt[wv] = __popcll(cm);
                csort[child][bin] = cand ? 1 : 0;  // candidate flags until ranked
                __syncthreads();
                // rank = the candidates ordered before this one: a wave
                // reads 64 categories' keys and flags per LDS load, then
                // compares with each candidate's key read from its lane.
                // Below 64 categories every candidate is in the half's
                // first wave: the half's four waves each compare the keys
                // of bins 0-63 with a quarter of the candidates, and the
                // quarters' counts are added up.
                const bool few = ncf < 64;  // block-uniform
                int rank = 0;
                {
                    const double kt = few ? ckey[child][lane] : key;  // the target: bin `lane`, or the own bin
                    const int bt = few ? lane : bin;
                    for (int u0 = 1; u0 <= ncf; u0 += 64) {
                        const int u = u0 + lane;
                        const bool ok = u <= ncf && csort[child][u] != 0;
                        const double ku = ok ? ckey[child][u] : 0.0;
                        unsigned long long m = __ballot(ok);
                        if (few) m &= 0xFFFFULL << (16 * cw);
                        for (; m; m &= m - 1ULL) {
                            const int l = (int)__builtin_ctzll(m);
                            const double kl = readlane_f64_early(ku, l);
                            rank += (kl < kt || (kl == kt && u0 + l < bt)) ? 1 : 0;
                        }
                    }
                    if (few) rpart[child][cw][lane] = rank;
                }
                const int used = cwcnt[child << 2] + cwcnt[(child << 2) + 1] + cwcnt[(child << 2) + 2] +
                                 cwcnt[(child << 2) + 3];
                __syncthreads();
                if (few && cw == 0)
                    rank = rpart[child][0][lane] + rpart[child][1][lane] + rpart[child][2][lane] + rpart[child][3][lane];
                if (cand) csort[child][rank] = bin;
                __syncthreads();
                // each direction's wave: its lanes load the steps' cells, a
                // uniform pass adds them in the walk's order and takes the
                // walk's decisions (continue / break / min_data_per_group
                // groups), then the evaluated steps are scored in parallel;
                // the first maximum wins (strict '>' along the walk)
                const int dthr = (tid & 255) >> 6;  // waves 0 and 1 of the half: directions 0 and 1
                if (dthr < 2) {
                    const int d = dthr;
                    double dg = 0.0;
                    int di = -1;
                    long long dl_ = 0;
                    if (used >= 2) {
                        int max_num_cat = hp.max_cat_threshold;
                        if ((used + 1) / 2 < max_num_cat) max_num_cat = (used + 1) / 2;
                        if (max_num_cat < 0) max_num_cat = 0;
                        const int steps = used < max_num_cat ? used : max_num_cat;
                        const double l2c = l2 + hp.cat_l2;
                        const int mdpg = hp.min_data_per_group;
                        // lane = step of the walk (64 per pass): the running
                        // sums are 32-bit integer prefix sums (exact in any
                        // order: every subset of a round's rows sums within
                        // int32, as the histogram cells do);
                        // the walk stops at the first step that leaves too
                        // little on the other side, and the groups of
                        // min_data_per_group rows are a scalar pass over the
                        // steps' counts before it
                        long long ag = 0, ah = 0;
                        long long ac = 0, agg = 0;
                        bool stop = false;
                        for (int c0 = 0; c0 < steps && !stop; c0 += 64) {
                            const int i = c0 + lane;
                            const bool in = i < steps;
                            const int tb = in ? csort[child][d == 0 ? i : used - 1 - i] : 0;
                            const int xg = in ? cg[child][tb] : 0, xh = in ? ch[child][tb] : 0;
                            const int xc = in ? cc[child][tb] : 0;
                            const long long mg = ag + (long long)wave_incl_scan_i(xg);
                            const long long mh = ah + (long long)wave_incl_scan_i(xh);
                            const long long mc = ac + (long long)wave_incl_scan_i(xc);
                            const bool valid = in && !(mc < min_c || mh < hmin);
                            const long long rc = TC - mc;
                            const unsigned long long sm =
                                __ballot(valid && (rc < min_c || rc < hp.min_data_per_group || TH - mh < hmin));
                            const int n_here = steps - c0 < 64 ? steps - c0 : 64;
                            const int s_at = sm ? (int)__builtin_ctzll(sm) : n_here;  // first stop, else the pass's end
                            const unsigned long long vm = __ballot(valid);
                            const unsigned long long before = s_at < 64 ? (1ULL << s_at) - 1ULL : ~0ULL;
                            unsigned long long evm = 0ULL;
                            if ((~__ballot(xc >= mdpg) & before) == 0ULL) {
                                // every step before the stop holds a group on
                                // its own: each valid one closes a group, and
                                // the open count is what follows the last
                                evm = vm & before;
                                if (s_at > 0) {
                                    const long long last = readlane_i64(mc, s_at - 1);
                                    agg = evm ? last - readlane_i64(mc, 63 - (int)__builtin_clzll(evm)) : agg + (last - ac);
                                }
                            } else {
                                for (int k = 0; k < s_at; ++k) {
                                    agg += __builtin_amdgcn_readlane(xc, k);
                                    if (((vm >> k) & 1ULL) && agg >= mdpg) {
                                        evm |= 1ULL << k;
                                        agg = 0;
                                    }
                                }
                            }
                            const bool mev = (evm >> lane) & 1ULL;
                            stop = sm != 0ULL;
                            ag = readlane_i64(mg, 63);
                            ah = readlane_i64(mh, 63);
                            ac = readlane_i64(mc, 63);
                            double bg = 0.0;
                            int bo = 0x7FFFFFFF;
                            if (mev) {
                                const double g_ = qscore(mg, mh, gu, hu, l1, l2c) + qscore(TG - mg, TH - mh, gu, hu, l1, l2c) - parent;
                                if (g_ > 0.0) {
                                    bg = g_;
                                    bo = i;
                                }
                            }
                            const int mine = bo;
                            wave_argmax(bg, bo);
                            if (bo != 0x7FFFFFFF && bg > dg) {
                                const unsigned long long wl = __ballot(mine == bo);
                                dg = bg;
                                di = bo;
                                dl_ = __builtin_amdgcn_readlane((int)mc, (int)__builtin_ctzll(wl));
                            }
                        }
                    }
                    if (lane == 0) {
                        cdg[child][d] = dg;
                        cdi[child][d] = di;
                        cdl[child][d] = dl_;
                    }
                }
                __syncthreads();
            }
        } else if (!gated) {
            const int mg = mbf >= 0 ? cg[child][mbf] : 0, mh = mbf >= 0 ? ch[child][mbf] : 0,
                      mc = mbf >= 0 ? cc[child][mbf] : 0;
            const long long min_c = hp.min_data_in_leaf;
            const int n_scan = mbf >= 0 ? mbf : nb;
            int lim = n_scan < s.widths[f] ? n_scan : s.widths[f];
            if (mc == 0 && lim > n_scan - 1) lim = n_scan - 1;
            if (bin < lim) {
                const double parent = qscore(TG, TH, gu, hu, l1, l2);
                if (mbf >= 0) {
                    const int ag = lg + mg, ah = lh + mh, ac = lc + mc;
                    const int rg = TG - ag, rh = TH - ah, rc = TC - ac;
                    if (!(ah < hmin || rh < hmin || ac < min_c || rc < min_c)) {
                        const double gain =
                            qscore(ag, ah, gu, hu, l1, l2) + qscore(rg, rh, gu, hu, l1, l2) - parent;
                        if (gain > best_gain) {
                            best_gain = gain;
                            best_order = 2 * bin;
                            best_left = ac;
                        }
                    }
                }
                if (mbf < 0 || mc > 0) {
                    const int rg = TG - lg, rh = TH - lh, rc = TC - lc;
                    if (!(lh < hmin || rh < hmin || lc < min_c || rc < min_c)) {
                        const double gain =
                            qscore(lg, lh, gu, hu, l1, l2) + qscore(rg, rh, gu, hu, l1, l2) - parent;
                        if (gain > best_gain) {
                            best_gain = gain;
                            best_order = 2 * bin + 1;
                            best_left = lc;
                        }
                    }
                }
            }
        }
        {
            // argmax carrying the winner's left count (orders are distinct
            // per lane, so the winner is the lane that held the final order)
            const int mine = best_order;
            wave_argmax(best_gain, best_order);
            const unsigned long long wins = __ballot(mine == best_order && best_order != 0x7FFFFFFF);
            const int srcl = wins ? (int)__ffsll((long long)wins) - 1 : 0;
            best_left = __shfl(best_left, srcl, 64);
        }
        if (lane == 0) {
            wgain[wv] = best_gain;
            word[wv] = best_order;
            wleft[wv] = best_left;
        }
        __syncthreads();
        if (ncf > 0) {
            if ((tid & 255) == 0 && !(root_mode && child == 1)) {
                ScanResult rs;
                unsigned long long bits[4] = {0ULL, 0ULL, 0ULL, 0ULL};
                rs.gain = 0.0;
                rs.found = 0;
                rs.n_left = 0;
                if (cat_sorted) {
                    // direction 0 first, then direction 1 on a strictly larger gain
                    int d = -1;
                    if (cdi[child][0] >= 0) d = 0;
                    if (cdi[child][1] >= 0 && (d < 0 || cdg[child][1] > cdg[child][0])) d = 1;
                    if (d >= 0) {
                        int used = 0;
                        for (int k = 0; k < 4; ++k) used += cwcnt[(child << 2) + k];
                        for (int i = 0; i <= cdi[child][d]; ++i) {
                            const int tb = csort[child][d == 0 ? i : used - 1 - i];
                            bits[tb >> 6] |= 1ULL << (tb & 63);
                        }
                        rs.gain = cdg[child][d];
                        rs.found = 1;
                        rs.n_left = cdl[child][d];
                    }
                } else {
                    double bgn = wgain[child << 2];
                    int bo = word[child << 2];
                    long long bleft = wleft[child << 2];
                    for (int k = 1; k < 4; ++k) {
                        const double og = wgain[(child << 2) + k];
                        const int oo = word[(child << 2) + k];
                        if (og > bgn || (og == bgn && oo < bo)) {
                            bgn = og;
                            bo = oo;
                            bleft = wleft[(child << 2) + k];
                        }
                    }
                    if (bo != 0x7FFFFFFF) {
                        bits[bo >> 6] |= 1ULL << (bo & 63);
                        rs.gain = bgn;
                        rs.found = 1;
                        rs.n_left = bleft;
                    }
                }
                rs.bin = -1;
                rs.default_left = 0;
                rs.cat = rs.found;
                rs.tot_g = TG;
                rs.tot_h = TH;
                rs.tot_c = TC;
                const size_t ri = (size_t)(j * 2 + child) * F + f;
                s.scan[ri] = rs;
                s.scan_gain[ri] = rs.found ? rs.gain : -1.0;
#pragma unroll
                for (int w = 0; w < 4; ++w) s.scan_cat[ri * 4 + w] = bits[w];
            }
        } else if ((tid & 255) == 0 && !(root_mode && child == 1)) {
            double bgn = wgain[child << 2];
            int bo = word[child << 2];
            long long bleft = wleft[child << 2];
            for (int k = 1; k < 4; ++k) {
                const double og = wgain[(child << 2) + k];
                const int oo = word[(child << 2) + k];
                if (og > bgn || (og == bgn && oo < bo)) {
                    bgn = og;
                    bo = oo;
                    bleft = wleft[(child << 2) + k];
                }
            }
            ScanResult rs;
            rs.gain = bgn;
            rs.found = bo != 0x7FFFFFFF;
            rs.bin = rs.found ? bo >> 1 : -1;
            rs.default_left = rs.found ? ((bo & 1) == 0) : 0;
            rs.cat = 0;
            rs.tot_g = TG;
            rs.tot_h = TH;
            rs.tot_c = TC;
            rs.n_left = rs.found ? bleft : 0;
            s.scan[(size_t)(j * 2 + child) * F + f] = rs;
            s.scan_gain[(size_t)(j * 2 + child) * F + f] = rs.found ? rs.gain : -1.0;
        }
        __syncthreads();
    }
}

// Scan, fp32-gradient path. Same task layout as k_scan. The merge sums the
// fp64 partials; the sibling is parent - built in fp64 (subtract_histogram,
// histogram.mojo:3747). Then one thread per child runs the reference's
// sequential arithmetic of split.find_best_split (split.mojo:601-1360):
// totals over 8 interleaved lanes reduced pairwise plus the tail, the
// running left prefix in ascending bin order, and the serial sum over all
// bins that tree._leaf_value (tree.mojo:1961-1995) uses; every thread then
// scores its bin's candidates from those prefixes with the reference's gain
// expression. Given identical histograms the gains are identical; the
// histograms themselves differ from the reference's only in the rounding of
// their fp64 sums.
// kCat as in k_scan; without categorical features at most 128 VGPRs (two
// blocks per CU), with them uncapped (the category search would spill).
// k_scan for narrow histograms (at most 64 bins per feature) without
// categorical features: a block takes kNarrowFeat features of one leaf, so
// that every thread has a bin. The merge maps thread -> (feature, half,
// bin); the scan gives one wave to each (feature, child), lane = bin, so a
// child's prefix sums are one wave scan and its best split one wave argmax,
// with no block barrier. Candidates, guards and tie rules are k_scan's.
constexpr int kNarrowFeat = kScanThreads / 128;
__global__ __launch_bounds__(kScanThreads, 4) void k_scan_narrow(DevState s, int root_mode) {
    __shared__ int acc[kNarrowFeat][3][64];
    __shared__ int cv[kNarrowFeat][2][3][64];  // (g, h, c) of the accumulated child (0) and the sibling (1)
    const int tid = threadIdx.x, lane = lane_id(), wv = tid >> 6;
    const HyperParams &hp = s.hp;
    const int F = s.n_features, nb = s.n_bins;
    const size_t hsz = (size_t)F * nb * 3;
    const int n_items = root_mode ? 1 : s.batch->n_items;
    const int n_groups = (F + kNarrowFeat - 1) / kNarrowFeat;
    const int n_tasks = n_items * n_groups;
    if ((int)blockIdx.x >= n_tasks) return;
    const Round rd = *s.round;
    if (rd.stopped) return;
    const double gu = rd.grad_units, hu = rd.hess_units;
    const double l1 = hp.lambda_l1, l2 = hp.lambda_l2;
    long long hmin = 0;  // hessian_units_at_least: min_sum_hessian in lattice units, rounded up
    if (hp.min_sum_hessian > 0.0) {
        const double u = hp.min_sum_hessian * hu;
        double fl = floor(u);
        if (fl < u) fl += 1.0;
        hmin = (long long)fl;
    }
    // every wave holds the batch's items, lane i item i (n_items <= 64): a
    // task reads its item's fields from registers, not from memory
    Item my{};
    if (!root_mode && lane < n_items) my = s.items[lane];
    for (int task = blockIdx.x; task < n_tasks; task += gridDim.x) {
        const int j = task / n_groups;
        const int f0 = (task - j * n_groups) * kNarrowFeat;
        // the scan phase's feature (this wave's: f0 + wave / 2) metadata,
        // requested with the task's first loads
        const int fs = f0 + (wv >> 1);
        int mbf_s = -1, fwidth = 0;
        bool fmask = false;
        if (fs < F) {
            mbf_s = s.missing_bin[fs];
            fwidth = s.widths[fs];
            fmask = s.feature_mask[(size_t)rd.tree_index * F + fs];
        }
        Item it;
        int64_t m_built, m_sib;
        if (root_mode) {
            m_built = root_rows(s);
            m_sib = 0;
            it.part_off = 0;
            const int64_t chk = hist_chunk(s, m_built);
            it.part_cnt = m_built > 0 ? (int)((m_built + chk - 1) / chk) : 0;
            it.hist_built = 0;
            it.hist_sib = 0;
            it.depth_child = 0;
        } else {
            it.begin = readlane_i64(my.begin, j);
            it.end = readlane_i64(my.end, j);
            it.n_left = readlane_i64(my.n_left, j);
            it.builds_left = __builtin_amdgcn_readlane(my.builds_left, j);
            it.hist_built = __builtin_amdgcn_readlane(my.hist_built, j);
            it.hist_sib = __builtin_amdgcn_readlane(my.hist_sib, j);
            it.depth_child = __builtin_amdgcn_readlane(my.depth_child, j);
            it.part_off = __builtin_amdgcn_readlane(my.part_off, j);
            it.part_cnt = __builtin_amdgcn_readlane(my.part_cnt, j);
            const int64_t m = it.end - it.begin;
            m_built = it.builds_left ? it.n_left : m - it.n_left;
            m_sib = m - m_built;
        }
        // ---- merge the accumulated child's partials: thread -> (feature, half, bin)
        {
            const int q = tid >> 7, half = (tid >> 6) & 1, bin = lane;
            const int f = f0 + q;
            int g = 0, h = 0, c = 0;
            // the parent's cells (the sibling is parent - accumulated) are
            // loaded with the partials, one memory round trip for both
            int32_t *pp = nullptr;
            int pg0 = 0, ph0 = 0, pc0 = 0;
            if (half == 0 && !root_mode && f < F && bin < nb) {
                pp = s.hist + (size_t)it.hist_sib * hsz + ((size_t)f * nb + bin) * 3;
                pg0 = pp[0];
                ph0 = pp[1];
                pc0 = pp[2];
            }
            if (f < F && bin < nb) {
                const size_t pstride = (size_t)F * s.part_stride;
                const unsigned long long *p =
                    s.part + (size_t)it.part_off * pstride + (size_t)f * s.part_stride + bin;
                const int np = it.part_cnt;
                int b = half;
                if (hp.wide) {
                    const uint32_t *pc =
                        s.part_c + (size_t)it.part_off * pstride + (size_t)f * s.part_stride + bin;
                    uint32_t ug = 0u, uh = 0u, uc = 0u;
                    for (; b < np; b += 2) {
                        const unsigned long long vv = p[(size_t)b * pstride];
                        ug += (uint32_t)(vv >> 32);
                        uh += (uint32_t)vv;
                        uc += pc[(size_t)b * pstride];
                    }
                    g = (int)ug;
                    h = (int)uh;
                    c = (int)uc;
                } else {
                    for (; b + 14 < np; b += 16) {
                        unsigned long long vv[8];
#pragma unroll
                        for (int u = 0; u < 8; ++u) vv[u] = p[(size_t)(b + 2 * u) * pstride];
#pragma unroll
                        for (int u = 0; u < 8; ++u) {
                            c += (int)(vv[u] & 0xFFFFFULL);
                            h += (int)((vv[u] >> 20) & 0x3FFFFFULL);
                            g += (int)((long long)vv[u] >> 42);
                        }
                    }
                    for (; b < np; b += 2) {
                        const unsigned long long vv = p[(size_t)b * pstride];
                        c += (int)(vv & 0xFFFFFULL);
                        h += (int)((vv >> 20) & 0x3FFFFFULL);
                        g += (int)((long long)vv >> 42);
                    }
                }
            }
            if (half == 1) {
                acc[q][0][bin] = g;
                acc[q][1][bin] = h;
                acc[q][2][bin] = c;
            }
            __syncthreads();
            if (half == 0) {
                g += acc[q][0][bin];
                h += acc[q][1][bin];
                c += acc[q][2][bin];
                cv[q][0][0][bin] = g;
                cv[q][0][1][bin] = h;
                cv[q][0][2][bin] = c;
                int sgv = 0, shv = 0, scv = 0;
                if (f < F && bin < nb) {
                    int32_t *ob = s.hist + (size_t)it.hist_built * hsz + ((size_t)f * nb + bin) * 3;
                    ob[0] = g;
                    ob[1] = h;
                    ob[2] = c;
                    if (!root_mode) {
                        sgv = pg0 - g;
                        shv = ph0 - h;
                        scv = pc0 - c;
                        pp[0] = sgv;
                        pp[1] = shv;
                        pp[2] = scv;
                    }
                }
                cv[q][1][0][bin] = sgv;
                cv[q][1][1][bin] = shv;
                cv[q][1][2][bin] = scv;
            }
            __syncthreads();
        }
        // ---- scan: wave -> (feature, child), lane = bin
        const int q = wv >> 1, child = wv & 1, bin = lane;
        const int f = f0 + q;
        if (f < F && !(root_mode && child == 1)) {  // wave-uniform
            const int vg = cv[q][child][0][bin], vh = cv[q][child][1][bin], vc = cv[q][child][2][bin];
            const int lg = wave_incl_scan_i(vg), lh = wave_incl_scan_i(vh), lc = wave_incl_scan_i(vc);
            const int TG = __builtin_amdgcn_readlane(lg, 63), TH = __builtin_amdgcn_readlane(lh, 63),
                      TC = __builtin_amdgcn_readlane(lc, 63);
            const int64_t n_child = child == 0 ? m_built : m_sib;
            const int mbf = mbf_s;  // f == fs
            const bool gated = (hp.max_depth > 0 && it.depth_child >= hp.max_depth) ||
                               n_child < 2 * (int64_t)hp.min_data_in_leaf || n_child < 2 || !fmask;
            double best_gain = 0.0;
            int best_order = 0x7FFFFFFF;
            int best_left = 0;
            if (!gated) {
                const int mg = mbf >= 0 ? cv[q][child][0][mbf] : 0, mh = mbf >= 0 ? cv[q][child][1][mbf] : 0,
                          mc = mbf >= 0 ? cv[q][child][2][mbf] : 0;
                const long long min_c = hp.min_data_in_leaf;
                const int n_scan = mbf >= 0 ? mbf : nb;
                int lim = n_scan < fwidth ? n_scan : fwidth;
                if (mc == 0 && lim > n_scan - 1) lim = n_scan - 1;
                if (bin < lim) {
                    const double parent = qscore(TG, TH, gu, hu, l1, l2);
                    if (mbf >= 0) {
                        const int ag = lg + mg, ah = lh + mh, ac = lc + mc;
                        const int rg = TG - ag, rh = TH - ah, rc = TC - ac;
                        if (!(ah < hmin || rh < hmin || ac < min_c || rc < min_c)) {
                            const double gain =
                                qscore(ag, ah, gu, hu, l1, l2) + qscore(rg, rh, gu, hu, l1, l2) - parent;
                            if (gain > best_gain) {
                                best_gain = gain;
                                best_order = 2 * bin;
                                best_left = ac;
                            }
                        }
                    }
                    if (mbf < 0 || mc > 0) {
                        const int rg = TG - lg, rh = TH - lh, rc = TC - lc;
                        if (!(lh < hmin || rh < hmin || lc < min_c || rc < min_c)) {
                            const double gain =
                                qscore(lg, lh, gu, hu, l1, l2) + qscore(rg, rh, gu, hu, l1, l2) - parent;
                            if (gain > best_gain) {
                                best_gain = gain;
                                best_order = 2 * bin + 1;
                                best_left = lc;
                            }
                        }
                    }
                }
            }
            const int mine = best_order;
            wave_argmax(best_gain, best_order);
            const unsigned long long wins = __ballot(mine == best_order && best_order != 0x7FFFFFFF);
            const int srcl = wins ? (int)__ffsll((long long)wins) - 1 : 0;
            best_left = __shfl(best_left, srcl, 64);
            if (lane == 0) {
                ScanResult rs;
                rs.gain = best_gain;
                rs.found = best_order != 0x7FFFFFFF;
                rs.bin = rs.found ? best_order >> 1 : -1;
                rs.default_left = rs.found ? ((best_order & 1) == 0) : 0;
                rs.cat = 0;
                rs.tot_g = TG;
                rs.tot_h = TH;
                rs.tot_c = TC;
                rs.n_left = rs.found ? best_left : 0;
                const size_t ri = (size_t)(j * 2 + child) * F + f;
                s.scan[ri] = rs;
                s.scan_gain[ri] = rs.found ? rs.gain : -1.0;
            }
        }
        __syncthreads();  // the LDS tiles are rewritten by the next task
    }
}

template <bool kCat>
__global__ __launch_bounds__(kScanThreads, kCat ? 1 : 4) void k_scan_f(DevState s, int root_mode) {
    __shared__ __align__(16) double cg[2][256], ch[2][256];
    __shared__ int cc[2][256];
    __shared__ __align__(16) double pg_[2][256], ph_[2][256];
    __shared__ int pc_[2][256];
    __shared__ double accg[256], acch[256];
    __shared__ double ckey[2][256];
    __shared__ int csort[2][256];
    __shared__ int cwcnt[8];
    __shared__ double cdg[2][2];
    __shared__ int cdi[2][2];
    __shared__ long long cdl[2][2];
    __shared__ int accc[256];
    __shared__ double s_tg[2], s_th[2], s_sg[2], s_sh[2];
    __shared__ long long s_tc[2];
    __shared__ double wgain[8];
    __shared__ int word[8];
    __shared__ long long wleft[8];
    const int tid = threadIdx.x, lane = lane_id(), wv = tid >> 6;
    const HyperParams &hp = s.hp;
    const int F = s.n_features, nb = s.n_bins;
    const size_t hsz = (size_t)F * nb;
    const int n_items = root_mode ? 1 : s.batch->n_items;
    const int n_tasks = n_items * F;
    if ((int)blockIdx.x >= n_tasks) return;
    const Round rd = *s.round;
    if (rd.stopped) return;
    const double l1 = hp.lambda_l1, l2 = hp.lambda_l2, min_h = hp.min_sum_hessian;
    const long long min_c = hp.min_data_in_leaf;
    for (int task = blockIdx.x; task < n_tasks; task += gridDim.x) {
        // with category-set features, tasks go feature-major in scan_order
        // (those features first: their searches run longest, so the
        // shorter numerical tasks fill in behind them)
        int j, f;
        if (kCat && s.scan_order != nullptr) {
            const int pos = task / n_items;
            j = task - pos * n_items;
            f = s.scan_order[pos];
        } else {
            j = task / F;
            f = task - j * F;
        }
        Item it;
        int64_t m_built, m_sib;
        if (root_mode) {
            m_built = root_rows(s);
            m_sib = 0;
            it.part_off = 0;
            const int64_t chk = hist_chunk(s, m_built);
            it.part_cnt = m_built > 0 ? (int)((m_built + chk - 1) / chk) : 0;
            it.hist_built = 0;
            it.hist_sib = 0;
            it.depth_child = 0;
        } else {
            it = s.items[j];
            const int64_t m = it.end - it.begin;
            m_built = it.builds_left ? it.n_left : m - it.n_left;
            m_sib = m - m_built;
        }
        // ---- merge (thread -> (bin, half))
        {
            const int bin = tid & 255, half = tid >> 8;
            double g = 0.0, h = 0.0;
            int c = 0;
            // the parent's cell (the sibling is parent - accumulated) is
            // loaded with the partials, one memory round trip for both
            HistF *pp = nullptr;
            HistF pv{};
            if (half == 0 && !root_mode && bin < nb) {
                pp = s.histf + (size_t)it.hist_sib * hsz + (size_t)f * nb + bin;
                pv = *pp;
            }
            if (bin < nb) {
                const size_t pstride = (size_t)F * s.part_stride;
                // the item's partials of this feature through buffer loads
                // (a 32-bit offset per load instead of a 64-bit address, so
                // kMU partials' loads fit in flight); added in partial order
                constexpr int kMU = 6;
                const size_t ubase = (size_t)it.part_off * pstride + (size_t)f * s.part_stride;
                const int np = it.part_cnt;
                // byte offsets of the item's partials fit 32 bits (else
                // the addresses are formed in 64 bits, one partial at a time)
                const bool fits = (uint64_t)np * (uint64_t)pstride * 8ull < (1ull << 32);  // task-uniform
                const uint32_t span = fits ? (uint32_t)((size_t)np * pstride) : 0u;  // elements
                const __amdgpu_buffer_rsrc_t rg = buffer_rsrc(s.fpart_g + ubase, span * 8u);
                const __amdgpu_buffer_rsrc_t rh = buffer_rsrc(s.fpart_h + ubase, span * 8u);
                const __amdgpu_buffer_rsrc_t rc = buffer_rsrc(s.fpart_c + ubase, span * 4u);
                auto ld = [&](uint32_t e, double &xg, double &xh, uint32_t &xc) {
                    xg = __builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(rg, e * 8u, 0, 0));
                    xh = __builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(rh, e * 8u, 0, 0));
                    xc = __builtin_amdgcn_raw_buffer_load_b32(rc, e * 4u, 0, 0);
                };
                int b = half;
                if (!fits) {
                    for (; b < np; b += 2) {
                        const size_t at = ubase + (size_t)b * pstride + bin;
                        g += s.fpart_g[at];
                        h += s.fpart_h[at];
                        c += (int)s.fpart_c[at];
                    }
                }
                for (; b + 2 * kMU - 2 < np; b += 2 * kMU) {
                    double vg[kMU], vh[kMU];
                    uint32_t vc[kMU];
#pragma unroll
                    for (int u = 0; u < kMU; ++u)
                        ld((uint32_t)bin + (uint32_t)(b + 2 * u) * (uint32_t)pstride, vg[u], vh[u], vc[u]);
#pragma unroll
                    for (int u = 0; u < kMU; ++u) {
                        g += vg[u];
                        h += vh[u];
                        c += (int)vc[u];
                    }
                }
                for (; b < np; b += 2) {
                    double xg, xh;
                    uint32_t xc;
                    ld((uint32_t)bin + (uint32_t)b * (uint32_t)pstride, xg, xh, xc);
                    g += xg;
                    h += xh;
                    c += (int)xc;
                }
            }
            if (half == 1) {
                accg[bin] = g;
                acch[bin] = h;
                accc[bin] = c;
            }
            __syncthreads();
            if (half == 0) {
                g += accg[bin];
                h += acch[bin];
                c += accc[bin];
                cg[0][bin] = g;
                ch[0][bin] = h;
                cc[0][bin] = c;
                double sgv = 0.0, shv = 0.0;
                int scv = 0;
                if (bin < nb) {
                    HistF *ob = s.histf + (size_t)it.hist_built * hsz + (size_t)f * nb + bin;
                    ob->g = g;
                    ob->h = h;
                    ob->c = c;
                    if (!root_mode) {
                        sgv = pv.g - g;
                        shv = pv.h - h;
                        scv = (int)(pv.c - c);
                        pp->g = sgv;
                        pp->h = shv;
                        pp->c = scv;
                    }
                }
                cg[1][bin] = sgv;
                ch[1][bin] = shv;
                cc[1][bin] = scv;
            }
            __syncthreads();
        }
        const int child = tid >> 8;
        const int bin = tid & 255;
        // ---- the reference's sums per child, split over four waves:
        //  wave 0: the sequential prefix sums (lane 2c + q: child c, grad
        //    cells for q = 0, hess for q = 1), eight cells per step with the
        //    next eight in flight;
        //  wave 1: the eight-way totals (lane 16c + 8q + k sums cells k,
        //    k + 8, ... of the full 8-cell blocks in order, then the lanes
        //    pair up as (k, k + 4), (k, k + 2), (0, 1) and the last partial
        //    block is added in order);
        //  waves 2, 3: the count prefixes of child 0, 1 (integers: a wave
        //    scan gives the same values as the sequential sum; the last
        //    prefix is the total).
        if (wv == 0) {
            if (lane < 4) {
                const int c = lane >> 1, q = lane & 1;
                const double *src = q ? ch[c] : cg[c];
                double *dst = q ? ph_[c] : pg_[c];
                double r = 0.0;
                int b = 0;
                if (nb >= 8) {
                    // two register blocks of eight cells taking turns: one is
                    // added while the other's cells are requested (loads
                    // clamped in bounds of the 256-cell rows; past the last
                    // full block unused)
                    double2 xa[4], xb[4];
                    auto ld8 = [&](double2 *x, int at) {
                        const int c8 = at <= 248 ? at : 248;
#pragma unroll
                        for (int u = 0; u < 4; ++u) x[u] = ((const double2 *)(src + c8))[u];
                    };
                    auto add8 = [&](const double2 *x, int at) {
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            r += x[u].x;
                            const double r0 = r;
                            r += x[u].y;
                            ((double2 *)(dst + at))[u] = make_double2(r0, r);
                        }
                    };
                    ld8(xa, 0);
                    for (; b + 16 <= nb; b += 16) {
                        ld8(xb, b + 8);
                        add8(xa, b);
                        ld8(xa, b + 16);
                        add8(xb, b + 8);
                    }
                    if (b + 8 <= nb) {
                        add8(xa, b);
                        b += 8;
                    }
                }
                for (; b < nb; ++b) {
                    r += src[b];
                    dst[b] = r;
                }
                if (q == 0) s_sg[c] = r;
                else s_sh[c] = r;
            }
        } else if (wv == 1) {
            const int c = (lane >> 4) & 1, q = (lane >> 3) & 1, kk = lane & 7;
            const double *src = q ? ch[c] : cg[c];
            const int full = nb & ~7;  // cells in full 8-cell blocks
            double a = 0.0;
            int j = kk;
            for (; j + 24 < full; j += 32) {
                const double v0 = src[j], v1 = src[j + 8], v2 = src[j + 16], v3 = src[j + 24];
                a += v0;
                a += v1;
                a += v2;
                a += v3;
            }
            for (; j < full; j += 8) a += src[j];
            a += __shfl_down(a, 4, 64);
            a += __shfl_down(a, 2, 64);
            a += __shfl_down(a, 1, 64);
            if (lane < 32 && kk == 0) {
                double t = a;
                for (int bb = full; bb < nb; ++bb) t += src[bb];
                if (q == 0) s_tg[c] = t;
                else s_th[c] = t;
            }
        } else if (wv < 4) {
            const int c = wv - 2;
            const int *csrc = cc[c];
            int *cdst = pc_[c];
            int pfx[4];
            int run = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int cell = 4 * lane + i;
                run += cell < nb ? csrc[cell] : 0;
                pfx[i] = run;
            }
            int incl = run;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const int o = __shfl_up(incl, d, 64);
                incl += lane >= d ? o : 0;
            }
            const int excl = incl - run;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int cell = 4 * lane + i;
                if (cell < nb) cdst[cell] = excl + pfx[i];
            }
            if (lane == 63) s_tc[c] = incl;
        }
        __syncthreads();
        const double TG = s_tg[child], TH = s_th[child];
        const long long TC = s_tc[child];
        const int64_t n_child = child == 0 ? m_built : m_sib;
        const int mbf = s.missing_bin[f];
        const bool gated = (root_mode && child == 1) ||
                           (hp.max_depth > 0 && it.depth_child >= hp.max_depth) ||
                           n_child < 2 * (int64_t)hp.min_data_in_leaf || n_child < 2 ||
                           !s.feature_mask[(size_t)rd.tree_index * F + f];
        double best_gain = 0.0;
        int best_order = 0x7FFFFFFF;
        long long best_left = 0;
        // a categorical feature: category sets over the Float64 cells, the
        // oracle's arithmetic (categorical.find_best_categorical_split,
        // categorical.mojo:684-782) with the totals above; the walk adds the
        // sorted categories' sums in order, one thread per direction
        const int ncf = kCat && s.ncat ? s.ncat[f] : 0;  // block-uniform
        const bool cat_onehot = ncf > 0 && (hp.one_hot_max_size >= 0 ? ncf <= hp.one_hot_max_size
                                                                      : ncf + 1 <= hp.max_cat_to_onehot);
        bool cat_sorted = false;
        auto leaf = [&](double g, double h, double l2x) {
            const double tl = soft_threshold_l1(g, l1);
            return tl * tl / (h + l2x);
        };
        if (ncf > 0) {
            const double parent = leaf(TG, TH, l2);
            const double vg = cg[child][bin], vh = ch[child][bin];
            const long long vc = cc[child][bin];
            if (cat_onehot) {
                if (!gated && ncf >= 2 && bin >= 1 && bin <= ncf && !(vc < min_c || vh < min_h) &&
                    !(TC - vc < min_c) && !(TH - vh < min_h)) {
                    const double gain = leaf(vg, vh, l2) + leaf(TG - vg, TH - vh, l2) - parent;
                    if (gain > best_gain) {
                        best_gain = gain;
                        best_order = bin;
                        best_left = vc;
                    }
                }
            } else {
                cat_sorted = true;
                const bool cand = !gated && ncf >= 2 && bin >= 1 && bin <= ncf && (double)vc >= hp.cat_smooth;
                const double key = vg / (vh + hp.cat_smooth);
                ckey[child][bin] = cand ? key : 0.0;
                const unsigned long long cm = __ballot(cand);
                if (lane == 0) cwcnt[wv] = __popcll(cm);
                csort[child][bin] = cand ? 1 : 0;
                __syncthreads();
                int rank = 0;
                if (cand)
                    for (int u = 1; u <= ncf; ++u) {
                        const double ku = ckey[child][u];
                        rank += (csort[child][u] != 0 && (ku < key || (ku == key && u < bin))) ? 1 : 0;
                    }
                const int used = cwcnt[child << 2] + cwcnt[(child << 2) + 1] + cwcnt[(child << 2) + 2] +
                                 cwcnt[(child << 2) + 3];
                __syncthreads();
                if (cand) csort[child][rank] = bin;
                __syncthreads();
                // each direction's wave: its lanes load the steps' cells, a
                // uniform pass adds them in the walk's order and takes the
                // walk's decisions (continue / break / min_data_per_group
                // groups), then the evaluated steps are scored in parallel;
                // the first maximum wins (strict '>' along the walk)
                const int dthr = (tid & 255) >> 6;  // waves 0 and 1 of the half: directions 0 and 1
                if (dthr < 2) {
                    const int d = dthr;
                    double dg = 0.0;
                    int di = -1;
                    long long dl_ = 0;
                    if (used >= 2) {
                        int max_num_cat = hp.max_cat_threshold;
                        if ((used + 1) / 2 < max_num_cat) max_num_cat = (used + 1) / 2;
                        if (max_num_cat < 0) max_num_cat = 0;
                        const int steps = used < max_num_cat ? used : max_num_cat;
                        const double l2c = l2 + hp.cat_l2;
                        double ag = 0.0, ah = 0.0;
                        long long ac = 0, agg = 0;
                        bool stop = false;
                        for (int c0 = 0; c0 < steps && !stop; c0 += 64) {
                            const int i = c0 + lane;
                            const bool in = i < steps;
                            const int tb = in ? csort[child][d == 0 ? i : used - 1 - i] : 0;
                            const double xg = in ? cg[child][tb] : 0.0, xh = in ? ch[child][tb] : 0.0;
                            const int xc = in ? (int)cc[child][tb] : 0;
                            double mg = 0.0, mh = 0.0;
                            long long mc = 0;
                            bool mev = false;
                            const int n_here = steps - c0 < 64 ? steps - c0 : 64;
                            for (int k = 0; k < n_here; ++k) {
                                ag = ag + rl_f64(xg, k);
                                ah = ah + rl_f64(xh, k);
                                const long long kc = __builtin_amdgcn_readlane(xc, k);
                                ac += kc;
                                agg += kc;
                                bool ev = false;
                                if (!(ac < min_c || ah < min_h)) {
                                    const long long rc = TC - ac;
                                    if (rc < min_c || rc < hp.min_data_per_group || TH - ah < min_h) {
                                        stop = true;
                                        break;
                                    }
                                    if (agg >= hp.min_data_per_group) {
                                        ev = true;
                                        agg = 0;
                                    }
                                }
                                if (lane == k) {
                                    mg = ag;
                                    mh = ah;
                                    mc = ac;
                                    mev = ev;
                                }
                            }
                            double bg = 0.0;
                            int bo = 0x7FFFFFFF;
                            if (mev) {
                                const double g_ = leaf(mg, mh, l2c) + leaf(TG - mg, TH - mh, l2c) - parent;
                                if (g_ > 0.0) {
                                    bg = g_;
                                    bo = i;
                                }
                            }
                            const int mine = bo;
                            wave_argmax(bg, bo);
                            if (bo != 0x7FFFFFFF && bg > dg) {
                                const unsigned long long wl = __ballot(mine == bo);
                                dg = bg;
                                di = bo;
                                dl_ = __builtin_amdgcn_readlane((int)mc, (int)__builtin_ctzll(wl));
                            }
                        }
                    }
                    if (lane == 0) {
                        cdg[child][d] = dg;
                        cdi[child][d] = di;
                        cdl[child][d] = dl_;
                    }
                }
                __syncthreads();
            }
        } else if (!gated) {
            const double mg = mbf >= 0 ? cg[child][mbf] : 0.0, mh = mbf >= 0 ? ch[child][mbf] : 0.0;
            const long long mc = mbf >= 0 ? cc[child][mbf] : 0;
            const int n_scan = mbf >= 0 ? mbf : nb;
            int lim = n_scan < s.widths[f] ? n_scan : s.widths[f];
            if (mc == 0 && lim > n_scan - 1) lim = n_scan - 1;
            if (bin < lim) {
                const double pgs = soft_threshold_l1(TG, l1);
                const double parent_score = pgs * pgs / (TH + l2);
                const double lgs = pg_[child][bin], lhs = ph_[child][bin];
                const long long lcs = pc_[child][bin];
                if (mbf >= 0) {
                    const double a = lgs + mg, ah = lhs + mh;
                    const long long ac = lcs + mc;
                    const double rg = TG - a, rh = TH - ah;
                    if (!(ah < min_h || rh < min_h || ac < min_c || TC - ac < min_c)) {
                        const double tl = soft_threshold_l1(a, l1), tr = soft_threshold_l1(rg, l1);
                        const double gain = tl * tl / (ah + l2) + tr * tr / (rh + l2) - parent_score;
                        if (gain > best_gain) {
                            best_gain = gain;
                            best_order = 2 * bin;
                            best_left = ac;
                        }
                    }
                }
                if (mbf < 0 || mc > 0) {
                    const double rg = TG - lgs, rh = TH - lhs;
                    if (!(lhs < min_h || rh < min_h || lcs < min_c || TC - lcs < min_c)) {
                        const double tl = soft_threshold_l1(lgs, l1), tr = soft_threshold_l1(rg, l1);
                        const double gain = tl * tl / (lhs + l2) + tr * tr / (rh + l2) - parent_score;
                        if (gain > best_gain) {
                            best_gain = gain;
                            best_order = 2 * bin + 1;
                            best_left = lcs;
                        }
                    }
                }
            }
        }
        {
            const int mine = best_order;
            wave_argmax(best_gain, best_order);
            const unsigned long long wins = __ballot(mine == best_order && best_order != 0x7FFFFFFF);
            const int srcl = wins ? (int)__ffsll((long long)wins) - 1 : 0;
            best_left = __shfl(best_left, srcl, 64);
        }
        if (lane == 0) {
            wgain[wv] = best_gain;
            word[wv] = best_order;
            wleft[wv] = best_left;
        }
        __syncthreads();
        if ((tid & 255) == 0 && !(root_mode && child == 1)) {
            double bgn = wgain[child << 2];
            int bo = word[child << 2];
            long long bleft = wleft[child << 2];
            for (int k = 1; k < 4; ++k) {
                const double og = wgain[(child << 2) + k];
                const int oo = word[(child << 2) + k];
                if (og > bgn || (og == bgn && oo < bo)) {
                    bgn = og;
                    bo = oo;
                    bleft = wleft[(child << 2) + k];
                }
            }
            ScanResult rs;
            unsigned long long cbits[4] = {0ULL, 0ULL, 0ULL, 0ULL};
            if (ncf > 0) {
                rs.gain = 0.0;
                rs.found = 0;
                rs.n_left = 0;
                if (cat_sorted) {
                    int d = -1;
                    if (cdi[child][0] >= 0) d = 0;
                    if (cdi[child][1] >= 0 && (d < 0 || cdg[child][1] > cdg[child][0])) d = 1;
                    if (d >= 0) {
                        int used = 0;
                        for (int k = 0; k < 4; ++k) used += cwcnt[(child << 2) + k];
                        for (int i = 0; i <= cdi[child][d]; ++i) {
                            const int tb = csort[child][d == 0 ? i : used - 1 - i];
                            cbits[tb >> 6] |= 1ULL << (tb & 63);
                        }
                        rs.gain = cdg[child][d];
                        rs.found = 1;
                        rs.n_left = cdl[child][d];
                    }
                } else if (bo != 0x7FFFFFFF) {
                    cbits[bo >> 6] |= 1ULL << (bo & 63);
                    rs.gain = bgn;
                    rs.found = 1;
                    rs.n_left = bleft;
                }
                rs.bin = -1;
                rs.default_left = 0;
                rs.cat = rs.found;
            } else {
                rs.gain = bgn;
                rs.found = bo != 0x7FFFFFFF;
                rs.bin = rs.found ? bo >> 1 : -1;
                rs.default_left = rs.found ? ((bo & 1) == 0) : 0;
                rs.cat = 0;
                rs.n_left = rs.found ? bleft : 0;
            }
            rs.tot_g = 0;
            rs.tot_h = 0;
            rs.tot_c = TC;
            rs.fg = s_sg[child];
            rs.fh = s_sh[child];
            const size_t ri = (size_t)(j * 2 + child) * F + f;
            s.scan[ri] = rs;
            s.scan_gain[ri] = rs.found ? rs.gain : -1.0;
            if (ncf > 0)
                for (int w = 0; w < 4; ++w) s.scan_cat[ri * 4 + w] = cbits[w];
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------- pair fold
// With more than 64 features the planner cannot take a pair's per-feature
// gains in one wave load: one block per (child) pair folds them here, after
// the scan -- the feature of largest gain (gain > 0, lowest feature on equal
// gains, as the planner's own fold) -- so the planner's single block reads
// one (gain, feature) per pair instead of F gains (C4: 2000 features x 64
// pairs, a megabyte through one CU).
constexpr int kFoldThreads = 256;
__global__ __launch_bounds__(kFoldThreads) void k_fold(DevState s, int root_mode) {
    __shared__ double wg[kFoldThreads / 64];
    __shared__ int wf[kFoldThreads / 64];
    const int n_pairs = root_mode ? 1 : 2 * s.batch->n_items;
    const int pr = blockIdx.x;
    if (pr >= n_pairs) return;
    const int F = s.n_features, tid = threadIdx.x, lane = lane_id(), wv = tid >> 6;
    const double *q = s.scan_gain + (size_t)pr * F;
    double bg = 0.0;
    int bf = 0x7FFFFFFF;
    // eight loads in flight per thread, ascending features per thread (strict
    // '>' keeps the lowest of equal gains)
    for (int f0 = tid; f0 < F; f0 += 8 * kFoldThreads) {
        double v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int f = f0 + u * kFoldThreads;
            v[u] = f < F ? q[f] : -1.0;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int f = f0 + u * kFoldThreads;
            if (v[u] > 0.0 && v[u] > bg) {
                bg = v[u];
                bf = f;
            }
        }
    }
    wave_argmax_lex(bg, bf);
    if (lane == 0) {
        wg[wv] = bg;
        wf[wv] = bf;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < kFoldThreads / 64; ++w)
            if (wg[w] > bg || (wg[w] == bg && wf[w] < bf)) {
                bg = wg[w];
                bf = wf[w];
            }
        s.pair_gain[pr] = bf != 0x7FFFFFFF ? bg : 0.0;
        s.pair_feat[pr] = bf;
    }
}

// ------------------------------------------------------------------ planner
// Single block of kPlanThreads, after every scan launch.
//
// 1. Fold: for each child of each expanded item, the feature of largest gain
//    (strict '>', lowest feature on ties, gain > 0) becomes the child's best
//    split; with the child's totals and leaf value (quantized_leaf_output)
//    it is stored in the child's explored node.
// 2. Replay: the reference's best-first order (tree.grow_tree_leaves_profiled;
//    growth_policy.GrowthSchedule.next_leaf, src/mojotrees/growth_policy.mojo:
//    659-677: the frontier slot of largest gain wins, lowest slot on ties,
//    gain must be > 0, stop at num_leaves) over the explored nodes: each pick
//    whose leaf is already expanded is committed -- node ids left = n_nodes,
//    right = n_nodes + 1, the left child keeps the parent's slot, the right
//    one takes slot n_leaves -- until a pick needs an unexpanded leaf or the
//    tree is complete.
// 3. Selection: best-first continues over the explored tree as if every
//    expanded leaf were committed; each pick that is not expanded joins the
//    next batch and counts as one split, until num_leaves would be reached
//    or the batch holds min(kmax, remaining splits, free expansions -
//    (remaining splits - 1)) leaves. The first pick is the leaf the replay
//    waits for; the budget rule leaves an expansion for every split the
//    replay can still need. Expanding ahead this way follows the order the
//    replay will take, so speculative expansions are mostly used.
constexpr int kPlanThreads = 1024;

// LDS layout of the planner (byte offsets), shared by the host's size query
// and the kernel.
// The fields of a selected leaf's explored node the batch setup needs.
struct SelNode {
    int64_t begin, end, n_left;
    int32_t buf, hist, depth, feature, bin, default_left, cat, pad_;
};

struct PlanLayout {
    size_t sn, mbin;
    size_t wg, eg, sg, cb, kr, wf, el, ep, rw, fr, ci, sl_e, sl_fid, cm_e, cm_fid, cm_lf, sel_e, pcnt, poff, qcnt, qoff, it;
    size_t total;
};

__host__ __device__ inline PlanLayout plan_layout(int L, int E, int K, int F) {
    PlanLayout p;
    size_t o = 0;
    auto take = [&o](size_t bytes, size_t align) {
        o = (o + align - 1) & ~(align - 1);
        const size_t at = o;
        o += bytes;
        return at;
    };
    p.wg = take((size_t)8 * 2 * K, 8);       // pair's best gain
    p.eg = take((size_t)8 * E, 8);           // explored node's gain view
    p.sg = take((size_t)8 * L, 8);           // frontier slot's gain
    p.cb = take((size_t)8 * E, 8);           // replay: left child's gain; selection: bottleneck values
    p.kr = take((size_t)8 * E, 8);           // replay: right child's gain; selection: fr, ci
    p.fr = p.kr;                             // in the committed frontier
    p.ci = p.kr + (size_t)4 * E;             // jump pointers, then candidates' node ids
    p.wf = take((size_t)4 * 2 * K, 4);       // pair's best feature
    p.el = take((size_t)4 * E, 4);           // explored node's left child
    p.ep = take((size_t)4 * E, 4);           // explored node's parent
    p.rw = take((size_t)4 * E, 4);           // explored node's rows
    p.sl_e = take((size_t)4 * L, 4);
    p.sl_fid = take((size_t)4 * L, 4);
    p.cm_e = take((size_t)4 * L, 4);
    p.cm_fid = take((size_t)4 * L, 4);
    p.cm_lf = take((size_t)4 * L, 4);
    p.sel_e = take((size_t)4 * K, 4);
    p.pcnt = take((size_t)4 * K, 4);
    p.poff = take((size_t)4 * (K + 1), 4);
    p.qcnt = take((size_t)4 * K, 4);
    p.qoff = take((size_t)4 * (K + 1), 4);
    p.it = take(sizeof(Item) * K, 16);
    p.sn = take(sizeof(SelNode) * K, 16);    // the selected leaves' nodes
    p.mbin = take((size_t)4 * F, 4);         // missing bin per feature
    p.total = o;
    return p;
}

struct PlanView {
    SelNode *sn;
    int32_t *mbin;
    double *wg, *eg, *sg, *cb, *gr;
    int32_t *wf, *el, *ep, *rw, *fr, *ci, *sl_e, *sl_fid, *cm_e, *cm_fid, *cm_lf, *sel_e, *pcnt, *poff, *qcnt, *qoff;
    Item *it;
};

__device__ PlanView plan_view(const DevState &s, unsigned char *smem) {
    const PlanLayout p = plan_layout(s.hp.num_leaves, s.e_cap, s.kmax, s.n_features);
    PlanView v;
    v.wg = (double *)(smem + p.wg);
    v.eg = (double *)(smem + p.eg);
    v.sg = (double *)(smem + p.sg);
    v.cb = (double *)(smem + p.cb);
    v.gr = (double *)(smem + p.kr);
    v.wf = (int32_t *)(smem + p.wf);
    v.el = (int32_t *)(smem + p.el);
    v.ep = (int32_t *)(smem + p.ep);
    v.rw = (int32_t *)(smem + p.rw);
    v.fr = (int32_t *)(smem + p.fr);
    v.ci = (int32_t *)(smem + p.ci);
    v.sl_e = (int32_t *)(smem + p.sl_e);
    v.sl_fid = (int32_t *)(smem + p.sl_fid);
    v.cm_e = (int32_t *)(smem + p.cm_e);
    v.cm_fid = (int32_t *)(smem + p.cm_fid);
    v.cm_lf = (int32_t *)(smem + p.cm_lf);
    v.sel_e = (int32_t *)(smem + p.sel_e);
    v.pcnt = (int32_t *)(smem + p.pcnt);
    v.poff = (int32_t *)(smem + p.poff);
    v.qcnt = (int32_t *)(smem + p.qcnt);
    v.qoff = (int32_t *)(smem + p.qoff);
    v.it = (Item *)(smem + p.it);
    v.sn = (SelNode *)(smem + p.sn);
    v.mbin = (int32_t *)(smem + p.mbin);
    return v;
}

// Maximum of a 64-bit unsigned value over the 64 lanes (every lane active),
// returned wave-uniform: the DPP steps of wave_max_u32 on both halves, one
// 64-bit compare per step.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ unsigned long long dpp_max_u64_step(unsigned long long x) {
    const unsigned long long o = ((unsigned long long)dpp_u32<CTRL, ROW_MASK>((unsigned)(x >> 32)) << 32) |
                                 dpp_u32<CTRL, ROW_MASK>((unsigned)x);
    return o > x ? o : x;
}
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long x) {
    x = dpp_max_u64_step<0xB1, 0xF>(x);
    x = dpp_max_u64_step<0x4E, 0xF>(x);
    x = dpp_max_u64_step<0x141, 0xF>(x);
    x = dpp_max_u64_step<0x140, 0xF>(x);
    x = dpp_max_u64_step<0x142, 0xA>(x);
    x = dpp_max_u64_step<0x143, 0xC>(x);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(x >> 32), 63);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)x, 63);
    return ((unsigned long long)hi << 32) | lo;
}

// Bitonic sort of 2^LOGN 32-bit keys, descending, one key per thread of a
// kPlanThreads block (thread = position; threads past 2^LOGN pass through).
// Fully unrolled, so every exchange distance j is a constant: quad
// permutations (DPP) for j = 1, 2; a row shift each way and a select for
// j = 4, 8 (row_shl:j reads lane + j, row_shr:j lane - j, both inside the
// lane's row of 16); a swizzle within 32 lanes for 16; a crossbar shuffle
// for 32; through LDS for 64 and more, alternating between two buffers so
// that each such step takes one barrier (a buffer is rewritten two steps
// later, after every thread has passed the barrier between). Only the waves
// that hold the 2^LOGN positions compare and exchange (a position's partners
// are all below 2^LOGN); the others take the LDS steps' barriers and nothing
// else, so they leave the SIMDs to the sorting waves.
template <int LOGN>
__device__ __forceinline__ unsigned bitonic_desc(unsigned x, unsigned (*keys)[kPlanThreads]) {
    const int tid = threadIdx.x, lane = lane_id();
    constexpr int kWaves = (1 << LOGN) > 64 ? (1 << LOGN) / 64 : 1;
    if ((tid >> 6) >= kWaves) {  // wave-uniform
        constexpr int kLdsSteps = LOGN > 6 ? (LOGN - 6) * (LOGN - 5) / 2 : 0;  // steps with j >= 64
#pragma unroll
        for (int i = 0; i < kLdsSteps; ++i) __syncthreads();
        return x;
    }
    int buf = 1;
#pragma unroll
    for (int lk = 1; lk <= LOGN; ++lk) {
        const int k = 1 << lk;
#pragma unroll
        for (int lj = lk - 1; lj >= 0; --lj) {
            const int j = 1 << lj;
            unsigned y;
            if (j >= 64) {
                keys[buf][tid] = x;
                __syncthreads();
                y = keys[buf][tid ^ j];
                buf ^= 1;
            } else if (j == 1) {
                y = dpp_u32<0xB1, 0xF>(x);  // quad_perm [1,0,3,2]
            } else if (j == 2) {
                y = dpp_u32<0x4E, 0xF>(x);  // quad_perm [2,3,0,1]
            } else if (j == 4) {
                const unsigned up = dpp_u32<0x104, 0xF>(x), dn = dpp_u32<0x114, 0xF>(x);
                y = (lane & 4) ? dn : up;
            } else if (j == 8) {
                const unsigned up = dpp_u32<0x108, 0xF>(x), dn = dpp_u32<0x118, 0xF>(x);
                y = (lane & 8) ? dn : up;
            } else if (j == 16) {
                y = (unsigned)__builtin_amdgcn_ds_swizzle((int)x, 0x401F);  // and 0x1F, xor 0x10
            } else {
                y = (unsigned)__shfl_xor((int)x, 32, 64);
            }
            const bool desc = (tid & k) == 0, lower = (tid & j) == 0;
            x = (lower == desc) ? max(x, y) : min(x, y);
        }
    }
    return x;
}

__device__ __forceinline__ double readlane_f64(double d, int l) {
    const unsigned long long b = (unsigned long long)__double_as_longlong(d);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(b >> 32), l);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)b, l);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

// Best-first replay by one wave (tree.grow_tree_leaves_profiled with
// growth_policy.GrowthSchedule.next_leaf: the frontier slot of largest gain
// splits next, lowest slot on ties, gain > 0, until num_leaves). The frontier
// lives in registers: lane l holds slots l, l + 64, ... (QS of them: gain,
// explored node, node id) and its own best slot with that slot's children
// (left child's explored id and both children's gains, loaded from LDS each
// time the lane's best changes, behind the next pick). A pick is the wave
// maximum of the lanes' best gains (non-negative binary64 values order like
// their bits): a 32-bit maximum of the high words and a ballot find the lane
// that holds it; only when several lanes share that high word does a 64-bit
// maximum decide, and only when several hold exactly the same gain does a
// wave minimum pick the lowest slot. A commit rewrites two slots -- the left
// child keeps the parent's slot, the right one takes slot n_leaves; node ids
// left = n_nodes, right = n_nodes + 1 -- and the two lanes holding them
// recompute their best. The replay stops at a pick whose leaf has not been
// expanded yet (x) or when the tree is complete (done).
template <int QS>
__device__ void replay_wave(PlanView &v, int L, int &nl, int &nn, int &nc, int &done, int &x) {
    const int lane = lane_id();
    double sg[QS];
    int se[QS], sf[QS];
#pragma unroll
    for (int q = 0; q < QS; ++q) {
        const int slot = lane + 64 * q;
        const bool in = slot < nl;
        sg[q] = in ? v.sg[slot] : 0.0;  // 0 is never picked (gain must be > 0)
        se[q] = in ? v.sl_e[slot] : 0;
        sf[q] = in ? v.sl_fid[slot] : -1;
    }
    double lbg, kgl, kgr;
    int lbi, lbe, lbf, kle;
    auto local_best = [&]() {
        lbg = 0.0;
        lbi = 0x7FFFFFFF;
        lbe = 0;
        lbf = -1;
#pragma unroll
        for (int q = 0; q < QS; ++q) {
            const bool t = sg[q] > lbg;  // ascending slots: strict '>' keeps the lowest
            lbg = t ? sg[q] : lbg;
            lbi = t ? lane + 64 * q : lbi;
            lbe = t ? se[q] : lbe;
            lbf = t ? sf[q] : lbf;
        }
        kle = v.el[lbe];
        kgl = v.cb[lbe];
        kgr = v.gr[lbe];
    };
    local_best();
    for (;;) {
        if (nl >= L) {
            done = 1;
            break;
        }
        const unsigned long long mine = (unsigned long long)__double_as_longlong(lbg);
        const unsigned hi = (unsigned)(mine >> 32);
        const unsigned mh = wave_max_u32(hi);
        int ol;
        const unsigned long long t1 = __ballot(hi == mh);
        if (mh != 0u && (t1 & (t1 - 1ULL)) == 0ULL) {
            ol = (int)__builtin_ctzll(t1);
        } else {
            // several lanes share the high word (or every best is below
            // 2^-1022): the full 64-bit maximum among them
            const unsigned long long m = wave_max_u64(hi == mh ? mine : 0ULL);
            if (m == 0ULL) {  // no slot with a positive gain
                done = 1;
                break;
            }
            const unsigned long long t2 = __ballot(mine == m);
            if ((t2 & (t2 - 1ULL)) == 0ULL) ol = (int)__builtin_ctzll(t2);
            else ol = (int)(wave_min_u32(mine == m ? (unsigned)lbi : 0xFFFFFFFFu) & 63u);
        }
        const int bi = __builtin_amdgcn_readlane(lbi, ol);
        const int X = __builtin_amdgcn_readlane(lbe, ol);
        const int fid = __builtin_amdgcn_readlane(lbf, ol);
        const int le = __builtin_amdgcn_readlane(kle, ol);
        if (le < 0) {
            x = X;
            break;
        }
        const double gl = readlane_f64(kgl, ol), gr = readlane_f64(kgr, ol);
        if (lane == 0) {
            v.cm_e[nc] = X;
            v.cm_fid[nc] = fid;
            v.cm_lf[nc] = nn;
        }
        const int q = bi >> 6, q2 = nl >> 6, ol2 = nl & 63;
#pragma unroll
        for (int qq = 0; qq < QS; ++qq) {
            if (lane == ol && qq == q) {
                sg[qq] = gl;
                se[qq] = le;
                sf[qq] = nn;
            }
            if (lane == ol2 && qq == q2) {
                sg[qq] = gr;
                se[qq] = le + 1;
                sf[qq] = nn + 1;
            }
        }
        if (lane == ol || lane == ol2) local_best();
        ++nl;
        nn += 2;
        ++nc;
    }
#pragma unroll
    for (int q = 0; q < QS; ++q) {
        const int slot = lane + 64 * q;
        if (slot < nl) {
            v.sg[slot] = sg[q];
            v.sl_e[slot] = se[q];
            v.sl_fid[slot] = sf[q];
        }
    }
}

// The batch header into pinned host memory by system-scope stores (they
// reach host memory whatever the allocation's caching; the host reads them
// after the launch's completion event).
__device__ __forceinline__ void publish_header(Batch *host, const Batch &b) {
    const int32_t *src = (const int32_t *)&b;
    int32_t *dst = (int32_t *)host;
#pragma unroll
    for (int i = 0; i < (int)(sizeof(Batch) / sizeof(int32_t)); ++i)
        __hip_atomic_store(dst + i, src[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// host: when not null (the last planning launch of a group), the batch
// header is also written there, to pinned host memory the host reads after
// the group's event instead of copying the header with a launch of its own.
__global__ __launch_bounds__(kPlanThreads) void k_plan(DevState s, int root_mode, Batch *host) {
    extern __shared__ unsigned char plan_smem[];
    __shared__ Grow g;
    __shared__ int s_nc, s_done, s_ncand, s_nsel, s_total, s_x, s_vf;
    __shared__ unsigned long long s_rows_built, s_rows_parted;
    __shared__ long long s_chunk, s_chunk_p;
    __shared__ int s_total_p;
    const int tid = threadIdx.x, lane = lane_id(), wv = tid >> 6;
    const int nthr = blockDim.x, nwaves = blockDim.x >> 6;
    const int L = s.hp.num_leaves, F = s.n_features;
    const HyperParams &hp = s.hp;
    // When the explored nodes, the frontier, the features and the items fit
    // one per thread, every array the set-up needs is read up to its
    // capacity first, with the batch header below in flight at the same
    // time: one memory round trip instead of two (entries past the header's
    // counts are allocated, read and never used).
    constexpr int kPW = 8;  // fold: pairs per wave (16 waves x 8 >= 2 x 64)
    static_assert(kPlanThreads / 64 * kPW >= 2 * 64, "every pair of a batch in one pass");
    const bool pre = s.e_cap <= kPlanThreads && L <= kPlanThreads;  // launch-uniform
    const bool folded = F > 64;  // k_fold left one (gain, feature) per pair
    double p_eg = 0.0, gq[kPW], p_pg = 0.0;
    int p_pf = 0x7FFFFFFF;
    int p_el = 0, p_ep = 0, p_rw = 0, p_se = 0, p_sf = 0, p_mb = 0;
    static_assert(sizeof(Item) == 64, "an item is four 16-byte words");
    uint4 p_i0 = make_uint4(0, 0, 0, 0), p_i1 = p_i0, p_i2 = p_i0, p_i3 = p_i0;
    if (pre) {
        if (tid < s.e_cap) {
            p_eg = s.e_gain[tid];
            p_el = s.e_left[tid];
            p_ep = s.e_parent[tid];
            p_rw = s.e_rows[tid];
        }
        if (tid < L) {
            p_se = s.slot_e[tid];
            p_sf = s.slot_fid[tid];
        }
        if (tid < F) p_mb = s.missing_bin[tid];
        if (tid < s.kmax) {
            const uint4 *q = (const uint4 *)&s.items[tid];
            p_i0 = q[0];
            p_i1 = q[1];
            p_i2 = q[2];
            p_i3 = q[3];
        }
        if (!folded) {
#pragma unroll
            for (int k = 0; k < kPW; ++k) {
                int pr = wv + k * nwaves;
                pr = pr < 2 * s.kmax ? pr : 0;
                gq[k] = s.scan_gain[(size_t)pr * F + (lane < F ? lane : 0)];
            }
        } else if (tid < 2 * s.kmax) {
            p_pg = s.pair_gain[tid];
            p_pf = s.pair_feat[tid];
        }
    }
    // the batch size, the round and the growth counters in one memory round
    // trip (every thread reads the counters itself, a broadcast load, instead
    // of waiting at a barrier for one thread's copy)
    const int n_items = root_mode ? 1 : s.batch->n_items;
    const Round rd = *s.round;
    const int ne = root_mode ? 1 : s.grow->n_explored, nl0 = root_mode ? 1 : s.grow->n_leaves;
    if (n_items <= 0) {  // the tree is complete
        if (host != nullptr && tid == 0) publish_header(host, *s.batch);
        return;
    }
    PlanView v = plan_view(s, plan_smem);
    if (rd.stopped) {
        // training has stopped: an empty tree, nothing to expand
        if (tid == 0) {
            s.t_meta[0] = 1;
            s.t_meta[1] = 1;
            Batch b;
            b.n_items = 0;
            b.n_blocks = 0;
            b.done = 1;
            b.iters = 0;
            b.n_acc = 0;
            b.chunk_p = b.chunk_a = b.pad_ = 0;
            *s.batch = b;
            if (host != nullptr) publish_header(host, b);
        }
        return;
    }
    const double gu = rd.grad_units, hu = rd.hess_units;
    if (tid == 0) {
        if (root_mode) {
            g.n_leaves = 1;
            g.n_nodes = 1;
            g.n_explored = 1;
            g.n_hist = 1;
            g.expansions = 0;
            g.iterations = 0;
            g.rows_built = 0;
            g.rows_parted = 0;
        } else {
            g = *s.grow;
        }
        s_rows_built = 0;
        s_rows_parted = 0;
        s_ncand = 0;
    }
    // ---- 1. fold (one wave per pair over the pair's per-feature results).
    // The fold's gains, the items, the explored nodes and the frontier are
    // all loaded in one memory round trip, the gains first.
    const int n_pairs = root_mode ? 1 : 2 * n_items;
    // The fold reads the dense gains (scan_gain: the gain of a found split,
    // else -1), 8 bytes per (pair, feature): the planner's one CU moves a
    // few lines per wave load instead of a line per lane. Every load
    // unconditional (a branch between dependent loads would cost a memory
    // round trip each): when F <= 64 wave w takes pairs w + 16 k, k < kPW,
    // lane = feature; the argmax keeps the lowest feature on equal gains.
    // With more features k_fold has already folded each pair (same rule),
    // and thread p reads pair p's (gain, feature).
    if (pre) {
        if (!root_mode && tid < n_items) {
            uint4 *q = (uint4 *)&v.it[tid];
            q[0] = p_i0;
            q[1] = p_i1;
            q[2] = p_i2;
            q[3] = p_i3;
        }
        if (tid < F) v.mbin[tid] = p_mb;
        for (int f = tid + nthr; f < F; f += nthr) v.mbin[f] = s.missing_bin[f];  // F > kPlanThreads
        if (tid < ne) {
            v.eg[tid] = p_eg;
            v.el[tid] = p_el;
            v.ep[tid] = p_ep;
            v.rw[tid] = p_rw;
        }
        if (!root_mode && tid < nl0) {
            v.sl_e[tid] = p_se;
            v.sl_fid[tid] = p_sf;
        }
    } else {
        if (folded) {
            if (tid < n_pairs) {
                p_pg = s.pair_gain[tid];
                p_pf = s.pair_feat[tid];
            }
        } else {
#pragma unroll
            for (int k = 0; k < kPW; ++k) {
                int pr = wv + k * nwaves;
                pr = pr < n_pairs ? pr : 0;
                gq[k] = s.scan_gain[(size_t)pr * F + (lane < F ? lane : 0)];
            }
        }
        if (!root_mode)
            for (int jj = tid; jj < n_items; jj += nthr) v.it[jj] = s.items[jj];
        for (int f = tid; f < F; f += nthr) v.mbin[f] = s.missing_bin[f];
        for (int i = tid; i < ne; i += nthr) {
            v.eg[i] = s.e_gain[i];
            v.el[i] = s.e_left[i];
            v.ep[i] = s.e_parent[i];
            v.rw[i] = s.e_rows[i];
        }
        if (!root_mode)
            for (int i = tid; i < nl0; i += nthr) {
                v.sl_e[i] = s.slot_e[i];
                v.sl_fid[i] = s.slot_fid[i];
            }
    }
    if (hp.quantized) {
        if (tid == 0) s_vf = 0;  // unused: integer sums give the leaf values
    } else if (tid < 64) {
        // the tree's first selected feature (the fp32 path's leaf value sums)
        int vf = F - 1;
        for (int f0 = 0; f0 < F; f0 += 64) {
            const unsigned long long m =
                __ballot(f0 + lane < F && s.feature_mask[(size_t)rd.tree_index * F + f0 + lane]);
            if (m) {
                vf = f0 + (int)__builtin_ctzll(m);
                break;
            }
        }
        if (lane == 0) s_vf = vf;
    }
    if (folded) {
        if (tid < n_pairs) {
            v.wg[tid] = p_pg;
            v.wf[tid] = p_pf;
        }
    } else {  // F <= 64
#pragma unroll
        for (int k = 0; k < kPW; ++k) {
            const int pr = wv + k * nwaves;
            if (pr >= n_pairs) break;  // wave-uniform
            const bool ok = lane < F && gq[k] > 0.0;
            double bg = ok ? gq[k] : 0.0;
            int bf = ok ? lane : 0x7FFFFFFF;
            wave_argmax_lex(bg, bf);
            if (lane == 0) {
                v.wg[pr] = bg;
                v.wf[pr] = bf;
            }
        }
    }
    __syncthreads();
    for (int pr = tid; pr < n_pairs; pr += nthr) {
        int e_id = 0;
        if (!root_mode) {
            const Item &it = v.it[pr >> 1];
            const bool built = (pr & 1) == 0;
            e_id = (built == (it.builds_left != 0)) ? it.left_e : it.left_e + 1;
        }
        const ScanResult *base = &s.scan[(size_t)pr * F];
        const int bf = v.wf[pr];
        const bool found = bf != 0x7FFFFFFF;
        // the three results this pair needs, loaded together
        const long long G = base->tot_g, H = base->tot_h, C = base->tot_c;
        const double fg = base[s_vf].fg, fh = base[s_vf].fh;
        const ScanResult &qb = base[found ? bf : 0];
        const int q_bin = qb.bin, q_dl = qb.default_left, q_cat = qb.cat;
        const long long q_nl = qb.n_left;
        // leaf value: integer sums are the same on every feature; the fp32
        // path sums the tree's first selected feature serially, as
        // tree._leaf_value does (value_feature = tree_features[0])
        const double value = hp.quantized ? qleaf(G, H, gu, hu, hp.lambda_l1, hp.lambda_l2)
                                          : -soft_threshold_l1(fg, hp.lambda_l1) / (fh + hp.lambda_l2);
        ENode *e = &s.enodes[e_id];
        if (root_mode) {
            e->begin = 0;
            e->end = C;
            e->buf = 0;
            e->hist = 0;
            e->depth = 0;
            e->left_e = -1;
            e->right_e = -1;
            s.t_value[0] = value;
            s.t_count[0] = (double)C;
        }
        e->tot_g = G;
        e->tot_h = H;
        e->tot_c = C;
        e->value = value;
        e->found = found ? 1 : 0;
        e->cat = found && q_cat ? 1 : 0;
        if (found && q_cat) {
            const unsigned long long *sb = s.scan_cat + ((size_t)pr * F + bf) * 4;
#pragma unroll
            for (int w = 0; w < 4; ++w) s.e_cat[(size_t)e_id * 4 + w] = sb[w];
        }
        if (found) {
            e->gain = v.wg[pr];
            e->feature = bf;
            e->bin = q_bin;
            e->default_left = q_dl;
            e->n_left = q_nl;
        } else {
            e->gain = 0.0;
            e->feature = -1;
            e->bin = -1;
            e->default_left = 0;
            e->n_left = 0;
        }
        const double eg = found ? v.wg[pr] : -1.0;  // a found split has gain > 0
        v.eg[e_id] = eg;
        s.e_gain[e_id] = eg;
        if (root_mode) {
            v.el[0] = -1;
            v.ep[0] = -1;
            v.rw[0] = (int32_t)C;
            s.e_left[0] = -1;
            s.e_parent[0] = -1;
            s.e_rows[0] = (int32_t)C;
        }
    }
    if (root_mode && tid == 0) {
        v.sl_e[0] = 0;
        v.sl_fid[0] = 0;
    }
    __syncthreads();
    for (int i = tid; i < nl0; i += nthr) v.sg[i] = v.eg[v.sl_e[i]];
    __syncthreads();
    // ---- 2. replay (wave 0), see replay_wave. Each explored node's
    // children gains sit beside it (cb = left, gr = right) so a commit costs
    // one LDS round trip.
    for (int i = tid; i < ne; i += nthr) {
        const int le = v.el[i];
        v.cb[i] = le >= 0 ? v.eg[le] : 0.0;
        v.gr[i] = le >= 0 ? v.eg[le + 1] : 0.0;
    }
    __syncthreads();
    if (tid < 64) {
        int nl = nl0, nn = g.n_nodes, nc = 0, done = 0, x = -1;
        if (L <= 256) replay_wave<4>(v, L, nl, nn, nc, done, x);
        else if (L <= 512) replay_wave<8>(v, L, nl, nn, nc, done, x);
        else replay_wave<16>(v, L, nl, nn, nc, done, x);
        if (lane == 0) {
            s_nc = nc;
            s_done = done;
            s_x = x;
            g.n_leaves = nl;
            g.n_nodes = nn;
        }
        // the committed frontier's marks for the selection (fr reuses the
        // replay's right-child gains, free now); one wave's LDS writes land
        // in order
        for (int i = lane; i < ne; i += 64) v.fr[i] = 0;
        __asm__ volatile("" ::: "memory");
        for (int i = lane; i < nl; i += 64) v.fr[v.sl_e[i]] = 1;
    }
    __syncthreads();
    const int nc = s_nc, nl = g.n_leaves, nn = g.n_nodes;
    // committed splits -> tree arrays
    auto write_commits = [&]() {
        for (int c = tid; c < nc; c += nthr) {
            const ENode *e = &s.enodes[v.cm_e[c]];
            const int fx = v.cm_fid[c], lf = v.cm_lf[c];
            const int le = v.el[v.cm_e[c]];
            // every load first, then the stores
            const int feat = e->feature, ecat = e->cat, ebin = e->bin, edl = e->default_left;
            const double egain = e->gain;
            const double v0 = s.enodes[le].value, v1 = s.enodes[le + 1].value;
            const int64_t c0 = s.enodes[le].tot_c, c1 = s.enodes[le + 1].tot_c;
            s.t_feature[fx] = feat;
            s.t_threshold[fx] = ecat ? -1 : ebin;
            s.t_left[fx] = lf;
            s.t_right[fx] = lf + 1;
            s.t_default_left[fx] = ecat ? 0 : edl;
            // tree._set_split (tree.mojo:462-481): a categorical node has no
            // threshold and no missing bin, only its set
            s.t_missing_bin[fx] = ecat ? -1 : v.mbin[feat];
            if (s.t_cat) {
#pragma unroll
                for (int w = 0; w < 4; ++w)
                    s.t_cat[(size_t)fx * 4 + w] = ecat ? s.e_cat[(size_t)v.cm_e[c] * 4 + w] : 0ULL;
            }
            s.t_gain[fx] = egain;
            s.t_value[lf] = v0;
            s.t_count[lf] = (double)c0;
            s.t_value[lf + 1] = v1;
            s.t_count[lf + 1] = (double)c1;
        }
    };
    auto finish = [&](int err_code) {
        if (tid == 0) {
            if (err_code) atomicOr(s.error, err_code);
            s.t_meta[0] = nn;
            s.t_meta[1] = nl;
            *s.grow = g;
            Batch b;
            b.n_items = 0;
            b.n_blocks = 0;
            b.done = 1;
            b.iters = g.iterations;
            b.n_acc = 0;
            b.chunk_p = b.chunk_a = b.pad_ = 0;
            *s.batch = b;
            if (host != nullptr) publish_header(host, b);
        }
    };
    if (s_done) {
        write_commits();
        for (int i = tid; i < nl; i += nthr) {
            const int fid = v.sl_fid[i];
            s.t_feature[fid] = -1;
            s.t_threshold[fid] = -1;
            s.t_left[fid] = -1;
            s.t_right[fid] = -1;
            s.t_default_left[fid] = 0;
            s.t_missing_bin[fid] = -1;
            s.t_gain[fid] = 0.0;
            if (s.t_cat)
                for (int w = 0; w < 4; ++w) s.t_cat[(size_t)fid * 4 + w] = 0ULL;
        }
        finish(0);
        return;
    }
    // the committed frontier is kept for the next launch
    for (int i = tid; i < nl; i += nthr) {
        s.slot_e[i] = v.sl_e[i];
        s.slot_fid[i] = v.sl_fid[i];
    }
    // ---- 3. selection. Best-first over a tree pops nodes in non-increasing
    // order of their bottleneck value b(v) = the smallest gain on the path
    // from the committed frontier down to v; continuing the replay as if
    // every expanded leaf were committed therefore visits the explored nodes
    // of largest b first. A visited node that is not expanded joins the
    // batch. The visit stops after num_leaves - n_leaves splits (each visit
    // adds one leaf) or when the batch holds `cap` leaves. Ties are broken
    // by node index; the selection only steers speed, never the tree.
    const int r = L - nl;
    int cap = r < s.kmax ? r : s.kmax;
    const int room = (s.max_exp - g.expansions) - (r - 1);
    if (room < cap) cap = room;
    // A speculative leaf (any but the one the replay waits for) joins the
    // batch only when its partition and accumulation cost little against
    // the waited-for leaf's: at most max(n / 2, 2 x its rows) rows. Late in
    // training a root split often peels off a small high-gain region that
    // takes every split while its large sibling never splits; expanding that
    // sibling's subtree ahead doubled the rows a tree partitions and
    // accumulated. Deferred leaves are expanded when the replay reaches them
    // (measured on C2: 45M instead of 76M rows partitioned per tree, 22.1
    // instead of 20.0 iterations, 6 % less time).
    const int64_t spec_rows = s_x >= 0 ? max((int64_t)(s.n / 2), (int64_t)2 * v.rw[s_x]) : (int64_t)s.n;
    // b by pointer chasing: node i carries the smallest gain on its path up
    // to (excluding) up[i]; up = -1 once a frontier node was passed
    // (inside), -2 at the root without one (a committed internal node).
    // Each node's (b, up) is one 64-bit LDS word (b rounded to binary32:
    // the rounding is monotone and b only orders the selection), read and
    // written whole, so a node that follows an ancestor's word always reads
    // a consistent pair -- the ancestor's start or any later step of its own
    // chase -- and takes the min and the pointer from it. Every thread
    // follows its nodes' chains to the end with no barrier between steps
    // (chains are at most the tree's depth and shortened by ancestors that
    // have progressed). Nodes per thread: ne <= e_cap <= 4 x 1024.
    constexpr int kJ = 4;
    unsigned long long *bw = (unsigned long long *)v.cb;
    auto pack_b = [](float b, int up) {
        return ((unsigned long long)__float_as_uint(b) << 32) | (unsigned long long)(uint32_t)up;
    };
    float jv[kJ];
    int ju[kJ];
#pragma unroll
    for (int k = 0; k < kJ; ++k) {
        const int i = tid + k * nthr;
        jv[k] = -1.0f;
        ju[k] = -2;
        if (i < ne) {
            jv[k] = (float)v.eg[i];
            ju[k] = v.fr[i] ? -1 : (v.ep[i] < 0 ? -2 : v.ep[i]);
            __hip_atomic_store(&bw[i], pack_b(jv[k], ju[k]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    }
    __syncthreads();  // every node's starting word is in place
#pragma unroll
    for (int k = 0; k < kJ; ++k) {
        const int i = tid + k * nthr;
        while (ju[k] >= 0) {
            const unsigned long long w = __hip_atomic_load(&bw[ju[k]], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            const float pv = __uint_as_float((unsigned)(w >> 32));
            jv[k] = pv < jv[k] ? pv : jv[k];
            ju[k] = (int)(uint32_t)w;
            __hip_atomic_store(&bw[i], pack_b(jv[k], ju[k]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    }
    // candidates: b > 0 inside the region below the frontier, compacted by
    // wave ballots into (cb, ci): b and the node id, bit 31 set when the
    // node is expanded; the pending (unexpanded) ones are also listed, by
    // their candidate index, in fr (free once the jump pointers are done).
    // The kJ x nwaves ballot counts are scanned by wave 0 in one pass.
    static_assert(kPlanThreads / 64 * kJ == 64, "one wave scans the ballot counts");
    __shared__ int s_wcnt[64], s_pcnt[64];
    __shared__ int s_npend;
    __shared__ unsigned s_keys[2][kPlanThreads];  // the sort's keys (up to kPlanThreads candidates), two buffers
    int myb[kJ], myp[kJ];
#pragma unroll
    for (int k = 0; k < kJ; ++k) {
        const int i = tid + k * nthr;
        const bool c = i < ne && ju[k] == -1 && v.eg[i] > 0.0 && jv[k] > 0.0;
        const bool pend = c && v.el[i] < 0 && (i == s_x || v.rw[i] <= spec_rows);
        const unsigned long long m = __ballot(c), mp = __ballot(pend);
        const unsigned long long below = (1ULL << lane) - 1ULL;
        myb[k] = c ? (int)__popcll(m & below) : -1;
        myp[k] = pend ? (int)__popcll(mp & below) : -1;
        if (lane == 0) {
            s_wcnt[k * nwaves + wv] = __popcll(m);
            s_pcnt[k * nwaves + wv] = __popcll(mp);
        }
    }
    __syncthreads();
    if (tid < 64) {
        const int a = s_wcnt[lane], b = s_pcnt[lane];
        const int ia = wave_incl_scan_i(a), ib = wave_incl_scan_i(b);
        s_wcnt[lane] = ia - a;
        s_pcnt[lane] = ib - b;
        if (lane == 63) {
            s_ncand = ia;
            s_npend = ib;
            s_nsel = 0;
        }
    }
    __syncthreads();
    // up to kPlanThreads candidates are ranked by a sort of 32-bit keys:
    // b rounded to binary32 (a positive float orders like its bits; the
    // rounding is monotone) with the low 12 bits replaced by 0xFFF - node id
    // (ne <= 4096), so that a descending sort puts larger b first and, among
    // b equal to 11 mantissa bits, the lower node id. Keys are at least
    // 0x1000, above the padding 0. The order only steers which leaves are
    // expanded ahead, never the tree.
    const bool by_sort = s_ncand <= kPlanThreads;
#pragma unroll
    for (int k = 0; k < kJ; ++k) {
        if (myb[k] < 0) continue;
        const int i = tid + k * nthr;
        const int kk = s_wcnt[k * nwaves + wv] + myb[k];
        if (by_sort) {
            const unsigned fb = __float_as_uint(jv[k]) & ~0xFFFu;
            s_keys[0][kk] = (fb > 0x1000u ? fb : 0x1000u) | (unsigned)(0xFFF - i);
        } else {
            v.cb[kk] = jv[k];
            v.ci[kk] = i | (myp[k] < 0 ? (int)0x80000000 : 0);
            if (myp[k] >= 0) v.fr[s_pcnt[k * nwaves + wv] + myp[k]] = kk;
        }
    }
    __syncthreads();
    const int ncand = s_ncand, npend = s_npend;
    if (by_sort) {
        // Bitonic sort, descending, one key per thread (tid = position):
        // partners within a wave by lane shuffles, farther ones through LDS.
        // A candidate's position is the number of candidates before it; the
        // pending ones before it, an exclusive count over positions, is its
        // batch slot. Pending candidates at positions below r with a slot
        // below cap join the batch.
        int lg = 0;
        while ((1 << lg) < ncand) ++lg;
        unsigned x = tid < ncand ? s_keys[0][tid] : 0u;
        static_assert(kPlanThreads == 1024, "sorts of up to 2^10 keys");
        switch (lg) {  // block-uniform
        case 1: x = bitonic_desc<1>(x, s_keys); break;
        case 2: x = bitonic_desc<2>(x, s_keys); break;
        case 3: x = bitonic_desc<3>(x, s_keys); break;
        case 4: x = bitonic_desc<4>(x, s_keys); break;
        case 5: x = bitonic_desc<5>(x, s_keys); break;
        case 6: x = bitonic_desc<6>(x, s_keys); break;
        case 7: x = bitonic_desc<7>(x, s_keys); break;
        case 8: x = bitonic_desc<8>(x, s_keys); break;
        case 9: x = bitonic_desc<9>(x, s_keys); break;
        case 10: x = bitonic_desc<10>(x, s_keys); break;
        default: break;  // one candidate
        }
        const bool isc = tid < ncand;
        const int id = isc ? (int)(0xFFF - (int)(x & 0xFFFu)) : 0;
        const bool pend = isc && v.el[id] < 0 && (id == s_x || v.rw[id] <= spec_rows);
        const bool in_r = pend && tid < r;
        const unsigned long long pm = __ballot(pend), rm = __ballot(in_r);
        if (lane == 0) {
            s_wcnt[wv] = __popcll(pm);
            s_pcnt[wv] = __popcll(rm);
        }
        __syncthreads();
        if (tid == 0) {
            int a = 0, t = 0;
            for (int w = 0; w < nwaves; ++w) {
                const int c = s_wcnt[w];
                s_wcnt[w] = a;
                a += c;
                t += s_pcnt[w];
            }
            s_nsel = t < cap ? t : cap;  // pending candidates before position r, at most cap
        }
        __syncthreads();
        const int slot = s_wcnt[wv] + (int)__popcll(pm & ((1ULL << lane) - 1ULL));
        if (in_r && slot < cap) v.sel_e[slot] = id;
    }
    // A pending candidate joins the batch when fewer than r candidates and
    // fewer than cap pending ones come before it in (b descending, node id
    // ascending) order; its rank among the pending ones is its batch slot.
    // One wave ranks two pending candidates at a time, its lanes striding
    // over all candidates with four independent loads in flight.
    auto before = [](double bq, int iq, double bk, int ik) -> unsigned {
        return (bq > bk || (bq == bk && iq < ik)) ? 1u : 0u;
    };
    // (more candidates than threads: the same rule by counting, pending
    // candidate against every candidate)
    for (int p = 2 * wv; !by_sort && p < npend; p += 2 * nwaves) {
        const bool two = p + 1 < npend;
        const int ka = v.fr[p], kb = v.fr[two ? p + 1 : p];
        const double ba = v.cb[ka], bb = v.cb[kb];
        const int ca = v.ci[ka], cb = v.ci[kb];
        unsigned raa = 0, rpa = 0, rab = 0, rpb = 0;
        for (int q0 = lane; q0 < ncand; q0 += 256) {
            double bq[4];
            int cq[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int q = q0 + 64 * u;
                const int qq = q < ncand ? q : q0;
                bq[u] = v.cb[qq];
                cq[u] = v.ci[qq];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const unsigned in = q0 + 64 * u < ncand ? 1u : 0u;
                const int iq = cq[u] & 0x7FFFFFFF;
                const unsigned pq = cq[u] >= 0 ? 1u : 0u;
                const unsigned xa = in & before(bq[u], iq, ba, ca);
                const unsigned xb = in & before(bq[u], iq, bb, cb);
                raa += xa;
                rpa += xa & pq;
                rab += xb;
                rpb += xb & pq;
            }
        }
        raa = wave_add_u32(raa);
        rpa = wave_add_u32(rpa);
        rab = wave_add_u32(rab);
        rpb = wave_add_u32(rpb);
        if (lane == 0) {
            if ((int)raa < r && (int)rpa < cap) {
                v.sel_e[rpa] = ca;
                atomicAdd(&s_nsel, 1);
            }
            if (two && (int)rab < r && (int)rpb < cap) {
                v.sel_e[rpb] = cb;
                atomicAdd(&s_nsel, 1);
            }
        }
    }
    __syncthreads();
    if (tid < 64) {
        // the leaf the replay waits for is always in the batch
        int n = s_nsel;
        const bool has = __ballot(lane < n && v.sel_e[lane] == s_x) != 0ULL;  // n <= cap <= kmax <= 64
        if (!has && cap > 0) {
            if (n < cap) ++n;
            if (lane == 0) v.sel_e[n - 1] = s_x;
        }
        if (lane == 0) s_nsel = n;
    }
    __syncthreads();
    const int nsel = s_nsel;
    {
        // unreachable while the expansion budget holds; each check has its
        // own code in the sticky error word
        const int bad = (cap <= 0 ? 8 : 0) | (nsel <= 0 ? 16 : 0) | (ne + 2 * nsel > s.e_cap ? 64 : 0) |
                        (g.n_hist + nsel > 1 + s.max_exp ? 128 : 0);
        if (bad) {
            finish(bad);
            return;
        }
    }
    // Rows per task, one value per kind for the whole batch. Accumulation:
    // the batch's accumulated rows spread over about pb_launch tasks (one
    // per resident block), at least hist_chunk_min rows each (fewer tasks
    // mean fewer partials to store and merge; a batch never needs more than
    // n / hist_chunk_min + nsel of them). Partition: the batch's parent rows
    // spread over about part_target tasks (one output reservation each),
    // kPartChunkMin to kPartChunk rows each.
    // the selected leaves' nodes and the committed splits' tree entries, one
    // memory round trip for both
    {
        SelNode sn;
        if (tid < nsel) {
            const ENode *e = &s.enodes[v.sel_e[tid]];
            sn.begin = e->begin;
            sn.end = e->end;
            sn.n_left = e->n_left;
            sn.buf = e->buf;
            sn.hist = e->hist;
            sn.depth = e->depth;
            sn.feature = e->feature;
            sn.bin = e->bin;
            sn.default_left = e->default_left;
            sn.cat = e->cat;
            sn.pad_ = 0;
        }
        write_commits();
        if (tid < nsel) v.sn[tid] = sn;
    }
    __syncthreads();
    if (tid < 64) {  // wave 0: totals, chunks, task counts and their prefixes (nsel <= kmax <= 64)
        // (row counts below n < 2^31 and task counts: 32-bit DPP sums and scans)
        long long m = 0, mb = 0;
        if (lane < nsel) {
            const SelNode &sn = v.sn[lane];
            m = sn.end - sn.begin;
            mb = sn.n_left <= m - sn.n_left ? sn.n_left : m - sn.n_left;
        }
        const long long rows_total = wave_add_u32((unsigned)m), built_total = wave_add_u32((unsigned)mb);
        int64_t chunk = (built_total + s.pb_launch - 1) / s.pb_launch;
        if (chunk < s.hist_chunk_min) chunk = s.hist_chunk_min;
        if (chunk > s.hist_chunk_limit) chunk = s.hist_chunk_limit;
        const int pc = lane < nsel ? (int)((mb + chunk - 1) / chunk) : 0;
        long long chunk_p = (rows_total + s.part_target - 1) / s.part_target;
        chunk_p = (chunk_p + kPartChunkStep - 1) / kPartChunkStep * kPartChunkStep;
        // the root's batch has a launch of its own with larger tasks
        const long long cmax = s.rcp ? (long long)kPartRecThreads * kPartRows
                               : root_mode && s.part_root ? kPartChunkRoot : kPartChunk;
        chunk_p = chunk_p < kPartChunkMin ? kPartChunkMin : chunk_p > cmax ? cmax : chunk_p;
        const int qc = lane < nsel ? (int)((m + chunk_p - 1) / chunk_p) : 0;
        const int pi = wave_incl_scan_i(pc), qi = wave_incl_scan_i(qc);
        if (lane < nsel) {
            v.pcnt[lane] = (int)pc;
            v.qcnt[lane] = (int)qc;
            v.poff[lane] = (int)(pi - pc);
            v.qoff[lane] = (int)(qi - qc);
        }
        if (lane == 63) {
            v.poff[nsel] = (int)pi;
            v.qoff[nsel] = (int)qi;
            s_total = (int)pi;
            s_total_p = (int)qi;
            s_chunk = chunk;
            s_chunk_p = chunk_p;
            s_rows_parted = (unsigned long long)rows_total;
            s_rows_built = (unsigned long long)built_total;
        }
    }
    __syncthreads();
    const int64_t chunk = s_chunk;
    const int64_t chunk_p = s_chunk_p;
    const int total = s_total, total_p = s_total_p;
    if (total > s.pb_grid || total_p > s.part_grid) {  // the leaves of a batch are disjoint, so never
        finish(4);
        return;
    }
    for (int jj = tid; jj < nsel; jj += nthr) {
        const int Xs = v.sel_e[jj];
        ENode *e = &s.enodes[Xs];
        const SelNode &sn = v.sn[jj];
        const int64_t b0 = sn.begin, e0 = sn.end, nlft = sn.n_left;
        const int64_t m = e0 - b0;
        const int ebuf = sn.buf, ehist = sn.hist, edep = sn.depth;
        const bool bl = nlft <= m - nlft;
        const int le = ne + 2 * jj, hb = g.n_hist + jj;
        Item it;
        it.begin = b0;
        it.end = e0;
        it.n_left = nlft;
        it.parent_e = Xs;
        it.left_e = le;
        it.src_buf = ebuf;
        it.builds_left = bl ? 1 : 0;
        it.hist_built = hb;
        it.hist_sib = ehist;
        it.depth_child = edep + 1;
        it.part_off = v.poff[jj];
        it.part_cnt = v.pcnt[jj];
        it.pad_ = 0;
        s.items[jj] = it;
        v.it[jj] = it;
        ENode c;
        c.n_left = 0;
        c.tot_g = c.tot_h = c.tot_c = 0;
        c.gain = 0.0;
        c.value = 0.0;
        c.buf = 1 - ebuf;
        c.depth = edep + 1;
        c.found = 0;
        c.feature = -1;
        c.bin = -1;
        c.default_left = 0;
        c.left_e = -1;
        c.right_e = -1;
        c.cat = 0;
        c.begin = b0;
        c.end = b0 + nlft;
        c.hist = bl ? hb : ehist;
        s.enodes[le] = c;
        c.begin = b0 + nlft;
        c.end = e0;
        c.hist = bl ? ehist : hb;
        s.enodes[le + 1] = c;
        s.e_gain[le] = -1.0;
        s.e_gain[le + 1] = -1.0;
        s.e_left[le] = -1;
        s.e_left[le + 1] = -1;
        s.e_parent[le] = Xs;
        s.e_parent[le + 1] = Xs;
        s.e_rows[le] = (int32_t)nlft;
        s.e_rows[le + 1] = (int32_t)(m - nlft);
        e->left_e = le;
        e->right_e = le + 1;
        s.e_left[Xs] = le;
        s.cursor[2 + 2 * jj] = 0;
        s.cursor[3 + 2 * jj] = 0;
        // the item's partition and accumulation work; each task of the
        // launches finds its item from these (no per-task descriptors)
        PartItem pi;
        pi.begin = b0;
        pi.n_left = nlft;
        pi.m = m;
        pi.qoff = v.qoff[jj];
        pi.src_buf = ebuf;
        pi.feature = sn.feature;
        pi.bin = sn.bin;
        pi.default_left = sn.default_left;
        pi.missing_bin = v.mbin[sn.feature];
        pi.cat_e = sn.cat ? Xs : -1;
        // the root of an unsampled round spans every row in order: its
        // partition computes the ids instead of reading an identity list
        pi.direct = (Xs == 0 && !rd.sampled) ? 1 : 0;
        pi.root = Xs == 0 ? 1 : 0;
        pi.pad_ = 0;
        s.part_items[jj] = pi;
        AccItem ai;
        ai.lo = bl ? b0 : b0 + nlft;
        ai.hi = bl ? b0 + nlft : e0;
        ai.poff = v.poff[jj];
        ai.buf = 1 - ebuf;
        s.acc_items[jj] = ai;
    }
    __syncthreads();
    __syncthreads();
    if (tid == 0) {
        if (s.iter_log && g.iterations < s.iter_stride) {
            int64_t *lg = s.iter_log + 2 * ((size_t)rd.tree_index * s.iter_stride + g.iterations);
            lg[0] = (int64_t)s_rows_parted;
            lg[1] = (int64_t)s_rows_built;
        }
        g.n_explored = ne + 2 * nsel;
        g.n_hist += nsel;
        g.expansions += nsel;
        g.iterations += 1;
        g.rows_built += (int64_t)s_rows_built;
        g.rows_parted += (int64_t)s_rows_parted;
        *s.grow = g;
        Batch b;
        b.n_items = nsel;
        b.n_blocks = total_p;
        b.done = 0;
        b.iters = g.iterations;
        b.n_acc = total;
        b.chunk_p = (int32_t)chunk_p;
        b.chunk_a = (int32_t)chunk;
        b.pad_ = 0;
        *s.batch = b;
        if (host != nullptr) publish_header(host, b);
    }
}

// ------------------------------------------------------------- score update
// raw[r] += lr * value(leaf of r), fused (boosting._add_by_leaf,
// src/mojotrees/boosting.mojo:1991-2112), by walking the tree for every row
// over the row's record (its bins are contiguous), so sampled-out rows are
// covered too (the traversal route, :1947). A single-leaf tree whose value is
// below 1e-12 is the reference's stopping condition (:2898-2907) and adds
// nothing.
// The finished tree in LDS, one 64-bit word per node: feature (16 bits,
// 0xFFFF for a leaf), threshold bin (8), missing bin + 1 (9), default_left
// (1), left child (16); the right child is always left + 1 (node ids are
// given in pairs). One LDS read per level of a walk.
struct PackedTree {
    const unsigned long long *node;
    const double *value;
    const unsigned long long *cat;  // 4 words per node: a categorical node's left set
};

// tree.goes_left for a packed node: bit 50 marks a categorical node, routed
// by its set (bin 0, missing or unseen, is in no set); otherwise the missing
// bin follows default_left and bin <= threshold goes left. The numerical rule
// in integer arithmetic, 1 when bin b goes left: le ^ (miss & (le ^ dl)) is
// dl for the missing bin and le otherwise (no boolean select for the compiler
// to turn into a branch).
__device__ __forceinline__ unsigned packed_left_bit(unsigned long long w, int b) {
    const unsigned thr = (unsigned)(w >> 16) & 255u;
    const unsigned mbin = ((unsigned)(w >> 24) & 511u) - 1u;  // 0xFFFFFFFF: no missing bin
    const unsigned dl = (unsigned)(w >> 33) & 1u;
    const unsigned le = (unsigned)b <= thr ? 1u : 0u;
    const unsigned miss = (unsigned)b == mbin ? 1u : 0u;
    return le ^ (miss & (le ^ dl));
}

__device__ __forceinline__ PackedTree load_packed_tree(const DevState &s, unsigned char *smem) {
    unsigned long long *pn = (unsigned long long *)smem;
    double *vals = (double *)(pn + s.max_nodes);
    unsigned long long *cats = (unsigned long long *)(vals + s.max_nodes);  // when s.t_cat
    const int n_nodes = s.t_meta[0];
    for (int i = threadIdx.x; i < n_nodes; i += blockDim.x) {
        const int f = s.t_feature[i];
        unsigned long long w;
        if (f < 0) {
            w = 0xFFFFULL;
        } else {
            const bool cat = s.t_threshold[i] < 0;  // a categorical node has no threshold
            w = (unsigned long long)(uint32_t)f | ((unsigned long long)(s.t_threshold[i] & 255) << 16) |
                ((unsigned long long)((s.t_missing_bin[i] + 1) & 511) << 24) |
                ((unsigned long long)(s.t_default_left[i] ? 1 : 0) << 33) |
                ((unsigned long long)(s.t_left[i] & 0xFFFF) << 34) | ((unsigned long long)(cat ? 1 : 0) << 50);
            if (cat)
                for (int k = 0; k < 4; ++k) cats[(size_t)i * 4 + k] = s.t_cat[(size_t)i * 4 + k];
        }
        pn[i] = w;
        vals[i] = s.t_value[i];
    }
    __syncthreads();
    return PackedTree{pn, vals, cats};
}

// Leaf of a row: bin(f) gives the row's bin of feature f. The missing bin
// follows default_left, otherwise bin <= threshold goes left
// (tree.goes_left, src/mojotrees/tree.mojo:483-505). Children always have
// larger ids than their parent, so a walk ends within n_nodes steps.
// 1 when bin b goes left at node `node` (word w): with kCat, a categorical
// node's set bit is read for every node (in bounds; used only where bit 50
// marks the node categorical) and selected, so the step has no branch.
template <bool kCat>
__device__ __forceinline__ unsigned packed_left(const PackedTree &t, unsigned long long w, int node, int b) {
    const unsigned num = packed_left_bit(w, b);
    if (!kCat) return num;
    const unsigned set = (unsigned)(t.cat[(size_t)node * 4 + (b >> 6)] >> (b & 63)) & 1u;
    return ((w >> 50) & 1ULL) ? set : num;
}

template <bool kCat, class BinOf>
__device__ __forceinline__ int walk_packed(const PackedTree &t, int n_nodes, BinOf bin) {
    // no branch inside the step (a lane leaves the loop at its leaf)
    int node = 0;
    unsigned long long w = t.node[0];
    for (int d = 0; d < n_nodes; ++d) {
        const int f = (int)(w & 0xFFFFULL);
        if (f == 0xFFFF) break;
        const int c = (int)((w >> 34) & 0xFFFFULL) + 1 - (int)packed_left<kCat>(t, w, node, bin(f));
        node = (unsigned)c < (unsigned)n_nodes ? c : 0;
        w = t.node[node];
    }
    return node;
}

// Two independent walks advanced together, so each level's LDS round trips
// of one row overlap the other's.
template <bool kCat, class BinA, class BinB>
__device__ __forceinline__ void walk_packed2(const PackedTree &t, int n_nodes, BinA bin_a, BinB bin_b, int &na,
                                             int &nb) {
    // both rows step until both reach their leaves; a row at its leaf keeps
    // it and reads feature 0 (selects, no branch inside the step)
    int a = 0, b = 0;
    unsigned long long wa = t.node[0], wb = wa;
    for (int d = 0; d < n_nodes; ++d) {
        const int fa = (int)(wa & 0xFFFFULL), fb = (int)(wb & 0xFFFFULL);
        const bool la = fa == 0xFFFF, lb = fb == 0xFFFF;
        if (la && lb) break;
        const int ba = bin_a(la ? 0 : fa), bb = bin_b(lb ? 0 : fb);
        const int ca = (int)((wa >> 34) & 0xFFFFULL) + 1 - (int)packed_left<kCat>(t, wa, a, ba);
        const int cb = (int)((wb >> 34) & 0xFFFFULL) + 1 - (int)packed_left<kCat>(t, wb, b, bb);
        a = la ? a : ((unsigned)ca < (unsigned)n_nodes ? ca : 0);
        b = lb ? b : ((unsigned)cb < (unsigned)n_nodes ? cb : 0);
        wa = t.node[a];
        wb = t.node[b];
    }
    na = a;
    nb = b;
}

__global__ __launch_bounds__(256) void k_score(DevState s) {
    extern __shared__ unsigned char score_smem[];
    const int n_nodes = s.t_meta[0];
    const int n_leaves = s.t_meta[1];
    if (s.round->stopped) return;
    // a single output stops before adding a degenerate tree; a multiclass
    // round adds every class tree and decides afterwards
    // (boosting.mojo:2898-2907, :3876-4165)
    if (s.hp.num_class == 1 && n_leaves == 1 && fabs(s.t_value[0]) < 1e-12) return;
    const PackedTree tree = load_packed_tree(s, score_smem);
    const bool has_cat = s.t_cat != nullptr;  // categorical nodes possible (launch-uniform)
    const double lr = s.hp.learning_rate;
    const int k = s.round->class_k;
    const int rec = s.rec_bytes, tf = s.tile_f;
    const size_t tile_bytes = (size_t)s.n * rec;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t n = s.n;
    double *raw = s.raw + (size_t)k * n;  // class-major (k = 0 for a single output)
    const int64_t r0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (s.n_tiles == 1 && rec <= 64) {
        // one tile of at most 64 bytes: the row's record is copied into this
        // thread's 64 LDS bytes and walked there, the next row's record and
        // raw score loaded (unconditionally, the last row again past the
        // end) while the current row walks
        __shared__ uint4 srec[256 * 4];
        uint4 *mine4 = srec + threadIdx.x * 4;
        const uint8_t *mine = (const uint8_t *)mine4;
        const uint4 *R = (const uint4 *)s.records;
        const int per = rec / 16;  // 1, 2 or 4 uint4 per record
        const int o1 = per > 1 ? 1 : 0, o2 = per > 2 ? 2 : per - 1, o3 = per - 1;
        int64_t q = r0 < n ? r0 : n - 1;
        uint4 c0 = R[q * per], c1 = R[q * per + o1], c2 = R[q * per + o2], c3 = R[q * per + o3];
        double cv = raw[q];
        for (int64_t r = r0; r < n; r += stride) {
            q = r + stride < n ? r + stride : n - 1;
            const uint4 n0 = R[q * per], n1 = R[q * per + o1], n2 = R[q * per + o2], n3 = R[q * per + o3];
            const double nv = raw[q];
            mine4[0] = c0;  // this thread's own bytes: no barrier
            mine4[1] = c1;
            mine4[2] = c2;
            mine4[3] = c3;
            auto bin = [&](int f) { return (int)mine[f]; };
            const int node = has_cat ? walk_packed<true>(tree, n_nodes, bin) : walk_packed<false>(tree, n_nodes, bin);
            raw[r] = fma(lr, tree.value[node], cv);
            c0 = n0;
            c1 = n1;
            c2 = n2;
            c3 = n3;
            cv = nv;
        }
        return;
    }
    for (int64_t r = r0; r < n; r += stride) {
        const uint8_t *rb = s.records + r * rec;
        auto bin = [&](int f) {
            const int t = f / tf;
            return (int)rb[(size_t)t * tile_bytes + (f - t * tf)];
        };
        const int node = has_cat ? walk_packed<true>(tree, n_nodes, bin) : walk_packed<false>(tree, n_nodes, bin);
        raw[r] = fma(lr, tree.value[node], raw[r]);
    }
}

// Score update of the finished tree fused with the next round's objective,
// for single-output L2 and binary objectives: per row, raw += lr x leaf
// value (k_score) and then the next round's g, h from the updated raw score
// and max |g|, |h| over the next round's bag (k_objective), so raw scores are
// read once and written once per round. Training that stops at this tree
// never reads these g, h. With one feature tile of at most 32 bytes the
// row's record is loaded whole (one or two 16-byte loads) into the thread's
// LDS slot and the walk reads its bins there.
// kL8: the labels as bytes (labels8, every label an integer in [0, 255]):
// a row's label costs 1 byte of HBM instead of 8.
template <bool kL8>
__global__ __launch_bounds__(256) void k_score_objective(DevState s) {
    extern __shared__ unsigned char score_smem[];
    __shared__ float red_g[4], red_h[4];
    __shared__ uint4 srec[256 * 4];     // each thread's two records (at most 32 bytes each)
    const Round rd = *s.round;
    if (rd.stopped) return;
    const HyperParams &hp = s.hp;
    const int n_nodes = s.t_meta[0];
    const bool add = !(s.t_meta[1] == 1 && fabs(s.t_value[0]) < 1e-12);
    const PackedTree tree = load_packed_tree(s, score_smem);
    const bool has_cat = s.t_cat != nullptr;  // categorical nodes possible (launch-uniform)
    const double lr = hp.learning_rate;
    const int rec = s.rec_bytes;
    const bool in_regs = s.n_tiles == 1 && rec <= 32;
    const int np = 1 - rd.parity;  // the next tree's magnitude-stats pair
    const uint64_t bstream = hp.bagging ? bag_stream_of(hp, rd.round + 1) : 0;
    const int64_t bfall = hp.bagging ? bag_fallback_of(s, rd.round + 1) : -1;
    if (blockIdx.x == 0 && threadIdx.x == 0) s.cursor[0] = 0;  // the next root row count
    float mg = 0.0f, mh = 0.0f;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    // the row's next-round objective and the bag's magnitude stats
    auto objective = [&](int64_t r, double raw, double y) {
        float g, h;
        if (hp.objective == kObjBinary) {
            const double w = s.weights ? s.weights[r] : 1.0;
            const double p = sigmoid(raw);
            g = (float)(w * (p - y));
            double hh = p * (1.0 - p);
            if (hh < 1e-16) hh = 1e-16;
            h = (float)(w * hh);
        } else {
            const double w = s.weights ? s.weights[r] : 1.0;
            g = (float)(w * (raw - y));
            h = (float)(w * 1.0);
        }
        if (s.gh2) {
            ((float2 *)s.gh2)[r] = make_float2(g, h);
        } else {
            s.grad[r] = g;
            s.hess[r] = h;
        }
        const float ag = fabsf(g), ah = fabsf(h);
        const bool sel = !hp.bagging || in_bag(s, bstream, bfall, r);
        if (sel && isfinite(ag) && isfinite(ah)) {
            mg = fmaxf(mg, ag);
            mh = fmaxf(mh, ah);
        }
    };
    const int64_t r0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (in_regs) {
        // one feature tile of at most 32 bytes: the next row's record, raw
        // score and label are loaded (unconditionally, the last row again
        // past the end) while the current row walks the tree
        const uint4 *R = (const uint4 *)s.records;
        const int per = rec / 16;  // 1 or 2 uint4 per record
        uint8_t *mine = (uint8_t *)&srec[threadIdx.x * 2];
        auto fetch = [&](int64_t r, uint4 &a, uint4 &b, double &raw, double &y) {
            const int64_t q = r < s.n ? r : s.n - 1;
            a = R[q * per];
            b = R[q * per + per - 1];
            raw = s.raw[q];
            y = kL8 ? (double)s.labels8[q] : s.labels[q];
        };
        // two rows per step (r and r + stride), walked together
        uint8_t *mine2 = (uint8_t *)&srec[256 * 2 + threadIdx.x * 2];
        uint4 ca, cb, ca2, cb2;
        double craw, cy, craw2, cy2;
        fetch(r0, ca, cb, craw, cy);
        fetch(r0 + stride, ca2, cb2, craw2, cy2);
        for (int64_t r = r0; r < s.n; r += 2 * stride) {
            uint4 na, nb, na2, nb2;
            double nraw, ny, nraw2, ny2;
            fetch(r + 2 * stride, na, nb, nraw, ny);
            fetch(r + 3 * stride, na2, nb2, nraw2, ny2);
            const int64_t r2 = r + stride;
            double raw = craw, raw2 = craw2;
            if (add) {
                srec[threadIdx.x * 2] = ca;
                srec[threadIdx.x * 2 + 1] = cb;  // this thread's own slots: no barrier needed
                srec[256 * 2 + threadIdx.x * 2] = ca2;
                srec[256 * 2 + threadIdx.x * 2 + 1] = cb2;
                int n1, n2;
                auto bin1 = [&](int f) { return (int)mine[f]; };
                auto bin2 = [&](int f) { return (int)mine2[f]; };
                if (has_cat) walk_packed2<true>(tree, n_nodes, bin1, bin2, n1, n2);
                else walk_packed2<false>(tree, n_nodes, bin1, bin2, n1, n2);
                raw = fma(lr, tree.value[n1], raw);
                s.raw[r] = raw;
                raw2 = fma(lr, tree.value[n2], raw2);
                if (r2 < s.n) s.raw[r2] = raw2;
            }
            objective(r, raw, cy);
            if (r2 < s.n) objective(r2, raw2, cy2);
            ca = na;
            cb = nb;
            craw = nraw;
            cy = ny;
            ca2 = na2;
            cb2 = nb2;
            craw2 = nraw2;
            cy2 = ny2;
        }
    } else {
        const int tf = s.tile_f;
        const size_t tile_bytes = (size_t)s.n * rec;
        for (int64_t r = r0; r < s.n; r += stride) {
            double raw = s.raw[r];
            if (add) {
                const uint8_t *rb = s.records + r * rec;
                auto bin = [&](int f) {
                    const int t = f / tf;
                    return (int)rb[(size_t)t * tile_bytes + (f - t * tf)];
                };
                const int node =
                    has_cat ? walk_packed<true>(tree, n_nodes, bin) : walk_packed<false>(tree, n_nodes, bin);
                raw = fma(lr, tree.value[node], raw);
                s.raw[r] = raw;
            }
            objective(r, raw, kL8 ? (double)s.labels8[r] : s.labels[r]);
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
        atomicMax(&s.stats[stat_slot(np, 0, blockIdx.x)], __float_as_uint(mg));
        atomicMax(&s.stats[stat_slot(np, 1, blockIdx.x)], __float_as_uint(mh));
    }
}

// Archive the finished tree and advance the round state (one block).
__device__ __forceinline__ void round_end_body(const DevState &s) {
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
        if (s.arc_cat)
            for (int w = 0; w < 4; ++w)
                s.arc_cat[((size_t)rd.tree_index * mn + i) * 4 + w] = s.t_cat[(size_t)i * 4 + w];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        ai[6 * mn + 0] = n_nodes;
        ai[6 * mn + 1] = s.t_meta[1];
        const Grow g = *s.grow;
        int64_t *ax = s.arc_aux + (size_t)rd.tree_index * 4;
        ax[0] = g.rows_built;
        ax[1] = g.iterations;
        ax[2] = g.expansions;
        ax[3] = g.rows_parted;
        Round nr = rd;
        if (!rd.stopped) {
            // boosting._boost_rounds' stop rule: a tree of one leaf whose
            // value is below 1e-12 ends training unless rows are sampled;
            // for multiclass, a round none of whose trees does better
            const bool degenerate = s.t_meta[1] == 1 && fabs(s.t_value[0]) < 1e-12;
            const int K = s.hp.num_class;
            const bool sampling = s.hp.bagging || s.hp.goss;
            if (K == 1) {
                if (degenerate && !sampling) nr.stopped = 1;
            } else {
                // progress over this state's trees of the round; with several
                // states side by side, k_round_combine judges the round
                const bool first = rd.class_k < s.hp.class_stride;
                nr.progress = (first ? 0 : rd.progress) | (degenerate ? 0 : 1);
                if (s.hp.class_stride == 1 && rd.class_k == K - 1 && !nr.progress && !sampling) nr.stopped = 1;
            }
        }
        // this state's next class tree: class_k + stride, or its first class
        // of the next round
        const int S = s.hp.class_stride;
        nr.class_k = rd.class_k + S;
        if (nr.class_k >= s.hp.num_class) {
            nr.class_k = rd.class_k % S;
            nr.round = rd.round + 1;
        }
        nr.tree_index = (int32_t)(nr.round * s.hp.num_class + nr.class_k);
        nr.parity = 1 - rd.parity;
        *s.round = nr;
    }
}

__global__ __launch_bounds__(256) void k_round_end(DevState s) { round_end_body(s); }

// The end of a tree and the next tree's one-block quantizer launch in one
// (both one block, in order): used when no launch comes between them (one
// output, the objective fused into the score update, no GOSS, no
// magnitude-sum lattice, the pairs written by the root build).
__global__ __launch_bounds__(256) void k_round_end_quantize(DevState s) {
    round_end_body(s);
    __syncthreads();  // the advanced round state, written by thread 0
    quantize_body(s, 0);
}

// The round's stop rule when several states grow its class trees side by
// side (one thread, after every state finished the round): boosting.
// train_multiclass judges the round's K trees together -- a round none of
// whose trees split or moved ends training unless rows are sampled
// (boosting.mojo:3876-4165) -- so the states' progress flags are combined
// and every state stops.
__global__ void k_round_combine(RoundStates rs, int sampling) {
    if (threadIdx.x != 0) return;
    bool stopped = false, progress = false;
    for (int i = 0; i < rs.n; ++i) {
        stopped |= rs.r[i]->stopped != 0;
        progress |= rs.r[i]->progress != 0;
    }
    if (!stopped && !progress && !sampling)
        for (int i = 0; i < rs.n; ++i) rs.r[i]->stopped = 1;
}

// Bins column-major -> tile-major row records (each tile: its features' bin
// bytes, then zeros up to the g/h pair, which starts at zero too).
__global__ __launch_bounds__(256) void k_build_records(const uint8_t *bins_cm, uint8_t *records,
                                                       int64_t n, int F, int rec, int tile_f, int n_tiles) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t total = n * n_tiles;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int t = (int)(i / n);
        const int64_t r = i - (int64_t)t * n;
        const int f0 = t * tile_f;
        const int ft = min(tile_f, F - f0);
        uint8_t *o = records + i * rec;
        for (int j = 0; j < rec; ++j) o[j] = j < ft ? bins_cm[(size_t)(f0 + j) * n + r] : 0;
    }
}

// Raw scores of a flat ensemble (Tree.predict_row, src/mojotrees/tree.mojo:
// 483-505; Booster.predict_raw_row, src/mojotrees/boosting.mojo:1722-1760):
// a row's bin for a node's feature comes from its record; the missing bin
// follows the default direction, otherwise bin <= threshold goes left. The
// class's trees are added in ascending order as fma(learning_rate, value,
// score), the host predictor's fused update, so the scores are its bits.
__global__ __launch_bounds__(256) void k_predict(PredictArgs a) {
    const int k = blockIdx.y;
    const int K = a.num_class;
    const int tf = a.tile_f;
    const bool tiled = a.n_tiles > 1;
    const size_t tile_bytes = (size_t)a.n * a.rec_bytes;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < a.n; r += stride) {
        const uint8_t *rb = a.records + r * a.rec_bytes;
        double acc = a.base ? a.base[k] : 0.0;
        for (int64_t t = a.t0 + k; t < a.t1; t += K) {
            int node = a.root[t];
            int4 nd = a.nodes[node];
            // children have larger indices than their parent (host-checked),
            // so a walk ends within the tree's node count
            for (int d = 0; nd.x >= 0 && d < a.max_steps; ++d) {
                int b;
                if (tiled) {
                    const int tt = nd.x / tf;
                    b = rb[(size_t)tt * tile_bytes + (nd.x - tt * tf)];
                } else {
                    b = rb[nd.x];
                }
                const int md = a.md[node];
                const bool left = nd.y < 0 ? ((a.cat[(size_t)node * 4 + (b >> 6)] >> (b & 63)) & 1ULL) != 0
                                           : (b == (md >> 1)) ? (md & 1) : (b <= nd.y);
                node = left ? nd.z : nd.w;
                nd = a.nodes[node];
            }
            acc = fma(a.learning_rate, a.value[node], acc);
        }
        a.out[r * K + k] = acc;
    }
}

// The initial raw scores, class-major: class k of row r at k n + r.
__global__ __launch_bounds__(256) void k_fill_f64(double *p, int64_t n, int K, const double *base) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n * K; i += stride)
        p[i] = base[i / n];
}

__global__ void k_exp_sigmoid(const double *x, double *e, double *sg, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        e[i] = ref_exp(x[i]);
        sg[i] = sigmoid(x[i]);
    }
}

// ------------------------------------------------------------------ launch
size_t rank_lds_bytes(const DevState &s) { return (size_t)s.rank_pad * 49; }
hipError_t launch_objective(const DevState &s, int grid, hipStream_t st) {
    if (s.hp.objective == kObjLambdarank) {
        const int g = s.n_queries < 4 * grid ? s.n_queries : 4 * grid;
        hipLaunchKernelGGL(k_lambdarank, dim3(g > 0 ? g : 1), dim3(256), rank_lds_bytes(s), st, s);
        if (s.n_big > 0) {
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
            hipLaunchKernelGGL(k_lambdarank_big, dim3(s.rank_big_slots), dim3(256), 0, st, s);
        }
    } else {
        hipLaunchKernelGGL(k_objective, dim3(grid), dim3(256), 0, st, s);
    }
    return hipGetLastError();
}
hipError_t launch_softmax(const DevState &s, int grid, hipStream_t st) {
    hipLaunchKernelGGL(k_softmax, dim3(grid), dim3(256), 0, st, s);
    return hipGetLastError();
}
hipError_t launch_goss(const DevState &s, int grid_rows, hipStream_t st) {
    if (s.hp.num_class > 1) hipLaunchKernelGGL(k_goss_importance, dim3(grid_rows), dim3(256), 0, st, s);
    hipLaunchKernelGGL(k_goss_setup, dim3(1), dim3(256), 0, st, s);
    for (int pass = 0; pass < 8; ++pass)
        hipLaunchKernelGGL(k_goss_digits, dim3(kGossDigitBlocks), dim3(256), 0, st, s, pass);
    hipLaunchKernelGGL(k_goss_pick, dim3(1), dim3(64), 0, st, s);
    const dim3 blocks(s.goss_nblk);
    const size_t walk_lds = (size_t)2 * kGossTile * sizeof(int32_t);
    int64_t *n_unc = &s.gst->n_uncertain;
    int64_t *bag_n = &s.gst->bag_n;
    // top rows: counts, prefix; kappa and the band's classes
    hipLaunchKernelGGL(k_goss_count, blocks, dim3(kGossRowThreads), 0, st, s, 0);
    hipLaunchKernelGGL(k_goss_scan, dim3(1), dim3(1024), 0, st, s, s.goss_blk, (int64_t *)nullptr, (int32_t *)nullptr,
                       (int64_t *)nullptr);
    hipLaunchKernelGGL(k_goss_kappa, blocks, dim3(kGossRowThreads), 0, st, s);
    // the open rows: list, sequential count, decisions
    // the kept and the open rows' block counts, one block each
    hipLaunchKernelGGL(k_goss_scan, dim3(2), dim3(1024), 0, st, s, s.goss_blk, (int64_t *)nullptr, s.goss_blk_u,
                       n_unc);
    hipLaunchKernelGGL(k_goss_compact, blocks, dim3(kGossRowThreads), 0, st, s);
    hipLaunchKernelGGL(k_goss_walk, dim3(1), dim3(1024), walk_lds, st, s, 1);
    hipLaunchKernelGGL(k_goss_apply, dim3(256), dim3(256), 0, st, s);
    // the check, and the full count when it fails
    hipLaunchKernelGGL(k_goss_count, blocks, dim3(kGossRowThreads), 0, st, s, 2);
    hipLaunchKernelGGL(k_goss_scan, dim3(1), dim3(1024), 0, st, s, s.goss_blk, (int64_t *)nullptr, (int32_t *)nullptr,
                       (int64_t *)nullptr);
    hipLaunchKernelGGL(k_goss_verify, blocks, dim3(kGossRowThreads), 0, st, s);
    hipLaunchKernelGGL(k_goss_walk, dim3(1), dim3(1024), walk_lds, st, s, 0);
    // the sample: top rows and kept rows, ascending
    hipLaunchKernelGGL(k_goss_count, blocks, dim3(kGossRowThreads), 0, st, s, 1);
    hipLaunchKernelGGL(k_goss_scan, dim3(1), dim3(1024), 0, st, s, s.goss_blk, bag_n, (int32_t *)nullptr,
                       (int64_t *)nullptr);
    hipLaunchKernelGGL(k_goss_scatter, blocks, dim3(kGossRowThreads), 0, st, s);
    return hipGetLastError();
}
hipError_t launch_goss_stats(const DevState &s, int grid_rows, hipStream_t st) {
    hipLaunchKernelGGL(k_goss_stats, dim3(grid_rows), dim3(256), 0, st, s);
    return hipGetLastError();
}
hipError_t launch_magnitude(const DevState &s, hipStream_t st) {
    hipLaunchKernelGGL(k_magsum, dim3(kMagBlocks), dim3(kMagThreads), 0, st, s);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_magfold, dim3(1), dim3(64), 0, st, s);
    return hipGetLastError();
}
hipError_t launch_quantize(const DevState &s, int grid, hipStream_t st, bool write_pairs) {
    hipLaunchKernelGGL(k_quantize, dim3(grid), dim3(256), 0, st, s, write_pairs ? 1 : 0);
    return hipGetLastError();
}
size_t score_lds_bytes(const DevState &s) { return (size_t)s.max_nodes * (s.t_cat ? 48 : 16); }
size_t pb_lds_bytes_for(int tile_f, int lds_stride, int kind) {
    return kind == kAccQuant  ? QAcc::lds_bytes(tile_f, lds_stride)
           : kind == kAccWide ? WAcc::lds_bytes(tile_f, lds_stride)
                              : FAcc::lds_bytes(tile_f, lds_stride);
}
size_t hist_lds_bytes(const DevState &s) { return pb_lds_bytes_for(s.tile_f, s.lds_stride, acc_kind(s.hp)); }
size_t plan_lds_bytes(const DevState &s) {
    return plan_layout(s.hp.num_leaves, s.e_cap, s.kmax, s.n_features).total;
}

#define MB_SET_LDS(fn, bytes)                                                                     \
    do {                                                                                          \
        hipError_t e_ = hipFuncSetAttribute((const void *)(fn), hipFuncAttributeMaxDynamicSharedMemorySize, \
                                            (int)(bytes));                                        \
        if (e_ != hipSuccess) return e_;                                                          \
    } while (0)

hipError_t prepare_kernels(const DevState &s) {
    const size_t h = hist_lds_bytes(s);
    if (s.hp.objective == kObjLambdarank) MB_SET_LDS(k_lambdarank, rank_lds_bytes(s));
    if (s.hp.stage16) {
        MB_SET_LDS((k_hist<1, WAcc16>), h);
        MB_SET_LDS((k_hist<2, WAcc16>), h);
        MB_SET_LDS((k_hist<4, WAcc16>), h);
        MB_SET_LDS((k_hist<8, WAcc16>), h);
        MB_SET_LDS((k_accum<1, WAcc16>), h);
        MB_SET_LDS((k_accum<2, WAcc16>), h);
        MB_SET_LDS((k_accum<4, WAcc16>), h);
        MB_SET_LDS((k_accum<8, WAcc16>), h);
    } else if (s.hp.wide) {
        MB_SET_LDS((k_hist<1, WAcc>), h);
        MB_SET_LDS((k_hist<2, WAcc>), h);
        MB_SET_LDS((k_hist<4, WAcc>), h);
        MB_SET_LDS((k_hist<8, WAcc>), h);
        MB_SET_LDS((k_accum<1, WAcc>), h);
        MB_SET_LDS((k_accum<2, WAcc>), h);
        MB_SET_LDS((k_accum<4, WAcc>), h);
        MB_SET_LDS((k_accum<8, WAcc>), h);
    } else if (s.hp.quantized) {
        MB_SET_LDS((k_hist<1, QAcc>), h);
        MB_SET_LDS((k_hist<2, QAcc>), h);
        MB_SET_LDS((k_hist<4, QAcc>), h);
        MB_SET_LDS((k_hist<8, QAcc>), h);
        MB_SET_LDS((k_accum<1, QAcc>), h);
        MB_SET_LDS((k_accum<2, QAcc>), h);
        MB_SET_LDS((k_accum<4, QAcc>), h);
        MB_SET_LDS((k_accum<8, QAcc>), h);
        MB_SET_LDS(k_accum_rec<1>, h);
        MB_SET_LDS(k_accum_rec<2>, h);
        MB_SET_LDS(k_accum_rec<4>, h);
    } else {
        MB_SET_LDS((k_hist<1, FAcc>), h);
        MB_SET_LDS((k_hist<2, FAcc>), h);
        MB_SET_LDS((k_hist<4, FAcc>), h);
        MB_SET_LDS((k_hist<8, FAcc>), h);
        MB_SET_LDS((k_accum<1, FAcc>), h);
        MB_SET_LDS((k_accum<2, FAcc>), h);
        MB_SET_LDS((k_accum<4, FAcc>), h);
        MB_SET_LDS((k_accum<8, FAcc>), h);
    }
    MB_SET_LDS(k_plan, plan_lds_bytes(s));
    MB_SET_LDS(k_goss_walk, (size_t)2 * kGossTile * sizeof(int32_t));
    MB_SET_LDS(k_score, score_lds_bytes(s));
    MB_SET_LDS(k_score_objective<false>, score_lds_bytes(s));
    MB_SET_LDS(k_score_objective<true>, score_lds_bytes(s));
    return hipSuccess;
}
// A launch of kernel k with DevState s; with both events given, the runtime
// records them at the kernel's own start and end (hipExtLaunchKernel), so
// their elapsed time is the kernel's duration without the queue gaps that
// stream events around the launch would add.
template <class K>
hipError_t launch_timed(K k, dim3 grid, dim3 block, size_t lds, hipStream_t st, const DevState &s,
                        hipEvent_t ev0, hipEvent_t ev1) {
    if (ev0 && ev1) hipExtLaunchKernelGGL(k, grid, block, (uint32_t)lds, st, ev0, ev1, 0u, s);
    else hipLaunchKernelGGL(k, grid, block, lds, st, s);
    return hipGetLastError();
}
template <class Acc, bool kQ = false>
hipError_t launch_hist_t(const DevState &s, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    const size_t lds = hist_lds_bytes(s);
    const dim3 grid(s.hist_grid, s.n_tiles), block(kHistThreads);
    switch (s.rec_bytes / 16) {
    case 1: return launch_timed(k_hist<1, Acc, kQ>, grid, block, lds, st, s, ev0, ev1);
    case 2: return launch_timed(k_hist<2, Acc, kQ>, grid, block, lds, st, s, ev0, ev1);
    case 4: return launch_timed(k_hist<4, Acc, kQ>, grid, block, lds, st, s, ev0, ev1);
    case 8: return launch_timed(k_hist<8, Acc, kQ>, grid, block, lds, st, s, ev0, ev1);
    default: return hipErrorInvalidValue;
    }
}
hipError_t launch_hist(const DevState &s, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1, bool quantize) {
    if (quantize && s.hp.quantized && !s.hp.wide && !s.hp.stage16 && !s.hp.grad64)
        return launch_hist_t<QAcc, true>(s, st, ev0, ev1);
    return s.hp.stage16     ? launch_hist_t<WAcc16>(s, st, ev0, ev1)
           : s.hp.wide      ? launch_hist_t<WAcc>(s, st, ev0, ev1)
           : s.hp.quantized ? launch_hist_t<QAcc>(s, st, ev0, ev1)
                            : launch_hist_t<FAcc>(s, st, ev0, ev1);
}
hipError_t launch_partition(const DevState &s, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1, bool root) {
    if (s.rcp) {
        // a CU holds several record-partition blocks: the grid is widened
        // to keep the same rows in flight
        const dim3 grid(s.part_launch * (kPartThreads / kPartRecThreads)), block(kPartRecThreads);
        switch (s.rec_bytes / 16) {
        case 1: return launch_timed(k_partition_rec<1>, grid, block, 0, st, s, ev0, ev1);
        case 2: return launch_timed(k_partition_rec<2>, grid, block, 0, st, s, ev0, ev1);
        case 4: return launch_timed(k_partition_rec<4>, grid, block, 0, st, s, ev0, ev1);
        default: return hipErrorInvalidValue;
        }
    }
    if (root) return launch_timed(k_partition<kPartRowsRoot>, dim3(s.part_launch), dim3(kPartThreads), 0, st, s, ev0, ev1);
    return launch_timed(k_partition<kPartRows>, dim3(s.part_launch), dim3(kPartThreads), 0, st, s, ev0, ev1);
}
template <class Acc>
hipError_t launch_accum_t(const DevState &s, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    const size_t lds = hist_lds_bytes(s);
    const dim3 grid(s.pb_launch, s.n_tiles), block(kAccThreads);
    switch (s.rec_bytes / 16) {
    case 1: return launch_timed(k_accum<1, Acc>, grid, block, lds, st, s, ev0, ev1);
    case 2: return launch_timed(k_accum<2, Acc>, grid, block, lds, st, s, ev0, ev1);
    case 4: return launch_timed(k_accum<4, Acc>, grid, block, lds, st, s, ev0, ev1);
    case 8: return launch_timed(k_accum<8, Acc>, grid, block, lds, st, s, ev0, ev1);
    default: return hipErrorInvalidValue;
    }
}
hipError_t launch_accum(const DevState &s, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    if (s.rcp) {
        const size_t lds = hist_lds_bytes(s);
        const dim3 grid(s.pb_launch), block(kAccThreads);
        switch (s.rec_bytes / 16) {
        case 1: return launch_timed(k_accum_rec<1>, grid, block, lds, st, s, ev0, ev1);
        case 2: return launch_timed(k_accum_rec<2>, grid, block, lds, st, s, ev0, ev1);
        case 4: return launch_timed(k_accum_rec<4>, grid, block, lds, st, s, ev0, ev1);
        default: return hipErrorInvalidValue;
        }
    }
    return s.hp.stage16     ? launch_accum_t<WAcc16>(s, st, ev0, ev1)
           : s.hp.wide      ? launch_accum_t<WAcc>(s, st, ev0, ev1)
           : s.hp.quantized ? launch_accum_t<QAcc>(s, st, ev0, ev1)
                            : launch_accum_t<FAcc>(s, st, ev0, ev1);
}
hipError_t launch_fold(const DevState &s, int root_mode, hipStream_t st) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || s.n_features <= 64) return e;
    hipLaunchKernelGGL(k_fold, dim3(root_mode ? 1 : 2 * s.kmax), dim3(kFoldThreads), 0, st, s, root_mode);
    return hipGetLastError();
}
hipError_t launch_scan(const DevState &s, int root_mode, hipStream_t st) {
    if (s.hp.quantized && !s.ncat && s.n_bins <= 64) {
        const int groups = (s.n_features + kNarrowFeat - 1) / kNarrowFeat;
        const int grid = root_mode ? groups : std::min(s.scan_grid, s.kmax * groups);
        hipLaunchKernelGGL(k_scan_narrow, dim3(grid), dim3(kScanThreads), 0, st, s, root_mode);
        return launch_fold(s, root_mode, st);
    }
    const int grid = root_mode ? s.n_features : s.scan_grid;
    if (s.hp.quantized && s.ncat)
        hipLaunchKernelGGL(k_scan<true>, dim3(grid), dim3(kScanThreads), 0, st, s, root_mode);
    else if (s.hp.quantized)
        hipLaunchKernelGGL(k_scan<false>, dim3(grid), dim3(kScanThreads), 0, st, s, root_mode);
    else if (s.ncat)
        hipLaunchKernelGGL(k_scan_f<true>, dim3(grid), dim3(kScanThreads), 0, st, s, root_mode);
    else
        hipLaunchKernelGGL(k_scan_f<false>, dim3(grid), dim3(kScanThreads), 0, st, s, root_mode);
    return launch_fold(s, root_mode, st);
}
hipError_t launch_plan(const DevState &s, int root_mode, hipStream_t st, Batch *host) {
    hipLaunchKernelGGL(k_plan, dim3(1), dim3(kPlanThreads), plan_lds_bytes(s), st, s, root_mode, host);
    return hipGetLastError();
}
hipError_t launch_score(const DevState &s, int grid, hipStream_t st) {
    hipLaunchKernelGGL(k_score, dim3(grid), dim3(256), score_lds_bytes(s), st, s);
    return hipGetLastError();
}
hipError_t launch_score_objective(const DevState &s, int grid, hipStream_t st) {
    if (s.labels8 != nullptr)
        hipLaunchKernelGGL(k_score_objective<true>, dim3(grid), dim3(256), score_lds_bytes(s), st, s);
    else
        hipLaunchKernelGGL(k_score_objective<false>, dim3(grid), dim3(256), score_lds_bytes(s), st, s);
    return hipGetLastError();
}
int rows_grid(const DevState &s, RowsKernel k, int n_cu) {
    const void *fn = k == kRowsScore            ? (const void *)k_score
                     : k == kRowsSoftmax        ? (const void *)k_softmax
                     : s.labels8 != nullptr     ? (const void *)k_score_objective<true>
                                                : (const void *)k_score_objective<false>;
    const size_t lds = k == kRowsSoftmax ? 0 : score_lds_bytes(s);
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 256, lds) != hipSuccess) per_cu = 8;
    per_cu = per_cu < 1 ? 1 : per_cu > 8 ? 8 : per_cu;
    return per_cu * (n_cu < 1 ? 1 : n_cu);
}
hipError_t launch_round_combine(const RoundStates &rs, int sampling, hipStream_t st) {
    hipLaunchKernelGGL(k_round_combine, dim3(1), dim3(64), 0, st, rs, sampling);
    return hipGetLastError();
}
hipError_t launch_round_end(const DevState &s, hipStream_t st) {
    hipLaunchKernelGGL(k_round_end, dim3(1), dim3(256), 0, st, s);
    return hipGetLastError();
}
hipError_t launch_round_end_quantize(const DevState &s, hipStream_t st) {
    hipLaunchKernelGGL(k_round_end_quantize, dim3(1), dim3(256), 0, st, s);
    return hipGetLastError();
}
hipError_t launch_build_records(const uint8_t *bins_cm, uint8_t *records, int64_t n, int F, int rec,
                                int tile_f, int n_tiles, int grid, hipStream_t st) {
    hipLaunchKernelGGL(k_build_records, dim3(grid), dim3(256), 0, st, bins_cm, records, n, F, rec, tile_f,
                       n_tiles);
    return hipGetLastError();
}
hipError_t launch_predict(const PredictArgs &a, int grid, hipStream_t st) {
    hipLaunchKernelGGL(k_predict, dim3(grid, a.num_class), dim3(256), 0, st, a);
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
