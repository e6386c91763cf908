// CPU oracle: a plain C++ restatement of the reference's CPU GBDT training
// algorithm (ajhendel/mojoboost, package `mojotrees`, all Mojo).
//
// TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and
// bench.py's cpu_baseline leg as the checker. The product (mojoboost_amd/)
// never links or calls it.
//
// The reference cannot be built here (Mojo 1.0.0 / MAX 26.5.0 toolchain,
// pixi.toml:175-177), so nothing is compiled from /root/reference. What pins
// each part of this file:
//   splitmix64, uniform, quant_stream ... closed forms + the standard first
//        SplitMix64 output (tests/test_oracle_arith.py)
//   exp, log (the reference's Mojo stdlib algorithms, see ref_exp/ref_log),
//        objectives, base score, float histogram, float split search, leaf-wise
//        grower, score update, prediction, bin_equal_width, bagging, feature
//        fraction, softmax ........ the reference's golden bit patterns
//        (tests/golden/golden_bits.json from tests/test_golden_bits.mojo)
//   fit_bins/transform .............. golden "large" fixture + closed forms
//   quantizer (max-abs, stochastic) ... closed forms and the reference's
//        worked example y=-1.3,u=0.9 -> -2 (quantized_gradient.mojo:1502-1505)
//   magnitude-sum lattice: largest_power_of_two_at_most and
//        fixed_point_scale_pow2 .... closed forms (exact powers, binade
//        interiors, refusals) and the reference's assertions
//        (tests/test_cpu_quantized_grad.mojo:429-460: the factor is its own
//        power-of-two floor and <= 2^30 / sum|g|); magnitude_sums' fixed
//        reduction order ... a hand-derived binary32 total that any other
//        order, or a binary64 sum, misses (tests/test_oracle_magnitude.py)
//   integer histogram ................ brute force + float/int agreement
//   quantized split search ........... brute-force enumeration on tiny nodes
//   GOSS ........... the reference's GOSS properties (tests/test_goss.mojo:
//        counts, multiplier, top set, order, reseeding, unbiasedness, warmup,
//        sampled leaf counts) in tests/test_oracle_goss.py; the per-row draw
//        u(r) = uniform(splitmix64(seed ^ round * GOLDEN) + r) follows the
//        formula of goss.mojo:67-78 and no vector of drawn rows pins it
#include "oracle.h"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstdio>
#include <cstring>
#include <functional>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

namespace {

// ---------------------------------------------------------------- rng
// src/mojotrees/rng.mojo:35-46
inline uint64_t splitmix64(uint64_t state) {
    uint64_t z = state + 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}
const uint64_t GOLDEN = 0x9E3779B97F4A7C15ULL;
inline double uniform(uint64_t counter) {
    return (double)(splitmix64(counter) >> 11) * (1.0 / 9007199254740992.0);
}

// ---------------------------------------------------------------- exp
// The reference's exp: Mojo stdlib `exp` (mojo 1.0.0), called by the
// logistic sigmoid (src/mojotrees/boosting.mojo:261-266), the softmax
// (:3515-3573) and the response link. Its bits are not libm's: it reduces
// with one truncated ln2 constant, k = floor(x / ln2 + 0.5),
// r = x - k * 0x1.62e42fefa3000p-1, evaluates the degree-12 Taylor
// polynomial of e^r in fused Horner form and scales by 2^k. This restatement
// reproduces every golden prediction bit of the logit and multi fixtures
// (tests/test_oracle_golden.py). The clamp to [-709.436139303, 709.437] only
// matters beyond the range any fixture reaches (parity unpinned there).
const double REF_EXP_COEF[13] = {
    1.0, 1.0, 0.5, 0.16666666666666666667, 0.041666666666666666667,
    0.0083333333333333333333, 0.0013888888888888888889, 0.00019841269841269841270,
    0.000024801587301587301587, 2.7557319223985890653e-6, 2.7557319223985890653e-7,
    2.5052108385441718775e-8, 2.0876756987868098979e-9};

double ref_exp(double x) {
    if (x != x) return x;
    if (x < -709.436139303) x = -709.436139303;
    if (x > 709.437) x = 709.437;
    double k = std::floor(std::fma(x, 1.442695040888963407359924681001892137, 0.5));
    double r = std::fma(k, -0.69314718055966295651160180568695068359375, x);
    double y = REF_EXP_COEF[12];
    for (int i = 11; i >= 0; --i) y = std::fma(y, r, REF_EXP_COEF[i]);
    return std::ldexp(y, (int)k);
}

// The reference's natural log: Mojo stdlib `log` (mojo 1.0.0), called by
// boosting._base_score (src/mojotrees/boosting.mojo:556-567) and
// train_multiclass (:4231). Its bits are not a correctly rounded log: they are
// the Cephes `logf` algorithm (frexp to [sqrt(1/2), sqrt(2)), a degree-8
// polynomial in Horner form with fused steps, then e * ln2) carried out in
// binary64. This restatement reproduces every golden raw score of the logit
// and multi fixtures (tests/test_oracle_golden.py), which a correctly rounded
// log misses by ~7e-10 relative.
double ref_log(double xv) {
    static const double C[9] = {3.3333331174e-1, -2.4999993993e-1, 2.0000714765e-1,
                                -1.6668057665e-1, 1.4249322787e-1, -1.2420140846e-1,
                                1.1676998740e-1, -1.1514610310e-1, 7.0376836292e-2};
    int e = 0;
    double x1 = std::frexp(xv, &e);
    if (x1 < 0.70710678118654752440) {
        x1 = x1 * 2.0 - 1.0;
        e -= 1;
    } else {
        x1 = x1 - 1.0;
    }
    double x2 = x1 * x1;
    double y = C[8];
    for (int i = 7; i >= 0; --i) y = std::fma(y, x1, C[i]);
    y = x1 * x2 * y;
    y = std::fma(-0.5, x2, y);
    y = x1 + y;
    return std::fma((double)e, 0.69314718055994530942, y);
}

// Mojo stdlib `log2`, called for the LambdaRank position discounts and the
// per-query normalizer (src/mojotrees/ranking.mojo:240-244, :598). Restated
// as the same Cephes reduction and polynomial as ref_log with the result
// taken in base 2, y * log2(e) + e. The reference's own tests pin log2 only
// to 1e-8 (tests/test_ranking.mojo:5-8, :47-48), so its last bits are
// parity unpinned; exact at powers of two.
double ref_log2(double xv) {
    static const double C[9] = {3.3333331174e-1, -2.4999993993e-1, 2.0000714765e-1,
                                -1.6668057665e-1, 1.4249322787e-1, -1.2420140846e-1,
                                1.1676998740e-1, -1.1514610310e-1, 7.0376836292e-2};
    int e = 0;
    double x1 = std::frexp(xv, &e);
    if (x1 < 0.70710678118654752440) {
        x1 = x1 * 2.0 - 1.0;
        e -= 1;
    } else {
        x1 = x1 - 1.0;
    }
    double x2 = x1 * x1;
    double y = C[8];
    for (int i = 7; i >= 0; --i) y = std::fma(y, x1, C[i]);
    y = x1 * x2 * y;
    y = std::fma(-0.5, x2, y);
    y = x1 + y;
    return std::fma(y, 1.44269504088896340736, (double)e);
}

// src/mojotrees/boosting.mojo:261-266
inline double sigmoid(double x) {
    if (x >= 0.0) {
        double e = ref_exp(-x);
        return 1.0 / (1.0 + e);
    }
    double e = ref_exp(x);
    return e / (1.0 + e);
}

// src/mojotrees/boosting.mojo:269-275
inline double clamp_prob(double p) {
    if (p < 1e-15) return 1e-15;
    if (p > 1.0 - 1e-15) return 1.0 - 1e-15;
    return p;
}

// src/mojotrees/histogram.mojo:462-482 (derivative[narrow=True])
inline double narrow(double v) { return (double)(float)v; }

// ---------------------------------------------------------------- pool
class Pool {
public:
    explicit Pool(int n) : n_(n < 1 ? 1 : n) {
        for (int i = 1; i < n_; ++i) workers_.emplace_back([this] { loop(); });
    }
    ~Pool() {
        {
            std::lock_guard<std::mutex> g(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto &t : workers_) t.join();
    }
    int size() const { return n_; }
    // Run fn(i) for i in [0, n_tasks); each task owns disjoint outputs.
    void run(int64_t n_tasks, const std::function<void(int64_t)> &fn) {
        if (n_tasks <= 0) return;
        if (n_ == 1 || n_tasks == 1) {
            for (int64_t i = 0; i < n_tasks; ++i) fn(i);
            return;
        }
        {
            std::lock_guard<std::mutex> g(mu_);
            fn_ = &fn;
            n_tasks_ = n_tasks;
            next_.store(0);
            done_ = 0;
            ++gen_;
        }
        cv_.notify_all();
        work();
        std::unique_lock<std::mutex> lk(mu_);
        done_cv_.wait(lk, [this] { return done_ == n_ - 1; });
        fn_ = nullptr;
    }

private:
    void work() {
        for (;;) {
            int64_t i = next_.fetch_add(1);
            if (i >= n_tasks_) break;
            (*fn_)(i);
        }
    }
    void loop() {
        uint64_t seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [&] { return stop_ || gen_ != seen; });
                if (stop_) return;
                seen = gen_;
            }
            work();
            {
                std::lock_guard<std::mutex> g(mu_);
                ++done_;
            }
            done_cv_.notify_all();
        }
    }
    int n_;
    std::vector<std::thread> workers_;
    std::mutex mu_;
    std::condition_variable cv_, done_cv_;
    bool stop_ = false;
    uint64_t gen_ = 0;
    const std::function<void(int64_t)> *fn_ = nullptr;
    int64_t n_tasks_ = 0;
    std::atomic<int64_t> next_{0};
    int done_ = 0;
};

// ---------------------------------------------------------------- data
struct Data {
    const uint8_t *bins;  // column-major bins[f * n + r]
    int64_t n;
    int nf;
    int nb;
    std::vector<int> missing_bin;  // -1: none
    std::vector<int> widths;       // binning.histogram_widths
    std::vector<int> ncat;         // categories of a categorical feature, 0 numerical
    bool is_cat(int f) const { return !ncat.empty() && ncat[f] > 0; }
};

// src/mojotrees/binning.mojo:2303-2337
std::vector<int> histogram_widths(const Data &d) {
    std::vector<int> w(d.nf, 1);
    for (int f = 0; f < d.nf; ++f) {
        const uint8_t *col = d.bins + (int64_t)f * d.n;
        int mx = 0;
        for (int64_t r = 0; r < d.n; ++r) mx = std::max(mx, (int)col[r]);
        w[f] = std::max(w[f], mx + 1);
        int m = d.missing_bin[f] + 1;
        if (m > w[f]) w[f] = m;
        if (w[f] > d.nb) w[f] = d.nb;
    }
    return w;
}

struct Split {
    int feature = -1;
    int bin = -1;
    double gain = 0.0;
    bool found = false;
    bool default_left = false;
    bool cat = false;           // a category-set split: bins in `bits` go left
    uint64_t bits[4] = {0, 0, 0, 0};
};

inline bool cat_contains(const uint64_t *bits, int bin) {
    return (bits[bin >> 6] >> (bin & 63)) & 1ULL;
}

struct Params {
    orc_params p;
    bool const_hessian = false;
};

// src/mojotrees/gain.mojo:17-35
inline double soft_threshold_l1(double s, double l1) {
    if (l1 <= 0.0) return s;
    double mag = std::fabs(s) - l1;
    if (mag <= 0.0) return 0.0;
    return s > 0.0 ? mag : -mag;
}
inline double leaf_score(double g, double h, double l1, double l2) {
    double t = soft_threshold_l1(g, l1);
    return t * t / (h + l2);
}

// ------------------------------------------------------------ float hist
// Histogram cells are LightGBM's interleaved (grad, hess) pair plus a count
// plane (src/mojotrees/histogram.mojo:1002, :300-330).
struct FHist {
    std::vector<double> gh;  // 2 * cells
    std::vector<int64_t> c;
    void reset(int cells) {
        gh.assign(2 * (size_t)cells, 0.0);
        c.assign(cells, 0);
    }
};

// src/mojotrees/apple_cpu_policy.mojo:778-924 (row-block plan).
int plan_row_blocks(int64_t rows, int n_bins, int n_active) {
    if (rows <= 0 || n_bins <= 0 || n_active <= 0) return 1;
    int64_t cells = (int64_t)n_active * n_bins;
    int64_t per_block = cells * 3 * 8;
    int64_t by_bytes = (16LL * 1024 * 1024) / per_block;
    if (by_bytes < 1) by_bytes = 1;
    int64_t ceiling = by_bytes < 64 ? by_bytes : 64;
    int64_t min_rows = 2 * 8 * (int64_t)n_bins;
    int64_t blocks = rows / min_rows;
    if (blocks > ceiling) blocks = ceiling;
    if (blocks > rows) blocks = rows;
    if (blocks < 2) return 1;
    int64_t chunk = (rows + blocks - 1) / blocks;
    return (int)((rows + chunk - 1) / chunk);
}

// Feature-parallel float accumulation in ascending row order per cell
// (src/mojotrees/histogram.mojo:60-115, :1617, :2257), with contiguous
// ascending row blocks folded in block order when the plan blocks
// (:116-160, :2845).
void build_float(FHist &out, const Data &d, const std::vector<double> &grad,
                 const std::vector<double> &hess, const int32_t *rows,
                 int64_t m, const std::vector<int> &features, Pool &pool,
                 int forced_blocks = 0) {
    out.reset(d.nf * d.nb);
    int n_active = (int)features.size();
    int blocks = forced_blocks > 0 ? forced_blocks : plan_row_blocks(m, d.nb, n_active);
    int64_t chunk = blocks > 1 ? (m + blocks - 1) / blocks : m;
    if (blocks > 1) blocks = (int)((m + chunk - 1) / chunk);
    pool.run(n_active, [&](int64_t fi) {
        int f = features[fi];
        const uint8_t *col = d.bins + (int64_t)f * d.n;
        double *gh = out.gh.data() + 2 * (int64_t)f * d.nb;
        int64_t *cc = out.c.data() + (int64_t)f * d.nb;
        if (blocks <= 1) {
            for (int64_t i = 0; i < m; ++i) {
                int64_t r = rows ? rows[i] : i;
                int b = col[r];
                gh[2 * b] += grad[r];
                gh[2 * b + 1] += hess[r];
                cc[b] += 1;
            }
            return;
        }
        std::vector<double> part(2 * (size_t)d.nb);
        for (int blk = 0; blk < blocks; ++blk) {
            std::fill(part.begin(), part.end(), 0.0);
            int64_t lo = blk * chunk, hi = std::min(m, lo + chunk);
            for (int64_t i = lo; i < hi; ++i) {
                int64_t r = rows ? rows[i] : i;
                int b = col[r];
                part[2 * b] += grad[r];
                part[2 * b + 1] += hess[r];
                cc[b] += 1;
            }
            for (int b = 0; b < 2 * d.nb; ++b) {
                if (blk == 0) gh[b] = part[b];
                else gh[b] += part[b];
            }
        }
    });
}

// src/mojotrees/histogram.mojo:3760-3960
void subtract_float(FHist &out, const FHist &parent, const FHist &child) {
    size_t cells = parent.c.size();
    out.gh.resize(2 * cells);
    out.c.resize(cells);
    for (size_t i = 0; i < cells; ++i) {
        out.gh[2 * i] = parent.gh[2 * i] - child.gh[2 * i];
        out.gh[2 * i + 1] = parent.gh[2 * i + 1] - child.gh[2 * i + 1];
        out.c[i] = parent.c[i] - child.c[i];
    }
}

// tree._leaf_value (src/mojotrees/tree.mojo:1961-1995): serial sum over the
// value feature's bins, then -T(G) / (H + lambda_l2).
double leaf_value_float(const FHist &h, const Data &d, int value_feature,
                        const Params &P) {
    const double *gh = h.gh.data() + 2 * (int64_t)value_feature * d.nb;
    double g = 0.0, hh = 0.0;
    for (int b = 0; b < d.nb; ++b) {
        g += gh[2 * b];
        hh += gh[2 * b + 1];
    }
    return -soft_threshold_l1(g, P.p.lambda_l1) / (hh + P.p.lambda_l2);
}

// Mojo SIMD.reduce_add: pairwise halving of the lanes.
double reduce_lanes(const double *v, int w, bool tree) {
    if (!tree) {
        double s = v[0];
        for (int i = 1; i < w; ++i) s += v[i];
        return s;
    }
    double buf[64];
    for (int i = 0; i < w; ++i) buf[i] = v[i];
    while (w > 1) {
        int h = w / 2;
        for (int i = 0; i < h; ++i) buf[i] = buf[i] + buf[i + h];
        w = h;
    }
    return buf[0];
}

// ------------------------------------------------------------ categorical
// categorical.find_best_categorical_split (src/mojotrees/categorical.mojo:
// 684-782) with _onehot_search (:478-525) and _sorted_search (:527-623);
// the arithmetic helpers cat_sort_key, cat_enters_search, cat_side_cap,
// cat_partition_gain and cat_effective_l2 (tree_parameters_extra.mojo:
// 981-1042). Written once over a sums type S so the Float64 histograms and
// the integer (quantized) ones share it: Ops supplies a bin's sums, their
// sum and difference, the leaf score at an L2, the sort key, the Hessian
// guard and the count.
struct CatCfg {
    int max_cat_to_onehot, max_cat_threshold, min_data_per_group, one_hot_max_size;
    double cat_smooth, cat_l2;
};
CatCfg cat_cfg(const orc_params &p) {
    return CatCfg{p.max_cat_to_onehot, p.max_cat_threshold, p.min_data_per_group, p.one_hot_max_size,
                  p.cat_smooth, p.cat_l2};
}

// metrics._argsort (src/mojotrees/metrics.mojo:514-556): stable bottom-up
// merge sort, ascending, `<=` keeps the left run's element first.
std::vector<int> argsort_stable(const std::vector<double> &v) {
    const int n = (int)v.size();
    std::vector<int> idx(n), buf(n);
    for (int i = 0; i < n; ++i) idx[i] = i;
    for (int width = 1; width < n; width *= 2) {
        for (int lo = 0; lo < n; lo += 2 * width) {
            int mid = std::min(lo + width, n), hi = std::min(lo + 2 * width, n);
            int i = lo, j = mid, k = lo;
            while (i < mid && j < hi) buf[k++] = v[idx[i]] <= v[idx[j]] ? idx[i++] : idx[j++];
            while (i < mid) buf[k++] = idx[i++];
            while (j < hi) buf[k++] = idx[j++];
        }
        idx = buf;
    }
    return idx;
}

struct CatResult {
    double gain = 0.0;
    bool found = false;
    uint64_t bits[4] = {0, 0, 0, 0};
};

template <class Ops>
CatResult cat_search(const Ops &o, int n_cat, const typename Ops::S &total, double l2,
                     int64_t min_data_in_leaf, const CatCfg &c) {
    using S = typename Ops::S;
    CatResult best;
    if (n_cat < 2) return best;
    const double parent = o.score(total, l2);
    const bool one_hot = c.one_hot_max_size >= 0 ? n_cat <= c.one_hot_max_size
                                                   : n_cat + 1 <= c.max_cat_to_onehot;
    if (one_hot) {
        for (int t = 1; t <= n_cat; ++t) {
            const S left = o.cell(t);
            if (o.count(left) < min_data_in_leaf || o.low_hess(left)) continue;
            const S right = o.sub(total, left);
            if (o.count(right) < min_data_in_leaf) continue;
            if (o.low_hess(right)) continue;
            const double gain = o.score(left, l2) + o.score(right, l2) - parent;
            if (gain > best.gain) {
                best = CatResult();
                best.gain = gain;
                best.found = true;
                best.bits[t >> 6] |= 1ULL << (t & 63);
            }
        }
        return best;
    }
    std::vector<int> cand;
    std::vector<double> keys;
    for (int t = 1; t <= n_cat; ++t) {
        const S s = o.cell(t);
        if (!((double)o.count(s) >= c.cat_smooth)) continue;
        cand.push_back(t);
        keys.push_back(o.key(s, c.cat_smooth));
    }
    const int used = (int)cand.size();
    if (used < 2) return best;
    const std::vector<int> order = argsort_stable(keys);
    std::vector<int> sorted(used);
    for (int i = 0; i < used; ++i) sorted[i] = cand[order[i]];
    int max_num_cat = c.max_cat_threshold;
    if ((used + 1) / 2 < max_num_cat) max_num_cat = (used + 1) / 2;
    if (max_num_cat < 0) max_num_cat = 0;
    const double l2c = l2 + c.cat_l2;
    for (int d = 0; d < 2; ++d) {
        const int dir = d == 0 ? 1 : -1;
        const int start = d == 0 ? 0 : used - 1;
        int pos = start;
        int64_t group = 0;
        S left = o.zero();
        const int steps = used < max_num_cat ? used : max_num_cat;
        for (int i = 0; i < steps; ++i) {
            const int t = sorted[pos];
            pos += dir;
            const S s = o.cell(t);
            left = o.add(left, s);
            group += o.count(s);
            if (o.count(left) < min_data_in_leaf || o.low_hess(left)) continue;
            const S right = o.sub(total, left);
            if (o.count(right) < min_data_in_leaf || o.count(right) < c.min_data_per_group) break;
            if (o.low_hess(right)) break;
            if (group < c.min_data_per_group) continue;
            group = 0;
            const double gain = o.score(left, l2c) + o.score(right, l2c) - parent;
            if (gain > best.gain) {
                best = CatResult();
                best.gain = gain;
                best.found = true;
                int q = start;
                for (int k = 0; k <= i; ++k, q += dir) best.bits[sorted[q] >> 6] |= 1ULL << (sorted[q] & 63);
            }
        }
    }
    return best;
}

// Float64 sums (the reference's own histograms).
struct FloatCatOps {
    struct S {
        double g, h;
        int64_t c;
    };
    const double *gh;
    const int64_t *cnt;
    double l1, min_h;
    S cell(int t) const { return S{gh[2 * t], gh[2 * t + 1], cnt[t]}; }
    S zero() const { return S{0.0, 0.0, 0}; }
    S add(const S &a, const S &b) const { return S{a.g + b.g, a.h + b.h, a.c + b.c}; }
    S sub(const S &tot, const S &a) const { return S{tot.g - a.g, tot.h - a.h, tot.c - a.c}; }
    double score(const S &s, double l2) const { return leaf_score(s.g, s.h, l1, l2); }
    double key(const S &s, double smooth) const { return s.g / (s.h + smooth); }
    bool low_hess(const S &s) const { return s.h < min_h; }
    int64_t count(const S &s) const { return s.c; }
};

// split.find_best_split (src/mojotrees/split.mojo:601-1360), numerical
// features, L2 score, no extra-tree controls.
Split find_best_split_float(const FHist &hist, const Data &d,
                            const std::vector<int> &scan, const Params &P) {
    const int W = 8;  // SIMD_LANES = 4 * simd_width_of[float64] on arm64
    struct Slot {
        double gain = 0.0;
        int bin = -1;
        bool dl = false;
        bool found = false;
        bool cat = false;
        uint64_t bits[4] = {0, 0, 0, 0};
    };
    std::vector<Slot> slots(scan.size());
    const double l1 = P.p.lambda_l1, l2 = P.p.lambda_l2;
    const double min_h = P.p.min_sum_hessian;
    const int64_t min_c = P.p.min_data_in_leaf;
    for (size_t fi = 0; fi < scan.size(); ++fi) {
        int f = scan[fi];
        const double *gh = hist.gh.data() + 2 * (int64_t)f * d.nb;
        const int64_t *cc = hist.c.data() + (int64_t)f * d.nb;
        double lg[W] = {0}, lh[W] = {0};
        int64_t tc = 0;
        int b = 0;
        while (b + W <= d.nb) {
            for (int k = 0; k < W; ++k) {
                lg[k] += gh[2 * (b + k)];
                lh[k] += gh[2 * (b + k) + 1];
                tc += cc[b + k];
            }
            b += W;
        }
        double tg = reduce_lanes(lg, W, P.p.totals_tree_reduce != 0);
        double th = reduce_lanes(lh, W, P.p.totals_tree_reduce != 0);
        while (b < d.nb) {
            tg += gh[2 * b];
            th += gh[2 * b + 1];
            tc += cc[b];
            ++b;
        }
        if (d.is_cat(f)) {
            // a categorical feature is searched as category partitions
            // (split.mojo:1022-1066); bin 0 joins no set
            FloatCatOps ops{gh, cc, l1, min_h};
            CatResult cr = cat_search(ops, d.ncat[f], FloatCatOps::S{tg, th, tc}, l2, min_c, cat_cfg(P.p));
            Slot s;
            if (cr.found) {
                s.gain = cr.gain;
                s.found = true;
                s.cat = true;
                std::memcpy(s.bits, cr.bits, sizeof s.bits);
            }
            slots[fi] = s;
            continue;
        }
        int mb = d.missing_bin[f];
        double pg = soft_threshold_l1(tg, l1);
        double parent_score = pg * pg / (th + l2);
        int n_scan = mb >= 0 ? mb : d.nb;
        int n_lim = n_scan;
        if (!d.widths.empty() && d.widths[f] < n_lim) n_lim = d.widths[f];
        double mg = 0.0, mh = 0.0;
        int64_t mc = 0;
        if (mb >= 0) {
            mg = gh[2 * mb];
            mh = gh[2 * mb + 1];
            mc = cc[mb];
        }
        int scan_to = n_lim < n_scan ? n_lim : n_scan;
        double lgs = 0.0, lhs = 0.0;
        int64_t lcs = 0;
        Slot s;
        for (int bb = 0; bb < scan_to; ++bb) {
            if (bb == n_scan - 1 && mc == 0) break;
            lgs += gh[2 * bb];
            lhs += gh[2 * bb + 1];
            lcs += cc[bb];
            if (mb >= 0) {
                double a = lgs + mg, ah = lhs + mh;
                int64_t ac = lcs + mc;
                double rg = tg - a, rh = th - ah;
                if (!(ah < min_h || rh < min_h || ac < min_c || tc - ac < min_c)) {
                    double tl = soft_threshold_l1(a, l1), tr = soft_threshold_l1(rg, l1);
                    double gain = tl * tl / (ah + l2) + tr * tr / (rh + l2) - parent_score;
                    if (gain > s.gain) {
                        s.gain = gain;
                        s.bin = bb;
                        s.dl = true;
                        s.found = true;
                    }
                }
            }
            if (mb < 0 || mc > 0) {
                double rg = tg - lgs, rh = th - lhs;
                if (!(lhs < min_h || rh < min_h || lcs < min_c || tc - lcs < min_c)) {
                    double tl = soft_threshold_l1(lgs, l1), tr = soft_threshold_l1(rg, l1);
                    double gain = tl * tl / (lhs + l2) + tr * tr / (rh + l2) - parent_score;
                    if (gain > s.gain) {
                        s.gain = gain;
                        s.bin = bb;
                        s.dl = false;
                        s.found = true;
                    }
                }
            }
        }
        slots[fi] = s;
    }
    Split best;
    for (size_t fi = 0; fi < scan.size(); ++fi) {
        if (slots[fi].found && slots[fi].gain > best.gain) {
            best.gain = slots[fi].gain;
            best.feature = scan[fi];
            best.bin = slots[fi].bin;
            best.default_left = slots[fi].dl;
            best.found = true;
            best.cat = slots[fi].cat;
            std::memcpy(best.bits, slots[fi].bits, sizeof best.bits);
        }
    }
    return best;
}

// ------------------------------------------------------------ quantized
// src/mojotrees/quantized_gradient.mojo:475-492
uint64_t quant_stream(int64_t seed, int64_t round_index, int64_t class_index,
                      int64_t plane) {
    uint64_t h = splitmix64((uint64_t)(seed & 0x7FFFFFFFFFFFFFFFLL));
    h = splitmix64(h ^ (uint64_t)(round_index & 0x7FFFFFFFFFFFFFFFLL));
    h = splitmix64(h ^ (uint64_t)((class_index + 1) & 0x7FFFFFFFFFFFFFFFLL));
    return splitmix64(h ^ ((uint64_t)plane * GOLDEN));
}

// quantize_scalar (src/mojotrees/quantized_gradient.mojo:1479-1545)
inline int64_t quantize_scalar(double value, double units, int64_t max_unit,
                               bool stochastic, uint64_t counter) {
    double y = value * units;
    double lim = (double)max_unit;
    if (y > lim) y = lim;
    else if (y < -lim) y = -lim;
    if (stochastic) {
        double u = uniform(counter);
        if (y >= 0.0) return (int64_t)std::floor(y + u);
        return -(int64_t)std::floor(-y + u);
    }
    return (int64_t)std::round(y);  // ties away from zero
}

struct QScales {
    double gu = 1.0, hu = 1.0;
    int64_t gmax = 0, hmax = 0;
};

// The scale rules of derive_scales (quantized_gradient.mojo:1343-1453):
// LightGBM's max-abs lattice, or the reference's magnitude-sum power-of-two
// lattice (SCALE_MAGNITUDE_SUM at SCALE_SHAPE_POW2, the rule its GPU
// histogram ships and its CPU quantized path defaults to).
constexpr int kRuleMaxAbs = 0;
constexpr int kRuleMagnitudeSum = 1;
constexpr double kFixedOne = 1073741824.0;  // FIXED_ONE = 2^30 (quantized_gradient.mojo:418)
constexpr double kMagnitudeFloor = 1e-12;   // MAGNITUDE_FLOOR (quantized_gradient.mojo:428)

// largest_power_of_two_at_most (quantized_gradient.mojo:856-888): 2^floor(
// log2 x) for a positive normal x, by clearing the mantissa bits; zero,
// subnormal and non-finite inputs are refused.
double largest_power_of_two_at_most(double x) {
    if (!std::isfinite(x) || x <= 0.0) throw std::runtime_error("a power-of-two floor needs a positive finite value");
    uint64_t b;
    std::memcpy(&b, &x, 8);
    const uint64_t biased = (b >> 52) & 0x7FF;
    if (biased == 0) throw std::runtime_error("a power-of-two floor needs a normal value");
    const uint64_t out = biased << 52;
    double p;
    std::memcpy(&p, &out, 8);
    return p;
}

// fixed_point_scale_pow2 (quantized_gradient.mojo:908-1117): the power of two
// 2^k <= fl(2^30 / max(total, 1e-12)), which must be a binary32 value exactly
// (the width the device multiplies by).
double fixed_point_scale_pow2(double total) {
    if (!std::isfinite(total)) throw std::runtime_error("gradients and hessians must be finite");
    const double t = total < kMagnitudeFloor ? kMagnitudeFloor : total;
    const double q = kFixedOne / t;
    if (!std::isfinite(q) || q <= 0.0)
        throw std::runtime_error("gradient/hessian magnitudes are out of range for the fixed-point histogram");
    const double p = largest_power_of_two_at_most(q);
    const float f = (float)p;
    if (!std::isfinite(f) || f <= 0.0f || (double)f != p)
        throw std::runtime_error("gradient/hessian magnitudes are out of range for the fixed-point histogram");
    return p;
}

// The device magnitude reduction in its fixed order
// (gpu_objectives_native._abs_sum_kernel :982-1040 and sum_abs_partials
// :1100-1125): 256 workgroups of 256 threads; thread t of workgroup b adds
// |x| in binary32 for rows b * 256 + t, stepping by 65536; each workgroup
// halves its 256 sums in binary32 (s[t] += s[t + a] for a = 128, 64, .., 1);
// the 256 workgroup sums are added in binary64 in ascending order. Rows
// outside the round's sample (in_sample[r] == 0) add nothing, and rows whose
// gradient or hessian is not finite are left out, as gradient_stats
// (:762-810) leaves them out.
void magnitude_sums(const std::vector<double> &grad, const std::vector<double> &hess,
                    const std::vector<uint8_t> &in_sample, double &sum_g, double &sum_h) {
    constexpr int kBlocks = 256, kThreads = 256;
    const int64_t n = (int64_t)grad.size();
    std::vector<float> pg(kBlocks), ph(kBlocks);
    float sg[kThreads], sh[kThreads];
    for (int b = 0; b < kBlocks; ++b) {
        for (int t = 0; t < kThreads; ++t) {
            float ag = 0.0f, ah = 0.0f;
            for (int64_t r = (int64_t)b * kThreads + t; r < n; r += (int64_t)kBlocks * kThreads) {
                if (!in_sample.empty() && !in_sample[r]) continue;
                const float g = std::fabs((float)grad[r]), h = std::fabs((float)hess[r]);
                if (!(std::isfinite(g) && std::isfinite(h))) continue;
                ag += g;
                ah += h;
            }
            sg[t] = ag;
            sh[t] = ah;
        }
        for (int a = kThreads / 2; a > 0; a /= 2)
            for (int t = 0; t < a; ++t) {
                sg[t] = sg[t] + sg[t + a];
                sh[t] = sh[t] + sh[t + a];
            }
        pg[b] = sg[0];
        ph[b] = sh[0];
    }
    sum_g = 0.0;
    sum_h = 0.0;
    for (int b = 0; b < kBlocks; ++b) {
        sum_g += (double)pg[b];
        sum_h += (double)ph[b];
    }
}

// gradient_stats + derive_scales + quantize_round_cpu
// (src/mojotrees/quantized_gradient.mojo:762-810, :1343-1453, :2487-2565).
// Max-abs: units = (B / 2) / max|g| and B / max|h| (one unit over max|h|
// under a constant hessian), clamps B / 2 and B. Magnitude sum: units =
// fixed_point_scale_pow2(sum |g|) and (sum |h|) -- again 1 / max|h| with a
// one-unit clamp under a constant hessian -- and clamps 2^30. Every row is
// quantized; the sample decides the magnitudes.
QScales quantize_round(const std::vector<double> &grad,
                       const std::vector<double> &hess, const int32_t *rows,
                       int64_t n_sel, int quant_bins, bool stochastic,
                       int64_t seed, int64_t round_index, int64_t class_index,
                       bool const_hessian, int rule, int32_t *qg, int32_t *qh, Pool &pool) {
    int64_t n = (int64_t)grad.size();
    double max_g = 0.0, max_h = 0.0;
    int64_t count = rows ? n_sel : n;
    for (int64_t i = 0; i < count; ++i) {
        int64_t r = rows ? rows[i] : i;
        double g = std::fabs(grad[r]), h = std::fabs(hess[r]);
        if (!(std::isfinite(g) && std::isfinite(h))) continue;
        if (g > max_g) max_g = g;
        if (h > max_h) max_h = h;
    }
    QScales s;
    if (max_g < kMagnitudeFloor) max_g = kMagnitudeFloor;
    if (max_h < kMagnitudeFloor) max_h = kMagnitudeFloor;
    if (rule == kRuleMagnitudeSum) {
        std::vector<uint8_t> in_sample;
        if (rows) {
            in_sample.assign((size_t)n, 0);
            for (int64_t i = 0; i < n_sel; ++i) in_sample[(size_t)rows[i]] = 1;
        }
        double sum_g = 0.0, sum_h = 0.0;
        magnitude_sums(grad, hess, in_sample, sum_g, sum_h);
        s.gu = fixed_point_scale_pow2(sum_g);
        s.gmax = (int64_t)kFixedOne;
        if (const_hessian) {
            s.hu = 1.0 / max_h;
            s.hmax = 1;
        } else {
            s.hu = fixed_point_scale_pow2(sum_h);
            s.hmax = (int64_t)kFixedOne;
        }
    } else {
        s.gmax = quant_bins / 2;
        s.gu = (double)s.gmax / max_g;
        if (const_hessian) {
            s.hmax = 1;
            s.hu = 1.0 / max_h;
        } else {
            s.hmax = quant_bins;
            s.hu = (double)s.hmax / max_h;
        }
    }
    uint64_t gs = quant_stream(seed, round_index, class_index, 0);
    uint64_t hs = quant_stream(seed, round_index, class_index, 1);
    int64_t blocks = (n + 65535) / 65536;
    pool.run(blocks, [&](int64_t b) {
        int64_t lo = b * 65536, hi = std::min(n, lo + 65536);
        for (int64_t r = lo; r < hi; ++r) {
            qg[r] = (int32_t)quantize_scalar(grad[r], s.gu, s.gmax, stochastic, gs + (uint64_t)r);
            qh[r] = (int32_t)quantize_scalar(hess[r], s.hu, s.hmax, stochastic, hs + (uint64_t)r);
        }
    });
    return s;
}

struct QHist {
    std::vector<int64_t> v;  // 3 per cell: grad, hess, count
    void reset(int cells) { v.assign(3 * (size_t)cells, 0); }
};

// Integer accumulation: order-free (quantized_gradient.mojo:2688-2945).
void build_quant(QHist &out, const Data &d, const int32_t *qg, const int32_t *qh,
                 const int32_t *rows, int64_t m, const std::vector<int> &features,
                 Pool &pool) {
    out.reset(d.nf * d.nb);
    pool.run((int64_t)features.size(), [&](int64_t fi) {
        int f = features[fi];
        const uint8_t *col = d.bins + (int64_t)f * d.n;
        int64_t *cell = out.v.data() + 3 * (int64_t)f * d.nb;
        for (int64_t i = 0; i < m; ++i) {
            int64_t r = rows ? rows[i] : i;
            int64_t *c = cell + 3 * col[r];
            c[0] += qg[r];
            c[1] += qh[r];
            c[2] += 1;
        }
    });
}

// subtract_quantized (src/mojotrees/quantized_gradient.mojo:1989-2025)
void subtract_quant(QHist &out, const QHist &parent, const QHist &child) {
    out.v.resize(parent.v.size());
    for (size_t i = 0; i < parent.v.size(); ++i) out.v[i] = parent.v[i] - child.v[i];
}

// hessian_units_at_least (quantized_gradient.mojo:3336-3364)
int64_t hessian_units_at_least(double min_child_hess, const QScales &s) {
    if (min_child_hess <= 0.0) return 0;
    double units = min_child_hess * s.hu;
    double fl = std::floor(units);
    if (fl < units) fl += 1.0;
    return (int64_t)fl;
}

// quantized_leaf_score / quantized_split_gain / quantized_leaf_output
// (quantized_gradient.mojo:3252-3334), with dequant = Float64(q) / units.
inline double qscore(int64_t g, int64_t h, const QScales &s, double l1, double l2) {
    return leaf_score((double)g / s.gu, (double)h / s.hu, l1, l2);
}
inline double qleaf(int64_t g, int64_t h, const QScales &s, double l1, double l2) {
    return -soft_threshold_l1((double)g / s.gu, l1) / ((double)h / s.hu + l2);
}

// Integer sums on the (gu, hu) lattice: accumulated exactly, dequantized
// (Float64(q) / units) for every score and sort key, the Hessian guard in
// integer units (hessian_units_at_least), as the numerical quantized scan.
struct QuantCatOps {
    struct S {
        int64_t g, h, c;
    };
    const int64_t *cell3;  // {grad, hess, count} per bin
    double gu, hu, l1;
    int64_t hmin;
    S cell(int t) const { return S{cell3[3 * t], cell3[3 * t + 1], cell3[3 * t + 2]}; }
    S zero() const { return S{0, 0, 0}; }
    S add(const S &a, const S &b) const { return S{a.g + b.g, a.h + b.h, a.c + b.c}; }
    S sub(const S &tot, const S &a) const { return S{tot.g - a.g, tot.h - a.h, tot.c - a.c}; }
    double score(const S &s, double l2) const { return leaf_score((double)s.g / gu, (double)s.h / hu, l1, l2); }
    double key(const S &s, double smooth) const { return ((double)s.g / gu) / ((double)s.h / hu + smooth); }
    bool low_hess(const S &s) const { return s.h < hmin; }
    int64_t count(const S &s) const { return s.c; }
};

// The integer form of find_best_split: the same candidate order, guards and
// strict-greater fold as split.mojo:601-1360, with left/right/parent sums
// kept as exact integers and each candidate scored by quantized_split_gain.
Split find_best_split_quant(const QHist &hist, const Data &d,
                            const std::vector<int> &scan, const QScales &s,
                            const Params &P) {
    const double l1 = P.p.lambda_l1, l2 = P.p.lambda_l2;
    const int64_t hmin = hessian_units_at_least(P.p.min_sum_hessian, s);
    const int64_t min_c = P.p.min_data_in_leaf;
    Split best;
    for (size_t fi = 0; fi < scan.size(); ++fi) {
        int f = scan[fi];
        const int64_t *cell = hist.v.data() + 3 * (int64_t)f * d.nb;
        int64_t tg = 0, th = 0, tc = 0;
        for (int b = 0; b < d.nb; ++b) {
            tg += cell[3 * b];
            th += cell[3 * b + 1];
            tc += cell[3 * b + 2];
        }
        if (d.is_cat(f)) {
            QuantCatOps ops{cell, s.gu, s.hu, l1, hmin};
            CatResult cr = cat_search(ops, d.ncat[f], QuantCatOps::S{tg, th, tc}, l2, min_c, cat_cfg(P.p));
            if (cr.found && cr.gain > best.gain) {
                best = Split();
                best.gain = cr.gain;
                best.feature = f;
                best.found = true;
                best.cat = true;
                std::memcpy(best.bits, cr.bits, sizeof best.bits);
            }
            continue;
        }
        double parent = qscore(tg, th, s, l1, l2);
        int mb = d.missing_bin[f];
        int n_scan = mb >= 0 ? mb : d.nb;
        int n_lim = n_scan;
        if (!d.widths.empty() && d.widths[f] < n_lim) n_lim = d.widths[f];
        int64_t mg = 0, mh = 0, mc = 0;
        if (mb >= 0) {
            mg = cell[3 * mb];
            mh = cell[3 * mb + 1];
            mc = cell[3 * mb + 2];
        }
        int scan_to = n_lim < n_scan ? n_lim : n_scan;
        int64_t lg = 0, lh = 0, lc = 0;
        double f_gain = 0.0;
        int f_bin = -1;
        bool f_dl = false, f_found = false;
        for (int b = 0; b < scan_to; ++b) {
            if (b == n_scan - 1 && mc == 0) break;
            lg += cell[3 * b];
            lh += cell[3 * b + 1];
            lc += cell[3 * b + 2];
            if (mb >= 0) {
                int64_t ag = lg + mg, ah = lh + mh, ac = lc + mc;
                int64_t rg = tg - ag, rh = th - ah, rc = tc - ac;
                if (!(ah < hmin || rh < hmin || ac < min_c || rc < min_c)) {
                    double gain = qscore(ag, ah, s, l1, l2) + qscore(rg, rh, s, l1, l2) - parent;
                    if (gain > f_gain) {
                        f_gain = gain;
                        f_bin = b;
                        f_dl = true;
                        f_found = true;
                    }
                }
            }
            if (mb < 0 || mc > 0) {
                int64_t rg = tg - lg, rh = th - lh, rc = tc - lc;
                if (!(lh < hmin || rh < hmin || lc < min_c || rc < min_c)) {
                    double gain = qscore(lg, lh, s, l1, l2) + qscore(rg, rh, s, l1, l2) - parent;
                    if (gain > f_gain) {
                        f_gain = gain;
                        f_bin = b;
                        f_dl = false;
                        f_found = true;
                    }
                }
            }
        }
        if (f_found && f_gain > best.gain) {
            best = Split();
            best.gain = f_gain;
            best.feature = f;
            best.bin = f_bin;
            best.default_left = f_dl;
            best.found = true;
        }
    }
    return best;
}

// ---------------------------------------------------------------- tree
struct Tree {
    std::vector<int> feature, threshold, left, right, default_left, missing_bin;
    std::vector<double> value, gain, count;
    std::vector<uint64_t> cat;  // 4 words per node: the left set of a categorical node
    int n_leaves = 0;
    int add_node(double v, double cnt) {
        int id = (int)feature.size();
        cat.insert(cat.end(), 4, 0ULL);
        feature.push_back(-1);
        threshold.push_back(-1);
        left.push_back(-1);
        right.push_back(-1);
        default_left.push_back(0);
        missing_bin.push_back(-1);
        value.push_back(v);
        gain.push_back(0.0);
        count.push_back(cnt);
        return id;
    }
    bool is_cat(int node) const { return feature[node] >= 0 && threshold[node] < 0; }
    // tree.goes_left (src/mojotrees/tree.mojo:483-495): a categorical node
    // routes by set membership (bin 0 is never a member)
    bool goes_left(int node, int bin) const {
        if (is_cat(node)) return cat_contains(&cat[4 * (size_t)node], bin);
        if (bin == missing_bin[node]) return default_left[node] != 0;
        return bin <= threshold[node];
    }
    double predict(const Data &d, int64_t r) const {
        int node = 0;
        while (feature[node] >= 0) {
            int b = d.bins[(int64_t)feature[node] * d.n + r];
            node = goes_left(node, b) ? left[node] : right[node];
        }
        return value[node];
    }
};

// sampling.mojo:319-548 (feature_fraction per tree)
uint64_t sampling_stream(int64_t seed, int64_t tree_index, int64_t tag) {
    uint64_t h = splitmix64((uint64_t)(seed & 0x7FFFFFFFFFFFFFFFLL));
    h = splitmix64(h ^ (uint64_t)(tree_index & 0x7FFFFFFFFFFFFFFFLL));
    return splitmix64(h ^ (uint64_t)(tag & 0x7FFFFFFFFFFFFFFFLL));
}
int selection_count(int total, double fraction) {
    if (total <= 0) return 0;
    int count = (int)((double)total * fraction + 0.5);
    int floor_count = total >= 2 ? 2 : total;
    if (count < floor_count) count = floor_count;
    if (count > total) count = total;
    return count;
}
std::vector<int> select_tree_features(int nf, double fraction, int64_t seed,
                                      int64_t tree_index) {
    std::vector<int> pool(nf);
    for (int f = 0; f < nf; ++f) pool[f] = f;
    if (fraction >= 1.0) return pool;
    int count = selection_count(nf, fraction);
    uint64_t stream = sampling_stream(seed, tree_index, 0);
    std::vector<int> out;
    int chosen = 0;
    for (int i = 0; i < nf; ++i) {
        if (chosen >= count) break;
        double prob = (double)(count - chosen) / (double)(nf - i);
        if (uniform(stream + (uint64_t)i) < prob) {
            out.push_back(pool[i]);
            ++chosen;
        }
    }
    return out;
}

// tree.partition_rows_into (src/mojotrees/tree.mojo:733-826): stable.
void partition_rows(const Data &d, const std::vector<int32_t> &rows,
                    const Split &s, int missing_bin, std::vector<int32_t> &left,
                    std::vector<int32_t> &right) {
    left.clear();
    right.clear();
    const uint8_t *col = d.bins + (int64_t)s.feature * d.n;
    for (int32_t r : rows) {
        int b = col[r];
        bool gl = s.cat ? cat_contains(s.bits, b) : (b == missing_bin) ? s.default_left : (b <= s.bin);
        (gl ? left : right).push_back(r);
    }
}

template <class H>
struct Leaf {
    int node;
    std::vector<int32_t> rows;
    H hist;
    Split split;
    int depth;
};

struct FloatPolicy {
    const Data &d;
    const std::vector<double> &grad, &hess;
    const Params &P;
    Pool &pool;
    int value_feature;
    using H = FHist;
    void build(H &h, const int32_t *rows, int64_t m, const std::vector<int> &feats) {
        build_float(h, d, grad, hess, rows, m, feats, pool);
    }
    void subtract(H &o, const H &p, const H &c) { subtract_float(o, p, c); }
    double value(const H &h, int64_t) { return leaf_value_float(h, d, value_feature, P); }
    Split search(const H &h, const std::vector<int> &scan) {
        return find_best_split_float(h, d, scan, P);
    }
};

struct QuantPolicy {
    const Data &d;
    const int32_t *qg, *qh;
    const QScales &s;
    const Params &P;
    Pool &pool;
    int value_feature;
    using H = QHist;
    void build(H &h, const int32_t *rows, int64_t m, const std::vector<int> &feats) {
        build_quant(h, d, qg, qh, rows, m, feats, pool);
    }
    void subtract(H &o, const H &p, const H &c) { subtract_quant(o, p, c); }
    double value(const H &h, int64_t) {
        // Every row lands in one bin of every feature, so the value feature's
        // bins sum to the node totals (tree._leaf_value reads the same one).
        int64_t g = 0, hh = 0;
        const int64_t *cell = h.v.data() + 3 * (int64_t)value_feature * d.nb;
        for (int b = 0; b < d.nb; ++b) {
            g += cell[3 * b];
            hh += cell[3 * b + 1];
        }
        return qleaf(g, hh, s, P.p.lambda_l1, P.p.lambda_l2);
    }
    Split search(const H &h, const std::vector<int> &scan) {
        return find_best_split_quant(h, d, scan, s, P);
    }
};

// tree.grow_tree_leaves_profiled (src/mojotrees/tree.mojo:3125-4290),
// leaf-wise: growth_policy.GrowthSchedule.next_leaf (growth_policy.mojo:
// 659-677), smaller child built and its sibling derived by subtraction,
// left child replaces the parent's frontier slot, right child appended.
template <class Policy>
Tree grow_tree(Policy &pol, const Data &d, const Params &P,
               const std::vector<int32_t> *bag, int64_t tree_index,
               std::vector<std::pair<int, std::vector<int32_t>>> *leaf_rows) {
    using H = typename Policy::H;
    Tree tree;
    std::vector<int> tree_features = select_tree_features(
        d.nf, P.p.feature_fraction, P.p.feature_fraction_seed, tree_index);
    bool per_node_draw = (int)tree_features.size() != d.nf;
    std::vector<int> scan = tree_features;  // empty-vs-all: same scan order
    (void)per_node_draw;
    std::vector<Leaf<H>> frontier;
    Leaf<H> root;
    root.depth = 0;
    if (bag && !bag->empty()) {
        root.rows = *bag;
        pol.build(root.hist, root.rows.data(), (int64_t)root.rows.size(), tree_features);
    } else {
        root.rows.resize(d.n);
        for (int64_t r = 0; r < d.n; ++r) root.rows[r] = (int32_t)r;
        pol.build(root.hist, nullptr, d.n, tree_features);
    }
    int64_t n_root = (int64_t)root.rows.size();
    root.node = tree.add_node(pol.value(root.hist, n_root), (double)n_root);
    auto search = [&](const H &h, int64_t n_rows, int depth) {
        if (P.p.max_depth > 0 && depth >= P.p.max_depth) return Split();
        if (n_rows < 2 * (int64_t)P.p.min_data_in_leaf || n_rows < 2) return Split();
        return pol.search(h, scan);
    };
    root.split = search(root.hist, n_root, 0);
    frontier.push_back(std::move(root));
    int n_leaves = 1;
    while (n_leaves < P.p.num_leaves) {
        int best_i = -1;
        double best_gain = 0.0;
        for (size_t i = 0; i < frontier.size(); ++i) {
            const Split &s = frontier[i].split;
            if (s.found && s.gain > 0.0 && s.gain > best_gain) {
                best_gain = s.gain;
                best_i = (int)i;
            }
        }
        if (best_i < 0) break;
        Leaf<H> &par = frontier[best_i];
        Split split = par.split;
        // tree._set_split (src/mojotrees/tree.mojo:462-481): a categorical
        // node has no threshold and no missing bin
        int mbin = split.cat ? -1 : d.missing_bin[split.feature];
        std::vector<int32_t> lrows, rrows;
        partition_rows(d, par.rows, split, mbin, lrows, rrows);
        H lh, rh;
        bool builds_left = lrows.size() <= rrows.size();
        if (builds_left) {
            pol.build(lh, lrows.data(), (int64_t)lrows.size(), tree_features);
            pol.subtract(rh, par.hist, lh);
        } else {
            pol.build(rh, rrows.data(), (int64_t)rrows.size(), tree_features);
            pol.subtract(lh, par.hist, rh);
        }
        double lv = pol.value(lh, (int64_t)lrows.size());
        double rv = pol.value(rh, (int64_t)rrows.size());
        int ln = tree.add_node(lv, (double)lrows.size());
        int rn = tree.add_node(rv, (double)rrows.size());
        int pn = par.node;
        tree.left[pn] = ln;
        tree.right[pn] = rn;
        tree.feature[pn] = split.feature;
        tree.gain[pn] = split.gain;
        tree.threshold[pn] = split.cat ? -1 : split.bin;
        tree.default_left[pn] = split.default_left ? 1 : 0;
        tree.missing_bin[pn] = mbin;
        if (split.cat) std::memcpy(&tree.cat[4 * (size_t)pn], split.bits, sizeof split.bits);
        int cd = par.depth + 1;
        Split ls = search(lh, (int64_t)lrows.size(), cd);
        Split rs = search(rh, (int64_t)rrows.size(), cd);
        Leaf<H> L{ln, std::move(lrows), std::move(lh), ls, cd};
        Leaf<H> R{rn, std::move(rrows), std::move(rh), rs, cd};
        frontier[best_i] = std::move(L);
        frontier.push_back(std::move(R));
        ++n_leaves;
    }
    tree.n_leaves = n_leaves;
    if (leaf_rows) {
        leaf_rows->clear();
        for (auto &l : frontier) leaf_rows->emplace_back(l.node, std::move(l.rows));
    }
    return tree;
}

// bagging.sample_rows / refresh_bag (src/mojotrees/bagging.mojo:1-150)
void refresh_bag(std::vector<int32_t> &bag, const orc_params &p, int64_t n,
                 int64_t iteration) {
    if (!(p.bagging_freq > 0 && p.bagging_fraction < 1.0)) return;
    if (iteration % p.bagging_freq != 0) return;
    int64_t bag_index = iteration / p.bagging_freq;
    uint64_t stream = splitmix64((uint64_t)(p.bagging_seed & 0x7FFFFFFFFFFFFFFFLL) ^
                                 ((uint64_t)bag_index * GOLDEN));
    bag.clear();
    double min_draw = 2.0;
    int64_t min_row = 0;
    for (int64_t r = 0; r < n; ++r) {
        double u = uniform(stream + (uint64_t)r);
        if (u < p.bagging_fraction) bag.push_back((int32_t)r);
        if (u < min_draw) {
            min_draw = u;
            min_row = r;
        }
    }
    if (bag.empty()) bag.push_back((int32_t)min_row);
}

// ranking._refresh_query_bag / _expand_queries (src/mojotrees/ranking.mojo:
// 655-686): the same draw over query indices, then the rows of the drawn
// queries, ascending
void refresh_query_bag(std::vector<int32_t> &bag, const orc_params &p, const std::vector<int64_t> &starts,
                       int64_t iteration) {
    if (!(p.bagging_freq > 0 && p.bagging_fraction < 1.0)) return;
    if (iteration % p.bagging_freq != 0) return;
    std::vector<int32_t> qbag;
    refresh_bag(qbag, p, (int64_t)starts.size() - 1, iteration);
    bag.clear();
    for (int32_t q : qbag)
        for (int64_t r = starts[q]; r < starts[q + 1]; ++r) bag.push_back((int32_t)r);
}

// goss.mojo:240-396
double select_kth_desc(std::vector<double> &v, int64_t k) {
    auto median3 = [](double a, double b, double c) {
        if (a < b) {
            if (b < c) return b;
            return a < c ? c : a;
        }
        if (a < c) return a;
        return b < c ? c : b;
    };
    int64_t lo = 0, hi = (int64_t)v.size() - 1;
    while (lo < hi) {
        int64_t mid = lo + (hi - lo) / 2;
        double pivot = median3(v[lo], v[mid], v[hi]);
        int64_t i = lo, j = hi;
        while (i <= j) {
            while (v[i] > pivot) ++i;
            while (v[j] < pivot) --j;
            if (i <= j) {
                std::swap(v[i], v[j]);
                ++i;
                --j;
            }
        }
        if (k <= j) hi = j;
        else if (k >= i) lo = i;
        else return pivot;
    }
    return v[lo];
}

// goss_select (goss.mojo:308-357) over per-row importance: the sample in
// ascending row order into bag, other[r] = 1 for a sampled small-importance
// row (0 for every other row); returns the weight of those rows,
// (n - top_k) / other_k (1 when other_k is 0).
double goss_select(const std::vector<double> &imp, const orc_params &p, int64_t round,
                   std::vector<int32_t> &bag, std::vector<uint8_t> &other) {
    const int64_t n = (int64_t)imp.size();
    int64_t top_k = (int64_t)((double)n * p.top_rate);
    if (top_k < 1) top_k = 1;
    if (top_k > n) top_k = n;
    int64_t other_k = (int64_t)((double)n * p.other_rate);
    if (other_k > n - top_k) other_k = n - top_k;
    std::vector<double> scratch = imp;
    double threshold = select_kth_desc(scratch, top_k - 1);
    double mult = 1.0;
    if (other_k > 0) mult = (double)(n - top_k) / (double)other_k;
    uint64_t stream = splitmix64((uint64_t)(p.goss_seed & 0x7FFFFFFFFFFFFFFFLL) ^
                                 ((uint64_t)round * GOLDEN));
    bag.clear();
    other.assign((size_t)n, 0);
    int64_t n_top = 0, n_other = 0;
    for (int64_t r = 0; r < n; ++r) {
        if (imp[r] >= threshold) {
            bag.push_back((int32_t)r);
            ++n_top;
        } else {
            int64_t rest_need = other_k - n_other;
            int64_t rest_all = (n - r) - (top_k - n_top);
            double prob = rest_all <= 0 ? (rest_need > 0 ? 1.0 : 0.0)
                                        : (double)rest_need / (double)rest_all;
            if (uniform(stream + (uint64_t)r) < prob) {
                bag.push_back((int32_t)r);
                other[(size_t)r] = 1;
                ++n_other;
            }
        }
    }
    return mult;
}

// GossParams.active (goss.mojo:102-157): on, and past floor(1 / learning_rate)
// warmup rounds
bool goss_active(const orc_params &p, int64_t round) {
    if (!p.goss) return false;
    int64_t warm = p.learning_rate <= 0.0 ? 0 : (int64_t)(1.0 / p.learning_rate);
    return round >= warm;
}

// apply_goss_scaling (goss.mojo:360-373): the sampled small-importance rows'
// derivatives times the weight, in binary64
void goss_scale(const std::vector<uint8_t> &other, double mult, std::vector<double> &grad,
                std::vector<double> &hess, const std::vector<int32_t> &bag) {
    for (int32_t r : bag)
        if (other[(size_t)r]) {
            grad[r] *= mult;
            hess[r] *= mult;
        }
}

// goss_round (goss.mojo:376-396): a single-output round's sample from
// goss_importance = |grad * hess| (:294-305), its rows scaled in place.
// scale, when given, receives each sampled row's multiplier (1 for a top row).
bool goss_round(std::vector<int32_t> &bag, std::vector<double> &grad,
                std::vector<double> &hess, const orc_params &p, int64_t round,
                std::vector<double> *scale = nullptr) {
    if (!goss_active(p, round)) return false;
    const int64_t n = (int64_t)grad.size();
    std::vector<double> imp(n);
    for (int64_t r = 0; r < n; ++r) imp[r] = std::fabs(grad[r] * hess[r]);
    std::vector<uint8_t> other;
    const double mult = goss_select(imp, p, round, bag, other);
    goss_scale(other, mult, grad, hess, bag);
    if (scale) {
        scale->clear();
        for (int32_t r : bag) scale->push_back(other[(size_t)r] ? mult : 1.0);
    }
    return true;
}

// boosting._multiclass_goss_select (boosting.mojo:3680-3710): one sample for
// a whole multiclass round from each row's sum over the classes, in class
// order, of |grad_k * hess_k| with the derivatives at the round's precision
// (_fill_softmax_grad_hess, as the class trees will use them).
double goss_select_multiclass(const std::vector<double> &prob, const double *labels, int64_t n, int K,
                              const double *weights, const orc_params &p, int64_t round,
                              std::vector<int32_t> &bag, std::vector<uint8_t> &other);

// ---------------------------------------------------------------- ranking
// LambdaRank, LightGBM's LambdarankNDCG (src/mojotrees/ranking.mojo).
struct RankSpec {
    std::vector<int64_t> starts;  // n_queries + 1
    int truncation = 30;
    double sigmoid = 1.0;
    bool norm = true;
};

// label_gain (ranking.mojo:235-237)
inline double label_gain(int l) { return (double)((1LL << l) - 1); }

// _discounts (ranking.mojo:240-245)
std::vector<double> rank_discounts(int64_t n) {
    std::vector<double> d((size_t)n);
    for (int64_t i = 0; i < n; ++i) d[i] = 1.0 / ref_log2((double)i + 2.0);
    return d;
}

// _argsort_desc_range (ranking.mojo:248-289): stable descending, ties in
// input order.
std::vector<int64_t> argsort_desc(const double *v, int64_t cnt) {
    std::vector<int64_t> idx((size_t)cnt);
    for (int64_t i = 0; i < cnt; ++i) idx[i] = i;
    std::stable_sort(idx.begin(), idx.end(), [&](int64_t a, int64_t b) { return v[a] > v[b]; });
    return idx;
}

// max_dcg (ranking.mojo:306-323) over the query's labels, cutoff k
double max_dcg(const int *labels, int64_t cnt, int k) {
    std::vector<int> sorted(labels, labels + cnt);
    std::sort(sorted.begin(), sorted.end(), [](int a, int b) { return a > b; });
    const int64_t m = k < cnt ? k : cnt;
    std::vector<double> disc = rank_discounts(m);
    double total = 0.0;
    for (int64_t j = 0; j < m; ++j) total += label_gain(sorted[j]) * disc[j];
    return total;
}

// _pair_sigmoid (ranking.mojo:500-507)
inline double pair_sigmoid(double delta, double sigma) {
    const double z = sigma * delta;
    if (z >= 0.0) {
        const double e = ref_exp(-z);
        return e / (1.0 + e);
    }
    const double e = ref_exp(z);
    return 1.0 / (1.0 + e);
}

// _fill_query_lambdas (ranking.mojo:510-570)
void query_lambdas(const double *scores, const int *labels, int64_t cnt, double inv_max_dcg,
                   const std::vector<double> &disc, const RankSpec &rs, double *grad, double *hess) {
    for (int64_t i = 0; i < cnt; ++i) grad[i] = hess[i] = 0.0;
    if (cnt < 2) return;
    std::vector<int64_t> order = argsort_desc(scores, cnt);
    const double best = scores[order[0]], worst = scores[order[cnt - 1]];
    double sum_lambdas = 0.0;
    int64_t top = cnt - 1;
    if (rs.truncation < top) top = rs.truncation;
    for (int64_t i = 0; i < top; ++i)
        for (int64_t j = i + 1; j < cnt; ++j) {
            if (labels[order[i]] == labels[order[j]]) continue;
            int64_t hr, lr;
            if (labels[order[i]] > labels[order[j]]) {
                hr = i;
                lr = j;
            } else {
                hr = j;
                lr = i;
            }
            const int64_t high = order[hr], low = order[lr];
            const double delta_score = scores[high] - scores[low];
            const double dcg_gap = label_gain(labels[high]) - label_gain(labels[low]);
            const double paired = std::fabs(disc[hr] - disc[lr]);
            double delta_ndcg = dcg_gap * paired * inv_max_dcg;
            if (rs.norm && best != worst) delta_ndcg /= 0.01 + std::fabs(delta_score);
            double p_lambda = pair_sigmoid(delta_score, rs.sigmoid);
            double p_hess = p_lambda * (1.0 - p_lambda);
            p_lambda *= -rs.sigmoid * delta_ndcg;
            p_hess *= rs.sigmoid * rs.sigmoid * delta_ndcg;
            grad[low] -= p_lambda;
            hess[low] += p_hess;
            grad[high] += p_lambda;
            hess[high] += p_hess;
            sum_lambdas -= 2.0 * p_lambda;
        }
    if (rs.norm && sum_lambdas > 0.0) {
        const double factor = ref_log2(1.0 + sum_lambdas) / sum_lambdas;
        for (int64_t i = 0; i < cnt; ++i) {
            grad[i] *= factor;
            hess[i] *= factor;
        }
    }
}

// lambdarank_gradients / _fill_lambdas (ranking.mojo:573-654), unweighted:
// every query's lambdas, in binary64 (the reference's ranker does not narrow).
void fill_lambdas(const double *raw, const std::vector<int> &labels, const RankSpec &rs,
                  const std::vector<double> &inv_max_dcg, const std::vector<double> &disc,
                  double *grad, double *hess) {
    const int64_t nq = (int64_t)rs.starts.size() - 1;
    for (int64_t q = 0; q < nq; ++q) {
        const int64_t a = rs.starts[q], c = rs.starts[q + 1] - a;
        query_lambdas(raw + a, labels.data() + a, c, inv_max_dcg[q], disc, rs, grad + a, hess + a);
    }
}

RankSpec rank_spec(const orc_params &p, int64_t n) {
    RankSpec rs;
    if (!p.query_starts || p.n_queries < 1) throw std::runtime_error("lambdarank needs query boundaries");
    rs.starts.assign(p.query_starts, p.query_starts + p.n_queries + 1);
    if (rs.starts[0] != 0 || rs.starts.back() != n) throw std::runtime_error("query boundaries must span the rows");
    for (int64_t q = 0; q < p.n_queries; ++q)
        if (rs.starts[q + 1] <= rs.starts[q]) throw std::runtime_error("query boundaries must increase");
    rs.truncation = p.lambdarank_truncation_level;
    rs.sigmoid = p.lambdarank_sigmoid;
    rs.norm = p.lambdarank_norm != 0;
    if (rs.truncation < 1 || !(rs.sigmoid > 0.0)) throw std::runtime_error("bad lambdarank parameters");
    return rs;
}

}  // namespace

// ================================================================ model
struct orc_model {
    int num_class = 1;
    int objective = 0;
    double learning_rate = 0.1;
    bool fused_predict = true;
    std::vector<double> base;
    std::vector<Tree> trees;
    std::vector<double> train_raw;
    std::vector<double> round_seconds;
};

namespace {

void fill_grad_hess(int objective, const double *raw, const double *labels,
                    int64_t n, int k, int kk, double *grad, double *hess, const double *weights = nullptr) {
    // boosting._fill_grad_hess_into (src/mojotrees/boosting.mojo:676-811)
    // and _fill_softmax_grad_hess_at (:3621-3678), narrowed; w = 1.0 when
    // unweighted (the reference multiplies by it either way).
    if (objective == ORC_OBJ_BINARY) {
        for (int64_t r = 0; r < n; ++r) {
            double p = sigmoid(raw[r]);
            const double w = weights ? weights[r] : 1.0;
            grad[r] = narrow(w * (p - labels[r]));
            double h = p * (1.0 - p);
            if (h < 1e-16) h = 1e-16;
            hess[r] = narrow(w * h);
        }
    } else if (objective == ORC_OBJ_MULTICLASS) {
        double factor = (double)k / (double)(k - 1);
        for (int64_t r = 0; r < n; ++r) {
            // raw holds probabilities here (softmax already applied).
            double p = raw[r * k + kk];
            double y = ((int)labels[r] == kk) ? 1.0 : 0.0;
            const double w = weights ? weights[r] : 1.0;
            grad[r] = narrow(w * (p - y));
            double h = factor * p * (1.0 - p);
            if (h < 1e-16) h = 1e-16;
            hess[r] = narrow(w * h);
        }
    } else {
        for (int64_t r = 0; r < n; ++r) {
            const double w = weights ? weights[r] : 1.0;
            grad[r] = narrow(w * (raw[r] - labels[r]));
            hess[r] = narrow(w * 1.0);
        }
    }
}

// boosting._softmax_rows (src/mojotrees/boosting.mojo:3529-3573)
void softmax_rows(const std::vector<double> &raw, std::vector<double> &prob,
                  int64_t n, int k) {
    prob.resize(raw.size());
    for (int64_t r = 0; r < n; ++r) {
        const double *s = raw.data() + r * k;
        double *p = prob.data() + r * k;
        for (int i = 0; i < k; ++i) p[i] = s[i];
        double m = p[0];
        for (int i = 1; i < k; ++i)
            if (p[i] > m) m = p[i];
        double total = 0.0;
        for (int i = 0; i < k; ++i) {
            double e = ref_exp(p[i] - m);
            p[i] = e;
            total += e;
        }
        for (int i = 0; i < k; ++i) p[i] = p[i] / total;
    }
}

double goss_select_multiclass(const std::vector<double> &prob, const double *labels, int64_t n, int K,
                              const double *weights, const orc_params &p, int64_t round,
                              std::vector<int32_t> &bag, std::vector<uint8_t> &other) {
    std::vector<double> imp((size_t)n, 0.0), g((size_t)n), h((size_t)n);
    for (int k = 0; k < K; ++k) {
        fill_grad_hess(ORC_OBJ_MULTICLASS, prob.data(), labels, n, K, k, g.data(), h.data(), weights);
        for (int64_t r = 0; r < n; ++r) imp[r] += std::fabs(g[r] * h[r]);
    }
    return goss_select(imp, p, round, bag, other);
}

// One tree of a round: quantized or float, returns the tree and leaf rows.
Tree grow_one(const Data &d, const Params &P, std::vector<double> &grad,
              std::vector<double> &hess, const std::vector<int32_t> &bag,
              int64_t round, int64_t class_index, int64_t tree_index,
              std::vector<std::pair<int, std::vector<int32_t>>> &leaves,
              std::vector<int32_t> &qg, std::vector<int32_t> &qh, Pool &pool) {
    const std::vector<int32_t> *bagp = bag.empty() ? nullptr : &bag;
    std::vector<int> tf = select_tree_features(d.nf, P.p.feature_fraction,
                                               P.p.feature_fraction_seed, tree_index);
    if (P.p.use_quantized_grad) {
        qg.resize(d.n);
        qh.resize(d.n);
        QScales s = quantize_round(grad, hess, bag.empty() ? nullptr : bag.data(),
                                   (int64_t)bag.size(), P.p.num_grad_quant_bins,
                                   P.p.stochastic_rounding != 0, P.p.quant_seed, round,
                                   class_index, P.const_hessian, P.p.quant_scale_rule, qg.data(),
                                   qh.data(), pool);
        QuantPolicy pol{d, qg.data(), qh.data(), s, P, pool, tf[0]};
        return grow_tree(pol, d, P, bagp, tree_index, &leaves);
    }
    FloatPolicy pol{d, grad, hess, P, pool, tf[0]};
    return grow_tree(pol, d, P, bagp, tree_index, &leaves);
}

void add_tree_scores(std::vector<double> &raw, const Tree &t, const Data &d,
                     const std::vector<std::pair<int, std::vector<int32_t>>> &leaves,
                     bool by_leaf, double lr, int stride, int offset, bool fused) {
    // boosting._add_by_leaf (fma) / _add_by_traversal
    // (src/mojotrees/boosting.mojo:1947-2151).
    if (by_leaf) {
        for (auto &lf : leaves) {
            double v = t.value[lf.first];
            for (int32_t r : lf.second) {
                double &slot = raw[(int64_t)r * stride + offset];
                slot = fused ? std::fma(lr, v, slot) : slot + lr * v;
            }
        }
        return;
    }
    for (int64_t r = 0; r < d.n; ++r) {
        double &slot = raw[r * stride + offset];
        double v = t.predict(d, r);
        slot = fused ? std::fma(lr, v, slot) : slot + lr * v;
    }
}

}  // namespace

extern "C" {

uint64_t orc_splitmix64(uint64_t state) { return splitmix64(state); }
double orc_uniform(uint64_t counter) { return uniform(counter); }
double orc_exp(double x) { return ref_exp(x); }
double orc_log(double x) { return ref_log(x); }
double orc_sigmoid(double x) { return sigmoid(x); }
uint64_t orc_quant_stream(int64_t seed, int64_t round_index, int64_t class_index,
                          int64_t plane) {
    return quant_stream(seed, round_index, class_index, plane);
}

// binning.bin_equal_width (src/mojotrees/binning.mojo:4109-4166)
int32_t orc_bin_equal_width(const double *x, int64_t n, int32_t nf, int32_t nb,
                            uint8_t *out) {
    if (nb < 2 || nb > 256 || n < 1) return -1;
    for (int f = 0; f < nf; ++f) {
        const double *col = x + (int64_t)f * n;
        double lo = col[0], hi = lo;
        for (int64_t r = 1; r < n; ++r) {
            double v = col[r];
            if (v < lo) lo = v;
            if (v > hi) hi = v;
        }
        double width = (hi - lo) / (double)nb;
        for (int64_t r = 0; r < n; ++r) {
            double v = col[r];
            int64_t b;
            if (width <= 0.0 || v != v) {
                b = 0;
            } else {
                b = (int64_t)((v - lo) / width);
                if (b >= nb) b = nb - 1;
                if (b < 0) b = 0;
            }
            out[(int64_t)f * n + r] = (uint8_t)b;
        }
    }
    return 0;
}

}  // extern "C"

namespace {
// bin_construct_sample_rows (src/mojotrees/binning.mojo:1745-1785): Knuth's
// selection sampling, row r of the `left` still to consider taken when
// uniform(seed * GOLDEN + r) * left < need, every remaining row once need >=
// left; empty (every row) for sample_cnt <= 0 or >= n.
std::vector<int64_t> bin_sample_rows(int64_t n, int64_t sample_cnt, int64_t seed) {
    std::vector<int64_t> sample;
    if (n < 1 || sample_cnt <= 0 || sample_cnt >= n) return sample;
    sample.reserve((size_t)sample_cnt);
    const uint64_t base = (uint64_t)seed * GOLDEN;
    int64_t need = sample_cnt;
    for (int64_t r = 0; r < n && need > 0; ++r) {
        const int64_t left = n - r;
        if (need >= left) {
            sample.push_back(r);
            --need;
            continue;
        }
        if (uniform(base + (uint64_t)r) * (double)left < (double)need) {
            sample.push_back(r);
            --need;
        }
    }
    return sample;
}
}  // namespace

extern "C" {

int64_t orc_bin_sample_rows(int64_t n, int64_t sample_cnt, int64_t seed, int64_t *out) {
    const std::vector<int64_t> s = bin_sample_rows(n, sample_cnt, seed);
    if (out) std::memcpy(out, s.data(), s.size() * sizeof(int64_t));
    return (int64_t)s.size();
}

// binning.fit_bins, quantile border type, numerical features
// (src/mojotrees/binning.mojo:3565-4047; quantile_boundary_indices :558,
// emit_quantile_edges :583, bin_construct_sample_rows :1745). The
// selection-based branch (resolve_ranks) returns the same order statistics
// as the sort-based branch restated here.
int32_t orc_fit_bins(const double *x, int64_t n, int32_t nf, int32_t max_bins,
                     int32_t min_data_in_bin, int32_t use_missing, int64_t sample_cnt,
                     int64_t seed, double *out_edges, int32_t *out_n_edges,
                     int32_t *out_missing_bin) {
    if (max_bins < 2 || max_bins > 256 || n < 1 || min_data_in_bin < 1) return -1;
    const std::vector<int64_t> sample = bin_sample_rows(n, sample_cnt, seed);
    bool sampled = !sample.empty();
    int64_t n_sample = sampled ? (int64_t)sample.size() : n;
    int max_edges = max_bins - 1;
    for (int f = 0; f < nf; ++f) {
        const double *colp = x + (int64_t)f * n;
        std::vector<double> col;
        col.reserve(n_sample);
        for (int64_t i = 0; i < n_sample; ++i) {
            double v = colp[sampled ? sample[i] : i];
            if (v == v) col.push_back(v);
        }
        int64_t n_valid = (int64_t)col.size();
        bool reserve = use_missing && n_valid < n_sample;
        int n_ordinary = reserve ? max_bins - 1 : max_bins;
        std::sort(col.begin(), col.end());
        std::vector<double> below, above, edges;
        // distinct levels (collect_distinct, binning.mojo:1531)
        std::vector<double> dv;
        std::vector<int64_t> dc;
        bool distinct_ok = true;
        for (int64_t i = 0; i < n_valid;) {
            int64_t j = i;
            while (j < n_valid && col[j] == col[i]) ++j;
            dv.push_back(col[i]);
            dc.push_back(j - i);
            if ((int64_t)dv.size() > n_ordinary) {
                distinct_ok = false;
                break;
            }
            i = j;
        }
        if (distinct_ok) {
            if (min_data_in_bin <= 1) {
                for (size_t j = 0; j + 1 < dv.size(); ++j) {
                    below.push_back(dv[j]);
                    above.push_back(dv[j + 1]);
                }
            } else {
                int64_t acc = 0;
                for (size_t j = 0; j + 1 < dv.size(); ++j) {
                    acc += dc[j];
                    if (acc >= min_data_in_bin) {
                        below.push_back(dv[j]);
                        above.push_back(dv[j + 1]);
                        acc = 0;
                    }
                }
            }
        } else {
            int64_t n_ord = n_ordinary;
            if (min_data_in_bin > 1) {
                int64_t cap = n_valid / min_data_in_bin;
                if (cap < 1) cap = 1;
                if (cap < n_ord) n_ord = cap;
            }
            for (int64_t b = 1; b < n_ord; ++b) {
                int64_t idx = b * n_valid / n_ord;
                if (idx <= 0 || idx >= n_valid) continue;
                double w = col[idx - 1];
                below.push_back(w);
                int64_t e = std::upper_bound(col.begin() + idx, col.end(), w) - col.begin();
                above.push_back(e < n_valid ? col[e] : w);
            }
        }
        for (size_t j = 0; j < below.size() && j < above.size(); ++j) {
            double lo = below[j], hi = above[j];
            if (hi <= lo) continue;
            double edge = (lo + hi) / 2.0;
            if (edge != edge) edge = 0.0;
            else if (edge >= 1e300) edge = 1e300;
            else if (edge <= -1e300) edge = -1e300;
            if (!edges.empty() && edge <= edges.back()) continue;
            edges.push_back(edge);
        }
        if ((int)edges.size() > max_edges) return -2;
        for (size_t i = 0; i < edges.size(); ++i) out_edges[(int64_t)f * max_bins + i] = edges[i];
        out_n_edges[f] = (int32_t)edges.size();
        out_missing_bin[f] = reserve ? (int32_t)edges.size() + 1 : -1;
    }
    return 0;
}

// BinMapper.bin_value (src/mojotrees/binning.mojo:3242-3262)
int32_t orc_transform(const double *x, int64_t n, int32_t nf, int32_t max_bins,
                      const double *edges, const int32_t *n_edges,
                      const int32_t *missing_bin, uint8_t *out) {
    for (int f = 0; f < nf; ++f) {
        const double *e = edges + (int64_t)f * max_bins;
        int k = n_edges[f];
        for (int64_t r = 0; r < n; ++r) {
            double v = x[(int64_t)f * n + r];
            int b;
            if (v != v) {
                if (missing_bin[f] >= 0) {
                    out[(int64_t)f * n + r] = (uint8_t)missing_bin[f];
                    continue;
                }
                v = 0.0;
            }
            int lo = 0, hi = k;
            while (lo < hi) {
                int mid = (lo + hi) / 2;
                if (v <= e[mid]) hi = mid;
                else lo = mid + 1;
            }
            b = lo;
            out[(int64_t)f * n + r] = (uint8_t)b;
        }
    }
    return 0;
}

int32_t orc_grad_hess(int32_t objective, const double *raw, const double *labels,
                      int64_t n, int32_t num_class, int32_t class_k, double *grad,
                      double *hess) {
    fill_grad_hess(objective, raw, labels, n, num_class, class_k, grad, hess);
    return 0;
}
int32_t orc_grad_hess_w(int32_t objective, const double *raw, const double *labels, const double *weights,
                        int64_t n, int32_t num_class, int32_t class_k, double *grad, double *hess) {
    fill_grad_hess(objective, raw, labels, n, num_class, class_k, grad, hess, weights);
    return 0;
}

int32_t orc_quantize_rule(const double *grad, const double *hess, int64_t n,
                          const int32_t *rows, int64_t n_sel, int32_t quant_bins,
                          int32_t stochastic, int64_t seed, int64_t round_index,
                          int64_t class_index, int32_t const_hessian, int32_t rule,
                          int32_t *q_grad, int32_t *q_hess, double *out_scales) {
    std::vector<double> g(grad, grad + n), h(hess, hess + n);
    Pool pool(1);
    try {
        QScales s = quantize_round(g, h, rows, n_sel, quant_bins, stochastic != 0, seed,
                                   round_index, class_index, const_hessian != 0, rule, q_grad,
                                   q_hess, pool);
        out_scales[0] = s.gu;
        out_scales[1] = s.hu;
        out_scales[2] = (double)s.gmax;
        out_scales[3] = (double)s.hmax;
    } catch (const std::exception &) {
        return -1;
    }
    return 0;
}

int32_t orc_quantize(const double *grad, const double *hess, int64_t n,
                     const int32_t *rows, int64_t n_sel, int32_t quant_bins,
                     int32_t stochastic, int64_t seed, int64_t round_index,
                     int64_t class_index, int32_t const_hessian, int8_t *q_grad,
                     int8_t *q_hess, double *out_scales) {
    std::vector<int32_t> qg((size_t)n), qh((size_t)n);
    const int32_t rc = orc_quantize_rule(grad, hess, n, rows, n_sel, quant_bins, stochastic, seed,
                                         round_index, class_index, const_hessian, kRuleMaxAbs,
                                         qg.data(), qh.data(), out_scales);
    for (int64_t r = 0; r < n; ++r) {
        q_grad[r] = (int8_t)qg[(size_t)r];
        q_hess[r] = (int8_t)qh[(size_t)r];
    }
    return rc;
}

int32_t orc_magnitude_sums(const double *grad, const double *hess, int64_t n,
                           const uint8_t *in_sample, double *out_sums) {
    std::vector<double> g(grad, grad + n), h(hess, hess + n);
    std::vector<uint8_t> m;
    if (in_sample) m.assign(in_sample, in_sample + n);
    magnitude_sums(g, h, m, out_sums[0], out_sums[1]);
    return 0;
}

double orc_largest_power_of_two_at_most(double x) {
    try {
        return largest_power_of_two_at_most(x);
    } catch (const std::exception &) {
        return -1.0;
    }
}

double orc_fixed_point_scale_pow2(double total) {
    try {
        return fixed_point_scale_pow2(total);
    } catch (const std::exception &) {
        return -1.0;
    }
}

int32_t orc_hist_quantized32(const uint8_t *bins, int64_t n, int32_t nf, int32_t nb,
                             const int32_t *qg, const int32_t *qh, const int32_t *rows,
                             int64_t n_sel, int64_t *out) {
    Data d{bins, n, nf, nb, std::vector<int>(nf, -1), {}, {}};
    std::vector<int> feats(nf);
    for (int f = 0; f < nf; ++f) feats[f] = f;
    QHist h;
    Pool pool(1);
    build_quant(h, d, qg, qh, rows, rows ? n_sel : n, feats, pool);
    std::memcpy(out, h.v.data(), h.v.size() * sizeof(int64_t));
    return 0;
}

int32_t orc_hist_quantized(const uint8_t *bins, int64_t n, int32_t nf, int32_t nb,
                           const int8_t *qg, const int8_t *qh, const int32_t *rows,
                           int64_t n_sel, int64_t *out) {
    std::vector<int32_t> g(qg, qg + n), h(qh, qh + n);
    return orc_hist_quantized32(bins, n, nf, nb, g.data(), h.data(), rows, n_sel, out);
}

int32_t orc_hist_float(const uint8_t *bins, int64_t n, int32_t nf, int32_t nb,
                       const double *grad, const double *hess, const int32_t *rows,
                       int64_t n_sel, int32_t row_blocks, double *out_gh,
                       int64_t *out_count) {
    Data d{bins, n, nf, nb, std::vector<int>(nf, -1), {}, {}};
    std::vector<int> feats(nf);
    for (int f = 0; f < nf; ++f) feats[f] = f;
    std::vector<double> g(grad, grad + n), h(hess, hess + n);
    FHist hist;
    Pool pool(1);
    build_float(hist, d, g, h, rows, rows ? n_sel : n, feats, pool, row_blocks);
    std::memcpy(out_gh, hist.gh.data(), hist.gh.size() * sizeof(double));
    std::memcpy(out_count, hist.c.data(), hist.c.size() * sizeof(int64_t));
    return 0;
}

int32_t orc_lambdarank(const double *scores, const double *labels, const int64_t *starts,
                       int64_t n_queries, int32_t truncation, double sigma, int32_t norm,
                       double *grad, double *hess) {
    try {
        orc_params p{};
        p.query_starts = starts;
        p.n_queries = n_queries;
        p.lambdarank_truncation_level = truncation;
        p.lambdarank_sigmoid = sigma;
        p.lambdarank_norm = norm;
        const int64_t n = starts[n_queries];
        RankSpec rs = rank_spec(p, n);
        std::vector<int> lab(n);
        for (int64_t r = 0; r < n; ++r) {
            if (!(labels[r] >= 0.0 && labels[r] <= 30.0)) return -1;
            lab[r] = (int)labels[r];
        }
        std::vector<double> inv;
        int64_t max_size = 0;
        for (int64_t q = 0; q < n_queries; ++q) {
            const int64_t a = starts[q], c = starts[q + 1] - a;
            max_size = std::max(max_size, c);
            const double md = max_dcg(lab.data() + a, c, truncation);
            inv.push_back(md > 0.0 ? 1.0 / md : 0.0);
        }
        fill_lambdas(scores, lab, rs, inv, rank_discounts(max_size), grad, hess);
        return 0;
    } catch (const std::exception &) {
        return -1;
    }
}

double orc_log2(double x) { return ref_log2(x); }

// One GOSS selection (goss_importance + goss_select + apply_goss_scaling,
// goss.mojo:294-373) on caller arrays, warmup not applied. rows_out and
// scale_out need n entries; grad/hess are scaled in place like the trainer's.
int32_t orc_goss_select(double *grad, double *hess, int64_t n, double top_rate,
                        double other_rate, int32_t seed, int64_t round_index,
                        int32_t *rows_out, double *scale_out, int64_t *n_out) {
    if (n <= 0 || !grad || !hess || !rows_out || !scale_out || !n_out) return -1;
    orc_params p{};
    p.goss = 1;
    p.learning_rate = 0.0;  // no warmup
    p.top_rate = top_rate;
    p.other_rate = other_rate;
    p.goss_seed = seed;
    std::vector<double> g(grad, grad + n), h(hess, hess + n), sc;
    std::vector<int32_t> bag;
    goss_round(bag, g, h, p, round_index, &sc);
    for (size_t i = 0; i < bag.size(); ++i) {
        rows_out[i] = bag[i];
        scale_out[i] = sc[i];
    }
    std::memcpy(grad, g.data(), n * sizeof(double));
    std::memcpy(hess, h.data(), n * sizeof(double));
    *n_out = (int64_t)bag.size();
    return 0;
}

// One multiclass round's GOSS sample (_multiclass_goss_select,
// boosting.mojo:3680-3710) from the round's class probabilities (row-major,
// prob[r * K + k]), warmup not applied: rows_out (n entries) receives the
// sample ascending, other_out[r] (n entries) 1 for a sampled small-importance
// row, *mult_out their weight.
int32_t orc_goss_select_multiclass(const double *prob, const double *labels, int64_t n, int32_t K,
                                   const double *weights, double top_rate, double other_rate,
                                   int32_t seed, int64_t round_index, int32_t *rows_out,
                                   uint8_t *other_out, double *mult_out, int64_t *n_out) {
    if (n <= 0 || K < 2 || !prob || !labels || !rows_out || !other_out || !mult_out || !n_out) return -1;
    orc_params p{};
    p.goss = 1;
    p.learning_rate = 0.0;
    p.top_rate = top_rate;
    p.other_rate = other_rate;
    p.goss_seed = seed;
    std::vector<double> pr(prob, prob + n * K);
    std::vector<int32_t> bag;
    std::vector<uint8_t> other;
    *mult_out = goss_select_multiclass(pr, labels, n, K, weights, p, round_index, bag, other);
    for (size_t i = 0; i < bag.size(); ++i) rows_out[i] = bag[i];
    std::memcpy(other_out, other.data(), (size_t)n);
    *n_out = (int64_t)bag.size();
    return 0;
}

int32_t orc_split_quantized(const int64_t *hist, int32_t nf, int32_t nb,
                            const int32_t *missing_bin, const int32_t *widths,
                            double gu, double hu, double l1, double l2,
                            double min_sum_hessian, int32_t min_data_in_leaf,
                            int32_t *of, int32_t *ob, int32_t *odl, double *og) {
    Data d{nullptr, 0, nf, nb, std::vector<int>(missing_bin, missing_bin + nf),
           widths ? std::vector<int>(widths, widths + nf) : std::vector<int>(), {}};
    QHist h;
    h.v.assign(hist, hist + 3 * (int64_t)nf * nb);
    QScales s;
    s.gu = gu;
    s.hu = hu;
    Params P;
    std::memset(&P.p, 0, sizeof(P.p));
    P.p.lambda_l1 = l1;
    P.p.lambda_l2 = l2;
    P.p.min_sum_hessian = min_sum_hessian;
    P.p.min_data_in_leaf = min_data_in_leaf;
    std::vector<int> scan(nf);
    for (int f = 0; f < nf; ++f) scan[f] = f;
    Split b = find_best_split_quant(h, d, scan, s, P);
    *of = b.feature;
    *ob = b.bin;
    *odl = b.default_left ? 1 : 0;
    *og = b.gain;
    return b.found ? 1 : 0;
}

orc_model *orc_train(const uint8_t *bins, int64_t n, int32_t nf, int32_t nb,
                     const int32_t *missing_bin, const double *labels,
                     const orc_params *params, char *err, int32_t err_len) {
    try {
        Params P;
        P.p = *params;
        Data d{bins, n, nf, nb,
               missing_bin ? std::vector<int>(missing_bin, missing_bin + nf)
                           : std::vector<int>(nf, -1),
               {}, {}};
        if (P.p.n_categories) {
            d.ncat.assign(P.p.n_categories, P.p.n_categories + nf);
            for (int f = 0; f < nf; ++f)
                if (d.ncat[f] >= nb) throw std::runtime_error("categorical feature has more categories than bins");
        }
        d.widths = histogram_widths(d);
        int threads = P.p.n_threads > 0 ? P.p.n_threads
                                        : (int)std::max(1u, std::thread::hardware_concurrency());
        Pool pool(threads);
        auto *m = new orc_model();
        m->objective = P.p.objective;
        m->learning_rate = P.p.learning_rate;
        m->fused_predict = P.p.fused_predict != 0;
        int K = P.p.objective == ORC_OBJ_MULTICLASS ? P.p.num_class : 1;
        m->num_class = K;
        m->round_seconds.assign(P.p.num_iterations, 0.0);
        // boosting.round_has_constant_hessian: L2, unweighted, no GOSS.
        P.const_hessian = (P.p.objective == ORC_OBJ_L2) && !P.p.goss && !P.p.weights;
        std::vector<double> raw((size_t)n * K);
        const bool rank = P.p.objective == ORC_OBJ_LAMBDARANK;
        RankSpec rs;
        std::vector<int> rank_labels;
        std::vector<double> inv_max_dcg, rank_disc;
        if (rank) {
            // train_ranker (ranking.mojo:713-771): base score 0, labels in [0, 30]
            rs = rank_spec(P.p, n);
            rank_labels.resize(n);
            for (int64_t r = 0; r < n; ++r) {
                if (!(labels[r] >= 0.0 && labels[r] <= 30.0) || labels[r] != std::floor(labels[r]))
                    throw std::runtime_error("relevance labels must be integers in [0, 30]");
                rank_labels[r] = (int)labels[r];
            }
            int64_t max_size = 0;
            for (int64_t q = 0; q + 1 < (int64_t)rs.starts.size(); ++q) {
                const int64_t a = rs.starts[q], c = rs.starts[q + 1] - a;
                max_size = std::max(max_size, c);
                const double md = max_dcg(rank_labels.data() + a, c, rs.truncation);
                inv_max_dcg.push_back(md > 0.0 ? 1.0 / md : 0.0);
            }
            rank_disc = rank_discounts(max_size);
        }
        if (K == 1 && rank) {
            m->base.push_back(0.0);
            std::fill(raw.begin(), raw.end(), 0.0);
        } else if (K == 1) {
            // boosting._base_score (src/mojotrees/boosting.mojo:521-568)
            double mean = 0.0, tw = 0.0;
            for (int64_t r = 0; r < n; ++r) {
                const double w = P.p.weights ? P.p.weights[r] : 1.0;
                mean += w * labels[r];
                tw += w;
            }
            mean /= tw;
            double base = mean;
            if (P.p.objective == ORC_OBJ_BINARY) {
                double p = clamp_prob(mean);
                base = ref_log(p / (1.0 - p));
            }
            if (P.p.use_init_base) base = P.p.init_base;
            m->base.push_back(base);
            std::fill(raw.begin(), raw.end(), base);
        } else {
            // boosting.train_multiclass (src/mojotrees/boosting.mojo:4167-4250)
            std::vector<double> cw(K, 0.0);
            double tw = 0.0;
            for (int64_t r = 0; r < n; ++r) {
                const double w = P.p.weights ? P.p.weights[r] : 1.0;
                cw[(int)labels[r]] += w;
                tw += w;
            }
            for (int k = 0; k < K; ++k) m->base.push_back(ref_log(clamp_prob(cw[k] / tw)));
            for (int64_t r = 0; r < n; ++r)
                for (int k = 0; k < K; ++k) raw[r * K + k] = m->base[k];
        }
        std::vector<double> grad(n), hess(n), prob;
        std::vector<int32_t> bag;
        std::vector<int32_t> qg, qh;
        std::vector<std::pair<int, std::vector<int32_t>>> leaves;
        bool bagging = P.p.bagging_freq > 0 && P.p.bagging_fraction < 1.0;
        for (int it = 0; it < P.p.num_iterations; ++it) {
            auto t0 = std::chrono::steady_clock::now();
            if (rank)
                refresh_query_bag(bag, P.p, rs.starts, it);
            else
                refresh_bag(bag, P.p, n, it);
            if (K == 1) {
                if (rank) {
                    fill_lambdas(raw.data(), rank_labels, rs, inv_max_dcg, rank_disc, grad.data(), hess.data());
                    // lambdarank_gradients (ranking.mojo:613-616): weights
                    // scale the finished lambdas and hessians
                    if (P.p.weights)
                        for (int64_t r = 0; r < n; ++r) {
                            grad[r] *= P.p.weights[r];
                            hess[r] *= P.p.weights[r];
                        }
                } else
                    fill_grad_hess(P.p.objective, raw.data(), labels, n, 1, 0, grad.data(), hess.data(), P.p.weights);
                goss_round(bag, grad, hess, P.p, it);
                Tree t = grow_one(d, P, grad, hess, bag, it, 0, it, leaves, qg, qh, pool);
                if (t.n_leaves == 1 && std::fabs(t.value[0]) < 1e-12) {
                    if (bagging || P.p.goss) continue;
                    break;
                }
                bool by_leaf = bag.empty();
                add_tree_scores(raw, t, d, leaves, by_leaf, P.p.learning_rate, 1, 0,
                                P.p.fused_score_update != 0);
                m->trees.push_back(std::move(t));
            } else {
                // boosting._boost_rounds_multiclass (boosting.mojo:3876-4165)
                softmax_rows(raw, prob, n, K);
                // one GOSS sample for the whole round, drawn before any class's
                // tree (:4041-4053); each class's derivatives scaled by it
                std::vector<uint8_t> gother;
                double gmult = 1.0;
                const bool gactive = goss_active(P.p, it);
                if (gactive) gmult = goss_select_multiclass(prob, labels, n, K, P.p.weights, P.p, it, bag, gother);
                bool progress = false;
                std::vector<Tree> round_trees;
                for (int k = 0; k < K; ++k) {
                    fill_grad_hess(ORC_OBJ_MULTICLASS, prob.data(), labels, n, K, k,
                                   grad.data(), hess.data(), P.p.weights);
                    if (gactive) goss_scale(gother, gmult, grad, hess, bag);
                    Tree t = grow_one(d, P, grad, hess, bag, it, k, (int64_t)it * K + k,
                                      leaves, qg, qh, pool);
                    if (t.n_leaves > 1 || std::fabs(t.value[0]) >= 1e-12) progress = true;
                    add_tree_scores(raw, t, d, leaves, bag.empty(), P.p.learning_rate, K, k,
                                    P.p.fused_score_update != 0);
                    round_trees.push_back(std::move(t));
                }
                if (!progress) {
                    if (bagging || P.p.goss) continue;
                    break;
                }
                for (auto &t : round_trees) m->trees.push_back(std::move(t));
            }
            m->round_seconds[it] = std::chrono::duration<double>(
                                       std::chrono::steady_clock::now() - t0)
                                       .count();
        }
        m->train_raw = raw;
        return m;
    } catch (const std::exception &e) {
        if (err && err_len > 0) std::snprintf(err, err_len, "%s", e.what());
        return nullptr;
    }
}

void orc_model_free(orc_model *m) { delete m; }
int32_t orc_model_num_trees(const orc_model *m) { return (int32_t)m->trees.size(); }
int32_t orc_model_num_class(const orc_model *m) { return m->num_class; }
int64_t orc_model_total_nodes(const orc_model *m) {
    int64_t t = 0;
    for (auto &tr : m->trees) t += (int64_t)tr.feature.size();
    return t;
}
void orc_model_arrays(const orc_model *m, double *base, int64_t *off, int32_t *feature,
                      int32_t *thr, int32_t *left, int32_t *right, double *value,
                      int32_t *dl, int32_t *mb, double *gain, double *count) {
    for (int k = 0; k < m->num_class; ++k) base[k] = m->base[k];
    int64_t o = 0;
    for (size_t t = 0; t < m->trees.size(); ++t) {
        off[t] = o;
        const Tree &tr = m->trees[t];
        for (size_t i = 0; i < tr.feature.size(); ++i, ++o) {
            feature[o] = tr.feature[i];
            thr[o] = tr.threshold[i];
            left[o] = tr.left[i];
            right[o] = tr.right[i];
            value[o] = tr.value[i];
            dl[o] = tr.default_left[i];
            mb[o] = tr.missing_bin[i];
            gain[o] = tr.gain[i];
            count[o] = tr.count[i];
        }
    }
    off[m->trees.size()] = o;
}
void orc_model_cat_bits(const orc_model *m, uint64_t *out) {
    size_t o = 0;
    for (const Tree &tr : m->trees) {
        std::memcpy(out + o, tr.cat.data(), tr.cat.size() * sizeof(uint64_t));
        o += tr.cat.size();
    }
}
int32_t orc_cat_split(const double *gh, const int64_t *count, int32_t n_categories, double total_g,
                      double total_h, int64_t total_c, double lambda_l2, double lambda_l1,
                      double min_child_hess, int32_t min_data_in_leaf, int32_t max_cat_to_onehot,
                      int32_t max_cat_threshold, double cat_smooth, double cat_l2,
                      int32_t min_data_per_group, int32_t one_hot_max_size, double *out_gain,
                      uint64_t *out_bits) {
    FloatCatOps ops{gh, count, lambda_l1, min_child_hess};
    CatCfg c{max_cat_to_onehot, max_cat_threshold, min_data_per_group, one_hot_max_size, cat_smooth, cat_l2};
    CatResult r = cat_search(ops, n_categories, FloatCatOps::S{total_g, total_h, total_c}, lambda_l2,
                             min_data_in_leaf, c);
    *out_gain = r.gain;
    std::memcpy(out_bits, r.bits, sizeof r.bits);
    return r.found ? 1 : 0;
}
void orc_model_train_raw(const orc_model *m, double *out) {
    std::memcpy(out, m->train_raw.data(), m->train_raw.size() * sizeof(double));
}
void orc_model_round_seconds(const orc_model *m, double *out) {
    std::memcpy(out, m->round_seconds.data(), m->round_seconds.size() * sizeof(double));
}

// Booster.predict_raw_row / response (src/mojotrees/boosting.mojo:1722-1760)
// and MulticlassBooster softmax.
int32_t orc_predict_binned(const orc_model *m, const uint8_t *bins, int64_t n,
                           int32_t nf, double *raw, double *resp) {
    Data d{bins, n, nf, 256, std::vector<int>(nf, -1), {}, {}};
    int K = m->num_class;
    double lr = m->learning_rate;
    for (int64_t r = 0; r < n; ++r) {
        for (int k = 0; k < K; ++k) raw[r * K + k] = m->base[k];
        for (size_t t = 0; t < m->trees.size(); ++t) {
            int k = (int)(t % K);
            double v = m->trees[t].predict(d, r);
            double &s = raw[r * K + k];
            s = m->fused_predict ? std::fma(lr, v, s) : s + lr * v;
        }
        if (K == 1) {
            resp[r] = m->objective == ORC_OBJ_BINARY ? sigmoid(raw[r]) : raw[r];
        } else {
            double mx = raw[r * K];
            for (int k = 1; k < K; ++k) mx = std::max(mx, raw[r * K + k]);
            double tot = 0.0;
            for (int k = 0; k < K; ++k) {
                resp[r * K + k] = ref_exp(raw[r * K + k] - mx);
                tot += resp[r * K + k];
            }
            for (int k = 0; k < K; ++k) resp[r * K + k] /= tot;
        }
    }
    return 0;
}

}  // extern "C"
