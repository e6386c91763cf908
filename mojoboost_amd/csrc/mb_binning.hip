// mbh_bin_dense_device: the binning of mbh_bin_dense with the per-value
// transform on the GPU. The quantile fit (binning.fit_bins,
// src/mojotrees/binning.mojo:3565-4047, and categorical.fit_categorical_spec,
// src/mojotrees/categorical.mojo:419-464) stays on the host, where it reads
// a sample of at most bin_construct_sample_cnt rows; the transform
// (BinMapper.transform, binning.mojo:3264-3330, bin_value :3242-3262) reads
// every value once and is an HBM-bound byte map: 8 bytes in and 1 byte out
// per value.
//
// Device layout: the column-major doubles as the caller passes them
// (x[f * n + r]), the column-major uint8 bins out, and one table of
// kTable doubles per feature in LDS: a numerical feature's k ascending
// edges padded with +inf up to P, the smallest power of two above k (a
// sentinel never counts: +inf < v is false for every v). A value's bin is
// the number of edges strictly below it -- the first edge with v <= edge,
// which is bin_value's search -- found by a branch-free descent of log2 P
// steps. NaN takes the reserved missing bin, or the bin of 0.0 when none is
// reserved (the LightGBM rule bin_value follows). A categorical feature's
// table holds its kept codes ascending (int64), the i-th in bin i + 1; NaN,
// negative, >= 2^31, unseen and dropped codes take bin 0, a fraction
// truncates (CategoricalSpec.bin_of, categorical.mojo:296-322).
#include <hip/hip_runtime.h>

#include <chrono>
#include <cmath>
#include <cstdio>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/mojoboost_hip.h"
#include "../../include/mojotrees.h"
#include "mb_host.h"

namespace {

constexpr int kTable = 256;       // table entries per feature (uint8 bins: at most 255 edges or codes)
constexpr int kThreads = 256;
constexpr int kRowsPerThread = 8;  // rows a thread maps per block pass

struct FeatureTable {
    int32_t is_cat;    // 1: categorical codes, 0: numerical edges
    int32_t half;      // numerical: P / 2 (the descent's first step); categorical: code count
    int32_t nan_bin;   // numerical: the bin a NaN takes
    int32_t pad_;
};

// grid (row blocks, features); every row of the block pass is in range or
// masked, every table read is below kTable.
__global__ __launch_bounds__(kThreads) void k_bin_transform(const double *__restrict__ x, int64_t n,
                                                            const FeatureTable *__restrict__ ft,
                                                            const double *__restrict__ edges,
                                                            const long long *__restrict__ codes,
                                                            uint8_t *__restrict__ out) {
    __shared__ double t_edge[kTable];
    __shared__ long long t_code[kTable];
    const int f = blockIdx.y;
    const FeatureTable tb = ft[f];
    const int tid = threadIdx.x;
    if (tb.is_cat) t_code[tid] = codes[(size_t)f * kTable + tid];
    else t_edge[tid] = edges[(size_t)f * kTable + tid];
    __syncthreads();
    const double *col = x + (size_t)f * n;
    uint8_t *oc = out + (size_t)f * n;
    const int64_t base = (int64_t)blockIdx.x * (kThreads * kRowsPerThread) + tid;
    double v[kRowsPerThread];
#pragma unroll
    for (int u = 0; u < kRowsPerThread; ++u) {
        const int64_t r = base + (int64_t)u * kThreads;
        v[u] = r < n ? col[r] : 0.0;
    }
    if (tb.is_cat) {
#pragma unroll
        for (int u = 0; u < kRowsPerThread; ++u) {
            const int64_t r = base + (int64_t)u * kThreads;
            const double c = v[u];
            int b = 0;
            if (c >= 0.0 && c < 2147483648.0) {
                const long long code = (long long)c;  // truncation toward zero
                int lo = 0, hi = tb.half;             // lower_bound over the kept codes
                while (lo < hi) {
                    const int mid = (lo + hi) >> 1;
                    if (t_code[mid] < code) lo = mid + 1;
                    else hi = mid;
                }
                b = (lo < tb.half && t_code[lo] == code) ? lo + 1 : 0;
            }
            if (r < n) oc[r] = (uint8_t)b;
        }
        return;
    }
    // count of edges strictly below v, the rows' descents interleaved so
    // that their LDS reads of one step are in flight together; on NaN every
    // compare is false and the descent ends at 0, replaced by the NaN bin
    int pos[kRowsPerThread];
#pragma unroll
    for (int u = 0; u < kRowsPerThread; ++u) pos[u] = 0;
    for (int step = tb.half; step > 0; step >>= 1) {
#pragma unroll
        for (int u = 0; u < kRowsPerThread; ++u) pos[u] = (t_edge[pos[u] + step - 1] < v[u]) ? pos[u] + step : pos[u];
    }
#pragma unroll
    for (int u = 0; u < kRowsPerThread; ++u) {
        const int64_t r = base + (int64_t)u * kThreads;
        if (r < n) oc[r] = (uint8_t)((v[u] != v[u]) ? tb.nan_bin : pos[u]);
    }
}

void set_err(char *err, int32_t len, const std::string &m) {
    if (err && len > 0) std::snprintf(err, (size_t)len, "%s", m.c_str());
}

struct HipError {
    std::string what;
};
#define HIPB(x)                                                                           \
    do {                                                                                  \
        hipError_t e_ = (x);                                                              \
        if (e_ != hipSuccess) throw HipError{std::string(#x) + ": " + hipGetErrorString(e_)}; \
    } while (0)

// Device buffers of one call, released on every exit.
struct Buffers {
    std::vector<void *> p;
    hipEvent_t ev[4] = {nullptr, nullptr, nullptr, nullptr};
    template <class T>
    T *alloc(size_t count) {
        void *q = nullptr;
        HIPB(hipMalloc(&q, count * sizeof(T) > 0 ? count * sizeof(T) : 1));
        p.push_back(q);
        return (T *)q;
    }
    ~Buffers() {
        for (void *q : p) (void)hipFree(q);
        for (hipEvent_t e : ev)
            if (e) (void)hipEventDestroy(e);
    }
};

// The descent's answer for v (the host mirror of the kernel's numerical arm,
// used for the NaN bin of a feature without a reserved missing bin).
int descend(const double *tbl, int half, double v) {
    int pos = 0;
    for (int step = half; step > 0; step >>= 1) pos = (tbl[pos + step - 1] < v) ? pos + step : pos;
    return pos;
}

}  // namespace

extern "C" {

int32_t mbh_bin_dense_device(const double *data, int64_t n, int32_t F, int32_t max_bins, int32_t min_data_in_bin,
                             int32_t use_missing, int64_t sample_cnt, int64_t seed, const int32_t *categorical,
                             int32_t n_categorical, uint8_t *out_bins, int32_t *out_missing, int32_t *out_ncat,
                             double *out_times_ms, char *err, int32_t err_len) {
    if (!data || !out_bins || !out_missing || n <= 0 || F <= 0 || n_categorical < 0 ||
        (n_categorical > 0 && !categorical)) {
        set_err(err, err_len, "invalid arguments");
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    if (F > 65535) {
        set_err(err, err_len, "the device transform takes at most 65535 features");
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    const auto t0 = std::chrono::steady_clock::now();
    mb::BinMapper m;
    try {
        const std::vector<int> cats(categorical, categorical + n_categorical);
        m = mb::fit_bins(data, n, F, max_bins, min_data_in_bin, use_missing != 0, sample_cnt, seed, cats);
    } catch (const std::exception &e) {
        set_err(err, err_len, e.what());
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    const double fit_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    // per-feature tables
    std::vector<FeatureTable> ft(F);
    std::vector<double> edges((size_t)F * kTable, INFINITY);
    std::vector<long long> codes((size_t)F * kTable, 0);
    for (int f = 0; f < F; ++f) {
        FeatureTable t{};
        if (!m.is_cat.empty() && m.is_cat[f]) {
            const int64_t k = m.cat_offsets[f + 1] - m.cat_offsets[f];
            if (k > kTable - 1) {
                set_err(err, err_len, "a categorical feature keeps more than 255 codes");
                return MOJOTREES_ERROR_INVALID_ARGUMENT;
            }
            for (int64_t i = 0; i < k; ++i) codes[(size_t)f * kTable + i] = m.cat_codes[m.cat_offsets[f] + i];
            t.is_cat = 1;
            t.half = (int32_t)k;
            t.nan_bin = 0;
        } else {
            const int64_t k = m.edge_offsets[f + 1] - m.edge_offsets[f];
            if (k > kTable - 1) {
                set_err(err, err_len, "a feature has more than 255 bin edges");
                return MOJOTREES_ERROR_INVALID_ARGUMENT;
            }
            int P = 1;
            while (P <= k) P += P;
            for (int64_t i = 0; i < k; ++i) edges[(size_t)f * kTable + i] = m.edges[m.edge_offsets[f] + i];
            t.is_cat = 0;
            t.half = P >> 1;
            t.nan_bin = m.missing_bin[f] >= 0 ? m.missing_bin[f] : descend(&edges[(size_t)f * kTable], t.half, 0.0);
        }
        ft[f] = t;
    }
    try {
        Buffers b;
        double *dx = b.alloc<double>((size_t)n * F);
        uint8_t *dout = b.alloc<uint8_t>((size_t)n * F);
        FeatureTable *dft = b.alloc<FeatureTable>(F);
        double *dedge = b.alloc<double>((size_t)F * kTable);
        long long *dcode = b.alloc<long long>((size_t)F * kTable);
        for (auto &e : b.ev) HIPB(hipEventCreate(&e));
        hipStream_t st = nullptr;  // the null stream: the copies and the kernel in order
        HIPB(hipEventRecord(b.ev[0], st));
        HIPB(hipMemcpyAsync(dx, data, (size_t)n * F * sizeof(double), hipMemcpyHostToDevice, st));
        HIPB(hipMemcpyAsync(dft, ft.data(), ft.size() * sizeof(FeatureTable), hipMemcpyHostToDevice, st));
        HIPB(hipMemcpyAsync(dedge, edges.data(), edges.size() * sizeof(double), hipMemcpyHostToDevice, st));
        HIPB(hipMemcpyAsync(dcode, codes.data(), codes.size() * sizeof(long long), hipMemcpyHostToDevice, st));
        HIPB(hipEventRecord(b.ev[1], st));
        const int64_t per_block = (int64_t)kThreads * kRowsPerThread;
        const int64_t gx = (n + per_block - 1) / per_block;
        if (gx > 0x7FFFFFFF) throw HipError{"too many rows for one launch"};
        hipLaunchKernelGGL(k_bin_transform, dim3((unsigned)gx, (unsigned)F), dim3(kThreads), 0, st, dx, n, dft, dedge,
                           dcode, dout);
        HIPB(hipGetLastError());
        HIPB(hipEventRecord(b.ev[2], st));
        HIPB(hipMemcpyAsync(out_bins, dout, (size_t)n * F, hipMemcpyDeviceToHost, st));
        HIPB(hipEventRecord(b.ev[3], st));
        HIPB(hipStreamSynchronize(st));
        if (out_times_ms) {
            float a = 0.f, k = 0.f, c = 0.f;
            HIPB(hipEventElapsedTime(&a, b.ev[0], b.ev[1]));
            HIPB(hipEventElapsedTime(&k, b.ev[1], b.ev[2]));
            HIPB(hipEventElapsedTime(&c, b.ev[2], b.ev[3]));
            out_times_ms[0] = fit_ms;
            out_times_ms[1] = a;
            out_times_ms[2] = k;
            out_times_ms[3] = c;
        }
    } catch (const HipError &e) {
        set_err(err, err_len, e.what);
        return MOJOTREES_ERROR_TRAINING;
    }
    for (int f = 0; f < F; ++f) {
        out_missing[f] = m.missing_bin[f];
        if (out_ncat) out_ncat[f] = m.n_categories(f);
    }
    return MOJOTREES_OK;
}

}  // extern "C"
