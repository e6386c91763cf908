// mbh_histogram_noalloc: the quantized histogram of mbh_histogram for callers
// that cannot allocate device memory (code under HIP graph capture, serving
// loops, harnesses that forbid hipMalloc). Inputs and the output are the
// caller's device buffers; the block partials live in `scratch`, a static
// device array of kScratchBytes that each GPU the library runs on holds until
// the process ends. No hipMalloc, hipFree, hipMemset or allocating library
// routine is called on this path.
//
// In host code `scratch` names a host-side stand-in, not a device address:
// the address of each device's copy is taken once per device with
// hipGetSymbolAddress (with that device current) and only that address is
// handed to kernels.
//
// Calls on one GPU share its scratch: two calls that overlap on one GPU (on
// different streams, or from different host threads) race. Every partial cell
// a call reads is written by the same call first, so nothing is carried over
// from an earlier call.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>

#include "../../include/mojoboost_hip.h"
#include "../../include/mojotrees.h"

namespace {

constexpr size_t kScratchBytes = (size_t)MBH_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
constexpr int kThreads = 256;
constexpr int kMaxBlocks = 2048;       // row chunks of one call, at most
constexpr int kMinChunk = 2048;        // fewest rows a block is given
constexpr size_t kLdsBudget = 64 * 1024;  // one block's packed LDS histogram

__device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_mu;
void *g_scratch[kMaxDevices] = {};

void set_err(char *err, int32_t len, const char *m) {
    if (err && len > 0) std::snprintf(err, (size_t)len, "%s", m);
}

// The device address of the current device's scratch, looked up once per
// device (hipGetSymbolAddress with that device current).
hipError_t device_scratch(void **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_scratch[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return hipSuccess;
}

// Rows a block may pack into its 64-bit LDS counters (count in bits [0, 20),
// hessian sum in [20, 42), signed gradient sum in [42, 64)) before a field
// overflows, for |q_grad| <= B/2 + 1 and 0 <= q_hess <= B + 1.
int64_t chunk_limit(int B) {
    int64_t lim = (1 << 20) - 1;
    const int64_t h = ((1 << 22) - 1) / (B + 1);
    const int64_t g = ((1 << 21) - 1) / (B / 2 + 1);
    if (h < lim) lim = h;
    if (g < lim) lim = g;
    return lim;
}

__global__ void k_na_clear(int32_t *status) {
    if (status && threadIdx.x == 0 && blockIdx.x == 0) *status = 0;
}

// Block (x, y): rows [x * chunk, ...) of the selection, features
// [y * ft, y * ft + ft). Each thread takes one row at a time and adds a
// packed (grad, hess, 1) counter per feature of the tile into the block's
// LDS histogram; the block then writes every cell of its tile as partial x.
// Entries that are out of range (a row id outside [0, n), a quantized pair
// outside the lattice, a bin id >= n_bins) are not added and flag *status.
__global__ __launch_bounds__(kThreads) void k_na_hist(const uint8_t *bins_cm, int64_t n, int F, int nb,
                                                     const int8_t *qg, const int8_t *qh, const int32_t *rows,
                                                     int64_t m, int64_t chunk, int ft, int gmax, int hmax,
                                                     unsigned long long *part, int32_t *status) {
    extern __shared__ unsigned long long lds[];
    const int f0 = (int)blockIdx.y * ft;
    const int nf = min(ft, F - f0);
    for (int i = threadIdx.x; i < nf * nb; i += kThreads) lds[i] = 0ULL;
    __syncthreads();
    const int64_t c0 = (int64_t)blockIdx.x * chunk;
    const int64_t c1 = c0 + chunk < m ? c0 + chunk : m;
    bool bad = false;
    for (int64_t i = c0 + threadIdx.x; i < c1; i += kThreads) {
        const int64_t r = rows ? (int64_t)rows[i] : i;
        if (r < 0 || r >= n) {
            bad = true;
            continue;
        }
        const int g = qg[r], h = qh[r];
        if (g < -gmax || g > gmax || h < 0 || h > hmax) {
            bad = true;
            continue;
        }
        const unsigned long long packed =
            (unsigned long long)(((long long)g << 42) + ((long long)h << 20) + 1LL);
        for (int f = 0; f < nf; ++f) {
            const int b = bins_cm[(size_t)(f0 + f) * n + r];
            if (b >= nb) {
                bad = true;
                continue;
            }
            atomicAdd(&lds[f * nb + b], packed);
        }
    }
    if (bad && status) atomicOr(status, 1);
    __syncthreads();
    unsigned long long *out = part + ((size_t)blockIdx.x * F + f0) * nb;
    for (int i = threadIdx.x; i < nf * nb; i += kThreads) out[i] = lds[i];
}

// One thread per (feature, bin) cell: the sum of the blocks' partials,
// unpacked, as int32 {grad, hess, count}.
__global__ __launch_bounds__(kThreads) void k_na_merge(const unsigned long long *part, int blocks, int cells,
                                                      int32_t *out) {
    const int c = (int)(blockIdx.x * (unsigned)kThreads + threadIdx.x);
    if (c >= cells) return;
    long long g = 0, h = 0, cnt = 0;
    for (int b = 0; b < blocks; ++b) {
        const unsigned long long v = part[(size_t)b * cells + c];
        cnt += (long long)(v & 0xFFFFFULL);
        h += (long long)((v >> 20) & 0x3FFFFFULL);
        g += (long long)v >> 42;
    }
    out[3 * c + 0] = (int32_t)g;
    out[3 * c + 1] = (int32_t)h;
    out[3 * c + 2] = (int32_t)cnt;
}

}  // namespace

extern "C" int32_t mbh_histogram_noalloc(const uint8_t *bins_cm, int64_t n_rows, int32_t n_features,
                                         int32_t n_bins, const int8_t *q_grad, const int8_t *q_hess,
                                         const int32_t *rows, int64_t n_sel, int32_t B, int32_t *out,
                                         int32_t *status, void *stream, char *err, int32_t err_len) {
    if (!bins_cm || !q_grad || !q_hess || !out || n_rows <= 0 || n_features <= 0 || n_bins < 2 ||
        n_bins > 256 || (rows && n_sel <= 0)) {
        set_err(err, err_len, "invalid arguments");
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    if (n_rows >= ((int64_t)1 << 31)) {
        set_err(err, err_len, "n_rows must be below 2^31");
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    if (B < 2 || B > 126 || B % 2 != 0) {
        set_err(err, err_len, "num_grad_quant_bins must be even and in [2, 126]");
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    const int64_t m = rows ? n_sel : n_rows;
    if ((double)m * (double)(B + 1) >= 2147483647.0) {
        set_err(err, err_len, "rows * (num_grad_quant_bins + 1) must stay below 2^31 for int32 histogram cells");
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    // one partial in 64-bit arithmetic, checked before anything divides by
    // it or narrows the cell count (n_features * n_bins may exceed int)
    const int64_t cells64 = (int64_t)n_features * (int64_t)n_bins;
    const uint64_t partial_bytes = (uint64_t)cells64 * sizeof(unsigned long long);
    if (partial_bytes > (uint64_t)kScratchBytes) {
        set_err(err, err_len,
                "n_features * n_bins exceeds the no-alloc scratch (one partial of 8 bytes per cell must fit "
                "MBH_NOALLOC_SCRATCH_BYTES)");
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    const int cells = (int)cells64;  // at most kScratchBytes / 8 after the check
    int max_blocks = (int)(kScratchBytes / partial_bytes);
    if (max_blocks > kMaxBlocks) max_blocks = kMaxBlocks;
    const int64_t limit = chunk_limit(B);
    int64_t blocks = (m + kMinChunk - 1) / kMinChunk;
    if (blocks > max_blocks) blocks = max_blocks;
    if (blocks < 1) blocks = 1;
    const int64_t chunk = (m + blocks - 1) / blocks;
    if (chunk > limit) {
        set_err(err, err_len,
                "selection too large for the no-alloc scratch at this n_features * n_bins "
                "(the packed block counters would overflow)");
        return MOJOTREES_ERROR_INVALID_ARGUMENT;
    }
    int ft = (int)(kLdsBudget / ((size_t)n_bins * sizeof(unsigned long long)));
    if (ft > n_features) ft = n_features;
    const int tiles = (n_features + ft - 1) / ft;
    void *sp = nullptr;
    hipError_t e = device_scratch(&sp);
    if (e != hipSuccess) {
        set_err(err, err_len, hipGetErrorString(e));
        return MOJOTREES_ERROR_TRAINING;
    }
    auto *part = (unsigned long long *)sp;
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(k_na_clear, dim3(1), dim3(64), 0, st, status);
    hipLaunchKernelGGL(k_na_hist, dim3((unsigned)blocks, (unsigned)tiles), dim3(kThreads),
                       (size_t)ft * n_bins * sizeof(unsigned long long), st, bins_cm, n_rows, (int)n_features,
                       (int)n_bins, q_grad, q_hess, rows, m, chunk, ft, B / 2 + 1, B + 1, part, status);
    hipLaunchKernelGGL(k_na_merge, dim3((unsigned)((cells + kThreads - 1) / kThreads)), dim3(kThreads), 0, st,
                       (const unsigned long long *)part, (int)blocks, cells, out);
    e = hipGetLastError();
    if (e != hipSuccess) {
        set_err(err, err_len, hipGetErrorString(e));
        return MOJOTREES_ERROR_TRAINING;
    }
    return MOJOTREES_OK;
}
