// Scalar arithmetic shared by the HIP kernels and the host control plane.
//
// Every routine here is a fixed sequence of IEEE-754 binary64 operations
// (add, multiply, divide, explicit fma, floor, exact scaling). The library is
// compiled with -ffp-contract=off, so the device and the host produce the
// same bits for the same inputs; the fused steps are written as fma() where
// the reference's own arithmetic fuses them.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define MB_HD __host__ __device__ __forceinline__

namespace mb {

// splitmix64 finalizer and the 53-bit uniform built on it
// (reference src/mojotrees/rng.mojo:35-46).
MB_HD uint64_t splitmix64(uint64_t state) {
    uint64_t z = state + 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}
constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ULL;

MB_HD double uniform53(uint64_t counter) {
    return (double)(splitmix64(counter) >> 11) * (1.0 / 9007199254740992.0);
}

// Stochastic-rounding stream of one (round, class, plane)
// (reference src/mojotrees/quantized_gradient.mojo:475-492).
MB_HD uint64_t quant_stream(int64_t seed, int64_t round_index, int64_t class_index,
                            int64_t plane) {
    uint64_t h = splitmix64((uint64_t)(seed & 0x7FFFFFFFFFFFFFFFLL));
    h = splitmix64(h ^ (uint64_t)(round_index & 0x7FFFFFFFFFFFFFFFLL));
    h = splitmix64(h ^ (uint64_t)((class_index + 1) & 0x7FFFFFFFFFFFFFFFLL));
    return splitmix64(h ^ ((uint64_t)plane * kGolden));
}

// The exponential the reference trains with (the Mojo 1.0 stdlib `exp`
// called from boosting._sigmoid, src/mojotrees/boosting.mojo:261-266):
// k = floor(x / ln2 + 0.5), r = x - k * ln2 (one truncated constant), the
// degree-12 Taylor polynomial of e^r in fused Horner form, scaled by 2^k.
MB_HD double ref_exp(double x) {
    if (x != x) return x;
    if (x < -709.436139303) x = -709.436139303;
    if (x > 709.437) x = 709.437;
    const double c[13] = {1.0,
                          1.0,
                          0.5,
                          0.16666666666666666667,
                          0.041666666666666666667,
                          0.0083333333333333333333,
                          0.0013888888888888888889,
                          0.00019841269841269841270,
                          0.000024801587301587301587,
                          2.7557319223985890653e-6,
                          2.7557319223985890653e-7,
                          2.5052108385441718775e-8,
                          2.0876756987868098979e-9};
    double k = floor(fma(x, 1.442695040888963407359924681001892137, 0.5));
    double r = fma(k, -0.69314718055966295651160180568695068359375, x);
    double y = c[12];
#pragma unroll
    for (int i = 11; i >= 0; --i) y = fma(y, r, c[i]);
    return ldexp(y, (int)k);
}

// The natural log the reference's base score uses (Mojo 1.0 stdlib `log`,
// called from boosting._base_score, src/mojotrees/boosting.mojo:556-567, and
// train_multiclass, :4231): the Cephes logf reduction and polynomial carried
// out in binary64 with fused steps. Host-side only in practice.
MB_HD double ref_log(double xv) {
    const double c[9] = {3.3333331174e-1, -2.4999993993e-1, 2.0000714765e-1,
                         -1.6668057665e-1, 1.4249322787e-1, -1.2420140846e-1,
                         1.1676998740e-1, -1.1514610310e-1, 7.0376836292e-2};
    int e = 0;
    double x1 = frexp(xv, &e);
    if (x1 < 0.70710678118654752440) {
        x1 = x1 * 2.0 - 1.0;
        e -= 1;
    } else {
        x1 = x1 - 1.0;
    }
    double x2 = x1 * x1;
    double y = c[8];
    for (int i = 7; i >= 0; --i) y = fma(y, x1, c[i]);
    y = x1 * x2 * y;
    y = fma(-0.5, x2, y);
    y = x1 + y;
    return fma((double)e, 0.69314718055994530942, y);
}

// The reference's log2 (ranking.mojo:240-244, :598): the same reduction and
// polynomial as ref_log, taken in base 2 as y * log2(e) + e; exact at powers
// of two.
MB_HD double ref_log2(double xv) {
    const double c[9] = {3.3333331174e-1, -2.4999993993e-1, 2.0000714765e-1,
                         -1.6668057665e-1, 1.4249322787e-1, -1.2420140846e-1,
                         1.1676998740e-1, -1.1514610310e-1, 7.0376836292e-2};
    int e = 0;
    double x1 = frexp(xv, &e);
    if (x1 < 0.70710678118654752440) {
        x1 = x1 * 2.0 - 1.0;
        e -= 1;
    } else {
        x1 = x1 - 1.0;
    }
    double x2 = x1 * x1;
    double y = c[8];
    for (int i = 7; i >= 0; --i) y = fma(y, x1, c[i]);
    y = x1 * x2 * y;
    y = fma(-0.5, x2, y);
    y = x1 + y;
    return fma(y, 1.44269504088896340736, (double)e);
}

// LambdaRank pieces (ranking.mojo:235-237, :500-507): the label gain
// 2^l - 1 and the pairwise logistic 1 / (1 + exp(sigma * delta)).
MB_HD double label_gain(int l) { return (double)((1LL << l) - 1); }
MB_HD double pair_sigmoid(double delta, double sigma) {
    const double z = sigma * delta;
    if (z >= 0.0) {
        const double e = ref_exp(-z);
        return e / (1.0 + e);
    }
    const double e = ref_exp(z);
    return 1.0 / (1.0 + e);
}

// Logistic link in branch-on-sign form (boosting.mojo:261-266).
MB_HD double sigmoid(double x) {
    if (x >= 0.0) {
        double e = ref_exp(-x);
        return 1.0 / (1.0 + e);
    }
    double e = ref_exp(x);
    return e / (1.0 + e);
}

// LightGBM's ThresholdL1 and the leaf score (gain.mojo:17-35).
MB_HD double soft_threshold_l1(double s, double l1) {
    if (l1 <= 0.0) return s;
    double mag = fabs(s) - l1;
    if (mag <= 0.0) return 0.0;
    return s > 0.0 ? mag : -mag;
}

// Score of a leaf holding integer sums (g, h) on a (gu, hu) lattice:
// quantized_leaf_score (quantized_gradient.mojo:3252-3281).
MB_HD double qscore(int64_t g, int64_t h, double gu, double hu, double l1, double l2) {
    double t = soft_threshold_l1((double)g / gu, l1);
    return t * t / ((double)h / hu + l2);
}

// Newton step from integer sums: quantized_leaf_output (:3312-3334).
MB_HD double qleaf(int64_t g, int64_t h, double gu, double hu, double l1, double l2) {
    return -soft_threshold_l1((double)g / gu, l1) / ((double)h / hu + l2);
}

// One value onto the lattice, LightGBM's magnitude-symmetric stochastic
// rounding or round-half-away-from-zero (quantized_gradient.mojo:1479-1545).
MB_HD int32_t quantize_scalar(double value, double units, int32_t max_unit, bool stochastic,
                              uint64_t counter) {
    double y = value * units;
    double lim = (double)max_unit;
    if (y > lim) y = lim;
    else if (y < -lim) y = -lim;
    if (stochastic) {
        double u = uniform53(counter);
        if (y >= 0.0) return (int32_t)floor(y + u);
        return -(int32_t)floor(-y + u);
    }
    return (int32_t)round(y);
}

// The magnitude-sum lattice (quantized_gradient.mojo:856-1117): the scale is
// the power of two 2^k <= fl(2^30 / max(total, 1e-12)), found by clearing
// the mantissa bits of the quotient (largest_power_of_two_at_most), and must
// be a binary32 value exactly (the reference multiplies in binary32). ok is
// false for a non-finite total, a subnormal quotient or a power below 2^-149.
constexpr double kFixedOne = 1073741824.0;  // FIXED_ONE = 2^30
MB_HD double fixed_point_scale_pow2(double total, bool &ok) {
    ok = false;
    if (!(total == total) || total > 1.7976931348623157e308) return 1.0;
    const double t = total < 1e-12 ? 1e-12 : total;
    const double q = kFixedOne / t;
    if (!(q > 0.0) || q > 1.7976931348623157e308) return 1.0;
    unsigned long long b;
    __builtin_memcpy(&b, &q, 8);
    const unsigned long long biased = (b >> 52) & 0x7FFULL;
    if (biased == 0) return 1.0;
    const unsigned long long pb = biased << 52;
    double p;
    __builtin_memcpy(&p, &pb, 8);
    const float f = (float)p;
    if (!(f > 0.0f) || (double)f != p) return 1.0;
    ok = true;
    return p;
}

}  // namespace mb
