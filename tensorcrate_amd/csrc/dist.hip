// Distribution functions: `Kernels::vector_distribution`,
// `matrix_distribution` and `matrix_axis_distribution` (tensors/kernels.rs:
// 1046-1070; Host statistics/mod.rs:649-651, :733-735, :785-801).
//
// The Host evaluates every element in f64 and rounds once to the element type
// (statistics/special.rs:1-9, statistics/mod.rs:273-297), and so does this
// file: CDNA4 runs f64 at half the f32 vector rate, which keeps even the
// normal CDF (two exponentials, a rational and a division per element) within
// a small factor of the memory stream.  The special functions are the
// published methods the Host uses, evaluated in the same order:
//  - erf / erfc: W. J. Cody, "Rational Chebyshev approximations for the error
//    function", Math. Comp. 23 (1969), as in his CALERF routine: a rational in
//    x^2 up to 0.46875, exp(-x^2) times a rational up to 4, an asymptotic
//    rational beyond, with x^2 split at a multiple of 1/16 so exp(-x^2) stays
//    accurate;
//  - the normal quantile: M. J. Wichura, "Algorithm AS 241: The percentage
//    points of the normal distribution", Appl. Statist. 37 (1988), PPND16;
//  - the inverse Gaussian: its closed-form density and distribution function
//    (the second CDF term taken through ln erfc so exp(2 lambda/mu) cannot
//    overflow), and the quantile by a bracketed Newton iteration.
// Built with -ffp-contract=off, so no product is fused into a sum the Host
// rounds separately.

#include "common.hpp"

namespace tc {
namespace {

constexpr double kInvSqrtPi = 0.56418958354775628695;  // 1/sqrt(pi)
constexpr double kSqrt2Pi = 2.50662827463100050242;    // sqrt(2 pi)
constexpr double kInvSqrt2 = 0.70710678118654752440;   // 1/sqrt(2)
constexpr double kLn2 = 0.69314718055994530942;
constexpr double kTwoPi = 6.28318530717958647693;
constexpr double kErfCentral = 0.46875;
constexpr double kErfcAsymptotic = 4.0;
constexpr double kErfcUnderflow = 27.25;  // erfc(x) is below the least double beyond

// Cody's coefficients (CALERF): the central rational A/B, the shoulder C/D,
// the asymptotic P/Q.
__constant__ const double kCodyA[5] = {3.16112374387056560e00, 1.13864154151050156e02, 3.77485237685302021e02,
                                       3.20937758913846947e03, 1.85777706184603153e-1};
__constant__ const double kCodyB[4] = {2.36012909523441209e01, 2.44024637934444173e02, 1.28261652607737228e03,
                                       2.84423683343917062e03};
__constant__ const double kCodyC[9] = {5.64188496988670089e-1, 8.88314979438837594e00, 6.61191906371416295e01,
                                       2.98635138197400131e02, 8.81952221241769090e02, 1.71204761263407058e03,
                                       2.05107837782607147e03, 1.23033935479799725e03, 2.15311535474403846e-8};
__constant__ const double kCodyD[8] = {1.57449261107098347e01, 1.17693950891312499e02, 5.37181101862009858e02,
                                       1.62138957456669019e03, 3.29079923573345963e03, 4.36261909014324716e03,
                                       3.43936767414372164e03, 1.23033935480374942e03};
__constant__ const double kCodyP[6] = {3.05326634961232344e-1, 3.60344899949804439e-1, 1.25781726111229246e-1,
                                       1.60837851487422766e-2, 6.58749161529837803e-4, 1.63153871373020978e-2};
__constant__ const double kCodyQ[5] = {2.56852019228982242e00, 1.87295284992346047e00, 5.27905102951428412e-1,
                                       6.05183413124413191e-2, 2.33520497626869185e-3};

// Wichura's PPND16: numerator a0..a7 and denominator b1..b7 (b0 = 1) for
// |p - 1/2| <= 0.425, then c/d and e/f in r = sqrt(-ln min(p, 1-p)), split at
// r = 5.
__constant__ const double kAs241A[8] = {3.3871328727963666080e0, 1.3314166789178437745e2, 1.9715909503065514427e3,
                                        1.3731693765509461125e4, 4.5921953931549871457e4, 6.7265770927008700853e4,
                                        3.3430575583588128105e4, 2.5090809287301226727e3};
__constant__ const double kAs241B[7] = {4.2313330701600911252e1, 6.8718700749205790830e2, 5.3941960214247511077e3,
                                        2.1213794301586595867e4, 3.9307895800092710610e4, 2.8729085735721942674e4,
                                        5.2264952788528545610e3};
__constant__ const double kAs241C[8] = {1.42343711074968357734e0, 4.63033784615654529590e0, 5.76949722146069140550e0,
                                        3.64784832476320460504e0, 1.27045825245236838258e0, 2.41780725177450611770e-1,
                                        2.27238449892691845833e-2, 7.74545014278341407640e-4};
__constant__ const double kAs241D[7] = {2.05319162663775882187e0, 1.67638483018380384940e0, 6.89767334985100004550e-1,
                                        1.48103976427480074590e-1, 1.51986665636164571966e-2, 5.47593808499534494600e-4,
                                        1.05075007164441684324e-9};
__constant__ const double kAs241E[8] = {6.65790464350110377720e0, 5.46378491116411436990e0, 1.78482653991729133580e0,
                                        2.96560571828504891230e-1, 2.65321895265761230930e-2, 1.24266094738807843860e-3,
                                        2.71155556874348757815e-5, 2.01033439929228813265e-7};
__constant__ const double kAs241F[7] = {5.99832206555887937690e-1, 1.36929880922735805310e-1, 1.48753612908506148525e-2,
                                        7.86869131145613259100e-4, 1.84631831751005468180e-5, 1.42151175831644588870e-7,
                                        2.04426310338993978564e-15};

// c[0] + c[1] x + ... + c[n-1] x^(n-1), Horner from the top.
template <int N>
__device__ double horner(const double (&c)[N], double x) {
    double total = c[N - 1];
#pragma unroll
    for (int i = N - 2; i >= 0; i--) total = total * x + c[i];
    return total;
}

// erf on [-0.46875, 0.46875]: x times a rational in x^2.
__device__ double erf_central(double x) {
    const double z = x * x;
    double top = kCodyA[4] * z;
    double bottom = z;
#pragma unroll
    for (int i = 0; i < 3; i++) {
        top = (top + kCodyA[i]) * z;
        bottom = (bottom + kCodyB[i]) * z;
    }
    return x * (top + kCodyA[3]) / (bottom + kCodyB[3]);
}

// exp(x^2) erfc(x) for x > 0.46875.
__device__ double erfc_scaled(double x) {
    if (x <= kErfcAsymptotic) {
        double top = kCodyC[8] * x;
        double bottom = x;
#pragma unroll
        for (int i = 0; i < 7; i++) {
            top = (top + kCodyC[i]) * x;
            bottom = (bottom + kCodyD[i]) * x;
        }
        return (top + kCodyC[7]) / (bottom + kCodyD[7]);
    }
    const double z = 1.0 / (x * x);
    double top = kCodyP[5] * z;
    double bottom = z;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        top = (top + kCodyP[i]) * z;
        bottom = (bottom + kCodyQ[i]) * z;
    }
    const double correction = z * (top + kCodyP[4]) / (bottom + kCodyQ[4]);
    return (kInvSqrtPi - correction) / x;
}

// erfc for x > 0.46875: exp(-x^2) split as exp(-l^2) exp(-(x-l)(x+l)) with l
// = x truncated to a multiple of 1/16, so l^2 is exact.
__device__ double erfc_positive(double x) {
    if (x > kErfcUnderflow) return 0.0;
    const double leading = trunc(x * 16.0) / 16.0;
    const double correction = (x - leading) * (x + leading);
    return exp(-leading * leading) * exp(-correction) * erfc_scaled(x);
}

__device__ double erfc_of(double x) {
    if (isnan(x)) return x;
    if (x < -kErfCentral) return 2.0 - erfc_positive(-x);
    if (x <= kErfCentral) return 1.0 - erf_central(x);
    return erfc_positive(x);
}

// ln erfc(x), finite far past where erfc underflows.
__device__ double ln_erfc(double x) {
    if (isnan(x)) return x;
    if (x <= kErfCentral) return log(erfc_of(x));
    return log(erfc_scaled(x)) - x * x;
}

__device__ double standard_pdf(double z) { return exp(-0.5 * z * z) / kSqrt2Pi; }
__device__ double standard_cdf(double z) { return 0.5 * erfc_of(-z * kInvSqrt2); }
__device__ double standard_ln_cdf(double z) { return ln_erfc(-z * kInvSqrt2) - kLn2; }

__device__ double standard_ppf(double p) {
    if (!(p >= 0.0 && p <= 1.0)) return __builtin_nan("");
    if (p == 0.0) return -__builtin_inf();
    if (p == 1.0) return __builtin_inf();
    const double q = p - 0.5;
    if (fabs(q) <= 0.425) {
        const double r = 0.180625 - q * q;
        return q * horner(kAs241A, r) / (horner(kAs241B, r) * r + 1.0);
    }
    double r = sqrt(-log(q < 0.0 ? p : 1.0 - p));
    double value;
    if (r <= 5.0) {
        r = r - 1.6;
        value = horner(kAs241C, r) / (horner(kAs241D, r) * r + 1.0);
    } else {
        r = r - 5.0;
        value = horner(kAs241E, r) / (horner(kAs241F, r) * r + 1.0);
    }
    return q < 0.0 ? -value : value;
}

// Normal(mean, stddev); a scale that is not positive gives NaN.
__device__ double normal(uint32_t statistic, double x, double mean, double stddev) {
    if (!(stddev > 0.0)) return __builtin_nan("");
    switch (statistic) {
        case 0: return standard_pdf((x - mean) / stddev) / stddev;
        case 1: return standard_cdf((x - mean) / stddev);
        default: return mean + stddev * standard_ppf(x);
    }
}

__device__ double wald_pdf(double x, double mean, double shape) {
    if (x <= 0.0) return 0.0;
    const double deviation = x - mean;
    const double exponent = -shape * deviation * deviation / (2.0 * mean * mean * x);
    return sqrt(shape / (kTwoPi * x * x * x)) * exp(exponent);
}

// Phi(a) + exp(2 lambda/mu + ln Phi(-b)), capped at 1 (a NaN sum gives 1, as
// minNum does).
__device__ double wald_cdf(double x, double mean, double shape) {
    if (x <= 0.0) return 0.0;
    const double scale = sqrt(shape / x);
    const double ratio = x / mean;
    const double lower = scale * (ratio - 1.0);
    const double upper = scale * (ratio + 1.0);
    const double tail = 2.0 * shape / mean + standard_ln_cdf(-upper);
    return fmin(standard_cdf(lower) + exp(tail), 1.0);
}

// The quantile: bracket [low, high] by doubling from the mean, then at most
// 60 Newton steps, each replaced by a bisection when it leaves the bracket.
__device__ double wald_ppf(double p, double mean, double shape) {
    if (!(p >= 0.0 && p <= 1.0)) return __builtin_nan("");
    if (p == 0.0) return 0.0;
    if (p == 1.0) return __builtin_inf();
    double low = 0.0;
    double high = mean;
    while (wald_cdf(high, mean, shape) < p) {
        low = high;
        high = high * 2.0;
        if (isinf(high)) return __builtin_inf();
    }
    double guess = 0.5 * (low + high);
    for (int pass = 0; pass < 60; pass++) {
        const double error = wald_cdf(guess, mean, shape) - p;
        if (error > 0.0) {
            high = guess;
        } else {
            low = guess;
        }
        const double density = wald_pdf(guess, mean, shape);
        const double step = density > 0.0 ? guess - error / density : __builtin_nan("");
        const double next = (isfinite(step) && step > low && step < high) ? step : 0.5 * (low + high);
        if (next == guess) break;
        guess = next;
    }
    return guess;
}

__device__ double wald(uint32_t statistic, double x, double mean, double shape) {
    if (!(mean > 0.0) || !(shape > 0.0)) return __builtin_nan("");
    switch (statistic) {
        case 0: return wald_pdf(x, mean, shape);
        case 1: return wald_cdf(x, mean, shape);
        default: return wald_ppf(x, mean, shape);
    }
}

__device__ double evaluate(uint32_t family, uint32_t statistic, double x, double first, double second) {
    return family == 0 ? normal(statistic, x, first, second) : wald(statistic, x, first, second);
}

// f64 to the element type: to f32 by round-to-nearest-even, then (f16,
// bf16) to the type the same way, as the Host's `NumCast` does.
template <typename S>
__device__ S from_double(double v) {
    return Elem<S>::narrow(static_cast<float>(v));
}

template <typename S>
__global__ void __launch_bounds__(256) distribution_kernel(const S* __restrict__ a, S* __restrict__ out, uint64_t n,
                                                           uint32_t family, uint32_t statistic, double first,
                                                           double second) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        const double x = Elem<S>::widen(a[i]);
        out[i] = from_double<S>(evaluate(family, statistic, x, first, second));
    }
}

// One parameter pair per row (blockIdx.y walks rows) or per column.
template <typename S, bool PER_ROW>
__global__ void __launch_bounds__(256) axis_distribution_kernel(const S* __restrict__ a, S* __restrict__ out,
                                                                uint64_t rows, uint64_t cols, uint32_t family,
                                                                uint32_t statistic, const S* __restrict__ first,
                                                                const S* __restrict__ second) {
    using E = Elem<S>;
    for (uint64_t row = blockIdx.y; row < rows; row += gridDim.y) {
        const double row_first = PER_ROW ? E::widen(first[row]) : 0.0;
        const double row_second = PER_ROW ? E::widen(second[row]) : 0.0;
        const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
        for (uint64_t col = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; col < cols; col += stride) {
            const double p1 = PER_ROW ? row_first : E::widen(first[col]);
            const double p2 = PER_ROW ? row_second : E::widen(second[col]);
            const uint64_t i = row * cols + col;
            out[i] = from_double<S>(evaluate(family, statistic, E::widen(a[i]), p1, p2));
        }
    }
}

int check_codes(const char* what, uint32_t family, uint32_t statistic) {
    if (family > 1) return fail(TC_INVALID, std::string(what) + ": no Family " + std::to_string(family));
    if (statistic > 2) return fail(TC_INVALID, std::string(what) + ": no Statistic " + std::to_string(statistic));
    return TC_OK;
}

}  // namespace
}  // namespace tc

using namespace tc;

extern "C" {

int tc_distribution(uint32_t dtype, uint32_t family, uint32_t statistic, const void* a, void* out, uint64_t n,
                    float first, float second) {
    TC_STREAM(s);
    const int status = check_codes("distribution", family, statistic);
    if (status != TC_OK) return status;
    TC_DISPATCH_FLOAT(dtype, "distribution", S, {
        if (n == 0) return TC_OK;
        distribution_kernel<S><<<blocks_for(n, 1), 256, 0, s>>>(static_cast<const S*>(a), static_cast<S*>(out), n,
                                                                 family, statistic, first, second);
        return check_launch("distribution");
    });
    return TC_OK;
}

int tc_axis_distribution(uint32_t dtype, uint32_t family, uint32_t statistic, const void* a, uint64_t rows,
                         uint64_t cols, uint32_t axis, const void* first, const void* second, void* out) {
    TC_STREAM(s);
    int status = check_codes("axis distribution", family, statistic);
    if (status != TC_OK) return status;
    if (axis > TC_AXIS_COLUMNS) return fail(TC_INVALID, "axis distribution: no Axis " + std::to_string(axis));
    TC_DISPATCH_FLOAT(dtype, "axis distribution", S, {
        if (rows == 0 || cols == 0) return TC_OK;
        const uint32_t across = blocks_for(cols, 1) < 64 ? blocks_for(cols, 1) : 64;
        const uint64_t down_wanted = (uint64_t{1} << 14) / across;
        const uint32_t down = static_cast<uint32_t>(rows < down_wanted ? rows : (down_wanted > 0 ? down_wanted : 1));
        const dim3 grid(across, down);
        const S* in = static_cast<const S*>(a);
        S* o = static_cast<S*>(out);
        const S* p1 = static_cast<const S*>(first);
        const S* p2 = static_cast<const S*>(second);
        if (axis == TC_AXIS_ROWS) {
            axis_distribution_kernel<S, true><<<grid, 256, 0, s>>>(in, o, rows, cols, family, statistic, p1, p2);
        } else {
            axis_distribution_kernel<S, false><<<grid, 256, 0, s>>>(in, o, rows, cols, family, statistic, p1, p2);
        }
        return check_launch("axis distribution");
    });
    return TC_OK;
}

}  // extern "C"
