/*
 * CPU restatement of tensorcrate's Host backend for the Hip backend's hot
 * path.  TEST INFRASTRUCTURE: the checker the GPU results are compared with
 * and the timed CPU baseline, never part of the product (see oracle.h).
 *
 * Each function follows the reference's own loop structure and arithmetic
 * order, cited per function as src/<file>:<line> of arthurmburke/tensorcrate,
 * so that where the Host backend is deterministic (copies, elementwise ops,
 * sequential folds, the f32 FMA-chain product, the fused interpreter) this
 * gives its bits.  Built with -ffp-contract=off: every multiply and add the
 * reference writes separately stays separate, and FMA appears only where the
 * reference calls one (_mm256_fmadd_ps, restated with fmaf).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#if defined(__x86_64__)
#include <immintrin.h>
#endif

#define MAX_RANK 6

enum { F32 = 0, F16 = 1, BF16 = 2 };

/* ---- conversions (half 2.7.1, called at compact.rs:40-57) ---------------- */

static uint32_t bits_of(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    return x;
}

static float float_of(uint32_t x) {
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* Round-to-nearest-even with NaN quieting; the rule metal/common.h:153-165
 * restates from `half::bf16::from_f32`. */
uint16_t or_bf16_from_f32(float value) {
    uint32_t x = bits_of(value);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x0040u);
    uint32_t round_bit = 0x00008000u;
    if ((x & round_bit) != 0 && (x & (3u * round_bit - 1u)) != 0) return (uint16_t)((x >> 16) + 1);
    return (uint16_t)(x >> 16);
}

static float bf16_to_f32(uint16_t bits) { return float_of((uint32_t)bits << 16); }

/* `value >> shift` rounded to nearest, ties to even. */
static uint32_t shift_rne(uint32_t value, uint32_t shift) {
    if (shift == 0) return value;
    if (shift > 31) return 0;
    uint32_t q = value >> shift;
    uint32_t rem = value & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return q;
}

/* IEEE binary32 -> binary16, round to nearest even; NaNs keep their top
 * payload bits and are quieted, as `half::f16::from_f32` does. */
uint16_t or_f16_from_f32(float value) {
    uint32_t x = bits_of(value);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xffu) {
        if (man != 0) return (uint16_t)(sign | 0x7e00u | (man >> 13));
        return (uint16_t)(sign | 0x7c00u);
    }
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        /* A subnormal half: the value over 2^-24, rounded. */
        if (exp == 0) return (uint16_t)sign; /* f32 subnormals are far below half's */
        uint32_t significand = man | 0x800000u;
        uint32_t shift = (uint32_t)(126 - (int)exp);
        return (uint16_t)(sign | shift_rne(significand, shift));
    }
    /* Adding a rounded-up mantissa carries into the exponent, and from the
     * largest exponent into infinity, as it should. */
    uint32_t rounded = shift_rne(man, 13);
    return (uint16_t)(sign + ((uint32_t)e << 10) + rounded);
}

float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0x1fu) return float_of(sign | 0x7f800000u | (man << 13));
    if (exp == 0) {
        if (man == 0) return float_of(sign);
        /* subnormal: man * 2^-24, exact in f32 */
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return float_of(sign | ((exp - 15 + 127) << 23) | (man << 13));
}

static float widen_one(uint32_t dtype, const void* p, uint64_t i) {
    switch (dtype) {
        case F16: return or_f16_to_f32(((const uint16_t*)p)[i]);
        case BF16: return bf16_to_f32(((const uint16_t*)p)[i]);
        default: return ((const float*)p)[i];
    }
}

static void narrow_one(uint32_t dtype, void* p, uint64_t i, float v) {
    switch (dtype) {
        case F16: ((uint16_t*)p)[i] = or_f16_from_f32(v); break;
        case BF16: ((uint16_t*)p)[i] = or_bf16_from_f32(v); break;
        default: ((float*)p)[i] = v; break;
    }
}

/* A value rounded to the element type and back. */
static float in_type(uint32_t dtype, float v) {
    switch (dtype) {
        case F16: return or_f16_to_f32(or_f16_from_f32(v));
        case BF16: return bf16_to_f32(or_bf16_from_f32(v));
        default: return v;
    }
}

void or_narrow(uint32_t dtype, const float* in, void* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) narrow_one(dtype, out, i, in[i]);
}

void or_widen(uint32_t dtype, const void* in, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) out[i] = widen_one(dtype, in, i);
}

/* ---- layout walk (layout.rs:419-498) --------------------------------------- */

typedef struct walk {
    uint32_t rank;
    uint64_t shape[MAX_RANK];
    uint64_t strides[3][MAX_RANK];
} walk;

/* `coalesce` (layout.rs:419-449) over n operands. */
static walk coalesce(uint32_t rank, const uint64_t* shape, uint32_t n, const uint64_t* const* strides) {
    walk w;
    memset(&w, 0, sizeof w);
    for (uint32_t axis = 0; axis < rank; axis++) {
        uint64_t extent = shape[axis];
        if (extent == 1) continue;
        uint32_t r = w.rank;
        int joins = r > 0;
        for (uint32_t o = 0; joins && o < n; o++) joins = w.strides[o][r - 1] == strides[o][axis] * extent;
        if (joins) {
            w.shape[r - 1] *= extent;
            for (uint32_t o = 0; o < n; o++) w.strides[o][r - 1] = strides[o][axis];
        } else {
            w.shape[r] = extent;
            for (uint32_t o = 0; o < n; o++) w.strides[o][r] = strides[o][axis];
            w.rank++;
        }
    }
    return w;
}

typedef void (*run_fn)(void* context, const uint64_t* starts, uint64_t len, const uint64_t* steps);

/* `for_each_run` (layout.rs:457-498): one call per innermost run, in
 * row-major order; none for an empty shape, one of one element for a scalar. */
static void for_each_run(uint32_t rank, const uint64_t* shape, uint32_t n, const uint64_t* offsets,
                         const uint64_t* const* strides, run_fn run, void* context) {
    for (uint32_t k = 0; k < rank; k++)
        if (shape[k] == 0) return;
    walk w = coalesce(rank, shape, n, strides);
    uint64_t at[3] = {0, 0, 0};
    for (uint32_t o = 0; o < n; o++) at[o] = offsets[o];
    if (w.rank == 0) {
        uint64_t zero[3] = {0, 0, 0};
        run(context, at, 1, zero);
        return;
    }
    uint64_t inner = w.shape[w.rank - 1];
    uint64_t steps[3] = {0, 0, 0};
    for (uint32_t o = 0; o < n; o++) steps[o] = w.strides[o][w.rank - 1];
    uint64_t index[MAX_RANK] = {0};
    for (;;) {
        run(context, at, inner, steps);
        uint32_t axis = w.rank - 1;
        for (;;) {
            if (axis == 0) return;
            axis--;
            index[axis]++;
            for (uint32_t o = 0; o < n; o++) at[o] += w.strides[o][axis];
            if (index[axis] < w.shape[axis]) break;
            for (uint32_t o = 0; o < n; o++) at[o] -= w.strides[o][axis] * w.shape[axis];
            index[axis] = 0;
        }
    }
}

/* ---- strided copies (backend.rs:255-300) ----------------------------------- */

typedef struct copy_ctx {
    uint32_t width;
    const uint8_t* src;
    uint8_t* out;
    uint64_t written;
} copy_ctx;

static void copy_run(void* c, const uint64_t* starts, uint64_t len, const uint64_t* steps) {
    copy_ctx* ctx = (copy_ctx*)c;
    uint32_t w = ctx->width;
    if (steps[0] == 1) {
        memcpy(ctx->out + ctx->written * w, ctx->src + starts[0] * w, len * w);
    } else {
        for (uint64_t i = 0; i < len; i++)
            memcpy(ctx->out + (ctx->written + i) * w, ctx->src + (starts[0] + i * steps[0]) * w, w);
    }
    ctx->written += len;
}

uint64_t or_strided_copy(uint32_t width, const void* src, uint32_t rank, const uint64_t* shape, uint64_t offset,
                         const uint64_t* strides, void* out) {
    copy_ctx ctx = {width, (const uint8_t*)src, (uint8_t*)out, 0};
    const uint64_t* s[1] = {strides};
    uint64_t offsets[1] = {offset};
    for_each_run(rank, shape, 1, offsets, s, copy_run, &ctx);
    return ctx.written;
}

typedef struct write_ctx {
    uint32_t width;
    const uint8_t* src;
    uint8_t* target;
} write_ctx;

static void write_run(void* c, const uint64_t* starts, uint64_t len, const uint64_t* steps) {
    write_ctx* ctx = (write_ctx*)c;
    uint32_t w = ctx->width;
    for (uint64_t i = 0; i < len; i++)
        memcpy(ctx->target + (starts[1] + i * steps[1]) * w, ctx->src + (starts[0] + i * steps[0]) * w, w);
}

void or_strided_write(uint32_t width, const void* src, void* target, uint32_t rank, const uint64_t* shape,
                      uint64_t from_offset, const uint64_t* from_strides, uint64_t to_offset,
                      const uint64_t* to_strides) {
    write_ctx ctx = {width, (const uint8_t*)src, (uint8_t*)target};
    const uint64_t* s[2] = {from_strides, to_strides};
    uint64_t offsets[2] = {from_offset, to_offset};
    for_each_run(rank, shape, 2, offsets, s, write_run, &ctx);
}

/* ---- elementwise (kernels.rs:98-153, :431-441) ---------------------------- */

/* `Compare::value` (kernels.rs:138-153). */
static float compare_value(uint32_t op, float a, float b) {
    switch (op) {
        case 0: return fminf(a, b);
        case 1: return fmaxf(a, b);
        case 2: return a > b ? 1.0f : (a < b ? 0.0f : 0.5f);
        case 3: return a < b ? 1.0f : 0.0f;
        case 4: return a <= b ? 1.0f : 0.0f;
        case 5: return a > b ? 1.0f : 0.0f;
        default: return a >= b ? 1.0f : 0.0f;
    }
}

static float arithmetic_value(uint32_t op, float a, float b) {
    switch (op) {
        case 0: return a + b;
        case 1: return a - b;
        case 2: return a * b;
        case 3: return a / b;
        default: return fmodf(a, b); /* Rust `%` on floats: the truncated remainder */
    }
}

/* `Pairwise::value` (kernels.rs:431-441) for T of `dtype`: the f32 result
 * rounded to T once, which for f16 and bf16 is the correctly rounded value
 * `half`'s operators give; a power is f32 `powf` then one rounding
 * (numbers/primitive.rs:131-156). */
static float pairwise(uint32_t dtype, uint32_t kind, uint32_t op, float a, float b) {
    float v;
    if (kind == 0) v = arithmetic_value(op, a, b);
    else if (kind == 1) v = compare_value(op, a, b);
    else v = powf(a, b);
    return in_type(dtype, v);
}

typedef struct binary_ctx {
    uint32_t dtype, kind, op;
    const void *a, *b;
    void* out;
    uint64_t written;
} binary_ctx;

static void binary_run(void* c, const uint64_t* starts, uint64_t len, const uint64_t* steps) {
    binary_ctx* ctx = (binary_ctx*)c;
    for (uint64_t k = 0; k < len; k++) {
        float x = widen_one(ctx->dtype, ctx->a, starts[0] + k * steps[0]);
        float y = widen_one(ctx->dtype, ctx->b, starts[1] + k * steps[1]);
        narrow_one(ctx->dtype, ctx->out, ctx->written + k, pairwise(ctx->dtype, ctx->kind, ctx->op, x, y));
    }
    ctx->written += len;
}

void or_binary(uint32_t dtype, uint32_t kind, uint32_t op, uint32_t rank, const uint64_t* shape, const void* a,
               uint64_t a_offset, const uint64_t* a_strides, const void* b, uint64_t b_offset,
               const uint64_t* b_strides, void* out) {
    binary_ctx ctx = {dtype, kind, op, a, b, out, 0};
    const uint64_t* s[2] = {a_strides, b_strides};
    uint64_t offsets[2] = {a_offset, b_offset};
    for_each_run(rank, shape, 2, offsets, s, binary_run, &ctx);
}

void or_elementwise(uint32_t dtype, uint32_t kind, uint32_t op, const void* a, const void* b, void* out,
                    uint64_t n) {
    for (uint64_t i = 0; i < n; i++)
        narrow_one(dtype, out, i, pairwise(dtype, kind, op, widen_one(dtype, a, i), widen_one(dtype, b, i)));
}

void or_scalar(uint32_t dtype, uint32_t kind, uint32_t op, const void* a, float scalar, int scalar_left, void* out,
               uint64_t n) {
    for (uint64_t i = 0; i < n; i++) {
        float x = widen_one(dtype, a, i);
        float v = scalar_left ? pairwise(dtype, kind, op, scalar, x) : pairwise(dtype, kind, op, x, scalar);
        narrow_one(dtype, out, i, v);
    }
}

/* `clamp` (kernels.rs:856-863): the pair of comparisons in one pass. */
void or_clamp(uint32_t dtype, const void* a, float low, float high, void* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) narrow_one(dtype, out, i, fminf(fmaxf(widen_one(dtype, a, i), low), high));
}

/* ---- reductions (strided.rs:80-225) ---------------------------------------- */

static int in_axes(uint32_t axis, uint32_t naxes, const uint32_t* axes) {
    for (uint32_t k = 0; k < naxes; k++)
        if (axes[k] == axis) return 1;
    return 0;
}

/* `result_strides` (strided.rs:83-100). */
static void result_strides(uint32_t rank, const uint64_t* shape, uint32_t naxes, const uint32_t* axes,
                           uint64_t* out) {
    uint64_t kept[MAX_RANK];
    uint32_t nkept = 0;
    for (uint32_t a = 0; a < rank; a++)
        if (!in_axes(a, naxes, axes)) kept[nkept++] = shape[a];
    uint64_t kept_strides[MAX_RANK];
    uint64_t step = 1;
    for (int k = (int)nkept - 1; k >= 0; k--) {
        kept_strides[k] = step;
        step *= kept[k];
    }
    uint32_t next = 0;
    for (uint32_t a = 0; a < rank; a++) out[a] = in_axes(a, naxes, axes) ? 0 : kept_strides[next++];
}

enum { FOLD_SUM, FOLD_MIN, FOLD_MAX, FOLD_DEVIATION };

typedef struct fold_ctx {
    uint32_t dtype, mode;
    const void* input;
    float* acc;
    const float* means;
} fold_ctx;

/* `Reduce::combine` (kernels.rs:205-211) and the deviation fold of
 * strided.rs:150-153, into accumulator `slot`. */
static void fold_run(void* c, const uint64_t* starts, uint64_t len, const uint64_t* steps) {
    fold_ctx* ctx = (fold_ctx*)c;
    for (uint64_t k = 0; k < len; k++) {
        uint64_t slot = starts[1] + k * steps[1];
        float x = widen_one(ctx->dtype, ctx->input, starts[0] + k * steps[0]);
        float t = ctx->acc[slot];
        switch (ctx->mode) {
            case FOLD_SUM: t = t + x; break;
            case FOLD_MIN: t = fminf(t, x); break;
            case FOLD_MAX: t = fmaxf(t, x); break;
            default: {
                float d = x - ctx->means[slot];
                t = t + d * d;
            }
        }
        ctx->acc[slot] = t;
    }
}

static void fold_all(uint32_t dtype, const void* input, uint32_t rank, const uint64_t* shape, uint64_t offset,
                     const uint64_t* strides, const uint64_t* to, uint32_t mode, float* acc, const float* means) {
    fold_ctx ctx = {dtype, mode, input, acc, means};
    const uint64_t* s[2] = {strides, to};
    uint64_t offsets[2] = {offset, 0};
    for_each_run(rank, shape, 2, offsets, s, fold_run, &ctx);
}

/* `reduce_in` with the f32 accumulator (strided.rs:119-162). */
void or_reduce(uint32_t dtype, const void* input, uint32_t rank, const uint64_t* shape, uint64_t offset,
               const uint64_t* strides, uint32_t naxes, const uint32_t* axes, uint32_t kind, uint32_t op,
               uint64_t divisor, void* out) {
    uint64_t to[MAX_RANK];
    result_strides(rank, shape, naxes, axes, to);
    uint64_t results = 1, depth = 1;
    for (uint32_t a = 0; a < rank; a++) {
        if (in_axes(a, naxes, axes)) depth *= shape[a];
        else results *= shape[a];
    }
    float count = (float)(double)depth;
    float* totals = (float*)malloc((results ? results : 1) * sizeof(float));
    if (kind == 0) {
        float identity = op == 0 ? 0.0f : (op == 1 ? INFINITY : -INFINITY);
        for (uint64_t r = 0; r < results; r++) totals[r] = identity;
        fold_all(dtype, input, rank, shape, offset, strides, to, op == 0 ? FOLD_SUM : (op == 1 ? FOLD_MIN : FOLD_MAX),
                 totals, NULL);
    } else {
        for (uint64_t r = 0; r < results; r++) totals[r] = 0.0f;
        fold_all(dtype, input, rank, shape, offset, strides, to, FOLD_SUM, totals, NULL);
        for (uint64_t r = 0; r < results; r++) totals[r] = totals[r] / count;
        if (kind == 2) {
            float* means = totals;
            float* deviations = (float*)malloc((results ? results : 1) * sizeof(float));
            for (uint64_t r = 0; r < results; r++) deviations[r] = 0.0f;
            fold_all(dtype, input, rank, shape, offset, strides, to, FOLD_DEVIATION, deviations, means);
            float d = (float)(double)divisor;
            for (uint64_t r = 0; r < results; r++) totals[r] = deviations[r] / d;
            free(deviations);
        }
    }
    for (uint64_t r = 0; r < results; r++) narrow_one(dtype, out, r, totals[r]);
    free(totals);
}

typedef struct arg_ctx {
    uint32_t dtype, op;
    const void* input;
    float* best;
    uint32_t* positions;
} arg_ctx;

/* `replaces` (strided.rs:188-197): a number that beats the best so far, or
 * any number over a NaN best. */
static int replaces(uint32_t op, float x, float best) {
    if (isnan(x)) return 0;
    return isnan(best) || (op == 1 ? x < best : x > best);
}

static void arg_run(void* c, const uint64_t* starts, uint64_t len, const uint64_t* steps) {
    arg_ctx* ctx = (arg_ctx*)c;
    for (uint64_t k = 0; k < len; k++) {
        uint64_t slot = starts[1] + k * steps[1];
        float x = widen_one(ctx->dtype, ctx->input, starts[0] + k * steps[0]);
        if (replaces(ctx->op, x, ctx->best[slot])) {
            ctx->best[slot] = x;
            ctx->positions[slot] = (uint32_t)(starts[2] + k * steps[2]);
        }
    }
}

void or_arg_reduce(uint32_t dtype, const void* input, uint32_t rank, const uint64_t* shape, uint64_t offset,
                   const uint64_t* strides, uint32_t axis, uint32_t op, uint32_t* out) {
    uint64_t to[MAX_RANK], along[MAX_RANK] = {0};
    uint32_t axes[1] = {axis};
    result_strides(rank, shape, 1, axes, to);
    along[axis] = 1;
    uint64_t results = 1;
    for (uint32_t a = 0; a < rank; a++)
        if (a != axis) results *= shape[a];
    float* best = (float*)malloc((results ? results : 1) * sizeof(float));
    for (uint64_t r = 0; r < results; r++) {
        best[r] = NAN;
        out[r] = 0;
    }
    arg_ctx ctx = {dtype, op, input, best, out};
    const uint64_t* s[3] = {strides, to, along};
    uint64_t offsets[3] = {offset, 0, 0};
    for_each_run(rank, shape, 3, offsets, s, arg_run, &ctx);
    free(best);
}

/* ---- products (matrix.rs:580-745, simd_x86.rs:57-101, :1261-1327) --------- */

#define HOST_MATMUL_DISPATCH_OPS 512 /* tensors/mod.rs:167 */

static int has_avx2_fma(void) {
#if defined(__x86_64__)
    static int known = -1;
    if (known < 0) known = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
    return known;
#else
    return 0;
#endif
}

#if defined(__x86_64__)
__attribute__((target("avx2,fma"))) static void matmul_accumulate_avx(const float* a, const float* b, uint64_t m,
                                                                      uint64_t k, uint64_t n, float* out) {
    for (uint64_t i = 0; i < m; i++) {
        const uint64_t arow = i * k, orow = i * n;
        for (uint64_t p = 0; p < k; p++) {
            const float value = a[arow + p];
            const __m256 broadcast = _mm256_set1_ps(value);
            const uint64_t brow = p * n;
            uint64_t j = 0;
            for (; j + 8 <= n; j += 8) {
                __m256 rhs = _mm256_loadu_ps(b + brow + j);
                __m256 current = _mm256_loadu_ps(out + orow + j);
                _mm256_storeu_ps(out + orow + j, _mm256_fmadd_ps(broadcast, rhs, current));
            }
            for (; j < n; j++) out[orow + j] += value * b[brow + j];
        }
    }
}
#endif

/* `matmul_avx` (simd_x86.rs:1302-1327): i, p, j; each eight-lane block is one
 * FMA per element, the tail a separate multiply and add.  `fmaf` is the
 * same single rounding as `_mm256_fmadd_ps`. */
static void matmul_accumulate(const float* a, const float* b, uint64_t m, uint64_t k, uint64_t n, float* out) {
#if defined(__x86_64__)
    if (has_avx2_fma()) {
        matmul_accumulate_avx(a, b, m, k, n, out);
        return;
    }
#endif
    for (uint64_t i = 0; i < m; i++) {
        for (uint64_t p = 0; p < k; p++) {
            const float value = a[i * k + p];
            uint64_t j = 0;
            for (; j + 8 <= n; j += 8)
                for (uint64_t l = 0; l < 8; l++) out[i * n + j + l] = fmaf(value, b[p * n + j + l], out[i * n + j + l]);
            for (; j < n; j++) out[i * n + j] += value * b[p * n + j];
        }
    }
}

void or_matmul_f32(const float* a, const float* b, uint64_t m, uint64_t k, uint64_t n, float* out,
                   int accumulate) {
    if (m * k * n < HOST_MATMUL_DISPATCH_OPS) {
        if (accumulate) {
            /* matrix.rs:658-665: i, p, j onto the addend. */
            for (uint64_t i = 0; i < m; i++)
                for (uint64_t p = 0; p < k; p++)
                    for (uint64_t j = 0; j < n; j++) out[i * n + j] = out[i * n + j] + a[i * k + p] * b[p * n + j];
        } else {
            /* matrix.rs:601-609: i, j, then the sum over p from zero. */
            for (uint64_t i = 0; i < m; i++)
                for (uint64_t j = 0; j < n; j++) {
                    float sum = 0.0f;
                    for (uint64_t p = 0; p < k; p++) sum = sum + a[i * k + p] * b[p * n + j];
                    out[i * n + j] = sum;
                }
        }
        return;
    }
    if (!accumulate) memset(out, 0, m * n * sizeof(float)); /* f32k::matmul fills with zero */
    matmul_accumulate(a, b, m, k, n, out);
}

void or_matmul(uint32_t in_dtype, uint32_t out_dtype, const void* a, const void* b, uint64_t m, uint64_t k,
               uint64_t n, void* out, int accumulate) {
    if (in_dtype == F32) {
        or_matmul_f32((const float*)a, (const float*)b, m, k, n, (float*)out, accumulate);
        return;
    }
    float* wa = (float*)malloc((m * k + 1) * sizeof(float));
    float* wb = (float*)malloc((k * n + 1) * sizeof(float));
    float* wc = (float*)malloc((m * n + 1) * sizeof(float));
    or_widen(in_dtype, a, wa, m * k);
    or_widen(in_dtype, b, wb, k * n);
    if (accumulate) or_widen(out_dtype, out, wc, m * n);
    or_matmul_f32(wa, wb, m, k, n, wc, accumulate);
    or_narrow(out_dtype, wc, out, m * n);
    free(wa);
    free(wb);
    free(wc);
}

void or_transpose(uint32_t width, const void* src, uint64_t rows, uint64_t cols, void* out) {
    const uint8_t* s = (const uint8_t*)src;
    uint8_t* o = (uint8_t*)out;
    for (uint64_t j = 0; j < cols; j++)
        for (uint64_t i = 0; i < rows; i++) memcpy(o + (j * rows + i) * width, s + (i * cols + j) * width, width);
}

#if defined(__x86_64__)
__attribute__((target("avx2,fma"))) static float dot_avx(const float* a, const float* b, uint64_t n) {
    uint64_t i = 0;
    __m256 acc[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
    while (i + 32 <= n) {
        for (int lane = 0; lane < 4; lane++) {
            uint64_t offset = i + (uint64_t)lane * 8;
            acc[lane] = _mm256_fmadd_ps(_mm256_loadu_ps(a + offset), _mm256_loadu_ps(b + offset), acc[lane]);
        }
        i += 32;
    }
    __m256 total = _mm256_add_ps(_mm256_add_ps(acc[0], acc[1]), _mm256_add_ps(acc[2], acc[3]));
    float lanes[8];
    _mm256_storeu_ps(lanes, total);
    float sum = 0.0f;
    for (int l = 0; l < 8; l++) sum += lanes[l];
    while (i + 8 <= n) {
        __m256 product = _mm256_mul_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i));
        _mm256_storeu_ps(lanes, product);
        float part = 0.0f;
        for (int l = 0; l < 8; l++) part += lanes[l];
        sum += part;
        i += 8;
    }
    while (i < n) {
        sum += a[i] * b[i];
        i++;
    }
    return sum;
}
#endif

/* `f32k::dot` = `dot_avx` (simd_x86.rs:57-101), with the same association in
 * the scalar fallback. */
static float dot_simd(const float* a, const float* b, uint64_t n) {
#if defined(__x86_64__)
    if (has_avx2_fma()) return dot_avx(a, b, n);
#endif
    uint64_t i = 0;
    float acc[4][8] = {{0}};
    while (i + 32 <= n) {
        for (int lane = 0; lane < 4; lane++)
            for (int l = 0; l < 8; l++) acc[lane][l] = fmaf(a[i + lane * 8 + l], b[i + lane * 8 + l], acc[lane][l]);
        i += 32;
    }
    float sum = 0.0f;
    for (int l = 0; l < 8; l++) sum += (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
    while (i + 8 <= n) {
        float part = 0.0f;
        for (int l = 0; l < 8; l++) part += a[i + l] * b[i + l];
        sum += part;
        i += 8;
    }
    for (; i < n; i++) sum += a[i] * b[i];
    return sum;
}

/* `Vector::dot` (vector.rs:468-483): the SIMD dot from 16 elements
 * (simd_dispatch.rs:77-91), the plain loop below. */
static float dot_f32(const float* a, const float* b, uint64_t n) {
    if (n < 16) {
        float sum = 0.0f;
        for (uint64_t i = 0; i < n; i++) sum = sum + a[i] * b[i];
        return sum;
    }
    return dot_simd(a, b, n);
}

float or_dot(uint32_t dtype, const void* a, const void* b, uint64_t n) {
    if (dtype == F32) return dot_f32((const float*)a, (const float*)b, n);
    float total = 0.0f; /* compact.rs:177-179: each product exact, one rounding per term */
    for (uint64_t i = 0; i < n; i++) total = total + widen_one(dtype, a, i) * widen_one(dtype, b, i);
    return total;
}

void or_matvec(uint32_t dtype, const void* m, const void* v, uint64_t rows, uint64_t cols, void* out,
               int accumulate) {
    if (dtype != F32) {
        or_matmul(dtype, dtype, m, v, rows, cols, 1, out, accumulate);
        return;
    }
    const float* mm = (const float*)m;
    const float* vv = (const float*)v;
    float* o = (float*)out;
    int simd = rows * cols >= HOST_MATMUL_DISPATCH_OPS;
    for (uint64_t r = 0; r < rows; r++) {
        float sum;
        if (simd) {
            sum = dot_simd(mm + r * cols, vv, cols);
        } else {
            sum = 0.0f;
            for (uint64_t c = 0; c < cols; c++) sum = sum + mm[r * cols + c] * vv[c];
        }
        o[r] = accumulate ? o[r] + sum : sum;
    }
}

void or_vecmat(uint32_t dtype, const void* v, const void* m, uint64_t rows, uint64_t cols, void* out) {
    if (dtype != F32) {
        or_matmul(dtype, dtype, v, m, 1, rows, cols, out, 0);
        return;
    }
    const float* vv = (const float*)v;
    const float* mm = (const float*)m;
    float* o = (float*)out;
    if (rows * cols >= HOST_MATMUL_DISPATCH_OPS) {
        or_matmul_f32(vv, mm, 1, rows, cols, o, 0);
        return;
    }
    for (uint64_t j = 0; j < cols; j++) {
        float sum = 0.0f;
        for (uint64_t p = 0; p < rows; p++) sum = sum + vv[p] * mm[p * cols + j];
        o[j] = sum;
    }
}

/* ---- fused programs (fused/mod.rs:62-70, :3254-3268) ------------------------ */

static uint64_t place_at(const or_place* p, uint64_t row, uint64_t col) {
    uint64_t at = p->offset + col * p->col_step;
    if (p->lead > 0) {
        for (int k = (int)p->lead - 1; k > 0; k--) {
            at += (row % p->dims[k]) * p->steps[k];
            row /= p->dims[k];
        }
        at += row * p->steps[0];
    }
    return at;
}

/* `Analytic::value` (kernels.rs:334-354) in f32 libm; only `Sqrt`, which
 * is IEEE, is pinned bit for bit. */
static float analytic(uint32_t op, float x) {
    switch (op) {
        case 0: return sinf(x);
        case 1: return cosf(x);
        case 2: return tanf(x);
        case 3: return 1.0f / cosf(x);
        case 4: return 1.0f / sinf(x);
        case 5: return asinf(x);
        case 6: return acosf(x);
        case 7: return atanf(x);
        case 8: return expf(x);
        case 9: return logf(x);
        case 10: return sinhf(x);
        case 11: return coshf(x);
        case 12: return tanhf(x);
        case 13: return sqrtf(x);
        default: return NAN;
    }
}

void or_fused(uint32_t dtype, const or_encoded* code, uint32_t count, const or_place* places,
              const void* const* inputs, void* const* outputs, uint64_t rows, uint64_t cols) {
    float r[16] = {0};
    for (uint64_t row = 0; row < rows; row++) {
        for (uint64_t col = 0; col < cols; col++) {
            uint64_t element = row * cols + col;
            for (uint32_t pc = 0; pc < count; pc++) {
                const or_encoded* in = &code[pc];
                switch (in->kind) {
                    case 0:
                        r[in->dst] = in_type(dtype, widen_one(in->b, inputs[in->a], place_at(&places[in->op], row, col)));
                        break;
                    case 1: r[in->dst] = in->value; break;
                    case 2: r[in->dst] = in_type(dtype, arithmetic_value(in->op, r[in->a], r[in->b])); break;
                    case 3: r[in->dst] = in_type(dtype, analytic(in->op, r[in->a])); break;
                    case 4: r[in->dst] = in_type(dtype, compare_value(in->op, r[in->a], r[in->b])); break;
                    default: narrow_one(in->b, outputs[in->aux], element, r[in->a]); break;
                }
            }
        }
    }
}

/* ---- the composed Kernels members (kernels.rs:1090-1149) ------------------- */

static size_t elem_bytes(uint32_t dtype) { return dtype == F32 ? 4 : 2; }

void or_row_moments(uint32_t dtype, uint32_t input_dtype, const void* input, const or_place* place, uint64_t rows,
                    uint64_t cols, void* means, void* deviations) {
    float* row = (float*)malloc((cols ? cols : 1) * sizeof(float));
    for (uint64_t r = 0; r < rows; r++) {
        if (cols == 0) {
            narrow_one(dtype, means, r, NAN);
            narrow_one(dtype, deviations, r, NAN);
            continue;
        }
        for (uint64_t c = 0; c < cols; c++) row[c] = in_type(dtype, widen_one(input_dtype, input, place_at(place, r, c)));
        float total = 0.0f;
        for (uint64_t c = 0; c < cols; c++) total = total + row[c];
        const float mean = total / (float)cols;
        float squares = 0.0f;
        for (uint64_t c = 0; c < cols; c++) {
            const float d = row[c] - mean;
            squares = squares + d * d;
        }
        narrow_one(dtype, means, r, mean);
        narrow_one(dtype, deviations, r, squares);
    }
    free(row);
}

void or_fused_sum(uint32_t dtype, const or_encoded* code, uint32_t count, const or_place* places,
                  const void* const* inputs, uint64_t rows, uint64_t cols, uint32_t axis, void* out) {
    const uint64_t n = rows * cols;
    void* data = malloc((n ? n : 1) * elem_bytes(dtype));
    void* outputs[1] = {data};
    or_fused(dtype, code, count, places, inputs, outputs, rows, cols);
    const uint64_t len = axis == 0 ? cols : rows;
    void* ones = malloc((len ? len : 1) * elem_bytes(dtype));
    for (uint64_t i = 0; i < len; i++) narrow_one(dtype, ones, i, 1.0f);
    if (axis == 0) {
        or_matvec(dtype, data, ones, rows, cols, out, 0);
    } else {
        or_vecmat(dtype, ones, data, rows, cols, out);
    }
    free(ones);
    free(data);
}

void or_matmul_epilogue(uint32_t dtype, const or_encoded* code, uint32_t count, const or_place* places,
                        const void* a, const void* b, uint64_t m, uint64_t k, uint64_t n, const void* const* inputs,
                        uint32_t input_count, void* const* outputs) {
    void* product = malloc((m * n > 0 ? m * n : 1) * elem_bytes(dtype));
    or_matmul(dtype, dtype, a, b, m, k, n, product, 0);
    const void** all = (const void**)malloc((input_count + 1) * sizeof(void*));
    all[0] = product;
    for (uint32_t s = 0; s < input_count; s++) all[s + 1] = inputs[s];
    or_fused(dtype, code, count, places, all, outputs, m, n);
    free(all);
    free(product);
}

/* ---- analytic functions and powers (kernels.rs:293-385, analytic.rs:405-540) -- */

static float analytic_in(uint32_t dtype, uint32_t op, float x) {
    if (op == 3) return 1.0f / in_type(dtype, cosf(x));
    if (op == 4) return 1.0f / in_type(dtype, sinf(x));
    return analytic(op, x);
}

static float derivative_in(uint32_t dtype, uint32_t op, float x) {
#define R(v) in_type(dtype, (v))
#define VALUE(f) R(analytic_in(dtype, (f), x))
    switch (op) {
        case 0: return VALUE(1);
        case 1: return -VALUE(0);
        case 2: { float c = VALUE(1); return R(1.0f / R(c * c)); }
        case 3: { float c = VALUE(1); return R(VALUE(0) / R(c * c)); }
        case 4: { float s = VALUE(0); return R(-VALUE(1) / R(s * s)); }
        case 5: return R(1.0f / R(sqrtf(R(1.0f - R(x * x)))));
        case 6: return -R(1.0f / R(sqrtf(R(1.0f - R(x * x)))));
        case 7: return R(1.0f / R(1.0f + R(x * x)));
        case 8: return VALUE(8);
        case 9: return R(1.0f / x);
        case 10: return VALUE(11);
        case 11: return VALUE(10);
        case 12: { float t = VALUE(12); return R(1.0f - R(t * t)); }
        default: return R(1.0f / R(2.0f * VALUE(13)));
    }
#undef VALUE
#undef R
}

void or_unary(uint32_t dtype, uint32_t op, const void* a, void* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) narrow_one(dtype, out, i, analytic_in(dtype, op, widen_one(dtype, a, i)));
}

void or_unary_dual(uint32_t dtype, uint32_t op, const void* value, const void* tangent, void* out_value,
                   void* out_tangent, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) {
        const float x = widen_one(dtype, value, i);
        narrow_one(dtype, out_value, i, analytic_in(dtype, op, x));
        narrow_one(dtype, out_tangent, i, derivative_in(dtype, op, x) * widen_one(dtype, tangent, i));
    }
}

void or_power(uint32_t dtype, const void* a, const void* b, void* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) narrow_one(dtype, out, i, powf(widen_one(dtype, a, i), widen_one(dtype, b, i)));
}

void or_power_scalar(uint32_t dtype, const void* a, float scalar, int scalar_left, void* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) {
        const float x = widen_one(dtype, a, i);
        float y;
        if (scalar_left) {
            y = powf(scalar, x);
        } else if (dtype == F32 && scalar == 0.0f) {
            y = 1.0f;
        } else if (dtype == F32 && scalar == 1.0f) {
            y = x;
        } else if (dtype == F32 && scalar == 2.0f) {
            y = x * x;
        } else if (dtype == F32 && scalar == 0.5f) {
            y = x == -INFINITY ? INFINITY : sqrtf(x) + 0.0f;
        } else if (dtype == F32 && scalar == -1.0f) {
            y = 1.0f / x;
        } else {
            y = powf(x, scalar);
        }
        narrow_one(dtype, out, i, y);
    }
}

void or_moments(uint32_t dtype, const void* a, uint64_t n, float* out) {
    if (n == 0) {
        out[0] = out[1] = NAN;
        return;
    }
    float total = 0.0f;
    for (uint64_t i = 0; i < n; i++) total = total + widen_one(dtype, a, i);
    const float mean = total / (float)n;
    float squares = 0.0f;
    for (uint64_t i = 0; i < n; i++) {
        const float d = widen_one(dtype, a, i) - mean;
        squares = squares + d * d;
    }
    out[0] = mean;
    out[1] = squares;
}

/* ---- correlation, padding, flipping (kernels.rs:1514-1600, :1720-1794) ------ */

void or_correlate(uint32_t dtype, const void* input, uint64_t rows, uint64_t cols, const void* window,
                  uint64_t window_rows, uint64_t window_cols, int flip, void* out) {
    const uint64_t out_rows = rows - window_rows + 1, out_cols = cols - window_cols + 1;
    for (uint64_t row = 0; row < out_rows; row++) {
        for (uint64_t col = 0; col < out_cols; col++) {
            float sum = 0.0f;
            for (uint64_t i = 0; i < window_rows; i++) {
                for (uint64_t j = 0; j < window_cols; j++) {
                    const uint64_t tap_row = flip ? window_rows - 1 - i : i;
                    const uint64_t tap_col = flip ? window_cols - 1 - j : j;
                    sum = sum + widen_one(dtype, input, (row + i) * cols + col + j) *
                                    widen_one(dtype, window, tap_row * window_cols + tap_col);
                }
            }
            narrow_one(dtype, out, row * out_cols + col, sum);
        }
    }
}

void or_correlate_input_gradient(uint32_t dtype, const void* adjoint, uint64_t adjoint_rows, uint64_t adjoint_cols,
                                 const void* window, uint64_t window_rows, uint64_t window_cols, int forward_flip,
                                 void* out) {
    const uint64_t rows = adjoint_rows + window_rows - 1, cols = adjoint_cols + window_cols - 1;
    for (uint64_t row = 0; row < rows; row++) {
        for (uint64_t col = 0; col < cols; col++) {
            float sum = 0.0f;
            for (uint64_t i = 0; i < window_rows; i++) {
                for (uint64_t j = 0; j < window_cols; j++) {
                    if (row < i || col < j) continue;
                    const uint64_t source_row = row - i, source_col = col - j;
                    if (source_row >= adjoint_rows || source_col >= adjoint_cols) continue;
                    const uint64_t tap_row = forward_flip ? window_rows - 1 - i : i;
                    const uint64_t tap_col = forward_flip ? window_cols - 1 - j : j;
                    sum = sum + widen_one(dtype, adjoint, source_row * adjoint_cols + source_col) *
                                    widen_one(dtype, window, tap_row * window_cols + tap_col);
                }
            }
            narrow_one(dtype, out, row * cols + col, sum);
        }
    }
}

void or_pad(uint32_t width, const void* input, uint64_t rows, uint64_t cols, uint64_t pad_rows, uint64_t pad_cols,
            void* out) {
    const uint64_t padded_rows = rows + 2 * pad_rows, padded_cols = cols + 2 * pad_cols;
    const uint8_t* in = (const uint8_t*)input;
    uint8_t* o = (uint8_t*)out;
    for (uint64_t row = 0; row < padded_rows; row++) {
        for (uint64_t col = 0; col < padded_cols; col++) {
            const int inside = row >= pad_rows && row < pad_rows + rows && col >= pad_cols && col < pad_cols + cols;
            uint8_t* at = o + (row * padded_cols + col) * width;
            if (inside) {
                memcpy(at, in + ((row - pad_rows) * cols + col - pad_cols) * width, width);
            } else {
                memset(at, 0, width);
            }
        }
    }
}

void or_flip(uint32_t width, const void* input, uint64_t rows, uint64_t cols, void* out) {
    const uint8_t* in = (const uint8_t*)input;
    uint8_t* o = (uint8_t*)out;
    for (uint64_t row = 0; row < rows; row++) {
        for (uint64_t col = 0; col < cols; col++) {
            memcpy(o + (row * cols + col) * width, in + ((rows - 1 - row) * cols + cols - 1 - col) * width, width);
        }
    }
}

/* ---- scans and sorts ----------------------------------------------------- */

/* compact.rs:209-221 (the Host `Vector::prefix_sum`, vector.rs:578-589, for
 * the three element types here): an inclusive running total kept in f32,
 * left to right, each output rounded to the element type once. */
void or_prefix_sum(uint32_t dtype, const void* a, uint64_t n, void* out) {
    float running = 0.0f;
    for (uint64_t i = 0; i < n; i++) {
        running += widen_one(dtype, a, i);
        narrow_one(dtype, out, i, running);
    }
}

/* IEEE totalOrder on raw bit patterns of `bits` width (`total_cmp`,
 * numbers/primitive.rs:70-72 via SortOrder::comparator, kernels.rs:259-266),
 * from its definition: a set sign bit orders first; among two non-negative
 * patterns the larger magnitude is larger; among two negative ones the larger
 * magnitude is smaller.  NaNs sit beyond the infinities by sign and payload. */
static int total_order(uint32_t x, uint32_t y, uint32_t bits) {
    const uint32_t sign = 1u << (bits - 1);
    const int nx = (x & sign) != 0, ny = (y & sign) != 0;
    if (nx != ny) return nx ? -1 : 1;
    const uint32_t mx = x & (sign - 1), my = y & (sign - 1);
    if (mx == my) return 0;
    if (nx) return mx > my ? -1 : 1;
    return mx < my ? -1 : 1;
}

static int ascending32(const void* l, const void* r) {
    return total_order(*(const uint32_t*)l, *(const uint32_t*)r, 32);
}
static int ascending16(const void* l, const void* r) {
    return total_order(*(const uint16_t*)l, *(const uint16_t*)r, 16);
}

/* vector.rs:874-884 (`sort` / `sorted`): sort_unstable_by the order's
 * comparator.  Elements equal under totalOrder are the same bit pattern, so
 * an unstable sort fixes the output; descending is the ascending output
 * reversed. */
void or_sort(uint32_t dtype, const void* a, uint64_t n, uint32_t order, void* out) {
    const size_t width = dtype == F32 ? 4 : 2;
    memcpy(out, a, n * width);
    qsort(out, n, width, width == 4 ? ascending32 : ascending16);
    if (order == 1) {
        uint8_t* o = (uint8_t*)out;
        uint8_t tmp[4];
        for (uint64_t i = 0, j = n ? n - 1 : 0; i < j; i++, j--) {
            memcpy(tmp, o + i * width, width);
            memcpy(o + i * width, o + j * width, width);
            memcpy(o + j * width, tmp, width);
        }
    }
}

/* ---- distributions ------------------------------------------------------- */

/* statistics/special.rs: every function in f64.  Cody's error function
 * (special.rs:48-200, coefficient tables :101-113, :145-180) and Wichura's
 * AS 241 quantile (:242-330), restated from the publications in the order the
 * reference evaluates them. */

static const double CODY_A[5] = {3.16112374387056560e00, 1.13864154151050156e02, 3.77485237685302021e02,
                                 3.20937758913846947e03, 1.85777706184603153e-1};
static const double CODY_B[4] = {2.36012909523441209e01, 2.44024637934444173e02, 1.28261652607737228e03,
                                 2.84423683343917062e03};
static const double CODY_C[9] = {5.64188496988670089e-1, 8.88314979438837594e00, 6.61191906371416295e01,
                                 2.98635138197400131e02, 8.81952221241769090e02, 1.71204761263407058e03,
                                 2.05107837782607147e03, 1.23033935479799725e03, 2.15311535474403846e-8};
static const double CODY_D[8] = {1.57449261107098347e01, 1.17693950891312499e02, 5.37181101862009858e02,
                                 1.62138957456669019e03, 3.29079923573345963e03, 4.36261909014324716e03,
                                 3.43936767414372164e03, 1.23033935480374942e03};
static const double CODY_P[6] = {3.05326634961232344e-1, 3.60344899949804439e-1, 1.25781726111229246e-1,
                                 1.60837851487422766e-2, 6.58749161529837803e-4, 1.63153871373020978e-2};
static const double CODY_Q[5] = {2.56852019228982242e00, 1.87295284992346047e00, 5.27905102951428412e-1,
                                 6.05183413124413191e-2, 2.33520497626869185e-3};
static const double PPND_A[8] = {3.3871328727963666080e0, 1.3314166789178437745e2, 1.9715909503065514427e3,
                                 1.3731693765509461125e4, 4.5921953931549871457e4, 6.7265770927008700853e4,
                                 3.3430575583588128105e4, 2.5090809287301226727e3};
static const double PPND_B[7] = {4.2313330701600911252e1, 6.8718700749205790830e2, 5.3941960214247511077e3,
                                 2.1213794301586595867e4, 3.9307895800092710610e4, 2.8729085735721942674e4,
                                 5.2264952788528545610e3};
static const double PPND_C[8] = {1.42343711074968357734e0, 4.63033784615654529590e0, 5.76949722146069140550e0,
                                 3.64784832476320460504e0, 1.27045825245236838258e0, 2.41780725177450611770e-1,
                                 2.27238449892691845833e-2, 7.74545014278341407640e-4};
static const double PPND_D[7] = {2.05319162663775882187e0, 1.67638483018380384940e0, 6.89767334985100004550e-1,
                                 1.48103976427480074590e-1, 1.51986665636164571966e-2, 5.47593808499534494600e-4,
                                 1.05075007164441684324e-9};
static const double PPND_E[8] = {6.65790464350110377720e0, 5.46378491116411436990e0, 1.78482653991729133580e0,
                                 2.96560571828504891230e-1, 2.65321895265761230930e-2, 1.24266094738807843860e-3,
                                 2.71155556874348757815e-5, 2.01033439929228813265e-7};
static const double PPND_F[7] = {5.99832206555887937690e-1, 1.36929880922735805310e-1, 1.48753612908506148525e-2,
                                 7.86869131145613259100e-4, 1.84631831751005468180e-5, 1.42151175831644588870e-7,
                                 2.04426310338993978564e-15};

/* special.rs:339-345: Horner from the constant term's end, starting at 0. */
static double poly(const double* c, int n, double x) {
    double total = 0.0;
    for (int i = n - 1; i >= 0; i--) total = total * x + c[i];
    return total;
}

/* special.rs:100-122 */
static double erf_central(double x) {
    double z = x * x, top = CODY_A[4] * z, bottom = z;
    for (int i = 0; i < 3; i++) {
        top = (top + CODY_A[i]) * z;
        bottom = (bottom + CODY_B[i]) * z;
    }
    return x * (top + CODY_A[3]) / (bottom + CODY_B[3]);
}

/* special.rs:144-200 */
static double erfc_scaled(double x) {
    if (x <= 4.0) {
        double top = CODY_C[8] * x, bottom = x;
        for (int i = 0; i < 7; i++) {
            top = (top + CODY_C[i]) * x;
            bottom = (bottom + CODY_D[i]) * x;
        }
        return (top + CODY_C[7]) / (bottom + CODY_D[7]);
    }
    double z = 1.0 / (x * x), top = CODY_P[5] * z, bottom = z;
    for (int i = 0; i < 4; i++) {
        top = (top + CODY_P[i]) * z;
        bottom = (bottom + CODY_Q[i]) * z;
    }
    double correction = z * (top + CODY_P[4]) / (bottom + CODY_Q[4]);
    return (0.5641895835477563 - correction) / x;
}

/* special.rs:133-140 */
static double erfc_positive(double x) {
    if (x > 27.25) return 0.0;
    double leading = trunc(x * 16.0) / 16.0;
    double correction = (x - leading) * (x + leading);
    return exp(-leading * leading) * exp(-correction) * erfc_scaled(x);
}

/* special.rs:48-60 */
double or_erf(double x) {
    if (isnan(x)) return x;
    if (fabs(x) <= 0.46875) return erf_central(x);
    double complement = 1.0 - erfc_positive(fabs(x));
    return x < 0.0 ? -complement : complement;
}

/* special.rs:64-79 */
double or_erfc(double x) {
    if (isnan(x)) return x;
    if (x < -0.46875) return 2.0 - erfc_positive(-x);
    if (x <= 0.46875) return 1.0 - erf_central(x);
    return erfc_positive(x);
}

/* special.rs:88-96 */
static double ln_erfc(double x) {
    if (isnan(x)) return x;
    if (x <= 0.46875) return log(or_erfc(x));
    return log(erfc_scaled(x)) - x * x;
}

/* special.rs:216-236 */
static double std_pdf(double z) { return exp(-0.5 * z * z) / 2.5066282746310002; }
static double std_cdf(double z) { return 0.5 * or_erfc(-z * 0.7071067811865476); }
static double std_ln_cdf(double z) { return ln_erfc(-z * 0.7071067811865476) - 0.6931471805599453; }

/* special.rs:242-331 */
double or_normal_quantile(double p) {
    if (isnan(p) || p < 0.0 || p > 1.0) return NAN;
    if (p == 0.0) return -INFINITY;
    if (p == 1.0) return INFINITY;
    double q = p - 0.5;
    if (fabs(q) <= 0.425) {
        double r = 0.180625 - q * q;
        return q * poly(PPND_A, 8, r) / (poly(PPND_B, 7, r) * r + 1.0);
    }
    double r = sqrt(-log(q < 0.0 ? p : 1.0 - p)), value;
    if (r <= 5.0) {
        r = r - 1.6;
        value = poly(PPND_C, 8, r) / (poly(PPND_D, 7, r) * r + 1.0);
    } else {
        r = r - 5.0;
        value = poly(PPND_E, 8, r) / (poly(PPND_F, 7, r) * r + 1.0);
    }
    return q < 0.0 ? -value : value;
}

/* special.rs:378-390 */
static double wald_pdf(double x, double mean, double shape) {
    if (x <= 0.0) return 0.0;
    double deviation = x - mean;
    double exponent = -shape * deviation * deviation / (2.0 * mean * mean * x);
    return sqrt(shape / (2.0 * 3.141592653589793 * x * x * x)) * exp(exponent);
}

/* special.rs:397-410: Rust's f64::min returns the number when the sum is NaN,
 * as fmin does. */
static double wald_cdf(double x, double mean, double shape) {
    if (x <= 0.0) return 0.0;
    double scale = sqrt(shape / x), ratio = x / mean;
    double lower = scale * (ratio - 1.0), upper = scale * (ratio + 1.0);
    double tail = 2.0 * shape / mean + std_ln_cdf(-upper);
    return fmin(std_cdf(lower) + exp(tail), 1.0);
}

/* special.rs:420-476 */
static double wald_ppf(double p, double mean, double shape) {
    if (isnan(p) || p < 0.0 || p > 1.0) return NAN;
    if (p == 0.0) return 0.0;
    if (p == 1.0) return INFINITY;
    double low = 0.0, high = mean;
    while (wald_cdf(high, mean, shape) < p) {
        low = high;
        high *= 2.0;
        if (isinf(high)) return INFINITY;
    }
    double guess = 0.5 * (low + high);
    for (int pass = 0; pass < 60; pass++) {
        double error = wald_cdf(guess, mean, shape) - p;
        if (error > 0.0) high = guess; else low = guess;
        double density = wald_pdf(guess, mean, shape);
        double step = density > 0.0 ? guess - error / density : NAN;
        double next = (isfinite(step) && step > low && step < high) ? step : 0.5 * (low + high);
        if (next == guess) break;
        guess = next;
    }
    return guess;
}

/* `Distribution::evaluate` (statistics/mod.rs:273-297) with the family and
 * statistic as codes: special.rs:348-370 for the normal, :378-476 for the
 * inverse Gaussian, each guarded by its parameter checks (:334-336). */
double or_evaluate(uint32_t family, uint32_t statistic, double x, double first, double second) {
    if (family == 0) {
        if (isnan(second) || second <= 0.0) return NAN;
        if (statistic == 0) return std_pdf((x - first) / second) / second;
        if (statistic == 1) return std_cdf((x - first) / second);
        return first + second * or_normal_quantile(x);
    }
    if (!(first > 0.0) || !(second > 0.0)) return NAN;
    if (statistic == 0) return wald_pdf(x, first, second);
    if (statistic == 1) return wald_cdf(x, first, second);
    return wald_ppf(x, first, second);
}

/* statistics/mod.rs:274-297's `cast` (`T::from`, half 2.7.1's `NumCast`
 * for f16/bf16 converts through f32): f64 to f32 by round-to-nearest-even,
 * then to the type. */
static void store_double(uint32_t dtype, void* out, uint64_t i, double v) {
    narrow_one(dtype, out, i, (float)v);
}

/* statistics/mod.rs:649-651 (`map` of `evaluate`). */
void or_distribution(uint32_t dtype, uint32_t family, uint32_t statistic, const void* a, void* out, uint64_t n,
                     float first, float second) {
    for (uint64_t i = 0; i < n; i++) {
        store_double(dtype, out, i, or_evaluate(family, statistic, widen_one(dtype, a, i), first, second));
    }
}

/* statistics/mod.rs:582-600: element i takes the pair of its row
 * (i / cols, `axis` 0) or column (i % cols, `axis` 1). */
void or_axis_distribution(uint32_t dtype, uint32_t family, uint32_t statistic, const void* a, uint64_t rows,
                          uint64_t cols, uint32_t axis, const void* first, const void* second, void* out) {
    for (uint64_t i = 0; i < rows * cols; i++) {
        uint64_t along = axis == 0 ? i / cols : i % cols;
        double x = widen_one(dtype, a, i);
        store_double(dtype, out, i,
                     or_evaluate(family, statistic, x, widen_one(dtype, first, along), widen_one(dtype, second, along)));
    }
}
