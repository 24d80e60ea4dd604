/*
 * CPU restatement of tensorcrate's Host backend for the Hip backend's hot
 * path: TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it, as the checker or the timed CPU
 * baseline; the product never calls it.  Every function names the reference
 * file:line it restates (paths under arthurmburke/tensorcrate's src/).
 *
 * Conventions match include/tchip.h: element counts and strides in
 * elements, dtype codes of `fused::DType`, op codes of the reference enums.
 */
#ifndef TC_ORACLE_H
#define TC_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* f32 -> bf16 / f16 bits, round to nearest even with NaNs quieted
 * (`half::bf16::from_f32`, `half::f16::from_f32`, half 2.7.1, as called at
 * compact.rs:40-57), and f16 bits -> f32 (exact). */
uint16_t or_bf16_from_f32(float value);
uint16_t or_f16_from_f32(float value);
float or_f16_to_f32(uint16_t bits);
void or_narrow(uint32_t dtype, const float* in, void* out, uint64_t n);
void or_widen(uint32_t dtype, const void* in, float* out, uint64_t n);

/* `Backend::strided_copy` on Host (backend.rs:255-274) over `coalesce` and
 * `for_each_run` (layout.rs:419-498).  Returns the element count. */
uint64_t or_strided_copy(uint32_t width, const void* src, uint32_t rank, const uint64_t* shape,
                         uint64_t offset, const uint64_t* strides, void* out);

/* `strided_write_slice` (backend.rs:277-300). */
void or_strided_write(uint32_t width, const void* src, void* target, uint32_t rank, const uint64_t* shape,
                      uint64_t from_offset, const uint64_t* from_strides, uint64_t to_offset,
                      const uint64_t* to_strides);

/* `strided::binary` (strided.rs:29-78) with `Pairwise::value`
 * (kernels.rs:431-441): kind 0 arithmetic, 1 compare, 2 power. */
void or_binary(uint32_t dtype, uint32_t kind, uint32_t op, uint32_t rank, const uint64_t* shape,
               const void* a, uint64_t a_offset, const uint64_t* a_strides, const void* b, uint64_t b_offset,
               const uint64_t* b_strides, void* out);

/* Same-shape elementwise ops (kernels.rs:1193-1240): a op b, a op s or s op a,
 * compare, compare_scalar, clamp. */
void or_elementwise(uint32_t dtype, uint32_t kind, uint32_t op, const void* a, const void* b, void* out,
                    uint64_t n);
void or_scalar(uint32_t dtype, uint32_t kind, uint32_t op, const void* a, float scalar, int scalar_left,
               void* out, uint64_t n);
void or_clamp(uint32_t dtype, const void* a, float low, float high, void* out, uint64_t n);

/* `strided::reduce` / `reduce_in` / `fold` (strided.rs:80-184): the input's
 * `rank`-axis layout folded over the ascending `axes`; kind 0 fold (op a
 * Reduce), 1 mean, 2 variance with `divisor`. */
void or_reduce(uint32_t dtype, const void* input, uint32_t rank, const uint64_t* shape, uint64_t offset,
               const uint64_t* strides, uint32_t naxes, const uint32_t* axes, uint32_t kind, uint32_t op,
               uint64_t divisor, void* out);

/* `strided::arg_reduce` and `replaces` (strided.rs:186-225). */
void or_arg_reduce(uint32_t dtype, const void* input, uint32_t rank, const uint64_t* shape, uint64_t offset,
                   const uint64_t* strides, uint32_t axis, uint32_t op, uint32_t* out);

/* `Matrix::matmul` / `matmul_add` on Host for f32 (matrix.rs:580-667 over
 * simd_dispatch.rs:558-620 and simd_x86.rs:1261-1327): the i-p-j loop, FMA
 * on eight-lane blocks and a separate multiply and add on the tail, behind
 * the 512-operation gate of tensors/mod.rs:167.  `accumulate` starts from
 * `out` as the addend. */
void or_matmul_f32(const float* a, const float* b, uint64_t m, uint64_t k, uint64_t n, float* out,
                   int accumulate);

/* `compact::matmul` (compact.rs:232-253): widen, f32 product, narrow once.
 * `out_dtype` may be F32 for `matmul_f32`. */
void or_matmul(uint32_t in_dtype, uint32_t out_dtype, const void* a, const void* b, uint64_t m, uint64_t k,
               uint64_t n, void* out, int accumulate);

/* `Matrix::transpose` (matrix.rs:740, :1173-1206). */
void or_transpose(uint32_t width, const void* src, uint64_t rows, uint64_t cols, void* out);

/* `f32k::dot` (simd_x86.rs:57-101) and the compact `dot` (compact.rs:162-180);
 * the f32 result, rounded to dtype by the caller. */
float or_dot(uint32_t dtype, const void* a, const void* b, uint64_t n);

/* `Matrix::matvec` / `matvec_add` (matrix.rs:675-737, simd_dispatch.rs:626-695)
 * and `Vector::vecmat` (vector.rs:491-514, simd_dispatch.rs:698-710). */
void or_matvec(uint32_t dtype, const void* m, const void* v, uint64_t rows, uint64_t cols, void* out,
               int accumulate);
void or_vecmat(uint32_t dtype, const void* v, const void* m, uint64_t rows, uint64_t cols, void* out);

/* One instruction of a fused program (`Encoded`, fused/mod.rs:1402-1410). */
typedef struct or_encoded {
    uint16_t kind;
    uint16_t op;
    uint8_t dst;
    uint8_t a;
    uint8_t b;
    uint8_t aux;
    float value;
} or_encoded;

/* Where element (row, col) reads a load (`Place`, fused/mod.rs:3229-3268). */
typedef struct or_place {
    uint64_t offset;
    uint64_t col_step;
    uint32_t lead;
    uint64_t dims[5];
    uint64_t steps[5];
} or_place;

/* The host interpreter's semantics (fused/mod.rs:62-70, :4055): for every
 * element of the rows x cols space, each instruction in order, in dtype T. */
void or_fused(uint32_t dtype, const or_encoded* code, uint32_t count, const or_place* places,
              const void* const* inputs, void* const* outputs, uint64_t rows, uint64_t cols);

/* `Analytic::value` applied to dtype elements as the host does
 * (vmath.rs:483-507), in f32 libm: the value rounded once; f16/bf16 `Sec`
 * and `Csc` the reciprocal in dtype of the rounded cosine or sine. */
void or_unary(uint32_t dtype, uint32_t op, const void* a, void* out, uint64_t n);

/* `(f(x), f'(x) * t)`, `Analytic::derivative` (kernels.rs:358-385) with one
 * rounding to dtype per operation (`vector_unary_dual`, kernels.rs:1284-1300). */
void or_unary_dual(uint32_t dtype, uint32_t op, const void* value, const void* tangent, void* out_value,
                   void* out_tangent, uint64_t n);

/* `powf` in f32 rounded once (primitive.rs:133-150), elementwise or with a
 * scalar on either side; `x^s` takes the f32 fast exponents
 * (analytic.rs:415-476). */
void or_power(uint32_t dtype, const void* a, const void* b, void* out, uint64_t n);
void or_power_scalar(uint32_t dtype, const void* a, float scalar, int scalar_left, void* out, uint64_t n);

/* `Kernels::row_moments` on the Host (`host_row_moments`, fused/mod.rs:
 * 4030-4041): the rows x cols matrix `place` reads of `input`, converted to
 * dtype (`input_matrix`, :3984-3991), and per row `moments_of`
 * (statistics/mod.rs:419-441): mean = sum / n, then the sum of squared
 * deviations from it, both sequential f32 folds (the compact types widen to
 * f32 and round the two results once); NaNs for an empty row. */
void or_row_moments(uint32_t dtype, uint32_t input_dtype, const void* input, const or_place* place, uint64_t rows,
                    uint64_t cols, void* means, void* deviations);

/* `vector_moments` / `matrix_moments` on the Host (`moments_of`,
 * statistics/mod.rs:419-441): out[0] the mean, out[1] the sum of squared
 * deviations, sequential f32 folds; NaNs for no elements. */
void or_moments(uint32_t dtype, const void* a, uint64_t n, float* out);

/* `correlate_values` (kernels.rs:1720-1750) and
 * `correlate_input_gradient_values` (:1754-1794), f32 accumulation for the
 * compact types rounded once (:1523-1527); `pad` (:1575-1600) and `flip`
 * (:1531-1542) over `width`-byte elements. */
void or_correlate(uint32_t dtype, const void* input, uint64_t rows, uint64_t cols, const void* window,
                  uint64_t window_rows, uint64_t window_cols, int flip, void* out);
void or_correlate_input_gradient(uint32_t dtype, const void* adjoint, uint64_t adjoint_rows, uint64_t adjoint_cols,
                                 const void* window, uint64_t window_rows, uint64_t window_cols, int forward_flip,
                                 void* out);
void or_pad(uint32_t width, const void* input, uint64_t rows, uint64_t cols, uint64_t pad_rows, uint64_t pad_cols,
            void* out);
void or_flip(uint32_t width, const void* input, uint64_t rows, uint64_t cols, void* out);

/* The inclusive prefix sum, f32 running total rounded per output
 * (compact.rs:209-221), and the sort in IEEE totalOrder, `order` 0
 * ascending or 1 descending (vector.rs:874-884, kernels.rs:252-267). */
void or_prefix_sum(uint32_t dtype, const void* a, uint64_t n, void* out);
void or_sort(uint32_t dtype, const void* a, uint64_t n, uint32_t order, void* out);

/* The Host's special functions in f64 (statistics/special.rs) and the
 * distribution members over them (statistics/mod.rs:273-297, :582-600,
 * :649-651): `family` 0 normal (mean, stddev), 1 inverse Gaussian (mean,
 * shape); `statistic` 0 pdf, 1 cdf, 2 ppf; results rounded to f32, then to
 * `dtype`. */
double or_erf(double x);
double or_erfc(double x);
double or_normal_quantile(double p);
double or_evaluate(uint32_t family, uint32_t statistic, double x, double first, double second);
void or_distribution(uint32_t dtype, uint32_t family, uint32_t statistic, const void* a, void* out, uint64_t n,
                     float first, float second);
void or_axis_distribution(uint32_t dtype, uint32_t family, uint32_t statistic, const void* a, uint64_t rows,
                          uint64_t cols, uint32_t axis, const void* first, const void* second, void* out);

/* `Kernels::fused_sum`'s default (kernels.rs:1120-1135): the program's one
 * output, then `axis_sum` (fused/mod.rs:4045-4051), its products with ones:
 * axis 0 (Rows) a matvec, axis 1 (Columns) a vecmat. */
void or_fused_sum(uint32_t dtype, const or_encoded* code, uint32_t count, const or_place* places,
                  const void* const* inputs, uint64_t rows, uint64_t cols, uint32_t axis, void* out);

/* `host_matmul` (fused/mod.rs:4754-4766): the product, then the interpreter
 * with it as input 0 and `inputs` (count `input_count`) from slot 1. */
void or_matmul_epilogue(uint32_t dtype, const or_encoded* code, uint32_t count, const or_place* places,
                        const void* a, const void* b, uint64_t m, uint64_t k, uint64_t n, const void* const* inputs,
                        uint32_t input_count, void* const* outputs);

#ifdef __cplusplus
}
#endif

#endif
