// The scalar arithmetic every kernel shares, and the source the fused-program
// compiler embeds in each kernel it generates at run time, so that compiled
// and interpreted programs compute with the very same functions.  It includes
// nothing: the runtime compiler has no C library headers.
//
// Operation codes are the reference's stable u16 values (`BinaryOp`,
// `Compare`, `Analytic`, `fused::DType`, tensors/kernels.rs:30-354,
// fused/mod.rs:145-150); common.hpp checks them against include/tchip.h.
#pragma once

namespace tc_ops {
enum : unsigned { ADD = 0, SUB = 1, MUL = 2, DIV = 3, REM = 4 };
enum : unsigned { MIN = 0, MAX = 1, MAX_SHARE = 2, LESS = 3, LESS_EQUAL = 4, GREATER = 5, GREATER_EQUAL = 6 };
enum : unsigned { F32 = 0, F16 = 1, BF16 = 2 };
enum : unsigned { SQRT = 13 };
}  // namespace tc_ops

// bf16 is the top half of an f32, so widening is a shift.
__host__ __device__ inline float tc_bf16_to_f32(unsigned short bits) {
    return __builtin_bit_cast(float, static_cast<unsigned>(bits) << 16);
}

// Round to nearest, ties to even, with NaNs quieted: the rule of
// `half::bf16::from_f32` that the reference narrows with.  Adding 0x7fff plus
// the kept half's lowest bit carries into the kept half exactly when the
// dropped half is above one half, or exactly one half with an odd kept half.
// On the device, gfx950's conversion instruction (v_cvt_pk_bf16_f32) is this
// rule exactly: run over every one of the 2^32 f32 bit patterns on MI355X it
// gave the bits below for all of them, NaN payloads included.
__host__ __device__ inline unsigned short tc_f32_to_bf16(float value) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_bit_cast(unsigned short, static_cast<__bf16>(value));
#else
    const unsigned x = __builtin_bit_cast(unsigned, value);
    const unsigned rounded = (x + 0x7fffu + ((x >> 16) & 1u)) >> 16;
    const unsigned quiet = (x >> 16) | 0x0040u;
    return static_cast<unsigned short>((x & 0x7fffffffu) > 0x7f800000u ? quiet : rounded);
#endif
}

// `BinaryOp` in f32 (kernels.rs:431-437); the caller rounds once.  `Rem` is
// Rust's `%`, the truncated remainder `fmod`, which is exact.
__device__ inline float tc_binary(unsigned op, float a, float b) {
    switch (op) {
        case tc_ops::ADD: return a + b;
        case tc_ops::SUB: return a - b;
        case tc_ops::MUL: return a * b;
        case tc_ops::DIV: return a / b;
        default: return fmodf(a, b);
    }
}

// `Compare::value` (kernels.rs:138-153): minNum/maxNum, the ½-at-ties share,
// and predicates that are false on NaN.
__device__ inline float tc_compare(unsigned op, float a, float b) {
    switch (op) {
        case tc_ops::MIN: return fminf(a, b);
        case tc_ops::MAX: return fmaxf(a, b);
        case tc_ops::MAX_SHARE: return a > b ? 1.0f : (a < b ? 0.0f : 0.5f);
        case tc_ops::LESS: return a < b ? 1.0f : 0.0f;
        case tc_ops::LESS_EQUAL: return a <= b ? 1.0f : 0.0f;
        case tc_ops::GREATER: return a > b ? 1.0f : 0.0f;
        default: return a >= b ? 1.0f : 0.0f;
    }
}

// `Analytic::value` (kernels.rs:334-354) in f32; the caller rounds once.
__device__ inline float tc_analytic(unsigned op, float x) {
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
        default: return __builtin_nanf("");
    }
}

// An f32 value rounded to the program type T and back.
template <int T>
__device__ inline float tc_round(float v) {
    if (T == tc_ops::F16) return static_cast<float>(static_cast<_Float16>(v));
    if (T == tc_ops::BF16) return tc_bf16_to_f32(tc_f32_to_bf16(v));
    return v;
}

// Each element of `v` rounded as tc_round<T> rounds it.  bf16 rounds two at
// a time: gfx950's pair conversion (v_cvt_pk_bf16_f32, the same rule as the
// one-value conversion) and one shift or mask each back to f32.
template <int T, int E>
__device__ inline void tc_round_run(float (&v)[E]) {
    if constexpr (T == tc_ops::BF16) {
        typedef float pair_f32 __attribute__((ext_vector_type(2)));
        typedef __bf16 pair_bf16 __attribute__((ext_vector_type(2)));
        int e = 0;
        for (; e + 1 < E; e += 2) {
            const unsigned w = __builtin_bit_cast(unsigned, __builtin_convertvector(pair_f32{v[e], v[e + 1]}, pair_bf16));
            v[e] = __uint_as_float(w << 16);
            v[e + 1] = __uint_as_float(w & 0xffff0000u);
        }
        if (e < E) v[e] = tc_round<T>(v[e]);
    } else if constexpr (T == tc_ops::F16) {
        for (int e = 0; e < E; e++) v[e] = tc_round<T>(v[e]);
    }
}
