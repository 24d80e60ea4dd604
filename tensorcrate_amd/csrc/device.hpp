// The device-side element types and operand addressing shared by the
// library's kernels and the kernels the runtime compiler builds from
// generated source (fused programs, product epilogues).  It includes only
// scalar_ops.h, so hiprtc can read it as it is.
#pragma once

#if defined(__HIPCC_RTC__)
using __hip_internal::uint16_t;
using __hip_internal::uint32_t;
using __hip_internal::uint64_t;
using __hip_internal::uint8_t;
#else
#include <hip/hip_runtime.h>
#include <stdint.h>
#endif

#include "scalar_ops.h"

namespace tc {

__host__ __device__ inline float bf16_bits_to_f32(uint16_t bits) { return tc_bf16_to_f32(bits); }
__host__ __device__ inline uint16_t f32_to_bf16_bits(float value) { return tc_f32_to_bf16(value); }

struct bf16_t {
    uint16_t bits;
};

// How a storage type widens to the f32 the kernels compute in, and rounds
// back once.  f32 is the identity; f16 uses the hardware conversion, which
// rounds to nearest even.
template <typename S>
struct Elem;

template <>
struct Elem<float> {
    static constexpr int dtype = tc_ops::F32;
    __device__ static float widen(float v) { return v; }
    __device__ static float narrow(float v) { return v; }
};

template <>
struct Elem<_Float16> {
    static constexpr int dtype = tc_ops::F16;
    __device__ static float widen(_Float16 v) { return static_cast<float>(v); }
    __device__ static _Float16 narrow(float v) { return static_cast<_Float16>(v); }
};

template <>
struct Elem<bf16_t> {
    static constexpr int dtype = tc_ops::BF16;
    __device__ static float widen(bf16_t v) { return bf16_bits_to_f32(v.bits); }
    __device__ static bf16_t narrow(float v) { return bf16_t{f32_to_bf16_bits(v)}; }
};

// ---- fused-program operands ---------------------------------------------------

constexpr int kPlaceLead = 5;  // a place's folded row axes (TC_FUSED_LEAD)

// The consecutive columns of one row a product epilogue's run form (`run`)
// takes at a time: 16 bytes of a 16-bit C.
constexpr int kEpilogueRun = 8;

// A load's place in device form (`Place`, fused/mod.rs:3230-3268): element
// (row, col) reads offset + col * col_step plus the row index spread over
// up to five folded axes.
struct DevicePlace {
    uint64_t offset;
    uint64_t col_step;
    uint32_t lead;
    uint32_t pad;
    uint64_t dims[kPlaceLead];
    uint64_t steps[kPlaceLead];
};

// The storage element element (row, col) reads through `place`
// (fused/mod.rs:3254-3268).
__device__ __forceinline__ uint64_t place_at(const DevicePlace& p, uint64_t row, uint64_t col) {
    uint64_t at = p.offset + col * p.col_step;
    if (p.lead == 1) return at + row * p.steps[0];
    if (p.lead > 1) {
        for (int k = static_cast<int>(p.lead) - 1; k > 0; k--) {
            at += (row % p.dims[k]) * p.steps[k];
            row /= p.dims[k];
        }
        at += row * p.steps[0];
    }
    return at;
}

__device__ __forceinline__ float load_as(const void* base, uint32_t dtype, uint64_t index) {
    switch (dtype) {
        case tc_ops::F16: return static_cast<float>(static_cast<const _Float16*>(base)[index]);
        case tc_ops::BF16: return bf16_bits_to_f32(static_cast<const uint16_t*>(base)[index]);
        default: return static_cast<const float*>(base)[index];
    }
}

__device__ __forceinline__ void store_as(void* base, uint32_t dtype, uint64_t index, float v) {
    switch (dtype) {
        case tc_ops::F16: static_cast<_Float16*>(base)[index] = static_cast<_Float16>(v); break;
        case tc_ops::BF16: static_cast<uint16_t*>(base)[index] = f32_to_bf16_bits(v); break;
        default: static_cast<float*>(base)[index] = v; break;
    }
}

// A 16-byte or 8-byte piece, with NT a non-temporal load (streaming past
// the caches, for data read once).
template <bool NT, typename W>
__device__ __forceinline__ W load_piece(const W* at) {
    if (NT) return __builtin_nontemporal_load(at);
    return *at;
}

// `E` consecutive elements from `index` on, as `load_as` reads them one by
// one, moved four at a time: 16 bytes for f32, 8 for the 16-bit types.
// `index` is a multiple of 4 and `base` aligned to the piece.  With NT the
// loads are non-temporal.
template <int E, bool NT = false>
__device__ __forceinline__ void load_run(const void* base, uint32_t dtype, uint64_t index, float (&out)[E]) {
    static_assert(E % 4 == 0, "whole runs of four");
    typedef uint32_t words4 __attribute__((ext_vector_type(4)));
    typedef uint32_t words2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int q = 0; q < E / 4; q++) {
        if (dtype == tc_ops::F32) {
            const words4 v =
                load_piece<NT>(reinterpret_cast<const words4*>(static_cast<const float*>(base) + index + 4 * q));
            out[4 * q] = __uint_as_float(v.x), out[4 * q + 1] = __uint_as_float(v.y);
            out[4 * q + 2] = __uint_as_float(v.z), out[4 * q + 3] = __uint_as_float(v.w);
        } else {
            const words2 v =
                load_piece<NT>(reinterpret_cast<const words2*>(static_cast<const uint16_t*>(base) + index + 4 * q));
            const uint16_t h[4] = {static_cast<uint16_t>(v.x), static_cast<uint16_t>(v.x >> 16),
                                   static_cast<uint16_t>(v.y), static_cast<uint16_t>(v.y >> 16)};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                out[4 * q + j] = dtype == tc_ops::F16 ? static_cast<float>(__builtin_bit_cast(_Float16, h[j]))
                                                      : bf16_bits_to_f32(h[j]);
            }
        }
    }
}

// `E` consecutive elements stored from `index` on, each converted as
// `store_as` converts it, four at a time; the same alignment as `load_run`.
// With NT the stores are non-temporal, as in `store_wide`.
template <int E, bool NT = false>
__device__ __forceinline__ void store_run(void* base, uint32_t dtype, uint64_t index, const float (&v)[E]) {
    static_assert(E % 4 == 0, "whole runs of four");
    typedef uint32_t words4 __attribute__((ext_vector_type(4)));
    typedef uint32_t words2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int q = 0; q < E / 4; q++) {
        if (dtype == tc_ops::F32) {
            float* at = static_cast<float*>(base) + index + 4 * q;
            const words4 w = {__float_as_uint(v[4 * q]), __float_as_uint(v[4 * q + 1]), __float_as_uint(v[4 * q + 2]),
                              __float_as_uint(v[4 * q + 3])};
            if (NT) {
                __builtin_nontemporal_store(w, reinterpret_cast<words4*>(at));
            } else {
                *reinterpret_cast<words4*>(at) = w;
            }
        } else {
            uint16_t h[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                h[j] = dtype == tc_ops::F16 ? __builtin_bit_cast(uint16_t, static_cast<_Float16>(v[4 * q + j]))
                                            : f32_to_bf16_bits(v[4 * q + j]);
            }
            uint16_t* at = static_cast<uint16_t*>(base) + index + 4 * q;
            const words2 w = {h[0] | (static_cast<uint32_t>(h[1]) << 16), h[2] | (static_cast<uint32_t>(h[3]) << 16)};
            if (NT) {
                __builtin_nontemporal_store(w, reinterpret_cast<words2*>(at));
            } else {
                *reinterpret_cast<words2*>(at) = w;
            }
        }
    }
}

// As `load_run`, in 16-byte pieces for every type: eight 16-bit elements or
// four f32 a piece.  `index` is a multiple of a piece's elements and `base`
// 16-byte aligned.
template <int E, bool NT = false>
__device__ __forceinline__ void load_wide(const void* base, uint32_t dtype, uint64_t index, float (&out)[E]) {
    static_assert(E % 8 == 0, "whole runs of eight");
    typedef uint32_t words4 __attribute__((ext_vector_type(4)));
    if (dtype == tc_ops::F32) {
#pragma unroll
        for (int q = 0; q < E / 4; q++) {
            const words4 v =
                load_piece<NT>(reinterpret_cast<const words4*>(static_cast<const float*>(base) + index + 4 * q));
            out[4 * q] = __uint_as_float(v.x), out[4 * q + 1] = __uint_as_float(v.y);
            out[4 * q + 2] = __uint_as_float(v.z), out[4 * q + 3] = __uint_as_float(v.w);
        }
        return;
    }
#pragma unroll
    for (int q = 0; q < E / 8; q++) {
        const words4 v =
            load_piece<NT>(reinterpret_cast<const words4*>(static_cast<const uint16_t*>(base) + index + 8 * q));
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint16_t h = static_cast<uint16_t>(w[j / 2] >> (16 * (j % 2)));
            out[8 * q + j] = dtype == tc_ops::F16 ? static_cast<float>(__builtin_bit_cast(_Float16, h))
                                                  : bf16_bits_to_f32(h);
        }
    }
}

// As `store_run`, in 16-byte pieces for every type (the alignment of
// `load_wide`); with NT the stores are non-temporal, streaming past the
// caches, for results no kernel of the same launch reads back.
template <int E, bool NT>
__device__ __forceinline__ void store_wide(void* base, uint32_t dtype, uint64_t index, const float (&v)[E]) {
    static_assert(E % 8 == 0, "whole runs of eight");
    typedef uint32_t words __attribute__((ext_vector_type(4)));
    auto put = [](uint4* at, uint4 value) {
        if (NT) {
            __builtin_nontemporal_store(words{value.x, value.y, value.z, value.w}, reinterpret_cast<words*>(at));
        } else {
            *at = value;
        }
    };
    if (dtype == tc_ops::F32) {
#pragma unroll
        for (int q = 0; q < E / 4; q++) {
            put(reinterpret_cast<uint4*>(static_cast<float*>(base) + index + 4 * q),
                make_uint4(__float_as_uint(v[4 * q]), __float_as_uint(v[4 * q + 1]), __float_as_uint(v[4 * q + 2]),
                           __float_as_uint(v[4 * q + 3])));
        }
        return;
    }
    typedef float pair_f32 __attribute__((ext_vector_type(2)));
    typedef __bf16 pair_bf16 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int q = 0; q < E / 8; q++) {
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float lo = v[8 * q + 2 * j], hi = v[8 * q + 2 * j + 1];
            if (dtype == tc_ops::F16) {
                w[j] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(lo)) |
                       (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(hi))) << 16);
            } else {
                // Both halves in one conversion (v_cvt_pk_bf16_f32, the
                // rounding f32_to_bf16_bits does), `lo` in the low half.
                w[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector(pair_f32{lo, hi}, pair_bf16));
            }
        }
        put(reinterpret_cast<uint4*>(static_cast<uint16_t*>(base) + index + 8 * q), make_uint4(w[0], w[1], w[2], w[3]));
    }
}

// q[e] = x[e] / d, each the IEEE f32 quotient, for a divisor the same for
// every element (a function of a row's statistics and constants), at about
// half the cost of E f32 divisions: one f64 reciprocal, then a product a
// quotient.  r = RN64(1/d) and RN64(x r) are within 2^-52 of x / d
// relatively, while x / d, a quotient of two 24-bit significands, lies at
// least 2^-49 from every midpoint between two normal floats (or the
// overflow threshold) unless it is one, which takes a 25-bit significand
// that no 24-bit x has: so rounding the product to f32 gives the
// correctly rounded quotient whenever that is a normal float.  Any other
// result (zero, subnormal, infinite, NaN; so any zero, infinite or NaN
// operand) is recomputed by the f32 division itself.
template <int E>
__device__ __forceinline__ void div_uniform(float (&q)[E], const float (&x)[E], float d) {
    const double r = 1.0 / static_cast<double>(d);
    bool other = false;
#pragma unroll
    for (int e = 0; e < E; e++) {
        q[e] = static_cast<float>(static_cast<double>(x[e]) * r);
        other |= !__builtin_amdgcn_classf(q[e], 0x108);  // not a normal float (class bits 3 and 8)
    }
    if (other) {
#pragma unroll
        for (int e = 0; e < E; e++) q[e] = x[e] / d;
    }
}

}  // namespace tc
