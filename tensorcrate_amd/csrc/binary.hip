// Elementwise kernels: the same-shape vector and matrix operations
// (`*_elementwise`, `*_broadcast`, `*_compare`, `*_compare_scalar`,
// `*_clamp`, tensors/kernels.rs:832-863, :912-938) and the broadcasting
// `strided_binary` (kernels.rs:1162-1166).
//
// Every result is computed in f32 and rounded to the element type once.  For
// f32 that is the IEEE operation itself, and for f16 and bf16 it is the
// correctly rounded 16-bit result, since f32 carries more than twice their
// precision plus two bits: the values `half`'s scalar operators produce
// (compact.rs:5-13).  The sources build with -ffp-contract=off, so no
// multiply and add are ever fused across two operations.
//
// Each thread moves 16 bytes of every unit-stride operand (4 f32 or 8
// f16/bf16 elements) with vector loads and stores, in one pass over a grid
// that covers the work; launches whose traffic exceeds the Infinity Cache
// stream with nontemporal accesses.

#include "common.hpp"

namespace tc {
namespace {

// ---- the operation functors ------------------------------------------------

template <uint32_t OP>
struct Arith {
    __device__ static float apply(float a, float b) { return binary_value(OP, a, b); }
};
template <uint32_t OP>
struct Cmp {
    __device__ static float apply(float a, float b) { return compare_value(OP, a, b); }
};
struct Pow {
    __device__ static float apply(float a, float b) { return powf(a, b); }
};

template <typename S>
struct alignas(16) Pack {
    static constexpr int N = 16 / sizeof(S);
    S v[N];
};

// ---- contiguous operands ---------------------------------------------------

// What one contiguous element computes: from two operands, from one and a
// scalar on either side, or the clamp.
template <typename Op>
struct Two {
    __device__ float operator()(float x, float y) const { return Op::apply(x, y); }
};
template <typename Op, bool LEFT>
struct WithScalar {
    float s;
    __device__ float operator()(float x, float) const { return LEFT ? Op::apply(s, x) : Op::apply(x, s); }
};
// `clamp(low, high)` = min(max(x, low), high) (kernels.rs:856-863).
struct ClampTo {
    float low, high;
    __device__ float operator()(float x, float) const { return fminf(fmaxf(x, low), high); }
};

// out[i] = f(a[i], b[i]) over n contiguous elements; `b` may be null when f
// ignores it.  PACKED kernels move 16-byte packs (all pointers aligned), U
// packs a thread a round with every load issued before any store, and block
// 0 finishes the last partial pack element by element; NT marks a streaming
// launch, whose loads are non-temporal and stores plain (same-shape add over
// 64 Mi f32: 6.55 -> 6.87 TB/s against non-temporal stores; the broadcasting
// kernel below measured the same either way and keeps them).  The grid normally covers the work in one round; the loop covers
// tensors past the 2^32 work-items one dispatch can hold.
template <typename S, typename F, bool PACKED, bool NT, int U>
__global__ void __launch_bounds__(256) map_kernel(const S* __restrict__ a, const S* __restrict__ b,
                                                  S* __restrict__ out, uint64_t n, F f) {
    using E = Elem<S>;
    constexpr int N = Pack<S>::N;
    const uint64_t step = static_cast<uint64_t>(gridDim.x) * 256 * U;
    if (PACKED) {
        const uint64_t packs = n / N;
        for (uint64_t base = static_cast<uint64_t>(blockIdx.x) * 256 * U + threadIdx.x; base < packs; base += step) {
            Pack<S> x[U], y[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const uint64_t i = base + u * 256;
                if (i < packs) {
                    x[u] = __builtin_bit_cast(Pack<S>, load_word<NT>(a + i * N));
                    if (b != nullptr) y[u] = __builtin_bit_cast(Pack<S>, load_word<NT>(b + i * N));
                }
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                const uint64_t i = base + u * 256;
                if (i < packs) {
                    Pack<S> z;
#pragma unroll
                    for (int k = 0; k < N; k++) {
                        const float yv = b != nullptr ? E::widen(y[u].v[k]) : 0.0f;
                        z.v[k] = E::narrow(f(E::widen(x[u].v[k]), yv));
                    }
                    store_word<false>(out + i * N, __builtin_bit_cast(uint4, z));
                }
            }
        }
        const uint64_t tail = n - packs * N;
        if (blockIdx.x == 0 && threadIdx.x < tail) {
            const uint64_t i = packs * N + threadIdx.x;
            const float yv = b != nullptr ? E::widen(b[i]) : 0.0f;
            out[i] = E::narrow(f(E::widen(a[i]), yv));
        }
    } else {
        for (uint64_t base = static_cast<uint64_t>(blockIdx.x) * 256 * U + threadIdx.x; base < n; base += step) {
#pragma unroll
            for (int u = 0; u < U; u++) {
                const uint64_t i = base + u * 256;
                if (i < n) {
                    const float yv = b != nullptr ? E::widen(b[i]) : 0.0f;
                    out[i] = E::narrow(f(E::widen(a[i]), yv));
                }
            }
        }
    }
}

template <typename S, typename F>
int launch_map(const void* a, const void* b, void* out, uint64_t n, F f, hipStream_t s, const char* what) {
    if (n == 0) return TC_OK;
    const S* pa = static_cast<const S*>(a);
    const S* pb = static_cast<const S*>(b);
    S* po = static_cast<S*>(out);
    const uint64_t bytes = n * sizeof(S) * (b == nullptr ? 2 : 3);
    if (aligned16(a) && (b == nullptr || aligned16(b)) && aligned16(out)) {
        const uint64_t packs = n / Pack<S>::N;
        if (bytes > kStreamBytes) {
            map_kernel<S, F, true, true, 4><<<blocks_for(packs, 4), 256, 0, s>>>(pa, pb, po, n, f);
        } else {
            map_kernel<S, F, true, false, 1><<<blocks_for(packs, 1), 256, 0, s>>>(pa, pb, po, n, f);
        }
    } else {
        map_kernel<S, F, false, false, 4><<<blocks_for(n, 4), 256, 0, s>>>(pa, pb, po, n, f);
    }
    return check_launch(what);
}

// Dispatch a (kind, op) pair to its functor type `Op`.
#define TC_DISPATCH_PAIRWISE(kind, op, Op, ...)                                              \
    if (kind == TC_PAIR_ARITHMETIC) {                                                        \
        switch (op) {                                                                        \
            case TC_ADD: { using Op = Arith<TC_ADD>; __VA_ARGS__; } break;                   \
            case TC_SUB: { using Op = Arith<TC_SUB>; __VA_ARGS__; } break;                   \
            case TC_MUL: { using Op = Arith<TC_MUL>; __VA_ARGS__; } break;                   \
            case TC_DIV: { using Op = Arith<TC_DIV>; __VA_ARGS__; } break;                   \
            case TC_REM: { using Op = Arith<TC_REM>; __VA_ARGS__; } break;                   \
            default: return fail(TC_INVALID, "no BinaryOp " + std::to_string(op));          \
        }                                                                                    \
    } else if (kind == TC_PAIR_COMPARE) {                                                    \
        switch (op) {                                                                        \
            case TC_MIN: { using Op = Cmp<TC_MIN>; __VA_ARGS__; } break;                     \
            case TC_MAX: { using Op = Cmp<TC_MAX>; __VA_ARGS__; } break;                     \
            case TC_MAX_SHARE: { using Op = Cmp<TC_MAX_SHARE>; __VA_ARGS__; } break;         \
            case TC_LESS: { using Op = Cmp<TC_LESS>; __VA_ARGS__; } break;                   \
            case TC_LESS_EQUAL: { using Op = Cmp<TC_LESS_EQUAL>; __VA_ARGS__; } break;       \
            case TC_GREATER: { using Op = Cmp<TC_GREATER>; __VA_ARGS__; } break;             \
            case TC_GREATER_EQUAL: { using Op = Cmp<TC_GREATER_EQUAL>; __VA_ARGS__; } break; \
            default: return fail(TC_INVALID, "no Compare " + std::to_string(op));           \
        }                                                                                    \
    } else if (kind == TC_PAIR_POWER) {                                                      \
        using Op = Pow;                                                                      \
        __VA_ARGS__;                                                                         \
    } else {                                                                                 \
        return fail(TC_INVALID, "no Pairwise kind " + std::to_string(kind));                \
    }

template <typename S>
int map_pair(uint32_t kind, uint32_t op, const void* a, const void* b, void* out, uint64_t n,
             const char* what) {
    TC_STREAM(s);
    TC_DISPATCH_PAIRWISE(kind, op, Op, return launch_map<S>(a, b, out, n, Two<Op>{}, s, what));
    return TC_OK;
}

template <typename S>
int map_scalar(uint32_t kind, uint32_t op, const void* a, float scalar, bool left, void* out, uint64_t n,
               const char* what) {
    TC_STREAM(s);
    if (left) {
        TC_DISPATCH_PAIRWISE(kind, op, Op,
                             return launch_map<S>(a, nullptr, out, n, WithScalar<Op, true>{scalar}, s, what));
    } else {
        TC_DISPATCH_PAIRWISE(kind, op, Op,
                             return launch_map<S>(a, nullptr, out, n, WithScalar<Op, false>{scalar}, s, what));
    }
    return TC_OK;
}

// ---- analytic functions and powers (kernels.rs:876-895, :941-949) -----------

// A value rounded to S and back: the host's arithmetic in S, one rounding per
// operation, with f32 the identity.
template <typename S>
__device__ __forceinline__ float in_s(float v) {
    return Elem<S>::widen(Elem<S>::narrow(v));
}

// `Analytic::value` as the host applies it to S (vmath.rs:483-507): in f32,
// the caller rounding once; for f16 and bf16 `Sec` and `Csc` are the
// reciprocal, in S, of the rounded cosine or sine.
template <typename S>
__device__ __forceinline__ float analytic_in(uint32_t op, float x) {
    if (op == 3) return 1.0f / in_s<S>(cosf(x));
    if (op == 4) return 1.0f / in_s<S>(sinf(x));
    return tc_analytic(op, x);
}

// `Analytic::derivative` (kernels.rs:358-385), every operation rounded to S
// as the host's arithmetic in S rounds it.
template <typename S>
__device__ float derivative_in(uint32_t op, float x) {
    auto r = [](float v) { return in_s<S>(v); };
    auto value = [&](uint32_t f) { return r(analytic_in<S>(f, x)); };
    switch (op) {
        case 0: return value(1);
        case 1: return -value(0);
        case 2: { const float c = value(1); return r(1.0f / r(c * c)); }
        case 3: { const float c = value(1); return r(value(0) / r(c * c)); }
        case 4: { const float sn = value(0); return r(-value(1) / r(sn * sn)); }
        case 5: return r(1.0f / r(sqrtf(r(1.0f - r(x * x)))));
        case 6: return -r(1.0f / r(sqrtf(r(1.0f - r(x * x)))));
        case 7: return r(1.0f / r(1.0f + r(x * x)));
        case 8: return value(8);
        case 9: return r(1.0f / x);
        case 10: return value(11);
        case 11: return value(10);
        case 12: { const float t = value(12); return r(1.0f - r(t * t)); }
        default: return r(1.0f / r(2.0f * value(13)));
    }
}

template <typename S>
struct UnaryOf {
    uint32_t op;
    __device__ float operator()(float x, float) const { return analytic_in<S>(op, x); }
};

// `x^s` with the host's fast exponents for f32 (analytic.rs:415-476): 0, 1,
// 2, 1/2 and -1 are single exact operations; anything else, and every f16 or
// bf16 exponent, is `powf` rounded once.
template <typename S>
struct PowerRight {
    float s;
    int fast;  // 0 none, 1 zero, 2 one, 3 square, 4 root, 5 reciprocal
    __device__ float operator()(float x, float) const {
        switch (fast) {
            case 1: return 1.0f;
            case 2: return x;
            case 3: return x * x;
            case 4: return x == -INFINITY ? INFINITY : sqrtf(x) + 0.0f;
            case 5: return 1.0f / x;
            default: return powf(x, s);
        }
    }
};

// `(f(x), f'(x) t)` over n elements, 16 bytes of each operand a thread.
template <typename S, bool PACKED>
__global__ void __launch_bounds__(256) dual_kernel(const S* __restrict__ value, const S* __restrict__ tangent,
                                                   S* __restrict__ out_value, S* __restrict__ out_tangent,
                                                   uint64_t n, uint32_t op) {
    using E = Elem<S>;
    constexpr int N = PACKED ? Pack<S>::N : 1;
    const uint64_t groups = PACKED ? n / N : n;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t g = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; g < groups; g += stride) {
        S x[N], t[N], fx[N], ft[N];
        if (PACKED) {
            __builtin_memcpy(x, value + g * N, 16);
            __builtin_memcpy(t, tangent + g * N, 16);
        } else {
            x[0] = value[g];
            t[0] = tangent[g];
        }
#pragma unroll
        for (int k = 0; k < N; k++) {
            const float v = E::widen(x[k]);
            fx[k] = E::narrow(analytic_in<S>(op, v));
            ft[k] = E::narrow(derivative_in<S>(op, v) * E::widen(t[k]));
        }
        if (PACKED) {
            __builtin_memcpy(out_value + g * N, fx, 16);
            __builtin_memcpy(out_tangent + g * N, ft, 16);
        } else {
            out_value[g] = fx[0];
            out_tangent[g] = ft[0];
        }
    }
    if (PACKED && blockIdx.x == 0 && threadIdx.x < n - groups * N) {
        const uint64_t i = groups * N + threadIdx.x;
        const float v = E::widen(value[i]);
        out_value[i] = E::narrow(analytic_in<S>(op, v));
        out_tangent[i] = E::narrow(derivative_in<S>(op, v) * E::widen(tangent[i]));
    }
}

template <typename S>
int launch_dual(const void* value, const void* tangent, void* out_value, void* out_tangent, uint64_t n, uint32_t op) {
    TC_STREAM(s);
    if (n == 0) return TC_OK;
    const S* v = static_cast<const S*>(value);
    const S* t = static_cast<const S*>(tangent);
    S* ov = static_cast<S*>(out_value);
    S* ot = static_cast<S*>(out_tangent);
    if (aligned16(v) && aligned16(t) && aligned16(ov) && aligned16(ot)) {
        dual_kernel<S, true><<<blocks_for(n / Pack<S>::N + 1, 1), 256, 0, s>>>(v, t, ov, ot, n, op);
    } else {
        dual_kernel<S, false><<<blocks_for(n, 1), 256, 0, s>>>(v, t, ov, ot, n, op);
    }
    return check_launch("unary_dual");
}

int fast_exponent(float e) {
    if (e == 0.0f) return 1;
    if (e == 1.0f) return 2;
    if (e == 2.0f) return 3;
    if (e == 0.5f) return 4;
    if (e == -1.0f) return 5;
    return 0;
}

// ---- strided, broadcasting operands ----------------------------------------

// How an operand steps along the innermost axis of a coalesced walk.
enum Step : uint32_t { kRepeat = 0, kUnit = 1, kStrided = 2 };

template <typename I>
struct BinaryWalk {
    int rank;  // axes; threads work along runs of the last one
    I shape[kMaxRank];
    Div<I> div[kMaxRank];
    I a[kMaxRank], b[kMaxRank];
    uint32_t step_a, step_b;  // each operand's Step along the run
    bool vec_a, vec_b;        // a unit-stride operand's groups are 16-byte aligned
};

// Work items are groups of V consecutive elements of one run (V divides the
// run).  The output is the row-major layout of the walk's shape.
template <typename S, typename Op, int V, bool NT, typename I>
__global__ void __launch_bounds__(256) strided_binary_kernel(const S* __restrict__ a,
                                                             const S* __restrict__ b,
                                                             S* __restrict__ out, BinaryWalk<I> w,
                                                             I groups, Div<I> per_run, I run_groups) {
    using E = Elem<S>;
    const int last = w.rank - 1;
    // One round normally; the loop (64-bit, so it cannot wrap) covers work
    // past what one dispatch holds.
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t item = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; item < groups;
         item += stride) {
        const I g = static_cast<I>(item);
        const I row = per_run.div(g);
        const I col = (g - row * run_groups) * V;
        // The run's start in each operand, from the row's coordinates.
        I at_a = 0, at_b = 0;
        I index = row;
        for (int k = last - 1; k > 0; k--) {
            I q = w.div[k].div(index);
            I c = index - q * w.shape[k];
            at_a += c * w.a[k];
            at_b += c * w.b[k];
            index = q;
        }
        if (last > 0) {
            at_a += index * w.a[0];
            at_b += index * w.b[0];
        }
        float x[V], y[V];
        if (V > 1 && w.step_a == kUnit && w.vec_a) {
            Pack<S> p = __builtin_bit_cast(Pack<S>, load_word<NT>(a + at_a + col));
#pragma unroll
            for (int k = 0; k < V; k++) x[k] = E::widen(p.v[k]);
        } else if (w.step_a == kRepeat) {
            const float v = E::widen(a[at_a]);
#pragma unroll
            for (int k = 0; k < V; k++) x[k] = v;
        } else {
#pragma unroll
            for (int k = 0; k < V; k++) x[k] = E::widen(a[at_a + (col + k) * w.a[last]]);
        }
        if (V > 1 && w.step_b == kUnit && w.vec_b) {
            Pack<S> p = __builtin_bit_cast(Pack<S>, load_word<NT>(b + at_b + col));
#pragma unroll
            for (int k = 0; k < V; k++) y[k] = E::widen(p.v[k]);
        } else if (w.step_b == kRepeat) {
            const float v = E::widen(b[at_b]);
#pragma unroll
            for (int k = 0; k < V; k++) y[k] = v;
        } else {
#pragma unroll
            for (int k = 0; k < V; k++) y[k] = E::widen(b[at_b + (col + k) * w.b[last]]);
        }
        const I o = row * w.shape[last] + col;
        if (V > 1) {
            Pack<S> z;
#pragma unroll
            for (int k = 0; k < V; k++) z.v[k] = E::narrow(Op::apply(x[k], y[k]));
            store_word<NT>(out + o, __builtin_bit_cast(uint4, z));
        } else {
            out[o] = E::narrow(Op::apply(x[0], y[0]));
        }
    }
}

template <typename S, typename Op, typename I>
int launch_strided_binary(const S* a, const S* b, S* out, const Walk<3>& walk, uint64_t count,
                          hipStream_t s) {
    if (walk.rank == 0) {
        // A single element: a run of one.
        BinaryWalk<I> w{};
        w.rank = 1;
        w.shape[0] = 1;
        w.div[0].set(1);
        w.step_a = w.step_b = kRepeat;
        Div<I> one;
        one.set(1);
        strided_binary_kernel<S, Op, 1, false, I><<<1, 64, 0, s>>>(a, b, out, w, I{1}, one, I{1});
        return check_launch("strided binary");
    }
    BinaryWalk<I> w{};
    w.rank = walk.rank;
    for (int k = 0; k < walk.rank; k++) {
        w.shape[k] = static_cast<I>(walk.shape[k]);
        w.div[k].set(walk.shape[k]);
        w.a[k] = static_cast<I>(walk.strides[0][k]);
        w.b[k] = static_cast<I>(walk.strides[1][k]);
    }
    const int last = walk.rank - 1;
    auto step_of = [](uint64_t stride) { return stride == 0 ? kRepeat : stride == 1 ? kUnit : kStrided; };
    w.step_a = step_of(walk.strides[0][last]);
    w.step_b = step_of(walk.strides[1][last]);
    auto runs_aligned = [&](const S* p, int operand) {
        if (!aligned16(p)) return false;
        for (int k = 0; k < last; k++) {
            if ((walk.strides[operand][k] * sizeof(S)) % 16 != 0) return false;
        }
        return true;
    };
    w.vec_a = runs_aligned(a, 0);
    w.vec_b = runs_aligned(b, 1);
    const uint64_t run = walk.shape[last];
    constexpr int V = Pack<S>::N;
    if (run % V == 0 && aligned16(out)) {
        const uint64_t run_groups = run / V;
        const uint64_t groups = count / V;
        Div<I> per_run;
        per_run.set(run_groups);
        // Streaming when the output alone exceeds the Infinity Cache.
        if (count * sizeof(S) > kStreamBytes) {
            strided_binary_kernel<S, Op, V, true, I><<<blocks_for(groups, 1), 256, 0, s>>>(
                a, b, out, w, static_cast<I>(groups), per_run, static_cast<I>(run_groups));
        } else {
            strided_binary_kernel<S, Op, V, false, I><<<blocks_for(groups, 1), 256, 0, s>>>(
                a, b, out, w, static_cast<I>(groups), per_run, static_cast<I>(run_groups));
        }
    } else {
        Div<I> per_run;
        per_run.set(run);
        strided_binary_kernel<S, Op, 1, false, I><<<blocks_for(count, 1), 256, 0, s>>>(
            a, b, out, w, static_cast<I>(count), per_run, static_cast<I>(run));
    }
    return check_launch("strided binary");
}

template <typename S>
int strided_binary_typed(uint32_t kind, uint32_t op, const void* a, const void* b, void* out,
                         const Walk<3>& walk, uint64_t count) {
    TC_STREAM(s);
    const S* pa = static_cast<const S*>(a) + walk.offsets[0];
    const S* pb = static_cast<const S*>(b) + walk.offsets[1];
    S* po = static_cast<S*>(out);
    bool small = count <= UINT32_MAX;
    for (int n = 0; n < 2 && small; n++) {
        uint64_t end = 0;
        small = reach(walk.rank, walk.shape, 0, walk.strides[n], &end) && end <= UINT32_MAX;
    }
    if (small) {
        TC_DISPATCH_PAIRWISE(kind, op, Op,
                             return launch_strided_binary<S, Op, uint32_t>(pa, pb, po, walk, count, s));
    } else {
        TC_DISPATCH_PAIRWISE(kind, op, Op,
                             return launch_strided_binary<S, Op, uint64_t>(pa, pb, po, walk, count, s));
    }
    return TC_OK;
}

}  // namespace
}  // namespace tc

using namespace tc;

extern "C" {

int tc_elementwise(uint32_t dtype, uint32_t op, const void* a, const void* b, void* out, uint64_t n) {
    if (n != 0 && any_null({a, b, out})) return null_operand("elementwise");
    TC_DISPATCH_FLOAT(dtype, "elementwise", S,
                      return map_pair<S>(TC_PAIR_ARITHMETIC, op, a, b, out, n, "elementwise"));
    return TC_OK;
}

int tc_broadcast(uint32_t dtype, uint32_t op, const void* a, float scalar, int scalar_left, void* out,
                 uint64_t n) {
    if (n != 0 && any_null({a, out})) return null_operand("broadcast");
    TC_DISPATCH_FLOAT(dtype, "broadcast", S,
                      return map_scalar<S>(TC_PAIR_ARITHMETIC, op, a, scalar, scalar_left != 0, out, n,
                                           "broadcast"));
    return TC_OK;
}

int tc_compare(uint32_t dtype, uint32_t op, const void* a, const void* b, void* out, uint64_t n) {
    if (n != 0 && any_null({a, b, out})) return null_operand("compare");
    TC_DISPATCH_FLOAT(dtype, "compare", S,
                      return map_pair<S>(TC_PAIR_COMPARE, op, a, b, out, n, "compare"));
    return TC_OK;
}

int tc_compare_scalar(uint32_t dtype, uint32_t op, const void* a, float scalar, int scalar_left,
                      void* out, uint64_t n) {
    if (n != 0 && any_null({a, out})) return null_operand("compare_scalar");
    TC_DISPATCH_FLOAT(dtype, "compare_scalar", S,
                      return map_scalar<S>(TC_PAIR_COMPARE, op, a, scalar, scalar_left != 0, out, n,
                                           "compare_scalar"));
    return TC_OK;
}

int tc_unary(uint32_t dtype, uint32_t op, const void* a, void* out, uint64_t n) {
    if (op > 13) return fail(TC_INVALID, "no Analytic " + std::to_string(op));
    if (n != 0 && any_null({a, out})) return null_operand("unary");
    TC_STREAM(s);
    TC_DISPATCH_FLOAT(dtype, "unary", S, return launch_map<S>(a, nullptr, out, n, UnaryOf<S>{op}, s, "unary"));
    return TC_OK;
}

int tc_unary_dual(uint32_t dtype, uint32_t op, const void* value, const void* tangent, void* out_value,
                  void* out_tangent, uint64_t n) {
    if (op > 13) return fail(TC_INVALID, "no Analytic " + std::to_string(op));
    if (n != 0 && any_null({value, tangent, out_value, out_tangent})) return null_operand("unary_dual");
    TC_DISPATCH_FLOAT(dtype, "unary_dual", S, return launch_dual<S>(value, tangent, out_value, out_tangent, n, op));
    return TC_OK;
}

int tc_power(uint32_t dtype, const void* a, const void* b, void* out, uint64_t n) {
    if (n != 0 && any_null({a, b, out})) return null_operand("power");
    TC_DISPATCH_FLOAT(dtype, "power", S, return map_pair<S>(TC_PAIR_POWER, 0, a, b, out, n, "power"));
    return TC_OK;
}

int tc_power_scalar(uint32_t dtype, const void* a, float scalar, int scalar_left, void* out, uint64_t n) {
    if (n != 0 && any_null({a, out})) return null_operand("power");
    if (scalar_left) {
        TC_DISPATCH_FLOAT(dtype, "power", S,
                          return map_scalar<S>(TC_PAIR_POWER, 0, a, scalar, true, out, n, "power"));
        return TC_OK;
    }
    TC_STREAM(s);
    const int fast = dtype == TC_F32 ? fast_exponent(scalar) : 0;
    TC_DISPATCH_FLOAT(dtype, "power", S,
                      return launch_map<S>(a, nullptr, out, n, PowerRight<S>{scalar, fast}, s, "power"));
    return TC_OK;
}

int tc_clamp(uint32_t dtype, const void* a, float low, float high, void* out, uint64_t n) {
    // Only an ordered pair the wrong way round is refused: a NaN bound is
    // inert, since max(x, NaN) and min(x, NaN) are x (shape.rs:30-43).
    if (low > high) return fail(TC_INVALID, "clamp: the lower bound exceeds the upper one");
    if (n != 0 && any_null({a, out})) return null_operand("clamp");
    TC_STREAM(s);
    TC_DISPATCH_FLOAT(dtype, "clamp", S, return launch_map<S>(a, nullptr, out, n, ClampTo{low, high}, s, "clamp"));
    return TC_OK;
}

int tc_strided_binary(uint32_t dtype, uint32_t kind, uint32_t op, uint32_t rank, const uint64_t* shape,
                      const void* a, uint64_t a_len, const tc_strided* a_at, const void* b, uint64_t b_len,
                      const tc_strided* b_at, void* out) {
    uint64_t count = 0;
    int status = check_strided(a_len, rank, shape, a_at->offset, a_at->strides, "strided binary", &count);
    if (status != TC_OK) return status;
    status = check_strided(b_len, rank, shape, b_at->offset, b_at->strides, "strided binary", &count);
    if (status != TC_OK) return status;
    if (count == 0) return TC_OK;
    if (any_null({a, b, out})) return null_operand("strided binary");
    uint64_t out_strides[kMaxRank] = {};
    uint64_t step = 1;
    for (int k = static_cast<int>(rank) - 1; k >= 0; k--) {
        out_strides[k] = step;
        step *= shape[k];
    }
    const uint64_t* strides[3] = {a_at->strides, b_at->strides, out_strides};
    const uint64_t offsets[3] = {a_at->offset, b_at->offset, 0};
    Walk<3> walk = coalesce<3>(rank, shape, strides, offsets);
    TC_DISPATCH_FLOAT(dtype, "strided binary", S,
                      return strided_binary_typed<S>(kind, op, a, b, out, walk, count));
    return TC_OK;
}

}  // extern "C"
