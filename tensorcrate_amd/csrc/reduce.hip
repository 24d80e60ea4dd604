// Reductions: `Kernels::reduce_axes` (tensors/kernels.rs:1175-1179),
// `Kernels::arg_reduce` (kernels.rs:1187), and the whole-buffer
// `vector_reduce` and `dot` (kernels.rs:867, :897).
//
// Every slice accumulates in f32 and rounds to the element type once, as the
// host's `reduce_in` does (strided.rs:102-162).  Min and max are minNum /
// maxNum, exact in any order; a sum is a tree here where the host folds left
// to right, so sums, means and variances agree with the host within rounding,
// as the reference's own Metal kernels do (kernels.rs:170-180).  The variance
// is single-pass: each thread folds exact two-pass moments of the values it
// holds in registers, and threads combine (count, mean, M2) triples with
// Chan, Golub and LeVeque's pairwise update, so no slice is read from HBM
// twice.  Argmax/argmin carry (value, index) pairs ordered by value and then
// by smaller index, which picks the first extreme whatever the tree's shape;
// NaNs never win, and a slice of NaNs answers index 0 (strided.rs:186-225).
//
// The host coalesces the kept and the folded axes separately and picks:
//  - rows: the folded axes are one contiguous run; one wave per slice, lanes
//    reading 16 bytes at a time, combined by a 64-lane shuffle tree;
//  - columns: the innermost kept axis is contiguous and the folded axes are
//    one strided axis; lanes take neighbouring columns so each row read is
//    coalesced, four row groups split the depth inside a block, and long
//    depths split across blocks, each result's splits then merged by one
//    wave in a fixed order;
//  - general: one thread per slice walking its elements in row-major order.

#include <math.h>

#include <mutex>
#include <unordered_map>

#include "common.hpp"

// The whole-buffer fold's block partials for `tc_vector_reduce_noalloc`,
// which allocates nothing: `total` launches at most four blocks a CU, so
// 4096 floats (16 KiB a GPU, held until the process ends) cover parts of up
// to 1024 CUs.
constexpr uint32_t kStaticPartials = 4096;
static __device__ __align__(256) float scratch[kStaticPartials];

namespace tc {
namespace {

// ---- accumulator policies ---------------------------------------------------

// Sum, Min, Max and Mean fold one f32.
template <uint32_t OP>
struct Fold {
    using State = float;
    __device__ static State init() {
        return OP == TC_REDUCE_SUM ? 0.0f : (OP == TC_REDUCE_MIN ? INFINITY : -INFINITY);
    }
    __device__ static State combine(State a, float x) {
        return OP == TC_REDUCE_SUM ? a + x : (OP == TC_REDUCE_MIN ? fminf(a, x) : fmaxf(a, x));
    }
    __device__ static void add(State& s, float x, uint32_t) { s = combine(s, x); }
    template <int N>
    __device__ static void add_chunk(State& s, const float (&x)[N], uint32_t) {
        State c = init();
#pragma unroll
        for (int k = 0; k < N; k++) c = combine(c, x[k]);
        s = combine(s, c);
    }
    // U packs of V elements, pack k starting at element first + k * step.
    template <int U, int V>
    __device__ static void add_packs(State& s, const float (&x)[U * V], uint32_t, uint32_t) {
        add_chunk(s, x, 0);
    }
    __device__ static State merge(State a, State b) { return combine(a, b); }
    __device__ static State shuffle(State s, int lane) { return __shfl(s, lane, 64); }
};

struct Moments {
    float n, mean, m2;
};

// Chan, Golub and LeVeque (1979): the moments of two disjoint sets.
__device__ inline Moments merge_moments(Moments a, Moments b) {
    if (a.n == 0.0f) return b;
    if (b.n == 0.0f) return a;
    const float n = a.n + b.n;
    const float share = b.n / n;
    const float d = b.mean - a.mean;
    return Moments{n, a.mean + d * share, a.m2 + b.m2 + d * d * a.n * share};
}

struct Var {
    using State = Moments;
    __device__ static State init() { return Moments{0.0f, 0.0f, 0.0f}; }
    __device__ static void add(State& s, float x, uint32_t) { s = merge_moments(s, Moments{1.0f, x, 0.0f}); }
    // A chunk's own moments are exact two-pass ones from registers.
    template <int N>
    __device__ static void add_chunk(State& s, const float (&x)[N], uint32_t) {
        float total = 0.0f;
#pragma unroll
        for (int k = 0; k < N; k++) total += x[k];
        const float mean = total / static_cast<float>(N);
        float m2 = 0.0f;
#pragma unroll
        for (int k = 0; k < N; k++) {
            const float d = x[k] - mean;
            m2 += d * d;
        }
        s = merge_moments(s, Moments{static_cast<float>(N), mean, m2});
    }
    // Every pack a lane holds is one chunk: the pairwise merge, with its
    // division, runs once per U * V elements instead of once per pack.
    template <int U, int V>
    __device__ static void add_packs(State& s, const float (&x)[U * V], uint32_t, uint32_t) {
        add_chunk(s, x, 0);
    }
    __device__ static State merge(State a, State b) { return merge_moments(a, b); }
    __device__ static State shuffle(State s, int lane) {
        return Moments{__shfl(s.n, lane, 64), __shfl(s.mean, lane, 64), __shfl(s.m2, lane, 64)};
    }
};

struct Arg {
    float value;  // NaN until the slice's first number
    uint32_t index;
};

// The later-or-better pair under "largest (or smallest) value, then smallest
// index, NaNs never": associative and commutative, so any tree finds the
// first extreme.
template <uint32_t OP>
struct ArgFold {
    using State = Arg;
    __device__ static State init() { return Arg{NAN, 0u}; }
    __device__ static bool better(Arg b, Arg a) {
        if (isnan(b.value)) return false;
        if (isnan(a.value)) return true;
        const bool past = OP == TC_REDUCE_MIN ? b.value < a.value : b.value > a.value;
        return past || (b.value == a.value && b.index < a.index);
    }
    __device__ static void add(State& s, float x, uint32_t index) {
        Arg c{x, index};
        if (better(c, s)) s = c;
    }
    template <int N>
    __device__ static void add_chunk(State& s, const float (&x)[N], uint32_t first) {
#pragma unroll
        for (int k = 0; k < N; k++) add(s, x[k], first + k);
    }
    template <int U, int V>
    __device__ static void add_packs(State& s, const float (&x)[U * V], uint32_t first, uint32_t step) {
#pragma unroll
        for (int k = 0; k < U; k++) {
#pragma unroll
            for (int j = 0; j < V; j++) add(s, x[k * V + j], first + k * step + j);
        }
    }
    __device__ static State merge(State a, State b) { return better(b, a) ? b : a; }
    __device__ static State shuffle(State s, int lane) {
        return Arg{__shfl(s.value, lane, 64), static_cast<uint32_t>(__shfl(static_cast<int>(s.index), lane, 64))};
    }
};

// Beside the public `tc_axis_reduction`s: a variance's two moments, the
// mean to `out` and the sum of squared deviations to `Finish::second`
// (`row_moments`, kernels.rs:1090).
constexpr uint32_t kAxisMoments = 3;

// What a finished slice writes.
struct Finish {
    uint32_t kind;     // tc_axis_reduction, or kAxisMoments
    float depth;       // the mean's count
    float divisor;     // the variance's divisor
    void* second;      // kAxisMoments: where the deviation sums go
};

template <typename S>
__device__ inline void write_result(S* out, uint64_t at, float value) {
    out[at] = Elem<S>::narrow(value);
}

template <typename P, typename S>
__device__ inline void finish(const typename P::State& s, const Finish& f, S* out, uint64_t at);

template <typename P>
struct Finisher {
    template <typename S>
    __device__ static void write(const typename P::State& s, const Finish& f, S* out, uint64_t at) {
        // Fold and Mean share the f32 state; the mean divides in f32.
        const float v = f.kind == TC_AXIS_MEAN ? s / f.depth : s;
        write_result(out, at, v);
    }
};
template <>
struct Finisher<Var> {
    template <typename S>
    __device__ static void write(const Moments& s, const Finish& f, S* out, uint64_t at) {
        if (f.kind == kAxisMoments) {
            write_result(out, at, s.mean);
            write_result(static_cast<S*>(f.second), at, s.m2);
        } else {
            write_result(out, at, s.m2 / f.divisor);
        }
    }
};
template <uint32_t OP>
struct Finisher<ArgFold<OP>> {
    template <typename S>
    __device__ static void write(const Arg& s, const Finish&, S*, uint64_t) {}
    __device__ static void write(const Arg& s, const Finish&, uint32_t* out, uint64_t at) { out[at] = s.index; }
};

template <typename P>
__device__ inline typename P::State wave_reduce(typename P::State s) {
    const int lane = threadIdx.x % 64;
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) {
        typename P::State other = P::shuffle(s, lane ^ offset);
        // The lower lane's state is the left operand, so the tree's order is
        // fixed and the result deterministic.
        s = (lane & offset) ? P::merge(other, s) : P::merge(s, other);
    }
    return s;
}

// The wave's moments in closed form rather than by six pairwise merges:
// with N = sum n_i and mean = sum n_i mean_i / N,
//     M2 = sum (M2_i + n_i (mean_i - mean)^2),
// the identity each of Chan's merges applies, taken over all 64 lanes at
// once.  Two shuffle-sum trees and one division instead of six divisions
// and eighteen shuffles; the fixed tree keeps the result deterministic.
// A butterfly sum: every lane ends with the same total (each step adds one
// pair, and addition is commutative).
__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, 64);
    return v;
}

template <>
__device__ inline Moments wave_reduce<Var>(Moments s) {
    const float n = wave_sum(s.n);
    if (n == 0.0f) return Var::init();
    const float mean = wave_sum(s.n * s.mean) / n;
    const float d = s.mean - mean;
    const float m2 = wave_sum(s.n == 0.0f ? 0.0f : s.m2 + s.n * d * d);
    return Moments{n, mean, m2};
}

// ---- layouts ----------------------------------------------------------------

template <typename I>
struct Kept {
    int rank;
    I shape[kMaxRank];
    Div<I> div[kMaxRank];
    I strides[kMaxRank];
};

template <typename I>
__device__ __forceinline__ I kept_offset(const Kept<I>& kept, I index) {
    I at = 0;
    for (int k = kept.rank - 1; k > 0; k--) {
        I q = kept.div[k].div(index);
        at += (index - q * kept.shape[k]) * kept.strides[k];
        index = q;
    }
    if (kept.rank > 0) at += index * kept.strides[0];
    return at;
}

template <typename I>
struct Folded {
    int rank;
    I shape[kMaxRank];
    I strides[kMaxRank];
};

template <typename S>
struct alignas(16) Pack {
    static constexpr int N = 16 / sizeof(S);
    S v[N];
};

// ---- rows: one wave per contiguous slice ------------------------------------

// U packs of one lane, 64 packs apart, loaded together and widened.
template <typename S, int U, bool NT>
__device__ __forceinline__ void load_packs(const Pack<S>* packs, float (&x)[U * Pack<S>::N]) {
    constexpr int V = Pack<S>::N;
    uint4 w[U];
#pragma unroll
    for (int k = 0; k < U; k++) w[k] = load_word<NT>(packs + k * 64);
#pragma unroll
    for (int k = 0; k < U; k++) {
        Pack<S> p;
        __builtin_memcpy(&p, &w[k], 16);
#pragma unroll
        for (int j = 0; j < V; j++) x[k * V + j] = Elem<S>::widen(p.v[j]);
    }
}

// With NT the input streams past the Infinity Cache (inputs larger than it).
template <typename S, typename P, typename O, bool PACKED, bool NT, typename I>
__global__ void __launch_bounds__(256) rows_kernel(const S* __restrict__ in, O* __restrict__ out,
                                                   Kept<I> kept, I results, I depth, Finish f) {
    using E = Elem<S>;
    constexpr int V = Pack<S>::N;
    // Four 16-byte packs in flight per lane: a 4 KiB row per wave at once.
    constexpr int U = 4;
    const int lane = threadIdx.x % 64;
    const I waves = static_cast<I>(gridDim.x) * (blockDim.x / 64);
    for (I r = static_cast<I>(blockIdx.x) * (blockDim.x / 64) + threadIdx.x / 64; r < results; r += waves) {
        const S* slice = in + kept_offset(kept, r);
        typename P::State s = P::init();
        if (PACKED) {
            const Pack<S>* packs = reinterpret_cast<const Pack<S>*>(slice);
            const I count = depth / V;
            I p = lane;
            for (; p + 64 * (U - 1) < count; p += 64 * U) {
                float x[U * V];
                load_packs<S, U, NT>(packs + p, x);
                P::template add_packs<U, V>(s, x, static_cast<uint32_t>(p * V), 64 * V);
            }
            for (; p < count; p += 64) {
                float x[V];
                load_packs<S, 1, NT>(packs + p, x);
                P::template add_packs<1, V>(s, x, static_cast<uint32_t>(p * V), 0);
            }
        } else {
            for (I i = lane; i < depth; i += 64) P::add(s, E::widen(slice[i]), static_cast<uint32_t>(i));
        }
        s = wave_reduce<P>(s);
        if (lane == 0) Finisher<P>::write(s, f, out, r);
    }
}

// ---- columns: lanes on neighbouring kept columns ----------------------------

constexpr int kColumns = 64;
constexpr int kGroups = 4;

// The columns' layout: results are [outer, columns] with the columns
// contiguous in the input; each column folds `depth` elements `step` apart.
template <typename I>
struct ColumnWalk {
    Kept<I> outer;  // the kept axes before the column axis
    I columns;
    I depth, step;
    I tiles;        // column tiles per outer index
    Div<I> tiles_div;
    I splits;       // depth splits across blocks
    I per_split;    // rows per split (the last may hold fewer)
};

// One block: kColumns lanes, each on VC neighbouring columns (VC > 1 reads
// them as one 16-byte word), times kGroups row groups over one split's rows.
// With splits == 1 it finishes the results; otherwise it writes its states
// to `partial[result * splits + split]` for the combine kernels.
template <typename S, typename P, typename O, int VC, bool NT, typename I>
__global__ void __launch_bounds__(256) columns_kernel(const S* __restrict__ in, O* __restrict__ out,
                                                      typename P::State* __restrict__ partial,
                                                      ColumnWalk<I> w, I blocks, Finish f) {
    using E = Elem<S>;
    using State = typename P::State;
    // Rows in flight per lane.
    constexpr int U = 8;
    __shared__ State stage[kGroups][VC][kColumns];
    const int lane = threadIdx.x % kColumns;
    const int group = threadIdx.x / kColumns;
    for (I block = blockIdx.x; block < blocks; block += gridDim.x) {
        // block -> (split, outer, tile), split outermost so neighbouring
        // blocks share rows.
        const I per_split_blocks = blocks / w.splits;
        const I split = block / per_split_blocks;
        const I rest = block - split * per_split_blocks;
        const I outer = w.tiles_div.div(rest);
        const I tile = rest - outer * w.tiles;
        // With VC > 1 the columns are a multiple of VC, so a lane's first
        // column in range puts all VC in range.
        const I column = (tile * kColumns + lane) * VC;
        const I row_begin = split * w.per_split;
        I row_end = row_begin + w.per_split;
        if (row_end > w.depth) row_end = w.depth;
        // Contiguous row ranges per group, so group order is index order.
        const I span = row_end - row_begin;
        const I per_group = (span + kGroups - 1) / kGroups;
        I first = row_begin + group * per_group;
        I last = first + per_group;
        if (last > row_end) last = row_end;
        if (first > row_end) first = row_end;
        State s[VC];
#pragma unroll
        for (int c = 0; c < VC; c++) s[c] = P::init();
        if (column < w.columns) {
            const S* base = in + kept_offset(w.outer, outer) + column;
            I row = first;
            if (VC == 1) {
                for (; row + U <= last; row += U) {
                    float x[U];
#pragma unroll
                    for (int k = 0; k < U; k++) x[k] = E::widen(base[(row + k) * w.step]);
                    P::add_chunk(s[0], x, static_cast<uint32_t>(row));
                }
                for (; row < last; row++) P::add(s[0], E::widen(base[row * w.step]), static_cast<uint32_t>(row));
            } else {
                for (; row + U <= last; row += U) {
                    S v[U][VC];
#pragma unroll
                    for (int k = 0; k < U; k++) {
                        const uint4 word = load_word<NT>(base + (row + k) * w.step);
                        __builtin_memcpy(v[k], &word, 16);
                    }
#pragma unroll
                    for (int c = 0; c < VC; c++) {
                        float x[U];
#pragma unroll
                        for (int k = 0; k < U; k++) x[k] = E::widen(v[k][c]);
                        P::add_chunk(s[c], x, static_cast<uint32_t>(row));
                    }
                }
                for (; row < last; row++) {
                    S v[VC];
                    const uint4 word = load_word<NT>(base + row * w.step);
                    __builtin_memcpy(v, &word, 16);
#pragma unroll
                    for (int c = 0; c < VC; c++) P::add(s[c], E::widen(v[c]), static_cast<uint32_t>(row));
                }
            }
        }
#pragma unroll
        for (int c = 0; c < VC; c++) stage[group][c][lane] = s[c];
        __syncthreads();
        if (group == 0 && column < w.columns) {
#pragma unroll
            for (int c = 0; c < VC; c++) {
                State t = s[c];
#pragma unroll
                for (int g = 1; g < kGroups; g++) t = P::merge(t, stage[g][c][lane]);
                const I result = outer * w.columns + column + c;
                if (w.splits == 1) {
                    Finisher<P>::write(t, f, out, result);
                } else {
                    partial[result * w.splits + split] = t;
                }
            }
        }
        __syncthreads();
    }
}

// Merge each result's split states and finish it: one wave per result,
// lanes taking the splits k = lane, lane + 64, ... in order and the wave's
// fixed shuffle tree merging the lanes, so the order is the same every run.
// A result's states are contiguous (`partial[result * splits + split]`), so
// each wave's loads are one run.
template <typename P, typename O, typename I>
__global__ void __launch_bounds__(256) combine_kernel(const typename P::State* __restrict__ partial,
                                                      O* __restrict__ out, I results, I splits, Finish f) {
    const int lane = threadIdx.x % 64;
    const I waves = static_cast<I>(gridDim.x) * (blockDim.x / 64);
    for (I r = static_cast<I>(blockIdx.x) * (blockDim.x / 64) + threadIdx.x / 64; r < results; r += waves) {
        typename P::State s = P::init();
        for (I k = lane; k < splits; k += 64) s = P::merge(s, partial[r * splits + k]);
        s = wave_reduce<P>(s);
        if (lane == 0) Finisher<P>::write(s, f, out, r);
    }
}

// The same merge for a few splits per result: one thread per result, folding
// its splits left to right.
template <typename P, typename O, typename I>
__global__ void __launch_bounds__(256) combine_few_kernel(const typename P::State* __restrict__ partial,
                                                          O* __restrict__ out, I results, I splits, Finish f) {
    const I stride = static_cast<I>(gridDim.x) * blockDim.x;
    for (I r = static_cast<I>(blockIdx.x) * blockDim.x + threadIdx.x; r < results; r += stride) {
        typename P::State s = partial[r * splits];
        for (I k = 1; k < splits; k++) s = P::merge(s, partial[r * splits + k]);
        Finisher<P>::write(s, f, out, r);
    }
}

// ---- general: one thread per slice -------------------------------------------

template <typename S, typename P, typename O, typename I>
__global__ void __launch_bounds__(256) general_kernel(const S* __restrict__ in, O* __restrict__ out,
                                                      Kept<I> kept, Folded<I> folded, I results, I depth,
                                                      Finish f) {
    using E = Elem<S>;
    const I stride = static_cast<I>(gridDim.x) * blockDim.x;
    for (I r = static_cast<I>(blockIdx.x) * blockDim.x + threadIdx.x; r < results; r += stride) {
        const S* slice = in + kept_offset(kept, r);
        typename P::State s = P::init();
        I index[kMaxRank] = {};
        I at = 0;
        for (I i = 0; i < depth; i++) {
            P::add(s, E::widen(slice[at]), static_cast<uint32_t>(i));
            // Advance the folded axes like an odometer (layout.rs:476-496).
            for (int k = folded.rank - 1; k >= 0; k--) {
                index[k]++;
                at += folded.strides[k];
                if (index[k] < folded.shape[k]) break;
                at -= folded.strides[k] * folded.shape[k];
                index[k] = 0;
            }
        }
        Finisher<P>::write(s, f, out, r);
    }
}

// ---- host-side planning -------------------------------------------------------

// One operand's axes with extent-one axes dropped and mergeable neighbours
// merged (layout.rs:419-449 for a single operand).
struct Axes {
    int rank = 0;
    uint64_t shape[kMaxRank] = {};
    uint64_t strides[kMaxRank] = {};
};

Axes coalesce_axes(uint32_t rank, const uint64_t* shape, const uint64_t* strides) {
    Axes axes;
    for (uint32_t k = 0; k < rank; k++) {
        if (shape[k] == 1) continue;
        if (axes.rank > 0 && axes.strides[axes.rank - 1] == strides[k] * shape[k]) {
            axes.shape[axes.rank - 1] *= shape[k];
            axes.strides[axes.rank - 1] = strides[k];
        } else {
            axes.shape[axes.rank] = shape[k];
            axes.strides[axes.rank] = strides[k];
            axes.rank++;
        }
    }
    return axes;
}

template <typename I>
Kept<I> make_kept(const Axes& axes, int rank) {
    Kept<I> kept{};
    kept.rank = rank;
    for (int k = 0; k < rank; k++) {
        kept.shape[k] = static_cast<I>(axes.shape[k]);
        kept.div[k].set(axes.shape[k]);
        kept.strides[k] = static_cast<I>(axes.strides[k]);
    }
    return kept;
}

struct Plan {
    Axes kept, folded;
    uint64_t results, depth;
};

// The columns kernel over a plan whose innermost kept axis is contiguous and
// whose one folded axis is strided; VC columns per lane.
template <typename S, typename P, typename O, int VC, bool NT, typename I>
int launch_columns(const S* in, O* out, const Plan& plan, const Finish& f, hipStream_t s, const char* what) {
    const Axes& kept = plan.kept;
    const uint64_t results = plan.results, depth = plan.depth;
    ColumnWalk<I> w{};
    w.outer = make_kept<I>(kept, kept.rank - 1);
    const uint64_t columns = kept.shape[kept.rank - 1];
    const uint64_t outer = results / columns;
    const uint64_t tiles = (columns + kColumns * VC - 1) / (kColumns * VC);
    w.columns = static_cast<I>(columns);
    w.depth = static_cast<I>(depth);
    w.step = static_cast<I>(plan.folded.strides[0]);
    w.tiles = static_cast<I>(tiles);
    w.tiles_div.set(tiles);
    // Split the depth across blocks until there are four blocks for every
    // CU, each row group keeping at least 32 rows (16 of 16-byte words); a
    // split costs one partial state per result, written and read back once.
    const uint64_t base_blocks = outer * tiles;
    const uint64_t want = static_cast<uint64_t>(compute_units()) * 4;
    uint64_t splits = 1;
    if (base_blocks < want) {
        splits = (want + base_blocks - 1) / base_blocks;
        const uint64_t most = depth / (kGroups * (VC == 1 ? 32 : 16));
        if (splits > most) splits = most;
        if (splits < 1) splits = 1;
    }
    const uint64_t per_split = (depth + splits - 1) / splits;
    splits = (depth + per_split - 1) / per_split;
    w.splits = static_cast<I>(splits);
    w.per_split = static_cast<I>(per_split);
    const uint64_t blocks = base_blocks * splits;
    typename P::State* partial = nullptr;
    if (splits > 1) {
        void* scratch = nullptr;
        int status = tc_alloc(splits * results * sizeof(typename P::State), &scratch);
        if (status != TC_OK) return status;
        partial = static_cast<typename P::State*>(scratch);
    }
    columns_kernel<S, P, O, VC, NT, I><<<grid_for(blocks, 1, 64), 256, 0, s>>>(in, out, partial, w,
                                                                                 static_cast<I>(blocks), f);
    int status = check_launch(what);
    if (status == TC_OK && splits > 1) {
        if (splits <= 8) {
            combine_few_kernel<P, O, I><<<grid_for(results, 256, 64), 256, 0, s>>>(
                partial, out, static_cast<I>(results), static_cast<I>(splits), f);
        } else {
            combine_kernel<P, O, I><<<grid_for(results, 4, 64), 256, 0, s>>>(
                partial, out, static_cast<I>(results), static_cast<I>(splits), f);
        }
        status = check_launch(what);
    }
    // Stream order keeps the block alive until both kernels have run.
    if (partial != nullptr) tc_free(partial);
    return status;
}

template <typename S, typename P, typename O, typename I>
int launch_reduce(const S* in, O* out, const Plan& plan, const Finish& f, hipStream_t s, const char* what) {
    const Axes& kept = plan.kept;
    const Axes& folded = plan.folded;
    const uint64_t results = plan.results, depth = plan.depth;
    // Rows: the slice is one contiguous run long enough to share a wave.
    if (folded.rank == 1 && folded.strides[0] == 1 && depth >= 64) {
        constexpr int V = Pack<S>::N;
        bool packed = depth % V == 0 && aligned16(in);
        for (int k = 0; packed && k < kept.rank; k++) packed = (kept.strides[k] * sizeof(S)) % 16 == 0;
        Kept<I> k = make_kept<I>(kept, kept.rank);
        const uint32_t blocks = grid_for(results, 4, 32);
        const bool stream = results * depth * sizeof(S) > kStreamBytes;
        if (packed && stream) {
            rows_kernel<S, P, O, true, true, I><<<blocks, 256, 0, s>>>(in, out, k, static_cast<I>(results),
                                                                       static_cast<I>(depth), f);
        } else if (packed) {
            rows_kernel<S, P, O, true, false, I><<<blocks, 256, 0, s>>>(in, out, k, static_cast<I>(results),
                                                                        static_cast<I>(depth), f);
        } else {
            rows_kernel<S, P, O, false, false, I><<<blocks, 256, 0, s>>>(in, out, k, static_cast<I>(results),
                                                                         static_cast<I>(depth), f);
        }
        return check_launch(what);
    }
    // Columns: contiguous neighbouring results, one strided folded axis.
    if (folded.rank == 1 && kept.rank >= 1 && kept.strides[kept.rank - 1] == 1 &&
        kept.shape[kept.rank - 1] >= 16) {
        // An input past the Infinity Cache streams with 16-byte words, VC
        // columns a lane; a smaller one runs a column a lane, which spreads
        // it over four times the blocks (measured faster below 256 MiB).
        constexpr int VC = 16 / sizeof(S);
        bool packed = results * depth * sizeof(S) > kStreamBytes && kept.shape[kept.rank - 1] % VC == 0 &&
                      folded.strides[0] % VC == 0 && aligned16(in);
        for (int k = 0; packed && k + 1 < kept.rank; k++) packed = kept.strides[k] % VC == 0;
        if (packed) return launch_columns<S, P, O, VC, true, I>(in, out, plan, f, s, what);
        return launch_columns<S, P, O, 1, false, I>(in, out, plan, f, s, what);
    }
    Kept<I> k = make_kept<I>(kept, kept.rank);
    Folded<I> fo{};
    fo.rank = folded.rank;
    for (int a = 0; a < folded.rank; a++) {
        fo.shape[a] = static_cast<I>(folded.shape[a]);
        fo.strides[a] = static_cast<I>(folded.strides[a]);
    }
    general_kernel<S, P, O, I><<<grid_for(results, 256), 256, 0, s>>>(in, out, k, fo, static_cast<I>(results),
                                                                      static_cast<I>(depth), f);
    return check_launch(what);
}

template <typename S, typename P, typename O>
int reduce_typed(const void* input, void* out, uint64_t offset, const Plan& plan, const Finish& f,
                 uint64_t input_len, const char* what) {
    TC_STREAM(s);
    const S* in = static_cast<const S*>(input) + offset;
    if (plan.results == 0) return TC_OK;
    bool small = plan.results <= UINT32_MAX && plan.depth <= UINT32_MAX && input_len <= UINT32_MAX;
    if (small) return launch_reduce<S, P, O, uint32_t>(in, static_cast<O*>(out), plan, f, s, what);
    return launch_reduce<S, P, O, uint64_t>(in, static_cast<O*>(out), plan, f, s, what);
}

int check_split(const tc_split* split, uint64_t input_len, const char* what, Plan* plan) {
    if (split->kept_rank + split->folded_rank > static_cast<uint32_t>(kMaxRank)) {
        return fail(TC_INVALID, std::string(what) + ": more than " + std::to_string(kMaxRank) + " axes");
    }
    uint64_t shape[kMaxRank], strides[kMaxRank];
    uint32_t rank = 0;
    for (uint32_t k = 0; k < split->kept_rank; k++, rank++) {
        shape[rank] = split->kept[k];
        strides[rank] = split->kept_strides[k];
    }
    for (uint32_t k = 0; k < split->folded_rank; k++, rank++) {
        shape[rank] = split->folded[k];
        strides[rank] = split->folded_strides[k];
    }
    uint64_t count = 0;
    int status = check_strided(input_len, rank, shape, split->offset, strides, what, &count);
    if (status != TC_OK) return status;
    if (!element_count(split->kept_rank, split->kept, &plan->results) ||
        !element_count(split->folded_rank, split->folded, &plan->depth)) {
        return fail(TC_INVALID, std::string(what) + ": too many elements");
    }
    plan->kept = coalesce_axes(split->kept_rank, split->kept, split->kept_strides);
    plan->folded = coalesce_axes(split->folded_rank, split->folded, split->folded_strides);
    return TC_OK;
}

template <typename S>
int moments_typed(const void* input, uint64_t input_len, const tc_split* split, void* means, void* deviations) {
    Plan plan;
    int status = check_split(split, input_len, "row_moments", &plan);
    if (status != TC_OK) return status;
    Finish f{kAxisMoments, static_cast<float>(plan.depth), 1.0f, deviations};
    return reduce_typed<S, Var, S>(input, means, split->offset, plan, f, input_len, "row_moments");
}

template <typename S>
int reduce_axes_typed(const void* input, uint64_t input_len, const tc_split* split, uint32_t kind,
                      uint32_t op, uint64_t divisor, void* out) {
    Plan plan;
    int status = check_split(split, input_len, "reduce_axes", &plan);
    if (status != TC_OK) return status;
    Finish f{kind, static_cast<float>(plan.depth), static_cast<float>(divisor), nullptr};
    const char* what = "reduce_axes";
    if (kind == TC_AXIS_VARIANCE) {
        return reduce_typed<S, Var, S>(input, out, split->offset, plan, f, input_len, what);
    }
    if (kind == TC_AXIS_MEAN) {
        return reduce_typed<S, Fold<TC_REDUCE_SUM>, S>(input, out, split->offset, plan, f, input_len, what);
    }
    if (kind != TC_AXIS_FOLD) return fail(TC_INVALID, "reduce_axes: no AxisReduction " + std::to_string(kind));
    switch (op) {
        case TC_REDUCE_SUM:
            return reduce_typed<S, Fold<TC_REDUCE_SUM>, S>(input, out, split->offset, plan, f, input_len, what);
        case TC_REDUCE_MIN:
            return reduce_typed<S, Fold<TC_REDUCE_MIN>, S>(input, out, split->offset, plan, f, input_len, what);
        case TC_REDUCE_MAX:
            return reduce_typed<S, Fold<TC_REDUCE_MAX>, S>(input, out, split->offset, plan, f, input_len, what);
        default:
            return fail(TC_INVALID, "reduce_axes: no Reduce " + std::to_string(op));
    }
}

template <typename S>
int arg_reduce_typed(const void* input, uint64_t input_len, const tc_split* split, uint32_t op,
                     uint32_t* out) {
    const char* what = "arg_reduce";
    if (split->folded_rank != 1) {
        return fail(TC_INVALID, "arg_reduce: folds " + std::to_string(split->folded_rank) +
                                    " axes, not one");
    }
    if (split->folded[0] == 0) return fail(TC_INVALID, "arg_reduce: the axis is empty");
    if (split->folded[0] > UINT32_MAX) {
        return fail(TC_INVALID, "arg_reduce: the axis's extent " + std::to_string(split->folded[0]) +
                                    " does not fit a u32");
    }
    Plan plan;
    int status = check_split(split, input_len, what, &plan);
    if (status != TC_OK) return status;
    Finish f{TC_AXIS_FOLD, 0.0f, 0.0f, nullptr};
    switch (op) {
        case TC_REDUCE_MIN:
            return reduce_typed<S, ArgFold<TC_REDUCE_MIN>, uint32_t>(input, out, split->offset, plan, f, input_len, what);
        case TC_REDUCE_MAX:
            return reduce_typed<S, ArgFold<TC_REDUCE_MAX>, uint32_t>(input, out, split->offset, plan, f, input_len, what);
        default:
            return fail(TC_INVALID, "arg_reduce: Reduce " + std::to_string(op) + " is not Min or Max");
    }
}

// ---- whole buffers ------------------------------------------------------------

// Stage one: each block folds a strided share into `partial[block]`; stage
// two: one block folds the partials in order into `result`.
// PACKED reads 16-byte packs, four per operand in flight per lane; NT
// streams inputs larger than the Infinity Cache past it.
template <typename S, uint32_t OP, bool DOT, bool PACKED, bool NT>
__global__ void __launch_bounds__(256) total_kernel(const S* __restrict__ a, const S* __restrict__ b,
                                                    uint64_t n, float* __restrict__ partial) {
    using E = Elem<S>;
    using P = Fold<OP>;
    constexpr int V = Pack<S>::N;
    constexpr int U = 4;
    __shared__ float stage[4];
    float s = P::init();
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    const uint64_t first = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (PACKED) {
        const Pack<S>* pa = reinterpret_cast<const Pack<S>*>(a);
        const Pack<S>* pb = reinterpret_cast<const Pack<S>*>(b);
        const uint64_t packs = n / V;
        uint64_t p = first;
        for (; p + (U - 1) * stride < packs; p += U * stride) {
            uint4 wa[U], wb[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                wa[u] = load_word<NT>(pa + p + u * stride);
                if (DOT) wb[u] = load_word<NT>(pb + p + u * stride);
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                Pack<S> x, y;
                __builtin_memcpy(&x, &wa[u], 16);
                if (DOT) __builtin_memcpy(&y, &wb[u], 16);
#pragma unroll
                for (int j = 0; j < V; j++) {
                    const float e = E::widen(x.v[j]);
                    P::add(s, DOT ? e * E::widen(y.v[j]) : e, 0);
                }
            }
        }
        for (; p < packs; p += stride) {
            Pack<S> x = pa[p];
#pragma unroll
            for (int j = 0; j < V; j++) {
                const float e = E::widen(x.v[j]);
                P::add(s, DOT ? e * E::widen(pb[p].v[j]) : e, 0);
            }
        }
        const uint64_t i = packs * V + first;
        if (i < n) {
            const float x = E::widen(a[i]);
            P::add(s, DOT ? x * E::widen(b[i]) : x, 0);
        }
    } else {
        for (uint64_t i = first; i < n; i += stride) {
            const float x = E::widen(a[i]);
            P::add(s, DOT ? x * E::widen(b[i]) : x, 0);
        }
    }
    s = wave_reduce<P>(s);
    if (threadIdx.x % 64 == 0) stage[threadIdx.x / 64] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = stage[0];
        for (int w = 1; w < 4; w++) t = P::merge(t, stage[w]);
        partial[blockIdx.x] = t;
    }
}

// 256 threads, each folding every 256th partial with four loads in flight,
// then the waves in order: a fixed order, so the result does not depend on
// timing, and a few load round trips rather than count / 64.
template <uint32_t OP>
__global__ void __launch_bounds__(256) finish_total_kernel(const float* __restrict__ partial, uint32_t count,
                                                           float* __restrict__ result) {
    using P = Fold<OP>;
    __shared__ float stage[4];
    float s = P::init();
    uint32_t i = threadIdx.x;
    for (; i + 3 * 256 < count; i += 4 * 256) {
        float x[4];
#pragma unroll
        for (int u = 0; u < 4; u++) x[u] = partial[i + u * 256];
#pragma unroll
        for (int u = 0; u < 4; u++) P::add(s, x[u], 0);
    }
    for (; i < count; i += 256) P::add(s, partial[i], 0);
    s = wave_reduce<P>(s);
    if (threadIdx.x % 64 == 0) stage[threadIdx.x / 64] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = stage[0];
        for (int w = 1; w < 4; w++) t = P::merge(t, stage[w]);
        *result = t;
    }
}

// Blocks of `total` for `n` elements: at most four a CU.
inline uint32_t total_blocks(uint64_t n) { return grid_for(n, 256 * 8, 4); }

// `total` with the blocks' partials in `partial` (total_blocks(n) floats),
// which every block writes before the finishing wave reads it: nothing in it
// has to start at zero.
template <typename S, uint32_t OP, bool DOT>
int total_into(const void* a, const void* b, uint64_t n, float* result, float* partial, const char* what,
               hipStream_t s) {
    const uint32_t blocks = total_blocks(n);
    const S* pa = static_cast<const S*>(a);
    const S* pb = static_cast<const S*>(b);
    const bool packed = aligned16(a) && (!DOT || aligned16(b));
    const bool stream = n * sizeof(S) * (DOT ? 2 : 1) >= kStreamBytes;
    if (packed && stream) {
        total_kernel<S, OP, DOT, true, true><<<blocks, 256, 0, s>>>(pa, pb, n, partial);
    } else if (packed) {
        total_kernel<S, OP, DOT, true, false><<<blocks, 256, 0, s>>>(pa, pb, n, partial);
    } else {
        total_kernel<S, OP, DOT, false, false><<<blocks, 256, 0, s>>>(pa, pb, n, partial);
    }
    int status = check_launch(what);
    if (status == TC_OK) {
        finish_total_kernel<OP><<<1, 256, 0, s>>>(partial, blocks, result);
        status = check_launch(what);
    }
    return status;
}

template <typename S, uint32_t OP, bool DOT>
int total(const void* a, const void* b, uint64_t n, float* result, const char* what) {
    TC_STREAM(s);
    void* scratch = nullptr;
    int status = tc_alloc(total_blocks(n) * sizeof(float), &scratch);
    if (status != TC_OK) return status;
    status = total_into<S, OP, DOT>(a, b, n, result, static_cast<float*>(scratch), what, s);
    tc_free(scratch);
    return status;
}

// ---- the whole-buffer fold without allocation ----------------------------
//
// Partials of `tc_vector_reduce_noalloc` live in the file-scope device array
// `scratch` (top of this file), one copy per GPU.  Host code reaches a GPU's
// copy only through the address hipGetSymbolAddress gives for it with that
// device current, looked up on the entry point's first call on the device
// and kept; the array's name in host code is a host-side stand-in, never
// passed to a kernel.
//
// Calls on one GPU share the array, so each GPU's copy has an owner: the
// stream of the last call that used it, with an event recorded after that
// call's kernels.  A call from another stream takes the array over only once
// that event has passed; while the owner's last use is still queued the call
// is refused (TC_UNSUPPORTED) rather than racing on the array.  The check,
// the launch and the event's record are one step under a lock, so two
// threads cannot both take the array over.  Replays of a captured call are
// not tracked: a graph holding one must not replay beside eager calls or
// other graphs holding one on that GPU.
struct StaticPartials {
    float* address = nullptr;
    hipEvent_t last_use = nullptr;
    hipStream_t owner = nullptr;
};

std::mutex scratch_mutex;
std::unordered_map<int, StaticPartials> scratch_by_device;

// The device's array, set up on its first call there; `scratch_mutex` held.
int static_partials(StaticPartials** out) {
    int device = -1;
    hipError_t error = hipGetDevice(&device);
    if (error != hipSuccess) return fail(TC_DEVICE, std::string("vector_reduce_noalloc: ") + hipGetErrorString(error));
    auto found = scratch_by_device.find(device);
    if (found == scratch_by_device.end()) {
        StaticPartials entry;
        void* address = nullptr;
        error = hipGetSymbolAddress(&address, HIP_SYMBOL(::scratch));
        if (error != hipSuccess || address == nullptr) {
            (void)hipGetLastError();
            return fail(TC_DEVICE, std::string("vector_reduce_noalloc: the partials array of device ") +
                                       std::to_string(device) + ": " + hipGetErrorString(error));
        }
        entry.address = static_cast<float*>(address);
        error = hipEventCreateWithFlags(&entry.last_use, hipEventDisableTiming);
        if (error != hipSuccess) {
            (void)hipGetLastError();
            return fail(TC_DEVICE, std::string("vector_reduce_noalloc: ") + hipGetErrorString(error));
        }
        found = scratch_by_device.emplace(device, entry).first;
    }
    *out = &found->second;
    return TC_OK;
}

template <typename S, uint32_t OP>
int total_noalloc(const void* a, uint64_t n, float* result) {
    TC_STREAM(s);
    const uint32_t blocks = total_blocks(n);
    if (blocks > kStaticPartials) {
        return fail(TC_UNSUPPORTED, "vector_reduce_noalloc: " + std::to_string(blocks) + " partials, over the " +
                                        std::to_string(kStaticPartials) + " the library holds");
    }
    std::lock_guard<std::mutex> lock(scratch_mutex);
    StaticPartials* partials = nullptr;
    int status = static_partials(&partials);
    if (status != TC_OK) return status;
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &capture) != hipSuccess) (void)hipGetLastError();
    if (partials->owner != nullptr && partials->owner != s) {
        const hipError_t state = hipEventQuery(partials->last_use);
        if (state != hipSuccess) {
            if (state != hipErrorNotReady) (void)hipGetLastError();
            return fail(TC_UNSUPPORTED, "vector_reduce_noalloc: the device's partials array is in use by another "
                                        "stream's call that has not finished");
        }
    }
    status = total_into<S, OP, false>(a, nullptr, n, result, partials->address, "vector_reduce_noalloc", s);
    if (status != TC_OK || capture != hipStreamCaptureStatusNone) return status;
    const hipError_t error = hipEventRecord(partials->last_use, s);
    if (error != hipSuccess) {
        (void)hipGetLastError();
        // Without the record, no later check could see this call: wait for
        // it, so the array is free when the next owner takes it.
        (void)host_wait(s);
        partials->owner = nullptr;
        return TC_OK;
    }
    partials->owner = s;
    return TC_OK;
}

// The moments of a whole buffer, in the manner of `total`: each block folds
// its grid-stride share (16-byte packs when aligned, each pack's exact
// two-pass moments merged in), the waves' states merge in the closed form,
// and one wave merges the blocks' states into `result[0]` (the mean) and
// `result[1]` (the sum of squared deviations), unrounded f32; NaNs for an
// empty buffer (statistics/mod.rs:428-434).
template <typename S, bool PACKED>
__global__ void __launch_bounds__(256) moments_total_kernel(const S* __restrict__ a, uint64_t n,
                                                            Moments* __restrict__ partial) {
    using E = Elem<S>;
    constexpr int V = Pack<S>::N;
    __shared__ Moments stage[4];
    Moments s = Var::init();
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    const uint64_t first = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (PACKED) {
        const uint64_t packs = n / V;
        for (uint64_t p = first; p < packs; p += stride) {
            float x[V];
            load_packs<S, 1, false>(reinterpret_cast<const Pack<S>*>(a) + p, x);
            Var::add_chunk(s, x, 0);
        }
        if (blockIdx.x == 0 && threadIdx.x < n - packs * V) Var::add(s, E::widen(a[packs * V + threadIdx.x]), 0);
    } else {
        for (uint64_t i = first; i < n; i += stride) Var::add(s, E::widen(a[i]), 0);
    }
    s = wave_reduce<Var>(s);
    if (threadIdx.x % 64 == 0) stage[threadIdx.x / 64] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        Moments t = stage[0];
        for (int w = 1; w < 4; w++) t = merge_moments(t, stage[w]);
        partial[blockIdx.x] = t;
    }
}

__global__ void __launch_bounds__(64) finish_moments_kernel(const Moments* __restrict__ partial, uint32_t count,
                                                            float* __restrict__ result) {
    Moments s = Var::init();
    for (uint32_t i = threadIdx.x; i < count; i += 64) s = merge_moments(s, partial[i]);
    s = wave_reduce<Var>(s);
    if (threadIdx.x == 0) {
        result[0] = s.n == 0.0f ? NAN : s.mean;
        result[1] = s.n == 0.0f ? NAN : s.m2;
    }
}

template <typename S>
int total_moments(const void* a, uint64_t n, float* result) {
    TC_STREAM(s);
    const uint32_t blocks = grid_for(n, 256 * 16, 4);
    void* scratch = nullptr;
    int status = tc_alloc(blocks * sizeof(Moments), &scratch);
    if (status != TC_OK) return status;
    Moments* partial = static_cast<Moments*>(scratch);
    const S* in = static_cast<const S*>(a);
    if (aligned16(in)) {
        moments_total_kernel<S, true><<<blocks, 256, 0, s>>>(in, n, partial);
    } else {
        moments_total_kernel<S, false><<<blocks, 256, 0, s>>>(in, n, partial);
    }
    status = check_launch("moments");
    if (status == TC_OK) {
        finish_moments_kernel<<<1, 64, 0, s>>>(partial, blocks, result);
        status = check_launch("moments");
    }
    tc_free(scratch);
    return status;
}

}  // namespace
}  // namespace tc

namespace tc {
int reduce_moments(uint32_t dtype, const void* input, uint64_t input_len, const tc_split* split, void* means,
                   void* deviations) {
    TC_DISPATCH_FLOAT(dtype, "row_moments", S, return moments_typed<S>(input, input_len, split, means, deviations));
    return TC_OK;
}
}  // namespace tc

using namespace tc;

namespace tc {
namespace {

// How many results a split keeps (the product of its kept extents; one for
// a full reduction).
uint64_t split_results(const tc_split* split) {
    uint64_t results = 1;
    for (uint32_t k = 0; k < split->kept_rank && k < static_cast<uint32_t>(kMaxRank); k++) results *= split->kept[k];
    return results;
}

}  // namespace
}  // namespace tc

extern "C" {

int tc_reduce_axes(uint32_t dtype, const void* input, uint64_t input_len, const tc_split* split,
                   uint32_t kind, uint32_t op, uint64_t divisor, void* out) {
    if ((input_len != 0 && input == nullptr) || (split_results(split) != 0 && out == nullptr)) {
        return null_operand("reduce_axes");
    }
    TC_DISPATCH_FLOAT(dtype, "reduce_axes", S,
                      return reduce_axes_typed<S>(input, input_len, split, kind, op, divisor, out));
    return TC_OK;
}

int tc_arg_reduce(uint32_t dtype, const void* input, uint64_t input_len, const tc_split* split,
                  uint32_t op, uint32_t* out) {
    if ((input_len != 0 && input == nullptr) || (split_results(split) != 0 && out == nullptr)) {
        return null_operand("arg_reduce");
    }
    TC_DISPATCH_FLOAT(dtype, "arg_reduce", S, return arg_reduce_typed<S>(input, input_len, split, op, out));
    return TC_OK;
}

int tc_vector_reduce(uint32_t dtype, const void* a, uint64_t n, uint32_t op, float* result) {
    if (result == nullptr || (n != 0 && a == nullptr)) return null_operand("vector_reduce");
    switch (op) {
        case TC_REDUCE_SUM:
            TC_DISPATCH_FLOAT(dtype, "vector_reduce", S,
                              return total<S, TC_REDUCE_SUM, false>(a, nullptr, n, result, "vector_reduce"));
            break;
        case TC_REDUCE_MIN:
            TC_DISPATCH_FLOAT(dtype, "vector_reduce", S,
                              return total<S, TC_REDUCE_MIN, false>(a, nullptr, n, result, "vector_reduce"));
            break;
        case TC_REDUCE_MAX:
            TC_DISPATCH_FLOAT(dtype, "vector_reduce", S,
                              return total<S, TC_REDUCE_MAX, false>(a, nullptr, n, result, "vector_reduce"));
            break;
        default:
            return fail(TC_INVALID, "vector_reduce: no Reduce " + std::to_string(op));
    }
    return TC_OK;
}

int tc_moments(uint32_t dtype, const void* a, uint64_t n, float* result) {
    if (result == nullptr || (n != 0 && a == nullptr)) return null_operand("moments");
    TC_DISPATCH_FLOAT(dtype, "moments", S, return total_moments<S>(a, n, result));
    return TC_OK;
}

int tc_vector_reduce_noalloc(uint32_t dtype, const void* a, uint64_t n, uint32_t op, float* result) {
    if (result == nullptr || (n != 0 && a == nullptr)) return null_operand("vector_reduce_noalloc");
    switch (op) {
        case TC_REDUCE_SUM:
            TC_DISPATCH_FLOAT(dtype, "vector_reduce_noalloc", S, return total_noalloc<S, TC_REDUCE_SUM>(a, n, result));
            break;
        case TC_REDUCE_MIN:
            TC_DISPATCH_FLOAT(dtype, "vector_reduce_noalloc", S, return total_noalloc<S, TC_REDUCE_MIN>(a, n, result));
            break;
        case TC_REDUCE_MAX:
            TC_DISPATCH_FLOAT(dtype, "vector_reduce_noalloc", S, return total_noalloc<S, TC_REDUCE_MAX>(a, n, result));
            break;
        default: return fail(TC_INVALID, "vector_reduce_noalloc: no Reduce " + std::to_string(op));
    }
    return TC_OK;
}

int tc_dot(uint32_t dtype, const void* a, const void* b, uint64_t n, float* result) {
    if (result == nullptr || (n != 0 && any_null({a, b}))) return null_operand("dot");
    TC_DISPATCH_FLOAT(dtype, "dot", S, return total<S, TC_REDUCE_SUM, true>(a, b, n, result, "dot"));
    return TC_OK;
}

}  // extern "C"
