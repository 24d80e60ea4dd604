// Matrix-vector products: `Kernels::matvec` / `matvec_add` (tensors/kernels.rs:901-908,
// matrix.rs:675-737) and `Kernels::vecmat` (kernels.rs:899, vector.rs:491).
//
// Both stream the matrix once from HBM, so both are bandwidth kernels:
//  - matvec: one wave per row, lanes reading 16 bytes of the row at a time
//    (eight such reads in flight per lane),
//    a 64-lane shuffle tree for the dot product.  The vector stays hot in L2.
// A matrix as large as the Infinity Cache is read with non-temporal loads,
// streaming past the caches so they keep the vector (measured at 8192 x 8192
// f32: matvec 72.7% -> 80.3% of HBM, vecmat 69.3% -> 74.2%).
//  - vecmat: lanes on neighbouring columns, 16 bytes of a row each, so
//    every row read is one coalesced run; four row groups split the rows
//    inside a block, and tall matrices split their rows across blocks,
//    combined in order by a second pass, so the result does not depend on
//    timing.
// Accumulation is f32, rounded once to the element type (compact.rs:223-231).

#include "common.hpp"

namespace tc {
namespace {

template <typename S>
struct alignas(16) Pack {
    static constexpr int N = 16 / sizeof(S);
    S v[N];
};

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, 64);
    return v;
}

template <typename S, bool PACKED, bool NT>
__global__ void __launch_bounds__(256) matvec_kernel(const S* __restrict__ m, const S* __restrict__ v,
                                                     S* __restrict__ y, uint64_t rows, uint64_t cols,
                                                     bool accumulate) {
    using E = Elem<S>;
    constexpr int N = Pack<S>::N;
    const int lane = threadIdx.x % 64;
    const uint64_t waves = static_cast<uint64_t>(gridDim.x) * (blockDim.x / 64);
    for (uint64_t r = static_cast<uint64_t>(blockIdx.x) * (blockDim.x / 64) + threadIdx.x / 64; r < rows;
         r += waves) {
        const S* row = m + r * cols;
        float total = 0.0f;
        if (PACKED) {
            // Eight 16-byte packs of the row in flight per lane (measured:
            // 73% of HBM at 8192 x 8192 f32, against 72% with four).
            const Pack<S>* pr = reinterpret_cast<const Pack<S>*>(row);
            const Pack<S>* pv = reinterpret_cast<const Pack<S>*>(v);
            const uint64_t packs = cols / N;
            uint64_t p = lane;
            for (; p + 7 * 64 < packs; p += 8 * 64) {
                Pack<S> a[8], b[8];
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const uint4 w = load_word<NT>(pr + p + u * 64);
                    __builtin_memcpy(&a[u], &w, 16);
                    b[u] = pv[p + u * 64];
                }
#pragma unroll
                for (int u = 0; u < 8; u++) {
#pragma unroll
                    for (int k = 0; k < N; k++) total += E::widen(a[u].v[k]) * E::widen(b[u].v[k]);
                }
            }
            for (; p < packs; p += 64) {
                Pack<S> a = pr[p], b = pv[p];
#pragma unroll
                for (int k = 0; k < N; k++) total += E::widen(a.v[k]) * E::widen(b.v[k]);
            }
        } else {
            for (uint64_t c = lane; c < cols; c += 64) total += E::widen(row[c]) * E::widen(v[c]);
        }
        total = wave_sum(total);
        if (lane == 0) {
            if (accumulate) total += E::widen(y[r]);
            y[r] = E::narrow(total);
        }
    }
}

constexpr int kGroups = 4;

// Block: 64 lanes x kGroups row groups.  A lane owns W packs of V columns,
// 64 packs apart, so one wave reads 64·V·W contiguous columns of a row (4 KiB
// for f32 at V = W = 4); `split` picks the rows.  With one split the block
// finishes its columns; otherwise it writes f32 partial sums to
// `partial[split][col]`.
template <typename S, int V, int W, bool NT>
__global__ void __launch_bounds__(256) vecmat_kernel(const S* __restrict__ v, const S* __restrict__ m,
                                                     S* __restrict__ y, float* __restrict__ partial,
                                                     uint64_t rows, uint64_t cols, uint64_t tiles,
                                                     uint64_t splits, uint64_t per_split, bool accumulate) {
    using E = Elem<S>;
    constexpr int kTile = 64 * V * W;
    __shared__ float stage[kGroups][kTile];
    const int lane = threadIdx.x % 64;
    const int group = threadIdx.x / 64;
    const uint64_t tile = blockIdx.x % tiles;
    const uint64_t split = blockIdx.x / tiles;
    const uint64_t base = tile * kTile + lane * V;
    const uint64_t begin = split * per_split;
    const uint64_t end = min(begin + per_split, rows);
    const uint64_t span = end > begin ? end - begin : 0;
    const uint64_t per_group = (span + kGroups - 1) / kGroups;
    const uint64_t first = min(begin + group * per_group, end);
    const uint64_t last = min(first + per_group, end);
    float acc[W][V];
#pragma unroll
    for (int u = 0; u < W; u++) {
#pragma unroll
        for (int k = 0; k < V; k++) acc[u][k] = 0.0f;
    }
    // Columns are whole packs (cols % V == 0 when V > 1), so a pack is either
    // inside the matrix or wholly past its last column.
    bool live[W];
#pragma unroll
    for (int u = 0; u < W; u++) live[u] = base + u * 64 * V < cols;
    uint64_t r = first;
    if (V > 1) {
        // Two rows' packs in flight per lane before any is used: measured at
        // 8192 x 8192 f32, four or eight rows in flight were slower (66% and
        // 61% of HBM against 70%).
        constexpr int R = 2;
        for (; r + R <= last; r += R) {
            Pack<S> p[R][W];
            float w[R];
#pragma unroll
            for (int q = 0; q < R; q++) {
                w[q] = E::widen(v[r + q]);
#pragma unroll
                for (int u = 0; u < W; u++) {
                    if (live[u]) {
                        const uint4 word = load_word<NT>(m + (r + q) * cols + base + u * 64 * V);
                        __builtin_memcpy(&p[q][u], &word, 16);
                    }
                }
            }
#pragma unroll
            for (int q = 0; q < R; q++) {
#pragma unroll
                for (int u = 0; u < W; u++) {
                    if (!live[u]) continue;
#pragma unroll
                    for (int k = 0; k < V; k++) acc[u][k] += w[q] * E::widen(p[q][u].v[k]);
                }
            }
        }
    }
    for (; r < last; r++) {
        const float w = E::widen(v[r]);
#pragma unroll
        for (int u = 0; u < W; u++) {
            if (!live[u]) continue;
            if (V > 1) {
                const uint4 word = load_word<NT>(m + r * cols + base + u * 64 * V);
                Pack<S> p;
                __builtin_memcpy(&p, &word, 16);
#pragma unroll
                for (int k = 0; k < V; k++) acc[u][k] += w * E::widen(p.v[k]);
            } else {
                acc[u][0] += w * E::widen(m[r * cols + base + u * 64]);
            }
        }
    }
#pragma unroll
    for (int u = 0; u < W; u++) {
#pragma unroll
        for (int k = 0; k < V; k++) stage[group][u * 64 * V + lane * V + k] = acc[u][k];
    }
    __syncthreads();
    if (group == 0) {
#pragma unroll
        for (int u = 0; u < W; u++) {
            if (!live[u]) continue;
            const uint64_t col = base + u * 64 * V;
#pragma unroll
            for (int k = 0; k < V; k++) {
                float total = stage[0][u * 64 * V + lane * V + k];
#pragma unroll
                for (int g = 1; g < kGroups; g++) total += stage[g][u * 64 * V + lane * V + k];
                if (splits == 1) {
                    if (accumulate) total += E::widen(y[col + k]);
                    y[col + k] = E::narrow(total);
                } else {
                    partial[split * cols + col + k] = total;
                }
            }
        }
    }
}

// The splits' partial sums of 64 columns a block: lane = column, each of
// the four waves folding a quarter of the splits in order (eight loads in
// flight), then the quarters in order, so the sum does not depend on timing.
template <typename S>
__global__ void __launch_bounds__(256) vecmat_combine_kernel(const float* __restrict__ partial, S* __restrict__ y,
                                                             uint64_t cols, uint64_t splits, bool accumulate) {
    __shared__ float quarter[kGroups][64];
    const int lane = threadIdx.x % 64;
    const int wave = threadIdx.x / 64;
    const uint64_t c = static_cast<uint64_t>(blockIdx.x) * 64 + lane;
    const uint64_t per_wave = (splits + kGroups - 1) / kGroups;
    const uint64_t k0 = min(wave * per_wave, splits);
    const uint64_t k1 = min(k0 + per_wave, splits);
    float total = 0.0f;
    if (c < cols) {
        uint64_t k = k0;
        for (; k + 8 <= k1; k += 8) {
            float x[8];
#pragma unroll
            for (int u = 0; u < 8; u++) x[u] = partial[(k + u) * cols + c];
#pragma unroll
            for (int u = 0; u < 8; u++) total += x[u];
        }
        for (; k < k1; k++) total += partial[k * cols + c];
    }
    quarter[wave][lane] = total;
    __syncthreads();
    if (wave == 0 && c < cols) {
        float sum = quarter[0][lane];
#pragma unroll
        for (int g = 1; g < kGroups; g++) sum += quarter[g][lane];
        if (accumulate) sum += Elem<S>::widen(y[c]);
        y[c] = Elem<S>::narrow(sum);
    }
}

template <typename S>
int matvec_typed(bool accumulate, uint64_t rows, uint64_t cols, const void* m, const void* v, void* y) {
    TC_STREAM(s);
    if (rows == 0) return TC_OK;
    const S* pm = static_cast<const S*>(m);
    const S* pv = static_cast<const S*>(v);
    S* py = static_cast<S*>(y);
    const bool packed = cols % Pack<S>::N == 0 && aligned16(m) && aligned16(v);
    const bool stream = rows * cols * sizeof(S) >= kStreamBytes;
    const uint32_t blocks = grid_for(rows, 4, 32);
    if (packed && stream) {
        matvec_kernel<S, true, true><<<blocks, 256, 0, s>>>(pm, pv, py, rows, cols, accumulate);
    } else if (packed) {
        matvec_kernel<S, true, false><<<blocks, 256, 0, s>>>(pm, pv, py, rows, cols, accumulate);
    } else {
        matvec_kernel<S, false, false><<<blocks, 256, 0, s>>>(pm, pv, py, rows, cols, accumulate);
    }
    return check_launch("matvec");
}

// `per_cu`: the blocks a CU that row splits fill, when the column tiles
// alone do not.
template <typename S, int V, int W, bool NT>
int launch_vecmat(const S* v, const S* m, S* y, uint64_t rows, uint64_t cols, bool accumulate, uint64_t per_cu,
                  hipStream_t s) {
    const uint64_t tiles = (cols + 64 * V * W - 1) / (64 * V * W);
    const uint64_t want = static_cast<uint64_t>(compute_units()) * per_cu;
    uint64_t splits = 1;
    if (tiles < want) {
        splits = (want + tiles - 1) / tiles;
        const uint64_t most = rows / (kGroups * 16);
        if (splits > most) splits = most;
        if (splits < 1) splits = 1;
    }
    const uint64_t per_split = (rows + splits - 1) / splits;
    splits = rows == 0 ? 1 : (rows + per_split - 1) / per_split;
    float* partial = nullptr;
    if (splits > 1) {
        void* scratch = nullptr;
        int status = tc_alloc(splits * cols * sizeof(float), &scratch);
        if (status != TC_OK) return status;
        partial = static_cast<float*>(scratch);
    }
    vecmat_kernel<S, V, W, NT><<<static_cast<uint32_t>(tiles * splits), 256, 0, s>>>(v, m, y, partial, rows, cols,
                                                                                 tiles, splits, per_split, accumulate);
    int status = check_launch("vecmat");
    if (status == TC_OK && splits > 1) {
        vecmat_combine_kernel<S><<<static_cast<uint32_t>((cols + 63) / 64), 256, 0, s>>>(partial, y, cols, splits, accumulate);
        status = check_launch("vecmat");
    }
    if (partial != nullptr) tc_free(partial);
    return status;
}

template <typename S>
int vecmat_typed(bool accumulate, uint64_t rows, uint64_t cols, const void* v, const void* m, void* y) {
    TC_STREAM(s);
    if (cols == 0) return TC_OK;
    const S* pv = static_cast<const S*>(v);
    const S* pm = static_cast<const S*>(m);
    S* py = static_cast<S*>(y);
    constexpr int V = Pack<S>::N;
    if (cols % V == 0 && aligned16(m)) {
        // Streamed: two packs a lane on two blocks a CU.  Measured at 8192 x
        // 8192 f32 with non-temporal loads, as a share of HBM: 78% against
        // 74% for one pack a lane on four blocks a CU (one pack on two: 65%;
        // four packs on two: 77%; two packs on one, four or eight: 60%,
        // 77% and 71%).  Before streaming, one pack a lane on four blocks a
        // CU led (70%, against 68% and 66% for two and four packs).
        if (rows * cols * sizeof(S) >= kStreamBytes) {
            return launch_vecmat<S, V, 2, true>(pv, pm, py, rows, cols, accumulate, 2, s);
        }
        return launch_vecmat<S, V, 1, false>(pv, pm, py, rows, cols, accumulate, 4, s);
    }
    return launch_vecmat<S, 1, 1, false>(pv, pm, py, rows, cols, accumulate, 4, s);
}

}  // namespace

int vector_product(uint32_t dtype, bool row_vector, bool accumulate, uint64_t rows, uint64_t cols, const void* matrix,
                   const void* vector, void* out) {
    if (row_vector) {
        TC_DISPATCH_FLOAT(dtype, "vecmat", S, return vecmat_typed<S>(accumulate, rows, cols, vector, matrix, out));
    } else {
        TC_DISPATCH_FLOAT(dtype, "matvec", S, return matvec_typed<S>(accumulate, rows, cols, matrix, vector, out));
    }
    return TC_OK;
}

}  // namespace tc

using namespace tc;

extern "C" {

int tc_matvec(uint32_t dtype, int accumulate, uint64_t rows, uint64_t cols, const void* matrix, const void* vector,
              void* out) {
    if (rows != 0 && (out == nullptr || (cols != 0 && (matrix == nullptr || vector == nullptr)))) {
        return fail(TC_INVALID, "matvec: a null operand");
    }
    TC_DISPATCH_FLOAT(dtype, "matvec", S, return matvec_typed<S>(accumulate != 0, rows, cols, matrix, vector, out));
    return TC_OK;
}

int tc_vecmat(uint32_t dtype, uint64_t rows, uint64_t cols, const void* vector, const void* matrix, void* out) {
    if (cols != 0 && (out == nullptr || (rows != 0 && (matrix == nullptr || vector == nullptr)))) {
        return fail(TC_INVALID, "vecmat: a null operand");
    }
    TC_DISPATCH_FLOAT(dtype, "vecmat", S, return vecmat_typed<S>(false, rows, cols, vector, matrix, out));
    return TC_OK;
}

}  // extern "C"
