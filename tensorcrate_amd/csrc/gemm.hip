// Matrix products on CDNA4 matrix cores: `Kernels::matmul`, `matmul_add`
// and `matmul_transposed_add` (tensors/kernels.rs:956-985), including the
// compact types' f32-output `matmul_f32` (tensors/backend.rs:904-922).
//
// The arithmetic is the reference's: f16 and bf16 operands widen exactly,
// every product accumulates in f32, and a 16-bit output rounds once, to
// nearest even (compact.rs:223-253).  The order of the f32 additions is the
// matrix cores', not the host's left-to-right FMA chain, so results agree
// with the host within the f32 tolerance the reference's Metal products keep.
//
// One kernel shape carries every product: C[M x N] (+)= A[M x K] . Bt[N x K]^T
// with both operands K-contiguous, which is how a matrix core wants its
// operands (each lane feeds it consecutive k).  A product whose operand is
// stored the other way round is first transposed into a scratch block with
// the LDS tile transpose.
//
//  - 16-bit operands: v_mfma_f32_32x32x16_{bf16,f16}.  A 256 x 128 block tile
//    and 64-deep k steps; four waves, each owning a 128 x 64 sub-tile as
//    4 x 2 matrix-core tiles (128 f32 accumulators per lane).
//  - f32 operands: v_mfma_f32_16x16x4_f32, the same block tile with 32-deep k
//    steps and 8 x 4 tiles of 16 x 16 per wave.  One 16-byte LDS read feeds
//    four consecutive matrix-core steps, since the sum over k does not care
//    which lane holds which k as long as both operands agree.
//
// Operands travel global -> registers -> LDS, double-buffered so the next k
// step's loads are in flight while the matrix cores work on this one; LDS
// rows are padded by 16 bytes so a wave's 16-byte operand reads spread over
// the banks.  Block tiles are ordered in groups of rows, and the linear
// block index is first spread so that the blocks one XCD runs are
// neighbours, which keeps each XCD's L2 working on a few A and B panels.

#include "common.hpp"

namespace tc {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBM = 256;
constexpr int kBN = 128;
constexpr int kThreads = 256;
constexpr int kGroupM = 8;  // block-tile rows per ordering group

template <typename S>
struct Mfma16;
template <>
struct Mfma16<bf16_t> {
    __device__ static f32x16 step(uint4 a, uint4 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    }
};
template <>
struct Mfma16<_Float16> {
    __device__ static f32x16 step(uint4 a, uint4 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
};

// The block tile a block computes, from its linear index: spread across the
// XCDs first (hardware hands consecutive blocks to consecutive XCDs), then
// grouped so that neighbouring blocks share rows of A.
__device__ __forceinline__ void tile_of(uint32_t block, uint32_t tiles_m, uint32_t tiles_n, uint32_t& tm,
                                        uint32_t& tn) {
    const uint32_t total = tiles_m * tiles_n;
    constexpr uint32_t kXcds = 8;
    if (total % kXcds == 0) {
        block = (block % kXcds) * (total / kXcds) + block / kXcds;
    }
    const uint32_t per_group = kGroupM * tiles_n;
    const uint32_t group = block / per_group;
    const uint32_t first_m = group * kGroupM;
    const uint32_t rows = min(tiles_m - first_m, static_cast<uint32_t>(kGroupM));
    const uint32_t in_group = block - group * per_group;
    tm = first_m + in_group % rows;
    tn = in_group / rows;
}

// 16 bytes of row `row`, from column `k`, of a K-contiguous operand with
// `rows` rows of `K` elements of `E` bytes; zeros outside it.  `fast` says the
// whole operand is 16-byte aligned row by row.
template <int E>
__device__ __forceinline__ uint4 load16(const uint8_t* base, uint32_t row, uint32_t k, uint32_t rows,
                                        uint32_t K, bool fast) {
    constexpr uint32_t per = 16 / E;
    if (row < rows && fast && k + per <= K) {
        return *reinterpret_cast<const uint4*>(base + (static_cast<uint64_t>(row) * K + k) * E);
    }
    uint8_t bytes[16] = {};
    if (row < rows) {
        for (uint32_t e = 0; e < per; e++) {
            if (k + e < K) {
                const uint8_t* at = base + (static_cast<uint64_t>(row) * K + k + e) * E;
                for (int b = 0; b < E; b++) bytes[e * E + b] = at[b];
            }
        }
    }
    uint4 out;
    __builtin_memcpy(&out, bytes, 16);
    return out;
}

template <typename O>
__device__ __forceinline__ void store_out(O* c, uint64_t at, float v, bool accumulate) {
    using E = Elem<O>;
    if (accumulate) v += E::widen(c[at]);
    c[at] = E::narrow(v);
}

// ---- 16-bit operands ------------------------------------------------------------

constexpr int kBK16 = 64;
constexpr int kLd16 = kBK16 + 8;  // padded LDS row, in elements

template <typename S, typename O>
__global__ void __launch_bounds__(kThreads) gemm16_kernel(const S* __restrict__ A, const S* __restrict__ Bt,
                                                          O* __restrict__ C, uint32_t M, uint32_t N,
                                                          uint32_t K, bool accumulate, bool fast) {
    __shared__ __attribute__((aligned(16))) S lds_a[2][kBM * kLd16];
    __shared__ __attribute__((aligned(16))) S lds_b[2][kBN * kLd16];
    const uint32_t tiles_m = (M + kBM - 1) / kBM;
    const uint32_t tiles_n = (N + kBN - 1) / kBN;
    uint32_t tm, tn;
    tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const uint32_t m0 = tm * kBM, n0 = tn * kBN;
    const int t = threadIdx.x;
    const int lane = t % 64;
    const int wave = t / 64;
    const int wm = wave / 2, wn = wave % 2;  // 2 x 2 waves of 128 x 64
    const uint8_t* a_bytes = reinterpret_cast<const uint8_t*>(A);
    const uint8_t* b_bytes = reinterpret_cast<const uint8_t*>(Bt);

    // Global chunk (row, 16-byte column) each thread stages: A has 8 per
    // thread, B 4; eight threads cover one 128-byte row segment.
    const uint32_t chunk_row = t / 8, chunk_col = (t % 8) * 8;
    uint4 stage_a[8], stage_b[4];
    auto fetch = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < 8; i++)
            stage_a[i] = load16<2>(a_bytes, m0 + chunk_row + 32 * i, k0 + chunk_col, M, K, fast);
#pragma unroll
        for (int i = 0; i < 4; i++)
            stage_b[i] = load16<2>(b_bytes, n0 + chunk_row + 32 * i, k0 + chunk_col, N, K, fast);
    };
    auto commit = [&](int buffer) {
#pragma unroll
        for (int i = 0; i < 8; i++)
            *reinterpret_cast<uint4*>(&lds_a[buffer][(chunk_row + 32 * i) * kLd16 + chunk_col]) = stage_a[i];
#pragma unroll
        for (int i = 0; i < 4; i++)
            *reinterpret_cast<uint4*>(&lds_b[buffer][(chunk_row + 32 * i) * kLd16 + chunk_col]) = stage_b[i];
    };

    f32x16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = f32x16{};

    const uint32_t steps = (K + kBK16 - 1) / kBK16;
    if (steps > 0) {
        fetch(0);
        commit(0);
        __syncthreads();
    }
    const int row_in = lane % 32;
    const int k_in = (lane / 32) * 8;
    for (uint32_t step = 0; step < steps; step++) {
        const int buffer = step & 1;
        const bool more = step + 1 < steps;
        if (more) fetch((step + 1) * kBK16);
        const S* la = lds_a[buffer];
        const S* lb = lds_b[buffer];
#pragma unroll
        for (int kk = 0; kk < kBK16; kk += 16) {
            uint4 a[4], b[2];
#pragma unroll
            for (int i = 0; i < 4; i++)
                a[i] = *reinterpret_cast<const uint4*>(&la[(wm * 128 + i * 32 + row_in) * kLd16 + kk + k_in]);
#pragma unroll
            for (int j = 0; j < 2; j++)
                b[j] = *reinterpret_cast<const uint4*>(&lb[(wn * 64 + j * 32 + row_in) * kLd16 + kk + k_in]);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 2; j++) acc[i][j] = Mfma16<S>::step(a[i], b[j], acc[i][j]);
        }
        if (more) commit(buffer ^ 1);
        __syncthreads();
    }

    // A 32 x 32 result tile: lane holds column lane % 32, and rows
    // 8 (e / 4) + 4 (lane / 32) + e % 4 for its 16 values e.
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint32_t col = n0 + wn * 64 + j * 32 + lane % 32;
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const uint32_t row = m0 + wm * 128 + i * 32 + 8 * (e / 4) + 4 * (lane / 32) + e % 4;
                if (row < M && col < N) store_out(C, static_cast<uint64_t>(row) * N + col, acc[i][j][e], accumulate);
            }
        }
    }
}

// ---- f32 operands ------------------------------------------------------------------

constexpr int kBK32 = 32;
constexpr int kLd32 = kBK32 + 4;

template <typename O>
__global__ void __launch_bounds__(kThreads) gemm32_kernel(const float* __restrict__ A, const float* __restrict__ Bt,
                                                          O* __restrict__ C, uint32_t M, uint32_t N,
                                                          uint32_t K, bool accumulate, bool fast) {
    __shared__ __attribute__((aligned(16))) float lds_a[2][kBM * kLd32];
    __shared__ __attribute__((aligned(16))) float lds_b[2][kBN * kLd32];
    const uint32_t tiles_m = (M + kBM - 1) / kBM;
    const uint32_t tiles_n = (N + kBN - 1) / kBN;
    uint32_t tm, tn;
    tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const uint32_t m0 = tm * kBM, n0 = tn * kBN;
    const int t = threadIdx.x;
    const int lane = t % 64;
    const int wave = t / 64;
    const int wm = wave / 2, wn = wave % 2;
    const uint8_t* a_bytes = reinterpret_cast<const uint8_t*>(A);
    const uint8_t* b_bytes = reinterpret_cast<const uint8_t*>(Bt);

    const uint32_t chunk_row = t / 8, chunk_col = (t % 8) * 4;
    uint4 stage_a[8], stage_b[4];
    auto fetch = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < 8; i++)
            stage_a[i] = load16<4>(a_bytes, m0 + chunk_row + 32 * i, k0 + chunk_col, M, K, fast);
#pragma unroll
        for (int i = 0; i < 4; i++)
            stage_b[i] = load16<4>(b_bytes, n0 + chunk_row + 32 * i, k0 + chunk_col, N, K, fast);
    };
    auto commit = [&](int buffer) {
#pragma unroll
        for (int i = 0; i < 8; i++)
            *reinterpret_cast<uint4*>(&lds_a[buffer][(chunk_row + 32 * i) * kLd32 + chunk_col]) = stage_a[i];
#pragma unroll
        for (int i = 0; i < 4; i++)
            *reinterpret_cast<uint4*>(&lds_b[buffer][(chunk_row + 32 * i) * kLd32 + chunk_col]) = stage_b[i];
    };

    f32x4 acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f32x4{};

    const uint32_t steps = (K + kBK32 - 1) / kBK32;
    if (steps > 0) {
        fetch(0);
        commit(0);
        __syncthreads();
    }
    const int row_in = lane % 16;
    const int k_in = (lane / 16) * 4;
    for (uint32_t step = 0; step < steps; step++) {
        const int buffer = step & 1;
        const bool more = step + 1 < steps;
        if (more) fetch((step + 1) * kBK32);
        const float* la = lds_a[buffer];
        const float* lb = lds_b[buffer];
#pragma unroll
        for (int kk = 0; kk < kBK32; kk += 16) {
            f32x4 a[8], b[4];
#pragma unroll
            for (int i = 0; i < 8; i++)
                a[i] = *reinterpret_cast<const f32x4*>(&la[(wm * 128 + i * 16 + row_in) * kLd32 + kk + k_in]);
#pragma unroll
            for (int j = 0; j < 4; j++)
                b[j] = *reinterpret_cast<const f32x4*>(&lb[(wn * 64 + j * 16 + row_in) * kLd32 + kk + k_in]);
#pragma unroll
            for (int e = 0; e < 4; e++)
#pragma unroll
                for (int i = 0; i < 8; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][e], b[j][e], acc[i][j], 0, 0, 0);
        }
        if (more) commit(buffer ^ 1);
        __syncthreads();
    }

    // A 16 x 16 result tile: lane holds column lane % 16 and rows
    // 4 (lane / 16) + e.
#pragma unroll
    for (int i = 0; i < 8; i++) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t col = n0 + wn * 64 + j * 16 + lane % 16;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t row = m0 + wm * 128 + i * 16 + 4 * (lane / 16) + e;
                if (row < M && col < N) store_out(C, static_cast<uint64_t>(row) * N + col, acc[i][j][e], accumulate);
            }
        }
    }
}

// ---- host side ---------------------------------------------------------------------

// A K-contiguous copy of an operand stored the other way round, in a block
// from the thread's cache: the `rows x cols` matrix `src` transposed.
int transposed_copy(const void* src, uint64_t rows, uint64_t cols, uint32_t width, void** out) {
    int status = tc_alloc(rows * cols * width, out);
    if (status != TC_OK) return status;
    status = tc_transpose(width, rows, cols, src, *out);
    if (status != TC_OK) tc_free(*out);
    return status;
}

template <typename S, typename O>
int launch_gemm(const S* a, const S* bt, O* c, uint64_t m, uint64_t k, uint64_t n, bool accumulate,
                hipStream_t s) {
    const uint32_t tiles = static_cast<uint32_t>(((m + kBM - 1) / kBM) * ((n + kBN - 1) / kBN));
    constexpr uint32_t E = sizeof(S);
    const bool fast = aligned16(a) && aligned16(bt) && (k * E) % 16 == 0;
    if constexpr (std::is_same<S, float>::value) {
        gemm32_kernel<O><<<tiles, kThreads, 0, s>>>(a, bt, c, static_cast<uint32_t>(m), static_cast<uint32_t>(n),
                                                    static_cast<uint32_t>(k), accumulate, fast);
    } else {
        gemm16_kernel<S, O><<<tiles, kThreads, 0, s>>>(a, bt, c, static_cast<uint32_t>(m),
                                                       static_cast<uint32_t>(n), static_cast<uint32_t>(k),
                                                       accumulate, fast);
    }
    return check_launch("matmul");
}

template <typename S, typename O>
int matmul_typed(uint32_t transposed, bool accumulate, uint64_t m, uint64_t k, uint64_t n, const void* a,
                 const void* b, void* c) {
    TC_STREAM(s);
    if (m == 0 || n == 0) return TC_OK;
    if (m > UINT32_MAX / 2 || n > UINT32_MAX / 2 || k > UINT32_MAX / 2 ||
        m * k > (uint64_t{1} << 40) || n * k > (uint64_t{1} << 40)) {
        return fail(TC_UNSUPPORTED, "matmul: extents beyond 2^31 rows or columns");
    }
    const S* pa = static_cast<const S*>(a);
    const S* pb = static_cast<const S*>(b);
    void* made_a = nullptr;
    void* made_b = nullptr;
    int status = TC_OK;
    // The kernel wants A as M x K and B as N x K.
    if (transposed == TC_LEFT) {  // A stored K x M
        status = transposed_copy(a, k, m, sizeof(S), &made_a);
        if (status != TC_OK) return status;
        pa = static_cast<const S*>(made_a);
    }
    if (transposed != TC_RIGHT) {  // B stored K x N
        status = transposed_copy(b, k, n, sizeof(S), &made_b);
        if (status != TC_OK) {
            if (made_a) tc_free(made_a);
            return status;
        }
        pb = static_cast<const S*>(made_b);
    }
    status = launch_gemm<S, O>(pa, pb, static_cast<O*>(c), m, k, n, accumulate, s);
    if (made_a) tc_free(made_a);
    if (made_b) tc_free(made_b);
    return status;
}

}  // namespace
}  // namespace tc

using namespace tc;

extern "C" int tc_matmul(uint32_t in_dtype, uint32_t out_dtype, uint32_t transposed, int accumulate, uint64_t m,
                         uint64_t k, uint64_t n, const void* a, const void* b, void* c) {
    if (transposed > TC_RIGHT) return fail(TC_INVALID, "matmul: no Transposed " + std::to_string(transposed));
    const bool acc = accumulate != 0;
    if (in_dtype == TC_F32 && out_dtype == TC_F32) return matmul_typed<float, float>(transposed, acc, m, k, n, a, b, c);
    if (in_dtype == TC_BF16 && out_dtype == TC_BF16) return matmul_typed<bf16_t, bf16_t>(transposed, acc, m, k, n, a, b, c);
    if (in_dtype == TC_BF16 && out_dtype == TC_F32) return matmul_typed<bf16_t, float>(transposed, acc, m, k, n, a, b, c);
    if (in_dtype == TC_F16 && out_dtype == TC_F16) return matmul_typed<_Float16, _Float16>(transposed, acc, m, k, n, a, b, c);
    if (in_dtype == TC_F16 && out_dtype == TC_F32) return matmul_typed<_Float16, float>(transposed, acc, m, k, n, a, b, c);
    return fail(TC_UNSUPPORTED, std::string("matmul: no kernel for ") + dtype_name(in_dtype) + " operands with " +
                                    dtype_name(out_dtype) + " output");
}
