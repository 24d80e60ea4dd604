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
// 16-bit operands (the tiled kernel below, v_mfma_f32_32x32x16_{bf16,f16})
// are read in whatever orientation they are stored in: a K-contiguous
// operand's LDS tile is read with ds_read_b128, a row-contiguous one's with
// gfx950's transposing ds_read_tr16_b64, so `matmul`, `matmul_add` and both
// `matmul_transposed_add` forms run the same kernel with no transpose pass.
// Blocks own 256 x 256 tiles of C over eight waves (128 x 128 over four for
// small products) and walk K 64 at a time.  HBM reaches LDS through buffer
// loads that write LDS directly (no staging registers), into XOR-swizzled,
// double-buffered tiles; out-of-range reads return zeros.  Each step's loads,
// LDS reads and matrix-core steps are woven with scheduling groups, and the
// step's barrier sits before its last slice so the next step's first
// fragments are read under that slice's matrix-core steps.
//
// f32 operands (v_mfma_f32_16x16x4_f32, the in-place f32 kernel) are read in
// place the same way, a row-contiguous operand's four k per lane coming from
// four LDS reads down its tile; 256 x 128 tiles (128 x 128 for products with
// fewer such tiles than CUs), 32-deep steps.  One 16-byte
// LDS read of a K-contiguous f32 tile feeds four consecutive matrix-core
// steps, since the sum over k does not care which lane holds which k as long
// as both operands agree.
//
// Operands whose rows are not 16-byte aligned, or past 2^31 bytes, take the
// general kernels: both operands K-contiguous, one stored the other way round
// first transposed into a scratch block, loads bounds-checked element by
// element.
//
// Block tiles are ordered in groups of rows, and the linear block index is
// first spread so that the blocks one XCD runs are neighbours, which keeps
// each XCD's L2 working on a few A and B panels.

#include <string.h>

#include <algorithm>

#include <type_traits>

#include "common.hpp"
#include "gemm_kernels.hpp"
#include "program.hpp"

namespace tc {
namespace {

// The program epilogue interpreted: the fused programs' interpreter over the
// tile's staged products, instruction by instruction.
template <int T>
struct ProgramStore {
    static constexpr bool kProgram = true;
    static constexpr int kElems = kLanesPerThread;
    Inline program;
    Buffers buffers;
    uint32_t count;

    __device__ __forceinline__ void group(const bool (&live)[4], const uint32_t (&rows)[4], const uint32_t (&cols)[4],
                                          uint32_t N, const float (&product)[4]) const {
        uint64_t row[4], col[4], element[4];
#pragma unroll
        for (int v = 0; v < 4; v++) {
            row[v] = rows[v];
            col[v] = cols[v];
            element[v] = row[v] * N + col[v];
        }
        Registers regs;
        for (uint32_t pc = 0; pc < count; pc++) {
            const tc_encoded in = program.code[pc];
            float value[4];
            bool writes = true;
            if (in.kind == 0 && in.a == 0) {
#pragma unroll
                for (int v = 0; v < 4; v++) value[v] = live[v] ? round_to<T>(product[v]) : 0.0f;
            } else {
                writes = evaluate<T>(regs, in, in.kind == 0 ? &program.places[in.op] : nullptr, buffers, live, row,
                                     col, element, value);
            }
            if (writes) write(regs, in.dst, value);
        }
    }
};

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

// The four-wave kernel's instances, named here: launched from a template
// alone, the host compiler emitted no launch stub for it (its step order is
// built from nested generic lambdas) and the library failed to load.
}  // namespace
template __global__ void gemm16x16_wide_kernel<bf16_t, bf16_t, true, true>(
    const bf16_t*, const bf16_t*, bf16_t*, uint32_t, uint32_t, uint32_t, bool, PlainStore);
template __global__ void gemm16x16_wide_kernel<bf16_t, bf16_t, true, false>(
    const bf16_t*, const bf16_t*, bf16_t*, uint32_t, uint32_t, uint32_t, bool, PlainStore);
template __global__ void gemm16x16_wide_kernel<bf16_t, bf16_t, false, false>(
    const bf16_t*, const bf16_t*, bf16_t*, uint32_t, uint32_t, uint32_t, bool, PlainStore);
template __global__ void gemm16x16_wide_kernel<_Float16, _Float16, true, true>(
    const _Float16*, const _Float16*, _Float16*, uint32_t, uint32_t, uint32_t, bool, PlainStore);
template __global__ void gemm16x16_wide_kernel<_Float16, _Float16, true, false>(
    const _Float16*, const _Float16*, _Float16*, uint32_t, uint32_t, uint32_t, bool, PlainStore);
template __global__ void gemm16x16_wide_kernel<_Float16, _Float16, false, false>(
    const _Float16*, const _Float16*, _Float16*, uint32_t, uint32_t, uint32_t, bool, PlainStore);
namespace {

// The tiled kernels' shapes: a 256 x 256 tile over eight waves of 128 x 64
// (two waves per SIMD, so one's waits overlap the other's matrix-core
// steps), and a 128 x 128 tile over four waves of 64 x 64 for products too
// small to give every CU a tile.  Products of at least a tile a CU run the
// 16 x 16 x 32 kernels: the four-wave one for a 16-bit C written whole over
// whole pairs of steps, the eight-wave persistent one for other plain stores
// and whole pairs of steps (on MI355X, bf16 8192^3: 1443 against 1395
// TFLOP/s a tile a block; f16 16384 x 4096 x 1024: 1203 against 1065 for
// the persistent 32 x 32 x 16 kernel it replaced), the one-tile kernel for
// program epilogues and odd step counts.
template <typename S, typename O, bool A_KC, bool B_KC, class EPI = PlainStore>
void launch_tiled16(const S* a, const S* b, O* c, uint32_t m, uint32_t k, uint32_t n, bool accumulate,
                    hipStream_t s, const EPI& epi = EPI{}) {
    const uint32_t large = ((m + 255) / 256) * ((n + 255) / 256);
    const uint32_t cus = static_cast<uint32_t>(compute_units());
    if (large >= cus) {
        if constexpr (!EPI::kProgram && sizeof(O) == 2) {
            // A 16-bit C written whole, by rows of 16-byte pieces, over whole
            // step pairs: the four-wave kernel.
            if (!accumulate && n % 8 == 0 && reinterpret_cast<uintptr_t>(c) % 16 == 0 && k % 128 == 0) {
                gemm16x16_wide_kernel<S, O, A_KC, B_KC><<<cus, 256, 0, s>>>(a, b, c, m, n, k, false, PlainStore{});
                return;
            }
        }
        if constexpr (!EPI::kProgram) {
            // k >= 8 here, so an even step count is at least two.
            if (((k + 63) / 64) % 2 == 0) {
                gemm16x16_persistent_kernel<S, O, A_KC, B_KC><<<cus, 512, 0, s>>>(a, b, c, m, n, k, accumulate,
                                                                                PlainStore{});
                return;
            }
        }
        gemm16x16_kernel<S, O, A_KC, B_KC, EPI><<<large, 512, 0, s>>>(a, b, c, m, n, k, accumulate, epi);
    } else {
        const uint32_t small = ((m + 127) / 128) * ((n + 127) / 128);
        direct16_kernel<S, O, A_KC, B_KC, 128, 128, 2, 2, 64, 2, EPI><<<small, 2 * 2 * 64, 0, s>>>(a, b, c, m, n, k,
                                                                                                 accumulate, epi);
    }
}

// The in-place f32 kernel's shape: 128 x 128 tiles over four waves of 64 x
// 64, whatever the product's size.  At 70 KiB of LDS and 82 VGPRs + 64 AGPRs
// two blocks share a CU, so one block's step barrier and first fragment
// reads overlap the other's matrix-core steps; 256 x 128 tiles (one block a
// CU) measured 4-16% slower on every shape tried on MI355X, from 2048^3 to
// 8192^3 in all three forms (4096^3: 132.2 / 133.6 / 129.4 TFLOP/s PLAIN /
// LEFT / RIGHT against 124.9 / 118.7 / 124.5), with the same bits.
template <typename O, bool A_KC, bool B_KC, class EPI = PlainStore>
void launch_inplace32(const float* a, const float* b, O* c, uint32_t m, uint32_t k, uint32_t n, bool accumulate,
                      hipStream_t s, const EPI& epi = EPI{}) {
    const uint32_t tiles = ((m + 127) / 128) * ((n + 127) / 128);
    // Too few 128 x 128 tiles for two blocks on every CU (a 4096 x 1024
    // product has 256): 128 x 64 tiles, twice the blocks, so the two-blocks-
    // a-CU overlap still happens.
    if constexpr (!EPI::kProgram) {
        if (tiles < 2 * static_cast<uint32_t>(compute_units())) {
            const uint32_t narrow = ((m + 127) / 128) * ((n + 63) / 64);
            inplace32_kernel<O, A_KC, B_KC, 128, 64, EPI><<<narrow, kThreads, 0, s>>>(a, b, c, m, n, k, accumulate,
                                                                                     epi);
            return;
        }
    }
    inplace32_kernel<O, A_KC, B_KC, 128, 128, EPI><<<tiles, kThreads, 0, s>>>(a, b, c, m, n, k, accumulate, epi);
}

// ---- products over a short K -----------------------------------------------------------
//
// A product with K below 8 (an outer product, K = 1, is how the tape
// broadcasts a bias: `outer`, tape/mod.rs:1000-1006) does too little
// arithmetic for the matrix cores and is bound by writing C.  Each thread
// forms four neighbouring outputs of one row with an FMA chain over k, in
// k order, and stores them as one 16-byte word where the row allows.  For
// K = 1 the result is the single rounding of a·b, the host's own.
template <typename S, typename O, bool A_KC, bool B_KC, bool VEC>
__global__ void __launch_bounds__(256) short_k_kernel(const S* __restrict__ A, const S* __restrict__ B,
                                                      O* __restrict__ C, uint32_t M, uint32_t N, uint32_t K,
                                                      bool accumulate) {
    using EA = Elem<S>;
    const uint32_t groups = (N + 3) / 4;
    const uint64_t items = static_cast<uint64_t>(M) * groups;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t item = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; item < items;
         item += stride) {
        const uint32_t row = static_cast<uint32_t>(item / groups);
        const uint32_t col = static_cast<uint32_t>(item - static_cast<uint64_t>(row) * groups) * 4;
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (uint32_t k = 0; k < K; k++) {
            const float a = EA::widen(A_KC ? A[static_cast<uint64_t>(row) * K + k] : A[static_cast<uint64_t>(k) * M + row]);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                if (VEC || col + e < N) {
                    const uint32_t j = col + e;
                    const float b = EA::widen(B_KC ? B[static_cast<uint64_t>(j) * K + k] : B[static_cast<uint64_t>(k) * N + j]);
                    acc[e] = fmaf(a, b, acc[e]);
                }
            }
        }
        const uint64_t at = static_cast<uint64_t>(row) * N + col;
        if constexpr (VEC) {
            float4* to = reinterpret_cast<float4*>(C + at);
            if (accumulate) {
                const float4 c = *to;
                acc[0] += c.x, acc[1] += c.y, acc[2] += c.z, acc[3] += c.w;
            }
            *to = make_float4(acc[0], acc[1], acc[2], acc[3]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                if (col + e < N) store_out(C, at + e, acc[e], accumulate);
            }
        }
    }
}

template <typename S, typename O, bool A_KC, bool B_KC>
int launch_short_k(const S* a, const S* b, O* c, uint64_t m, uint64_t k, uint64_t n, bool accumulate, hipStream_t s) {
    const uint32_t m32 = static_cast<uint32_t>(m), k32 = static_cast<uint32_t>(k), n32 = static_cast<uint32_t>(n);
    const uint32_t blocks = blocks_for(m * ((n + 3) / 4), 1);
    if (std::is_same<O, float>::value && n % 4 == 0 && aligned16(c)) {
        short_k_kernel<S, O, A_KC, B_KC, true><<<blocks, 256, 0, s>>>(a, b, c, m32, n32, k32, accumulate);
    } else {
        short_k_kernel<S, O, A_KC, B_KC, false><<<blocks, 256, 0, s>>>(a, b, c, m32, n32, k32, accumulate);
    }
    return check_launch("matmul");
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
    if constexpr (std::is_same<S, O>::value) {
        // One output column or row: the matrix-vector kernels, which spread
        // it over the whole part where a product's tiles would leave all but
        // a few CUs idle (MetalBuffer::product_into, metal/ops.rs:176-200).
        // Each form's vector is contiguous: B's one column (PLAIN, RIGHT),
        // A's one row (PLAIN, LEFT).
        if (k > 0 && (n == 1 || m == 1)) {
            const uint32_t dtype = Elem<S>::dtype;
            if (n == 1) {
                if (transposed == TC_LEFT) return vector_product(dtype, true, accumulate, k, m, a, b, c);  // b . A
                return vector_product(dtype, false, accumulate, m, k, a, b, c);                            // A . b
            }
            if (transposed == TC_RIGHT) return vector_product(dtype, false, accumulate, n, k, b, a, c);    // B . a
            return vector_product(dtype, true, accumulate, k, n, b, a, c);                                 // a . B
        }
    }
    if (k < 8) {
        O* pc = static_cast<O*>(c);
        if (transposed == TC_PLAIN) return launch_short_k<S, O, true, false>(pa, pb, pc, m, k, n, accumulate, s);
        if (transposed == TC_LEFT) return launch_short_k<S, O, false, false>(pa, pb, pc, m, k, n, accumulate, s);
        return launch_short_k<S, O, true, true>(pa, pb, pc, m, k, n, accumulate, s);
    }
    if constexpr (std::is_same<S, float>::value) {
        // f32 operands read in place whenever their rows are 16-byte aligned
        // and they stay under the buffer offsets' 2^31 bytes.
        const bool a_kc = transposed != TC_LEFT, b_kc = transposed == TC_RIGHT;
        const uint64_t limit = uint64_t{1} << 31;
        const bool in_place = aligned16(a) && aligned16(b) && (a_kc ? k % 4 == 0 : m % 4 == 0) &&
                              (b_kc ? k % 4 == 0 : n % 4 == 0) && m * k * 4 < limit && k * n * 4 < limit;
        if (in_place) {
            const uint32_t m32 = static_cast<uint32_t>(m), k32 = static_cast<uint32_t>(k),
                           n32 = static_cast<uint32_t>(n);
            O* pc = static_cast<O*>(c);
            if (a_kc && b_kc) {
                launch_inplace32<O, true, true>(pa, pb, pc, m32, k32, n32, accumulate, s);
            } else if (a_kc) {
                launch_inplace32<O, true, false>(pa, pb, pc, m32, k32, n32, accumulate, s);
            } else {
                launch_inplace32<O, false, false>(pa, pb, pc, m32, k32, n32, accumulate, s);
            }
            return check_launch("matmul");
        }
    } else {
        // 16-bit operands read in place whenever their rows are 16-byte
        // aligned: A is K-contiguous unless LEFT, B only when RIGHT.
        const bool a_kc = transposed != TC_LEFT, b_kc = transposed == TC_RIGHT;
        // The tiled kernel addresses each operand with 32-bit buffer offsets
        // and points the K tail past 2^31 bytes, so operands stay below it.
        const uint64_t limit = uint64_t{1} << 31;
        const bool in_place = aligned16(a) && aligned16(b) && (a_kc ? k % 8 == 0 : m % 8 == 0) &&
                              (b_kc ? k % 8 == 0 : n % 8 == 0) && m * k * sizeof(S) < limit &&
                              k * n * sizeof(S) < limit;
        if (in_place) {
            const uint32_t m32 = static_cast<uint32_t>(m), k32 = static_cast<uint32_t>(k),
                           n32 = static_cast<uint32_t>(n);
            O* pc = static_cast<O*>(c);
            if (a_kc && b_kc) {
                launch_tiled16<S, O, true, true>(pa, pb, pc, m32, k32, n32, accumulate, s);
            } else if (a_kc) {
                launch_tiled16<S, O, true, false>(pa, pb, pc, m32, k32, n32, accumulate, s);
            } else {
                launch_tiled16<S, O, false, false>(pa, pb, pc, m32, k32, n32, accumulate, s);
            }
            return check_launch("matmul");
        }
    }
    void* made_a = nullptr;
    void* made_b = nullptr;
    int status = TC_OK;
    // The general kernels want A as M x K and B as N x K.
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

// Elements a thread takes through a compiled epilogue at once: all their
// loads are in flight together.
constexpr int kCompiledElems = 16;

// The source the runtime compiler builds a program's product kernels from:
// the epilogue type CompiledStore with the program as straight-line code,
// after the product kernels' header; empty when the program has more
// constants than the kernels' arguments carry.
std::string epilogue_source(uint32_t dtype, const tc_encoded* code, uint32_t count, const tc_place* host_places,
                            std::vector<float>* constants, bool runs, bool* has_runs = nullptr) {
    const std::string body = epilogue_group(code, count, dtype, true, kCompiledElems, host_places, constants);
    // The run form, where the operands allow it (the caller's `runs`): runs
    // of eight for the four-wave kernel's 16-bit products, of four for the
    // f32 kernel.
    const std::string run_members =
        runs ? epilogue_runs(code, count, dtype, host_places, constants, dtype == TC_F32 ? 4 : kEpilogueRun)
             : std::string();
    if (constants->size() > static_cast<size_t>(kInlineCode)) return std::string();
    if (has_runs != nullptr) *has_runs = !run_members.empty();
    return "#include \"gemm_kernels.hpp\"\n"
           "struct CompiledStore {\n"
           "  static constexpr bool kProgram = true;\n"
           "  static constexpr bool kRuns = " + std::string(run_members.empty() ? "false" : "true") + ";\n"
           "  static constexpr int kElems = " + std::to_string(kCompiledElems) + ";\n" +
           compiled_members() +
           "  __device__ __forceinline__ void group(const bool (&live)[kElems], const uint32_t (&row)[kElems],\n"
           "      const uint32_t (&col)[kElems], uint32_t N, const float (&product)[kElems]) const {\n" +
           body + "  }\n" + run_members + "};\n";
}

// The most architectural VGPRs a four-wave instance with a compiled
// epilogue may use: a margin of 32 under the 256 a wave has, so spilled
// scalars find a free VGPR rather than an accumulator's AGPR (the library's
// own instances use 165-200).
constexpr uint32_t kWideVgprLimit = 224;

// The product kernels with `code` compiled into their epilogue, once the
// program has been seen before: true when they were launched.
bool run_compiled_epilogue(uint32_t dtype, uint32_t m, uint32_t k, uint32_t n, const void* a, const void* b,
                           const tc_encoded* code, uint32_t count, const tc_place* host_places,
                           const DevicePlace* places, uint32_t place_count,
                           const void* const* inputs, uint32_t input_count, void* const* outputs,
                           uint32_t output_count, hipStream_t s, int* status) {
    std::vector<float> constants;
    const bool runs = runs_allowed(n, code, count, host_places, inputs, outputs, output_count, true,
                                   dtype == TC_F32 ? 4 : kEpilogueRun);
    bool has_runs = false;
    const std::string source = epilogue_source(dtype, code, count, host_places, &constants, runs, &has_runs);
    if (source.empty()) return false;
    std::vector<std::string> kernels;
    uint32_t large = 0, small = 0, large_threads = 0, small_threads = 0;
    if (dtype == TC_F32) {
        // One shape for f32, as launch_inplace32 runs it.
        kernels = {"tc::inplace32_kernel<float, true, false, 128, 128, CompiledStore>"};
        large_threads = small_threads = kThreads;
    } else {
        const std::string type = dtype == TC_F16 ? "_Float16" : "tc::bf16_t";
        kernels = {"tc::gemm16x16_kernel<" + type + ", " + type + ", true, false, CompiledStore>",
                   "tc::direct16_kernel<" + type + ", " + type + ", true, false, 128, 128, 2, 2, 64, 2, CompiledStore>"};
        if (runtime_compiler_is_ours()) {
            kernels.push_back("tc::gemm16x16_persistent_kernel<" + type + ", " + type + ", true, false, CompiledStore>");
            // The four-wave kernel takes only the run form: the element
            // form's per-element addresses and stores cost it more than the
            // eight-wave kernel loses, and crowd its registers.
            if (has_runs) {
                kernels.push_back("tc::gemm16x16_wide_kernel<" + type + ", " + type + ", true, false, CompiledStore>");
            }
        }
        large = ((m + 255) / 256) * ((n + 255) / 256);
        large_threads = 512;
        small_threads = 2 * 2 * 64;
    }
    small = ((m + 127) / 128) * ((n + 127) / 128);
    hipFunction_t functions[4] = {};
    KernelResources resources[4];
    if (!compiled_kernels(source, kernels, functions, resources)) return false;
    CompiledArgsOf args{};
    for (uint32_t slot = 1; slot < input_count; slot++) args.in[slot] = inputs[slot];
    for (uint32_t slot = 0; slot < output_count; slot++) args.out[slot] = outputs[slot];
    for (uint32_t p = 0; p < place_count; p++) args.places[p] = places[p];
    for (size_t c = 0; c < constants.size(); c++) args.constants[c] = constants[c];
    void* none = nullptr;
    bool accumulate = false;
    void* params[] = {const_cast<void**>(&a), const_cast<void**>(&b), &none, &m, &n, &k, &accumulate, &args};
    const uint32_t cus = static_cast<uint32_t>(compute_units());
    const bool use_large = dtype != TC_F32 && large >= cus;
    // 16-bit products over whole step pairs take the persistent kernels, as
    // plain ones do (launch_tiled16): the four-wave one when K is a multiple
    // of 128, else the eight-wave one.
    // The four-wave kernel's matrix-core steps are inline assembly on
    // accumulators pinned in AGPRs, with their hazard cover written around
    // them.  An epilogue that crowds the registers breaks those assumptions:
    // with the architectural VGPRs nearly full the compiler parks spilled
    // values in AGPRs and moves accumulators out of them inside the main
    // loop (seen at 250 VGPRs), and past that it spills to scratch memory.
    // So an instance is launched only when the compile's resource report
    // shows no scratch and at most kWideVgprLimit VGPRs; otherwise the
    // eight-wave kernels take the product.
    const bool wide = kernels.size() == 4 && use_large && k % 128 == 0 && resources[3].scratch == 0 &&
                      resources[3].vgprs <= kWideVgprLimit;
    const bool persistent = kernels.size() == 4 && use_large && ((k + 63) / 64) % 2 == 0;
    hipFunction_t function = dtype == TC_F32 ? functions[0]
                             : wide          ? functions[3]
                             : persistent    ? functions[2]
                             : use_large     ? functions[0]
                                             : functions[1];
    const uint32_t grid = wide || persistent ? cus : use_large ? large : small;
    const uint32_t threads = wide ? 256 : use_large ? large_threads : small_threads;
    count_dispatch();
    const hipError_t error = hipModuleLaunchKernel(function, grid, 1, 1, threads, 1, 1, 0, s, params, nullptr);
    *status = error == hipSuccess ? TC_OK : fail(TC_DEVICE, std::string("fused matmul: ") + hipGetErrorString(error));
    return true;
}

}  // namespace

int matmul_program(uint32_t dtype, uint64_t m, uint64_t k, uint64_t n, const void* a, const void* b,
                   const tc_encoded* code, uint32_t count, const tc_place* places, uint32_t place_count,
                   const void* const* inputs, uint32_t input_count, void* const* outputs, uint32_t output_count,
                   bool* fused) {
    *fused = false;
    if (count > static_cast<uint32_t>(kInlineCode) || place_count > static_cast<uint32_t>(kInlinePlaces)) return TC_OK;
    if (k < 8 || m == 0 || n == 0 || m > UINT32_MAX / 2 || n > UINT32_MAX / 2 || k > UINT32_MAX / 2) return TC_OK;
    const size_t width = dtype == TC_F32 ? 4 : 2;
    const uint64_t limit = uint64_t{1} << 31;
    const uint64_t align = 16 / width;  // a row-major row of A (k) and of B (n) in whole 16-byte words
    if (!aligned16(a) || !aligned16(b) || k % align != 0 || n % align != 0 || m * k * width >= limit ||
        k * n * width >= limit) {
        return TC_OK;
    }
    TC_STREAM(s);
    const uint32_t m32 = static_cast<uint32_t>(m), k32 = static_cast<uint32_t>(k), n32 = static_cast<uint32_t>(n);
    int status = TC_OK;
    {
        DevicePlace device_places[kInlinePlaces] = {};
        status = to_device_places(places, place_count, device_places);
        if (status != TC_OK) return status;
        if (run_compiled_epilogue(dtype, m32, k32, n32, a, b, code, count, places, device_places, place_count, inputs,
                                  input_count, outputs, output_count, s, &status)) {
            *fused = true;
            return status;
        }
    }
    auto interpreted = [&](auto& epi) {
        memcpy(epi.program.code, code, count * sizeof(tc_encoded));
        status = to_device_places(places, place_count, epi.program.places);
        for (uint32_t slot = 1; slot < input_count; slot++) epi.buffers.inputs[slot] = inputs[slot];
        for (uint32_t slot = 0; slot < output_count; slot++) epi.buffers.outputs[slot] = outputs[slot];
        epi.count = count;
        return status == TC_OK;
    };
    switch (dtype) {
        case TC_F32: {
            ProgramStore<TC_F32> epi{};
            if (!interpreted(epi)) return status;
            launch_inplace32<float, true, false>(static_cast<const float*>(a), static_cast<const float*>(b), nullptr,
                                                 m32, k32, n32, false, s, epi);
            break;
        }
        case TC_F16: {
            ProgramStore<TC_F16> epi{};
            if (!interpreted(epi)) return status;
            launch_tiled16<_Float16, _Float16, true, false>(static_cast<const _Float16*>(a),
                                                            static_cast<const _Float16*>(b), nullptr, m32, k32, n32,
                                                            false, s, epi);
            break;
        }
        case TC_BF16: {
            ProgramStore<TC_BF16> epi{};
            if (!interpreted(epi)) return status;
            launch_tiled16<bf16_t, bf16_t, true, false>(static_cast<const bf16_t*>(a), static_cast<const bf16_t*>(b),
                                                        nullptr, m32, k32, n32, false, s, epi);
            break;
        }
        default: return TC_OK;
    }
    *fused = true;
    return check_launch("fused matmul");
}

}  // namespace tc

using namespace tc;

extern "C" int tc_matmul_epilogue_source(uint32_t dtype, const tc_encoded* code, uint32_t count,
                                         const tc_place* places, uint32_t place_count, uint32_t runs, char* out,
                                         uint64_t capacity, uint64_t* length) {
    if (dtype != TC_F32 && dtype != TC_F16 && dtype != TC_BF16) {
        return fail(TC_UNSUPPORTED, std::string("matmul epilogue source: no kernels for ") + dtype_name(dtype));
    }
    if (count > static_cast<uint32_t>(kInlineCode) || place_count > static_cast<uint32_t>(kInlinePlaces)) {
        return fail(TC_UNSUPPORTED, "matmul epilogue source: the program is not compiled into the product kernels");
    }
    std::vector<float> constants;
    const std::string source = epilogue_source(dtype, code, count, places, &constants, runs != 0);
    if (source.empty()) {
        return fail(TC_UNSUPPORTED, "matmul epilogue source: more constants than the kernels' arguments carry");
    }
    *length = source.size();
    if (out != nullptr && capacity > 0) {
        const size_t n = std::min<size_t>(source.size(), capacity - 1);
        memcpy(out, source.data(), n);
        out[n] = '\0';
    }
    return TC_OK;
}

extern "C" int tc_matmul(uint32_t in_dtype, uint32_t out_dtype, uint32_t transposed, int accumulate, uint64_t m,
                         uint64_t k, uint64_t n, const void* a, const void* b, void* c) {
    if (transposed > TC_RIGHT) return fail(TC_INVALID, "matmul: no Transposed " + std::to_string(transposed));
    if (m != 0 && n != 0 && (c == nullptr || (k != 0 && (a == nullptr || b == nullptr)))) {
        return fail(TC_INVALID, "matmul: a null operand");
    }
    const bool acc = accumulate != 0;
    if (in_dtype == TC_F32 && out_dtype == TC_F32) return matmul_typed<float, float>(transposed, acc, m, k, n, a, b, c);
    if (in_dtype == TC_BF16 && out_dtype == TC_BF16) return matmul_typed<bf16_t, bf16_t>(transposed, acc, m, k, n, a, b, c);
    if (in_dtype == TC_BF16 && out_dtype == TC_F32) return matmul_typed<bf16_t, float>(transposed, acc, m, k, n, a, b, c);
    if (in_dtype == TC_F16 && out_dtype == TC_F16) return matmul_typed<_Float16, _Float16>(transposed, acc, m, k, n, a, b, c);
    if (in_dtype == TC_F16 && out_dtype == TC_F32) return matmul_typed<_Float16, float>(transposed, acc, m, k, n, a, b, c);
    return fail(TC_UNSUPPORTED, std::string("matmul: no kernel for ") + dtype_name(in_dtype) + " operands with " +
                                    dtype_name(out_dtype) + " output");
}
