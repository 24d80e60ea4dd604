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

#include <type_traits>

#include "common.hpp"

namespace tc {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// The descriptor word that makes a gfx9-family buffer resource a plain,
// untyped byte range (32-bit data format, no swizzle, no stride).
constexpr int kBufferFlags = 0x00020000;

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

// ---- f32 operands in place ---------------------------------------------------------
//
// The f32 product with each operand read in its stored orientation, as the
// 16-bit kernel does, so `matmul_transposed_add` (the tape's backward
// products) and a plain `matmul` pay for no transpose pass.  A lane's four k
// for one tile row come from one ds_read_b128 of a K-contiguous tile, or
// four ds_read_b32 down a row-contiguous tile ([k][rows + 4]: the 4-float
// pad puts the four k-rows a wave reads on distinct bank quarters).  HBM is
// staged through buffer loads (zeros past the operand) into registers and
// then LDS, double-buffered, 256 x 128 or 128 x 128 tiles, 32-deep steps,
// four waves of a quarter tile.  Requirements as for the 16-bit kernel, with K (K-contiguous)
// or the contiguous extent (row-contiguous) a multiple of 4.

template <int ROWS, bool KC>
struct Stager32 {
    static constexpr int kRowChunks = KC ? kBK32 / 4 : ROWS / 4;  // 16-byte chunks per tile row
    static constexpr int kPassRows = kThreads / kRowChunks;
    static constexpr int kPasses = (KC ? ROWS : kBK32) / kPassRows;
    static constexpr int kLdsRow = KC ? kLd32 : ROWS + 4;
    __amdgpu_buffer_rsrc_t rsrc;
    uint32_t offset, pass_bytes, k_bytes, lds_at, k_in;

    __device__ void init(const float* p, uint32_t first, uint32_t rows, uint32_t ld, uint32_t depth, int t) {
        const uint32_t row = t / kRowChunks, part = (t % kRowChunks) * 4;
        if (KC) {
            rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p + static_cast<uint64_t>(first) * ld), 0,
                                                     (rows - first) * ld * 4, kBufferFlags);
            k_bytes = 4;
            k_in = part;
        } else {
            rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p + first), 0, (depth * ld - first) * 4,
                                                     kBufferFlags);
            k_bytes = ld * 4;
            k_in = 0;
        }
        offset = (row * ld + part) * 4;
        pass_bytes = kPassRows * ld * 4;
        lds_at = row * kLdsRow + part;
    }
    __device__ __forceinline__ void fetch(uint4 (&stage)[kPasses], uint32_t k0, uint32_t K, bool full) const {
        const uint32_t at = (full || !KC || k0 + k_in < K) ? offset : 0x80000000u;
#pragma unroll
        for (int i = 0; i < kPasses; i++) {
            auto v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, at, i * pass_bytes + k0 * k_bytes, 0);
            stage[i] = __builtin_bit_cast(uint4, v);
        }
    }
    __device__ __forceinline__ void commit(const uint4 (&stage)[kPasses], float* lds) const {
        uint4* to = reinterpret_cast<uint4*>(lds);
#pragma unroll
        for (int i = 0; i < kPasses; i++) to[(lds_at + i * kPassRows * kLdsRow) / 4] = stage[i];
    }
    // Lane `lane`'s four k (4 (lane / 16) + 0..3 of the slice at `kk`) of
    // tile row `row`.
    __device__ __forceinline__ f32x4 fragment(const float* lds, int row, int kk, int lane) const {
        const int k = kk + (lane / 16) * 4;
        if (KC) return reinterpret_cast<const f32x4*>(lds)[(row * kLdsRow + k) / 4];
        return f32x4{lds[k * kLdsRow + row], lds[(k + 1) * kLdsRow + row], lds[(k + 2) * kLdsRow + row],
                     lds[(k + 3) * kLdsRow + row]};
    }
};

// BM x BN tiles over four waves of (BM / 2) x (BN / 2).
template <typename O, bool A_KC, bool B_KC, int BM, int BN>
__global__ void __launch_bounds__(kThreads) inplace32_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                             O* __restrict__ C, uint32_t M, uint32_t N, uint32_t K,
                                                             bool accumulate) {
    using SA = Stager32<BM, A_KC>;
    using SB = Stager32<BN, B_KC>;
    constexpr int TM = BM / 32, TN = BN / 32;  // 16 x 16 tiles per wave
    constexpr int kA = A_KC ? BM * kLd32 : kBK32 * (BM + 4);
    constexpr int kB = B_KC ? BN * kLd32 : kBK32 * (BN + 4);
    __shared__ __attribute__((aligned(16))) float lds_a[2 * kA];
    __shared__ __attribute__((aligned(16))) float lds_b[2 * kB];
    const uint32_t tiles_m = (M + BM - 1) / BM;
    const uint32_t tiles_n = (N + BN - 1) / BN;
    uint32_t tm, tn;
    tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const int t = threadIdx.x;
    const int lane = t % 64;
    const int wave = t / 64;
    const int wm = wave / 2, wn = wave % 2;
    SA sa;
    SB sb;
    sa.init(A, m0, M, A_KC ? K : M, K, t);
    sb.init(B, n0, N, B_KC ? K : N, K, t);
    uint4 stage_a[SA::kPasses], stage_b[SB::kPasses];

    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = f32x4{};

    const uint32_t steps = (K + kBK32 - 1) / kBK32;
    if (steps > 0) {
        sa.fetch(stage_a, 0, K, kBK32 <= K);
        sb.fetch(stage_b, 0, K, kBK32 <= K);
        sa.commit(stage_a, lds_a);
        sb.commit(stage_b, lds_b);
        __syncthreads();
    }
    const int row_in = lane % 16;
    for (uint32_t step = 0; step < steps; step++) {
        const int buffer = step & 1;
        const bool more = step + 1 < steps;
        if (more) {
            const uint32_t k0 = (step + 1) * kBK32;
            sa.fetch(stage_a, k0, K, k0 + kBK32 <= K);
            sb.fetch(stage_b, k0, K, k0 + kBK32 <= K);
        }
        const float* la = lds_a + buffer * kA;
        const float* lb = lds_b + buffer * kB;
#pragma unroll
        for (int kk = 0; kk < kBK32; kk += 16) {
            f32x4 a[TM], b[TN];
#pragma unroll
            for (int i = 0; i < TM; i++) a[i] = sa.fragment(la, wm * (BM / 2) + i * 16 + row_in, kk, lane);
#pragma unroll
            for (int j = 0; j < TN; j++) b[j] = sb.fragment(lb, wn * (BN / 2) + j * 16 + row_in, kk, lane);
#pragma unroll
            for (int e = 0; e < 4; e++)
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][e], b[j][e], acc[i][j], 0, 0, 0);
        }
        if (more) {
            sa.commit(stage_a, lds_a + (buffer ^ 1) * kA);
            sb.commit(stage_b, lds_b + (buffer ^ 1) * kB);
        }
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < TM; i++) {
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const uint32_t col = n0 + wn * (BN / 2) + j * 16 + lane % 16;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t row = m0 + wm * (BM / 2) + i * 16 + 4 * (lane / 16) + e;
                if (row < M && col < N) store_out(C, static_cast<uint64_t>(row) * N + col, acc[i][j][e], accumulate);
            }
        }
    }
}

// ---- 16-bit operands in place ---------------------------------------------------------
//
// C[M x N] (+)= A . B with each operand read in the layout it is stored in:
// "K-contiguous" (A stored M x K, B stored N x K) or "row-contiguous" (A
// stored K x M, B stored K x N — B's ordinary row-major form).  Each block
// owns a BM x BN tile of C and walks K in 64-deep steps; the waves split the
// tile WM x WN, each owning (BM/WM) x (BN/WN) as 32 x 32 matrix-core tiles.
// A lane's 8-element fragment of a 32 x 32 x 16 step is row lane % 32 (the
// tile's M or N index) and k (lane / 32) * 8 .. + 8 of the slice:
//  - from a K-contiguous tile with one ds_read_b128;
//  - from a row-contiguous tile with gfx950's transposing ds_read_tr16_b64,
//    which hands each lane of a 16-lane group four k-consecutive values of
//    one column: when lane j of the group addresses (k0 + j / 4,
//    c0 + 4 (j % 4)), lane i receives rows k0 .. k0 + 3 of column c0 + i.
//    Two such reads give a lane the same fragment, so no operand is ever
//    transposed in HBM.
// Requirements (checked by the host): 16-byte aligned operands, K a multiple
// of 8 for K-contiguous operands, the contiguous extent a multiple of 8 for
// row-contiguous ones, and operands under 2^31 bytes.  M and N edges and the
// K tail load zeros (buffer reads past the operand) or values that only feed
// results that are never stored.

constexpr int kTileK = 64;

typedef short short4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ short4v read_tr16(const void* lds_addr) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) short4v*)(const_cast<void*>(lds_addr)));
}

// The order the scheduler is asked to keep within one step: F matrix-core
// steps per slice, each followed by its share of the step's HBM loads (first
// slice) and of the next slice's LDS reads (every slice but the last, whose
// reads the scheduler places itself; interleaving those too measured no
// faster).
template <int F, int LOADS, int READS, int SLICES, int Q = 0, int R = 0>
__device__ __forceinline__ void weave() {
    if constexpr (Q < SLICES) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // a matrix-core step
        constexpr int loads = LOADS * (R + 1) / F - LOADS * R / F;
        constexpr int reads = READS * (R + 1) / F - READS * R / F;
        if constexpr (Q == 0 && loads > 0) __builtin_amdgcn_sched_group_barrier(0x020, loads, 0);  // HBM loads
        if constexpr (Q + 1 < SLICES && reads > 0) __builtin_amdgcn_sched_group_barrier(0x100, reads, 0);  // LDS reads
        if constexpr (R + 1 < F) {
            weave<F, LOADS, READS, SLICES, Q, R + 1>();
        } else {
            weave<F, LOADS, READS, SLICES, Q + 1, 0>();
        }
    }
}

// ---- staging straight into LDS ------------------------------------------------
//
// HBM -> LDS staging is done by gfx950's buffer loads that write LDS directly
// (`buffer_load_dwordx4 ... lds`): no staging registers and no ds_write
// instructions.  Such a load writes 64 lanes x 16 bytes to consecutive LDS
// bytes, so tiles are unpadded and bank conflicts are avoided by
// XOR-swizzling each row's 16-byte chunks instead: a lane loads the global
// chunk that belongs at the LDS position it writes.
//  - K-contiguous tile, BK x 2-byte rows (CPR = BK / 8 chunks a row, RPW =
//    256 / (2 BK) rows per 256-byte bank window): logical chunk c of row r
//    lives at chunk c ^ ((r / RPW) % CPR), which spreads the 16 rows a
//    ds_read_b128 phase touches over all 16 bank groups.
//  - row-contiguous tile, ROWS x 2-byte rows: chunk c of k-row r lives at
//    c ^ ((r & 3) << 2), which spreads the four rows of a transposing read
//    over distinct bank groups.
// The K loop runs NS stages deep: each step issues the loads of the step
// NS - 1 ahead into the stage the previous step freed, then waits only for
// the next step's loads (vmcnt counts this wave's loads in issue order).
// Two 64-deep stages measure faster on MI355X than three or four 32-deep
// ones (1170 vs 950 TFLOP/s at 8192^3): the per-step barrier costs more
// than the extra latency cover buys.

template <int BK>
__device__ __forceinline__ int kc_swizzle(int row) {
    constexpr int kCpr = BK / 8, kRpw = 256 / (2 * BK);
    return (row / kRpw) % kCpr;
}
__device__ __forceinline__ int rc_swizzle(int row) { return (row & 3) << 2; }

template <typename S, int ROWS, bool KC, int WAVES, int BK>
struct DirectStager {
    static constexpr int kTileBytes = ROWS * BK * 2;
    static constexpr int kInstr = kTileBytes / 1024;  // one wave instruction moves 1 KiB
    static constexpr int kPer = kInstr / WAVES;
    static_assert(kInstr % WAVES == 0, "tile instructions must divide among the waves");
    static constexpr int kRowsPer = KC ? 1024 / (BK * 2) : 1024 / (ROWS * 2);  // tile rows one instruction fills
    static constexpr int kChunksPerRow = KC ? BK / 8 : ROWS / 8;

    __amdgpu_buffer_rsrc_t rsrc;
    uint32_t offset[kPer];  // this lane's chunk of each instruction, bytes at k0 = 0
    uint32_t k_of[kPer];    // its k within a step (K-contiguous only)
    uint32_t k_bytes;
    int wave;

    __device__ void init(const S* p, uint32_t first, uint32_t rows, uint32_t ld, uint32_t depth, int w, int lane) {
        wave = w;
        if (KC) {
            rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<S*>(p + static_cast<uint64_t>(first) * ld), 0,
                                                     (rows - first) * ld * sizeof(S), kBufferFlags);
            k_bytes = sizeof(S);
        } else {
            rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<S*>(p + first), 0, (depth * ld - first) * sizeof(S),
                                                     kBufferFlags);
            k_bytes = ld * sizeof(S);
        }
#pragma unroll
        for (int i = 0; i < kPer; i++) {
            const int first_row = kRowsPer * (w + WAVES * i);
            const int row = first_row + lane / kChunksPerRow;
            const int place = lane % kChunksPerRow;
            const int chunk = place ^ (KC ? kc_swizzle<BK>(row) : rc_swizzle(row));
            offset[i] = (static_cast<uint32_t>(row) * ld + chunk * 8) * sizeof(S);
            k_of[i] = KC ? chunk * 8 : 0;
        }
    }
    // Stage the step at `k0` into `tile` (the LDS stage).  Past K a
    // K-contiguous chunk is the next row's, so it is pointed past the
    // resource (operands are under 2^31 bytes) and loads zeros.
    __device__ __forceinline__ void fetch(S* tile, uint32_t k0, uint32_t K, bool full) const {
#pragma unroll
        for (int i = 0; i < kPer; i++) {
            const uint32_t at = (full || !KC || k0 + k_of[i] < K) ? offset[i] : 0x80000000u;
            uint8_t* dst = reinterpret_cast<uint8_t*>(tile) + 1024 * (wave + WAVES * i);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)dst, 16, at,
                                                     k0 * k_bytes, 0, 0);
        }
    }
};

// A lane's fragment of tile row `row_base + lane % 32` (the tile's M or N
// index) for the 16-deep slice at `k_base`, from a swizzled tile.
template <typename S, int ROWS, bool KC, int BK>
__device__ __forceinline__ uint4 swizzled_fragment(const S* lds, int row_base, int k_base, int lane) {
    if (KC) {
        const int row = row_base + lane % 32;
        const int chunk = (k_base / 8 + lane / 32) ^ kc_swizzle<BK>(row);
        return reinterpret_cast<const uint4*>(lds)[row * (BK / 8) + chunk];
    } else {
        const int g = lane / 16, j = lane % 16;
        const int k = k_base + (g / 2) * 8 + j / 4;
        const int col = row_base + (g % 2) * 16 + 4 * (j % 4);
        const int chunk = (col / 8) ^ rc_swizzle(k);  // k + 4 swizzles the same way
        const S* at = lds + k * ROWS + chunk * 8 + col % 8;
        short4v lo = read_tr16(at);
        short4v hi = read_tr16(at + 4 * ROWS);
        uint4 out;
        out.x = static_cast<uint16_t>(lo[0]) | (static_cast<uint32_t>(static_cast<uint16_t>(lo[1])) << 16);
        out.y = static_cast<uint16_t>(lo[2]) | (static_cast<uint32_t>(static_cast<uint16_t>(lo[3])) << 16);
        out.z = static_cast<uint16_t>(hi[0]) | (static_cast<uint32_t>(static_cast<uint16_t>(hi[1])) << 16);
        out.w = static_cast<uint16_t>(hi[2]) | (static_cast<uint32_t>(static_cast<uint16_t>(hi[3])) << 16);
        return out;
    }
}

// s_waitcnt's immediate for vmcnt(n), other counters not waited on
// (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
constexpr int vmcnt_wait(int n) { return (n & 0xf) | ((n >> 4) << 14) | (0x7 << 4) | (0xf << 8); }

// One LDS stage of an operand.  A separate array per stage gives every LDS
// read and every direct load a distinct, statically known object, so the
// compiler waits for a stage's loads only where that stage is read.
template <typename S, int ELEMS, int STAGE>
__device__ __forceinline__ S* stage_tile() {
    __shared__ __attribute__((aligned(1024))) S tile[ELEMS];
    return tile;
}

template <typename S, typename O, bool A_KC, bool B_KC, int BM, int BN, int WM, int WN, int BK, int NS>
__global__ void __launch_bounds__(WM * WN * 64) direct16_kernel(const S* __restrict__ A, const S* __restrict__ B,
                                                                O* __restrict__ C, uint32_t M, uint32_t N, uint32_t K,
                                                                bool accumulate) {
    constexpr int kWaves = WM * WN;
    constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
    constexpr int kA = BM * BK, kB = BN * BK;  // elements of one stage
    static_assert(NS >= 2 && NS <= 4, "two to four stages");

    const uint32_t tiles_m = (M + BM - 1) / BM;
    const uint32_t tiles_n = (N + BN - 1) / BN;
    uint32_t tm, tn;
    tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const int lane = threadIdx.x % 64;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int wm = wave / WN, wn = wave % WN;

    using StagerA = DirectStager<S, BM, A_KC, kWaves, BK>;
    using StagerB = DirectStager<S, BN, B_KC, kWaves, BK>;
    StagerA sa;
    StagerB sb;
    sa.init(A, m0, M, A_KC ? K : M, K, wave, lane);
    sb.init(B, n0, N, B_KC ? K : N, K, wave, lane);

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = f32x16{};

    uint4 fa[2][TM], fb[2][TN];
    auto read_fragments = [&](int slot, const S* la, const S* lb, int kk) {
#pragma unroll
        for (int i = 0; i < TM; i++)
            fa[slot][i] = swizzled_fragment<S, BM, A_KC, BK>(la, wm * (BM / WM) + i * 32, kk, lane);
#pragma unroll
        for (int j = 0; j < TN; j++)
            fb[slot][j] = swizzled_fragment<S, BN, B_KC, BK>(lb, wn * (BN / WN) + j * 32, kk, lane);
    };

    constexpr int kSlices = BK / 16;
    constexpr int kSteps = TM * TN;
    constexpr int kReads = (A_KC ? TM : 2 * TM) + (B_KC ? TN : 2 * TN);
    constexpr int kLoads = StagerA::kPer + StagerB::kPer;  // this wave's loads per step
    const uint32_t steps = (K + BK - 1) / BK;
    auto stage_of = [&](auto t, uint32_t s) {
        const uint32_t k0 = (s < steps ? s : steps - 1) * BK;  // past the end: a harmless reload
        sa.fetch(stage_tile<S, kA, 2 * decltype(t)::value>(), k0, K, k0 + BK <= K);
        sb.fetch(stage_tile<S, kB, 2 * decltype(t)::value + 1>(), k0, K, k0 + BK <= K);
    };
    // Step s computes from stage T = s % NS.  It first stages step s + NS - 1
    // into stage (T + NS - 1) % NS, which every wave finished reading before
    // the previous step's barrier; it waits for step s + 1 and meets the
    // others at a barrier before its last slice, whose fragments it already
    // holds, and reads step s + 1's first fragments under that slice.
    auto step = [&](auto t, uint32_t s) {
        constexpr int T = decltype(t)::value;
        const S* la = stage_tile<S, kA, 2 * T>();
        const S* lb = stage_tile<S, kB, 2 * T + 1>();
        stage_of(std::integral_constant<int, (T + NS - 1) % NS>{}, s + NS - 1);
#pragma unroll
        for (int q = 0; q + 1 < kSlices; q++) {
            read_fragments((q + 1) & 1, la, lb, (q + 1) * 16);
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) acc[i][j] = Mfma16<S>::step(fa[q & 1][i], fb[q & 1][j], acc[i][j]);
        }
        weave<kSteps, kLoads, kReads, kSlices - 1>();
        __builtin_amdgcn_s_waitcnt(vmcnt_wait(kLoads * (NS - 2)));  // step s + 1 is in LDS
        __syncthreads();
        constexpr int last = (kSlices - 1) & 1;
        constexpr int U = (T + 1) % NS;
        read_fragments(last ^ 1, stage_tile<S, kA, 2 * U>(), stage_tile<S, kB, 2 * U + 1>(), 0);
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) acc[i][j] = Mfma16<S>::step(fa[last][i], fb[last][j], acc[i][j]);
        weave<kSteps, 0, kReads, 2>();
    };
    if (steps > 0) {
        stage_of(std::integral_constant<int, 0>{}, 0);
        if constexpr (NS > 2) stage_of(std::integral_constant<int, 1>{}, 1);
        if constexpr (NS > 3) stage_of(std::integral_constant<int, 2>{}, 2);
        __builtin_amdgcn_s_waitcnt(vmcnt_wait(kLoads * (NS - 2)));  // step 0 is in LDS
        __syncthreads();
        read_fragments(0, stage_tile<S, kA, 0>(), stage_tile<S, kB, 1>(), 0);
    }
    for (uint32_t s = 0; s < steps; s += NS) {
        step(std::integral_constant<int, 0>{}, s);
        if (s + 1 < steps) step(std::integral_constant<int, 1 % NS>{}, s + 1);
        if constexpr (NS > 2) {
            if (s + 2 < steps) step(std::integral_constant<int, 2 % NS>{}, s + 2);
        }
        if constexpr (NS > 3) {
            if (s + 3 < steps) step(std::integral_constant<int, 3 % NS>{}, s + 3);
        }
    }

#pragma unroll
    for (int i = 0; i < TM; i++) {
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const uint32_t col = n0 + wn * (BN / WN) + j * 32 + lane % 32;
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const uint32_t row = m0 + wm * (BM / WM) + i * 32 + 8 * (e / 4) + 4 * (lane / 32) + e % 4;
                if (row < M && col < N) store_out(C, static_cast<uint64_t>(row) * N + col, acc[i][j][e], accumulate);
            }
        }
    }
}

// The tiled kernel's shapes: a 256 x 256 tile over eight waves of 128 x 64
// (two waves per SIMD, so one's waits overlap the other's matrix-core
// steps), and a 128 x 128 tile over four waves of 64 x 64 for products too
// small to give every CU a few large tiles.
template <typename S, typename O, bool A_KC, bool B_KC>
void launch_tiled16(const S* a, const S* b, O* c, uint32_t m, uint32_t k, uint32_t n, bool accumulate,
                    hipStream_t s) {
    const uint32_t large = ((m + 255) / 256) * ((n + 255) / 256);
    if (large >= static_cast<uint32_t>(compute_units())) {
        direct16_kernel<S, O, A_KC, B_KC, 256, 256, 2, 4, 64, 2><<<large, 2 * 4 * 64, 0, s>>>(a, b, c, m, n, k, accumulate);
    } else {
        const uint32_t small = ((m + 127) / 128) * ((n + 127) / 128);
        direct16_kernel<S, O, A_KC, B_KC, 128, 128, 2, 2, 64, 2><<<small, 2 * 2 * 64, 0, s>>>(a, b, c, m, n, k, accumulate);
    }
}

// The in-place f32 kernel's shapes: 256 x 128 tiles, or 128 x 128 when the
// larger ones would leave CUs without a tile (a 4096 x 1024 product has 128
// of them on 256 CUs).
template <typename O, bool A_KC, bool B_KC>
void launch_inplace32(const float* a, const float* b, O* c, uint32_t m, uint32_t k, uint32_t n, bool accumulate,
                      hipStream_t s) {
    const uint32_t large = ((m + kBM - 1) / kBM) * ((n + kBN - 1) / kBN);
    if (large >= static_cast<uint32_t>(compute_units())) {
        inplace32_kernel<O, A_KC, B_KC, kBM, kBN><<<large, kThreads, 0, s>>>(a, b, c, m, n, k, accumulate);
    } else {
        const uint32_t small = ((m + 127) / 128) * ((n + 127) / 128);
        inplace32_kernel<O, A_KC, B_KC, 128, 128><<<small, kThreads, 0, s>>>(a, b, c, m, n, k, accumulate);
    }
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
