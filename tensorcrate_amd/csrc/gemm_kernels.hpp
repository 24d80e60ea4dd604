// The matrix-core product kernels, shared by the library (gemm.hip) and the
// product kernels the runtime compiler builds with a program's epilogue
// compiled in: the tiled 16-bit kernel (`direct16_kernel`) and the in-place
// f32 kernel (`inplace32_kernel`), templated on how a tile is finished.  It
// includes only device.hpp and <type_traits>, which hiprtc provides.
#pragma once

#include <type_traits>

#include "device.hpp"

namespace tc {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Two f32 values rounded once to the 16-bit O and packed, the first in the
// low half: one gfx950 conversion instruction a pair, with the rounding of
// Elem<O>::narrow (IEEE round to nearest even; tc_f32_to_bf16's rule for bf16).
template <typename O>
__device__ __forceinline__ uint32_t pack_pair(float lo, float hi) {
    if constexpr (std::is_same<O, _Float16>::value) {
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, f16x2));
    } else {
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
    }
}

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

// ---- how a tile is finished ---------------------------------------------------------
//
// A product kernel ends either with plain stores, C (+)= A . B, or with a
// fused program run over its tile (`Kernels::matmul_epilogue`,
// kernels.rs:1142; `Program::run_matmul`, fused/mod.rs:1143-1215): the
// product is never written to memory unless the program stores it.  The
// tile's accumulators are staged through the LDS the main loop used, a pass
// of rows at a time, and the program then runs over the pass in row-major
// order, four elements a thread 64 apart as the fused kernel runs them, so
// its loads and stores are coalesced.  Input 0 is the product rounded to the
// program's type, as the host's product is before its program reads it.
//
// An epilogue type with kProgram set provides kElems and
//   group(live, row, col, N, product)
// for kElems elements of C: whether each is inside C, its row and column
// (its row-major index is row * N + col), and its f32 product.  The
// library's interprets the program; a compiled one is the program as
// straight-line code.

struct PlainStore {
    static constexpr bool kProgram = false;
};

// Whether an epilogue type also has the run form (`kRuns`, with
// `Invariant`, `invariant` and `run`); a type without the member has not.
template <class EPI, class = void>
struct HasRuns : std::false_type {};
template <class EPI>
struct HasRuns<EPI, std::void_t<decltype(EPI::kRuns)>> : std::integral_constant<bool, EPI::kRuns> {};
// The run form's invariant state where the epilogue has one, else nothing.
template <class EPI, bool = HasRuns<EPI>::value>
struct RunState {
    struct Invariant {};
};
template <class EPI>
struct RunState<EPI, true> {
    using Invariant = typename EPI::Invariant;
};

// A workgroup barrier ordering LDS alone: fences scoped to the workgroup and
// to LDS ("local") around the barrier, so LDS accesses stay on their side
// and only LDS traffic is waited for.  Unlike __syncthreads it does not wait
// for the epilogue's global stores, which only have to land by the end of
// the kernel.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Where tile column `col` of staged row `row` sits: groups of G lanes that
// store one row of a matrix-core tile, 4 rows apart, land on distinct banks.
// G = 0 is the 16 x 16 x 32 kernel's layout, where a lane stores four
// consecutive columns of one row as one 16-byte write and 16 lanes store 16
// consecutive rows: the row's low four bits pick the quad's 16-byte place
// within its 64 columns.
template <int G>
__device__ __forceinline__ uint32_t staged_col(uint32_t row, uint32_t col) {
    if constexpr (G == 0) {
        return col ^ ((row & 15) << 2);
    } else {
        return col ^ (((row >> 2) & (64 / G - 1)) * G);
    }
}

// The staged rows live in up to four LDS regions of REGION_ROWS rows each.
template <int BN, int G, int REGION_ROWS>
__device__ __forceinline__ float* staged_at(float* r0, float* r1, float* r2, float* r3, uint32_t row, uint32_t col) {
    const uint32_t region = row / REGION_ROWS;
    float* base = region == 0 ? r0 : region == 1 ? r1 : region == 2 ? r2 : r3;
    return base + (row % REGION_ROWS) * BN + staged_col<G>(row, col);
}

// The epilogue over `rows` x BN staged products, EPI::kElems elements a
// thread 64 apart in row-major order (each load and store instruction of a
// wave then touches one contiguous run), handed to `epi.group`.  A pass holds
// H rows of each wave row (WAVE_ROWS rows apart), its `pass`-th H: staged row
// rr is tile row (rr / H) * WAVE_ROWS + pass * H + rr % H, so every wave
// stages, and then stops holding, the same share of its accumulators in
// every pass.
template <int BN, int G, int REGION_ROWS, int H, int WAVE_ROWS, class EPI>
__device__ __forceinline__ void program_pass(const EPI& epi, float* r0, float* r1, float* r2, float* r3,
                                             uint32_t rows, uint32_t pass, uint32_t row_base, uint32_t col_base,
                                             uint32_t M, uint32_t N) {
    constexpr int E = EPI::kElems;
    const uint32_t total = rows * BN;
    const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const uint32_t per_round = blockDim.x * E;
    for (uint32_t base = 0; base < total; base += per_round) {
        uint32_t row[E], col[E];
        bool live[E];
        float product[E];
#pragma unroll
        for (int v = 0; v < E; v++) {
            const uint32_t at = base + wave * (64 * E) + v * 64 + lane;
            const uint32_t rr = at / BN, cc = at % BN;
            const bool inside = at < total;
            product[v] = inside ? *staged_at<BN, G, REGION_ROWS>(r0, r1, r2, r3, rr, cc) : 0.0f;
            row[v] = row_base + (rr / H) * WAVE_ROWS + pass * H + rr % H;
            col[v] = col_base + cc;
            live[v] = inside && row[v] < M && col[v] < N;
        }
        epi.group(live, row, col, N, product);
    }
}

// The run form of the same epilogue (EPI::run, runs of four columns): the
// staged rows read back one 16-byte run a thread, consecutive threads on
// consecutive runs, each thread on the same four columns in every round
// (BN / 4 divides the workgroup), whose row-invariant loads `inv` holds.
template <int BN, int G, int REGION_ROWS, int H, int WAVE_ROWS, class EPI>
__device__ __forceinline__ void program_runs(const EPI& epi, const typename EPI::Invariant& inv, float* region,
                                             uint32_t rows, uint32_t pass, uint32_t row_base, uint32_t col_base,
                                             uint32_t M, uint32_t N) {
    constexpr uint32_t kPerRow = BN / 4;
    const uint32_t runs = rows * kPerRow;
    for (uint32_t q = threadIdx.x; q < runs; q += blockDim.x) {
        const uint32_t rr = q / kPerRow, cc = (q % kPerRow) * 4;
        const float4 v =
            *reinterpret_cast<const float4*>(staged_at<BN, G, REGION_ROWS>(region, region, region, region, rr, cc));
        const float product[4] = {v.x, v.y, v.z, v.w};
        const uint32_t row = row_base + (rr / H) * WAVE_ROWS + pass * H + rr % H;
        const uint32_t col = col_base + cc;
        epi.run(inv, row < M && col < N, row, col, N, product);
    }
}

constexpr int kBK32 = 32;
constexpr int kLd32 = kBK32 + 4;

// ---- f32 operands in place ---------------------------------------------------------
//
// The f32 product with each operand read in its stored orientation, as the
// 16-bit kernel does, so `matmul_transposed_add` (the tape's backward
// products) and a plain `matmul` pay for no transpose pass.  A lane's four k
// for one tile row come from one ds_read_b128 of a K-contiguous tile, or
// four ds_read_b32 down a row-contiguous tile ([k][rows + 4]: the 4-float
// pad puts the four k-rows a wave reads on distinct bank quarters).  A
// K-contiguous tile's rows are 128 bytes, 16-byte chunk c of row r at
// c ^ ((r / 2) % 8): conflict-free for the 16 rows a ds_read_b128 reads,
// where rows padded to 144 bytes measured a 2-way conflict on every read
// (16.8M conflict cycles a 4096^3 launch for each such operand).  HBM is
// staged through buffer loads (zeros past the operand) into registers and
// then LDS, double-buffered, 256 x 128 or 128 x 128 tiles, 32-deep steps,
// four waves of a quarter tile.  Requirements as for the 16-bit kernel, with K (K-contiguous)
// or the contiguous extent (row-contiguous) a multiple of 4.

template <int ROWS, bool KC>
struct Stager32 {
    static constexpr int kRowChunks = KC ? kBK32 / 4 : ROWS / 4;  // 16-byte chunks per tile row
    static constexpr int kPassRows = kThreads / kRowChunks;
    static constexpr int kPasses = (KC ? ROWS : kBK32) / kPassRows;
    static constexpr int kLdsRow = KC ? kBK32 : ROWS + 4;
    static constexpr int kTile = KC ? ROWS * kLdsRow : kBK32 * kLdsRow;  // floats a stage
    static_assert(!KC || kPassRows % 16 == 0, "a pass's rows repeat the swizzle");
    __device__ static __forceinline__ int swizzle(int row) { return (row / 2) % 8; }
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
        lds_at = row * kLdsRow + (KC ? ((part / 4) ^ swizzle(row)) * 4 : part);
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
        if (KC) return reinterpret_cast<const f32x4*>(lds)[row * (kLdsRow / 4) + ((k / 4) ^ swizzle(row))];
        return f32x4{lds[k * kLdsRow + row], lds[(k + 1) * kLdsRow + row], lds[(k + 2) * kLdsRow + row],
                     lds[(k + 3) * kLdsRow + row]};
    }
};

// BM x BN tiles over four waves of (BM / 2) x (BN / 2).
template <typename O, bool A_KC, bool B_KC, int BM, int BN, class EPI = PlainStore>
__global__ void __launch_bounds__(kThreads) inplace32_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                             O* __restrict__ C, uint32_t M, uint32_t N, uint32_t K,
                                                             bool accumulate, EPI epi) {
    using SA = Stager32<BM, A_KC>;
    using SB = Stager32<BN, B_KC>;
    constexpr int TM = BM / 32, TN = BN / 32;  // 16 x 16 tiles per wave
    constexpr int kA = SA::kTile;
    constexpr int kB = SB::kTile;
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

    if constexpr (EPI::kProgram) {
        // Passes of a power-of-two number of rows that fit in both A stages,
        // each taking the same share of both wave rows.
        constexpr int kFit = 2 * kA / BN;
        constexpr int kPass = kFit >= 128 ? 128 : 64;
        constexpr int kPasses = BM / kPass, H = BM / 2 / kPasses;
        static_assert(kFit >= kPass && BM % kPass == 0 && H % 16 == 0, "a pass fits in LDS");
        // The run form loads what every row reads alike for the thread's
        // four columns before any store, so no load waits behind one.
        typename RunState<EPI>::Invariant inv{};
        if constexpr (HasRuns<EPI>::value) {
            static_assert(kThreads % (BN / 4) == 0, "a thread keeps its columns in every round");
            const uint32_t col = n0 + (threadIdx.x % (BN / 4)) * 4;
            epi.invariant(inv, col < N, col);
        }
#pragma unroll
        for (int pass = 0; pass < kPasses; pass++) {
            lds_barrier();  // every wave is done with LDS
#pragma unroll
            for (int i = pass * H / 16; i < (pass + 1) * H / 16; i++) {
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const uint32_t col = wn * (BN / 2) + j * 16 + lane % 16;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const uint32_t rr = wm * H + i * 16 - pass * H + 4 * (lane / 16) + e;
                        *staged_at<BN, 16, kPass>(lds_a, lds_a, lds_a, lds_a, rr, col) = acc[i][j][e];
                    }
                }
            }
            lds_barrier();
            if constexpr (HasRuns<EPI>::value) {
                program_runs<BN, 16, kPass, H, BM / 2>(epi, inv, lds_a, kPass, pass, m0, n0, M, N);
            } else {
                program_pass<BN, 16, kPass, H, BM / 2>(epi, lds_a, lds_a, lds_a, lds_a, kPass, pass, m0, n0, M, N);
            }
        }
    } else {
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
    // The same lanes' chunks of another block tile: only the resource
    // (its base and range) depends on the tile.
    __device__ __forceinline__ void retarget(const S* p, uint32_t first, uint32_t rows, uint32_t ld,
                                             uint32_t depth) {
        if (KC) {
            rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<S*>(p + static_cast<uint64_t>(first) * ld), 0,
                                                     (rows - first) * ld * sizeof(S), kBufferFlags);
        } else {
            rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<S*>(p + first), 0, (depth * ld - first) * sizeof(S),
                                                     kBufferFlags);
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

template <typename S, typename O, bool A_KC, bool B_KC, int BM, int BN, int WM, int WN, int BK, int NS,
          class EPI = PlainStore>
__global__ void __launch_bounds__(WM * WN * 64) direct16_kernel(const S* __restrict__ A, const S* __restrict__ B,
                                                                O* __restrict__ C, uint32_t M, uint32_t N, uint32_t K,
                                                                bool accumulate, EPI epi) {
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

    if constexpr (EPI::kProgram) {
        // The four stage arrays, BK / 2 rows of BN floats each, hold a pass
        // of 2 BK rows.
        static_assert(NS == 2 && BM == BN && kA == kB, "square tiles over two stages");
        constexpr int kRegionRows = kA * static_cast<int>(sizeof(S)) / 4 / BN;
        constexpr int kPass = 4 * kRegionRows;
        constexpr int kPasses = BM / kPass, H = BM / WM / kPasses;
        static_assert(BM % kPass == 0 && H % 32 == 0, "whole passes of whole matrix-core tiles");
        float* r0 = reinterpret_cast<float*>(stage_tile<S, kA, 0>());
        float* r1 = reinterpret_cast<float*>(stage_tile<S, kB, 1>());
        float* r2 = reinterpret_cast<float*>(stage_tile<S, kA, 2>());
        float* r3 = reinterpret_cast<float*>(stage_tile<S, kB, 3>());
        __builtin_amdgcn_s_waitcnt(vmcnt_wait(0));  // the last step's reload has landed
#pragma unroll
        for (int pass = 0; pass < kPasses; pass++) {
            lds_barrier();  // every wave is done with LDS
#pragma unroll
            for (int i = pass * H / 32; i < (pass + 1) * H / 32; i++) {
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const uint32_t col = wn * (BN / WN) + j * 32 + lane % 32;
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        const uint32_t rr = wm * H + i * 32 - pass * H + 8 * (e / 4) + 4 * (lane / 32) + e % 4;
                        *staged_at<BN, 32, kRegionRows>(r0, r1, r2, r3, rr, col) = acc[i][j][e];
                    }
                }
            }
            lds_barrier();
            program_pass<BN, 32, kRegionRows, H, BM / WM>(epi, r0, r1, r2, r3, kPass, pass, m0, n0, M,
                                                                           N);
        }
    } else if (m0 + BM <= M && n0 + BN <= N) {
        // A whole tile: no bounds to check, and each lane's column walks down
        // from one base pointer in steps of N.
        O* base = C + static_cast<uint64_t>(m0 + wm * (BM / WM) + 4 * (lane / 32)) * N + n0 + wn * (BN / WN) +
                  lane % 32;
#pragma unroll
        for (int i = 0; i < TM; i++) {
#pragma unroll
            for (int j = 0; j < TN; j++) {
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const uint32_t r = i * 32 + 8 * (e / 4) + e % 4;
                    store_out(base, static_cast<uint64_t>(r) * N + j * 32, acc[i][j][e], accumulate);
                }
            }
        }
    } else {
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
}
// ---- the 16 x 16 x 32 kernel ---------------------------------------------------
//
// The large-product kernel: 256 x 256 block tiles over eight waves of 128 x 64
// (two waves a SIMD), 16 x 16 x 32 matrix-core steps, 64-deep K steps in two
// LDS stages filled by direct loads.  Measured on MI355X against the 32 x 32
// x 16 kernel above at 8192^3 bf16, it holds a higher clock under sustained
// load (the smaller step moves fewer accumulator bytes through the register
// file per product), and the order below keeps the matrix cores busier:
//  - Operands are swapped into the matrix-core step (B's fragment first), so
//    a lane's four accumulators are four consecutive columns of C, stored as
//    one 8-byte write.
//  - Step s runs its first 32-deep slice from registers while reading the
//    second slice's fragments from stage s % 2; at the barrier that follows,
//    stage s % 2 is free and step s + 1 is visible, so step s + 2's loads go
//    into stage s % 2 at once: a load has a whole step to land.  The second
//    slice then runs while step s + 1's first fragments are read.
//  - A's fragments are read back into the same registers right after their
//    last use; B's are double-buffered.  Each slice is ordered as groups of
//    four matrix-core steps, each followed by its share of the LDS reads (all
//    issued before the slice's last group, so the wait at the barrier is
//    short) and of the direct loads.
//  - Barriers are bare s_barrier with explicit waits: __syncthreads' fence
//    would also wait for the loads of the step ahead.
// Row-contiguous stage tiles are swizzled so that the eight k-rows a
// half-wave's transposing read touches fall on distinct bank groups.

template <typename S>
struct Mfma16x16;
template <>
struct Mfma16x16<bf16_t> {
    __device__ static f32x4 step(uint4 a, uint4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                       0, 0, 0);
    }
};
template <>
struct Mfma16x16<_Float16> {
    __device__ static f32x4 step(uint4 a, uint4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                      0, 0);
    }
};

// s_waitcnt immediates: vmcnt(n) and lgkmcnt(0); lgkmcnt(0) alone.
constexpr int vmcnt_lgkm0(int n) { return (n & 0xf) | ((n >> 4) << 14) | (0x7 << 4); }

// A workgroup barrier that orders nothing by itself: callers wait for what
// they need first.  The compiler keeps memory accesses on their side.
__device__ __forceinline__ void bare_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// Chunk swizzle of a row-contiguous tile for the 16 x 16 x 32 reads: k-rows 0-3
// and 8-11 of a slice (one half-wave's transposing read) differ in the low
// four chunk bits.
__device__ __forceinline__ int rc16_swizzle(int k) { return ((k & 3) << 2) | (((k >> 3) & 1) << 1); }

// Direct-load staging of one operand's stage tile with per-lane offsets that
// repeat: the swizzle of a lane's chunk has a period of 16 rows, so when a
// wave's consecutive instructions are 16 rows apart (or a multiple) one
// offset serves them all, and when they are 8 rows apart (four waves over a
// row-contiguous tile) two alternate.  Instruction i adds a uniform stride
// (kept in a scalar register) to offset i % kPeriod.
template <typename S, int ROWS, bool KC, int WAVES, int BK>
struct StrideStager {
    static constexpr int kInstr = ROWS * BK * 2 / 1024;  // one wave instruction moves 1 KiB
    static constexpr int kPer = kInstr / WAVES;
    static constexpr int kRowsPer = KC ? 1024 / (BK * 2) : 1024 / (ROWS * 2);
    static constexpr int kChunksPerRow = KC ? BK / 8 : ROWS / 8;
    static constexpr int kApart = kRowsPer * WAVES;  // rows from one of a wave's instructions to the next
    static constexpr int kPeriod = kApart % 16 == 0 ? 1 : 16 / kApart;
    static_assert(kInstr % WAVES == 0, "whole instructions per wave");
    static_assert((kApart * kPeriod) % 16 == 0 && kPer % kPeriod == 0, "whole swizzle periods per wave");
    __amdgpu_buffer_rsrc_t rsrc;
    uint32_t offset[kPeriod];  // this lane's chunk of instructions 0 .. kPeriod - 1, bytes at k0 = 0
    uint32_t k_of[kPeriod];    // its k within a step (K-contiguous only)
    uint32_t stride;           // bytes from one period's rows to the next's
    uint32_t k_bytes;
    int wave;

    __device__ void init(const S* p, uint32_t first, uint32_t rows, uint32_t ld, uint32_t depth, int w, int lane) {
        wave = w;
#pragma unroll
        for (int q = 0; q < kPeriod; q++) {
            const int row = kRowsPer * w + kApart * q + lane / kChunksPerRow;
            const int chunk = (lane % kChunksPerRow) ^ (KC ? kc_swizzle<BK>(row) : rc16_swizzle(row));
            offset[q] = (static_cast<uint32_t>(row) * ld + chunk * 8) * sizeof(S);
            k_of[q] = KC ? chunk * 8 : 0;
        }
        stride = kApart * kPeriod * ld * sizeof(S);
        k_bytes = KC ? sizeof(S) : ld * sizeof(S);
        retarget(p, first, rows, ld, depth);
    }
    // Another block tile of the same operand: only the resource changes.
    __device__ __forceinline__ void retarget(const S* p, uint32_t first, uint32_t rows, uint32_t ld, uint32_t depth) {
        if (KC) {
            rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<S*>(p + static_cast<uint64_t>(first) * ld), 0,
                                                     (rows - first) * ld * sizeof(S), kBufferFlags);
        } else {
            rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<S*>(p + first), 0, (depth * ld - first) * sizeof(S),
                                                     kBufferFlags);
        }
    }
    // Stage the step at k0 into `tile`.  Past K a K-contiguous chunk is the
    // next row's, so it is pointed past the resource (operands are under
    // 2^31 bytes) and loads zeros.
    __device__ __forceinline__ void fetch(S* tile, uint32_t k0, uint32_t K, bool full) const {
#pragma unroll
        for (int i = 0; i < kPer; i++) {
            const int q = i % kPeriod;
            const uint32_t at = (full || !KC || k0 + k_of[q] < K) ? offset[q] : 0x80000000u;
            uint8_t* dst = reinterpret_cast<uint8_t*>(tile) + 1024 * (wave + WAVES * i);
            // The scalar offset is uniform; said so, the compiler keeps it in
            // a scalar register rather than looping over lanes.
            const uint32_t soffset = __builtin_amdgcn_readfirstlane(k0 * k_bytes + (i / kPeriod) * stride);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)dst, 16, at,
                                                     soffset, 0, 0);
        }
    }
    // Instruction i of this wave's share of a whole step (no K tail).
    __device__ __forceinline__ void fetch_one(S* tile, uint32_t k0, int i) const {
        const int q = i % kPeriod;
        uint8_t* dst = reinterpret_cast<uint8_t*>(tile) + 1024 * (wave + WAVES * i);
        const uint32_t soffset = __builtin_amdgcn_readfirstlane(k0 * k_bytes + (i / kPeriod) * stride);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)dst, 16, offset[q],
                                                 soffset, 0, 0);
    }
};

// Per-lane byte offsets of 16 x 16 x 32 operands in a 64-deep stage tile.  A
// lane's operand is tile row (first + 16 blk + lane % 16) at k = 32 q + 8 (lane
// / 16) .. + 8.  K-contiguous tile (rows of 128 bytes, chunk c of row r at
// c ^ ((r / 2) % 8)): offset(q) + 2048 blk.
__device__ __forceinline__ uint32_t kc16_offset(int lane, int first_row, int q) {
    const int r = first_row + lane % 16, g = lane / 16;
    return static_cast<uint32_t>(r * 128 + ((4 * q + g) ^ ((r / 2) % 8)) * 16);
}
// Row-contiguous tile (k-rows of ROWS elements): the transposing reads of
// column block `blk` are at offset(blk) + 32 q * ROWS * 2 and four k-rows on.
template <int ROWS>
__device__ __forceinline__ uint32_t rc16_offset(int lane, int first_col, int blk) {
    const int g = lane / 16, j = lane % 16;
    const int k = 8 * g + j / 4;
    const int col = first_col + 16 * blk + 4 * (j % 4);
    const int chunk = (col / 8) ^ rc16_swizzle(k);
    return static_cast<uint32_t>(k * ROWS * 2 + chunk * 16 + (col % 8) * 2);
}

template <typename S>
__device__ __forceinline__ uint4 lds_b128(const S* tile, uint32_t offset) {
    return *reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(tile) + offset);
}
template <typename S, int ROWS>
__device__ __forceinline__ uint4 lds_tr_pair(const S* tile, uint32_t offset) {
    const uint8_t* at = reinterpret_cast<const uint8_t*>(tile) + offset;
    short4v lo = read_tr16(at);
    short4v hi = read_tr16(at + 4 * ROWS * 2);
    uint4 out;
    out.x = static_cast<uint16_t>(lo[0]) | (static_cast<uint32_t>(static_cast<uint16_t>(lo[1])) << 16);
    out.y = static_cast<uint16_t>(lo[2]) | (static_cast<uint32_t>(static_cast<uint16_t>(lo[3])) << 16);
    out.z = static_cast<uint16_t>(hi[0]) | (static_cast<uint32_t>(static_cast<uint16_t>(hi[1])) << 16);
    out.w = static_cast<uint16_t>(hi[2]) | (static_cast<uint32_t>(static_cast<uint16_t>(hi[3])) << 16);
    return out;
}

// One slice's order: G groups of PER matrix-core steps, each followed by its
// share of READS LDS reads (spread over the first G - LAG groups) and of
// LOADS direct loads.
template <int G, int PER, int READS, int LOADS, int LAG, int g = 0>
__device__ __forceinline__ void weave16() {
    if constexpr (g < G) {
        __builtin_amdgcn_sched_group_barrier(0x008, PER, 0);  // matrix-core steps
        constexpr int RG = G - LAG;
        constexpr int r = g < RG ? READS * (g + 1) / RG - READS * g / RG : 0;
        constexpr int l = LOADS * (g + 1) / G - LOADS * g / G;
        if constexpr (r > 0) __builtin_amdgcn_sched_group_barrier(0x100, r, 0);  // LDS reads
        if constexpr (l > 0) __builtin_amdgcn_sched_group_barrier(0x020, l, 0);  // direct loads
        weave16<G, PER, READS, LOADS, LAG, g + 1>();
    }
}

// Four consecutive columns of C from a lane's accumulators, (+)=, rounded once
// (`at` aligned to four elements).
template <typename O>
__device__ __forceinline__ void store_quad(O* at, f32x4 v, bool accumulate) {
    using E = Elem<O>;
    if constexpr (sizeof(O) == 4) {
        if (accumulate) v += *reinterpret_cast<const f32x4*>(at);
        *reinterpret_cast<f32x4*>(at) = v;
    } else {
        if (accumulate) {
            const uint2 old = *reinterpret_cast<const uint2*>(at);
            v[0] += E::widen(__builtin_bit_cast(O, static_cast<uint16_t>(old.x & 0xffff)));
            v[1] += E::widen(__builtin_bit_cast(O, static_cast<uint16_t>(old.x >> 16)));
            v[2] += E::widen(__builtin_bit_cast(O, static_cast<uint16_t>(old.y & 0xffff)));
            v[3] += E::widen(__builtin_bit_cast(O, static_cast<uint16_t>(old.y >> 16)));
        }
        uint2 out;
        out.x = pack_pair<O>(v[0], v[1]);
        out.y = pack_pair<O>(v[2], v[3]);
        *reinterpret_cast<uint2*>(at) = out;
    }
}

// C (+)= A . B on 256 x 256 tiles, one tile a block, finished by plain
// stores or a program epilogue (how a tile is finished, above).  Operands are
// 16-byte aligned row by row and under 2^31 bytes.
template <typename S, typename O, bool A_KC, bool B_KC, class EPI = PlainStore>
__global__ void __launch_bounds__(512) gemm16x16_kernel(const S* __restrict__ A, const S* __restrict__ B,
                                                         O* __restrict__ C, uint32_t M, uint32_t N, uint32_t K,
                                                         bool accumulate, EPI epi) {
    constexpr int BM = 256, BN = 256, BK = 64, WM = 2, WN = 4, kWaves = WM * WN;
    constexpr int TM = BM / WM / 16, TN = BN / WN / 16;  // 16-wide blocks of a wave's 128 x 64
    constexpr int kA = BM * BK, kB = BN * BK;
    using StagerA = StrideStager<S, BM, A_KC, kWaves, BK>;
    using StagerB = StrideStager<S, BN, B_KC, kWaves, BK>;
    constexpr int kLoads = StagerA::kPer + StagerB::kPer;
    constexpr int kReads = TM * (A_KC ? 1 : 2) + TN * (B_KC ? 1 : 2);

    const uint32_t tiles_m = (M + BM - 1) / BM;
    const uint32_t tiles_n = (N + BN - 1) / BN;
    if (blockIdx.x >= tiles_m * tiles_n) return;
    uint32_t tm, tn;
    tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const int lane = threadIdx.x % 64;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int wm = wave / WN, wn = wave % WN;

    StagerA sa;
    StagerB sb;
    sa.init(A, m0, M, A_KC ? K : M, K, wave, lane);
    sb.init(B, n0, N, B_KC ? K : N, K, wave, lane);

    // Fragment offsets: K-contiguous operands one per slice, row-contiguous
    // ones one per 16-wide block.
    uint32_t a_off[A_KC ? 2 : TM], b_off[B_KC ? 2 : TN];
    if constexpr (A_KC) {
        a_off[0] = kc16_offset(lane, wm * (BM / WM), 0);
        a_off[1] = kc16_offset(lane, wm * (BM / WM), 1);
    } else {
#pragma unroll
        for (int i = 0; i < TM; i++) a_off[i] = rc16_offset<BM>(lane, wm * (BM / WM), i);
    }
    if constexpr (B_KC) {
        b_off[0] = kc16_offset(lane, wn * (BN / WN), 0);
        b_off[1] = kc16_offset(lane, wn * (BN / WN), 1);
    } else {
#pragma unroll
        for (int j = 0; j < TN; j++) b_off[j] = rc16_offset<BN>(lane, wn * (BN / WN), j);
    }
    auto frag_a = [&](const S* t, int i, int q) __attribute__((always_inline)) {
        return A_KC ? lds_b128(t, a_off[q] + 2048 * i) : lds_tr_pair<S, BM>(t, a_off[i] + q * 32 * BM * 2);
    };
    auto frag_b = [&](const S* t, int j, int q) __attribute__((always_inline)) {
        return B_KC ? lds_b128(t, b_off[q] + 2048 * j) : lds_tr_pair<S, BN>(t, b_off[j] + q * 32 * BN * 2);
    };

    f32x4 acc[TM][TN];
    uint4 fa[TM], fb[2][TN];
    const uint32_t steps = (K + BK - 1) / BK;
    // Step s; past the last step, a harmless reload of it.
    auto stage_of = [&](auto t, uint32_t s) __attribute__((always_inline)) {
        const uint32_t k0 = (s < steps ? s : steps - 1) * BK;
        sa.fetch(stage_tile<S, kA, 2 * decltype(t)::value>(), k0, K, k0 + BK <= K);
        sb.fetch(stage_tile<S, kB, 2 * decltype(t)::value + 1>(), k0, K, k0 + BK <= K);
    };
    auto read_b = [&](int slot, const S* lb, int q) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < TN; j++) fb[slot][j] = frag_b(lb, j, q);
    };
    // One slice's products; A's block i is re-read from (la, q) after its
    // last product.
    auto slice = [&](int slot, const S* la, int q) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < TM; i++) {
#pragma unroll
            for (int j = 0; j < TN; j++) acc[i][j] = Mfma16x16<S>::step(fb[slot][j], fa[i], acc[i][j]);
            fa[i] = frag_a(la, i, q);
        }
    };
    auto step = [&](auto t, uint32_t s) __attribute__((always_inline)) {
        constexpr int T = decltype(t)::value;
        constexpr int U = T ^ 1;
        read_b(1, stage_tile<S, kB, 2 * T + 1>(), 1);
        slice(0, stage_tile<S, kA, 2 * T>(), 1);
        weave16<TM, TN, kReads, 0, 1>();
        __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0(0));  // step s + 1 is in LDS; stage T is read
        bare_barrier();
        stage_of(t, s + 2);
        read_b(0, stage_tile<S, kB, 2 * U + 1>(), 0);
        slice(1, stage_tile<S, kA, 2 * U>(), 0);
        weave16<TM, TN, kReads, kLoads, 0>();
        __builtin_amdgcn_sched_barrier(0);
    };

    if (steps > 0) {
        stage_of(std::integral_constant<int, 0>{}, 0);
        stage_of(std::integral_constant<int, 1>{}, 1);
        __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0(kLoads));  // step 0 is in LDS
        bare_barrier();
        read_b(0, stage_tile<S, kB, 1>(), 0);
#pragma unroll
        for (int i = 0; i < TM; i++) fa[i] = frag_a(stage_tile<S, kA, 0>(), i, 0);
    }
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = f32x4{};
    for (uint32_t s = 0; s < steps; s += 2) {
        step(std::integral_constant<int, 0>{}, s);
        if (s + 1 < steps) step(std::integral_constant<int, 1>{}, s + 1);
    }
    // lane holds C[row][col .. col + 3] for row = m0 + wm*128 + 16 i + lane % 16,
    // col = n0 + wn*64 + 16 j + 4 (lane / 16).
    if constexpr (EPI::kProgram) {
        // The four stage arrays, BK / 2 rows of BN floats each, hold a pass of
        // 128 rows: 64 of each wave row, so each wave stages the same share of
        // its accumulators in every pass.
        constexpr int kRegionRows = kA * static_cast<int>(sizeof(S)) / 4 / BN;
        constexpr int kPass = 4 * kRegionRows;
        constexpr int kPasses = BM / kPass, H = BM / WM / kPasses;
        static_assert(BM == BN && kA == kB && BM % kPass == 0 && H % 16 == 0, "whole passes of whole 16-row blocks");
        float* r0 = reinterpret_cast<float*>(stage_tile<S, kA, 0>());
        float* r1 = reinterpret_cast<float*>(stage_tile<S, kB, 1>());
        float* r2 = reinterpret_cast<float*>(stage_tile<S, kA, 2>());
        float* r3 = reinterpret_cast<float*>(stage_tile<S, kB, 3>());
        __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0(0));  // the last step's reloads have landed
#pragma unroll
        for (int pass = 0; pass < kPasses; pass++) {
            lds_barrier();  // every wave is done with LDS
#pragma unroll
            for (int i = pass * H / 16; i < (pass + 1) * H / 16; i++) {
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const uint32_t rr = wm * H + 16 * i + lane % 16 - pass * H;
                    const uint32_t col = wn * (BN / WN) + 16 * j + 4 * (lane / 16);
                    *reinterpret_cast<f32x4*>(staged_at<BN, 0, kRegionRows>(r0, r1, r2, r3, rr, col)) = acc[i][j];
                }
            }
            lds_barrier();
            program_pass<BN, 0, kRegionRows, H, BM / WM>(epi, r0, r1, r2, r3, kPass, pass, m0, n0, M, N);
        }
        return;
    }
    const bool quads = (N % 4) == 0 && (reinterpret_cast<uint64_t>(C) % (4 * sizeof(O))) == 0;
    const uint32_t row0 = m0 + wm * (BM / WM) + lane % 16;
    const uint32_t col0 = n0 + wn * (BN / WN) + 4 * (lane / 16);
    O* base = C + static_cast<uint64_t>(row0) * N + col0;
#pragma unroll
    for (int i = 0; i < TM; i++) {
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const uint32_t row = row0 + 16 * i, col = col0 + 16 * j;
            O* at = base + static_cast<uint64_t>(16 * i) * N + 16 * j;
            if (quads && row < M && col + 4 <= N) {
                store_quad(at, acc[i][j], accumulate);
            } else if (row < M) {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (col + e < N) store_out(at, e, acc[i][j][e], accumulate);
            }
        }
    }
    // No direct load may still be writing LDS when the block ends.
    __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0(0));
}

// The 16 x 16 x 32 kernel made persistent: one block a CU walks every
// gridDim.x-th tile, so a tile's first loads and the previous tile's stores
// do not sit between two tiles' matrix-core steps.
//  - The step loop is the one-tile kernel's, in pairs; the last pair of a
//    tile fetches the next tile's first two steps (its operand resources are
//    retargeted at the top of that pair), and the last step's trailing reads
//    are the next tile's first fragments.  Steps must come in whole pairs
//    (an even count) so that every tile starts on stage 0.
//  - A whole tile of 16-bit C is stored as whole rows: each wave stages a
//    quarter of its 128 x 64 results at a time in its own 4 KiB of a further
//    32 KiB of LDS (16-byte chunk c of row r at c ^ (r % 8)) and writes them
//    back 16 bytes a lane, eight lanes a 128-byte row.  Measured on MI355X at
//    f16 16384 x 4096 x 1024, against 8-byte stores straight from the
//    accumulators (16 rows of 32 bytes an instruction): 114 against 129 us.
//    The staging's LDS accesses are written as inline assembly: the compiler
//    cannot tell the staging array from the stages the direct loads are
//    filling, and would otherwise wait for the next tile's loads before the
//    first staging write.  Within a wave, LDS accesses complete in order.
//  - Edge tiles, f32 C and accumulation store from the accumulators, as the
//    one-tile kernel does.
//  - A program epilogue runs wave by wave over the same 4 KiB: a wave
//    stages one 16-row block of its f32 results at a time (16-byte chunk c
//    of row r at c ^ r, conflict-free both ways) and hands the program
//    EPI::kElems elements a lane, 64 lanes on 64 neighbouring columns, so
//    its loads and stores are row runs.  No block barrier is needed: each
//    wave reads back only what it wrote.
template <typename S, typename O, bool A_KC, bool B_KC, class EPI = PlainStore>
__global__ void __launch_bounds__(512) gemm16x16_persistent_kernel(const S* __restrict__ A, const S* __restrict__ B,
                                                                    O* __restrict__ C, uint32_t M, uint32_t N,
                                                                    uint32_t K, bool accumulate, EPI epi) {
    constexpr int BM = 256, BN = 256, BK = 64, WM = 2, WN = 4, kWaves = WM * WN;
    constexpr int TM = BM / WM / 16, TN = BN / WN / 16;
    constexpr int kA = BM * BK, kB = BN * BK;
    using StagerA = StrideStager<S, BM, A_KC, kWaves, BK>;
    using StagerB = StrideStager<S, BN, B_KC, kWaves, BK>;
    constexpr int kLoads = StagerA::kPer + StagerB::kPer;
    constexpr int kReads = TM * (A_KC ? 1 : 2) + TN * (B_KC ? 1 : 2);
    constexpr int kRegion = 4096;  // staging bytes a wave

    const uint32_t tiles_m = (M + BM - 1) / BM;
    const uint32_t tiles_n = (N + BN - 1) / BN;
    const uint32_t tiles = tiles_m * tiles_n;
    uint32_t tile = blockIdx.x;
    if (tile >= tiles) return;
    uint32_t tm, tn;
    tile_of(tile, tiles_m, tiles_n, tm, tn);
    uint32_t m0 = tm * BM, n0 = tn * BN;
    const int lane = threadIdx.x % 64;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int wm = wave / WN, wn = wave % WN;

    StagerA sa;
    StagerB sb;
    sa.init(A, m0, M, A_KC ? K : M, K, wave, lane);
    sb.init(B, n0, N, B_KC ? K : N, K, wave, lane);

    uint32_t a_off[A_KC ? 2 : TM], b_off[B_KC ? 2 : TN];
    if constexpr (A_KC) {
        a_off[0] = kc16_offset(lane, wm * (BM / WM), 0);
        a_off[1] = kc16_offset(lane, wm * (BM / WM), 1);
    } else {
#pragma unroll
        for (int i = 0; i < TM; i++) a_off[i] = rc16_offset<BM>(lane, wm * (BM / WM), i);
    }
    if constexpr (B_KC) {
        b_off[0] = kc16_offset(lane, wn * (BN / WN), 0);
        b_off[1] = kc16_offset(lane, wn * (BN / WN), 1);
    } else {
#pragma unroll
        for (int j = 0; j < TN; j++) b_off[j] = rc16_offset<BN>(lane, wn * (BN / WN), j);
    }
    auto frag_a = [&](const S* t, int i, int q) __attribute__((always_inline)) {
        return A_KC ? lds_b128(t, a_off[q] + 2048 * i) : lds_tr_pair<S, BM>(t, a_off[i] + q * 32 * BM * 2);
    };
    auto frag_b = [&](const S* t, int j, int q) __attribute__((always_inline)) {
        return B_KC ? lds_b128(t, b_off[q] + 2048 * j) : lds_tr_pair<S, BN>(t, b_off[j] + q * 32 * BN * 2);
    };

    f32x4 acc[TM][TN];
    uint4 fa[TM], fb[2][TN];
    const uint32_t steps = (K + BK - 1) / BK;
    auto fetch = [&](auto t, uint32_t k0) __attribute__((always_inline)) {
        sa.fetch(stage_tile<S, kA, 2 * decltype(t)::value>(), k0, K, k0 + BK <= K);
        sb.fetch(stage_tile<S, kB, 2 * decltype(t)::value + 1>(), k0, K, k0 + BK <= K);
    };
    auto read_b = [&](int slot, const S* lb, int q) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < TN; j++) fb[slot][j] = frag_b(lb, j, q);
    };
    auto slice = [&](int slot, const S* la, int q) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < TM; i++) {
#pragma unroll
            for (int j = 0; j < TN; j++) acc[i][j] = Mfma16x16<S>::step(fb[slot][j], fa[i], acc[i][j]);
            fa[i] = frag_a(la, i, q);
        }
    };
    // One step from stage T; after its barrier, stage T takes the step at
    // `k_next` (of this tile or the next).
    auto step = [&](auto t, uint32_t k_next) __attribute__((always_inline)) {
        constexpr int T = decltype(t)::value;
        constexpr int U = T ^ 1;
        read_b(1, stage_tile<S, kB, 2 * T + 1>(), 1);
        slice(0, stage_tile<S, kA, 2 * T>(), 1);
        weave16<TM, TN, kReads, 0, 1>();
        __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0(0));  // the next step is in LDS; stage T is read
        bare_barrier();
        fetch(t, k_next);
        read_b(0, stage_tile<S, kB, 2 * U + 1>(), 0);
        slice(1, stage_tile<S, kA, 2 * U>(), 0);
        weave16<TM, TN, kReads, kLoads, 0>();
        __builtin_amdgcn_sched_barrier(0);
    };

    // Each lane's staging offsets: where it writes the quad of columns
    // 16 j + 4 (lane / 16) of row r (16-byte chunk 2 j + lane / 32), and
    // where it reads chunk lane % 8 of row lane / 8 (and 8, 16, 24 rows on,
    // which share the row's swizzle).
    __shared__ __attribute__((aligned(1024))) uint8_t rows_lds[kWaves * kRegion];
    const uint32_t region = static_cast<uint32_t>(reinterpret_cast<uint64_t>(
                                (__attribute__((address_space(3))) uint8_t*)(rows_lds))) +
                            wave * kRegion;
    const uint32_t read_at = region + (lane / 8) * 128 + (((lane % 8) ^ (lane / 8)) * 16);
    const uint32_t row_off = ((lane / 8) * N + 8 * (lane % 8)) * sizeof(O);
    const bool rows_ok = sizeof(O) == 2 && (N % 8) == 0 && (reinterpret_cast<uint64_t>(C) % 16) == 0 && !accumulate;

    fetch(std::integral_constant<int, 0>{}, 0);
    fetch(std::integral_constant<int, 1>{}, BK);
    __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0(kLoads));  // the first step is in LDS
    bare_barrier();
    read_b(0, stage_tile<S, kB, 1>(), 0);
#pragma unroll
    for (int i = 0; i < TM; i++) fa[i] = frag_a(stage_tile<S, kA, 0>(), i, 0);
    for (;;) {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) acc[i][j] = f32x4{};
        for (uint32_t s = 0; s < steps; s += 2) {
            uint32_t k_next = (s + 2) * BK;
            if (s + 2 == steps) {
                // After the last tile, its own first steps again: harmless
                // loads into stages nobody reads.
                const uint32_t next = tile + gridDim.x < tiles ? tile + gridDim.x : tile;
                uint32_t nm, nn;
                tile_of(next, tiles_m, tiles_n, nm, nn);
                sa.retarget(A, nm * BM, M, A_KC ? K : M, K);
                sb.retarget(B, nn * BN, N, B_KC ? K : N, K);
                k_next = 0;
            }
            step(std::integral_constant<int, 0>{}, k_next);
            step(std::integral_constant<int, 1>{}, k_next + BK);
        }
        // lane holds C[row][col .. col + 3] for row = m0 + wm*128 + 16 i + lane % 16,
        // col = n0 + wn*64 + 16 j + 4 (lane / 16).
        if constexpr (EPI::kProgram) {
            constexpr int E = EPI::kElems;
            static_assert(16 % E == 0, "whole groups of a staged block's 16 rows");
            float* staged = reinterpret_cast<float*>(rows_lds + wave * kRegion);
            const int r = lane % 16, g = lane / 16;
#pragma unroll
            for (int i = 0; i < TM; i++) {
#pragma unroll
                for (int j = 0; j < TN; j++)
                    *reinterpret_cast<f32x4*>(staged + r * 64 + (((4 * j + g) ^ r) * 4)) = acc[i][j];
#pragma unroll
                for (int v0 = 0; v0 < 16; v0 += E) {
                    bool live[E];
                    uint32_t row[E], col[E];
                    float product[E];
#pragma unroll
                    for (int e = 0; e < E; e++) {
                        const int v = v0 + e;
                        product[e] = staged[v * 64 + (((lane / 4) ^ v) * 4) + lane % 4];
                        row[e] = m0 + wm * (BM / WM) + 16 * i + v;
                        col[e] = n0 + wn * (BN / WN) + lane;
                        live[e] = row[e] < M && col[e] < N;
                    }
                    epi.group(live, row, col, N, product);
                }
            }
        } else if (rows_ok && m0 + BM <= M && n0 + BN <= N) {
          if constexpr (sizeof(O) == 2) {
            const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
                C + static_cast<uint64_t>(m0 + wm * (BM / WM)) * N + n0 + wn * (BN / WN), 0, 0x7fffffff,
                kBufferFlags);
            const int g = lane / 16;
#pragma unroll
            for (int p = 0; p < TM / 2; p++) {
#pragma unroll
                for (int ii = 0; ii < 2; ii++) {
                    const int r = ii * 16 + lane % 16;
#pragma unroll
                    for (int j = 0; j < TN; j++) {
                        const f32x4 v = acc[2 * p + ii][j];
                        const u32x2 out = {pack_pair<O>(v[0], v[1]), pack_pair<O>(v[2], v[3])};
                        const uint32_t at = region + r * 128 + (((2 * j + g / 2) ^ (r % 8)) * 16) + (g % 2) * 8;
                        asm volatile("ds_write_b64 %0, %1" ::"v"(at), "v"(out) : "memory");
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
                u32x4 v0, v1, v2, v3;
                asm volatile(
                    "ds_read_b128 %0, %4\n\t"
                    "ds_read_b128 %1, %4 offset:1024\n\t"
                    "ds_read_b128 %2, %4 offset:2048\n\t"
                    "ds_read_b128 %3, %4 offset:3072\n\t"
                    "s_waitcnt lgkmcnt(0)"
                    : "=&v"(v0), "=&v"(v1), "=&v"(v2), "=&v"(v3)
                    : "v"(read_at)
                    : "memory");
                const uint32_t first = __builtin_amdgcn_readfirstlane(32 * p * N * sizeof(O));
                const uint32_t eight = __builtin_amdgcn_readfirstlane(8 * N * sizeof(O));
                __builtin_amdgcn_raw_buffer_store_b128(v0, rc, row_off, first, 0);
                __builtin_amdgcn_raw_buffer_store_b128(v1, rc, row_off, first + eight, 0);
                __builtin_amdgcn_raw_buffer_store_b128(v2, rc, row_off, first + 2 * eight, 0);
                __builtin_amdgcn_raw_buffer_store_b128(v3, rc, row_off, first + 3 * eight, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
          }
        } else {
            const bool quads = (N % 4) == 0 && (reinterpret_cast<uint64_t>(C) % (4 * sizeof(O))) == 0;
            const uint32_t row0 = m0 + wm * (BM / WM) + lane % 16;
            const uint32_t col0 = n0 + wn * (BN / WN) + 4 * (lane / 16);
            O* base = C + static_cast<uint64_t>(row0) * N + col0;
#pragma unroll
            for (int i = 0; i < TM; i++) {
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const uint32_t row = row0 + 16 * i, col = col0 + 16 * j;
                    O* at = base + static_cast<uint64_t>(16 * i) * N + 16 * j;
                    if (quads && row < M && col + 4 <= N) {
                        store_quad(at, acc[i][j], accumulate);
                    } else if (row < M) {
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            if (col + e < N) store_out(at, e, acc[i][j][e], accumulate);
                    }
                }
            }
        }
        tile += gridDim.x;
        if (tile >= tiles) break;
        tile_of(tile, tiles_m, tiles_n, tm, tn);
        m0 = tm * BM;
        n0 = tn * BN;
    }
    // No direct load may still be writing LDS when the block ends.
    __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0(0));
}

// ---- the wide-wave product kernel ------------------------------------------------------
//
// The same 256 x 256 tiles, 64-deep steps and persistent tile walk as above,
// over four waves of 128 x 128 (one wave a SIMD) instead of eight of 128 x 64.
// A wave reads 16 KiB of operand fragments from LDS per 64 matrix-core steps
// rather than 24 KiB, and the whole loop is ordered by hand:
//  - The 256 accumulators of a 128 x 128 wave tile fill the AGPRs.  The
//    compiler's own allocation of that many MFMA accumulators copies them
//    between register files and spills; each matrix-core step is therefore
//    written as one in-place instruction on an AGPR operand, which pins them.
//    The compiler cannot see these instructions' hazards, so the code around
//    them supplies its own: fragments are read by LDS loads straight into
//    the operand registers (a load's wait count covers it), zeroed
//    accumulators stand five wait states before the first step reads them,
//    and 42 wait states separate the last step from the reads of its results.
//  - Every operand fragment is double-buffered: a step's 32-deep slice runs
//    from one slot while the next slice's fragments load into the other.
//  - Memory operations sit one at a time between matrix-core steps: with one
//    wave a SIMD, a burst of them would leave the matrix core idle.  Slice 0
//    reads slice 1's fragments after its odd steps 1-31; one block barrier
//    follows (the next step has landed, this one is in registers); slice 1
//    issues the 16 direct loads of the step after next after every fourth
//    step and reads the next step's first fragments after odd steps 3-33.
// Measured on MI355X against the eight-wave persistent kernel (stand-alone
// harness, same bits): bf16 8192^3 1518-1523 against 1411-1437 TFLOP/s,
// the matrix cores 82% busy at 1.81 GHz against 71-72% at 1.92; f16 16384 x
// 1024 x 4096 within 1%.  Spreading the memory operations mattered: placed
// in bursts after each group of eight steps the kernel ran no faster than
// the eight-wave one, and with the loads all in the first half of the slice
// 3% slower than evenly spread.
//
// For 16-bit C written whole (no accumulate), N a multiple of 8, C 16-byte
// aligned and K a multiple of 128: each tile leaves through the staged
// whole-row stores, a lane's 16-byte piece stored only where it lies inside
// C, so edge tiles need no other path.  A program epilogue (compiled) runs
// wave by wave over the same staging, as in the persistent kernel.
template <typename S>
struct InPlaceMfma;
template <>
struct InPlaceMfma<bf16_t> {
    __device__ static __forceinline__ void step(f32x4& c, const uint4& a, const uint4& b) {
        asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0"
                     : "+a"(c)
                     : "v"(__builtin_bit_cast(u32x4, a)), "v"(__builtin_bit_cast(u32x4, b)));
    }
};
template <>
struct InPlaceMfma<_Float16> {
    __device__ static __forceinline__ void step(f32x4& c, const uint4& a, const uint4& b) {
        asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0"
                     : "+a"(c)
                     : "v"(__builtin_bit_cast(u32x4, a)), "v"(__builtin_bit_cast(u32x4, b)));
    }
};

template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// What follows matrix-core step t (0-63) of a slice: fragment read r (even r
// an A fragment, odd a B fragment, of block r / 2), direct load 100 + i, or
// nothing.
// The cache policy of the four-wave kernel's C stores: non-temporal (the
// buffer instruction's nt bit), so C streams to memory instead of settling
// in the XCD's L2, where the A and B panels the other tiles of the round are
// still reading live.  A round's C is 4 MiB an XCD, the size of its L2.
// Measured on MI355X (stand-alone harness, same bits): bf16 8192^3 1560-1585
// against 1500-1505 TFLOP/s with plain stores; streaming the operand loads
// instead measured 1285.  The f32 kernel's 4-byte stores measured 0.4-1.5%
// slower streamed, so they stay plain.
constexpr int kStreamStore = 2;

template <int SLICE>
__device__ constexpr int wide_op_at(int t) {
    if (SLICE == 0) return t % 2 == 1 && t < 32 ? t / 2 : -1;
    if (t % 4 == 0) return 100 + t / 4;
    return t % 2 == 1 && t >= 3 && t <= 33 ? (t - 3) / 2 : -1;
}

template <typename S, typename O, bool A_KC, bool B_KC, class EPI = PlainStore>
__global__ void __launch_bounds__(256) gemm16x16_wide_kernel(const S* __restrict__ A, const S* __restrict__ B,
                                                             O* __restrict__ C, uint32_t M, uint32_t N, uint32_t K,
                                                             bool accumulate, EPI epi) {
    static_assert(sizeof(O) == 2, "16-bit C");
    (void)accumulate;  // C is written whole: launched with false
    constexpr int BM = 256, BN = 256, BK = 64, WM = 2, WN = 2, kWaves = WM * WN;
    constexpr int TM = BM / WM / 16, TN = BN / WN / 16;
    constexpr int kA = BM * BK, kB = BN * BK;
    using StagerA = StrideStager<S, BM, A_KC, kWaves, BK>;
    using StagerB = StrideStager<S, BN, B_KC, kWaves, BK>;
    static_assert(StagerA::kPer == 8 && StagerB::kPer == 8, "sixteen direct loads a step");
    static_assert(TM == 8 && TN == 8, "sixteen fragments a slice");
    constexpr int kRegion = 4096;  // staging bytes a wave

    const uint32_t tiles_m = (M + BM - 1) / BM;
    const uint32_t tiles_n = (N + BN - 1) / BN;
    const uint32_t tiles = tiles_m * tiles_n;
    uint32_t tile = blockIdx.x;
    if (tile >= tiles) return;
    uint32_t tm, tn;
    tile_of(tile, tiles_m, tiles_n, tm, tn);
    uint32_t m0 = tm * BM, n0 = tn * BN;
    const int lane = threadIdx.x % 64;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int wm = wave / WN, wn = wave % WN;

    StagerA sa;
    StagerB sb;
    sa.init(A, m0, M, A_KC ? K : M, K, wave, lane);
    sb.init(B, n0, N, B_KC ? K : N, K, wave, lane);

    uint32_t a_off[A_KC ? 2 : TM], b_off[B_KC ? 2 : TN];
    if constexpr (A_KC) {
        a_off[0] = kc16_offset(lane, wm * (BM / WM), 0);
        a_off[1] = kc16_offset(lane, wm * (BM / WM), 1);
    } else {
#pragma unroll
        for (int i = 0; i < TM; i++) a_off[i] = rc16_offset<BM>(lane, wm * (BM / WM), i);
    }
    if constexpr (B_KC) {
        b_off[0] = kc16_offset(lane, wn * (BN / WN), 0);
        b_off[1] = kc16_offset(lane, wn * (BN / WN), 1);
    } else {
#pragma unroll
        for (int j = 0; j < TN; j++) b_off[j] = rc16_offset<BN>(lane, wn * (BN / WN), j);
    }
    auto frag_a = [&](const S* t, int i, int q) __attribute__((always_inline)) {
        return A_KC ? lds_b128(t, a_off[q] + 2048 * i) : lds_tr_pair<S, BM>(t, a_off[i] + q * 32 * BM * 2);
    };
    auto frag_b = [&](const S* t, int j, int q) __attribute__((always_inline)) {
        return B_KC ? lds_b128(t, b_off[q] + 2048 * j) : lds_tr_pair<S, BN>(t, b_off[j] + q * 32 * BN * 2);
    };

    f32x4 acc[TM][TN];
    uint4 fa[2][TM], fb[2][TN];
    const uint32_t steps = K / BK;

    // One step from stage T: slice 0 from slot 0 (read during the previous
    // step), slice 1 from slot 1; stage T then takes the step at k_next.
    auto step = [&](auto t, uint32_t k_next) __attribute__((always_inline)) {
        constexpr int T = decltype(t)::value;
        constexpr int U = T ^ 1;
        const S* ca = stage_tile<S, kA, 2 * T>();
        const S* cb = stage_tile<S, kB, 2 * T + 1>();
        static_for<0, TM * TN>([&](auto x) __attribute__((always_inline)) {
            constexpr int s = decltype(x)::value;
            InPlaceMfma<S>::step(acc[s / TN][s % TN], fb[0][s % TN], fa[0][s / TN]);
            constexpr int op = wide_op_at<0>(s);
            if constexpr (op >= 0) {
                if constexpr (op % 2 == 0) fa[1][op / 2] = frag_a(ca, op / 2, 1);
                else fb[1][op / 2] = frag_b(cb, op / 2, 1);
            }
            __builtin_amdgcn_sched_barrier(0);
        });
        __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0(0));  // the next step is in LDS; this one is read
        bare_barrier();
        static_for<0, TM * TN>([&](auto x) __attribute__((always_inline)) {
            constexpr int s = decltype(x)::value;
            InPlaceMfma<S>::step(acc[s / TN][s % TN], fb[1][s % TN], fa[1][s / TN]);
            constexpr int op = wide_op_at<1>(s);
            if constexpr (op >= 100) {
                if constexpr (op < 108) sa.fetch_one(stage_tile<S, kA, 2 * T>(), k_next, op - 100);
                else sb.fetch_one(stage_tile<S, kB, 2 * T + 1>(), k_next, op - 108);
            } else if constexpr (op >= 0) {
                if constexpr (op % 2 == 0) fa[0][op / 2] = frag_a(stage_tile<S, kA, 2 * U>(), op / 2, 0);
                else fb[0][op / 2] = frag_b(stage_tile<S, kB, 2 * U + 1>(), op / 2, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        });
    };

    // Staging as in the persistent kernel, per half of a wave's 128 columns.
    __shared__ __attribute__((aligned(1024))) uint8_t rows_lds[kWaves * kRegion];
    const uint32_t region = static_cast<uint32_t>(reinterpret_cast<uint64_t>(
                                (__attribute__((address_space(3))) uint8_t*)(rows_lds))) +
                            wave * kRegion;
    const uint32_t read_at = region + (lane / 8) * 128 + (((lane % 8) ^ (lane / 8)) * 16);
    const uint32_t row_off = ((lane / 8) * N + 8 * (lane % 8)) * sizeof(O);

#pragma unroll
    for (int i = 0; i < StagerA::kPer; i++) sa.fetch_one(stage_tile<S, kA, 0>(), 0, i);
#pragma unroll
    for (int i = 0; i < StagerB::kPer; i++) sb.fetch_one(stage_tile<S, kB, 1>(), 0, i);
#pragma unroll
    for (int i = 0; i < StagerA::kPer; i++) sa.fetch_one(stage_tile<S, kA, 2>(), BK, i);
#pragma unroll
    for (int i = 0; i < StagerB::kPer; i++) sb.fetch_one(stage_tile<S, kB, 3>(), BK, i);
    __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0(StagerA::kPer + StagerB::kPer));  // the first step is in LDS
    bare_barrier();
#pragma unroll
    for (int i = 0; i < TM; i++) fa[0][i] = frag_a(stage_tile<S, kA, 0>(), i, 0);
#pragma unroll
    for (int j = 0; j < TN; j++) fb[0][j] = frag_b(stage_tile<S, kB, 1>(), j, 0);
    for (;;) {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) acc[i][j] = f32x4{};
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_nop 4" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        for (uint32_t s = 0; s < steps; s += 2) {
            uint32_t k_next = (s + 2) * BK;
            if (s + 2 == steps) {
                // After the last tile, its own first steps again: harmless
                // loads into stages nobody reads.
                const uint32_t next = tile + gridDim.x < tiles ? tile + gridDim.x : tile;
                uint32_t nm, nn;
                tile_of(next, tiles_m, tiles_n, nm, nn);
                sa.retarget(A, nm * BM, M, A_KC ? K : M, K);
                sb.retarget(B, nn * BN, N, B_KC ? K : N, K);
                k_next = 0;
            }
            step(std::integral_constant<int, 0>{}, k_next);
            step(std::integral_constant<int, 1>{}, k_next + BK);
        }
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        // lane's accumulators of block (i, j): C[row][col .. col + 3] for row =
        // m0 + wm*128 + 16 i + lane % 16, col = n0 + wn*128 + 16 j + 4 (lane / 16).
        if constexpr (EPI::kProgram && HasRuns<EPI>::value) {
            // The program over runs: each 16-row block of a 64-column half,
            // staged in f32 in the wave's own 4 KiB as below, is read back
            // eight consecutive columns of one row a lane (lane / 8 picks
            // the row, lane % 8 the eight columns), the same columns in
            // every block of the half, so what the program loads for every
            // row alike (a bias) is loaded once a half, for both halves
            // before the tile's first store: no load then waits behind the
            // tile's stores.  Each run leaves as one 16-byte store.
            constexpr int R = kEpilogueRun;
            static_assert(R == 8, "a lane's eight columns: two staged 16-byte chunks");
            float* staged = reinterpret_cast<float*>(rows_lds + wave * kRegion);
            const int r = lane % 16, g = lane / 16;
            typename EPI::Invariant inv[TN / 4];
            static_for<0, TN / 4>([&](auto x) __attribute__((always_inline)) {
                constexpr int h = decltype(x)::value;
                const uint32_t col = n0 + wn * (BN / WN) + 64 * h + 8 * (lane % 8);
                epi.invariant(inv[h], col < N, col);
            });
            static_for<0, (TN / 4) * TM>([&](auto x) __attribute__((always_inline)) {
                constexpr int h = decltype(x)::value / TM, i = decltype(x)::value % TM;
                static_for<0, 4>([&](auto y) __attribute__((always_inline)) {
                    constexpr int jj = decltype(y)::value;
                    *reinterpret_cast<f32x4*>(staged + r * 64 + (((4 * jj + g) ^ r) * 4)) = acc[i][4 * h + jj];
                });
                const uint32_t col = n0 + wn * (BN / WN) + 64 * h + 8 * (lane % 8);
#pragma unroll
                for (int half = 0; half < 2; half++) {
                    const int rr = 8 * half + lane / 8, c0 = 2 * (lane % 8);
                    const f32x4 lo = *reinterpret_cast<const f32x4*>(staged + rr * 64 + ((c0 ^ rr) * 4));
                    const f32x4 hi = *reinterpret_cast<const f32x4*>(staged + rr * 64 + (((c0 + 1) ^ rr) * 4));
                    const float product[R] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                    const uint32_t row = m0 + wm * (BM / WM) + 16 * i + rr;
                    epi.run(inv[h], row < M && col < N, row, col, N, product);
                }
            });
        } else if constexpr (EPI::kProgram) {
            // As in the persistent kernel, per 64-column half of the wave's
            // tile: one 16-row block of f32 results at a time in the wave's
            // own 4 KiB, handed to the program EPI::kElems rows a lane.
            constexpr int E = EPI::kElems;
            static_assert(16 % E == 0, "whole groups of a staged block's 16 rows");
            float* staged = reinterpret_cast<float*>(rows_lds + wave * kRegion);
            const int r = lane % 16, g = lane / 16;
            // Blocks visited by compile-time index (static_for rather than
            // an unroll hint), so the accumulators are never indexed at run
            // time: a large program made the compiler stop unrolling and
            // keep the whole accumulator array in scratch memory, where the
            // in-place matrix-core steps would read it back unguarded.
            static_for<0, (TN / 4) * TM>([&](auto x) __attribute__((always_inline)) {
                constexpr int h = decltype(x)::value / TM, i = decltype(x)::value % TM;
                static_for<0, 4>([&](auto y) __attribute__((always_inline)) {
                    constexpr int jj = decltype(y)::value;
                    *reinterpret_cast<f32x4*>(staged + r * 64 + (((4 * jj + g) ^ r) * 4)) = acc[i][4 * h + jj];
                });
#pragma unroll
                for (int v0 = 0; v0 < 16; v0 += E) {
                    bool live[E];
                    uint32_t row[E], col[E];
                    float product[E];
#pragma unroll
                    for (int e = 0; e < E; e++) {
                        const int v = v0 + e;
                        product[e] = staged[v * 64 + (((lane / 4) ^ v) * 4) + lane % 4];
                        row[e] = m0 + wm * (BM / WM) + 16 * i + v;
                        col[e] = n0 + wn * (BN / WN) + 64 * h + lane;
                        live[e] = row[e] < M && col[e] < N;
                    }
                    epi.group(live, row, col, N, product);
                }
            });
        } else {
        const bool whole = m0 + BM <= M && n0 + BN <= N;
        const int g = lane / 16;
#pragma unroll
        for (int h = 0; h < TN / 4; h++) {
            const uint32_t row0 = m0 + wm * (BM / WM), col0 = n0 + wn * (BN / WN) + 64 * h;
            const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
                C + static_cast<uint64_t>(row0) * N + col0, 0, 0x7fffffff, kBufferFlags);
            const bool col_ok = col0 + 8 * (lane % 8) < N;
#pragma unroll
            for (int p = 0; p < TM / 2; p++) {
#pragma unroll
                for (int ii = 0; ii < 2; ii++) {
                    const int r = ii * 16 + lane % 16;
#pragma unroll
                    for (int jj = 0; jj < 4; jj++) {
                        const f32x4 v = acc[2 * p + ii][4 * h + jj];
                        const u32x2 out = {pack_pair<O>(v[0], v[1]), pack_pair<O>(v[2], v[3])};
                        const uint32_t at = region + r * 128 + (((2 * jj + g / 2) ^ (r % 8)) * 16) + (g % 2) * 8;
                        asm volatile("ds_write_b64 %0, %1" ::"v"(at), "v"(out) : "memory");
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
                u32x4 v0, v1, v2, v3;
                asm volatile(
                    "ds_read_b128 %0, %4\n\t"
                    "ds_read_b128 %1, %4 offset:1024\n\t"
                    "ds_read_b128 %2, %4 offset:2048\n\t"
                    "ds_read_b128 %3, %4 offset:3072\n\t"
                    "s_waitcnt lgkmcnt(0)"
                    : "=&v"(v0), "=&v"(v1), "=&v"(v2), "=&v"(v3)
                    : "v"(read_at)
                    : "memory");
                const uint32_t first = __builtin_amdgcn_readfirstlane(32 * p * N * sizeof(O));
                const uint32_t eight = __builtin_amdgcn_readfirstlane(8 * N * sizeof(O));
                // Row 32 p + 8 e + lane / 8 of the wave's band.
                const uint32_t row = row0 + 32 * p + lane / 8;
                if (whole || (col_ok && row < M)) __builtin_amdgcn_raw_buffer_store_b128(v0, rc, row_off, first, kStreamStore);
                if (whole || (col_ok && row + 8 < M))
                    __builtin_amdgcn_raw_buffer_store_b128(v1, rc, row_off, first + eight, kStreamStore);
                if (whole || (col_ok && row + 16 < M))
                    __builtin_amdgcn_raw_buffer_store_b128(v2, rc, row_off, first + 2 * eight, kStreamStore);
                if (whole || (col_ok && row + 24 < M))
                    __builtin_amdgcn_raw_buffer_store_b128(v3, rc, row_off, first + 3 * eight, kStreamStore);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        }
        tile += gridDim.x;
        if (tile >= tiles) break;
        tile_of(tile, tiles_m, tiles_n, tm, tn);
        m0 = tm * BM;
        n0 = tn * BN;
    }
    // No direct load may still be writing LDS when the block ends.
    __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0(0));
}

}  // namespace tc
