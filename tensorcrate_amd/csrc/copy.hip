// Strided copies: `Backend::strided_copy`, `assemble` and `strided_write`
// (tensors/backend.rs:141-173), and `Kernels::transpose` (kernels.rs:987).
//
// A copy moves bits, so every kernel is instantiated by element width
// (1, 2, 4, 8 or 16 bytes) rather than by type.  The host coalesces the joint
// source/target layout (layout.rs:419-449) and picks one of three kernels:
//
//  - rows: both sides step by one along the innermost axis.  Each run is
//    copied with 16-byte vector accesses when both runs are 16-byte aligned,
//    which covers contiguous copies, slices and concatenation.
//  - tile: one side is contiguous along an axis the other is not (a permute
//    such as a transpose).  A tile is read along the source's contiguous
//    axis, held in LDS, and written along the target's, so both HBM streams
//    are coalesced: 128 x 64 four-byte elements moved 16 bytes a lane, in
//    diagonal block order, or 64 x 64 of any other width.
//  - gather: anything else (broadcasts along inner axes, general strides),
//    one element per thread with the coordinates recovered by multiply-shift
//    division.
//
// Indices are 32-bit whenever every offset a layout reaches fits, which is
// every layout under 2^32 elements; the 64-bit instantiation covers the rest
// of a 288 GB device.

#include <string.h>

#include "common.hpp"

namespace tc {
namespace {

template <int W>
struct Word;
template <> struct Word<1> { using type = uint8_t; };
template <> struct Word<2> { using type = uint16_t; };
template <> struct Word<4> { using type = uint32_t; };
template <> struct Word<8> { using type = uint64_t; };
template <> struct Word<16> { using type = uint4; };

// A coalesced two-operand layout in index type I.
template <typename I>
struct Layout2 {
    int rank;
    I shape[kMaxRank];
    Div<I> div[kMaxRank];
    I src[kMaxRank];
    I dst[kMaxRank];
};

template <typename I>
Layout2<I> make_layout(const Walk<2>& walk) {
    Layout2<I> layout{};
    layout.rank = walk.rank;
    for (int k = 0; k < walk.rank; k++) {
        layout.shape[k] = static_cast<I>(walk.shape[k]);
        layout.div[k].set(walk.shape[k]);
        layout.src[k] = static_cast<I>(walk.strides[0][k]);
        layout.dst[k] = static_cast<I>(walk.strides[1][k]);
    }
    return layout;
}

// Element `index` of the walk over axes [0, last): its source and target
// offsets.
template <typename I>
__device__ __forceinline__ void locate(const Layout2<I>& layout, int last, I index, I& src, I& dst) {
    src = 0;
    dst = 0;
    for (int k = last - 1; k > 0; k--) {
        I q = layout.div[k].div(index);
        I c = index - q * layout.shape[k];
        src += c * layout.src[k];
        dst += c * layout.dst[k];
        index = q;
    }
    if (last > 0) {
        src += index * layout.src[0];
        dst += index * layout.dst[0];
    }
}

template <typename T, typename I>
__global__ void __launch_bounds__(256) gather_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                                     Layout2<I> layout, I count) {
    I stride = static_cast<I>(gridDim.x) * blockDim.x;
    for (I i = static_cast<I>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride) {
        I from, to;
        locate(layout, layout.rank, i, from, to);
        dst[to] = src[from];
    }
}

// Rows of `run` words each, a word being one element or 16 bytes of them.
// `run_div` divides a flat (row, word) index by the words per row.  One word
// a thread, over a grid that covers them; NT (16-byte words only) marks a
// copy that streams past the Infinity Cache: its loads are non-temporal, its
// stores plain (config 3's slice 6.22 -> 6.48 TB/s and concat 6.18 -> 6.50
// against non-temporal stores).
template <typename T, bool NT, typename I, int U = 1>
__global__ void __launch_bounds__(256) rows_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                                   Layout2<I> layout, Div<I> run_div, I run, I total) {
    // U words a thread, a grid apart, all loads issued before any store; one
    // round normally, the loop (64-bit, so it cannot wrap) covering work past
    // what one dispatch holds.
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t base = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; base < total;
         base += stride * U) {
        T value[U];
        I to[U];
#pragma unroll
        for (int k = 0; k < U; k++) {
            const uint64_t item = base + k * stride;
            if (item < total) {
                const I i = static_cast<I>(item);
                I row = run_div.div(i);
                I word = i - row * run;
                I from;
                locate(layout, layout.rank - 1, row, from, to[k]);
                to[k] += word;
                if constexpr (NT) {
                    value[k] = load_word<true>(src + from + word);
                } else {
                    value[k] = src[from + word];
                }
            }
        }
#pragma unroll
        for (int k = 0; k < U; k++) {
            if (base + k * stride < total) {
                dst[to[k]] = value[k];
            }
        }
    }
}

constexpr int kTile = 64;
constexpr int kTileRows = 4;  // 256 threads: 64 columns x 4 rows per pass

// A batched tile transpose.  Axis `a` is the one the source steps along by
// one and `b` the one the target does; the tile is read with lanes along `a`
// and written with lanes along `b`.  Every other axis is a batch axis.
template <typename I>
struct TileLayout {
    I extent_a, extent_b;
    I src_b, dst_a;  // the strides that are not one
    Div<I> tiles_a_div, tiles_b_div;
    I tiles_a, tiles_b;
    int batch_rank;
    I batch_shape[kMaxRank];
    Div<I> batch_div[kMaxRank];
    I batch_src[kMaxRank];
    I batch_dst[kMaxRank];
};

template <typename T, typename I>
__global__ void __launch_bounds__(256) tile_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                                   TileLayout<I> t, I blocks) {
    __shared__ T tile[kTile][kTile + 1];
    const int tx = threadIdx.x % kTile;
    const int ty = threadIdx.x / kTile;
    for (I block = blockIdx.x; block < blocks; block += gridDim.x) {
        I rest = t.tiles_a_div.div(block);
        I tile_a = block - rest * t.tiles_a;
        I batch = t.tiles_b_div.div(rest);
        I tile_b = rest - batch * t.tiles_b;
        I from = 0, to = 0;
        for (int k = t.batch_rank - 1; k > 0; k--) {
            I q = t.batch_div[k].div(batch);
            I c = batch - q * t.batch_shape[k];
            from += c * t.batch_src[k];
            to += c * t.batch_dst[k];
            batch = q;
        }
        if (t.batch_rank > 0) {
            from += batch * t.batch_src[0];
            to += batch * t.batch_dst[0];
        }
        const I a0 = tile_a * kTile;
        const I b0 = tile_b * kTile;
        // Read: lanes walk `a`, where the source is contiguous.
        const I a = a0 + tx;
        if (a < t.extent_a) {
#pragma unroll
            for (int r = 0; r < kTile; r += kTileRows) {
                const I b = b0 + ty + r;
                if (b < t.extent_b) tile[ty + r][tx] = src[from + a + b * t.src_b];
            }
        }
        __syncthreads();
        // Write: lanes walk `b`, where the target is contiguous.
        const I b = b0 + tx;
        if (b < t.extent_b) {
#pragma unroll
            for (int r = 0; r < kTile; r += kTileRows) {
                const I aa = a0 + ty + r;
                if (aa < t.extent_a) dst[to + b + aa * t.dst_a] = tile[tx][ty + r];
            }
        }
        __syncthreads();
    }
}

// The same transpose for 4-byte elements moving 16 bytes a lane on both
// sides, over TA x TB tiles (TA along `a`, TB along `b`).  A lane reads four
// elements along `a` and writes them to LDS as one 16-byte word; after the
// barrier it reads a 4 x 4 block (four 16-byte words from four consecutive
// `b` rows), transposes it in registers and writes four 16-byte words along
// `b`.  So the LDS sees a quarter of the instructions a word-at-a-time
// exchange would, and no padding: the 16-byte chunks of tile row r sit at
// chunk ^ ((r / 4) % 16), which puts the 16 rows a quarter-wave reads on
// distinct bank groups in the second phase and permutes a row's chunks in
// the first (the period is the smaller of a row's chunks and TB / 4).
// Needs every extent, offset and stride that steps along a vector to be a
// multiple of 4, which the host checks.  NT marks a transpose that streams
// past the Infinity Cache: its loads are non-temporal, its stores plain
// (config-3 permute of [256, 512, 512] f32: 5.99 TB/s with both streamed,
// 6.50 with plain stores).
template <typename I, bool NT, int TA, int TB>
__global__ void __launch_bounds__(256) tile4_kernel(const uint32_t* __restrict__ src, uint32_t* __restrict__ dst,
                                                    TileLayout<I> t, I tiles) {
    constexpr int kReadQuads = TA / 4, kReadRows = 256 / kReadQuads;  // first phase: lanes along `a`
    constexpr int kBlocksB = TB / 4;                                   // second phase: 4 x 4 blocks along `b`
    constexpr int kBlockRows = 256 / kBlocksB;                         // ... and along `a`, per pass
    // The swizzle's period: at most a row's chunks, so it stays within a row.
    constexpr int kSwizzle = TA / 4 < TB / 4 ? TA / 4 : TB / 4;
    static_assert((kSwizzle & (kSwizzle - 1)) == 0, "the swizzle stays within a row");
    __shared__ __attribute__((aligned(16))) uint32_t tile[TB][TA];
    auto chunk_at = [](int r, int chunk) { return (chunk ^ ((r / 4) % kSwizzle)) * 4; };
    // Where tile `block` starts in the source (`from`, plus a0 along `a` and
    // b0 along `b`) and in the target (`to`).
    struct Place {
        I from, to, a0, b0;
    };
    auto place_of = [&](I block) {
        I rest = t.tiles_a_div.div(block);
        const I tile_a = block - rest * t.tiles_a;
        I batch = t.tiles_b_div.div(rest);
        I tile_b = rest - batch * t.tiles_b;
        // Diagonal order: the blocks running together (neighbouring tile_a)
        // take different tile_b, so their writes land in different columns
        // rather than all in the same few (long target rows would otherwise
        // put them on the same HBM channels: an 8192 x 8192 transpose runs at
        // 3.9 TB/s without this, 5.8 with it).
        tile_b += tile_a - t.tiles_b_div.div(tile_a) * t.tiles_b;
        if (tile_b >= t.tiles_b) tile_b -= t.tiles_b;
        Place p{0, 0, tile_a * TA, tile_b * TB};
        for (int k = t.batch_rank - 1; k > 0; k--) {
            I q = t.batch_div[k].div(batch);
            I c = batch - q * t.batch_shape[k];
            p.from += c * t.batch_src[k];
            p.to += c * t.batch_dst[k];
            batch = q;
        }
        if (t.batch_rank > 0) {
            p.from += batch * t.batch_src[0];
            p.to += batch * t.batch_dst[0];
        }
        return p;
    };
    const int quad = threadIdx.x % kReadQuads, row = threadIdx.x / kReadQuads;
    uint4 v[TB / kReadRows];
    auto load = [&](const Place& p) {
        const I a = p.a0 + quad * 4;
#pragma unroll
        for (int pass = 0; pass < TB / kReadRows; pass++) {
            const I b = p.b0 + row + pass * kReadRows;
            if (a < t.extent_a && b < t.extent_b) v[pass] = load_word<NT>(src + p.from + a + b * t.src_b);
        }
    };
    // Each block walks every gridDim.x-th tile; the next tile's loads are
    // in flight while this one's stores go out.
    I block = blockIdx.x;
    Place here = place_of(block);
    load(here);
    for (;;) {
#pragma unroll
        for (int pass = 0; pass < TB / kReadRows; pass++) {
            const int r = row + pass * kReadRows;
            *reinterpret_cast<uint4*>(&tile[r][chunk_at(r, quad)]) = v[pass];
        }
        __syncthreads();
        const I next = block + gridDim.x;
        Place there{};
        if (next < tiles) {
            there = place_of(next);
            load(there);
        }
        const int cb = threadIdx.x % kBlocksB;
        const I b = here.b0 + cb * 4;
#pragma unroll
        for (int pass = 0; pass < TA / 4 / kBlockRows; pass++) {
            const int ca = threadIdx.x / kBlocksB + pass * kBlockRows;
            uint4 q[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                q[r] = *reinterpret_cast<const uint4*>(&tile[cb * 4 + r][chunk_at(cb * 4 + r, ca)]);
            }
            const I aa = here.a0 + ca * 4;
            uint32_t* out = dst + here.to + b + aa * t.dst_a;
            if (b < t.extent_b) {
                if (aa < t.extent_a) store_word<false>(out, uint4{q[0].x, q[1].x, q[2].x, q[3].x});
                if (aa + 1 < t.extent_a) store_word<false>(out + t.dst_a, uint4{q[0].y, q[1].y, q[2].y, q[3].y});
                if (aa + 2 < t.extent_a) store_word<false>(out + 2 * t.dst_a, uint4{q[0].z, q[1].z, q[2].z, q[3].z});
                if (aa + 3 < t.extent_a) store_word<false>(out + 3 * t.dst_a, uint4{q[0].w, q[1].w, q[2].w, q[3].w});
            }
        }
        if (next >= tiles) break;
        __syncthreads();  // every wave has read the tile before the next is written
        block = next;
        here = there;
    }
}

bool fits32(const Walk<2>& walk, uint64_t count) {
    if (count > UINT32_MAX) return false;
    for (int n = 0; n < 2; n++) {
        uint64_t end = 0;
        if (!reach(walk.rank, walk.shape, 0, walk.strides[n], &end) || end > UINT32_MAX) return false;
    }
    return true;
}

template <typename T, typename I>
int launch_copy(const T* src, T* dst, const Walk<2>& walk, uint64_t count, bool stream, hipStream_t s) {
    const int rank = walk.rank;
    if (rank == 0) {
        Layout2<I> layout{};
        gather_kernel<T, I><<<1, 64, 0, s>>>(src, dst, layout, I{1});
        return check_launch("strided copy");
    }
    const uint64_t inner_src = walk.strides[0][rank - 1];
    const uint64_t inner_dst = walk.strides[1][rank - 1];
    if (inner_src == 1 && inner_dst == 1) {
        Layout2<I> layout = make_layout<I>(walk);
        const uint64_t run = walk.shape[rank - 1];
        const uint64_t rows = count / run;
        // 16-byte words when every run starts 16-byte aligned.
        bool wide = sizeof(T) < 16 && (run * sizeof(T)) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(src) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(dst) % 16 == 0;
        for (int k = 0; wide && k < rank - 1; k++) {
            wide = (walk.strides[0][k] * sizeof(T)) % 16 == 0 && (walk.strides[1][k] * sizeof(T)) % 16 == 0;
        }
        if (wide) {
            const uint64_t per = 16 / sizeof(T);
            Layout2<I> words = layout;
            for (int k = 0; k < rank - 1; k++) {
                words.src[k] = static_cast<I>(walk.strides[0][k] / per);
                words.dst[k] = static_cast<I>(walk.strides[1][k] / per);
            }
            const uint64_t run_words = run / per;
            Div<I> run_div;
            run_div.set(run_words);
            const uint64_t total = rows * run_words;
            if (stream) {
                rows_kernel<uint4, true, I><<<blocks_for(total, 1), 256, 0, s>>>(
                    reinterpret_cast<const uint4*>(src), reinterpret_cast<uint4*>(dst), words, run_div,
                    static_cast<I>(run_words), static_cast<I>(total));
            } else {
                rows_kernel<uint4, false, I><<<blocks_for(total, 1), 256, 0, s>>>(
                    reinterpret_cast<const uint4*>(src), reinterpret_cast<uint4*>(dst), words, run_div,
                    static_cast<I>(run_words), static_cast<I>(total));
            }
        } else {
            Div<I> run_div;
            run_div.set(run);
            rows_kernel<T, false, I><<<blocks_for(count, 1), 256, 0, s>>>(
                src, dst, layout, run_div, static_cast<I>(run), static_cast<I>(count));
        }
        return check_launch("strided copy");
    }
    // A permute: find the axis the source is contiguous along and the one
    // the target is, distinct and both long enough to fill a tile.
    int axis_a = -1, axis_b = -1;
    for (int k = 0; k < rank; k++) {
        if (walk.strides[0][k] == 1 && axis_a < 0) axis_a = k;
        if (walk.strides[1][k] == 1 && axis_b < 0) axis_b = k;
    }
    if (sizeof(T) <= 8 && axis_a >= 0 && axis_b >= 0 && axis_a != axis_b &&
        walk.shape[axis_a] >= 16 && walk.shape[axis_b] >= 16) {
        TileLayout<I> t{};
        t.extent_a = static_cast<I>(walk.shape[axis_a]);
        t.extent_b = static_cast<I>(walk.shape[axis_b]);
        t.src_b = static_cast<I>(walk.strides[0][axis_b]);
        t.dst_a = static_cast<I>(walk.strides[1][axis_a]);
        uint64_t batches = 1;
        for (int k = 0; k < rank; k++) {
            if (k == axis_a || k == axis_b) continue;
            t.batch_shape[t.batch_rank] = static_cast<I>(walk.shape[k]);
            t.batch_div[t.batch_rank].set(walk.shape[k]);
            t.batch_src[t.batch_rank] = static_cast<I>(walk.strides[0][k]);
            t.batch_dst[t.batch_rank] = static_cast<I>(walk.strides[1][k]);
            t.batch_rank++;
            batches *= walk.shape[k];
        }
        // Tiles of `ta` x `tb`; the number of blocks that covers them.
        auto tiled = [&](uint64_t ta, uint64_t tb) {
            const uint64_t tiles_a = (walk.shape[axis_a] + ta - 1) / ta;
            const uint64_t tiles_b = (walk.shape[axis_b] + tb - 1) / tb;
            t.tiles_a = static_cast<I>(tiles_a);
            t.tiles_b = static_cast<I>(tiles_b);
            t.tiles_a_div.set(tiles_a);
            t.tiles_b_div.set(tiles_b);
            return tiles_a * tiles_b * batches;
        };
        // Four-byte elements whose rows start on 16-byte boundaries move 16
        // bytes a lane; a block walks several tiles.  Streaming transposes
        // take 64 x 128 tiles (256-byte reads and 512-byte writes per row):
        // measured on MI355X over ten shapes from 2048^2 to [1024, 256, 256],
        // streaming, with inputs and outputs both cold, they averaged 5.55
        // TB/s against 5.46 for 128 x 64 and 5.49 for 256 x 32 (the config-3
        // permute 5.89 against 5.69).  Streaming both sides beat plain
        // accesses on every shape there, but writing into a target that is
        // still in the Infinity Cache it loses (a 4096^2 transpose into one
        // reused target: 4.86 against 5.18 TB/s), and streamed loads with
        // plain stores beat both (the kernel's stores are now always plain);
        // as for every copy, only traffic past that cache streams.  Smaller
        // transposes take 64 x 64 tiles, twice the blocks for the same work:
        // 4096^2 5.22 -> 5.55 TB/s, 2048^2 4.05 -> 4.29, 2048 x 8192 5.55 ->
        // 5.42; 32 x 128 and 128 x 64 measured slower than both.
        const bool stream_tiles = stream;
        const int ta = 64, tb = stream_tiles ? 128 : 64;
        uint64_t blocks = tiled(ta, tb);
        bool wide = sizeof(T) == 4 && blocks <= UINT32_MAX && walk.shape[axis_a] % 4 == 0 &&
                    walk.shape[axis_b] % 4 == 0 && walk.strides[0][axis_b] % 4 == 0 &&
                    walk.strides[1][axis_a] % 4 == 0 && aligned16(src) && aligned16(dst);
        for (int k = 0; wide && k < t.batch_rank; k++) wide = t.batch_src[k] % 4 == 0 && t.batch_dst[k] % 4 == 0;
        if (wide) {
            const uint32_t* s32 = reinterpret_cast<const uint32_t*>(src);
            uint32_t* d32 = reinterpret_cast<uint32_t*>(dst);
            // At most four blocks a CU for the 64 x 128 tiles (32 KiB of LDS
            // each), eight for 64 x 64 (16 KiB), each block walking the same
            // number of tiles, so no second round runs part-empty.  Four
            // rather than the five that fit: 8192^2 transpose 6.44 -> 6.70
            // TB/s, config-3 permute 6.52 -> 6.67 (8192 tiles: 1024 blocks of
            // eight, four on every CU, rather than 1171 of seven).
            const uint64_t resident = (stream_tiles ? 4 : 8) * static_cast<uint64_t>(compute_units());
            const uint64_t per_block = (blocks + resident - 1) / resident;
            const uint32_t grid = static_cast<uint32_t>((blocks + per_block - 1) / per_block);
            if (stream_tiles) {
                tile4_kernel<I, true, 64, 128><<<grid, 256, 0, s>>>(s32, d32, t, static_cast<I>(blocks));
            } else {
                tile4_kernel<I, false, 64, 64><<<grid, 256, 0, s>>>(s32, d32, t, static_cast<I>(blocks));
            }
            return check_launch("strided copy");
        }
        blocks = tiled(kTile, kTile);
        tile_kernel<T, I><<<grid_for(blocks, 1, 64), 256, 0, s>>>(src, dst, t, static_cast<I>(blocks));
        return check_launch("strided copy");
    }
    Layout2<I> layout = make_layout<I>(walk);
    gather_kernel<T, I><<<grid_for(count, 256 * 4), 256, 0, s>>>(src, dst, layout, static_cast<I>(count));
    return check_launch("strided copy");
}

template <typename T>
int copy_walk(const void* src, void* dst, const Walk<2>& walk, uint64_t count, bool stream, hipStream_t s) {
    if (count == 0) return TC_OK;
    const T* from = static_cast<const T*>(src) + walk.offsets[0];
    T* to = static_cast<T*>(dst) + walk.offsets[1];
    if (fits32(walk, count)) return launch_copy<T, uint32_t>(from, to, walk, count, stream, s);
    return launch_copy<T, uint64_t>(from, to, walk, count, stream, s);
}

// `traffic` is the bytes the whole operation moves: one as large as the
// Infinity Cache streams past it, however it is split into launches.
int copy_by_width(uint32_t width, const void* src, void* dst, const Walk<2>& walk, uint64_t count,
                  uint64_t traffic, const char* operation) {
    TC_STREAM(s);
    const bool stream = traffic >= kStreamBytes;
    switch (width) {
        case 1: return copy_walk<Word<1>::type>(src, dst, walk, count, stream, s);
        case 2: return copy_walk<Word<2>::type>(src, dst, walk, count, stream, s);
        case 4: return copy_walk<Word<4>::type>(src, dst, walk, count, stream, s);
        case 8: return copy_walk<Word<8>::type>(src, dst, walk, count, stream, s);
        case 16: return copy_walk<Word<16>::type>(src, dst, walk, count, stream, s);
        default:
            return fail(TC_UNSUPPORTED, std::string(operation) + ": no kernel for " +
                                            std::to_string(width) + "-byte elements");
    }
}

// One region: `shape` from `source` at `from` to `target` at `to`, as part
// of an operation moving `traffic` bytes (0: just this region).
int write_region(uint32_t width, const void* source, uint64_t source_len, void* target,
                 uint64_t target_len, uint32_t rank, const uint64_t* shape, const tc_strided& from,
                 const tc_strided& to, uint64_t traffic, const char* operation) {
    uint64_t count = 0;
    int status = check_strided(source_len, rank, shape, from.offset, from.strides,
                               (std::string(operation) + " source").c_str(), &count);
    if (status != TC_OK) return status;
    status = check_strided(target_len, rank, shape, to.offset, to.strides,
                           (std::string(operation) + " target").c_str(), &count);
    if (status != TC_OK) return status;
    const uint64_t* strides[2] = {from.strides, to.strides};
    const uint64_t offsets[2] = {from.offset, to.offset};
    Walk<2> walk = coalesce<2>(rank, shape, strides, offsets);
    if (traffic == 0) traffic = 2 * count * width;
    return copy_by_width(width, source, target, walk, count, traffic, operation);
}

}  // namespace
}  // namespace tc

using namespace tc;

extern "C" {

int tc_strided_copy(uint32_t width, const void* src, uint64_t src_len, uint32_t rank,
                    const uint64_t* shape, const tc_strided* from, void* dst) {
    if (rank > static_cast<uint32_t>(kMaxRank)) {
        return fail(TC_INVALID, "strided copy: shape " + shape_text(shape, rank) + " has more than " +
                                    std::to_string(kMaxRank) + " axes");
    }
    uint64_t count = 0;
    int status = check_strided(src_len, rank, shape, from->offset, from->strides, "strided copy", &count);
    if (status != TC_OK) return status;
    if (count != 0 && any_null({src, dst})) return null_operand("strided copy");
    // The target is the row-major layout of `shape`.
    tc_strided to{};
    uint64_t step = 1;
    for (int k = static_cast<int>(rank) - 1; k >= 0; k--) {
        to.strides[k] = step;
        step *= shape[k];
    }
    const uint64_t* strides[2] = {from->strides, to.strides};
    const uint64_t offsets[2] = {from->offset, 0};
    Walk<2> walk = coalesce<2>(rank, shape, strides, offsets);
    return copy_by_width(width, src, dst, walk, count, 2 * count * width, "strided copy");
}

int tc_assemble(uint32_t width, void* dst, uint64_t len, const tc_region* regions, uint32_t count) {
    // Every region is checked before anything is queued, so a bad one
    // leaves the target untouched.
    uint64_t traffic = 0;
    for (uint32_t r = 0; r < count; r++) {
        const tc_region& region = regions[r];
        uint64_t elements = 0;
        int status = check_strided(region.source_len, region.rank, region.shape, region.from.offset,
                                   region.from.strides, "assemble", &elements);
        if (status != TC_OK) return status;
        status = check_strided(len, region.rank, region.shape, region.to.offset, region.to.strides,
                               "assemble", &elements);
        if (status != TC_OK) return status;
        if (elements != 0 && any_null({region.source, dst})) return null_operand("assemble");
        traffic += 2 * elements * width;
    }
    for (uint32_t r = 0; r < count; r++) {
        const tc_region& region = regions[r];
        int status = write_region(width, region.source, region.source_len, dst, len, region.rank,
                                  region.shape, region.from, region.to, traffic, "assemble");
        if (status != TC_OK) return status;
    }
    return TC_OK;
}

int tc_strided_write(uint32_t width, void* target, uint64_t target_len, const tc_region* region) {
    return write_region(width, region->source, region->source_len, target, target_len, region->rank,
                        region->shape, region->from, region->to, 0, "strided write");
}

int tc_transpose(uint32_t width, uint64_t rows, uint64_t cols, const void* src, void* dst) {
    // Output (c, r) is input (r, c): a copy of the shape [cols, rows] read
    // with strides [1, cols].
    uint64_t shape[2] = {cols, rows};
    tc_strided from{};
    from.strides[0] = 1;
    from.strides[1] = cols;
    uint64_t len = rows * cols;
    return tc_strided_copy(width, src, len, 2, shape, &from, dst);
}

}  // extern "C"
