// `Kernels::vector_prefix_sum` and `vector_sort` (tensors/kernels.rs:870-873).
//
// The prefix sum is inclusive, accumulated in f32 and rounded to the element
// type per output (compact.rs:209-221; vector.rs:578-589).  It runs as three
// deterministic passes, so a given length always adds in the same order:
//  1. each block of 4096 elements sums its tile (a fixed tree);
//  2. one block scans the tile sums into each tile's offset, 256 at a time
//     with a carry;
//  3. each block scans its tile from LDS, each thread 16 consecutive
//     elements, the threads' totals scanned across the block, and adds the
//     tile's offset.
// The order differs from the host's left-to-right running sum, so results
// agree within the rounding a sum of that many terms can carry.
//
// The sort is exact: f32, f16 and bf16 bit patterns are mapped to unsigned
// keys whose order is IEEE totalOrder (the `total_cmp` order `SortOrder`
// compares with, kernels.rs:252-270: -NaN < -inf < ... < -0 < +0 < ... <
// +inf < +NaN), complemented for a descending sort, put in order by a
// least-significant-digit radix sort of 8-bit digits (four passes for f32,
// two for f16 and bf16), and mapped back.  Each pass counts every 4096-key
// tile's digits, scans the counts digit-major (so digit d of tile t lands
// after every smaller digit and after digit d of every earlier tile), and
// scatters each tile's keys to those offsets in their input order, which
// keeps the sort stable from pass to pass.  Within a tile a key's place
// among the keys of its digit comes from wave ballots on the digit's bits
// (the lanes holding the same digit, counted below this lane) and from the
// counts of the waves and rounds before it.

#include "common.hpp"

namespace tc {
namespace {

constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;
constexpr int kScanTile = kScanThreads * kScanItems;

// A scan of one value a thread across the block (Hillis-Steele in LDS: a
// fixed order).  Returns the inclusive sum; `exclusive` receives the sum of
// the threads before this one, read from the scan itself (thread t - 1's
// inclusive sum, zero for thread 0), never as the inclusive sum minus the
// value: a later infinity, NaN or very large element then cannot reach the
// sums before it.  `total` receives the block's sum.
__device__ float block_scan(float v, float* lds, float* exclusive, float* total) {
    const int t = threadIdx.x;
    lds[t] = v;
    __syncthreads();
    for (int offset = 1; offset < kScanThreads; offset <<= 1) {
        const float add = t >= offset ? lds[t - offset] : 0.0f;
        __syncthreads();
        if (t >= offset) lds[t] = lds[t] + add;
        __syncthreads();
    }
    const float out = lds[t];
    *exclusive = t > 0 ? lds[t - 1] : 0.0f;
    *total = lds[kScanThreads - 1];
    __syncthreads();
    return out;
}

template <typename S>
__global__ void __launch_bounds__(kScanThreads) tile_sums_kernel(const S* __restrict__ a, uint64_t n,
                                                                 float* __restrict__ sums) {
    __shared__ float lds[kScanThreads];
    const uint64_t base = static_cast<uint64_t>(blockIdx.x) * kScanTile;
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < kScanItems; k++) {
        const uint64_t i = base + k * kScanThreads + threadIdx.x;
        if (i < n) s = s + Elem<S>::widen(a[i]);
    }
    float before, total;
    block_scan(s, lds, &before, &total);
    if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

// Exclusive scan of the tile sums in place, 256 at a time with a carry.
__global__ void __launch_bounds__(kScanThreads) scan_sums_kernel(float* __restrict__ sums, uint32_t count) {
    __shared__ float lds[kScanThreads];
    float carry = 0.0f;
    for (uint32_t first = 0; first < count; first += kScanThreads) {
        const uint32_t i = first + threadIdx.x;
        const float v = i < count ? sums[i] : 0.0f;
        float before, total;
        block_scan(v, lds, &before, &total);
        if (i < count) sums[i] = carry + before;
        carry = carry + total;
    }
}

template <typename S>
__global__ void __launch_bounds__(kScanThreads) tile_scan_kernel(const S* __restrict__ a, S* __restrict__ out,
                                                                 uint64_t n, const float* __restrict__ offsets) {
    using E = Elem<S>;
    __shared__ float tile[kScanTile + kScanTile / 32];  // one pad word per 32 against bank conflicts
    __shared__ float lds[kScanThreads];
    auto slot = [](int i) { return i + i / 32; };
    const uint64_t base = static_cast<uint64_t>(blockIdx.x) * kScanTile;
#pragma unroll
    for (int k = 0; k < kScanItems; k++) {
        const int i = k * kScanThreads + threadIdx.x;
        tile[slot(i)] = base + i < n ? E::widen(a[base + i]) : 0.0f;
    }
    __syncthreads();
    float run[kScanItems];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < kScanItems; k++) {
        s = s + tile[slot(threadIdx.x * kScanItems + k)];
        run[k] = s;
    }
    float before, total;
    block_scan(s, lds, &before, &total);
    const float offset = offsets[blockIdx.x] + before;
#pragma unroll
    for (int k = 0; k < kScanItems; k++) tile[slot(threadIdx.x * kScanItems + k)] = offset + run[k];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kScanItems; k++) {
        const int i = k * kScanThreads + threadIdx.x;
        if (base + i < n) out[base + i] = E::narrow(tile[slot(i)]);
    }
}

template <typename S>
int prefix_sum_typed(const void* a, void* out, uint64_t n) {
    TC_STREAM(s);
    if (n == 0) return TC_OK;
    const uint64_t tiles = (n + kScanTile - 1) / kScanTile;
    if (tiles > 0xffffffu) return fail(TC_UNSUPPORTED, "prefix_sum: more than 2^24 tiles");
    void* scratch = nullptr;
    int status = tc_alloc(tiles * sizeof(float), &scratch);
    if (status != TC_OK) return status;
    float* sums = static_cast<float*>(scratch);
    const S* in = static_cast<const S*>(a);
    tile_sums_kernel<S><<<static_cast<uint32_t>(tiles), kScanThreads, 0, s>>>(in, n, sums);
    status = check_launch("prefix_sum");
    if (status == TC_OK) {
        scan_sums_kernel<<<1, kScanThreads, 0, s>>>(sums, static_cast<uint32_t>(tiles));
        status = check_launch("prefix_sum");
    }
    if (status == TC_OK) {
        tile_scan_kernel<S><<<static_cast<uint32_t>(tiles), kScanThreads, 0, s>>>(in, static_cast<S*>(out), n, sums);
        status = check_launch("prefix_sum");
    }
    tc_free(scratch);
    return status;
}

constexpr int kRadixBits = 8;
constexpr int kRadix = 1 << kRadixBits;
constexpr int kSortThreads = 256;  // one thread a digit in the block steps
constexpr int kSortItems = 16;
constexpr int kSortTile = kSortThreads * kSortItems;

template <typename K>
__device__ __forceinline__ uint32_t digit_of(K key, uint32_t shift) {
    return (static_cast<uint32_t>(key) >> shift) & (kRadix - 1);
}

// Digit counts of each tile, digit-major: counts[d * tiles + tile].
template <typename K>
__global__ void __launch_bounds__(kSortThreads) digit_counts_kernel(const K* __restrict__ keys, uint64_t n,
                                                                    uint32_t shift, uint32_t* __restrict__ counts,
                                                                    uint32_t tiles) {
    __shared__ uint32_t bins[kRadix];
    bins[threadIdx.x] = 0;
    __syncthreads();
    const uint64_t base = static_cast<uint64_t>(blockIdx.x) * kSortTile;
#pragma unroll 4
    for (int r = 0; r < kSortItems; r++) {
        const uint64_t i = base + r * kSortThreads + threadIdx.x;
        if (i < n) atomicAdd(&bins[digit_of(keys[i], shift)], 1u);
    }
    __syncthreads();
    counts[static_cast<uint64_t>(threadIdx.x) * tiles + blockIdx.x] = bins[threadIdx.x];
}

// An exclusive scan of `count` u32 in place, in three passes over tiles of
// 4096 (integer sums, so any order gives the same values).
__global__ void __launch_bounds__(kScanThreads) count_sums_kernel(const uint32_t* __restrict__ v, uint64_t count,
                                                                  uint32_t* __restrict__ sums) {
    __shared__ uint32_t lds[kScanThreads];
    const uint64_t base = static_cast<uint64_t>(blockIdx.x) * kScanTile;
    uint32_t s = 0;
    for (int k = 0; k < kScanItems; k++) {
        const uint64_t i = base + k * kScanThreads + threadIdx.x;
        if (i < count) s += v[i];
    }
    lds[threadIdx.x] = s;
    __syncthreads();
    for (int half = kScanThreads / 2; half > 0; half >>= 1) {
        if (threadIdx.x < half) lds[threadIdx.x] += lds[threadIdx.x + half];
        __syncthreads();
    }
    if (threadIdx.x == 0) sums[blockIdx.x] = lds[0];
}

__device__ uint32_t block_exclusive_u32(uint32_t v, uint32_t* lds, uint32_t* total) {
    const int t = threadIdx.x;
    lds[t] = v;
    __syncthreads();
    for (int offset = 1; offset < kScanThreads; offset <<= 1) {
        const uint32_t add = t >= offset ? lds[t - offset] : 0u;
        __syncthreads();
        lds[t] += add;
        __syncthreads();
    }
    const uint32_t inclusive = lds[t];
    *total = lds[kScanThreads - 1];
    __syncthreads();
    return inclusive - v;
}

__global__ void __launch_bounds__(kScanThreads) scan_count_sums_kernel(uint32_t* __restrict__ sums, uint32_t count) {
    __shared__ uint32_t lds[kScanThreads];
    uint32_t carry = 0;
    for (uint32_t first = 0; first < count; first += kScanThreads) {
        const uint32_t i = first + threadIdx.x;
        uint32_t total;
        const uint32_t before = block_exclusive_u32(i < count ? sums[i] : 0u, lds, &total);
        if (i < count) sums[i] = carry + before;
        carry += total;
    }
}

__global__ void __launch_bounds__(kScanThreads) scan_counts_kernel(uint32_t* __restrict__ v, uint64_t count,
                                                                   const uint32_t* __restrict__ sums) {
    __shared__ uint32_t lds[kScanThreads];
    const uint64_t base = static_cast<uint64_t>(blockIdx.x) * kScanTile;
    uint32_t run[kScanItems];
    uint32_t s = 0;
    for (int k = 0; k < kScanItems; k++) {
        const uint64_t i = base + threadIdx.x * kScanItems + k;
        run[k] = s;
        s += i < count ? v[i] : 0u;
    }
    uint32_t total;
    const uint32_t before = block_exclusive_u32(s, lds, &total) + sums[blockIdx.x];
    for (int k = 0; k < kScanItems; k++) {
        const uint64_t i = base + threadIdx.x * kScanItems + k;
        if (i < count) v[i] = before + run[k];
    }
}

// One pass: each tile's keys to their digit's place, in input order.  Round
// r takes keys base + 256 r + thread, so (round, wave, lane) is input order.
template <typename K>
__global__ void __launch_bounds__(kSortThreads) scatter_kernel(const K* __restrict__ in, K* __restrict__ out,
                                                               uint64_t n, uint32_t shift,
                                                               const uint32_t* __restrict__ offsets, uint32_t tiles) {
    constexpr int kWaves = kSortThreads / 64;
    __shared__ uint32_t placed[kRadix];            // keys of each digit placed so far
    __shared__ uint32_t before[kWaves][kRadix];    // a round's counts, then its places
    const int t = threadIdx.x, lane = t % 64, wave = t / 64;
    placed[t] = offsets[static_cast<uint64_t>(t) * tiles + blockIdx.x];
    const uint64_t base = static_cast<uint64_t>(blockIdx.x) * kSortTile;
    for (int r = 0; r < kSortItems; r++) {
#pragma unroll
        for (int w = 0; w < kWaves; w++) before[w][t] = 0;
        const uint64_t i = base + r * kSortThreads + t;
        const bool valid = i < n;
        const K key = valid ? in[i] : K(0);
        const uint32_t d = digit_of(key, shift);
        uint64_t peers = __ballot(valid);
#pragma unroll
        for (int b = 0; b < kRadixBits; b++) {
            const bool bit = (d >> b) & 1u;
            const uint64_t set = __ballot(bit);
            peers &= bit ? set : ~set;
        }
        const uint32_t rank = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(peers >> 32),
                                                        __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(peers), 0u));
        __syncthreads();
        // The lowest lane of each group of equal digits posts the group's size.
        if (valid && rank == 0) before[wave][d] = static_cast<uint32_t>(__popcll(peers));
        __syncthreads();
        {
            uint32_t at = placed[t];
#pragma unroll
            for (int w = 0; w < kWaves; w++) {
                const uint32_t c = before[w][t];
                before[w][t] = at;
                at += c;
            }
            placed[t] = at;
        }
        __syncthreads();
        if (valid) out[before[wave][d] + rank] = key;
        __syncthreads();
    }
}

// Float bit patterns <-> unsigned keys in totalOrder: negative values have
// every bit flipped, non-negative ones only the sign; a descending sort
// complements the keys.
template <typename K>
__global__ void __launch_bounds__(256) to_keys_kernel(const K* __restrict__ in, K* __restrict__ out, uint64_t n,
                                                      bool descending) {
    constexpr K kSign = static_cast<K>(K(1) << (sizeof(K) * 8 - 1));
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        const K v = in[i];
        const K key = (v & kSign) ? static_cast<K>(~v) : static_cast<K>(v | kSign);
        out[i] = descending ? static_cast<K>(~key) : key;
    }
}

template <typename K>
__global__ void __launch_bounds__(256) from_keys_kernel(K* __restrict__ data, uint64_t n, bool descending) {
    constexpr K kSign = static_cast<K>(K(1) << (sizeof(K) * 8 - 1));
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        const K key = descending ? static_cast<K>(~data[i]) : data[i];
        data[i] = (key & kSign) ? static_cast<K>(key & static_cast<K>(~kSign)) : static_cast<K>(~key);
    }
}

template <typename K>
int sort_typed(const void* a, void* out, uint64_t n, bool descending) {
    TC_STREAM(s);
    if (n == 0) return TC_OK;
    if (n > 0xffffffffu) return fail(TC_UNSUPPORTED, "sort: more than 2^32 elements");
    const uint64_t tiles = (n + kSortTile - 1) / kSortTile;
    const uint64_t counts = tiles * kRadix;
    const uint64_t count_tiles = (counts + kScanTile - 1) / kScanTile;
    // Scratch: the other ping-pong buffer of keys, the counts, their tile sums.
    const uint64_t keys_bytes = (n * sizeof(K) + 255) / 256 * 256;
    const uint64_t counts_bytes = (counts * sizeof(uint32_t) + 255) / 256 * 256;
    void* scratch = nullptr;
    int status = tc_alloc(keys_bytes + counts_bytes + count_tiles * sizeof(uint32_t), &scratch);
    if (status != TC_OK) return status;
    K* other = static_cast<K*>(scratch);
    uint32_t* digit_counts = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(scratch) + keys_bytes);
    uint32_t* sums = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(scratch) + keys_bytes + counts_bytes);
    K* keys = static_cast<K*>(out);
    to_keys_kernel<K><<<blocks_for(n, 1), 256, 0, s>>>(static_cast<const K*>(a), keys, n, descending);
    status = check_launch("sort");
    // An even number of passes: the sorted keys end in `out`.
    constexpr uint32_t kPasses = sizeof(K) * 8 / kRadixBits;
    static_assert(kPasses % 2 == 0, "passes end where they began");
    for (uint32_t pass = 0; pass < kPasses && status == TC_OK; pass++) {
        const K* from = pass % 2 == 0 ? keys : other;
        K* to = pass % 2 == 0 ? other : keys;
        const uint32_t shift = pass * kRadixBits;
        digit_counts_kernel<K><<<static_cast<uint32_t>(tiles), kSortThreads, 0, s>>>(from, n, shift, digit_counts,
                                                                                  static_cast<uint32_t>(tiles));
        status = check_launch("sort");
        if (status == TC_OK) {
            count_sums_kernel<<<static_cast<uint32_t>(count_tiles), kScanThreads, 0, s>>>(digit_counts, counts, sums);
            status = check_launch("sort");
        }
        if (status == TC_OK) {
            scan_count_sums_kernel<<<1, kScanThreads, 0, s>>>(sums, static_cast<uint32_t>(count_tiles));
            status = check_launch("sort");
        }
        if (status == TC_OK) {
            scan_counts_kernel<<<static_cast<uint32_t>(count_tiles), kScanThreads, 0, s>>>(digit_counts, counts, sums);
            status = check_launch("sort");
        }
        if (status == TC_OK) {
            scatter_kernel<K><<<static_cast<uint32_t>(tiles), kSortThreads, 0, s>>>(from, to, n, shift, digit_counts,
                                                                                 static_cast<uint32_t>(tiles));
            status = check_launch("sort");
        }
    }
    if (status == TC_OK) {
        from_keys_kernel<K><<<blocks_for(n, 1), 256, 0, s>>>(keys, n, descending);
        status = check_launch("sort");
    }
    tc_free(scratch);
    return status;
}

}  // namespace
}  // namespace tc

using namespace tc;

extern "C" {

int tc_prefix_sum(uint32_t dtype, const void* a, void* out, uint64_t n) {
    TC_DISPATCH_FLOAT(dtype, "prefix_sum", S, return prefix_sum_typed<S>(a, out, n));
    return TC_OK;
}

int tc_sort(uint32_t dtype, const void* a, void* out, uint64_t n, uint32_t order) {
    if (order > 1) return fail(TC_INVALID, "sort: no SortOrder " + std::to_string(order));
    switch (dtype) {
        case TC_F32: return sort_typed<uint32_t>(a, out, n, order == 1);
        case TC_F16:
        case TC_BF16: return sort_typed<uint16_t>(a, out, n, order == 1);
        default: return fail(TC_UNSUPPORTED, std::string("sort: no kernel for ") + dtype_name(dtype));
    }
}

}  // extern "C"
