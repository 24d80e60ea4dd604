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
// +inf < +NaN), sorted by rocPRIM's device radix sort, and mapped back.

#include <rocprim/device/device_radix_sort.hpp>

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

// Float bit patterns <-> unsigned keys in totalOrder: negative values have
// every bit flipped, non-negative ones only the sign.
template <typename K>
__global__ void __launch_bounds__(256) order_keys_kernel(const K* __restrict__ in, K* __restrict__ out, uint64_t n,
                                                         bool forward) {
    constexpr K kSign = static_cast<K>(K(1) << (sizeof(K) * 8 - 1));
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        const K v = in[i];
        if (forward) {
            out[i] = (v & kSign) ? static_cast<K>(~v) : static_cast<K>(v | kSign);
        } else {
            out[i] = (v & kSign) ? static_cast<K>(v & static_cast<K>(~kSign)) : static_cast<K>(~v);
        }
    }
}

template <typename K>
int sort_typed(const void* a, void* out, uint64_t n, bool descending) {
    TC_STREAM(s);
    if (n == 0) return TC_OK;
    if (n > 0xffffffffu) return fail(TC_UNSUPPORTED, "sort: more than 2^32 elements");
    void* keys = nullptr;
    int status = tc_alloc(n * sizeof(K), &keys);
    if (status != TC_OK) return status;
    K* k = static_cast<K*>(keys);
    K* o = static_cast<K*>(out);
    order_keys_kernel<K><<<blocks_for(n, 1), 256, 0, s>>>(static_cast<const K*>(a), k, n, true);
    status = check_launch("sort");
    size_t bytes = 0;
    const unsigned size = static_cast<unsigned>(n);
    constexpr unsigned kBits = sizeof(K) * 8;
    hipError_t error = descending ? rocprim::radix_sort_keys_desc(nullptr, bytes, k, o, size, 0, kBits, s)
                                  : rocprim::radix_sort_keys(nullptr, bytes, k, o, size, 0, kBits, s);
    void* temp = nullptr;
    if (status == TC_OK && error == hipSuccess) status = tc_alloc(bytes > 0 ? bytes : 1, &temp);
    if (status == TC_OK && error == hipSuccess) {
        error = descending ? rocprim::radix_sort_keys_desc(temp, bytes, k, o, size, 0, kBits, s)
                           : rocprim::radix_sort_keys(temp, bytes, k, o, size, 0, kBits, s);
    }
    if (status == TC_OK && error != hipSuccess) status = fail(TC_DEVICE, std::string("sort: ") + hipGetErrorString(error));
    if (status == TC_OK) {
        order_keys_kernel<K><<<blocks_for(n, 1), 256, 0, s>>>(o, o, n, false);
        status = check_launch("sort");
    }
    if (temp != nullptr) tc_free(temp);
    tc_free(keys);
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
