// The runtime under every entry point: per-thread error state and stream,
// the stream-ordered storage cache, transfers and fills, and timing.
//
// It takes the roles the reference's Metal runtime splits across
// metal/device.rs (the thread-local device and queue), metal/pool.rs (buffer
// reuse fenced against queued work), metal/buffer.rs (reads that wait for
// the GPU), metal/sync.rs (failure reported at the next wait) and
// counters.rs (operations queued and host waits), re-cut for HIP: one
// in-order stream per host thread makes reuse of a freed block safe without
// fences, because any later use of it is queued behind every earlier one.
//
// Stream capture breaks that premise: work captured into a HIP graph runs
// again at every replay, after anything queued eagerly in between.  So a
// block allocated or freed while the thread's stream is capturing belongs
// to the graphs: freed during the capture that made it, it is reused only
// by later allocations of that same capture (whose graph replays in the
// order it was captured); freed after, or left over when the capture ends,
// it is retired, handed to nothing, until tc_release_graph_memory says the
// graphs are gone.

#include <stdio.h>
#include <string.h>

#include <map>
#include <mutex>
#include <sstream>
#include <unordered_map>

#include "common.hpp"

namespace tc {

namespace {

thread_local std::string last_error;

struct ThreadState {
    int device = -1;
    hipStream_t stream = nullptr;
    hipEvent_t timer_start = nullptr;
    hipEvent_t timer_stop = nullptr;
    // Freed blocks by their rounded size, and the size of every live block.
    std::multimap<size_t, void*> cached;
    std::unordered_map<void*, size_t> live;
    size_t cached_bytes = 0;
    // Blocks that captured graphs may touch on replay (allocated or freed
    // while capturing): live ones, those free for reuse within the capture
    // `capture_id` (0: none), and retired ones, reused by nothing.
    std::unordered_map<void*, size_t> graph_live;
    std::multimap<size_t, void*> capture_free;
    std::vector<std::pair<void*, size_t>> retired;
    unsigned long long capture_id = 0;
    // Operations queued on the stream and times the host waited for it.
    uint64_t dispatches = 0;
    uint64_t waits = 0;
    // Nothing is released at thread exit: the HIP runtime may already be
    // gone by then, and the device reclaims everything with the process.
};

thread_local ThreadState state;

int cus = 0;
std::once_flag cus_once;

int hip_fail(hipError_t error, const char* what) {
    return fail(error == hipErrorOutOfMemory ? TC_OUT_OF_MEMORY : TC_DEVICE,
                std::string(what) + ": " + hipGetErrorString(error));
}

// Blocks are rounded so that a tape's many same-shaped temporaries reuse one
// another: to 512 bytes below 1 MiB and to 2 MiB above.
size_t rounded(size_t bytes) {
    if (bytes == 0) bytes = 1;
    size_t quantum = bytes < (size_t{1} << 20) ? 512 : (size_t{2} << 20);
    return (bytes + quantum - 1) / quantum * quantum;
}

}  // namespace

int fail(int status, const std::string& message) {
    last_error = message;
    return status;
}

int init_device(int device) {
    if (state.stream != nullptr) {
        if (state.device == device) return TC_OK;
        return fail(TC_INVALID, "tc_init: this thread already uses device " +
                                    std::to_string(state.device));
    }
    int count = 0;
    hipError_t error = hipGetDeviceCount(&count);
    if (error != hipSuccess || count == 0) {
        return fail(TC_DEVICE, "no HIP device is available; Host fallback is disabled");
    }
    if (device < 0 || device >= count) {
        return fail(TC_INVALID, "tc_init: device " + std::to_string(device) + " of " +
                                    std::to_string(count));
    }
    if ((error = hipSetDevice(device)) != hipSuccess) return hip_fail(error, "hipSetDevice");
    hipStream_t created = nullptr;
    if ((error = hipStreamCreateWithFlags(&created, hipStreamNonBlocking)) != hipSuccess) {
        return hip_fail(error, "hipStreamCreate");
    }
    state.stream = created;
    state.device = device;
    return TC_OK;
}

hipStream_t stream() {
    if (state.stream == nullptr && init_device(0) != TC_OK) return nullptr;
    return state.stream;
}

int check_launch(const char* what) {
    state.dispatches++;
    hipError_t error = hipGetLastError();
    if (error != hipSuccess) return hip_fail(error, what);
    return TC_OK;
}

void count_dispatch() { state.dispatches++; }

hipError_t host_wait(hipStream_t s) {
    state.waits++;
    return hipStreamSynchronize(s);
}

hipError_t host_wait(hipEvent_t e) {
    state.waits++;
    return hipEventSynchronize(e);
}

namespace {

// The capture the thread's stream is in (0: none), ending the previous one
// first if it is over: its free blocks are retired.
unsigned long long current_capture(hipStream_t s) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    unsigned long long id = 0;
    if (hipStreamGetCaptureInfo(s, &status, &id) != hipSuccess) {
        (void)hipGetLastError();
        status = hipStreamCaptureStatusNone;
    }
    if (status != hipStreamCaptureStatusActive) id = 0;
    if (id != state.capture_id) {
        for (auto& entry : state.capture_free) state.retired.emplace_back(entry.second, entry.first);
        state.capture_free.clear();
        state.capture_id = id;
    }
    return id;
}

}  // namespace

int compute_units() {
    std::call_once(cus_once, [] {
        int device = 0;
        (void)hipGetDevice(&device);
        hipDeviceProp_t props;
        cus = hipGetDeviceProperties(&props, device) == hipSuccess ? props.multiProcessorCount : 256;
        if (cus <= 0) cus = 256;
    });
    return cus;
}

std::string shape_text(const uint64_t* values, uint32_t rank) {
    std::ostringstream text;
    text << "[";
    for (uint32_t k = 0; k < rank; k++) text << (k ? ", " : "") << values[k];
    text << "]";
    return text.str();
}

int check_strided(uint64_t len, uint32_t rank, const uint64_t* shape, uint64_t offset,
                  const uint64_t* strides, const char* operation, uint64_t* count) {
    std::string shape_str = shape_text(shape, rank);
    if (rank > static_cast<uint32_t>(kMaxRank)) {
        return fail(TC_INVALID, std::string(operation) + ": shape " + shape_str +
                                    " has more than " + std::to_string(kMaxRank) + " axes");
    }
    if (!element_count(rank, shape, count)) {
        return fail(TC_INVALID, std::string(operation) + ": shape " + shape_str +
                                    " has more elements than fit in a usize");
    }
    uint64_t end = 0;
    bool fits = reach(rank, shape, offset, strides, &end);
    if (!fits || end > len) {
        return fail(TC_INVALID, std::string(operation) + ": shape " + shape_str +
                                    " with strides " + shape_text(strides, rank) +
                                    " from offset " + std::to_string(offset) +
                                    " reaches past " + std::to_string(len) + " elements");
    }
    return TC_OK;
}

// ---- fill -------------------------------------------------------------------

template <typename W>
__global__ void fill_kernel(W* __restrict__ dst, uint64_t count, W value) {
    uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += stride) {
        dst[i] = value;
    }
}

// A fill of `width`-byte elements as 16-byte stores where the run allows:
// the pattern of one element repeated to 16 bytes is stored with uint4.
int fill(void* dst, uint64_t count, uint32_t width, const void* value) {
    TC_STREAM(s);
    if (count == 0) return TC_OK;
    if (width != 1 && width != 2 && width != 4 && width != 8 && width != 16) {
        return fail(TC_UNSUPPORTED, "fill: no kernel for " + std::to_string(width) +
                                        "-byte elements");
    }
    uint64_t bytes = count * width;
    uint8_t pattern[16];
    for (uint32_t at = 0; at < 16; at += width) memcpy(pattern + at, value, width);
    uint4 wide;
    memcpy(&wide, pattern, 16);
    uint8_t* base = static_cast<uint8_t*>(dst);
    if (reinterpret_cast<uintptr_t>(base) % 16 == 0 && bytes >= 16) {
        uint64_t vectors = bytes / 16;
        fill_kernel<uint4><<<grid_for(vectors, 256 * 4), 256, 0, s>>>(
            reinterpret_cast<uint4*>(base), vectors, wide);
        base += vectors * 16;
        bytes -= vectors * 16;
    }
    if (bytes > 0) {
        uint64_t tail = bytes / width;
        switch (width) {
            case 1: fill_kernel<uint8_t><<<grid_for(tail, 256), 256, 0, s>>>(base, tail, pattern[0]); break;
            case 2: {
                uint16_t v; memcpy(&v, pattern, 2);
                fill_kernel<uint16_t><<<grid_for(tail, 256), 256, 0, s>>>(reinterpret_cast<uint16_t*>(base), tail, v);
                break;
            }
            case 4: {
                uint32_t v; memcpy(&v, pattern, 4);
                fill_kernel<uint32_t><<<grid_for(tail, 256), 256, 0, s>>>(reinterpret_cast<uint32_t*>(base), tail, v);
                break;
            }
            case 8: {
                uint64_t v; memcpy(&v, pattern, 8);
                fill_kernel<uint64_t><<<grid_for(tail, 256), 256, 0, s>>>(reinterpret_cast<uint64_t*>(base), tail, v);
                break;
            }
            default:
                fill_kernel<uint4><<<grid_for(tail, 256), 256, 0, s>>>(reinterpret_cast<uint4*>(base), tail, wide);
                break;
        }
    }
    return check_launch("fill");
}

}  // namespace tc

using namespace tc;

extern "C" {

int tc_init(int device) { return init_device(device); }

const char* tc_last_error(void) { return last_error.c_str(); }

int tc_sync(void) {
    TC_STREAM(s);
    hipError_t error = host_wait(s);
    if (error != hipSuccess) return hip_fail(error, "the GPU failed; its output is invalid");
    return TC_OK;
}

int tc_stream(void** out) {
    TC_STREAM(s);
    *out = s;
    return TC_OK;
}

int tc_device_info(char* name, size_t name_len, char* arch, size_t arch_len) {
    TC_STREAM(s);
    (void)s;
    hipDeviceProp_t props;
    hipError_t error = hipGetDeviceProperties(&props, state.device);
    if (error != hipSuccess) return hip_fail(error, "hipGetDeviceProperties");
    if (name && name_len) snprintf(name, name_len, "%s", props.name);
    if (arch && arch_len) snprintf(arch, arch_len, "%s", props.gcnArchName);
    return TC_OK;
}

int tc_timer_begin(void) {
    TC_STREAM(s);
    hipError_t error;
    if (state.timer_start == nullptr) {
        if ((error = hipEventCreate(&state.timer_start)) != hipSuccess) return hip_fail(error, "hipEventCreate");
        if ((error = hipEventCreate(&state.timer_stop)) != hipSuccess) return hip_fail(error, "hipEventCreate");
    }
    if ((error = hipEventRecord(state.timer_start, s)) != hipSuccess) return hip_fail(error, "hipEventRecord");
    return TC_OK;
}

int tc_timer_end(float* milliseconds) {
    TC_STREAM(s);
    if (state.timer_start == nullptr) return fail(TC_INVALID, "tc_timer_end without tc_timer_begin");
    hipError_t error;
    if ((error = hipEventRecord(state.timer_stop, s)) != hipSuccess) return hip_fail(error, "hipEventRecord");
    if ((error = host_wait(state.timer_stop)) != hipSuccess) return hip_fail(error, "the GPU failed; its output is invalid");
    if ((error = hipEventElapsedTime(milliseconds, state.timer_start, state.timer_stop)) != hipSuccess) {
        return hip_fail(error, "hipEventElapsedTime");
    }
    return TC_OK;
}

int tc_alloc(size_t bytes, void** out) {
    TC_STREAM(s);
    size_t size = rounded(bytes);
    const bool capturing = current_capture(s) != 0;
    if (capturing) {
        auto hit = state.capture_free.find(size);
        if (hit != state.capture_free.end()) {
            *out = hit->second;
            state.capture_free.erase(hit);
            state.graph_live[*out] = size;
            return TC_OK;
        }
    }
    auto hit = state.cached.find(size);
    if (hit != state.cached.end()) {
        *out = hit->second;
        state.cached.erase(hit);
        state.cached_bytes -= size;
        (capturing ? state.graph_live : state.live)[*out] = size;
        return TC_OK;
    }
    void* pointer = nullptr;
    hipError_t error = hipMalloc(&pointer, size);
    if (error == hipErrorOutOfMemory && !state.cached.empty() && !capturing) {
        // Give the cache back and try once more before reporting.
        (void)hipGetLastError();
        (void)host_wait(s);
        for (auto& entry : state.cached) (void)hipFree(entry.second);
        state.cached.clear();
        state.cached_bytes = 0;
        error = hipMalloc(&pointer, size);
    }
    if (error != hipSuccess) {
        (void)hipGetLastError();
        return hip_fail(error, ("allocating " + std::to_string(bytes) + " bytes").c_str());
    }
    (capturing ? state.graph_live : state.live)[pointer] = size;
    *out = pointer;
    return TC_OK;
}

int tc_free(void* pointer) {
    if (pointer == nullptr) return TC_OK;
    TC_STREAM(s);
    const bool capturing = current_capture(s) != 0;
    auto found = state.live.find(pointer);
    size_t size = 0;
    bool graphs = capturing;
    if (found != state.live.end()) {
        size = found->second;
        state.live.erase(found);
    } else {
        auto owned = state.graph_live.find(pointer);
        if (owned == state.graph_live.end()) {
            return fail(TC_INVALID, "tc_free: the pointer was not allocated by tc_alloc on this thread");
        }
        size = owned->second;
        state.graph_live.erase(owned);
        graphs = true;
    }
    if (!graphs) {
        state.cached.emplace(size, pointer);
        state.cached_bytes += size;
    } else if (capturing) {
        state.capture_free.emplace(size, pointer);
    } else {
        state.retired.emplace_back(pointer, size);
    }
    return TC_OK;
}

int tc_release_graph_memory(void) {
    TC_STREAM(s);
    if (current_capture(s) != 0) {
        return fail(TC_INVALID, "tc_release_graph_memory: the stream is capturing");
    }
    for (auto& entry : state.retired) {
        state.cached.emplace(entry.second, entry.first);
        state.cached_bytes += entry.second;
    }
    state.retired.clear();
    for (auto& entry : state.graph_live) state.live.emplace(entry.first, entry.second);
    state.graph_live.clear();
    return TC_OK;
}

int tc_graph_memory(uint64_t* live_bytes, uint64_t* retired_bytes) {
    TC_STREAM(s);
    (void)current_capture(s);
    uint64_t live = 0, retired = 0;
    for (auto& entry : state.graph_live) live += entry.second;
    for (auto& entry : state.capture_free) retired += entry.first;
    for (auto& entry : state.retired) retired += entry.second;
    *live_bytes = live;
    *retired_bytes = retired;
    return TC_OK;
}

int tc_empty_cache(void) {
    TC_STREAM(s);
    if (current_capture(s) != 0) return fail(TC_INVALID, "tc_empty_cache: the stream is capturing");
    hipError_t error = host_wait(s);
    if (error != hipSuccess) return hip_fail(error, "the GPU failed; its output is invalid");
    for (auto& entry : state.cached) (void)hipFree(entry.second);
    state.cached.clear();
    state.cached_bytes = 0;
    return TC_OK;
}

int tc_activity(uint64_t* dispatches, uint64_t* waits) {
    *dispatches = state.dispatches;
    *waits = state.waits;
    return TC_OK;
}

// Transfers this large go through the thread's pinned staging
// (tc_upload_staged, persist.hip), at about twice the runtime's pageable
// rate up and three times down; smaller ones cost less as one runtime copy.
constexpr size_t kStagedBytes = size_t{8} << 20;

int tc_upload(void* dst, const void* src, size_t bytes) {
    TC_STREAM(s);
    if (bytes == 0) return TC_OK;
    if (bytes >= kStagedBytes) return tc_upload_staged(dst, src, bytes);
    // A pageable source: the runtime stages it before the call returns, so
    // the caller's buffer is free to reuse at once.
    hipError_t error = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s);
    if (error != hipSuccess) return hip_fail(error, "upload");
    error = host_wait(s);
    if (error != hipSuccess) return hip_fail(error, "upload");
    return TC_OK;
}

int tc_download(void* dst, const void* src, size_t bytes) {
    TC_STREAM(s);
    if (bytes == 0) return TC_OK;
    if (bytes >= kStagedBytes) return tc_download_staged(dst, src, bytes);
    hipError_t error = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s);
    if (error != hipSuccess) return hip_fail(error, "download");
    error = host_wait(s);
    if (error != hipSuccess) return hip_fail(error, "the GPU failed; its output is invalid");
    return TC_OK;
}

int tc_copy(void* dst, const void* src, size_t bytes) {
    TC_STREAM(s);
    if (bytes == 0) return TC_OK;
    // From 16 MiB, whole 16-byte words go through the copy kernel (one word
    // a thread, streaming past the Infinity Cache when large): measured on
    // MI355X, 6.5-6.7 TB/s from 64 MiB up against the runtime's 5.1-5.6.
    if (bytes >= (size_t{16} << 20) && bytes % 16 == 0 && reinterpret_cast<uintptr_t>(src) % 16 == 0 &&
        reinterpret_cast<uintptr_t>(dst) % 16 == 0) {
        const uint64_t words = bytes / 4;
        const uint64_t shape[1] = {words};
        tc_strided from{};
        from.strides[0] = 1;
        return tc_strided_copy(4, src, words, 1, shape, &from, dst);
    }
    count_dispatch();
    hipError_t error = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, s);
    if (error != hipSuccess) return hip_fail(error, "duplicate");
    return TC_OK;
}

int tc_fill(void* dst, uint64_t count, uint32_t width, const void* value) {
    return tc::fill(dst, count, width, value);
}

}  // extern "C"
