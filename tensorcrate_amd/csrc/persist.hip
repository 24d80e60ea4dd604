// Host memory and files to and from HBM through pinned staging: pageable
// uploads (`to_backend`, tensors/backend.rs) and the `TCR1` tensor format
// (persist.rs:44-93), read and written straight between the file and the
// device.
//
// Each thread owns two pinned staging buffers.  A transfer moves in chunks
// of one buffer: while the DMA engine copies chunk i between a buffer and
// HBM, the CPU fills (from user memory or the file) or drains the other, so
// the file or memcpy time and the PCIe time overlap; the host side of a
// chunk is itself split over four CPU threads.  The buffers are allocated on
// first use and held until the process ends.
//
// The TCR1 checks and their messages are the reference's (persist.rs:
// 266-330): magic, version, kind, element tag, extents.  Payload bytes move
// as they are, so every element type's bits survive the round trip; the
// element tag fixes the element size (a prefix code: Complex and Dual hold
// two of what follows, FixedPoint<N> an i64).

#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <functional>
#include <sstream>
#include <thread>
#include <vector>

#include "common.hpp"

namespace tc {
namespace {

constexpr size_t kStageBytes = size_t{16} << 20;

struct Staging {
    void* buffer[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    bool pending[2] = {false, false};
};

thread_local Staging staging;

int staging_ready() {
    for (int k = 0; k < 2; k++) {
        if (staging.buffer[k] == nullptr) {
            hipError_t error = hipHostMalloc(&staging.buffer[k], kStageBytes, hipHostMallocDefault);
            if (error != hipSuccess) {
                staging.buffer[k] = nullptr;
                return fail(TC_OUT_OF_MEMORY, std::string("staging buffer: ") + hipGetErrorString(error));
            }
        }
        if (staging.done[k] == nullptr) {
            hipError_t error = hipEventCreateWithFlags(&staging.done[k], hipEventDisableTiming);
            if (error != hipSuccess) {
                staging.done[k] = nullptr;
                return fail(TC_DEVICE, std::string("staging event: ") + hipGetErrorString(error));
            }
        }
    }
    return TC_OK;
}

// `work(offset, n)` over [0, bytes) in up to four pieces at once (one on the
// calling thread): a single CPU thread copies at about half of what PCIe
// moves, so a chunk's host side is split.  The first failing piece's
// status is returned.
int in_parallel(size_t bytes, const std::function<int(size_t, size_t)>& work) {
    constexpr size_t kPieces = 4, kMinPiece = size_t{1} << 20;
    const size_t pieces = bytes / kMinPiece < kPieces ? (bytes / kMinPiece > 0 ? bytes / kMinPiece : 1) : kPieces;
    if (pieces == 1) return work(0, bytes);
    const size_t piece = (bytes + pieces - 1) / pieces;
    std::vector<int> status(pieces, TC_OK);
    std::vector<std::string> message(pieces);  // a helper's error, recorded on its own thread
    std::vector<std::thread> helpers;
    for (size_t k = 1; k < pieces; k++) {
        const size_t at = k * piece;
        const size_t n = at < bytes ? (bytes - at < piece ? bytes - at : piece) : 0;
        helpers.emplace_back([&, k, at, n] {
            status[k] = n ? work(at, n) : TC_OK;
            if (status[k] != TC_OK) message[k] = tc_last_error();
        });
    }
    status[0] = work(0, piece < bytes ? piece : bytes);
    for (std::thread& t : helpers) t.join();
    if (status[0] != TC_OK) return status[0];
    for (size_t k = 1; k < pieces; k++) {
        if (status[k] != TC_OK) return fail(status[k], message[k]);
    }
    return TC_OK;
}

// Wait until the DMA last queued on buffer `k` is done with it.
int wait_buffer(int k) {
    if (!staging.pending[k]) return TC_OK;
    hipError_t error = host_wait(staging.done[k]);
    staging.pending[k] = false;
    return error == hipSuccess ? TC_OK : fail(TC_DEVICE, std::string("staging: ") + hipGetErrorString(error));
}

// `bytes` into `device_dst`, `fill(host, offset, n)` producing each chunk.
template <typename Fill>
int staged_upload(void* device_dst, size_t bytes, Fill fill) {
    TC_STREAM(s);
    int status = staging_ready();
    if (status != TC_OK) return status;
    int k = 0;
    for (size_t done = 0; done < bytes; done += kStageBytes, k ^= 1) {
        const size_t n = bytes - done < kStageBytes ? bytes - done : kStageBytes;
        if ((status = wait_buffer(k)) != TC_OK) return status;
        if ((status = fill(staging.buffer[k], done, n)) != TC_OK) return status;
        count_dispatch();
        hipError_t error = hipMemcpyAsync(static_cast<char*>(device_dst) + done, staging.buffer[k], n,
                                          hipMemcpyHostToDevice, s);
        if (error == hipSuccess) error = hipEventRecord(staging.done[k], s);
        if (error != hipSuccess) return fail(TC_DEVICE, std::string("staged upload: ") + hipGetErrorString(error));
        staging.pending[k] = true;
    }
    // The source is consumed once both buffers have drained.
    if ((status = wait_buffer(0)) != TC_OK) return status;
    return wait_buffer(1);
}

// `bytes` from `device_src`, `drain(host, offset, n)` taking each chunk; the
// next chunk's DMA runs while the CPU drains this one.
template <typename Drain>
int staged_download(const void* device_src, size_t bytes, Drain drain) {
    TC_STREAM(s);
    int status = staging_ready();
    if (status != TC_OK) return status;
    auto issue = [&](size_t at, int k) -> int {
        const size_t n = bytes - at < kStageBytes ? bytes - at : kStageBytes;
        count_dispatch();
        hipError_t error = hipMemcpyAsync(staging.buffer[k], static_cast<const char*>(device_src) + at, n,
                                          hipMemcpyDeviceToHost, s);
        if (error == hipSuccess) error = hipEventRecord(staging.done[k], s);
        if (error != hipSuccess) return fail(TC_DEVICE, std::string("staged download: ") + hipGetErrorString(error));
        staging.pending[k] = true;
        return TC_OK;
    };
    if (bytes == 0) return TC_OK;
    if ((status = issue(0, 0)) != TC_OK) return status;
    int k = 0;
    for (size_t done = 0; done < bytes; done += kStageBytes, k ^= 1) {
        const size_t n = bytes - done < kStageBytes ? bytes - done : kStageBytes;
        if (done + n < bytes) {
            if ((status = wait_buffer(k ^ 1)) != TC_OK) return status;
            if ((status = issue(done + n, k ^ 1)) != TC_OK) return status;
        }
        if ((status = wait_buffer(k)) != TC_OK) return status;
        if ((status = drain(staging.buffer[k], done, n)) != TC_OK) return status;
    }
    return TC_OK;
}

// ---- small reads, queued --------------------------------------------------------

// A reduction's result read back without a wait at the time it is asked for
// (the tape's unread loss, tape/mod.rs:253-295): the copy is queued behind the
// thread's work into one of its pinned slots, and only reading the ticket
// waits, for that copy alone.
constexpr uint64_t kSlots = 1024;
constexpr size_t kSlotBytes = 64;

struct Slots {
    uint8_t* pinned = nullptr;
    hipEvent_t done[kSlots] = {};
    uint64_t issued = 0;  // tickets handed out; ticket t lives in slot t % kSlots
};

thread_local Slots slots;

// ---- TCR1 -------------------------------------------------------------------

constexpr uint8_t kMagic[4] = {'T', 'C', 'R', '1'};
constexpr uint8_t kVersion = 1;
constexpr uint8_t kComplex = 0x20, kDual = 0x21, kFixedPoint = 0x30;

// persist.rs:190-225: the type a tag names, as the reference prints it.
std::string describe(const uint8_t* tag, uint32_t length) {
    uint32_t at = 0;
    std::function<std::string()> walk = [&]() -> std::string {
        if (at >= length) return "?";
        const uint8_t code = tag[at++];
        static const char* const kLeaves[] = {nullptr, "i8", "u8", "i16", "u16", "i32", "u32", "i64", "u64"};
        if (code >= 0x01 && code <= 0x08) return kLeaves[code];
        switch (code) {
            case 0x10: return "f32";
            case 0x11: return "f64";
            case 0x12: return "f16";
            case 0x13: return "bf16";
            case kComplex: return "Complex<" + walk() + ">";
            case kDual: return "Dual<" + walk() + ">";
            case kFixedPoint: {
                const std::string precision = at < length ? std::to_string(tag[at]) : "?";
                at++;
                return "FixedPoint<" + precision + ">";
            }
            default: {
                char hex[8];
                snprintf(hex, sizeof(hex), "%02x", code);
                return std::string("<unknown tag 0x") + hex + ">";
            }
        }
    };
    return walk();
}

// Bytes one element of the tag's type occupies, or 0 for a tag this library
// cannot size (reserved and unknown codes, or a malformed prefix).
uint64_t element_bytes(const uint8_t* tag, uint32_t length, uint32_t* at) {
    if (*at >= length) return 0;
    const uint8_t code = tag[(*at)++];
    switch (code) {
        case 0x01: case 0x02: return 1;
        case 0x03: case 0x04: case 0x12: case 0x13: return 2;
        case 0x05: case 0x06: case 0x10: return 4;
        case 0x07: case 0x08: case 0x11: return 8;
        case kComplex: case kDual: return 2 * element_bytes(tag, length, at);
        case kFixedPoint: return ++(*at) <= length ? 8 : 0;
        default: return 0;
    }
}

const char* name_of_kind(uint32_t kind) {
    switch (kind) {
        case 0: return "vector";
        case 1: return "matrix";
        case 2: return "tensor";
        default: return "tensor of unknown kind";
    }
}

std::string bytes_text(const uint8_t* b, int n) {
    std::ostringstream out;
    out << "[";
    for (int k = 0; k < n; k++) out << (k ? ", " : "") << int(b[k]);
    out << "]";
    return out.str();
}

struct File {
    int fd = -1;
    ~File() {
        if (fd >= 0) close(fd);
    }
};

// Exactly `n` bytes at `offset`, or the reference's end-of-input error.
int read_exact(int fd, void* out, size_t n, uint64_t offset) {
    size_t got = 0;
    while (got < n) {
        const ssize_t r = pread(fd, static_cast<char*>(out) + got, n - got, static_cast<off_t>(offset + got));
        if (r < 0) return fail(TC_IO, std::string("read: ") + strerror(errno));
        if (r == 0) return fail(TC_IO, "failed to fill whole buffer");
        got += static_cast<size_t>(r);
    }
    return TC_OK;
}

int write_all(int fd, const void* data, size_t n) {
    size_t put = 0;
    while (put < n) {
        const ssize_t w = write(fd, static_cast<const char*>(data) + put, n - put);
        if (w < 0) return fail(TC_IO, std::string("write: ") + strerror(errno));
        put += static_cast<size_t>(w);
    }
    return TC_OK;
}

int open_for(const char* path, int flags, File* file) {
    file->fd = open(path, flags, 0644);
    if (file->fd < 0) return fail(TC_IO, std::string(path) + ": " + strerror(errno));
    return TC_OK;
}

}  // namespace
}  // namespace tc

using namespace tc;

extern "C" {

int tc_upload_staged(void* device_dst, const void* host_src, size_t bytes) {
    return staged_upload(device_dst, bytes, [&](void* host, size_t at, size_t n) -> int {
        return in_parallel(n, [&](size_t part, size_t len) {
            memcpy(static_cast<char*>(host) + part, static_cast<const char*>(host_src) + at + part, len);
            return TC_OK;
        });
    });
}

int tc_download_staged(void* host_dst, const void* device_src, size_t bytes) {
    return staged_download(device_src, bytes, [&](const void* host, size_t at, size_t n) -> int {
        return in_parallel(n, [&](size_t part, size_t len) {
            memcpy(static_cast<char*>(host_dst) + at + part, static_cast<const char*>(host) + part, len);
            return TC_OK;
        });
    });
}

int tc_read_async(const void* device_src, size_t bytes, uint64_t* ticket) {
    TC_STREAM(s);
    if (bytes > kSlotBytes) return fail(TC_INVALID, "read_async: " + std::to_string(bytes) + " bytes, over 64");
    if (slots.pinned == nullptr) {
        void* block = nullptr;
        hipError_t error = hipHostMalloc(&block, kSlots * kSlotBytes, hipHostMallocDefault);
        if (error != hipSuccess) return fail(TC_OUT_OF_MEMORY, std::string("read slots: ") + hipGetErrorString(error));
        slots.pinned = static_cast<uint8_t*>(block);
    }
    const uint64_t t = slots.issued;
    const uint64_t slot = t % kSlots;
    if (slots.done[slot] == nullptr) {
        hipError_t error = hipEventCreateWithFlags(&slots.done[slot], hipEventDisableTiming);
        if (error != hipSuccess) return fail(TC_DEVICE, std::string("read slot event: ") + hipGetErrorString(error));
    } else {
        // The slot's previous read must land before this one overwrites it.
        hipError_t error = host_wait(slots.done[slot]);
        if (error != hipSuccess) return fail(TC_DEVICE, std::string("read slot: ") + hipGetErrorString(error));
    }
    count_dispatch();
    hipError_t error = hipMemcpyAsync(slots.pinned + slot * kSlotBytes, device_src, bytes, hipMemcpyDeviceToHost, s);
    if (error == hipSuccess) error = hipEventRecord(slots.done[slot], s);
    if (error != hipSuccess) return fail(TC_DEVICE, std::string("read_async: ") + hipGetErrorString(error));
    slots.issued = t + 1;
    *ticket = t;
    return TC_OK;
}

int tc_read_wait(uint64_t ticket, void* host_dst, size_t bytes) {
    if (bytes > kSlotBytes) return fail(TC_INVALID, "read_wait: " + std::to_string(bytes) + " bytes, over 64");
    if (ticket >= slots.issued || slots.issued - ticket > kSlots) {
        return fail(TC_INVALID, "read_wait: ticket " + std::to_string(ticket) +
                                    (ticket >= slots.issued ? " was never issued on this thread"
                                                            : " was reused by 1024 later reads"));
    }
    const uint64_t slot = ticket % kSlots;
    hipError_t error = host_wait(slots.done[slot]);
    if (error != hipSuccess) return fail(TC_DEVICE, std::string("the GPU failed; its output is invalid: ") +
                                                        hipGetErrorString(error));
    memcpy(host_dst, slots.pinned + slot * kSlotBytes, bytes);
    return TC_OK;
}

int tc_tcr1_read_header(const char* path, uint64_t offset, const uint8_t* tag, uint32_t tag_length,
                        uint32_t kind, tc_tcr1* out) {
    File file;
    int status = open_for(path, O_RDONLY, &file);
    if (status != TC_OK) return status;
    uint8_t prefix[7];
    if ((status = read_exact(file.fd, prefix, 7, offset)) != TC_OK) return status;
    if (memcmp(prefix, kMagic, 4) != 0) {
        return fail(TC_FORMAT, "not a tensor file: expected magic " + bytes_text(kMagic, 4) + ", found " +
                                   bytes_text(prefix, 4));
    }
    const uint8_t version = prefix[4], stored_kind = prefix[5], stored_length = prefix[6];
    if (version != kVersion) {
        return fail(TC_FORMAT, "format version " + std::to_string(version) +
                                   " is not supported; this build reads version " + std::to_string(kVersion));
    }
    // A tensor target also reads vector and matrix records (persist.rs:459).
    const bool kind_ok = kind == 2 ? stored_kind <= 2 : stored_kind == kind;
    if (!kind_ok) {
        return fail(TC_FORMAT, std::string("expected a ") + name_of_kind(kind) + ", found a " +
                                   name_of_kind(stored_kind));
    }
    uint8_t stored_tag[255];
    if ((status = read_exact(file.fd, stored_tag, stored_length, offset + 7)) != TC_OK) return status;
    if (stored_length != tag_length || memcmp(stored_tag, tag, tag_length) != 0) {
        return fail(TC_FORMAT, "element type is " + describe(stored_tag, stored_length) + ", but the target holds " +
                                   describe(tag, tag_length));
    }
    tc_tcr1 header{};
    header.kind = stored_kind;
    uint64_t at = offset + 7 + stored_length;
    uint64_t first[2] = {0, 0};
    if ((status = read_exact(file.fd, first, stored_kind == 2 ? 8 : 16, at)) != TC_OK) return status;
    if (stored_kind == 2) {
        const uint64_t rank = first[0];
        if (rank > TC_MAX_RANK) {
            return fail(TC_FORMAT, "stored tensor has " + std::to_string(rank) +
                                       " axes; a tensor may have at most " + std::to_string(TC_MAX_RANK));
        }
        header.rank = static_cast<uint32_t>(rank);
        if ((status = read_exact(file.fd, header.shape, 8 * rank, at + 8)) != TC_OK) return status;
        at += 8 + 8 * rank;
    } else {
        header.rank = stored_kind == 0 ? 1 : 2;
        header.shape[0] = first[0];
        if (stored_kind == 1) header.shape[1] = first[1];
        at += 16;
    }
    uint64_t count = 1;
    for (uint32_t d = 0; d < header.rank; d++) {
        if (header.shape[d] != 0 && count > UINT64_MAX / header.shape[d]) {
            if (stored_kind == 1) {
                return fail(TC_FORMAT, "stored tensor is " + std::to_string(header.shape[0]) + "×" +
                                           std::to_string(header.shape[1]) +
                                           ", which overflows this platform's address space");
            }
            return fail(TC_FORMAT, "stored tensor of shape " + shape_text(header.shape, header.rank) +
                                       " overflows this platform's address space");
        }
        count *= header.shape[d];
    }
    uint32_t parsed = 0;
    const uint64_t width = element_bytes(tag, tag_length, &parsed);
    if (width == 0 || parsed != tag_length) {
        return fail(TC_UNSUPPORTED, "TCR1: no fixed element size for " + describe(tag, tag_length));
    }
    if (count > UINT64_MAX / width) {
        return fail(TC_FORMAT, "stored tensor of shape " + shape_text(header.shape, header.rank) +
                                   " overflows this platform's address space");
    }
    header.count = count;
    header.element_bytes = width;
    header.data_offset = at;
    header.end_offset = at + count * width;
    struct stat info;
    if (fstat(file.fd, &info) != 0) return fail(TC_IO, std::string("stat: ") + strerror(errno));
    if (static_cast<uint64_t>(info.st_size) < header.end_offset) return fail(TC_IO, "failed to fill whole buffer");
    *out = header;
    return TC_OK;
}

int tc_tcr1_load(const char* path, const tc_tcr1* header, void* device_dst) {
    File file;
    int status = open_for(path, O_RDONLY, &file);
    if (status != TC_OK) return status;
    const uint64_t bytes = header->count * header->element_bytes;
    return staged_upload(device_dst, bytes, [&](void* host, size_t at, size_t n) -> int {
        return in_parallel(n, [&](size_t part, size_t len) {
            return read_exact(file.fd, static_cast<char*>(host) + part, len, header->data_offset + at + part);
        });
    });
}

int tc_tcr1_save(const char* path, int append, uint32_t kind, uint32_t rank, const uint64_t* shape,
                 const uint8_t* tag, uint32_t tag_length, const void* device_src) {
    if (kind > 2) return fail(TC_INVALID, "TCR1: no kind " + std::to_string(kind));
    if (tag_length == 0 || tag_length > 255) return fail(TC_FORMAT, "element tag is " + std::to_string(tag_length) + " bytes, limit 255");
    if ((kind == 0 && rank != 1) || (kind == 1 && rank != 2) || rank > TC_MAX_RANK) {
        return fail(TC_INVALID, "TCR1: a " + std::string(name_of_kind(kind)) + " of " + std::to_string(rank) + " axes");
    }
    uint32_t parsed = 0;
    const uint64_t width = element_bytes(tag, tag_length, &parsed);
    if (width == 0 || parsed != tag_length) {
        return fail(TC_UNSUPPORTED, "TCR1: no fixed element size for " + describe(tag, tag_length));
    }
    uint64_t count = 1;
    for (uint32_t d = 0; d < rank; d++) count *= shape[d];
    std::string head(reinterpret_cast<const char*>(kMagic), 4);
    head += static_cast<char>(kVersion);
    head += static_cast<char>(kind);
    head += static_cast<char>(tag_length);
    head.append(reinterpret_cast<const char*>(tag), tag_length);
    auto u64 = [&](uint64_t v) { head.append(reinterpret_cast<const char*>(&v), 8); };  // little-endian host
    if (kind == 2) {
        u64(rank);
        for (uint32_t d = 0; d < rank; d++) u64(shape[d]);
    } else {
        u64(shape[0]);
        u64(kind == 1 ? shape[1] : 1);
    }
    File file;
    int status = open_for(path, O_WRONLY | O_CREAT | (append ? O_APPEND : O_TRUNC), &file);
    if (status != TC_OK) return status;
    if ((status = write_all(file.fd, head.data(), head.size())) != TC_OK) return status;
    return staged_download(device_src, count * width, [&](const void* host, size_t, size_t n) -> int {
        return write_all(file.fd, host, n);
    });
}

}  // extern "C"
