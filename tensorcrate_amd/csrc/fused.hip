// Fused elementwise programs: `Kernels::fused` (tensors/kernels.rs:1077-1082),
// the kernel an `Adam` step runs as (optim.rs:1048-1135).
//
// A program is a short register program over a rows x cols space, encoded
// twelve bytes an instruction (fused/mod.rs:1387-1410), and each element runs
// it in order.  The program and its load places are copied into LDS once per
// block; every wave then walks them in lockstep, so each instruction's
// operands are wave-uniform, and the register file is a small array indexed
// by those uniform numbers.  Each thread runs four elements 64 apart, so
// every load and store instruction of a wave touches one contiguous run.
//
// A program computes in its own type T (f32, f16 or bf16): loads convert
// their storage type to T, every operation rounds to T, and stores convert T
// to the output's storage type — the exact per-instruction arithmetic of the
// host interpreter (fused/mod.rs:62-70), since each operation computed in
// f32 and rounded once is T's own correctly rounded result.  No
// multiply-add is ever contracted.

#include <math.h>
#include <string.h>

#include "common.hpp"

namespace tc {
namespace {

constexpr int kLanesPerThread = 4;

struct DevicePlace {
    uint64_t offset;
    uint64_t col_step;
    uint32_t lead;
    uint32_t pad;
    uint64_t dims[TC_FUSED_LEAD];
    uint64_t steps[TC_FUSED_LEAD];
};

// Round an f32 value to the program's type T and back.
template <int T>
__device__ __forceinline__ float round_to(float v) {
    if (T == TC_F16) return static_cast<float>(static_cast<_Float16>(v));
    if (T == TC_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
    return v;
}

__device__ __forceinline__ float load_as(const void* base, uint32_t dtype, uint64_t index) {
    switch (dtype) {
        case TC_F16: return static_cast<float>(static_cast<const _Float16*>(base)[index]);
        case TC_BF16: return bf16_bits_to_f32(static_cast<const uint16_t*>(base)[index]);
        default: return static_cast<const float*>(base)[index];
    }
}

__device__ __forceinline__ void store_as(void* base, uint32_t dtype, uint64_t index, float v) {
    switch (dtype) {
        case TC_F16: static_cast<_Float16*>(base)[index] = static_cast<_Float16>(v); break;
        case TC_BF16: static_cast<uint16_t*>(base)[index] = f32_to_bf16_bits(v); break;
        default: static_cast<float*>(base)[index] = v; break;
    }
}

// `Analytic::value` (kernels.rs:334-354), in f32; the program rounds the
// result to T.
__device__ __forceinline__ float analytic_value(uint32_t op, float x) {
    switch (op) {
        case 0: return sinf(x);
        case 1: return cosf(x);
        case 2: return tanf(x);
        case 3: return 1.0f / cosf(x);
        case 4: return 1.0f / sinf(x);
        case 5: return asinf(x);
        case 6: return acosf(x);
        case 7: return atanf(x);
        case 8: return expf(x);
        case 9: return logf(x);
        case 10: return sinhf(x);
        case 11: return coshf(x);
        case 12: return tanhf(x);
        case 13: return sqrtf(x);
        default: return NAN;
    }
}

// The storage element element (row, col) reads through `place`
// (fused/mod.rs:3254-3268).
__device__ __forceinline__ uint64_t place_at(const DevicePlace& p, uint64_t row, uint64_t col) {
    uint64_t at = p.offset + col * p.col_step;
    if (p.lead == 1) return at + row * p.steps[0];
    if (p.lead > 1) {
        for (int k = static_cast<int>(p.lead) - 1; k > 0; k--) {
            at += (row % p.dims[k]) * p.steps[k];
            row /= p.dims[k];
        }
        at += row * p.steps[0];
    }
    return at;
}

struct Buffers {
    const void* inputs[TC_FUSED_MAX_INPUTS];
    void* outputs[TC_FUSED_MAX_OUTPUTS];
};

template <int T>
__global__ void __launch_bounds__(256) fused_kernel(const tc_encoded* __restrict__ code, uint32_t count,
                                                    const DevicePlace* __restrict__ places, uint32_t place_count,
                                                    Buffers buffers, uint64_t rows, uint64_t cols, DivMod cols_div,
                                                    bool small) {
    __shared__ tc_encoded lds_code[TC_FUSED_MAX_INSTRUCTIONS];
    __shared__ DevicePlace lds_places[TC_FUSED_MAX_LOADS];
    for (uint32_t i = threadIdx.x; i < count; i += blockDim.x) lds_code[i] = code[i];
    for (uint32_t i = threadIdx.x; i < place_count; i += blockDim.x) lds_places[i] = places[i];
    __syncthreads();

    const uint64_t total = rows * cols;
    const uint64_t per_block = static_cast<uint64_t>(blockDim.x) * kLanesPerThread;
    const int lane = threadIdx.x % 64;
    const int wave = threadIdx.x / 64;
    for (uint64_t base = static_cast<uint64_t>(blockIdx.x) * per_block; base < total;
         base += static_cast<uint64_t>(gridDim.x) * per_block) {
        // This thread's elements: four, 64 apart, within its wave's run.
        uint64_t element[kLanesPerThread], row[kLanesPerThread], col[kLanesPerThread];
        bool live[kLanesPerThread];
#pragma unroll
        for (int v = 0; v < kLanesPerThread; v++) {
            element[v] = base + wave * 64 * kLanesPerThread + v * 64 + lane;
            live[v] = element[v] < total;
            if (small) {
                const uint32_t e = static_cast<uint32_t>(element[v]);
                const uint32_t r = cols_div.div(e);
                row[v] = r;
                col[v] = e - r * static_cast<uint32_t>(cols);
            } else {
                row[v] = element[v] / cols;
                col[v] = element[v] - row[v] * cols;
            }
        }
        float r0[TC_FUSED_REGISTERS], r1[TC_FUSED_REGISTERS], r2[TC_FUSED_REGISTERS], r3[TC_FUSED_REGISTERS];
        float* regs[kLanesPerThread] = {r0, r1, r2, r3};
        for (uint32_t pc = 0; pc < count; pc++) {
            const tc_encoded in = lds_code[pc];
            switch (in.kind) {
                case 0: {  // load
                    const DevicePlace& p = lds_places[in.op];
                    const void* src = buffers.inputs[in.a];
#pragma unroll
                    for (int v = 0; v < kLanesPerThread; v++) {
                        regs[v][in.dst] = live[v] ? round_to<T>(load_as(src, in.b, place_at(p, row[v], col[v]))) : 0.0f;
                    }
                    break;
                }
                case 1:  // const: a T value, which f32 holds exactly
#pragma unroll
                    for (int v = 0; v < kLanesPerThread; v++) regs[v][in.dst] = in.value;
                    break;
                case 2:
#pragma unroll
                    for (int v = 0; v < kLanesPerThread; v++)
                        regs[v][in.dst] = round_to<T>(binary_value(in.op, regs[v][in.a], regs[v][in.b]));
                    break;
                case 3:
#pragma unroll
                    for (int v = 0; v < kLanesPerThread; v++)
                        regs[v][in.dst] = round_to<T>(analytic_value(in.op, regs[v][in.a]));
                    break;
                case 4:
#pragma unroll
                    for (int v = 0; v < kLanesPerThread; v++)
                        regs[v][in.dst] = round_to<T>(compare_value(in.op, regs[v][in.a], regs[v][in.b]));
                    break;
                default: {  // store
                    void* dst = buffers.outputs[in.aux];
#pragma unroll
                    for (int v = 0; v < kLanesPerThread; v++) {
                        if (live[v]) store_as(dst, in.b, element[v], regs[v][in.a]);
                    }
                    break;
                }
            }
        }
    }
}

// Host-side validation of what the kernel would otherwise trust.
int check_program(const tc_encoded* code, uint32_t count, uint32_t place_count, uint32_t input_count,
                  uint32_t output_count) {
    if (count > TC_FUSED_MAX_INSTRUCTIONS) return fail(TC_INVALID, "fused program: " + std::to_string(count) + " instructions, over the 256 limit");
    if (place_count > TC_FUSED_MAX_LOADS) return fail(TC_INVALID, "fused program: " + std::to_string(place_count) + " loads, over the 64 limit");
    if (input_count > TC_FUSED_MAX_INPUTS) return fail(TC_INVALID, "fused program: " + std::to_string(input_count) + " inputs, over the 16 limit");
    if (output_count > TC_FUSED_MAX_OUTPUTS) return fail(TC_INVALID, "fused program: " + std::to_string(output_count) + " outputs, over the 8 limit");
    for (uint32_t pc = 0; pc < count; pc++) {
        const tc_encoded& in = code[pc];
        const std::string at = "fused program: instruction " + std::to_string(pc);
        if (in.kind > 5) return fail(TC_INVALID, at + ": no kind " + std::to_string(in.kind));
        if (in.kind != 5 && in.dst >= TC_FUSED_REGISTERS) return fail(TC_INVALID, at + ": register out of range");
        if ((in.kind >= 2 && in.a >= TC_FUSED_REGISTERS) || ((in.kind == 2 || in.kind == 4) && in.b >= TC_FUSED_REGISTERS)) {
            return fail(TC_INVALID, at + ": register out of range");
        }
        if (in.kind == 0) {
            if (in.op >= place_count) return fail(TC_INVALID, at + ": no such load");
            if (in.a >= input_count) return fail(TC_INVALID, at + ": no such input");
            if (in.b > TC_BF16) return fail(TC_UNSUPPORTED, at + ": no kernel loads " + dtype_name(in.b));
        }
        if (in.kind == 2 && in.op > TC_REM) return fail(TC_INVALID, at + ": no BinaryOp " + std::to_string(in.op));
        if (in.kind == 3 && in.op > 13) return fail(TC_INVALID, at + ": no Analytic " + std::to_string(in.op));
        if (in.kind == 4 && in.op > TC_GREATER_EQUAL) return fail(TC_INVALID, at + ": no Compare " + std::to_string(in.op));
        if (in.kind == 5) {
            if (in.a >= TC_FUSED_REGISTERS) return fail(TC_INVALID, at + ": register out of range");
            if (in.aux >= output_count) return fail(TC_INVALID, at + ": no such output");
            if (in.b > TC_BF16) return fail(TC_UNSUPPORTED, at + ": no kernel stores " + dtype_name(in.b));
        }
    }
    return TC_OK;
}

}  // namespace
}  // namespace tc

using namespace tc;

// One past the last element `place` reads over a rows x cols space
// (`Place::end`, fused/mod.rs:3306-3319), or false on overflow.
static bool place_end(const tc_place& p, uint64_t rows, uint64_t cols, uint64_t* end) {
    uint64_t shape[TC_FUSED_LEAD + 1], strides[TC_FUSED_LEAD + 1];
    uint32_t rank = 0;
    uint64_t folded = 1;
    for (uint32_t d = 0; d < p.lead; d++, rank++) {
        shape[rank] = p.dims[d];
        strides[rank] = p.steps[d];
        folded *= p.dims[d];
    }
    if (p.lead == 0) folded = rows;  // no row axis: every row reads the same run
    if (p.lead > 0 && folded != rows) return false;
    shape[rank] = cols;
    strides[rank] = p.col_step;
    rank++;
    return reach(rank, shape, p.offset, strides, end);
}

extern "C" int tc_fused(uint32_t dtype, const tc_encoded* code, uint32_t count, const tc_place* places,
                        uint32_t place_count, const void* const* inputs, const uint64_t* input_lens,
                        uint32_t input_count, void* const* outputs, const uint64_t* output_lens,
                        uint32_t output_count, uint64_t rows, uint64_t cols) {
    int status = check_program(code, count, place_count, input_count, output_count);
    if (status != TC_OK) return status;
    if (dtype > TC_BF16) return fail(TC_UNSUPPORTED, std::string("fused program: no kernel computes in ") + dtype_name(dtype));
    TC_STREAM(s);
    if (rows == 0 || cols == 0 || count == 0) return TC_OK;
    // Every load stays inside its input and every store inside its output.
    for (uint32_t pc = 0; pc < count; pc++) {
        const tc_encoded& in = code[pc];
        if (in.kind == 0) {
            if (places[in.op].lead > TC_FUSED_LEAD) return fail(TC_INVALID, "fused program: a place folds more than 5 axes");
            uint64_t end = 0;
            if (!place_end(places[in.op], rows, cols, &end) || end > input_lens[in.a]) {
                return fail(TC_INVALID, "fused program: load " + std::to_string(in.op) + " reaches past input " +
                                            std::to_string(in.a) + "'s " + std::to_string(input_lens[in.a]) +
                                            " elements");
            }
        } else if (in.kind == 5 && output_lens[in.aux] < rows * cols) {
            return fail(TC_INVALID, "fused program: output " + std::to_string(in.aux) + " holds " +
                                        std::to_string(output_lens[in.aux]) + " elements, not " +
                                        std::to_string(rows * cols));
        }
    }
    // The program and its places travel in one block of device memory,
    // freed once the kernel has been queued (stream order keeps it alive).
    const size_t code_bytes = (count * sizeof(tc_encoded) + 15) / 16 * 16;
    const size_t place_bytes = place_count * sizeof(DevicePlace);
    std::vector<uint8_t> host(code_bytes + place_bytes);
    memcpy(host.data(), code, count * sizeof(tc_encoded));
    for (uint32_t k = 0; k < place_count; k++) {
        DevicePlace p{};
        p.offset = places[k].offset;
        p.col_step = places[k].col_step;
        p.lead = places[k].lead;
        if (p.lead > TC_FUSED_LEAD) return fail(TC_INVALID, "fused program: a place folds more than 5 axes");
        for (int d = 0; d < TC_FUSED_LEAD; d++) {
            p.dims[d] = places[k].dims[d];
            p.steps[d] = places[k].steps[d];
            if (d < static_cast<int>(p.lead) && p.dims[d] == 0) {
                return fail(TC_INVALID, "fused program: a place has an empty axis");
            }
        }
        memcpy(host.data() + code_bytes + k * sizeof(DevicePlace), &p, sizeof(DevicePlace));
    }
    void* device = nullptr;
    status = tc_alloc(host.size(), &device);
    if (status != TC_OK) return status;
    hipError_t error = hipMemcpyAsync(device, host.data(), host.size(), hipMemcpyHostToDevice, s);
    if (error != hipSuccess) {
        tc_free(device);
        return fail(TC_DEVICE, std::string("fused program upload: ") + hipGetErrorString(error));
    }
    Buffers buffers{};
    for (uint32_t k = 0; k < input_count; k++) buffers.inputs[k] = inputs[k];
    for (uint32_t k = 0; k < output_count; k++) buffers.outputs[k] = outputs[k];
    const uint64_t total = rows * cols;
    const bool small = total <= UINT32_MAX && cols <= UINT32_MAX;
    DivMod cols_div(small ? static_cast<uint32_t>(cols) : 1u);
    const uint32_t blocks = grid_for(total, 256 * kLanesPerThread, 8);
    const tc_encoded* dcode = static_cast<const tc_encoded*>(device);
    const DevicePlace* dplaces = reinterpret_cast<const DevicePlace*>(static_cast<uint8_t*>(device) + code_bytes);
    switch (dtype) {
        case TC_F32: fused_kernel<TC_F32><<<blocks, 256, 0, s>>>(dcode, count, dplaces, place_count, buffers, rows, cols, cols_div, small); break;
        case TC_F16: fused_kernel<TC_F16><<<blocks, 256, 0, s>>>(dcode, count, dplaces, place_count, buffers, rows, cols, cols_div, small); break;
        default: fused_kernel<TC_BF16><<<blocks, 256, 0, s>>>(dcode, count, dplaces, place_count, buffers, rows, cols, cols_div, small); break;
    }
    status = check_launch("fused program");
    tc_free(device);
    return status;
}
