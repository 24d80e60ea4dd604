// The fused-program interpreter's device side, shared by the fused kernels
// and the matrix product's program epilogue: places, the operand and output
// tables, a program small enough to travel in kernel arguments, and `run`,
// which applies one instruction to each of a thread's four elements.
//
// Arithmetic follows the host interpreter instruction by instruction
// (fused/mod.rs:62-70): one working type T per program (f32, f16 or bf16),
// loads rounded to T, each operation done in f32 and rounded to T, stores
// converted from T to the output's element type; multiply and add are
// never fused.

#pragma once

#include <math.h>

#include "common.hpp"

namespace tc {
namespace {

constexpr int kLanesPerThread = 4;

template <int T>
__device__ __forceinline__ float round_to(float v) {
    return tc_round<T>(v);
}

__device__ __forceinline__ float analytic_value(uint32_t op, float x) { return tc_analytic(op, x); }

struct Buffers {
    const void* inputs[TC_FUSED_MAX_INPUTS];
    void* outputs[TC_FUSED_MAX_OUTPUTS];
};

// A program small enough to travel in the kernel's argument segment, where
// the scalar unit reads it directly; larger ones are read from a device
// block.  Either way every instruction and place is fetched by scalar loads
// at a wave-uniform index, so the opcode, the register numbers and the
// place are SGPR values and every lane runs the same instruction.
constexpr int kInlineCode = 48;
constexpr int kInlinePlaces = 8;

// The arguments of a compiled program (an epilogue's `CompiledStore` or a
// general program's `Program`), laid out as the generated source declares
// its members.
struct CompiledArgsOf {
    const void* in[TC_FUSED_MAX_INPUTS];
    void* out[TC_FUSED_MAX_OUTPUTS];
    DevicePlace places[8];
    float constants[48];
};

static_assert(TC_FUSED_MAX_INPUTS == 16 && TC_FUSED_MAX_OUTPUTS == 8 && kInlinePlaces == 8 && kInlineCode == 48,
              "the generated members' extents");

// The generated declaration of those members.
inline const char* compiled_members() {
    return "  const void* in[16];\n  void* out[8];\n  tc::DevicePlace places[8];\n  float constants[48];\n";
}

struct Inline {
    tc_encoded code[kInlineCode];
    DevicePlace places[kInlinePlaces];
};

// The interpreter's register file: one 16-wide vector register per element
// a thread runs, indexed only by uniform register numbers, so each stays in
// VGPRs (indexed moves) rather than going to scratch memory.
typedef float Regs16 __attribute__((ext_vector_type(TC_FUSED_REGISTERS)));

struct Registers {
    Regs16 r[kLanesPerThread];
    template <int V>
    __device__ __forceinline__ float get(uint32_t i) const {
        return r[V][i];
    }
    template <int V>
    __device__ __forceinline__ void set(uint32_t i, float v) {
        r[V][i] = v;
    }
};

// The rare analytic functions, kept out of line so the interpreter's hot
// path stays small; `Sqrt`, the one Adam runs, is inline.
__device__ __noinline__ float analytic_slow(uint32_t op, float x) { return analytic_value(op, x); }

// Every element of one instruction, dispatched once on the (uniform) kind and
// operation, then applied to each of a thread's elements.
#define TC_EACH(body)                        \
    {                                        \
        constexpr int V = 0;                 \
        body;                                \
    }                                        \
    {                                        \
        constexpr int V = 1;                 \
        body;                                \
    }                                        \
    {                                        \
        constexpr int V = 2;                 \
        body;                                \
    }                                        \
    {                                        \
        constexpr int V = 3;                 \
        body;                                \
    }

// One instruction's results for a thread's four elements into `value`, or
// its stores; true when it writes register `in.dst`.  The register file is
// only read here: writing it once, after the dispatch (`run`), keeps each
// indexed write in place instead of copying the whole file in every branch.
template <int T>
__device__ __forceinline__ bool evaluate(const Registers& regs, const tc_encoded& in, const DevicePlace* place,
                                         const Buffers& buffers, const bool (&live)[kLanesPerThread],
                                         const uint64_t (&row)[kLanesPerThread],
                                         const uint64_t (&col)[kLanesPerThread],
                                         const uint64_t (&element)[kLanesPerThread], float (&value)[kLanesPerThread]) {
    static_assert(kLanesPerThread == 4, "TC_EACH covers four elements");
    switch (in.kind) {
        case 0: {  // load
            const void* src = buffers.inputs[in.a];
            TC_EACH(value[V] = live[V] ? round_to<T>(load_as(src, in.b, place_at(*place, row[V], col[V]))) : 0.0f);
            return true;
        }
        case 1:  // const: a T value, which f32 holds exactly
            TC_EACH(value[V] = in.value);
            return true;
        case 2:
            switch (in.op) {
                case TC_ADD: TC_EACH(value[V] = round_to<T>(regs.get<V>(in.a) + regs.get<V>(in.b))); break;
                case TC_SUB: TC_EACH(value[V] = round_to<T>(regs.get<V>(in.a) - regs.get<V>(in.b))); break;
                case TC_MUL: TC_EACH(value[V] = round_to<T>(regs.get<V>(in.a) * regs.get<V>(in.b))); break;
                case TC_DIV: TC_EACH(value[V] = round_to<T>(regs.get<V>(in.a) / regs.get<V>(in.b))); break;
                default: TC_EACH(value[V] = round_to<T>(fmodf(regs.get<V>(in.a), regs.get<V>(in.b)))); break;
            }
            return true;
        case 3:
            if (in.op == 13) {
                TC_EACH(value[V] = round_to<T>(sqrtf(regs.get<V>(in.a))));
            } else {
                TC_EACH(value[V] = round_to<T>(analytic_slow(in.op, regs.get<V>(in.a))));
            }
            return true;
        case 4:
            TC_EACH(value[V] = round_to<T>(compare_value(in.op, regs.get<V>(in.a), regs.get<V>(in.b))));
            return true;
        default: {  // store
            void* dst = buffers.outputs[in.aux];
            TC_EACH(if (live[V]) store_as(dst, in.b, element[V], regs.get<V>(in.a)));
            return false;
        }
    }
}

__device__ __forceinline__ void write(Registers& regs, uint32_t dst, const float (&value)[kLanesPerThread]) {
    regs.set<0>(dst, value[0]);
    regs.set<1>(dst, value[1]);
    regs.set<2>(dst, value[2]);
    regs.set<3>(dst, value[3]);
}

template <int T>
__device__ __forceinline__ void run(Registers& regs, const tc_encoded& in, const DevicePlace* place,
                                    const Buffers& buffers, const bool (&live)[kLanesPerThread],
                                    const uint64_t (&row)[kLanesPerThread], const uint64_t (&col)[kLanesPerThread],
                                    const uint64_t (&element)[kLanesPerThread]) {
    float value[kLanesPerThread];
    if (evaluate<T>(regs, in, place, buffers, live, row, col, element, value)) write(regs, in.dst, value);
}

#undef TC_EACH

// The host's places in the device form, refusing the ones no kernel walks.
inline int to_device_places(const tc_place* places, uint32_t count, DevicePlace* out) {
    for (uint32_t k = 0; k < count; k++) {
        DevicePlace& p = out[k];
        p = DevicePlace{};
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
    }
    return TC_OK;
}

}  // namespace
}  // namespace tc
