// Fused elementwise programs: `Kernels::fused` (tensors/kernels.rs:1077-1082),
// the kernel an `Adam` step runs as (optim.rs:1048-1135).
//
// A program is a short register program over a rows x cols space, encoded
// twelve bytes an instruction (fused/mod.rs:1387-1410), and each element runs
// it in order.  Every wave walks the program in lockstep, fetching each
// instruction and load place with scalar loads (from the kernel's argument
// segment for programs of up to 48 instructions, such as Adam's, from a
// device block otherwise), so the opcode and register numbers are SGPRs,
// each instruction is dispatched once per wave, and the register file — one
// 16-wide vector per element — is indexed with indexed VGPR moves, never
// scratch memory.  Each thread runs four elements 64 apart, so every load
// and store instruction of a wave touches one contiguous run.
//
// Arithmetic follows the host interpreter instruction by instruction
// (fused/mod.rs:62-70): a program has one working type T (f32, f16 or bf16);
// every load widens its storage element and rounds it to T, every operation
// is done in f32 and rounded to T once — which is T's correctly rounded
// result — and every store converts from T to the output's element type.
// Multiply and add are never fused.

#include <dlfcn.h>
#include <hip/hiprtc.h>
#include <limits.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>
#include <sstream>
#include <unordered_map>
#include <utility>

#include "common.hpp"
#include "program.hpp"

namespace tc {
namespace {

template <int T, bool INLINE>
__global__ void __launch_bounds__(256) fused_kernel(Inline small_program, const tc_encoded* __restrict__ code,
                                                    const DevicePlace* __restrict__ places, uint32_t count,
                                                    Buffers buffers, uint64_t rows, uint64_t cols, DivMod cols_div,
                                                    bool small) {
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
        Registers regs;
        for (uint32_t pc = 0; pc < count; pc++) {
            const tc_encoded in = INLINE ? small_program.code[pc] : code[pc];
            const DevicePlace* place = nullptr;
            if (in.kind == 0) place = INLINE ? &small_program.places[in.op] : &places[in.op];
            run<T>(regs, in, place, buffers, live, row, col, element);
        }
    }
}

// ---- the dense path ------------------------------------------------------
//
// A program whose every load reads its tensor in element order and whose
// loads all come before its stores — a whole-tensor update such as Adam —
// runs four consecutive elements per thread: all of a chunk's loads are
// issued first, as one 16-byte (f32) or 8-byte (16-bit) vector load each, so
// every thread has its whole working set in flight at once, and each store
// writes its four elements with one vector store.  Load instruction j of the
// program reads staging slot j.

constexpr int kDenseLoads = 8;
typedef float Stage __attribute__((ext_vector_type(4 * kDenseLoads)));

struct DenseLoads {
    const void* base[kDenseLoads];  // the input with the place's offset applied
    uint32_t dtype[kDenseLoads];
};

__device__ __forceinline__ void load4(const void* base, uint32_t dtype, uint64_t first, float (&out)[4]) {
    if (dtype == TC_F32) {
        const float4 v = reinterpret_cast<const float4*>(base)[first / 4];
        out[0] = v.x, out[1] = v.y, out[2] = v.z, out[3] = v.w;
    } else {
        const uint2 v = reinterpret_cast<const uint2*>(base)[first / 4];
        const uint16_t h[4] = {static_cast<uint16_t>(v.x), static_cast<uint16_t>(v.x >> 16),
                               static_cast<uint16_t>(v.y), static_cast<uint16_t>(v.y >> 16)};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            out[e] = dtype == TC_F16 ? static_cast<float>(__builtin_bit_cast(_Float16, h[e])) : bf16_bits_to_f32(h[e]);
        }
    }
}

__device__ __forceinline__ void store4(void* base, uint32_t dtype, uint64_t first, const float (&v)[4]) {
    if (dtype == TC_F32) {
        reinterpret_cast<float4*>(base)[first / 4] = make_float4(v[0], v[1], v[2], v[3]);
    } else {
        uint16_t h[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            h[e] = dtype == TC_F16 ? __builtin_bit_cast(uint16_t, static_cast<_Float16>(v[e])) : f32_to_bf16_bits(v[e]);
        }
        reinterpret_cast<uint2*>(base)[first / 4] =
            make_uint2(h[0] | (static_cast<uint32_t>(h[1]) << 16), h[2] | (static_cast<uint32_t>(h[3]) << 16));
    }
}

template <int T>
__global__ void __launch_bounds__(256) fused_dense_kernel(Inline program, uint32_t count, DenseLoads loads,
                                                          uint32_t load_count, Buffers buffers, uint64_t chunks) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t chunk = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; chunk < chunks;
         chunk += stride) {
        const uint64_t first = chunk * 4;
        Stage stage;
        for (uint32_t j = 0; j < load_count; j++) {
            float v[4];
            load4(loads.base[j], loads.dtype[j], first, v);
#pragma unroll
            for (int e = 0; e < 4; e++) stage[4 * j + e] = v[e];
        }
        Registers regs;
        uint32_t next_load = 0;
        for (uint32_t pc = 0; pc < count; pc++) {
            const tc_encoded in = program.code[pc];
            if (in.kind == 0) {
                const uint32_t j = next_load++;
                regs.set<0>(in.dst, round_to<T>(stage[4 * j + 0]));
                regs.set<1>(in.dst, round_to<T>(stage[4 * j + 1]));
                regs.set<2>(in.dst, round_to<T>(stage[4 * j + 2]));
                regs.set<3>(in.dst, round_to<T>(stage[4 * j + 3]));
            } else if (in.kind == 5) {
                const float v[4] = {regs.get<0>(in.a), regs.get<1>(in.a), regs.get<2>(in.a), regs.get<3>(in.a)};
                store4(buffers.outputs[in.aux], in.b, first, v);
            } else {
                const bool live[4] = {true, true, true, true};
                const uint64_t none[4] = {0, 0, 0, 0};
                run<T>(regs, in, nullptr, buffers, live, none, none, none);
            }
        }
    }
}

// Whether `code` runs on the dense path over a rows x cols space, and if so
// the staging it reads.
bool dense_plan(const tc_encoded* code, uint32_t count, const tc_place* places, const void* const* inputs,
                void* const* outputs, uint64_t rows, uint64_t cols, DenseLoads* plan, uint32_t* load_count) {
    if (count > static_cast<uint32_t>(kInlineCode) || (rows * cols) % 4 != 0) return false;
    uint32_t loads = 0;
    bool stored = false;
    for (uint32_t pc = 0; pc < count; pc++) {
        const tc_encoded& in = code[pc];
        const size_t size = in.b == TC_F32 ? 4 : 2;
        if (in.kind == 0) {
            if (stored || loads == static_cast<uint32_t>(kDenseLoads)) return false;
            const tc_place& p = places[in.op];
            // Element order: (row, col) reads offset + row * cols + col.
            const bool in_order = p.col_step == 1 && (rows == 1 || (p.lead == 1 && p.steps[0] == cols));
            const uint8_t* base = static_cast<const uint8_t*>(inputs[in.a]) + p.offset * size;
            if (!in_order || reinterpret_cast<uintptr_t>(base) % (4 * size) != 0) return false;
            plan->base[loads] = base;
            plan->dtype[loads] = in.b;
            loads++;
        } else if (in.kind == 5) {
            stored = true;
            if (reinterpret_cast<uintptr_t>(outputs[in.aux]) % (4 * size) != 0) return false;
        }
    }
    *load_count = loads;
    return true;
}

// ---- compiled programs -----------------------------------------------------
//
// Specialisation (the reference's Metal backend does the same for its fused
// programs, metal/codegen.rs:1-40): the second time a dense program is seen,
// it is turned into HIP source with no interpreter loop left — each value a
// local variable, each opcode and storage type a literal the compiler can
// fold — built with hiprtc and this library's code-generation flags, and
// launched instead of the interpreter from then on.  The generated code
// calls scalar_ops.h, the functions the interpreter uses, so both give the
// same bits.  Literal constants are passed as kernel arguments rather than
// written into the source, which lets a program rebuilt each step with new
// constants (an optimizer's) reuse its kernel; kernels are kept, keyed by
// source, until the process ends.  A program seen only once is never
// compiled, so a one-off never waits for the compiler.

// The headers hiprtc reads, embedded by the build.
extern "C" const char tc_scalar_ops_source[];
extern "C" const char tc_device_source[];
extern "C" const char tc_gemm_kernels_source[];

constexpr int kCompiledConstants = kInlineCode;

struct CompiledArgs {
    const void* in[kDenseLoads];
    void* out[TC_FUSED_MAX_OUTPUTS];
    float constants[kCompiledConstants];
    uint64_t chunks;
};

// Bytes one chunk (four elements) of a dense program loads and stores.
uint64_t dense_chunk_bytes(const tc_encoded* code, uint32_t count) {
    uint64_t bytes = 0;
    for (uint32_t pc = 0; pc < count; pc++) {
        if (code[pc].kind == 0 || code[pc].kind == 5) bytes += code[pc].b == TC_F32 ? 16 : 8;
    }
    return bytes;
}

// The generated source of a dense program, and the order its constants
// take in `CompiledArgs::constants`.  A streaming program (one whose traffic
// exceeds the Infinity Cache) loads with nontemporal hints and stores
// plainly (the Adam update over 25 M f32 parameters: 6.06 -> 6.64 TB/s
// against nontemporal stores).
std::string dense_source(const tc_encoded* code, uint32_t count, uint32_t dtype, bool stream,
                         std::vector<float>* constants) {
    static const char* const kRound[] = {"tc_round<0>", "tc_round<1>", "tc_round<2>"};
    static const char* const kBinary[] = {"+", "-", "*", "/"};
    const char* round = kRound[dtype];
    std::ostringstream src;
    src << "#include \"scalar_ops.h\"\n"
        << "typedef float tc_f4 __attribute__((ext_vector_type(4)));\n"
        << "typedef unsigned tc_u2 __attribute__((ext_vector_type(2)));\n"
        << (stream ? "#define TC_LD(p) __builtin_nontemporal_load(p)\n#define TC_ST(v, p) (*(p) = (v))\n"
                   : "#define TC_LD(p) (*(p))\n#define TC_ST(v, p) (*(p) = (v))\n")
        << "struct Args { const void* in[" << kDenseLoads << "]; void* out[" << TC_FUSED_MAX_OUTPUTS
        << "]; float constants[" << kCompiledConstants << "]; unsigned long long chunks; };\n"
        << "extern \"C\" __global__ void __launch_bounds__(256) tc_fused_program(Args a) {\n"
        << "  const unsigned long long stride = (unsigned long long)gridDim.x * blockDim.x;\n"
        << "  for (unsigned long long chunk = (unsigned long long)blockIdx.x * blockDim.x + threadIdx.x;"
        << " chunk < a.chunks; chunk += stride) {\n";
    std::string reg[TC_FUSED_REGISTERS];
    uint32_t loads = 0;
    for (uint32_t pc = 0; pc < count; pc++) {
        const tc_encoded& in = code[pc];
        const std::string v = "v" + std::to_string(pc);
        auto at = [&](uint8_t r) { return reg[r].empty() ? std::string("0.0f") : reg[r] + "[e]"; };
        if (in.kind == 5) {
            const std::string value = reg[in.a].empty() ? "zero" : reg[in.a];
            if (reg[in.a].empty()) src << "    const float zero[4] = {0.0f, 0.0f, 0.0f, 0.0f};\n";
            if (in.b == TC_F32) {
                src << "    TC_ST(((tc_f4){" << value << "[0], " << value << "[1], " << value << "[2], " << value
                    << "[3]}), (tc_f4*)a.out[" << int(in.aux) << "] + chunk);\n";
            } else {
                const std::string narrow = in.b == TC_F16 ? "__builtin_bit_cast(unsigned short, (_Float16)(" : "tc_f32_to_bf16((";
                src << "    { unsigned short h[4]; for (int e = 0; e < 4; e++) h[e] = " << narrow << value << "[e]));\n"
                    << "      TC_ST(((tc_u2){h[0] | ((unsigned)h[1] << 16), h[2] | ((unsigned)h[3] << 16)}), (tc_u2*)a.out["
                    << int(in.aux) << "] + chunk); }\n";
            }
            continue;
        }
        src << "    float " << v << "[4];\n";
        switch (in.kind) {
            case 0: {
                const uint32_t j = loads++;
                if (in.b == TC_F32) {
                    src << "    { const tc_f4 w = TC_LD((const tc_f4*)a.in[" << j << "] + chunk); " << v << "[0] = " << round
                        << "(w.x); " << v << "[1] = " << round << "(w.y); " << v << "[2] = " << round << "(w.z); " << v
                        << "[3] = " << round << "(w.w); }\n";
                } else {
                    const std::string widen = in.b == TC_F16 ? "(float)__builtin_bit_cast(_Float16, (unsigned short)(" : "tc_bf16_to_f32((unsigned short)(";
                    src << "    { const tc_u2 w = TC_LD((const tc_u2*)a.in[" << j << "] + chunk);\n"
                        << "      const unsigned hw[4] = {w.x & 0xffffu, w.x >> 16, w.y & 0xffffu, w.y >> 16};\n"
                        << "      for (int e = 0; e < 4; e++) " << v << "[e] = " << round << "(" << widen << "hw[e]))); }\n";
                }
                break;
            }
            case 1: {
                src << "    for (int e = 0; e < 4; e++) " << v << "[e] = a.constants[" << constants->size() << "];\n";
                constants->push_back(in.value);
                break;
            }
            case 2:
                if (in.op == TC_REM) {
                    src << "    for (int e = 0; e < 4; e++) " << v << "[e] = " << round << "(fmodf(" << at(in.a) << ", "
                        << at(in.b) << "));\n";
                } else {
                    src << "    for (int e = 0; e < 4; e++) " << v << "[e] = " << round << "(" << at(in.a) << " "
                        << kBinary[in.op] << " " << at(in.b) << ");\n";
                }
                break;
            case 3:
                src << "    for (int e = 0; e < 4; e++) " << v << "[e] = " << round << "(tc_analytic(" << in.op << "u, "
                    << at(in.a) << "));\n";
                break;
            default:  // compare
                src << "    for (int e = 0; e < 4; e++) " << v << "[e] = " << round << "(tc_compare(" << in.op << "u, "
                    << at(in.a) << ", " << at(in.b) << "));\n";
                break;
        }
        reg[in.dst] = v;
    }
    src << "  }\n}\n";
    return src.str();
}

struct Compiled {
    uint32_t seen = 0;
    bool failed = false;
    hipModule_t module = nullptr;
    std::vector<hipFunction_t> functions;
    // Each function's resources, from the compiler's resource report.
    std::vector<KernelResources> resources;
    // The code object the module was loaded from.  The loader reports this
    // buffer to tools (profilers, debuggers) as the loaded code object's
    // storage and they read it back while the module lives, so it lives as
    // long as the module: for the process, as cached modules are never
    // unloaded.
    std::vector<char> image;
};

// Programs too large for kernel arguments, resident on the device for the
// process by their bytes (the host copy is kept beside each, the source of
// its one upload), up to `resident_limit` of them.  A program first seen
// while the stream is being captured is refused: its upload would be a node
// of the graph reading host memory.  Past the limit, an uncaptured run
// uploads its program into a stream-ordered block of its own, freed once the
// kernel is queued (`transient_program`), so a stream of distinct programs
// (new shapes, offsets or constants each call) keeps running and holds no
// device memory beyond the limit's.
struct ResidentProgram {
    std::string host;
    void* device = nullptr;
};
std::mutex resident_mutex;
std::unordered_map<std::string, ResidentProgram> resident_programs;
size_t resident_limit = 4096;

// Host copies of transient uploads, each kept until the event recorded
// after its copy has passed: the copy reads host memory when the stream
// reaches it, not when it is queued.  Never destroyed (the process's end
// releases it), so no thread's exit races another's upload.
struct PendingUpload {
    hipEvent_t done;
    std::string host;
};
std::vector<PendingUpload>* pending_uploads = new std::vector<PendingUpload>();

void release_finished_uploads() {
    auto& pending = *pending_uploads;
    size_t kept = 0;
    for (size_t i = 0; i < pending.size(); i++) {
        const hipError_t state = hipEventQuery(pending[i].done);
        if (state == hipSuccess) {
            (void)hipEventDestroy(pending[i].done);
            continue;
        }
        if (state != hipErrorNotReady) (void)hipGetLastError();
        if (kept != i) pending[kept] = std::move(pending[i]);
        kept++;
    }
    pending.resize(kept);
}

// `key` uploaded into a block from the thread's stream-ordered cache, which
// the caller frees with `tc_free` once its kernel is queued.
int transient_program(const std::string& key, hipStream_t s, void** device) {
    release_finished_uploads();
    int status = tc_alloc(key.size(), device);
    if (status != TC_OK) return status;
    PendingUpload upload{nullptr, key};
    hipError_t error = hipEventCreateWithFlags(&upload.done, hipEventDisableTiming);
    if (error == hipSuccess) {
        count_dispatch();
        error = hipMemcpyAsync(*device, upload.host.data(), key.size(), hipMemcpyHostToDevice, s);
        if (error == hipSuccess) error = hipEventRecord(upload.done, s);
    }
    if (error != hipSuccess) {
        (void)hipGetLastError();
        if (upload.done != nullptr) {
            // The copy may have been queued before the record failed: wait
            // for the stream before the host copy goes.
            (void)hipStreamSynchronize(s);
            (void)hipEventDestroy(upload.done);
        }
        tc_free(*device);
        *device = nullptr;
        return fail(TC_DEVICE, std::string("fused program upload: ") + hipGetErrorString(error));
    }
    pending_uploads->push_back(std::move(upload));
    return TC_OK;
}

// The device copy of a large program: resident (`*transient` false) or, past
// the limit, a transient block the caller frees after its launch.
int resident_program(const std::string& key, hipStream_t s, void** device, bool* transient) {
    std::lock_guard<std::mutex> lock(resident_mutex);
    *transient = false;
    auto found = resident_programs.find(key);
    if (found != resident_programs.end()) {
        *device = found->second.device;
        return TC_OK;
    }
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &capture) != hipSuccess) (void)hipGetLastError();
    if (capture != hipStreamCaptureStatusNone) {
        return fail(TC_UNSUPPORTED, "fused program: a program of more than " + std::to_string(kInlineCode) +
                                        " instructions or " + std::to_string(kInlinePlaces) +
                                        " places must run once before it is captured");
    }
    if (resident_programs.size() >= resident_limit) {
        *transient = true;
        return transient_program(key, s, device);
    }
    ResidentProgram entry;
    entry.host = key;
    hipError_t error = hipMalloc(&entry.device, key.size());
    if (error != hipSuccess) {
        (void)hipGetLastError();
        return fail(TC_OUT_OF_MEMORY, std::string("fused program upload: ") + hipGetErrorString(error));
    }
    count_dispatch();
    auto placed = resident_programs.emplace(key, std::move(entry)).first;
    error = hipMemcpyAsync(placed->second.device, placed->second.host.data(), key.size(), hipMemcpyHostToDevice, s);
    if (error != hipSuccess) {
        (void)hipGetLastError();
        // The entry never held the program: drop it, so a later run of the
        // same program uploads again rather than reading unwritten memory.
        // The copy failed to queue, so nothing on the device reads the block.
        (void)hipFree(placed->second.device);
        resident_programs.erase(placed);
        return fail(TC_DEVICE, std::string("fused program upload: ") + hipGetErrorString(error));
    }
    *device = placed->second.device;
    return TC_OK;
}

std::mutex compiled_mutex;
std::unordered_map<std::string, Compiled> compiled_programs;
uint64_t compiled_count = 0;

// hiprtc's flags: the library's own (see _build.py), and the compiler's
// per-function resource report into the compile log, where each kernel's
// scratch and register use is read (`resources_by_function`).
const char* const kCompileFlags[] = {"--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
                                     "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                                     "-Rpass-analysis=kernel-resource-usage"};

// The resources each function of a compile log uses: the log's resource
// remarks name a function ("Function Name: <mangled>") and then report,
// among others, its "VGPRs: <n>" (indented, unlike "TotalSGPRs" and
// "VGPRs Spill") and "ScratchSize [bytes/lane]: <n>".
std::unordered_map<std::string, KernelResources> resources_by_function(const std::string& log) {
    std::unordered_map<std::string, KernelResources> out;
    static const std::string kName = "remark: Function Name: ", kScratch = "ScratchSize [bytes/lane]: ",
                             kVgprs = " VGPRs: ";
    std::string current;
    size_t at = 0;
    while (at < log.size()) {
        size_t end = log.find('\n', at);
        if (end == std::string::npos) end = log.size();
        const std::string line = log.substr(at, end - at);
        size_t found = line.find(kName);
        if (found != std::string::npos) {
            const size_t first = found + kName.size();
            current = line.substr(first, line.find(' ', first) - first);
        } else if (!current.empty() && (found = line.find(kScratch)) != std::string::npos) {
            out[current].scratch = static_cast<uint32_t>(strtoul(line.c_str() + found + kScratch.size(), nullptr, 10));
        } else if (!current.empty() && (found = line.find(kVgprs)) != std::string::npos) {
            out[current].vgprs = static_cast<uint32_t>(strtoul(line.c_str() + found + kVgprs.size(), nullptr, 10));
        }
        at = end + 1;
    }
    return out;
}

// Compile `source` with the embedded headers and look up `kernels`, each an
// extern "C" name or a template-id whose lowered name hiprtc reports.
bool compile_program(const std::string& source, const std::vector<std::string>& kernels, Compiled* out) {
    hiprtcProgram program;
    const char* headers[] = {tc_scalar_ops_source, tc_device_source, tc_gemm_kernels_source};
    const char* names[] = {"scalar_ops.h", "device.hpp", "gemm_kernels.hpp"};
    if (hiprtcCreateProgram(&program, source.c_str(), "tc_fused_program.hip", 3, headers, names) != HIPRTC_SUCCESS) {
        return false;
    }
    for (const std::string& kernel : kernels) {
        if (kernel.find('<') != std::string::npos) (void)hiprtcAddNameExpression(program, kernel.c_str());
    }
    bool ok = hiprtcCompileProgram(program, sizeof(kCompileFlags) / sizeof(kCompileFlags[0]), kCompileFlags) ==
              HIPRTC_SUCCESS;
    std::vector<char> binary;
    std::vector<std::string> lowered;
    std::unordered_map<std::string, KernelResources> resources;
    if (ok) {
        size_t log_size = 0;
        if (hiprtcGetProgramLogSize(program, &log_size) == HIPRTC_SUCCESS && log_size > 0) {
            std::string log(log_size, '\0');
            if (hiprtcGetProgramLog(program, &log[0]) == HIPRTC_SUCCESS) resources = resources_by_function(log);
        }
        size_t size = 0;
        ok = hiprtcGetCodeSize(program, &size) == HIPRTC_SUCCESS && size > 0;
        if (ok) {
            binary.resize(size);
            ok = hiprtcGetCode(program, binary.data()) == HIPRTC_SUCCESS;
        }
        for (const std::string& kernel : kernels) {
            const char* name = kernel.c_str();
            if (ok && kernel.find('<') != std::string::npos) {
                ok = hiprtcGetLoweredName(program, kernel.c_str(), &name) == HIPRTC_SUCCESS;
            }
            lowered.push_back(ok ? std::string(name) : std::string());
        }
    }
    hiprtcDestroyProgram(&program);
    if (!ok) return false;
    out->image = std::move(binary);
    if (hipModuleLoadData(&out->module, out->image.data()) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    for (const std::string& name : lowered) {
        hipFunction_t function = nullptr;
        if (hipModuleGetFunction(&function, out->module, name.c_str()) != hipSuccess) {
            (void)hipGetLastError();
            return false;
        }
        out->functions.push_back(function);
        const auto known = resources.find(name);
        out->resources.push_back(known == resources.end() ? KernelResources{} : known->second);
    }
    return true;
}

// The cached kernels of `source` for this device, compiled on the source's
// second request; false (run something else) before that or if it does not
// compile.
bool cached_kernels(const std::string& source, const std::vector<std::string>& kernels, hipFunction_t* out,
                    KernelResources* resources = nullptr) {
    int device = 0;
    (void)hipGetDevice(&device);
    std::lock_guard<std::mutex> lock(compiled_mutex);
    Compiled& entry = compiled_programs["device " + std::to_string(device) + "\n" + source];
    if (entry.failed) return false;
    if (entry.functions.empty()) {
        if (++entry.seen < 2) return false;
        if (!compile_program(source, kernels, &entry)) {
            entry.failed = true;
            return false;
        }
        compiled_count++;
    }
    for (size_t k = 0; k < entry.functions.size(); k++) {
        out[k] = entry.functions[k];
        if (resources != nullptr) resources[k] = entry.resources[k];
    }
    return true;
}

// The straight-line form of a program over `elems` of a thread's elements:
// the body of an epilogue's `group(live, row, col, N, product)`, each
// value a local, each load through `places[j]` of the epilogue's arguments,
// each constant from `constants[]` (appended to `*constants`).  With
// `product_input`, input 0 is the product rather than a load.
// The element index of `place` (the device copy named `p`) at row `r`,
// column `c`: column steps of 0 and 1 and a row step of 0, the usual
// broadcast and contiguous places, are written without their multiply, so
// the kernel's source (and its cache key) carries them.
std::string place_index(const tc_place& place, const std::string& p, const std::string& r, const std::string& c) {
    if (place.lead > 1) return "tc::place_at(" + p + ", " + r + ", " + c + ")";
    std::string index = p + ".offset";
    if (place.col_step == 1) {
        index += " + (uint64_t)" + c;
    } else if (place.col_step != 0) {
        index += " + (uint64_t)" + c + " * " + p + ".col_step";
    }
    if (place.lead == 1 && place.steps[0] != 0) index += " + (uint64_t)" + r + " * " + p + ".steps[0]";
    return index;
}

// Whether `value` is a value of `dtype` (rounding it to the type changes no
// bit): every f32 is; for the 16-bit types, on the host's conversions.
bool holds_exactly(uint32_t dtype, float value) {
    uint32_t bits = 0, back = 0;
    memcpy(&bits, &value, 4);
    if (dtype == TC_BF16) {
        back = static_cast<uint32_t>(tc_f32_to_bf16(value)) << 16;
    } else if (dtype == TC_F16) {
        const float wide = static_cast<float>(static_cast<_Float16>(value));
        memcpy(&back, &wide, 4);
    } else {
        return true;
    }
    return bits == back;
}

// `held`, when given, marks the loads (by instruction index) whose values
// the kernel already holds, rounded to the program's type: they read
// `held[e]` instead of memory.  `runs`, when given, marks the loads and
// stores that may move the group as one run: the kernel calls the group
// with elements that are consecutive columns of one row, all live or none,
// and these instructions' pieces are aligned (load_run / store_run; with
// `wide`, 16-byte pieces, load_wide / store_wide; with `stream` the stores
// and the loads of places that walk rows are non-temporal).
// `invariant`, when given, marks loads whose run is the same for every row
// of the kernel's runs: they read `inv.i<pc>[e]`, loaded before the runs.
std::string group_body(const tc_encoded* code, uint32_t count, uint32_t dtype, bool product_input, int elems,
                       const tc_place* places, std::vector<float>* constants, bool sum_store = false,
                       int stat_first = -1, const std::vector<bool>* held = nullptr,
                       const std::vector<bool>* runs = nullptr, const std::vector<bool>* invariant = nullptr,
                       bool wide = false, bool stream = false, bool sum_each = false) {
    static const char* const kBinary[] = {"+", "-", "*", "/"};
    const std::string round_run = "    tc_round_run<" + std::to_string(dtype) + ">(";
    std::ostringstream src;
    std::string reg[TC_FUSED_REGISTERS];
    // Whether a register's every element is already a value of the type
    // (rounding it again changes no bit): what a rounding wrote, a constant
    // the type holds exactly, a predicate's 0, 1/2 or 1.  An unwritten
    // register reads 0.
    bool exact[TC_FUSED_REGISTERS];
    for (bool& e : exact) e = true;
    // Whether a register holds the same value for every element of a group
    // (a function of constants and the row's statistics, whose groups lie
    // in one row): a division by such a value takes tc::div_uniform.
    bool uniform[TC_FUSED_REGISTERS];
    for (bool& u : uniform) u = true;
    auto at = [&](uint8_t r) { return reg[r].empty() ? std::string("0.0f") : reg[r] + "[e]"; };
    const std::string each = "    for (int e = 0; e < " + std::to_string(elems) + "; e++) ";
    for (uint32_t pc = 0; pc < count; pc++) {
        const tc_encoded& in = code[pc];
        if (in.kind == 5) {
            if (sum_store && sum_each) {  // each element's own running sum, in f32
                src << each << "sum[e] += live[e] ? " << at(in.a) << " : 0.0f;\n";
            } else if (sum_store) {  // the one output, already in its type, summed in f32 in element order
                src << each << "sum += live[e] ? " << at(in.a) << " : 0.0f;\n";
            } else if (runs != nullptr && (*runs)[pc] && !reg[in.a].empty()) {
                src << "    if (live[0]) tc::" << (wide ? "store_wide<" : "store_run<") << elems
                    << (stream ? ", true" : ", false") << ">(out[" << int(in.aux) << "], " << int(in.b)
                    << "u, (uint64_t)row[0] * N + col[0], " << reg[in.a] << ");\n";
            } else {
                src << each << "if (live[e]) tc::store_as(out[" << int(in.aux) << "], " << int(in.b)
                    << "u, (uint64_t)row[e] * N + col[e], " << at(in.a) << ");\n";
            }
            continue;
        }
        const std::string v = "v" + std::to_string(pc);
        // Each value is computed in f32 and the array then rounded to the
        // type (tc_round_run, as tc_round rounds one value) unless `rounded`
        // is left false because the rounding could change no bit.
        bool rounded = true;
        bool same = true;  // the value is uniform, as defined above
        switch (in.kind) {
            case 0: same = stat_first >= 0 && in.a >= stat_first; break;
            case 1: break;
            case 3: same = uniform[in.a]; break;
            default: same = uniform[in.a] && uniform[in.b]; break;
        }
        if (in.kind == 2 && in.op == TC_DIV && uniform[in.b] && !same && !reg[in.a].empty()) {
            src << "    float " << v << "[" << elems << "];\n    tc::div_uniform<" << elems << ">(" << v << ", "
                << reg[in.a] << ", " << (reg[in.b].empty() ? std::string("0.0f") : reg[in.b] + "[0]") << ");\n"
                << round_run << v << ");\n";
            reg[in.dst] = v;
            exact[in.dst] = true;
            uniform[in.dst] = false;
            continue;
        }
        src << "    float " << v << "[" << elems << "];\n" << each << v << "[e] = ";
        switch (in.kind) {
            case 0:
                if (product_input && in.a == 0) {
                    src << "live[e] ? product[e] : 0.0f;\n";
                } else if (stat_first >= 0 && in.a >= stat_first) {
                    // A row statistic, one value a row, already in the type.
                    src << "stat[" << (in.a - stat_first) << "];\n";
                    rounded = false;
                } else if (held != nullptr && (*held)[pc]) {
                    src << "held[e];\n";
                    rounded = false;
                } else if (invariant != nullptr && (*invariant)[pc]) {
                    src << "inv.i" << pc << "[e];\n";
                    rounded = false;
                } else if (runs != nullptr && (*runs)[pc]) {
                    // The run from its first element's index, loaded only
                    // when live; in a streaming program, a place that walks
                    // rows is read once and its loads are non-temporal (a
                    // run every row reads stays cached).
                    const std::string p = "places[" + std::to_string(in.op) + "]";
                    const tc_place& lp = places[in.op];
                    const bool walks_rows = lp.lead > 1 || (lp.lead == 1 && lp.steps[0] != 0);
                    src << "0.0f;\n    if (live[0]) tc::" << (wide ? "load_wide<" : "load_run<") << elems
                        << (stream && walks_rows ? ", true" : "") << ">(in[" << int(in.a) << "], " << int(in.b)
                        << "u, " << place_index(lp, p, "row[0]", "col[0]") << ", " << v << ");\n";
                } else {
                    // Every lane loads, an element outside C at (0, 0), so
                    // no load waits on a branch; the place's row walk is
                    // written out for the usual one or no folded axes.
                    const std::string p = "places[" + std::to_string(in.op) + "]";
                    const std::string r = "(live[e] ? row[e] : 0u)", c = "(live[e] ? col[e] : 0u)";
                    std::string index = place_index(places[in.op], p, r, c);
                    src << "live[e] ? tc::load_as(in[" << int(in.a) << "], " << int(in.b) << "u, " << index
                        << ") : 0.0f;\n";
                }
                break;
            case 1:
                // Constants are used as given; one the type holds exactly
                // counts as rounded.
                src << "constants[" << constants->size() << "];\n";
                constants->push_back(in.value);
                rounded = false;
                exact[in.dst] = holds_exactly(dtype, in.value);
                break;
            case 2:
                if (in.op == TC_REM) {
                    src << "fmodf(" << at(in.a) << ", " << at(in.b) << ");\n";
                } else {
                    src << at(in.a) << " " << kBinary[in.op] << " " << at(in.b) << ";\n";
                }
                break;
            case 3:
                src << "tc_analytic(" << int(in.op) << "u, " << at(in.a) << ");\n";
                break;
            default:
                src << "tc_compare(" << int(in.op) << "u, " << at(in.a) << ", " << at(in.b) << ");\n";
                // A predicate is 0, 1/2 or 1; the minimum or maximum of two
                // values of the type is one of them (or a quiet NaN the type
                // holds).
                rounded = (in.op == TC_MIN || in.op == TC_MAX) && !(exact[in.a] && exact[in.b]);
                break;
        }
        if (rounded) src << round_run << v << ");\n";
        reg[in.dst] = v;
        if (in.kind != 1) exact[in.dst] = true;
        uniform[in.dst] = same;
    }
    return src.str();
}

// Run `code` compiled when it has been seen before and compiles; false when
// the interpreter should run it instead.
bool run_compiled(const tc_encoded* code, uint32_t count, uint32_t dtype, const DenseLoads& loads,
                  uint32_t load_count, const Buffers& buffers, uint64_t chunks, hipStream_t s, int* status) {
    std::vector<float> constants;
    const bool stream = chunks * dense_chunk_bytes(code, count) > kStreamBytes;
    const std::string source = dense_source(code, count, dtype, stream, &constants);
    if (constants.size() > static_cast<size_t>(kCompiledConstants)) return false;
    hipFunction_t function = nullptr;
    if (!cached_kernels(source, {"tc_fused_program"}, &function)) return false;
    CompiledArgs args{};
    for (uint32_t j = 0; j < load_count; j++) args.in[j] = loads.base[j];
    for (int k = 0; k < TC_FUSED_MAX_OUTPUTS; k++) args.out[k] = buffers.outputs[k];
    for (size_t k = 0; k < constants.size(); k++) args.constants[k] = constants[k];
    args.chunks = chunks;
    size_t size = sizeof(args);
    void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, &args, HIP_LAUNCH_PARAM_BUFFER_SIZE, &size, HIP_LAUNCH_PARAM_END};
    const uint32_t blocks = blocks_for(chunks, 1);
    count_dispatch();
    hipError_t error = hipModuleLaunchKernel(function, blocks, 1, 1, 256, 1, 1, 0, s, nullptr, config);
    *status = error == hipSuccess ? TC_OK : fail(TC_DEVICE, std::string("fused program: ") + hipGetErrorString(error));
    return true;
}

}  // namespace

bool runs_allowed(uint64_t cols, const tc_encoded* code, uint32_t count, const tc_place* places,
                  const void* const* inputs, void* const* outputs, uint32_t output_count, bool product_input,
                  int width) {
    // A piece is 16 bytes of the run, or the whole run when that is shorter,
    // and it starts on its own size.
    auto piece = [&](uint32_t element_dtype) -> uint64_t {
        const uint64_t size = element_dtype == TC_F32 ? 4 : 2;
        return width * size < 16 ? width * size : 16;
    };
    if (width <= 0 || cols % static_cast<uint64_t>(width) != 0) return false;
    for (uint32_t pc = 0; pc < count; pc++) {
        const tc_encoded& in = code[pc];
        if (in.kind == 5) {
            if (in.aux < output_count && reinterpret_cast<uintptr_t>(outputs[in.aux]) % piece(in.b) != 0) return false;
            continue;
        }
        if (in.kind != 0 || (product_input && in.a == 0)) continue;
        const tc_place& place = places[in.op];
        if (place.lead > 1 || (place.col_step != 0 && place.col_step != 1)) return false;
        if (place.col_step != 1) continue;
        const uint64_t size = in.b == TC_F32 ? 4 : 2, align = piece(in.b);
        if ((reinterpret_cast<uintptr_t>(inputs[in.a]) + place.offset * size) % align != 0) return false;
        if (place.lead == 1 && (place.steps[0] * size) % align != 0) return false;
    }
    return true;
}

namespace {

// The columns a thread of the run form takes (`runs_allowed` at that
// width), or 0 for the element form: eight (16 bytes of a 16-bit type)
// unless the program stores f32 or its operands allow only runs of four,
// then four (each f32 store one 16-byte piece, so a wave's store
// instruction writes one contiguous kilobyte; 8-byte pieces of the 16-bit
// types).  Eight f32 a thread stored as two pieces left each instruction
// half of every line it touched, and the non-temporal halves reached HBM as
// 1.56 times the output's bytes.
int run_width(const tc_encoded* code, uint32_t count, const tc_place* places, const void* const* inputs,
              void* const* outputs, uint64_t cols) {
    bool f32_store = false;
    for (uint32_t pc = 0; pc < count; pc++) f32_store |= code[pc].kind == 5 && code[pc].b == TC_F32;
    if (!f32_store && runs_allowed(cols, code, count, places, inputs, outputs, TC_FUSED_MAX_OUTPUTS, false)) {
        return kEpilogueRun;
    }
    return runs_allowed(cols, code, count, places, inputs, outputs, TC_FUSED_MAX_OUTPUTS, false, 4) ? 4 : 0;
}

// A program over whole runs (`runs_allowed`): a kernel over the rows x cols
// space in runs of `run_elems` consecutive columns of one row, a run a
// thread, consecutive threads on consecutive runs.  Each load of contiguous
// columns moves the run's pieces (a row-invariant one, a bias, from the
// cache), a load of one value a row loads it once a run, and each store is
// whole pieces, non-temporal when the program moves more than kStreamBytes.
// From the program's second appearance, like the other compiled forms.
std::string general_runs_source(const tc_encoded* code, uint32_t count, uint32_t dtype, const tc_place* places,
                                uint64_t rows, uint64_t cols, int E, std::vector<float>* constants) {
    const uint64_t runs = rows * cols / E;
    std::vector<bool> marks(count, false);
    uint64_t bytes = 0;  // a run's, loads of contiguous columns and stores
    for (uint32_t pc = 0; pc < count; pc++) {
        const tc_encoded& in = code[pc];
        const uint64_t size = in.b == TC_F32 ? 4 : 2;
        if (in.kind == 5 || (in.kind == 0 && places[in.op].col_step == 1)) {
            marks[pc] = true;
            bytes += size * E;
        }
    }
    const bool stream = runs * bytes > kStreamBytes;
    const std::string body = group_body(code, count, dtype, false, E, places, constants, false, -1, nullptr, &marks,
                                        nullptr, E % 8 == 0, stream);
    if (constants->size() > static_cast<size_t>(kInlineCode)) return std::string();
    const std::string e = std::to_string(E);
    return "#include \"device.hpp\"\n"
           "struct Program {\n" + std::string(compiled_members()) +
           "  __device__ __forceinline__ void run(uint32_t r, uint32_t c, uint32_t N) const {\n"
           "    bool live[" + e + "];\n    uint32_t row[" + e + "], col[" + e + "];\n"
           "    for (int e = 0; e < " + e + "; e++) live[e] = true, row[e] = r, col[e] = c + e;\n" + body + "  }\n};\n"
           "extern \"C\" __global__ void __launch_bounds__(256) tc_fused_runs(Program p, uint32_t cols, uint32_t per_row,\n"
           "                                                                 uint32_t runs) {\n"
           "  const uint32_t stride = gridDim.x * 256u;\n"
           "  uint32_t at = blockIdx.x * 256u + threadIdx.x;\n"
           "  if (at >= runs) return;\n"
           "  // The run's row and its place in the row, then stepped by the grid's\n"
           "  // stride without a division.\n"
           "  uint32_t r = at / per_row, c = at - r * per_row;\n"
           "  const uint32_t step_rows = stride / per_row, step_runs = stride - step_rows * per_row;\n"
           "  for (; at < runs; at += stride) {\n"
           "    p.run(r, c * " + e + "u, cols);\n"
           "    r += step_rows;\n"
           "    c += step_runs;\n"
           "    if (c >= per_row) { c -= per_row; r++; }\n"
           "  }\n"
           "}\n";
}

bool run_general_runs(const tc_encoded* code, uint32_t count, uint32_t dtype, const tc_place* places,
                      uint32_t place_count, const Buffers& buffers, uint64_t rows, uint64_t cols, int E,
                      hipStream_t s, int* status) {
    const uint64_t runs = rows * cols / E;
    std::vector<float> constants;
    const std::string source = general_runs_source(code, count, dtype, places, rows, cols, E, &constants);
    if (source.empty()) return false;
    hipFunction_t function = nullptr;
    if (!cached_kernels(source, {"tc_fused_runs"}, &function)) return false;
    CompiledArgsOf args{};
    for (int k = 0; k < TC_FUSED_MAX_INPUTS; k++) args.in[k] = buffers.inputs[k];
    for (int k = 0; k < TC_FUSED_MAX_OUTPUTS; k++) args.out[k] = buffers.outputs[k];
    int place_status = to_device_places(places, place_count, args.places);
    if (place_status != TC_OK) {
        *status = place_status;
        return true;
    }
    for (size_t c = 0; c < constants.size(); c++) args.constants[c] = constants[c];
    uint32_t cols32 = static_cast<uint32_t>(cols), per_row = static_cast<uint32_t>(cols / E),
             runs32 = static_cast<uint32_t>(runs);
    void* params[] = {&args, &cols32, &per_row, &runs32};
    // A run a thread: a thread's loads then never wait behind its own
    // stores of a run before (loads and stores retire in order), as in a
    // grid of eight workgroups a CU stepping over the runs (the composed
    // layer norm's program pass over 8192 x 8192 f32: 3.52 TB/s for the
    // pair, against 3.02).
    const uint32_t blocks = blocks_for(runs, 1);
    count_dispatch();
    const hipError_t error = hipModuleLaunchKernel(function, blocks, 1, 1, 256, 1, 1, 0, s, params, nullptr);
    *status = error == hipSuccess ? TC_OK : fail(TC_DEVICE, std::string("fused program: ") + hipGetErrorString(error));
    return true;
}

// A program whose loads do not all walk in element order (a broadcast
// operand, a transposed view) runs compiled too, from its second
// appearance: a kernel over the rows x cols space, 16 elements a thread 64
// apart (each load and store instruction of a wave one contiguous run), a
// thread's first element's row and column by one 32-bit division and the
// rest by stepping 64 columns on, the program as the same
// straight-line code a product epilogue runs.
constexpr int kGeneralElems = 16;

std::string general_source(const tc_encoded* code, uint32_t count, uint32_t dtype, const tc_place* places,
                           std::vector<float>* constants);
bool launch_general(hipFunction_t function, const std::vector<float>& constants, const tc_place* places,
                    uint32_t place_count, const Buffers& buffers, uint64_t total, uint64_t cols, hipStream_t s,
                    int* status);

bool run_general_compiled(const tc_encoded* code, uint32_t count, uint32_t dtype, const tc_place* places,
                          uint32_t place_count, const Buffers& buffers, uint64_t rows, uint64_t cols, hipStream_t s,
                          int* status) {
    const uint64_t total = rows * cols;
    // 32-bit element indices: below 2^31, so no index of the last pass wraps.
    if (place_count > static_cast<uint32_t>(kInlinePlaces) || total > (uint64_t{1} << 31)) return false;
    const int E = run_width(code, count, places, buffers.inputs, buffers.outputs, cols);
    if (E != 0) return run_general_runs(code, count, dtype, places, place_count, buffers, rows, cols, E, s, status);
    std::vector<float> constants;
    const std::string source = general_source(code, count, dtype, places, &constants);
    if (source.empty()) return false;
    hipFunction_t function = nullptr;
    if (!cached_kernels(source, {"tc_fused_general"}, &function)) return false;
    return launch_general(function, constants, places, place_count, buffers, rows * cols, cols, s, status);
}

std::string general_source(const tc_encoded* code, uint32_t count, uint32_t dtype, const tc_place* places,
                           std::vector<float>* constants) {
    const std::string body = group_body(code, count, dtype, false, kGeneralElems, places, constants);
    if (constants->size() > static_cast<size_t>(kInlineCode)) return std::string();
    const std::string E = std::to_string(kGeneralElems);
    return
        "#include \"device.hpp\"\n"
        "struct Program {\n" + std::string(compiled_members()) +
        "  __device__ __forceinline__ void group(const bool (&live)[" + E + "], const uint32_t (&row)[" + E + "],\n"
        "      const uint32_t (&col)[" + E + "], uint32_t N) const {\n" + body + "  }\n};\n"
        "extern \"C\" __global__ void __launch_bounds__(256) tc_fused_general(Program p, uint32_t cols, uint32_t total) {\n"
        "  const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64;\n"
        "  const uint32_t per_block = 256u * " + E + ";\n"
        "  for (uint32_t base = blockIdx.x * per_block; base < total; base += gridDim.x * per_block) {\n"
        "    uint32_t row[" + E + "], col[" + E + "];\n"
        "    bool live[" + E + "];\n"
        "    const uint32_t first = base + wave * (64u * " + E + ") + lane;\n"
        "    uint32_t r = first / cols, c = first - r * cols;\n"
        "    for (int v = 0; v < " + E + "; v++) {\n"
        "      const uint32_t at = first + v * 64u;\n"
        "      live[v] = at < total;\n"
        "      if (v > 0) {\n"
        "        // 64 elements on: one step of the row walk when rows are at\n"
        "        // least 64 long, a division otherwise.\n"
        "        if (cols >= 64u) {\n"
        "          c += 64u;\n"
        "          if (c >= cols) { c -= cols; r++; }\n"
        "        } else {\n"
        "          r = at / cols;\n"
        "          c = at - r * cols;\n"
        "        }\n"
        "      }\n"
        "      row[v] = r;\n"
        "      col[v] = c;\n"
        "    }\n"
        "    p.group(live, row, col, cols);\n"
        "  }\n"
        "}\n";
}

bool launch_general(hipFunction_t function, const std::vector<float>& constants, const tc_place* places,
                    uint32_t place_count, const Buffers& buffers, uint64_t total, uint64_t cols, hipStream_t s,
                    int* status) {
    CompiledArgsOf args{};
    for (int k = 0; k < TC_FUSED_MAX_INPUTS; k++) args.in[k] = buffers.inputs[k];
    for (int k = 0; k < TC_FUSED_MAX_OUTPUTS; k++) args.out[k] = buffers.outputs[k];
    int place_status = to_device_places(places, place_count, args.places);
    if (place_status != TC_OK) {
        *status = place_status;
        return true;
    }
    for (size_t c = 0; c < constants.size(); c++) args.constants[c] = constants[c];
    uint32_t cols32 = static_cast<uint32_t>(cols), total32 = static_cast<uint32_t>(total);
    void* params[] = {&args, &cols32, &total32};
    // A thread's elements once, as in the run form (the composed layer norm
    // over 8192 x 8188 f32, whose program takes this form: 2.15 TB/s for the
    // pair, against 2.01 on a grid of eight workgroups a CU).
    const uint32_t blocks = blocks_for(total, kGeneralElems);
    count_dispatch();
    const hipError_t error = hipModuleLaunchKernel(function, blocks, 1, 1, 256, 1, 1, 0, s, params, nullptr);
    *status = error == hipSuccess ? TC_OK : fail(TC_DEVICE, std::string("fused program: ") + hipGetErrorString(error));
    return true;
}

// A program's one output summed along its rows (`fused_sum` over
// `Axis::Rows`, kernels.rs:1120-1135) in one kernel, from the program's second
// appearance: a wave a row, each lane summing its elements in the order it
// takes them (runs of four columns, or 16 elements 64 apart) and the wave in
// a fixed shuffle tree, so the output itself is never stored.
// The bytes an element the program's loads read through places that walk
// rows (a row-invariant place reads the same run in every row).
uint64_t walked_bytes(const tc_encoded* code, uint32_t count, const tc_place* places) {
    uint64_t bytes = 0;
    for (uint32_t pc = 0; pc < count; pc++) {
        if (code[pc].kind != 0) continue;
        const tc_place& p = places[code[pc].op];
        if (p.lead > 1 || (p.lead == 1 && p.steps[0] != 0)) bytes += code[pc].b == TC_F32 ? 4 : 2;
    }
    return bytes;
}

bool run_compiled_row_sums(const tc_encoded* code, uint32_t count, uint32_t dtype, const tc_place* places,
                           uint32_t place_count, const Buffers& buffers, uint64_t rows, uint64_t cols, void* out,
                           hipStream_t s, int* status) {
    if (place_count > static_cast<uint32_t>(kInlinePlaces) || rows * cols > (uint64_t{1} << 31)) return false;
    // Where the operands allow the run form, a lane takes four consecutive
    // columns at a time (the program's contiguous loads one 16-byte run of
    // f32), four runs 256 columns apart in flight; otherwise 16 elements 64
    // apart.  Either way each lane adds its elements in the order it takes
    // them, cols / 64 of them.
    const bool runs = runs_allowed(cols, code, count, places, buffers.inputs, nullptr, 0, false, 4);
    std::vector<bool> marks(count, false);
    for (uint32_t pc = 0; runs && pc < count; pc++) {
        marks[pc] = code[pc].kind == 0 && places[code[pc].op].col_step == 1;
    }
    const int elems = runs ? 4 : kGeneralElems;
    // Runs over 256 MiB or more are read with non-temporal loads.
    const bool stream = runs && rows * cols * walked_bytes(code, count, places) >= kStreamBytes;
    std::vector<float> constants;
    const std::string body = group_body(code, count, dtype, false, elems, places, &constants, true, -1, nullptr,
                                        runs ? &marks : nullptr, nullptr, false, stream);
    if (constants.size() > static_cast<size_t>(kInlineCode)) return false;
    const std::string E = std::to_string(elems);
    const std::string walk =
        runs ? "    for (uint32_t c0 = 0; c0 < cols; c0 += 1024u) {\n"
               "#pragma unroll\n"
               "      for (uint32_t u = 0; u < 4u; u++) {\n"
               "        uint32_t row[4], col[4];\n"
               "        bool live[4];\n"
               "        const uint32_t c = c0 + u * 256u + lane * 4u;\n"
               "        for (int v = 0; v < 4; v++) col[v] = c + v, row[v] = r, live[v] = c < cols;\n"
               "        p.group(live, row, col, cols, sum);\n"
               "      }\n"
               "    }\n"
             : "    for (uint32_t c0 = 0; c0 < cols; c0 += 64u * " + E + ") {\n"
               "      uint32_t row[" + E + "], col[" + E + "];\n"
               "      bool live[" + E + "];\n"
               "      for (int v = 0; v < " + E + "; v++) {\n"
               "        col[v] = c0 + v * 64u + lane;\n"
               "        row[v] = r;\n"
               "        live[v] = col[v] < cols;\n"
               "      }\n"
               "      p.group(live, row, col, cols, sum);\n"
               "    }\n";
    const std::string source =
        "#include \"device.hpp\"\n"
        "struct Program {\n" + std::string(compiled_members()) +
        "  __device__ __forceinline__ void group(const bool (&live)[" + E + "], const uint32_t (&row)[" + E + "],\n"
        "      const uint32_t (&col)[" + E + "], uint32_t N, float& sum) const {\n" + body + "  }\n};\n"
        "extern \"C\" __global__ void __launch_bounds__(256) tc_fused_row_sums(Program p, uint32_t rows,\n"
        "    uint32_t cols, void* sums) {\n"
        "  const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64;\n"
        "  for (uint32_t r = blockIdx.x * 4 + wave; r < rows; r += gridDim.x * 4) {\n"
        "    float sum = 0.0f;\n" + walk +
        "    for (int offset = 32; offset > 0; offset >>= 1) sum += __shfl_xor(sum, offset);\n"
        "    if (lane == 0) tc::store_as(sums, " + std::to_string(dtype) + "u, r, sum);\n"
        "  }\n"
        "}\n";
    hipFunction_t function = nullptr;
    if (!cached_kernels(source, {"tc_fused_row_sums"}, &function)) return false;
    CompiledArgsOf args{};
    for (int k = 0; k < TC_FUSED_MAX_INPUTS; k++) args.in[k] = buffers.inputs[k];
    int place_status = to_device_places(places, place_count, args.places);
    if (place_status != TC_OK) {
        *status = place_status;
        return true;
    }
    for (size_t c = 0; c < constants.size(); c++) args.constants[c] = constants[c];
    uint32_t rows32 = static_cast<uint32_t>(rows), cols32 = static_cast<uint32_t>(cols);
    void* params[] = {&args, &rows32, &cols32, &out};
    const uint64_t wanted = (rows + 3) / 4;
    const uint32_t blocks = static_cast<uint32_t>(wanted < 0xffffffu ? wanted : 0xffffffu);
    count_dispatch();
    const hipError_t error = hipModuleLaunchKernel(function, blocks, 1, 1, 256, 1, 1, 0, s, params, nullptr);
    *status = error == hipSuccess ? TC_OK : fail(TC_DEVICE, std::string("fused sum: ") + hipGetErrorString(error));
    return true;
}

// A program's one output summed along its columns (`fused_sum` over
// `Axis::Columns`, kernels.rs:1120-1135) from the program's second
// appearance, the output never stored: a workgroup takes 256 columns, four
// consecutive ones a lane (the program's contiguous loads one 16-byte run of
// f32, 8 bytes of a 16-bit type), over a split of the rows, its four waves
// consecutive quarters of the split, each lane summing its columns in f32 in
// row order, eight rows' programs at a time; the waves' sums are added in
// order, and the splits' (when the rows are split to fill the GPU) by a
// second kernel in split order.  Taken when the program's operands allow
// the run form (`runs_allowed`).
bool run_compiled_column_sums(const tc_encoded* code, uint32_t count, uint32_t dtype, const tc_place* places,
                              uint32_t place_count, const Buffers& buffers, uint64_t rows, uint64_t cols, void* out,
                              hipStream_t s, int* status) {
    constexpr int E = 4;
    if (place_count > static_cast<uint32_t>(kInlinePlaces) || rows * cols > (uint64_t{1} << 31)) return false;
    if (!runs_allowed(cols, code, count, places, buffers.inputs, nullptr, 0, false, 4)) return false;
    std::vector<bool> runs(count, false);
    for (uint32_t pc = 0; pc < count; pc++) {
        runs[pc] = code[pc].kind == 0 && places[code[pc].op].col_step == 1;
    }
    // Runs over 256 MiB or more are read with non-temporal loads.
    const bool stream = rows * cols * walked_bytes(code, count, places) >= kStreamBytes;
    std::vector<float> constants;
    const std::string body = group_body(code, count, dtype, false, E, places, &constants, true, -1, nullptr, &runs,
                                        nullptr, false, stream, true);
    if (constants.size() > static_cast<size_t>(kInlineCode)) return false;
    const std::string T = std::to_string(dtype);
    const std::string source =
        "#include \"device.hpp\"\n"
        "struct Program {\n" + std::string(compiled_members()) +
        "  __device__ __forceinline__ void group(const bool (&live)[4], const uint32_t (&row)[4],\n"
        "      const uint32_t (&col)[4], uint32_t N, float (&sum)[4]) const {\n" + body + "  }\n};\n"
        "extern \"C\" __global__ void __launch_bounds__(256) tc_fused_column_sums(Program p, uint32_t rows,\n"
        "    uint32_t cols, uint32_t tiles, uint32_t per_split, uint32_t splits, void* sums, float* partial) {\n"
        "  __shared__ float quarter[4][256];\n"
        "  const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64;\n"
        "  const uint32_t tile = blockIdx.x % tiles, split = blockIdx.x / tiles;\n"
        "  const uint32_t c = (tile * 64u + lane) * 4u;\n"
        "  const bool alive = c < cols;\n"
        "  const uint32_t begin = split * per_split;\n"
        "  const uint32_t end = min(begin + per_split, rows);\n"
        "  const uint32_t per_wave = (end - begin + 3u) / 4u;\n"
        "  const uint32_t first = min(begin + wave * per_wave, end), last = min(first + per_wave, end);\n"
        "  float sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};\n"
        "  auto one = [&](uint32_t r) {\n"
        "    bool live[4];\n"
        "    uint32_t row[4], col[4];\n"
        "    for (int e = 0; e < 4; e++) live[e] = alive, row[e] = r, col[e] = c + e;\n"
        "    p.group(live, row, col, cols, sum);\n"
        "  };\n"
        "  uint32_t r = first;\n"
        "  for (; r + 8u <= last; r += 8u) {\n"
        "#pragma unroll\n"
        "    for (int u = 0; u < 8; u++) one(r + u);\n"
        "  }\n"
        "  for (; r < last; r++) one(r);\n"
        "  for (int e = 0; e < 4; e++) quarter[wave][lane * 4u + e] = sum[e];\n"
        "  __syncthreads();\n"
        "  if (wave == 0 && alive) {\n"
        "    for (int e = 0; e < 4; e++) {\n"
        "      const uint32_t at = lane * 4u + e;\n"
        "      const float total = ((quarter[0][at] + quarter[1][at]) + quarter[2][at]) + quarter[3][at];\n"
        "      if (splits == 1u) tc::store_as(sums, " + T + "u, c + e, total);\n"
        "      else partial[(uint64_t)split * cols + c + e] = total;\n"
        "    }\n"
        "  }\n"
        "}\n"
        "// The splits' sums of 64 columns a workgroup: lane = column, each wave\n"
        "// adding a quarter of the splits in order (eight loads in flight), then\n"
        "// the quarters in order.\n"
        "extern \"C\" __global__ void __launch_bounds__(256) tc_fused_column_sums_combine(uint32_t cols,\n"
        "    uint32_t splits, const float* partial, void* sums) {\n"
        "  __shared__ float quarter[4][64];\n"
        "  const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64;\n"
        "  const uint32_t c = blockIdx.x * 64u + lane;\n"
        "  const uint32_t per_wave = (splits + 3u) / 4u;\n"
        "  const uint32_t k0 = min(wave * per_wave, splits), k1 = min(k0 + per_wave, splits);\n"
        "  float total = 0.0f;\n"
        "  if (c < cols) {\n"
        "    uint32_t k = k0;\n"
        "    for (; k + 8u <= k1; k += 8u) {\n"
        "      float x[8];\n"
        "      for (int u = 0; u < 8; u++) x[u] = partial[(uint64_t)(k + u) * cols + c];\n"
        "      for (int u = 0; u < 8; u++) total += x[u];\n"
        "    }\n"
        "    for (; k < k1; k++) total += partial[(uint64_t)k * cols + c];\n"
        "  }\n"
        "  quarter[wave][lane] = total;\n"
        "  __syncthreads();\n"
        "  if (wave == 0 && c < cols) {\n"
        "    tc::store_as(sums, " + T + "u, c, ((quarter[0][lane] + quarter[1][lane]) + quarter[2][lane]) + quarter[3][lane]);\n"
        "  }\n"
        "}\n";
    hipFunction_t functions[2] = {};
    if (!cached_kernels(source, {"tc_fused_column_sums", "tc_fused_column_sums_combine"}, functions)) return false;
    CompiledArgsOf args{};
    for (int k = 0; k < TC_FUSED_MAX_INPUTS; k++) args.in[k] = buffers.inputs[k];
    int place_status = to_device_places(places, place_count, args.places);
    if (place_status != TC_OK) {
        *status = place_status;
        return true;
    }
    for (size_t c = 0; c < constants.size(); c++) args.constants[c] = constants[c];
    // The rows split until there are four workgroups a CU, each wave keeping
    // at least sixteen rows.
    const uint64_t tiles = (cols + 255) / 256;
    const uint64_t want = static_cast<uint64_t>(compute_units()) * 4;
    uint64_t splits = 1;
    if (tiles < want) {
        splits = (want + tiles - 1) / tiles;
        const uint64_t most = rows / (4 * 16);
        if (splits > most) splits = most;
        if (splits < 1) splits = 1;
    }
    const uint64_t per_split = (rows + splits - 1) / splits;
    splits = (rows + per_split - 1) / per_split;
    void* partial = nullptr;
    if (splits > 1) {
        *status = tc_alloc(splits * cols * sizeof(float), &partial);
        if (*status != TC_OK) return true;
    }
    uint32_t rows32 = static_cast<uint32_t>(rows), cols32 = static_cast<uint32_t>(cols),
             tiles32 = static_cast<uint32_t>(tiles), per32 = static_cast<uint32_t>(per_split),
             splits32 = static_cast<uint32_t>(splits);
    void* params[] = {&args, &rows32, &cols32, &tiles32, &per32, &splits32, &out, &partial};
    count_dispatch();
    hipError_t error = hipModuleLaunchKernel(functions[0], static_cast<uint32_t>(tiles * splits), 1, 1, 256, 1, 1, 0,
                                             s, params, nullptr);
    if (error == hipSuccess && splits > 1) {
        void* finish[] = {&cols32, &splits32, &partial, &out};
        count_dispatch();
        error = hipModuleLaunchKernel(functions[1], static_cast<uint32_t>((cols + 63) / 64), 1, 1, 256, 1, 1, 0, s,
                                      finish, nullptr);
    }
    // Stream order keeps the partial sums alive until both kernels have run.
    if (partial != nullptr) tc_free(partial);
    *status = error == hipSuccess ? TC_OK : fail(TC_DEVICE, std::string("fused sum: ") + hipGetErrorString(error));
    return true;
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

std::string epilogue_group(const tc_encoded* code, uint32_t count, uint32_t dtype, bool product_input, int elems,
                           const tc_place* places, std::vector<float>* constants) {
    return group_body(code, count, dtype, product_input, elems, places, constants);
}

std::string epilogue_runs(const tc_encoded* code, uint32_t count, uint32_t dtype, const tc_place* places,
                          std::vector<float>* constants, int E) {
    // Runs of eight (16-bit products) move 16-byte pieces and stream their
    // stores; runs of four (f32 products) move one 16-byte piece, stored
    // plainly as the f32 kernel's own stores are.
    const bool wide = E % 8 == 0;
    const std::string round = "tc_round<" + std::to_string(dtype) + ">";
    const std::string each = "    for (int e = 0; e < " + std::to_string(E) + "; e++) ";
    std::vector<bool> runs(count, false), invariant(count, false);
    std::ostringstream members, loader;
    for (uint32_t pc = 0; pc < count; pc++) {
        const tc_encoded& in = code[pc];
        if (in.kind == 5) {
            runs[pc] = true;
            continue;
        }
        if (in.kind != 0 || in.a == 0) continue;  // input 0 is the product
        const tc_place& place = places[in.op];
        if (place.lead > 1) return std::string();
        const bool same_rows = place.lead == 0 || place.steps[0] == 0;
        const std::string p = "places[" + std::to_string(in.op) + "]", name = "inv.i" + std::to_string(pc);
        if (same_rows && (place.col_step == 1 || place.col_step == 0)) {
            invariant[pc] = true;
            members << "    float i" << pc << "[" << E << "];\n";
            if (place.col_step == 1) {
                loader << each << name << "[e] = 0.0f;\n    if (live) tc::" << (wide ? "load_wide<" : "load_run<") << E
                       << ">(in[" << int(in.a) << "], " << int(in.b) << "u, " << place_index(place, p, "0u", "col")
                       << ", " << name << ");\n" << each << name << "[e] = " << round << "(" << name << "[e]);\n";
            } else {
                loader << "    {\n      const float x = live ? " << round << "(tc::load_as(in[" << int(in.a) << "], "
                       << int(in.b) << "u, " << place_index(place, p, "0u", "0u") << ")) : 0.0f;\n  " << each
                       << name << "[e] = x;\n    }\n";
            }
        } else if (place.col_step == 1) {
            runs[pc] = true;
        } else if (place.col_step != 0) {
            return std::string();
        }
    }
    const std::string body =
        group_body(code, count, dtype, true, E, places, constants, false, -1, nullptr, &runs, &invariant, wide, wide);
    const std::string e = std::to_string(E);
    return "  struct Invariant {\n" + members.str() + "  };\n"
           "  __device__ __forceinline__ void invariant(Invariant& inv, bool live, uint32_t col) const {\n" +
           loader.str() + "  }\n"
           "  __device__ __forceinline__ void run(const Invariant& inv, bool alive, uint32_t r, uint32_t c, uint32_t N,\n"
           "      const float (&product)[" + e + "]) const {\n"
           "    bool live[" + e + "];\n    uint32_t row[" + e + "], col[" + e + "];\n" + each +
           "live[e] = alive, row[e] = r, col[e] = c + e;\n" + body + "  }\n";
}

bool compiled_kernels(const std::string& source, const std::vector<std::string>& kernels, hipFunction_t* out,
                      KernelResources* resources) {
    return cached_kernels(source, kernels, out, resources);
}

// hiprtc hands the compile to the code-object compiler library (comgr) that
// the process has loaded under its soname.  A PyTorch build bundles an older
// one under the same soname, and in a process that imported it first hiprtc
// compiles with that: it handles the one-tile product kernels with a program
// epilogue but crashes on the persistent one (ROCm 7.0's, measured).  So that
// kernel is compiled only when comgr is not loaded yet (the system's will be)
// or the loaded one is the file of the ROCm this library was built with.
bool runtime_compiler_is_ours() {
    static const bool ours = [] {
        void* handle = dlopen("libamd_comgr.so.3", RTLD_NOW | RTLD_NOLOAD);
        if (handle == nullptr) return true;
        bool same = false;
        void* symbol = dlsym(handle, "amd_comgr_get_version");
        Dl_info info{};
        if (symbol != nullptr && dladdr(symbol, &info) != 0 && info.dli_fname != nullptr) {
            char loaded[PATH_MAX], built[PATH_MAX];
            same = realpath(info.dli_fname, loaded) != nullptr &&
                   realpath(TC_ROCM_LIB "/libamd_comgr.so.3", built) != nullptr && strcmp(loaded, built) == 0;
        }
        dlclose(handle);
        return same;
    }();
    return ours;
}

int fused_row_sums(uint32_t dtype, const tc_encoded* code, uint32_t count, const tc_place* places,
                   uint32_t place_count, const void* const* inputs, const uint64_t* input_lens, uint32_t input_count,
                   uint64_t rows, uint64_t cols, void* out, bool* done) {
    *done = false;
    const uint64_t lens[1] = {rows * cols};
    int status = check_fused(dtype, code, count, places, place_count, input_lens, input_count, lens, 1, rows, cols);
    if (status != TC_OK) return status;
    TC_STREAM(s);
    Buffers buffers{};
    for (uint32_t k = 0; k < input_count; k++) buffers.inputs[k] = inputs[k];
    *done = run_compiled_row_sums(code, count, dtype, places, place_count, buffers, rows, cols, out, s, &status);
    return status;
}

int fused_column_sums(uint32_t dtype, const tc_encoded* code, uint32_t count, const tc_place* places,
                      uint32_t place_count, const void* const* inputs, const uint64_t* input_lens,
                      uint32_t input_count, uint64_t rows, uint64_t cols, void* out, bool* done) {
    *done = false;
    const uint64_t lens[1] = {rows * cols};
    int status = check_fused(dtype, code, count, places, place_count, input_lens, input_count, lens, 1, rows, cols);
    if (status != TC_OK) return status;
    TC_STREAM(s);
    Buffers buffers{};
    for (uint32_t k = 0; k < input_count; k++) buffers.inputs[k] = inputs[k];
    *done = run_compiled_column_sums(code, count, dtype, places, place_count, buffers, rows, cols, out, s, &status);
    return status;
}

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

int tc::check_fused(uint32_t dtype, const tc_encoded* code, uint32_t count, const tc_place* places,
                    uint32_t place_count, const uint64_t* input_lens, uint32_t input_count,
                    const uint64_t* output_lens, uint32_t output_count, uint64_t rows, uint64_t cols) {
    int status = check_program(code, count, place_count, input_count, output_count);
    if (status != TC_OK) return status;
    if (dtype > TC_BF16) return fail(TC_UNSUPPORTED, std::string("fused program: no kernel computes in ") + dtype_name(dtype));
    if (rows == 0 || cols == 0) return TC_OK;
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
    return TC_OK;
}

extern "C" int tc_fused(uint32_t dtype, const tc_encoded* code, uint32_t count, const tc_place* places,
                        uint32_t place_count, const void* const* inputs, const uint64_t* input_lens,
                        uint32_t input_count, void* const* outputs, const uint64_t* output_lens,
                        uint32_t output_count, uint64_t rows, uint64_t cols) {
    int status = check_fused(dtype, code, count, places, place_count, input_lens, input_count, output_lens,
                             output_count, rows, cols);
    if (status != TC_OK) return status;
    if (null_slot(inputs, input_lens, input_count) || null_slot(outputs, output_lens, output_count)) {
        return null_operand("fused program");
    }
    TC_STREAM(s);
    if (rows == 0 || cols == 0 || count == 0) return TC_OK;
    Buffers buffers{};
    for (uint32_t k = 0; k < input_count; k++) buffers.inputs[k] = inputs[k];
    for (uint32_t k = 0; k < output_count; k++) buffers.outputs[k] = outputs[k];
    DenseLoads dense{};
    uint32_t dense_loads = 0;
    if (dense_plan(code, count, places, inputs, outputs, rows, cols, &dense, &dense_loads)) {
        const uint64_t chunks = rows * cols / 4;
        if (run_compiled(code, count, dtype, dense, dense_loads, buffers, chunks, s, &status)) return status;
        Inline program{};
        memcpy(program.code, code, count * sizeof(tc_encoded));
        const uint32_t blocks = grid_for(chunks, 256, 8);
        switch (dtype) {
            case TC_F32: fused_dense_kernel<TC_F32><<<blocks, 256, 0, s>>>(program, count, dense, dense_loads, buffers, chunks); break;
            case TC_F16: fused_dense_kernel<TC_F16><<<blocks, 256, 0, s>>>(program, count, dense, dense_loads, buffers, chunks); break;
            default: fused_dense_kernel<TC_BF16><<<blocks, 256, 0, s>>>(program, count, dense, dense_loads, buffers, chunks); break;
        }
        return check_launch("fused program");
    }
    if (run_general_compiled(code, count, dtype, places, place_count, buffers, rows, cols, s, &status)) return status;
    std::vector<DevicePlace> device_places(place_count);
    status = to_device_places(places, place_count, device_places.data());
    if (status != TC_OK) return status;
    const uint64_t total = rows * cols;
    const bool small = total <= UINT32_MAX && cols <= UINT32_MAX;
    DivMod cols_div(small ? static_cast<uint32_t>(cols) : 1u);
    const uint32_t blocks = grid_for(total, 256 * kLanesPerThread, 8);
    Inline program{};
    const bool inline_program = count <= static_cast<uint32_t>(kInlineCode) &&
                                place_count <= static_cast<uint32_t>(kInlinePlaces);
    void* device = nullptr;
    bool transient = false;
    const tc_encoded* dcode = nullptr;
    const DevicePlace* dplaces = nullptr;
    if (inline_program) {
        memcpy(program.code, code, count * sizeof(tc_encoded));
        if (place_count) memcpy(program.places, device_places.data(), place_count * sizeof(DevicePlace));
    } else {
        // A larger program and its places travel in one block of device
        // memory, uploaded on the program's first sight and kept for the
        // process, keyed by its bytes: a later run, captured into a graph or
        // not, reads it in place.  Past the resident limit the block is this
        // call's own, freed below once the kernel is queued.
        const size_t code_bytes = (count * sizeof(tc_encoded) + 15) / 16 * 16;
        std::string key(code_bytes + place_count * sizeof(DevicePlace), '\0');
        memcpy(&key[0], code, count * sizeof(tc_encoded));
        if (place_count) memcpy(&key[code_bytes], device_places.data(), place_count * sizeof(DevicePlace));
        status = resident_program(key, s, &device, &transient);
        if (status != TC_OK) return status;
        dcode = static_cast<const tc_encoded*>(device);
        dplaces = reinterpret_cast<const DevicePlace*>(static_cast<uint8_t*>(device) + code_bytes);
    }
#define TC_FUSED_LAUNCH(T, INLINE)                                                                  \
    fused_kernel<T, INLINE><<<blocks, 256, 0, s>>>(program, dcode, dplaces, count, buffers, rows, cols, \
                                                   cols_div, small)
    if (inline_program) {
        switch (dtype) {
            case TC_F32: TC_FUSED_LAUNCH(TC_F32, true); break;
            case TC_F16: TC_FUSED_LAUNCH(TC_F16, true); break;
            default: TC_FUSED_LAUNCH(TC_BF16, true); break;
        }
    } else {
        switch (dtype) {
            case TC_F32: TC_FUSED_LAUNCH(TC_F32, false); break;
            case TC_F16: TC_FUSED_LAUNCH(TC_F16, false); break;
            default: TC_FUSED_LAUNCH(TC_BF16, false); break;
        }
    }
#undef TC_FUSED_LAUNCH
    status = check_launch("fused program");
    // Stream order keeps a transient block alive until the kernel has run.
    if (transient) tc_free(device);
    return status;
}

extern "C" int tc_fused_compiled(uint64_t* count) {
    std::lock_guard<std::mutex> lock(compiled_mutex);
    *count = compiled_count;
    return TC_OK;
}

extern "C" int tc_fused_resident(uint64_t limit, uint64_t* resident, uint64_t* current_limit) {
    std::lock_guard<std::mutex> lock(resident_mutex);
    if (limit != 0) resident_limit = static_cast<size_t>(limit);
    if (resident != nullptr) *resident = resident_programs.size();
    if (current_limit != nullptr) *current_limit = resident_limit;
    return TC_OK;
}

namespace tc {
namespace {

// The moments' merge and the wave's fold, shared by both forms of the
// statistics kernel's source.
const char* const kMomentsSource =
    "struct Moments { float n, mean, m2; };\n"
    "// Chan's pairwise merge of two (count, mean, squared deviations).\n"
    "__device__ __forceinline__ Moments merge(Moments a, Moments b) {\n"
    "  if (b.n == 0.0f) return a;\n"
    "  if (a.n == 0.0f) return b;\n"
    "  const float n = a.n + b.n, delta = b.mean - a.mean, share = b.n / n;\n"
    "  return Moments{n, a.mean + delta * share, a.m2 + b.m2 + delta * delta * (a.n * share)};\n"
    "}\n"
    "// Every lane ends with the same bits: each step merges the lower\n"
    "// lane's moments with the higher lane's, on both lanes.\n"
    "__device__ __forceinline__ Moments wave_merge(Moments m, uint32_t lane) {\n"
    "  for (int offset = 1; offset < 64; offset <<= 1) {\n"
    "    const Moments o{__shfl_xor(m.n, offset), __shfl_xor(m.mean, offset), __shfl_xor(m.m2, offset)};\n"
    "    m = (lane & offset) == 0 ? merge(m, o) : merge(o, m);\n"
    "  }\n"
    "  return m;\n"
    "}\n";

// The statistics kernel for one source whose place is its own rows x cols
// row-major matrix (a layer norm's x): one to four waves a row (`waves`),
// the row loaded once as 16-byte packs into registers (the row's lane t
// holds packs t, t + 64 waves, ...), each lane's moments taken in two passes
// over its registers, the wave's lanes merged by Chan's update in a fixed
// shuffle tree and the row's waves through LDS in a fixed tree, and the
// program then run over the held packs, a pack's elements a call, its
// loads of that same matrix reading the registers.  The row is read from
// memory once, where the general form reads it again for the program.
// Long rows take more waves, so a lane holds at most 32 values where it
// can: a wave per row of up to 2048 elements, two up to 4096, else four.
// The program's loads of what every row reads alike (a row vector, a
// scalar) are issued once for each of the lane's packs, behind the row's
// loads: left inside the program, each would wait for the stores before
// it, loads and stores retiring in order.  A workgroup takes one group of
// rows, and the launch as many workgroups as there are groups.  Taken when
// the source is 16-byte aligned, rows are whole packs and a lane holds at
// most 64 values (cols up to 16384; the row and a row vector then take
// about 150 registers); false otherwise.
bool held_row_source(const tc_encoded* code, uint32_t count, uint32_t dtype, const tc_place* places,
                     const void* const* inputs, uint32_t input_count, void* const* outputs, uint64_t rows, uint64_t cols,
                     const tc_row_stat& st, uint32_t sources, const tc_row_stat* statistics,
                     uint32_t statistic_count, std::vector<float>* constants, std::string* out,
                     uint32_t* waves_out) {
    if (sources != 1) return false;
    const uint32_t size = st.source_dtype == TC_F32 ? 4 : (st.source_dtype == TC_F16 || st.source_dtype == TC_BF16) ? 2 : 0;
    if (size == 0) return false;
    const uint32_t per = 16 / size;
    const tc_place& sp = st.place;
    if (sp.offset != 0 || sp.col_step != 1 || sp.lead != 1 || sp.steps[0] != cols || cols % per != 0 ||
        reinterpret_cast<uintptr_t>(st.source) % 16 != 0) {
        return false;
    }
    const uint32_t waves = cols <= 2048 ? 1 : cols <= 4096 ? 2 : 4;  // waves a row
    // A source as large as the Infinity Cache is read with non-temporal
    // loads (cache policy 2, nt), each row once; the stores stay plain.
    // Layer norm over 8192 x 8192 f32: 5.50 -> 6.04 TB/s, against 5.62 with
    // the stores non-temporal as well.
    const std::string policy = rows * cols * size >= kStreamBytes ? "2" : "0";
    const uint64_t lanes = 64 * waves;
    const uint64_t packs = (cols + lanes * per - 1) / (lanes * per);  // packs a lane holds
    if (packs * per > 64) return false;
    // The program's loads of the same elements: the same storage, type and
    // place.
    std::vector<bool> held(count, false);
    for (uint32_t pc = 0; pc < count; pc++) {
        const tc_encoded& in = code[pc];
        if (in.kind != 0 || in.a >= input_count || inputs[in.a] != st.source || in.b != st.source_dtype) continue;
        const tc_place& lp = places[in.op];
        held[pc] = lp.offset == sp.offset && lp.col_step == sp.col_step && lp.lead == sp.lead &&
                   lp.dims[0] == sp.dims[0] && lp.steps[0] == sp.steps[0];
    }
    // The other loads and the stores move a pack's elements as one run
    // where their pieces are aligned: a store to an aligned output (its row
    // of cols elements is whole pieces), a load through a place that walks
    // columns one by one from an aligned input, offset and row step.
    // `outputs` may be null (a diagnostic): outputs then count as aligned.
    auto aligned = [](const void* pointer, uint32_t element_dtype) {
        return reinterpret_cast<uintptr_t>(pointer) % (element_dtype == TC_F32 ? 16 : 8) == 0;
    };
    std::vector<bool> runs(count, false);
    for (uint32_t pc = 0; pc < count; pc++) {
        const tc_encoded& in = code[pc];
        if (in.kind == 5) {
            runs[pc] = outputs == nullptr || aligned(outputs[in.aux], in.b);
        } else if (in.kind == 0 && !held[pc] && in.a < input_count) {
            const tc_place& lp = places[in.op];
            runs[pc] = lp.lead <= 1 && lp.col_step == 1 && lp.offset % 4 == 0 &&
                       (lp.lead == 0 || lp.steps[0] % 4 == 0) && aligned(inputs[in.a], in.b);
        }
    }
    // Loads that read the same elements in every row (a row vector such as
    // a layer norm's gamma, a scalar) are loaded for every pack of the lane
    // once, before the loop over rows: a load inside the program would wait
    // for the stores before it, as loads and stores retire in order.
    std::vector<bool> invariant(count, false);
    const std::string round = "tc_round<" + std::to_string(dtype) + ">";
    const std::string each_pack = "    for (int e = 0; e < " + std::to_string(per) + "; e++) ";
    std::ostringstream members, loader;
    for (uint32_t pc = 0; pc < count; pc++) {
        const tc_encoded& in = code[pc];
        if (in.kind != 0 || held[pc] || in.a >= input_count) continue;
        const tc_place& lp = places[in.op];
        const bool same_rows = lp.lead == 0 || (lp.lead == 1 && lp.steps[0] == 0);
        if (!same_rows || (lp.col_step != 0 && !runs[pc])) continue;
        invariant[pc] = true;
        runs[pc] = false;
        const std::string name = "inv.i" + std::to_string(pc), pl = "places[" + std::to_string(in.op) + "]";
        members << "    float i" << pc << "[" << per << "];\n";
        if (lp.col_step == 1) {
            loader << each_pack << name << "[e] = 0.0f;\n    if (live) tc::load_run<" << per << ">(in["
                   << int(in.a) << "], " << int(in.b) << "u, " << place_index(lp, pl, "0u", "col") << ", " << name
                   << ");\n" << each_pack << name << "[e] = " << round << "(" << name << "[e]);\n";
        } else {
            loader << "    {\n      const float x = live ? " << round << "(tc::load_as(in[" << int(in.a) << "], "
                   << int(in.b) << "u, " << place_index(lp, pl, "0u", "0u") << ")) : 0.0f;\n  " << each_pack
                   << name << "[e] = x;\n    }\n";
        }
    }
    const std::string body = group_body(code, count, dtype, false, static_cast<int>(per), places, constants, false,
                                        static_cast<int>(input_count), &held, &runs, &invariant);
    if (constants->size() > static_cast<size_t>(kInlineCode)) return false;
    const std::string P = std::to_string(per), K = std::to_string(packs), S = std::to_string(statistic_count),
                      T = std::to_string(dtype);
    // A pack's elements from its 16 bytes, rounded to the program's type as
    // a load of them is.
    std::string unpack;
    if (st.source_dtype == TC_F32) {
        unpack = "  const uint32_t bits[4] = {w.x, w.y, w.z, w.w};\n"
                 "  for (int j = 0; j < 4; j++) x[j] = tc_round<" + T + ">(__builtin_bit_cast(float, bits[j]));\n";
    } else {
        const std::string widen = st.source_dtype == TC_F16
                                      ? "static_cast<float>(__builtin_bit_cast(_Float16, h))"
                                      : "tc::bf16_bits_to_f32(h)";
        unpack = "  const uint32_t words[4] = {w.x, w.y, w.z, w.w};\n"
                 "  for (int j = 0; j < 8; j++) {\n"
                 "    const uint16_t h = static_cast<uint16_t>(words[j / 2] >> (16 * (j % 2)));\n"
                 "    x[j] = tc_round<" + T + ">(" + widen + ");\n"
                 "  }\n";
    }
    const std::string W = std::to_string(waves), L = std::to_string(lanes),
                      B = std::to_string(lanes * 16), R = std::to_string(4 / waves);
    std::ostringstream src;
    src << "#include \"device.hpp\"\n"
           "struct Program {\n" << compiled_members()
        << "  struct Invariant {\n" << members.str() << "  };\n"
           "  __device__ __forceinline__ void invariant(Invariant& inv, bool live, uint32_t col) const {\n"
        << loader.str() << "  }\n"
           "  __device__ __forceinline__ void group(const bool (&live)[" << P << "], const uint32_t (&row)[" << P
        << "],\n      const uint32_t (&col)[" << P << "], uint32_t N, const float (&stat)[" << S
        << "], const float (&held)[" << P << "],\n      const Invariant& inv) const {\n"
        << body << "  }\n};\n"
           "struct Sources { const void* in[4]; tc::DevicePlace places[4]; };\n"
        << kMomentsSource
        << "__device__ __forceinline__ void unpack(const uint4 w, float (&x)[" << P << "]) {\n" << unpack << "}\n"
           "extern \"C\" __global__ void __launch_bounds__(256)\n"
           "tc_fused_row_statistics(Program p, Sources src,\n"
           "    uint32_t rows, uint32_t cols) {\n"
           "  // " << W << " wave(s) a row, " << R << " row(s) a block: the wave, its row\n"
           "  // and its part of the row are uniform, so the row's buffer\n"
           "  // resource lives in scalar registers.\n"
           "  const uint32_t lane = threadIdx.x % 64, wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);\n"
           "  const uint32_t part = wave % " << W << "u, at = part * 64u + lane;\n";
    if (waves > 1) {
        src << "  // Each wave's merged moments.\n"
               "  __shared__ float parts[4][3];\n";
    }
    src << "  // The workgroup's row for this wave (one past the last row repeats\n"
           "  // the last row's work and stores nothing, so the workgroup's\n"
           "  // barrier is met by all of its waves).\n"
           "  const uint32_t first_row = blockIdx.x * " << R << "u + wave / " << W << "u;\n"
           "  const bool on = first_row < rows;\n"
           "  const uint32_t r = on ? first_row : rows - 1;\n"
           "  // The row as a buffer of its own bytes: a pack past its end loads\n"
           "  // zeros, with no branch, and every load's address is the lane's\n"
           "  // offset plus a constant.\n"
           "  const __amdgpu_buffer_rsrc_t line = __builtin_amdgcn_make_buffer_rsrc(\n"
           "      const_cast<uint8_t*>(static_cast<const uint8_t*>(src.in[0]) + (uint64_t)r * cols * " << size
        << "u), 0,\n      cols * " << size << "u, 0x00020000);\n"
           "  // The row's packs as loaded (16-bit elements stay packed, two a\n"
           "  // register), unpacked at each use.\n"
           "  uint4 w[" << K << "];\n"
           "#pragma unroll\n"
           "  for (int k = 0; k < " << K << "; k++)\n"
           "    w[k] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(line, at * 16u, k * " << B
        << "u, " << policy << "));\n";
    if (waves > 1) {
        src << "  // The row's first pack, which every lane loads (lane 0 of the\n"
               "  // row's first wave holds it in w[0] as well).\n"
               "  const uint4 head = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(line, 0u, 0u, "
            << policy << "));\n";
    }
    src << "  // The program's loads of what every row reads alike, for each of\n"
           "  // the lane's packs, issued behind the row's.\n"
           "  typename Program::Invariant inv[" << K << "];\n"
           "#pragma unroll\n"
           "  for (int k = 0; k < " << K << "; k++) {\n"
           "    const uint32_t col = (at + " << L << "u * k) * " << P << "u;\n"
           "    p.invariant(inv[k], col < cols, col);\n"
           "  }\n"
           "  {\n"
           "    // The lane's values in two passes: their mean, then the squared\n"
           "    // deviations from it; then the wave's lanes merged.\n"
           "    // The row's first element, when finite, is subtracted first and\n"
           "    // added back to the mean once: rows whose mean is large against\n"
           "    // their spread keep their accuracy through the lanes' merges.\n"
           "    float first[" << P << "];\n";
    if (waves == 1) {
        src << "    unpack(w[0], first);\n"
               "    float shift = __shfl(first[0], 0, 64);\n";
    } else {
        src << "    unpack(head, first);\n"
               "    float shift = first[0];\n";
    }
    src << "    if (!isfinite(shift)) shift = 0.0f;\n"
           "    float n = 0.0f, sum = 0.0f;\n"
           "#pragma unroll\n"
           "    for (int k = 0; k < " << K << "; k++) {\n"
           "      if ((at + " << L << "u * k) * " << P << "u < cols) {\n"
           "        float x[" << P << "];\n"
           "        unpack(w[k], x);\n"
           "        for (int j = 0; j < " << P << "; j++) sum += x[j] - shift;\n"
           "        n += " << per << ".0f;\n"
           "      }\n"
           "    }\n"
           "    const float lane_mean = n > 0.0f ? sum / n : 0.0f;\n"
           "    // The same value, made opaque: the second pass recomputes each\n"
           "    // x - shift rather than keeping the first pass's in registers.\n"
           "    asm volatile(\"\" : \"+v\"(shift));\n"
           "    float q = 0.0f;\n"
           "#pragma unroll\n"
           "    for (int k = 0; k < " << K << "; k++) {\n"
           "      if ((at + " << L << "u * k) * " << P << "u < cols) {\n"
           "        float x[" << P << "];\n"
           "        unpack(w[k], x);\n"
           "        for (int j = 0; j < " << P << "; j++) {\n"
           "          const float d = (x[j] - shift) - lane_mean;\n"
           "          q += d * d;\n"
           "        }\n"
           "      }\n"
           "    }\n";
    if (waves == 1) {
        src << "    const Moments m = wave_merge(Moments{n, lane_mean, q}, lane);\n";
    } else {
        src << "    const Moments mine = wave_merge(Moments{n, lane_mean, q}, lane);\n"
               "    if (lane == 0) {\n"
               "      parts[wave][0] = mine.n;\n"
               "      parts[wave][1] = mine.mean;\n"
               "      parts[wave][2] = mine.m2;\n"
               "    }\n"
               "    __syncthreads();\n"
               "    // The row's waves in a fixed tree, the same bits on each.\n"
               "    Moments each[" << W << "];\n"
               "    for (uint32_t v = 0; v < " << W << "u; v++) {\n"
               "      const float* slot = parts[wave - part + v];\n"
               "      each[v] = Moments{slot[0], slot[1], slot[2]};\n"
               "    }\n";
        if (waves == 2) {
            src << "    const Moments m = merge(each[0], each[1]);\n";
        } else {
            src << "    const Moments m = merge(merge(each[0], each[1]), merge(each[2], each[3]));\n";
        }
    }
    src << "    float stat[" << S << "];\n";
    for (uint32_t i = 0; i < statistic_count; i++) {
        src << "    stat[" << i << "] = tc_round<" << T << ">("
            << (statistics[i].which == TC_STAT_MEAN ? "m.mean + shift" : "m.m2") << ");\n";
    }
    src << "    // The lane's index made opaque here, so the columns of every pack\n"
           "    // are computed where they are used rather than hoisted out of the\n"
           "    // row loop, where they would hold a register each.\n"
           "    uint32_t at_lane = at;\n"
           "    asm volatile(\"\" : \"+v\"(at_lane));\n"
           "#pragma unroll\n"
           "    for (int k = 0; k < " << K << "; k++) {\n"
           "      uint32_t row[" << P << "], col[" << P << "];\n"
           "      bool live[" << P << "];\n"
           "      for (int j = 0; j < " << P << "; j++) {\n"
           "        col[j] = (at_lane + " << L << "u * k) * " << P << "u + j;\n"
           "        row[j] = r;\n"
           "        live[j] = on && col[j] < cols;\n"
           "      }\n"
           "      float x[" << P << "];\n"
           "      unpack(w[k], x);\n"
           "      p.group(live, row, col, cols, stat, x, inv[k]);\n"
           "      // One pack's program at a time: hoisting every pack's loads\n"
           "      // ahead of the others' arithmetic would spill the row.\n"
           "      __builtin_amdgcn_sched_barrier(0);\n"
           "    }\n"
           "  }\n"
           "}\n";
    *waves_out = waves;
    *out = src.str();
    return true;
}

}  // namespace
}  // namespace tc

// `fused_with_statistics` (kernels.rs:1103-1113) as one compiled kernel, from
// the program's second appearance.  The held form (`held_row_source`) keeps
// each row in registers; the general form here runs a wave a row.  For each
// distinct source
// one pass over the row (through the source's place, rounded to the
// program's type) takes each lane's batches of 16 elements, their mean and
// squared deviations from it, and merges them into the lane's running
// moments (Chan's pairwise update), then merges the wave's lanes in a fixed
// tree; mean and deviations are rounded to the program's type, as the
// composed form stores them, and the program then runs over the row with
// each statistic read from a register.  The row's second read, for the
// program, mostly hits the caches.
namespace tc {
namespace {

// The one-kernel form's plan: its source (empty when the program does not
// take that form), its constants, and its distinct sources.
struct RowStatisticsPlan {
    std::string source;
    std::vector<float> constants;
    const tc_row_stat* first[4] = {};
    uint32_t sources = 0;
    bool held = false;    // the form that holds each row in registers
    uint32_t waves = 1;   // the held form's waves a row (1, 2 or 4)
};

int plan_row_statistics(uint32_t dtype, const tc_encoded* code, uint32_t count, const tc_place* places,
                        uint32_t place_count, const void* const* inputs, uint32_t input_count,
                        void* const* outputs, uint64_t rows, uint64_t cols, const tc_row_stat* statistics,
                        uint32_t statistic_count, RowStatisticsPlan* plan) {
    plan->source.clear();
    constexpr uint32_t kMaxSources = 4;
    if (statistic_count == 0 || statistic_count > 8 || place_count > static_cast<uint32_t>(kInlinePlaces) ||
        rows == 0 || cols == 0 || rows * cols > (uint64_t{1} << 31)) {
        return TC_OK;
    }
    // Every load of a statistic reads one value a row, in the program's type.
    for (uint32_t pc = 0; pc < count; pc++) {
        const tc_encoded& in = code[pc];
        if (in.kind != 0 || in.a < input_count) continue;
        if (in.op >= place_count || in.b != dtype) return TC_OK;
        const tc_place& p = places[in.op];
        if (p.offset != 0 || p.col_step != 0 || p.lead != 1 || p.dims[0] != rows || p.steps[0] != 1) return TC_OK;
    }
    // The distinct sources, each with its place checked against its length.
    uint32_t source_of[8];
    uint32_t& sources = plan->sources;
    const tc_row_stat** first = plan->first;
    for (uint32_t i = 0; i < statistic_count; i++) {
        const tc_row_stat& st = statistics[i];
        uint32_t j = 0;
        for (; j < sources; j++) {
            const tc_row_stat& f = *first[j];
            bool same = f.source == st.source && f.source_dtype == st.source_dtype && f.place.offset == st.place.offset &&
                        f.place.col_step == st.place.col_step && f.place.lead == st.place.lead;
            for (uint32_t d = 0; same && d < st.place.lead; d++) {
                same = f.place.dims[d] == st.place.dims[d] && f.place.steps[d] == st.place.steps[d];
            }
            if (same) break;
        }
        if (j == sources) {
            if (sources == kMaxSources) return TC_OK;
            uint64_t end = 0;
            if (!place_end(st.place, rows, cols, &end) || end > st.source_len) {
                return fail(TC_INVALID, "fused with statistics: statistic " + std::to_string(i) +
                                            " reads past its source's " + std::to_string(st.source_len) + " elements");
            }
            first[sources++] = &st;
        }
        source_of[i] = j;
    }
    std::vector<float>& constants = plan->constants;
    const std::string S = std::to_string(statistic_count), T = std::to_string(dtype);
    std::ostringstream src;
    std::string held_source;
    if (held_row_source(code, count, dtype, places, inputs, input_count, outputs, rows, cols, *first[0], sources,
                        statistics, statistic_count, &constants, &held_source, &plan->waves)) {
        src << held_source;
        plan->held = true;
    } else {
        constants.clear();
        const std::string body = group_body(code, count, dtype, false, kGeneralElems, places, &constants, false,
                                            static_cast<int>(input_count));
        if (constants.size() > static_cast<size_t>(kInlineCode)) return TC_OK;
        const std::string E = std::to_string(kGeneralElems);
        src << "#include \"device.hpp\"\n"
               "struct Program {\n" << compiled_members()
            << "  __device__ __forceinline__ void group(const bool (&live)[" << E << "], const uint32_t (&row)[" << E
            << "],\n      const uint32_t (&col)[" << E << "], uint32_t N, const float (&stat)[" << S << "]) const {\n"
            << body << "  }\n};\n"
               "struct Sources { const void* in[4]; tc::DevicePlace places[4]; };\n"
            << kMomentsSource <<
               "extern \"C\" __global__ void __launch_bounds__(256) tc_fused_row_statistics(Program p, Sources src,\n"
               "    uint32_t rows, uint32_t cols) {\n"
               "  const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64;\n"
               "  for (uint32_t r = blockIdx.x * 4 + wave; r < rows; r += gridDim.x * 4) {\n"
               "    float stat[" << S << "];\n";
        for (uint32_t j = 0; j < sources; j++) {
            const std::string J = std::to_string(j), D = std::to_string(first[j]->source_dtype);
            // Sixteen loads in flight a lane; each lane still adds its
            // elements in column order.
            const std::string value = "tc_round<" + T + ">(tc::load_as(src.in[" + J + "], " + D + "u, " +
                                      place_index(first[j]->place, "src.places[" + J + "]", "r", "c") + "))";
            const std::string batch = "      for (uint32_t c0 = lane; c0 < cols; c0 += 64u * 16u) {\n"
                                      "        float x[16];\n"
                                      "        for (int u = 0; u < 16; u++) {\n"
                                      "          const uint32_t c = c0 + 64u * u;\n"
                                      "          x[u] = c < cols ? " + value + " : 0.0f;\n"
                                      "        }\n";
            // One pass: each batch's own mean and squared deviations, merged
            // into the lane's running moments, then the wave's lanes merged.
            // The row's first element, when finite, is subtracted before the
            // moments are taken and added back to the mean once: rows whose
            // mean is large against their spread keep the accuracy of two
            // passes through the merges.
            const std::string first_value = "tc_round<" + T + ">(tc::load_as(src.in[" + J + "], " + D + "u, " +
                                            place_index(first[j]->place, "src.places[" + J + "]", "r", "0u") + "))";
            src << "    {\n"
                   "      float shift = " << first_value << ";\n"
                   "      if (!isfinite(shift)) shift = 0.0f;\n"
                   "      Moments m{0.0f, 0.0f, 0.0f};\n" << batch <<
                   "        for (int u = 0; u < 16; u++) x[u] -= shift;\n"
                   "        float bs = 0.0f, bn = 0.0f;\n"
                   "        for (int u = 0; u < 16; u++) if (c0 + 64u * u < cols) { bs += x[u]; bn += 1.0f; }\n"
                   "        const float bm = bn > 0.0f ? bs / bn : 0.0f;\n"
                   "        float bq = 0.0f;\n"
                   "        for (int u = 0; u < 16; u++) {\n"
                   "          const float d = x[u] - bm;\n"
                   "          if (c0 + 64u * u < cols) bq += d * d;\n"
                   "        }\n"
                   "        m = merge(m, Moments{bn, bm, bq});\n"
                   "      }\n"
                   "      m = wave_merge(m, lane);\n"
                   "      const float mean = m.mean + shift, deviations = m.m2;\n";
            for (uint32_t i = 0; i < statistic_count; i++) {
                if (source_of[i] != j) continue;
                src << "      stat[" << i << "] = tc_round<" << T << ">("
                    << (statistics[i].which == TC_STAT_MEAN ? "mean" : "deviations") << ");\n";
            }
            src << "    }\n";
        }
        src << "    for (uint32_t c0 = 0; c0 < cols; c0 += 64u * " << E << ") {\n"
               "      uint32_t row[" << E << "], col[" << E << "];\n"
               "      bool live[" << E << "];\n"
               "      for (int v = 0; v < " << E << "; v++) {\n"
               "        col[v] = c0 + v * 64u + lane;\n"
               "        row[v] = r;\n"
               "        live[v] = col[v] < cols;\n"
               "      }\n"
               "      p.group(live, row, col, cols, stat);\n"
               "    }\n"
               "  }\n"
               "}\n";
    }
    plan->source = src.str();
    return TC_OK;
}

}  // namespace
}  // namespace tc

int tc::fused_row_statistics(uint32_t dtype, const tc_encoded* code, uint32_t count, const tc_place* places,
                             uint32_t place_count, const void* const* inputs, const uint64_t* input_lens,
                             uint32_t input_count, void* const* outputs, const uint64_t* output_lens,
                             uint32_t output_count, uint64_t rows, uint64_t cols, const tc_row_stat* statistics,
                             uint32_t statistic_count, bool* done) {
    *done = false;
    (void)input_lens;
    (void)output_lens;
    RowStatisticsPlan plan;
    int status = plan_row_statistics(dtype, code, count, places, place_count, inputs, input_count, outputs, rows,
                                     cols, statistics, statistic_count, &plan);
    if (status != TC_OK || plan.source.empty()) return status;
    const std::vector<float>& constants = plan.constants;
    const uint32_t sources = plan.sources;
    const tc_row_stat* const* first = plan.first;
    hipFunction_t function = nullptr;
    if (!cached_kernels(plan.source, {"tc_fused_row_statistics"}, &function)) return TC_OK;
    TC_STREAM(s);
    CompiledArgsOf args{};
    for (uint32_t k = 0; k < input_count; k++) args.in[k] = inputs[k];
    for (uint32_t k = 0; k < output_count; k++) args.out[k] = outputs[k];
    status = to_device_places(places, place_count, args.places);
    if (status != TC_OK) return status;
    for (size_t c = 0; c < constants.size(); c++) args.constants[c] = constants[c];
    struct {
        const void* in[4];
        DevicePlace places[4];
    } where{};
    for (uint32_t j = 0; j < sources; j++) {
        where.in[j] = first[j]->source;
        status = to_device_places(&first[j]->place, 1, &where.places[j]);
        if (status != TC_OK) return status;
    }
    uint32_t rows32 = static_cast<uint32_t>(rows), cols32 = static_cast<uint32_t>(cols);
    void* params[] = {&args, &where, &rows32, &cols32};
    // The general form: four workgroups a CU, each wave walking rows:
    // enough loads in flight for HBM, while the rows in flight stay few
    // enough that a row's second read, for the program, finds it in the
    // caches (layer norm over 8192 x 8192 f32: 3.10 TB/s, against 2.91 at
    // eight a CU).  The held form reads each row once and takes a workgroup
    // for each 4 / waves rows, as many as there are: the rows of a launch
    // spread over every CU as workgroups end, where a grid of eight a CU
    // looping over them ends on a few CUs still at their last rows (the
    // same layer norm, four waves a row: 5.16 TB/s, against 5.00 at eight a
    // CU; a wave a row, 4.70 at eight a CU).
    const uint64_t per_block = plan.held ? 4 / plan.waves : 4;
    const uint64_t wanted = (rows + per_block - 1) / per_block,
                   cap = plan.held ? wanted : static_cast<uint64_t>(compute_units()) * 4;
    const uint32_t blocks = static_cast<uint32_t>(wanted < cap ? wanted : cap);
    count_dispatch();
    const hipError_t error = hipModuleLaunchKernel(function, blocks, 1, 1, 256, 1, 1, 0, s, params, nullptr);
    if (error != hipSuccess) return fail(TC_DEVICE, std::string("fused with statistics: ") + hipGetErrorString(error));
    *done = true;
    return TC_OK;
}

using tc::RowStatisticsPlan;
using tc::plan_row_statistics;

extern "C" int tc_fused_with_statistics_source(uint32_t dtype, const tc_encoded* code, uint32_t count,
                                               const tc_place* places, uint32_t place_count,
                                               const void* const* inputs, uint32_t input_count, uint64_t rows,
                                               uint64_t cols, const tc_row_stat* statistics,
                                               uint32_t statistic_count, char* out, uint64_t capacity,
                                               uint64_t* length) {
    RowStatisticsPlan plan;
    const int status = plan_row_statistics(dtype, code, count, places, place_count, inputs, input_count, nullptr,
                                           rows, cols, statistics, statistic_count, &plan);
    if (status != TC_OK) return status;
    if (plan.source.empty()) {
        return fail(TC_UNSUPPORTED, "fused with statistics source: the program does not take the one-kernel form");
    }
    *length = plan.source.size();
    if (out != nullptr && capacity > 0) {
        const size_t n = plan.source.size() < capacity - 1 ? plan.source.size() : capacity - 1;
        memcpy(out, plan.source.data(), n);
        out[n] = '\0';
    }
    return TC_OK;
}

extern "C" int tc_fused_source(uint32_t dtype, const tc_encoded* code, uint32_t count, const tc_place* places,
                               uint32_t place_count, const void* const* inputs, uint32_t input_count, uint64_t rows,
                               uint64_t cols, char* out, uint64_t capacity, uint64_t* length) {
    if (dtype > TC_BF16) return fail(TC_UNSUPPORTED, std::string("fused source: no kernels for ") + dtype_name(dtype));
    if (input_count > TC_FUSED_MAX_INPUTS || rows == 0 || cols == 0) {
        return fail(TC_INVALID, "fused source: inputs, rows and columns as tc_fused takes them");
    }
    const void* in[TC_FUSED_MAX_INPUTS] = {};
    for (uint32_t k = 0; k < input_count; k++) in[k] = inputs[k];
    void* const outs[TC_FUSED_MAX_OUTPUTS] = {};  // outputs count as 16-byte aligned
    std::vector<float> constants;
    std::string source;
    tc::DenseLoads dense{};
    uint32_t dense_loads = 0;
    if (tc::dense_plan(code, count, places, in, outs, rows, cols, &dense, &dense_loads)) {
        const bool stream = rows * cols / 4 * tc::dense_chunk_bytes(code, count) > kStreamBytes;
        source = tc::dense_source(code, count, dtype, stream, &constants);
    } else if (place_count <= static_cast<uint32_t>(kInlinePlaces) && rows * cols <= (uint64_t{1} << 31)) {
        const int width = tc::run_width(code, count, places, in, outs, cols);
        source = width != 0 ? tc::general_runs_source(code, count, dtype, places, rows, cols, width, &constants)
                            : tc::general_source(code, count, dtype, places, &constants);
    }
    if (source.empty()) return fail(TC_UNSUPPORTED, "fused source: the program runs interpreted");
    *length = source.size();
    if (out != nullptr && capacity > 0) {
        const size_t n = source.size() < capacity - 1 ? source.size() : capacity - 1;
        memcpy(out, source.data(), n);
        out[n] = '\0';
    }
    return TC_OK;
}
