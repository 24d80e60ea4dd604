// Shared by every translation unit of libtchip: the runtime hooks the entry
// points use (error state, the calling thread's stream, launch checks), the
// element types and their conversions, and the index arithmetic the strided
// kernels run on.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "../../include/tchip.h"
#include "device.hpp"
#include "scalar_ops.h"

// The codes scalar_ops.h (which the runtime compiler also reads) uses are
// the C ABI's.
static_assert(tc_ops::ADD == TC_ADD && tc_ops::SUB == TC_SUB && tc_ops::MUL == TC_MUL && tc_ops::DIV == TC_DIV &&
                  tc_ops::REM == TC_REM,
              "BinaryOp codes");
static_assert(tc_ops::MIN == TC_MIN && tc_ops::MAX == TC_MAX && tc_ops::MAX_SHARE == TC_MAX_SHARE &&
                  tc_ops::LESS == TC_LESS && tc_ops::LESS_EQUAL == TC_LESS_EQUAL && tc_ops::GREATER == TC_GREATER &&
                  tc_ops::GREATER_EQUAL == TC_GREATER_EQUAL,
              "Compare codes");
static_assert(tc_ops::F32 == TC_F32 && tc_ops::F16 == TC_F16 && tc_ops::BF16 == TC_BF16, "DType codes");
static_assert(tc::kPlaceLead == TC_FUSED_LEAD, "a place's folded axes");

namespace tc {

constexpr int kMaxRank = TC_MAX_RANK;

// ---- runtime hooks (runtime.hip) -------------------------------------------

// Record `message` as this thread's last error and return `status`.
int fail(int status, const std::string& message);
// The calling thread's stream, initialising device 0 on first use; nullptr
// (with the error recorded) if the device cannot be set up.
hipStream_t stream();
// TC_OK, or the HIP error from the launch just made, recorded under `what`;
// counts the launch as one operation queued on the thread's stream.
int check_launch(const char* what);
// Count an operation queued without check_launch (a module launch, a copy).
void count_dispatch();
// Wait for the stream or an event on the host, counted as a host wait.
hipError_t host_wait(hipStream_t s);
hipError_t host_wait(hipEvent_t e);
// A call with work to do refuses a null device pointer on the host, before
// any device work: a kernel would read or write address 0.  `null_operand`
// records the refusal under `what`; `null_slot` is true when a slot of an
// input or output array has elements but no storage.
inline bool any_null(std::initializer_list<const void*> pointers) {
    for (const void* p : pointers) {
        if (p == nullptr) return true;
    }
    return false;
}
inline int null_operand(const char* what) { return fail(TC_INVALID, std::string(what) + ": a null operand"); }
inline bool null_slot(const void* const* pointers, const uint64_t* lens, uint32_t count) {
    for (uint32_t k = 0; k < count; k++) {
        if (lens[k] != 0 && pointers[k] == nullptr) return true;
    }
    return false;
}

// Shorthand: set up the thread's stream or return its failure.
#define TC_STREAM(var)                                \
    hipStream_t var = ::tc::stream();                 \
    if (var == nullptr) return TC_DEVICE

// Number of compute units, for sizing persistent and split grids.
int compute_units();

// Each slice's mean into `means` and its sum of squared deviations into
// `deviations`, both of `dtype`, in one pass (reduce.hip; the moments
// `row_moments` returns).
int reduce_moments(uint32_t dtype, const void* input, uint64_t input_len, const tc_split* split, void* means,
                   void* deviations);

// Everything `tc_fused` checks before a launch: the program's registers,
// kinds and codes, and every load and store inside its buffer over a rows x
// cols space (fused.hip).
int check_fused(uint32_t dtype, const tc_encoded* code, uint32_t count, const tc_place* places,
                uint32_t place_count, const uint64_t* input_lens, uint32_t input_count, const uint64_t* output_lens,
                uint32_t output_count, uint64_t rows, uint64_t cols);

// The product a . b (m x k by k x n, row-major, `dtype` operands) with the
// checked program run over it in the product kernel's epilogue, input 0 the
// product rounded to `dtype` (gemm.hip).  Sets `*fused` false, launching
// nothing, when the product does not take the matrix-core kernels or the
// program does not fit in kernel arguments.
int matmul_program(uint32_t dtype, uint64_t m, uint64_t k, uint64_t n, const void* a, const void* b,
                   const tc_encoded* code, uint32_t count, const tc_place* places, uint32_t place_count,
                   const void* const* inputs, uint32_t input_count, void* const* outputs, uint32_t output_count,
                   bool* fused);

// The matrix-vector kernels (gemv.hip): out[rows] (+)= matrix[rows x cols] .
// vector[cols], or with `row_vector` out[cols] (+)= vector[rows] .
// matrix[rows x cols]; `dtype` operands and output.
int vector_product(uint32_t dtype, bool row_vector, bool accumulate, uint64_t rows, uint64_t cols, const void* matrix,
                   const void* vector, void* out);

// Runtime compilation (fused.hip).  The straight-line body of an
// epilogue's `group(live, row, col, N, product)` over `elems` elements, for
// `code` computing in `dtype` with loads through `places` (their folded axes
// are written into the source), its constants appended to `*constants`
// (input 0 the product when `product_input`); and the kernels `kernels` of
// `source`, compiled by hiprtc with the embedded headers on the source's
// second request and cached for the process (false until then, or if it
// does not compile).
std::string epilogue_group(const tc_encoded* code, uint32_t count, uint32_t dtype, bool product_input, int elems,
                           const tc_place* places, std::vector<float>* constants);
// The run form of the same program, for a kernel that hands it whole runs
// of E consecutive columns of one row (all inside C or none) and loads what
// every row shares once: the members `Invariant`, `invariant(inv, live,
// col)` (the runs starting at column `col`, loaded when `live`) and
// `run(inv, live, row, col, N, product)`.  Loads of contiguous columns and
// stores move 16-byte pieces: E = kEpilogueRun (16-bit products) streams its
// stores past the caches, E = 4 (f32 products, one piece a run) stores
// plainly; the caller checks their alignment.  Empty when a load's place
// steps through its columns other than by 0 or 1, or folds rows.
std::string epilogue_runs(const tc_encoded* code, uint32_t count, uint32_t dtype, const tc_place* places,
                          std::vector<float>* constants, int E = kEpilogueRun);
// Whether a program over `cols` columns may run in runs of `width` columns
// moved in 16-byte pieces, or as one piece when the run is shorter (four
// 16-bit elements: 8 bytes): `cols` a multiple of the run, every output
// it stores and every load of contiguous columns starting on a piece, every
// load's rows stepping by whole pieces, and no place stepping through its
// columns other than by 0 or 1 or folding more than one row axis.  With
// `product_input`, input 0 is a product kernel's own result and not checked.
bool runs_allowed(uint64_t cols, const tc_encoded* code, uint32_t count, const tc_place* places,
                  const void* const* inputs, void* const* outputs, uint32_t output_count, bool product_input,
                  int width = kEpilogueRun);
// What the compiler's resource report says of a compiled kernel: scratch
// bytes a lane and architectural VGPRs (UINT32_MAX where it said nothing).
struct KernelResources {
    uint32_t scratch = UINT32_MAX;
    uint32_t vgprs = UINT32_MAX;
};
bool compiled_kernels(const std::string& source, const std::vector<std::string>& kernels, hipFunction_t* out,
                      KernelResources* resources = nullptr);
// Whether hiprtc in this process compiles with the code-object compiler of
// the ROCm the library was built against (fused.hip).
bool runtime_compiler_is_ours();

// `fused_sum` over rows as one compiled kernel (fused.hip): the checked
// program's one output summed per row into `out`, rounded once to `dtype`.
// Sets `*done` false, launching nothing, until the program has been seen
// before (or when it does not fit the compiled form).
int fused_row_sums(uint32_t dtype, const tc_encoded* code, uint32_t count, const tc_place* places,
                   uint32_t place_count, const void* const* inputs, const uint64_t* input_lens, uint32_t input_count,
                   uint64_t rows, uint64_t cols, void* out, bool* done);
// The same along columns: the output summed per column, the rows split
// over workgroups when there are few columns, the splits' sums added by a
// second kernel in split order.
int fused_column_sums(uint32_t dtype, const tc_encoded* code, uint32_t count, const tc_place* places,
                      uint32_t place_count, const void* const* inputs, const uint64_t* input_lens,
                      uint32_t input_count, uint64_t rows, uint64_t cols, void* out, bool* done);

// `fused_with_statistics` as one compiled kernel (fused.hip), for a checked
// program: each row's statistics computed in registers and the program run
// over that row.  Sets `*done` false, launching nothing, until the program
// has been seen before or when it does not fit the compiled form (a
// statistic read other than one value a row, more than four sources).
int fused_row_statistics(uint32_t dtype, const tc_encoded* code, uint32_t count, const tc_place* places,
                         uint32_t place_count, const void* const* inputs, const uint64_t* input_lens,
                         uint32_t input_count, void* const* outputs, const uint64_t* output_lens,
                         uint32_t output_count, uint64_t rows, uint64_t cols, const tc_row_stat* statistics,
                         uint32_t statistic_count, bool* done);

std::string shape_text(const uint64_t* values, uint32_t rank);

// ---- element types (device.hpp) ---------------------------------------------

inline size_t dtype_size(uint32_t dtype) {
    switch (dtype) {
        case TC_F32: return 4;
        case TC_F16:
        case TC_BF16: return 2;
        case TC_F64: return 8;
        default: return 0;
    }
}

inline const char* dtype_name(uint32_t dtype) {
    switch (dtype) {
        case TC_F32: return "f32";
        case TC_F16: return "f16";
        case TC_BF16: return "bf16";
        case TC_F64: return "f64";
        default: return "unknown";
    }
}

// Call `body` with a value of the storage type `dtype` names (only its type
// matters); unsupported types are reported, never computed some other way.
#define TC_DISPATCH_FLOAT(dtype, what, S, ...)                                        \
    switch (dtype) {                                                                  \
        case TC_F32: { using S = float; __VA_ARGS__; break; }                         \
        case TC_F16: { using S = _Float16; __VA_ARGS__; break; }                      \
        case TC_BF16: { using S = ::tc::bf16_t; __VA_ARGS__; break; }                 \
        default:                                                                      \
            return ::tc::fail(TC_UNSUPPORTED, std::string(what) + ": no kernel for " + \
                                                  ::tc::dtype_name(dtype));           \
    }

// ---- the scalar operations every kernel shares -----------------------------

__device__ inline float binary_value(uint32_t op, float a, float b) { return tc_binary(op, a, b); }
__device__ inline float compare_value(uint32_t op, float a, float b) { return tc_compare(op, a, b); }

// `Pairwise::value` (kernels.rs:431-441); a power is f32 `powf`
// (numbers/primitive.rs:131-156).
__device__ inline float pairwise_value(uint32_t kind, uint32_t op, float a, float b) {
    if (kind == TC_PAIR_ARITHMETIC) return binary_value(op, a, b);
    if (kind == TC_PAIR_COMPARE) return compare_value(op, a, b);
    return powf(a, b);
}

// ---- index arithmetic -------------------------------------------------------

// Unsigned 32-bit division by an invariant divisor as a multiply and a shift
// (Granlund and Montgomery, "Division by invariant integers using
// multiplication", 1994): with l = ceil(log2 d) and
// m = floor(2^32 (2^l - d) / d) + 1, n / d = (mulhi(m, n) + n) >> l for every
// n < 2^32.
struct DivMod {
    uint32_t divisor = 1;
    uint32_t multiplier = 0;
    uint32_t shift = 0;

    DivMod() = default;
    explicit DivMod(uint32_t d) : divisor(d) {
        uint32_t l = 0;
        while (l < 32 && (uint64_t{1} << l) < d) l++;
        shift = l;
        multiplier = static_cast<uint32_t>(((uint64_t{1} << 32) * ((uint64_t{1} << l) - d)) / d + 1);
    }
    __device__ __forceinline__ uint32_t div(uint32_t n) const {
        uint32_t t = __umulhi(n, multiplier);
        return static_cast<uint32_t>((static_cast<uint64_t>(t) + n) >> shift);
    }
};

// Division by an extent in index type I: multiply-shift for 32-bit indices,
// a plain divide for 64-bit ones.
template <typename I>
struct Div;
template <>
struct Div<uint32_t> {
    DivMod dm;
    void set(uint64_t d) { dm = DivMod(static_cast<uint32_t>(d)); }
    __device__ __forceinline__ uint32_t div(uint32_t n) const { return dm.div(n); }
};
template <>
struct Div<uint64_t> {
    uint64_t d = 1;
    void set(uint64_t v) { d = v; }
    __device__ __forceinline__ uint64_t div(uint64_t n) const { return n / d; }
};

inline bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

// ---- streaming ------------------------------------------------------------------

// A kernel whose traffic exceeds MI355X's 256 MiB Infinity Cache streams
// from HBM: its 16-byte loads and stores then carry the nontemporal hint, so
// lines that will not be reused do not displace ones that will, and each
// thread moves four 16-byte words per pass.  Below it, the data is mostly
// cache-resident and plain accesses, one word per thread, are faster
// (measured on MI355X: 6.3 vs 4.9 TB/s for a 768 MiB add; 7.5 vs 6.3 TB/s
// for a 96 MiB one).
constexpr uint64_t kStreamBytes = uint64_t{256} << 20;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ uint4 load_word(const void* p) {
    if (NT) {
        const u32x4 v = __builtin_nontemporal_load(static_cast<const u32x4*>(p));
        return uint4{v.x, v.y, v.z, v.w};
    }
    return *static_cast<const uint4*>(p);
}

template <bool NT>
__device__ __forceinline__ void store_word(void* p, uint4 v) {
    if (NT) {
        __builtin_nontemporal_store(u32x4{v.x, v.y, v.z, v.w}, static_cast<u32x4*>(p));
    } else {
        *static_cast<uint4*>(p) = v;
    }
}

// Blocks of 256 threads for a one-pass kernel over `work` items, `per_thread`
// items a thread (never zero blocks).  A dispatch holds fewer than 2^32
// work-items, so past 2^24 - 1 blocks the kernels loop.
inline uint32_t blocks_for(uint64_t work, uint32_t per_thread) {
    const uint64_t per_block = uint64_t{256} * per_thread;
    uint64_t blocks = (work + per_block - 1) / per_block;
    if (blocks == 0) blocks = 1;
    if (blocks > 0xffffffu) blocks = 0xffffffu;
    return static_cast<uint32_t>(blocks);
}

// A joint layout of up to `kMaxRank` axes over `N` operands, after
// coalescing: the extents, a divider per axis, and each operand's strides.
template <int N>
struct Walk {
    int rank = 0;
    uint64_t shape[kMaxRank] = {};
    uint64_t strides[N][kMaxRank] = {};
    uint64_t offsets[N] = {};
};

// `coalesce` (tensors/layout.rs:419-449): axes of one element dropped, and an
// axis merged into the one before it wherever every operand steps across the
// pair as across one axis.  The row-major walk order is unchanged.
template <int N>
Walk<N> coalesce(uint32_t rank, const uint64_t* shape, const uint64_t* const* strides,
                 const uint64_t* offsets) {
    Walk<N> walk;
    for (int n = 0; n < N; n++) walk.offsets[n] = offsets[n];
    for (uint32_t axis = 0; axis < rank; axis++) {
        uint64_t extent = shape[axis];
        if (extent == 1) continue;
        int r = walk.rank;
        bool joins = r > 0;
        for (int n = 0; joins && n < N; n++) {
            joins = walk.strides[n][r - 1] == strides[n][axis] * extent;
        }
        if (joins) {
            walk.shape[r - 1] *= extent;
            for (int n = 0; n < N; n++) walk.strides[n][r - 1] = strides[n][axis];
        } else {
            walk.shape[r] = extent;
            for (int n = 0; n < N; n++) walk.strides[n][r] = strides[n][axis];
            walk.rank++;
        }
    }
    return walk;
}

// The number of elements of `shape`, or false on overflow (layout.rs:96-103).
inline bool element_count(uint32_t rank, const uint64_t* shape, uint64_t* count) {
    uint64_t total = 1;
    for (uint32_t k = 0; k < rank; k++) {
        if (shape[k] != 0 && total > UINT64_MAX / shape[k]) return false;
        total *= shape[k];
    }
    *count = total;
    return true;
}

// One past the last element a layout reads, 0 if it reads none, or false on
// overflow (`reach`, layout.rs:138-149).
inline bool reach(uint32_t rank, const uint64_t* shape, uint64_t offset, const uint64_t* strides,
                  uint64_t* end) {
    for (uint32_t k = 0; k < rank; k++) {
        if (shape[k] == 0) {
            *end = 0;
            return true;
        }
    }
    uint64_t at = offset;
    for (uint32_t k = 0; k < rank; k++) {
        uint64_t extent = shape[k] - 1;
        if (strides[k] != 0 && extent > (UINT64_MAX - at) / strides[k]) return false;
        at += extent * strides[k];
    }
    if (at == UINT64_MAX) return false;
    *end = at + 1;
    return true;
}

// `check_strided` (tensors/backend.rs:226-252): TC_OK with the element count,
// or TC_INVALID with the reference's message.
int check_strided(uint64_t len, uint32_t rank, const uint64_t* shape, uint64_t offset,
                  const uint64_t* strides, const char* operation, uint64_t* count);

// Blocks for a grid-stride kernel over `work` items of `per_block` each,
// capped so the grid stays a few waves deep on every CU.
inline uint32_t grid_for(uint64_t work, uint32_t per_block, uint32_t cap_per_cu = 16) {
    uint64_t blocks = (work + per_block - 1) / per_block;
    uint64_t cap = static_cast<uint64_t>(compute_units()) * cap_per_cu;
    if (blocks > cap) blocks = cap;
    if (blocks == 0) blocks = 1;
    return static_cast<uint32_t>(blocks);
}

}  // namespace tc
