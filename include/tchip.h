/*
 * tchip.h — the C ABI of the MI355X `Hip` storage and kernel backend for
 * tensorcrate.
 *
 * Every entry point takes plain device pointers, element counts and small
 * plain-old-data layout structs; nothing here names a C++ or torch type, so a
 * Rust `extern "C"` block (or ctypes, or cgo) binds it directly.  Each
 * declaration cites the reference interface it stands in for, as
 * `<file>:<line>` under arthurmburke/tensorcrate's `src/`.
 *
 * Conventions
 *  - Every function returns a `tc_status`.  On failure `tc_last_error()` holds
 *    a message for the calling thread, worded like the reference's panic for
 *    the same mistake ("strided copy: shape [..] ... reaches past N
 *    elements").  Layout checks run on the host before any launch, so a bad
 *    layout never reaches the GPU.  A call with elements to read or write
 *    refuses a null device pointer the same way (TC_INVALID, "<operation>: a
 *    null operand"); an empty call may pass null.
 *  - All work is queued asynchronously on one HIP stream per host thread and
 *    ordered on it; `tc_sync` waits for it.  Host pointers passed to
 *    `tc_upload` / `tc_download` are done with when the call returns.
 *  - Element counts and strides are in elements of the operand's type, not
 *    bytes, as the reference's `Strided`/`Region` are (backend.rs:199-213).
 *  - Storage is not shared between threads: a pointer is allocated, used and
 *    freed on one thread, as the reference's Metal tensors are not `Send`.
 */
#ifndef TCHIP_H
#define TCHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The deepest layout a strided operation takes: `MAX_RANK` (tensors/layout.rs:16). */
#define TC_MAX_RANK 6
/* Registers, inputs, outputs, instructions and loads of one fused program
 * (tensors/fused/mod.rs:119-132, :483). */
#define TC_FUSED_REGISTERS 16
#define TC_FUSED_MAX_INPUTS 16
#define TC_FUSED_MAX_OUTPUTS 8
#define TC_FUSED_MAX_INSTRUCTIONS 256
#define TC_FUSED_MAX_LOADS 64
/* Row axes a fused program's place folds together (fused/mod.rs:3236). */
#define TC_FUSED_LEAD 5

typedef enum tc_status {
    TC_OK = 0,
    TC_INVALID = 1,     /* a shape, layout or argument the reference would panic on */
    TC_UNSUPPORTED = 2, /* a type or operation with no kernel: never a silent fallback */
    TC_DEVICE = 3,      /* a HIP runtime error */
    TC_OUT_OF_MEMORY = 4,
    TC_FORMAT = 5, /* a stored tensor this build does not read: the reference's `Error::Format` */
    TC_IO = 6      /* a file that cannot be opened, read or written, or ends early: `Error::Io` */
} tc_status;

/* Storage and arithmetic types: `fused::DType` (fused/mod.rs:145-150). */
typedef enum tc_dtype { TC_F32 = 0, TC_F16 = 1, TC_BF16 = 2, TC_F64 = 3 } tc_dtype;

/* `BinaryOp` (tensors/kernels.rs:32-38). */
typedef enum tc_binary_op { TC_ADD = 0, TC_SUB = 1, TC_MUL = 2, TC_DIV = 3, TC_REM = 4 } tc_binary_op;

/* `Compare` (tensors/kernels.rs:106-122). */
typedef enum tc_compare_op {
    TC_MIN = 0, TC_MAX = 1, TC_MAX_SHARE = 2,
    TC_LESS = 3, TC_LESS_EQUAL = 4, TC_GREATER = 5, TC_GREATER_EQUAL = 6
} tc_compare_op;

/* `Reduce` (tensors/kernels.rs:183-187). */
typedef enum tc_reduce_op { TC_REDUCE_SUM = 0, TC_REDUCE_MIN = 1, TC_REDUCE_MAX = 2 } tc_reduce_op;

/* `Pairwise` (tensors/kernels.rs:411-415): the kind, then the `BinaryOp` or
 * `Compare` code in a separate argument. */
typedef enum tc_pairwise { TC_PAIR_ARITHMETIC = 0, TC_PAIR_COMPARE = 1, TC_PAIR_POWER = 2 } tc_pairwise;

/* `AxisReduction` (tensors/kernels.rs:449-457): `Fold(Reduce)`, `Mean`, or
 * `Variance { divisor }`. */
typedef enum tc_axis_reduction { TC_AXIS_FOLD = 0, TC_AXIS_MEAN = 1, TC_AXIS_VARIANCE = 2 } tc_axis_reduction;

/* `Axis` (tensors/kernels.rs:482-487): fold each row, or each column. */
typedef enum tc_axis { TC_AXIS_ROWS = 0, TC_AXIS_COLUMNS = 1 } tc_axis;

/* `Transposed` (tensors/kernels.rs:462-467), with `TC_PLAIN` for neither. */
typedef enum tc_transposed { TC_PLAIN = 0, TC_LEFT = 1, TC_RIGHT = 2 } tc_transposed;

/* One side of a strided copy: element [i0..] of a shape is storage element
 * `offset + sum(i_k * strides[k])` (`Strided`, tensors/backend.rs:199-202). */
typedef struct tc_strided {
    uint64_t offset;
    uint64_t strides[TC_MAX_RANK];
} tc_strided;

/* One block of an assemble or a strided write: `shape` copied from `source`
 * (holding `source_len` elements) at `from` to the target at `to`
 * (`Region`, tensors/backend.rs:208-213). */
typedef struct tc_region {
    const void* source;
    uint64_t source_len;
    uint32_t rank;
    uint64_t shape[TC_MAX_RANK];
    tc_strided from;
    tc_strided to;
} tc_region;

/* How a reduction walks its input (`Split`, tensors/layout.rs:370-376): the
 * output at kept index [k..] reduces the storage elements at
 * offset + Σ k_i·kept_strides[i] + Σ f_j·folded_strides[j], for every folded
 * index [f..] within `folded`. */
typedef struct tc_split {
    uint64_t offset;
    uint32_t kept_rank;
    uint64_t kept[TC_MAX_RANK];
    uint64_t kept_strides[TC_MAX_RANK];
    uint32_t folded_rank;
    uint64_t folded[TC_MAX_RANK];
    uint64_t folded_strides[TC_MAX_RANK];
} tc_split;

/* One instruction of a fused program as the kernels read it, twelve bytes
 * (`Encoded`, tensors/fused/mod.rs:1391-1410):
 *   kind 0 load  : op = load index, dst, a = input slot, b = storage dtype
 *   kind 1 const : dst, value
 *   kind 2 binary: op = BinaryOp, dst, a, b
 *   kind 3 unary : op = Analytic, dst, a
 *   kind 4 cmp   : op = Compare, dst, a, b
 *   kind 5 store : a = source register, b = storage dtype, aux = output slot */
typedef struct tc_encoded {
    uint16_t kind;
    uint16_t op;
    uint8_t dst;
    uint8_t a;
    uint8_t b;
    uint8_t aux;
    float value;
} tc_encoded;

/* Where element (row, col) of a rows x cols walk reads a load: storage
 * element `offset + col*col_step`, plus the row split over the `lead` axes
 * it folds together, outermost first (`Place`, fused/mod.rs:3229-3268). */
typedef struct tc_place {
    uint64_t offset;
    uint64_t col_step;
    uint32_t lead;
    uint64_t dims[TC_FUSED_LEAD];
    uint64_t steps[TC_FUSED_LEAD];
} tc_place;

/* ---- context, stream, errors ------------------------------------------- */

/* Select the device for the calling thread and create its stream.  Every
 * other entry point calls it for device 0 if the thread has not.  Replaces
 * the thread-local Metal device (metal/device.rs:309-313). */
int tc_init(int device);

/* The last failure's message on this thread ("" when none).  The Rust side
 * maps it onto the panic `require_metal` raises (tensors/backend.rs:422-426). */
const char* tc_last_error(void);

/* Wait for all work queued by this thread, and report any asynchronous
 * failure — the HIP form of `sync` (metal/sync.rs:225-259). */
int tc_sync(void);

/* The calling thread's HIP stream (a `hipStream_t`), for callers that order
 * their own work against this library's. */
int tc_stream(void** stream);

/* The device's marketing name and architecture string, e.g. "gfx950". */
int tc_device_info(char* name, size_t name_len, char* arch, size_t arch_len);

/* GPU time between `tc_timer_begin` and `tc_timer_end` on this thread's
 * stream, in milliseconds; `tc_timer_end` waits for the stream. */
int tc_timer_begin(void);
int tc_timer_end(float* milliseconds);

/* ---- storage (Backend, tensors/backend.rs:86-111) ---------------------- */

/* Device storage of `bytes` from this thread's stream-ordered cache.
 * `Backend::store` / `from_vec` allocate with this and then upload. */
int tc_alloc(size_t bytes, void** out);
/* Return storage to the calling thread's cache; work already queued that
 * reads it still completes first (the pool fence of metal/pool.rs:34-48).
 * Storage allocated or freed while the thread's stream is being captured
 * into a HIP graph stays with the graphs, which touch it again on every
 * replay: it is reused only within the capture that freed it, and after
 * that capture ends it is retired, handed to no other allocation. */
int tc_free(void* pointer);
/* Give every cached, unused block back to the device (retired graph
 * storage excepted).  Refused while the stream is capturing. */
int tc_empty_cache(void);
/* The caller's promise that no graph captured on this thread will run
 * again: retired graph storage returns to the cache and live graph storage
 * becomes ordinary.  No reference counterpart (Metal has no graphs); the
 * fence of metal/pool.rs:34-48 applied to replays. */
int tc_release_graph_memory(void);
/* Bytes of live and of retired (or capture-free) graph storage. */
int tc_graph_memory(uint64_t* live_bytes, uint64_t* retired_bytes);
/* This thread's operations queued on its stream (kernel launches and device
 * copies) and the times the host waited for the stream, since the thread
 * began: the `dispatches` and `syncs` of counters::Counts
 * (src/counters.rs:33-57, recorded at :100-135). */
int tc_activity(uint64_t* dispatches, uint64_t* waits);
/* Host to device, device to host (`as_slice`, backend.rs:99; the download
 * waits for queued work), and device to device (`duplicate`, backend.rs:111).
 * From 8 MiB up the first two take the pinned staging of tc_upload_staged. */
int tc_upload(void* device_dst, const void* host_src, size_t bytes);
int tc_download(void* host_dst, const void* device_src, size_t bytes);
int tc_copy(void* device_dst, const void* device_src, size_t bytes);
/* `count` elements of `width` bytes set to `*value` on the device: the
 * device-side `Vector::filled` / `Matrix::filled` (vector.rs:101,
 * matrix.rs:112), so a zero adjoint is never a host upload. */
int tc_fill(void* dst, uint64_t count, uint32_t width, const void* value);

/* ---- strided copies (Backend, tensors/backend.rs:141-173) --------------- */

/* `Backend::strided_copy` (backend.rs:141-145; Host backend.rs:255-274):
 * the `rank`-axis layout `from` of `src` (holding `src_len` elements of
 * `width` bytes, width 1/2/4/8/16) copied row-major into `dst`, which holds
 * the product of `shape` elements. */
int tc_strided_copy(uint32_t width, const void* src, uint64_t src_len, uint32_t rank,
                    const uint64_t* shape, const tc_strided* from, void* dst);

/* `Backend::assemble` (backend.rs:157-160; Host backend.rs:303-323): each
 * region copied into `dst` of `len` elements.  Elements no region writes are
 * left as they were (the reference leaves them unspecified). */
int tc_assemble(uint32_t width, void* dst, uint64_t len, const tc_region* regions, uint32_t count);

/* `Backend::strided_write` (backend.rs:170-173; Host backend.rs:277-300):
 * `region` copied into `target` (holding `target_len` elements) in place. */
int tc_strided_write(uint32_t width, void* target, uint64_t target_len, const tc_region* region);

/* ---- elementwise (Kernels, tensors/kernels.rs:832-863, :912-938) -------- */

/* `vector_elementwise` / `matrix_elementwise` (kernels.rs:832, :912):
 * out[i] = a[i] op b[i], one rounding to `dtype`. */
int tc_elementwise(uint32_t dtype, uint32_t op, const void* a, const void* b, void* out, uint64_t n);
/* `vector_broadcast` / `matrix_broadcast` (kernels.rs:838, :918):
 * out[i] = a[i] op s, or s op a[i] when `scalar_left`.  `scalar` is a value
 * of `dtype`, which float holds exactly. */
int tc_broadcast(uint32_t dtype, uint32_t op, const void* a, float scalar, int scalar_left,
                 void* out, uint64_t n);
/* `vector_compare` / `matrix_compare` (kernels.rs:846, :926). */
int tc_compare(uint32_t dtype, uint32_t op, const void* a, const void* b, void* out, uint64_t n);
/* `vector_compare_scalar` / `matrix_compare_scalar` (kernels.rs:849, :929). */
int tc_compare_scalar(uint32_t dtype, uint32_t op, const void* a, float scalar, int scalar_left,
                      void* out, uint64_t n);
/* `vector_clamp` / `matrix_clamp` (kernels.rs:863, :938): min(max(x, low),
 * high).  Fails when low > high (shape.rs:30-43); a NaN bound passes and is
 * inert. */
int tc_clamp(uint32_t dtype, const void* a, float low, float high, void* out, uint64_t n);

/* `Kernels::strided_binary` (kernels.rs:1162-1166; Host strided.rs:29-78):
 * out = op(a, b) element by element over `shape`, written row-major; a and b
 * are addressed through their own strided layouts, so a stride of 0 reuses
 * one element along that axis (broadcasting) without copying.  `kind` is a
 * `tc_pairwise`; `op` its BinaryOp or Compare. */
int tc_strided_binary(uint32_t dtype, uint32_t kind, uint32_t op, uint32_t rank,
                      const uint64_t* shape, const void* a, uint64_t a_len, const tc_strided* a_at,
                      const void* b, uint64_t b_len, const tc_strided* b_at, void* out);

/* ---- transfers and the TCR1 format (persist.rs:44-93) -------------------- */

/* Host memory to and from HBM through the thread's two pinned staging
 * buffers (16 MiB each, allocated on first use and held until the process
 * ends), the CPU copying one chunk while the DMA engine moves the other.
 * For pageable memory (`to_backend`, `as_slice`, tensors/backend.rs); the
 * host buffer is free again when the call returns. */
int tc_upload_staged(void* device_dst, const void* host_src, size_t bytes);
int tc_download_staged(void* host_dst, const void* device_src, size_t bytes);

/* A small read (at most 64 bytes, such as a reduction's scalar) queued
 * behind the thread's work into one of its 1024 pinned slots, returning at
 * once with a `ticket` (the tape's unread loss, `Lazy`, tape/mod.rs:253-295:
 * the value is only waited for when something reads it). */
int tc_read_async(const void* device_src, size_t bytes, uint64_t* ticket);
/* Wait for that read alone and copy its bytes to `host_dst`; TC_INVALID for
 * a ticket this thread never issued or whose slot 1024 later reads reused. */
int tc_read_wait(uint64_t ticket, void* host_dst, size_t bytes);

/* A TCR1 record's header (persist.rs:44-93): `kind` 0 vector, 1 matrix, 2
 * tensor; `rank` extents in `shape` (a vector's length, a matrix's rows and
 * columns); `count` elements of `element_bytes` each, the payload at byte
 * `data_offset` of the file and the record ending at `end_offset` (where a
 * next record may begin). */
typedef struct tc_tcr1 {
    uint32_t kind;
    uint32_t rank;
    uint64_t shape[TC_MAX_RANK];
    uint64_t count;
    uint64_t element_bytes;
    uint64_t data_offset;
    uint64_t end_offset;
} tc_tcr1;

/* `read_from`'s header checks (persist.rs:266-330, :330-333, :453-480) for
 * the record at byte `offset` of `path`, read into a target whose element
 * tag is `tag` (persist.rs:105-189: f32 0x10, f16 0x12, bf16 0x13, ...) and
 * whose kind is `kind` (a tensor target, 2, also reads vector and matrix
 * records): TC_FORMAT with the reference's message for a wrong magic,
 * version, kind, element type or too many axes; TC_IO for a file that ends
 * before the record does. */
int tc_tcr1_read_header(const char* path, uint64_t offset, const uint8_t* tag, uint32_t tag_length,
                        uint32_t kind, tc_tcr1* out);

/* The record's payload, as stored, into `device_dst` (`count *
 * element_bytes` bytes): read from the file into pinned staging and copied
 * to HBM, the two overlapped. */
int tc_tcr1_load(const char* path, const tc_tcr1* header, void* device_dst);

/* `write_to` (persist.rs:350-430) from the device: the header for `kind`,
 * `rank` extents and element `tag`, then the `count * element size` bytes
 * at `device_src`, copied to pinned staging and written to `path`
 * (truncated, or appended to when `append` is nonzero). */
int tc_tcr1_save(const char* path, int append, uint32_t kind, uint32_t rank, const uint64_t* shape,
                 const uint8_t* tag, uint32_t tag_length, const void* device_src);

/* ---- scans and sorts (kernels.rs:870-873) -------------------------------- */

/* `Kernels::vector_prefix_sum` (kernels.rs:870; Host vector.rs:578-589,
 * compact.rs:209-221): the inclusive running sum of `n` elements,
 * accumulated in f32 and rounded to `dtype` per output.  A deterministic
 * tree order (the same bits every run); within the rounding of a sum of
 * that many terms of the host's left-to-right order. */
int tc_prefix_sum(uint32_t dtype, const void* a, void* out, uint64_t n);

/* `Kernels::vector_sort` (kernels.rs:873; Host `Vector::sorted`): the `n`
 * elements in `order` (a `SortOrder`, kernels.rs:252-255: 0 ascending, 1
 * descending) of IEEE totalOrder (`total_cmp`), exactly. */
int tc_sort(uint32_t dtype, const void* a, void* out, uint64_t n, uint32_t order);

/* ---- analytic functions and powers (kernels.rs:876-895, :941-949) ------- */

/* `Kernels::vector_unary` / `matrix_unary` (kernels.rs:876, :941): `op` (an
 * `Analytic`, kernels.rs:293-308) of each element, in f32 and rounded to
 * `dtype` once; for f16 and bf16, `Sec` and `Csc` are the reciprocal in
 * `dtype` of the rounded cosine or sine (vmath.rs:483-507).  The device's
 * own f32 functions stand in for the host's `vmath` ones: within a few ulp
 * of each other, both within a few ulp of the exact value. */
int tc_unary(uint32_t dtype, uint32_t op, const void* a, void* out, uint64_t n);

/* `Kernels::vector_unary_dual` / `matrix_unary_dual` (kernels.rs:891, :949):
 * `out_value = op(value)` and `out_tangent = op'(value) * tangent`, the
 * derivative as `Analytic::derivative` composes it (kernels.rs:358-385),
 * one rounding to `dtype` per operation. */
int tc_unary_dual(uint32_t dtype, uint32_t op, const void* value, const void* tangent, void* out_value,
                  void* out_tangent, uint64_t n);

/* `Kernels::vector_power` / `matrix_power` (kernels.rs:884, :944): elementwise
 * `a^b`, `powf` in f32 rounded once (primitive.rs:133-150). */
int tc_power(uint32_t dtype, const void* a, const void* b, void* out, uint64_t n);

/* `Kernels::vector_power_scalar` / `matrix_power_scalar` (kernels.rs:888,
 * :947): `scalar^x` when `scalar_left`, else `x^scalar`, the latter with the
 * host's exact fast exponents 0, 1, 2, 1/2 and -1 for f32
 * (analytic.rs:415-476). */
int tc_power_scalar(uint32_t dtype, const void* a, float scalar, int scalar_left, void* out, uint64_t n);

/* ---- reductions (kernels.rs:867, :1175, :1187) -------------------------- */

/* `Kernels::reduce_axes` (kernels.rs:1175-1179; Host strided.rs:105-162):
 * one result per kept index, folded over `split->folded`, accumulated in f32
 * and rounded to `dtype` once.  `kind` is a `tc_axis_reduction`; `op` the
 * `Reduce` of a fold; `divisor` the variance's divisor
 * (statistics/mod.rs:96-101).  Every slice holds at least one element. */
int tc_reduce_axes(uint32_t dtype, const void* input, uint64_t input_len, const tc_split* split,
                   uint32_t kind, uint32_t op, uint64_t divisor, void* out);

/* `Kernels::arg_reduce` (kernels.rs:1187; Host strided.rs:186-225): the
 * u32 position along the one folded axis of each slice's first maximum
 * (`op` TC_REDUCE_MAX) or minimum (TC_REDUCE_MIN); NaNs are passed over and
 * an all-NaN slice answers 0.  `split` folds exactly one axis. */
int tc_arg_reduce(uint32_t dtype, const void* input, uint64_t input_len, const tc_split* split,
                  uint32_t op, uint32_t* out);

/* `Kernels::vector_reduce` (kernels.rs:867): the whole buffer folded; the
 * f32 accumulator is written to the device scalar `result`, unrounded, as
 * Metal's `reduce` returns it (tensors/backend.rs:813-818). */
int tc_vector_reduce(uint32_t dtype, const void* a, uint64_t n, uint32_t op, float* result);

/* `tc_vector_reduce` that allocates nothing, with identical results: its
 * block partials go to a 16 KiB array the library holds on each GPU (4096
 * f32, enough for any length on parts of up to 1024 CUs; more partials are
 * refused with TC_UNSUPPORTED).  No counterpart in the reference: it is for
 * callers that cannot allocate (code under HIP graph capture, tight serving
 * loops).  Every call on one GPU shares that array, which belongs to the
 * stream of the last call that used it: a call from another stream while
 * that call is still queued is refused with TC_UNSUPPORTED instead of
 * racing.  Replays of a captured call are not tracked, so a graph holding
 * one must not replay beside other users of the array on that GPU. */
int tc_vector_reduce_noalloc(uint32_t dtype, const void* a, uint64_t n, uint32_t op, float* result);

/* `Kernels::vector_moments` / `matrix_moments` (kernels.rs:1035-1038; Host
 * `moments_of`, statistics/mod.rs:419-441): the mean of all `n` elements into
 * the device f32 `result[0]` and the sum of squared deviations from it into
 * `result[1]`, unrounded (the caller rounds to the element type, as the
 * compact types do); NaNs for no elements. */
int tc_moments(uint32_t dtype, const void* a, uint64_t n, float* result);

/* `Kernels::matrix_axis_moments` (kernels.rs:1042; Host
 * statistics/mod.rs:451-520): per row (`axis` TC_AXIS_ROWS) or per column
 * of the row-major rows x cols matrix `a`, the mean into `means` and the sum
 * of squared deviations into `deviations`, accumulated in f32 and rounded to
 * `dtype` once; NaNs along an empty axis. */
int tc_axis_moments(uint32_t dtype, const void* a, uint64_t rows, uint64_t cols, uint32_t axis, void* means,
                    void* deviations);

/* `Family` and `Statistic` (kernels.rs:536-590), the reference's u16 codes. */
typedef enum tc_family { TC_NORMAL = 0, TC_INVERSE_GAUSSIAN = 1 } tc_family;
typedef enum tc_statistic { TC_PDF = 0, TC_CDF = 1, TC_PPF = 2 } tc_statistic;

/* `Kernels::vector_distribution` / `matrix_distribution` (kernels.rs:
 * 1046-1059; Host statistics/mod.rs:649-651, :733-735): `statistic` of the
 * `family` distribution with parameters (first, second) -- (mean, stddev)
 * for the normal, (mean, shape) for the inverse Gaussian, each a `dtype`
 * value widened exactly to f32 -- at each of the `n` elements, evaluated in
 * f64 by the Host's methods (statistics/special.rs) and rounded once to f32,
 * then to `dtype`.  Parameters that are not positive give NaNs. */
int tc_distribution(uint32_t dtype, uint32_t family, uint32_t statistic, const void* a, void* out, uint64_t n,
                    float first, float second);

/* `Kernels::matrix_axis_distribution` (kernels.rs:1063-1070; Host
 * `distribution_axis`, statistics/mod.rs:785-801, :582-600): as
 * tc_distribution over the row-major rows x cols `a`, with the parameter
 * pair of each element's row (`axis` TC_AXIS_ROWS: `first`/`second` hold
 * `rows` device values of `dtype`) or column (TC_AXIS_COLUMNS: `cols`). */
int tc_axis_distribution(uint32_t dtype, uint32_t family, uint32_t statistic, const void* a, uint64_t rows,
                         uint64_t cols, uint32_t axis, const void* first, const void* second, void* out);

/* `Kernels::dot` (kernels.rs:897): sum a[i]*b[i] into the device f32 scalar
 * `result`, unrounded. */
int tc_dot(uint32_t dtype, const void* a, const void* b, uint64_t n, float* result);

/* ---- products (kernels.rs:897-908, :956-987) ---------------------------- */

/* `Kernels::matmul` / `matmul_add` / `matmul_transposed_add`
 * (kernels.rs:956, :963, :975; Host matrix.rs:580-667, compact.rs:232-253):
 *   transposed TC_PLAIN: C[m x n] (+)= A[m x k] . B[k x n]
 *   transposed TC_LEFT : C (+)= A^T . B with A stored k x m
 *   transposed TC_RIGHT: C (+)= A . B^T with B stored n x k
 * all row-major.  `accumulate` adds to C (the addend the reference consumes
 * as its accumulator) instead of overwriting it.  A and B are `in_dtype`,
 * accumulation is f32, and C is `out_dtype`: `in_dtype` itself, or TC_F32
 * for the compact types' `matmul_f32`.  k == 0 gives zeros (or the addend). */
int tc_matmul(uint32_t in_dtype, uint32_t out_dtype, uint32_t transposed, int accumulate,
              uint64_t m, uint64_t k, uint64_t n, const void* a, const void* b, void* c);

/* `Kernels::matvec` / `matvec_add` (kernels.rs:901-908; Host matrix.rs:675-737):
 * y[rows] (+)= M[rows x cols] . v[cols]. */
int tc_matvec(uint32_t dtype, int accumulate, uint64_t rows, uint64_t cols,
              const void* matrix, const void* vector, void* out);

/* `Kernels::vecmat` (kernels.rs:899; vector.rs:491): y[cols] = v[rows] . M[rows x cols]. */
int tc_vecmat(uint32_t dtype, uint64_t rows, uint64_t cols, const void* vector,
              const void* matrix, void* out);

/* `Kernels::transpose` (kernels.rs:987; matrix.rs:740, :1173-1206): the
 * cols x rows transpose of a rows x cols matrix of `width`-byte elements. */
int tc_transpose(uint32_t width, uint64_t rows, uint64_t cols, const void* src, void* dst);

/* ---- correlation, padding, flipping (kernels.rs:990-1029) --------------- */

/* `Kernels::correlate` (kernels.rs:998; Host `correlate_values`,
 * kernels.rs:1720-1750): the valid correlation of the row-major rows x cols
 * `input` with the window_rows x window_cols `window` into
 * (rows - window_rows + 1) x (cols - window_cols + 1) `out`; `flip` reverses
 * the window (convolution).  Each output sums its taps in row-major tap
 * order, a separate multiply and add each, in f32, rounded to `dtype` once:
 * the host's bits.  `correlate_window_gradient` is this with the adjoint as
 * the window (kernels.rs:1544-1551).  A window larger than the input is
 * refused with the reference's message. */
int tc_correlate(uint32_t dtype, const void* input, uint64_t rows, uint64_t cols, const void* window,
                 uint64_t window_rows, uint64_t window_cols, int flip, void* out);

/* `Kernels::correlate_input_gradient` (kernels.rs:1017; Host
 * kernels.rs:1754-1794): the full correlation of the adjoint_rows x
 * adjoint_cols `adjoint` with the window, the taps applied the other way
 * round from the forward pass's `forward_flip`, into the
 * (adjoint_rows + window_rows - 1) x (adjoint_cols + window_cols - 1) `out`;
 * the same order of operations as the host. */
int tc_correlate_input_gradient(uint32_t dtype, const void* adjoint, uint64_t adjoint_rows, uint64_t adjoint_cols,
                                const void* window, uint64_t window_rows, uint64_t window_cols, int forward_flip,
                                void* out);

/* `Kernels::pad` (kernels.rs:1025; Host kernels.rs:1575-1600): the rows x cols
 * matrix of `width`-byte elements surrounded by `pad_rows` and `pad_cols`
 * zeros on every side, into (rows + 2 pad_rows) x (cols + 2 pad_cols) `out`. */
int tc_pad(uint32_t width, const void* input, uint64_t rows, uint64_t cols, uint64_t pad_rows, uint64_t pad_cols,
           void* out);

/* `Kernels::flip` (kernels.rs:1028; Host kernels.rs:1531-1542): both axes of a
 * rows x cols matrix of `width`-byte elements reversed. */
int tc_flip(uint32_t width, const void* input, uint64_t rows, uint64_t cols, void* out);

/* ---- fused programs (kernels.rs:1077-1082; fused/mod.rs:959-1011) ------- */

/* `Kernels::fused`: run `count` encoded instructions for every element of a
 * rows x cols space, computing in `dtype`.  Load `k` reads through
 * `places[k]` from `inputs[slot]`; a store writes element row*cols + col of
 * `outputs[slot]`.  An in-place tensor is both an input and an output, and
 * is loaded unremapped before it is stored, so every element is read by the
 * thread that writes it.  `code`, `places` and the two length arrays are
 * host arrays; `input_lens[k]` / `output_lens[k]` count the elements of
 * each buffer, and a load or store that would reach past one is refused
 * before launch (`Program::run`'s checks, fused/mod.rs:978-986). */
int tc_fused(uint32_t dtype, const tc_encoded* code, uint32_t count, const tc_place* places,
             uint32_t place_count, const void* const* inputs, const uint64_t* input_lens,
             uint32_t input_count, void* const* outputs, const uint64_t* output_lens,
             uint32_t output_count, uint64_t rows, uint64_t cols);

/* `Kernels::row_moments` (kernels.rs:1090-1097; Host `host_row_moments`,
 * fused/mod.rs:4030-4041, and `moments_of`, statistics/mod.rs:419-441): the
 * rows x cols matrix `place` reads of `input` (stored as `input_dtype`,
 * `input_len` elements), converted to `dtype`, and per row its mean into
 * `means[rows]` and its sum of squared deviations from that mean into
 * `deviations[rows]`, accumulated in f32 and rounded to `dtype` once.  A
 * matrix with no columns gives NaNs. */
int tc_row_moments(uint32_t dtype, uint32_t input_dtype, const void* input, uint64_t input_len,
                   const tc_place* place, uint64_t rows, uint64_t cols, void* means, void* deviations);

/* One row statistic a program reads (`RowStatistic`, fused/mod.rs:547-553):
 * the mean, or the sum of squared deviations from it, of each row of the
 * rows x cols matrix `place` reads of `source` (stored as `source_dtype`,
 * `source_len` elements), as `tc_row_moments` gives them. */
typedef enum tc_row_statistic { TC_STAT_MEAN = 0, TC_STAT_DEVIATIONS = 1 } tc_row_statistic;
typedef struct tc_row_stat {
    const void* source;
    uint64_t source_len;
    uint32_t source_dtype;
    uint32_t which; /* a tc_row_statistic */
    tc_place place;
} tc_row_stat;

/* `Kernels::fused_with_statistics` (kernels.rs:1103-1113; `row_statistics`,
 * fused/mod.rs:3995-4027): run a program, as `tc_fused` does, whose inputs
 * are `inputs` followed by `statistic_count` row statistics, statistic i
 * being input slot `input_count + i`, a vector of `rows` values of `dtype`.
 * By default each distinct (source, type, place) has its moments computed
 * once by `tc_row_moments` and the program then runs with them; from the
 * program's second appearance, when every statistic is read one value a row
 * and at most four sources are involved, one compiled kernel computes each
 * row's statistics and runs the program over that row, so the statistics
 * are never stored.  Results then agree with the composition within the
 * statistics' rounding (the moments fold in another order). */
int tc_fused_with_statistics(uint32_t dtype, const tc_encoded* code, uint32_t count, const tc_place* places,
                             uint32_t place_count, const void* const* inputs, const uint64_t* input_lens,
                             uint32_t input_count, void* const* outputs, const uint64_t* output_lens,
                             uint32_t output_count, uint64_t rows, uint64_t cols, const tc_row_stat* statistics,
                             uint32_t statistic_count);

/* `Kernels::fused_sum` (kernels.rs:1120-1135; `Program::run_sum`,
 * fused/mod.rs:1048-1082; `axis_sum`, :4045-4051): run a program whose one
 * output is of type `dtype` (every store to output 0 as `dtype`) over a
 * rows x cols space, as `tc_fused` does, and sum that output along `axis`
 * (a `tc_axis`) into `out`: `rows` sums of rows, or `cols` sums of columns,
 * accumulated in f32 and rounded once.  The output itself is not returned. */
int tc_fused_sum(uint32_t dtype, const tc_encoded* code, uint32_t count, const tc_place* places,
                 uint32_t place_count, const void* const* inputs, const uint64_t* input_lens, uint32_t input_count,
                 uint64_t rows, uint64_t cols, uint32_t axis, void* out);

/* `Kernels::matmul_epilogue` (kernels.rs:1142-1149; Host `host_matmul`,
 * fused/mod.rs:4754-4766; checks in `Program::run_matmul`, :1143-1200): the
 * product A[m x k] . B[k x n] (row-major, `dtype`, as `tc_matmul` forms it)
 * is the program's input 0, read unremapped over the m x n space, and
 * `inputs` fill slots 1 on; outputs as `tc_fused`.  The program runs in the
 * product kernel's epilogue, so the product is not written to memory; the
 * results are the bits of `tc_matmul` then `tc_fused`.  A load of input 0
 * through any other place, or as another type, is refused. */
int tc_matmul_epilogue(uint32_t dtype, const tc_encoded* code, uint32_t count, const tc_place* places,
                       uint32_t place_count, uint64_t m, uint64_t k, uint64_t n, const void* a, const void* b,
                       const void* const* inputs, const uint64_t* input_lens, uint32_t input_count,
                       void* const* outputs, const uint64_t* output_lens, uint32_t output_count);

/* The source the runtime compiler builds `tc_matmul_epilogue`'s product
 * kernels from for this program (after the product kernels' header, the
 * epilogue type `CompiledStore`, its program as straight-line code), into
 * `out` (NUL-terminated, cut at `capacity` - 1 bytes) with its full length
 * in `*length`; `out` may be NULL to ask for the length.  `runs` nonzero
 * asks for the source of a launch whose operands allow the four-wave
 * kernel's run form (N a multiple of 8, 16-byte aligned operands), which it
 * contains when the program's places allow it too.  Needs no device.
 * No counterpart in the reference's interface: a diagnostic, so that tests
 * can compile and inspect the very instances the runtime compiles. */
int tc_matmul_epilogue_source(uint32_t dtype, const tc_encoded* code, uint32_t count, const tc_place* places,
                              uint32_t place_count, uint32_t runs, char* out, uint64_t capacity, uint64_t* length);

/* The source the runtime compiler builds for `tc_fused` with this program
 * over rows x cols (the arguments as that call takes them; `inputs` are
 * only checked for alignment, never read; outputs count as 16-byte
 * aligned): the dense form, the run form or the general form, as the call
 * would pick, into `out` as `tc_matmul_epilogue_source` does.
 * TC_UNSUPPORTED when the program runs interpreted.  Needs no device.  No
 * counterpart in the reference's interface: a diagnostic, so that tests can
 * compile the very source the runtime compiles. */
int tc_fused_source(uint32_t dtype, const tc_encoded* code, uint32_t count, const tc_place* places,
                    uint32_t place_count, const void* const* inputs, uint32_t input_count, uint64_t rows,
                    uint64_t cols, char* out, uint64_t capacity, uint64_t* length);

/* The source the runtime compiler builds `tc_fused_with_statistics`'s one
 * kernel from for this program and these statistics (the arguments as that
 * call takes them; `inputs` and the statistics' sources are only compared
 * and checked for alignment, never read; outputs count as 16-byte aligned),
 * into `out` as `tc_matmul_epilogue_source` does.
 * TC_UNSUPPORTED when the program runs as the composition instead.  Needs no
 * device.  No counterpart in the reference's interface: a diagnostic, so
 * that tests can compile the very source the runtime compiles. */
int tc_fused_with_statistics_source(uint32_t dtype, const tc_encoded* code, uint32_t count, const tc_place* places,
                                    uint32_t place_count, const void* const* inputs, uint32_t input_count,
                                    uint64_t rows, uint64_t cols, const tc_row_stat* statistics,
                                    uint32_t statistic_count, char* out, uint64_t capacity, uint64_t* length);

/* How many fused programs this process has compiled into kernels of their
 * own.  A dense program (every load in element order, every load before any
 * store) is compiled on its second appearance and cached by its source, as
 * the reference's Metal backend does (metal/codegen.rs:1-40); others, and
 * any that fail to compile, run on the interpreter.  No counterpart in the
 * reference's interface: a diagnostic in the manner of its `counters`
 * feature (counters.rs:1-110), for tests and profiling. */
int tc_fused_compiled(uint64_t* count);

/* Programs beyond what kernel arguments carry (more than 48 instructions or
 * 8 places) run from a device copy kept for the process, keyed by their
 * bytes, up to a limit (4096 by default); past it an uncaptured run uploads
 * its program into a block of its own, freed once its kernel is queued, and
 * a captured run of a program not yet resident is refused.  Reports how many
 * are resident and the limit in force, after setting it to `limit` if that
 * is not 0 (lowering it keeps what is resident).  No counterpart in the
 * reference's interface: a diagnostic and tuning hook, for tests. */
int tc_fused_resident(uint64_t limit, uint64_t* resident, uint64_t* current_limit);

#ifdef __cplusplus
}
#endif

#endif /* TCHIP_H */
