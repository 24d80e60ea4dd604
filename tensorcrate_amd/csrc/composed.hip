// The `Kernels` members that compose a fused program with a product or a
// reduction: `row_moments` (kernels.rs:1090), `fused_sum` (kernels.rs:1120)
// and `matmul_epilogue` (kernels.rs:1142); and `matrix_axis_moments`
// (kernels.rs:1042), the moments reduction along an axis; and
// `fused_with_statistics` (kernels.rs:1103): from a program's second
// appearance one compiled kernel (fused.hip), otherwise `row_moments` for
// each statistic the program derives, then `tc_fused` with those as extra
// inputs, as the trait's default does.
//
// Each runs as the Host backend defines it, over device storage:
//  - row_moments: the rows x cols matrix a place reads of an input, in the
//    program's type, and per row its mean and sum of squared deviations
//    (fused/mod.rs:4030-4041, statistics/mod.rs:419-491), from one pass of
//    the reduction kernels' variance fold.  An input stored as the program's
//    type and read through a place the reduction walk can take is read in
//    place; any other is first converted into a scratch matrix by a two-
//    instruction fused program.
//  - fused_sum: the program's one output summed along the axis
//    (`axis_sum`, fused/mod.rs:4045-4051, defines the sums as products with
//    ones; here f32 accumulation rounded once).  Row sums of a program seen
//    before run as one compiled kernel (fused.hip) and never store the
//    output; otherwise the output goes to scratch and the reduction kernels
//    sum it.
//  - matmul_epilogue: the program in the product kernel's epilogue
//    (gemm.hip); only a product that takes neither matrix-core kernel is
//    formed into scratch first, then the program runs with it as input 0
//    (`host_matmul`, fused/mod.rs:4754-4766).
// Scratch blocks come from the thread's stream-ordered cache and are
// returned to it once the work that reads them is queued.

#include <string.h>

#include "common.hpp"

namespace tc {
namespace {

// A scratch block freed when it leaves scope (stream order keeps it alive
// until the queued work has read it).
struct Scratch {
    void* ptr = nullptr;
    int status = TC_OK;
    explicit Scratch(uint64_t bytes) { status = tc_alloc(bytes, &ptr); }
    ~Scratch() {
        if (ptr != nullptr) tc_free(ptr);
    }
    Scratch(const Scratch&) = delete;
    Scratch& operator=(const Scratch&) = delete;
};

int fill_nan(uint32_t dtype, void* out, uint64_t n) {
    if (n == 0) return TC_OK;
    if (dtype == TC_F32) {
        const float nan = __builtin_nanf("");
        return tc_fill(out, n, 4, &nan);
    }
    const uint16_t bits = dtype == TC_F16 ? 0x7e00 : 0x7fc0;
    return tc_fill(out, n, 2, &bits);
}

// The split a place reads over a rows x cols walk, folding each row: the
// row axes the place's lead axes give (or one repeated row), and the row
// itself `col_step` apart.  False when the lead axes do not multiply out to
// `rows` exactly.
bool place_split(const tc_place& place, uint64_t rows, uint64_t cols, tc_split* split) {
    memset(split, 0, sizeof(*split));
    split->offset = place.offset;
    if (place.lead == 0) {
        split->kept_rank = 1;
        split->kept[0] = rows;
        split->kept_strides[0] = 0;
    } else {
        if (place.lead > TC_FUSED_LEAD) return false;
        uint64_t inner = 1;
        for (uint32_t d = 1; d < place.lead; d++) {
            if (place.dims[d] == 0) return false;
            inner *= place.dims[d];
        }
        if (inner == 0 || rows % inner != 0) return false;
        split->kept_rank = place.lead;
        split->kept[0] = rows / inner;
        split->kept_strides[0] = place.steps[0];
        for (uint32_t d = 1; d < place.lead; d++) {
            split->kept[d] = place.dims[d];
            split->kept_strides[d] = place.steps[d];
        }
    }
    split->folded_rank = 1;
    split->folded[0] = cols;
    split->folded_strides[0] = place.col_step;
    return true;
}

bool is_float(uint32_t dtype) { return dtype == TC_F32 || dtype == TC_F16 || dtype == TC_BF16; }

}  // namespace
}  // namespace tc

using namespace tc;

extern "C" {

int tc_row_moments(uint32_t dtype, uint32_t input_dtype, const void* input, uint64_t input_len,
                   const tc_place* place, uint64_t rows, uint64_t cols, void* means, void* deviations) {
    if (!is_float(dtype) || !is_float(input_dtype)) {
        return fail(TC_UNSUPPORTED, std::string("row_moments: no kernel for ") + dtype_name(input_dtype) +
                                        " input in " + dtype_name(dtype));
    }
    if (place->lead > TC_FUSED_LEAD) return fail(TC_INVALID, "row_moments: a place folds more than 5 axes");
    if (rows == 0) return TC_OK;
    if (any_null({means, deviations}) || (cols != 0 && input_len != 0 && input == nullptr)) {
        return null_operand("row_moments");
    }
    if (cols == 0) {  // moments of nothing (statistics/mod.rs:428-434)
        int status = fill_nan(dtype, means, rows);
        return status == TC_OK ? fill_nan(dtype, deviations, rows) : status;
    }
    tc_split split;
    if (input_dtype == dtype && place_split(*place, rows, cols, &split)) {
        return reduce_moments(dtype, input, input_len, &split, means, deviations);
    }
    // The matrix the place reads, converted to the program's type.
    const uint64_t n = rows * cols;
    Scratch matrix(n * dtype_size(dtype));
    if (matrix.status != TC_OK) return matrix.status;
    const tc_encoded code[2] = {
        {0, 0, 0, 0, static_cast<uint8_t>(input_dtype), 0, 0.0f},  // load input 0 through place 0
        {5, 0, 0, 0, static_cast<uint8_t>(dtype), 0, 0.0f},        // store it to output 0
    };
    const void* inputs[1] = {input};
    void* outputs[1] = {matrix.ptr};
    const uint64_t output_lens[1] = {n};
    int status = tc_fused(dtype, code, 2, place, 1, inputs, &input_len, 1, outputs, output_lens, 1, rows, cols);
    if (status != TC_OK) return status;
    memset(&split, 0, sizeof(split));
    split.kept_rank = 1;
    split.kept[0] = rows;
    split.kept_strides[0] = cols;
    split.folded_rank = 1;
    split.folded[0] = cols;
    split.folded_strides[0] = 1;
    return reduce_moments(dtype, matrix.ptr, n, &split, means, deviations);
}

int tc_fused_with_statistics(uint32_t dtype, const tc_encoded* code, uint32_t count, const tc_place* places,
                             uint32_t place_count, const void* const* inputs, const uint64_t* input_lens,
                             uint32_t input_count, void* const* outputs, const uint64_t* output_lens,
                             uint32_t output_count, uint64_t rows, uint64_t cols, const tc_row_stat* statistics,
                             uint32_t statistic_count) {
    if (!is_float(dtype)) {
        return fail(TC_UNSUPPORTED, std::string("fused with statistics: no kernel computes in ") + dtype_name(dtype));
    }
    if (input_count + statistic_count > TC_FUSED_MAX_INPUTS) {
        return fail(TC_INVALID, "fused with statistics: " + std::to_string(input_count + statistic_count) +
                                    " inputs with the statistics, over the " + std::to_string(TC_FUSED_MAX_INPUTS) +
                                    " limit");
    }
    for (uint32_t i = 0; i < statistic_count; i++) {
        const tc_row_stat& st = statistics[i];
        if (st.which > TC_STAT_DEVIATIONS || !is_float(st.source_dtype) || st.place.lead > TC_FUSED_LEAD) {
            return fail(TC_INVALID, "fused with statistics: statistic " + std::to_string(i) + " is malformed");
        }
        if (st.source == nullptr && st.source_len != 0) return null_operand("fused with statistics");
    }
    if (null_slot(inputs, input_lens, input_count) || null_slot(outputs, output_lens, output_count)) {
        return null_operand("fused with statistics");
    }
    const void* all[TC_FUSED_MAX_INPUTS] = {};
    uint64_t all_lens[TC_FUSED_MAX_INPUTS] = {};
    for (uint32_t k = 0; k < input_count; k++) {
        all[k] = inputs[k];
        all_lens[k] = input_lens[k];
    }
    for (uint32_t i = 0; i < statistic_count; i++) all_lens[input_count + i] = rows;
    const uint32_t total = input_count + statistic_count;
    int status = check_fused(dtype, code, count, places, place_count, all_lens, total, output_lens, output_count,
                             rows, cols);
    if (status != TC_OK) return status;
    if (rows == 0) return TC_OK;
    if (statistic_count == 0) {
        return tc_fused(dtype, code, count, places, place_count, all, all_lens, total, outputs, output_lens,
                        output_count, rows, cols);
    }
    bool done = false;
    status = fused_row_statistics(dtype, code, count, places, place_count, all, all_lens, input_count, outputs,
                                  output_lens, output_count, rows, cols, statistics, statistic_count, &done);
    if (status != TC_OK || done) return status;
    // The trait's default: each distinct source's moments once, then the
    // program with them as inputs.
    const uint64_t width = dtype_size(dtype);
    Scratch moments(2 * statistic_count * rows * width);
    if (moments.status != TC_OK) return moments.status;
    uint8_t* base = static_cast<uint8_t*>(moments.ptr);
    uint32_t computed[8];
    uint32_t distinct = 0;
    for (uint32_t i = 0; i < statistic_count; i++) {
        const tc_row_stat& st = statistics[i];
        uint32_t j = 0;
        for (; j < distinct; j++) {
            const tc_row_stat& f = statistics[computed[j]];
            bool same = f.source == st.source && f.source_dtype == st.source_dtype &&
                        f.place.offset == st.place.offset && f.place.col_step == st.place.col_step &&
                        f.place.lead == st.place.lead;
            for (uint32_t d = 0; same && d < st.place.lead; d++) {
                same = f.place.dims[d] == st.place.dims[d] && f.place.steps[d] == st.place.steps[d];
            }
            if (same) break;
        }
        void* means = base + 2 * j * rows * width;
        void* deviations = base + (2 * j + 1) * rows * width;
        if (j == distinct) {
            if (distinct == 8) return fail(TC_INVALID, "fused with statistics: more than 8 statistics");
            computed[distinct++] = i;
            status = tc_row_moments(dtype, st.source_dtype, st.source, st.source_len, &st.place, rows, cols, means,
                                    deviations);
            if (status != TC_OK) return status;
        }
        all[input_count + i] = st.which == TC_STAT_MEAN ? means : deviations;
    }
    return tc_fused(dtype, code, count, places, place_count, all, all_lens, total, outputs, output_lens,
                    output_count, rows, cols);
}

int tc_axis_moments(uint32_t dtype, const void* a, uint64_t rows, uint64_t cols, uint32_t axis, void* means,
                    void* deviations) {
    if (axis > TC_AXIS_COLUMNS) return fail(TC_INVALID, "axis moments: no Axis " + std::to_string(axis));
    if (!is_float(dtype)) return fail(TC_UNSUPPORTED, std::string("axis moments: no kernel for ") + dtype_name(dtype));
    const uint64_t results = axis == TC_AXIS_ROWS ? rows : cols;
    const uint64_t depth = axis == TC_AXIS_ROWS ? cols : rows;
    if (results == 0) return TC_OK;
    if (depth == 0) {  // moments of nothing (statistics/mod.rs:470-476)
        int status = fill_nan(dtype, means, results);
        return status == TC_OK ? fill_nan(dtype, deviations, results) : status;
    }
    tc_split split;
    memset(&split, 0, sizeof(split));
    split.kept_rank = 1;
    split.folded_rank = 1;
    split.kept[0] = results;
    split.folded[0] = depth;
    split.kept_strides[0] = axis == TC_AXIS_ROWS ? cols : 1;
    split.folded_strides[0] = axis == TC_AXIS_ROWS ? 1 : cols;
    return reduce_moments(dtype, a, rows * cols, &split, means, deviations);
}

int tc_fused_sum(uint32_t dtype, const tc_encoded* code, uint32_t count, const tc_place* places,
                 uint32_t place_count, const void* const* inputs, const uint64_t* input_lens, uint32_t input_count,
                 uint64_t rows, uint64_t cols, uint32_t axis, void* out) {
    if (axis > TC_AXIS_COLUMNS) return fail(TC_INVALID, "fused sum: no Axis " + std::to_string(axis));
    if (!is_float(dtype)) return fail(TC_UNSUPPORTED, std::string("fused sum: no kernel for ") + dtype_name(dtype));
    for (uint32_t pc = 0; pc < count; pc++) {
        if (code[pc].kind == 5 && (code[pc].aux != 0 || code[pc].b != dtype)) {
            return fail(TC_INVALID, std::string("fused sum: the program must have one ") + dtype_name(dtype) +
                                        " output, update nothing in place and compute no row statistics");
        }
    }
    const uint64_t results = axis == TC_AXIS_ROWS ? rows : cols;
    const uint64_t depth = axis == TC_AXIS_ROWS ? cols : rows;
    if (results == 0) return TC_OK;
    if (out == nullptr || null_slot(inputs, input_lens, input_count)) return null_operand("fused sum");
    if (depth == 0) {  // sums of nothing
        const uint32_t zero = 0;
        return tc_fill(out, results, static_cast<uint32_t>(dtype_size(dtype)), &zero);
    }
    {
        bool done = false;
        int status = axis == TC_AXIS_ROWS
                         ? fused_row_sums(dtype, code, count, places, place_count, inputs, input_lens, input_count,
                                          rows, cols, out, &done)
                         : fused_column_sums(dtype, code, count, places, place_count, inputs, input_lens,
                                             input_count, rows, cols, out, &done);
        if (status != TC_OK || done) return status;
    }
    const uint64_t n = rows * cols;
    Scratch data(n * dtype_size(dtype));
    if (data.status != TC_OK) return data.status;
    void* outputs[1] = {data.ptr};
    const uint64_t output_lens[1] = {n};
    int status = tc_fused(dtype, code, count, places, place_count, inputs, input_lens, input_count, outputs,
                          output_lens, 1, rows, cols);
    if (status != TC_OK) return status;
    tc_split split;
    memset(&split, 0, sizeof(split));
    split.kept_rank = 1;
    split.folded_rank = 1;
    split.kept[0] = results;
    split.folded[0] = depth;
    split.kept_strides[0] = axis == TC_AXIS_ROWS ? cols : 1;
    split.folded_strides[0] = axis == TC_AXIS_ROWS ? 1 : cols;
    return tc_reduce_axes(dtype, data.ptr, n, &split, TC_AXIS_FOLD, TC_REDUCE_SUM, 0, out);
}

}  // extern "C"

// Whether `p` reads element (row, col) of a row-major rows x cols matrix at
// row * cols + col: no offset, unit column step, and lead axes that fold
// the row index contiguously.
static bool reads_in_order(const tc_place& p, uint64_t rows, uint64_t cols) {
    if (p.offset != 0 || (p.col_step != 1 && cols > 1)) return false;
    if (p.lead == 0) return rows <= 1;
    if (p.lead > TC_FUSED_LEAD) return false;
    uint64_t step = cols, folded = 1;
    for (int d = static_cast<int>(p.lead) - 1; d >= 0; d--) {
        if (p.dims[d] > 1 && p.steps[d] != step) return false;
        step *= p.dims[d];
        folded *= p.dims[d];
    }
    return folded == rows;
}

extern "C" {

int tc_matmul_epilogue(uint32_t dtype, const tc_encoded* code, uint32_t count, const tc_place* places,
                       uint32_t place_count, uint64_t m, uint64_t k, uint64_t n, const void* a, const void* b,
                       const void* const* inputs, const uint64_t* input_lens, uint32_t input_count,
                       void* const* outputs, const uint64_t* output_lens, uint32_t output_count) {
    if (!is_float(dtype)) return fail(TC_UNSUPPORTED, std::string("fused matmul: no kernel for ") + dtype_name(dtype));
    if (input_count + 1 > TC_FUSED_MAX_INPUTS) {
        return fail(TC_INVALID, "fused program: " + std::to_string(input_count + 1) + " inputs, over the 16 limit");
    }
    // fused/mod.rs:1185-1196: the product is input 0, read without a remap.
    for (uint32_t pc = 0; pc < count; pc++) {
        if (code[pc].kind == 0 && code[pc].a == 0) {
            if (code[pc].op >= place_count || !reads_in_order(places[code[pc].op], m, n)) {
                return fail(TC_INVALID, "fused matmul: the product is read through a remap");
            }
            if (code[pc].b != dtype) return fail(TC_INVALID, "fused matmul: the product is stored as the program's type");
        }
    }
    if (m == 0 || n == 0) return TC_OK;
    if (k != 0 && (a == nullptr || b == nullptr)) return fail(TC_INVALID, "fused matmul: a null operand");
    for (uint32_t s = 0; s < input_count; s++) {
        if (inputs[s] == nullptr && input_lens[s] != 0) return fail(TC_INVALID, "fused matmul: a null input");
    }
    for (uint32_t s = 0; s < output_count; s++) {
        if (outputs[s] == nullptr && output_lens[s] != 0) return fail(TC_INVALID, "fused matmul: a null output");
    }
    const uint64_t cells = m * n;
    {
        const void* all[TC_FUSED_MAX_INPUTS] = {};
        uint64_t lens[TC_FUSED_MAX_INPUTS] = {};
        lens[0] = cells;
        for (uint32_t s = 0; s < input_count; s++) {
            all[s + 1] = inputs[s];
            lens[s + 1] = input_lens[s];
        }
        int status = check_fused(dtype, code, count, places, place_count, lens, input_count + 1, output_lens,
                                 output_count, m, n);
        if (status != TC_OK) return status;
        bool fused = false;
        status = matmul_program(dtype, m, k, n, a, b, code, count, places, place_count, all, input_count + 1, outputs,
                                output_count, &fused);
        if (status != TC_OK || fused) return status;
    }
    Scratch product(cells * dtype_size(dtype));
    if (product.status != TC_OK) return product.status;
    int status = tc_matmul(dtype, dtype, TC_PLAIN, 0, m, k, n, a, b, product.ptr);
    if (status != TC_OK) return status;
    const void* all[TC_FUSED_MAX_INPUTS];
    uint64_t lens[TC_FUSED_MAX_INPUTS];
    all[0] = product.ptr;
    lens[0] = cells;
    for (uint32_t s = 0; s < input_count; s++) {
        all[s + 1] = inputs[s];
        lens[s + 1] = input_lens[s];
    }
    return tc_fused(dtype, code, count, places, place_count, all, lens, input_count + 1, outputs, output_lens,
                    output_count, m, n);
}

}  // extern "C"
