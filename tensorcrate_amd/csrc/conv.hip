// Valid correlation and its gradients, padding and flipping: `Kernels::
// correlate`, `correlate_window_gradient`, `correlate_input_gradient`, `pad`
// and `flip` (tensors/kernels.rs:990-1029).
//
// Each output of a correlation is its own sum, taken over the window in row-
// major tap order with a separate multiply and add per tap, f32 throughout
// (f16 and bf16 widened, rounded once at the end) — the host's loop
// (kernels.rs:1720-1794), so the results are the host's bits.  One thread
// per output; the window's taps are read by every thread of a block at once
// and come from the cache.  The window gradient is the correlation of the
// input with the adjoint (kernels.rs:1544-1551), so it needs no kernel of
// its own.  `pad` and `flip` move bits, by element width.

#include "common.hpp"

namespace tc {
namespace {

template <typename S, bool FLIP>
__global__ void __launch_bounds__(256) correlate_kernel(const S* __restrict__ input, const S* __restrict__ window,
                                                        S* __restrict__ out, uint64_t cols, uint64_t window_rows,
                                                        uint64_t window_cols, uint64_t out_cols, uint64_t count) {
    using E = Elem<S>;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t at = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; at < count; at += stride) {
        const uint64_t row = at / out_cols, col = at - row * out_cols;
        float sum = 0.0f;
        for (uint64_t i = 0; i < window_rows; i++) {
            const S* line = input + (row + i) * cols + col;
            for (uint64_t j = 0; j < window_cols; j++) {
                const uint64_t tap = FLIP ? (window_rows - 1 - i) * window_cols + (window_cols - 1 - j)
                                          : i * window_cols + j;
                sum = sum + E::widen(line[j]) * E::widen(window[tap]);
            }
        }
        out[at] = E::narrow(sum);
    }
}

// X̄[p][q] = Σ Ȳ[p-i][q-j] K[tap(i, j)] over the taps whose adjoint index
// is in range, in tap order (kernels.rs:1754-1794).
template <typename S, bool FLIP>
__global__ void __launch_bounds__(256) input_gradient_kernel(const S* __restrict__ adjoint,
                                                             const S* __restrict__ window, S* __restrict__ out,
                                                             uint64_t adjoint_rows, uint64_t adjoint_cols,
                                                             uint64_t window_rows, uint64_t window_cols,
                                                             uint64_t cols, uint64_t count) {
    using E = Elem<S>;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t at = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; at < count; at += stride) {
        const uint64_t row = at / cols, col = at - row * cols;
        float sum = 0.0f;
        for (uint64_t i = 0; i < window_rows; i++) {
            if (row < i || row - i >= adjoint_rows) continue;
            for (uint64_t j = 0; j < window_cols; j++) {
                if (col < j || col - j >= adjoint_cols) continue;
                const uint64_t tap = FLIP ? (window_rows - 1 - i) * window_cols + (window_cols - 1 - j)
                                          : i * window_cols + j;
                sum = sum + E::widen(adjoint[(row - i) * adjoint_cols + (col - j)]) * E::widen(window[tap]);
            }
        }
        out[at] = E::narrow(sum);
    }
}

template <typename T>
__global__ void __launch_bounds__(256) pad_kernel(const T* __restrict__ input, T* __restrict__ out, uint64_t rows,
                                                  uint64_t cols, uint64_t pad_rows, uint64_t pad_cols,
                                                  uint64_t padded_cols, uint64_t count) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t at = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; at < count; at += stride) {
        const uint64_t row = at / padded_cols, col = at - row * padded_cols;
        const bool inside = row >= pad_rows && row < pad_rows + rows && col >= pad_cols && col < pad_cols + cols;
        out[at] = inside ? input[(row - pad_rows) * cols + (col - pad_cols)] : T{};
    }
}

// Reversing both axes of a row-major matrix reverses its storage.
template <typename T>
__global__ void __launch_bounds__(256) reverse_kernel(const T* __restrict__ input, T* __restrict__ out,
                                                      uint64_t count) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t at = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; at < count; at += stride) {
        out[at] = input[count - 1 - at];
    }
}

template <typename S>
int correlate_typed(const void* input, uint64_t cols, const void* window, uint64_t window_rows,
                    uint64_t window_cols, bool flip, void* out, uint64_t out_rows, uint64_t out_cols) {
    TC_STREAM(s);
    const uint64_t count = out_rows * out_cols;
    if (count == 0) return TC_OK;
    const S* in = static_cast<const S*>(input);
    const S* w = static_cast<const S*>(window);
    S* o = static_cast<S*>(out);
    if (flip) {
        correlate_kernel<S, true><<<blocks_for(count, 1), 256, 0, s>>>(in, w, o, cols, window_rows, window_cols,
                                                                        out_cols, count);
    } else {
        correlate_kernel<S, false><<<blocks_for(count, 1), 256, 0, s>>>(in, w, o, cols, window_rows, window_cols,
                                                                         out_cols, count);
    }
    return check_launch("correlate");
}

template <typename S>
int input_gradient_typed(const void* adjoint, uint64_t adjoint_rows, uint64_t adjoint_cols, const void* window,
                         uint64_t window_rows, uint64_t window_cols, bool flip, void* out) {
    TC_STREAM(s);
    const uint64_t rows = adjoint_rows + window_rows - 1, cols = adjoint_cols + window_cols - 1;
    const uint64_t count = rows * cols;
    if (count == 0) return TC_OK;
    const S* a = static_cast<const S*>(adjoint);
    const S* w = static_cast<const S*>(window);
    S* o = static_cast<S*>(out);
    if (flip) {
        input_gradient_kernel<S, true><<<blocks_for(count, 1), 256, 0, s>>>(a, w, o, adjoint_rows, adjoint_cols,
                                                                             window_rows, window_cols, cols, count);
    } else {
        input_gradient_kernel<S, false><<<blocks_for(count, 1), 256, 0, s>>>(a, w, o, adjoint_rows, adjoint_cols,
                                                                              window_rows, window_cols, cols, count);
    }
    return check_launch("correlate input gradient");
}

}  // namespace
}  // namespace tc

using namespace tc;

extern "C" {

int tc_correlate(uint32_t dtype, const void* input, uint64_t rows, uint64_t cols, const void* window,
                 uint64_t window_rows, uint64_t window_cols, int flip, void* out) {
    if (window_rows > rows || window_cols > cols) {  // `correlation_shape` (kernels.rs:1841-1851)
        return fail(TC_INVALID, "correlate: a " + std::to_string(window_rows) + "×" + std::to_string(window_cols) +
                                    " window does not fit in a " + std::to_string(rows) + "×" + std::to_string(cols) +
                                    " input");
    }
    const uint64_t out_rows = rows - window_rows + 1, out_cols = cols - window_cols + 1;
    TC_DISPATCH_FLOAT(dtype, "correlate", S,
                      return correlate_typed<S>(input, cols, window, window_rows, window_cols, flip != 0, out,
                                                out_rows, out_cols));
    return TC_OK;
}

int tc_correlate_input_gradient(uint32_t dtype, const void* adjoint, uint64_t adjoint_rows, uint64_t adjoint_cols,
                                const void* window, uint64_t window_rows, uint64_t window_cols, int forward_flip,
                                void* out) {
    if (window_rows == 0 || window_cols == 0) {
        return fail(TC_INVALID, "correlate input gradient: an empty window");
    }
    TC_DISPATCH_FLOAT(dtype, "correlate input gradient", S,
                      return input_gradient_typed<S>(adjoint, adjoint_rows, adjoint_cols, window, window_rows,
                                                     window_cols, forward_flip != 0, out));
    return TC_OK;
}

int tc_pad(uint32_t width, const void* input, uint64_t rows, uint64_t cols, uint64_t pad_rows, uint64_t pad_cols,
           void* out) {
    TC_STREAM(s);
    const uint64_t padded_cols = cols + 2 * pad_cols;
    const uint64_t count = (rows + 2 * pad_rows) * padded_cols;
    if (count == 0) return TC_OK;
    const uint32_t blocks = blocks_for(count, 1);
#define TC_PAD(T)                                                                                                     \
    pad_kernel<T><<<blocks, 256, 0, s>>>(static_cast<const T*>(input), static_cast<T*>(out), rows, cols, pad_rows, \
                                         pad_cols, padded_cols, count)
    switch (width) {
        case 1: TC_PAD(uint8_t); break;
        case 2: TC_PAD(uint16_t); break;
        case 4: TC_PAD(uint32_t); break;
        case 8: TC_PAD(uint64_t); break;
        case 16: TC_PAD(uint4); break;
        default: return fail(TC_UNSUPPORTED, "pad: no kernel for " + std::to_string(width) + "-byte elements");
    }
#undef TC_PAD
    return check_launch("pad");
}

int tc_flip(uint32_t width, const void* input, uint64_t rows, uint64_t cols, void* out) {
    TC_STREAM(s);
    const uint64_t count = rows * cols;
    if (count == 0) return TC_OK;
    const uint32_t blocks = blocks_for(count, 1);
#define TC_FLIP(T) reverse_kernel<T><<<blocks, 256, 0, s>>>(static_cast<const T*>(input), static_cast<T*>(out), count)
    switch (width) {
        case 1: TC_FLIP(uint8_t); break;
        case 2: TC_FLIP(uint16_t); break;
        case 4: TC_FLIP(uint32_t); break;
        case 8: TC_FLIP(uint64_t); break;
        case 16: TC_FLIP(uint4); break;
        default: return fail(TC_UNSUPPORTED, "flip: no kernel for " + std::to_string(width) + "-byte elements");
    }
#undef TC_FLIP
    return check_launch("flip");
}

}  // extern "C"
