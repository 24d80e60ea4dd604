// The host side of the `Hip` backend in C++: tensorcrate's `Backend` storage
// and the `Kernels<T>` operations the tape and the optimizers are written in
// (src/tensors/backend.rs:77-178, src/tensors/kernels.rs:829-1188), as types
// over the C ABI of include/tchip.h.
//
// The reference's host code is Rust and reaches a device backend through
// `B: Kernels<T>`; this mirror keeps its names, argument meanings and error
// behaviour so the code above it (tape.hpp, optim.hpp) reads like the
// reference's own.  Shape mistakes throw `std::invalid_argument` with the
// reference's panic wording before anything reaches the device
// (tensors/shape.rs:9-60); a failed device call throws `hip::Error` with the
// library's message, the analogue of `require_metal`'s panic
// (backend.rs:422-426).  Nothing here computes on the host: every operation
// is one or two calls into libtchip.
#pragma once

#include <stdint.h>

#include <algorithm>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "tchip.h"

namespace tensorcrate {
namespace hip {

struct Error : std::runtime_error {
    int status;
    Error(int s, const std::string& message) : std::runtime_error(message), status(s) {}
};

inline void check(int status) {
    if (status != TC_OK) throw Error(status, tc_last_error());
}

// `BinaryOp`, `Compare`, `Reduce`, `Transposed` (kernels.rs:30-187, :461).
enum class BinaryOp : uint32_t { Add = TC_ADD, Sub = TC_SUB, Mul = TC_MUL, Div = TC_DIV, Rem = TC_REM };
enum class Compare : uint32_t {
    Min = TC_MIN, Max = TC_MAX, MaxShare = TC_MAX_SHARE,
    Less = TC_LESS, LessEqual = TC_LESS_EQUAL, Greater = TC_GREATER, GreaterEqual = TC_GREATER_EQUAL
};
enum class Reduce : uint32_t { Sum = TC_REDUCE_SUM, Min = TC_REDUCE_MIN, Max = TC_REDUCE_MAX };
enum class Transposed : uint32_t { Left = TC_LEFT, Right = TC_RIGHT };

// The element types a kernel computes in; only f32 is instantiated here.
template <typename T>
struct DType;
template <>
struct DType<float> {
    static constexpr uint32_t code = TC_F32;
};

// `Backend::Storage<T>` for Hip (backend.rs:86-111): one device allocation
// from the calling thread's stream-ordered cache, freed back to it.  Like a
// Metal tensor it belongs to the thread that made it.
template <typename T>
class Storage {
   public:
    explicit Storage(size_t len) : len_(len) { check(tc_alloc(len * sizeof(T), &ptr_)); }
    ~Storage() {
        if (ptr_ != nullptr) tc_free(ptr_);
    }
    Storage(const Storage&) = delete;
    Storage& operator=(const Storage&) = delete;
    Storage(Storage&& other) noexcept : ptr_(other.ptr_), len_(other.len_) {
        other.ptr_ = nullptr;
        other.len_ = 0;
    }
    Storage& operator=(Storage&& other) noexcept {
        std::swap(ptr_, other.ptr_);
        std::swap(len_, other.len_);
        return *this;
    }

    // `Backend::store` (backend.rs:89): one upload.
    static Storage store(const T* values, size_t len) {
        Storage s(len);
        check(tc_upload(s.ptr_, values, len * sizeof(T)));
        return s;
    }
    // `Vector::filled` on the device: a fill kernel, not an upload of a
    // host vector as the reference's generic `filled` makes (vector.rs:101-106).
    static Storage filled(size_t len, T value) {
        Storage s(len);
        check(tc_fill(s.ptr_, len, sizeof(T), &value));
        return s;
    }
    // `Backend::duplicate` (backend.rs:111): a device-to-device copy.
    Storage duplicate() const {
        Storage s(len_);
        check(tc_copy(s.ptr_, ptr_, len_ * sizeof(T)));
        return s;
    }
    // `Backend::as_slice` (backend.rs:99): waits for queued work, downloads.
    std::vector<T> to_host() const {
        std::vector<T> out(len_);
        check(tc_download(out.data(), ptr_, len_ * sizeof(T)));
        return out;
    }

    void* ptr() { return ptr_; }
    const void* ptr() const { return ptr_; }
    size_t len() const { return len_; }

   private:
    void* ptr_ = nullptr;
    size_t len_ = 0;
};

// `Vector<T, Hip>` (tensors/vector.rs).
template <typename T>
class Vector {
   public:
    explicit Vector(Storage<T> s) : storage_(std::move(s)) {}
    static Vector filled(size_t len, T value) { return Vector(Storage<T>::filled(len, value)); }
    static Vector from_host(const std::vector<T>& values) { return Vector(Storage<T>::store(values.data(), values.size())); }
    Vector duplicate() const { return Vector(storage_.duplicate()); }
    std::vector<T> to_host() const { return storage_.to_host(); }
    size_t len() const { return storage_.len(); }
    Storage<T>& storage() { return storage_; }
    const Storage<T>& storage() const { return storage_; }
    Storage<T> into_storage() && { return std::move(storage_); }

   private:
    Storage<T> storage_;
};

// `Matrix<T, Hip>` (tensors/matrix.rs:23): row-major `rows x cols`.
template <typename T>
class Matrix {
   public:
    Matrix(size_t rows, size_t cols, Storage<T> s) : rows_(rows), cols_(cols), storage_(std::move(s)) {
        if (storage_.len() != rows * cols) {
            throw std::invalid_argument("from_storage: " + std::to_string(storage_.len()) + " elements for a " +
                                        std::to_string(rows) + "×" + std::to_string(cols) + " matrix");
        }
    }
    static Matrix filled(size_t rows, size_t cols, T value) {
        return Matrix(rows, cols, Storage<T>::filled(rows * cols, value));
    }
    static Matrix from_host(size_t rows, size_t cols, const std::vector<T>& values) {
        return Matrix(rows, cols, Storage<T>::store(values.data(), values.size()));
    }
    Matrix duplicate() const { return Matrix(rows_, cols_, storage_.duplicate()); }
    std::vector<T> to_host() const { return storage_.to_host(); }
    size_t rows() const { return rows_; }
    size_t cols() const { return cols_; }
    std::pair<size_t, size_t> shape() const { return {rows_, cols_}; }
    size_t len() const { return rows_ * cols_; }
    Storage<T>& storage() { return storage_; }
    const Storage<T>& storage() const { return storage_; }
    Storage<T> into_storage() && { return std::move(storage_); }

   private:
    size_t rows_, cols_;
    Storage<T> storage_;
};

// `Analytic` (kernels.rs:293-308), numbered as the kernels read it.
enum class Analytic : uint32_t {
    Sin = 0, Cos, Tan, Sec, Csc, Arcsin, Arccos, Arctan, Exp, Ln, Sinh, Cosh, Tanh, Sqrt
};

using Shape = std::vector<size_t>;

inline size_t element_count(const Shape& shape) {
    size_t n = 1;
    for (size_t extent : shape) n *= extent;
    return n;
}

inline std::string shape_text(const Shape& shape) {
    std::string text = "[";
    for (size_t k = 0; k < shape.size(); k++) text += (k ? ", " : "") + std::to_string(shape[k]);
    return text + "]";
}

// `Tensor<T, Hip>` (tensors/tensor.rs:50): a shape over one row-major
// storage.  The reference's views (offset + strides) are not kept: every
// layout operation here makes its contiguous copy at once, one strided-copy
// kernel, which is what a view's `contiguous()` costs when a kernel reads it.
template <typename T>
class Tensor {
   public:
    Tensor(Shape shape, Storage<T> s) : shape_(std::move(shape)), storage_(std::move(s)) {
        if (shape_.size() > TC_MAX_RANK) {
            throw std::invalid_argument("tensor: shape " + shape_text(shape_) + " has more than " +
                                        std::to_string(TC_MAX_RANK) + " axes");
        }
        if (storage_.len() != element_count(shape_)) {
            throw std::invalid_argument("from_storage: " + std::to_string(storage_.len()) +
                                        " elements for shape " + shape_text(shape_));
        }
    }
    static Tensor filled(Shape shape, T value) {
        const size_t n = element_count(shape);
        return Tensor(std::move(shape), n ? Storage<T>::filled(n, value) : Storage<T>(0));
    }
    static Tensor from_host(Shape shape, const std::vector<T>& values) {
        return Tensor(std::move(shape), Storage<T>::store(values.data(), values.size()));
    }
    Tensor duplicate() const { return Tensor(shape_, len() ? storage_.duplicate() : Storage<T>(0)); }
    std::vector<T> to_host() const { return len() ? storage_.to_host() : std::vector<T>(); }
    // `Tensor::reshape` (tensor.rs): the same storage under `shape`.
    Tensor reshape(Shape shape) && {
        if (element_count(shape) != len()) {
            throw std::invalid_argument("reshape: shape " + shape_text(shape_) + " holds " + std::to_string(len()) +
                                        " elements, which " + shape_text(shape) + " cannot");
        }
        return Tensor(std::move(shape), std::move(storage_));
    }
    const Shape& shape() const { return shape_; }
    size_t rank() const { return shape_.size(); }
    size_t len() const { return storage_.len(); }
    Storage<T>& storage() { return storage_; }
    const Storage<T>& storage() const { return storage_; }
    Storage<T> into_storage() && { return std::move(storage_); }

   private:
    Shape shape_;
    Storage<T> storage_;
};

// ---- the reference's shape checks (tensors/shape.rs:9-60) ----------------------

inline std::string dims(std::pair<size_t, size_t> s) {
    return std::to_string(s.first) + "×" + std::to_string(s.second);
}

inline void assert_same_len(size_t left, size_t right, const char* operation) {
    if (left != right) {
        throw std::invalid_argument(std::string(operation) + ": vector lengths differ, " + std::to_string(left) +
                                    " and " + std::to_string(right));
    }
}

inline void assert_same_shape(std::pair<size_t, size_t> left, std::pair<size_t, size_t> right, const char* operation) {
    if (left != right) {
        throw std::invalid_argument(std::string(operation) + ": matrix shapes differ, " + dims(left) + " and " +
                                    dims(right));
    }
}

inline void assert_inner(std::pair<size_t, size_t> left, std::pair<size_t, size_t> right, const char* operation) {
    if (left.second != right.first) {
        throw std::invalid_argument(std::string(operation) + ": inner dimensions differ, " + dims(left) + " times " +
                                    dims(right));
    }
}

// ---- Kernels<T> for Hip (kernels.rs:829-1188) -----------------------------------

template <typename T>
struct Kernels {
    static constexpr uint32_t dtype = DType<T>::code;

    // `vector_elementwise` (kernels.rs:832).
    static Vector<T> vector_elementwise(const Vector<T>& a, const Vector<T>& b, BinaryOp op) {
        assert_same_len(a.len(), b.len(), "elementwise");
        Storage<T> out(a.len());
        check(tc_elementwise(dtype, static_cast<uint32_t>(op), a.storage().ptr(), b.storage().ptr(), out.ptr(), a.len()));
        return Vector<T>(std::move(out));
    }
    // `matrix_elementwise` (kernels.rs:912).
    static Matrix<T> matrix_elementwise(const Matrix<T>& a, const Matrix<T>& b, BinaryOp op) {
        assert_same_shape(a.shape(), b.shape(), "elementwise");
        Storage<T> out(a.len());
        check(tc_elementwise(dtype, static_cast<uint32_t>(op), a.storage().ptr(), b.storage().ptr(), out.ptr(), a.len()));
        return Matrix<T>(a.rows(), a.cols(), std::move(out));
    }
    // `vector_broadcast` / `matrix_broadcast` (kernels.rs:838, :918):
    // x op s, or s op x when `scalar_left`.
    static Vector<T> vector_broadcast(const Vector<T>& a, T scalar, BinaryOp op, bool scalar_left) {
        Storage<T> out(a.len());
        check(tc_broadcast(dtype, static_cast<uint32_t>(op), a.storage().ptr(), scalar, scalar_left, out.ptr(), a.len()));
        return Vector<T>(std::move(out));
    }
    static Matrix<T> matrix_broadcast(const Matrix<T>& a, T scalar, BinaryOp op, bool scalar_left) {
        Storage<T> out(a.len());
        check(tc_broadcast(dtype, static_cast<uint32_t>(op), a.storage().ptr(), scalar, scalar_left, out.ptr(), a.len()));
        return Matrix<T>(a.rows(), a.cols(), std::move(out));
    }
    // `matrix_compare` / `matrix_compare_scalar` (kernels.rs:926, :929).
    static Matrix<T> matrix_compare(const Matrix<T>& a, const Matrix<T>& b, Compare op) {
        assert_same_shape(a.shape(), b.shape(), "compare");
        Storage<T> out(a.len());
        check(tc_compare(dtype, static_cast<uint32_t>(op), a.storage().ptr(), b.storage().ptr(), out.ptr(), a.len()));
        return Matrix<T>(a.rows(), a.cols(), std::move(out));
    }
    static Matrix<T> matrix_compare_scalar(const Matrix<T>& a, T scalar, Compare op, bool scalar_left) {
        Storage<T> out(a.len());
        check(tc_compare_scalar(dtype, static_cast<uint32_t>(op), a.storage().ptr(), scalar, scalar_left, out.ptr(),
                                a.len()));
        return Matrix<T>(a.rows(), a.cols(), std::move(out));
    }
    // `matmul` (kernels.rs:956): (R×K)·(K×C).
    static Matrix<T> matmul(const Matrix<T>& a, const Matrix<T>& b) {
        assert_inner(a.shape(), b.shape(), "matmul");
        Storage<T> out(a.rows() * b.cols());
        check(tc_matmul(dtype, dtype, TC_PLAIN, 0, a.rows(), a.cols(), b.cols(), a.storage().ptr(), b.storage().ptr(),
                        out.ptr()));
        return Matrix<T>(a.rows(), b.cols(), std::move(out));
    }
    // `matmul_add` (kernels.rs:963): the addend is consumed as the accumulator.
    static Matrix<T> matmul_add(const Matrix<T>& a, const Matrix<T>& b, Matrix<T> addend) {
        assert_inner(a.shape(), b.shape(), "matmul_add");
        assert_same_shape(addend.shape(), {a.rows(), b.cols()}, "matmul_add");
        check(tc_matmul(dtype, dtype, TC_PLAIN, 1, a.rows(), a.cols(), b.cols(), a.storage().ptr(), b.storage().ptr(),
                        addend.storage().ptr()));
        return addend;
    }
    // `matmul_transposed_add` (kernels.rs:975-985): addend + Aᵀ·B (Left) or
    // addend + A·Bᵀ (Right), the transposed operand read in place.
    static Matrix<T> matmul_transposed_add(const Matrix<T>& a, const Matrix<T>& b, Transposed which, Matrix<T> addend) {
        size_t m, k, n;
        if (which == Transposed::Left) {
            assert_inner({a.cols(), a.rows()}, b.shape(), "matmul_transposed_add");
            m = a.cols(), k = a.rows(), n = b.cols();
        } else {
            assert_inner(a.shape(), {b.cols(), b.rows()}, "matmul_transposed_add");
            m = a.rows(), k = a.cols(), n = b.rows();
        }
        assert_same_shape(addend.shape(), {m, n}, "matmul_transposed_add");
        check(tc_matmul(dtype, dtype, static_cast<uint32_t>(which), 1, m, k, n, a.storage().ptr(), b.storage().ptr(),
                        addend.storage().ptr()));
        return addend;
    }
    // `matvec` (kernels.rs:901): M·v.
    static Vector<T> matvec(const Matrix<T>& m, const Vector<T>& v) {
        if (m.cols() != v.len()) {
            throw std::invalid_argument("matvec: a " + dims(m.shape()) + " matrix times a length-" +
                                        std::to_string(v.len()) + " vector");
        }
        Storage<T> out(m.rows());
        check(tc_matvec(dtype, 0, m.rows(), m.cols(), m.storage().ptr(), v.storage().ptr(), out.ptr()));
        return Vector<T>(std::move(out));
    }
    // `matvec_add` (kernels.rs:908): M·v + addend, the addend consumed as
    // the accumulator.
    static Vector<T> matvec_add(const Matrix<T>& m, const Vector<T>& v, Vector<T> addend) {
        if (m.cols() != v.len() || m.rows() != addend.len()) {
            throw std::invalid_argument("matvec_add: a " + dims(m.shape()) + " matrix times a length-" +
                                        std::to_string(v.len()) + " vector plus a length-" +
                                        std::to_string(addend.len()) + " vector");
        }
        check(tc_matvec(dtype, 1, m.rows(), m.cols(), m.storage().ptr(), v.storage().ptr(), addend.storage().ptr()));
        return addend;
    }
    // `vecmat` (kernels.rs:899): vᵀ·M.
    static Vector<T> vecmat(const Vector<T>& v, const Matrix<T>& m) {
        if (m.rows() != v.len()) {
            throw std::invalid_argument("vecmat: a length-" + std::to_string(v.len()) + " vector times a " +
                                        dims(m.shape()) + " matrix");
        }
        Storage<T> out(m.cols());
        check(tc_vecmat(dtype, m.rows(), m.cols(), v.storage().ptr(), m.storage().ptr(), out.ptr()));
        return Vector<T>(std::move(out));
    }
    // `transpose` (kernels.rs:987).
    static Matrix<T> transpose(const Matrix<T>& m) {
        Storage<T> out(m.len());
        check(tc_transpose(sizeof(T), m.rows(), m.cols(), m.storage().ptr(), out.ptr()));
        return Matrix<T>(m.cols(), m.rows(), std::move(out));
    }
    // `vector_reduce` (kernels.rs:867) queued, its result read back behind
    // it: the ticket's value is waited for only when it is read.
    static uint64_t reduce_async(const Storage<T>& values, Reduce op) {
        float* result = nullptr;
        check(tc_alloc(sizeof(float), reinterpret_cast<void**>(&result)));
        int status = tc_vector_reduce(dtype, values.ptr(), values.len(), static_cast<uint32_t>(op), result);
        uint64_t ticket = 0;
        if (status == TC_OK) status = tc_read_async(result, sizeof(float), &ticket);
        tc_free(result);  // reused only by work queued after the read
        check(status);
        return ticket;
    }
    static T read(uint64_t ticket) {
        float host = 0.0f;
        check(tc_read_wait(ticket, &host, sizeof(float)));
        return static_cast<T>(host);
    }
    // `vector_reduce` (kernels.rs:867): the whole buffer folded; reading the
    // value waits for the device.
    static T reduce(const Storage<T>& values, Reduce op) {
        float* result = nullptr;
        check(tc_alloc(sizeof(float), reinterpret_cast<void**>(&result)));
        int status = tc_vector_reduce(dtype, values.ptr(), values.len(), static_cast<uint32_t>(op), result);
        float host = 0.0f;
        if (status == TC_OK) status = tc_download(&host, result, sizeof(float));
        tc_free(result);
        check(status);
        return static_cast<T>(host);
    }

    // ---- tensors: the trait's strided and axis operations -----------------

    // `Pairwise::name` (kernels.rs:419-426) for a shape error.
    static const char* pairwise_name(uint32_t kind, uint32_t op) {
        if (kind == TC_PAIR_POWER) return "power";
        if (kind == TC_PAIR_COMPARE) return op == TC_MIN ? "min" : op == TC_MAX ? "max" : "compare";
        static const char* const names[] = {"add", "subtract", "multiply", "divide", "remainder"};
        return op < 5 ? names[op] : "elementwise";
    }

    // `broadcast_shape` (layout.rs:316-340): numpy's rule from the last axis;
    // false when the shapes do not broadcast.
    static bool broadcast_shape(const Shape& left, const Shape& right, Shape& out) {
        const size_t rank = std::max(left.size(), right.size());
        out.assign(rank, 1);
        for (size_t axis = 0; axis < rank; axis++) {
            const size_t from_end = rank - axis;
            const size_t l = left.size() >= from_end ? left[left.size() - from_end] : 1;
            const size_t r = right.size() >= from_end ? right[right.size() - from_end] : 1;
            if (l == r || r == 1) {
                out[axis] = l;
            } else if (l == 1) {
                out[axis] = r;
            } else {
                return false;
            }
        }
        return true;
    }

    // The layout that reads a row-major `from` as `to` (`broadcast_strides`,
    // layout.rs:347-363): an axis of extent 1 stretched to more repeats its
    // element with stride 0.
    static tc_strided broadcast_layout(const Shape& from, const Shape& to) {
        tc_strided at{};
        if (to.size() > TC_MAX_RANK) {
            throw std::invalid_argument("broadcast_to: shape " + shape_text(to) + " has more than " +
                                        std::to_string(TC_MAX_RANK) + " axes");
        }
        const size_t added = to.size() - from.size();
        size_t step = 1;
        for (size_t axis = from.size(); axis-- > 0;) {
            const size_t wanted = to[added + axis];
            if (from[axis] == wanted) {
                at.strides[added + axis] = step;
            } else if (from[axis] != 1) {
                throw std::invalid_argument("broadcast_to: shape " + shape_text(from) + " does not broadcast to " +
                                            shape_text(to));
            }
            step *= from[axis];
        }
        return at;
    }

    // `TensorView::zip` (tensor_ops.rs:71-91): two tensors of one shape take
    // the vector kernel, anything else one strided kernel over both operands
    // broadcast to their common shape and read in place.
    static Tensor<T> zip(const Tensor<T>& a, const Tensor<T>& b, uint32_t kind, uint32_t op) {
        Shape shape;
        if (!broadcast_shape(a.shape(), b.shape(), shape)) {
            throw std::invalid_argument(std::string(pairwise_name(kind, op)) + ": tensor shapes differ, " +
                                        shape_text(a.shape()) + " and " + shape_text(b.shape()) +
                                        ", and do not broadcast");
        }
        Storage<T> out(element_count(shape));
        if (out.len() == 0) return Tensor<T>(std::move(shape), std::move(out));
        if (a.shape() == b.shape() && kind != TC_PAIR_POWER) {
            if (kind == TC_PAIR_ARITHMETIC) {
                check(tc_elementwise(dtype, op, a.storage().ptr(), b.storage().ptr(), out.ptr(), out.len()));
            } else {
                check(tc_compare(dtype, op, a.storage().ptr(), b.storage().ptr(), out.ptr(), out.len()));
            }
            return Tensor<T>(std::move(shape), std::move(out));
        }
        if (a.shape() == b.shape() && kind == TC_PAIR_POWER) {
            check(tc_power(dtype, a.storage().ptr(), b.storage().ptr(), out.ptr(), out.len()));
            return Tensor<T>(std::move(shape), std::move(out));
        }
        const tc_strided a_at = broadcast_layout(a.shape(), shape);
        const tc_strided b_at = broadcast_layout(b.shape(), shape);
        const std::vector<uint64_t> dims(shape.begin(), shape.end());
        check(tc_strided_binary(dtype, kind, op, static_cast<uint32_t>(shape.size()), dims.data(),
                                a.storage().ptr(), a.len(), &a_at, b.storage().ptr(), b.len(), &b_at, out.ptr()));
        return Tensor<T>(std::move(shape), std::move(out));
    }
    static Tensor<T> elementwise(const Tensor<T>& a, const Tensor<T>& b, BinaryOp op) {
        return zip(a, b, TC_PAIR_ARITHMETIC, static_cast<uint32_t>(op));
    }
    static Tensor<T> compare(const Tensor<T>& a, const Tensor<T>& b, Compare op) {
        return zip(a, b, TC_PAIR_COMPARE, static_cast<uint32_t>(op));
    }
    static Tensor<T> power(const Tensor<T>& a, const Tensor<T>& b) { return zip(a, b, TC_PAIR_POWER, 0); }

    // `with_scalar`, `compare_scalar`, `power_scalar`, `unary`,
    // `unary_dual` over the flat storage (tensor_ops.rs:93-199).
    static Tensor<T> with_scalar(const Tensor<T>& a, T scalar, BinaryOp op, bool scalar_left) {
        Storage<T> out(a.len());
        if (a.len()) {
            check(tc_broadcast(dtype, static_cast<uint32_t>(op), a.storage().ptr(), scalar, scalar_left, out.ptr(),
                               a.len()));
        }
        return Tensor<T>(a.shape(), std::move(out));
    }
    static Tensor<T> scale(const Tensor<T>& a, T factor) { return with_scalar(a, factor, BinaryOp::Mul, false); }
    static Tensor<T> compare_scalar(const Tensor<T>& a, T scalar, Compare op, bool scalar_left) {
        Storage<T> out(a.len());
        if (a.len()) {
            check(tc_compare_scalar(dtype, static_cast<uint32_t>(op), a.storage().ptr(), scalar, scalar_left,
                                    out.ptr(), a.len()));
        }
        return Tensor<T>(a.shape(), std::move(out));
    }
    static Tensor<T> power_scalar(const Tensor<T>& a, T scalar, bool scalar_left) {
        Storage<T> out(a.len());
        if (a.len()) check(tc_power_scalar(dtype, a.storage().ptr(), scalar, scalar_left, out.ptr(), a.len()));
        return Tensor<T>(a.shape(), std::move(out));
    }
    static Tensor<T> unary(const Tensor<T>& a, Analytic f) {
        Storage<T> out(a.len());
        if (a.len()) check(tc_unary(dtype, static_cast<uint32_t>(f), a.storage().ptr(), out.ptr(), a.len()));
        return Tensor<T>(a.shape(), std::move(out));
    }
    // f(x) and f'(x)·tangent in one dispatch (kernels.rs:891).
    static std::pair<Tensor<T>, Tensor<T>> unary_dual(const Tensor<T>& x, const Tensor<T>& tangent, Analytic f) {
        if (x.shape() != tangent.shape()) {
            throw std::invalid_argument("unary_dual: tensor shapes differ, " + shape_text(x.shape()) + " and " +
                                        shape_text(tangent.shape()));
        }
        Storage<T> value(x.len()), product(x.len());
        if (x.len()) {
            check(tc_unary_dual(dtype, static_cast<uint32_t>(f), x.storage().ptr(), tangent.storage().ptr(),
                                value.ptr(), product.ptr(), x.len()));
        }
        return {Tensor<T>(x.shape(), std::move(value)), Tensor<T>(x.shape(), std::move(product))};
    }

    // `TensorView::broadcast_to(..).contiguous()` (view.rs:370, :407): one
    // strided copy with the stretched axes at stride 0.
    static Tensor<T> broadcast_to(const Tensor<T>& a, const Shape& shape) {
        if (shape.size() < a.rank()) {
            throw std::invalid_argument("broadcast_to: shape " + shape_text(a.shape()) + " does not broadcast to " +
                                        shape_text(shape));
        }
        const tc_strided from = broadcast_layout(a.shape(), shape);
        return copy_through(a, shape, from);
    }
    // `permute(..).contiguous()` (view.rs:133-160): axis k of the result is
    // axis `axes[k]` of `a`.
    static Tensor<T> permute(const Tensor<T>& a, const std::vector<size_t>& axes) {
        std::vector<bool> seen(a.rank(), false);
        bool valid = axes.size() == a.rank();
        for (size_t axis : axes) {
            if (!valid || axis >= a.rank() || seen[axis]) {
                valid = false;
                break;
            }
            seen[axis] = true;
        }
        if (!valid) throw std::invalid_argument("permute: the axes are not a permutation of " + shape_text(a.shape()));
        std::vector<size_t> strides(a.rank());
        size_t step = 1;
        for (size_t axis = a.rank(); axis-- > 0;) {
            strides[axis] = step;
            step *= a.shape()[axis];
        }
        Shape shape(a.rank());
        tc_strided from{};
        for (size_t k = 0; k < axes.size(); k++) {
            shape[k] = a.shape()[axes[k]];
            from.strides[k] = strides[axes[k]];
        }
        return copy_through(a, shape, from);
    }

    // The axes of a reduction resolved against `rank`, negative ones from the
    // end, sorted; out-of-range and repeated axes are refused with the
    // reference's wording (layout.rs:205-238).
    static std::vector<size_t> resolve_axes(const std::vector<long>& axes, const Shape& shape, const char* operation) {
        std::vector<size_t> resolved;
        const long rank = static_cast<long>(shape.size());
        for (long axis : axes) {
            const long k = axis < 0 ? axis + rank : axis;
            if (k < 0 || k >= rank) {
                throw std::invalid_argument(std::string(operation) + ": axis " + std::to_string(axis) +
                                            " is out of range for shape " + shape_text(shape) + " (" +
                                            std::to_string(rank) + " axes)");
            }
            resolved.push_back(static_cast<size_t>(k));
        }
        std::sort(resolved.begin(), resolved.end());
        if (std::adjacent_find(resolved.begin(), resolved.end()) != resolved.end()) {
            std::string named = "[";
            for (size_t k = 0; k < axes.size(); k++) named += (k ? ", " : "") + std::to_string(axes[k]);
            throw std::invalid_argument(std::string(operation) + ": axes " + named + "] are not distinct axes of shape " +
                                        shape_text(shape));
        }
        return resolved;
    }

    // `reduce_axes` (kernels.rs:1175-1179) over a row-major tensor: the kept
    // axes index the result, the folded ones (`axes`, resolved and sorted)
    // are summed, averaged, or folded to their extreme; `divisor` is the
    // variance's.  A slice with no elements gives `empty` (0 for a sum, the
    // fold's identity, NaN for a mean or a variance), as the reference's host
    // kernels do, without a launch.
    static Tensor<T> reduce_axes(const Tensor<T>& a, const std::vector<size_t>& axes, bool keep_dims, uint32_t kind,
                                 Reduce op, size_t divisor, bool divisor_defined, T empty) {
        std::vector<size_t> strides(a.rank());
        size_t step = 1;
        for (size_t axis = a.rank(); axis-- > 0;) {
            strides[axis] = step;
            step *= a.shape()[axis];
        }
        tc_split split{};
        Shape shape;
        size_t depth = 1;
        for (size_t axis = 0; axis < a.rank(); axis++) {
            const bool folded = std::find(axes.begin(), axes.end(), axis) != axes.end();
            if (folded) {
                split.folded[split.folded_rank] = a.shape()[axis];
                split.folded_strides[split.folded_rank++] = strides[axis];
                depth *= a.shape()[axis];
                if (keep_dims) shape.push_back(1);
            } else {
                split.kept[split.kept_rank] = a.shape()[axis];
                split.kept_strides[split.kept_rank++] = strides[axis];
                shape.push_back(a.shape()[axis]);
            }
        }
        const size_t results = element_count(shape);
        if (!divisor_defined || depth == 0 || results == 0) return Tensor<T>::filled(std::move(shape), empty);
        Storage<T> out(results);
        check(tc_reduce_axes(dtype, a.storage().ptr(), a.len(), &split, kind, static_cast<uint32_t>(op), divisor,
                             out.ptr()));
        return Tensor<T>(std::move(shape), std::move(out));
    }

    // ---- slices: `narrow`, `write_slice`, `concat` (view.rs, tensor.rs:504,
    // backend.rs:157-173) ----

    static std::vector<size_t> strides_of(const Shape& shape) {
        std::vector<size_t> strides(shape.size());
        size_t step = 1;
        for (size_t axis = shape.size(); axis-- > 0;) {
            strides[axis] = step;
            step *= shape[axis];
        }
        return strides;
    }
    static void check_range(const Shape& shape, size_t axis, size_t start, size_t len, const char* operation) {
        if (axis >= shape.size() || start > shape[axis] || len > shape[axis] - start) {
            throw std::invalid_argument(std::string(operation) + ": " + std::to_string(start) + ".." +
                                        std::to_string(start + len) + " is out of range for axis " +
                                        std::to_string(axis) + " of shape " + shape_text(shape));
        }
    }
    // Elements `start..start + len` of `axis`, copied out.
    static Tensor<T> narrow(const Tensor<T>& a, size_t axis, size_t start, size_t len) {
        check_range(a.shape(), axis, start, len, "narrow");
        const std::vector<size_t> strides = strides_of(a.shape());
        Shape shape = a.shape();
        shape[axis] = len;
        tc_strided from{};
        from.offset = start * strides[axis];
        for (size_t k = 0; k < strides.size(); k++) from.strides[k] = strides[k];
        return copy_through(a, shape, from);
    }
    // `Tensor::write_slice` (tensor.rs:504): `delta` written over elements
    // `start..` of `axis` of `target`, in place (`Backend::strided_write`).
    static void write_slice(Tensor<T>& target, size_t axis, size_t start, const Tensor<T>& delta) {
        if (delta.rank() != target.rank()) {
            throw std::invalid_argument("write_slice: shape " + shape_text(delta.shape()) + " into " +
                                        shape_text(target.shape()));
        }
        check_range(target.shape(), axis, start, delta.shape()[axis], "write_slice");
        if (delta.len() == 0) return;
        const tc_region place = slice_region(delta, target.shape(), axis, start);
        check(tc_strided_write(sizeof(T), target.storage().ptr(), target.len(), &place));
    }
    // The elements `start..` of `axis` of `current` plus `delta`, reading
    // `current` in place: one strided kernel, no copy of the slice.
    static Tensor<T> narrow_add(const Tensor<T>& current, size_t axis, size_t start, const Tensor<T>& delta) {
        if (delta.rank() != current.rank()) {
            throw std::invalid_argument("narrow: shape " + shape_text(delta.shape()) + " against " +
                                        shape_text(current.shape()));
        }
        check_range(current.shape(), axis, start, delta.shape()[axis], "narrow");
        Storage<T> out(delta.len());
        if (out.len()) {
            const tc_region place = slice_region(delta, current.shape(), axis, start);
            const std::vector<uint64_t> dims(delta.shape().begin(), delta.shape().end());
            check(tc_strided_binary(dtype, TC_PAIR_ARITHMETIC, TC_ADD, static_cast<uint32_t>(delta.rank()),
                                    dims.data(), current.storage().ptr(), current.len(), &place.to,
                                    delta.storage().ptr(), delta.len(), &place.from, out.ptr()));
        }
        return Tensor<T>(delta.shape(), std::move(out));
    }
    // `Tensor::concat` (tensor.rs): the pieces joined along `axis`, one
    // assemble of every piece's region.
    static Tensor<T> concat(const std::vector<const Tensor<T>*>& pieces, size_t axis) {
        if (pieces.empty()) throw std::invalid_argument("concat: there are no tensors to join");
        Shape shape = pieces[0]->shape();
        if (axis >= shape.size()) throw std::invalid_argument("concat: axis out of range for " + shape_text(shape));
        shape[axis] = 0;
        const Shape off_axis = shape;
        for (const Tensor<T>* piece : pieces) {
            Shape other = piece->shape();
            if (other.size() != shape.size()) {
                throw std::invalid_argument("concat: shapes " + shape_text(pieces[0]->shape()) + " and " +
                                            shape_text(other) + " differ off axis " + std::to_string(axis));
            }
            const size_t extent = other[axis];
            other[axis] = 0;
            if (other != off_axis) {
                throw std::invalid_argument("concat: shapes " + shape_text(pieces[0]->shape()) + " and " +
                                            shape_text(piece->shape()) + " differ off axis " + std::to_string(axis));
            }
            shape[axis] += extent;
        }
        Storage<T> out(element_count(shape));
        std::vector<tc_region> regions;
        size_t start = 0;
        for (const Tensor<T>* piece : pieces) {
            if (piece->len()) regions.push_back(slice_region(*piece, shape, axis, start));
            start += piece->shape()[axis];
        }
        if (out.len() && !regions.empty()) {
            check(tc_assemble(sizeof(T), out.ptr(), out.len(), regions.data(), static_cast<uint32_t>(regions.size())));
        }
        return Tensor<T>(std::move(shape), std::move(out));
    }

   private:
    // `delta` (row-major) as the block at `start` of `axis` in a row-major
    // tensor of `shape`: `from` reads `delta`, `to` addresses the block.
    static tc_region slice_region(const Tensor<T>& delta, const Shape& shape, size_t axis, size_t start) {
        tc_region region{};
        region.source = delta.storage().ptr();
        region.source_len = delta.len();
        region.rank = static_cast<uint32_t>(delta.rank());
        const std::vector<size_t> from = strides_of(delta.shape());
        const std::vector<size_t> to = strides_of(shape);
        for (size_t k = 0; k < delta.rank(); k++) {
            region.shape[k] = delta.shape()[k];
            region.from.strides[k] = from[k];
            region.to.strides[k] = to[k];
        }
        region.to.offset = start * to[axis];
        return region;
    }
    static Tensor<T> copy_through(const Tensor<T>& a, const Shape& shape, const tc_strided& from) {
        Storage<T> out(element_count(shape));
        if (out.len()) {
            const std::vector<uint64_t> dims(shape.begin(), shape.end());
            check(tc_strided_copy(sizeof(T), a.storage().ptr(), a.len(), static_cast<uint32_t>(shape.size()),
                                  dims.data(), &from, out.ptr()));
        }
        return Tensor<T>(shape, std::move(out));
    }
};

}  // namespace hip
}  // namespace tensorcrate
