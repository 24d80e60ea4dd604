// Reverse-mode differentiation over Hip storage: tensorcrate's `Tape`, its
// nodes and the scalar, vector, matrix and tensor variables with their
// backward rules (src/tensors/tape/mod.rs, tape/tensor.rs), restated in C++
// over backend.hpp.
//
// The structure is the reference's: every operation computes its value now,
// through `Kernels`, and records a rule that pushes the node's adjoint into
// its operands; `backward_with` clears every adjoint, seeds the output, and
// runs the rules in reverse recording order (tape/mod.rs:507-529).  Adjoints
// start absent and are summed with `add` when a second contribution arrives
// (`Node::accumulate`, :316-323); a product's rule accumulates straight into
// a copy of the current adjoint, or a fresh zero, with one accumulating
// product (`current_or_zeros`, :325-330; `MatrixVar::matmul`, :1195-1216).
// A scalar reduced from device storage is recorded unread and read only when
// something asks for its value (`Lazy`, :253-295), so a training step never
// waits on its loss unless the caller reads it.  Zeros are device fills, not
// host uploads.
#pragma once

#include <cmath>
#include <functional>
#include <limits>
#include <memory>
#include <optional>
#include <stdexcept>
#include <utility>
#include <vector>

#include "backend.hpp"

namespace tensorcrate {
namespace hip {

// `TapeValue` (tape/mod.rs:175-240): a zero of the same shape, a copy, a sum.
template <typename T>
struct TapeValue;

template <>
struct TapeValue<float> {
    static float zeros_like(const float&) { return 0.0f; }
    static float duplicate(const float& v) { return v; }
    static float add(const float& a, const float& b) { return a + b; }
};

template <typename T>
struct TapeValue<Vector<T>> {
    static Vector<T> zeros_like(const Vector<T>& v) { return Vector<T>::filled(v.len(), T(0)); }
    static Vector<T> duplicate(const Vector<T>& v) { return v.duplicate(); }
    static Vector<T> add(const Vector<T>& a, const Vector<T>& b) {
        return Kernels<T>::vector_elementwise(a, b, BinaryOp::Add);
    }
};

template <typename T>
struct TapeValue<Tensor<T>> {
    static Tensor<T> zeros_like(const Tensor<T>& t) { return Tensor<T>::filled(t.shape(), T(0)); }
    static Tensor<T> duplicate(const Tensor<T>& t) { return t.duplicate(); }
    static Tensor<T> add(const Tensor<T>& a, const Tensor<T>& b) {
        return Kernels<T>::elementwise(a, b, BinaryOp::Add);
    }
};

template <typename T>
struct TapeValue<Matrix<T>> {
    static Matrix<T> zeros_like(const Matrix<T>& m) { return Matrix<T>::filled(m.rows(), m.cols(), T(0)); }
    static Matrix<T> duplicate(const Matrix<T>& m) { return m.duplicate(); }
    static Matrix<T> add(const Matrix<T>& a, const Matrix<T>& b) {
        return Kernels<T>::matrix_elementwise(a, b, BinaryOp::Add);
    }
};

// Holds a node's value, either at once or as a thunk run the first time the
// value is asked for: a loss reduced on the device stays queued until the
// host reads it (`Lazy`, tape/mod.rs:253-295).
template <typename V>
class Lazy {
   public:
    static Lazy ready(V value) {
        Lazy l;
        l.value_.emplace(std::move(value));
        return l;
    }
    static Lazy deferred(std::function<V()> compute) {
        Lazy l;
        l.pending_ = std::move(compute);
        return l;
    }
    const V& get() {
        if (!value_) {
            value_.emplace(pending_());
            pending_ = nullptr;
        }
        return *value_;
    }
    bool is_ready() const { return value_.has_value(); }

   private:
    std::optional<V> value_;
    std::function<V()> pending_;
};

// What the tape calls on every node without knowing its value type
// (`Backprop`, tape/mod.rs:333-346).
struct Backprop {
    virtual ~Backprop() = default;
    virtual void propagate() = 0;
    virtual void clear() = 0;
};

template <typename V>
struct Node : Backprop {
    size_t index = 0;
    Lazy<V> value;
    std::optional<V> adjoint;  // absent: a zero not yet allocated
    std::function<void(const V&)> rule;  // empty for a leaf

    explicit Node(Lazy<V> v) : value(std::move(v)) {}

    const V& get() { return value.get(); }

    // `Node::accumulate` (tape/mod.rs:316-323).
    void accumulate(V delta) {
        if (adjoint) {
            adjoint.emplace(TapeValue<V>::add(*adjoint, delta));
        } else {
            adjoint.emplace(std::move(delta));
        }
    }
    // `Node::current_or_zeros` (tape/mod.rs:325-330).
    V current_or_zeros() {
        if (adjoint) return TapeValue<V>::duplicate(*adjoint);
        return TapeValue<V>::zeros_like(get());
    }
    void propagate() override {
        if (adjoint && rule) rule(*adjoint);
    }
    void clear() override { adjoint.reset(); }
};

class Tape;

// `Var<'t, U, B>`: a handle on one recorded node.
template <typename V>
class Var {
   public:
    Var(Tape* tape, std::shared_ptr<Node<V>> node) : tape_(tape), node_(std::move(node)) {}

    const V& value() const { return node_->get(); }
    // The accumulated adjoint after `backward` (`Var::grad`): a zero of the
    // value's shape when nothing reached this node.
    V grad() const {
        if (node_->adjoint) return TapeValue<V>::duplicate(*node_->adjoint);
        return TapeValue<V>::zeros_like(value());
    }
    // `backward_with` (tape/mod.rs:507-529).
    void backward_with(V seed) const;

    Tape* tape() const { return tape_; }
    const std::shared_ptr<Node<V>>& node() const { return node_; }

   protected:
    void assert_same_tape(Tape* other) const {
        if (other != tape_) throw std::invalid_argument("reverse-mode operands belong to different tapes");
    }
    template <typename U>
    Var<U> record(U value, std::function<void(const U&)> rule) const;
    template <typename U>
    Var<U> record_lazy(Lazy<U> value, std::function<void(const U&)> rule) const;

    Tape* tape_;
    std::shared_ptr<Node<V>> node_;
};

// `Tape` (tape/mod.rs:349-420): the recording, in order.
class Tape {
   public:
    template <typename V>
    Var<V> push(Lazy<V> value, std::function<void(const V&)> rule) {
        auto node = std::make_shared<Node<V>>(std::move(value));
        node->index = nodes_.size();
        node->rule = std::move(rule);
        nodes_.push_back(node);
        return Var<V>(this, node);
    }
    // Inputs: `Tape::scalar`, `vector`, `matrix` (tape/mod.rs:372-404).
    Var<float> scalar(float value) { return push<float>(Lazy<float>::ready(value), nullptr); }
    template <typename T>
    Var<Vector<T>> vector(Vector<T> value) {
        return push<Vector<T>>(Lazy<Vector<T>>::ready(std::move(value)), nullptr);
    }
    template <typename T>
    Var<Matrix<T>> matrix(Matrix<T> value) {
        return push<Matrix<T>>(Lazy<Matrix<T>>::ready(std::move(value)), nullptr);
    }
    template <typename T>
    Var<Tensor<T>> tensor(Tensor<T> value) {
        return push<Tensor<T>>(Lazy<Tensor<T>>::ready(std::move(value)), nullptr);
    }
    size_t len() const { return nodes_.size(); }
    // `Tape::zero_grad` (tape/mod.rs:416-420).
    void zero_grad() {
        for (auto& node : nodes_) node->clear();
    }

    template <typename V>
    void backward_from(Node<V>& output, V seed) {
        for (auto& node : nodes_) node->clear();
        output.accumulate(std::move(seed));
        for (size_t i = output.index + 1; i-- > 0;) nodes_[i]->propagate();
    }

   private:
    std::vector<std::shared_ptr<Backprop>> nodes_;
};

template <typename V>
void Var<V>::backward_with(V seed) const {
    tape_->backward_from(*node_, std::move(seed));
}

template <typename V>
template <typename U>
Var<U> Var<V>::record(U value, std::function<void(const U&)> rule) const {
    return tape_->push<U>(Lazy<U>::ready(std::move(value)), std::move(rule));
}

template <typename V>
template <typename U>
Var<U> Var<V>::record_lazy(Lazy<U> value, std::function<void(const U&)> rule) const {
    return tape_->push<U>(std::move(value), std::move(rule));
}

template <typename T>
using K = Kernels<T>;

// u ⊗ v, computed as the product of u as one column with v as one row
// (`outer`, tape/mod.rs:1000-1006).
template <typename T>
Matrix<T> outer(const Vector<T>& u, const Vector<T>& v) {
    Matrix<T> column(u.len(), 1, u.duplicate().into_storage());
    Matrix<T> row(1, v.len(), v.duplicate().into_storage());
    return K<T>::matmul(column, row);
}

template <typename T>
Matrix<T> matrix_op(const Matrix<T>& a, const Matrix<T>& b, BinaryOp op) {
    return K<T>::matrix_elementwise(a, b, op);
}

template <typename T>
Matrix<T> negated_matrix(const Matrix<T>& m) {
    return K<T>::matrix_broadcast(m, T(-1), BinaryOp::Mul, false);
}

template <typename T>
class MatrixVar;
template <typename T>
class TensorVar;

// `ScalarVar` (tape/mod.rs:600-760): the scalar operations a loss needs.
class ScalarVar : public Var<float> {
   public:
    ScalarVar(Var<float> v) : Var<float>(std::move(v)) {}  // NOLINT: the reference's alias

    // `ScalarVar::scale` (tape/mod.rs:715-720): lazy when its operand is.
    ScalarVar scale(float factor) const {
        auto parent = node_;
        Lazy<float> value = parent->value.is_ready()
                                ? Lazy<float>::ready(parent->get() * factor)
                                : Lazy<float>::deferred([parent, factor] { return parent->get() * factor; });
        return record_lazy<float>(std::move(value), [parent, factor](const float& adjoint) {
            parent->accumulate(adjoint * factor);
        });
    }
    // `ScalarVar::add`, the `Add` arm of `ScalarVar::binary` (tape/mod.rs:611-640,
    // :1385-1392): lazy when either operand is.
    ScalarVar add(const ScalarVar& other) const {
        assert_same_tape(other.tape());
        auto left = node_;
        auto right = other.node_;
        Lazy<float> value = left->value.is_ready() && right->value.is_ready()
                                ? Lazy<float>::ready(left->get() + right->get())
                                : Lazy<float>::deferred([left, right] { return left->get() + right->get(); });
        return record_lazy<float>(std::move(value), [left, right](const float& adjoint) {
            left->accumulate(adjoint);
            right->accumulate(adjoint);
        });
    }
    // `ScalarVar::backward` (tape/mod.rs:547-551): seed 1.
    void backward() const { backward_with(1.0f); }
};

// `VectorVar` (tape/mod.rs:760-1000): what a bias needs.
template <typename T>
class VectorVar : public Var<Vector<T>> {
    using Base = Var<Vector<T>>;

   public:
    VectorVar(Var<Vector<T>> v) : Base(std::move(v)) {}  // NOLINT

    size_t len() const { return this->value().len(); }

    // `VectorVar::outer` (tape/mod.rs:979-987): ū += Ȳ·v, v̄ += uᵀ·Ȳ.
    MatrixVar<T> outer(const VectorVar& other) const;

    VectorVar operator+(const VectorVar& rhs) const { return binary(rhs, BinaryOp::Add); }
    VectorVar operator-(const VectorVar& rhs) const { return binary(rhs, BinaryOp::Sub); }
    VectorVar operator*(const VectorVar& rhs) const { return binary(rhs, BinaryOp::Mul); }
    VectorVar operator/(const VectorVar& rhs) const { return binary(rhs, BinaryOp::Div); }

    // `VectorVar::binary` (tape/mod.rs:764-810): the matrix rules over
    // vectors; `Rem` is refused on the device as `MatrixVar`'s is.
    VectorVar binary(const VectorVar& rhs, BinaryOp op) const {
        this->assert_same_tape(rhs.tape());
        if (op == BinaryOp::Rem) {
            throw Error(TC_UNSUPPORTED, "Hip % could not execute on the GPU; Host fallback is disabled");
        }
        using V = Vector<T>;
        auto left = this->node_;
        auto right = rhs.node_;
        auto apply = [](const V& a, const V& b, BinaryOp o) { return K<T>::vector_elementwise(a, b, o); };
        return this->template record<V>(apply(this->value(), rhs.value(), op), [left, right, op, apply](const V& adjoint) {
            switch (op) {
                case BinaryOp::Add:
                    left->accumulate(adjoint.duplicate());
                    right->accumulate(adjoint.duplicate());
                    break;
                case BinaryOp::Sub:
                    left->accumulate(adjoint.duplicate());
                    right->accumulate(K<T>::vector_broadcast(adjoint, T(-1), BinaryOp::Mul, false));
                    break;
                case BinaryOp::Mul:
                    left->accumulate(apply(adjoint, right->get(), BinaryOp::Mul));
                    right->accumulate(apply(adjoint, left->get(), BinaryOp::Mul));
                    break;
                case BinaryOp::Div: {
                    left->accumulate(apply(adjoint, right->get(), BinaryOp::Div));
                    V squared = apply(right->get(), right->get(), BinaryOp::Mul);
                    V scaled = apply(apply(adjoint, left->get(), BinaryOp::Mul), squared, BinaryOp::Div);
                    right->accumulate(K<T>::vector_broadcast(scaled, T(-1), BinaryOp::Mul, false));
                    break;
                }
                default:
                    break;
            }
        });
    }

    // `VectorVar::to_tensor` (tape/tensor.rs:764-778): the same storage
    // viewed with `shape`; backward reads the gradient as a flat vector.
    TensorVar<T> to_tensor(const Shape& shape) const;

    // `VectorVar::scale`.
    VectorVar scale(T factor) const {
        auto parent = this->node_;
        return this->template record<Vector<T>>(
            K<T>::vector_broadcast(this->value(), factor, BinaryOp::Mul, false),
            [parent, factor](const Vector<T>& adjoint) {
                parent->accumulate(K<T>::vector_broadcast(adjoint, factor, BinaryOp::Mul, false));
            });
    }
};

// `MatrixVar` (tape/mod.rs:1010-1300).
template <typename T>
class MatrixVar : public Var<Matrix<T>> {
    using Base = Var<Matrix<T>>;
    using M = Matrix<T>;

   public:
    MatrixVar(Var<Matrix<T>> v) : Base(std::move(v)) {}  // NOLINT

    std::pair<size_t, size_t> shape() const { return this->value().shape(); }
    size_t rows() const { return this->value().rows(); }
    size_t cols() const { return this->value().cols(); }

    MatrixVar operator+(const MatrixVar& rhs) const { return binary(rhs, BinaryOp::Add); }
    MatrixVar operator-(const MatrixVar& rhs) const { return binary(rhs, BinaryOp::Sub); }
    MatrixVar operator*(const MatrixVar& rhs) const { return binary(rhs, BinaryOp::Mul); }
    MatrixVar operator/(const MatrixVar& rhs) const { return binary(rhs, BinaryOp::Div); }

    // `MatrixVar::binary` (tape/mod.rs:1026-1065).  `Rem` needs a truncated
    // quotient that has no kernel; like Metal's `Rem`, it is refused on the
    // device rather than computed on the host.
    MatrixVar binary(const MatrixVar& rhs, BinaryOp op) const {
        this->assert_same_tape(rhs.tape());
        if (op == BinaryOp::Rem) {
            throw Error(TC_UNSUPPORTED, "Hip % could not execute on the GPU; Host fallback is disabled");
        }
        auto left = this->node_;
        auto right = rhs.node_;
        return this->template record<M>(matrix_op(this->value(), rhs.value(), op), [left, right, op](const M& adjoint) {
            switch (op) {
                case BinaryOp::Add:
                    left->accumulate(adjoint.duplicate());
                    right->accumulate(adjoint.duplicate());
                    break;
                case BinaryOp::Sub:
                    left->accumulate(adjoint.duplicate());
                    right->accumulate(negated_matrix(adjoint));
                    break;
                case BinaryOp::Mul:
                    left->accumulate(matrix_op(adjoint, right->get(), BinaryOp::Mul));
                    right->accumulate(matrix_op(adjoint, left->get(), BinaryOp::Mul));
                    break;
                case BinaryOp::Div: {
                    left->accumulate(matrix_op(adjoint, right->get(), BinaryOp::Div));
                    M squared = matrix_op(right->get(), right->get(), BinaryOp::Mul);
                    M scaled = matrix_op(matrix_op(adjoint, left->get(), BinaryOp::Mul), squared, BinaryOp::Div);
                    right->accumulate(negated_matrix(scaled));
                    break;
                }
                default:
                    break;
            }
        });
    }

    // `maximum` / `minimum` (tape/mod.rs:1067-1097): the adjoint splits by
    // the ½-at-ties share.
    MatrixVar maximum(const MatrixVar& other) const { return select(other, true); }
    MatrixVar minimum(const MatrixVar& other) const { return select(other, false); }

    // `clamp_min`, `clamp_max`, `relu` (tape/mod.rs:1099-1133).
    MatrixVar clamp_min(T floor) const { return select_scalar(floor, true); }
    MatrixVar clamp_max(T ceiling) const { return select_scalar(ceiling, false); }
    MatrixVar relu() const { return clamp_min(T(0)); }

    // `scale` / `shift` / `neg` (tape/mod.rs:1162-1180).
    MatrixVar scale(T factor) const {
        auto parent = this->node_;
        return this->template record<M>(K<T>::matrix_broadcast(this->value(), factor, BinaryOp::Mul, false),
                                        [parent, factor](const M& adjoint) {
                                            parent->accumulate(
                                                K<T>::matrix_broadcast(adjoint, factor, BinaryOp::Mul, false));
                                        });
    }
    MatrixVar shift(T offset) const {
        auto parent = this->node_;
        return this->template record<M>(K<T>::matrix_broadcast(this->value(), offset, BinaryOp::Add, false),
                                        [parent](const M& adjoint) { parent->accumulate(adjoint.duplicate()); });
    }
    MatrixVar neg() const { return scale(T(-1)); }

    // `MatrixVar::matmul` (tape/mod.rs:1195-1216): Ā += C̄·Bᵀ, B̄ += Aᵀ·C̄,
    // each one accumulating product into the current adjoint (or zeros).
    MatrixVar matmul(const MatrixVar& other) const {
        this->assert_same_tape(other.tape());
        auto left = this->node_;
        auto right = other.node_;
        return this->template record<M>(K<T>::matmul(this->value(), other.value()), [left, right](const M& adjoint) {
            M left_adjoint = K<T>::matmul_transposed_add(adjoint, right->get(), Transposed::Right,
                                                         left->current_or_zeros());
            left->adjoint.emplace(std::move(left_adjoint));
            M right_adjoint = K<T>::matmul_transposed_add(left->get(), adjoint, Transposed::Left,
                                                          right->current_or_zeros());
            right->adjoint.emplace(std::move(right_adjoint));
        });
    }

    // `MatrixVar::matmul_add` (tape/mod.rs:1219-1246).
    MatrixVar matmul_add(const MatrixVar& other, const MatrixVar& addend) const {
        this->assert_same_tape(other.tape());
        this->assert_same_tape(addend.tape());
        auto left = this->node_;
        auto right = other.node_;
        auto bias = addend.node_;
        return this->template record<M>(
            K<T>::matmul_add(this->value(), other.value(), addend.value().duplicate()),
            [left, right, bias](const M& adjoint) {
                M left_adjoint = K<T>::matmul_transposed_add(adjoint, right->get(), Transposed::Right,
                                                             left->current_or_zeros());
                left->adjoint.emplace(std::move(left_adjoint));
                M right_adjoint = K<T>::matmul_transposed_add(left->get(), adjoint, Transposed::Left,
                                                              right->current_or_zeros());
                right->adjoint.emplace(std::move(right_adjoint));
                bias->accumulate(adjoint.duplicate());
            });
    }

    // `MatrixVar::matvec` / `matvec_add` (tape/mod.rs:1249-1274):
    // M̄ += ȳ ⊗ v, v̄ += ȳᵀ·M, and the addend's adjoint is ȳ.
    VectorVar<T> matvec(const VectorVar<T>& v) const {
        this->assert_same_tape(v.tape());
        auto matrix = this->node_;
        auto vector = v.node();
        return VectorVar<T>(this->template record<Vector<T>>(
            K<T>::matvec(this->value(), v.value()), [matrix, vector](const Vector<T>& adjoint) {
                matrix->accumulate(hip::outer(adjoint, vector->get()));
                vector->accumulate(K<T>::vecmat(adjoint, matrix->get()));
            }));
    }
    VectorVar<T> matvec_add(const VectorVar<T>& v, const VectorVar<T>& addend) const {
        this->assert_same_tape(v.tape());
        this->assert_same_tape(addend.tape());
        auto matrix = this->node_;
        auto vector = v.node();
        auto bias = addend.node();
        return VectorVar<T>(this->template record<Vector<T>>(
            K<T>::matvec_add(this->value(), v.value(), addend.value().duplicate()),
            [matrix, vector, bias](const Vector<T>& adjoint) {
                matrix->accumulate(hip::outer(adjoint, vector->get()));
                vector->accumulate(K<T>::vecmat(adjoint, matrix->get()));
                bias->accumulate(adjoint.duplicate());
            }));
    }

    // `MatrixVar::transpose` (tape/mod.rs:1272-1279).
    MatrixVar transpose() const {
        auto parent = this->node_;
        return this->template record<M>(K<T>::transpose(this->value()),
                                        [parent](const M& adjoint) { parent->accumulate(K<T>::transpose(adjoint)); });
    }

    // `MatrixVar::sum` (tape/mod.rs:1286-1297): recorded unread -- the
    // reduction and the read of its result are queued now, and only reading
    // the value waits, for that read; the adjoint is a device fill of the
    // scalar adjoint.
    ScalarVar sum() const {
        auto parent = this->node_;
        const uint64_t ticket = K<T>::reduce_async(parent->get().storage(), Reduce::Sum);
        Lazy<float> total = Lazy<float>::deferred([ticket] { return static_cast<float>(K<T>::read(ticket)); });
        return ScalarVar(this->template record_lazy<float>(std::move(total), [parent](const float& adjoint) {
            const M& value = parent->get();
            parent->accumulate(M::filled(value.rows(), value.cols(), adjoint));
        }));
    }

    // `MatrixVar::to_tensor` (tape/tensor.rs:744-761): the row-major storage
    // viewed with `shape`; backward reads the gradient as rows × cols.
    TensorVar<T> to_tensor(const Shape& shape) const;

    // `MatrixVar::frobenius_dot` (tape/mod.rs:1299-1302).
    ScalarVar frobenius_dot(const MatrixVar& other) const { return binary(other, BinaryOp::Mul).sum(); }

   private:
    MatrixVar select(const MatrixVar& other, bool largest) const {
        this->assert_same_tape(other.tape());
        auto left = this->node_;
        auto right = other.node_;
        const Compare op = largest ? Compare::Max : Compare::Min;
        return this->template record<M>(
            K<T>::matrix_compare(this->value(), other.value(), op), [left, right, largest](const M& adjoint) {
                M share = K<T>::matrix_compare(left->get(), right->get(), Compare::MaxShare);
                M complement = K<T>::matrix_broadcast(share, T(1), BinaryOp::Sub, true);
                const M& mine = largest ? share : complement;
                const M& theirs = largest ? complement : share;
                left->accumulate(K<T>::matrix_elementwise(adjoint, mine, BinaryOp::Mul));
                right->accumulate(K<T>::matrix_elementwise(adjoint, theirs, BinaryOp::Mul));
            });
    }

    MatrixVar select_scalar(T scalar, bool largest) const {
        auto parent = this->node_;
        const Compare op = largest ? Compare::Max : Compare::Min;
        return this->template record<M>(
            K<T>::matrix_compare_scalar(this->value(), scalar, op, false), [parent, scalar, largest](const M& adjoint) {
                M share = K<T>::matrix_compare_scalar(parent->get(), scalar, Compare::MaxShare, false);
                M weight = largest ? std::move(share) : K<T>::matrix_broadcast(share, T(1), BinaryOp::Sub, true);
                parent->accumulate(K<T>::matrix_elementwise(adjoint, weight, BinaryOp::Mul));
            });
    }

    friend class VectorVar<T>;
};

// `sum_to_shape` (tape/tensor.rs:18-37): the adjoint of a broadcast, summed
// down to the operand's `shape`: one reduction folds the gradient's extra
// leading axes and each axis that broadcasting stretched from extent 1.
template <typename T>
Tensor<T> sum_to_shape(const Tensor<T>& gradient, const Shape& shape) {
    if (gradient.shape() == shape) return gradient.duplicate();
    const size_t added = gradient.rank() - shape.size();
    std::vector<size_t> axes;
    for (size_t axis = 0; axis < gradient.rank(); axis++) {
        if (axis < added || (shape[axis - added] == 1 && gradient.shape()[axis] != 1)) axes.push_back(axis);
    }
    Tensor<T> summed = axes.empty() ? gradient.duplicate()
                                    : K<T>::reduce_axes(gradient, axes, true, TC_AXIS_FOLD, Reduce::Sum, 0, true, T(0));
    return std::move(summed).reshape(shape);
}

// `Node::accumulate_slice` (tape/tensor.rs:55-82): adds `delta` to one
// window along `axis` (from index `start`) of the node's gradient.  A node
// without a gradient yet gets a zero tensor with `delta` written into the
// window; otherwise only the window is read, summed and written back.
template <typename T>
void accumulate_slice(Node<Tensor<T>>& node, size_t axis, size_t start, const Tensor<T>& delta) {
    if (node.adjoint) {
        Tensor<T> sum = K<T>::narrow_add(*node.adjoint, axis, start, delta);
        K<T>::write_slice(*node.adjoint, axis, start, sum);
    } else {
        Tensor<T> zeros = Tensor<T>::filled(node.get().shape(), T(0));
        K<T>::write_slice(zeros, axis, start, delta);
        node.adjoint.emplace(std::move(zeros));
    }
}

// `Correction` (statistics/mod.rs:80-101): the variance's divisor n, or
// n − 1 for a sample; too few elements leave it undefined.
enum class Correction { Population, Sample };

// `TensorVar` (tape/tensor.rs): an N-dimensional value recorded on the tape.
// Its backward rules call only the device kernels of backend.hpp, so the
// whole backward pass runs on the GPU; a gradient flowing to a broadcast
// operand is reduced to that operand's shape first.
template <typename T>
class TensorVar : public Var<Tensor<T>> {
    using Base = Var<Tensor<T>>;
    using X = Tensor<T>;

   public:
    TensorVar(Var<Tensor<T>> v) : Base(std::move(v)) {}  // NOLINT

    const Shape& shape() const { return this->value().shape(); }
    size_t rank() const { return this->value().rank(); }
    size_t len() const { return this->value().len(); }

    TensorVar operator+(const TensorVar& rhs) const { return binary(rhs, BinaryOp::Add); }
    TensorVar operator-(const TensorVar& rhs) const { return binary(rhs, BinaryOp::Sub); }
    TensorVar operator*(const TensorVar& rhs) const { return binary(rhs, BinaryOp::Mul); }
    TensorVar operator/(const TensorVar& rhs) const { return binary(rhs, BinaryOp::Div); }

    // `TensorVar::binary` (tape/tensor.rs:126-160): c = a op b with
    // broadcasting; both gradients are reduced to their operands' shapes.
    // Remainder has no rule here, as in the reference.
    TensorVar binary(const TensorVar& rhs, BinaryOp op) const {
        this->assert_same_tape(rhs.tape());
        if (op == BinaryOp::Rem) throw std::invalid_argument("no tensor remainder is recorded");
        auto left = this->node_;
        auto right = rhs.node_;
        return this->template record<X>(K<T>::elementwise(this->value(), rhs.value(), op), [left, right, op](const X& adjoint) {
            const X& a = left->get();
            const X& b = right->get();
            switch (op) {
                case BinaryOp::Add:
                    left->accumulate(sum_to_shape(adjoint, a.shape()));
                    right->accumulate(sum_to_shape(adjoint, b.shape()));
                    break;
                case BinaryOp::Sub:
                    left->accumulate(sum_to_shape(adjoint, a.shape()));
                    right->accumulate(K<T>::scale(sum_to_shape(adjoint, b.shape()), T(-1)));
                    break;
                case BinaryOp::Mul:
                    left->accumulate(sum_to_shape(K<T>::elementwise(adjoint, b, op), a.shape()));
                    right->accumulate(sum_to_shape(K<T>::elementwise(adjoint, a, op), b.shape()));
                    break;
                case BinaryOp::Div: {
                    // d(a/b)/da = 1/b, d(a/b)/db = −a/b²
                    X over = K<T>::elementwise(adjoint, b, BinaryOp::Div);
                    X scaled = K<T>::elementwise(K<T>::elementwise(over, a, BinaryOp::Mul), b, BinaryOp::Div);
                    left->accumulate(sum_to_shape(over, a.shape()));
                    right->accumulate(K<T>::scale(sum_to_shape(scaled, b.shape()), T(-1)));
                    break;
                }
                default:
                    break;
            }
        });
    }

    // `TensorVar::power` (tape/tensor.rs:162-185): d(a^b)/da = b·a^(b−1)
    // and d(a^b)/db = a^b·ln a, each gradient reduced to its operand's shape.
    TensorVar power(const TensorVar& exponent) const {
        this->assert_same_tape(exponent.tape());
        auto base = this->node_;
        auto power = exponent.node_;
        return this->template record<X>(K<T>::power(this->value(), exponent.value()), [base, power](const X& adjoint) {
            const X& a = base->get();
            const X& b = power->get();
            X lowered = K<T>::with_scalar(b, T(1), BinaryOp::Sub, false);
            X slope = K<T>::elementwise(K<T>::power(a, lowered), b, BinaryOp::Mul);
            base->accumulate(sum_to_shape(K<T>::elementwise(adjoint, slope, BinaryOp::Mul), a.shape()));
            X growth = K<T>::elementwise(K<T>::power(a, b), K<T>::unary(a, Analytic::Ln), BinaryOp::Mul);
            power->accumulate(sum_to_shape(K<T>::elementwise(adjoint, growth, BinaryOp::Mul), b.shape()));
        });
    }

    // `TensorVar::power_scalar` (tape/tensor.rs:187-208): x^s, or s^x when
    // `scalar_left`.
    TensorVar power_scalar(T scalar, bool scalar_left) const {
        auto parent = this->node_;
        return this->template record<X>(
            K<T>::power_scalar(this->value(), scalar, scalar_left), [parent, scalar, scalar_left](const X& adjoint) {
                const X& x = parent->get();
                X slope = scalar_left ? K<T>::scale(K<T>::power_scalar(x, scalar, true), T(std::log(scalar)))
                                      : K<T>::scale(K<T>::power_scalar(x, scalar - T(1), false), scalar);
                parent->accumulate(K<T>::elementwise(adjoint, slope, BinaryOp::Mul));
            });
    }

    // `maximum` / `minimum` (tape/tensor.rs:210-250): the gradient follows
    // the operand the result came from; equal operands share it in halves.
    TensorVar maximum(const TensorVar& other) const { return select_pair(other, true); }
    TensorVar minimum(const TensorVar& other) const { return select_pair(other, false); }

    // `clamp_min`, `clamp_max`, `clamp`, `relu`, `abs` (tape/tensor.rs:252-281).
    TensorVar clamp_min(T floor) const { return select_scalar(floor, true); }
    TensorVar clamp_max(T ceiling) const { return select_scalar(ceiling, false); }
    TensorVar clamp(T floor, T ceiling) const {
        if (floor > ceiling) throw std::invalid_argument("clamp: the lower bound exceeds the upper one");
        return clamp_min(floor).clamp_max(ceiling);
    }
    TensorVar relu() const { return clamp_min(T(0)); }
    TensorVar abs() const { return maximum(scale(T(-1))); }

    // `TensorVar::analytic` (tape/tensor.rs:299-310): x̄ += f'(x)·ȳ in one
    // dual dispatch.
    TensorVar analytic(Analytic f) const {
        auto parent = this->node_;
        return this->template record<X>(K<T>::unary(this->value(), f), [parent, f](const X& adjoint) {
            parent->accumulate(std::move(K<T>::unary_dual(parent->get(), adjoint, f).second));
        });
    }

    // `neg`, `scale`, `shift` (tape/tensor.rs:311-333).
    TensorVar neg() const { return scale(T(-1)); }
    TensorVar scale(T factor) const {
        auto parent = this->node_;
        return this->template record<X>(K<T>::scale(this->value(), factor), [parent, factor](const X& adjoint) {
            parent->accumulate(K<T>::scale(adjoint, factor));
        });
    }
    TensorVar shift(T offset) const {
        auto parent = this->node_;
        return this->template record<X>(K<T>::with_scalar(this->value(), offset, BinaryOp::Add, false),
                                        [parent](const X& adjoint) { parent->accumulate(adjoint.duplicate()); });
    }

    // ---- layout (tape/tensor.rs:335-420, :555-570) ----

    // `reshape` (:335-350): backward views the gradient in the input's shape.
    TensorVar reshape(const Shape& shape) const {
        auto parent = this->node_;
        return this->template record<X>(this->value().duplicate().reshape(shape), [parent](const X& adjoint) {
            parent->accumulate(adjoint.duplicate().reshape(parent->get().shape()));
        });
    }
    // `contiguous` (:371-377): a copy; the adjoint passes through.
    TensorVar contiguous() const {
        auto parent = this->node_;
        return this->template record<X>(this->value().duplicate(),
                                        [parent](const X& adjoint) { parent->accumulate(adjoint.duplicate()); });
    }
    // `permute` (:379-400): the adjoint permuted back by the inverse.
    TensorVar permute(const std::vector<size_t>& axes) const {
        X value = K<T>::permute(this->value(), axes);
        std::vector<size_t> inverse(axes.size());
        for (size_t k = 0; k < axes.size(); k++) inverse[axes[k]] = k;
        auto parent = this->node_;
        return this->template record<X>(std::move(value), [parent, inverse](const X& adjoint) {
            parent->accumulate(K<T>::permute(adjoint, inverse));
        });
    }
    // `transpose` (:402-420): two axes swapped, negative ones from the end.
    TensorVar transpose(long a, long b) const {
        const std::vector<size_t> ab = K<T>::resolve_axes({a}, shape(), "transpose");
        const std::vector<size_t> bb = K<T>::resolve_axes({b}, shape(), "transpose");
        std::vector<size_t> axes(rank());
        for (size_t k = 0; k < axes.size(); k++) axes[k] = k;
        std::swap(axes[ab[0]], axes[bb[0]]);
        return permute(axes);
    }
    // `squeeze` / `unsqueeze` (:351-370): reshapes that drop or add an
    // axis of extent 1.
    TensorVar squeeze(long axis) const {
        const size_t k = K<T>::resolve_axes({axis}, shape(), "squeeze")[0];
        if (shape()[k] != 1) {
            throw std::invalid_argument("squeeze: axis " + std::to_string(axis) + " of shape " + shape_text(shape()) +
                                        " is not of extent 1");
        }
        Shape s = shape();
        s.erase(s.begin() + static_cast<long>(k));
        return reshape(s);
    }
    TensorVar unsqueeze(long axis) const {
        const long rank = static_cast<long>(this->rank()) + 1;
        const long k = axis < 0 ? axis + rank : axis;
        if (k < 0 || k >= rank) {
            throw std::invalid_argument("unsqueeze: axis " + std::to_string(axis) + " is out of range for shape " +
                                        shape_text(shape()) + " (" + std::to_string(rank) + " axes)");
        }
        Shape s = shape();
        s.insert(s.begin() + k, 1);
        return reshape(s);
    }

    // `narrow` (:422-435): the adjoint written back where the slice came
    // from (`accumulate_slice`); `slice` takes a range of the same axis.
    TensorVar narrow(long axis, size_t start, size_t len) const {
        const size_t k = K<T>::resolve_axes({axis}, shape(), "narrow")[0];
        auto parent = this->node_;
        return this->template record<X>(K<T>::narrow(this->value(), k, start, len), [parent, k, start](const X& adjoint) {
            accumulate_slice(*parent, k, start, adjoint);
        });
    }
    TensorVar slice(long axis, size_t start, size_t end) const {
        if (end < start) throw std::invalid_argument("slice: the range " + std::to_string(start) + ".." +
                                                     std::to_string(end) + " runs backwards");
        return narrow(axis, start, end - start);
    }
    // `select` (:448-462): index `index` of `axis`, the axis dropped.
    TensorVar select(long axis, size_t index) const {
        const size_t k = K<T>::resolve_axes({axis}, shape(), "select")[0];
        if (index >= shape()[k]) {
            throw std::invalid_argument("select: index " + std::to_string(index) + " is out of range for axis " +
                                        std::to_string(k) + " of shape " + shape_text(shape()));
        }
        Shape dropped = shape();
        dropped.erase(dropped.begin() + static_cast<long>(k));
        auto parent = this->node_;
        X value = K<T>::narrow(this->value(), k, index, 1).reshape(dropped);
        return this->template record<X>(std::move(value), [parent, k, index](const X& adjoint) {
            Shape kept = adjoint.shape();
            kept.insert(kept.begin() + static_cast<long>(k), 1);
            accumulate_slice(*parent, k, index, adjoint.duplicate().reshape(kept));
        });
    }
    // `split` (:464-487): consecutive narrows of `sizes`, which must cover
    // the axis; `chunk` (:489-500): `parts` equal pieces.
    std::vector<TensorVar> split(long axis, const std::vector<size_t>& sizes) const {
        const size_t k = K<T>::resolve_axes({axis}, shape(), "split")[0];
        size_t total = 0;
        for (size_t size : sizes) total += size;
        if (total != shape()[k]) {
            throw std::invalid_argument("split: sizes adding to " + std::to_string(total) + " for axis " +
                                        std::to_string(k) + " of shape " + shape_text(shape()));
        }
        std::vector<TensorVar> pieces;
        size_t start = 0;
        for (size_t size : sizes) {
            pieces.push_back(narrow(static_cast<long>(k), start, size));
            start += size;
        }
        return pieces;
    }
    std::vector<TensorVar> chunk(long axis, size_t parts) const {
        const size_t k = K<T>::resolve_axes({axis}, shape(), "chunk")[0];
        if (parts == 0 || shape()[k] % parts != 0) {
            throw std::invalid_argument("chunk: axis " + std::to_string(k) + " of shape " + shape_text(shape()) +
                                        " does not split into " + std::to_string(parts) + " equal parts");
        }
        return split(static_cast<long>(k), std::vector<size_t>(parts, shape()[k] / parts));
    }
    // `concat` (:502-533): backward hands each input the window of the
    // gradient that its elements occupy.
    static TensorVar concat(const std::vector<TensorVar>& pieces, long axis) {
        if (pieces.empty()) throw std::invalid_argument("concat: there are no tensors to join");
        const TensorVar& first = pieces[0];
        std::vector<const X*> values;
        std::vector<std::shared_ptr<Node<X>>> nodes;
        for (const TensorVar& piece : pieces) {
            first.assert_same_tape(piece.tape());
            values.push_back(&piece.value());
            nodes.push_back(piece.node_);
        }
        const size_t k = K<T>::resolve_axes({axis}, first.shape(), "concat")[0];
        return first.template record<X>(K<T>::concat(values, k), [nodes, k](const X& adjoint) {
            size_t start = 0;
            for (const auto& node : nodes) {
                const size_t len = node->get().shape()[k];
                node->accumulate(K<T>::narrow(adjoint, k, start, len));
                start += len;
            }
        });
    }
    // `stack` (:535-553): the pieces joined along a new axis, each lifted
    // by `unsqueeze` and then one `concat`; the adjoints are the same blocks
    // the reference's `select`s give.
    static TensorVar stack(const std::vector<TensorVar>& pieces, long axis) {
        if (pieces.empty()) throw std::invalid_argument("stack: there are no tensors to stack");
        std::vector<TensorVar> lifted;
        for (const TensorVar& piece : pieces) {
            if (piece.shape() != pieces[0].shape()) {
                throw std::invalid_argument("stack: shapes " + shape_text(pieces[0].shape()) + " and " +
                                            shape_text(piece.shape()) + " differ");
            }
            lifted.push_back(piece.unsqueeze(axis));
        }
        const long rank = static_cast<long>(pieces[0].rank()) + 1;
        return concat(lifted, axis < 0 ? axis + rank : axis);
    }

    // `broadcast_to` (:555-570): the adjoint summed back to this shape.
    TensorVar broadcast_to(const Shape& shape) const {
        auto parent = this->node_;
        return this->template record<X>(K<T>::broadcast_to(this->value(), shape), [parent](const X& adjoint) {
            parent->accumulate(sum_to_shape(adjoint, parent->get().shape()));
        });
    }

    // ---- reductions (tape/tensor.rs:572-684) ----

    // `sum_axes`: backward broadcasts each output's gradient over the inputs
    // it summed.
    TensorVar sum_axes(const std::vector<long>& axes, bool keep_dims) const {
        const Folding f = folding(axes, "sum_axes");
        auto parent = this->node_;
        X value = K<T>::reduce_axes(this->value(), f.folded, keep_dims, TC_AXIS_FOLD, Reduce::Sum, 0, true, T(0));
        return this->template record<X>(std::move(value), [parent, f](const X& adjoint) {
            parent->accumulate(K<T>::broadcast_to(adjoint.duplicate().reshape(f.kept), parent->get().shape()));
        });
    }
    // `mean_axes`: as the sum, divided by the number of elements averaged.
    TensorVar mean_axes(const std::vector<long>& axes, bool keep_dims) const {
        const Folding f = folding(axes, "mean_axes");
        auto parent = this->node_;
        X value = K<T>::reduce_axes(this->value(), f.folded, keep_dims, TC_AXIS_MEAN, Reduce::Sum, 0, true,
                                    std::numeric_limits<T>::quiet_NaN());
        const T share = T(1.0 / static_cast<double>(f.count));
        return this->template record<X>(std::move(value), [parent, f, share](const X& adjoint) {
            X scaled = K<T>::scale(adjoint, share);
            parent->accumulate(K<T>::broadcast_to(std::move(scaled).reshape(f.kept), parent->get().shape()));
        });
    }
    // `var_axes`: dvar/dx = 2(x − mean)/d with d the divisor the correction
    // gives; where there are too few elements for it, value and gradient are
    // both NaN.
    TensorVar var_axes(const std::vector<long>& axes, Correction correction, bool keep_dims) const {
        const Folding f = folding(axes, "var_axes");
        const bool sample = correction == Correction::Sample;
        const bool defined = sample ? f.count >= 2 : f.count >= 1;
        const size_t divisor = defined ? (sample ? f.count - 1 : f.count) : 0;
        const T nan = std::numeric_limits<T>::quiet_NaN();
        X value = K<T>::reduce_axes(this->value(), f.folded, keep_dims, TC_AXIS_VARIANCE, Reduce::Sum, divisor,
                                    defined, nan);
        const T factor = defined ? T(2.0 / static_cast<double>(divisor)) : nan;
        auto parent = this->node_;
        return this->template record<X>(std::move(value), [parent, f, factor](const X& adjoint) {
            const X& x = parent->get();
            X mean = K<T>::reduce_axes(x, f.folded, true, TC_AXIS_MEAN, Reduce::Sum, 0, true,
                                       std::numeric_limits<T>::quiet_NaN());
            X deviation = K<T>::elementwise(x, mean, BinaryOp::Sub);
            X weight = K<T>::scale(adjoint, factor);
            parent->accumulate(K<T>::elementwise(deviation, std::move(weight).reshape(f.kept), BinaryOp::Mul));
        });
    }
    // `max_axes` / `min_axes` through `extreme_axes`: the adjoint goes to
    // the elements equal to their slice's extreme, shared evenly among ties;
    // NaNs, which the fold passes over, receive none.
    TensorVar max_axes(const std::vector<long>& axes, bool keep_dims) const {
        return extreme_axes(axes, keep_dims, Reduce::Max, "max_axes");
    }
    TensorVar min_axes(const std::vector<long>& axes, bool keep_dims) const {
        return extreme_axes(axes, keep_dims, Reduce::Min, "min_axes");
    }

    // `TensorVar::sum` (tape/tensor.rs:686-697): recorded unread, as
    // `MatrixVar::sum` is; each element's adjoint is the scalar's, a fill.
    ScalarVar sum() const {
        auto parent = this->node_;
        Lazy<float> total = Lazy<float>::ready(0.0f);
        if (parent->get().len()) {
            const uint64_t ticket = K<T>::reduce_async(parent->get().storage(), Reduce::Sum);
            total = Lazy<float>::deferred([ticket] { return static_cast<float>(K<T>::read(ticket)); });
        }
        return ScalarVar(this->template record_lazy<float>(std::move(total), [parent](const float& adjoint) {
            parent->accumulate(X::filled(parent->get().shape(), T(adjoint)));
        }));
    }
    // `TensorVar::mean` (:699-701).
    ScalarVar mean() const { return sum().scale(static_cast<float>(1.0 / static_cast<double>(len()))); }

    // `TensorVar::to_vector` (tape/tensor.rs:733-742): the row-major storage
    // as one vector; backward views the gradient in the tensor's shape.
    VectorVar<T> to_vector() const {
        auto parent = this->node_;
        Vector<T> value(this->value().duplicate().into_storage());
        return VectorVar<T>(this->template record<Vector<T>>(std::move(value), [parent](const Vector<T>& adjoint) {
            parent->accumulate(X(parent->get().shape(), adjoint.duplicate().into_storage()));
        }));
    }

    // `TensorVar::to_matrix` (tape/tensor.rs:703-731): the row-major storage
    // as rows × cols; backward views the gradient in the tensor's shape.
    MatrixVar<T> to_matrix(size_t rows, size_t cols) const {
        if (rows * cols != len()) {
            throw std::invalid_argument("to_matrix: shape " + shape_text(shape()) + " holds " + std::to_string(len()) +
                                        " elements, which " + std::to_string(rows) + "×" + std::to_string(cols) +
                                        " cannot");
        }
        auto parent = this->node_;
        Matrix<T> value(rows, cols, this->value().duplicate().into_storage());
        return MatrixVar<T>(this->template record<Matrix<T>>(std::move(value), [parent](const Matrix<T>& adjoint) {
            parent->accumulate(X(parent->get().shape(), adjoint.duplicate().into_storage()));
        }));
    }

   private:
    // `folding` (tape/tensor.rs:39-53): which axes a reduction folds, the
    // input shape with those axes set to 1, and how many inputs each output
    // reduces.
    struct Folding {
        std::vector<size_t> folded;
        Shape kept;
        size_t count;
    };
    Folding folding(const std::vector<long>& axes, const char* operation) const {
        Folding f{K<T>::resolve_axes(axes, shape(), operation), shape(), 1};
        for (size_t axis : f.folded) {
            f.count *= f.kept[axis];
            f.kept[axis] = 1;
        }
        return f;
    }

    TensorVar extreme_axes(const std::vector<long>& axes, bool keep_dims, Reduce op, const char* operation) const {
        const Folding f = folding(axes, operation);
        const T identity = op == Reduce::Max ? -std::numeric_limits<T>::infinity() : std::numeric_limits<T>::infinity();
        X value = K<T>::reduce_axes(this->value(), f.folded, keep_dims, TC_AXIS_FOLD, op, 0, true, identity);
        const Compare attains = op == Reduce::Max ? Compare::GreaterEqual : Compare::LessEqual;
        auto parent = this->node_;
        return this->template record<X>(std::move(value), [parent, f, op, attains, identity](const X& adjoint) {
            const X& x = parent->get();
            X extreme = K<T>::reduce_axes(x, f.folded, true, TC_AXIS_FOLD, op, 0, true, identity);
            X mask = K<T>::compare(x, extreme, attains);
            X ties = K<T>::compare_scalar(
                K<T>::reduce_axes(mask, f.folded, true, TC_AXIS_FOLD, Reduce::Sum, 0, true, T(0)), T(1),
                Compare::Max, false);
            X share = K<T>::elementwise(adjoint.duplicate().reshape(f.kept), ties, BinaryOp::Div);
            parent->accumulate(K<T>::elementwise(mask, share, BinaryOp::Mul));
        });
    }

    TensorVar select_pair(const TensorVar& other, bool largest) const {
        this->assert_same_tape(other.tape());
        auto left = this->node_;
        auto right = other.node_;
        const Compare op = largest ? Compare::Max : Compare::Min;
        return this->template record<X>(
            K<T>::compare(this->value(), other.value(), op), [left, right, largest](const X& adjoint) {
                const X& a = left->get();
                const X& b = right->get();
                X share = K<T>::compare(a, b, Compare::MaxShare);
                X complement = K<T>::with_scalar(share, T(1), BinaryOp::Sub, true);
                const X& mine = largest ? share : complement;
                const X& theirs = largest ? complement : share;
                left->accumulate(sum_to_shape(K<T>::elementwise(adjoint, mine, BinaryOp::Mul), a.shape()));
                right->accumulate(sum_to_shape(K<T>::elementwise(adjoint, theirs, BinaryOp::Mul), b.shape()));
            });
    }

    TensorVar select_scalar(T scalar, bool largest) const {
        auto parent = this->node_;
        const Compare op = largest ? Compare::Max : Compare::Min;
        return this->template record<X>(
            K<T>::compare_scalar(this->value(), scalar, op, false), [parent, scalar, largest](const X& adjoint) {
                X share = K<T>::compare_scalar(parent->get(), scalar, Compare::MaxShare, false);
                X weight = largest ? std::move(share) : K<T>::with_scalar(share, T(1), BinaryOp::Sub, true);
                parent->accumulate(K<T>::elementwise(adjoint, weight, BinaryOp::Mul));
            });
    }
};

template <typename T>
TensorVar<T> VectorVar<T>::to_tensor(const Shape& shape) const {
    auto parent = this->node_;
    Tensor<T> value = Tensor<T>(Shape{this->len()}, this->value().duplicate().into_storage()).reshape(shape);
    return TensorVar<T>(this->template record<Tensor<T>>(std::move(value), [parent](const Tensor<T>& adjoint) {
        parent->accumulate(Vector<T>(adjoint.duplicate().into_storage()));
    }));
}

template <typename T>
TensorVar<T> MatrixVar<T>::to_tensor(const Shape& shape) const {
    auto parent = this->node_;
    Tensor<T> value = Tensor<T>(Shape{this->rows(), this->cols()}, this->value().duplicate().into_storage()).reshape(shape);
    return TensorVar<T>(this->template record<Tensor<T>>(std::move(value), [parent](const Tensor<T>& adjoint) {
        const Matrix<T>& m = parent->get();
        parent->accumulate(Matrix<T>(m.rows(), m.cols(), adjoint.duplicate().into_storage()));
    }));
}

template <typename T>
MatrixVar<T> VectorVar<T>::outer(const VectorVar& other) const {
    this->assert_same_tape(other.tape());
    auto left = this->node_;
    auto right = other.node_;
    return MatrixVar<T>(this->template record<Matrix<T>>(
        hip::outer(this->value(), other.value()), [left, right](const Matrix<T>& adjoint) {
            left->accumulate(K<T>::matvec(adjoint, right->get()));
            right->accumulate(K<T>::vecmat(left->get(), adjoint));
        }));
}

}  // namespace hip
}  // namespace tensorcrate
