// Reverse-mode differentiation over Hip storage: tensorcrate's `Tape`, its
// nodes and the scalar, vector and matrix variables with their backward
// rules (src/tensors/tape/mod.rs), restated in C++ over backend.hpp.
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

#include <functional>
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
struct TapeValue<Matrix<T>> {
    static Matrix<T> zeros_like(const Matrix<T>& m) { return Matrix<T>::filled(m.rows(), m.cols(), T(0)); }
    static Matrix<T> duplicate(const Matrix<T>& m) { return m.duplicate(); }
    static Matrix<T> add(const Matrix<T>& a, const Matrix<T>& b) {
        return Kernels<T>::matrix_elementwise(a, b, BinaryOp::Add);
    }
};

// A node's value, computed when recorded or — for a scalar reduced from
// device storage — when first read (`Lazy`, tape/mod.rs:253-295).
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

// The type-erased face of a node (`Backprop`, tape/mod.rs:333-346).
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

// The outer product u ⊗ v as a (u.len × 1)·(1 × v.len) product
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
