// A tape of tensor variables driven through C entry points
// (include/tchip_host.h): each call records one `TensorVar` operation of
// tape.hpp (src/tensors/tape/tensor.rs) by handle, so the backward rules can
// be checked operation by operation from Python against finite differences,
// the way tests/tensor_autodiff.rs drives them in the reference.
//
// Handles index the variables in recording order; a handle names either a
// tensor or a scalar (a whole-tensor sum or mean).

#include <memory>
#include <string>
#include <variant>
#include <vector>

#include "backend.hpp"
#include "entry.hpp"
#include "tape.hpp"
#include "tchip_host.h"

using namespace tensorcrate::hip;

struct tch_tape {
    Tape tape;
    std::vector<std::variant<TensorVar<float>, ScalarVar>> vars;

    uint32_t add(std::variant<TensorVar<float>, ScalarVar> v) {
        vars.push_back(std::move(v));
        return static_cast<uint32_t>(vars.size() - 1);
    }
    const std::variant<TensorVar<float>, ScalarVar>& at(uint32_t handle) const {
        if (handle >= vars.size()) throw std::invalid_argument("tape: no variable " + std::to_string(handle));
        return vars[handle];
    }
    const TensorVar<float>& tensor(uint32_t handle) const {
        const auto& v = at(handle);
        if (!std::holds_alternative<TensorVar<float>>(v)) {
            throw std::invalid_argument("tape: variable " + std::to_string(handle) + " is a scalar, not a tensor");
        }
        return std::get<TensorVar<float>>(v);
    }
    const ScalarVar& scalar(uint32_t handle) const {
        const auto& v = at(handle);
        if (!std::holds_alternative<ScalarVar>(v)) {
            throw std::invalid_argument("tape: variable " + std::to_string(handle) + " is a tensor, not a scalar");
        }
        return std::get<ScalarVar>(v);
    }
};

namespace {

Shape shape_of(uint32_t rank, const uint64_t* dims) {
    return Shape(dims, dims + rank);
}

std::vector<long> axes_of(uint32_t count, const int64_t* axes) {
    return std::vector<long>(axes, axes + count);
}

// `a`'s last axis against the k × n matrix `b`, through `to_matrix`,
// `MatrixVar::matmul` and `to_tensor`, as the reference's matrix round trip
// does (tests/tensor_autodiff.rs:247-250).
TensorVar<float> product(const TensorVar<float>& a, const TensorVar<float>& b) {
    if (a.rank() == 0 || b.rank() != 2) {
        throw std::invalid_argument("matmul: shapes " + shape_text(a.shape()) + " and " + shape_text(b.shape()) +
                                    " are not a tensor and a matrix");
    }
    const size_t k = a.shape().back();
    const size_t rows = k ? a.len() / k : 0;
    Shape out(a.shape().begin(), a.shape().end() - 1);
    out.push_back(b.shape()[1]);
    return a.to_matrix(rows, k).matmul(b.to_matrix(b.shape()[0], b.shape()[1])).to_tensor(out);
}

}  // namespace

extern "C" {

int tch_tape_create(tch_tape** out) {
    return guarded([&] { *out = new tch_tape(); });
}

void tch_tape_destroy(tch_tape* tape) { delete tape; }

int tch_tape_tensor(tch_tape* t, uint32_t rank, const uint64_t* shape, const float* values, uint32_t* out) {
    return guarded([&] {
        Shape s = shape_of(rank, shape);
        const size_t n = element_count(s);
        Tensor<float> value(s, n ? Storage<float>::store(values, n) : Storage<float>(0));
        *out = t->add(TensorVar<float>(t->tape.tensor(std::move(value))));
    });
}

int tch_tape_binary(tch_tape* t, uint32_t op, uint32_t a, uint32_t b, uint32_t* out) {
    return guarded([&] {
        const TensorVar<float>& x = t->tensor(a);
        const TensorVar<float>& y = t->tensor(b);
        switch (op) {
            case TCH_ADD: *out = t->add(x + y); break;
            case TCH_SUB: *out = t->add(x - y); break;
            case TCH_MUL: *out = t->add(x * y); break;
            case TCH_DIV: *out = t->add(x / y); break;
            case TCH_MAXIMUM: *out = t->add(x.maximum(y)); break;
            case TCH_MINIMUM: *out = t->add(x.minimum(y)); break;
            case TCH_POWER: *out = t->add(x.power(y)); break;
            case TCH_MATMUL: *out = t->add(product(x, y)); break;
            case TCH_MATVEC: {
                if (x.rank() != 2 || y.rank() != 1) {
                    throw std::invalid_argument("matvec: shapes " + shape_text(x.shape()) + " and " +
                                                shape_text(y.shape()) + " are not a matrix and a vector");
                }
                MatrixVar<float> m = x.to_matrix(x.shape()[0], x.shape()[1]);
                *out = t->add(m.matvec(y.to_vector()).to_tensor({x.shape()[0]}));
                break;
            }
            case TCH_VECTOR_MUL: {
                // `to_vector`, `VectorVar`'s product, `to_tensor`: one flat
                // variable when both operands are the same tensor, as in
                // tests/tensor_autodiff.rs:251-254.
                if (x.len() != y.len()) {
                    throw std::invalid_argument("elementwise: vector lengths differ, " + std::to_string(x.len()) +
                                                " and " + std::to_string(y.len()));
                }
                VectorVar<float> fa = x.to_vector();
                VectorVar<float> fb = a == b ? fa : y.to_vector();
                *out = t->add((fa * fb).to_tensor(x.shape()));
                break;
            }
            default: throw std::invalid_argument("tape: no binary operation " + std::to_string(op));
        }
    });
}

int tch_tape_matvec_add(tch_tape* t, uint32_t m, uint32_t v, uint32_t addend, uint32_t* out) {
    return guarded([&] {
        const TensorVar<float>& x = t->tensor(m);
        const TensorVar<float>& y = t->tensor(v);
        const TensorVar<float>& z = t->tensor(addend);
        if (x.rank() != 2 || y.rank() != 1 || z.rank() != 1) {
            throw std::invalid_argument("matvec_add: shapes " + shape_text(x.shape()) + ", " + shape_text(y.shape()) +
                                        " and " + shape_text(z.shape()) + " are not a matrix and two vectors");
        }
        MatrixVar<float> matrix = x.to_matrix(x.shape()[0], x.shape()[1]);
        *out = t->add(matrix.matvec_add(y.to_vector(), z.to_vector()).to_tensor({x.shape()[0]}));
    });
}

int tch_tape_unary(tch_tape* t, uint32_t op, uint32_t a, float first, float second, uint32_t* out) {
    return guarded([&] {
        const TensorVar<float>& x = t->tensor(a);
        if (op >= TCH_ANALYTIC && op < TCH_ANALYTIC + 14) {
            *out = t->add(x.analytic(static_cast<Analytic>(op - TCH_ANALYTIC)));
            return;
        }
        switch (op) {
            case TCH_CLAMP_MIN: *out = t->add(x.clamp_min(first)); break;
            case TCH_CLAMP_MAX: *out = t->add(x.clamp_max(first)); break;
            case TCH_CLAMP: *out = t->add(x.clamp(first, second)); break;
            case TCH_RELU: *out = t->add(x.relu()); break;
            case TCH_ABS: *out = t->add(x.abs()); break;
            case TCH_NEG: *out = t->add(x.neg()); break;
            case TCH_SCALE: *out = t->add(x.scale(first)); break;
            case TCH_SHIFT: *out = t->add(x.shift(first)); break;
            case TCH_POWER_SCALAR: *out = t->add(x.power_scalar(first, false)); break;
            case TCH_POWER_SCALAR_LEFT: *out = t->add(x.power_scalar(first, true)); break;
            case TCH_CONTIGUOUS: *out = t->add(x.contiguous()); break;
            default: throw std::invalid_argument("tape: no unary operation " + std::to_string(op));
        }
    });
}

int tch_tape_layout(tch_tape* t, uint32_t op, uint32_t a, uint32_t count, const int64_t* values, uint32_t* out) {
    return guarded([&] {
        const TensorVar<float>& x = t->tensor(a);
        const bool axis_first = op == TCH_NARROW || op == TCH_SELECT || op == TCH_SLICE || op == TCH_SQUEEZE ||
                                op == TCH_UNSQUEEZE;
        const uint32_t fixed[] = {0, 0, 2, 0, 3, 2, 3, 1, 1};
        if (op < sizeof(fixed) / sizeof(fixed[0]) && fixed[op] && count != fixed[op]) {
            throw std::invalid_argument("tape: layout operation " + std::to_string(op) + " takes " +
                                        std::to_string(fixed[op]) + " values, not " + std::to_string(count));
        }
        Shape dims;
        for (uint32_t k = 0; k < count; k++) {
            if (values[k] < 0 && op != TCH_TRANSPOSE && !(axis_first && k == 0)) {
                throw std::invalid_argument("tape: a negative extent or axis " + std::to_string(values[k]));
            }
            dims.push_back(static_cast<size_t>(values[k]));
        }
        switch (op) {
            case TCH_RESHAPE: *out = t->add(x.reshape(dims)); break;
            case TCH_PERMUTE: *out = t->add(x.permute(dims)); break;
            case TCH_BROADCAST_TO: *out = t->add(x.broadcast_to(dims)); break;
            case TCH_TRANSPOSE: *out = t->add(x.transpose(values[0], values[1])); break;
            case TCH_NARROW: *out = t->add(x.narrow(values[0], dims[1], dims[2])); break;
            case TCH_SELECT: *out = t->add(x.select(values[0], dims[1])); break;
            case TCH_SLICE: *out = t->add(x.slice(values[0], dims[1], dims[2])); break;
            case TCH_SQUEEZE: *out = t->add(x.squeeze(values[0])); break;
            case TCH_UNSQUEEZE: *out = t->add(x.unsqueeze(values[0])); break;
            default: throw std::invalid_argument("tape: no layout operation " + std::to_string(op));
        }
    });
}

int tch_tape_reduce(tch_tape* t, uint32_t op, uint32_t a, uint32_t count, const int64_t* axes, int keep_dims,
                    uint32_t* out) {
    return guarded([&] {
        const TensorVar<float>& x = t->tensor(a);
        std::vector<long> named = axes_of(count, axes);
        const bool keep = keep_dims != 0;
        switch (op) {
            case TCH_SUM_AXES: *out = t->add(x.sum_axes(named, keep)); break;
            case TCH_MEAN_AXES: *out = t->add(x.mean_axes(named, keep)); break;
            case TCH_VAR_AXES: *out = t->add(x.var_axes(named, Correction::Population, keep)); break;
            case TCH_VAR_AXES_SAMPLE: *out = t->add(x.var_axes(named, Correction::Sample, keep)); break;
            case TCH_MAX_AXES: *out = t->add(x.max_axes(named, keep)); break;
            case TCH_MIN_AXES: *out = t->add(x.min_axes(named, keep)); break;
            case TCH_SUM: *out = t->add(x.sum()); break;
            case TCH_MEAN: *out = t->add(x.mean()); break;
            default: throw std::invalid_argument("tape: no reduction " + std::to_string(op));
        }
    });
}

int tch_tape_split(tch_tape* t, uint32_t a, int64_t axis, uint32_t count, const uint64_t* sizes, uint32_t* out) {
    return guarded([&] {
        const TensorVar<float>& x = t->tensor(a);
        std::vector<TensorVar<float>> pieces =
            sizes ? x.split(axis, std::vector<size_t>(sizes, sizes + count)) : x.chunk(axis, count);
        for (size_t k = 0; k < pieces.size(); k++) out[k] = t->add(std::move(pieces[k]));
    });
}

int tch_tape_join(tch_tape* t, uint32_t op, uint32_t count, const uint32_t* handles, int64_t axis, uint32_t* out) {
    return guarded([&] {
        std::vector<TensorVar<float>> pieces;
        for (uint32_t k = 0; k < count; k++) pieces.push_back(t->tensor(handles[k]));
        if (op == TCH_CONCAT) {
            *out = t->add(TensorVar<float>::concat(pieces, axis));
        } else if (op == TCH_STACK) {
            *out = t->add(TensorVar<float>::stack(pieces, axis));
        } else {
            throw std::invalid_argument("tape: no join " + std::to_string(op));
        }
    });
}

int tch_tape_add_scalars(tch_tape* t, uint32_t a, uint32_t b, uint32_t* out) {
    return guarded([&] { *out = t->add(t->scalar(a).add(t->scalar(b))); });
}

int tch_tape_backward(tch_tape* t, uint32_t output, const float* seed) {
    return guarded([&] {
        const auto& v = t->at(output);
        if (std::holds_alternative<ScalarVar>(v)) {
            std::get<ScalarVar>(v).backward_with(seed ? *seed : 1.0f);
            return;
        }
        const TensorVar<float>& x = std::get<TensorVar<float>>(v);
        if (seed == nullptr) throw std::invalid_argument("backward: a tensor output needs a seed");
        const size_t n = x.len();
        x.backward_with(Tensor<float>(x.shape(), n ? Storage<float>::store(seed, n) : Storage<float>(0)));
    });
}

int tch_tape_shape(tch_tape* t, uint32_t handle, uint32_t* rank, uint64_t* shape) {
    return guarded([&] {
        const auto& v = t->at(handle);
        if (std::holds_alternative<ScalarVar>(v)) {
            *rank = 0;
            return;
        }
        const Shape& s = std::get<TensorVar<float>>(v).shape();
        *rank = static_cast<uint32_t>(s.size());
        for (size_t k = 0; k < s.size(); k++) shape[k] = s[k];
    });
}

int tch_tape_read(tch_tape* t, uint32_t handle, int gradient, float* out) {
    return guarded([&] {
        const auto& v = t->at(handle);
        if (std::holds_alternative<ScalarVar>(v)) {
            const ScalarVar& s = std::get<ScalarVar>(v);
            *out = gradient ? s.grad() : s.value();
            return;
        }
        const TensorVar<float>& x = std::get<TensorVar<float>>(v);
        const std::vector<float> host = gradient ? x.grad().to_host() : x.value().to_host();
        std::copy(host.begin(), host.end(), out);
    });
}

int tch_tape_zero_grad(tch_tape* t) {
    return guarded([&] { t->tape.zero_grad(); });
}

}  // extern "C"
