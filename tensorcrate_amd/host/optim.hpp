// The Adam rule over Hip storage: one fused program per step, run by
// `tc_fused` (src/optim.rs:986-1136; `Kernels::fused`, kernels.rs:1077).
//
// `program` encodes the program `Adam::program` builds (optim.rs:1048-1100)
// as the Host runs it, with the uniforms bound to their values: `1 - beta`
// folded into constants computed once in the element type, and the bias
// corrections `1 / (1 - beta^t)` computed on the host in the element type as
// `Adam::update` does (optim.rs:1106-1124), with `powi` as square-and-multiply
// from the low bit, each product rounded (compiler-rt's __powisf2, what
// Rust's f32::powi lowers to).  The first step returns fresh moments; later
// steps update parameters and both moments in place, reading and writing
// each once.
//
// The Host optimizes a built program under the thread's `Algebra`
// (fused/mod.rs:2473-2491): `Exact` keeps the construction order,
// ((m' c1) / d) rate; `Reassociate`, the default, regroups the product chain
// m' . c1 / d . rate, whose inner links nothing else reads, and folds its two
// constants into one in the element type: (m' fl(c1 rate)) / d
// (fusion/src/rewrite.rs:324-399), the plan the optimizer's cost model picks
// (fusion/src/optimize.rs:152-215).
#pragma once

#include <stdint.h>

#include <cmath>
#include <optional>
#include <vector>

#include "backend.hpp"

namespace tensorcrate {
namespace hip {

// `Float::powi` for f32: square and multiply from the low bit.
inline float powi(float base, int exponent) {
    float result = 1.0f;
    float a = base;
    unsigned b = exponent < 0 ? static_cast<unsigned>(-exponent) : static_cast<unsigned>(exponent);
    while (true) {
        if (b & 1u) result *= a;
        b /= 2;
        if (b == 0) break;
        a *= a;
    }
    return exponent < 0 ? 1.0f / result : result;
}

// `Algebra` (fused/mod.rs:2473-2491).
enum class Algebra { Exact, Reassociate };

// `Adam` (optim.rs:1001-1136) for f32 parameters of one shape.
class Adam {
   public:
    // `Adam::new`: beta1 0.9, beta2 0.999, epsilon 1e-8 (optim.rs:1029-1041);
    // the algebra is fixed when the rule is made (optim.rs:727-733).
    explicit Adam(float rate, Algebra algebra = Algebra::Reassociate) : rate_(rate), algebra_(algebra) {}

    size_t steps() const { return steps_; }

    // `Rule::update` (optim.rs:1106-1135) for a parameter tensor of `len`
    // elements and its gradient.
    void update(Storage<float>& parameters, const Storage<float>& gradient) {
        if (parameters.len() != gradient.len()) {
            throw std::invalid_argument("update: vector lengths differ, " + std::to_string(parameters.len()) +
                                        " and " + std::to_string(gradient.len()));
        }
        steps_ += 1;
        const float one = 1.0f;
        const float first_correction = one / (one - powi(first_decay_, static_cast<int>(steps_)));
        const float second_correction = one / (one - powi(second_decay_, static_cast<int>(steps_)));
        const bool resumed = first_.has_value();
        const size_t n = parameters.len();
        if (!resumed) {
            first_.emplace(n);
            second_.emplace(n);
        }
        std::vector<tc_encoded> code = program(resumed, first_correction, second_correction);
        // Every load reads its tensor in its own order: one row of n.
        tc_place place{};
        place.offset = 0;
        place.col_step = 1;
        place.lead = 1;
        place.dims[0] = 1;
        place.steps[0] = n;
        const int loads = resumed ? 4 : 2;
        std::vector<tc_place> places(loads, place);
        std::vector<const void*> inputs = {gradient.ptr(), parameters.ptr()};
        if (resumed) {
            inputs.push_back(first_->ptr());
            inputs.push_back(second_->ptr());
        }
        std::vector<uint64_t> input_lens(inputs.size(), n);
        void* outputs[3] = {parameters.ptr(), first_->ptr(), second_->ptr()};
        uint64_t output_lens[3] = {n, n, n};
        check(tc_fused(TC_F32, code.data(), static_cast<uint32_t>(code.size()), places.data(),
                       static_cast<uint32_t>(places.size()), inputs.data(), input_lens.data(),
                       static_cast<uint32_t>(inputs.size()), outputs, output_lens, 3, 1, n));
    }

   private:
    // The encoded step (optim.rs:1048-1100).  Inputs: 0 the gradient, 1 the
    // parameters, then (resumed) 2 and 3 the moments; outputs: 0 the
    // parameters, 1 and 2 the moments.
    std::vector<tc_encoded> program(bool resumed, float first_correction, float second_correction) const {
        enum : uint16_t { LOAD = 0, CONST = 1, BINARY = 2, UNARY = 3, STORE = 5 };
        constexpr uint16_t kSqrt = 13;  // Analytic::Sqrt (kernels.rs:307)
        auto op = [](uint16_t kind, uint16_t code, uint8_t dst, uint8_t a, uint8_t b, uint8_t aux, float value) {
            return tc_encoded{kind, code, dst, a, b, aux, value};
        };
        const float first_share = 1.0f - first_decay_, second_share = 1.0f - second_decay_;
        std::vector<tc_encoded> code = {
            op(LOAD, 0, 0, 0, TC_F32, 0, 0.0f),           // r0 = g
            op(CONST, 0, 1, 0, 0, 0, first_share),         // r1 = 1 - beta1
            op(BINARY, TC_MUL, 2, 0, 1, 0, 0.0f),          // r2 = g (1 - beta1)
            op(BINARY, TC_MUL, 3, 0, 0, 0, 0.0f),          // r3 = g g
            op(CONST, 0, 4, 0, 0, 0, second_share),        // r4 = 1 - beta2
            op(BINARY, TC_MUL, 5, 3, 4, 0, 0.0f),          // r5 = g g (1 - beta2)
        };
        uint8_t first = 2, second = 5;
        if (resumed) {
            const tc_encoded more[] = {
                op(LOAD, 2, 6, 2, TC_F32, 0, 0.0f),        // r6 = m
                op(CONST, 0, 7, 0, 0, 0, first_decay_),
                op(BINARY, TC_MUL, 6, 6, 7, 0, 0.0f),      // m beta1
                op(BINARY, TC_ADD, 6, 6, 2, 0, 0.0f),      // first moment
                op(LOAD, 3, 8, 3, TC_F32, 0, 0.0f),        // r8 = v
                op(CONST, 0, 9, 0, 0, 0, second_decay_),
                op(BINARY, TC_MUL, 8, 8, 9, 0, 0.0f),      // v beta2
                op(BINARY, TC_ADD, 8, 8, 5, 0, 0.0f),      // second moment
            };
            code.insert(code.end(), std::begin(more), std::end(more));
            first = 6;
            second = 8;
        }
        const bool regrouped = algebra_ == Algebra::Reassociate;
        // Regrouped, c1 and the rate are one constant, folded in f32.
        const float numerator_factor = regrouped ? first_correction * rate_ : first_correction;
        const tc_encoded middle[] = {
            op(CONST, 0, 10, 0, 0, 0, numerator_factor),
            op(BINARY, TC_MUL, 11, first, 10, 0, 0.0f),    // m' c1, or m' fl(c1 rate)
            op(CONST, 0, 12, 0, 0, 0, second_correction),
            op(BINARY, TC_MUL, 13, second, 12, 0, 0.0f),   // corrected second
            op(UNARY, kSqrt, 13, 13, 0, 0, 0.0f),          // root
            op(CONST, 0, 14, 0, 0, 0, epsilon_),
            op(BINARY, TC_ADD, 13, 13, 14, 0, 0.0f),       // denominator
            op(BINARY, TC_DIV, 11, 11, 13, 0, 0.0f),       // step
        };
        code.insert(code.end(), std::begin(middle), std::end(middle));
        if (!regrouped) {
            code.push_back(op(CONST, 0, 15, 0, 0, 0, rate_));
            code.push_back(op(BINARY, TC_MUL, 11, 11, 15, 0, 0.0f));  // step rate
        }
        const tc_encoded tail[] = {
            op(LOAD, 1, 7, 1, TC_F32, 0, 0.0f),            // r7 = p
            op(BINARY, TC_SUB, 7, 7, 11, 0, 0.0f),         // p - step rate
            op(STORE, 0, 0, 7, TC_F32, 0, 0.0f),
            op(STORE, 0, 0, first, TC_F32, 1, 0.0f),
            op(STORE, 0, 0, second, TC_F32, 2, 0.0f),
        };
        code.insert(code.end(), std::begin(tail), std::end(tail));
        return code;
    }

    float rate_;
    Algebra algebra_;
    float first_decay_ = 0.9f, second_decay_ = 0.999f, epsilon_ = 1e-8f;
    size_t steps_ = 0;
    std::optional<Storage<float>> first_, second_;
};

}  // namespace hip
}  // namespace tensorcrate
