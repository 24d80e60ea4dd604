// The dense-network training step of tensorcrate's benchmark harness,
// `mlp_step` (benches/nn_ops.rs:875-921), on the C++ host mirror: a tape
// records W·H + b⊗1 per layer with ReLU between layers, the mean squared
// residual against the targets is differentiated, and every weight and
// bias takes one Adam step.  The reference runs two layers; `widths` here
// gives any depth, and the configuration the bench quotes is
// 1024 -> 4096 -> 4096 -> 1024 over a batch of 4096.
//
// Activations are features x batch, as the reference's are (`matrix(inputs,
// batch)`), so each layer is one (out x in)·(in x batch) product.  The
// operations, their order and their arguments are the reference's: the
// parameters are copied onto a fresh tape each step (`to_backend`), biases
// broadcast through `outer` with a vector of ones, and the loss is
// `residual.frobenius_dot(residual).scale(1 / (outputs · batch))`.
//
// The C entry points (include/tchip_host.h) drive this from Python and
// return a status; the message of a failure is `tch_last_error()` (entry.hpp).

#include "tchip_host.h"

#include <memory>
#include <string>
#include <vector>

#include "backend.hpp"
#include "entry.hpp"
#include "optim.hpp"
#include "tape.hpp"

using namespace tensorcrate::hip;


struct tch_mlp {
    std::vector<size_t> widths;
    size_t batch;
    std::vector<Matrix<float>> weights;
    std::vector<Vector<float>> biases;
    Matrix<float> inputs, targets;
    Vector<float> ones;
    std::vector<Adam> weight_rules, bias_rules;
    // The last step's gradients and its (unread) loss.
    std::vector<Matrix<float>> weight_grads;
    std::vector<Vector<float>> bias_grads;
    std::shared_ptr<Node<float>> loss;

    tch_mlp(std::vector<size_t> w, size_t b, std::vector<Matrix<float>> ws, std::vector<Vector<float>> bs,
            Matrix<float> x, Matrix<float> y, float rate)
        : widths(std::move(w)),
          batch(b),
          weights(std::move(ws)),
          biases(std::move(bs)),
          inputs(std::move(x)),
          targets(std::move(y)),
          ones(Vector<float>::filled(b, 1.0f)) {
        for (size_t l = 0; l + 1 < widths.size(); l++) {
            weight_rules.emplace_back(rate);
            bias_rules.emplace_back(rate);
        }
    }

    // One `mlp_step` (benches/nn_ops.rs:896-920); `update` false stops after
    // the backward pass, leaving the parameters as they were.
    void step(bool update) {
        Tape tape;
        const size_t layers = widths.size() - 1;
        std::vector<MatrixVar<float>> w;
        std::vector<VectorVar<float>> b;
        for (size_t l = 0; l < layers; l++) {
            w.emplace_back(tape.matrix(weights[l].duplicate()));
            b.emplace_back(tape.vector(biases[l].duplicate()));
        }
        VectorVar<float> one = tape.vector(ones.duplicate());
        MatrixVar<float> hidden = tape.matrix(inputs.duplicate());
        for (size_t l = 0; l < layers; l++) {
            MatrixVar<float> z = w[l].matmul(hidden) + b[l].outer(one);
            hidden = l + 1 < layers ? z.relu() : z;
        }
        MatrixVar<float> residual = hidden - MatrixVar<float>(tape.matrix(targets.duplicate()));
        const float scale = 1.0f / static_cast<float>(widths.back() * batch);
        ScalarVar total = residual.frobenius_dot(residual).scale(scale);
        total.backward();
        weight_grads.clear();
        bias_grads.clear();
        for (size_t l = 0; l < layers; l++) {
            weight_grads.push_back(w[l].grad());
            bias_grads.push_back(b[l].grad());
        }
        loss = total.node();
        if (!update) return;
        for (size_t l = 0; l < layers; l++) {
            weight_rules[l].update(weights[l].storage(), weight_grads[l].storage());
            bias_rules[l].update(biases[l].storage(), bias_grads[l].storage());
        }
    }
};

extern "C" {

const char* tch_last_error(void) { return host_error.c_str(); }

int tch_mlp_create(uint32_t layers, const uint64_t* widths, uint64_t batch, const float* const* weights,
                   const float* const* biases, const float* inputs, const float* targets, float rate,
                   tch_mlp** out) {
    return guarded([&] {
        if (layers == 0 || batch == 0) throw std::invalid_argument("mlp: no layers or an empty batch");
        std::vector<size_t> w(widths, widths + layers + 1);
        for (size_t width : w) {
            if (width == 0) throw std::invalid_argument("mlp: a layer of width zero");
        }
        std::vector<Matrix<float>> ws;
        std::vector<Vector<float>> bs;
        for (uint32_t l = 0; l < layers; l++) {
            ws.push_back(Matrix<float>(w[l + 1], w[l], Storage<float>::store(weights[l], w[l + 1] * w[l])));
            bs.push_back(Vector<float>(Storage<float>::store(biases[l], w[l + 1])));
        }
        Matrix<float> x(w[0], batch, Storage<float>::store(inputs, w[0] * batch));
        Matrix<float> y(w.back(), batch, Storage<float>::store(targets, w.back() * batch));
        *out = new tch_mlp(std::move(w), batch, std::move(ws), std::move(bs), std::move(x), std::move(y), rate);
    });
}

int tch_mlp_step(tch_mlp* mlp, int update) {
    return guarded([&] { mlp->step(update != 0); });
}

int tch_mlp_loss(tch_mlp* mlp, float* loss) {
    return guarded([&] {
        if (!mlp->loss) throw std::invalid_argument("mlp: no step has run");
        *loss = mlp->loss->get();
    });
}

int tch_mlp_parameters(tch_mlp* mlp, uint32_t layer, float* weights, float* bias) {
    return guarded([&] {
        if (layer + 1 >= mlp->widths.size()) throw std::invalid_argument("mlp: no layer " + std::to_string(layer));
        check(tc_download(weights, mlp->weights[layer].storage().ptr(), mlp->weights[layer].len() * sizeof(float)));
        check(tc_download(bias, mlp->biases[layer].storage().ptr(), mlp->biases[layer].len() * sizeof(float)));
    });
}

int tch_mlp_gradients(tch_mlp* mlp, uint32_t layer, float* weights, float* bias) {
    return guarded([&] {
        if (layer >= mlp->weight_grads.size()) throw std::invalid_argument("mlp: no gradient of layer " + std::to_string(layer));
        check(tc_download(weights, mlp->weight_grads[layer].storage().ptr(),
                          mlp->weight_grads[layer].len() * sizeof(float)));
        check(tc_download(bias, mlp->bias_grads[layer].storage().ptr(), mlp->bias_grads[layer].len() * sizeof(float)));
    });
}

void tch_mlp_destroy(tch_mlp* mlp) { delete mlp; }

}  // extern "C"
