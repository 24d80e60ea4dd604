/*
 * tchip_host.h — C entry points of the C++ host mirror (libtchip_host.so):
 * tensorcrate's reverse-mode tape and Adam rule (src/tensors/tape/mod.rs,
 * src/optim.rs) running on the Hip backend through include/tchip.h.
 *
 * These are not FFI replacement points: the reference's own code above the
 * `Kernels` trait is generic over the backend and needs no binding.  They
 * drive the C++ restatement of that code from Python, so the tape's backward
 * rules and the training step of tensorcrate's benchmark harness can be
 * checked against the CPU oracle and timed on the GPU.
 *
 * Every function returns a `tc_status`; on failure `tch_last_error()` holds
 * the message for the calling thread.
 */
#ifndef TCHIP_HOST_H
#define TCHIP_HOST_H

#include <stdint.h>

#include "tchip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct tch_mlp tch_mlp;

const char* tch_last_error(void);

/* A dense network of `layers` layers trained as `mlp_step` does
 * (benches/nn_ops.rs:875-921): widths[0] inputs, widths[layers] outputs,
 * layer l mapping widths[l] -> widths[l+1] through W_l (widths[l+1] x
 * widths[l], row-major) and b_l (widths[l+1]), ReLU between layers, squared
 * error against `targets` averaged over outputs x batch, Adam at `rate` for
 * every W_l and b_l.  `inputs` is widths[0] x batch and `targets`
 * widths[layers] x batch, row-major (features x batch).  Host arrays are
 * copied; the network lives on the device until `tch_mlp_destroy`. */
int tch_mlp_create(uint32_t layers, const uint64_t* widths, uint64_t batch, const float* const* weights,
                   const float* const* biases, const float* inputs, const float* targets, float rate,
                   tch_mlp** out);

/* One training step: a fresh tape, forward, backward, then (when `update`
 * is non-zero) one Adam step of every parameter.  Queued asynchronously;
 * nothing is read back. */
int tch_mlp_step(tch_mlp* mlp, int update);

/* The last step's loss, read from the device (waits for it). */
int tch_mlp_loss(tch_mlp* mlp, float* loss);

/* Layer `layer`'s current parameters, and the last step's gradients of
 * them, downloaded into host arrays of widths[l+1] x widths[l] and
 * widths[l+1] floats. */
int tch_mlp_parameters(tch_mlp* mlp, uint32_t layer, float* weights, float* bias);
int tch_mlp_gradients(tch_mlp* mlp, uint32_t layer, float* weights, float* bias);

void tch_mlp_destroy(tch_mlp* mlp);

#ifdef __cplusplus
}
#endif

#endif /* TCHIP_HOST_H */
