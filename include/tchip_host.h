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

/* ---- a tape of tensor variables (src/tensors/tape/tensor.rs) ------------
 *
 * Each call records one `TensorVar` operation and answers its handle; the
 * handles number the variables in recording order.  A handle names a tensor,
 * or a scalar for `TCH_SUM` / `TCH_MEAN` and `tch_tape_add_scalars`.  Values
 * are f32, row-major; shapes have at most TC_MAX_RANK axes. */

typedef struct tch_tape tch_tape;

/* Binary operations, broadcasting (tape/tensor.rs:126-250);  TCH_MATMUL is
 * the last axis of `a` times the k x n tensor `b`, through `to_matrix`,
 * `MatrixVar::matmul` and `to_tensor` (tape/tensor.rs:703-761);
 * TCH_VECTOR_MUL the elementwise product of two tensors of one length
 * through `to_vector`, `VectorVar`'s product and `to_tensor` back to `a`'s
 * shape (tape/tensor.rs:733-778); TCH_MATVEC the r x c tensor `a` times
 * the length-c tensor `b` through `MatrixVar::matvec` (tape/mod.rs:1249-1257). */
typedef enum tch_binary {
    TCH_ADD = 0, TCH_SUB = 1, TCH_MUL = 2, TCH_DIV = 3,
    TCH_MAXIMUM = 4, TCH_MINIMUM = 5, TCH_POWER = 6, TCH_MATMUL = 7, TCH_VECTOR_MUL = 8, TCH_MATVEC = 9
} tch_binary;

/* Unary operations (tape/tensor.rs:187-333); `first` and `second` are the
 * scalar, factor, offset or bounds; TCH_ANALYTIC + k is `analytic` of the
 * k-th `Analytic` (kernels.rs:293-308). */
typedef enum tch_unary {
    TCH_CLAMP_MIN = 0, TCH_CLAMP_MAX = 1, TCH_CLAMP = 2, TCH_RELU = 3, TCH_ABS = 4, TCH_NEG = 5,
    TCH_SCALE = 6, TCH_SHIFT = 7, TCH_POWER_SCALAR = 8, TCH_POWER_SCALAR_LEFT = 9, TCH_CONTIGUOUS = 10,
    TCH_ANALYTIC = 32
} tch_unary;

/* Layout operations (tape/tensor.rs:335-462, :555-570): `values` is the new
 * shape, the permutation, the two axes to swap, the shape to broadcast to,
 * (axis, start, len) of a narrow, (axis, index) of a select, (axis, start,
 * end) of a slice, or the one axis to squeeze or unsqueeze.  Axes may be
 * negative, counted from the end. */
typedef enum tch_layout {
    TCH_RESHAPE = 0, TCH_PERMUTE = 1, TCH_TRANSPOSE = 2, TCH_BROADCAST_TO = 3,
    TCH_NARROW = 4, TCH_SELECT = 5, TCH_SLICE = 6, TCH_SQUEEZE = 7, TCH_UNSQUEEZE = 8
} tch_layout;

/* Joins (tape/tensor.rs:502-553): along an existing axis, or a new one. */
typedef enum tch_join { TCH_CONCAT = 0, TCH_STACK = 1 } tch_join;

/* Reductions (tape/tensor.rs:572-701): over `axes` (negative from the end),
 * or, for TCH_SUM and TCH_MEAN, over everything to a scalar. */
typedef enum tch_reduction {
    TCH_SUM_AXES = 0, TCH_MEAN_AXES = 1, TCH_VAR_AXES = 2, TCH_VAR_AXES_SAMPLE = 3,
    TCH_MAX_AXES = 4, TCH_MIN_AXES = 5, TCH_SUM = 6, TCH_MEAN = 7
} tch_reduction;

int tch_tape_create(tch_tape** out);
void tch_tape_destroy(tch_tape* tape);
/* A leaf: `values` holds the product of `shape` floats, copied to the device. */
int tch_tape_tensor(tch_tape* tape, uint32_t rank, const uint64_t* shape, const float* values, uint32_t* out);
int tch_tape_binary(tch_tape* tape, uint32_t op, uint32_t a, uint32_t b, uint32_t* out);
/* `MatrixVar::matvec_add` (tape/mod.rs:1259-1274): the r x c tensor `m`
 * times the length-c tensor `v` plus the length-r tensor `addend`. */
int tch_tape_matvec_add(tch_tape* tape, uint32_t m, uint32_t v, uint32_t addend, uint32_t* out);
int tch_tape_unary(tch_tape* tape, uint32_t op, uint32_t a, float first, float second, uint32_t* out);
int tch_tape_layout(tch_tape* tape, uint32_t op, uint32_t a, uint32_t count, const int64_t* values, uint32_t* out);
int tch_tape_reduce(tch_tape* tape, uint32_t op, uint32_t a, uint32_t count, const int64_t* axes, int keep_dims,
                    uint32_t* out);
/* `split` into pieces of `sizes` along `axis`, or with `sizes` NULL
 * `chunk` into `count` equal pieces (tape/tensor.rs:464-500); `out` receives
 * `count` handles. */
int tch_tape_split(tch_tape* tape, uint32_t a, int64_t axis, uint32_t count, const uint64_t* sizes, uint32_t* out);
/* `concat` or `stack` of `count` tensors along `axis`. */
int tch_tape_join(tch_tape* tape, uint32_t op, uint32_t count, const uint32_t* handles, int64_t axis, uint32_t* out);
/* The sum of two scalars (`ScalarVar::add`). */
int tch_tape_add_scalars(tch_tape* tape, uint32_t a, uint32_t b, uint32_t* out);
/* `backward_with` (tape/mod.rs:507-529) from `output`, seeded with `seed`
 * (one float per element of a tensor output; for a scalar, NULL seeds 1). */
int tch_tape_backward(tch_tape* tape, uint32_t output, const float* seed);
/* A variable's shape (rank 0 for a scalar) into `shape`, which holds
 * TC_MAX_RANK entries. */
int tch_tape_shape(tch_tape* tape, uint32_t handle, uint32_t* rank, uint64_t* shape);
/* A variable's value, or (`gradient` non-zero) its accumulated adjoint, a
 * zero where the last backward pass did not reach it, into `out`, which
 * holds one float per element; waits for the device. */
int tch_tape_read(tch_tape* tape, uint32_t handle, int gradient, float* out);
/* `Tape::zero_grad` (tape/mod.rs:416-420). */
int tch_tape_zero_grad(tch_tape* tape);

#ifdef __cplusplus
}
#endif

#endif /* TCHIP_HOST_H */
