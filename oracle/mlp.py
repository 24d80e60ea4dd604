"""CPU restatement of tensorcrate's dense-network training step.

TEST INFRASTRUCTURE ONLY: the checker for the C++ host mirror's tape and
Adam (tensorcrate_amd/host/) and for bench.py's CPU baseline; the product
never imports it.

It follows `mlp_step` (benches/nn_ops.rs:875-921) and the backward rules the
reference's tape runs for it, in the same order and the same element type:

- forward, per layer: `W·H + b ⊗ 1` (`MatrixVar::matmul`, tape/mod.rs:1195;
  `VectorVar::outer`, :979; `binary` Add, :1026), then `relu`
  (`select_scalar`, :1119-1133) between layers;
- loss: `(Y_hat - Y).frobenius_dot(same).scale(1 / (outputs * batch))`
  (:1299-1302, :715-720);
- backward: the scale's factor, the sum's fill (:1286-1297), the product's
  two contributions to the one residual node summed (:316-323), the
  difference's pass-through, the bias through `matvec(adjoint, ones)`
  (:984), the product's `adjoint · Hᵀ` and `Wᵀ · adjoint` (:1199-1214), and
  the rectifier's ½-at-ties share `MaxShare(z, 0)` (:1122-1130, kernels.rs:138-153);
- Adam: the program of optim.rs:1048-1100 with the corrections of :1106-1124,
  as the Host runs it under its default `Algebra::Reassociate`: the product
  chain m' . c1 / d . rate regrouped as (m' . fl(c1 rate)) / d, the plan
  `oracle/fusion.py`'s restatement of the reference's optimizer chooses for
  it (fusion/src/rewrite.rs:324-399, optimize.rs:152-215); `algebra="exact"`
  gives the construction order.

`dtype` float32 gives the step as the f32 kernels compute it up to the
order of each product's and sum's additions; float64 gives the tolerance
reference.
"""

from __future__ import annotations

import numpy as np


def powi(base, exponent: int, dtype=np.float32):
    """`Float::powi`: square and multiply from the low bit, each product rounded."""
    result, a, b = dtype(1.0), dtype(base), abs(exponent)
    while True:
        if b & 1:
            result = dtype(result * a)
        b //= 2
        if b == 0:
            break
        a = dtype(a * a)
    return dtype(dtype(1.0) / result) if exponent < 0 else result


class Adam:
    """`Adam` (optim.rs:1001-1136) over one array."""

    def __init__(self, rate, dtype=np.float32, algebra="reassociate"):
        if algebra not in ("exact", "reassociate"):
            raise ValueError(f"no Algebra {algebra!r}")
        self.algebra = algebra
        self.dtype = dtype
        self.rate = dtype(rate)
        self.b1, self.b2, self.eps = dtype(0.9), dtype(0.999), dtype(1e-8)
        self.steps = 0
        self.m = self.v = None

    def update(self, p: np.ndarray, g: np.ndarray) -> np.ndarray:
        t = self.dtype
        self.steps += 1
        one = t(1.0)
        c1 = t(one / t(one - powi(self.b1, self.steps, t)))
        c2 = t(one / t(one - powi(self.b2, self.steps, t)))
        fresh_first = g * t(one - self.b1)
        fresh_second = (g * g) * t(one - self.b2)
        if self.m is None:
            m, v = fresh_first, fresh_second
        else:
            m = self.m * self.b1 + fresh_first
            v = self.v * self.b2 + fresh_second
        denominator = np.sqrt(v * c2) + self.eps
        self.m, self.v = m, v
        if self.algebra == "reassociate":
            return p - (m * t(c1 * self.rate)) / denominator
        return p - ((m * c1) / denominator) * self.rate


def forward(weights, biases, x, y, dtype):
    """Pre-activations, activations and the loss of one forward pass."""
    t = dtype
    batch = x.shape[1]
    ones = np.ones(batch, t)
    h = [x.astype(t)]
    z = []
    for l, (w, b) in enumerate(zip(weights, biases)):
        pre = (w.astype(t) @ h[-1]) + np.outer(b.astype(t), ones)
        z.append(pre)
        h.append(np.maximum(pre, t(0)) if l + 1 < len(weights) else pre)
    residual = h[-1] - y.astype(t)
    scale = t(1.0) / t(y.shape[0] * batch)
    loss = t(np.sum((residual * residual).astype(np.float64))) * scale
    return z, h, residual, t(loss)


def gradients(weights, biases, x, y, dtype=np.float64):
    """The loss and every W and b gradient, by the tape's rules."""
    t = dtype
    z, h, residual, loss = forward(weights, biases, x, y, t)
    scale = t(1.0) / t(y.shape[0] * x.shape[1])
    adjoint = scale * residual  # the fill of the sum's adjoint times each factor
    d = adjoint + adjoint      # both of the product's contributions to one node
    ones = np.ones(x.shape[1], t)
    gw, gb = [None] * len(weights), [None] * len(weights)
    for l in range(len(weights) - 1, -1, -1):
        gw[l] = d @ h[l].T
        gb[l] = d @ ones
        if l > 0:
            dh = weights[l].astype(t).T @ d
            share = np.where(z[l - 1] > 0, t(1), np.where(z[l - 1] < 0, t(0), t(0.5)))
            d = dh * share
    return loss, gw, gb


def train(weights, biases, x, y, rate, steps, dtype=np.float32, algebra="reassociate"):
    """`steps` training steps; the loss before each, and the final parameters."""
    weights = [w.astype(dtype) for w in weights]
    biases = [b.astype(dtype) for b in biases]
    rules = [(Adam(rate, dtype, algebra), Adam(rate, dtype, algebra)) for _ in weights]
    losses = []
    for _ in range(steps):
        loss, gw, gb = gradients(weights, biases, x, y, dtype)
        losses.append(float(loss))
        for l, (rw, rb) in enumerate(rules):
            weights[l] = rw.update(weights[l], gw[l].astype(dtype))
            biases[l] = rb.update(biases[l], gb[l].astype(dtype))
    return losses, weights, biases


def he_init(widths, seed):
    """Config 5's synthetic network: He-initialised weights N(0, 2/fan_in),
    zero biases, inputs and targets N(0, 1), from numpy's PCG64 at `seed`."""
    rng = np.random.default_rng(seed)
    weights = [(rng.standard_normal((widths[l + 1], widths[l]), dtype=np.float32) *
                np.float32(np.sqrt(2.0 / widths[l]))) for l in range(len(widths) - 1)]
    biases = [np.zeros(widths[l + 1], np.float32) for l in range(len(widths) - 1)]
    return weights, biases


def batch_of(widths, batch, seed):
    rng = np.random.default_rng(seed + 1000)
    x = rng.standard_normal((widths[0], batch), dtype=np.float32)
    y = rng.standard_normal((widths[-1], batch), dtype=np.float32)
    return x, y
