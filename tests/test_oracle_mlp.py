"""The CPU restatement of the training step (oracle/mlp.py) pinned by what
the mathematics fixes, before any GPU result is compared with it: central
finite differences of the loss (tests/tensor_autodiff.rs:327-359 and
tests/reverse.rs:316-347 do the same for the reference's tape), the
rectifier's ½ share at a tie (tape/mod.rs:1122-1130), Adam's first step of
−rate·sign(g) (tests/optim.rs:71-101), and `powi` on exact powers."""

import numpy as np
import pytest

from oracle import mlp


def tiny(seed=0, widths=(3, 5, 4, 2), batch=6):
    weights, biases = mlp.he_init(widths, seed)
    rng = np.random.default_rng(seed + 7)
    biases = [rng.uniform(-0.5, 0.5, b.shape).astype(np.float32) for b in biases]
    x, y = mlp.batch_of(widths, batch, seed)
    return weights, biases, x, y


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_gradients_match_central_differences(seed):
    weights, biases, x, y = tiny(seed)
    w64 = [w.astype(np.float64) for w in weights]
    b64 = [b.astype(np.float64) for b in biases]
    _, gw, gb = mlp.gradients(w64, b64, x, y)
    h = 1e-6

    def loss(ws, bs):
        return float(mlp.forward(ws, bs, x, y, np.float64)[3])

    rng = np.random.default_rng(seed)
    for layer in range(len(w64)):
        for _ in range(4):
            i, j = rng.integers(w64[layer].shape[0]), rng.integers(w64[layer].shape[1])
            up = [w.copy() for w in w64]
            down = [w.copy() for w in w64]
            up[layer][i, j] += h
            down[layer][i, j] -= h
            numeric = (loss(up, b64) - loss(down, b64)) / (2 * h)
            assert abs(numeric - gw[layer][i, j]) <= 1e-6 + 1e-5 * abs(numeric)
        i = rng.integers(b64[layer].shape[0])
        up = [b.copy() for b in b64]
        down = [b.copy() for b in b64]
        up[layer][i] += h
        down[layer][i] -= h
        numeric = (loss(w64, up) - loss(w64, down)) / (2 * h)
        assert abs(numeric - gb[layer][i]) <= 1e-6 + 1e-5 * abs(numeric)


def test_a_rectifier_tie_passes_half_the_adjoint():
    # W1 = 0 and b1 = 0 put every hidden pre-activation exactly at the kink.
    w = [np.zeros((1, 1)), np.array([[0.75]])]
    b = [np.zeros(1), np.array([0.25])]
    x = np.array([[1.0, -2.0, 3.0]])
    y = np.array([[0.5, -1.0, 2.0]])
    _, gw, gb = mlp.gradients(w, b, x, y)
    d2 = 2 * (0.25 - y) / y.size
    assert np.isclose(gb[1][0], d2.sum())
    assert np.isclose(gb[0][0], 0.5 * 0.75 * d2.sum())


def test_adams_first_step_is_the_rate_against_the_gradient():
    g = np.array([3.0, -2.0, 1e-3, -4e-2, 7.0], np.float32)
    p = np.zeros_like(g)
    rule = mlp.Adam(1e-3)
    out = rule.update(p, g)
    assert np.allclose(out, -1e-3 * np.sign(g), rtol=1e-5)


def test_adam_moments_follow_the_recurrence():
    rng = np.random.default_rng(3)
    g1, g2 = rng.standard_normal(8), rng.standard_normal(8)
    rule = mlp.Adam(0.01, np.float64)
    p = rule.update(np.zeros(8), g1)
    p = rule.update(p, g2)
    m = 0.9 * (0.1 * g1) + 0.1 * g2
    v = 0.999 * (0.001 * g1 * g1) + 0.001 * g2 * g2
    step2 = (m / (1 - 0.9 ** 2)) / (np.sqrt(v / (1 - 0.999 ** 2)) + 1e-8)
    first = -0.01 * (g1 * 0.1 / 0.1) / (np.sqrt(g1 * g1 * 0.001 / 0.001) + 1e-8)
    assert np.allclose(p, first - 0.01 * step2, rtol=1e-10, atol=1e-14)


def test_powi_is_exact_on_exact_powers_and_close_otherwise():
    assert mlp.powi(2.0, 10) == np.float32(1024.0)
    assert mlp.powi(0.5, -3) == np.float32(8.0)
    for t in (1, 2, 7, 100, 1000):
        assert abs(float(mlp.powi(0.999, t)) - 0.999 ** t) <= 1e-6 * t


def test_f32_training_follows_f64():
    weights, biases, x, y = tiny(4, (6, 10, 8, 3), 12)
    l32, _, _ = mlp.train(weights, biases, x, y, 1e-2, 5, np.float32)
    l64, _, _ = mlp.train(weights, biases, x, y, 1e-2, 5, np.float64)
    assert np.allclose(l32, l64, rtol=1e-4)
    assert l64[-1] < l64[0]
