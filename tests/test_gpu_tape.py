"""The reverse-mode tape and Adam on the GPU (tensorcrate_amd/host/: the
C++ mirror of tape/mod.rs and optim.rs over libtchip) against the pinned
CPU restatement, oracle/mlp.py.

Tolerances: gradients within 1e-4 of the f64 restatement, normwise (the
largest error over the largest magnitude of each gradient array; the f32
products and sums reorder additions, nothing else differs); losses along a
training run within 1e-4 relative of the f32 restatement, which runs the
same Adam program in f32.
"""

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import mlp
from tensorcrate_amd import lib

pytestmark = pytest.mark.gpu


def network(widths, batch, seed):
    weights, biases = mlp.he_init(widths, seed)
    rng = np.random.default_rng(seed + 11)
    biases = [rng.uniform(-0.1, 0.1, b.shape).astype(np.float32) for b in biases]
    x, y = mlp.batch_of(widths, batch, seed)
    return weights, biases, x, y


def normwise(got, want):
    return float(np.max(np.abs(got.astype(np.float64) - want)) / max(np.max(np.abs(want)), 1e-30))


@pytest.mark.parametrize("widths,batch", [((24, 40, 32, 16), 48), ((7, 13, 5), 9), ((64, 256, 256, 64), 128)])
def test_gradients_match_the_restatement(widths, batch):
    weights, biases, x, y = network(widths, batch, 5)
    net = lib.Mlp(widths, batch, weights, biases, x, y, 1e-3)
    net.step(update=False)
    loss, gw, gb = mlp.gradients([w.astype(np.float64) for w in weights], [b.astype(np.float64) for b in biases],
                                 x, y)
    assert abs(net.loss() - loss) <= 1e-5 * abs(loss)
    for layer in range(len(widths) - 1):
        w, b = net.gradients(layer)
        assert normwise(w, gw[layer]) <= 1e-4, layer
        assert normwise(b, gb[layer]) <= 1e-4, layer
        # Without an update the parameters are untouched.
        pw, pb = net.parameters(layer)
        assert np.array_equal(pw, weights[layer]) and np.array_equal(pb, biases[layer])
    net.close()


def test_ten_adam_steps_follow_the_restatement():
    widths, batch = (32, 64, 64, 16), 40
    weights, biases, x, y = network(widths, batch, 6)
    net = lib.Mlp(widths, batch, weights, biases, x, y, 1e-3)
    losses = []
    for _ in range(10):
        net.step()
        losses.append(net.loss())
    want, w_final, b_final = mlp.train(weights, biases, x, y, 1e-3, 10, np.float32)
    assert np.allclose(losses, want, rtol=1e-4), (losses, want)
    assert losses[-1] < losses[0]
    for layer in range(len(widths) - 1):
        w, b = net.parameters(layer)
        # Ten steps of at most ~rate each: agreement far inside the distance moved.
        assert np.max(np.abs(w - w_final[layer])) <= 1e-4
        assert np.max(np.abs(b - b_final[layer])) <= 1e-4
    net.close()


def test_a_network_without_layers_is_refused():
    with pytest.raises(lib.HipError, match="no layers"):
        lib.Mlp([4], 3, [], [], np.zeros((4, 3)), np.zeros((4, 3)), 1e-3)


def test_gradients_behind_a_dead_rectifier_are_zeros():
    # A first layer whose pre-activations are all negative: the rectifier's
    # share is 0 everywhere (MaxShare, kernels.rs:138-153), so no adjoint
    # reaches that layer and its weight and bias gradients are exact zeros,
    # while the last layer's are not.
    widths, batch = (6, 5, 3), 4
    weights, biases, x, y = network(widths, batch, 9)
    biases[0] = np.full(widths[1], -100.0, np.float32)
    net = lib.Mlp(widths, batch, weights, biases, x, y, 1e-3)
    net.step(update=False)
    w, b = net.gradients(0)
    assert np.all(w == 0) and np.all(b == 0)
    _, last_bias = net.gradients(1)
    assert np.any(last_bias != 0)
    _, _, gb = mlp.gradients([p.astype(np.float64) for p in weights], [p.astype(np.float64) for p in biases], x, y)
    assert normwise(last_bias, gb[1]) <= 1e-4 and np.all(gb[0] == 0)
    net.close()


def test_config5_mlp_step_at_full_size():
    # 1024 -> 4096 -> 4096 -> 1024, batch 4096, He init, seed 4: the first
    # step's loss against the f32 restatement's forward pass, then three
    # training steps that must lower it.
    widths, batch = (1024, 4096, 4096, 1024), 4096
    weights, biases = mlp.he_init(widths, 4)
    x, y = mlp.batch_of(widths, batch, 4)
    net = lib.Mlp(widths, batch, weights, biases, x, y, 1e-3)
    net.step(update=False)
    want = float(mlp.forward(weights, biases, x, y, np.float32)[3])
    assert abs(net.loss() - want) <= 1e-4 * want
    first = None
    for _ in range(3):
        net.step()
        first = net.loss() if first is None else first
    net.step(update=False)
    assert net.loss() < first
    net.close()


def test_config5_loss_curve_at_full_size():
    # Configuration 5's ten training steps (the harness's `mlp_step`,
    # benches/nn_ops.rs:875-921; Adam trajectories as in
    # tests/tensor_autodiff.rs:596) against the f32 restatement's curve,
    # kept as a fixture (tests/golden/make_mlp_curve.py writes it).  The
    # GPU's products and sums add in another order than numpy's, nothing
    # else differs; each loss must agree within 1e-4 relative.
    curve = json.loads((Path(__file__).parent / "golden" / "mlp_config5_curve.json").read_text())
    widths, batch = tuple(curve["widths"]), curve["batch"]
    weights, biases = mlp.he_init(widths, curve["seed"])
    x, y = mlp.batch_of(widths, batch, curve["seed"])
    net = lib.Mlp(widths, batch, weights, biases, x, y, curve["rate"])
    losses = []
    for _ in range(curve["steps"]):
        net.step()
        losses.append(net.loss())
    net.close()
    want = np.array(curve["losses"])
    print("losses", losses, "relative", (np.array(losses) - want) / want, flush=True)
    assert np.allclose(losses, want, rtol=1e-4, atol=0), (losses, list(want))
