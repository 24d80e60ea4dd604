"""Writes ``mlp_config5_curve.json``: configuration 5's ten-step loss curve
by the f32 CPU restatement (oracle/mlp.py).

The network is BASELINE's configs[4]: 1024 -> 4096 -> 4096 -> 1024, ReLU,
batch 4096, He-initialised weights, zero biases, inputs and targets N(0, 1),
seed 4, MSE loss, Adam at rate 1e-3 (the reference harness's `mlp_step`,
benches/nn_ops.rs:875-921), its step as the Host runs it under the default
`Algebra::Reassociate`.  The curve takes minutes of CPU, so it is kept
as a fixture that the GPU test compares against rather than recomputed on
the GPU box.  Run from the repository root:

    python tests/golden/make_mlp_curve.py
"""

import json
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import mlp  # noqa: E402

WIDTHS, BATCH, SEED, RATE, STEPS = (1024, 4096, 4096, 1024), 4096, 4, 1e-3, 10


def main() -> None:
    start = time.time()
    weights, biases = mlp.he_init(WIDTHS, SEED)
    x, y = mlp.batch_of(WIDTHS, BATCH, SEED)
    losses, _, _ = mlp.train(weights, biases, x, y, RATE, STEPS, np.float32)
    out = {"widths": list(WIDTHS), "batch": BATCH, "seed": SEED, "rate": RATE, "steps": STEPS,
           "dtype": "f32", "losses": losses,
           "algebra": "reassociate",
           "source": "oracle/mlp.py train(), f32, numpy " + np.__version__}
    path = Path(__file__).with_name("mlp_config5_curve.json")
    path.write_text(json.dumps(out, indent=1) + "\n")
    print(f"{path}: {losses} ({time.time() - start:.0f} s)")


if __name__ == "__main__":
    main()
