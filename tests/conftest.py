"""Test configuration: the ``gpu`` marker and the import path.

``-m "not gpu"`` runs everywhere: the oracle against the reference's known
answers, the host-side logic, and that the C ABI library loads and exports
every declared symbol.  ``-m gpu`` runs the parity tests proper on an MI355X,
through the C ABI.
"""

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
