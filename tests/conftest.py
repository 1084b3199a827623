import os
import sys
from pathlib import Path

# Strict mode: no fast path may absorb an error and fall back (talm_amd/state.py), so a test
# can only pass on the HIP kernels themselves.
os.environ.setdefault("TALM_STRICT", "1")

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
