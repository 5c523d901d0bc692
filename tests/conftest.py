"""Shared test setup. `gpu`-marked tests need an MI355X (HIP device) and the
built libtensor_ops_rocm.so; everything else runs on the CPU."""
import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

# torch first: its wheel carries its own HIP and HSA runtimes, and the
# library's libamdhip64.so.7 then resolves to the one already loaded. Loaded
# the other way round, a process holds two HIP runtimes and the library's
# finds no device once torch has claimed it. (Any test may load mod_amd.)
try:
    import torch  # noqa: F401
except ImportError:
    pass


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X) and the built ROCm library")


def assert_rel(got, ref, rtol, what=""):
    """Elementwise relative check with a floor: |got-ref| <= rtol*max(|ref|, 1e-2*rms(ref)).
    The floor keeps outputs that happen to sit near zero (a random dot product
    can) from demanding an accuracy no fp32 summation order has."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    if ref.size == 0:
        return
    rms = float(np.sqrt(np.mean(ref * ref))) or 1.0
    denom = np.maximum(np.abs(ref), 1e-2 * rms)
    err = np.abs(got - ref) / denom
    worst = float(err.max())
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    assert worst <= rtol, f"{what}: max rel err {worst:.3e} > {rtol:.1e} at {np.unravel_index(err.argmax(), err.shape)}"


@pytest.fixture(scope="session")
def torch_dev():
    """cuda:0 on the GPU box; skips the test elsewhere."""
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda:0")
