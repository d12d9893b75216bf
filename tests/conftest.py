"""Shared fixtures. ``-m "not gpu"`` runs the oracle-pinning and ABI tests on the CPU;
``-m gpu`` runs the parity tests of the HIP kernels on an MI355X."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parents[1]
GOLDEN = REPO / "tests" / "golden"
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libldx.so")


@pytest.fixture(scope="session")
def pkg():
    """The product package (loads libldx.so; fails loudly if it is missing)."""
    import __graft_entry__

    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device (run them on the MI355X box)")
    return torch.device("cuda:0")


def load_fixture(name: str) -> dict[str, np.ndarray]:
    """A recorded reference fixture (inputs and Torch-CPU outputs), loaded without pickle."""
    with np.load(GOLDEN / "reference" / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def half_spacing(values: np.ndarray) -> np.ndarray:
    """Half the float16 spacing at ``values`` (tests/test_native_kernels.py:47-49)."""
    return np.spacing(np.abs(values).astype(np.float16)).astype(np.float64) / 2


ACCUMULATION_EPS = 8 * 2.0 ** -23   # tests/test_native_kernels.py:37
OPERAND_ROUNDING = 2.0 ** -11       # tests/test_native_kernels.py:38


def assert_fp16_bar(actual: np.ndarray, expected: np.ndarray, *, max_abs: float = 2e-2,
                    rel_l2: float = 1e-3) -> None:
    """The fp16-path parity bar: max abs error <= 2e-2 and relative L2 <= 1e-3 against
    a float64/fp32 reference."""
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    assert actual.shape == expected.shape, (actual.shape, expected.shape)
    assert np.all(np.isfinite(actual)), "non-finite output"
    err = np.abs(actual - expected)
    assert err.max() <= max_abs, f"max abs error {err.max():.3e} > {max_abs}"
    denom = max(np.linalg.norm(expected), 1e-30)
    rel = np.linalg.norm(actual - expected) / denom
    assert rel <= rel_l2, f"relative L2 {rel:.3e} > {rel_l2}"
