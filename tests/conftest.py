"""Shared fixtures.  Tests marked ``gpu`` need an AMD GPU and the built HIP
library; everything else runs on the CPU (oracle, host logic, the C-ABI's
symbol table)."""

from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

# Radius added to r_cut by the reference's SOAP graph: sigma * sqrt(-2 ln 1e-3)
# (cpp/src/standalone/soap.cpp:1214) at sigma = 1.
SOAP_PAD = float(np.sqrt(-2.0 * np.log(1e-3)))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct GPU and the built libmdx_hip.so")


def load_batch(path: Path) -> SimpleNamespace:
    data = np.load(path)
    return SimpleNamespace(numbers=data["numbers"], positions=data["positions"], cells=data["cells"],
                           pbc=data["pbc"], offsets=data["offsets"])


def load_golden(family: str, manifest: str) -> tuple[dict, SimpleNamespace, dict]:
    folder = GOLDEN / family
    meta = json.loads((folder / manifest).read_text())
    batch = load_batch(folder / meta["input"])
    expected = dict(np.load(folder / meta["expected_output"]))
    return meta, batch, expected


@pytest.fixture(scope="session")
def oracle():
    """The CPU oracle module, built on first use if its library is missing."""

    from oracle import oracle as module

    if not module.ORACLE_LIB.is_file():
        subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "oracle"], check=True)
    return module


@pytest.fixture(scope="session")
def hip_context():
    """One HIP context for the GPU tests; the library must be built."""

    from mdescriptor_amd import _hip

    if not _hip.LIBRARY_PATH.is_file():
        pytest.fail(f"{_hip.LIBRARY_PATH} is not built (python -m mdescriptor_amd.build)")
    ctx = _hip.Context(0)
    yield ctx
    ctx.close()


def scaled_error(values: np.ndarray, reference: np.ndarray) -> float:
    """max |v - r| / (|r| + max|row of r|): a relative error with an atol
    floor of one row maximum, since near-zero high-l features make a purely
    relative comparison ill-posed."""

    values = np.asarray(values, dtype=np.float64)
    reference = np.asarray(reference, dtype=np.float64)
    if reference.size == 0:
        return 0.0
    rowmax = np.max(np.abs(reference), axis=1, keepdims=True)
    return float(np.max(np.abs(values - reference) / (np.abs(reference) + rowmax + 1e-300)))
