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


def edge_batch() -> SimpleNamespace:
    """Empty structure, single isolated atom, a tiny periodic cell that needs
    several image shells, atoms outside the home cell, and an isolated
    molecule, in one batch."""

    rng = np.random.default_rng(5)
    tiny = np.array([[1.9, 0.0, 0.0], [0.3, 2.1, 0.0], [0.2, -0.4, 2.3]])
    big = np.diag([7.0, 7.5, 8.0])
    parts = [
        (np.array([], np.int32), np.zeros((0, 3)), np.zeros((3, 3)), [0, 0, 0]),
        (np.array([8]), np.array([[0.1, 0.2, 0.3]]), np.zeros((3, 3)), [0, 0, 0]),
        (np.array([1, 8]), rng.uniform(0, 1, (2, 3)) @ tiny, tiny, [1, 1, 1]),
        (np.array([8, 1, 1, 6]), rng.uniform(-0.5, 1.5, (4, 3)) @ big, big, [1, 1, 1]),
        (np.array([6, 1, 1, 1, 8]), rng.normal(size=(5, 3)) * 1.3, np.zeros((3, 3)), [0, 0, 0]),
    ]
    numbers = np.concatenate([p[0] for p in parts]).astype(np.int32)
    positions = np.concatenate([p[1] for p in parts])
    offsets = np.concatenate([[0], np.cumsum([len(p[0]) for p in parts])])
    return SimpleNamespace(numbers=numbers, positions=positions, cells=np.stack([p[2] for p in parts]),
                           pbc=np.array([p[3] for p in parts]), offsets=offsets,
                           ids=tuple(f"edge{i}" for i in range(len(parts))))


def table_samples(table: np.ndarray, row_offsets: np.ndarray, atom_offsets: np.ndarray) -> np.ndarray:
    """``[structure, local_i, local_j, sa, sb, sc]`` of DescriptorPairTable
    rows, the conversion of the reference's pair_samples
    (src/mdescriptor/core/result.py:257-300)."""

    row_offsets = np.asarray(row_offsets, dtype=np.int64)
    atom_offsets = np.asarray(atom_offsets, dtype=np.int64)
    structure = np.repeat(np.arange(len(row_offsets) - 1, dtype=np.int64), np.diff(row_offsets))
    first = atom_offsets[structure]
    records = np.asarray(table[:, :5], dtype=np.int64)
    return np.column_stack((structure, records[:, 0] - first, records[:, 1] - first, records[:, 2:5]))


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
