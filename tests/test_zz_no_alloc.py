"""mdx_hip_soap_run_noalloc against mdx_hip_soap_run, through the C-ABI.

The no-allocation entry point runs the same kernels with the run's scratch
(neighbour graph, partial sums) in the library's static device array, so its
rows must equal mdx_hip_soap_run's bit for bit.  Each case makes two calls in
a row, the second on a smaller batch, so the second starts from the array the
first left behind; a batch whose scratch exceeds the array is refused with a
message naming the maximum, and a call after the refusal works again.
"""

from __future__ import annotations

import ctypes
import re
from types import SimpleNamespace

import numpy as np
import pytest

from conftest import ROOT
from mdescriptor_amd import _hip, workloads
from mdescriptor_amd.descriptors.basis import basis_gto

pytestmark = pytest.mark.gpu


def _max_scratch() -> int:
    text = (ROOT / "include" / "mdx_hip.h").read_text()
    value, shift = re.search(r"MDX_NOALLOC_SCRATCH_BYTES\s+\((\d+)u\s*<<\s*(\d+)\)", text).groups()
    return int(value) << int(shift)


def _head(batch, structures: int) -> SimpleNamespace:
    """The first `structures` structures of a batch."""

    end = int(batch.offsets[structures])
    return SimpleNamespace(numbers=batch.numbers[:end], positions=batch.positions[:end],
                           cells=batch.cells[:structures], pbc=batch.pbc[:structures],
                           offsets=batch.offsets[:structures + 1])


def _smaller(batch) -> SimpleNamespace:
    """Half the structures of a batch; of a one-structure batch, the same cell
    with the first half of its atoms."""

    structures = len(batch.offsets) - 1
    if structures > 1:
        return _head(batch, structures // 2)
    atoms = int(batch.offsets[1]) // 2
    return SimpleNamespace(numbers=batch.numbers[:atoms], positions=batch.positions[:atoms], cells=batch.cells,
                           pbc=batch.pbc, offsets=np.array([0, atoms], np.int64))


def _plan(ctx, params, average, dtype):
    alphas, betas = basis_gto(params["r_cut"], params["n_max"], params["l_max"])
    return _hip.SoapPlan(ctx, species=params["species"], n_max=params["n_max"], l_max=params["l_max"],
                         r_cut=params["r_cut"], sigma=params.get("sigma", 1.0), alphas=alphas, betas=betas,
                         average=average, dtype=dtype)


def _run(ctx, plan, batch, entry: str):
    """Rows of one device-resident run through `entry`, and its timing."""

    device_batch = _hip.DeviceBatch(plan, batch)
    pitch = plan.features * plan.dtype.itemsize
    memory = _hip.DeviceMemory(max(1, device_batch.rows * pitch))
    timing = _hip.Timing()
    try:
        status = getattr(ctx.lib, entry)(ctx.handle, plan.handle, device_batch.handle,
                                         ctypes.c_void_p(memory.address), pitch, None, ctypes.byref(timing))
        ctx.check(status)
        rows = memory.to_host(np.empty((device_batch.rows, plan.features), plan.dtype))
    finally:
        memory.free()
        device_batch.close()
    return rows, timing


def _free_device_bytes() -> int:
    rt = _hip.DeviceMemory.runtime()
    rt.hipMemGetInfo.argtypes = [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]
    rt.hipMemGetInfo.restype = ctypes.c_int
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert rt.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return int(free.value)


@pytest.fixture(scope="module")
def context():
    ctx = _hip.Context(0)
    yield ctx
    ctx.close()


@pytest.mark.parametrize("config,average,dtype", [
    (1, "off", "float64"),
    (2, "off", "float64"),
    (2, "off", "float32"),
    (3, "inner", "float64"),
    (3, "outer", "float32"),
    (4, "off", "float32"),
    (5, "off", "float64"),
])
def test_noalloc_matches_device_run(context, config, average, dtype):
    work = workloads.config(config, "small")
    plan = _plan(context, work.params, average, dtype)
    try:
        for batch in (work.batch, _smaller(work.batch)):
            print(f"config {config} average {average} {dtype}: {len(batch.numbers)} atoms", flush=True)
            expected, reference = _run(context, plan, batch, "mdx_hip_soap_run")
            rows, timing = _run(context, plan, batch, "mdx_hip_soap_run_noalloc")
            assert rows.shape == expected.shape
            np.testing.assert_array_equal(rows, expected)
            assert timing.pairs == reference.pairs > 0
            assert timing.expansion_tiles == reference.expansion_tiles
            if average == "off" and config != 3:
                assert timing.expansion_tiles <= -1000  # the register-coefficient kernel
    finally:
        plan.close()


def test_noalloc_allocates_no_device_memory(context):
    """After one warm-up call, runs on new batches of other sizes leave the
    device's free memory unchanged (a device-batch run would grow the batch's
    graph buffers)."""

    work = workloads.config(3, "small")
    plan = _plan(context, work.params, "off", "float64")
    try:
        pitch = plan.features * 8
        device_batch = _hip.DeviceBatch(plan, work.batch)
        memory = _hip.DeviceMemory(device_batch.rows * pitch)
        smaller = [_hip.DeviceBatch(plan, _head(work.batch, k)) for k in (50, 120, 20)]  # of 200
        run = context.lib.mdx_hip_soap_run_noalloc
        context.check(run(context.handle, plan.handle, device_batch.handle, ctypes.c_void_p(memory.address), pitch,
                          None, None))
        free = _free_device_bytes()
        for b in smaller + [device_batch]:
            context.check(run(context.handle, plan.handle, b.handle, ctypes.c_void_p(memory.address), pitch, None,
                              None))
        assert _free_device_bytes() == free
        for b in smaller + [device_batch]:
            b.close()
        memory.free()
    finally:
        plan.close()


def test_noalloc_refuses_batches_beyond_the_array(context):
    """A batch whose graph outgrows the static array is refused with
    MDX_INVALID_ARGUMENT and a message naming the maximum; the next call on a
    batch that fits works again and still matches mdx_hip_soap_run."""

    limit = _max_scratch()
    rng = np.random.default_rng(11)
    # one species, one non-periodic structure: the binned images alone take
    # 44 bytes per atom and the centre arrays 28 more
    atoms = limit // 60
    edge = (atoms / 0.05) ** (1.0 / 3.0)
    big = SimpleNamespace(numbers=np.full(atoms, 14, np.int32), positions=rng.uniform(0.0, edge, (atoms, 3)),
                          cells=np.zeros((1, 3, 3)), pbc=np.zeros((1, 3), bool),
                          offsets=np.array([0, atoms], np.int64))
    params = dict(species=[14], n_max=4, l_max=3, r_cut=3.0)
    plan = _plan(context, params, "off", "float64")
    try:
        device_batch = _hip.DeviceBatch(plan, big)
        pitch = plan.features * 8
        memory = _hip.DeviceMemory(device_batch.rows * pitch)
        status = context.lib.mdx_hip_soap_run_noalloc(context.handle, plan.handle, device_batch.handle,
                                                      ctypes.c_void_p(memory.address), pitch, None, None)
        message = context.lib.mdx_hip_last_error(context.handle).decode()
        memory.free()
        device_batch.close()
        assert status == _hip.MDX_INVALID_ARGUMENT
        assert str(limit) in message
        # 2000 of its atoms at the same density
        small = SimpleNamespace(numbers=big.numbers[:2000], positions=big.positions[:2000] * (35.0 / edge),
                                cells=big.cells, pbc=big.pbc, offsets=np.array([0, 2000], np.int64))
        expected, reference = _run(context, plan, small, "mdx_hip_soap_run")
        rows, timing = _run(context, plan, small, "mdx_hip_soap_run_noalloc")
        assert timing.pairs == reference.pairs > 2000
        np.testing.assert_array_equal(rows, expected)
    finally:
        plan.close()


def test_noalloc_slot_overflow_matches_device_run(context):
    """A dense cluster whose every centre has more rows than the static
    graph's first slot width: the no-allocation run lays the overflowing
    batch out compactly in place (counting the true per-species rows again),
    and its rows equal mdx_hip_soap_run's on both calls (the second with the
    wider slot the first left behind) and on a smaller batch after them."""

    rng = np.random.default_rng(7)
    atoms = 640
    dense = SimpleNamespace(numbers=np.where(np.arange(atoms) % 3 == 0, 8, 1).astype(np.int32),
                            positions=rng.uniform(0.0, 3.5, (atoms, 3)), cells=np.zeros((1, 3, 3)),
                            pbc=np.zeros((1, 3), np.int32), offsets=np.array([0, atoms], np.int64))
    params = {"species": [1, 8], "n_max": 3, "l_max": 2, "r_cut": 3.0}
    for average in ("off", "inner"):
        plan = _plan(context, params, average, "float64")
        try:
            for batch in (dense, dense, _smaller(dense)):
                print(f"dense cluster {average}: {len(batch.numbers)} atoms", flush=True)
                expected, reference = _run(context, plan, batch, "mdx_hip_soap_run")
                rows, timing = _run(context, plan, batch, "mdx_hip_soap_run_noalloc")
                assert timing.pairs == reference.pairs
                np.testing.assert_array_equal(rows, expected)
        finally:
            plan.close()


@pytest.mark.parametrize("average", ["off", "inner"])
def test_noalloc_weighted_plan_matches_device_run(context, average):
    """A weighted plan (pow with w0): the per-row weights of the
    register-coefficient kernel sit in the static array beside the graph and
    the partial rows."""

    from test_oracle_vs_reference import option_arguments

    work = workloads.config(2, "small")
    p = work.params
    alphas, betas = basis_gto(p["r_cut"], p["n_max"], p["l_max"])
    options = option_arguments("pow_w0", p["species"], p["r_cut"], p["n_max"])
    plan = _hip.SoapPlan(context, species=p["species"], n_max=p["n_max"], l_max=p["l_max"], r_cut=p["r_cut"],
                         sigma=1.0, alphas=alphas, betas=betas, average=average, dtype="float64", options=options)
    try:
        for batch in (work.batch, _smaller(work.batch)):
            print(f"weighted {average}: {len(batch.numbers)} atoms", flush=True)
            expected, reference = _run(context, plan, batch, "mdx_hip_soap_run")
            rows, timing = _run(context, plan, batch, "mdx_hip_soap_run_noalloc")
            np.testing.assert_array_equal(rows, expected)
            assert timing.expansion_tiles == reference.expansion_tiles <= -1000
    finally:
        plan.close()
