"""New frames of a device-resident batch, the large-structure binning path and
slot overflows, against the CPU oracle through the C-ABI.

Everything of the neighbour search that depends on positions (cell grid,
regions of interest, binning path of each structure, home cells, search
lists) is rebuilt on the device at the start of every graph build.  These
tests move the atoms of a resident batch (``mdx_hip_batch_set_positions``,
from host and from device memory), including moves that change a structure's
binning path, and require the rows of the next run to match the oracle on the
new positions, the pair count to equal the oracle graph's, and the rows to
equal a fresh ``mdx_hip_soap_compute`` on the same positions bit for bit.

Structures with more than 2,048 ROI cells are binned by image-level atomics
(``k_bin_atoms``) and sorted per cell; a sparse box and a 64,000-atom liquid
silicon cell take that path, and their graph, SOAP rows and NeighborList
table must equal the oracle's.

A centre with more rows than its slot makes the run build the graph again
(mdx_hip_soap_run, plan compute) or lay it out compactly in place
(mdx_hip_soap_run_noalloc): every averaging mode, a weighted and an mu1nu1
plan are checked on the call that overflows.
"""

from __future__ import annotations

import ctypes
from types import SimpleNamespace

import numpy as np
import pytest

from conftest import SOAP_PAD, edge_batch, scaled_error
from mdescriptor_amd import _hip, workloads
from mdescriptor_amd.descriptors.basis import basis_gto

pytestmark = pytest.mark.gpu

F64_GATE = 1e-10
F32_GATE = 2e-5


def _plan(ctx, params, average, dtype, options=None):
    alphas, betas = basis_gto(params["r_cut"], params["n_max"], params["l_max"])
    plan = _hip.SoapPlan(ctx, species=params["species"], n_max=params["n_max"], l_max=params["l_max"],
                         r_cut=params["r_cut"], sigma=1.0, alphas=alphas, betas=betas, average=average, dtype=dtype,
                         options=options)
    return plan, (alphas, betas)


def _oracle_soap(oracle, batch, params, basis, average, options=None):
    return oracle.soap(batch, species=params["species"], n_max=params["n_max"], l_max=params["l_max"],
                       r_cut=params["r_cut"], sigma=1.0, alphas=basis[0], betas=basis[1], average=average,
                       options=options, num_threads=0)


def _moved(batch, positions):
    return SimpleNamespace(numbers=batch.numbers, positions=np.asarray(positions, np.float64), cells=batch.cells,
                           pbc=batch.pbc, offsets=batch.offsets)


def _gate(dtype):
    return F64_GATE if dtype == "float64" else F32_GATE


def _frames(batch, seed):
    """Three new frames: a small jitter, a larger one, and every structure
    stretched about its first atom by 1.6 (molecules outgrow one cell, boxes
    reach more cells: binning paths change)."""

    rng = np.random.default_rng(seed)
    base = np.asarray(batch.positions, np.float64)
    stretched = base.copy()
    offsets = np.asarray(batch.offsets)
    for s in range(len(offsets) - 1):
        a, b = int(offsets[s]), int(offsets[s + 1])
        if b > a:
            stretched[a:b] = base[a] + 1.6 * (base[a:b] - base[a])
    return [base + rng.normal(0.0, 0.05, base.shape), base + rng.normal(0.0, 0.4, base.shape), stretched]


class _Resident:
    """A device batch and its output buffer."""

    def __init__(self, plan, batch):
        self.plan = plan
        self.batch = _hip.DeviceBatch(plan, batch)
        self.pitch = plan.features * plan.dtype.itemsize
        self.out = _hip.DeviceMemory(max(1, self.batch.rows * self.pitch))

    def run(self, entry="mdx_hip_soap_run"):
        ctx = self.plan.context
        timing = _hip.Timing()
        ctx.check(getattr(ctx.lib, entry)(ctx.handle, self.plan.handle, self.batch.handle,
                                          ctypes.c_void_p(self.out.address), self.pitch, None, ctypes.byref(timing)))
        rows = self.out.to_host(np.empty((self.batch.rows, self.plan.features), self.plan.dtype))
        return rows, timing.as_dict()

    def close(self):
        self.out.free()
        self.batch.close()


def _frame_batches():
    cases = []
    for index in (1, 2, 3):
        work = workloads.config(index, "small")
        cases.append((f"config{index}", work.batch, work.params))
    edge = edge_batch()
    cases.append(("edge", edge, {"species": [1, 6, 8], "n_max": 4, "l_max": 4, "r_cut": 3.5}))
    return cases


FRAME_CASES = _frame_batches()


@pytest.mark.parametrize("case", range(len(FRAME_CASES)), ids=[c[0] for c in FRAME_CASES])
@pytest.mark.parametrize("average,dtype", [("off", "float64"), ("inner", "float64"), ("off", "float32")])
def test_new_frames_match_oracle(hip_context, oracle, case, average, dtype):
    name, batch, params = FRAME_CASES[case]
    plan, basis = _plan(hip_context, params, average, dtype)
    resident = _Resident(plan, batch)
    device_positions = None
    try:
        first, _ = resident.run()
        expected = _oracle_soap(oracle, batch, params, basis, average)
        assert scaled_error(first, expected) <= _gate(dtype)
        for k, positions in enumerate(_frames(batch, 31 + case)):
            print(f"{name} {average} {dtype}: frame {k}", flush=True)
            moved = _moved(batch, positions)
            if k == 1:
                # device-memory positions: copied on the context's stream
                device_positions = _hip.DeviceMemory(positions.nbytes).from_host(positions)
                resident.batch.set_positions(device_positions.address)
            else:
                resident.batch.set_positions(positions)
            rows, timing = resident.run()
            expected = _oracle_soap(oracle, moved, params, basis, average)
            assert rows.shape == expected.shape
            error = scaled_error(rows, expected)
            assert error <= _gate(dtype), f"{name} frame {k}: scaled error {error:.3e}"
            graph = oracle.graph(moved, params["r_cut"] + SOAP_PAD)
            assert timing["pairs"] == len(graph["atoms"])
            fresh, _ = plan.compute(moved)
            np.testing.assert_array_equal(rows, fresh)
            if device_positions is not None:
                device_positions.free()
                device_positions = None
    finally:
        resident.close()
        plan.close()


def test_frames_alternate_between_binning_paths(hip_context, oracle):
    """Molecules that fit one cell, then spread over many (the per-molecule
    wavefront binning and one-cell search give way to the multi-kernel
    binning and workgroup search), then back."""

    work = workloads.config(3, "small")
    params = work.params
    plan, basis = _plan(hip_context, params, "inner", "float64")
    resident = _Resident(plan, work.batch)
    base = np.asarray(work.batch.positions, np.float64)
    try:
        for k, scale in enumerate((1.0, 6.0, 1.0, 3.0)):
            positions = base * scale
            resident.batch.set_positions(positions)
            rows, timing = resident.run()
            moved = _moved(work.batch, positions)
            expected = _oracle_soap(oracle, moved, params, basis, "inner")
            assert scaled_error(rows, expected) <= F64_GATE, f"frame {k} (scale {scale})"
            assert timing["pairs"] == len(oracle.graph(moved, params["r_cut"] + SOAP_PAD)["atoms"])
    finally:
        resident.close()
        plan.close()


def test_non_finite_positions_are_rejected(hip_context):
    work = workloads.config(2, "small")
    plan, _ = _plan(hip_context, work.params, "off", "float64")
    resident = _Resident(plan, work.batch)
    try:
        good, _ = resident.run()
        bad = np.array(work.batch.positions, np.float64)
        bad[17, 1] = np.nan
        with pytest.raises(ValueError, match="positions must be finite"):
            resident.batch.set_positions(bad)
        memory = _hip.DeviceMemory(bad.nbytes).from_host(bad)
        resident.batch.set_positions(memory.address)
        with pytest.raises(ValueError, match="positions must be finite"):
            resident.run()
        memory.free()
        resident.batch.set_positions(np.asarray(work.batch.positions, np.float64))
        again, _ = resident.run()
        np.testing.assert_array_equal(again, good)
    finally:
        resident.close()
        plan.close()


def _roi_cells(batch, cutoff):
    """ROI cells of each structure by the reference's grid (build_grid,
    neighbor.cpp:135-194): to confirm which binning path a test reaches."""

    out = []
    offsets = np.asarray(batch.offsets)
    for s in range(len(offsets) - 1):
        pos = np.asarray(batch.positions[offsets[s]:offsets[s + 1]], np.float64)
        cell = np.asarray(batch.cells[s], np.float64)
        if np.all(np.asarray(batch.pbc[s]) == 1):
            inv = np.linalg.inv(cell)
            b = np.floor(cutoff * np.linalg.norm(inv, axis=0) + 1.0).astype(int)
            shifts = np.array([[i, j, k] for i in range(-b[0], b[0] + 1) for j in range(-b[1], b[1] + 1)
                               for k in range(-b[2], b[2] + 1)], np.float64) @ cell
        else:
            shifts = np.zeros((1, 3))
        lo = pos.min(axis=0) + shifts.min(axis=0) - 1e-10
        hi = pos.max(axis=0) + shifts.max(axis=0) + 1e-10
        dims = np.maximum(1, ((hi - lo) / cutoff).astype(int))
        spacing = np.maximum(cutoff, (hi - lo) / dims)
        c = np.clip(((pos - lo) / spacing).astype(int), 0, dims - 1)
        roi = np.minimum(dims - 1, c.max(axis=0) + 1) - np.maximum(0, c.min(axis=0) - 1) + 1
        out.append(int(np.prod(roi)))
    return out


def _sparse_box():
    rng = np.random.default_rng(2024)
    atoms, length = 2000, 120.0
    return SimpleNamespace(numbers=rng.choice([1, 6, 8], size=atoms).astype(np.int32),
                           positions=rng.uniform(0.0, length, (atoms, 3)), cells=np.eye(3)[None] * length,
                           pbc=np.ones((1, 3), np.int32), offsets=np.array([0, atoms], np.int64))


LARGE_CASES = {
    "sparse-box": (_sparse_box, {"species": [1, 6, 8], "n_max": 4, "l_max": 4, "r_cut": 3.0}),
    "liquid-si-64000": (lambda: workloads.liquid_si(20).batch,
                        {"species": [14], "n_max": 12, "l_max": 9, "r_cut": 5.5}),
}


@pytest.mark.parametrize("name", sorted(LARGE_CASES))
def test_large_structure_binning_matches_oracle(hip_context, oracle, name):
    make, params = LARGE_CASES[name]
    batch = make()
    cutoff = params["r_cut"] + SOAP_PAD
    assert max(_roi_cells(batch, cutoff)) > 2048  # the image-atomics binning path
    print(f"{name}: {batch.offsets[-1]} atoms, ROI cells {_roi_cells(batch, cutoff)}", flush=True)
    ours = _hip.neighbor_graph(hip_context, batch, cutoff)
    theirs = oracle.graph(batch, cutoff)
    for key in theirs:
        np.testing.assert_array_equal(ours[key], theirs[key], err_msg=f"{name}: {key}")
    del ours, theirs
    for dtype in ("float64", "float32"):
        plan, basis = _plan(hip_context, params, "off", dtype)
        try:
            values, _ = plan.compute(batch)
        finally:
            plan.close()
        expected = _oracle_soap(oracle, batch, params, basis, "off")
        error = scaled_error(values, expected)
        assert error <= _gate(dtype), f"{name} {dtype}: scaled error {error:.3e}"
    list_cutoff = params["r_cut"]
    listed = _hip.neighbor_list(hip_context, batch, list_cutoff, full_neighbor_list=True, table=True)
    table, offsets = oracle.neighbor_list(batch, list_cutoff, full_neighbor_list=True, self_pairs=False)
    np.testing.assert_array_equal(listed["offsets"], offsets)
    np.testing.assert_array_equal(listed["table"], table)


def _dense_cluster():
    rng = np.random.default_rng(7)
    atoms = 640
    return SimpleNamespace(numbers=np.where(np.arange(atoms) % 3 == 0, 8, 1).astype(np.int32),
                           positions=rng.uniform(0.0, 3.5, (atoms, 3)), cells=np.zeros((1, 3, 3)),
                           pbc=np.zeros((1, 3), np.int32), offsets=np.array([0, atoms]))


def _two_dense_clusters():
    one = _dense_cluster()
    return SimpleNamespace(numbers=np.concatenate([one.numbers, one.numbers]),
                           positions=np.concatenate([one.positions, one.positions[::-1] + 40.0]),
                           cells=np.zeros((2, 3, 3)), pbc=np.zeros((2, 3), np.int32),
                           offsets=np.array([0, 640, 1280]))


OVERFLOW_PLANS = {
    "default": None,
    "weighted": {"weighting": {"function": "pow", "r0": 2.0, "c": 2.0, "d": 1.0, "m": 3.0, "w0": 0.5}},
    "mu1nu1": {"compression": "mu1nu1"},
}
OVERFLOW_PARAMS = {"species": [1, 8], "n_max": 3, "l_max": 2, "r_cut": 3.0}


@pytest.mark.parametrize("options", sorted(OVERFLOW_PLANS))
@pytest.mark.parametrize("average", ["off", "inner", "outer"])
@pytest.mark.parametrize("entry", ["compute", "mdx_hip_soap_run"])
def test_slot_overflow_on_the_first_call(hip_context, oracle, options, average, entry):
    """Every centre of these clusters has more than 512 rows, so the first
    call on a fresh plan and batch overflows its slots and runs the graph and
    the expansion again; its rows must match the oracle."""

    batch = _two_dense_clusters()
    opts = OVERFLOW_PLANS[options]
    plan, basis = _plan(hip_context, OVERFLOW_PARAMS, average, "float64", opts)
    try:
        if entry == "compute":
            rows, timing = plan.compute(batch)
        else:
            resident = _Resident(plan, batch)
            try:
                rows, timing = resident.run()
            finally:
                resident.close()
        assert timing["pairs"] > 512 * 1280
        expected = _oracle_soap(oracle, batch, OVERFLOW_PARAMS, basis, average, opts)
        error = scaled_error(rows, expected)
        assert error <= F64_GATE, f"{options} {average} {entry}: scaled error {error:.3e}"
    finally:
        plan.close()


def _pipelined(plan, batch, frames, device_frames=()):
    """Rows of each frame through mdx_hip_soap_run_frame (all queued, one
    wait at the end), each frame into its own output buffer; frames whose
    index is in device_frames hand their positions over in device memory."""

    resident = _Resident(plan, batch)
    outs = [_hip.DeviceMemory(max(1, resident.batch.rows * resident.pitch)) for _ in frames]
    staged = []
    try:
        for k, positions in enumerate(frames):
            print(f"pipelined frame {k}", flush=True)
            if k in device_frames:
                staged.append(_hip.DeviceMemory(positions.nbytes).from_host(positions))
                resident.batch.run_frame(staged[-1].address, outs[k].address, resident.pitch)
            else:
                resident.batch.run_frame(positions, outs[k].address, resident.pitch)
        resident.batch.wait()
        shape = (resident.batch.rows, plan.features)
        return [out.to_host(np.empty(shape, plan.dtype)) for out in outs]
    finally:
        for memory in (*outs, *staged):
            memory.free()
        resident.close()


def _sequential(plan, batch, frames):
    resident = _Resident(plan, batch)
    try:
        rows = []
        for positions in frames:
            resident.batch.set_positions(positions)
            rows.append(resident.run()[0])
        return rows
    finally:
        resident.close()


@pytest.mark.parametrize("case", range(len(FRAME_CASES)), ids=[c[0] for c in FRAME_CASES])
@pytest.mark.parametrize("average,dtype", [("off", "float64"), ("inner", "float64"), ("outer", "float64"),
                                           ("off", "float32")])
def test_pipelined_frames_equal_synchronous_runs(hip_context, oracle, case, average, dtype):
    """Frames queued back to back (graph of frame k+1 built beside the
    expansion of frame k, the two buffer sets of the batch alternating) give
    the rows of one synchronous run per frame, bit for bit; the last frame is
    also checked against the oracle."""

    name, batch, params = FRAME_CASES[case]
    plan, basis = _plan(hip_context, params, average, dtype)
    base = np.asarray(batch.positions, np.float64)
    frames = [base, *_frames(batch, 57 + case), base + 0.01]
    try:
        expected = _sequential(plan, batch, frames)
        got = _pipelined(plan, batch, frames, device_frames=(2,))
        for k, (rows, want) in enumerate(zip(got, expected)):
            np.testing.assert_array_equal(rows, want, err_msg=f"{name} {average} {dtype} frame {k}")
        last = _oracle_soap(oracle, _moved(batch, frames[-1]), params, basis, average)
        assert scaled_error(got[-1], last) <= _gate(dtype)
    finally:
        plan.close()


WEIGHTED_FRAMES = {"weighting": {"function": "pow", "r0": 2.5, "c": 1.0, "d": 1.0, "m": 2.0, "w0": 0.5}}


@pytest.mark.parametrize("case", range(len(FRAME_CASES)), ids=[c[0] for c in FRAME_CASES])
@pytest.mark.parametrize("average,dtype", [("off", "float64"), ("inner", "float64"), ("off", "float32")])
def test_pipelined_weighted_frames_equal_synchronous_runs(hip_context, oracle, case, average, dtype):
    """A weighted plan's frames queued back to back (each frame's per-row
    weight pass queued behind its graph, beside the previous frame's
    expansion) give the rows of one synchronous run per frame, bit for bit;
    the last frame is also checked against the oracle."""

    name, batch, params = FRAME_CASES[case]
    plan, basis = _plan(hip_context, params, average, dtype, WEIGHTED_FRAMES)
    base = np.asarray(batch.positions, np.float64)
    frames = [base, *_frames(batch, 91 + case), base - 0.01]
    try:
        expected = _sequential(plan, batch, frames)
        got = _pipelined(plan, batch, frames, device_frames=(1,))
        for k, (rows, want) in enumerate(zip(got, expected)):
            np.testing.assert_array_equal(rows, want, err_msg=f"{name} {average} {dtype} frame {k}")
        last = _oracle_soap(oracle, _moved(batch, frames[-1]), params, basis, average, WEIGHTED_FRAMES)
        assert scaled_error(got[-1], last) <= _gate(dtype)
    finally:
        plan.close()


@pytest.mark.parametrize("options", ["default", "weighted"])
@pytest.mark.parametrize("average", ["off", "outer"])
def test_pipelined_frames_with_slot_overflow(hip_context, oracle, average, options):
    """Both buffer sets start with slots smaller than a centre's rows: the
    first frame on each overflows and is built again inside the call (a
    weighted plan's weights computed again for the larger slots)."""

    batch = _two_dense_clusters()
    chosen = OVERFLOW_PLANS[options]
    plan, basis = _plan(hip_context, OVERFLOW_PARAMS, average, "float64", chosen)
    base = np.asarray(batch.positions, np.float64)
    rng = np.random.default_rng(5)
    frames = [base + rng.normal(0.0, 0.02, base.shape) for _ in range(4)]
    try:
        got = _pipelined(plan, batch, frames)
        for k, positions in enumerate(frames):
            expected = _oracle_soap(oracle, _moved(batch, positions), OVERFLOW_PARAMS, basis, average, chosen)
            error = scaled_error(got[k], expected)
            assert error <= F64_GATE, f"{average} {options} frame {k}: scaled error {error:.3e}"
    finally:
        plan.close()


def test_pipelined_frame_rejects_non_finite_positions(hip_context):
    """A non-finite frame (host or device memory) fails its call; the frames
    before it and after it are unaffected."""

    work = workloads.config(2, "small")
    plan, _ = _plan(hip_context, work.params, "off", "float64")
    base = np.asarray(work.batch.positions, np.float64)
    bad = base.copy()
    bad[17, 1] = np.inf
    resident = _Resident(plan, work.batch)
    outs = [_hip.DeviceMemory(max(1, resident.batch.rows * resident.pitch)) for _ in range(2)]
    memory = _hip.DeviceMemory(bad.nbytes).from_host(bad)
    try:
        resident.batch.run_frame(base, outs[0].address, resident.pitch)
        with pytest.raises(ValueError, match="positions must be finite"):
            resident.batch.run_frame(bad, outs[1].address, resident.pitch)
        with pytest.raises(ValueError, match="positions must be finite"):
            resident.batch.run_frame(memory.address, outs[1].address, resident.pitch)
        resident.batch.run_frame(base, outs[1].address, resident.pitch)
        resident.batch.wait()
        shape = (resident.batch.rows, plan.features)
        first = outs[0].to_host(np.empty(shape, plan.dtype))
        second = outs[1].to_host(np.empty(shape, plan.dtype))
        fresh, _ = plan.compute(work.batch)
        np.testing.assert_array_equal(first, fresh)
        np.testing.assert_array_equal(second, fresh)
    finally:
        memory.free()
        for out in outs:
            out.free()
        resident.close()
        plan.close()


def test_pipelined_frames_share_one_output(hip_context, oracle):
    """Every frame into the same output buffer, the first frames overflowing
    their slots: the frame built and expanded again lands before the next
    frame's expansion, so the buffer ends with the last frame's rows."""

    batch = _two_dense_clusters()
    plan, basis = _plan(hip_context, OVERFLOW_PARAMS, "off", "float64")
    base = np.asarray(batch.positions, np.float64)
    rng = np.random.default_rng(9)
    resident = _Resident(plan, batch)
    try:
        for count in (1, 2, 3):
            frames = [base + rng.normal(0.0, 0.02, base.shape) for _ in range(count)]
            for positions in frames:
                resident.batch.run_frame(positions, resident.out.address, resident.pitch)
            resident.batch.wait()
            rows = resident.out.to_host(np.empty((resident.batch.rows, plan.features), plan.dtype))
            expected = _oracle_soap(oracle, _moved(batch, frames[-1]), OVERFLOW_PARAMS, basis, "off")
            error = scaled_error(rows, expected)
            assert error <= F64_GATE, f"{count} frames: scaled error {error:.3e}"
    finally:
        resident.close()
        plan.close()
