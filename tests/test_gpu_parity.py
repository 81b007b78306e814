"""Parity of the HIP library with the CPU oracle, through the C-ABI.

Gates: the neighbour graph is identical to the oracle's in every field and
order (d^2 bit-identical); float64 features satisfy
|delta| <= 1e-10 (|ref| + max|row|) and float32 features the same form at
2e-5 (the oracle's float64 result is the reference); samples, labels and
row offsets are identical.  The reference goldens are also checked end to end
through the public ``SOAP`` class.  Full-size configurations are checked
through properties that do not need a CPU run of the whole batch: one
structure against the oracle, translation invariance and periodic-supercell
replication.
"""

from __future__ import annotations

import ctypes
from types import SimpleNamespace

import numpy as np
import pytest

import mdescriptor_amd as mdx
from conftest import SOAP_PAD, edge_batch, load_golden, scaled_error
from mdescriptor_amd import _hip, workloads
from mdescriptor_amd.descriptors.basis import basis_gto

pytestmark = pytest.mark.gpu

F64_GATE = 1e-10
F32_GATE = 2e-5


def _plan(ctx, params, average=None, dtype=None):
    p = dict(params)
    alphas, betas = basis_gto(p["r_cut"], p["n_max"], p["l_max"])
    return _hip.SoapPlan(ctx, species=p["species"], n_max=p["n_max"], l_max=p["l_max"], r_cut=p["r_cut"],
                         sigma=p.get("sigma", 1.0), alphas=alphas, betas=betas,
                         average=average or p["average"], dtype=dtype or p["dtype"]), (alphas, betas)


def _oracle_soap(oracle, batch, params, basis, average):
    return oracle.soap(batch, species=params["species"], n_max=params["n_max"], l_max=params["l_max"],
                       r_cut=params["r_cut"], sigma=params.get("sigma", 1.0), alphas=basis[0], betas=basis[1],
                       average=average, num_threads=0)


def _check(ctx, oracle, batch, params, average, dtype):
    plan, basis = _plan(ctx, params, average, dtype)
    try:
        values, timing = plan.compute(batch)
    finally:
        plan.close()
    expected = _oracle_soap(oracle, batch, params, basis, average)
    assert values.dtype == np.dtype(dtype)
    assert values.shape == expected.shape
    assert np.all(np.isfinite(values))
    error = scaled_error(values, expected)
    assert error <= (F64_GATE if dtype == "float64" else F32_GATE), f"scaled error {error:.3e}"
    return values, timing


@pytest.fixture(scope="module", params=[1, 2, 3, 4, 5])
def workload(request):
    return workloads.config(request.param, "small")


def test_graph_identical_to_oracle(hip_context, oracle, workload):
    cutoff = workload.params["r_cut"] + SOAP_PAD
    ours = _hip.neighbor_graph(hip_context, workload.batch, cutoff)
    theirs = oracle.graph(workload.batch, cutoff)
    for key in theirs:
        np.testing.assert_array_equal(ours[key], theirs[key], err_msg=key)


@pytest.mark.parametrize("average", ["off", "inner", "outer"])
@pytest.mark.parametrize("dtype", ["float64", "float32"])
def test_soap_matches_oracle(hip_context, oracle, workload, average, dtype):
    _check(hip_context, oracle, workload.batch, workload.params, average, dtype)


@pytest.mark.parametrize("kernel", ["generic", "mfma", "quad", "block"])
def test_every_expansion_kernel_matches(hip_context, oracle, monkeypatch, kernel):
    """The plan picks the register-coefficient kernel for the default options
    with atom-level rows, inner averages, or outer averages of large
    structures where its shape is compiled, else
    the 4x4-block kernel
    where it fits (n_max <= 8), else the 16x16-tile kernel, with the generic
    kernel as the last fallback.  Each stays parity-green when forced."""

    monkeypatch.setenv("MDX_HIP_SOAP_KERNEL", kernel)
    work = workloads.config(2, "small")
    for average in ("off", "inner", "outer"):
        _, timing = _check(hip_context, oracle, work.batch, work.params, average, "float64")
        tiles = timing["expansion_tiles"]
        expected = {"block": tiles <= -1000, "quad": -1000 < tiles < 0, "mfma": tiles > 0, "generic": tiles == 0}
        assert expected[kernel], tiles


def test_default_plan_runs_the_block_kernel(hip_context, oracle):
    work = workloads.config(2, "small")
    for average, tiles in (("off", -1004), ("inner", -1004), ("outer", -1004)):
        _, timing = _check(hip_context, oracle, work.batch, work.params, average, "float32")
        # four wavefronts for n_max 8, l_max 6; inner averages of two 512-atom
        # structures (too few for a workgroup each) as runs of centres into
        # partial rows and a launch per structure; outer averages as float64
        # rows per centre, reduced per structure
        assert timing["expansion_tiles"] == tiles
    molecules = workloads.config(3, "small")
    _, timing = _check(hip_context, oracle, molecules.batch, molecules.params, "inner", "float64")
    # inner averages of molecules (at most 64 atoms): a workgroup per structure
    assert timing["expansion_tiles"] <= -1000
    # their outer averages too: each centre's power spectrum summed into the
    # structure's row in LDS
    _, timing = _check(hip_context, oracle, molecules.batch, molecules.params, "outer", "float64")
    assert timing["expansion_tiles"] <= -1000


def _random_cluster(seed, atoms, species):
    """A dense periodic box and an isolated cluster, both with every species."""

    rng = np.random.default_rng(seed)
    numbers = np.array([species[i % len(species)] for i in range(2 * atoms)], np.int32)
    box = 6.0
    positions = np.concatenate([rng.uniform(0.0, box, (atoms, 3)), rng.uniform(0.0, 4.0, (atoms, 3))])
    cells = np.stack([np.eye(3) * box, np.zeros((3, 3))])
    pbc = np.array([[1, 1, 1], [0, 0, 0]], np.int32)
    return SimpleNamespace(numbers=numbers, positions=positions, cells=cells, pbc=pbc,
                           offsets=np.array([0, atoms, 2 * atoms]))


def test_slot_overflow_falls_back_to_the_compact_layout(hip_context, oracle):
    """The SOAP graph keeps 512 rows per centre in one search pass; a centre
    with more neighbours makes that call lay the rows out compactly and the
    next call use larger slots.  Both calls, and a normal batch after them,
    must match the oracle."""

    rng = np.random.default_rng(7)
    atoms = 640
    dense = SimpleNamespace(numbers=np.where(np.arange(atoms) % 3 == 0, 8, 1).astype(np.int32),
                            positions=rng.uniform(0.0, 3.5, (atoms, 3)), cells=np.zeros((1, 3, 3)),
                            pbc=np.zeros((1, 3), np.int32), offsets=np.array([0, atoms]))
    params = {"species": [1, 8], "n_max": 3, "l_max": 2, "r_cut": 3.0}
    plan, basis = _plan(hip_context, params, "off", "float64")
    try:
        expected = _oracle_soap(oracle, dense, params, basis, "off")
        for _ in range(2):
            values, timing = plan.compute(dense)
            assert timing["pairs"] > 512 * atoms // 2
            assert scaled_error(values, expected) <= F64_GATE
        work = workloads.config(1, "small")
        values, _ = plan.compute(work.batch)
        assert scaled_error(values, _oracle_soap(oracle, work.batch, params, basis, "off")) <= F64_GATE
    finally:
        plan.close()


def _small_periodic_batch(seed, species, boxes=3, atoms=150, box=8.0):
    """Periodic boxes of 27 images each (cutoff below the box length), a
    five-atom molecule whose region is one cell, and an empty structure: a
    batch whose structures each fit one binning workgroup."""

    rng = np.random.default_rng(seed)
    parts, cells, pbc, offsets = [], [], [], [0]
    for _ in range(boxes):
        parts.append(rng.uniform(0.0, box, (atoms, 3)))
        cells.append(np.eye(3) * box)
        pbc.append([1, 1, 1])
        offsets.append(offsets[-1] + atoms)
    parts.append(rng.uniform(0.0, 1.5, (5, 3)))
    cells.append(np.zeros((3, 3)))
    pbc.append([0, 0, 0])
    offsets.append(offsets[-1] + 5)
    cells.append(np.zeros((3, 3)))
    pbc.append([0, 0, 0])
    offsets.append(offsets[-1])
    n = offsets[-1]
    numbers = np.array([species[i % len(species)] for i in range(n)], np.int32)
    return SimpleNamespace(numbers=numbers, positions=np.concatenate(parts), cells=np.stack(cells),
                           pbc=np.array(pbc, np.int32), offsets=np.array(offsets))


@pytest.mark.parametrize("species", [[14], [1, 8], [1, 6, 8]])
def test_one_workgroup_per_structure_binning(hip_context, oracle, species):
    """Batches whose structures each have at most 2,048 region cells and
    8,192 images (1,024 or more on average) are binned one structure per
    workgroup, and structures of at most 64 images one per wavefront, each
    structure's bins from its first extended index.  The graph, the SOAP
    rows and the NeighborList must match the oracle as on the multi-kernel
    path, with one species and several, a one-cell molecule (binned and
    searched by wavefronts) and an empty structure in the batch."""

    batch = _small_periodic_batch(11 + len(species), species)
    params = {"species": species, "n_max": 4, "l_max": 3, "r_cut": 3.0}
    cutoff = params["r_cut"] + SOAP_PAD
    ours = _hip.neighbor_graph(hip_context, batch, cutoff)
    theirs = oracle.graph(batch, cutoff)
    for key in theirs:
        np.testing.assert_array_equal(ours[key], theirs[key], err_msg=key)
    for average in ("off", "inner"):
        _check(hip_context, oracle, batch, params, average, "float64")
    for full in (True, False):
        listed = _hip.neighbor_list(hip_context, batch, params["r_cut"], full_neighbor_list=full, table=True)
        table, offsets = oracle.neighbor_list(batch, params["r_cut"], full_neighbor_list=full, self_pairs=False)
        np.testing.assert_array_equal(listed["offsets"], offsets)
        np.testing.assert_array_equal(listed["table"], table)


@pytest.mark.parametrize("n_max,l_max", [(1, 0), (2, 1), (3, 2), (4, 3), (4, 7), (5, 4), (6, 5), (7, 9),
                                         (8, 6), (8, 8), (8, 10)])
def test_quad_kernel_shapes(hip_context, oracle, monkeypatch, n_max, l_max):
    """Every radial-group count (n_max <= 4: one group, 5-8: two) and a range
    of degrees, so that plans with 1-7 wavefronts, split degrees and idle
    blocks all run against the oracle."""

    monkeypatch.setenv("MDX_HIP_SOAP_KERNEL", "quad")
    species = [1, 8]
    batch = _random_cluster(100 * n_max + l_max, 24, species)
    params = {"species": species, "n_max": n_max, "l_max": l_max, "r_cut": 3.0}
    # the inner average keeps a second coefficient block in LDS: past 64 KiB
    # at l_max 10, within the 160 KiB a gfx950 workgroup may use
    for average in ("off", "outer", "inner"):
        _, timing = _check(hip_context, oracle, batch, params, average, "float64")
        assert timing["expansion_tiles"] < 0


@pytest.mark.parametrize("species,n_max,l_max,r_cut", [
    ([1, 8], 4, 3, 3.0), ([1, 8], 3, 3, 3.0),       # one radial group, four step phases per exp register
    ([1, 6, 7, 8], 8, 6, 3.0), ([1, 6, 8], 7, 6, 3.0),  # two radial groups, two coefficient registers
    ([1, 6, 7, 8, 9], 6, 4, 3.0), ([24, 26, 27, 28, 29], 8, 8, 3.0),  # five species: three registers
    ([14], 12, 9, 6.0), ([14], 9, 9, 3.0),          # three radial groups: rotated beta fold
])
def test_block_kernel_shapes(hip_context, oracle, monkeypatch, species, n_max, l_max, r_cut):
    """Every compiled shape of the register-coefficient kernel (one, two and
    three radial groups; one to three coefficient registers; pad channels)
    against the oracle, float64 and float32 rows.  Twelve GTO channels get a
    6 A cutoff: packed into 3 A their overlap matrix is so ill-conditioned
    (max |beta| 1.6e7) that any two summation orders, the oracle's and every
    GPU kernel's alike, differ by 1e-9."""

    monkeypatch.setenv("MDX_HIP_SOAP_KERNEL", "block")
    batch = _random_cluster(10 * n_max + l_max, 30, species)
    params = {"species": species, "n_max": n_max, "l_max": l_max, "r_cut": r_cut}
    for dtype, average in (("float64", "off"), ("float32", "off"), ("float64", "inner"), ("float32", "inner")):
        _, timing = _check(hip_context, oracle, batch, params, average, dtype)
        assert timing["expansion_tiles"] == -1004


@pytest.mark.parametrize("kernel", ["block", "quad", "mfma"])
def test_far_translated_structures(hip_context, oracle, monkeypatch, kernel):
    """Molecules placed 1e4-3e4 A from the origin and from each other: a pad
    slot of a chunk may hold the position of another structure's atom, which
    must not reach an exp (a far-out argument overflows the table exp's
    exponent); every matrix-core kernel against the oracle."""

    monkeypatch.setenv("MDX_HIP_SOAP_KERNEL", kernel)
    work = workloads.config(3, "small")
    part = work.batch._slice_view(0, 12)
    shifts = np.repeat(np.array([[1e4 * (s + 1), -2e4 * (s % 2), 3e4 * (s % 3)] for s in range(part.structures)]),
                       np.diff(part.offsets), axis=0)
    batch = mdx.StructureBatch(part.numbers, part.positions + shifts, part.cells, part.pbc, part.offsets,
                               list(part.ids))
    for average in ("off", "inner", "outer"):
        _check(hip_context, oracle, batch, work.params, average, "float64")


def test_block_kernel_inner_average_with_empty_structures(hip_context, oracle, monkeypatch):
    """Inner averages on the register-coefficient kernel: a workgroup streams
    the centres of several whole structures and writes one row per structure;
    structures without atoms (first, inside, last) get zero rows."""

    monkeypatch.setenv("MDX_HIP_SOAP_KERNEL", "block")
    work = workloads.config(3, "small")
    b = work.batch
    keep = [b._slice_view(0, 40), b._slice_view(40, b.structures)]
    numbers = np.concatenate([keep[0].numbers, keep[1].numbers])
    positions = np.concatenate([keep[0].positions, keep[1].positions])
    sizes = [0] + list(np.diff(keep[0].offsets)) + [0, 0] + list(np.diff(keep[1].offsets)) + [0]
    offsets = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    structures = len(sizes)
    batch = mdx.StructureBatch(numbers, positions, np.zeros((structures, 3, 3)), np.zeros((structures, 3)),
                               offsets, [str(i) for i in range(structures)])
    for dtype in ("float64", "float32"):
        values, timing = _check(hip_context, oracle, batch, work.params, "inner", dtype)
        assert timing["expansion_tiles"] == -1004
        assert values.shape[0] == structures
        for row in np.flatnonzero(np.diff(offsets) == 0):
            assert np.all(values[row] == 0.0)


@pytest.mark.parametrize("cutoff", [3.5, 3.5 + SOAP_PAD])
def test_golden_graphs(hip_context, oracle, cutoff):
    _, batch, _ = load_golden("reference_soap", "manifest.json")
    ours = _hip.neighbor_graph(hip_context, batch, cutoff)
    theirs = oracle.graph(batch, cutoff)
    for key in theirs:
        np.testing.assert_array_equal(ours[key], theirs[key], err_msg=key)


@pytest.mark.parametrize("manifest", ["manifest.json", "external_manifest.json"])
def test_neighbor_list_goldens(hip_context, manifest):
    """The device graph reproduces the reference NeighborList pairs, in order."""

    meta, batch, expected = load_golden("reference_neighborlist", manifest)
    g = _hip.neighbor_graph(hip_context, batch, meta["configuration"]["parameters"]["cutoff"])
    offsets = np.asarray(batch.offsets)
    centre = np.repeat(np.arange(len(g["offsets"]) - 1), np.diff(g["offsets"]))
    keep = ~((g["atoms"] == centre) & np.all(g["shifts"] == 0, axis=1))
    structure = np.searchsorted(offsets, centre, side="right") - 1
    samples = np.column_stack((structure, centre - offsets[structure], g["atoms"] - offsets[structure],
                               g["shifts"]))[keep]
    np.testing.assert_array_equal(samples, expected["samples"])
    values = np.column_stack((g["displacements"], np.sqrt(g["distance2"])))[keep]
    np.testing.assert_allclose(values, expected["values"], rtol=1e-9, atol=1e-11)


def test_graph_boundary_inclusive_and_exclusive(hip_context):
    batch = SimpleNamespace(numbers=np.array([1, 8], np.int32), positions=np.array([[0.0, 0, 0], [1.0, 0, 0]]),
                            cells=np.zeros((1, 3, 3)), pbc=np.zeros((1, 3), np.int32), offsets=np.array([0, 2]))
    inclusive = _hip.neighbor_graph(hip_context, batch, 1.0, include_boundary=True)
    assert inclusive["offsets"].tolist() == [0, 2, 4] and 1.0 in inclusive["distance2"].tolist()
    exclusive = _hip.neighbor_graph(hip_context, batch, 1.0, include_boundary=False)
    assert exclusive["offsets"].tolist() == [0, 1, 2]


@pytest.mark.parametrize("manifest", ["manifest.json", "external_manifest.json"])
@pytest.mark.parametrize("dtype", ["float64", "float32"])
def test_public_soap_reproduces_goldens(manifest, dtype):
    meta, raw, expected = load_golden("reference_soap", manifest)
    p = meta["configuration"]["parameters"]
    ids = meta["result"]["structure_ids"]
    batch = mdx.StructureBatch(raw.numbers, raw.positions, raw.cells, raw.pbc, raw.offsets, ids)
    with mdx.SOAP(species=p["species"], r_cut=p["r_cut"], n_max=p["n_max"], l_max=p["l_max"],
                  sigma=p.get("sigma", 1.0), average=p["average"],
                  output=mdx.OutputOptions(dtype=dtype)) as soap:
        result = soap.compute(batch)
    tol = meta["tolerance"]
    if dtype == "float64":
        np.testing.assert_allclose(result.values, expected["values"], rtol=tol["rtol"], atol=tol["atol"])
    else:
        assert result.values.dtype == np.float32
        assert scaled_error(result.values, expected["values"]) <= F32_GATE
    assert list(result.labels) == meta["result"]["labels"]
    assert result.level.value == meta["result"]["level"]
    assert list(result.structure_ids) == ids
    expected_offsets = meta["result"]["row_offsets"]
    assert (result.row_offsets is None and expected_offsets is None) or \
        result.row_offsets.tolist() == expected_offsets
    if "samples" in expected:
        np.testing.assert_array_equal(result.samples, expected["samples"])
    assert result.metadata["backend"] == "mdescriptor-hip"
    assert result.metadata["execution"]["device"] == "hip"
    assert not result.values.flags.writeable


def _edge_batch():
    raw = edge_batch()
    return mdx.StructureBatch(raw.numbers, raw.positions, raw.cells, raw.pbc, raw.offsets, list(raw.ids))


@pytest.mark.parametrize("average", ["off", "inner", "outer"])
def test_edge_cases(hip_context, oracle, average):
    params = dict(species=[1, 6, 8], r_cut=4.0, n_max=4, l_max=4, dtype="float64")
    values, _ = _check(hip_context, oracle, _edge_batch(), params, average, "float64")
    if average != "off":
        assert np.all(values[0] == 0.0)


def test_empty_batch(hip_context):
    batch = mdx.StructureBatch(np.zeros(0, np.int32), np.zeros((0, 3)), np.zeros((0, 3, 3)), np.zeros((0, 3)), [0],
                               [])
    for average in ("off", "inner"):
        plan, _ = _plan(hip_context, dict(species=[1, 8], r_cut=4.0, n_max=2, l_max=2, dtype="float64"), average)
        values, _ = plan.compute(batch)
        plan.close()
        assert values.shape == (0, plan.features)


def test_invalid_batch_is_rejected_on_the_host(hip_context):
    batch = SimpleNamespace(numbers=np.array([1, 8], np.int32), positions=np.zeros((2, 3)),
                            cells=np.zeros((1, 3, 3)), pbc=np.ones((1, 3), np.int32), offsets=np.array([0, 2]))
    plan, _ = _plan(hip_context, dict(species=[1, 8], r_cut=4.0, n_max=2, l_max=2, dtype="float64"), "off")
    with pytest.raises(ValueError):
        plan.compute(batch)
    undeclared = SimpleNamespace(numbers=np.array([1, 9], np.int32), positions=np.eye(2, 3),
                                 cells=np.zeros((1, 3, 3)), pbc=np.zeros((1, 3), np.int32), offsets=np.array([0, 2]))
    with pytest.raises(ValueError):
        plan.compute(undeclared)
    plan.close()


def test_cancellation_flag(hip_context):
    work = workloads.config(1, "small")
    plan, _ = _plan(hip_context, work.params, "off")
    flag = ctypes.c_int32(1)
    with pytest.raises(_hip.HipCancelledError):
        plan.compute(work.batch, flag)
    flag.value = 0
    values, _ = plan.compute(work.batch, flag)
    plan.close()
    assert np.all(np.isfinite(values))
    control = mdx.ComputeControl()
    control.cancel()
    with pytest.raises(mdx.CancelledError):
        mdx.SOAP(species=[1, 8], r_cut=4.5, n_max=4, l_max=3, average="off").compute(work.batch, control=control)


def test_public_api_matches_c_abi_and_block_splitting(hip_context):
    work = workloads.config(3, "small")
    p = work.params
    plan, _ = _plan(hip_context, p)
    direct, _ = plan.compute(work.batch)
    plan.close()
    soap = mdx.SOAP(species=p["species"], r_cut=p["r_cut"], n_max=p["n_max"], l_max=p["l_max"],
                    average=p["average"], output=mdx.OutputOptions(dtype=p["dtype"]))
    control = mdx.ComputeControl()
    result = soap.compute(work.batch, control=control)
    np.testing.assert_array_equal(result.values, direct)
    assert control.completed() == control.total() == work.batch.structures
    soap._backend.atom_budget = 700
    split = soap.compute(work.batch)
    np.testing.assert_array_equal(split.values, direct)
    soap.close()


def test_device_resident_run_matches_compute(hip_context):
    work = workloads.config(2, "small")
    plan, _ = _plan(hip_context, work.params)
    host, _ = plan.compute(work.batch)
    device_batch = _hip.DeviceBatch(plan, work.batch)
    pitch = plan.features * host.itemsize
    memory = _hip.DeviceMemory(device_batch.rows * pitch)
    device_batch.run(memory.address, pitch)
    resident = memory.to_host(np.empty_like(host))
    np.testing.assert_array_equal(resident, host)
    memory.free()
    device_batch.close()
    plan.close()


def test_download_paths_agree(hip_context):
    """Pinned destinations take one DMA; pageable ones go through the pinned
    staging ring (several 64 MB chunks here) and host threads; a pitched
    pageable destination is written row by row and its padding left alone."""

    work = workloads.config(4, "small")
    plan, _ = _plan(hip_context, dict(work.params, dtype="float64"), "off")
    pinned, _ = plan.compute(work.batch)
    assert _hip.is_pinned(pinned)
    pageable = np.empty_like(np.asarray(pinned))
    plan.compute(work.batch, out=pageable)
    np.testing.assert_array_equal(pageable, pinned)
    rows, features = pinned.shape
    pitched = np.full((rows, features + 5), -7.0)
    arrays = _hip._BatchArrays(work.batch)
    hip_context.check(hip_context.lib.mdx_hip_soap_compute(
        hip_context.handle, plan.handle, ctypes.byref(arrays.view), pitched.ctypes.data_as(ctypes.c_void_p), rows,
        pitched.strides[0], None, None))
    np.testing.assert_array_equal(pitched[:, :features], pinned)
    assert np.all(pitched[:, features:] == -7.0)
    plan.close()


def test_compute_into_a_torch_tensor():
    """Device-resident public output: SOAP.compute_into writes the rows of
    compute() into a torch tensor on the GPU (also a pitched view, and block
    by block when the batch is split), bit for bit."""

    torch = pytest.importorskip("torch")
    work = workloads.config(3, "small")
    p = work.params
    for average, dtype in (("off", "float32"), ("inner", "float64"), ("outer", "float64")):
        soap = mdx.SOAP(species=p["species"], r_cut=p["r_cut"], n_max=p["n_max"], l_max=p["l_max"],
                        average=average, output=mdx.OutputOptions(dtype=dtype))
        host = soap.compute(work.batch).values
        tdtype = torch.float32 if dtype == "float32" else torch.float64
        out = torch.full(host.shape, -1.0, dtype=tdtype, device="cuda:0")
        assert soap.compute_into(work.batch, out) is out
        np.testing.assert_array_equal(out.cpu().numpy(), host)
        wide = torch.full((host.shape[0], host.shape[1] + 7), -3.0, dtype=tdtype, device="cuda:0")
        soap._backend.atom_budget = 700
        control = mdx.ComputeControl()
        soap.compute_into(work.batch, wide[:, :host.shape[1]], control=control)
        assert control.completed() == work.batch.structures
        np.testing.assert_array_equal(wide[:, :host.shape[1]].cpu().numpy(), host)
        assert bool(torch.all(wide[:, host.shape[1]:] == -3.0))
        soap.close()


def test_overlapped_download_matches(hip_context):
    """Atom-level rows into page-locked memory leave in several launches'
    worth of slices on the copy stream while later launches compute (12288
    rows: three slices of 4096); a pitched page-locked destination keeps
    its padding.  Both equal the staged pageable download."""

    work = workloads.config(1)
    plan, _ = _plan(hip_context, work.params, "off", "float64")
    pageable = np.empty((work.batch.atoms, plan.features))
    plan.compute(work.batch, out=pageable)
    pinned, timing = plan.compute(work.batch)
    assert _hip.is_pinned(pinned) and timing["expansion_launches"] == 3
    np.testing.assert_array_equal(pinned, pageable)
    rows, features = pageable.shape
    pitch = (features + 3) * 8
    block = ctypes.c_void_p()
    assert hip_context.lib.mdx_hip_host_alloc(rows * pitch, ctypes.byref(block)) == 0
    try:
        pitched = np.ctypeslib.as_array(ctypes.cast(block, ctypes.POINTER(ctypes.c_double)),
                                        shape=(rows, features + 3))
        pitched[:] = -7.0
        arrays = _hip._BatchArrays(work.batch)
        hip_context.check(hip_context.lib.mdx_hip_soap_compute(
            hip_context.handle, plan.handle, ctypes.byref(arrays.view), block, rows, pitch, None, None))
        np.testing.assert_array_equal(pitched[:, :features], pageable)
        assert np.all(pitched[:, features:] == -7.0)
    finally:
        hip_context.lib.mdx_hip_host_free(block)
    plan.close()


def test_full_config2_structure_against_oracle(hip_context, oracle):
    """Headline configuration at full size: every row finite, and the rows of
    one 4096-atom cell equal to the oracle's for that cell alone."""

    work = workloads.config(2)
    plan, basis = _plan(hip_context, work.params)
    values, timing = plan.compute(work.batch)
    staged = np.empty((65536, 3696), dtype=np.float32)
    plan.compute(work.batch, out=staged)
    plan.close()
    assert values.shape == (65536, 3696) and values.dtype == np.float32
    np.testing.assert_array_equal(staged, values)
    assert np.all(np.isfinite(values))
    assert timing["pairs"] > 17_000_000
    for s in (0, 15):
        part = work.batch._slice_view(s, s + 1)
        expected = _oracle_soap(oracle, part, work.params, basis, "off")
        rows = values[work.batch.offsets[s]:work.batch.offsets[s + 1]]
        assert scaled_error(rows, expected) <= F32_GATE


@pytest.mark.parametrize("index", [1, 3, 4])
def test_full_size_configs_match_oracle(hip_context, oracle, index):
    """Seeded full-size configurations 1 (12,288 water atoms), 3 (20,000
    molecules, structure averages) and 4 (32,000-atom alloy) against the
    oracle over the whole batch, at each configuration's own average mode
    and output type."""

    work = workloads.config(index)
    p = work.params
    print(f"config {index} ({work.name}): {work.batch.atoms} atoms", flush=True)
    plan, basis = _plan(hip_context, p)
    try:
        values, timing = plan.compute(work.batch)
    finally:
        plan.close()
    expected = _oracle_soap(oracle, work.batch, p, basis, p["average"])
    assert values.shape == expected.shape and values.dtype == np.dtype(p["dtype"])
    assert np.all(np.isfinite(values))
    error = scaled_error(values, expected)
    assert error <= (F64_GATE if p["dtype"] == "float64" else F32_GATE), f"scaled error {error:.3e}"


def test_supercell_replication_at_full_size(hip_context):
    """A periodic cell tiled 2x2x2 gives every image the same features as its
    original atom (the 32000-atom HEA size, built from a 4000-atom cell)."""

    base = workloads.hea_fcc(10)
    p = base.params
    cell = base.batch.cells[0]
    shifts = np.array([[i, j, k] for i in range(2) for j in range(2) for k in range(2)], dtype=np.float64)
    positions = np.concatenate([base.batch.positions + s @ cell for s in shifts])
    numbers = np.tile(base.batch.numbers, 8)
    big = mdx.StructureBatch(numbers, positions, (2 * cell)[None], [[1, 1, 1]], [0, len(numbers)], ["tiled"])
    plan, _ = _plan(hip_context, p, "off", "float64")
    small_values, _ = plan.compute(base.batch)
    big_values, _ = plan.compute(big)
    plan.close()
    assert big_values.shape[0] == 32000
    n = base.batch.atoms
    for image in range(8):
        assert scaled_error(big_values[image * n:(image + 1) * n], small_values) <= 1e-9


def test_translation_invariance_full_config5(hip_context):
    work = workloads.config(5)
    plan, _ = _plan(hip_context, work.params, "off", "float32")
    first, timing = plan.compute(work.batch)
    moved = mdx.StructureBatch(work.batch.numbers, work.batch.positions + np.array([1.37, -2.11, 0.53]),
                               work.batch.cells, work.batch.pbc, work.batch.offsets, work.batch.ids)
    second, _ = plan.compute(moved)
    plan.close()
    assert first.shape == (216000, 780)
    assert scaled_error(second, first.astype(np.float64)) <= F32_GATE
