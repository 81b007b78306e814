"""Parity of the device NeighborList with the CPU oracle, through the C-ABI.

Gate: bit-identical.  The table (centre, neighbour, shifts, displacement,
distance) equals the oracle's in every value and in order, for every
(full_neighbor_list, self_pairs) setting; the values and samples outputs are
the table's columns in the public layout.  The reference's NeighborList
goldens are checked end to end through the public ``NeighborList`` class.  At
the headline configuration's full size (65536 atoms, 3.4 million pairs at
its 5 Angstrom cutoff) the full/half identity is checked on the whole batch and one
structure against the oracle.
"""

from __future__ import annotations

import ctypes
import itertools

import numpy as np
import pytest

import mdescriptor_amd as mdx
from conftest import edge_batch, load_golden, table_samples
from mdescriptor_amd import _hip, workloads

pytestmark = pytest.mark.gpu

SETTINGS = list(itertools.product([True, False], [False, True]))


def _device(ctx, batch, cutoff, full, self_pairs):
    return _hip.neighbor_list(ctx, batch, cutoff, full_neighbor_list=full, self_pairs=self_pairs, table=True)


def _check(ctx, oracle, batch, cutoff, full, self_pairs):
    ours = _device(ctx, batch, cutoff, full, self_pairs)
    table, offsets = oracle.neighbor_list(batch, cutoff, full_neighbor_list=full, self_pairs=self_pairs)
    np.testing.assert_array_equal(ours["offsets"], offsets)
    np.testing.assert_array_equal(ours["table"], table)
    np.testing.assert_array_equal(ours["values"], table[:, 5:])
    np.testing.assert_array_equal(ours["samples"], table_samples(table, offsets, batch.offsets))
    return ours


@pytest.fixture(scope="module", params=[1, 2, 3, 4, 5])
def workload(request):
    return workloads.config(request.param, "small")


@pytest.mark.parametrize("full, self_pairs", SETTINGS)
def test_table_identical_to_oracle(hip_context, oracle, workload, full, self_pairs):
    _check(hip_context, oracle, workload.batch, workload.params["r_cut"], full, self_pairs)


@pytest.mark.parametrize("full, self_pairs", SETTINGS)
@pytest.mark.parametrize("cutoff", [1.2, 4.5, 9.0])
def test_edge_cases_identical_to_oracle(hip_context, oracle, full, self_pairs, cutoff):
    _check(hip_context, oracle, edge_batch(), cutoff, full, self_pairs)


@pytest.mark.parametrize("manifest", ["manifest.json", "external_manifest.json"])
@pytest.mark.parametrize("dtype", ["float64", "float32"])
def test_public_neighbor_list_reproduces_goldens(manifest, dtype):
    meta, raw, expected = load_golden("reference_neighborlist", manifest)
    p = meta["configuration"]["parameters"]
    ids = meta.get("result", {}).get("structure_ids") or [f"s{i}" for i in range(len(raw.offsets) - 1)]
    batch = mdx.StructureBatch(raw.numbers, raw.positions, raw.cells, raw.pbc, raw.offsets, ids)
    with mdx.NeighborList(cutoff=p["cutoff"], full_neighbor_list=p["full_neighbor_list"],
                          self_pairs=p["self_pairs"], output=mdx.OutputOptions(dtype=dtype)) as descriptor:
        result = descriptor.compute(batch)
        configuration = descriptor.configuration.to_dict()
    if dtype == "float64":
        np.testing.assert_array_equal(result.values, expected["values"])
    else:
        assert result.values.dtype == np.float32
        np.testing.assert_array_equal(result.values, expected["values"].astype(np.float32))
    np.testing.assert_array_equal(result.samples, expected["samples"])
    assert result.level.value == "pair" and list(result.labels) == ["dx", "dy", "dz", "distance"]
    assert result.feature_count == 4 and list(result.structure_ids) == ids
    if "result" in meta:
        assert result.row_offsets.tolist() == meta["result"]["row_offsets"]
        reference = dict(meta["result"]["metadata"])
        ours = dict(result.metadata)
        assert ours.pop("backend") == "mdescriptor-hip" and reference.pop("backend") == "mdescriptor-cpp"
        assert ours.pop("execution")["device"] == "hip"
        reference.pop("execution")
        reference["output"] = {"dtype": dtype, "sparse": False}
        assert ours == reference
    for key in ("cutoff", "full_neighbor_list", "self_pairs"):
        assert configuration["parameters"][key] == p[key]
    assert not result.values.flags.writeable


def test_device_outputs_match_host_outputs(hip_context):
    """Device pointers are written in place by the fill kernel; host ones go
    through the staging area.  Both give the same bytes."""

    batch = workloads.config(3, "small").batch
    host = _device(hip_context, batch, 5.0, False, True)
    rows = len(host["values"])
    sizes = {"table": rows * 72, "values": rows * 32, "samples": rows * 48, "offsets": len(host["offsets"]) * 8}
    memory = {k: _hip.DeviceMemory(v) for k, v in sizes.items()}
    lib = hip_context.lib
    hip_context.check(lib.mdx_hip_neighbor_list_fetch(
        hip_context.handle, *(ctypes.c_void_p(memory[k].address) for k in ("table", "values", "samples", "offsets"))))
    _hip.DeviceMemory.synchronize()
    for key, like in (("table", host["table"]), ("values", host["values"]), ("samples", host["samples"]),
                      ("offsets", host["offsets"])):
        np.testing.assert_array_equal(memory[key].to_host(np.empty_like(like)), like, err_msg=key)
        memory[key].free()
    # a device destination the 8-byte stores cannot take in place receives a copy
    shifted = _hip.DeviceMemory(rows * 32 + 8)
    hip_context.check(lib.mdx_hip_neighbor_list_fetch(hip_context.handle, None,
                                                      ctypes.c_void_p(shifted.address + 4), None, None))
    _hip.DeviceMemory.synchronize()
    raw = shifted.to_host(np.empty(rows * 32 + 8, dtype=np.uint8))
    np.testing.assert_array_equal(raw[4:4 + rows * 32].view(np.float64).reshape(rows, 4), host["values"])
    shifted.free()
    # pageable host destinations take the staged download
    table = np.empty((rows, 9))
    hip_context.check(lib.mdx_hip_neighbor_list_fetch(hip_context.handle, table.ctypes.data_as(ctypes.c_void_p),
                                                      None, None, None))
    np.testing.assert_array_equal(table, host["table"])


def test_fetch_needs_a_fresh_list(hip_context):
    batch = workloads.config(1, "small").batch
    _device(hip_context, batch, 4.0, True, False)
    hip_context.check(hip_context.lib.mdx_hip_neighbors_build(
        hip_context.handle, ctypes.byref(_hip._BatchArrays(batch).view), 4.0, 1, None))
    with pytest.raises(ValueError, match="no neighbour list"):
        hip_context.check(hip_context.lib.mdx_hip_neighbor_list_fetch(hip_context.handle, None, None, None, None))


def test_public_block_splitting_and_control(hip_context):
    work = workloads.config(3, "small")
    direct = _device(hip_context, work.batch, 5.0, True, False)
    descriptor = mdx.NeighborList(cutoff=5.0)
    control = mdx.ComputeControl()
    whole = descriptor.compute(work.batch, control=control)
    assert control.completed() == control.total() == work.batch.structures
    descriptor._backend.atom_budget = 700
    split = descriptor.compute(work.batch)
    descriptor.close()
    for result in (whole, split):
        np.testing.assert_array_equal(result.values, direct["values"])
        np.testing.assert_array_equal(result.samples, direct["samples"])
        np.testing.assert_array_equal(result.row_offsets, direct["offsets"])


def test_empty_batch_and_empty_structures(hip_context, oracle):
    empty = mdx.StructureBatch(np.zeros(0, np.int32), np.zeros((0, 3)), np.zeros((0, 3, 3)), np.zeros((0, 3)), [0],
                               [])
    result = mdx.NeighborList(cutoff=3.0).compute(empty)
    assert result.values.shape == (0, 4) and result.samples.shape == (0, 6) and result.row_offsets.tolist() == [0]
    lonely = mdx.StructureBatch(np.array([8, 1], np.int32), np.array([[0.0, 0, 0], [10.0, 0, 0]]),
                                np.zeros((2, 3, 3)), np.zeros((2, 3)), [0, 1, 2], ["a", "b"])
    for self_pairs in (False, True):
        result = mdx.NeighborList(cutoff=3.0, self_pairs=self_pairs).compute(lonely)
        assert result.row_offsets.tolist() == ([0, 1, 2] if self_pairs else [0, 0, 0])
        _check(hip_context, oracle, lonely, 3.0, False, self_pairs)


def test_cancellation_and_invalid_cutoff(hip_context):
    batch = workloads.config(1, "small").batch
    flag = ctypes.c_int32(1)
    with pytest.raises(_hip.HipCancelledError):
        _hip.neighbor_list(hip_context, batch, 4.0, cancel=flag)
    control = mdx.ComputeControl()
    control.cancel()
    with pytest.raises(mdx.CancelledError):
        mdx.NeighborList(cutoff=4.0).compute(batch, control=control)
    for cutoff in (float("inf"), float("nan")):
        with pytest.raises(mdx.DescriptorInputError, match="finite and positive"):
            mdx.NeighborList(cutoff=cutoff).compute(batch)


def test_sparse_output(hip_context):
    batch = workloads.config(1, "small").batch
    dense = mdx.NeighborList(cutoff=4.0).compute(batch)
    sparse = mdx.NeighborList(cutoff=4.0, output=mdx.OutputOptions(sparse=True)).compute(batch)
    np.testing.assert_array_equal(sparse.values.toarray(), dense.values)
    np.testing.assert_array_equal(sparse.samples, dense.samples)


def test_full_size_config2(hip_context, oracle):
    """Headline configuration at full size: the full list is the half list
    plus its reversal, and one 4096-atom cell equals the oracle's list for
    that cell alone."""

    work = workloads.config(2)
    cutoff = work.params["r_cut"]
    full = _hip.neighbor_list(hip_context, work.batch, cutoff, full_neighbor_list=True)
    half = _hip.neighbor_list(hip_context, work.batch, cutoff, full_neighbor_list=False)
    assert len(full["values"]) > 3_000_000
    assert len(full["values"]) == 2 * len(half["values"])
    key_full = full["samples"].copy()
    reversed_half = half["samples"][:, [0, 2, 1, 3, 4, 5]].copy()
    reversed_half[:, 3:] *= -1
    both = np.concatenate([half["samples"], reversed_half])
    order_a = np.lexsort(key_full.T[::-1])
    order_b = np.lexsort(both.T[::-1])
    np.testing.assert_array_equal(key_full[order_a], both[order_b])
    distance = np.concatenate([half["values"][:, 3], half["values"][:, 3]])
    np.testing.assert_allclose(full["values"][order_a, 3], distance[order_b], rtol=1e-13)
    assert np.all(full["values"][:, 3] <= cutoff)
    for s in (0, 15):
        part = work.batch._slice_view(s, s + 1)
        table, offsets = oracle.neighbor_list(part, cutoff)
        lo, hi = full["offsets"][s], full["offsets"][s + 1]
        np.testing.assert_array_equal(full["values"][lo:hi], table[:, 5:])
        expected = table_samples(table, offsets, part.offsets)
        expected[:, 0] = s
        np.testing.assert_array_equal(full["samples"][lo:hi], expected)
