"""The CPU oracle against the reference's own golden fixtures.

* ``reference_soap/manifest.json``: the reference project's SOAP output for a
  periodic 32-atom HEA cell and an isolated water trimer, seven species,
  ``average="inner"`` (tolerance rtol 1e-9, atol 1e-11 from the manifest).
* ``reference_soap/external_manifest.json``: DScribe 2.1.2's output for a
  periodic water cell, ``average="off"``, sigma 0.5.
* ``reference_neighborlist/*``: the reference NeighborList (full list, no
  self pairs, cutoff 3.5) -- 448 pairs in graph order, and six pairs from
  the external provider.  The pair order pins the graph's visiting order.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import load_golden
from mdescriptor_amd.descriptors.basis import basis_gto


@pytest.mark.parametrize("manifest", ["manifest.json", "external_manifest.json"])
def test_oracle_matches_reference_soap_goldens(oracle, manifest):
    meta, batch, expected = load_golden("reference_soap", manifest)
    p = meta["configuration"]["parameters"]
    alphas, betas = basis_gto(p["r_cut"], p["n_max"], p["l_max"])
    values = oracle.soap(batch, species=p["species"], n_max=p["n_max"], l_max=p["l_max"], r_cut=p["r_cut"],
                         sigma=p.get("sigma", 1.0), alphas=alphas, betas=betas, average=p["average"])
    tol = meta["tolerance"]
    assert values.shape == expected["values"].shape
    np.testing.assert_allclose(values, expected["values"], rtol=tol["rtol"], atol=tol["atol"])


def _pair_table(oracle, batch, cutoff):
    """(samples, values) of a full neighbour list without self pairs, in graph
    order, from the oracle graph (neighbor_list.cpp:31-60)."""

    g = oracle.graph(batch, cutoff)
    offsets = np.asarray(batch.offsets)
    centre = np.repeat(np.arange(len(g["offsets"]) - 1), np.diff(g["offsets"]))
    keep = ~((g["atoms"] == centre) & np.all(g["shifts"] == 0, axis=1))
    structure = np.searchsorted(offsets, centre, side="right") - 1
    samples = np.column_stack((structure, centre - offsets[structure], g["atoms"] - offsets[structure],
                               g["shifts"]))[keep]
    values = np.column_stack((g["displacements"], np.sqrt(np.maximum(g["distance2"], 0.0))))[keep]
    return samples.astype(np.int64), values


@pytest.mark.parametrize("manifest", ["manifest.json", "external_manifest.json"])
def test_oracle_graph_matches_reference_neighbor_list(oracle, manifest):
    meta, batch, expected = load_golden("reference_neighborlist", manifest)
    cutoff = meta["configuration"]["parameters"]["cutoff"]
    samples, values = _pair_table(oracle, batch, cutoff)
    np.testing.assert_array_equal(samples, expected["samples"])
    np.testing.assert_allclose(values, expected["values"], rtol=1e-9, atol=1e-11)


def test_soap_golden_labels_follow_feature_layout():
    """Label order of the golden manifest == pair -> l -> n1 -> n2 layout."""

    from mdescriptor_amd.descriptors.soap import SoapSettings

    for manifest in ("manifest.json", "external_manifest.json"):
        meta, _, expected = load_golden("reference_soap", manifest)
        p = meta["configuration"]["parameters"]
        settings = SoapSettings(species=p["species"], n_max=p["n_max"], l_max=p["l_max"], r_cut=p["r_cut"],
                                sigma=p.get("sigma", 1.0), average=p["average"])
        assert list(settings.labels()) == meta["result"]["labels"]
        assert settings.feature_count == meta["result"]["feature_count"] == expected["values"].shape[1]
