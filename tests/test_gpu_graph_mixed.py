"""Neighbour graph and NeighborList of seeded mixed batches against the oracle.

Each batch mixes periodic boxes (orthorhombic and tilted), molecules, empty
structures and, in some seeds, a box of more than 8,192 periodic images,
with one to six species.  Depending on the mix the library bins each
structure on its own (a wavefront per structure of at most 64 images, a
workgroup per structure of at most 8,192) or runs the multi-kernel binning
(count, scan, fill, sort); the search then reads each cell's species runs.
The graph (pairs, shifts, displacements, d^2) and the NeighborList table
must be identical to the oracle's, element for element, on every path.
"""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest

from conftest import SOAP_PAD
from mdescriptor_amd import _hip

pytestmark = pytest.mark.gpu

SPECIES_SETS = [[14], [1, 8], [1, 6, 7], [1, 6, 7, 8, 9, 16]]


def _mixed_batch(seed: int) -> SimpleNamespace:
    rng = np.random.default_rng(seed)
    species = SPECIES_SETS[seed % len(SPECIES_SETS)]
    kinds = list(rng.choice(["box", "tilted", "molecule", "molecule", "empty"], size=int(rng.integers(3, 8))))
    if seed % 3 == 0:
        kinds.append("big")
    parts, cells, pbc, counts = [], [], [], []
    for kind in kinds:
        if kind in ("box", "tilted", "big"):
            n = 400 if kind == "big" else int(rng.integers(20, 160))
            length = 14.0 if kind == "big" else float(rng.uniform(6.5, 10.0))
            cell = np.eye(3) * length
            if kind == "tilted":
                cell[1, 0] = rng.uniform(-1.5, 1.5)
                cell[2, 0] = rng.uniform(-1.5, 1.5)
                cell[2, 1] = rng.uniform(-1.5, 1.5)
            parts.append(rng.uniform(0.0, 1.0, (n, 3)) @ cell)
            cells.append(cell)
            pbc.append([1, 1, 1])
        elif kind == "molecule":
            n = int(rng.integers(1, 40))
            parts.append(rng.normal(0.0, 1.5, (n, 3)) + rng.uniform(-50.0, 50.0, 3))
            cells.append(np.zeros((3, 3)))
            pbc.append([0, 0, 0])
        else:
            n = 0
            parts.append(np.zeros((0, 3)))
            cells.append(np.zeros((3, 3)))
            pbc.append([0, 0, 0])
        counts.append(n)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    numbers = rng.choice(species, size=int(offsets[-1])).astype(np.int32)
    return SimpleNamespace(numbers=numbers, positions=np.concatenate(parts), cells=np.stack(cells),
                           pbc=np.array(pbc, np.int32), offsets=offsets, species=species)


@pytest.mark.parametrize("seed", range(12))
def test_mixed_batch_graph_and_list(hip_context, oracle, seed):
    batch = _mixed_batch(seed)
    print(f"mixed batch seed {seed}: {len(batch.offsets) - 1} structures, {batch.offsets[-1]} atoms", flush=True)
    cutoff = 3.0 + SOAP_PAD
    ours = _hip.neighbor_graph(hip_context, batch, cutoff)
    theirs = oracle.graph(batch, cutoff)
    for key in theirs:
        np.testing.assert_array_equal(ours[key], theirs[key], err_msg=f"seed {seed}: {key}")
    for full in (True, False):
        listed = _hip.neighbor_list(hip_context, batch, 3.0, full_neighbor_list=full, table=True)
        table, offsets = oracle.neighbor_list(batch, 3.0, full_neighbor_list=full, self_pairs=False)
        np.testing.assert_array_equal(listed["offsets"], offsets, err_msg=f"seed {seed}")
        np.testing.assert_array_equal(listed["table"], table, err_msg=f"seed {seed}")
