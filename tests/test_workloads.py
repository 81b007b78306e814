"""The seeded benchmark workloads follow BASELINE.json's configuration text:
sizes, species, densities and geometric constraints."""

from __future__ import annotations

import numpy as np
import pytest

from mdescriptor_amd import workloads


@pytest.fixture(scope="module")
def molecules():
    return workloads.config(3).batch


def test_config3_sizes_are_uniform_9_to_29(molecules):
    sizes = np.diff(molecules.offsets)
    assert molecules.structures == 20000
    assert sizes.min() == 9 and sizes.max() == 29
    assert abs(sizes.mean() - 19.0) < 0.15
    counts = np.bincount(sizes, minlength=30)[9:30]
    # 20000 / 21 = 952 per size; 5 sigma of a multinomial count is ~150
    assert counts.min() > 800 and counts.max() < 1100


def test_config3_chemistry_and_geometry(molecules):
    b = molecules
    assert set(np.unique(b.numbers)) <= {1, 6, 7, 8, 9}
    assert np.all(b.pbc == 0) and np.all(b.cells == 0)
    valence = {6: 4, 7: 3, 8: 2, 9: 1}
    for s in range(0, b.structures, 53):
        z = b.numbers[b.offsets[s]:b.offsets[s + 1]]
        p = b.positions[b.offsets[s]:b.offsets[s + 1]]
        d = np.sqrt(((p[:, None] - p[None]) ** 2).sum(-1))
        np.fill_diagonal(d, np.inf)
        bonded = d <= 1.5 + 1e-9
        # bonds are 1.0-1.5 A, every other pair at least 1.8 A apart
        assert np.all(d[bonded] >= 1.0 - 1e-9)
        assert np.all((d >= 1.8 - 1e-9) | bonded)
        # saturated: every heavy atom has its valence in bonds, every H one bond
        degree = bonded.sum(1)
        assert np.all(degree[z == 1] == 1)
        for atom in np.flatnonzero(z != 1):
            assert degree[atom] == valence[int(z[atom])]
        # a tree: atoms - 1 bonds, one connected piece
        assert bonded.sum() // 2 == len(z) - 1


def test_config3_is_independent_of_worker_count():
    seeds = np.random.SeedSequence(workloads.SEED_BASE + 3).spawn(64)
    serial = [workloads._molecule(seed) for seed in seeds]
    batch = workloads.molecules(64).batch
    np.testing.assert_array_equal(batch.numbers, np.concatenate([g[0] for g in serial]))
    np.testing.assert_array_equal(batch.positions, np.concatenate([g[1] for g in serial]))


@pytest.mark.parametrize("index,atoms,structures,species", [
    (1, 12288, 64, {1, 8}),
    (2, 65536, 16, {1, 6, 7, 8}),
    (4, 32000, 1, {24, 26, 27, 28, 29}),
    (5, 216000, 1, {14}),
])
def test_periodic_configs(index, atoms, structures, species):
    w = workloads.config(index)
    b = w.batch
    assert (b.atoms, b.structures) == (atoms, structures)
    assert set(np.unique(b.numbers)) == species
    assert np.all(b.pbc == 1)
    volume = abs(np.linalg.det(b.cells[0]))
    density = int(b.offsets[1]) / volume
    expected = {1: 192 / 12.42**3, 2: 0.10, 4: 4 / 3.6**3, 5: 0.055}[index]
    assert density == pytest.approx(expected, rel=1e-3)


def test_config2_species_fractions_and_min_distance():
    b = workloads.config(2, "small").batch
    z = b.numbers[: b.offsets[1]]
    fractions = [np.mean(z == e) for e in (1, 6, 7, 8)]
    np.testing.assert_allclose(fractions, [0.5, 0.3, 0.1, 0.1], atol=0.03)
    cell = b.cells[0]
    p = b.positions[: b.offsets[1]]
    frac = p @ np.linalg.inv(cell)
    delta = frac[:, None] - frac[None]
    delta -= np.round(delta)
    d = np.sqrt(((delta @ cell) ** 2).sum(-1))
    np.fill_diagonal(d, np.inf)
    assert d.min() >= 0.9 - 1e-9
