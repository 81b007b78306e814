"""Seeded synthetic structures for the five benchmark configurations.

Each generator returns a :class:`~mdescriptor_amd.core.input.StructureBatch`
plus the SOAP parameters of its configuration.  Seeds are fixed
(``numpy.random.PCG64(20261201 + cfg)``) so every run, test and benchmark
sees the same atoms.  ``scale`` shrinks a configuration for quick checks
(fewer structures or a smaller supercell) without changing its density or
chemistry.

  cfg 1  64 periodic boxes of 64 H2O, L = 12.42 A, species [1, 8],
         r_cut 4.5, n 4, l 3, average off, float64
  cfg 2  16 periodic cells of 4096 H/C/N/O atoms at 0.10 A^-3 (L = 34.47 A),
         fractions 0.5/0.3/0.1/0.1, min distance 0.9 A; r_cut 5, n 8, l 6,
         average off, float32 (the headline configuration)
  cfg 3  20000 isolated molecules of 9-29 atoms (C/N/O/F heavy atoms with
         saturating H); r_cut 5, n 6, l 4, average inner, float64
  cfg 4  FCC high-entropy alloy, 20^3 cells (32000 atoms, a = 3.6 A),
         species [24, 26, 27, 28, 29]; r_cut 6, n 8, l 8, off, float32
  cfg 5  liquid-like Si, 216000 atoms at 0.055 A^-3; r_cut 5.5, n 12, l 9,
         off, float32
"""

from __future__ import annotations

import multiprocessing
import os
import sys
from concurrent.futures import ProcessPoolExecutor
from dataclasses import dataclass
from typing import Any

import numpy as np

from .core.input import StructureBatch

SEED_BASE = 20261201


@dataclass(frozen=True)
class Workload:
    name: str
    batch: StructureBatch
    params: dict[str, Any]


def _rng(cfg: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(SEED_BASE + cfg))


def _random_rotation(rng: np.random.Generator) -> np.ndarray:
    q = rng.normal(size=4)
    q /= np.linalg.norm(q)
    a, b, c, d = q
    return np.array([
        [a * a + b * b - c * c - d * d, 2 * (b * c - a * d), 2 * (b * d + a * c)],
        [2 * (b * c + a * d), a * a - b * b + c * c - d * d, 2 * (c * d - a * b)],
        [2 * (b * d - a * c), 2 * (c * d + a * b), a * a - b * b - c * c + d * d],
    ])


def _pack(numbers: list[np.ndarray], positions: list[np.ndarray], cells: list[np.ndarray],
          pbc: list[Any], name: str) -> StructureBatch:
    offsets = np.concatenate([[0], np.cumsum([len(n) for n in numbers])]).astype(np.int64)
    return StructureBatch(
        np.concatenate(numbers).astype(np.int32),
        np.concatenate(positions).astype(np.float64),
        np.asarray(cells, dtype=np.float64),
        np.asarray(pbc, dtype=np.int32),
        offsets,
        tuple(f"{name}-{i}" for i in range(len(numbers))),
    )


def water_boxes(boxes: int = 64) -> Workload:
    """Configuration 1: periodic water boxes."""

    rng = _rng(1)
    length = 12.42
    spacing = length / 4.0
    angle = np.deg2rad(104.5)
    numbers, positions, cells = [], [], []
    for _ in range(boxes):
        grid = np.stack(np.meshgrid(np.arange(4), np.arange(4), np.arange(4), indexing="ij"), -1).reshape(-1, 3)
        oxygen = (grid + 0.5) * spacing + rng.uniform(-0.5, 0.5, size=(64, 3))
        local_h = 0.96 * np.array([[np.sin(angle / 2), 0.0, np.cos(angle / 2)],
                                   [-np.sin(angle / 2), 0.0, np.cos(angle / 2)]])
        pos = []
        num = []
        for o in oxygen:
            rot = _random_rotation(rng)
            pos.append(o)
            pos.extend(o + local_h @ rot.T)
            num.extend([8, 1, 1])
        numbers.append(np.asarray(num))
        positions.append(np.asarray(pos))
        cells.append(np.eye(3) * length)
    batch = _pack(numbers, positions, cells, [[1, 1, 1]] * boxes, "water")
    return Workload("water-64x192", batch, dict(species=[1, 8], r_cut=4.5, n_max=4, l_max=3, average="off",
                                                 dtype="float64"))


def _random_dense_cell(rng: np.random.Generator, natoms: int, length: float, min_distance: float) -> np.ndarray:
    """Uniform positions in a cubic box with sequential rejection at a minimum
    minimum-image distance, using a small cell list for the rejection test."""

    ncell = max(1, int(length // min_distance))
    width = length / ncell
    cells: dict[tuple[int, int, int], list[int]] = {}
    accepted = np.empty((natoms, 3))
    count = 0
    d2min = min_distance * min_distance
    while count < natoms:
        trial = rng.uniform(0.0, length, size=3)
        key = tuple(int(v) % ncell for v in trial // width)
        ok = True
        for dx in (-1, 0, 1):
            for dy in (-1, 0, 1):
                for dz in (-1, 0, 1):
                    for idx in cells.get(((key[0] + dx) % ncell, (key[1] + dy) % ncell, (key[2] + dz) % ncell), ()):
                        d = accepted[idx] - trial
                        d -= length * np.round(d / length)
                        if d @ d < d2min:
                            ok = False
                            break
                    if not ok:
                        break
                if not ok:
                    break
            if not ok:
                break
        if ok:
            accepted[count] = trial
            cells.setdefault(key, []).append(count)
            count += 1
    return accepted


def hcno_cells(cells_count: int = 16, natoms: int = 4096) -> Workload:
    """Configuration 2: random H/C/N/O cells at 0.10 atoms per cubic angstrom."""

    rng = _rng(2)
    length = (natoms / 0.10) ** (1.0 / 3.0)
    n_h = natoms // 2
    n_n = int(round(natoms * 0.1))
    n_o = int(round(natoms * 0.1)) - (1 if natoms == 4096 else 0)
    n_c = natoms - n_h - n_n - n_o
    base = np.array([1] * n_h + [6] * n_c + [7] * n_n + [8] * n_o)
    numbers, positions, cells = [], [], []
    for _ in range(cells_count):
        numbers.append(rng.permutation(base))
        positions.append(_random_dense_cell(rng, natoms, length, 0.9))
        cells.append(np.eye(3) * length)
    batch = _pack(numbers, positions, cells, [[1, 1, 1]] * cells_count, "hcno")
    return Workload(f"hcno-{cells_count}x{natoms}", batch, dict(species=[1, 6, 7, 8], r_cut=5.0, n_max=8, l_max=6,
                                                               average="off", dtype="float32"))


_VALENCE = {6: 4, 7: 3, 8: 2, 9: 1}
# tetrahedral bond directions: the bonds of a heavy atom point along the
# first `valence` of them (the first facing the atom's parent)
_TETRAHEDRON = np.array([[1.0, 1.0, 1.0], [1.0, -1.0, -1.0], [-1.0, 1.0, -1.0], [-1.0, -1.0, 1.0]]) / np.sqrt(3.0)


def _rotation_to(u: np.ndarray, v: np.ndarray) -> np.ndarray:
    """A rotation taking unit vector u onto unit vector v."""

    axis = np.cross(u, v)
    s, c = np.linalg.norm(axis), float(np.dot(u, v))
    if s < 1e-12:
        if c > 0:
            return np.eye(3)
        # half turn about any axis normal to u
        normal = np.cross(u, [1.0, 0.0, 0.0] if abs(u[0]) < 0.9 else [0.0, 1.0, 0.0])
        normal /= np.linalg.norm(normal)
        return 2.0 * np.outer(normal, normal) - np.eye(3)
    k = axis / s
    kx = np.array([[0.0, -k[2], k[1]], [k[2], 0.0, -k[0]], [-k[1], k[0], 0.0]])
    return np.eye(3) + s * kx + (1.0 - c) * kx @ kx


def _random_rotations(rng: np.random.Generator, count: int) -> np.ndarray:
    """`count` uniformly random rotation matrices (unit quaternions)."""

    q = rng.normal(size=(count, 4))
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    a, b, c, d = q.T
    return np.stack([
        np.stack([a * a + b * b - c * c - d * d, 2 * (b * c - a * d), 2 * (b * d + a * c)], -1),
        np.stack([2 * (b * c + a * d), a * a - b * b + c * c - d * d, 2 * (c * d - a * b)], -1),
        np.stack([2 * (b * d - a * c), 2 * (c * d + a * b), a * a - b * b - c * c + d * d], -1),
    ], 1)


def _twisted(directions: np.ndarray, axis: np.ndarray, angles: np.ndarray) -> np.ndarray:
    """directions (k, 3) rotated about the unit axis by each angle: (R, k, 3)."""

    cos, sin = np.cos(angles)[:, None, None], np.sin(angles)[:, None, None]
    along = (directions @ axis)[None, :, None] * axis
    return directions[None] * cos + np.cross(axis, directions)[None] * sin + along * (1.0 - cos)


def _grow_molecule(rng: np.random.Generator, target: int) -> tuple[np.ndarray, np.ndarray] | None:
    """One molecule of exactly `target` atoms, or None when this attempt
    fails (the caller regrows).

    Topology: a tree of heavy atoms (C/N/O/F drawn independently with
    probabilities 0.70/0.15/0.12/0.03) grows from an atom with free valence,
    the newest one with probability 0.7 so that chains grow away from the
    rest; a heavy atom of valence v adds v - 1 atoms to the saturated size
    sum(v) - h + 2, so heavy atoms are added until the saturated size
    reaches the target (an overshoot fails the attempt), and every free
    valence carries one H.

    Geometry, heavy atoms in growth order: an atom's bonds point along a
    tetrahedron whose first vertex faces its parent, twisted about that bond
    at random, each bond 1.0-1.5 A long.  Of 128 random twists and lengths
    whose new atoms keep 1.8 A from every atom but their bonded parent (and
    from each other), the least crowded by the atoms already placed (sum of
    d^-6) is taken; when none does, the attempt fails."""

    heavy_choice = np.array([6, 7, 8, 9])
    heavy_prob = np.array([0.70, 0.15, 0.12, 0.03])
    heavy = [int(rng.choice(heavy_choice, p=heavy_prob))]
    parent_of = [-1]
    free = [_VALENCE[heavy[0]]]
    size = free[0] + 1
    while size < target:
        element = int(rng.choice(heavy_choice, p=heavy_prob))
        open_atoms = [i for i, f in enumerate(free) if f > 0]
        if not open_atoms or size + _VALENCE[element] - 1 > target:
            return None
        parent = open_atoms[-1] if rng.random() < 0.7 else open_atoms[int(rng.integers(len(open_atoms)))]
        heavy.append(element)
        parent_of.append(parent)
        free.append(_VALENCE[element] - 1)
        free[parent] -= 1
        size += _VALENCE[element] - 1

    elements = np.empty(target, dtype=np.int64)
    coords = np.empty((target, 3))
    slot = [0] * len(heavy)  # atom index of each heavy atom
    elements[0], coords[0] = heavy[0], 0.0
    placed = 1
    trials = 128
    for h in range(len(heavy)):
        centre = coords[slot[h]]
        children = [c for c in range(len(heavy)) if parent_of[c] == h]
        bonds = [heavy[c] for c in children] + [1] * free[h]
        k = len(bonds)
        if k == 0:
            continue
        p = parent_of[h]
        # `trials` candidate arrangements of the k bonds at once
        if p >= 0:
            back = coords[slot[p]] - centre
            back /= np.linalg.norm(back)
            base = (_rotation_to(_TETRAHEDRON[0], back) @ _TETRAHEDRON[1:1 + k].T).T
            directions = _twisted(base, back, rng.uniform(0.0, 2.0 * np.pi, size=trials))
        else:
            directions = np.einsum("rij,kj->rki", _random_rotations(rng, trials), _TETRAHEDRON[:k])
        positions = centre + directions * rng.uniform(1.0, 1.5, size=(trials, k, 1))
        # 1.8 A from every placed atom but this centre, and between the new atoms
        d2 = np.sum((positions[:, :, None, :] - coords[None, None, :placed, :]) ** 2, axis=3)
        d2[:, :, slot[h]] = np.inf
        clear = np.all(d2 >= 1.8 * 1.8, axis=(1, 2))
        if k > 1:
            mutual = np.sum((positions[:, :, None, :] - positions[:, None, :, :]) ** 2, axis=3)
            mutual[:, np.arange(k), np.arange(k)] = np.inf
            clear &= np.all(mutual >= 1.8 * 1.8, axis=(1, 2))
        if not np.any(clear):
            return None
        crowding = np.where(clear, np.sum(1.0 / d2 ** 3, axis=(1, 2)), np.inf)
        coords[placed:placed + k] = positions[int(np.argmin(crowding))]
        elements[placed:placed + k] = bonds
        for b, c in enumerate(children):
            slot[c] = placed + b
        placed += k
    return elements, coords


def _molecule(seed: np.random.SeedSequence) -> tuple[np.ndarray, np.ndarray]:
    """One configuration-3 molecule from its own seed: a size drawn uniformly
    in 9-29, grown (and regrown) until it has exactly that many atoms, then
    placed at a random offset in a 40 A box."""

    rng = np.random.Generator(np.random.PCG64(seed))
    target = int(rng.integers(9, 30))
    grown = None
    while grown is None:
        grown = _grow_molecule(rng, target)
    elements, coords = grown
    return elements, coords + rng.uniform(-20.0, 20.0, size=3)


def molecules(count: int = 20000) -> Workload:
    """Configuration 3: isolated molecules of 9-29 atoms (uniform), grown by
    random self-avoiding steps.  Each molecule has its own seed, spawned
    from the configuration's, so the batch is the same whether it is grown
    in this process or, for large counts run from a script file, by a pool
    of spawned (never forked) worker processes."""

    seeds = np.random.SeedSequence(SEED_BASE + 3).spawn(count)
    main = sys.modules.get("__main__")
    main_file = getattr(main, "__file__", None)
    workers = min(16, os.cpu_count() or 1)
    if count >= 2000 and workers > 1 and main_file is not None and os.path.isfile(main_file):
        with ProcessPoolExecutor(max_workers=workers, mp_context=multiprocessing.get_context("spawn")) as pool:
            grown = list(pool.map(_molecule, seeds, chunksize=max(1, count // (4 * workers))))
    else:
        grown = [_molecule(seed) for seed in seeds]
    batch = _pack([g[0] for g in grown], [g[1] for g in grown], [np.zeros((3, 3))] * count, [[0, 0, 0]] * count,
                  "molecule")
    return Workload(f"molecules-{count}", batch, dict(species=[1, 6, 7, 8, 9], r_cut=5.0, n_max=6, l_max=4,
                                                      average="inner", dtype="float64"))


def hea_fcc(repeat: int = 20) -> Workload:
    """Configuration 4: FCC high-entropy alloy supercell."""

    rng = _rng(4)
    a = 3.6
    basis = np.array([[0, 0, 0], [0.5, 0.5, 0], [0.5, 0, 0.5], [0, 0.5, 0.5]])
    grid = np.stack(np.meshgrid(*(np.arange(repeat),) * 3, indexing="ij"), -1).reshape(-1, 1, 3)
    pos = ((grid + basis[None]) * a).reshape(-1, 3)
    pos = pos + rng.normal(scale=0.1, size=pos.shape)
    species = np.array([24, 26, 27, 28, 29])
    numbers = rng.choice(species, size=len(pos))
    batch = _pack([numbers], [pos], [np.eye(3) * a * repeat], [[1, 1, 1]], "hea")
    return Workload(f"hea-fcc-{len(pos)}", batch, dict(species=species.tolist(), r_cut=6.0, n_max=8, l_max=8,
                                                       average="off", dtype="float32"))


def liquid_si(repeat: int = 30) -> Workload:
    """Configuration 5: diamond Si with large displacements, rescaled to 0.055 A^-3."""

    rng = _rng(5)
    a = 5.43
    basis = np.array([[0, 0, 0], [0, 0.5, 0.5], [0.5, 0, 0.5], [0.5, 0.5, 0],
                      [0.25, 0.25, 0.25], [0.25, 0.75, 0.75], [0.75, 0.25, 0.75], [0.75, 0.75, 0.25]])
    grid = np.stack(np.meshgrid(*(np.arange(repeat),) * 3, indexing="ij"), -1).reshape(-1, 1, 3)
    pos = ((grid + basis[None]) * a).reshape(-1, 3)
    pos = pos + rng.normal(scale=0.4, size=pos.shape)
    natoms = len(pos)
    length = a * repeat
    target = (natoms / 0.055) ** (1.0 / 3.0)
    pos *= target / length
    batch = _pack([np.full(natoms, 14)], [pos], [np.eye(3) * target], [[1, 1, 1]], "si")
    return Workload(f"liquid-si-{natoms}", batch, dict(species=[14], r_cut=5.5, n_max=12, l_max=9, average="off",
                                                       dtype="float32"))


def config(index: int, scale: str = "full") -> Workload:
    """Workload of benchmark configuration 1-5; ``scale="small"`` gives a
    reduced variant of the same chemistry for tests."""

    small = scale == "small"
    if index == 1:
        return water_boxes(4 if small else 64)
    if index == 2:
        return hcno_cells(2, 512) if small else hcno_cells()
    if index == 3:
        return molecules(200 if small else 20000)
    if index == 4:
        return hea_fcc(4 if small else 20)
    if index == 5:
        return liquid_si(4 if small else 30)
    raise ValueError("configuration index must be 1-5")


__all__ = ["Workload", "config", "hcno_cells", "hea_fcc", "liquid_si", "molecules", "water_boxes"]
