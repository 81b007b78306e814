"""TEST INFRASTRUCTURE ONLY — ctypes access to the CPU oracle.

Two libraries are reachable from here:

* ``oracle/_bin/libmdx_oracle.so``: the C restatement in ``soap_oracle.c``
  of the reference's neighbour graph (cpp/src/common/neighbor.cpp:423-768),
  NeighborList descriptor (cpp/src/standalone/neighbor_list.cpp:15-78) and
  SOAP (cpp/src/standalone/soap.cpp:494-1246);
* ``oracle/_ref/libmdx_ref.so``: the reference's own C++ compiled in place
  (``oracle/Makefile``), present only where it was built.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, and only as the checker or the
timed CPU baseline.  The product package never imports it.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path
from typing import Any

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_LIB = HERE / "_bin" / "libmdx_oracle.so"
REF_LIB = HERE / "_ref" / "libmdx_ref.so"

_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_f64p = ctypes.POINTER(ctypes.c_double)


class _Graph(ctypes.Structure):
    _fields_ = [
        ("atoms", ctypes.c_int64),
        ("pairs", ctypes.c_int64),
        ("offsets", _i64p),
        ("neighbors", _i32p),
        ("shifts", _i32p),
        ("disp", _f64p),
        ("d2", _f64p),
    ]


class _PairTable(ctypes.Structure):
    """mdxo_pair_table / mdxr_pair_table: DescriptorPairTable
    (cpp/include/mdescriptor/local_descriptors.hpp:29-34)."""

    _fields_ = [
        ("rows", ctypes.c_int64),
        ("structures", ctypes.c_int64),
        ("values", _f64p),
        ("offsets", _i64p),
    ]


class _Options(ctypes.Structure):
    """mdxo_soap_options / mdxr_soap_options (the SoapOptions fields beyond
    the GTO, uncompressed, unweighted default; descriptor.hpp:17-43)."""

    _fields_ = [
        ("weighting_function", ctypes.c_int32),
        ("weighting_has_w0", ctypes.c_int32),
        ("weighting_r0", ctypes.c_double),
        ("weighting_c", ctypes.c_double),
        ("weighting_d", ctypes.c_double),
        ("weighting_m", ctypes.c_double),
        ("weighting_w0", ctypes.c_double),
        ("species_weights", _f64p),
        ("compression", ctypes.c_int32),
        ("radial_basis", ctypes.c_int32),
        ("grid_size", ctypes.c_int32),
        ("radial_grid", _f64p),
        ("radial_weights", _f64p),
        ("radial_values", _f64p),
    ]


_COMPRESSION = {"off": 0, "mu2": 1, "mu1nu1": 2, "crossover": 3}
_WEIGHTING = {"poly": 1, "pow": 2, "exp": 3}


def feature_count(S: int, n: int, l_max: int, compression: str = "off") -> int:
    """soap_features (soap.cpp:373-387)."""

    L = l_max + 1
    if compression == "mu2":
        return n * (n + 1) // 2 * L
    if compression == "mu1nu1":
        return S * n * n * L
    if compression == "crossover":
        return S * n * (n + 1) // 2 * L
    w = S * n
    return w * (w + 1) // 2 * L


def _options(options: dict | None, S: int, keep: list) -> Any:
    """A ctypes options struct (or None) from
    {"weighting": {...}, "species_weights": [...], "compression": str,
     "polynomial": (grid, weights, values)}; `keep` holds the arrays alive."""

    if not options:
        return None
    o = _Options()
    weighting = dict(options.get("weighting") or {})
    if "function" in weighting:
        o.weighting_function = _WEIGHTING[weighting["function"]]
    o.weighting_has_w0 = 1 if "w0" in weighting else 0
    o.weighting_r0 = float(weighting.get("r0", 1.0))
    o.weighting_c = float(weighting.get("c", 1.0))
    o.weighting_d = float(weighting.get("d", 0.0))
    o.weighting_m = float(weighting.get("m", 1.0))
    o.weighting_w0 = float(weighting.get("w0", 1.0))
    if options.get("species_weights") is not None:
        sw = np.ascontiguousarray(options["species_weights"], dtype=np.float64)
        if sw.shape != (S,):
            raise ValueError("species_weights needs one value per species")
        keep.append(sw)
        o.species_weights = _ptr(sw, _f64p)
    o.compression = _COMPRESSION[options.get("compression", "off")]
    if options.get("polynomial") is not None:
        grid, weights, values = (np.ascontiguousarray(a, dtype=np.float64) for a in options["polynomial"])
        keep.extend([grid, weights, values])
        o.radial_basis = 1
        o.grid_size = len(grid)
        o.radial_grid = _ptr(grid, _f64p)
        o.radial_weights = _ptr(weights, _f64p)
        o.radial_values = _ptr(values.ravel(), _f64p)
    return ctypes.pointer(o)


_loaded: dict[str, Any] = {}


def build(reference_root: str | None = "/root/reference") -> None:
    """Compile the oracle (and the reference harness when its sources exist)."""

    targets = ["oracle"]
    if reference_root and Path(reference_root, "cpp", "src", "standalone", "soap.cpp").is_file():
        targets.append("ref")
    env = dict(os.environ)
    if reference_root:
        env["REF"] = reference_root
    subprocess.run(["make", "-s", "-C", str(HERE), *targets], check=True, env=env)


def _load(kind: str) -> Any:
    if kind in _loaded:
        return _loaded[kind]
    path = ORACLE_LIB if kind == "oracle" else REF_LIB
    if not path.is_file():
        if kind == "oracle":
            raise FileNotFoundError(f"oracle library is not built: {path} (run `make -C oracle`)")
        return None
    lib = ctypes.CDLL(str(path))
    if kind == "oracle":
        lib.mdxo_graph_build.restype = ctypes.c_int
        lib.mdxo_graph_build.argtypes = [
            _i32p, _f64p, _f64p, _i32p, _i64p, ctypes.c_int64, ctypes.c_int64,
            ctypes.c_double, ctypes.c_int, ctypes.POINTER(_Graph), ctypes.c_char_p, ctypes.c_int,
        ]
        lib.mdxo_graph_free.argtypes = [ctypes.POINTER(_Graph)]
        lib.mdxo_neighbor_list.restype = ctypes.c_int
        lib.mdxo_neighbor_list.argtypes = [
            _i32p, _f64p, _f64p, _i32p, _i64p, ctypes.c_int64, ctypes.c_int64,
            ctypes.c_double, ctypes.c_int, ctypes.c_int, ctypes.POINTER(_PairTable), ctypes.c_char_p, ctypes.c_int,
        ]
        lib.mdxo_pair_table_free.argtypes = [ctypes.POINTER(_PairTable)]
        lib.mdxo_soap.restype = ctypes.c_int
        lib.mdxo_soap.argtypes = [
            _i32p, _f64p, _f64p, _i32p, _i64p, ctypes.c_int64, ctypes.c_int64,
            _i32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_double, ctypes.c_double,
            _f64p, _f64p, ctypes.POINTER(_Options), ctypes.c_int, ctypes.c_int, ctypes.c_int, _f64p,
            ctypes.POINTER(ctypes.c_int32), ctypes.c_char_p, ctypes.c_int,
        ]
        lib.mdxo_solid_harmonics.restype = None
        lib.mdxo_solid_harmonics.argtypes = [
            ctypes.c_double, ctypes.c_double, ctypes.c_double, ctypes.c_int, _f64p,
        ]
        lib.mdxo_soap_feature_count.restype = ctypes.c_int64
        lib.mdxo_soap_feature_count.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int]
    else:
        lib.mdxr_graph_build.restype = ctypes.c_int
        lib.mdxr_graph_build.argtypes = [
            _i32p, _f64p, _f64p, _i32p, _i64p, ctypes.c_int64, ctypes.c_int64,
            ctypes.c_double, ctypes.c_int, ctypes.c_int, ctypes.POINTER(_Graph),
            ctypes.c_char_p, ctypes.c_int,
        ]
        lib.mdxr_graph_free.argtypes = [ctypes.POINTER(_Graph)]
        lib.mdxr_neighbor_list.restype = ctypes.c_int
        lib.mdxr_neighbor_list.argtypes = [
            _i32p, _f64p, _f64p, _i32p, _i64p, ctypes.c_int64, ctypes.c_int64,
            ctypes.c_double, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(_PairTable),
            ctypes.c_char_p, ctypes.c_int,
        ]
        lib.mdxr_pair_table_free.argtypes = [ctypes.POINTER(_PairTable)]
        lib.mdxr_soap.restype = ctypes.c_int
        lib.mdxr_soap.argtypes = [
            _i32p, _f64p, _f64p, _i32p, _i64p, ctypes.c_int64, ctypes.c_int64,
            _i32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_double, ctypes.c_double,
            _f64p, _f64p, ctypes.POINTER(_Options), ctypes.c_int, ctypes.c_int, _f64p, ctypes.c_char_p,
            ctypes.c_int,
        ]
    _loaded[kind] = lib
    return lib


def reference_available() -> bool:
    return _load("ref") is not None


def _ptr(array: np.ndarray, ctype: Any) -> Any:
    return array.ctypes.data_as(ctype)


def _batch_arrays(batch: Any) -> tuple[np.ndarray, ...]:
    numbers = np.ascontiguousarray(batch.numbers, dtype=np.int32)
    positions = np.ascontiguousarray(batch.positions, dtype=np.float64).reshape(-1, 3)
    cells = np.ascontiguousarray(batch.cells, dtype=np.float64).reshape(-1, 3, 3)
    pbc = np.ascontiguousarray(batch.pbc, dtype=np.int32).reshape(-1, 3)
    offsets = np.ascontiguousarray(batch.offsets, dtype=np.int64)
    return numbers, positions, cells, pbc, offsets


def graph(batch: Any, cutoff: float, *, include_boundary: bool = True, kind: str = "oracle",
          num_threads: int = 1) -> dict[str, np.ndarray]:
    """Neighbour graph of every structure: CSR with global atom indices."""

    lib = _load(kind)
    if lib is None:
        raise FileNotFoundError("reference harness is not built")
    numbers, positions, cells, pbc, offsets = _batch_arrays(batch)
    out = _Graph()
    err = ctypes.create_string_buffer(512)
    args = (
        _ptr(numbers, _i32p), _ptr(positions, _f64p), _ptr(cells, _f64p), _ptr(pbc, _i32p),
        _ptr(offsets, _i64p), len(offsets) - 1, len(numbers), float(cutoff), int(include_boundary),
    )
    if kind == "oracle":
        rc = lib.mdxo_graph_build(*args, ctypes.byref(out), err, 512)
        free = lib.mdxo_graph_free
    else:
        rc = lib.mdxr_graph_build(*args, int(num_threads), ctypes.byref(out), err, 512)
        free = lib.mdxr_graph_free
    if rc != 0:
        raise ValueError(err.value.decode())
    try:
        p = int(out.pairs)
        n = int(out.atoms)
        result = {
            "offsets": np.ctypeslib.as_array(out.offsets, shape=(n + 1,)).copy(),
            "atoms": np.ctypeslib.as_array(out.neighbors, shape=(max(p, 1),))[:p].copy(),
            "shifts": np.ctypeslib.as_array(out.shifts, shape=(max(3 * p, 1),))[: 3 * p].reshape(p, 3).copy(),
            "displacements": np.ctypeslib.as_array(out.disp, shape=(max(3 * p, 1),))[: 3 * p].reshape(p, 3).copy(),
            "distance2": np.ctypeslib.as_array(out.d2, shape=(max(p, 1),))[:p].copy(),
        }
    finally:
        free(ctypes.byref(out))
    return result


def neighbor_list(batch: Any, cutoff: float, *, full_neighbor_list: bool = True, self_pairs: bool = False,
                  kind: str = "oracle", num_threads: int = 1) -> tuple[np.ndarray, np.ndarray]:
    """NeighborList table of the batch: ``(values[rows, 9], offsets[structures + 1])``
    as ``_cpp.compute_neighbor_list`` returns it (cpp/src/bindings/module.cpp:772-798)."""

    lib = _load(kind)
    if lib is None:
        raise FileNotFoundError("reference harness is not built")
    numbers, positions, cells, pbc, offsets = _batch_arrays(batch)
    out = _PairTable()
    err = ctypes.create_string_buffer(512)
    args = (
        _ptr(numbers, _i32p), _ptr(positions, _f64p), _ptr(cells, _f64p), _ptr(pbc, _i32p),
        _ptr(offsets, _i64p), len(offsets) - 1, len(numbers), float(cutoff), int(bool(full_neighbor_list)),
        int(bool(self_pairs)),
    )
    if kind == "oracle":
        rc = lib.mdxo_neighbor_list(*args, ctypes.byref(out), err, 512)
        free = lib.mdxo_pair_table_free
    else:
        rc = lib.mdxr_neighbor_list(*args, int(num_threads), ctypes.byref(out), err, 512)
        free = lib.mdxr_pair_table_free
    if rc != 0:
        raise ValueError(err.value.decode())
    try:
        rows, structures = int(out.rows), int(out.structures)
        values = np.ctypeslib.as_array(out.values, shape=(rows * 9 + 1,))[: rows * 9].reshape(rows, 9).copy()
        table_offsets = np.ctypeslib.as_array(out.offsets, shape=(structures + 1,)).copy()
    finally:
        free(ctypes.byref(out))
    return values, table_offsets


_AVERAGE = {"off": 0, "inner": 1, "outer": 2}


def soap(batch: Any, *, species: Any, n_max: int, l_max: int, r_cut: float, sigma: float,
         alphas: np.ndarray | None = None, betas: np.ndarray | None = None, average: str = "off",
         num_threads: int = 0, decomposition: int = 0, kind: str = "oracle", cancel: Any = None,
         options: dict | None = None) -> np.ndarray:
    """SOAP features (float64, rows x features) from the oracle or the reference.

    ``options`` (see ``_options``) selects weighting, species weights,
    compression and the polynomial basis; None is the GTO default."""

    lib = _load(kind)
    if lib is None:
        raise FileNotFoundError("reference harness is not built")
    numbers, positions, cells, pbc, offsets = _batch_arrays(batch)
    species_arr = np.ascontiguousarray(species, dtype=np.int32)
    alphas = np.ascontiguousarray(alphas if alphas is not None else np.zeros(1), dtype=np.float64).ravel()
    betas = np.ascontiguousarray(betas if betas is not None else np.zeros(1), dtype=np.float64).ravel()
    S = len(species_arr)
    keep: list = []
    opt = _options(options, S, keep)
    features = feature_count(S, n_max, l_max, (options or {}).get("compression", "off"))
    structures = len(offsets) - 1
    rows = structures if average in ("inner", "outer") else len(numbers)
    output = np.zeros((rows, features), dtype=np.float64)
    err = ctypes.create_string_buffer(512)
    common = (
        _ptr(numbers, _i32p), _ptr(positions, _f64p), _ptr(cells, _f64p), _ptr(pbc, _i32p),
        _ptr(offsets, _i64p), structures, len(numbers), _ptr(species_arr, _i32p), S,
        int(n_max), int(l_max), float(r_cut), float(sigma), _ptr(alphas, _f64p), _ptr(betas, _f64p),
        opt, _AVERAGE[average], int(num_threads),
    )
    if kind == "oracle":
        flag = cancel if cancel is not None else None
        rc = lib.mdxo_soap(*common, int(decomposition), _ptr(output, _f64p), flag, err, 512)
    else:
        rc = lib.mdxr_soap(*common, _ptr(output, _f64p), err, 512)
    if rc == 4:
        raise RuntimeError("cancelled")
    if rc != 0:
        raise ValueError(err.value.decode())
    return output


def solid_harmonics(vector: Any, l_max: int) -> np.ndarray:
    lib = _load("oracle")
    out = np.zeros((l_max + 1) ** 2, dtype=np.float64)
    x, y, z = (float(v) for v in vector)
    lib.mdxo_solid_harmonics(x, y, z, int(l_max), _ptr(out, _f64p))
    return out
