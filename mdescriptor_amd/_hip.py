"""The HIP plugin: a ctypes binding of ``_lib/libmdx_hip.so``.

It mirrors the reference's CUDA plugin contract (``cpp/cuda/src/bindings.cu:
15-57``): ``create_backend(name, options) -> Backend`` with
``Backend.compute(batch, control) -> dict`` (``values``, ``level``,
``row_offsets``, ``labels``, ``metadata``, ``_mdescriptor_owned_values``),
``Backend.feature_count``, ``Backend.metadata()`` and ``Backend.close()``,
plus ``MODEL_SNAPSHOT_ABI``.  The library's C ABI is declared in
``include/mdx_hip.h``; ctypes releases the GIL around every call.

Errors map onto the reference's families (``src/mdescriptor/core/errors.py:
215-248``): a missing library or device raises :class:`HipUnavailable`
(an ``ImportError``), device allocation failure :class:`HipOutOfMemory`
(a ``MemoryError``), invalid input ``ValueError``, cancellation
:class:`HipCancelledError`.  There is no CPU fallback: without the built
library nothing here computes.
"""

from __future__ import annotations

import ctypes
import os
import threading
from collections.abc import Mapping
from pathlib import Path
from typing import Any

import numpy as np

MODEL_SNAPSHOT_ABI = 1
LIBRARY_PATH = Path(__file__).resolve().parent / "_lib" / "libmdx_hip.so"

MDX_OK = 0
MDX_INVALID_ARGUMENT = 1
MDX_OUT_OF_MEMORY = 2
MDX_DEVICE_UNAVAILABLE = 3
MDX_CANCELLED = 4
MDX_INTERNAL = 5


class HipUnavailable(ImportError):
    """The HIP library or a HIP device is not available."""


class HipOutOfMemory(MemoryError):
    """A device allocation failed."""


class HipCancelledError(RuntimeError):
    """The computation was cancelled through its control."""


class HipError(RuntimeError):
    """An internal failure of the HIP backend."""


_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_f64p = ctypes.POINTER(ctypes.c_double)


class BatchView(ctypes.Structure):
    _fields_ = [
        ("numbers", _i32p),
        ("positions", _f64p),
        ("cells", _f64p),
        ("pbc", _i32p),
        ("offsets", _i64p),
        ("structures", ctypes.c_int64),
        ("atoms", ctypes.c_int64),
    ]


class SoapOptions(ctypes.Structure):
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


class SoapParams(ctypes.Structure):
    _fields_ = [
        ("species", _i32p),
        ("n_species", ctypes.c_int32),
        ("n_max", ctypes.c_int32),
        ("l_max", ctypes.c_int32),
        ("r_cut", ctypes.c_double),
        ("sigma", ctypes.c_double),
        ("alphas", _f64p),
        ("betas", _f64p),
        ("average", ctypes.c_int32),
        ("out_dtype", ctypes.c_int32),
        ("options", ctypes.POINTER(SoapOptions)),
    ]


COMPRESSION_MODES = {"off": 0, "mu2": 1, "mu1nu1": 2, "crossover": 3}
WEIGHTING_FUNCTIONS = {"poly": 1, "pow": 2, "exp": 3}


def soap_options(options: dict | None, n_species: int, keep: list) -> Any:
    """A SoapOptions pointer (None for the defaults) from
    ``{"weighting": {function, r0, c, d, m, w0}, "species_weights": [...],
    "compression": "off"|"mu2"|"mu1nu1"|"crossover",
    "polynomial": (grid, weights, values)}``, the fields SoapKernel fills
    (core.py:241-270).  ``keep`` receives the arrays the struct points to."""

    if not options:
        return None
    o = SoapOptions()
    weighting = dict(options.get("weighting") or {})
    if weighting.get("function") is not None:
        o.weighting_function = WEIGHTING_FUNCTIONS[str(weighting["function"])]
    o.weighting_has_w0 = 1 if "w0" in weighting else 0
    o.weighting_r0 = float(weighting.get("r0", 1.0))
    o.weighting_c = float(weighting.get("c", 1.0))
    o.weighting_d = float(weighting.get("d", 0.0))
    o.weighting_m = float(weighting.get("m", 1.0))
    o.weighting_w0 = float(weighting.get("w0", 1.0))
    if options.get("species_weights") is not None:
        weights = np.ascontiguousarray(options["species_weights"], dtype=np.float64)
        if weights.shape != (n_species,):
            raise ValueError("species_weights needs one value per species")
        keep.append(weights)
        o.species_weights = weights.ctypes.data_as(_f64p)
    o.compression = COMPRESSION_MODES[str(options.get("compression", "off"))]
    if options.get("polynomial") is not None:
        grid, weights, values = (np.ascontiguousarray(a, dtype=np.float64) for a in options["polynomial"])
        keep.extend([grid, weights, values])
        o.radial_basis = 1
        o.grid_size = int(grid.shape[0])
        o.radial_grid = grid.ctypes.data_as(_f64p)
        o.radial_weights = weights.ctypes.data_as(_f64p)
        o.radial_values = values.ctypes.data_as(_f64p)
    keep.append(o)
    return ctypes.pointer(o)


class Timing(ctypes.Structure):
    _fields_ = [
        ("graph_ms", ctypes.c_double),
        ("expansion_ms", ctypes.c_double),
        ("finalize_ms", ctypes.c_double),
        ("total_ms", ctypes.c_double),
        ("h2d_ms", ctypes.c_double),
        ("d2h_ms", ctypes.c_double),
        ("pairs", ctypes.c_int64),
        ("binned", ctypes.c_int64),
        ("expansion_launches", ctypes.c_int64),
        ("expansion_tiles", ctypes.c_int64),
    ]

    def as_dict(self) -> dict[str, float]:
        return {name: getattr(self, name) for name, _ in self._fields_}


# Every symbol include/mdx_hip.h declares, with its ctypes signature.
class ListTiming(ctypes.Structure):
    """mdx_list_timing: device stage times of the last neighbour list."""

    _fields_ = [
        ("graph_ms", ctypes.c_double),
        ("count_ms", ctypes.c_double),
        ("fill_ms", ctypes.c_double),
        ("graph_pairs", ctypes.c_int64),
        ("pairs", ctypes.c_int64),
        ("binned", ctypes.c_int64),
    ]

    def as_dict(self) -> dict[str, float]:
        return {name: float(getattr(self, name)) for name, _ in self._fields_}


SIGNATURES: dict[str, tuple[Any, list[Any]]] = {
    "mdx_hip_create": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(ctypes.c_void_p)]),
    "mdx_hip_destroy": (None, [ctypes.c_void_p]),
    "mdx_hip_last_error": (ctypes.c_char_p, [ctypes.c_void_p]),
    "mdx_hip_soap_plan_create": (
        ctypes.c_int,
        [ctypes.c_void_p, ctypes.POINTER(SoapParams), ctypes.POINTER(ctypes.c_void_p), _i64p],
    ),
    "mdx_hip_soap_plan_destroy": (None, [ctypes.c_void_p]),
    "mdx_hip_soap_rows": (ctypes.c_int64, [ctypes.c_void_p, ctypes.POINTER(BatchView)]),
    "mdx_hip_soap_compute": (
        ctypes.c_int,
        [ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(BatchView), ctypes.c_void_p, ctypes.c_int64,
         ctypes.c_int64, _i32p, ctypes.POINTER(Timing)],
    ),
    "mdx_hip_batch_upload": (
        ctypes.c_int,
        [ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(BatchView), ctypes.POINTER(ctypes.c_void_p)],
    ),
    "mdx_hip_batch_destroy": (None, [ctypes.c_void_p]),
    "mdx_hip_batch_set_positions": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]),
    "mdx_hip_soap_run": (
        ctypes.c_int,
        [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, _i32p,
         ctypes.POINTER(Timing)],
    ),
    "mdx_hip_soap_run_noalloc": (
        ctypes.c_int,
        [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, _i32p,
         ctypes.POINTER(Timing)],
    ),
    "mdx_hip_soap_run_frame": (
        ctypes.c_int,
        [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
         _i32p],
    ),
    "mdx_hip_batch_wait": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
    "mdx_hip_neighbors_build": (
        ctypes.c_int,
        [ctypes.c_void_p, ctypes.POINTER(BatchView), ctypes.c_double, ctypes.c_int32, _i64p],
    ),
    "mdx_hip_neighbors_fetch": (
        ctypes.c_int,
        [ctypes.c_void_p, _i64p, _i32p, _i32p, _f64p, _f64p],
    ),
    "mdx_hip_neighbor_list": (
        ctypes.c_int,
        [ctypes.c_void_p, ctypes.POINTER(BatchView), ctypes.c_double, ctypes.c_int32, ctypes.c_int32, _i32p, _i64p],
    ),
    "mdx_hip_neighbor_list_fetch": (
        ctypes.c_int,
        [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p],
    ),
    "mdx_hip_neighbor_list_timing": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ListTiming)]),
    "mdx_hip_host_alloc": (ctypes.c_int, [ctypes.c_size_t, ctypes.POINTER(ctypes.c_void_p)]),
    "mdx_hip_host_free": (None, [ctypes.c_void_p]),
    "mdx_hip_version": (ctypes.c_char_p, []),
}

_lock = threading.Lock()
_library: Any = None


def load_library() -> Any:
    """Load the in-tree HIP library, or raise :class:`HipUnavailable`."""

    global _library
    with _lock:
        if _library is not None:
            return _library
        if not LIBRARY_PATH.is_file():
            raise HipUnavailable(
                f"the HIP SOAP library is not built ({LIBRARY_PATH}); run `python -m mdescriptor_amd.build`"
            )
        try:
            lib = ctypes.CDLL(str(LIBRARY_PATH))
        except OSError as exc:
            raise HipUnavailable(f"cannot load {LIBRARY_PATH.name}: {exc}") from exc
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _library = lib
        return lib


def _raise_for(status: int, message: str) -> None:
    if status == MDX_OK:
        return
    if status == MDX_INVALID_ARGUMENT:
        raise ValueError(message or "invalid argument")
    if status == MDX_OUT_OF_MEMORY:
        raise HipOutOfMemory(message or "HIP backend ran out of memory")
    if status == MDX_DEVICE_UNAVAILABLE:
        raise HipUnavailable(message or "HIP device unavailable")
    if status == MDX_CANCELLED:
        raise HipCancelledError(message or "descriptor computation was cancelled")
    raise HipError(message or f"HIP backend failed with status {status}")


class _BatchArrays:
    """C-contiguous copies of a batch's five arrays and the ctypes view on them."""

    def __init__(self, batch: Any) -> None:
        self.numbers = np.ascontiguousarray(batch.numbers, dtype=np.int32)
        self.positions = np.ascontiguousarray(batch.positions, dtype=np.float64).reshape(-1, 3)
        self.cells = np.ascontiguousarray(batch.cells, dtype=np.float64).reshape(-1, 3, 3)
        self.pbc = np.ascontiguousarray(batch.pbc, dtype=np.int32).reshape(-1, 3)
        self.offsets = np.ascontiguousarray(batch.offsets, dtype=np.int64)
        self.view = BatchView(
            self.numbers.ctypes.data_as(_i32p),
            self.positions.ctypes.data_as(_f64p),
            self.cells.ctypes.data_as(_f64p),
            self.pbc.ctypes.data_as(_i32p),
            self.offsets.ctypes.data_as(_i64p),
            len(self.offsets) - 1,
            len(self.numbers),
        )


class Context:
    """One HIP device context (stream, device arena, pinned staging)."""

    def __init__(self, device: int = 0) -> None:
        self.lib = load_library()
        handle = ctypes.c_void_p()
        status = self.lib.mdx_hip_create(int(device), ctypes.byref(handle))
        _raise_for(status, (self.lib.mdx_hip_last_error(None) or b"").decode())
        self.handle = handle
        self.device = int(device)

    def check(self, status: int) -> None:
        if status != MDX_OK:
            _raise_for(status, (self.lib.mdx_hip_last_error(self.handle) or b"").decode())

    def close(self) -> None:
        if getattr(self, "handle", None) is not None and self.handle.value:
            self.lib.mdx_hip_destroy(self.handle)
        self.handle = None

    def __del__(self) -> None:  # pragma: no cover - interpreter shutdown order
        try:
            self.close()
        except Exception:
            pass


class PinnedPool:
    """Page-locked host blocks for result matrices, reused across calls.

    A result written into pinned memory arrives with one DMA at the PCIe rate
    (pageable destinations are staged by the library).  Pinning costs a few
    milliseconds per gigabyte, so released blocks are kept, up to
    ``cache_bytes`` in total, and handed out again to requests of at least
    half their size.
    """

    GRAIN = 2 << 20

    def __init__(self, cache_bytes: int = 4 << 30) -> None:
        self.cache_bytes = int(cache_bytes)
        self._free: list[tuple[int, int]] = []  # (size, address)
        self._cached = 0
        self._lock = threading.Lock()

    def acquire(self, nbytes: int) -> tuple[int, int] | None:
        size = max(self.GRAIN, -(-int(nbytes) // self.GRAIN) * self.GRAIN)
        with self._lock:
            best = None
            for i, (have, address) in enumerate(self._free):
                if size <= have <= 2 * size and (best is None or have < self._free[best][0]):
                    best = i
            if best is not None:
                have, address = self._free.pop(best)
                self._cached -= have
                return address, have
        lib = load_library()
        pointer = ctypes.c_void_p()
        if lib.mdx_hip_host_alloc(size, ctypes.byref(pointer)) != MDX_OK or not pointer.value:
            return None
        return int(pointer.value), size

    def release(self, address: int, size: int) -> None:
        with self._lock:
            if self._cached + size <= self.cache_bytes:
                self._free.append((size, address))
                self._cached += size
                return
        load_library().mdx_hip_host_free(ctypes.c_void_p(address))

    def clear(self) -> None:
        with self._lock:
            blocks, self._free, self._cached = self._free, [], 0
        for _, address in blocks:
            load_library().mdx_hip_host_free(ctypes.c_void_p(address))


class _PinnedArrayBase:
    """Owner of one pinned block, exposed to NumPy through the array interface;
    the block returns to the pool when the last array viewing it is gone."""

    def __init__(self, pool: PinnedPool, address: int, size: int, shape: tuple[int, ...], dtype: np.dtype) -> None:
        self._pool, self._address, self._size = pool, address, size
        self.__array_interface__ = {"shape": shape, "typestr": dtype.str, "data": (address, False), "version": 3}

    def __del__(self) -> None:  # pragma: no cover - runs at garbage collection
        try:
            self._pool.release(self._address, self._size)
        except Exception:
            pass


pinned_pool = PinnedPool(int(os.environ.get("MDX_HIP_PINNED_CACHE_MB", "4096")) << 20)


def pinned_empty(shape: tuple[int, ...], dtype: Any) -> np.ndarray:
    """Uninitialised C-contiguous array in page-locked host memory (pageable
    memory when pinning fails or the array is empty)."""

    dtype = np.dtype(dtype)
    shape = tuple(int(v) for v in shape)
    nbytes = int(np.prod(shape, dtype=np.int64)) * dtype.itemsize
    if nbytes == 0:
        return np.empty(shape, dtype=dtype)
    block = pinned_pool.acquire(nbytes)
    if block is None:
        return np.empty(shape, dtype=dtype)
    return np.asarray(_PinnedArrayBase(pinned_pool, block[0], block[1], shape, dtype))


def is_pinned(array: np.ndarray) -> bool:
    base = array
    while isinstance(base, np.ndarray):
        base = base.base
    return isinstance(base, _PinnedArrayBase)


class SoapPlan:
    """Device-resident SOAP plan on a context."""

    def __init__(self, context: Context, *, species: Any, n_max: int, l_max: int, r_cut: float, sigma: float,
                 alphas: np.ndarray | None, betas: np.ndarray | None, average: str, dtype: str,
                 options: dict | None = None) -> None:
        self.context = context
        self._species = np.ascontiguousarray(species, dtype=np.int32)
        self._alphas = np.ascontiguousarray(alphas if alphas is not None else np.zeros(1), dtype=np.float64).ravel()
        self._betas = np.ascontiguousarray(betas if betas is not None else np.zeros(1), dtype=np.float64).ravel()
        self.average = str(average)
        self.dtype = np.dtype(dtype)
        self._keep: list = []
        opt = soap_options(options, len(self._species), self._keep)
        params = SoapParams(
            self._species.ctypes.data_as(_i32p), len(self._species), int(n_max), int(l_max), float(r_cut),
            float(sigma), self._alphas.ctypes.data_as(_f64p) if alphas is not None else None,
            self._betas.ctypes.data_as(_f64p) if betas is not None else None,
            {"off": 0, "inner": 1, "outer": 2}[self.average], int(self.dtype.itemsize), opt,
        )
        handle = ctypes.c_void_p()
        features = ctypes.c_int64()
        context.check(context.lib.mdx_hip_soap_plan_create(context.handle, ctypes.byref(params),
                                                           ctypes.byref(handle), ctypes.byref(features)))
        self.handle = handle
        self.features = int(features.value)

    def rows(self, batch: Any) -> int:
        return (len(batch.offsets) - 1) if self.average != "off" else len(batch.numbers)

    def compute(self, batch: Any, cancel: ctypes.c_int32 | None = None,
                out: np.ndarray | None = None) -> tuple[np.ndarray, dict[str, float]]:
        """Compute one batch into ``out`` (allocated when None), a C-contiguous
        ``(rows, features)`` array of the plan's dtype."""

        arrays = _BatchArrays(batch)
        rows = self.rows(batch)
        if out is None:
            out = pinned_empty((rows, self.features), self.dtype)
        elif (out.shape != (rows, self.features) or out.dtype != self.dtype or not out.flags.c_contiguous
              or not out.flags.writeable):
            raise ValueError(f"output must be a writable C-contiguous {self.dtype} array of shape "
                             f"({rows}, {self.features})")
        timing = Timing()
        flag = ctypes.pointer(cancel) if cancel is not None else None
        lib = self.context.lib
        self.context.check(lib.mdx_hip_soap_compute(
            self.context.handle, self.handle, ctypes.byref(arrays.view), out.ctypes.data_as(ctypes.c_void_p),
            rows, out.strides[0] if rows > 0 else self.features * self.dtype.itemsize, flag, ctypes.byref(timing)))
        return out, timing.as_dict()

    def close(self) -> None:
        if getattr(self, "handle", None) is not None and self.handle.value:
            self.context.lib.mdx_hip_soap_plan_destroy(self.handle)
        self.handle = None

    def __del__(self) -> None:  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass


class DeviceBatch:
    """A batch validated, prepared and resident in HBM for one plan."""

    def __init__(self, plan: SoapPlan, batch: Any) -> None:
        self.plan = plan
        self.arrays = _BatchArrays(batch)
        self.rows = plan.rows(batch)
        ctx = plan.context
        handle = ctypes.c_void_p()
        ctx.check(ctx.lib.mdx_hip_batch_upload(ctx.handle, plan.handle, ctypes.byref(self.arrays.view),
                                               ctypes.byref(handle)))
        self.handle = handle

    def set_positions(self, positions: Any) -> None:
        """New positions for the resident batch (a new frame of the same
        system): a host array of shape (atoms, 3), or the device address (an
        int) of atoms * 3 float64 values.  Everything that depends on
        positions is rebuilt on the device by the next :meth:`run`."""

        ctx = self.plan.context
        if isinstance(positions, int):
            address = ctypes.c_void_p(positions)
            keep = None
        else:
            keep = np.ascontiguousarray(positions, dtype=np.float64)
            if keep.size != 3 * len(self.arrays.numbers):
                raise ValueError("positions must hold atoms * 3 values")
            address = keep.ctypes.data_as(ctypes.c_void_p)
        ctx.check(ctx.lib.mdx_hip_batch_set_positions(ctx.handle, self.handle, address))
        del keep

    def run(self, out_device_ptr: int, pitch_bytes: int, cancel: ctypes.c_int32 | None = None) -> dict[str, float]:
        ctx = self.plan.context
        timing = Timing()
        flag = ctypes.pointer(cancel) if cancel is not None else None
        ctx.check(ctx.lib.mdx_hip_soap_run(ctx.handle, self.plan.handle, self.handle, ctypes.c_void_p(out_device_ptr),
                                           int(pitch_bytes), flag, ctypes.byref(timing)))
        return timing.as_dict()

    def run_frame(self, positions: Any, out_device_ptr: int, pitch_bytes: int,
                  cancel: ctypes.c_int32 | None = None) -> None:
        """One trajectory frame without waiting for it: new positions (a host
        array of shape (atoms, 3), or the device address of atoms * 3 float64
        values) and the descriptors of them into out_device_ptr.  The output
        is complete after :meth:`wait`; the next frame's graph is built while
        this frame's search and expansion run."""

        ctx = self.plan.context
        if isinstance(positions, int):
            address = ctypes.c_void_p(positions)
            keep = None
        else:
            keep = np.ascontiguousarray(positions, dtype=np.float64)
            if keep.size != 3 * len(self.arrays.numbers):
                raise ValueError("positions must hold atoms * 3 values")
            address = keep.ctypes.data_as(ctypes.c_void_p)
        flag = ctypes.pointer(cancel) if cancel is not None else None
        ctx.check(ctx.lib.mdx_hip_soap_run_frame(ctx.handle, self.plan.handle, self.handle, address,
                                                 ctypes.c_void_p(out_device_ptr), int(pitch_bytes), flag))
        del keep

    def wait(self) -> None:
        """Settle and wait for the frames queued by :meth:`run_frame`."""

        ctx = self.plan.context
        ctx.check(ctx.lib.mdx_hip_batch_wait(ctx.handle, self.handle))

    def close(self) -> None:
        if getattr(self, "handle", None) is not None and self.handle.value:
            self.plan.context.lib.mdx_hip_batch_destroy(self.handle)
        self.handle = None

    def __del__(self) -> None:  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass


class DeviceArray:
    """Address, shape, dtype, row pitch and device of a caller's 2-D device
    array: a torch tensor on a HIP device, or any object exposing
    ``__cuda_array_interface__`` (taken to live on device 0).  Rows may be
    pitched; elements inside a row must be contiguous."""

    def __init__(self, out: Any) -> None:
        module = type(out).__module__
        if module.startswith("torch"):
            if not getattr(out, "is_cuda", False):
                raise ValueError("the output tensor must live on a HIP device")
            if out.dim() != 2 or (out.shape[0] > 0 and out.shape[1] > 1 and out.stride(1) != 1):
                raise ValueError("the output tensor must be two-dimensional with contiguous rows")
            names = {"torch.float32": "float32", "torch.float64": "float64"}
            if str(out.dtype) not in names:
                raise ValueError(f"unsupported output tensor dtype {out.dtype}")
            self.dtype = np.dtype(names[str(out.dtype)])
            self.shape = (int(out.shape[0]), int(out.shape[1]))
            self.address = int(out.data_ptr())
            self.pitch = int(out.stride(0)) * self.dtype.itemsize if self.shape[0] > 1 else \
                self.shape[1] * self.dtype.itemsize
            self.device = int(out.device.index or 0)
            self.torch_stream_owner = out
            return
        interface = getattr(out, "__cuda_array_interface__", None)
        if interface is None:
            raise ValueError("the output must be a torch tensor on a HIP device or expose __cuda_array_interface__")
        shape = tuple(int(v) for v in interface["shape"])
        if len(shape) != 2:
            raise ValueError("the output array must be two-dimensional")
        address, readonly = interface["data"]
        if readonly:
            raise ValueError("the output array is read-only")
        self.dtype = np.dtype(interface["typestr"])
        self.shape = shape
        self.address = int(address)
        strides = interface.get("strides")
        if strides is None:
            self.pitch = shape[1] * self.dtype.itemsize
        else:
            if shape[0] > 0 and shape[1] > 1 and int(strides[1]) != self.dtype.itemsize:
                raise ValueError("the output array's rows must be contiguous")
            self.pitch = int(strides[0]) if shape[0] > 1 else shape[1] * self.dtype.itemsize
        self.device = 0
        self.torch_stream_owner = None

    def check(self, rows: int, features: int, dtype: Any) -> None:
        if self.shape != (rows, features):
            raise ValueError(f"the output array must have shape ({rows}, {features}), not {self.shape}")
        if self.dtype != np.dtype(dtype):
            raise ValueError(f"the output array must be {np.dtype(dtype)}, not {self.dtype}")
        if rows > 0 and self.pitch < features * self.dtype.itemsize:
            raise ValueError("the output array's rows overlap")
        if self.device != 0:
            raise ValueError("the HIP backend computes on device 0")

    def settle(self) -> None:
        """Wait for work a torch stream may still have queued on the array."""

        if self.torch_stream_owner is not None:
            import torch

            torch.cuda.current_stream(self.torch_stream_owner.device).synchronize()


def neighbor_graph(context: Context, batch: Any, cutoff: float, *, include_boundary: bool = True
                   ) -> dict[str, np.ndarray]:
    """Device neighbour graph in the layout of ``_native.build_neighbor_graph``
    (``cpp/src/bindings/module.cpp:887-935``): offsets, atoms, shifts,
    displacements, distance2 — over every structure of the batch."""

    arrays = _BatchArrays(batch)
    lib = context.lib
    pairs = ctypes.c_int64()
    context.check(lib.mdx_hip_neighbors_build(context.handle, ctypes.byref(arrays.view), float(cutoff),
                                              1 if include_boundary else 0, ctypes.byref(pairs)))
    p = int(pairs.value)
    n = len(arrays.numbers)
    offsets = np.zeros(n + 1, dtype=np.int64)
    atoms = np.zeros(max(p, 1), dtype=np.int32)
    shifts = np.zeros((max(p, 1), 3), dtype=np.int32)
    disp = np.zeros((max(p, 1), 3), dtype=np.float64)
    d2 = np.zeros(max(p, 1), dtype=np.float64)
    context.check(lib.mdx_hip_neighbors_fetch(
        context.handle, offsets.ctypes.data_as(_i64p), atoms.ctypes.data_as(_i32p), shifts.ctypes.data_as(_i32p),
        disp.ctypes.data_as(_f64p), d2.ctypes.data_as(_f64p)))
    return {
        "offsets": offsets,
        "atoms": atoms[:p],
        "shifts": shifts[:p],
        "displacements": disp[:p],
        "distance2": d2[:p],
    }


def neighbor_list(context: Context, batch: Any, cutoff: float, *, full_neighbor_list: bool = True,
                  self_pairs: bool = False, cancel: ctypes.c_int32 | None = None, table: bool = False,
                  values: bool = True, samples: bool = True) -> dict[str, np.ndarray]:
    """NeighborList of a batch on the device (``mdx_hip_neighbor_list``).

    Returns ``offsets`` (first pair of each structure) and, as asked,
    ``table`` (rows x 9, the layout of ``_cpp.compute_neighbor_list``,
    ``cpp/src/bindings/module.cpp:772-798``), ``values`` (rows x 4: dx, dy,
    dz, distance) and ``samples`` (rows x 6: structure, local centre, local
    neighbour, cell shifts), the last two in page-locked memory."""

    arrays = _BatchArrays(batch)
    lib = context.lib
    rows = ctypes.c_int64()
    flag = ctypes.pointer(cancel) if cancel is not None else None
    context.check(lib.mdx_hip_neighbor_list(context.handle, ctypes.byref(arrays.view), float(cutoff),
                                            1 if full_neighbor_list else 0, 1 if self_pairs else 0, flag,
                                            ctypes.byref(rows)))
    n = int(rows.value)
    result: dict[str, np.ndarray] = {"offsets": np.zeros(len(arrays.offsets), dtype=np.int64)}
    if table:
        result["table"] = pinned_empty((n, 9), np.float64)
    if values:
        result["values"] = pinned_empty((n, 4), np.float64)
    if samples:
        result["samples"] = pinned_empty((n, 6), np.int64)

    def address(key: str) -> Any:
        array = result.get(key)
        return None if array is None or array.size == 0 else array.ctypes.data_as(ctypes.c_void_p)

    context.check(lib.mdx_hip_neighbor_list_fetch(context.handle, address("table"), address("values"),
                                                  address("samples"), address("offsets")))
    return result


def neighbor_list_timing(context: Context) -> dict[str, float]:
    """Stage times of the context's last neighbour list (``mdx_hip_neighbor_list_timing``)."""

    timing = ListTiming()
    context.check(context.lib.mdx_hip_neighbor_list_timing(context.handle, ctypes.byref(timing)))
    return timing.as_dict()


_contexts: dict[int, Context] = {}


def shared_context(device: int = 0) -> Context:
    """Process-wide context per device, created on first use."""

    with _lock:
        ctx = _contexts.get(device)
    if ctx is None:
        ctx = Context(device)
        with _lock:
            _contexts.setdefault(device, ctx)
            ctx = _contexts[device]
    return ctx


class Backend:
    """SOAP on one HIP device, created lazily by :func:`create_backend`."""

    def __init__(self, name: str, options: Mapping[str, Any]) -> None:
        if name != "SOAP":
            raise ValueError(f"the HIP backend implements SOAP only, not {name!r}")
        payload = options.get("_hip_payload")
        if not isinstance(payload, Mapping):
            raise ValueError("SOAP HIP backend requires the private _hip_payload")
        radial = payload["radial_basis"]
        if "alphas" not in radial and "radial_grid" not in radial:
            raise ValueError("the SOAP payload carries neither a GTO nor a polynomial radial basis")
        self.name = name
        self.options = dict(options)
        self._labels = tuple(options.get("_hip_labels") or payload.get("labels") or ())
        output = options.get("output") or {}
        self._dtype = output.get("dtype", "float64") if isinstance(output, Mapping) else getattr(output, "dtype", "float64")
        execution = options.get("execution") or {}
        num_threads = execution.get("num_threads") if isinstance(execution, Mapping) else getattr(execution, "num_threads", None)
        self._num_threads = num_threads
        self._average = str(options.get("average", "inner"))
        self._context = shared_context(0)
        species = [int(z) for z in options["species"]]
        self._plan = SoapPlan(
            self._context, species=species, n_max=int(options["n_max"]), l_max=int(options["l_max"]),
            r_cut=float(options["r_cut"]), sigma=float(options.get("sigma", 1.0)),
            alphas=np.asarray(radial["alphas"]) if "alphas" in radial else None,
            betas=np.asarray(radial["betas"]) if "betas" in radial else None, average=self._average,
            dtype=self._dtype, options=plan_options(options, species, radial),
        )
        self._lock = threading.Lock()
        self._closed = False
        self.last_timing: dict[str, float] = {}

    @property
    def feature_count(self) -> int:
        return self._plan.features

    def metadata(self) -> dict[str, Any]:
        return {
            "descriptor": self.name,
            "backend": "mdescriptor-hip",
            "execution": {"device": "hip", "num_threads": self._num_threads},
        }

    def compute(self, batch: Any, control: Any = None, out: np.ndarray | None = None) -> dict[str, Any]:
        with self._lock:
            if self._closed:
                raise RuntimeError("HIP backend is closed")
            flag = getattr(control, "_hip_cancel_flag", None) if control is not None else None
            values, timing = self._plan.compute(batch, flag, out)
            self.last_timing = timing
            level = "structure" if self._average in ("inner", "outer") else "atom"
            result: dict[str, Any] = {
                "values": values,
                "level": level,
                "labels": self._labels,
                "metadata": self.metadata(),
                "_mdescriptor_owned_values": True,
            }
            if level == "atom":
                result["row_offsets"] = np.asarray(batch.offsets, dtype=np.int64).copy()
            return result

    def compute_into(self, batch: Any, address: int, pitch: int, control: Any = None) -> dict[str, float]:
        """Compute one batch into device memory at ``address`` (rows of
        ``pitch`` bytes) through the device-resident path: no host copy of
        the values."""

        with self._lock:
            if self._closed:
                raise RuntimeError("HIP backend is closed")
            flag = getattr(control, "_hip_cancel_flag", None) if control is not None else None
            device_batch = DeviceBatch(self._plan, batch)
            try:
                timing = device_batch.run(address, pitch, flag)
            finally:
                device_batch.close()
            self.last_timing = timing
            return timing

    def close(self) -> None:
        with self._lock:
            if not self._closed:
                self._plan.close()
            self._closed = True


class NeighborListBackend:
    """NeighborList on one HIP device, the counterpart of the CUDA plugin's
    NeighborList branch (``cpp/cuda/src/backend.cu:358-471``): pair-level
    values (dx, dy, dz, distance), per-structure row offsets and, instead of
    the raw pair records, the pair samples already in the public
    ``[structure, local_i, local_j, sa, sb, sc]`` form."""

    feature_count = 4
    labels = ("dx", "dy", "dz", "distance")

    def __init__(self, name: str, options: Mapping[str, Any]) -> None:
        self.name = name
        self.options = dict(options)
        self.cutoff = float(options.get("cutoff", 6.0))
        self.full_neighbor_list = bool(options.get("full_neighbor_list", True))
        self.self_pairs = bool(options.get("self_pairs", False))
        execution = options.get("execution") or {}
        self._num_threads = (execution.get("num_threads") if isinstance(execution, Mapping)
                             else getattr(execution, "num_threads", None))
        self._context = shared_context(0)
        self._lock = threading.Lock()
        self._closed = False
        self.last_timing: dict[str, float] = {}

    def metadata(self) -> dict[str, Any]:
        return {
            "descriptor": self.name,
            "backend": "mdescriptor-hip",
            "execution": {"device": "hip", "num_threads": self._num_threads},
        }

    def compute(self, batch: Any, control: Any = None, out: np.ndarray | None = None) -> dict[str, Any]:
        if out is not None:
            raise ValueError("the NeighborList backend allocates its own pair-level output")
        with self._lock:
            if self._closed:
                raise RuntimeError("HIP backend is closed")
            flag = getattr(control, "_hip_cancel_flag", None) if control is not None else None
            raw = neighbor_list(self._context, batch, self.cutoff, full_neighbor_list=self.full_neighbor_list,
                                self_pairs=self.self_pairs, cancel=flag)
            return {
                "values": raw["values"],
                "level": "pair",
                "row_offsets": raw["offsets"],
                "samples": raw["samples"],
                "labels": self.labels,
                "metadata": self.metadata(),
                "_mdescriptor_owned_values": True,
            }

    def close(self) -> None:
        with self._lock:
            self._closed = True


def plan_options(options: Mapping[str, Any], species: list[int], radial: Mapping[str, Any]) -> dict | None:
    """The SoapPlan options of a backend configuration: the canonical
    ``weighting`` mapping, ``compression`` (mode and ``species_weighting``,
    a mapping from atomic number to weight) and the polynomial basis arrays of
    the payload, mapped as SoapKernel._ensure_native maps them
    (core.py:241-270).  None for the GTO / uncompressed / unweighted default."""

    weighting = dict(options.get("weighting") or {})
    compression = dict(options.get("compression") or {})
    mode = str(compression.get("mode", "off"))
    species_weighting = compression.get("species_weighting")
    species_weights = None
    if species_weighting is not None:
        keys = {int(k) for k in species_weighting}
        if keys != set(species):
            raise ValueError("species_weighting must contain exactly the configured species")
        by_number = {int(k): float(v) for k, v in species_weighting.items()}
        species_weights = [by_number[z] for z in species]
    result: dict[str, Any] = {}
    if weighting:
        result["weighting"] = weighting
    if species_weights is not None:
        result["species_weights"] = species_weights
    if mode != "off":
        result["compression"] = mode
    if "radial_grid" in radial:
        result["polynomial"] = (np.asarray(radial["radial_grid"]), np.asarray(radial["radial_weights"]),
                                np.asarray(radial["radial_values"]))
    return result or None


def create_backend(name: str, options: Mapping[str, Any]) -> Backend | NeighborListBackend:
    """Plugin factory, the counterpart of ``_cuda.create_backend`` (bindings.cu:30-40)."""

    if name == "NeighborList":
        return NeighborListBackend(name, options)
    return Backend(name, options)


def version() -> str:
    return load_library().mdx_hip_version().decode()


__all__ = [
    "Backend",
    "Context",
    "DeviceArray",
    "DeviceBatch",
    "HipCancelledError",
    "HipError",
    "HipOutOfMemory",
    "HipUnavailable",
    "MODEL_SNAPSHOT_ABI",
    "NeighborListBackend",
    "SoapPlan",
    "create_backend",
    "load_library",
    "neighbor_graph",
    "neighbor_list",
    "neighbor_list_timing",
    "shared_context",
]


class DeviceMemory:
    """Raw device allocation through the HIP runtime (for device-resident
    outputs in benchmarks and tests; the library itself never needs it)."""

    _runtime: Any = None

    @classmethod
    def runtime(cls) -> Any:
        if cls._runtime is None:
            load_library()  # the runtime is a dependency of the library
            rt = ctypes.CDLL("libamdhip64.so")
            rt.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
            rt.hipMalloc.restype = ctypes.c_int
            rt.hipFree.argtypes = [ctypes.c_void_p]
            rt.hipFree.restype = ctypes.c_int
            rt.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
            rt.hipMemcpy.restype = ctypes.c_int
            rt.hipDeviceSynchronize.argtypes = []
            rt.hipDeviceSynchronize.restype = ctypes.c_int
            rt.hipSetDevice.argtypes = [ctypes.c_int]
            rt.hipSetDevice.restype = ctypes.c_int
            cls._runtime = rt
        return cls._runtime

    def __init__(self, nbytes: int, device: int = 0) -> None:
        rt = self.runtime()
        if rt.hipSetDevice(int(device)) != 0:
            raise HipUnavailable("hipSetDevice failed")
        ptr = ctypes.c_void_p()
        if rt.hipMalloc(ctypes.byref(ptr), max(1, int(nbytes))) != 0:
            raise HipOutOfMemory(f"hipMalloc of {nbytes} bytes failed")
        self.ptr = ptr
        self.nbytes = int(nbytes)

    @property
    def address(self) -> int:
        return int(self.ptr.value or 0)

    def to_host(self, out: np.ndarray) -> np.ndarray:
        if out.nbytes > self.nbytes:
            raise ValueError("host buffer larger than the device allocation")
        if self.runtime().hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), self.ptr, out.nbytes, 2) != 0:
            raise HipError("hipMemcpy device-to-host failed")
        return out

    def from_host(self, array: np.ndarray) -> "DeviceMemory":
        data = np.ascontiguousarray(array)
        if data.nbytes > self.nbytes:
            raise ValueError("host array larger than the device allocation")
        if self.runtime().hipMemcpy(self.ptr, data.ctypes.data_as(ctypes.c_void_p), data.nbytes, 1) != 0:
            raise HipError("hipMemcpy host-to-device failed")
        return self

    @classmethod
    def synchronize(cls) -> None:
        if cls.runtime().hipDeviceSynchronize() != 0:
            raise HipError("hipDeviceSynchronize failed")

    def free(self) -> None:
        if getattr(self, "ptr", None) is not None and self.ptr.value:
            self.runtime().hipFree(self.ptr)
        self.ptr = None

    def __del__(self) -> None:  # pragma: no cover
        try:
            self.free()
        except Exception:
            pass
