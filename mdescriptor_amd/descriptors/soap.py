"""The public ``SOAP`` descriptor, executed on one AMD Instinct GPU.

Mirrors the reference's public class and its validation kernel:

* keyword-only constructor ``SOAP(*, species, rbf="gto", n_max=8, l_max=6,
  sigma=1.0, average="inner", weighting=None, r_cut=None, compression=None,
  output=None, execution=None)`` (``src/mdescriptor/core/adapter.py:927-984``,
  defaults ``src/mdescriptor/registry/builtins.py:218-278``);
* parameter checks, ``feature_count``, labels and metadata of ``SoapKernel``
  (``src/mdescriptor/descriptors/_kernels/core.py:156-371``);
* the private backend payload (radial basis, labels, feature count) handed to
  the device plugin exactly as ``_cuda_payload`` is (``core.py:331-355``,
  ``adapter.py:528-603``), keyed ``_hip_*`` here.

Every SOAP option of the reference runs on the GPU: both radial bases (GTO
and polynomial), distance weighting (poly, pow, exp, w0), species weights and
the four compression modes, on the matrix-core kernel.
"""

from __future__ import annotations

import threading
from collections.abc import Mapping
from typing import Any

import numpy as np

from ..core.backends import HipBackend
from ..core.descriptor import Descriptor
from ..core.errors import DescriptorConfigError, DescriptorInputError
from ..core.options import CONFIGURATION_SCHEMA_VERSION, ExecutionOptions, OutputOptions, coerce_options
from ..core.result import DescriptorResult, format_values, metadata_envelope, owned_values
from ..core.species import require_species, validate_batch_species
from .basis import basis_gto, basis_polynomial

# Limits of the HIP library (mdx_hip_soap_plan_create): species, radial
# channels and coefficient storage per centre.
HIP_MAX_SPECIES = 16
HIP_MAX_N = 16
HIP_MAX_L = 20
HIP_MAX_COEFF_BYTES = 96 * 1024
SUPPORTED_DEVICES = ("hip",)


class _KernelValueError(ValueError):
    def __init__(self, message: str, path: list[str]) -> None:
        super().__init__(message)
        self.path = path


# Per weighting function: the shape parameters it takes besides r0 and c, in
# the order they are checked; each defaults to -1 (absent, hence rejected).
# pow and exp also take a positive threshold (default 1e-2), used only to
# infer a missing cutoff.  (Contract of core.py:97-153: the same messages,
# defaults and cutoff formulas.)
_WEIGHTING_SHAPES = {"poly": ("m",), "pow": ("d", "m"), "exp": ("d",)}
_SHAPE_ERRORS = {"d": "SOAP pow/exp weighting requires d >= 0", "m": "SOAP {} weighting requires m >= 0"}


def _poly_cutoff(options: dict[str, Any]) -> float:
    return options["r0"]


def _pow_cutoff(options: dict[str, Any]) -> float:
    base = options["c"] / options["threshold"] - options["d"]
    if options["m"] <= 0.0 or base <= 0.0:
        raise ValueError("cannot infer SOAP pow weighting cutoff")
    return options["r0"] * base ** (1.0 / options["m"])


def _exp_cutoff(options: dict[str, Any]) -> float:
    base = options["c"] / options["threshold"] - options["d"]
    if base <= 1.0:
        raise ValueError("cannot infer SOAP exp weighting cutoff")
    return float(options["r0"] * np.log(base))


# the radius where each weighting function falls to the threshold
_CUTOFF_RULES = {"poly": _poly_cutoff, "pow": _pow_cutoff, "exp": _exp_cutoff}


def _weighting_config(weighting: Mapping[str, Any] | None, r_cut: float | None) -> tuple[dict[str, Any], float]:
    """Canonical weighting options and the resolved cutoff (core.py:97-153).

    Without a weighting function the cutoff must be given (else 6 A).  With
    one, a missing cutoff is inferred from the function: ``r0`` for ``poly``,
    ``r0 (c/threshold - d)^(1/m)`` for ``pow`` and ``r0 ln(c/threshold - d)``
    for ``exp``.
    """

    options = dict(weighting or {})
    kind = options.get("function")
    if kind is not None:
        kind = str(kind)
        shapes = _WEIGHTING_SHAPES.get(kind)
        if shapes is None:
            raise ValueError("SOAP weighting function must be 'poly', 'pow', or 'exp'")
        r0, c = float(options.get("r0", 0.0)), float(options.get("c", -1.0))
        if r0 <= 0.0 or c < 0.0:
            raise ValueError("SOAP weighting requires r0 > 0 and c >= 0")
        options["r0"], options["c"] = r0, c
        for name in shapes:
            value = float(options.get(name, -1.0))
            if value < 0.0:
                raise ValueError(_SHAPE_ERRORS[name].format(kind))
            options[name] = value
        if "d" in shapes:
            options["threshold"] = float(options.get("threshold", 1e-2))
            if options["threshold"] <= 0.0:
                raise ValueError("SOAP weighting threshold must be positive")
    if "w0" in options:
        options["w0"] = float(options["w0"])
        if options["w0"] < 0.0:
            raise ValueError("SOAP weighting w0 must be non-negative")
    if r_cut is not None:
        return options, float(r_cut)
    rule = _CUTOFF_RULES.get(kind) if kind is not None else None
    return options, 6.0 if rule is None else rule(options)


class SoapSettings:
    """Validated SOAP parameters with the reference's derived quantities."""

    name = "SOAP"

    def __init__(self, species: Any = None, rbf: str = "gto", n_max: int = 8, l_max: int = 6, sigma: float = 1.0,
                 average: str = "inner", weighting: Mapping[str, Any] | None = None, r_cut: float | None = None,
                 compression: Mapping[str, Any] | None = None, dtype: str = "float64", sparse: bool = False) -> None:
        for key, value in (("n_max", n_max), ("l_max", l_max)):
            if isinstance(value, bool) or (isinstance(value, float) and not float(value).is_integer()):
                raise _KernelValueError(f"{key} must be an integer", [key])
        self.rbf = str(rbf)
        self.n_max = int(n_max)
        self.l_max = int(l_max)
        self.sigma = float(sigma)
        self.average = str(average)
        self.dtype = str(dtype)
        self.sparse = bool(sparse)
        self.weighting, self.r_cut = _weighting_config(weighting, r_cut)
        compression = compression or {"mode": "off", "species_weighting": None}
        if not isinstance(compression, Mapping):
            raise ValueError("compression must be a dictionary")
        self.compression = dict(compression)
        self.compression_mode = str(self.compression.get("mode", "off"))
        if self.compression_mode not in {"off", "mu2", "mu1nu1", "crossover"}:
            raise ValueError("invalid SOAP compression mode")
        if self.rbf not in {"gto", "polynomial"}:
            raise ValueError("rbf must be 'gto' or 'polynomial'")
        bad: list[str] | None = None
        if self.r_cut <= 0:
            bad = ["r_cut"]
        elif self.n_max < 1:
            bad = ["n_max"]
        elif self.l_max < 0 or self.l_max > 20:
            bad = ["l_max"]
        elif self.sigma <= 0:
            bad = ["sigma"]
        if bad is not None:
            raise _KernelValueError("invalid SOAP parameters", bad)
        if not np.isfinite(self.r_cut):
            raise _KernelValueError("SOAP parameters must be finite", ["r_cut"])
        if not np.isfinite(self.sigma):
            raise _KernelValueError("SOAP parameters must be finite", ["sigma"])
        if self.rbf == "gto" and self.r_cut <= 1.0:
            raise ValueError("SOAP GTO radial basis requires r_cut > 1")
        if self.average not in {"off", "inner", "outer"}:
            raise ValueError("average must be 'off', 'inner', or 'outer'")
        self.species = require_species(species, descriptor=self.name)
        species_weighting = self.compression.get("species_weighting")
        if species_weighting is not None and not isinstance(species_weighting, Mapping):
            raise ValueError("species_weighting must be a dictionary or None")
        self.species_weighting = None if species_weighting is None else dict(species_weighting)

    @property
    def feature_count(self) -> int:
        """Columns of one row (core.py:272-284)."""

        s, n, degrees = len(self.species), self.n_max, self.l_max + 1
        if self.compression_mode == "mu2":
            return n * (n + 1) // 2 * degrees
        if self.compression_mode == "mu1nu1":
            return s * n * n * degrees
        if self.compression_mode == "crossover":
            return s * n * (n + 1) // 2 * degrees
        width = s * n
        return width * (width + 1) // 2 * degrees

    def labels(self) -> tuple[str, ...]:
        """Column labels in output order (core.py:306-329).

        Uncompressed: species pairs ``z1 <= z2`` in declaration order, then
        degree ``l``, then ``n1``, then ``n2`` (``n2 >= n1`` when the two
        species are equal).
        """

        degrees, n = range(self.l_max + 1), range(self.n_max)
        if self.compression_mode == "mu2":
            return tuple(f"soap:compression=mu2,l={l},n1={a},n2={b}" for l in degrees for a in n for b in n if b >= a)
        if self.compression_mode == "mu1nu1":
            return tuple(f"soap:compression=mu1nu1,z1={z},l={l},n1={a},n2={b}"
                         for z in self.species for l in degrees for a in n for b in n)
        if self.compression_mode == "crossover":
            pairs = [(z, z) for z in self.species]
        else:
            pairs = [(z1, z2) for i, z1 in enumerate(self.species) for z2 in self.species[i:]]
        return tuple(f"soap:z1={z1},z2={z2},l={l},n1={a},n2={b}"
                     for z1, z2 in pairs for l in degrees for a in n for b in n if z1 != z2 or b >= a)

    def details(self) -> dict[str, Any]:
        """Backend-independent metadata details (core.py:357-371)."""

        return {
            "species": list(self.species),
            "average": self.average,
            "r_cut": self.r_cut,
            "n_max": self.n_max,
            "l_max": self.l_max,
            "sigma": self.sigma,
            "rbf": self.rbf,
            "weighting": dict(self.weighting),
            "compression": dict(self.compression),
        }

    def hip_payload(self) -> dict[str, Any]:
        """Radial basis, labels and width for the device plugin (core.py:331-355)."""

        if self.rbf == "gto":
            alphas, betas = basis_gto(self.r_cut, self.n_max, self.l_max)
            radial = {"alphas": alphas, "betas": betas}
        else:
            grid, weights, values = basis_polynomial(self.r_cut, self.n_max)
            radial = {"radial_grid": grid, "radial_weights": weights, "radial_values": values}
        return {
            "radial_basis": radial,
            "feature_count": self.feature_count,
            "labels": self.labels(),
        }

    def hip_unsupported(self) -> tuple[str, str] | None:
        """First option the HIP library does not implement, as (path, reason):
        none since every option runs on the device.  The species weighting
        must name exactly the configured species (core.py:262-265)."""

        if self.species_weighting is not None and {int(k) for k in self.species_weighting} != set(self.species):
            raise ValueError("species_weighting must contain exactly the configured species")
        return None


_PUBLIC_OPTIONS = ("species", "rbf", "n_max", "l_max", "sigma", "average", "weighting", "r_cut", "compression")


class SOAP(Descriptor):
    """Smooth overlap of atomic positions, computed on an AMD GPU."""

    name = "SOAP"
    supported_devices = SUPPORTED_DEVICES

    def __init__(self, *, species: Any = None, rbf: str | None = None, n_max: int | None = None,
                 l_max: int | None = None, sigma: float | None = None, average: str | None = None,
                 weighting: Mapping[str, Any] | None = None, r_cut: float | None = None,
                 compression: Mapping[str, Any] | None = None, output: Any = None, execution: Any = None) -> None:
        super().__init__()
        self._output_options = coerce_options(output, OutputOptions, "output")
        self._execution_options = coerce_options(execution, ExecutionOptions, "execution")
        device = self._execution_options.device
        if device not in self.supported_devices:
            raise DescriptorConfigError(
                f"{self.name} does not support execution.device={device!r}; supported devices: "
                + ", ".join(self.supported_devices),
                code="unsupported_device",
                path=["execution", "device"],
                details={"supported": list(self.supported_devices)},
            )
        given = {"species": species, "rbf": rbf, "n_max": n_max, "l_max": l_max, "sigma": sigma,
                 "average": average, "weighting": weighting, "r_cut": r_cut, "compression": compression}
        kwargs = {k: v for k, v in given.items() if v is not None}
        try:
            settings = SoapSettings(**kwargs, dtype=self._output_options.dtype, sparse=self._output_options.sparse)
            unsupported = settings.hip_unsupported()
        except (DescriptorConfigError, DescriptorInputError):
            raise
        except (TypeError, ValueError) as exc:
            raise DescriptorConfigError(f"invalid {self.name} configuration: {exc}", code="invalid_configuration",
                                        path=getattr(exc, "path", None)) from exc
        if unsupported is not None:
            raise DescriptorConfigError(f"{self.name} on device 'hip': {unsupported[1]}", code="unsupported_option",
                                        path=["parameters", unsupported[0]], details={"device": "hip"})
        self._check_device_limits(settings)
        try:
            payload = settings.hip_payload()
        except ValueError as exc:
            raise DescriptorConfigError(f"invalid {self.name} configuration: {exc}", code="invalid_configuration",
                                        path=["parameters", "n_max"]) from exc
        self._settings = settings
        parameters: dict[str, Any] = {key: given[key] for key in _PUBLIC_OPTIONS}
        parameters["species"] = list(settings.species)
        parameters["output"] = self._output_options.to_dict()
        parameters["execution"] = self._execution_options.to_dict()
        self._set_configuration(CONFIGURATION_SCHEMA_VERSION, parameters)
        backend_options: dict[str, Any] = {
            "species": list(settings.species), "n_max": settings.n_max, "l_max": settings.l_max,
            "r_cut": settings.r_cut, "sigma": settings.sigma, "average": settings.average,
            "rbf": settings.rbf, "weighting": dict(settings.weighting), "compression": dict(settings.compression),
            "output": self._output_options.to_dict(), "execution": self._execution_options.to_dict(),
            "_hip_payload": payload, "_hip_labels": payload["labels"], "_hip_feature_count": settings.feature_count,
        }
        self._backend = HipBackend(self.name, backend_options, settings.feature_count)
        self._labels = payload["labels"]
        self._lock = threading.Lock()
        self._metadata_snapshot = self._envelope()

    def _check_device_limits(self, settings: SoapSettings) -> None:
        coeff_bytes = len(settings.species) * settings.n_max * (settings.l_max + 1) ** 2 * 8
        for parameter, value, maximum in (("species", len(settings.species), HIP_MAX_SPECIES),
                                          ("n_max", settings.n_max, HIP_MAX_N),
                                          ("l_max", settings.l_max, HIP_MAX_L),
                                          ("n_max", coeff_bytes, HIP_MAX_COEFF_BYTES)):
            if value > maximum:
                raise DescriptorConfigError(
                    f"{self.name} {parameter}={value!r} exceeds the hip limit of {maximum}",
                    code="invalid_parameter", path=["parameters", parameter],
                    details={"device": "hip", "provided": value, "maximum": maximum})

    @property
    def feature_count(self) -> int:
        return self._settings.feature_count

    @property
    def settings(self) -> SoapSettings:
        return self._settings

    def _envelope(self) -> dict[str, Any]:
        level = "atom" if self._settings.average == "off" else "structure"
        raw = {"backend": "mdescriptor-hip", "descriptor": self.name, "details": self._settings.details(),
               "output": self._output_options.to_dict(), "execution": self._execution_options.to_dict()}
        return metadata_envelope(raw, level, self.feature_count)

    def _validate_batch(self, batch: Any) -> None:
        validate_batch_species(batch, self._settings.species, descriptor=self.name)

    def _compute_batch(self, batch: Any, *, control: Any = None) -> DescriptorResult:
        try:
            raw = self._backend.compute(batch, control)
        except DescriptorInputError:
            raise
        except ValueError as exc:
            raise DescriptorInputError(str(exc), path=["input"]) from exc
        values = raw["values"]
        options = self._output_options
        if options.sparse:
            values = format_values(values, dtype=options.dtype, sparse=True)
        elif values.dtype != np.dtype(options.dtype):
            values = owned_values(np.ascontiguousarray(values, dtype=options.dtype))
        else:
            values = owned_values(values)
        metadata = self._envelope()
        result = DescriptorResult(values, raw["level"], batch.ids, raw.get("row_offsets"), raw["labels"], metadata,
                                  feature_count=self.feature_count)
        self._metadata_snapshot = metadata
        return result

    def compute_into(self, value: Any, out: Any, *, control: Any = None) -> Any:
        """Compute one batch straight into device memory and return ``out``.

        ``out`` is a writable two-dimensional device array of shape
        ``(rows, feature_count)`` and the output dtype: a torch tensor on a
        HIP device, or any object exposing ``__cuda_array_interface__``.
        Rows are those of :meth:`compute` (atoms in batch order, or one per
        structure when averaging); rows may be pitched.  The values never
        touch host memory.  This entry has no counterpart in the reference,
        whose results are always host arrays."""

        from .. import _hip

        batch = self._admit(value, control)
        try:
            target = _hip.DeviceArray(out)
            rows = batch.atoms if self._settings.average == "off" else batch.structures
            target.check(rows, self.feature_count, self._output_options.dtype)
        except ValueError as exc:
            raise DescriptorInputError(str(exc), path=["out"]) from exc
        target.settle()
        try:
            self._backend.compute_into(batch, target.address, target.pitch, control)
        except DescriptorInputError:
            raise
        except ValueError as exc:
            raise DescriptorInputError(str(exc), path=["input"]) from exc
        self._release(control)
        return out

    def close(self) -> None:
        if not self.closed:
            self._backend.close()
        super().close()


__all__ = ["SOAP", "SoapSettings"]
