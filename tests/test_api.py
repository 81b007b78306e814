"""Host-side contract of the public API (no GPU needed).

Follows the reference's contract tests: keyword-only construction and
parameter validation (``core.py:156-231``), labels and feature count
(``core.py:272-329``), the metadata envelope of the golden manifests, result
samples and offsets (``result.py:234-420``), the compute-control contract
(``cpp/tests/test_public_api.cpp:41-53``), batch validation
(``core/input.py:39-122``) and the device-unavailable error path.
"""

from __future__ import annotations

import pickle

import numpy as np
import pytest

import mdescriptor_amd as mdx
from conftest import load_golden
from mdescriptor_amd.core.backends import structure_blocks
from mdescriptor_amd.core.result import atom_samples, format_values


def _water(n_structures=1):
    numbers = np.tile([8, 1, 1], n_structures)
    positions = np.concatenate([np.array([[0, 0, 0], [0.96, 0, 0], [-0.24, 0.93, 0]]) + 5 * s
                                for s in range(n_structures)])
    return mdx.StructureBatch(numbers, positions, np.zeros((n_structures, 3, 3)), np.zeros((n_structures, 3)),
                              np.arange(n_structures + 1) * 3, [f"w{s}" for s in range(n_structures)])


def test_soap_defaults_and_layout():
    soap = mdx.SOAP(species=[1, 6, 7, 8], r_cut=5.0)
    assert (soap.settings.n_max, soap.settings.l_max, soap.settings.sigma, soap.settings.average) == (8, 6, 1.0,
                                                                                                        "inner")
    assert soap.feature_count == 3696
    assert len(soap.settings.labels()) == 3696
    assert soap.settings.labels()[0] == "soap:z1=1,z2=1,l=0,n1=0,n2=0"
    assert soap.settings.labels()[-1] == "soap:z1=8,z2=8,l=6,n1=7,n2=7"
    config = soap.configuration.to_dict()
    assert config["descriptor"] == "SOAP" and config["schema_version"] == 1
    assert config["parameters"]["execution"] == {"device": "hip", "num_threads": None}


def test_soap_is_keyword_only():
    with pytest.raises(TypeError):
        mdx.SOAP([1, 8], 5.0)  # type: ignore[misc]


@pytest.mark.parametrize("kwargs,path", [
    (dict(r_cut=-1.0), ["r_cut"]),
    (dict(r_cut=5.0, n_max=0), ["n_max"]),
    (dict(r_cut=5.0, l_max=21), ["l_max"]),
    (dict(r_cut=5.0, sigma=0.0), ["sigma"]),
    (dict(r_cut=float("inf")), ["r_cut"]),
])
def test_invalid_parameters_carry_paths(kwargs, path):
    with pytest.raises(mdx.DescriptorConfigError) as info:
        mdx.SOAP(species=[1, 8], **kwargs)
    assert info.value.code == "invalid_configuration"
    assert list(info.value.path) == path


@pytest.mark.parametrize("kwargs", [dict(r_cut=1.0), dict(r_cut=5.0, average="sum"), dict(r_cut=5.0, rbf="bessel"),
                                    dict(r_cut=5.0, compression={"mode": "bogus"}), dict(r_cut=5.0, species=[]),
                                    dict(r_cut=5.0, species=[1, 1]), dict(r_cut=5.0, species=[0, 1]),
                                    dict(r_cut=5.0, n_max=2.5)])
def test_invalid_configurations(kwargs):
    kwargs.setdefault("species", [1, 8])
    with pytest.raises(mdx.DescriptorConfigError):
        mdx.SOAP(**kwargs)


def test_species_required():
    with pytest.raises(mdx.DescriptorConfigError) as info:
        mdx.SOAP(r_cut=5.0)
    assert list(info.value.path) == ["species"]


@pytest.mark.parametrize("device", ["cpu", "cuda"])
def test_other_devices_are_rejected(device):
    with pytest.raises(mdx.DescriptorConfigError) as info:
        mdx.SOAP(species=[1, 8], r_cut=5.0, execution=mdx.ExecutionOptions(device=device))
    assert info.value.code == "unsupported_device"
    assert info.value.details == {"supported": ["hip"]}


def test_unknown_device_is_invalid():
    with pytest.raises(mdx.DescriptorConfigError) as info:
        mdx.ExecutionOptions(device="tpu")
    assert info.value.code == "invalid_device"


@pytest.mark.parametrize("kwargs,features", [
    (dict(rbf="polynomial"), (2 * 8) * (2 * 8 + 1) // 2 * 7),
    (dict(weighting={"function": "poly", "r0": 4.0, "c": 1.0, "m": 2.0}), (2 * 8) * (2 * 8 + 1) // 2 * 7),
    (dict(weighting={"w0": 0.5}), (2 * 8) * (2 * 8 + 1) // 2 * 7),
    (dict(compression={"mode": "mu2"}), 8 * 9 // 2 * 7),
    (dict(compression={"mode": "mu1nu1"}), 2 * 8 * 8 * 7),
    (dict(compression={"mode": "crossover"}), 2 * 8 * 9 // 2 * 7),
    (dict(compression={"mode": "off", "species_weighting": {1: 2.0, 8: 1.0}}), (2 * 8) * (2 * 8 + 1) // 2 * 7),
])
def test_every_soap_option_is_accepted(kwargs, features):
    """Weighting, compression, species weights and the polynomial basis run on
    the device; the width follows soap_features (soap.cpp:373-387)."""

    soap = mdx.SOAP(species=[1, 8], r_cut=5.0, **kwargs)
    assert soap.feature_count == features
    assert len(soap.settings.labels()) == features


def test_species_weighting_must_name_the_species():
    with pytest.raises(mdx.DescriptorConfigError) as info:
        mdx.SOAP(species=[1, 8], r_cut=5.0, compression={"mode": "off", "species_weighting": {1: 2.0}})
    assert info.value.code == "invalid_configuration"


def test_unit_species_weights_are_accepted():
    soap = mdx.SOAP(species=[1, 8], r_cut=5.0, compression={"mode": "off", "species_weighting": {1: 1.0, 8: 1}})
    assert soap.feature_count == (2 * 8) * (2 * 8 + 1) // 2 * 7


def test_device_limits():
    with pytest.raises(mdx.DescriptorConfigError) as info:
        mdx.SOAP(species=list(range(1, 18)), r_cut=5.0, n_max=2, l_max=2)
    assert info.value.code == "invalid_parameter" and info.value.details["maximum"] == 16


def test_weighting_cutoff_inference():
    from mdescriptor_amd.descriptors.soap import SoapSettings

    s = SoapSettings(species=[1], weighting={"function": "poly", "r0": 4.0, "c": 1.0, "m": 2.0})
    assert s.r_cut == 4.0
    s = SoapSettings(species=[1], weighting={"function": "exp", "r0": 1.0, "c": 1.0, "d": 0.0})
    assert s.r_cut == pytest.approx(np.log(100.0))
    assert SoapSettings(species=[1]).r_cut == 6.0


# (weighting, r_cut, expected cutoff or the first error message): the checks of
# _soap_weighting_config (core.py:97-153) in their order -- function, then r0
# and c, then d before m for pow, then the threshold, then w0 -- and the
# inferred cutoffs r0, r0 (c/t - d)^(1/m), r0 ln(c/t - d)
WEIGHTING_CASES = [
    ({"function": "gauss", "r0": 1.0, "c": 1.0}, None, "must be 'poly', 'pow', or 'exp'"),
    ({"function": "poly", "c": 1.0, "m": 1.0}, None, "requires r0 > 0 and c >= 0"),
    ({"function": "pow", "r0": 1.0, "m": 1.0, "d": 0.0}, None, "requires r0 > 0 and c >= 0"),
    ({"function": "poly", "r0": 1.0, "c": 1.0}, None, "SOAP poly weighting requires m >= 0"),
    ({"function": "pow", "r0": 1.0, "c": 1.0}, None, "SOAP pow/exp weighting requires d >= 0"),
    ({"function": "pow", "r0": 1.0, "c": 1.0, "d": 0.5}, None, "SOAP pow weighting requires m >= 0"),
    ({"function": "exp", "r0": 1.0, "c": 1.0}, None, "SOAP pow/exp weighting requires d >= 0"),
    ({"function": "exp", "r0": 1.0, "c": 1.0, "d": 0.0, "threshold": 0.0}, None, "threshold must be positive"),
    ({"function": "poly", "r0": 2.5, "c": 1.0, "m": 2.0, "w0": -1.0}, None, "w0 must be non-negative"),
    ({"w0": 0.25}, None, 6.0),
    ({"function": "poly", "r0": 2.5, "c": 0.0, "m": 0.0}, None, 2.5),
    ({"function": "poly", "r0": 2.5, "c": 1.0, "m": 2.0}, 4.0, 4.0),
    ({"function": "pow", "r0": 2.0, "c": 1.0, "d": 1.0, "m": 2.0, "threshold": 0.5}, None, 2.0),
    ({"function": "pow", "r0": 2.0, "c": 1.0, "d": 0.0, "m": 0.0}, None, "cannot infer SOAP pow"),
    ({"function": "pow", "r0": 2.0, "c": 1.0, "d": 200.0, "m": 1.0}, None, "cannot infer SOAP pow"),
    ({"function": "exp", "r0": 3.0, "c": 2.0, "d": 1.0, "threshold": 0.1}, None, 3.0 * np.log(19.0)),
    ({"function": "exp", "r0": 3.0, "c": 0.01, "d": 0.0}, None, "cannot infer SOAP exp"),
]


@pytest.mark.parametrize("case", range(len(WEIGHTING_CASES)))
def test_weighting_checks_and_cutoffs(case):
    from mdescriptor_amd.descriptors.soap import _weighting_config

    weighting, r_cut, expected = WEIGHTING_CASES[case]
    if isinstance(expected, str):
        with pytest.raises(ValueError, match=expected):
            _weighting_config(weighting, r_cut)
        return
    options, cutoff = _weighting_config(weighting, r_cut)
    assert cutoff == pytest.approx(expected, rel=1e-15)
    if weighting.get("function") in ("pow", "exp"):
        assert options["threshold"] == weighting.get("threshold", 1e-2)
        assert list(options)[-1] == "threshold" or "threshold" in weighting


@pytest.mark.parametrize("manifest", ["manifest.json", "external_manifest.json"])
def test_metadata_envelope_matches_golden(manifest):
    meta, _, _ = load_golden("reference_soap", manifest)
    p = meta["configuration"]["parameters"]
    soap = mdx.SOAP(species=p["species"], r_cut=p["r_cut"], n_max=p["n_max"], l_max=p["l_max"],
                    sigma=p.get("sigma", 1.0), average=p["average"])
    expected = dict(meta["result"]["metadata"])
    ours = soap.metadata
    assert ours["backend"] == "mdescriptor-hip" and ours["execution"]["device"] == "hip"
    for key in ("backend", "execution"):
        expected.pop(key)
        ours.pop(key)
    assert ours == expected


def test_compute_validates_before_touching_the_device():
    soap = mdx.SOAP(species=[1, 6], r_cut=4.0, n_max=2, l_max=2)
    with pytest.raises(mdx.DescriptorInputError) as info:
        soap.compute(_water())
    assert list(info.value.path) == ["input", "numbers"]
    control = mdx.ComputeControl()
    control.cancel()
    with pytest.raises(mdx.CancelledError):
        mdx.SOAP(species=[1, 8], r_cut=4.0, n_max=2, l_max=2).compute(_water(), control=control)


class _DeviceArrayStub:
    """An object exposing __cuda_array_interface__ at address 0: enough for
    the output checks, which run before any device work."""

    def __init__(self, shape, typestr="<f8", readonly=False, strides=None):
        self.__cuda_array_interface__ = {"shape": shape, "typestr": typestr, "data": (0, readonly),
                                         "strides": strides, "version": 3}


def test_compute_into_checks_the_output_before_touching_the_device():
    soap = mdx.SOAP(species=[1, 8], r_cut=4.0, n_max=2, l_max=2, average="off")
    batch = _water()
    rows, features = batch.atoms, soap.feature_count
    for bad in (_DeviceArrayStub((rows - 1, features)), _DeviceArrayStub((rows, features), "<f4"),
                _DeviceArrayStub((rows, features), readonly=True),
                _DeviceArrayStub((rows, features), strides=(8, rows * 8)), _DeviceArrayStub((rows * features,)),
                np.zeros((rows, features))):
        with pytest.raises(mdx.DescriptorInputError) as info:
            soap.compute_into(batch, bad)
        assert list(info.value.path) == ["out"]
    inner = mdx.SOAP(species=[1, 8], r_cut=4.0, n_max=2, l_max=2, output=mdx.OutputOptions(dtype="float32"))
    with pytest.raises(mdx.DescriptorInputError, match=r"shape \(1, "):
        inner.compute_into(batch, _DeviceArrayStub((rows, features), "<f4"))


def test_closed_descriptor_and_pickling():
    soap = mdx.SOAP(species=[1, 8], r_cut=4.0, n_max=2, l_max=2)
    with pytest.raises(TypeError):
        pickle.dumps(soap)
    snapshot = soap.metadata
    soap.close()
    assert soap.closed and soap.metadata == snapshot
    with pytest.raises(mdx.ClosedDescriptorError):
        soap.compute(_water())
    with mdx.SOAP(species=[1, 8], r_cut=4.0, n_max=2, l_max=2) as inner:
        assert not inner.closed
    assert inner.closed


def test_missing_device_fails_loudly(monkeypatch):
    """With no usable device the product path raises device_unavailable; it
    never computes on the CPU."""

    from mdescriptor_amd import _hip

    def unavailable(*args, **kwargs):
        raise _hip.HipUnavailable("no HIP device is available")

    monkeypatch.setattr(_hip, "shared_context", unavailable)
    soap = mdx.SOAP(species=[1, 8], r_cut=4.0, n_max=2, l_max=2)
    with pytest.raises(mdx.MDescriptorError) as info:
        soap.compute(_water())
    assert info.value.code == "device_unavailable"


def test_compute_control_contract():
    control = mdx.ComputeControl()
    control.reset(2)
    assert (control.total(), control.completed(), control.cancelled()) == (2, 0, False)
    control.mark_completed()
    assert control.completed() == 1
    control.cancel()
    assert control.cancelled() and control._hip_cancel_flag.value == 1
    control.reset(3)
    assert not control.cancelled()
    with pytest.raises(ValueError):
        control.reset(-1)


def test_result_samples_and_validation():
    values = np.arange(12, dtype=np.float64).reshape(4, 3)
    result = mdx.DescriptorResult(values, "atom", ("a", "b", "c"), np.array([0, 1, 1, 4]), ("x", "y", "z"))
    assert result.samples.tolist() == [[0, 0], [2, 0], [2, 1], [2, 2]]
    assert not result.values.flags.writeable
    values[0, 0] = 99.0
    assert result.values[0, 0] == 0.0
    with pytest.raises(ValueError):
        mdx.DescriptorResult(values, "atom", ("a",), np.array([0, 4]), ("x", "y"))
    with pytest.raises(ValueError):
        mdx.DescriptorResult(values, "structure", ("a", "b"), None, ("x", "y", "z"))
    structure = mdx.DescriptorResult(values[:2], "structure", ("a", "b"), None, ("x", "y", "z"))
    assert structure.samples.tolist() == [[0], [1]] and structure.row_offsets is None
    assert atom_samples(np.array([0, 0, 2])).tolist() == [[1, 0], [1, 1]]


def test_format_values_dense_and_sparse():
    dense = format_values(np.eye(3), dtype="float32")
    assert dense.dtype == np.float32
    sparse = format_values(np.eye(3), dtype="float64", sparse=True)
    assert sparse.nnz == 3 and sparse.dtype == np.float64


def test_structure_blocks():
    offsets = np.array([0, 3, 3, 10, 11, 30])
    assert structure_blocks(offsets, budget=10) == [(0, 3), (3, 4), (4, 5)]
    assert structure_blocks(offsets, budget=100) == [(0, 5)]
    assert structure_blocks(offsets, budget=1) == [(0, 1), (1, 2), (2, 3), (3, 4), (4, 5)]
    assert structure_blocks(np.array([0]), budget=5) == []
    covered = [s for a, b in structure_blocks(offsets, budget=4) for s in range(a, b)]
    assert covered == list(range(5))


def test_batch_validation():
    with pytest.raises(ValueError):
        mdx.StructureBatch([1, 1], np.zeros((2, 3)), np.eye(3)[None], [[1, 0, 1]], [0, 2], ["mixed"])
    with pytest.raises(ValueError):
        mdx.StructureBatch([1, 1], np.zeros((2, 3)), np.zeros((1, 3, 3)), [[1, 1, 1]], [0, 2], ["singular"])
    with pytest.raises(ValueError):
        mdx.StructureBatch([1, 1], np.zeros((2, 3)), np.zeros((1, 3, 3)), [[0, 0, 0]], [0, 3], ["offsets"])
    with pytest.raises(ValueError):
        mdx.StructureBatch([1, 0], np.zeros((2, 3)), np.zeros((1, 3, 3)), [[0, 0, 0]], [0, 2], ["z"])
    with pytest.raises(ValueError):
        mdx.StructureBatch([1, 1], np.full((2, 3), np.nan), np.zeros((1, 3, 3)), [[0, 0, 0]], [0, 2], ["nan"])
    batch = _water(3)
    assert batch.structures == 3 and batch.atoms == 9
    view = batch._slice_view(1, 3)
    assert view.offsets.tolist() == [0, 3, 6] and view.ids == ("w1", "w2")


@pytest.mark.parametrize("species,message", [
    (5, "species must be a sequence of atomic numbers"),
    ([1, True], "species must contain integer atomic numbers"),
    ([1, "x"], "species must contain integer atomic numbers"),
    ([1, 2.5], "species must contain integer atomic numbers"),
    ([1, float("nan")], "species must contain integer atomic numbers"),
    ([], "species must be a non-empty sequence of unique atomic numbers"),
    ([8, 8], "species must be a non-empty sequence of unique atomic numbers"),
    ([0, 0], "species must be a non-empty sequence of unique atomic numbers"),
    ([1, -8], "species must contain positive atomic numbers"),
])
def test_species_declaration_messages(species, message):
    """Messages and path of the species contract (src/mdescriptor/core/species.py:16-58)."""

    from mdescriptor_amd.core.species import normalize_species

    with pytest.raises(mdx.DescriptorConfigError) as info:
        normalize_species(species)
    assert str(info.value) == message or info.value.message == message
    assert list(info.value.path) == ["species"]


def test_species_accepts_integral_values():
    from mdescriptor_amd.core.species import normalize_species, validate_batch_species

    assert normalize_species([np.int64(8), 1.0, "6"]) == (8, 1, 6)
    assert normalize_species(None) is None
    with pytest.raises(mdx.DescriptorInputError, match=r"outside its declaration: \[8\]"):
        validate_batch_species(_water(), [1], descriptor="SOAP")


def test_batch_field_conversion_messages():
    base = dict(numbers=[1, 1], positions=np.zeros((2, 3)), cells=np.zeros((1, 3, 3)), pbc=[[0, 0, 0]],
                offsets=[0, 2], ids=["a"])
    for field, value, message in [
        ("numbers", [True, True], "numbers must contain integers, not booleans"),
        ("numbers", [1.5, 1.0], "numbers must contain finite integers"),
        ("numbers", ["a", "b"], "numbers must contain integers"),
        ("offsets", [0.0, 2.0], None),
        ("pbc", [[False, False, False]], None),
        ("positions", [["x", 0, 0], [0, 0, 0]], "positions must be a numeric array"),
        ("positions", np.full((2, 3), np.inf), "positions must be finite"),
        ("numbers", [2**40, 1], "numbers contains values outside"),
    ]:
        kwargs = dict(base, **{field: value})
        if message is None:
            mdx.StructureBatch(**kwargs)
            continue
        with pytest.raises(ValueError, match=message) as info:
            mdx.StructureBatch(**kwargs)
        assert list(info.value.path) == ["input", field]
