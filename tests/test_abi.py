"""The C-ABI library without a GPU: it loads, exports every function that
include/mdx_hip.h declares, and the ctypes mirror of its structs has the
layout a C compiler gives them.  No compute entry point is called here."""

from __future__ import annotations

import ctypes
import re
import subprocess
import sys

import pytest

from conftest import ROOT

HEADER = ROOT / "include" / "mdx_hip.h"


def _declared_functions() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(mdx_hip_[a-z0-9_]+)\s*\(", text))


@pytest.fixture(scope="module")
def hip():
    from mdescriptor_amd import _hip

    if not _hip.LIBRARY_PATH.is_file():
        subprocess.run([sys.executable, "-m", "mdescriptor_amd.build"], check=True, cwd=ROOT)
    return _hip


def test_library_exports_every_declared_function(hip):
    declared = _declared_functions()
    assert len(declared) >= 13
    lib = ctypes.CDLL(str(hip.LIBRARY_PATH))
    missing = [name for name in sorted(declared) if not hasattr(lib, name)]
    assert not missing
    exported = subprocess.run(["nm", "-D", "--defined-only", str(hip.LIBRARY_PATH)], capture_output=True,
                              text=True, check=True).stdout
    assert all(re.search(rf"\bT {name}$", exported, flags=re.M) for name in declared)


def test_ctypes_signatures_cover_header(hip):
    assert set(hip.SIGNATURES) == _declared_functions()
    lib = hip.load_library()
    assert "gfx950" in lib.mdx_hip_version().decode()
    assert lib.mdx_hip_last_error(None) is not None


def test_status_codes_match_header(hip):
    text = HEADER.read_text()
    for name in ("MDX_OK", "MDX_INVALID_ARGUMENT", "MDX_OUT_OF_MEMORY", "MDX_DEVICE_UNAVAILABLE", "MDX_CANCELLED",
                 "MDX_INTERNAL"):
        value = int(re.search(rf"\b{name}\s*=\s*(\d+)", text).group(1))
        assert getattr(hip, name) == value


def test_struct_layout_matches_c(hip, tmp_path):
    """sizeof/offsetof of the five public structs, compiled by gcc from the
    header, against the ctypes mirror."""

    structs = {"mdx_batch_view": hip.BatchView, "mdx_soap_params": hip.SoapParams, "mdx_timing": hip.Timing,
               "mdx_soap_options": hip.SoapOptions, "mdx_list_timing": hip.ListTiming}
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "mdx_hip.h"', "int main(void) {"]
    for cname, ctype in structs.items():
        lines.append(f'printf("{cname} %zu\\n", sizeof({cname}));')
        for field, _ in ctype._fields_:
            lines.append(f'printf("{cname}.{field} %zu\\n", offsetof({cname}, {field}));')
    lines.append("return 0; }")
    source = tmp_path / "layout.c"
    source.write_text("\n".join(lines))
    binary = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", f"-I{ROOT / 'include'}", str(source), "-o", str(binary)], check=True)
    printed = dict(line.rsplit(" ", 1) for line in subprocess.run([str(binary)], capture_output=True, text=True,
                                                                  check=True).stdout.splitlines())
    for cname, ctype in structs.items():
        assert int(printed[cname]) == ctypes.sizeof(ctype), cname
        for field, _ in ctype._fields_:
            assert int(printed[f"{cname}.{field}"]) == getattr(ctype, field).offset, f"{cname}.{field}"
