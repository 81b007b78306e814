"""Build the gfx950 SOAP library in-tree: ``mdescriptor_amd/_lib/libmdx_hip.so``
(and the peak-rate probes of the roofline, ``libmdx_peaks.so``).

Run ``python -m mdescriptor_amd.build``.  Every source under ``csrc/`` is
compiled with hipcc for gfx950 only, with FP contraction off (the device code
spells out its fused multiply-adds, so the graph arithmetic rounds like the
reference's) and packed-FP32 instruction selection disabled.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
OBJ_DIR = PACKAGE / "_build"
LIB_DIR = PACKAGE / "_lib"
LIBRARY = LIB_DIR / "libmdx_hip.so"
SOURCES = ("graph.hip", "frame.hip", "soap.hip", "soap_mfma.hip", "soap_quad.hip", "soap_block.hip", "neighbor_list.hip",
           "api.hip")
# peak-rate probes for the roofline (bench.py --peaks), a library of their own
PEAKS_SOURCE = "peaks.hip"
PEAKS_LIBRARY = LIB_DIR / "libmdx_peaks.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # matrix-core accumulators in ordinary VGPRs (gfx950 allows both forms):
    # avoids copies between AGPRs and VGPRs around every MFMA step
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-result",
]


def _hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise FileNotFoundError("hipcc was not found; the HIP library cannot be built")
    return found


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every source and link the shared library; returns its path."""

    hipcc = _hipcc()
    OBJ_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)

    def compile_one(name: str) -> Path:
        obj = OBJ_DIR / (Path(name).stem + ".o")
        cmd = [hipcc, *HIPCC_FLAGS, "-c", str(CSRC / name), "-o", str(obj)]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        messages = "\n".join(
            line for line in (proc.stdout + proc.stderr).splitlines()
            if "packed-fp32-ops" not in line
        )
        if proc.returncode != 0:
            raise RuntimeError(f"hipcc failed for {name}:\n{messages}")
        if verbose and messages.strip():
            print(messages, file=sys.stderr)
        return obj

    workers = jobs or min(len(SOURCES) + 1, int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=max(1, workers)) as pool:
        objects = list(pool.map(compile_one, (*SOURCES, PEAKS_SOURCE)))
    for library, parts in ((LIBRARY, objects[:-1]), (PEAKS_LIBRARY, objects[-1:])):
        tmp = library.with_suffix(".so.tmp")
        cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *map(str, parts)]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"linking {library.name} failed:\n{proc.stdout}{proc.stderr}")
        os.replace(tmp, library)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose=True))
