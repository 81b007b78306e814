#!/usr/bin/env python
"""SOAP atom-environments per second on one MI355X (benchmark configuration 2).

One step is one pass of the hot path over a new frame of the batch resident
in HBM, through ``mdx_hip_soap_run_frame``: the frame's positions (from one
of four frames uploaded before timing, a device-to-device copy), everything
of the neighbour search that depends on positions (cell grid, regions of
interest, binning paths, home cells, search lists, built on the device), the
neighbour graph (kernel 1) and the per-centre expansion, power spectrum and
float32 write (kernels 2-4).  The frames are the seeded configuration
jittered by 0.02 A (Gaussian, per coordinate), a different frame every step,
each written to one of two output buffers on the device.  Steps are
pipelined: the graph of frame k+1 is built on the context's second stream
while the expansion of frame k runs; the timed region ends after every step
has finished (``mdx_hip_batch_wait``).  The same steps as one synchronous
``mdx_hip_batch_set_positions`` + ``mdx_hip_soap_run`` each are timed before
it (``sequential``), and give the per-stage breakdown and the expansion
kernel's launch time.

Prints one JSON line with the metric of BASELINE.json, a ``roofline`` object
for the dominant kernel (the expansion kernel; bound by FP64 or HBM,
whichever roofline time of the configuration is longer: algorithmic FP64
flops, or algorithmic bytes (output plus 28 B of numbers and positions per
atom), per launch over its launch time from HIP events on the library's stream;
``profile_launch_ms`` is the same kernel's average in the committed rocprofv3
kernel-trace summary ``profiles/<kernel>_<workload>_kernel_trace.md``, for a
cross-check) and a ``cpu_baseline`` object: the reference's own C++ SOAP
compiled in place (``oracle/_ref``) on this host, decomposed as the reference
does (structures in parallel, threads capped at the structure count; one
structure: centres in parallel), on OMP_NUM_THREADS threads (else every CPU
the process may use), with the host's CPU count, model and OMP_NUM_THREADS.
Its sample is the whole batch, except for configuration 5 a 46,656-atom cell
of the same generator.

``--peaks`` only measures this device's FP64 (vector FMA, 16x16x4 MFMA) and
HBM copy rates with the probes of ``mdescriptor_amd/csrc/peaks.hip``.

``--config N`` selects benchmark configuration 1-5 (default 2, the headline);
``--options NAME`` runs the line with SOAP options (mu1nu1 compression, pow
weighting with w0, crossover with exp weighting) on that configuration.

``roofline.traffic`` (HBM bytes per launch of that kernel) is read from the
committed counter summary ``profiles/<kernel>_<workload>_traffic.txt``
when it exists for the benchmarked workload; it comes from two rocprofv3
``--pmc`` runs (FETCH_SIZE, WRITE_SIZE) of this script, each scaled by the
same counter on a device copy of known size (``--calibrate-copy``).

``--calibrate-copy MIB`` only runs that copy: five launches of a plain
device-to-device copy of MIB mebibytes, then exits.

``--path neighbor-list`` measures the NeighborList descriptor instead, on the
same configuration's structures at ``--nl-cutoff`` (default 6, the
descriptor's default): one step is ``mdx_hip_neighbor_list`` + a fetch of the
public values and samples into device memory.  Its ``value`` is kept pairs
per second of device time (graph + keep-count + fill, HIP events); the
roofline object covers the fill kernel (``k_list_fill``, HBM-bound) and the
CPU baseline is the reference's ``compute_neighbor_list`` (``oracle/_ref``).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "SOAP atom-envs/sec (4 spec, n8 l6, rc5) on 1 MI355X; % of FP64/HBM roofline"
FP64_PEAK_TFLOPS = 78.6  # MI355X dense FP64 (vector and MFMA)
HBM_PEAK_GBS = 8000.0


# SOAP options of the option bench lines (--options): the parameters of the
# option parity cases, and the average mode where a line sets its own
POW_W0 = {"function": "pow", "r0": 2.0, "c": 2.0, "d": 1.0, "m": 3.0, "w0": 0.5}
BENCH_OPTIONS = {
    "off": (None, None),
    "mu1nu1": ({"compression": "mu1nu1"}, None),
    "mu2": ({"compression": "mu2"}, None),
    "pow_w0": ({"weighting": POW_W0}, None),
    "crossover": ({"compression": "crossover", "weighting": {"function": "exp", "r0": 2.0, "c": 1.0, "d": 0.2}}, None),
    "polynomial": ({"polynomial": "basis"}, None),
    "outer": (None, "outer"),
    "inner": (None, "inner"),
    "inner_pow_w0": ({"weighting": POW_W0}, "inner"),
}


def describe_options(options: dict | None):
    """JSON-safe description of a line's SOAP options."""

    if not options:
        return "default (GTO, no weighting, compression off)"
    out = {k: v for k, v in options.items() if k != "polynomial"}
    if options.get("polynomial") is not None:
        out["radial_basis"] = f"polynomial ({len(options['polynomial'][0])}-point radial grid)"
    return out


def bench_options(name: str, params: dict) -> tuple[dict | None, str]:
    """The SOAP options and average mode of option line `name` on a
    configuration (the polynomial basis built for its r_cut and n_max)."""

    from mdescriptor_amd.descriptors.basis import basis_polynomial

    options, average = BENCH_OPTIONS[name]
    if options is not None and options.get("polynomial") == "basis":
        options = dict(options, polynomial=basis_polynomial(params["r_cut"], params["n_max"]))
    return options, average or params["average"]


def algorithmic_flops(envs: int, rows: int, kbar: float, S: int, n: int, l_max: int, features: int | None = None,
                      coefficient_species: int | None = None) -> float:
    """Algorithmic FP64 flops of one pass (FMA = 2): accumulation 2*K*n*H
    per environment; per output row (a centre, or with inner averages a
    structure, whose coefficients are averaged before the fold) the beta
    contraction 2*Sc*n^2*H (Sc coefficient species: 1 for mu2, else S) and
    the power spectrum, 2*(2l+1) per feature of degree l, i.e.
    features/(l_max+1) * 2H (with compression off S*n*(S*n+1)*H).""" 

    L = l_max + 1
    H = L * L
    if features is None:
        features = S * n * (S * n + 1) // 2 * L
    sc = S if coefficient_species is None else coefficient_species
    return envs * 2.0 * kbar * n * H + rows * (2.0 * sc * n * n * H + features / L * 2.0 * H)


def algorithmic_bytes(envs: int, rows: int, features: int, itemsize: int) -> float:
    """Algorithmic HBM bytes of one pass: every output value written once,
    numbers and positions (28 B) of every atom read once."""

    return rows * features * itemsize + 28.0 * envs


def roofline_bound(flops: float, nbytes: float) -> str:
    """The configuration's bound: FP64 ("mfma") or HBM ("hbm"), whichever
    roofline time is longer (T_roof = max(flops / FP64 peak, bytes / HBM peak))."""

    return "mfma" if flops / (FP64_PEAK_TFLOPS * 1e12) >= nbytes / (HBM_PEAK_GBS * 1e9) else "hbm"


FRAMES = 4
FRAME_JITTER = 0.02


def frame_positions(batch, count: int) -> list[np.ndarray]:
    """`count` frames of the batch: its positions plus seeded Gaussian noise of
    FRAME_JITTER angstrom per coordinate (frame 0 included)."""

    rng = np.random.Generator(np.random.PCG64(20261202))
    base = np.ascontiguousarray(batch.positions, dtype=np.float64).reshape(-1, 3)
    return [np.ascontiguousarray(base + rng.normal(0.0, FRAME_JITTER, base.shape)) for _ in range(count)]


def profile_average_us(workload_name: str, kernel: str) -> tuple[float | None, str | None]:
    """Average duration of `kernel` over the synchronous steps in the
    committed rocprofv3 kernel-trace summary of this workload (the third
    column of its ``| name | calls | average us (synchronous) | ...`` table)."""

    path = ROOT / "profiles" / f"{kernel.split('<')[0]}_{workload_name}_kernel_trace.md"
    if not path.is_file():
        return None, None
    for line in path.read_text().splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 3 and cells[0].startswith(kernel):
            try:
                return float(cells[2]), str(path.relative_to(ROOT))
            except ValueError:
                continue
    return None, None


def host_facts() -> dict:
    """The host the CPU baseline ran on: logical CPUs, the ones this process
    may use, OMP_NUM_THREADS and the CPU model."""

    model = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)),
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS"), "cpu_model": model}


def traffic_from_profile(workload_name: str, kernel: str = "k_soap_mfma") -> tuple[float | None, str | None]:
    """HBM bytes per launch recorded in the committed counter summary."""

    path = ROOT / "profiles" / f"{kernel}_{workload_name}_traffic.txt"
    if not path.is_file():
        return None, None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch="):
            return float(line.split("=", 1)[1]), str(path.relative_to(ROOT))
    return None, None


def calibrate_copy(mib: int) -> int:
    import torch

    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": n * 4, "copy_bytes_written": n * 4, "launches": 5}))
    return 0


def peaks() -> dict:
    """Measured peak rates of this device, for reading the roofline against
    them: FP64 FMA on the vector ALU, FP64 16x16x4 MFMA, and a 1 GiB HBM copy
    (mdescriptor_amd/csrc/peaks.hip)."""

    import ctypes

    lib = ctypes.CDLL(str(ROOT / "mdescriptor_amd" / "_lib" / "libmdx_peaks.so"))
    lib.mdx_peak_run.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int, ctypes.POINTER(ctypes.c_double),
                                 ctypes.POINTER(ctypes.c_double)]
    lib.mdx_peak_run.restype = ctypes.c_int
    report = {}
    for which, name, size, repeats, unit, scale, published in (
            (0, "fp64_valu_fma", 0, 10, "TFLOP/s", 1e12, FP64_PEAK_TFLOPS),
            (1, "fp64_mfma_16x16x4", 0, 10, "TFLOP/s", 1e12, FP64_PEAK_TFLOPS),
            (2, "hbm_copy", 1 << 30, 20, "GB/s", 1e9, HBM_PEAK_GBS),
            (3, "hbm_copy_stream", 4 << 30, 20, "GB/s", 1e9, HBM_PEAK_GBS),
            (4, "hbm_read_stream", 4 << 30, 20, "GB/s", 1e9, HBM_PEAK_GBS),
            (5, "hbm_write_stream", 4 << 30, 20, "GB/s", 1e9, HBM_PEAK_GBS)):
        seconds, work = ctypes.c_double(), ctypes.c_double()
        rc = lib.mdx_peak_run(which, size, repeats, ctypes.byref(seconds), ctypes.byref(work))
        if rc != 0:
            raise RuntimeError(f"peak probe {name} failed with HIP error {rc}")
        rate = work.value / seconds.value / scale
        report[name] = {"value": rate, "unit": unit, "published_peak": published, "frac": rate / published,
                        "launch_ms": seconds.value * 1e3, "work_per_launch": work.value}
    return report


def end_to_end(plan, batch, repeats: int = 3) -> dict:
    """compute() from host arrays into a host matrix: upload, graph,
    expansion and the device-to-host copy of the whole output -- into the
    page-locked result the API returns by default, and into a caller's
    pageable array (staged by the library)."""

    report = {}
    for name, make_out in (("pinned", lambda: None),
                           ("pageable", lambda: np.empty((plan.rows(batch), plan.features), dtype=plan.dtype))):
        seconds = []
        for _ in range(repeats):
            out = make_out()
            t0 = time.perf_counter()
            values, timing = plan.compute(batch, out=out)
            seconds.append(time.perf_counter() - t0)
            del values, out
        best = min(seconds)
        report[name] = {"envs_per_s": batch.atoms / best, "seconds": best, "d2h_ms": timing["d2h_ms"],
                        "h2d_ms": timing["h2d_ms"], "device_ms": timing["total_ms"]}
    return report


def cpu_sample(index: int, workload):
    """The batch the CPU baseline times: the whole benchmark batch, except
    for configuration 5 (216,000 atoms, minutes of CPU time) a 46,656-atom
    cell of the same generator (same density, displacements and species)."""

    from mdescriptor_amd import workloads

    if index == 5:
        return workloads.liquid_si(18)
    return workload


def cpu_baseline(index: int, workload, alphas, betas, threads: int, options: dict | None, average: str,
                 budget_s: float = 30.0) -> dict:
    """The reference's SOAP (compiled in place under oracle/_ref; else the
    oracle port) on this host, as the reference runs it: structures in
    parallel (threads capped at the structure count) or, for one structure,
    centres in parallel."""

    from oracle import oracle

    kind = "reference" if oracle.reference_available() else "port"
    sample = cpu_sample(index, workload)
    p = workload.params
    batch = sample.batch
    times = []
    while True:
        t0 = time.perf_counter()
        oracle.soap(batch, species=p["species"], n_max=p["n_max"], l_max=p["l_max"], r_cut=p["r_cut"],
                    sigma=1.0, alphas=alphas, betas=betas, average=average, num_threads=threads,
                    kind="ref" if kind == "reference" else "oracle", options=options)
        times.append(time.perf_counter() - t0)
        if len(times) >= 3 or sum(times) + times[-1] > budget_s:
            break
    seconds = statistics.median(times)
    used = min(threads, batch.structures) if batch.structures > 1 else threads
    decomposition = (f"structure-parallel over {batch.structures} structures" if batch.structures > 1
                     else "centre-parallel over one structure")
    return {
        "value": batch.atoms / seconds,
        "unit": "atom-envs/s",
        "cores": used,
        "kind": kind,
        "sample": (f"{sample.name} ({batch.atoms} envs, {batch.structures} structures), {decomposition}, "
                   f"{used} of {threads} threads, float64 compute, median of {len(times)} run(s) of "
                   f"{seconds:.2f}s"),
        "host": host_facts(),
    }


def list_fill_bytes(graph_pairs: int, pairs: int, atoms: int, binned: int) -> int:
    """Algorithmic HBM bytes of one k_list_fill launch writing values and
    samples, each datum counted once: per graph pair its bin index (4 B); per
    binned image its atom, image index and position (32 B); per centre its
    pair range, first row, position, structure and atom offset (52 B); per
    kept pair its records (32 + 48 B)."""

    return 4 * graph_pairs + 32 * binned + 52 * atoms + 80 * pairs


def neighbor_list_bench(args, workload) -> dict:
    import ctypes

    from mdescriptor_amd import _hip

    batch = workload.batch
    ctx = _hip.Context(0)
    arrays = _hip._BatchArrays(batch)
    lib = ctx.lib
    rows = ctypes.c_int64()
    full = not args.half

    def build() -> int:
        ctx.check(lib.mdx_hip_neighbor_list(ctx.handle, ctypes.byref(arrays.view), float(args.nl_cutoff),
                                            1 if full else 0, 0, None, ctypes.byref(rows)))
        return int(rows.value)

    n = build()
    values = _hip.DeviceMemory(max(1, n) * 32)
    samples = _hip.DeviceMemory(max(1, n) * 48)
    offsets = _hip.DeviceMemory((batch.structures + 1) * 8)

    def fetch() -> None:
        ctx.check(lib.mdx_hip_neighbor_list_fetch(ctx.handle, None, ctypes.c_void_p(values.address),
                                                  ctypes.c_void_p(samples.address), ctypes.c_void_p(offsets.address)))

    for _ in range(args.warmup):
        build()
        fetch()
    timings = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        build()
        fetch()
        timings.append(_hip.neighbor_list_timing(ctx))
    _hip.DeviceMemory.synchronize()
    wall = time.perf_counter() - t0
    graph_ms = statistics.mean(t["graph_ms"] for t in timings)
    count_ms = statistics.mean(t["count_ms"] for t in timings)
    fill_ms = statistics.mean(t["fill_ms"] for t in timings)
    device_ms = graph_ms + count_ms + fill_ms
    graph_pairs = int(timings[-1]["graph_pairs"])
    fill_bytes = list_fill_bytes(graph_pairs, n, batch.atoms, int(timings[-1]["binned"]))
    achieved = fill_bytes / (fill_ms * 1e-3) / 1e9
    traffic, traffic_source = traffic_from_profile(f"{workload.name}_rc{args.nl_cutoff:g}", "k_list_fill")
    result = {
        "metric": f"NeighborList pairs/sec (rc {args.nl_cutoff:g}, {'full' if full else 'half'} list) on 1 MI355X",
        "value": n / (device_ms * 1e-3),
        "unit": "pairs/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": device_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64",
        "data": "synthetic (seeded generator, mdescriptor_amd/workloads.py)",
        "config": {
            "workload": workload.name,
            "structures": batch.structures,
            "atoms": batch.atoms,
            "cutoff": args.nl_cutoff,
            "full_neighbor_list": full,
            "self_pairs": False,
            "outputs": "values (f64 x4) + samples (i64 x6), device memory",
            "parallelism": "single-gpu",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic,
            "kernel": "k_list_fill (keep filter + record fill)",
            "bytes_per_launch": fill_bytes,
            "launch_ms": fill_ms,
            "traffic_source": traffic_source,
        },
        "breakdown": {
            "graph_ms": graph_ms,
            "count_ms": count_ms,
            "fill_ms": fill_ms,
            "graph_pairs": graph_pairs,
            "binned": int(timings[-1]["binned"]),
            "pairs": n,
            "wall_ms_per_step": 1e3 * wall / args.steps,
        },
    }
    if not args.no_cpu_baseline:
        from oracle import oracle

        kind = "reference" if oracle.reference_available() else "port"
        threads = args.cpu_threads or int(os.environ.get("OMP_NUM_THREADS") or 0) or len(os.sched_getaffinity(0))
        times = []
        while True:
            t1 = time.perf_counter()
            table, _ = oracle.neighbor_list(batch, args.nl_cutoff, full_neighbor_list=full,
                                            kind="ref" if kind == "reference" else "oracle", num_threads=threads)
            times.append(time.perf_counter() - t1)
            if len(times) >= 3 or sum(times) + times[-1] > 30.0:
                break
        seconds = statistics.median(times)
        result["cpu_baseline"] = {
            "value": len(table) / seconds,
            "unit": "pairs/s",
            "cores": threads,
            "kind": kind,
            "sample": f"full {workload.name} batch ({len(table)} pairs), median of {len(times)} run(s) of "
                      f"{seconds:.3f}s",
            "host": host_facts(),
        }
    values.free()
    samples.free()
    offsets.free()
    ctx.close()
    return result


def soap_bench(args, workload) -> dict:
    """One configuration's SOAP line: `steps` device-resident runs of the hot
    path (graph + expansion + write) after `warmup` untimed ones."""

    from mdescriptor_amd import _hip
    from mdescriptor_amd.descriptors.basis import basis_gto

    p = workload.params
    batch = workload.batch
    options, average = bench_options(args.options, p)
    alphas, betas = basis_gto(p["r_cut"], p["n_max"], p["l_max"])
    ctx = _hip.Context(0)
    plan = _hip.SoapPlan(ctx, species=p["species"], n_max=p["n_max"], l_max=p["l_max"], r_cut=p["r_cut"],
                         sigma=1.0, alphas=alphas, betas=betas, average=average, dtype=p["dtype"],
                         options=options)
    dbatch = _hip.DeviceBatch(plan, batch)
    itemsize = np.dtype(p["dtype"]).itemsize
    pitch = plan.features * itemsize
    out = _hip.DeviceMemory(dbatch.rows * pitch)
    frames = frame_positions(batch, FRAMES)
    on_device = [_hip.DeviceMemory(f.nbytes).from_host(f) for f in frames]

    outs = [out, _hip.DeviceMemory(dbatch.rows * pitch)]

    def step(k: int) -> dict:
        dbatch.set_positions(on_device[k % FRAMES].address)
        return dbatch.run(out.address, pitch)

    def frame(k: int) -> None:
        dbatch.run_frame(on_device[k % FRAMES].address, outs[k % 2].address, pitch)

    # one synchronous run per frame (first: it also brings the device up to
    # its clocks): per-stage device times for the breakdown and the expansion
    # kernel's launch time for the roofline
    for k in range(args.warmup):
        step(k)
    _hip.DeviceMemory.synchronize()
    timings = []
    t1 = time.perf_counter()
    for k in range(args.steps):
        timings.append(step(args.warmup + k))
    _hip.DeviceMemory.synchronize()
    sequential = time.perf_counter() - t1
    # pipelined frames (the timed figure): each call builds its frame's graph
    # on the context's second stream while the previous frame's expansion runs
    for k in range(args.warmup):
        frame(k)
    dbatch.wait()
    _hip.DeviceMemory.synchronize()
    t0 = time.perf_counter()
    for k in range(args.steps):
        frame(args.warmup + k)
    dbatch.wait()
    _hip.DeviceMemory.synchronize()
    elapsed = time.perf_counter() - t0

    for memory in on_device:
        memory.free()
    outs[1].free()

    envs = batch.atoms
    ms_per_step = 1e3 * elapsed / args.steps
    value = envs * args.steps / elapsed
    pairs = timings[-1]["pairs"]
    kbar = pairs / envs
    S, n, l_max = len(p["species"]), p["n_max"], p["l_max"]
    compression = (options or {}).get("compression", "off")
    # the fold and the spectrum run once per output row, except for outer
    # averages (once per centre, the spectra then averaged)
    rows = batch.structures if average != "off" else envs
    fold_rows = batch.structures if average == "inner" else envs
    total_flops = algorithmic_flops(envs, fold_rows, kbar, S, n, l_max, plan.features,
                                    1 if compression == "mu2" else S)
    per_env = total_flops / envs
    launches = max(1, int(timings[-1]["expansion_launches"]))
    flops_launch = total_flops / launches
    launch_ms = statistics.mean(t["expansion_ms"] for t in timings) / launches
    total_bytes = algorithmic_bytes(envs, rows, plan.features, itemsize)
    bytes_launch = total_bytes / launches
    bound = roofline_bound(total_flops, total_bytes)
    if bound == "mfma":
        achieved = flops_launch / (launch_ms * 1e-3) / 1e12
        peak, unit = FP64_PEAK_TFLOPS, "TFLOP/s"
    else:
        achieved = bytes_launch / (launch_ms * 1e-3) / 1e9
        peak, unit = HBM_PEAK_GBS, "GB/s"
    tiles = int(timings[-1]["expansion_tiles"])
    if tiles <= -1000:
        family = "k_soap_block"
        kernel = (f"k_soap_block ({-1000 - tiles} wavefronts per workgroup, one degree set each; register "
                  f"coefficients on 4x4x4 and 16x16x4 FP64 MFMA; expansion + beta + power spectrum + write)")
    elif tiles < 0:
        family = "k_soap_quad"
        kernel = f"k_soap_quad ({-tiles} wavefronts of 4x4x4 FP64 MFMA; expansion + beta + power spectrum + write)"
    elif tiles > 0:
        family = "k_soap_mfma"
        kernel = f"k_soap_mfma<{tiles}> (expansion + beta + power spectrum + write)"
    else:
        family = "k_soap_expand"
        kernel = "k_soap_expand (expansion + beta + power spectrum + write)"
    label = workload.name + ("" if args.options == "off" else f"_{args.options}")
    traffic, traffic_source = traffic_from_profile(label, family)
    profile_us, profile_source = profile_average_us(label, family)
    result = {
        "metric": METRIC,
        "value": value,
        "unit": "atom-envs/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64",
        "data": "synthetic (seeded generator, mdescriptor_amd/workloads.py)",
        "config": {
            "workload": workload.name,
            "structures": batch.structures,
            "atoms": envs,
            "species": p["species"],
            "n_max": n,
            "l_max": l_max,
            "r_cut": p["r_cut"],
            "sigma": 1.0,
            "average": average,
            "output_dtype": p["dtype"],
            "options": describe_options(options),
            "parallelism": "single-gpu",
        },
        "roofline": {
            "bound": bound,
            "achieved": achieved,
            "peak": peak,
            "unit": unit,
            "frac": achieved / peak,
            "traffic": traffic,
            "kernel": kernel,
            "flops_per_launch": flops_launch,
            "bytes_per_launch": bytes_launch,
            "fp64_frac": flops_launch / (launch_ms * 1e-3) / 1e12 / FP64_PEAK_TFLOPS,
            "hbm_frac": bytes_launch / (launch_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "roofline_ms": 1e3 * max(total_flops / (FP64_PEAK_TFLOPS * 1e12), total_bytes / (HBM_PEAK_GBS * 1e9)),
            "launch_ms": launch_ms,
            "traffic_source": traffic_source,
            "profile_launch_ms": None if profile_us is None else profile_us * 1e-3,
            "profile_source": profile_source,
        },
        "frames": f"{FRAMES} frames (seeded positions + N(0, {FRAME_JITTER} A) per coordinate), a new one each step",
        "stepping": "pipelined (mdx_hip_soap_run_frame: graph of frame k+1 beside the expansion of frame k)",
        "sequential": {
            "value": envs * args.steps / sequential,
            "ms_per_step": 1e3 * sequential / args.steps,
            "entry": "mdx_hip_batch_set_positions + mdx_hip_soap_run (one synchronous run per frame)",
        },
        "breakdown": {
            "graph_ms": statistics.mean(t["graph_ms"] for t in timings),
            "expansion_ms": statistics.mean(t["expansion_ms"] for t in timings),
            "device_total_ms": statistics.mean(t["total_ms"] for t in timings),
            "pairs": pairs,
            "kbar": kbar,
            "output_bytes": dbatch.rows * pitch,
            "output_gbs": dbatch.rows * pitch / (launch_ms * launches * 1e-3) / 1e9,
            "features": plan.features,
            "exps_per_env": kbar * (l_max + 1) * n,
            "flops_per_env": per_env,
            "H": (l_max + 1) ** 2,
        },
    }
    if not args.no_end_to_end:
        result["end_to_end"] = end_to_end(plan, batch)
    dbatch.close()
    plan.close()
    out.free()
    ctx.close()
    if not args.no_cpu_baseline:
        threads = args.cpu_threads or int(os.environ.get("OMP_NUM_THREADS") or 0) or len(os.sched_getaffinity(0))
        result["cpu_baseline"] = cpu_baseline(args.config, workload, alphas, betas, threads, options, average)
    return result


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--config", type=int, default=2, help="benchmark configuration 1-5 (default 2)")
    parser.add_argument("--options", choices=sorted(BENCH_OPTIONS), default="off",
                        help="SOAP options of the line (default: GTO, no weighting, compression off)")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--cpu-threads", type=int, default=0,
                        help="CPU baseline threads (default OMP_NUM_THREADS, else every CPU this process may use)")
    parser.add_argument("--no-end-to-end", action="store_true")
    parser.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB")
    parser.add_argument("--peaks", action="store_true", help="only measure this device's FP64 and HBM peak rates")
    parser.add_argument("--path", choices=("soap", "neighbor-list"), default="soap")
    parser.add_argument("--nl-cutoff", type=float, default=6.0)
    parser.add_argument("--half", action="store_true", help="neighbor-list path: half list")
    args = parser.parse_args()
    if args.calibrate_copy:
        return calibrate_copy(args.calibrate_copy)
    if args.peaks:
        print(json.dumps(peaks()))
        return 0
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; the SOAP path would shard by structure or "
                                   "centre range across GPUs, but no multi-GPU run is provided",
                          "n_gpus": args.gpus}))
        return 2

    from mdescriptor_amd import workloads

    workload = workloads.config(args.config)
    if args.path == "neighbor-list":
        print(json.dumps(neighbor_list_bench(args, workload)))
        return 0
    print(json.dumps(soap_bench(args, workload)))
    return 0


if __name__ == "__main__":
    sys.exit(main())
