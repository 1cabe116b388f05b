#!/usr/bin/env python3
"""Q4_K matvec effective HBM bandwidth on one MI355X.

Workload: Q4_K weights 14336 x 4096 (the 8B-class gate/up projection) times
one fp32 activation vector (decode, N = 1), plus the same matrix at N = 8
(the small-N path) reported beside it. A step is one kernel launch over one
weight matrix; weights and activations are resident in HBM before timing.

- Enough distinct weight copies rotate to exceed twice the 256 MB Infinity
  Cache, so every step streams its weights from HBM.
- Every weight copy is read once before timing (its pages mapped and
  translated), then a 64 MiB device copy is enqueued just before the start
  event, so the host has queued the timed launches before the GPU reaches
  them; HIP
  events on that stream bracket the timed steps, so the span holds GPU work
  only, also at the driver's 20 steps (a HIP graph of 20 launches measured
  0.5 us per step slower to start; --launch graph times one).
- `value` = algorithmic bytes per step (packed weights + 4*cols*N +
  4*rows*N) / average step time.
- read_ceiling: a plain streaming read of the same weight bytes over the
  same rotation and launch method (nya_hip_read), the time this matvec can
  approach; `structures` times every read shape of nya_hip_read_shaped
  (wavefronts, loads in flight, workgroups per CU, load kind, and a read
  that also stores its output as every kernel does), `sizes` the plain and
  the fastest read at 16.5 .. 264 MB with a fit of the per-dispatch floor
  and the streaming rate (--no-read-legs skips both).
- traffic: HBM bytes per dispatch of the N=1 and N=8 matvecs and the read,
  from rocprofv3 FETCH_SIZE and WRITE_SIZE passes over child runs of this
  script (before the parent touches the GPU), scaled by what the same
  counters read for a 256 MiB copy; roofline.traffic and n8.traffic carry
  them (--no-traffic skips the passes).
- cpu_baseline: the reference CPU provider (built from the reference sources
  into oracle/_ref) on the same weights, on this host's cores, at the
  reference's default thread count, at the CPUs this process may use and at
  one thread; else this repository's C port of the scalar path.
- resident: the provider's resident plan (a whole token forward on the GPU)
  on synthetic dense LLaMAs of two shapes: an 8B-class model (tg: decode
  tokens/s with logits every token, and its weight bytes per token over the
  token time) and TinyLlama 1.1B (tg128 and pp512, the reference's published
  end-to-end metrics); on the 8B-class model also batched verification of
  k draft tokens (one nya_compute_plan_verify) against k decode steps, and
  tg_at_4096 (a 4096-token prefill, then decode past it); a 12B-class Gemma
  layout through the Gemma branch (tg and tg_at_4096); `attention` times
  one token's attention of the 8B heads per launch, one workgroup per head
  against the split over positions, by cached length.
- --sweep prints one line per configuration instead: the decode, small-N and
  prefill shapes of the benchmarked models and the dense F32/F16/BF16 GEMM.
- prefill: the same matrix times 512 tokens through the fp16-MFMA prefill
  GEMM (one call = activation split + GEMM): useful TFLOP/s (2 M N K) against
  the dense fp16 MFMA peak, and the fp16 work the matrix cores issue (two
  activation pieces per token) beside it.

Prints one JSON line.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

from fyodor_amd import BF16, F16, F32, Q4_0, Q4_K, Q6_K, Q8_0, TYPE_NAMES, storage_bytes, synth  # noqa: E402
from fyodor_amd.hip import Graph, Kernels, Runtime  # noqa: E402

METRIC = "Q4_K matvec effective HBM GB/s (% of peak), 14336x4096, N=1 and N=8"
ROWS, COLS = 14336, 4096
PEAK_HBM_GBS = 8000.0
PEAK_FP16_TFLOPS = 2500.0      # dense fp16 MFMA, MI355X
# The prefill GEMM multiplies each token's activations as two fp16 pieces
# (hi + lo) by exact fp16 integer weights: two MFMA products per useful
# multiply-add.
PREFILL_PIECES = 2
PREFILL_TOKENS = 512
MALL_BYTES = 256 * 1024 * 1024


TRAFFIC_COUNTERS = ("FETCH_SIZE", "WRITE_SIZE")
CALIBRATION_BYTES = 256 << 20
PROBE_LAUNCHES = 40


def traffic_probe() -> int:
    """The launches the traffic counters are read on (run under rocprofv3 by
    measure_traffic): a 256 MiB copy of known read and write bytes, then the
    benchmark's N=1 and N=8 matvecs and the plain read, each over the same
    rotating weight copies as the timed steps."""
    rt, kern = Runtime(), Kernels()
    stream = rt.stream()
    src, dst = rt.malloc(CALIBRATION_BYTES), rt.malloc(CALIBRATION_BYTES)
    for _ in range(3):
        kern.copy(dst, src, CALIBRATION_BYTES, stream)
    rt.sync(stream)
    rt.free(src)
    rt.free(dst)
    wbytes = storage_bytes(Q4_K, ROWS, COLS)
    copies = max(2, math.ceil(2 * MALL_BYTES / wbytes) + 2)
    dev_w = kern.device_weights(synth.weights(Q4_K, ROWS, COLS, seed=1234), Q4_K, ROWS, COLS)
    weights = []
    for _ in range(copies):
        p = rt.malloc(wbytes)
        rt.upload(p, dev_w)
        weights.append(p)
    x8 = synth.activations(8, COLS, seed=1234)
    x_dev, y_dev, sink = rt.malloc(x8.nbytes), rt.malloc(8 * ROWS * 4), rt.malloc(4096)
    rt.upload(x_dev, x8)
    for batch in (1, 8):
        for i in range(PROBE_LAUNCHES):
            kern.matmul(weights[i % copies], Q4_K, ROWS, COLS, x_dev, y_dev, batch, 0, 0, stream)
    for i in range(PROBE_LAUNCHES):
        kern.read(weights[i % copies], wbytes, sink, stream)
    rt.sync(stream)
    print(json.dumps({"copy": "copy16", "n1": kern.kernel_name(Q4_K, ROWS, COLS, 1),
                      "n8": kern.kernel_name(Q4_K, ROWS, COLS, 8), "read": "read16"}), flush=True)
    return 0


def measure_traffic(timeout_s: float = 120.0) -> dict:
    """HBM bytes per launch, measured in this run: one rocprofv3 pass per
    counter (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch) over
    traffic_probe() in a child process, each scaled by what it reads on the
    256 MiB copy (FETCH_SIZE counts half the bytes on gfx950). Run before this
    process touches the GPU. Returns {"n1": bytes, "n8": bytes, "read": bytes,
    ...} or {"error": why}."""
    import csv
    import shutil
    import signal
    import statistics
    import subprocess
    import tempfile

    prof = shutil.which("rocprofv3")
    if not prof:
        return {"error": "rocprofv3 not found"}
    medians, kern_names = {}, None
    for counter in TRAFFIC_COUNTERS:
        out_dir = tempfile.mkdtemp(prefix="fy_traffic_", dir="/tmp")
        cmd = [prof, "--pmc", counter, "--output-format", "csv", "-d", out_dir, "-o", "run", "--",
               sys.executable, str(REPO / "bench.py"), "--traffic-probe"]
        env = dict(os.environ, TMPDIR="/tmp")
        proc = subprocess.Popen(cmd, cwd="/tmp", env=env, stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                                start_new_session=True)
        try:
            out_text, err = proc.communicate(timeout=timeout_s)
        except subprocess.TimeoutExpired:
            os.killpg(proc.pid, signal.SIGKILL)
            proc.wait()
            shutil.rmtree(out_dir, ignore_errors=True)
            return {"error": f"rocprofv3 --pmc {counter} did not finish in {timeout_s:.0f} s"}
        rows = []
        for path in Path(out_dir).rglob("*counter_collection.csv"):
            with open(path) as f:
                rows += list(csv.DictReader(f))
        shutil.rmtree(out_dir, ignore_errors=True)
        if not rows:
            tail = err.decode(errors="replace").strip().splitlines()[-1:] if err else []
            return {"error": f"rocprofv3 --pmc {counter} exited {proc.returncode} without counters {tail}"}
        if kern_names is None:
            names = [l for l in out_text.decode(errors="replace").splitlines() if l.startswith("{")]
            if not names:
                return {"error": f"rocprofv3 --pmc {counter}: the probe printed no kernel names"}
            kern_names = json.loads(names[-1])
        per_kernel = {}
        for r in rows:
            if r.get("Counter_Name") == counter:
                per_kernel.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
        for key, pattern in kern_names.items():
            vals = [v for name, vs in per_kernel.items()
                    if pattern in name.replace("(anonymous namespace)", "").split("(")[0] for v in vs]
            if not vals:
                return {"error": f"no {counter} dispatches of {pattern}"}
            medians[(key, counter)] = statistics.median(vals) * 1024.0
    fetch_scale = CALIBRATION_BYTES / medians[("copy", "FETCH_SIZE")]
    write_scale = CALIBRATION_BYTES / medians[("copy", "WRITE_SIZE")]
    out = {key: int(round(medians[(key, "FETCH_SIZE")] * fetch_scale + medians[(key, "WRITE_SIZE")] * write_scale))
           for key in kern_names if key != "copy"}
    out["scale"] = {"FETCH_SIZE": round(fetch_scale, 5), "WRITE_SIZE": round(write_scale, 5)}
    out["source"] = ("median per dispatch of rocprofv3 --pmc FETCH_SIZE and --pmc WRITE_SIZE (separate child runs "
                     f"of bench.py --traffic-probe, {PROBE_LAUNCHES} launches each over the rotating copies), "
                     f"scaled by the counters on a {CALIBRATION_BYTES >> 20} MiB copy")
    return out


def device(rt) -> str:
    """The device's name, or its compute-unit count when it reports none."""
    name = rt.device_name()
    return name if name else f"gfx950, {rt.attribute(63)} CUs"   # 63: hipDeviceAttributeMultiprocessorCount


def algorithmic_bytes(rows: int, cols: int, batch: int) -> int:
    return storage_bytes(Q4_K, rows, cols) + 4 * cols * batch + 4 * rows * batch


class Settle:
    """A 64 MiB device copy enqueued before a start event: the GPU is busy
    for tens of microseconds while the host submits what follows, so the
    timed span starts with the first timed launch already queued. Before it,
    touch() reads every weight copy once (nya_hip_read), so the pages of all
    inputs are mapped and translated when timing starts, also where the
    timed steps outnumber the warmup steps (a larger copy here measured
    slower at 20 steps: it displaced those translations)."""

    BYTES = 64 << 20

    def __init__(self, rt, kern):
        self.rt, self.kern = rt, kern
        self.src, self.dst = rt.malloc(self.BYTES), rt.malloc(self.BYTES)
        self.sink = rt.malloc(1 << 20)

    def touch(self, buffers, stream):
        for p, nbytes in buffers:
            self.kern.read(p, nbytes, self.sink, stream)

    def __call__(self, stream):
        self.kern.copy(self.dst, self.src, self.BYTES, stream)

    def close(self):
        for p in (self.src, self.dst, self.sink):
            self.rt.free(p)


def time_launches(rt, stream, settle, launch, steps: int, warm: int, mode: str, touch=()) -> float:
    """Milliseconds per launch over `steps` launches launch(0..steps-1),
    after `warm` untimed ones, between HIP events that bracket GPU work only
    (the settle copy runs before the start event while the host queues the
    launches; `touch`: (pointer, bytes) of the input buffers, read once
    before it). mode "stream": direct launches; "graph": one HIP graph."""
    graph = Graph(rt, stream, [lambda i=i: launch(i) for i in range(steps)]) if mode == "graph" else None
    for i in range(warm):
        launch(i)
    settle.touch(touch, stream)
    rt.sync(stream)
    start, end = rt.event(), rt.event()
    settle(stream)
    rt.record(start, stream)
    if graph:
        graph.launch()
    else:
        for i in range(steps):
            launch(i)
    rt.record(end, stream)
    ms = rt.elapsed_ms(start, end)
    rt.sync(stream)
    if graph:
        graph.close()
    return ms / steps


def time_steps(rt, kern, stream, settle, weights, x_dev, y_dev, batch, steps, warmup, mode, work, work_bytes):
    """Average milliseconds per step over `steps` timed launches."""
    copies = len(weights)

    def launch(i):
        kern.matmul(weights[i % copies], Q4_K, ROWS, COLS, x_dev, y_dev, batch, work, work_bytes, stream)

    wbytes = storage_bytes(Q4_K, ROWS, COLS)
    return time_launches(rt, stream, settle, launch, steps, warmup, mode, [(p, wbytes) for p in weights])


def read_ceiling(rt, kern, stream, settle, weights, steps, warmup, mode, matvec_ms, shapes=True, sizes=True) -> dict:
    """The plain streaming read of the same weight bytes, same rotation and
    launch method as the timed matvec steps."""
    wbytes = storage_bytes(Q4_K, ROWS, COLS)
    sink = rt.malloc(1 << 20)   # the store form writes 256 bytes per workgroup
    copies = len(weights)

    def launch(i):
        kern.read(weights[i % copies], wbytes, sink, stream)

    ms = time_launches(rt, stream, settle, launch, steps, warmup, mode, [(p, wbytes) for p in weights])
    out = {"kernel": "read16 (nya_hip_read)", "bytes": wbytes, "us_per_step": round(ms * 1e3, 3),
           "GBps": round(wbytes / (ms * 1e-3) / 1e9, 2), "frac": round(wbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
           "matvec_over_read": round(matvec_ms / ms, 4)}
    if shapes:
        out["structures"] = read_structures(rt, kern, stream, settle, weights, wbytes, sink)
    if sizes:
        best = out.get("structures", {}).get("best")
        out["sizes"] = read_sizes(rt, kern, stream, settle, weights[0], wbytes, sink, best)
    rt.free(sink)
    return out


# Read structures tried at the matrix's size: (wavefronts per workgroup,
# 16-byte loads in flight per lane), workgroups per CU, and where the loads
# land (0 registers, non-temporal; 1 registers, default cache policy; 2 LDS).
READ_SHAPES = [(4, 32), (4, 16), (8, 16), (8, 8), (16, 8), (16, 4)]
READ_MODES = {0: "nontemporal", 1: "default", 2: "lds", 3: "nontemporal+store"}
# Read sizes as multiples of the matrix's bytes (16.5 .. 264 MB).
READ_SIZE_FACTORS = (0.5, 1, 2, 4, 8)


def read_structures(rt, kern, stream, settle, weights, wbytes, sink, steps: int = 200) -> dict:
    """Every read shape over the same rotating weight copies as the matvec:
    microseconds per launch, and the fastest."""
    copies = len(weights)
    table = []
    for waves, depth in READ_SHAPES:
        for per_cu in (1, 2):
            for mode in READ_MODES:
                def launch(i, w=waves, d=depth, c=per_cu, m=mode):
                    kern.read_shaped(weights[i % copies], wbytes, sink, w, d, c, m, stream)
                ms = time_launches(rt, stream, settle, launch, steps, 10, "stream", [(p, wbytes) for p in weights])
                table.append({"waves": waves, "depth": depth, "per_cu": per_cu, "loads": READ_MODES[mode],
                              "us_per_step": round(ms * 1e3, 3),
                              "frac": round(wbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)})
    best = min((r for r in table if r["loads"] != READ_MODES[3]), key=lambda r: r["us_per_step"])
    best_store = min((r for r in table if r["loads"] == READ_MODES[3]), key=lambda r: r["us_per_step"])
    return {"bytes": wbytes, "steps": steps, "best": best, "best_with_store": best_store, "table": table}


def read_sizes(rt, kern, stream, settle, src_weights, wbytes, sink, best, steps: int = 200) -> dict:
    """The plain read (and the fastest structure at the matrix's size) over
    16.5 .. 264 MB, each size over rotating copies that exceed twice the
    Infinity Cache, plus a least-squares line us = floor + bytes / rate:
    the per-dispatch floor and the streaming rate."""
    sizes = [int(wbytes * f) // 1024 * 1024 for f in READ_SIZE_FACTORS]
    need = max(s * (math.ceil(2 * MALL_BYTES / s) + 1) for s in sizes)
    arena = rt.malloc(need)
    # Fill the arena with the matrix's own bytes (data-dependent power
    # stays that of the matvec's inputs).
    for off in range(0, need, wbytes):
        kern.copy(arena + off, src_weights, min(wbytes, need - off) // 16 * 16, stream)
    rt.sync(stream)
    legs = {"read16": lambda p, n: kern.read(p, n, sink, stream)}
    if best:
        legs["best"] = lambda p, n: kern.read_shaped(p, n, sink, best["waves"], best["depth"], best["per_cu"],
                                                    {v: k for k, v in READ_MODES.items()}[best["loads"]], stream)
    out = {}
    for name, fn in legs.items():
        rows = []
        for s in sizes:
            copies = math.ceil(2 * MALL_BYTES / s) + 1
            ptrs = [arena + k * s for k in range(copies)]
            ms = time_launches(rt, stream, settle, lambda i: fn(ptrs[i % copies], s), steps, 10, "stream",
                               [(p, s) for p in ptrs])
            rows.append({"bytes": s, "us_per_step": round(ms * 1e3, 3),
                         "frac": round(s / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)})
        xs = np.array([r["bytes"] for r in rows], dtype=np.float64)
        ts = np.array([r["us_per_step"] for r in rows], dtype=np.float64)
        slope, floor = np.polyfit(xs, ts, 1)
        out[name] = {"table": rows, "fit": {"floor_us": round(float(floor), 3),
                                            "stream_GBps": round(1e-3 / float(slope), 1),
                                            "stream_frac": round(1e-3 / float(slope) / PEAK_HBM_GBS, 4)}}
    rt.free(arena)
    return out


def call_latency(kern, rt, stream, weights, x_dev, y_dev, host_w: np.ndarray, x_host: np.ndarray,
                 calls: int = 200) -> dict:
    """Wall time of single N=1 calls, each waited for, at the two boundaries:
    nya_hip_matmul on device buffers plus a stream synchronize, and the
    provider's matvec on host buffers (x staged and copied up, the kernel
    writing y into pinned host memory, one synchronize; the engine's
    contract, rocm/rocm.c:111-139) with the weights already in its cache."""
    abi = []
    for i in range(calls + 5):
        t0 = time.perf_counter()
        kern.matmul(weights[i % len(weights)], Q4_K, ROWS, COLS, x_dev, y_dev, 1, 0, 0, stream)
        rt.sync(stream)
        abi.append(time.perf_counter() - t0)
    from fyodor_amd import Compute
    host = []
    with Compute("rocm") as c:
        c.matvec_typed(host_w, ROWS, COLS, Q4_K, x_host)          # uploads the packed weights once
        for _ in range(calls + 5):
            t0 = time.perf_counter()
            c.matvec_typed(host_w, ROWS, COLS, Q4_K, x_host)
            host.append(time.perf_counter() - t0)
    med_abi, med_host = float(np.median(abi[5:])), float(np.median(host[5:]))
    return {"abi_us": round(med_abi * 1e6, 2), "provider_host_us": round(med_host * 1e6, 2),
            "provider_host_GBps": round(algorithmic_bytes(ROWS, COLS, 1) / med_host / 1e9, 2),
            "sample": f"median of {calls} N=1 calls of each, one at a time; the ABI calls rotate over the "
                      f"{len(weights)} weight copies, the provider reuses its one cached copy"}


def host_cpu() -> dict:
    """The host CPU as /proc/cpuinfo and sysfs describe it, and the SIMD path
    the reference provider selects on it (backend/core/cpu_kernels.c:91-100:
    AVX-512 F+BW, else AVX2+F16C, else scalar)."""
    info, flags = {}, set()
    try:
        for line in open("/proc/cpuinfo"):
            key, _, value = line.partition(":")
            key = key.strip()
            if key in ("model name", "vendor_id", "cpu family", "model", "stepping") and key not in info:
                info[key] = value.strip()
            elif key == "flags" and not flags:
                flags = set(value.split())
    except OSError:
        pass
    isa = "scalar"
    if {"avx2", "f16c"} <= flags:
        isa = "avx512" if {"avx512f", "avx512bw"} <= flags else "avx2"
    model = info.get("model name", "unknown")
    ident = "family {} model {} stepping {}".format(info.get("cpu family", "?"), info.get("model", "?"),
                                                   info.get("stepping", "?"))
    return {"model": f"{model} ({info.get('vendor_id', '?')}, {ident})", "isa": isa,
            "online_cpus": os.cpu_count() or 1, "affinity_cpus": len(os.sched_getaffinity(0)),
            "l3_bytes": l3_bytes()}


def l3_bytes() -> int:
    """Total last-level cache of the host: the sum over distinct L3
    instances in sysfs (0 when sysfs does not say)."""
    seen, total = set(), 0
    base = Path("/sys/devices/system/cpu")
    for cache in base.glob("cpu[0-9]*/cache/index[0-9]*"):
        try:
            if (cache / "level").read_text().strip() != "3":
                continue
            shared = (cache / "shared_cpu_list").read_text().strip()
            if shared in seen:
                continue
            seen.add(shared)
            size = (cache / "size").read_text().strip().upper()
            total += int(size[:-1]) * {"K": 1 << 10, "M": 1 << 20}.get(size[-1], 1) if size[-1] in "KM" else int(size)
        except (OSError, ValueError):
            continue
    return total


def cpu_baseline(weights_host: np.ndarray, x: np.ndarray, y_gpu: np.ndarray, seconds: float) -> dict:
    """The reference CPU provider (or the C port) on the same workload: at
    the reference's default thread count (NYA_CPU_THREADS unset: online
    CPUs, at most 64, backend/core/cpu_backend.c:113-151), at the CPUs this
    process may run on, and at one thread. The weights rotate over enough
    host copies to exceed twice the host's L3."""
    sys.path.insert(0, str(REPO))
    from oracle import Oracle, Reference  # the oracle; only this leg uses it

    host = host_cpu()
    default_threads = min(host["online_cpus"], 64)
    affinity = host["affinity_cpus"]
    n_copies = max(2, math.ceil(2 * host["l3_bytes"] / weights_host.nbytes) + 1)
    copies = [weights_host] + [weights_host.copy() for _ in range(n_copies - 1)]
    y = np.empty(ROWS, dtype=np.float32)
    kind = "reference" if Reference.available() else "port"
    ref = Reference() if kind == "reference" else None
    orc = None if ref else Oracle()

    def leg(n, budget: float, cap: int):
        """Median seconds per matvec and the output of the first call; n None:
        the provider's own default thread count."""
        ctx = None
        if ref:
            # The provider reads its thread count when created
            # (backend/core/cpu_backend.c:147-151).
            saved = os.environ.pop("NYA_CPU_THREADS", None)
            if n is not None:
                os.environ["NYA_CPU_THREADS"] = str(n)
            ctx = ref.cpu_provider()
            os.environ.pop("NYA_CPU_THREADS", None)
            if saved is not None:
                os.environ["NYA_CPU_THREADS"] = saved

            def run(w):
                ref.provider_matmul(ctx, w, Q4_K, x, ROWS, COLS, 1, y)
        else:
            def run(w):
                y[:] = orc.matmul(w, Q4_K, x, ROWS, COLS, 1, threads=n or default_threads)[0]
        run(copies[0])
        first = y.copy()
        run(copies[1])
        times, i, began = [], 0, time.perf_counter()
        while (time.perf_counter() - began < budget or len(times) < 5) and len(times) < cap:
            t0 = time.perf_counter()
            run(copies[i % len(copies)])
            times.append(time.perf_counter() - t0)
            i += 1
        if ctx is not None:
            ref.free(ctx)
        return float(np.median(times)), len(times), first

    nbytes = algorithmic_bytes(ROWS, COLS, 1)
    med, count, y_cpu = leg(None, seconds * 0.5, 5000)
    med_a, count_a, _ = leg(affinity, seconds * 0.3, 5000)
    med1, count1, _ = leg(1, seconds * 0.2, 200)
    parity = float(np.linalg.norm(y_gpu.astype(np.float64) - y_cpu) / np.linalg.norm(y_cpu.astype(np.float64)))
    return {
        "value": round(nbytes / med / 1e9, 2), "unit": "GB/s", "cores": default_threads, "kind": kind,
        "sample": f"{count} Q4_K 14336x4096 N=1 matvecs over {n_copies} rotating host copies of the same "
                  f"synthetic weights (more than twice the host's {host['l3_bytes'] >> 20} MiB of L3), median "
                  f"time {med * 1e3:.3f} ms, at the reference's default thread count (online CPUs capped at 64)"
                  + (" (reference backend/core/cpu_backend.c provider)" if kind == "reference"
                     else " (scalar C port, rows split over threads)"),
        "affinity": {"value": round(nbytes / med_a / 1e9, 2), "unit": "GB/s", "cores": affinity,
                     "sample": f"{count_a} matvecs of the same workload on the {affinity} CPUs this process may "
                               f"use, median time {med_a * 1e3:.3f} ms"},
        "one_thread": {"value": round(nbytes / med1 / 1e9, 2), "unit": "GB/s", "cores": 1,
                       "sample": f"{count1} matvecs of the same workload, median time {med1 * 1e3:.3f} ms"},
        "isa": host["isa"] if kind == "reference" else "scalar",
        "cpu_model": host["model"],
        "online_cpus": host["online_cpus"],
        "parity_rel_l2_vs_gpu": parity,
    }


def prefill(rt, kern, stream, settle, weights, steps: int, m: int = PREFILL_TOKENS) -> dict:
    """Q4_K 14336x4096 times m tokens on the prefill GEMM."""
    x = synth.activations(m, COLS, seed=99)
    x_dev, y_dev = rt.malloc(x.nbytes), rt.malloc(4 * ROWS * m)
    rt.upload(x_dev, x)
    need = kern.workspace_bytes(Q4_K, ROWS, COLS, m)
    work = rt.malloc(need)
    copies = len(weights)

    def launch(i):
        kern.matmul(weights[i % copies], Q4_K, ROWS, COLS, x_dev, y_dev, m, work, need, stream)

    wbytes = storage_bytes(Q4_K, ROWS, COLS)
    ms = time_launches(rt, stream, settle, launch, steps, 2, "stream", [(p, wbytes) for p in weights])
    for p in (x_dev, y_dev, work):
        rt.free(p)
    useful = 2.0 * ROWS * COLS * m / (ms * 1e-3) / 1e12          # 2 M N K per call
    issued = useful * PREFILL_PIECES                               # fp16 work on the matrix cores
    return {
        "workload": f"Q4_K {ROWS}x{COLS} x {m} tokens (prefill GEMM)", "kernel": kern.kernel_name(Q4_K, ROWS, COLS, m),
        "ms_per_call": round(ms, 5), "calls": steps, "useful_tflops": round(useful, 2),
        "roofline": {"bound": "mfma", "achieved": round(useful, 2), "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(useful / PEAK_FP16_TFLOPS, 4)},
        "issued": {"tflops": round(issued, 2), "frac": round(issued / PEAK_FP16_TFLOPS, 4),
                   "note": "fp16 MFMA work including the second activation piece of every token"},
    }


# Resident plan workloads: dense LLaMAs with a Q4_K_M-like type mix (Q4_K
# attention, gate and up; Q6_K down and output; Q4_K embedding), and a
# Gemma layout.
# "llama-8b": embedding 4096, 32 heads of 128 with 8 KV heads, feed-forward
# 14336, 32 blocks, vocabulary 128256. "tinyllama-1.1b": embedding 2048, 32
# heads of 64 with 4 KV heads, feed-forward 5632, 22 blocks, vocabulary
# 32000 — the model of the reference's published end-to-end table
# (backend/README.md:796-803: tg128 and pp512 tokens/s).
RESIDENT_TYPES = {"embedding": Q4_K, "output": Q6_K, "attention": Q4_K, "gate_up": Q4_K, "down": Q6_K}
# The tied Gemma embedding is also the vocabulary matrix: Q6_K, as the
# output matrices here.
GEMMA_TYPES = {"embedding": Q6_K, "output": Q6_K, "attention": Q4_K, "gate_up": Q4_K, "down": Q6_K}
RESIDENT_MODELS = {
    "llama-8b": dict(embedding=4096, heads=32, kv_heads=8, hidden=14336, blocks=32, vocabulary=128256),
    "tinyllama-1.1b": dict(embedding=2048, heads=32, kv_heads=4, hidden=5632, blocks=22, vocabulary=32000),
    # A 12B-class Gemma layout (Gemma 3 12B's published dimensions: 48
    # blocks of 16 heads / 8 KV heads of 256, five local 1024-position
    # windows to one global block, feed-forward 15360, 262144 tokens, tied
    # output), run through the Gemma branch with a final soft cap.
    "gemma-12b-class": dict(family="gemma", embedding=3840, heads=16, kv_heads=8, width=256, local_width=256,
                            hidden=15360, local=(1, 1, 1, 1, 1, 0) * 8, window=1024, vocabulary=262144,
                            shared_kv_layers=0, global_value=True, output_scales=(), softcap=30.0),
}


VERIFY_TOKENS = (1, 2, 4, 8, 16, 33)


LONG_CONTEXT = 4096


def resident(name: str, tg: int, pp: int, blocks: int | None = None, verify=(), long_tg: int = 0) -> dict:
    """The provider's resident plan on a synthetic model of `name`'s shape:
    tg = tokens/s of `tg` decode steps from position 0 (each with its logits
    downloaded and checked, as llama-bench's tg counts a generated token),
    pp = tokens/s of one plan_prefill of `pp` prompt tokens from position 0
    (logits of the last). Host wall clock around the plan calls; the plan
    is warmed first. HBM figure: weight bytes a decode step reads (every
    block's matrices, the output matrix, one embedding row) over its time."""
    from fyodor_amd import Compute
    from fyodor_amd.model import (GemmaModel, GemmaShape, LlamaModel, LlamaShape, Plan, gemma_tensors,
                                  llama_tensors)

    shape_args = dict(RESIDENT_MODELS[name])
    gemma = shape_args.pop("family", "llama") == "gemma"
    context = max(tg, pp) + 8
    if long_tg:
        context = max(context, LONG_CONTEXT + long_tg + 8)
    if gemma:
        if blocks:   # the first blocks, the last of them global
            shape_args["local"] = tuple(shape_args["local"][:blocks - 1]) + (0,)
        shape = GemmaShape(**shape_args, context=context, types=GEMMA_TYPES, seed=7)
        model = GemmaModel(shape, gemma_tensors(shape, shared_blocks=True))
        kinds = f"{sum(shape.local)} local ({shape.window}-position window) + {shape.blocks - sum(shape.local)} global"
        out = {"workload": (f"Gemma branch, embedding {shape.embedding}, {shape.heads} heads / {shape.kv_heads} KV of "
                            f"{shape.width}, feed-forward {shape.hidden} (GELU gate), {shape.blocks} blocks "
                            f"({kinds}), vocabulary {shape.vocabulary} tied, soft cap {shape.softcap}, Q4_K "
                            f"attention/gate/up + Q6_K down/embedding")}
    else:
        if blocks:
            shape_args["blocks"] = blocks
        shape = LlamaShape(**shape_args, context=context, types=RESIDENT_TYPES, seed=7)
        model = LlamaModel(shape, llama_tensors(shape, shared_blocks=True))
        out = {"workload": (f"dense LLaMA, embedding {shape.embedding}, {shape.heads} heads / {shape.kv_heads} KV "
                            f"of {shape.embedding // shape.heads}, feed-forward {shape.hidden}, {shape.blocks} "
                            f"blocks, vocabulary {shape.vocabulary}, Q4_K attention/gate/up + Q6_K down/output")}
    ids = [(7 * i + 11) % shape.vocabulary for i in range(max(tg, pp))]
    compute = Compute("rocm")
    try:
        t0 = time.perf_counter()
        plan = Plan(compute, model, shape.context)
        out["plan_open_s"] = round(time.perf_counter() - t0, 2)
        try:
            for i in range(8):
                plan.token(ids[i], i)
            if tg:
                before = plan.stats()["kernel_launches"]
                start = time.perf_counter()
                for i in range(tg):
                    plan.token(ids[i], i)
                wall = time.perf_counter() - start
                launches = (plan.stats()["kernel_launches"] - before) / tg
                # Every block's matrices and vectors, the output matrix (the
                # embedding itself when tied) and one embedding row.
                embd = next(a for a in model.arrays if a[0] == "token_embd.weight")
                wbytes = sum(a[3].nbytes for a in model.arrays if a[0] != "token_embd.weight") + \
                    embd[3].nbytes // shape.vocabulary + (embd[3].nbytes if gemma and shape.tied_output else 0)
                gbs = wbytes * tg / wall / 1e9
                out[f"tg{tg}"] = {"tokens_per_s": round(tg / wall, 2), "us_per_token": round(wall / tg * 1e6, 1),
                                  "weight_bytes_per_token": wbytes, "effective_gbs": round(gbs, 1),
                                  "hbm_frac": round(gbs / PEAK_HBM_GBS, 4), "launches_per_token": round(launches, 1),
                                  "logits_finite": bool(np.all(np.isfinite(plan.logits)))}
            if verify:
                # Batched verification (nya_compute_plan_verify): the target
                # runs k draft tokens at once and returns its greedy choice
                # after each; serial verification is k decode steps.
                step_us = out[f"tg{tg}"]["us_per_token"] if tg else None
                out["verify"] = {}
                for k in verify:
                    toks = ids[8:8 + k]
                    plan.verify(toks, 8)
                    reps = 20
                    start = time.perf_counter()
                    for _ in range(reps):
                        plan.verify(toks, 8)
                    wall = (time.perf_counter() - start) / reps
                    leg = {"us_per_call": round(wall * 1e6, 1), "target_tokens_per_s": round(k / wall, 1)}
                    if step_us:
                        leg["speedup_vs_serial_steps"] = round(k * step_us / (wall * 1e6), 2)
                    out["verify"][str(k)] = leg
            if long_tg:
                # Decode past a 4096-token context (prefilled first): the
                # attention reads 4096+ cached positions per layer.
                long_ids = [(7 * i + 11) % shape.vocabulary for i in range(LONG_CONTEXT + long_tg)]
                t0 = time.perf_counter()
                plan.prefill(long_ids[:LONG_CONTEXT], 0)
                prefill_s = time.perf_counter() - t0
                for i in range(LONG_CONTEXT, LONG_CONTEXT + 4):
                    plan.token(long_ids[i], i)
                start = time.perf_counter()
                for i in range(LONG_CONTEXT + 4, LONG_CONTEXT + long_tg):
                    plan.token(long_ids[i], i)
                wall = time.perf_counter() - start
                n = long_tg - 4
                out[f"tg_at_{LONG_CONTEXT}"] = {
                    "tokens_per_s": round(n / wall, 2), "us_per_token": round(wall / n * 1e6, 1),
                    "positions": [LONG_CONTEXT + 4, LONG_CONTEXT + long_tg - 1],
                    "prefill_4096_s": round(prefill_s, 3), "logits_finite": bool(np.all(np.isfinite(plan.logits)))}
            if pp:
                plan.prefill(ids[:pp], 0)
                start = time.perf_counter()
                plan.prefill(ids[:pp], 0)
                wall = time.perf_counter() - start
                out[f"pp{pp}"] = {"tokens_per_s": round(pp / wall, 2), "ms": round(wall * 1e3, 2)}
            out["device_weight_bytes"] = plan.stats()["weights_bytes"]
        finally:
            plan.close()
    finally:
        compute.close()
    return out


def attention_leg(heads: int = 32, kv_heads: int = 8, width: int = 128, layers: int = 32, steps: int = 200) -> dict:
    """One decode token's attention of the 8B-class head layout, timed per
    launch with events over back-to-back launches that rotate through
    `layers` distinct KV caches (every layer's cache is its own, as in a
    decode step): one workgroup per query head at 136 and 4096 positions, and
    the split form (the plan's splits: 512 / KV heads, 8 to 64) at 4096."""
    from fyodor_amd.hip import Kernels, Runtime
    rt, kern = Runtime(), Kernels()
    L = kern.lib
    up, sz = ctypes.c_uint64, ctypes.c_size_t
    L.nya_hip_attention.argtypes = [up, sz, up, up, up, up, up, sz, sz, sz, sz, sz, sz, ctypes.c_float, up]
    L.nya_hip_attention_split.argtypes = [up, sz, up, up, up, up, up, sz, sz, sz, sz, sz, sz, sz, ctypes.c_float, up]
    stream = rt.stream()
    max_length = LONG_CONTEXT + 64
    kv_bytes = max_length * kv_heads * width * 4
    rng = np.random.default_rng(3)
    cache = rng.standard_normal(max_length * kv_heads * width).astype(np.float32)
    keys, values = [], []
    for _ in range(layers):
        k, v = rt.malloc(kv_bytes), rt.malloc(kv_bytes)
        rt.upload(k, cache)
        rt.upload(v, cache)
        keys.append(k)
        values.append(v)
    q_stride = (heads + 2 * kv_heads) * width
    qd, od = rt.malloc(4 * q_stride), rt.malloc(4 * heads * width)
    rt.upload(qd, rng.standard_normal(q_stride).astype(np.float32))
    splits = min(64, max(8, 512 // kv_heads))
    part = rt.malloc(4 * heads * splits * (width + 2))
    pos = rt.malloc(4)
    scale = 1.0 / math.sqrt(width)
    out = {"workload": f"{heads} query heads / {kv_heads} KV heads of {width}, one token, {layers} rotating KV caches"}

    def time_it(length, split):
        rt.upload(pos, np.array([length - 1], dtype=np.int32))
        def launch(i):
            if split:
                st = L.nya_hip_attention_split(qd, q_stride, keys[i % layers], values[i % layers], od, part, pos, 1,
                                               heads, kv_heads, width, max_length, 0, splits, scale, stream)
            else:
                st = L.nya_hip_attention(qd, q_stride, keys[i % layers], values[i % layers], od, 0, pos, 1, heads,
                                         kv_heads, width, max_length, 0, scale, stream)
            assert st == 0
        for i in range(20):
            launch(i)
        rt.sync(stream)
        start, end = rt.event(), rt.event()
        rt.record(start, stream)
        for i in range(steps):
            launch(i)
        rt.record(end, stream)
        us = rt.elapsed_ms(start, end) / steps * 1e3
        rt.sync(stream)
        return round(us, 2)

    out["per_head_136_us"] = time_it(136, False)
    out["per_head_4096_us"] = time_it(LONG_CONTEXT, False)
    out["split_4096_us"] = time_it(LONG_CONTEXT, True)
    out["by_length"] = {str(n): {"per_head_us": time_it(n, False), "split_us": time_it(n, True)}
                        for n in (64, 136, 257, 512, 1024, 2048)}
    out["split_splits"] = splits
    out["split_4096_over_per_head_136"] = round(out["split_4096_us"] / out["per_head_136_us"], 3)
    out["kv_bytes_4096"] = 2 * LONG_CONTEXT * kv_heads * width * 4
    out["split_4096_GBps"] = round(out["kv_bytes_4096"] / (out["split_4096_us"] * 1e-6) / 1e9, 1)
    for p in keys + values + [qd, od, part, pos]:
        rt.free(p)
    return out


def resident_legs(tg: int, pp: int, blocks: int | None, long_tg: int = 36, models=None) -> dict:
    """Every resident model (or the named ones; then without the attention
    leg and with long_tg as given)."""
    names = models or list(RESIDENT_MODELS)
    legs = {name: resident(name, tg, pp if name == "tinyllama-1.1b" else 0, blocks,
                           VERIFY_TOKENS if name == "llama-8b" and not models else (),
                           long_tg if name != "tinyllama-1.1b" else 0) for name in names}
    if not models:
        legs["attention"] = attention_leg()
    legs["reference_published"] = {
        "tinyllama-1.1b": {"tg128": 205.48, "pp512": 1374.38, "hardware": "RTX 5060 Ti",
                           "source": "backend/README.md:796-803 (Stage 2 Fyodor CUDA resident)"}}
    legs["timing"] = "host wall clock around plan_token / plan_prefill calls; synthetic weights of the named shape"
    return legs


# The measured configurations: decode and small-N shapes (type, rows, cols,
# batches), then prefill GEMM shapes (type, rows, cols, tokens).
SWEEP_MATVEC = [
    (Q4_K, 14336, 4096, (1, 2, 4, 8)), (Q4_K, 4096, 4096, (1, 2, 4, 8)), (Q4_K, 1024, 4096, (1, 8)),
    (Q8_0, 4096, 4096, (1, 8)), (Q4_0, 4096, 4096, (1, 8)), (Q4_0, 11008, 4096, (1, 8)),
    (Q4_0, 4096, 11008, (1, 8)), (Q6_K, 4096, 14336, (1, 8)), (Q6_K, 128256, 4096, (1, 8)),
]
SWEEP_PREFILL = [(t, rows, 4096, m) for t in (Q4_K, Q8_0) for rows in (4096, 14336) for m in (512, 2048)]
# Dense weights at prefill batches (the fp32-MFMA GEMM): type, rows, cols, tokens.
SWEEP_DENSE = [(t, 4096, 4096, m) for t in (F32, F16, BF16) for m in (64, 512)]
PEAK_FP32_MFMA_TFLOPS = 157.3


def time_case(rt, kern, stream, settle, t, rows, cols, batch, steps):
    """Milliseconds per call of one matmul shape: direct launches behind the
    settle copy, over enough rotating weight copies that every call streams
    its weights from HBM."""
    wbytes = storage_bytes(t, rows, cols)
    copies = max(2, math.ceil(2 * MALL_BYTES / wbytes) + 1)
    dev = kern.device_weights(synth.weights(t, rows, cols, seed=7), t, rows, cols)
    weights = []
    for _ in range(copies):
        p = rt.malloc(wbytes)
        rt.upload(p, dev)
        weights.append(p)
    x = synth.activations(batch, cols, seed=8)
    x_dev, y_dev = rt.malloc(x.nbytes), rt.malloc(4 * rows * batch)
    rt.upload(x_dev, x)
    need = kern.workspace_bytes(t, rows, cols, batch)
    work = rt.malloc(max(need, 16))

    def launch(i):
        kern.matmul(weights[i % copies], t, rows, cols, x_dev, y_dev, batch, work, need, stream)

    ms = time_launches(rt, stream, settle, launch, steps, min(copies, 8), "stream", [(p, wbytes) for p in weights])
    for p in weights + [x_dev, y_dev, work]:
        rt.free(p)
    return ms


def sweep(rt, kern, stream, settle) -> int:
    """One JSON line per configuration: matvec / small-N effective HBM GB/s,
    prefill useful TFLOP/s (2 M N K per call)."""
    for t, rows, cols, batches in SWEEP_MATVEC:
        wbytes = storage_bytes(t, rows, cols)
        for batch in batches:
            steps = max(40, min(2000, int(4e9 / wbytes)))
            ms = time_case(rt, kern, stream, settle, t, rows, cols, batch, steps)
            nbytes = wbytes + 4 * cols * batch + 4 * rows * batch
            gbs = nbytes / (ms * 1e-3) / 1e9
            print(json.dumps({"sweep": "matvec", "type": TYPE_NAMES[t], "rows": rows, "cols": cols, "batch": batch,
                              "kernel": kern.kernel_name(t, rows, cols, batch), "calls": steps,
                              "us_per_call": round(ms * 1e3, 3), "GB/s": round(gbs, 1),
                              "frac_hbm": round(gbs / PEAK_HBM_GBS, 4)}), flush=True)
    for t, rows, cols, m in SWEEP_PREFILL:
        ms = time_case(rt, kern, stream, settle, t, rows, cols, m, 20)
        useful = 2.0 * rows * cols * m / (ms * 1e-3) / 1e12
        print(json.dumps({"sweep": "prefill", "type": TYPE_NAMES[t], "rows": rows, "cols": cols, "tokens": m,
                          "kernel": kern.kernel_name(t, rows, cols, m), "calls": 20,
                          "us_per_call": round(ms * 1e3, 2), "useful_tflops": round(useful, 1),
                          "frac_fp16": round(useful / PEAK_FP16_TFLOPS, 4),
                          "issued_frac_fp16": round(useful * PREFILL_PIECES / PEAK_FP16_TFLOPS, 4)}), flush=True)
    for t, rows, cols, m in SWEEP_DENSE:
        ms = time_case(rt, kern, stream, settle, t, rows, cols, m, 20)
        useful = 2.0 * rows * cols * m / (ms * 1e-3) / 1e12
        print(json.dumps({"sweep": "dense", "type": TYPE_NAMES[t], "rows": rows, "cols": cols, "tokens": m,
                          "kernel": kern.kernel_name(t, rows, cols, m), "calls": 20,
                          "us_per_call": round(ms * 1e3, 2), "tflops": round(useful, 1),
                          "frac_fp32_mfma": round(useful / PEAK_FP32_MFMA_TFLOPS, 4),
                          "weight_GBps": round(storage_bytes(t, rows, cols) / (ms * 1e-3) / 1e9, 1)}), flush=True)
    return 0


def calibrate_copy(rt, kern, stream, steps: int) -> int:
    """Copies of a known size: rocprofv3 FETCH_SIZE / WRITE_SIZE per
    dispatch divided into these bytes give the counters' scale factor."""
    nbytes = 256 << 20
    src, dst = rt.malloc(nbytes), rt.malloc(nbytes)
    for _ in range(steps):
        kern.copy(dst, src, nbytes, stream)
    rt.sync(stream)
    rt.free(src)
    rt.free(dst)
    print(json.dumps({"calibration": "nya_hip_copy", "read_bytes": nbytes, "write_bytes": nbytes, "launches": steps}))
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--launch", choices=["stream", "graph"], default="stream",
                    help="direct launches behind the settle copy (default), or one HIP graph per timed run")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-call-latency", action="store_true",
                    help="skip the per-call wall times at the C-ABI and provider boundaries")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the rocprofv3 FETCH_SIZE / WRITE_SIZE child runs that measure HBM bytes per launch")
    ap.add_argument("--traffic-probe", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--no-read-legs", action="store_true",
                    help="skip the read structures and read sizes beside the read ceiling")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only the plain 256 MiB device copy used to calibrate HBM byte counters")
    ap.add_argument("--prefill-steps", type=int, default=20, help="timed prefill GEMM calls (0: skip)")
    ap.add_argument("--prefill-only", action="store_true", help="run only the prefill GEMM measurement")
    ap.add_argument("--prefill-tokens", type=int, default=PREFILL_TOKENS,
                    help="tokens of the --prefill-only measurement (the line always uses 512)")
    ap.add_argument("--resident-tg", type=int, default=128, help="timed decode tokens of the resident plans (0: skip)")
    ap.add_argument("--resident-pp", type=int, default=512, help="prompt tokens of the timed resident prefill")
    ap.add_argument("--resident-blocks", type=int, default=0, help="override the resident models' block count")
    ap.add_argument("--resident-only", action="store_true", help="run only the resident plan measurements")
    ap.add_argument("--resident-models", default="",
                    help="with --resident-only: comma-separated models to run (" + ", ".join(RESIDENT_MODELS) +
                         "), decode only")
    ap.add_argument("--sweep", action="store_true",
                    help="time every decode, small-N and prefill configuration instead (one JSON line each)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this library has no multi-GPU path (a matrix's rows would be "
              "sharded across GPUs with no exchange between them). Run with --gpus 1.", file=sys.stderr)
        return 2

    if args.traffic_probe:
        return traffic_probe()
    # The counter passes run first: child processes started before this one
    # touches the GPU.
    traffic = measure_traffic() if not (args.no_traffic or args.sweep or args.prefill_only or args.resident_only
                                        or args.calibrate_copy) else {"error": "not measured (--no-traffic)"}
    if args.resident_only:
        models = [m for m in args.resident_models.split(",") if m]
        unknown = [m for m in models if m not in RESIDENT_MODELS]
        if unknown:
            print(f"unknown resident models: {unknown} (known: {list(RESIDENT_MODELS)})", file=sys.stderr)
            return 2
        legs = resident_legs(args.resident_tg, args.resident_pp, args.resident_blocks or None,
                             0 if models else 36, models or None)
        print(json.dumps({"resident": legs}), flush=True)
        return 0
    rt = Runtime()
    kern = Kernels()
    stream = rt.stream()
    if args.calibrate_copy:
        return calibrate_copy(rt, kern, stream, max(args.steps, 1))
    settle = Settle(rt, kern)
    if args.sweep:
        return sweep(rt, kern, stream, settle)
    wbytes = storage_bytes(Q4_K, ROWS, COLS)
    copies = max(2, math.ceil(2 * MALL_BYTES / wbytes) + 2)
    host_w = synth.weights(Q4_K, ROWS, COLS, seed=1234)
    dev_w = kern.device_weights(host_w, Q4_K, ROWS, COLS)
    weights = []
    for _ in range(copies):
        p = rt.malloc(wbytes)
        rt.upload(p, dev_w)
        weights.append(p)
    x8 = synth.activations(8, COLS, seed=1234)
    x_dev = rt.malloc(x8.nbytes)
    rt.upload(x_dev, x8)
    y_dev = rt.malloc(8 * ROWS * 4)
    work_bytes = max(kern.workspace_bytes(Q4_K, ROWS, COLS, b) for b in (1, 8))
    work = rt.malloc(max(work_bytes, 16))

    if args.prefill_only:
        print(json.dumps({"prefill": prefill(rt, kern, stream, settle, weights, max(args.prefill_steps, 1),
                                             args.prefill_tokens)}),
              flush=True)
        for p in weights + [work]:
            rt.free(p)
        return 0

    results = {}
    for batch in (1, 8):
        ms = time_steps(rt, kern, stream, settle, weights, x_dev, y_dev, batch, args.steps, args.warmup, args.launch,
                        work, kern.workspace_bytes(Q4_K, ROWS, COLS, batch))
        nbytes = algorithmic_bytes(ROWS, COLS, batch)
        results[batch] = (ms, nbytes / (ms * 1e-3) / 1e9, nbytes)

    # One plain N=1 call for the parity figure next to the CPU baseline.
    kern.matmul(weights[0], Q4_K, ROWS, COLS, x_dev, y_dev, 1, 0, 0, stream)
    rt.sync(stream)
    y1 = rt.download(y_dev, np.empty(ROWS, dtype=np.float32))

    ms1, gbs1, bytes1 = results[1]
    ms8, gbs8, bytes8 = results[8]
    line = {
        "metric": METRIC,
        "value": round(gbs1, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms1, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded Q4_K blocks, x ~ N(0,1))",
        "config": {"workload": "Q4_K matvec 14336x4096, N=1 (decode)", "rows": ROWS, "cols": COLS,
                   "batch": 1, "weight_copies": copies, "launch": args.launch,
                   "kernel": kern.kernel_name(Q4_K, ROWS, COLS, 1), "device": device(rt)},
        "roofline": {"bound": "hbm", "achieved": round(gbs1, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs1 / PEAK_HBM_GBS, 4), "traffic": traffic.get("n1"),
                     "algorithmic_bytes": bytes1},
        "n8": {"value": round(gbs8, 2), "unit": "GB/s", "ms_per_step": round(ms8, 6),
               "frac": round(gbs8 / PEAK_HBM_GBS, 4), "algorithmic_bytes": bytes8, "traffic": traffic.get("n8"),
               "kernel": kern.kernel_name(Q4_K, ROWS, COLS, 8)},
        "traffic": traffic,
    }
    line["read_ceiling"] = read_ceiling(rt, kern, stream, settle, weights, args.steps, args.warmup, args.launch, ms1,
                                        shapes=not args.no_read_legs, sizes=not args.no_read_legs)
    if not args.no_call_latency:
        line["call_latency"] = call_latency(kern, rt, stream, weights, x_dev, y_dev, host_w, x8[0].copy())
    if args.prefill_steps > 0:
        line["prefill"] = prefill(rt, kern, stream, settle, weights, args.prefill_steps)
    for p in weights + [work, x_dev, y_dev]:
        rt.free(p)
    settle.close()
    if args.resident_tg > 0:
        line["resident"] = resident_legs(args.resident_tg, args.resident_pp, args.resident_blocks or None)
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(host_w, x8[0].copy(), y1, args.cpu_seconds)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
