"""Benchmark of the gfx950 GDN decode step (one GPU).

    python bench.py [--steps K] [--warmup W] [--config NAME]

A step is one decode step (T=1) over one batch, updating the fp32 state in
place, with every input already resident in HBM.  The headline workload is
B=256 sequences of the qk16_v32 head layout (16 q/k heads, 32 v-heads,
K=V=128, q/k L2-norm on): 1,080,066,304 algorithmic bytes per step.

Steps run back to back and rotate over several layer states (as consecutive
GDN layers of a model do) totalling at least 1 GiB, so each step reads a
state that is no longer cached and pays for the write-back of the previous
step's dirty lines: the steady state of serving.  Prints ONE JSON line:

* ``value``: whole-job throughput in GB/s of algorithmic bytes, from the
  wall clock over K timed steps;
* ``roofline``: the decode kernel's achieved HBM GB/s, from HIP events
  around every timed launch on the launch stream, against MI355X's 8 TB/s;
  ``traffic`` is the measured HBM bytes per launch from the committed
  rocprofv3 counter summary, when there is one;
* ``b1``: time per decode step at B=1 (qk16_v32, L2-norm).  ``us_per_step``:
  steps back to back from a HIP graph, one per layer state (>= 1 GiB of
  states, so every step reads its state from HBM), HIP events around the
  replays: kernel plus launch gap per step, with the GPU never idle as in a
  model's decode loop.  ``kernel_trace``: rocprofv3 kernel-trace durations
  (the analogue of the reference's CUPTI timings) of isolated launches ~12 us
  apart and right after a 1 GiB read: a child process, started under
  ``rocprofv3 --kernel-trace`` before this process touches the GPU,
  launches every per-config shape through the product entry point, and its
  dispatches are attributed back to the shapes;
* ``per_config``: kernel times for every benchmark shape and for the
  reference's qk4_v8 definition at its workload batch sizes, plus bf16-state
  and multi-token (T = 2, 4) steps, in three regimes: steady (as above),
  warm (one state, repeatedly: cache-resident below 256 MiB) and cold (a
  1 GiB read evicts the caches just before the launch; the launch's own
  writes may still be in cache when it ends); ``us_*`` from events the
  kernel dispatch stamps (hipExtLaunchKernelGGL: ~2.5 us of their own
  overhead, so only meaningful above ~10 us), ``trace_us_*`` from the
  kernel trace;
* ``b1.kernel_trace.floor`` and ``b1.stamped.floor_same_timer``: each timer
  on reference kernels that move only the state bytes (an in-place
  read-modify-write of the B=1 state, and of the B=256 state under the
  stamped events) and on an empty kernel, so that the decode times read
  against the floor of their own traffic; ``b1.serving``: host-inclusive
  time per step of 48 back-to-back B=1 steps, eager and replayed from a
  HIP graph;
* ``cpu_baseline``: the reference's PyTorch-eager step (the oracle's
  loop-for-loop restatement) timed on this host's cores on a bounded sample;
* ``prefill``: the variable-length prefill workloads, each with the whole
  call's time and its three kernels' times (events the library records
  between its launches); ``prefill_roofline``: the largest workload's
  algorithmic FLOP rate against the bf16 MFMA peak and its preparation
  kernel's HBM rate; ``prefill_cpu_baseline``: the reference's prefill loop
  (the oracle) on a bounded sample, in tokens/s.

Algorithmic bytes per step: state read + write (B*HV*128*128*4*2, half that
for a bf16 state), and per token q and k (2*B*H*128*2), v (B*HV*128*2),
output (B*HV*128*2), a and b (2*B*HV*2); A_log and dt_bias (2*HV*4).
"""

from __future__ import annotations

import argparse
import csv
import ctypes
import json
import math
import os
import shutil
import statistics
import subprocess
import sys
import tempfile
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import flashinfer_competition_codebase_amd as gdn  # noqa: E402
from flashinfer_competition_codebase_amd import _lib  # noqa: E402
from flashinfer_competition_codebase_amd.build import (  # noqa: E402
    DECODE_SOURCES, PREFILL_SOURCES)
from flashinfer_competition_codebase_amd.build import sources_sha as _sources_sha  # noqa: E402

METRIC = ("GDN decode µs/step at B=1; achieved HBM GB/s (% of peak) at B=256")
PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0      # dense bf16 MFMA, MI355X
TRAFFIC_SUMMARY = ROOT / "profiles" / "gdn_decode_b256_qk16v32_traffic.json"
PREFILL_TRAFFIC_SUMMARY = ROOT / "profiles" / "gdn_prefill_traffic.json"

# name -> (B, H, HV, use_qk_l2norm)
CONFIGS = {
    "b1_qk16_v32_l2": (1, 16, 32, True),
    "b8_qk16_v32_l2": (8, 16, 32, True),
    "b64_qk16_v32_l2": (64, 16, 32, True),
    "b256_qk16_v32_l2": (256, 16, 32, True),
    "b128_qk8_v32_raw": (128, 8, 32, False),
}
REF_BATCHES = (1, 4, 8, 16, 32, 48, 64)


def step_bytes(B: int, H: int, HV: int, K: int = 128, V: int = 128, T: int = 1,
               state_elem: int = 4) -> int:
    """Algorithmic bytes of one launch: the state read and written once,
    q, k, v, output, a and b for each of T tokens, A_log and dt_bias."""
    return (B * HV * K * V * state_elem * 2 + T * (2 * B * H * K * 2 + B * HV * V * 2
            + B * HV * V * 2 + 2 * B * HV * 2) + 2 * HV * 4)


def make_device_inputs(B, H, HV, device, seed, T=1, state_dtype=torch.float32):
    """Seeded synthetic inputs generated on the device: q, k, v ~ N(0,1)
    bf16; state ~ N(0, 0.05^2) (fp32, or rounded to bf16); a, b ~ N(0,1)
    bf16 [B,T,HV]; A_log = log(U[1,16]); dt_bias ~ U[-1,1];
    scale = 1/sqrt(128)."""
    g = torch.Generator(device=device).manual_seed(seed)
    K = V = 128
    f = dict(device=device)
    q = torch.randn(B, T, H, K, generator=g, **f).to(torch.bfloat16)
    k = torch.randn(B, T, H, K, generator=g, **f).to(torch.bfloat16)
    v = torch.randn(B, T, HV, V, generator=g, **f).to(torch.bfloat16)
    state = torch.randn(B, HV, V, K, generator=g, **f).mul_(0.05).to(state_dtype)
    a = torch.randn(B, T, HV, generator=g, **f).to(torch.bfloat16)
    b = torch.randn(B, T, HV, generator=g, **f).to(torch.bfloat16)
    A_log = torch.log(torch.rand(HV, generator=g, **f) * 15.0 + 1.0)
    dt_bias = torch.rand(HV, generator=g, **f) * 2.0 - 1.0
    output = torch.empty(B, T, HV, V, dtype=torch.bfloat16, **f)
    return dict(q=q, k=k, v=v, state=state, A_log=A_log, a=a, dt_bias=dt_bias, b=b,
                scale=1.0 / math.sqrt(K), output=output, new_state=state)


class KernelStamps:
    """HIP events that a launch stamps with the kernel's own start and end
    timestamps (hipExtLaunchKernelGGL through gdn_decode_step_shaped), so the
    elapsed time is the kernel's duration, free of event-marker overhead.
    Uses the HIP runtime already loaded by torch (same soname)."""

    def __init__(self, n: int):
        self.hip = ctypes.CDLL("libamdhip64.so.7")
        self.start = [self._create() for _ in range(n)]
        self.stop = [self._create() for _ in range(n)]

    def _create(self):
        ev = ctypes.c_void_p()
        if self.hip.hipEventCreate(ctypes.byref(ev)) != 0:
            raise RuntimeError("hipEventCreate failed")
        return ev

    def elapsed_us(self, i: int) -> float:
        ms = ctypes.c_float()
        if self.hip.hipEventSynchronize(self.stop[i]) != 0:
            raise RuntimeError("hipEventSynchronize failed")
        if self.hip.hipEventElapsedTime(ctypes.byref(ms), self.start[i], self.stop[i]) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value * 1e3

    def between_us(self, a, b) -> float:
        ms = ctypes.c_float()
        if self.hip.hipEventElapsedTime(ctypes.byref(ms), a, b) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value * 1e3

    def close(self) -> None:
        for ev in self.start + self.stop:
            self.hip.hipEventDestroy(ev)


STEADY_BYTES = 1 << 30


def layer_states(state: torch.Tensor) -> list:
    """``state`` plus copies: at least two, and at least 1 GiB in total."""
    n = max(2, -(-STEADY_BYTES // (state.numel() * state.element_size())))
    return [state] + [state.clone() for _ in range(n - 1)]


def kernel_times_us(t, l2, iters, *, mode, flush=None):
    """Per-launch kernel durations in µs, stamped by the kernel dispatch
    itself, with the launch shape gdn_decode_step uses.

    steady: back-to-back launches rotating over ``layer_states``;
    warm: back-to-back launches on one state;
    cold: each launch right after reading a 1 GiB buffer (more than the
    32 MiB of L2 plus the 256 MiB MALL; a read leaves no dirty lines)."""
    B, T, HV = t["v"].shape[0], t["v"].shape[1], t["v"].shape[2]
    ns, waves, policy, _ = _lib.launch_shape(B, HV, T, t["state"].dtype == torch.bfloat16)
    states = layer_states(t["state"]) if mode == "steady" else [t["state"]]
    iters = max(iters, 2 * len(states)) if mode == "steady" else iters
    stamps = KernelStamps(iters)
    try:
        for i in range(iters):
            if mode == "cold":
                flush.sum()
            s = states[i % len(states)]
            gdn.kernel_hip_shaped(**{**t, "state": s, "new_state": s}, use_qk_l2norm=l2,
                                  rows_per_lane_group=ns, waves_per_block=waves,
                                  cache_policy=policy, start_event=stamps.start[i].value,
                                  stop_event=stamps.stop[i].value)
        torch.cuda.synchronize()
        d = [stamps.elapsed_us(i) for i in range(iters)]
        # steady: drop the first pass over the states (still warm from setup)
        return d[len(states):] if mode == "steady" else d
    finally:
        stamps.close()


def per_config_shapes():
    """(name, B, H, HV, use_qk_l2norm, T, state dtype) of every per-config
    shape: the benchmark configs, the reference's qk4_v8 definition at its
    workload batch sizes, bf16-state and multi-token steps."""
    f32, bf16 = torch.float32, torch.bfloat16
    shapes = [(n, *c, 1, f32) for n, c in CONFIGS.items()]
    shapes += [(f"qk4_v8_b{bb}", bb, 4, 8, False, 1, f32) for bb in REF_BATCHES]
    shapes += [(f"{n}_bf16_state", *CONFIGS[n], 1, bf16)
               for n in ("b1_qk16_v32_l2", "b8_qk16_v32_l2", "b256_qk16_v32_l2")]
    shapes += [(f"{n}_t{tt}", *CONFIGS[n], tt, f32)
               for n in ("b1_qk16_v32_l2", "b256_qk16_v32_l2") for tt in (2, 4)]
    # the shapes of FlashInfer's published decode tables (bf16 state at T = 1..4,
    # fp32 state, up to B = 512; findings/fi-gdn-decode-kernel.md:26-60)
    shapes += [(f"{n}_bf16_state_t{tt}", *CONFIGS[n], tt, bf16)
               for n in ("b1_qk16_v32_l2", "b256_qk16_v32_l2") for tt in (2, 4)]
    shapes += [("b512_qk16_v32_l2", 512, 16, 32, True, 1, f32),
               ("b512_qk16_v32_l2_bf16_state", 512, 16, 32, True, 1, bf16)]
    return shapes


# Kernel-name substrings in the trace: the decode kernel and the floor
# kernels of libgdn_calib.so.
TRACE_DECODE = "gdn_decode_"      # gdn_decode_k128 and gdn_decode_block
TRACE_RMW = "gdn_calib::rmw"
TRACE_EMPTY = "gdn_calib::empty"
TRACE_WARMUP = 5


def trace_child(device, manifest_path: str, iters: int) -> None:
    """The launches the kernel-trace leg records (run by ``kernel_trace_leg``
    under rocprofv3).  Per shape: warmup launches, steady launches rotating
    over layer states, then cold launches each right after a 1 GiB read, all
    through the product entry point ``kernel_hip``; then the floor kernels
    (the B=1 state's in-place read-modify-write, steady, and an empty kernel
    on the B=1 decode grid).  Writes the launch counts, in launch order, to
    ``manifest_path``."""
    flush = torch.ones(1 << 28, device=device)
    manifest = []
    for name, b_, h_, hv_, l2_, t_, sd_ in per_config_shapes():
        tc = make_device_inputs(b_, h_, hv_, device, seed=7, T=t_, state_dtype=sd_)
        for _ in range(TRACE_WARMUP):
            gdn.kernel_hip(**tc, use_qk_l2norm=l2_)
        states = layer_states(tc["state"])
        n_steady = max(iters, 2 * len(states))
        for i in range(n_steady):
            s_ = states[i % len(states)]
            gdn.kernel_hip(**{**tc, "state": s_, "new_state": s_}, use_qk_l2norm=l2_)
        for _ in range(iters):
            flush.sum()
            gdn.kernel_hip(**tc, use_qk_l2norm=l2_)
        torch.cuda.synchronize()
        # steady: the first pass over the states is still warm from setup
        manifest.append({"name": name, "warmup": TRACE_WARMUP, "steady": n_steady,
                         "steady_skip": len(states), "cold": iters})
        print(f"[trace] {name}: {TRACE_WARMUP} + {n_steady} + {iters} launches",
              file=sys.stderr, flush=True)
        del tc, states
    cal = Calib()
    bufs = layer_states(torch.zeros(32 * 128 * 128, device=device))
    n_rmw = max(iters, 2 * len(bufs))
    for i in range(n_rmw):
        cal.rmw(bufs[i % len(bufs)], None, None)
    _, _, _, b1_blocks = _lib.launch_shape(1, 32)
    for _ in range(iters):
        cal.empty(b1_blocks, None, None)
    torch.cuda.synchronize()
    floor = {"rmw": n_rmw, "rmw_skip": len(bufs), "empty": iters, "empty_blocks": b1_blocks}
    Path(manifest_path).write_text(json.dumps({"decode": manifest, "floor": floor}))


def attribute_kernel_trace(trace_csv, manifest: dict) -> dict:
    """Median kernel-trace duration (µs) per shape and regime: the decode
    dispatches of the trace, in start order, are the launches the manifest
    lists, in launch order."""
    rows = {TRACE_DECODE: [], TRACE_RMW: [], TRACE_EMPTY: []}
    with open(trace_csv) as f:
        for r in csv.DictReader(f):
            for key, lst in rows.items():
                if key in r["Kernel_Name"]:
                    lst.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    for lst in rows.values():
        lst.sort()
    dec = rows[TRACE_DECODE]
    need = sum(m["warmup"] + m["steady"] + m["cold"] for m in manifest["decode"])
    if len(dec) != need:
        raise ValueError(f"{len(dec)} decode dispatches in the trace, {need} launched")

    def med(span):
        return round(statistics.median((e - s) / 1e3 for s, e in span), 3)

    shapes, i = {}, 0
    for m in manifest["decode"]:
        i += m["warmup"]
        steady = dec[i + m["steady_skip"]: i + m["steady"]]
        i += m["steady"]
        cold = dec[i: i + m["cold"]]
        i += m["cold"]
        shapes[m["name"]] = {"steady": med(steady), "cold": med(cold),
                             "steady_avg": round(statistics.fmean(
                                 (e - s) / 1e3 for s, e in steady), 3),
                             "n_steady": len(steady), "n_cold": len(cold)}
    fl = manifest["floor"]
    floor = None
    if len(rows[TRACE_RMW]) == fl["rmw"] and len(rows[TRACE_EMPTY]) == fl["empty"]:
        floor = {"b1_rmw_us": med(rows[TRACE_RMW][fl["rmw_skip"]:]),
                 "empty_us": med(rows[TRACE_EMPTY]), "empty_blocks": fl["empty_blocks"]}
    return {"shapes": shapes, "floor": floor}


def kernel_trace_leg(iters: int, timeout_s: float = 300.0) -> dict:
    """rocprofv3 kernel-trace medians of the decode kernel per shape (steady
    and cold) and of the floor kernels: ``trace_child`` run as a separate
    program under ``rocprofv3 --kernel-trace``.  Called before this process
    initialises the GPU; skipped when this process itself runs under
    rocprofv3 (which sets ROCPROF_OUTPUT_PATH for the program it profiles)."""
    if "ROCPROF_OUTPUT_PATH" in os.environ:
        return {"skipped": "bench.py runs under rocprofv3"}
    exe = shutil.which("rocprofv3")
    if exe is None:
        return {"skipped": "rocprofv3 not on PATH"}
    with tempfile.TemporaryDirectory(prefix="gdn_trace_", dir="/tmp") as d:
        manifest = os.path.join(d, "manifest.json")
        cmd = [exe, "--kernel-trace", "--output-format", "csv", "-d", d, "-o", "trace", "--",
               sys.executable, str(ROOT / "bench.py"), "--trace-child", manifest,
               "--iters", str(iters)]
        sys.stderr.flush()
        try:
            # the child's output goes to stderr: stdout carries only the JSON line
            proc = subprocess.run(cmd, cwd="/tmp", env=dict(os.environ, TMPDIR="/tmp"),
                                  stdout=sys.stderr, stderr=sys.stderr, timeout=timeout_s)
        except subprocess.TimeoutExpired:
            return {"skipped": f"traced run exceeded {timeout_s:.0f} s"}
        traces = sorted(Path(d).rglob("*kernel_trace.csv"))
        # rocprofv3 may end with a signal after the program has finished and
        # its output is whole: the manifest and the trace decide.
        if not os.path.exists(manifest) or not traces:
            return {"skipped": f"traced run exited {proc.returncode} without a trace"}
        try:
            res = attribute_kernel_trace(traces[0], json.loads(Path(manifest).read_text()))
        except (OSError, ValueError, KeyError) as e:
            return {"skipped": f"trace not attributable: {e}"}
    res["timer"] = "rocprofv3 --kernel-trace, median per shape and regime"
    return res


def timed_steps(t, l2, steps, states):
    """Wall clock over ``steps`` back-to-back launches of the product entry
    point, rotating over ``states``, and the GPU time of the same region from
    one pair of HIP events on the launch stream (torch's current stream, the
    one ``kernel_hip`` launches on) around all of them: the average launch
    duration, gaps between back-to-back launches included, with nothing
    between the launches.  Returns (wall seconds, GPU µs per launch)."""
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    views = [{**t, "state": s, "new_state": s} for s in states]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for i in range(steps):
        gdn.kernel_hip(**views[i % len(views)], use_qk_l2norm=l2)
    stop.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall, start.elapsed_time(stop) * 1e3 / steps


def cpu_baseline(seconds: float):
    """The reference's eager PyTorch step (oracle_loop, a loop-for-loop
    restatement of solution/triton/kernel.py:72-118) on this host's cores,
    on a bounded sample of the B=256 qk16_v32 workload: the first Bs batch
    rows, repeated until about ``seconds`` of CPU work."""
    from oracle.gdn_decode_oracle import make_inputs, oracle_loop

    threads = host_threads()
    torch.set_num_threads(threads["affinity_cores"])
    torch.set_float32_matmul_precision("highest")
    Bs = 8
    t = make_inputs(Bs, 16, 32, seed=1003)
    oracle_loop(**t, use_qk_l2norm=True)           # warmup
    reps, elapsed = 0, 0.0
    t0 = time.perf_counter()
    while elapsed < seconds:
        oracle_loop(**t, use_qk_l2norm=True)
        reps += 1
        elapsed = time.perf_counter() - t0
    per_step = elapsed / reps
    t1 = make_inputs(1, 16, 32, seed=1000)
    b1 = []
    for _ in range(5):
        s = time.perf_counter()
        oracle_loop(**t1, use_qk_l2norm=True)
        b1.append((time.perf_counter() - s) * 1e6)
    return {
        "value": round(step_bytes(Bs, 16, 32) / per_step / 1e9, 4),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"a rate: B={Bs} of the B=256 qk16_v32 L2-norm workload ({Bs * 32} of its "
                   f"8192 heads; the per-head loop makes the rate independent of B), "
                   f"{reps} steps in {elapsed:.1f} s; {per_step * 1e3:.1f} ms per B={Bs} step, "
                   f"{per_step * 32e3:.0f} ms per B=256 step at this rate"),
        "b1_us_per_step": round(statistics.median(b1), 1),
        "cpu": _cpu_model(),
        "threads": {**threads, "torch_num_threads": torch.get_num_threads()},
    }


def host_threads() -> dict:
    """Host cores for the CPU baseline: every core of this process's
    affinity mask (``torch.set_num_threads(len(os.sched_getaffinity(0)))``),
    with the cgroup CPU quota recorded beside it when one is set."""
    res = {"affinity_cores": len(os.sched_getaffinity(0)), "os_cpu_count": os.cpu_count()}
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        res["cgroup_cpu_quota"] = None if quota == "max" else round(int(quota) / int(period), 2)
    except (OSError, ValueError):
        pass
    return res


def _cpu_model() -> str:
    """The host CPU's model name with its family, model and stepping numbers
    (a virtualised host may report a generic name such as "AMD EPYC")."""
    fields = {}
    try:
        for line in open("/proc/cpuinfo"):
            key, _, val = line.partition(":")
            key = key.strip()
            if key in ("model name", "cpu family", "model", "stepping") and key not in fields:
                fields[key] = val.strip()
            if not line.strip() and fields:
                break                                   # the first processor's entry
    except OSError:
        pass
    name = fields.get("model name", "unknown")
    ids = ", ".join(f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields)
    return f"{name} ({ids})" if ids else name


def decode_kernel_name(ns: int, waves: int, l2: bool, policy: int, bf16: bool = False,
                       multi: bool = False) -> str:
    """Name prefix of the decode kernel instantiation a launch shape runs,
    as rocprofv3 reports it."""
    b = lambda x: "true" if x else "false"  # noqa: E731
    if ns in (16, 32, 64):    # the block kernel (T = 2..4): 16-row tiles per wave
        return f"gdn::gdn_decode_block<{ns // 16}, {waves}, {b(l2)}, {b(bf16)}>"
    return (f"gdn::gdn_decode_k128<{ns}, {waves}, {b(l2)}, {policy}, {b(bf16)}, {b(multi)}, "
            f"false>")




def sources_sha(paths) -> str:
    """Hash of the given sources under this checkout (``ROOT``)."""
    return _sources_sha(paths, ROOT)


def _traffic(kernel: str) -> tuple[int | None, str]:
    """Measured HBM bytes per launch from the committed counter summary, if
    it was measured on ``kernel`` (the instantiation the timed launches
    run) built from the current sources; else None and the reason."""
    try:
        summary = json.loads(TRAFFIC_SUMMARY.read_text())
    except (OSError, ValueError) as e:
        return None, f"no counter summary: {e}"
    measured = summary.get("kernel", "")
    if not measured.startswith(kernel):
        return None, f"counter summary measured {measured.split('(')[0]!r}, not {kernel!r}"
    if summary.get("sources_sha") != sources_sha(DECODE_SOURCES):
        return None, "counter summary measured other decode sources (sources_sha differs)"
    return summary.get("traffic_bytes_per_launch"), str(TRAFFIC_SUMMARY.relative_to(ROOT))


PMC_DECODE_COMMANDS = [
    "cd /tmp && export TMPDIR=/tmp && timeout -s KILL 90 rocprofv3 --pmc FETCH_SIZE "
    "--output-format csv -d $REPO/gpurun_out/pmc_fetch -o pmc -- python3 $REPO/bench.py --pmc-pass",
    "cd /tmp && export TMPDIR=/tmp && timeout -s KILL 90 rocprofv3 --pmc WRITE_SIZE "
    "--output-format csv -d $REPO/gpurun_out/pmc_write -o pmc -- python3 $REPO/bench.py --pmc-pass",
    "python3 bench.py --summarize-pmc gpurun_out/pmc_fetch/pmc_counter_collection.csv "
    "gpurun_out/pmc_write/pmc_counter_collection.csv",
]
PMC_COPY_BYTES = 256 * 1024 * 1024


def summarize_pmc(fetch_csv: str, write_csv: str) -> dict:
    """The committed counter summary of the B=256 qk16_v32 decode launches
    of ``--pmc-pass`` (two rocprofv3 runs, FETCH_SIZE then WRITE_SIZE)."""
    from flashinfer_competition_codebase_amd.rocprof import pmc_traffic

    B, H, HV, l2 = CONFIGS["b256_qk16_v32_l2"]
    ns, waves, policy, _ = _lib.launch_shape(B, HV)
    res = pmc_traffic(fetch_csv, write_csv, decode_kernel_name(ns, waves, l2, policy),
                      PMC_COPY_BYTES, copies=3, skip=2)
    nbytes = step_bytes(B, H, HV)
    return {"kernel": res.pop("kernel"), "sources_sha": sources_sha(DECODE_SOURCES),
            "workload": ("B=256 qk16_v32 K=V=128 T=1, q/k L2-norm on, fp32 state updated in "
                         "place, steps rotating over 2 layer states"),
            "commands": PMC_DECODE_COMMANDS, **res,
            "algorithmic_bytes_per_launch": nbytes,
            "traffic_over_algorithmic": round(res["traffic_bytes_per_launch"] / nbytes, 4),
            "note": ("Counter values are KiB per dispatch.  Each counter is scaled by what it "
                     "reads for the three 256 MiB copies the run makes first (bytes = KiB * "
                     "1024 / factor); the decode value is the median over the launches after "
                     "the first two, whose states were still warm from setup.")}


def roofline_line(kernel: str, nbytes: int, kavg: float, traced: dict | None,
                  ref_stream: dict) -> dict:
    """The ``roofline`` object: algorithmic bytes per launch over the average
    launch duration of the timed region (HIP events around it), against the
    8 TB/s HBM peak; ``traffic``: measured HBM bytes per launch from the
    committed counter summary when it was measured on the same kernel
    instantiation; ``trace``: the same shape's average and median kernel
    duration in the kernel-trace leg (rocprofv3), steady regime."""
    achieved = nbytes / (kavg * 1e-6) / 1e9
    traffic, source = _traffic(kernel)
    line = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
            "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": traffic,
            "traffic_source": source, "kernel": kernel, "algorithmic_bytes": nbytes,
            "kernel_us_avg": round(kavg, 3),
            "timer": "HIP events on the launch stream around the timed launches"}
    if traced is not None and "steady_avg" in traced:
        t_avg = traced["steady_avg"]
        line["trace"] = {"avg_us": t_avg, "median_us": traced["steady"],
                         "frac": round(nbytes / (t_avg * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
                         "launches": traced["n_steady"],
                         "timer": "rocprofv3 --kernel-trace (the kernel-trace leg), steady"}
    line["reference_stream"] = ref_stream
    return line


def b1_serving(device, layers: int = 48, reps: int = 20):
    """Host-inclusive time per decode step at B=1 qk16_v32 (L2-norm) when a
    model issues one step per GDN layer (``layers`` states, inputs shared),
    wall clock from a synchronised GPU to the end of the last step, median
    over ``reps`` passes, divided by ``layers``:

    * ``eager``: a ``kernel_hip`` call per step (validation every call);
    * ``plan``: a bound ``DecodePlan.run()`` per step;
    * ``layers_run``: ``DecodeLayers.run()``, all steps from one native call;
    * ``graph``: ``DecodeLayers.replay()``, one HIP graph of all steps;
    * ``torch_graph``: the ``kernel_hip`` calls captured by torch.cuda.graph.
    """
    from flashinfer_competition_codebase_amd.serving import DecodeLayers

    t = make_device_inputs(1, 16, 32, device, seed=11)
    states = [t["state"]] + [t["state"].clone() for _ in range(layers - 1)]
    views = [{**t, "state": s_, "new_state": s_} for s_ in states]
    bound = DecodeLayers(views, use_qk_l2norm=True)
    bound.capture()

    def eager():
        for v_ in views:
            gdn.kernel_hip(**v_, use_qk_l2norm=True)

    def plans():
        for p_ in bound.plans:
            p_.run()

    eager()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        eager()
    torch.cuda.synchronize()
    res = {}
    for name, fn in (("eager", eager), ("plan", plans), ("layers_run", bound.run),
                     ("graph", bound.replay), ("torch_graph", graph.replay)):
        fn()
        per = []
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            per.append((time.perf_counter() - t0) * 1e6 / layers)
        res[f"{name}_us_per_step"] = round(statistics.median(per), 2)
    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(reps)]
    for a_, b_ in ev:
        a_.record(stream)
        bound.replay()
        b_.record(stream)
    torch.cuda.synchronize()
    res["graph_gpu_us_per_step"] = round(
        statistics.median(a_.elapsed_time(b_) * 1e3 for a_, b_ in ev) / layers, 3)
    res["layers"] = layers
    bound.close()
    del graph
    return res


def b1_back_to_back(device, reps: int = 20):
    """Time per decode step at B=1 qk16_v32 (L2-norm) when steps run back to
    back with the GPU never idle, as in a model's decode loop: one HIP graph
    of one step per layer state (``layer_states``: >= 1 GiB in total, so
    every step reads a state that is no longer cached), replayed; HIP events
    on the replay stream around each replay.  Per step: kernel plus the gap
    to the next kernel, an upper bound on the kernel's duration."""
    t = make_device_inputs(1, 16, 32, device, seed=12)
    states = layer_states(t["state"])
    views = [{**t, "state": s_, "new_state": s_} for s_ in states]

    def steps():
        for v_ in views:
            gdn.kernel_hip(**v_, use_qk_l2norm=True)

    steps()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        steps()
    torch.cuda.synchronize()
    for _ in range(2):
        graph.replay()
    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(reps)]
    for a_, b_ in ev:
        a_.record(stream)
        graph.replay()
        b_.record(stream)
    torch.cuda.synchronize()
    per = statistics.median(a_.elapsed_time(b_) * 1e3 for a_, b_ in ev) / len(views)
    del graph
    return {"us_per_step": round(per, 3), "steps_per_replay": len(views),
            "state_bytes_rotated": len(views) * states[0].numel() * 4}


def reference_stream(device, iters: int = 20):
    """GB/s of torch's in-place elementwise add over a 512 MiB fp32 buffer:
    512 MiB read and 512 MiB written, the state traffic of one B=256
    qk16_v32 step, through a plain streaming kernel.  A reference point for
    the practical read+write bandwidth of the box, timed with event markers."""
    buf = torch.zeros(1 << 27, device=device)
    for _ in range(3):
        buf.add_(1.0)
    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(iters)]
    for a, b in ev:
        a.record(stream)
        buf.add_(1.0)
        b.record(stream)
    torch.cuda.synchronize()
    us = statistics.median(a.elapsed_time(b) * 1e3 for a, b in ev)
    return {"kernel": "torch add_ (in place), 512 MiB fp32", "us": round(us, 2),
            "gbs": round(2 * buf.numel() * 4 / (us * 1e-6) / 1e9, 1)}


class Calib:
    """The reference kernels of ``libgdn_calib.so`` (same-bytes in-place
    read-modify-write, empty kernel), launched with kernel stamps."""

    def __init__(self):
        from flashinfer_competition_codebase_amd.build import CALIB_PATH

        if not CALIB_PATH.exists():
            raise RuntimeError(f"{CALIB_PATH} not built; run "
                               "`python -m flashinfer_competition_codebase_amd.build`")
        self.lib = ctypes.CDLL(str(CALIB_PATH))
        P, LL, F, I = ctypes.c_void_p, ctypes.c_longlong, ctypes.c_float, ctypes.c_int
        self.lib.gdn_calib_rmw.argtypes = [P, LL, F, I, P, P, P]
        self.lib.gdn_calib_rmw.restype = I
        self.lib.gdn_calib_empty.argtypes = [LL, P, P, P]
        self.lib.gdn_calib_empty.restype = I

    def rmw(self, buf, start, stop):
        code = self.lib.gdn_calib_rmw(buf.data_ptr(), buf.numel(), 0.999, 1, start, stop,
                                      torch.cuda.current_stream().cuda_stream)
        _lib.check(code, "gdn_calib_rmw")

    def empty(self, blocks, start, stop):
        code = self.lib.gdn_calib_empty(blocks, start, stop,
                                        torch.cuda.current_stream().cuda_stream)
        _lib.check(code, "gdn_calib_empty")


def traffic_floor(device, iters: int):
    """Kernel-stamped medians, steady regime, of the reference kernels that
    move only a decode step's state bytes: an in-place nontemporal
    read-modify-write of the B=1 qk16_v32 state (2 MiB, 256 workgroups of
    128 threads, as the decode launch at B=1) and of the B=256 state
    (512 MiB), and an empty kernel on 256 workgroups.  The decode kernel's
    times under the same timer compare directly."""
    cal = Calib()
    out = {}
    for name, nfloat in (("b1", 32 * 128 * 128), ("b256", 256 * 32 * 128 * 128)):
        bufs = layer_states(torch.zeros(nfloat, device=device))
        n = max(iters, 2 * len(bufs))
        stamps = KernelStamps(n)
        try:
            for i in range(n):
                cal.rmw(bufs[i % len(bufs)], stamps.start[i].value, stamps.stop[i].value)
            torch.cuda.synchronize()
            d = [stamps.elapsed_us(i) for i in range(len(bufs), n)]
        finally:
            stamps.close()
        us = statistics.median(d)
        out[f"{name}_rmw_us"] = round(us, 3)
        out[f"{name}_rmw_gbs"] = round(2 * nfloat * 4 / (us * 1e-6) / 1e9, 1)
        del bufs
    stamps = KernelStamps(iters)
    try:
        for i in range(iters):
            cal.empty(256, stamps.start[i].value, stamps.stop[i].value)
        torch.cuda.synchronize()
        out["empty_us"] = round(statistics.median(stamps.elapsed_us(i) for i in range(iters)), 3)
    finally:
        stamps.close()
    return out


# Prefill workloads: name -> (sequence lengths, H, HV).  The reference's
# prefill workload 0 is one 6-token sequence (findings/research.md:1029).
PREFILL_CONFIGS = {
    "prefill_qk4_v8_1x6": ([6], 4, 8),
    "prefill_qk4_v8_1x16384": ([16384], 4, 8),
    "prefill_qk4_v8_16x1024": ([1024] * 16, 4, 8),
    "prefill_qk16_v32_1x8192": ([8192], 16, 32),
    "prefill_qk16_v32_64x512": ([512] * 64, 16, 32),
}
# Algorithmic flops of the chunkwise prefill per (64-token chunk, v-head):
# K K^T and Q K^T (2 x 64x64x128), W and U (2 x 64x64x128), Delta = U - W S,
# Q S and K^T Delta (3 x 64x128x128), P Delta (64x64x128); multiply-adds x 2.
PREFILL_FLOP_PER_CHUNK_HEAD = 2 * (4 * 64 * 64 * 128 + 3 * 64 * 128 * 128 + 64 * 64 * 128)


def prefill_bytes(lens, H, HV) -> int:
    """Unique HBM bytes of one prefill: q, k, v, output, a, b per token,
    state read and written per sequence, A_log, dt_bias, cu_seqlens."""
    L, N = sum(lens), len(lens)
    return (L * (2 * H * 128 * 2 + 2 * HV * 128 * 2 + 2 * HV * 2)
            + N * HV * 128 * 128 * 4 * 2 + 2 * HV * 4 + (N + 1) * 4)


def prefill_workspace_bytes(lens, H, HV) -> int:
    """Bytes the preparation kernel writes: a slot per (chunk, v-head), the
    six lower 16 x 32 operand blocks of T diag(beta) as bf16 hi/lo and eight
    rows of 64 fp32 scales (six used)."""
    chunks = sum((n + 63) // 64 for n in lens)
    vslot = 2 * 6 * 16 * 32 * 2 + 8 * 64 * 4
    return chunks * HV * vslot


PREFILL_ROOFLINE_WORKLOAD = "prefill_qk16_v32_64x512"


PREFILL_PREP_KERNEL = "gdn_pf::prep_kernel<false>"
PREFILL_SCAN_KERNEL = "gdn_pf::scan_kernel<false, false, true, false, 8>"
PMC_PREFILL_COMMANDS = [
    "cd /tmp && export TMPDIR=/tmp && timeout -s KILL 90 rocprofv3 --pmc FETCH_SIZE "
    "--output-format csv -d $REPO/gpurun_out/pmcp1 -o p -- python3 $REPO/bench.py --pmc-prefill",
    "cd /tmp && export TMPDIR=/tmp && timeout -s KILL 90 rocprofv3 --pmc WRITE_SIZE "
    "--output-format csv -d $REPO/gpurun_out/pmcp2 -o p -- python3 $REPO/bench.py --pmc-prefill",
    "python3 bench.py --summarize-pmc-prefill gpurun_out/pmcp1/p_counter_collection.csv "
    "gpurun_out/pmcp2/p_counter_collection.csv",
]


def summarize_pmc_prefill(fetch_csv: str, write_csv: str) -> dict:
    """The committed counter summary of the 64 x 512 qk16_v32 prefills of
    ``--pmc-prefill`` (two rocprofv3 runs, FETCH_SIZE then WRITE_SIZE): HBM
    bytes per launch of the preparation and scan kernels."""
    from flashinfer_competition_codebase_amd.rocprof import pmc_traffic

    lens, H, HV = PREFILL_CONFIGS[PREFILL_ROOFLINE_WORKLOAD]
    kernels = {}
    for key, name in (("prep", PREFILL_PREP_KERNEL), ("scan", PREFILL_SCAN_KERNEL)):
        kernels[key] = pmc_traffic(fetch_csv, write_csv, name, PMC_COPY_BYTES, copies=3, skip=1)
    total = kernels["prep"]["traffic_bytes_per_launch"] + kernels["scan"]["traffic_bytes_per_launch"]
    alg = prefill_bytes(lens, H, HV)
    return {"workload": f"{PREFILL_ROOFLINE_WORKLOAD}: {len(lens)} x {lens[0]} tokens, "
                        f"H={H} HV={HV}, 3 prefills (the first one skipped)",
            "sources_sha": sources_sha(PREFILL_SOURCES), "commands": PMC_PREFILL_COMMANDS,
            "kernels": kernels, "traffic_bytes_per_prefill": total,
            "algorithmic_bytes_per_prefill": alg,
            "workspace_bytes_written": prefill_workspace_bytes(lens, H, HV),
            "traffic_over_algorithmic": round(total / alg, 4),
            "note": ("Counter values are KiB per dispatch, each scaled by what it reads for "
                     "the three 256 MiB copies the run makes first (bytes = KiB * 1024 / "
                     "factor); per kernel the median over the prefills after the first.")}


def _prefill_traffic() -> dict | None:
    """Measured HBM bytes per launch of the 64 x 512 qk16_v32 prefill kernels,
    from the committed counter summary when it was measured on the current
    prefill sources; else None."""
    try:
        summary = json.loads(PREFILL_TRAFFIC_SUMMARY.read_text())
        if summary.get("sources_sha") != sources_sha(PREFILL_SOURCES):
            return None
        k = summary["kernels"]
        return {"prep": k["prep"]["traffic_bytes_per_launch"],
                "scan": k["scan"]["traffic_bytes_per_launch"]}
    except (OSError, ValueError, KeyError):
        return None


def prefill_roofline(prefill: dict) -> dict:
    """Roofline of the largest prefill workload against the roof that binds
    it: its algorithmic bytes (q, k, v, a, b, output, states in and out) and
    FLOP give a floor time on each roof (HBM at 8 TB/s, bf16 dense MFMA), and
    the larger floor names ``bound``; ``achieved`` / ``frac`` are on that
    roof over the whole prefill's kernel time, and ``mfma`` / ``hbm`` carry
    both roofs' fractions.  ``prep``: the preparation kernel's HBM bytes
    (inputs read + workspace written) per its time; ``traffic``: measured
    HBM bytes of prep + scan per prefill and the HBM rate they make over the
    kernels' times."""
    r = prefill[PREFILL_ROOFLINE_WORKLOAD]
    lens_h = PREFILL_CONFIGS[PREFILL_ROOFLINE_WORKLOAD]
    lens, H, HV = lens_h
    chunks = sum((n + 63) // 64 for n in lens)
    flop = chunks * HV * PREFILL_FLOP_PER_CHUNK_HEAD
    alg_bytes = prefill_bytes(lens, H, HV)
    ku = r["kernel_us"]
    achieved = flop / (ku["kernels"] * 1e-6) / 1e12
    hbm_gbs = alg_bytes / (ku["kernels"] * 1e-6) / 1e9
    floor_hbm_us = alg_bytes / (PEAK_HBM_GBS * 1e3)
    floor_mfma_us = flop / (PEAK_BF16_TFLOPS * 1e6)
    mfma = {"achieved": round(achieved, 1), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "floor_us": round(floor_mfma_us, 1),
            "flop": flop}
    hbm = {"achieved": round(hbm_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
           "frac": round(hbm_gbs / PEAK_HBM_GBS, 4), "floor_us": round(floor_hbm_us, 1),
           "algorithmic_bytes": alg_bytes}
    binding = hbm if floor_hbm_us >= floor_mfma_us else mfma
    L = sum(lens)
    prep_in = L * (H * 128 * 2 + 2 * HV * 2)              # k, a, b
    prep_bytes = prep_in + r["prep_workspace_bytes"]
    prep_gbs = prep_bytes / (ku["prep"] * 1e-6) / 1e9
    tr = _prefill_traffic()
    traffic = None
    if tr is not None:
        total = tr["prep"] + tr["scan"]
        gbs = total / ((ku["prep"] + ku["scan"]) * 1e-6) / 1e9
        traffic = {"bytes": total, "prep_bytes": tr["prep"], "scan_bytes": tr["scan"],
                   "hbm_gbs": round(gbs, 1), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4),
                   "source": str(PREFILL_TRAFFIC_SUMMARY.relative_to(ROOT))}
    return {"workload": PREFILL_ROOFLINE_WORKLOAD,
            "bound": "hbm" if binding is hbm else "mfma",
            "achieved": binding["achieved"], "peak": binding["peak"], "unit": binding["unit"],
            "frac": binding["frac"], "hbm": hbm, "mfma": mfma, "traffic": traffic,
            "kernel_us": ku,
            "prep": {"hbm_bytes": prep_bytes, "gbs": round(prep_gbs, 1),
                     "frac_of_hbm_peak": round(prep_gbs / PEAK_HBM_GBS, 4)}}


def prefill_cpu_baseline(seconds: float, gpu_tokens_per_s: float | None):
    """The reference's prefill loop (prefill_loop, a restatement of
    solution/triton/prefill_kernel.py:85-183) on this host's cores, on a
    bounded sample of the 16 x 1024 qk4_v8 workload: one 256-token sequence,
    repeated until about ``seconds`` of CPU work; and the 6-token workload."""
    from oracle.gdn_prefill_oracle import make_prefill_inputs, prefill_loop

    torch.set_num_threads(host_threads()["affinity_cores"])
    t = make_prefill_inputs([256], 4, 8, seed=5)
    prefill_loop(**t)                              # warmup
    reps, elapsed = 0, 0.0
    t0 = time.perf_counter()
    while elapsed < seconds:
        prefill_loop(**t)
        reps += 1
        elapsed = time.perf_counter() - t0
    tps = 256 * reps / elapsed
    t6 = make_prefill_inputs([6], 4, 8, seed=6)
    w0 = []
    for _ in range(5):
        s_ = time.perf_counter()
        prefill_loop(**t6)
        w0.append((time.perf_counter() - s_) * 1e6)
    return {"value": round(tps, 1), "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": (f"one 256-token sequence of the 16 x 1024 qk4_v8 workload, {reps} "
                       f"prefills in {elapsed:.1f} s"),
            "gpu_tokens_per_s_same_workload": gpu_tokens_per_s,
            "workload0_1x6_us": round(statistics.median(w0), 1)}


def prefill_inputs(name: str, device) -> dict:
    """DPS arguments of one prefill workload, seeded on the device."""
    lens, H, HV = PREFILL_CONFIGS[name]
    L, N = sum(lens), len(lens)
    g = torch.Generator(device=device).manual_seed(17)
    f = dict(device=device)
    q = torch.randn(L, H, 128, generator=g, **f)
    k = torch.randn(L, H, 128, generator=g, **f)
    t = dict(q=(q / q.norm(dim=-1, keepdim=True)).to(torch.bfloat16),
             k=(k / k.norm(dim=-1, keepdim=True)).to(torch.bfloat16),
             v=torch.randn(L, HV, 128, generator=g, **f).to(torch.bfloat16),
             state=torch.randn(N, HV, 128, 128, generator=g, **f).mul_(0.05),
             A_log=torch.log(torch.rand(HV, generator=g, **f) * 15.0 + 1.0),
             a=torch.randn(L, HV, generator=g, **f).to(torch.bfloat16),
             dt_bias=torch.rand(HV, generator=g, **f) * 2.0 - 1.0,
             b=torch.randn(L, HV, generator=g, **f).to(torch.bfloat16),
             scale=1.0 / math.sqrt(128))
    cu = torch.zeros(N + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens), 0)
    t["cu_seqlens"] = cu.to(device)
    t["output"] = torch.empty(L, HV, 128, dtype=torch.bfloat16, **f)
    t["new_state"] = torch.empty_like(t["state"])
    return t


def pmc_prefill(device):
    """Short run for rocprofv3 counter passes over the prefill: three plain
    256 MiB copies (calibrate FETCH_SIZE / WRITE_SIZE against known bytes),
    then three prefills of the 64 x 512 qk16_v32 workload."""
    n = 256 * 1024 * 1024 // 4
    src = torch.randn(n, device=device)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    for name in (PREFILL_ROOFLINE_WORKLOAD,):
        t = prefill_inputs(name, device)
        for _ in range(3):
            gdn.kernel_prefill_hip(**t)
        torch.cuda.synchronize()
        del t
    print(json.dumps({"pmc_prefill": "done", "copy_bytes": n * 4}), flush=True)


def prefill_bench(device, iters: int = 20):
    """Per prefill workload: median time of the whole prefill call from
    torch events around it, and of each of its three kernels from HIP events
    the library records between its launches (gdn_prefill_timed);
    algorithmic TFLOP/s and GB/s.  Inputs: unit-norm q/k rows (the model's
    normalisation), the decode benchmark's other distributions."""
    out = {}
    stamps = KernelStamps(2 * iters)              # 4 events per timed prefill
    for name, (lens, H, HV) in PREFILL_CONFIGS.items():
        L, N = sum(lens), len(lens)
        t = prefill_inputs(name, device)
        for _ in range(PREFILL_WARMUP_CALLS):
            gdn.kernel_prefill_hip(**t)
        stream = torch.cuda.current_stream()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(iters)]
        for a_, b_ in ev:
            a_.record(stream)
            gdn.kernel_prefill_hip(**t)
            b_.record(stream)
        torch.cuda.synchronize()
        us = statistics.median(a_.elapsed_time(b_) * 1e3 for a_, b_ in ev)
        parts = {"offsets": [], "prep": [], "scan": [], "kernels": []}
        for i in range(iters):
            e4 = [stamps.start[2 * i], stamps.stop[2 * i], stamps.start[2 * i + 1],
                  stamps.stop[2 * i + 1]]
            gdn.kernel_prefill_hip_timed(**t, events=e4)
            torch.cuda.synchronize()
            d = [stamps.between_us(e4[j], e4[j + 1]) for j in range(3)]
            for key, val in zip(("offsets", "prep", "scan"), d):
                parts[key].append(val)
            parts["kernels"].append(sum(d))
        med = {key: statistics.median(v) for key, v in parts.items()}
        chunks = sum((n + 63) // 64 for n in lens)
        flop = chunks * HV * PREFILL_FLOP_PER_CHUNK_HEAD
        nb = prefill_bytes(lens, H, HV)
        out[name] = {"seqs": N, "tokens": L, "H": H, "HV": HV, "us": round(us, 2),
                     "kernel_us": {key: round(v, 2) for key, v in med.items()},
                     "tflops": round(flop / (us * 1e-6) / 1e12, 2),
                     "gbs": round(nb / (us * 1e-6) / 1e9, 1),
                     "tokens_per_s": round(L / (us * 1e-6), 1),
                     "prep_workspace_bytes": prefill_workspace_bytes(lens, H, HV)}
        del t
    stamps.close()
    return out


PREFILL_WARMUP_CALLS = 3


def summarize_prefill_trace(trace_csv: str, iters: int = 20) -> str:
    """Per prefill workload of a ``--prefill-only`` run under ``rocprofv3
    --kernel-trace``: the median kernel-trace duration of each kernel and of
    the whole call (first start to last end) over the timed calls, as a
    markdown table.  The run's calls are, per workload in order, the warmup
    calls, ``iters`` event-timed calls and ``iters`` calls of the timed entry,
    each of ``gdn_prefill_dispatches`` kernels."""
    with open(trace_csv, newline="") as f:
        rows = [r for r in csv.DictReader(f) if "gdn" in r["Kernel_Name"]]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    lib = _lib.load_prefill()
    lines = ["| workload | kernels per call | kernel: median us | call, first start to "
             "last end: median us |", "|---|---|---|---|"]
    i = 0
    for name, (lens, H, HV) in PREFILL_CONFIGS.items():
        nd = lib.gdn_prefill_dispatches(sum(lens), len(lens), HV)
        calls = []
        for _ in range(PREFILL_WARMUP_CALLS + 2 * iters):
            calls.append(rows[i:i + nd])
            i += nd
        per: dict[str, list[float]] = {}
        span = []
        for call in calls[PREFILL_WARMUP_CALLS:]:
            for r in call:
                k = r["Kernel_Name"].replace("void ", "").split("(")[0]
                per.setdefault(k, []).append(
                    (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
            span.append((int(call[-1]["End_Timestamp"]) - int(call[0]["Start_Timestamp"])) / 1e3)
        kern = "; ".join(f"`{k}` {statistics.median(v):.2f}" + (f" (x{len(v) // (2 * iters)})"
                         if len(v) > 2 * iters else "") for k, v in per.items())
        lines.append(f"| {name} ({len(lens)} x {lens[0]}, H={H} HV={HV}) | {nd} | {kern} | "
                     f"{statistics.median(span):.2f} |")
    if i != len(rows):
        raise ValueError(f"{trace_csv}: {len(rows)} prefill kernels, expected {i}")
    return "\n".join(lines)


def pmc_pass(device, shape: str = "b256_qk16_v32_l2"):
    """Short run for rocprofv3 counter passes (FETCH_SIZE, WRITE_SIZE, or
    others): three plain 256 MiB copies (calibrate the byte counters against
    known bytes), then six decode steps of one per-config shape (by default
    the B=256 qk16_v32 headline) rotating over two layer states, as in the
    timed region."""
    n = 256 * 1024 * 1024 // 4
    src = torch.randn(n, device=device)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    shapes = {sh[0]: sh[1:] for sh in per_config_shapes()}
    B, H, HV, l2, T, sd = shapes[shape]
    t = make_device_inputs(B, H, HV, device, seed=1003, T=T, state_dtype=sd)
    states = layer_states(t["state"])[:2]
    for i in range(6):
        s_ = states[i % len(states)]
        gdn.kernel_hip(**{**t, "state": s_, "new_state": s_}, use_qk_l2norm=l2)
    torch.cuda.synchronize()
    ns, waves, policy, _ = _lib.launch_shape(B, HV, T, sd == torch.bfloat16)
    print(json.dumps({"pmc_pass": shape, "copy_bytes": n * 4,
                      "kernel": decode_kernel_name(ns, waves, l2, policy, sd == torch.bfloat16,
                                                   T > 1),
                      "decode_bytes": step_bytes(B, H, HV, T=T,
                                                 state_elem=t["state"].element_size())}),
          flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="b256_qk16_v32_l2", choices=list(CONFIGS))
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--prefill-cpu-seconds", type=float, default=8.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-per-config", action="store_true")
    ap.add_argument("--iters", type=int, default=100,
                    help="launches per per-config kernel-time measurement")
    ap.add_argument("--pmc-pass", action="store_true")
    ap.add_argument("--pmc-shape", default="b256_qk16_v32_l2",
                    help="per-config shape the --pmc-pass run launches")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="write the decode counter summary from two --pmc-pass runs")
    ap.add_argument("--pmc-prefill", action="store_true",
                    help="short prefill run for rocprofv3 counter passes")
    ap.add_argument("--summarize-pmc-prefill", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="write the prefill counter summary from two --pmc-prefill runs")
    ap.add_argument("--summarize-prefill-trace", metavar="TRACE_CSV",
                    help="print per-workload kernel medians of a traced --prefill-only run")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--prefill-only", action="store_true",
                    help="time the prefill workloads only and print them as JSON")
    ap.add_argument("--serving-only", action="store_true",
                    help="time the B=1 serving paths only and print them as JSON")
    ap.add_argument("--no-kernel-trace", action="store_true",
                    help="skip the rocprofv3 kernel-trace leg")
    ap.add_argument("--trace-child", metavar="MANIFEST",
                    help="(internal) the launches the kernel-trace leg records")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(the decode step shards by batch or v-head with no communication)",
              file=sys.stderr)
        sys.exit(1)

    log = lambda *a: print(*a, file=sys.stderr, flush=True)  # noqa: E731
    if args.summarize_pmc:
        summary = summarize_pmc(*args.summarize_pmc)
        TRAFFIC_SUMMARY.write_text(json.dumps(summary, indent=1) + "\n")
        log(f"[bench] wrote {TRAFFIC_SUMMARY.relative_to(ROOT)}: "
            f"{summary['traffic_bytes_per_launch']} B per launch "
            f"({summary['traffic_over_algorithmic']}x algorithmic)")
        return
    if args.summarize_pmc_prefill:
        summary = summarize_pmc_prefill(*args.summarize_pmc_prefill)
        PREFILL_TRAFFIC_SUMMARY.write_text(json.dumps(summary, indent=1) + "\n")
        log(f"[bench] wrote {PREFILL_TRAFFIC_SUMMARY.relative_to(ROOT)}: "
            f"{summary['traffic_bytes_per_prefill']} B per prefill "
            f"({summary['traffic_over_algorithmic']}x algorithmic)")
        return
    if args.summarize_prefill_trace:
        print(summarize_prefill_trace(args.summarize_prefill_trace))
        return
    trace = None
    if not (args.trace_child or args.no_kernel_trace or args.no_per_config or args.pmc_pass
            or args.pmc_prefill or args.prefill_only or args.serving_only):
        # before this process touches the GPU: the traced run is its own program
        log("[bench] kernel-trace leg: every per-config shape under rocprofv3")
        trace = kernel_trace_leg(args.iters)
        log(f"[bench] kernel-trace leg: {trace.get('skipped', 'done')}")

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    _lib.get_lib()
    if args.trace_child:
        trace_child(device, args.trace_child, args.iters)
        return
    if args.pmc_pass:
        pmc_pass(device, args.pmc_shape)
        return
    if args.pmc_prefill:
        pmc_prefill(device)
        return
    if args.serving_only:
        print(json.dumps({"b1_serving": b1_serving(device),
                          "b1_back_to_back": b1_back_to_back(device)}), flush=True)
        return
    if args.prefill_only:
        pf = prefill_bench(device)
        print(json.dumps({"prefill": pf, "prefill_roofline": prefill_roofline(pf)}), flush=True)
        return

    B, H, HV, l2 = CONFIGS[args.config]
    nbytes = step_bytes(B, H, HV)
    t = make_device_inputs(B, H, HV, device, seed=1003)
    ns, waves, policy, blocks = _lib.launch_shape(B, HV)
    log(f"[bench] {args.config}: B={B} H={H} HV={HV} l2={l2} bytes/step={nbytes} "
        f"launch ns={ns} waves={waves} policy={policy} blocks={blocks}")
    states = layer_states(t["state"])
    log(f"[bench] rotating over {len(states)} layer states")
    for i in range(args.warmup):
        s_ = states[i % len(states)]
        gdn.kernel_hip(**{**t, "state": s_, "new_state": s_}, use_qk_l2norm=l2)
    torch.cuda.synchronize()
    wall, kavg = timed_steps(t, l2, args.steps, states)
    del states
    ms_per_step = wall * 1e3 / args.steps
    value = nbytes / (wall / args.steps) / 1e9
    achieved = nbytes / (kavg * 1e-6) / 1e9
    kernel = decode_kernel_name(ns, waves, l2, policy)
    log(f"[bench] timed {args.steps} steps: {ms_per_step * 1e3:.2f} us/step wall, "
        f"{kavg:.2f} us/launch on the GPU (events around the region), "
        f"{achieved:.0f} GB/s = {achieved / PEAK_HBM_GBS:.1%} of peak; kernel {kernel}")

    flush = torch.ones(1 << 28, device=device)     # 1 GiB > 32 MiB L2 + 256 MiB MALL
    per_config = {}
    traced = (trace or {}).get("shapes", {})
    if not args.no_per_config:
        bf16 = torch.bfloat16
        for name, b_, h_, hv_, l2_, t_, sd_ in per_config_shapes():
            tc = make_device_inputs(b_, h_, hv_, device, seed=7, T=t_, state_dtype=sd_)
            for _ in range(5):
                gdn.kernel_hip(**tc, use_qk_l2norm=l2_)
            med = {m: statistics.median(kernel_times_us(tc, l2_, args.iters, mode=m,
                                                        flush=flush))
                   for m in ("steady", "warm", "cold")}
            nb = step_bytes(b_, h_, hv_, T=t_, state_elem=tc["state"].element_size())
            sm = med["steady"]
            per_config[name] = {
                "B": b_, "H": h_, "HV": hv_, "T": t_, "l2norm": l2_,
                "state": "bf16" if sd_ == bf16 else "fp32", "bytes": nb,
                "launch": list(_lib.launch_shape(b_, hv_, t_, sd_ == bf16)),
                "us_steady": round(sm, 3), "us_warm": round(med["warm"], 3),
                "us_cold": round(med["cold"], 3),
                "steady_hbm_gbs": round(nb / (sm * 1e-6) / 1e9, 1),
                "steady_frac_of_peak": round(nb / (sm * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
            }
            tr = traced.get(name)
            if tr is not None:
                per_config[name].update({
                    "trace_us_steady": tr["steady"], "trace_us_cold": tr["cold"],
                    "trace_steady_hbm_gbs": round(nb / (tr["steady"] * 1e-6) / 1e9, 1)})
            log(f"[bench] {name}: steady {sm:.2f} us ({per_config[name]['steady_hbm_gbs']:.0f}"
                f" GB/s), warm {med['warm']:.2f} us, cold {med['cold']:.2f} us"
                + (f"; kernel trace steady {tr['steady']:.2f} us, cold {tr['cold']:.2f} us"
                   if tr is not None else ""))
            del tc

    floor = traffic_floor(device, args.iters)
    log(f"[bench] floor, same timer: B=1 state bytes in-place RMW {floor['b1_rmw_us']} us, "
        f"empty kernel {floor['empty_us']} us; B=256 state RMW {floor['b256_rmw_us']} us "
        f"({floor['b256_rmw_gbs']} GB/s)")

    prefill, prefill_rl = {}, None
    if not args.no_prefill:
        prefill = prefill_bench(device)
        for name, r in prefill.items():
            log(f"[bench] {name}: {r['us']} us, {r['tflops']} TFLOP/s, {r['gbs']} GB/s, "
                f"kernels {r['kernel_us']}")
        prefill_rl = prefill_roofline(prefill)

    serving = b1_serving(device)
    log(f"[bench] B=1 serving, {serving['layers']} layer steps (us/step, host wall): "
        + ", ".join(f"{k[:-12]} {v}" for k, v in serving.items() if k.endswith("_us_per_step"))
        + f"; graph on the GPU {serving['graph_gpu_us_per_step']} us/step")
    b2b = b1_back_to_back(device)
    log(f"[bench] B=1 back to back over {b2b['steps_per_replay']} layer states "
        f"({b2b['state_bytes_rotated'] >> 20} MiB): {b2b['us_per_step']} us/step")
    ref_stream = reference_stream(device)
    log(f"[bench] reference stream: {ref_stream['gbs']:.0f} GB/s ({ref_stream['us']} us)")

    cpu, prefill_cpu = None, None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(args.cpu_seconds)
        log(f"[bench] cpu baseline: {cpu['value']} GB/s on {cpu['cores']} threads "
            f"({cpu['sample']}); B=1 {cpu['b1_us_per_step']} us/step")
        if prefill:
            prefill_cpu = prefill_cpu_baseline(
                args.prefill_cpu_seconds, prefill["prefill_qk4_v8_16x1024"]["tokens_per_s"])
            log(f"[bench] prefill cpu baseline: {prefill_cpu['value']} tokens/s "
                f"({prefill_cpu['sample']})")

    b1 = per_config.get("b1_qk16_v32_l2")
    b1_line = {"target_us": 3.0, "us_per_step": b2b["us_per_step"],
               "timer": ("HIP events around replays of a HIP graph of back-to-back steps, "
                         "one per layer state (>= 1 GiB of states: every step reads its "
                         "state from HBM); per step = kernel + gap to the next kernel"),
               "back_to_back": b2b}
    if b1 and "trace_us_steady" in b1:
        b1_line["kernel_trace"] = {
            "us_isolated": b1["trace_us_steady"], "us_after_flush": b1["trace_us_cold"],
            "floor": trace["floor"],
            "timer": (trace["timer"] + "; launches ~12 us apart from Python (the GPU idles "
                      "between them), rotating over >= 1 GiB of states; after_flush: right "
                      "after a 1 GiB read")}
    else:
        b1_line["kernel_trace"] = {"skipped": (trace or {}).get("skipped", "not run")}
    if b1:
        b1_line["stamped"] = {"us_steady": b1["us_steady"], "us_warm": b1["us_warm"],
                              "us_cold": b1["us_cold"],
                              "timer": "kernel-stamped HIP events (hipExtLaunchKernelGGL)",
                              "floor_same_timer": floor}
    else:
        b1_line["stamped"] = {"floor_same_timer": floor}
    b1_line["serving"] = serving
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": ("synthetic, seeded on the device: q,k,v,a,b ~ N(0,1) bf16; state ~ "
                 "N(0,0.05^2) fp32; A_log = log U[1,16]; dt_bias ~ U[-1,1]"),
        "config": {
            "workload": (f"GDN decode step, qk{H}_v{HV}_d128 k-last fp32 state, B={B}, "
                         f"T=1, q/k L2-norm {'on' if l2 else 'off'}, in-place state update"),
            "B": B, "H": H, "HV": HV, "K": 128, "V": 128,
            "bytes_per_step": nbytes,
            "launch": {"rows_per_lane_group": ns, "waves_per_block": waves,
                       "cache_policy": policy, "blocks": blocks},
        },
        "b1": b1_line,
        "roofline": roofline_line(kernel, nbytes, kavg, traced.get(args.config), ref_stream),
        "cpu_baseline": cpu,
        "per_config": per_config,
        "prefill": prefill,
        "prefill_roofline": prefill_rl,
        "prefill_cpu_baseline": prefill_cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
