"""flashinfer-bench-style evaluation of the decode and prefill entry points on
MI355X.

The reference evaluates a solution with flashinfer-bench over the contest's
workloads of a definition (scripts/run_local.py:31-98): for each workload it
checks the outputs against the definition's reference implementation
(atol = rtol = 1e-2, CLAUDE.md:158), times the DPS entry point with the
cache flushed and the tensor arguments cloned before every iteration
(CLAUDE.md:151-157), and prints one line per workload
(``PASSED | µs | speedup | abs_err, rel_err``, scripts/run_local.py:101-120).
The contest score of a definition is the arithmetic mean of the per-workload
speedups (FAQ.md:27-33).  This module does the same for the entry points of
this package, with the workload inputs synthesised (the contest dataset is
external to the reference, CLAUDE.md:164-168):

* ``contest_decode_workloads()``: the 54 ``gdn_decode_qk4_v8_d128_k_last``
  workloads, batch sizes 1 x10, 4 x8, 8 x7, 16 x7, 32 x7, 48 x7, 64 x8
  (CLAUDE.md:139-140), each with its own seed;
* ``prefill_workloads()``: a seeded mix of 20 ``gdn_prefill_qk4_v8_d128_k_last``
  workloads (variable-length sequences packed with ``cu_seqlens``): the
  reference's workload 0 (one 6-token sequence, findings/research.md:1029),
  single sequences of 1 to 16384 tokens, uniform and ragged batches and
  empty sequences.  The contest's 100 prefill workloads are not recorded in
  the reference (CLAUDE.md:159), so the mix is this package's own;
* ``evaluate(fn, workloads, ...)``: correctness against a caller-supplied
  reference (a value-returning ``ref(**inputs) -> (output, new_state)``, the
  role the definition's ``reference`` plays) and timing in the reference's
  three tiers (findings/research.md:348-356): "event" (events around each
  call, the flashinfer-bench / NVBench tier), "sync" (wall clock with a
  device synchronisation around each call, the tier of flashinfer-bench's
  old ``do_bench``) and "trace" (kernel durations from a rocprofv3 kernel
  trace of the run, the CUPTI tier: ``evaluate`` writes a manifest of its
  calls and ``attribute_trace`` assigns the trace's dispatches to them);
* speedups against the reference's published B200 kernel times: per batch
  size for the decode (CUPTI medians of fla-recurrent and of the FlashInfer
  baseline, CLAUDE.md:229-238), and for prefill workload 0 (CUPTI medians of
  FLA's chunkwise prefill and of the FlashInfer baseline, CLAUDE.md:333-337);
  the contest's own speedup is against the definition's reference on the
  same GPU, which is not available here.

Command line (arguments as scripts/shared.py:93-142):

    python -m flashinfer_competition_codebase_amd.harness run --algo hip [-n N]
        [--definition gdn_prefill_qk4_v8_d128_k_last --algo prefill-hip]
        [--workload-id PREFIX] [--iterations 100] [--num-trials 5] [--tier event]
        [--manifest calls.json] [--json results.json]
    rocprofv3 --kernel-trace --output-format csv -d out -o run -- python3 -m \\
        flashinfer_competition_codebase_amd.harness run --manifest calls.json
    python -m flashinfer_competition_codebase_amd.harness attribute \\
        --trace out/run_kernel_trace.csv --manifest calls.json [--definition ...]

In the trace tier a prefill call is its dispatches (``prefill_dispatches``:
the chunk-offsets scan for several sequences, preparation and scan, two more
with segments, the token-by-token kernel first for a batch that may be all
short sequences -- or that kernel alone for a prefill of at most 56 tokens,
or the one-chunk kernel alone for 57 to 64), timed from the first one's
start to the last one's end.
"""

from __future__ import annotations

import argparse
import csv
import json
import math
import statistics
import sys
import time
from dataclasses import asdict, dataclass, field
from pathlib import Path
from typing import Callable, Optional

import torch

DECODE_DEFINITION = "gdn_decode_qk4_v8_d128_k_last"
PREFILL_DEFINITION = "gdn_prefill_qk4_v8_d128_k_last"
DEFINITIONS = (DECODE_DEFINITION, PREFILL_DEFINITION)

# Batch sizes of the contest's 54 decode workloads and how many of each
# (CLAUDE.md:139-140).
CONTEST_BATCHES = ((1, 10), (4, 8), (8, 7), (16, 7), (32, 7), (48, 7), (64, 8))

# Published B200 kernel times (CUPTI medians, µs) per batch size for the
# qk4_v8 decode definition, CLAUDE.md:229-238: fla-recurrent with adaptive
# warps, and the FlashInfer baseline (gated_delta_rule_decode_pretranspose).
B200_CUPTI_US = {
    "fla-b200": {1: 2.46, 4: 3.10, 8: 4.10, 16: 5.47, 32: 8.80, 48: 12.35, 64: 15.01},
    "fi-b200": {1: 3.36, 4: 3.65, 8: 4.22, 16: 5.31, 32: 7.71, 48: 10.50, 64: 12.74},
}
BASELINE_LABELS = {"fla-b200": "B200 fla-recurrent", "fi-b200": "B200 FlashInfer"}

# Published B200 times (CUPTI medians, µs) of the qk4_v8 prefill definition's
# workload 0, CLAUDE.md:333-337 (findings/research.md:1075-1080): FLA's
# chunkwise prefill and the FlashInfer baseline.  No other prefill workload
# has a published time.
PREFILL_WORKLOAD0_LENS = (6,)
B200_PREFILL_US = {"fla-b200": 1536.0, "fi-b200": 185.0}
PREFILL_BASELINE_LABELS = {"fla-b200": "B200 fla-chunk", "fi-b200": "B200 FlashInfer"}

# Kernel-name substrings of the dispatches one call makes, per definition (a
# prefill of a few tokens is one launch of the decode kernel's
# variable-length mode).
TRACE_KERNELS = {DECODE_DEFINITION: ("gdn_decode",),
                 PREFILL_DEFINITION: ("gdn_pf::", "gdn_decode_k128")}

ATOL = 1e-2
RTOL = 1e-2
TIERS = ("event", "sync")
FLUSH_BYTES = 1 << 30   # > 32 MiB of L2 plus the 256 MiB MALL


@dataclass(frozen=True)
class Workload:
    """One decode workload: shapes, seed and options (T tokens, L2-norm)."""
    uuid: str
    B: int
    H: int = 4
    HV: int = 8
    T: int = 1
    seed: int = 0
    use_qk_l2norm: bool = False


def contest_decode_workloads() -> list:
    """The 54 qk4_v8 decode workloads of the contest mix, in batch order."""
    out = []
    for B, count in CONTEST_BATCHES:
        for i in range(count):
            out.append(Workload(uuid=f"qk4v8-b{B:02d}-{i:02d}", B=B, seed=10_000 + 100 * B + i))
    return out


@dataclass(frozen=True)
class PrefillWorkload:
    """One prefill workload: sequence lengths (packed with cu_seqlens), head
    counts, seed and the L2-norm option."""
    uuid: str
    lens: tuple
    H: int = 4
    HV: int = 8
    seed: int = 0
    use_qk_l2norm: bool = False

    @property
    def L(self) -> int:
        return sum(self.lens)

    @property
    def N(self) -> int:
        return len(self.lens)

    @property
    def B(self) -> int:               # sequences: the batch of a prefill
        return self.N

    @property
    def dispatches(self) -> int:      # kernels one prefill call launches
        from .prefill import prefill_dispatches
        return prefill_dispatches(self.L, self.N, self.HV)


def prefill_workloads() -> list:
    """A seeded mix of 21 qk4_v8 prefill workloads: the reference's workload 0
    (one 6-token sequence), single sequences across the chunk boundaries and
    up to 16384 tokens, uniform and ragged batches, empty sequences, and a
    batch of short sequences past the total-token switch (4 x 20)."""
    g = torch.Generator().manual_seed(4242)

    def ragged(n, hi):
        return tuple(int(x) for x in torch.randint(1, hi + 1, (n,), generator=g))

    mixes = [
        (6,), (1,), (64,), (65,), (127,), (512,), (1000,), (2048,), (4096,), (8192,),
        (16384,), (100, 200, 300, 400), (128,) * 8, (256,) * 16, (1024,) * 16,
        (512,) * 32, (64,) * 64, ragged(24, 2048), ragged(8, 8192), (0, 17, 0, 300),
        (20,) * 4,
    ]
    return [PrefillWorkload(uuid=f"prefill-w{i:02d}", lens=lens, seed=20_000 + i)
            for i, lens in enumerate(mixes)]


def make_prefill_inputs(w: PrefillWorkload, device) -> dict:
    """Seeded inputs of prefill workload ``w`` on ``device``: q and k rows of
    unit norm (a model normalises them; unnormalised N(0, 1) keys make the
    delta rule diverge over long sequences), v, a, b ~ N(0, 1) bf16; state
    ~ N(0, 0.05^2) fp32; A_log = log U[1, 16]; dt_bias ~ U[-1, 1];
    cu_seqlens int32; scale = 1/sqrt(128).  Drawn on the CPU."""
    g = torch.Generator().manual_seed(w.seed)
    K = V = 128
    L, N = w.L, w.N
    q = torch.randn(L, w.H, K, generator=g)
    k = torch.randn(L, w.H, K, generator=g)
    cu = torch.zeros(N + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(w.lens, dtype=torch.int64), 0).to(torch.int32)
    t = dict(
        q=(q / q.norm(dim=-1, keepdim=True)).to(torch.bfloat16),
        k=(k / k.norm(dim=-1, keepdim=True)).to(torch.bfloat16),
        v=torch.randn(L, w.HV, V, generator=g).to(torch.bfloat16),
        state=torch.randn(N, w.HV, V, K, generator=g) * 0.05,
        A_log=torch.log(torch.rand(w.HV, generator=g) * 15.0 + 1.0),
        a=torch.randn(L, w.HV, generator=g).to(torch.bfloat16),
        dt_bias=torch.rand(w.HV, generator=g) * 2.0 - 1.0,
        b=torch.randn(L, w.HV, generator=g).to(torch.bfloat16),
        cu_seqlens=cu,
    )
    t = {n: x.to(device) for n, x in t.items()}
    t["scale"] = 1.0 / math.sqrt(K)
    return t


def make_inputs(w: Workload, device) -> dict:
    """Seeded inputs of workload ``w`` on ``device`` with the benchmark's
    distributions: q, k, v, a, b ~ N(0, 1) bf16; state ~ N(0, 0.05^2) fp32;
    A_log = log U[1, 16]; dt_bias ~ U[-1, 1]; scale = 1/sqrt(128).  Drawn on
    the CPU so every device sees the same bits."""
    g = torch.Generator().manual_seed(w.seed)
    K = V = 128
    t = dict(
        q=torch.randn(w.B, w.T, w.H, K, generator=g).to(torch.bfloat16),
        k=torch.randn(w.B, w.T, w.H, K, generator=g).to(torch.bfloat16),
        v=torch.randn(w.B, w.T, w.HV, V, generator=g).to(torch.bfloat16),
        state=torch.randn(w.B, w.HV, V, K, generator=g) * 0.05,
        A_log=torch.log(torch.rand(w.HV, generator=g) * 15.0 + 1.0),
        a=torch.randn(w.B, w.T, w.HV, generator=g).to(torch.bfloat16),
        dt_bias=torch.rand(w.HV, generator=g) * 2.0 - 1.0,
        b=torch.randn(w.B, w.T, w.HV, generator=g).to(torch.bfloat16),
    )
    t = {n: x.to(device) for n, x in t.items()}
    t["scale"] = 1.0 / math.sqrt(K)
    return t


def _dps_outputs(inputs: dict) -> dict:
    """Caller-allocated outputs of the DPS form (scripts/profile_proton.py:106-110):
    decode ``output [B, T, HV, V]``, ``new_state [B, HV, V, K]``; prefill
    ``output [L, HV, V]``, ``new_state [N, HV, V, K]``."""
    if "cu_seqlens" in inputs:
        L, HV, V = inputs["v"].shape
        K = inputs["q"].shape[-1]
        N = inputs["cu_seqlens"].numel() - 1
        dev = inputs["q"].device
        return dict(output=torch.empty(L, HV, V, dtype=torch.bfloat16, device=dev),
                    new_state=torch.empty(N, HV, V, K, dtype=torch.float32, device=dev))
    B, T, HV, V = inputs["v"].shape
    K = inputs["q"].shape[-1]
    dev = inputs["q"].device
    return dict(output=torch.empty(B, T, HV, V, dtype=torch.bfloat16, device=dev),
                new_state=torch.empty(B, HV, V, K, dtype=torch.float32, device=dev))


def compare(out, ref, atol: float = ATOL, rtol: float = RTOL):
    """flashinfer-bench's element-wise criterion ``|x - y| <= atol + rtol |y|``
    for one tensor; returns (status, max_abs_error, max_rel_error)."""
    if tuple(out.shape) != tuple(ref.shape):
        return "INCORRECT_SHAPE", math.inf, math.inf
    if out.dtype != ref.dtype:
        return "INCORRECT_DTYPE", math.inf, math.inf
    x, y = out.detach().float().cpu(), ref.detach().float().cpu()
    if not bool(torch.isfinite(x).all()):
        return "INCORRECT_NUMERICAL", math.inf, math.inf
    diff = (x - y).abs()
    max_abs = diff.max().item() if diff.numel() else 0.0
    max_rel = (diff / y.abs().clamp_min(1e-12)).max().item() if diff.numel() else 0.0
    ok = bool((diff <= atol + rtol * y.abs()).all())
    return ("PASSED" if ok else "INCORRECT_NUMERICAL"), max_abs, max_rel


@dataclass
class Result:
    """One workload's evaluation (scripts/run_local.py:79-96 fields); ``B`` is
    the batch (sequences of a prefill)."""
    uuid: str
    B: int
    status: str
    latency_us: Optional[float] = None
    latency_median_us: Optional[float] = None
    max_abs_error: Optional[float] = None
    max_rel_error: Optional[float] = None
    speedup: Optional[float] = None
    timings_us: list = field(default_factory=list, repr=False)


class Manifest:
    """The ordered list of solution calls of a run, for ``attribute_trace``:
    each call is (workload uuid, phase, dispatches) with phase "check",
    "warmup" or "timed" and the number of kernel dispatches the call makes."""

    def __init__(self):
        self.calls = []

    def add(self, uuid: str, phase: str, dispatches: int = 1) -> None:
        self.calls.append([uuid, phase, dispatches])

    def write(self, path) -> None:
        Path(path).write_text(json.dumps({"calls": self.calls, "sources_sha": run_sources_sha()}))


def run_sources_sha() -> dict:
    """Hash of the kernel sources of each library (build.sources_sha): what a
    run measured, recorded in its manifest and printed with its results."""
    from .build import DECODE_SOURCES, PREFILL_SOURCES, sources_sha

    return {"decode": sources_sha(DECODE_SOURCES), "prefill": sources_sha(PREFILL_SOURCES)}


def baseline_us(w, baseline: Optional[str]) -> Optional[float]:
    """The published B200 time the speedup of workload ``w`` is taken
    against, or None: the decode per batch size at the qk4_v8 shape (T = 1),
    the prefill for the reference's workload 0 only."""
    if not baseline:
        return None
    if isinstance(w, PrefillWorkload):
        if tuple(w.lens) == PREFILL_WORKLOAD0_LENS and (w.H, w.HV) == (4, 8):
            return B200_PREFILL_US.get(baseline)
        return None
    table = B200_CUPTI_US.get(baseline)
    if table and w.B in table and w.T == 1 and (w.H, w.HV) == (4, 8):
        return table[w.B]
    return None


def _call(fn, dps: bool, inputs: dict, outputs: dict):
    if dps:
        fn(**inputs, **outputs)
        return outputs["output"], outputs["new_state"]
    return fn(**inputs)


def evaluate(fn: Callable, workloads, *, dps: bool = True, reference: Optional[Callable] = None,
             reference_device="cpu", device="cuda:0", warmup: int = 3, iterations: int = 100,
             num_trials: int = 5, tier: str = "event", flush: str = "read",
             clone: bool = True, manifest: Optional[Manifest] = None,
             baseline: str = "fla-b200", log=None) -> list:
    """Evaluate entry point ``fn`` on each workload (``Workload`` for the
    decode definition, ``PrefillWorkload`` for the prefill definition).

    ``dps``: ``fn`` is destination-passing (writes ``output`` and
    ``new_state``) or value-returning (returns them), the two forms of
    scripts/shared.py:37.  ``reference``: value-returning reference run on
    ``reference_device`` with the same inputs; None skips the check (status
    "UNCHECKED").  Timing: ``num_trials`` x (``warmup`` untimed calls, then
    ``iterations`` timed calls); before each call the cache is flushed
    (``flush``: "read" reads 1 GiB, "zero" zero-fills 1 GiB as
    flashinfer-bench zero-fills 256 MB, "none") and, with ``clone``, the
    tensor arguments are cloned, outside the timed region (CLAUDE.md:151-157:
    the clone re-warms the cache with the arguments, as it does there).
    ``clone=False`` reuses one set of arguments for every call, as FlashInfer's
    ``bench_gpu_time`` does in scripts/bench_fi_timing.py:43-48 -- the
    methodology of the published B200 per-batch times.  ``latency_us`` is the
    mean over all timed calls (the flashinfer-bench statistic), with the
    median beside it.
    """
    if tier not in TIERS:
        raise ValueError(f"tier must be one of {TIERS}")
    if flush not in ("read", "zero", "none"):
        raise ValueError("flush must be 'read', 'zero' or 'none'")
    device = torch.device(device)
    flush_buf = None
    if flush != "none":
        flush_buf = torch.empty(FLUSH_BYTES // 4, dtype=torch.float32, device=device)
        flush_buf.fill_(1.0)
    results = []
    for w in workloads:
        prefill = isinstance(w, PrefillWorkload)
        base = make_prefill_inputs(w, device) if prefill else make_inputs(w, device)
        nd = w.dispatches if prefill else 1
        if log:
            log(f"[harness] {w.uuid}: " + (f"N={w.N} L={w.L} H={w.H} HV={w.HV}" if prefill
                                           else f"B={w.B} H={w.H} HV={w.HV} T={w.T}"))
        # correctness on one call with pristine inputs
        inputs = {n: (x.clone() if isinstance(x, torch.Tensor) else x) for n, x in base.items()}
        outputs = _dps_outputs(inputs) if dps else {}
        try:
            if manifest is not None:
                manifest.add(w.uuid, "check", nd)
            out, new_state = _call(fn, dps, inputs, outputs)
            torch.cuda.synchronize(device)
        except Exception as exc:  # noqa: BLE001 - reported as the workload's status
            results.append(Result(w.uuid, w.B, f"RUNTIME_ERROR: {exc}"))
            continue
        res = Result(w.uuid, w.B, "UNCHECKED")
        if reference is not None:
            rin = {n: (x.to(reference_device) if isinstance(x, torch.Tensor) else x)
                   for n, x in base.items()}
            ref_out, ref_state = reference(**rin)
            s1, a1, r1 = compare(out, ref_out)
            s2, a2, r2 = compare(new_state, ref_state)
            res.status = s1 if s1 != "PASSED" else s2
            res.max_abs_error, res.max_rel_error = max(a1, a2), max(r1, r2)
        # timing
        times = []
        for _ in range(num_trials):
            for i in range(warmup + iterations):
                timed = i >= warmup
                if flush == "read":
                    flush_buf.sum()
                elif flush == "zero":
                    flush_buf.zero_()
                if clone or i == 0:
                    args = {n: (x.clone() if isinstance(x, torch.Tensor) else x)
                            for n, x in base.items()}
                    outs = _dps_outputs(args) if dps else {}
                if manifest is not None:
                    manifest.add(w.uuid, "timed" if timed else "warmup", nd)
                if tier == "event":
                    ev0 = torch.cuda.Event(enable_timing=True)
                    ev1 = torch.cuda.Event(enable_timing=True)
                    ev0.record()
                    _call(fn, dps, args, outs)
                    ev1.record()
                    if timed:
                        times.append((ev0, ev1))
                else:
                    torch.cuda.synchronize(device)
                    t0 = time.perf_counter()
                    _call(fn, dps, args, outs)
                    torch.cuda.synchronize(device)
                    if timed:
                        times.append((time.perf_counter() - t0) * 1e6)
            torch.cuda.synchronize(device)
        if tier == "event":
            times = [a.elapsed_time(b) * 1e3 for a, b in times]
        res.timings_us = times
        res.latency_us = statistics.fmean(times)
        res.latency_median_us = statistics.median(times)
        ref_us = baseline_us(w, baseline)
        if ref_us is not None:
            res.speedup = ref_us / res.latency_us
        results.append(res)
    return results


def mean_speedup(results) -> Optional[float]:
    """Arithmetic mean of the per-workload speedups (FAQ.md:27-33)."""
    s = [r.speedup for r in results if r.speedup is not None]
    return statistics.fmean(s) if s else None


def attribute_trace(trace_csv, manifest_calls, *, kernel_substring="gdn_decode",
                    baseline: str = "fla-b200", workloads=None) -> list:
    """Kernel-trace tier: assign the dispatches of kernels whose name
    contains ``kernel_substring`` (a string or a tuple of alternatives) in a
    rocprofv3 ``kernel_trace.csv`` (in
    start-time order) to the manifest's calls, each call taking as many
    consecutive dispatches as it made, and return one Result per workload with
    the mean and median of its timed calls' times (first dispatch's start to
    last dispatch's end).  Raises if the counts differ."""
    subs = (kernel_substring,) if isinstance(kernel_substring, str) else tuple(kernel_substring)
    rows = []
    with open(trace_csv) as f:
        for r in csv.DictReader(f):
            if any(x in r["Kernel_Name"] for x in subs):
                rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    rows.sort()
    counts = [int(c[2]) if len(c) > 2 else 1 for c in manifest_calls]
    if len(rows) != sum(counts):
        raise ValueError(f"{len(rows)} {'/'.join(subs)} dispatches in the trace but "
                         f"{sum(counts)} in the manifest's {len(manifest_calls)} calls")
    per = {}
    i = 0
    for call, n in zip(manifest_calls, counts):
        uuid, phase = call[0], call[1]
        if phase == "timed":
            per.setdefault(uuid, []).append((rows[i + n - 1][1] - rows[i][0]) / 1e3)
        i += n
    by_uuid = {w.uuid: w for w in (workloads or contest_decode_workloads() + prefill_workloads())}
    out = []
    for uuid, d in per.items():
        w = by_uuid.get(uuid)
        B = w.B if w else -1
        res = Result(uuid, B, "TRACED", latency_us=statistics.fmean(d),
                     latency_median_us=statistics.median(d), timings_us=d)
        ref_us = baseline_us(w, baseline) if w is not None else None
        if ref_us is not None:
            res.speedup = ref_us / res.latency_us
        out.append(res)
    return out


def print_results(results, definition: str = DECODE_DEFINITION, baseline: str = "fla-b200",
                  file=None) -> None:
    """One line per workload in the layout of scripts/run_local.py:101-120,
    then the mean speedup."""
    file = file or sys.stdout
    labels = PREFILL_BASELINE_LABELS if definition == PREFILL_DEFINITION else BASELINE_LABELS
    label = labels.get(baseline, baseline)
    print(f"\n{definition}:", file=file)
    for r in results:
        line = f"  Workload {r.uuid}: {r.status}"
        if r.latency_us is not None:
            line += f" | {r.latency_us:.3f} µs"
        if r.speedup is not None:
            line += f" | {r.speedup:.2f}x vs {label}"
        if r.max_abs_error is not None:
            line += f" | abs_err={r.max_abs_error:.2e}, rel_err={r.max_rel_error:.2e}"
        print(line, file=file)
    ms = mean_speedup(results)
    if ms is not None:
        print(f"  mean speedup vs {label} over {sum(r.speedup is not None for r in results)} "
              f"workloads: {ms:.3f}x", file=file)


def per_workload_summary(results) -> dict:
    """Median latency (µs) per workload."""
    return {r.uuid: round(r.latency_median_us, 3) for r in results
            if r.latency_median_us is not None}


def per_batch_summary(results) -> dict:
    """Median latency (µs) per batch size."""
    by_b = {}
    for r in results:
        if r.latency_us is not None:
            by_b.setdefault(r.B, []).append(r.latency_median_us)
    return {b: round(statistics.median(v), 3) for b, v in sorted(by_b.items())}


def _select(workloads, num_workloads: int, workload_id: Optional[str]):
    if workload_id:
        workloads = [w for w in workloads if w.uuid.startswith(workload_id)]
        if not workloads:
            raise ValueError(f"No workload found matching '{workload_id}'")
    if num_workloads > 0:
        workloads = workloads[:num_workloads]
    return workloads


def _parser():
    ap = argparse.ArgumentParser(prog="python -m flashinfer_competition_codebase_amd.harness",
                                 description="Evaluate the GDN decode or prefill entry points "
                                             "over a workload mix of the definition")
    sub = ap.add_subparsers(dest="cmd", required=True)
    r = sub.add_parser("run", help="check and time an entry point over the workloads")
    r.add_argument("--algo", default="hip", help="entry point name (ENTRY_POINTS)")
    r.add_argument("--definition", default=DECODE_DEFINITION, choices=DEFINITIONS)
    r.add_argument("-n", "--num-workloads", type=int, default=0)
    r.add_argument("--workload-id", default=None,
                   help="workload name prefix, e.g. qk4v8-b16 or prefill-w0")
    r.add_argument("--iterations", type=int, default=100)
    r.add_argument("--num-trials", type=int, default=5)
    r.add_argument("--warmup", type=int, default=3)
    r.add_argument("--tier", choices=TIERS, default="event")
    r.add_argument("--flush", choices=("read", "zero", "none"), default="read")
    r.add_argument("--no-clone", action="store_true",
                   help="reuse one set of arguments (bench_gpu_time's methodology)")
    r.add_argument("--baseline", choices=sorted(B200_CUPTI_US), default="fla-b200")
    r.add_argument("--manifest", type=Path, default=None,
                   help="write the ordered call list for 'attribute'")
    r.add_argument("--json", type=Path, default=None, help="write the results as JSON")
    a = sub.add_parser("attribute", help="kernel-trace tier from a rocprofv3 trace of 'run'")
    a.add_argument("--trace", type=Path, required=True)
    a.add_argument("--manifest", type=Path, required=True)
    a.add_argument("--definition", default=DECODE_DEFINITION, choices=DEFINITIONS)
    a.add_argument("--baseline", choices=sorted(B200_CUPTI_US), default="fla-b200")
    a.add_argument("--json", type=Path, default=None)
    return ap


def _dump(results, path, extra=None) -> None:
    doc = {"results": [{k: v for k, v in asdict(r).items() if k != "timings_us"}
                       for r in results],
           "mean_speedup": mean_speedup(results),
           "per_batch_median_us": per_batch_summary(results),
           "per_workload_median_us": per_workload_summary(results)}
    doc.update(extra or {})
    Path(path).write_text(json.dumps(doc, indent=1))


def main(argv=None) -> int:
    args = _parser().parse_args(argv)
    prefill = args.definition == PREFILL_DEFINITION
    if args.cmd == "attribute":
        doc = json.loads(args.manifest.read_text())
        calls = doc["calls"]
        results = attribute_trace(args.trace, calls, baseline=args.baseline,
                                  kernel_substring=TRACE_KERNELS[args.definition])
        print(f"Sources of the traced run (sources_sha): {doc.get('sources_sha', 'not recorded')}")
        print_results(results, definition=args.definition, baseline=args.baseline)
        if prefill:
            print(f"  per-workload median kernel time (µs): {per_workload_summary(results)}")
        else:
            print(f"  per-batch median kernel time (µs): {per_batch_summary(results)}")
        if args.json:
            _dump(results, args.json, {"tier": "trace", "baseline": args.baseline,
                                       "definition": args.definition,
                                       "sources_sha": doc.get("sources_sha")})
        return 0

    from . import ENTRY_POINTS, NO_DPS

    algos = sorted(a for a in ENTRY_POINTS if a.startswith("prefill") == prefill)
    if args.algo not in algos:
        raise SystemExit(f"algo {args.algo!r} is not an entry point of this package for "
                         f"{args.definition}; available: {algos}")
    workloads = _select(prefill_workloads() if prefill else contest_decode_workloads(),
                        args.num_workloads, args.workload_id)
    manifest = Manifest() if args.manifest else None
    print(f"Algorithm: {args.algo} ({'value-returning' if args.algo in NO_DPS else 'DPS'}), "
          f"{len(workloads)} workloads, tier {args.tier}, flush {args.flush}, "
          f"{'one set of arguments' if args.no_clone else 'arguments cloned per call'}; "
          f"sources_sha {run_sources_sha()}", flush=True)
    results = evaluate(ENTRY_POINTS[args.algo], workloads, dps=args.algo not in NO_DPS,
                       warmup=args.warmup, iterations=args.iterations,
                       num_trials=args.num_trials, tier=args.tier, flush=args.flush,
                       clone=not args.no_clone, manifest=manifest, baseline=args.baseline,
                       log=lambda m: print(m, file=sys.stderr, flush=True))
    print_results(results, definition=args.definition, baseline=args.baseline)
    if prefill:
        print(f"  per-workload median latency (µs, {args.tier} tier): "
              f"{per_workload_summary(results)}")
    else:
        print(f"  per-batch median latency (µs, {args.tier} tier): {per_batch_summary(results)}")
    if manifest is not None:
        manifest.write(args.manifest)
    if args.json:
        _dump(results, args.json, {"tier": args.tier, "baseline": args.baseline,
                                   "algo": args.algo, "flush": args.flush,
                                   "clone": not args.no_clone, "definition": args.definition,
                                   "sources_sha": run_sources_sha()})
    return 0


if __name__ == "__main__":
    sys.exit(main())
