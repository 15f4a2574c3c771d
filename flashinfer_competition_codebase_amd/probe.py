"""Where a small decode step's time goes: phase stamps and counter regimes.

A B = 1 decode step takes ~2.4 µs when steps run back to back, ~3 µs when
launched alone, and 4-5 µs right after a large streaming kernel (the
reference's timing methodology flushes the caches with a 256 MB+ write
before every call, CLAUDE.md:151-158).  This module measures the phases
of the step in those regimes:

* ``stamps``: the instrumented copy of the single-token kernel
  (``gdn_decode_step_stamped``) writes per wavefront the shader clock at
  entry, after its loads are issued, after the per-head math (small inputs
  arrived), at the state's arrival, after the state stores are issued and
  when every store has completed, plus the 100 MHz real-time clock at entry
  and end (the phases of the reference's clock64 plan,
  findings/potential-cuda-improvement.md:457-496).  Reported per regime:
  medians over launches of the per-launch median phase durations (µs) and
  of the spread of wavefront start times.
* ``regimes``: the product kernel launched in the same regimes in a fixed
  order, for a ``rocprofv3 --pmc`` run (translation misses, L2 hits, read
  latency per dispatch); ``pmc-summary`` attributes the counter CSV back to
  the regimes.

Regimes: ``back_to_back`` (a burst of launches rotating over >= 1 GiB of
layer states, the GPU never idle), ``after_flush`` (each launch right after
a 1 GiB read, the reference's cold-cache methodology), ``isolated`` (each
launch after the GPU idled ~2 ms).

    python -m flashinfer_competition_codebase_amd.probe stamps [--shape NAME ...]
    python -m flashinfer_competition_codebase_amd.probe regimes
    python -m flashinfer_competition_codebase_amd.probe pmc-summary COUNTER_CSV MANIFEST
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import statistics
import sys
import time

import torch

from . import _lib

# name -> (B, H, HV, q/k L2-norm)
SHAPES = {"b1_qk16_v32_l2": (1, 16, 32, True), "qk4_v8_b1": (1, 4, 8, False),
          "qk4_v8_b4": (4, 4, 8, False)}
REGIMES = ("back_to_back", "after_flush", "isolated")
STEADY_BYTES = 1 << 30
STAMPS_PER_WAVE = 8
REALTIME_HZ = 100e6


def _inputs(B, H, HV, device, seed=21):
    g = torch.Generator(device=device).manual_seed(seed)
    f = dict(device=device)
    t = dict(q=torch.randn(B, 1, H, 128, generator=g, **f).to(torch.bfloat16),
             k=torch.randn(B, 1, H, 128, generator=g, **f).to(torch.bfloat16),
             v=torch.randn(B, 1, HV, 128, generator=g, **f).to(torch.bfloat16),
             state=torch.randn(B, HV, 128, 128, generator=g, **f).mul_(0.05),
             A_log=torch.log(torch.rand(HV, generator=g, **f) * 15.0 + 1.0),
             a=torch.randn(B, 1, HV, generator=g, **f).to(torch.bfloat16),
             dt_bias=torch.rand(HV, generator=g, **f) * 2.0 - 1.0,
             b=torch.randn(B, 1, HV, generator=g, **f).to(torch.bfloat16),
             output=torch.empty(B, 1, HV, 128, dtype=torch.bfloat16, **f))
    n = max(2, -(-STEADY_BYTES // (t["state"].numel() * 4)))
    t["states"] = [t["state"]] + [t["state"].clone() for _ in range(n - 1)]
    return t


def _regime_schedule(n: int):
    """(regime, launch slot, measured) in launch order: a back-to-back burst
    of 2n (the first n warm the states' rotation), then n after a flush,
    then n isolated; slots 0 .. 4n - 1."""
    sched = [("back_to_back", i, i >= n) for i in range(2 * n)]
    sched += [("after_flush", 2 * n + i, True) for i in range(n)]
    sched += [("isolated", 3 * n + i, True) for i in range(n)]
    return sched


def _run_schedule(t, n, launch, flush):
    """Launch per the schedule; ``launch(state, slot)`` issues one step."""
    states = t["states"]
    for regime, slot, _ in _regime_schedule(n):
        s = states[slot % len(states)]
        if regime == "after_flush":
            flush.sum()
        elif regime == "isolated":
            torch.cuda.synchronize()
            time.sleep(0.002)
        launch(s, slot)
        if regime != "back_to_back":
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def stamps(device, shapes, n: int = 32) -> dict:
    """Phase medians (µs) per shape and regime from the stamped kernel."""
    lib = _lib.get_lib()
    flush = torch.ones(1 << 28, device=device)
    out = {}
    for name in shapes:
        B, H, HV, l2 = SHAPES[name]
        ns, waves, _, blocks = _lib.launch_shape(B, HV)
        t = _inputs(B, H, HV, device)
        n_waves = blocks * waves
        total = 4 * n                                    # launch slots of the schedule
        buf = torch.zeros(total, n_waves * STAMPS_PER_WAVE, dtype=torch.int64, device=device)
        stream = torch.cuda.current_stream().cuda_stream
        scale = 1.0 / math.sqrt(128)

        def launch(s, slot):
            ptr = ctypes.cast(buf[slot].data_ptr(), ctypes.POINTER(ctypes.c_ulonglong))
            code = lib.gdn_decode_step_stamped(
                t["q"].data_ptr(), t["k"].data_ptr(), t["v"].data_ptr(), s.data_ptr(),
                t["A_log"].data_ptr(), t["a"].data_ptr(), t["dt_bias"].data_ptr(),
                t["b"].data_ptr(), scale, t["output"].data_ptr(), s.data_ptr(), B, H, HV, 128,
                128, int(l2), ns, waves, ptr, n_waves * STAMPS_PER_WAVE, stream)
            _lib.check(code, "gdn_decode_step_stamped")

        _run_schedule(t, n, launch, flush)
        st = buf.view(total, n_waves, STAMPS_PER_WAVE).cpu().double()
        res = {}
        sched = _regime_schedule(n)
        for regime in REGIMES:
            slots = [slot for r, slot, m in sched if r == regime and m]
            res[regime] = _phases(st[slots])
        out[name] = {"launch": {"rows_per_lane_group": ns, "waves_per_block": waves,
                                "blocks": blocks, "wavefronts": n_waves}, **res}
        del t, buf
    return out


def _phases(st: torch.Tensor) -> dict:
    """st: [launches, waves, 8] stamps -> medians over launches (µs)."""
    rt0, t0, t1, t2, t3, t4, t5, rt1 = (st[..., i] for i in range(STAMPS_PER_WAVE))
    # shader clock rate per wave from the real-time clock over the same span
    hz = ((t5 - t0) / ((rt1 - rt0) / REALTIME_HZ).clamp_min(1e-9)).median().item()
    cyc = lambda x: x / hz * 1e6  # noqa: E731

    def med(x):
        return round(statistics.median(x.median(dim=1).values.tolist()), 3)

    return {
        "shader_clock_ghz": round(hz / 1e9, 3),
        "issue_loads_us": med(cyc(t1 - t0)),
        "small_inputs_and_head_math_us": med(cyc(t2 - t1)),
        "state_arrival_after_entry_us": med(cyc(t3 - t0)),
        "state_stores_issued_us": med(cyc(t4 - t3)),
        "stores_complete_us": med(cyc(t5 - t4)),
        "wave_total_us": med(cyc(t5 - t0)),
        "wave_start_spread_us": round(statistics.median(
            ((rt0.max(dim=1).values - rt0.min(dim=1).values) / REALTIME_HZ * 1e6).tolist()), 3),
        "first_start_to_last_end_us": round(statistics.median(
            ((rt1.max(dim=1).values - rt0.min(dim=1).values) / REALTIME_HZ * 1e6).tolist()), 3),
    }


def regimes(device, n: int = 32, manifest_path: str | None = None) -> dict:
    """The product kernel (``kernel_hip``) in every regime, for each shape, in
    the order ``pmc_summary`` expects; writes the manifest."""
    from .kernel import kernel_hip

    flush = torch.ones(1 << 28, device=device)
    manifest = []
    for name, (B, H, HV, l2) in SHAPES.items():
        t = _inputs(B, H, HV, device)
        scale = 1.0 / math.sqrt(128)
        common = {k: t[k] for k in ("q", "k", "v", "A_log", "a", "dt_bias", "b", "output")}

        def launch(s, slot):
            kernel_hip(**common, state=s, new_state=s, scale=scale, use_qk_l2norm=l2)

        _run_schedule(t, n, launch, flush)
        manifest.append({"shape": name, "schedule": [[r, m] for r, _, m in _regime_schedule(n)]})
        print(f"[probe] {name}: {len(manifest[-1]['schedule'])} launches", file=sys.stderr,
              flush=True)
        del t
    # B = 1 qk16_v32 through other launch shapes (workgroup counts 1024 to 32)
    from .kernel import kernel_hip_shaped

    t = _inputs(1, 16, 32, device)
    common = {k: t[k] for k in ("q", "k", "v", "A_log", "a", "dt_bias", "b", "output")}
    for ns, waves in ((1, 1), (8, 1), (8, 4)):
        def shaped(s, slot, ns=ns, waves=waves):
            kernel_hip_shaped(**common, state=s, new_state=s, scale=1.0 / math.sqrt(128),
                              use_qk_l2norm=True, rows_per_lane_group=ns,
                              waves_per_block=waves, cache_policy=1)

        _run_schedule(t, n, shaped, flush)
        manifest.append({"shape": f"b1_qk16_v32_l2_shape_{ns}x{waves}",
                         "schedule": [[r, m] for r, _, m in _regime_schedule(n)]})
    del t
    # an empty kernel of 8 to 1024 workgroups in the same regimes: what a
    # dispatch costs with no work in it
    from .build import CALIB_PATH

    cal = ctypes.CDLL(str(CALIB_PATH))
    cal.gdn_calib_empty.argtypes = [ctypes.c_longlong, ctypes.c_void_p, ctypes.c_void_p,
                                    ctypes.c_void_p]
    cal.gdn_calib_empty.restype = ctypes.c_int
    t = {"states": [None]}
    for blocks in (8, 256, 1024):
        def empty(_s, _slot, blocks=blocks):
            _lib.check(cal.gdn_calib_empty(blocks, None, None,
                                           torch.cuda.current_stream().cuda_stream),
                       "gdn_calib_empty")

        _run_schedule(t, n, empty, flush)
        manifest.append({"shape": f"empty_kernel_{blocks}_blocks", "kernel": "gdn_calib::empty",
                         "schedule": [[r, m] for r, _, m in _regime_schedule(n)]})
    doc = {"shapes": manifest}
    if manifest_path:
        with open(manifest_path, "w") as f:
            json.dump(doc, f)
    return doc


def pmc_summary(counter_csv: str, manifest_path: str) -> dict:
    """Median counter values (and kernel durations) per shape and regime: the
    decode dispatches of a ``regimes`` run under ``rocprofv3 --pmc`` (or
    ``--kernel-trace``: durations only), in dispatch order."""
    import csv

    manifest = json.load(open(manifest_path))["shapes"]
    kernels = tuple({m.get("kernel", "gdn_decode_k128") for m in manifest})
    per = {}
    with open(counter_csv, newline="") as f:
        for r in csv.DictReader(f):
            if not any(k in r["Kernel_Name"] for k in kernels):
                continue
            d = int(r["Dispatch_Id"])
            row = per.setdefault(d, {"dur_us": (int(r["End_Timestamp"]) -
                                                int(r["Start_Timestamp"])) / 1e3})
            if "Counter_Name" in r:
                name = r["Counter_Name"]
                row[name] = row.get(name, 0.0) + float(r["Counter_Value"])
    rows = [per[d] for d in sorted(per)]
    need = sum(len(m["schedule"]) for m in manifest)
    if len(rows) != need:
        raise ValueError(f"{len(rows)} decode dispatches in {counter_csv}, {need} launched")
    out, i = {}, 0
    for m in manifest:
        res = {}
        for regime, measured in m["schedule"]:
            if measured:
                res.setdefault(regime, []).append(rows[i])
            i += 1
        out[m["shape"]] = {
            regime: {k: round(statistics.median(r[k] for r in rs), 2) for k in rs[0]}
            for regime, rs in res.items()}
    return out


def main(argv=None) -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stamps")
    s.add_argument("--shape", action="append", choices=list(SHAPES))
    s.add_argument("-n", type=int, default=32)
    r = sub.add_parser("regimes")
    r.add_argument("--manifest", required=True)
    r.add_argument("-n", type=int, default=32)
    p = sub.add_parser("pmc-summary")
    p.add_argument("counter_csv")
    p.add_argument("manifest")
    a = ap.parse_args(argv)
    if a.cmd == "pmc-summary":
        res = pmc_summary(a.counter_csv, a.manifest)
    else:
        device = torch.device("cuda:0")
        torch.cuda.set_device(device)
        if a.cmd == "stamps":
            res = stamps(device, a.shape or list(SHAPES), a.n)
        else:
            res = regimes(device, a.n, a.manifest)
    json.dump(res, sys.stdout, indent=1)
    sys.stdout.write("\n")


if __name__ == "__main__":
    main()
