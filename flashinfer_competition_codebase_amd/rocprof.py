"""Summaries of rocprofv3 output for the measurements ``bench.py`` reports.

rocprofv3 writes one CSV row per dispatch (``*_kernel_trace.csv``) or per
dispatch and counter (``*_counter_collection.csv``).  This module turns
those files into the short summaries kept with the results:

* ``pmc_traffic``: HBM bytes per launch of one kernel from two counter runs
  (``FETCH_SIZE``, then ``WRITE_SIZE``, KiB per dispatch), each scaled by
  what the same counter reads for plain copies of known size made earlier
  in the same program (the first ``copies`` ``__amd_rocclr_copyBuffer``
  dispatches);
* ``trace_average``: the average duration of a kernel's dispatches
  ``[skip, skip + count)`` in a kernel trace (the timed region of a run), and
  the average over all of its dispatches;
* ``trace_groups``: every decode/calibration kernel's dispatches grouped by
  instantiation and grid, with the median duration overall, right after a
  cache-evicting read, and otherwise (the per-shape table of a bench run).

Command line (prints JSON):

    python -m flashinfer_competition_codebase_amd.rocprof pmc FETCH_CSV WRITE_CSV \
        --kernel NAME_PREFIX --copy-bytes N [--skip 2] [--copies 3]
    python -m flashinfer_competition_codebase_amd.rocprof trace TRACE_CSV \
        --kernel NAME_PREFIX --skip W --count K
    python -m flashinfer_competition_codebase_amd.rocprof groups TRACE_CSV

The reference profiles with NVIDIA's tools (scripts/profile_ncu.py,
scripts/profile_proton.py); this is the rocprofv3 side of the same job.
"""

from __future__ import annotations

import argparse
import csv
import json
import statistics
import sys

COPY_KERNEL = "__amd_rocclr_copyBuffer"


def _rows(path: str) -> list[dict]:
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def _kernel_name(row: dict) -> str:
    """The kernel name without the ``void `` rocprofv3 puts before it."""
    name = row["Kernel_Name"]
    return name[5:] if name.startswith("void ") else name


def counter_values(path: str, counter: str) -> list[tuple[str, float]]:
    """(kernel name, value) per dispatch, in dispatch order, for one counter
    (summed when a dispatch has several rows for it)."""
    per = {}
    for r in _rows(path):
        if r["Counter_Name"] != counter:
            continue
        d = int(r["Dispatch_Id"])
        name, val = per.get(d, (_kernel_name(r), 0.0))
        per[d] = (name, val + float(r["Counter_Value"]))
    return [per[d] for d in sorted(per)]


def _scaled(path: str, counter: str, kernel: str, copy_bytes: int, copies: int,
            skip: int) -> dict:
    vals = counter_values(path, counter)
    cal = [v for n, v in vals if n.startswith(COPY_KERNEL)][:copies]
    if len(cal) < copies:
        raise ValueError(f"{path}: {len(cal)} calibration copies, expected {copies}")
    launches = [(n, v) for n, v in vals if n.startswith(kernel)]
    if len(launches) <= skip:
        raise ValueError(f"{path}: {len(launches)} dispatches of {kernel}, need more than {skip}")
    factor = statistics.median(cal) * 1024 / copy_bytes
    used = [v for _, v in launches[skip:]]
    return {"kib_per_copy": cal, "factor": round(factor, 5),
            "kib_per_launch": [round(v, 3) for _, v in launches],
            "bytes_per_launch": round(statistics.median(used) * 1024 / factor),
            "kernel": launches[0][0]}


def pmc_traffic(fetch_csv: str, write_csv: str, kernel: str, copy_bytes: int,
                copies: int = 3, skip: int = 2) -> dict:
    """HBM bytes per launch of ``kernel`` (dispatches whose name starts with
    it): the median over its dispatches after the first ``skip`` of
    FETCH_SIZE and of WRITE_SIZE (KiB), each divided by what that counter
    reads per byte of the calibration copies (``copy_bytes`` read and
    written each)."""
    fe = _scaled(fetch_csv, "FETCH_SIZE", kernel, copy_bytes, copies, skip)
    wr = _scaled(write_csv, "WRITE_SIZE", kernel, copy_bytes, copies, skip)
    if fe["kernel"] != wr["kernel"]:
        raise ValueError(f"the two runs profiled different kernels: {fe['kernel']!r}, "
                         f"{wr['kernel']!r}")
    return {
        "kernel": fe["kernel"],
        "calibration": {"copy_bytes": copy_bytes, "fetch_size_kib_per_copy": fe["kib_per_copy"],
                        "write_size_kib_per_copy": wr["kib_per_copy"],
                        "fetch_factor": fe["factor"], "write_factor": wr["factor"]},
        "fetch_size_kib_per_launch": fe["kib_per_launch"],
        "write_size_kib_per_launch": wr["kib_per_launch"],
        "launches_skipped": skip,
        "fetch_bytes_per_launch": fe["bytes_per_launch"],
        "write_bytes_per_launch": wr["bytes_per_launch"],
        "traffic_bytes_per_launch": fe["bytes_per_launch"] + wr["bytes_per_launch"],
    }


def trace_average(trace_csv: str, kernel: str, skip: int, count: int) -> dict:
    """Average duration (µs) of the dispatches ``[skip, skip + count)`` of
    ``kernel`` (name prefix) in start order, and over all its dispatches."""
    spans = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), _kernel_name(r))
                   for r in _rows(trace_csv) if _kernel_name(r).startswith(kernel))
    if len(spans) < skip + count:
        raise ValueError(f"{trace_csv}: {len(spans)} dispatches of {kernel}, need {skip + count}")
    sel = [(e - s) / 1e3 for s, e, _ in spans[skip:skip + count]]
    every = [(e - s) / 1e3 for s, e, _ in spans]
    return {"kernel": spans[0][2], "dispatches": len(spans), "skip": skip, "count": count,
            "avg_us": round(statistics.fmean(sel), 3),
            "median_us": round(statistics.median(sel), 3),
            "avg_us_all_dispatches": round(statistics.fmean(every), 3)}


def trace_groups(trace_csv: str, prefixes=("gdn::", "gdn_calib::"),
                 after: str = "reduce_kernel") -> list[dict]:
    """Dispatches of the kernels whose names start with one of ``prefixes``,
    grouped by instantiation and grid (in order of first appearance): count
    and median duration (µs) over all of them, over those that start right
    after a dispatch whose name contains ``after`` (a cache-evicting read),
    and over the others.  Grid as ``X x Y x Z / workgroup`` in work-items."""
    rows = sorted(_rows(trace_csv), key=lambda r: int(r["Start_Timestamp"]))
    groups: dict[tuple, dict] = {}
    prev = ""
    for r in rows:
        name = _kernel_name(r)
        if name.startswith(prefixes):
            key = (name.split("(")[0],
                   f"{r['Grid_Size_X']}x{r['Grid_Size_Y']}x{r['Grid_Size_Z']} / "
                   f"{r['Workgroup_Size_X']}")
            g = groups.setdefault(key, {"kernel": key[0], "grid": key[1], "all": [],
                                        "after": [], "other": []})
            d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            g["all"].append(d)
            g["after" if after in prev else "other"].append(d)
        prev = name
    out = []
    for g in groups.values():
        med = {k: (round(statistics.median(g[k]), 2) if g[k] else None)
               for k in ("all", "after", "other")}
        out.append({"kernel": g["kernel"], "grid": g["grid"], "dispatches": len(g["all"]),
                    "median_us": med["all"], "median_us_after_read": med["after"],
                    "median_us_otherwise": med["other"]})
    return out


def groups_table(groups: list[dict]) -> str:
    """``trace_groups`` as a Markdown table."""
    lines = ["| kernel | grid / block | dispatches | median all (us) | "
             "median after a cache-evicting read (us) | median otherwise (us) |",
             "|---|---|---|---|---|---|"]
    fmt = lambda x: "-" if x is None else f"{x:.2f}"  # noqa: E731
    for g in groups:
        lines.append(f"| `{g['kernel']}` | {g['grid']} | {g['dispatches']} | "
                     f"{fmt(g['median_us'])} | {fmt(g['median_us_after_read'])} | "
                     f"{fmt(g['median_us_otherwise'])} |")
    return "\n".join(lines)


def main(argv=None) -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    p = sub.add_parser("pmc")
    p.add_argument("fetch_csv")
    p.add_argument("write_csv")
    p.add_argument("--kernel", required=True)
    p.add_argument("--copy-bytes", type=int, required=True)
    p.add_argument("--copies", type=int, default=3)
    p.add_argument("--skip", type=int, default=2)
    t = sub.add_parser("trace")
    t.add_argument("trace_csv")
    t.add_argument("--kernel", required=True)
    t.add_argument("--skip", type=int, required=True)
    t.add_argument("--count", type=int, required=True)
    g = sub.add_parser("groups")
    g.add_argument("trace_csv")
    a = ap.parse_args(argv)
    if a.cmd == "groups":
        sys.stdout.write(groups_table(trace_groups(a.trace_csv)) + "\n")
        return
    if a.cmd == "pmc":
        res = pmc_traffic(a.fetch_csv, a.write_csv, a.kernel, a.copy_bytes, a.copies, a.skip)
    else:
        res = trace_average(a.trace_csv, a.kernel, a.skip, a.count)
    json.dump(res, sys.stdout, indent=1)
    sys.stdout.write("\n")


if __name__ == "__main__":
    main()
