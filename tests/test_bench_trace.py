"""bench.py's kernel-trace attribution: host logic on a synthetic rocprofv3
kernel_trace.csv (no GPU)."""

import csv
import random

import pytest

import bench

DECODE = "void gdn::gdn_decode_k128<2, 2, true, 1, false, false>(void const*, ...)"


def _write_trace(path, spans):
    """spans: (kernel name, duration ns) in launch order, 10 us apart."""
    rows = []
    for i, (name, dur) in enumerate(spans):
        start = 1_000_000 + 10_000 * i
        rows.append({"Kernel_Name": name, "Start_Timestamp": start,
                     "End_Timestamp": start + dur})
    random.Random(0).shuffle(rows)          # the parser orders by start time
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        w.writerows(rows)


MANIFEST = {
    "decode": [
        {"name": "x", "warmup": 1, "steady": 4, "steady_skip": 2, "cold": 2},
        {"name": "y", "warmup": 0, "steady": 3, "steady_skip": 1, "cold": 1},
    ],
    "floor": {"rmw": 3, "rmw_skip": 1, "empty": 2, "empty_blocks": 256},
}


def _spans():
    flush = ("void at::native::reduce_kernel<512, 1>(...)", 90_000)
    return [
        (DECODE, 50_000),                                 # x warmup
        (DECODE, 1), (DECODE, 1), (DECODE, 3000), (DECODE, 5000),   # x steady
        flush, (DECODE, 6000), flush, (DECODE, 8000),     # x cold
        (DECODE, 7), (DECODE, 2000), (DECODE, 2200),      # y steady
        flush, (DECODE, 4400),                            # y cold
        ("gdn_calib::rmw<true>(float*, float)", 1), ("gdn_calib::rmw<true>(float*, float)", 2500),
        ("gdn_calib::rmw<true>(float*, float)", 2700),
        ("gdn_calib::empty()", 1400), ("gdn_calib::empty()", 1600),
    ]


def test_attribution_by_launch_order(tmp_path):
    p = tmp_path / "trace_kernel_trace.csv"
    _write_trace(p, _spans())
    res = bench.attribute_kernel_trace(p, MANIFEST)
    x, y = res["shapes"]["x"], res["shapes"]["y"]
    assert (x["steady"], x["cold"], x["n_steady"], x["n_cold"]) == (4.0, 7.0, 2, 2)
    assert (y["steady"], y["cold"], y["n_steady"], y["n_cold"]) == (2.1, 4.4, 2, 1)
    assert res["floor"] == {"b1_rmw_us": 2.6, "empty_us": 1.5, "empty_blocks": 256}


def test_dispatch_count_mismatch_raises(tmp_path):
    p = tmp_path / "trace_kernel_trace.csv"
    _write_trace(p, _spans()[1:])           # one decode dispatch missing
    with pytest.raises(ValueError, match="decode dispatches"):
        bench.attribute_kernel_trace(p, MANIFEST)


def test_floor_omitted_when_counts_differ(tmp_path):
    p = tmp_path / "trace_kernel_trace.csv"
    _write_trace(p, _spans()[:-1])          # one empty kernel missing
    assert bench.attribute_kernel_trace(p, MANIFEST)["floor"] is None


def test_leg_skipped_under_rocprofv3(monkeypatch):
    monkeypatch.setenv("ROCPROF_OUTPUT_PATH", "/tmp")
    assert "skipped" in bench.kernel_trace_leg(10)
