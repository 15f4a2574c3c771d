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


def test_steady_average_beside_the_median(tmp_path):
    p = tmp_path / "trace_kernel_trace.csv"
    _write_trace(p, _spans())
    x = bench.attribute_kernel_trace(p, MANIFEST)["shapes"]["x"]
    assert x["steady_avg"] == 4.0            # (3000 + 5000) / 2 ns


def _pmc_csv(path, counter, dispatches):
    """dispatches: (kernel name, value) in order, one counter row each."""
    fields = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=fields)
        w.writeheader()
        for i, (name, val) in enumerate(dispatches):
            w.writerow({"Dispatch_Id": i + 1, "Kernel_Name": name, "Counter_Name": counter,
                        "Counter_Value": val})


def test_counter_summary_scales_by_the_calibration_copies(tmp_path):
    """FETCH_SIZE reading half the copy's bytes doubles the kernel's fetch;
    the first two launches are skipped; the summary names the kernel."""
    from flashinfer_competition_codebase_amd.rocprof import pmc_traffic

    copy = "__amd_rocclr_copyBuffer"
    kern = "void gdn::gdn_decode_k128<2, 4, true, 1, false, false, false>(void const*)"
    mib = 1024 * 1024
    _pmc_csv(tmp_path / "f.csv", "FETCH_SIZE",
             [(copy, 512.0)] * 3 + [(kern, 9999.0), (kern, 9999.0), (kern, 1000.0), (kern, 1002.0),
                                    (kern, 1004.0), (copy, 7.0)])
    _pmc_csv(tmp_path / "w.csv", "WRITE_SIZE",
             [(copy, 1024.0)] * 3 + [(kern, 1.0), (kern, 1.0), (kern, 2048.0)] * 1
             + [(kern, 2048.0), (kern, 2048.0)])
    res = pmc_traffic(tmp_path / "f.csv", tmp_path / "w.csv",
                      "gdn::gdn_decode_k128<2, 4, true, 1, false, false, false>", mib)
    assert res["calibration"]["fetch_factor"] == 0.5
    assert res["fetch_bytes_per_launch"] == 1002 * 1024 * 2
    assert res["write_bytes_per_launch"] == 2048 * 1024
    assert res["kernel"].startswith("gdn::gdn_decode_k128<2, 4, true, 1")


def test_traffic_only_from_a_summary_of_the_timed_kernel(tmp_path, monkeypatch):
    import json

    kernel = bench.decode_kernel_name(2, 4, True, 1)
    assert kernel == "gdn::gdn_decode_k128<2, 4, true, 1, false, false, false>"
    path = tmp_path / "traffic.json"
    monkeypatch.setattr(bench, "TRAFFIC_SUMMARY", path)
    monkeypatch.setattr(bench, "ROOT", tmp_path)
    for rel in bench.DECODE_SOURCES:
        (tmp_path / rel).parent.mkdir(parents=True, exist_ok=True)
        (tmp_path / rel).write_text(rel)
    sha = bench.sources_sha(bench.DECODE_SOURCES)
    path.write_text(json.dumps({"kernel": kernel + "(void const*)", "sources_sha": sha,
                                "traffic_bytes_per_launch": 123}))
    assert bench._traffic(kernel) == (123, "traffic.json")
    assert bench._traffic(bench.decode_kernel_name(4, 4, True, 1))[0] is None
    path.write_text(json.dumps({"kernel": kernel, "sources_sha": "0" * 16,
                                "traffic_bytes_per_launch": 123}))
    assert bench._traffic(kernel)[0] is None


def test_prefill_counter_summary_and_its_sources_check(tmp_path, monkeypatch):
    """The prefill summary scales prep and scan by the calibration copies,
    skips the first prefill, and the roofline reads it only while the
    prefill sources are the ones it was measured on."""
    import json

    copy = "__amd_rocclr_copyBuffer"
    prep = "void gdn_pf::prep_kernel<false>(gdn_pf::Params)"
    scan = "void gdn_pf::scan_kernel<false, false, true, false, 8>(gdn_pf::Params)"
    off = "gdn_pf::chunk_offsets_kernel(gdn_pf::Params, int*, int __vector(4)*)"
    mib = 1024 * 1024
    calls = [(off, 1.0), (prep, 5.0), (scan, 7.0)] + [(off, 1.0), (prep, 100.0), (scan, 300.0)] * 2
    _pmc_csv(tmp_path / "f.csv", "FETCH_SIZE", [(copy, 128.0 * 1024)] * 3 + calls)
    _pmc_csv(tmp_path / "w.csv", "WRITE_SIZE", [(copy, 256.0 * 1024)] * 3 + calls)
    monkeypatch.setattr(bench, "ROOT", tmp_path)
    for rel in bench.PREFILL_SOURCES:
        (tmp_path / rel).parent.mkdir(parents=True, exist_ok=True)
        (tmp_path / rel).write_text(rel)
    res = bench.summarize_pmc_prefill(tmp_path / "f.csv", tmp_path / "w.csv")
    assert res["kernels"]["prep"]["fetch_bytes_per_launch"] == 100 * 1024 * 2   # fetch reads half
    assert res["kernels"]["scan"]["write_bytes_per_launch"] == 300 * 1024
    assert res["traffic_bytes_per_prefill"] == (100 * 2 + 100 + 300 * 2 + 300) * 1024
    lens, H, HV = bench.PREFILL_CONFIGS[bench.PREFILL_ROOFLINE_WORKLOAD]
    assert res["algorithmic_bytes_per_prefill"] == bench.prefill_bytes(lens, H, HV)
    path = tmp_path / "prefill_traffic.json"
    monkeypatch.setattr(bench, "PREFILL_TRAFFIC_SUMMARY", path)
    path.write_text(json.dumps(res))
    assert bench._prefill_traffic() == {"prep": 300 * 1024, "scan": 900 * 1024}
    (tmp_path / bench.PREFILL_SOURCES[0]).write_text("changed")
    assert bench._prefill_traffic() is None


def test_trace_groups_splits_after_read(tmp_path):
    """rocprof.trace_groups: per instantiation and grid, in first-seen order,
    medians over all dispatches, those right after a reduce_kernel (a
    cache-evicting read), and the others."""
    from flashinfer_competition_codebase_amd import rocprof

    cols = ("Kernel_Name", "Start_Timestamp", "End_Timestamp", "Grid_Size_X", "Grid_Size_Y",
            "Grid_Size_Z", "Workgroup_Size_X")
    rows = [("void gdn::gdn_decode_k128<2, 4>(int)", 0, 2000, 256, 16, 1, 256),
            ("reduce_kernel", 3000, 4000, 64, 1, 1, 64),
            ("void gdn::gdn_decode_k128<2, 4>(int)", 5000, 9000, 256, 16, 1, 256),
            ("void gdn::gdn_decode_block<4, 2, true, true>(int)", 10000, 13000, 128, 16, 1, 128),
            ("void gdn::gdn_decode_k128<2, 4>(int)", 14000, 17000, 256, 16, 1, 256),
            ("void gdn::gdn_decode_k128<2, 4>(int)", 18000, 19000, 256, 16, 2, 256)]
    path = tmp_path / "trace.csv"
    path.write_text(",".join(cols) + "\n" + "".join(",".join(f'"{x}"' for x in r) + "\n"
                                                    for r in rows))
    g = rocprof.trace_groups(str(path))
    assert [x["kernel"] for x in g] == ["gdn::gdn_decode_k128<2, 4>",
                                        "gdn::gdn_decode_block<4, 2, true, true>",
                                        "gdn::gdn_decode_k128<2, 4>"]
    assert g[0]["grid"] == "256x16x1 / 256" and g[0]["dispatches"] == 3
    assert g[0]["median_us"] == 3.0                      # 2, 4, 3 us
    assert g[0]["median_us_after_read"] == 4.0
    assert g[0]["median_us_otherwise"] == 2.5
    assert g[2]["grid"] == "256x16x2 / 256" and g[2]["median_us_after_read"] is None
    assert "| `gdn::gdn_decode_block<4, 2, true, true>` | 128x16x1 / 128 | 1 |" in \
        rocprof.groups_table(g)


def test_prefill_roofline_reports_the_binding_roof(monkeypatch):
    """The prefill line names the roof whose floor time is larger (the 64 x
    512 qk16_v32 workload: 175 FLOP/B, under the bf16 ridge of 312 FLOP/B,
    so HBM) and carries both roofs' fractions, each computed from the
    workload's algorithmic bytes / FLOP over the kernel time."""
    monkeypatch.setattr(bench, "_prefill_traffic", lambda: None)
    lens, H, HV = bench.PREFILL_CONFIGS[bench.PREFILL_ROOFLINE_WORKLOAD]
    ku = {"offsets": 6.0, "prep": 110.0, "scan": 400.0, "kernels": 516.0}
    res = bench.prefill_roofline({bench.PREFILL_ROOFLINE_WORKLOAD: {
        "kernel_us": ku, "prep_workspace_bytes": 0}})
    alg = bench.prefill_bytes(lens, H, HV)
    flop = sum((n + 63) // 64 for n in lens) * HV * bench.PREFILL_FLOP_PER_CHUNK_HEAD
    assert flop / alg < bench.PEAK_BF16_TFLOPS * 1e12 / (bench.PEAK_HBM_GBS * 1e9)
    assert res["bound"] == "hbm" and res["unit"] == "GB/s"
    hbm_frac = alg / 516e-6 / 1e9 / bench.PEAK_HBM_GBS
    assert res["frac"] == pytest.approx(hbm_frac, abs=1e-4) == res["hbm"]["frac"]
    assert res["mfma"]["frac"] == pytest.approx(
        flop / 516e-6 / 1e12 / bench.PEAK_BF16_TFLOPS, abs=1e-4)
    assert res["hbm"]["floor_us"] > res["mfma"]["floor_us"]
