"""Host-side logic of the flashinfer-bench-style harness (no GPU needed)."""

from __future__ import annotations

import io
import json
import math

import pytest
import torch

from flashinfer_competition_codebase_amd import harness


def test_contest_mix_is_the_54_workload_decode_set():
    ws = harness.contest_decode_workloads()
    assert len(ws) == 54
    counts = {}
    for w in ws:
        counts[w.B] = counts.get(w.B, 0) + 1
        assert (w.H, w.HV, w.T, w.use_qk_l2norm) == (4, 8, 1, False)
    assert counts == {1: 10, 4: 8, 8: 7, 16: 7, 32: 7, 48: 7, 64: 8}   # CLAUDE.md:139-140
    assert len({w.uuid for w in ws}) == 54
    assert len({w.seed for w in ws}) == 54


def test_inputs_are_seeded_and_shaped_like_the_definition():
    w = harness.contest_decode_workloads()[12]
    t1 = harness.make_inputs(w, "cpu")
    t2 = harness.make_inputs(w, "cpu")
    for name in ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b"):
        assert torch.equal(t1[name], t2[name]), name
    B = w.B
    assert t1["q"].shape == (B, 1, 4, 128) and t1["q"].dtype == torch.bfloat16
    assert t1["v"].shape == (B, 1, 8, 128)
    assert t1["state"].shape == (B, 8, 128, 128) and t1["state"].dtype == torch.float32
    assert t1["a"].shape == (B, 1, 8) and t1["A_log"].shape == (8,)
    assert bool((t1["A_log"] >= 0).all()) and bool((t1["A_log"] <= math.log(16) + 1e-6).all())
    assert t1["scale"] == pytest.approx(1 / math.sqrt(128))
    outs = harness._dps_outputs(t1)
    assert outs["output"].shape == (B, 1, 8, 128) and outs["output"].dtype == torch.bfloat16
    assert outs["new_state"].shape == (B, 8, 128, 128)


def test_compare_is_the_allclose_criterion():
    y = torch.tensor([1.0, -2.0, 0.0, 100.0])
    assert harness.compare(y.clone(), y)[0] == "PASSED"
    # |x - y| <= 1e-2 + 1e-2 |y|: 100 -> 101 is allowed (1.0 <= 1.01), 0 -> 0.011 is not
    ok = y.clone()
    ok[3] = 101.0
    assert harness.compare(ok, y)[0] == "PASSED"
    bad = y.clone()
    bad[2] = 0.011
    status, max_abs, max_rel = harness.compare(bad, y)
    assert status == "INCORRECT_NUMERICAL"
    assert max_abs == pytest.approx(0.011)
    assert harness.compare(y[:3], y)[0] == "INCORRECT_SHAPE"
    assert harness.compare(y.double(), y)[0] == "INCORRECT_DTYPE"
    nan = y.clone()
    nan[0] = float("nan")
    assert harness.compare(nan, y)[0] == "INCORRECT_NUMERICAL"


def _trace_csv(tmp_path, durations_ns, other_every=2):
    """A rocprofv3-style kernel_trace.csv: one gdn dispatch per duration, with
    unrelated dispatches interleaved, rows shuffled out of time order."""
    rows = []
    t = 1000
    for i, d in enumerate(durations_ns):
        if i % other_every == 0:
            rows.append(("void at::native::reduce_kernel<512, 1>", t, t + 500))
            t += 1000
        rows.append(("void gdn::gdn_decode_k128<1, 1, false, 1, false, false>(void const*)",
                     t, t + d))
        t += d + 100
    rows.reverse()
    path = tmp_path / "kernel_trace.csv"
    with open(path, "w") as f:
        f.write('"Kind","Kernel_Name","Start_Timestamp","End_Timestamp"\n')
        for name, s, e in rows:
            f.write(f'"KERNEL_DISPATCH","{name}",{s},{e}\n')
    return path


def test_trace_attribution_assigns_dispatches_in_time_order(tmp_path):
    ws = harness.contest_decode_workloads()
    w1, w4 = ws[0], ws[10]                     # B=1 and B=4
    m = harness.Manifest()
    durs = []
    for w, base in ((w1, 3000), (w4, 5000)):
        m.add(w.uuid, "check"); durs.append(99_000)
        m.add(w.uuid, "warmup"); durs.append(77_000)
        for i in range(3):
            m.add(w.uuid, "timed"); durs.append(base + 100 * i)
    path = _trace_csv(tmp_path, durs)
    res = {r.uuid: r for r in harness.attribute_trace(path, m.calls)}
    assert res[w1.uuid].timings_us == [3.0, 3.1, 3.2]
    assert res[w4.uuid].latency_us == pytest.approx(5.1)
    assert res[w1.uuid].speedup == pytest.approx(2.46 / 3.1)
    assert res[w4.uuid].speedup == pytest.approx(3.10 / 5.1)
    with pytest.raises(ValueError):
        harness.attribute_trace(path, m.calls[:-1])


def test_cli_attribute_and_output_format(tmp_path, capsys):
    ws = harness.contest_decode_workloads()
    m = harness.Manifest()
    durs = []
    for w in ws[:2]:
        m.add(w.uuid, "timed")
        durs.append(2000)
    mpath = tmp_path / "calls.json"
    m.write(mpath)
    tpath = _trace_csv(tmp_path, durs)
    jpath = tmp_path / "res.json"
    assert harness.main(["attribute", "--trace", str(tpath), "--manifest", str(mpath),
                         "--baseline", "fi-b200", "--json", str(jpath)]) == 0
    out = capsys.readouterr().out
    assert "gdn_decode_qk4_v8_d128_k_last:" in out
    assert f"Workload {ws[0].uuid}: TRACED | 2.000 µs | 1.68x vs B200 FlashInfer" in out
    assert "mean speedup vs B200 FlashInfer over 2 workloads: 1.680x" in out
    doc = json.loads(jpath.read_text())
    assert doc["mean_speedup"] == pytest.approx(3.36 / 2.0)
    assert doc["per_batch_median_us"] == {"1": 2.0}


def test_print_results_layout_matches_the_reference_runner():
    r = harness.Result("qk4v8-b01-00", 1, "PASSED", latency_us=4.448, max_abs_error=3.05e-05,
                       max_rel_error=9.11e-02, speedup=0.55)
    buf = io.StringIO()
    harness.print_results([r], file=buf)
    line = buf.getvalue().splitlines()[2]
    assert line == ("  Workload qk4v8-b01-00: PASSED | 4.448 µs | 0.55x vs B200 fla-recurrent"
                    " | abs_err=3.05e-05, rel_err=9.11e-02")


def test_workload_selection():
    ws = harness.contest_decode_workloads()
    assert [w.B for w in harness._select(ws, 0, "qk4v8-b16")] == [16] * 7
    assert len(harness._select(ws, 5, None)) == 5
    with pytest.raises(ValueError):
        harness._select(ws, 0, "nope")


def test_evaluate_rejects_unknown_tier_and_flush():
    with pytest.raises(ValueError):
        harness.evaluate(lambda **k: None, [], tier="cupti")
    with pytest.raises(ValueError):
        harness.evaluate(lambda **k: None, [], flush="l2")
