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


# --- prefill definition ---------------------------------------------------------

def test_prefill_mix():
    ws = harness.prefill_workloads()
    assert len(ws) == 21
    assert len({w.uuid for w in ws}) == 21 and len({w.seed for w in ws}) == 21
    assert ws[20].lens == (20,) * 4                  # short sequences past the total switch
    assert ws[0].lens == (6,)                        # the reference's workload 0
    assert all((w.H, w.HV, w.use_qk_l2norm) == (4, 8, False) for w in ws)
    assert any(0 in w.lens for w in ws)              # empty sequences
    assert max(max(w.lens) for w in ws) == 16384   # longest single sequence
    # 6 and 1 tokens: the token path; 64 tokens: the one-chunk kernel; 65: prep and scan
    assert [w.dispatches for w in ws[:4]] == [1, 1, 1, 2]
    from flashinfer_competition_codebase_amd.prefill import token_path_max_tokens
    from tests.gdn_cases import prefill_segment_plan
    small = token_path_max_tokens()
    def expected(w):
        slots = min((w.L + 63) // 64 + w.N, w.L)
        if w.L <= small:
            return 1                                  # the token path
        if w.L <= 64 and 2 * w.N * w.HV <= 256:
            return 1                                  # the one-chunk kernel
        offsets = 0 if w.N == 1 or (w.N <= 64 and slots * w.HV <= 2048) else 1
        token = 1 if 2 <= w.N <= 64 and w.L <= w.N * small else 0   # token kernel first
        if prefill_segment_plan(w.L, w.N, w.HV)[0]:
            return token + offsets + 4                # segments
        return token + offsets + 2

    assert all(w.dispatches == expected(w) for w in ws)
    assert harness.prefill_workloads() == ws         # seeded: the same mix every time


def test_prefill_inputs_are_seeded_and_shaped_like_the_definition():
    w = harness.prefill_workloads()[11]              # lens 100, 200, 300, 400
    t1 = harness.make_prefill_inputs(w, "cpu")
    t2 = harness.make_prefill_inputs(w, "cpu")
    for name in ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens"):
        assert torch.equal(t1[name], t2[name]), name
    L, N = 1000, 4
    assert t1["q"].shape == (L, 4, 128) and t1["q"].dtype == torch.bfloat16
    assert t1["v"].shape == (L, 8, 128) and t1["a"].shape == (L, 8)
    assert t1["state"].shape == (N, 8, 128, 128) and t1["state"].dtype == torch.float32
    assert t1["cu_seqlens"].tolist() == [0, 100, 300, 600, 1000]
    assert t1["cu_seqlens"].dtype == torch.int32
    norms = t1["k"].float().norm(dim=-1)
    assert bool(((norms - 1).abs() < 1e-2).all())   # unit rows up to bf16 rounding
    outs = harness._dps_outputs(t1)
    assert outs["output"].shape == (L, 8, 128) and outs["output"].dtype == torch.bfloat16
    assert outs["new_state"].shape == (N, 8, 128, 128)


def test_prefill_baseline_is_workload_0_only():
    ws = harness.prefill_workloads()
    assert harness.baseline_us(ws[0], "fla-b200") == 1536.0    # CLAUDE.md:333-337
    assert harness.baseline_us(ws[0], "fi-b200") == 185.0
    assert all(harness.baseline_us(w, "fi-b200") is None for w in ws[1:])
    dec = harness.contest_decode_workloads()[0]
    assert harness.baseline_us(dec, "fla-b200") == 2.46
    assert harness.baseline_us(dec, None) is None


def _prefill_trace_csv(tmp_path, calls):
    """calls: list of lists of (start offset, duration) ns per dispatch; a
    one-dispatch call is the token-by-token kernel."""
    names = ["void gdn_pf::chunk_offsets_kernel(gdn_pf::Params, int*, int*)",
             "void gdn_pf::prep_kernel(gdn_pf::Params)",
             "void gdn_pf::scan_kernel<1>(gdn_pf::Params)"]
    token = "void gdn::gdn_decode_k128<1, 1, false, 0, false, true, true>(void const*)"
    rows, t = [], 10_000
    for disp in calls:
        rows.append(("void at::native::reduce_kernel<512, 1>", t, t + 700))
        t += 1000
        for j, (off, dur) in enumerate(disp):
            name = token if len(disp) == 1 else names[j + 3 - len(disp)]
            rows.append((name, t + off, t + off + dur))
        t += 100_000
    rows.reverse()
    path = tmp_path / "kernel_trace.csv"
    with open(path, "w") as f:
        f.write('"Kind","Kernel_Name","Start_Timestamp","End_Timestamp"\n')
        for name, s, e in rows:
            f.write(f'"KERNEL_DISPATCH","{name}",{s},{e}\n')
    return path


def test_prefill_trace_attribution_spans_the_calls_dispatches(tmp_path):
    ws = harness.prefill_workloads()
    w0, w2 = ws[0], ws[3]                            # 1 and 2 dispatches per call
    w11 = harness.PrefillWorkload(uuid="prefill-70x1", lens=(1,) * 70, seed=1)   # 3
    assert (w0.dispatches, w2.dispatches, w11.dispatches) == (1, 2, 3)
    m = harness.Manifest()
    calls = []
    m.add(w0.uuid, "check", w0.dispatches); calls.append([(0, 5000)])
    m.add(w0.uuid, "timed", w0.dispatches); calls.append([(0, 4000)])
    m.add(w2.uuid, "timed", w2.dispatches); calls.append([(0, 9000), (10_000, 6000)])
    m.add(w11.uuid, "timed", w11.dispatches)
    calls.append([(0, 3000), (4000, 20_000), (25_000, 30_000)])
    path = _prefill_trace_csv(tmp_path, calls)
    subs = harness.TRACE_KERNELS[harness.PREFILL_DEFINITION]
    res = {r.uuid: r for r in harness.attribute_trace(path, m.calls, kernel_substring=subs,
                                                      baseline="fi-b200")}
    assert res[w0.uuid].timings_us == [4.0]
    assert res[w2.uuid].timings_us == [16.0]         # first start to last end
    assert res[w11.uuid].timings_us == [55.0]
    assert res[w0.uuid].speedup == pytest.approx(185.0 / 4.0)
    assert res[w2.uuid].speedup is None
    with pytest.raises(ValueError, match="dispatches"):
        harness.attribute_trace(path, m.calls[:-1], kernel_substring=subs)


def test_cli_prefill_attribute(tmp_path, capsys):
    ws = harness.prefill_workloads()
    m = harness.Manifest()
    m.add(ws[0].uuid, "timed", 1)
    mpath = tmp_path / "calls.json"
    m.write(mpath)
    tpath = _prefill_trace_csv(tmp_path, [[(0, 20_000)]])
    assert harness.main(["attribute", "--trace", str(tpath), "--manifest", str(mpath),
                         "--definition", harness.PREFILL_DEFINITION]) == 0
    out = capsys.readouterr().out
    assert "gdn_prefill_qk4_v8_d128_k_last:" in out
    assert "Workload prefill-w00: TRACED | 20.000 µs | 76.80x vs B200 fla-chunk" in out


def test_cli_rejects_an_entry_point_of_the_other_definition():
    with pytest.raises(SystemExit, match="prefill-hip"):
        harness.main(["run", "--algo", "hip", "--definition", harness.PREFILL_DEFINITION])
    with pytest.raises(SystemExit, match="available"):
        harness.main(["run", "--algo", "prefill-hip"])


def test_prefill_dispatch_count_follows_the_token_path_threshold():
    from flashinfer_competition_codebase_amd.prefill import (prefill_dispatches,
                                                            token_path_max_tokens)
    m = token_path_max_tokens()
    assert m == 56
    assert prefill_dispatches(m, 1, 8) == 1 and prefill_dispatches(0, 5, 8) == 1
    # past it, at most one chunk (64 tokens) in all and at most 128 (sequence,
    # v-head) pairs: the one-chunk kernel alone
    assert prefill_dispatches(m + 1, 1, 8) == 1 and prefill_dispatches(64, 1, 8) == 1
    assert prefill_dispatches(64, 16, 8) == 1 and prefill_dispatches(64, 4, 32) == 1
    assert prefill_dispatches(65, 1, 8) == 2              # two chunks: prep and scan
    # 2..64 sequences of at most m tokens on average: the token kernel first
    # (it runs if every sequence is that short), then prep and scan
    assert prefill_dispatches(64, 17, 8) == 3             # 136 pairs: no one-chunk kernel
    assert prefill_dispatches(65, 2, 8) == 3
    assert prefill_dispatches(2 * m, 2, 8) == 3 and prefill_dispatches(2 * m + 1, 2, 8) == 2
    assert prefill_dispatches(80, 4, 8) == 3              # 4 x 20 tokens
    assert prefill_dispatches(m + 1, 64, 8) == 3          # slots found in the kernels
    assert prefill_dispatches(m + 1, 65, 8) == 3          # the chunk-offsets scan first
    assert prefill_dispatches(65 * m + 1, 65, 8) == 3
    assert prefill_dispatches(640, 8, 8) == 2             # 10 chunks + 8: slots in the kernels
    assert prefill_dispatches(8192, 8, 8) == 4            # 8 x 16 chunks at 8 v-heads: segments
    assert prefill_dispatches(8192, 16, 32) == 3          # (128 + 16) x 32 = 4608, 512 heads
    assert prefill_dispatches(16384, 1, 128) == 2         # one sequence: never offsets
    assert prefill_dispatches(16384, 1, 32) == 4          # ... cut into segments
    assert prefill_dispatches(39503, 8, 8) == 5           # offsets, then segments
    assert prefill_dispatches(m, 70_000, 8) == 3         # past the grid's z limit
    assert prefill_dispatches(100, 0, 8) == 0
