"""The harness over the 54-workload contest mix on MI355X, checked against the
oracle (the role the contest definition's reference plays)."""

from __future__ import annotations

import sys

import pytest
import torch

import flashinfer_competition_codebase_amd as gdn
from flashinfer_competition_codebase_amd import _lib, harness
from oracle.gdn_decode_oracle import oracle_vec

pytestmark = pytest.mark.gpu


def _announce(case):
    sys.stdout.write(f"[gpu case] {case}\n")
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _library_present():
    _lib.get_lib()


def test_contest_mix_passes_with_the_dps_entry(hip_device):
    _announce("harness: 54 contest workloads, DPS entry, event tier")
    ws = harness.contest_decode_workloads()
    m = harness.Manifest()
    res = harness.evaluate(gdn.kernel_hip, ws, dps=True, reference=oracle_vec,
                           device=hip_device, warmup=1, iterations=2, num_trials=1,
                           manifest=m)
    assert [r.status for r in res] == ["PASSED"] * 54, [(r.uuid, r.status) for r in res]
    assert len(m.calls) == 54 * (1 + 1 + 2)
    assert all(r.latency_us > 0 and len(r.timings_us) == 2 for r in res)
    assert all(r.max_abs_error < 1e-2 for r in res)
    assert harness.mean_speedup(res) > 0


def test_value_returning_entry_and_sync_tier(hip_device):
    _announce("harness: value-returning entry, sync tier")
    ws = [w for w in harness.contest_decode_workloads() if w.uuid.endswith("-00")]
    res = harness.evaluate(gdn.run, ws, dps=False, reference=oracle_vec, device=hip_device,
                           warmup=1, iterations=2, num_trials=1, tier="sync", flush="zero")
    assert [r.status for r in res] == ["PASSED"] * len(ws)


def test_a_wrong_solution_is_flagged(hip_device):
    """A solution that skips the decay fails the allclose check."""
    _announce("harness: planted wrong solution")

    def no_decay(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state):
        gdn.kernel_hip(q, k, v, state, torch.full_like(A_log, -float("inf")), a, dt_bias, b,
                       scale, output, new_state)

    w = harness.contest_decode_workloads()[20]
    res = harness.evaluate(no_decay, [w], reference=oracle_vec, device=hip_device, warmup=0,
                           iterations=1, num_trials=1, flush="none")
    assert res[0].status == "INCORRECT_NUMERICAL"


def test_prefill_mix_short_workloads_pass(hip_device):
    """The prefill definition through the harness: the short workloads of the
    mix (including empty sequences), DPS and value-returning entries, checked
    against the oracle's token loop."""
    from oracle.gdn_prefill_oracle import prefill_loop

    _announce("harness: prefill mix, short workloads, DPS and value-returning")
    ws = [w for w in harness.prefill_workloads() if w.L <= 1000]
    m = harness.Manifest()
    res = harness.evaluate(gdn.kernel_prefill_hip, ws, dps=True, reference=prefill_loop,
                           device=hip_device, warmup=1, iterations=2, num_trials=1, manifest=m)
    assert [r.status for r in res] == ["PASSED"] * len(ws), [(r.uuid, r.status) for r in res]
    assert len(m.calls) == len(ws) * 4
    assert all(c[2] == w.dispatches for w in ws for c in m.calls if c[0] == w.uuid)
    assert res[0].speedup is not None and res[0].speedup > 0     # workload 0 vs B200
    res2 = harness.evaluate(gdn.prefill_run, ws[:3], dps=False, reference=prefill_loop,
                            device=hip_device, warmup=0, iterations=1, num_trials=1,
                            tier="sync", flush="none")
    assert [r.status for r in res2] == ["PASSED"] * 3
