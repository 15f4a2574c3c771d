"""Host-side contract of the Python entry points (runs without a GPU).

Mirrors the reference's calling conventions (solution/triton/kernel.py:22-197,
solution/cuda/binding.py:35-60, scripts/shared.py:19-37) and checks that every
malformed argument raises before the C ABI is reached.
"""

from __future__ import annotations

import inspect
import math

import pytest
import torch

import flashinfer_competition_codebase_amd as gdn
from flashinfer_competition_codebase_amd import _lib
from oracle.gdn_decode_oracle import make_inputs

REF_ARGS = ["q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "scale"]


def test_signatures_match_reference_names():
    p = inspect.signature(gdn.run).parameters
    assert [n for n, x in p.items() if x.kind is x.POSITIONAL_OR_KEYWORD] == REF_ARGS
    assert p["use_qk_l2norm"].kind is inspect.Parameter.KEYWORD_ONLY
    assert p["use_qk_l2norm"].default is False
    p = inspect.signature(gdn.kernel_hip).parameters
    assert [n for n, x in p.items() if x.kind is x.POSITIONAL_OR_KEYWORD] == (
        REF_ARGS + ["output", "new_state"])
    assert gdn.ENTRY_POINTS["hip"] is gdn.kernel_hip
    assert gdn.run_dps is gdn.kernel_hip
    assert gdn.ENTRY_POINTS["hip-run"] is gdn.run
    assert gdn.NO_DPS == {"hip-run", "prefill-hip-run"}
    # prefill: kernel_prefill_reference / kernel_prefill_fla_chunk argument names
    # (solution/triton/prefill_kernel.py:10-12, 85-87)
    pref = REF_ARGS[:8] + ["cu_seqlens", "scale"]
    p = inspect.signature(gdn.prefill_run).parameters
    assert [n for n, x in p.items() if x.kind is x.POSITIONAL_OR_KEYWORD] == pref
    p = inspect.signature(gdn.kernel_prefill_hip).parameters
    assert [n for n, x in p.items() if x.kind is x.POSITIONAL_OR_KEYWORD] == (
        pref + ["output", "new_state"])


@pytest.mark.parametrize("scale,expect", [
    (None, 1 / math.sqrt(128)), (0, 1 / math.sqrt(128)), (0.0, 1 / math.sqrt(128)),
    (0.25, 0.25), (torch.tensor(0.5), 0.5), (torch.tensor([0.5]), 0.5),
    (torch.tensor(0.0), 1 / math.sqrt(128)),
])
def test_resolve_scale(scale, expect):
    assert gdn.resolve_scale(scale, 128) == pytest.approx(expect)


def test_resolve_scale_rejects_vectors():
    with pytest.raises(ValueError):
        gdn.resolve_scale(torch.ones(2), 128)


@pytest.fixture
def no_lib(monkeypatch):
    """Fail the test if anything reaches the native library."""
    def boom():
        raise AssertionError("validation let a malformed call reach the C ABI")
    monkeypatch.setattr(_lib, "get_lib", boom)


def _inputs(B=2, H=2, HV=4):
    t = make_inputs(B, H, HV, seed=3)
    t["output"] = torch.empty(B, 1, HV, 128, dtype=torch.bfloat16)
    t["new_state"] = torch.empty(B, HV, 128, 128)
    return t


def _bad(name, value):
    t = _inputs()
    t[name] = value
    return t


BAD_CASES = {
    "T=0": ({**_inputs(), "q": torch.zeros(2, 0, 2, 128, dtype=torch.bfloat16)}, ValueError),
    "T=2 q only": ({**_inputs(), "q": torch.zeros(2, 2, 2, 128, dtype=torch.bfloat16)}, ValueError),
    "K=64": ({**_inputs(), "q": torch.zeros(2, 1, 2, 64, dtype=torch.bfloat16)}, ValueError),
    "HV%H": ({**_inputs(), "q": torch.zeros(2, 1, 3, 128, dtype=torch.bfloat16)}, ValueError),
    "q fp32": (_bad("q", torch.zeros(2, 1, 2, 128)), TypeError),
    "k shape": (_bad("k", torch.zeros(2, 1, 1, 128, dtype=torch.bfloat16)), ValueError),
    "v noncontig": (_bad("v", torch.zeros(2, 1, 128, 4, dtype=torch.bfloat16).transpose(2, 3)),
                    ValueError),
    "state fp16": (_bad("state", torch.zeros(2, 4, 128, 128, dtype=torch.float16)), TypeError),
    "new_state dtype": (_bad("new_state", torch.empty(2, 4, 128, 128, dtype=torch.bfloat16)),
                        TypeError),
    "state shape": (_bad("state", torch.zeros(2, 4, 128, 64)), ValueError),
    "A_log shape": (_bad("A_log", torch.zeros(2)), ValueError),
    "dt_bias f64": (_bad("dt_bias", torch.zeros(4, dtype=torch.float64)), TypeError),
    "a shape": (_bad("a", torch.zeros(2, 4, 1, dtype=torch.bfloat16)), ValueError),
    "b fp32": (_bad("b", torch.zeros(2, 1, 4)), TypeError),
    "output dtype": (_bad("output", torch.empty(2, 1, 4, 128)), TypeError),
    "new_state shape": (_bad("new_state", torch.empty(2, 4, 128, 127)), ValueError),
    "q not tensor": (_bad("q", [[1.0]]), ValueError),
    "v 3-D": (_bad("v", torch.zeros(2, 4, 128, dtype=torch.bfloat16)), ValueError),
}


@pytest.mark.parametrize("case", list(BAD_CASES))
def test_malformed_arguments_raise_before_the_abi(case, no_lib):
    t, exc = BAD_CASES[case]
    with pytest.raises(exc):
        gdn.kernel_hip(**t)
    t = {n: x for n, x in t.items() if n not in ("output", "new_state")}
    if case not in ("output dtype", "new_state shape", "new_state dtype"):
        with pytest.raises(exc):
            gdn.run(**t)


def test_cpu_tensors_are_rejected_not_computed(no_lib):
    t = _inputs()
    with pytest.raises(ValueError, match="HIP device"):
        gdn.kernel_hip(**t)
    with pytest.raises(ValueError, match="HIP device"):
        gdn.run(**{n: x for n, x in t.items() if n not in ("output", "new_state")})


def test_mixed_devices_are_rejected(no_lib):
    t = _inputs()
    t["A_log"] = t["A_log"].to("meta")
    with pytest.raises(ValueError, match="one device"):
        gdn.kernel_hip(**t)


def test_dps_needs_outputs(no_lib):
    t = _inputs()
    t["output"] = None
    with pytest.raises(ValueError):
        gdn.kernel_hip(**t)


def test_gate_tensors_accept_both_reference_shapes(no_lib):
    t = _inputs()
    t["a"] = t["a"].reshape(2, 4)
    t["b"] = t["b"].reshape(2, 4)
    with pytest.raises(ValueError, match="HIP device"):   # shapes accepted, device refused
        gdn.kernel_hip(**t)


def test_multi_token_and_bf16_state_shapes_are_accepted(no_lib):
    t = make_inputs(2, 2, 4, seed=5, T=3)
    t["output"] = torch.empty(2, 3, 4, 128, dtype=torch.bfloat16)
    t["new_state"] = torch.empty(2, 4, 128, 128)
    with pytest.raises(ValueError, match="HIP device"):   # shapes accepted, device refused
        gdn.kernel_hip(**t)
    t["state"] = t["state"].to(torch.bfloat16)
    t["new_state"] = torch.empty(2, 4, 128, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="HIP device"):
        gdn.kernel_hip(**t)
    bad = {**t, "a": t["a"][:, :1]}                        # gates for one token only
    with pytest.raises(ValueError):
        gdn.kernel_hip(**bad)
    bad = {**t, "output": torch.empty(2, 1, 4, 128, dtype=torch.bfloat16)}
    with pytest.raises(ValueError):
        gdn.kernel_hip(**bad)


def test_nonzero_abi_code_raises(monkeypatch):
    class FakeLib:
        def gdn_decode_error_string(self, code):
            return b"invalid argument"
    monkeypatch.setattr(_lib, "get_lib", lambda: FakeLib())
    with pytest.raises(RuntimeError, match="invalid argument"):
        _lib.check(1, "gdn_decode_step")
    _lib.check(0, "gdn_decode_step")


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="not found"):
        _lib.load(tmp_path / "libgdn_decode.so")
