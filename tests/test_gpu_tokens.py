"""Multi-token decode (T > 1) and the bf16 state on MI355X, against the oracle.

T tokens per sequence read the state once, apply the per-token recurrence of
the reference's prefill oracle (solution/triton/prefill_kernel.py:144-178)
in order, and write the state once.  Bars: outputs as in
test_gpu_parity.py (1e-2 atol/rtol against the oracle's bf16 output, one
bf16 ulp against float64); fp32 states within 1e-3 relative + 1e-5; bf16
states within one bf16 ulp (2^-7 relative) of the oracle's bf16 state and
within half an ulp (2^-8 relative) plus 1e-6 of the float64 state, with at
most 0.1% of elements off by that ulp.
"""

from __future__ import annotations

import itertools
import sys

import pytest
import torch

import flashinfer_competition_codebase_amd as gdn
from flashinfer_competition_codebase_amd import _lib
from oracle.gdn_decode_oracle import make_inputs, oracle_loop, oracle_tokens, oracle_vec
from tests.gdn_cases import assert_output_close, assert_state_close

pytestmark = pytest.mark.gpu


def _announce(case):
    sys.stdout.write(f"[gpu case] {case}\n")
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _library_present():
    _lib.get_lib()


def _dev(t, device):
    return {n: (x.to(device) if isinstance(x, torch.Tensor) else x) for n, x in t.items()}


def _oracle(t, l2, state_dtype):
    B, HV = t["v"].shape[0], t["v"].shape[2]
    step = oracle_loop if B * HV <= 256 else oracle_vec
    ref_o, ref_s = oracle_tokens(step, **t, use_qk_l2norm=l2, state_dtype=state_dtype)

    def vec64(*args, **kw):
        return oracle_vec(*args, **kw, output_fp32=True, dtype=torch.float64)

    o64, s64 = oracle_tokens(vec64, **t, use_qk_l2norm=l2, state_dtype=None)
    return ref_o, ref_s, o64, s64


def _check_bf16_state(st, ref_s, s64, what):
    st = st.cpu().double()
    ref = ref_s.double()
    d_ref = (st - ref).abs()
    assert bool((d_ref <= 2.0 ** -7 * ref.abs() + 1e-6).all()), f"{what}: beyond one bf16 ulp"
    off = (d_ref > 0).double().mean().item()
    assert off <= 1e-3, f"{what}: {off:.2%} of elements differ from the oracle's bf16 state"
    d64 = (st - s64).abs()
    assert bool((d64 <= 2.0 ** -8 * s64.abs() + 1e-6).all()), f"{what}: not the RNE of the result"


@pytest.mark.parametrize("B,H,HV,T,l2", [
    (1, 16, 32, 2, True), (1, 16, 32, 4, True), (8, 16, 32, 3, True),
    (64, 16, 32, 4, True), (128, 8, 32, 2, False), (4, 4, 8, 8, False), (2, 5, 15, 3, True),
    # past 64 tokens the per-lane gate table is refilled (at token 64, 128);
    # unit keys (L2-norm) keep the state bounded over so many tokens (raw
    # N(0, 1) keys multiply it by ~|1 - beta |k|^2| ~ 60 per token)
    (1, 4, 8, 70, True), (2, 16, 32, 66, True), (1, 4, 8, 130, True),
])
def test_multi_token(B, H, HV, T, l2, hip_device):
    _announce(f"multi-token B={B} H={H} HV={HV} T={T} l2={l2}")
    t = make_inputs(B, H, HV, seed=5000 + 7 * B + T, T=T)
    out, new_state = gdn.run(**_dev(t, hip_device), use_qk_l2norm=l2)
    torch.cuda.synchronize()
    assert out.shape == (B, T, HV, 128)
    ref_o, ref_s, o64, s64 = _oracle(t, l2, torch.float32)
    assert_output_close(out.cpu(), ref_o, tight_ref64=o64, what="output")
    assert_state_close(new_state.cpu(), ref_s)
    assert (new_state.cpu().double() - s64).abs().max().item() < 1e-4


@pytest.mark.parametrize("B,H,HV,T", [(3, 16, 32, 4), (1, 4, 8, 70)])
def test_multi_token_agrees_with_chained_single_tokens(B, H, HV, T, hip_device):
    """One launch of T tokens against T chained T=1 launches (at T=70 across
    the refill of the per-lane gate table at token 64).  The multi-token loop
    applies each token's decay lazily (the state held divided by the decay
    not yet applied, one FMA per element per token), the single-token kernel
    directly, so the two round differently: outputs agree within one bf16
    ulp, states within 1e-5 relative + 1e-6."""
    _announce(f"multi-token vs chained B={B} H={H} HV={HV} T={T}")
    t = _dev(make_inputs(B, H, HV, seed=5100 + T, T=T), hip_device)
    out, st = gdn.run(**t, use_qk_l2norm=True)
    state = t["state"].clone()
    outs = []
    for tok in range(T):
        sl = slice(tok, tok + 1)
        o = torch.empty(B, 1, HV, 128, dtype=torch.bfloat16, device=hip_device)
        gdn.kernel_hip(q=t["q"][:, sl].contiguous(), k=t["k"][:, sl].contiguous(),
                       v=t["v"][:, sl].contiguous(), state=state, A_log=t["A_log"],
                       a=t["a"][:, sl].contiguous(), dt_bias=t["dt_bias"],
                       b=t["b"][:, sl].contiguous(), scale=t["scale"], output=o,
                       new_state=state, use_qk_l2norm=True)
        outs.append(o)
    torch.cuda.synchronize()
    chained = torch.cat(outs, dim=1).float()
    d_out = (chained - out.float()).abs()
    assert bool((d_out <= 2.0 ** -7 * out.float().abs() + 1e-6).all()), d_out.max()
    d_st = (state - st).abs()
    assert bool((d_st <= 1e-5 * st.abs() + 1e-6).all()), d_st.max()


@pytest.mark.parametrize("A_log_value,T", [(4.0, 8), (60.0, 5)])
def test_multi_token_extreme_decay(A_log_value, T, hip_device):
    """Decays far below the lazy loop's limit (2^-40 accumulated): with
    exp(A_log) = e^4 a token's decay is ~e^-40 .. e^-1, so the decay owed
    passes the limit within a token or two and is folded into the state;
    with e^60 every decay underflows to 0 in fp32 (g = 0: the state
    restarts from the token's own update).  Against the oracle."""
    _announce(f"multi-token extreme decay A_log={A_log_value} T={T}")
    t = make_inputs(4, 16, 32, seed=5150 + T, T=T)
    t["A_log"] = torch.full_like(t["A_log"], A_log_value)
    out, new_state = gdn.run(**_dev(t, hip_device), use_qk_l2norm=True)
    torch.cuda.synchronize()
    ref_o, ref_s, o64, s64 = _oracle(t, True, torch.float32)
    assert_output_close(out.cpu(), ref_o, tight_ref64=o64, what="output")
    assert_state_close(new_state.cpu(), ref_s)
    assert bool(torch.isfinite(new_state).all())


@pytest.mark.parametrize("B,H,HV,T,l2", [
    (1, 16, 32, 1, True), (8, 16, 32, 1, True), (4, 16, 32, 4, True), (64, 16, 32, 1, True),
    (16, 4, 8, 2, False),
])
def test_bf16_state(B, H, HV, T, l2, hip_device):
    _announce(f"bf16 state B={B} H={H} HV={HV} T={T} l2={l2}")
    t = make_inputs(B, H, HV, seed=5200 + B + T, T=T)
    t["state"] = t["state"].to(torch.bfloat16)
    out, new_state = gdn.run(**_dev(t, hip_device), use_qk_l2norm=l2)
    torch.cuda.synchronize()
    assert new_state.dtype == torch.bfloat16
    ref_o, ref_s, o64, s64 = _oracle(t, l2, torch.bfloat16)
    assert_output_close(out.cpu(), ref_o, tight_ref64=o64, what="output")
    _check_bf16_state(new_state, ref_s, s64, "bf16 state")


def test_bf16_state_in_place_and_none(hip_device):
    _announce("bf16 state in place / None")
    t = _dev(make_inputs(4, 16, 32, seed=5300, T=2), hip_device)
    t["state"] = t["state"].to(torch.bfloat16)
    ref_o, ref_s = gdn.run(**t, use_qk_l2norm=True)
    state = t["state"].clone()
    out = torch.empty_like(ref_o)
    gdn.kernel_hip(**{**t, "state": state}, output=out, new_state=state, use_qk_l2norm=True)
    torch.cuda.synchronize()
    assert torch.equal(out, ref_o) and torch.equal(state, ref_s)
    zero = torch.full_like(state, float("nan"))
    gdn.kernel_hip(**{**t, "state": None}, output=out, new_state=zero, use_qk_l2norm=True)
    out2, st2 = gdn.run(**{**t, "state": torch.zeros_like(state)}, use_qk_l2norm=True)
    torch.cuda.synchronize()
    assert torch.equal(out, out2) and torch.equal(zero, st2)


@pytest.mark.parametrize("T,bf16", [(3, False), (1, True), (2, True)])
def test_launch_shapes_agree_bitwise(T, bf16, hip_device):
    _announce(f"launch shapes T={T} bf16={bf16}")
    t = _dev(make_inputs(2, 16, 32, seed=5400 + T, T=T), hip_device)
    if bf16:
        t["state"] = t["state"].to(torch.bfloat16)
    ref_o, ref_s = gdn.run(**t, use_qk_l2norm=True)
    for ns, w, pol in itertools.product((1, 2, 4, 8), (1, 2, 4, 8), (0, 1)):
        if ns * w > 32:
            continue
        out, st = torch.empty_like(ref_o), torch.empty_like(ref_s)
        gdn.kernel_hip_shaped(**t, output=out, new_state=st, use_qk_l2norm=True,
                              rows_per_lane_group=ns, waves_per_block=w, cache_policy=pol)
        torch.cuda.synchronize()
        assert torch.equal(out, ref_o), (ns, w, pol)
        assert torch.equal(st, ref_s), (ns, w, pol)
    out, st = torch.empty_like(ref_o), torch.empty_like(ref_s)
    with pytest.raises(RuntimeError):   # split cache policies: single-token fp32 only
        gdn.kernel_hip_shaped(**t, output=out, new_state=st, rows_per_lane_group=2,
                              waves_per_block=1, cache_policy=2)


def test_multi_token_full_size(hip_device):
    """B=256 qk16_v32, T=2, L2-norm: the largest shape, against the oracle."""
    _announce("multi-token B=256 T=2")
    t = make_inputs(256, 16, 32, seed=5500, T=2)
    out, new_state = gdn.run(**_dev(t, hip_device), use_qk_l2norm=True)
    torch.cuda.synchronize()
    ref_o, ref_s = oracle_tokens(oracle_vec, **t, use_qk_l2norm=True)
    assert_output_close(out.cpu(), ref_o)
    assert_state_close(new_state.cpu(), ref_s)


@pytest.mark.parametrize("B,H,HV,T", [
    (129, 4, 8, 1),     # power-of-two grid sizes, a last run of 4 groups (shift path)
    (130, 3, 9, 1),     # GVA ratio 3 (division path), a last run of 6 groups
    (128, 5, 15, 2),    # multi-token loop, division path, whole runs
    (200, 3, 6, 4),     # T = 4 on the block kernel (1200 heads), division path
])
def test_xcd_grouped_launches(B, H, HV, T, hip_device):
    """Launches of 128 or more sequences with an fp32 state renumber their
    workgroups so that one sequence's share an XCD.  Against the oracle, and
    bitwise against the same batch as two launches of fewer than 128
    sequences (plain order: the per-head arithmetic does not depend on the
    mapping)."""
    _announce(f"xcd-grouped B={B} H={H} HV={HV} T={T}")
    t = make_inputs(B, H, HV, seed=5700 + B + T, T=T)
    td = _dev(t, hip_device)
    out, new_state = gdn.run(**td, use_qk_l2norm=True)
    torch.cuda.synchronize()
    ref_o, ref_s, o64, s64 = _oracle(t, True, torch.float32)
    assert_output_close(out.cpu(), ref_o, tight_ref64=o64, what="output")
    assert_state_close(new_state.cpu(), ref_s)
    half = B // 2
    parts = []
    for lo, hi in ((0, half), (half, B)):
        sl = {n: (x[lo:hi] if isinstance(x, torch.Tensor) and n not in ("A_log", "dt_bias")
                  else x) for n, x in td.items()}
        parts.append(gdn.run(**sl, use_qk_l2norm=True))
    torch.cuda.synchronize()
    assert torch.equal(out, torch.cat([p[0] for p in parts]))
    assert torch.equal(new_state, torch.cat([p[1] for p in parts]))
