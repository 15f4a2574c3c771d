"""The block decode kernel (T = 2..4 tokens applied as one block on the matrix
cores) on MI355X, against the oracle.

Every dot product of the block is taken against the state at the start of
the step and the tokens' effects on each other are a triangular recurrence
per state row; the oracle applies the reference's per-token recurrence
(solution/triton/prefill_kernel.py:144-178) token after token.  Bars as in
test_gpu_tokens.py: outputs within 1e-2 atol/rtol of the oracle's bf16
output and one bf16 ulp of float64; fp32 states within 1e-3 relative +
1e-5 (and 1e-4 absolute of float64); bf16 states within one bf16 ulp of the
oracle's bf16 state and half an ulp + 1e-6 of float64.
"""

from __future__ import annotations

import sys

import pytest
import torch

import flashinfer_competition_codebase_amd as gdn
from flashinfer_competition_codebase_amd import _lib
from oracle.gdn_decode_oracle import make_inputs, oracle_loop, oracle_tokens, oracle_vec
from tests.gdn_cases import assert_output_close, assert_state_close

pytestmark = pytest.mark.gpu

# (rows per wave, waves per block) of the block kernel: 16-row tiles, at most
# 128 rows (one head) per block.
BLOCK_SHAPES = [(16, 1), (16, 2), (16, 4), (16, 8), (32, 1), (32, 2), (32, 4), (64, 1), (64, 2)]


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


def _check_state(st, ref_s, s64, bf16, what):
    if bf16:
        st = st.cpu().double()
        ref = ref_s.double()
        d_ref = (st - ref).abs()
        assert bool((d_ref <= 2.0 ** -7 * ref.abs() + 1e-6).all()), f"{what}: beyond one bf16 ulp"
        off = (d_ref > 0).double().mean().item()
        assert off <= 1e-3, f"{what}: {off:.2%} of elements differ from the oracle's bf16 state"
        d64 = (st - s64).abs()
        assert bool((d64 <= 2.0 ** -8 * s64.abs() + 1e-6).all()), f"{what}: not the RNE"
    else:
        assert_state_close(st.cpu(), ref_s, what=what)
        assert (st.cpu().double() - s64).abs().max().item() < 1e-4, what


def _run_shaped(t, l2, rows, waves, state=None, new_state=None):
    B, T, HV = t["v"].shape[0], t["v"].shape[1], t["v"].shape[2]
    out = torch.empty(B, T, HV, 128, dtype=torch.bfloat16, device=t["q"].device)
    st = t["state"] if state is None else state
    if new_state is None:
        dtype = torch.float32 if st is None else st.dtype
        new_state = torch.empty(B, HV, 128, 128, dtype=dtype, device=t["q"].device)
    gdn.kernel_hip_shaped(**{**t, "state": st}, output=out, new_state=new_state,
                          use_qk_l2norm=l2, rows_per_lane_group=rows, waves_per_block=waves,
                          cache_policy=1)
    return out, new_state


@pytest.mark.parametrize("T", [2, 3, 4])
@pytest.mark.parametrize("bf16", [False, True])
def test_every_block_shape(T, bf16, hip_device):
    """All launch shapes of the block kernel at B=3 qk16_v32 with the L2-norm."""
    _announce(f"block shapes T={T} bf16={bf16}")
    t = make_inputs(3, 16, 32, seed=6000 + T, T=T)
    if bf16:
        t["state"] = t["state"].to(torch.bfloat16)
    sd = torch.bfloat16 if bf16 else torch.float32
    ref_o, ref_s, o64, s64 = _oracle(t, True, sd)
    td = _dev(t, hip_device)
    for rows, waves in BLOCK_SHAPES:
        out, st = _run_shaped(td, True, rows, waves)
        torch.cuda.synchronize()
        what = f"rows={rows} waves={waves}"
        assert_output_close(out.cpu(), ref_o, tight_ref64=o64, what=what)
        _check_state(st, ref_s, s64, bf16, what)


@pytest.mark.parametrize("B,H,HV,T,l2,bf16", [
    (4, 4, 8, 4, True, False), (5, 2, 6, 3, True, True), (2, 1, 4, 2, False, False),
    (3, 8, 32, 4, False, True), (2, 3, 12, 4, True, False), (6, 16, 32, 2, True, True),
])
def test_block_heads_and_norms(B, H, HV, T, l2, bf16, hip_device):
    """GVA ratios 1-4, the raw (unnormalised) keys, both state dtypes."""
    _announce(f"block B={B} H={H} HV={HV} T={T} l2={l2} bf16={bf16}")
    t = make_inputs(B, H, HV, seed=6100 + B * 7 + T, T=T)
    if bf16:
        t["state"] = t["state"].to(torch.bfloat16)
    sd = torch.bfloat16 if bf16 else torch.float32
    ref_o, ref_s, o64, s64 = _oracle(t, l2, sd)
    out, st = _run_shaped(_dev(t, hip_device), l2, 32, 2)
    torch.cuda.synchronize()
    assert_output_close(out.cpu(), ref_o, tight_ref64=o64)
    _check_state(st, ref_s, s64, bf16, "new_state")


@pytest.mark.parametrize("bf16", [False, True])
def test_block_null_state_and_in_place(bf16, hip_device):
    """state=None starts from zeros (nothing read); in place equals out of place."""
    _announce(f"block null state / in place bf16={bf16}")
    t = make_inputs(4, 16, 32, seed=6200, T=4)
    if bf16:
        t["state"] = t["state"].to(torch.bfloat16)
    sd = torch.bfloat16 if bf16 else torch.float32
    td = _dev(t, hip_device)
    ref_o, ref_s = _run_shaped(td, True, 32, 2)
    state = td["state"].clone()
    out, st = _run_shaped(td, True, 32, 2, state=state, new_state=state)
    torch.cuda.synchronize()
    assert torch.equal(out, ref_o) and torch.equal(state, ref_s)
    zero = torch.full_like(state, float("nan"))
    t0 = {**t, "state": None}
    out0, st0 = _run_shaped(_dev(t0, hip_device), True, 32, 2, state=None, new_state=zero)
    torch.cuda.synchronize()
    r_o, r_s, o64, s64 = _oracle({**t, "state": torch.zeros_like(t["state"])}, True, sd)
    assert_output_close(out0.cpu(), r_o, tight_ref64=o64)
    _check_state(st0, r_s, s64, bf16, "state=None")


@pytest.mark.parametrize("A_log_value", [4.0, 60.0])
def test_block_extreme_decay(A_log_value, hip_device):
    """exp(A_log) = e^4: decays ~e^-40 .. e^-1 whose products underflow over
    the block; e^60: every decay is 0 in fp32 (each token restarts from its
    own update).  No decay is divided by, so nothing overflows."""
    _announce(f"block extreme decay A_log={A_log_value}")
    t = make_inputs(4, 16, 32, seed=6300, T=4)
    t["A_log"] = torch.full_like(t["A_log"], A_log_value)
    ref_o, ref_s, o64, s64 = _oracle(t, True, torch.float32)
    out, st = _run_shaped(_dev(t, hip_device), True, 32, 2)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(st).all())
    assert_output_close(out.cpu(), ref_o, tight_ref64=o64)
    _check_state(st, ref_s, s64, False, "new_state")


@pytest.mark.parametrize("bf16", [False, True])
def test_block_full_size(bf16, hip_device):
    """B=256 qk16_v32, T=4, L2-norm (the largest multi-token shape)."""
    _announce(f"block B=256 T=4 bf16={bf16}")
    t = make_inputs(256, 16, 32, seed=6400 + bf16, T=4)
    if bf16:
        t["state"] = t["state"].to(torch.bfloat16)
    out, st = _run_shaped(_dev(t, hip_device), True, 32, 2)
    torch.cuda.synchronize()
    sd = torch.bfloat16 if bf16 else torch.float32
    ref_o, ref_s = oracle_tokens(oracle_vec, **t, use_qk_l2norm=True, state_dtype=sd)
    assert_output_close(out.cpu(), ref_o)
    if bf16:
        d = (st.cpu().double() - ref_s.double()).abs()
        assert bool((d <= 2.0 ** -7 * ref_s.double().abs() + 1e-6).all())
        assert (d > 0).double().mean().item() <= 1e-3
    else:
        assert_state_close(st.cpu(), ref_s)


def test_block_rejects_other_token_counts(hip_device):
    """The block kernel takes T = 2..4 and the nontemporal policy only."""
    _announce("block rejects T=1, T=5, policy 0")
    for T in (1, 5):
        td = _dev(make_inputs(2, 16, 32, seed=6500, T=T), hip_device)
        with pytest.raises(RuntimeError):
            _run_shaped(td, True, 32, 2)
    td = _dev(make_inputs(2, 16, 32, seed=6500, T=2), hip_device)
    out = torch.empty(2, 2, 32, 128, dtype=torch.bfloat16, device=hip_device)
    st = torch.empty_like(td["state"])
    with pytest.raises(RuntimeError):
        gdn.kernel_hip_shaped(**td, output=out, new_state=st, rows_per_lane_group=32,
                              waves_per_block=2, cache_policy=0)


@pytest.mark.parametrize("B,T,bf16", [(1, 4, True), (4, 2, True), (16, 4, True), (32, 3, True),
                                      (32, 2, True), (4, 4, False), (8, 4, False), (32, 3, False),
                                      (64, 4, False)])
def test_library_runs_block_kernel(B, T, bf16, hip_device):
    """Shapes at which the library's launch table picks the block kernel, through
    the value-returning entry point, against the oracle."""
    _announce(f"library block choice B={B} T={T} bf16={bf16}")
    ns, _, _, _ = _lib.launch_shape(B, 32, T, bf16)
    assert ns in (16, 32, 64), ns
    t = make_inputs(B, 16, 32, seed=6600 + B + T, T=T)
    if bf16:
        t["state"] = t["state"].to(torch.bfloat16)
    sd = torch.bfloat16 if bf16 else torch.float32
    ref_o, ref_s, o64, s64 = _oracle(t, True, sd)
    out, st = gdn.run(**_dev(t, hip_device), use_qk_l2norm=True)
    torch.cuda.synchronize()
    assert_output_close(out.cpu(), ref_o, tight_ref64=o64)
    _check_state(st, ref_s, s64, bf16, "new_state")
