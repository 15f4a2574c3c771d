"""Parity of the gfx950 decode kernel with the CPU oracle (needs a HIP device).

Every call goes through the package's entry points and so through the C ABI
in ``libgdn_decode.so``.  Bars: bf16 output within
atol = rtol = 1e-2 of the oracle's bf16 output, and within one bf16 ulp of
the float64 result; fp32 new state within 1e-3 relative + 1e-5 absolute of
the oracle (element-wise) and 1e-3 in relative Frobenius norm.  The oracle is
``oracle_loop`` (the loop-for-loop restatement of
solution/triton/kernel.py:72-118) where it finishes in seconds, else its
batched twin ``oracle_vec``.

Set ``GDN_PARITY_LOG=<path>`` to append one JSON line of measured errors per
case.
"""

from __future__ import annotations

import itertools
import json
import math
import os
import sys

import pytest
import torch

import flashinfer_competition_codebase_amd as gdn
from flashinfer_competition_codebase_amd import _lib
from oracle.gdn_decode_oracle import l2norm, make_inputs, oracle_loop, oracle_vec
from tests.gdn_cases import (
    CONFIG_SEEDS, CONFIGS, REF_BATCHES, assert_output_close, assert_state_close,
    load_golden)

pytestmark = pytest.mark.gpu


def _record(case, **metrics):
    path = os.environ.get("GDN_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps({"case": case, **metrics}) + "\n")


def _announce(case):
    sys.stdout.write(f"[gpu case] {case}\n")
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _library_present():
    # No skip: on a device host a missing or broken library is a failure.
    _lib.get_lib()


def _dev(t, device):
    return {n: (x.to(device) if isinstance(x, torch.Tensor) else x) for n, x in t.items()}


def _check_against_oracle(case, t, l2, out, new_state):
    B, HV = t["v"].shape[0], t["v"].shape[2]
    if B * HV <= 256:
        ref_o, ref_s = oracle_loop(**t, use_qk_l2norm=l2)
    else:
        ref_o, ref_s = oracle_vec(**t, use_qk_l2norm=l2)
    o64, s64 = oracle_vec(**t, use_qk_l2norm=l2, output_fp32=True, dtype=torch.float64)
    out_c, st_c = out.cpu(), new_state.cpu()
    assert_output_close(out_c, ref_o, tight_ref64=o64, what=f"{case} output")
    rel = assert_state_close(st_c, ref_s, what=f"{case} new_state")
    d64 = (st_c.double() - s64).abs()
    _record(case,
            out_max_abs_vs_oracle=(out_c.float() - ref_o.float()).abs().max().item(),
            out_max_abs_vs_fp64=(out_c.double() - o64).abs().max().item(),
            state_max_abs_vs_oracle=(st_c - ref_s).abs().max().item(),
            state_rel_fro_vs_oracle=rel,
            state_max_abs_vs_fp64=d64.max().item(),
            state_max_rel_vs_fp64=(d64 / s64.abs().clamp_min(1e-3)).max().item())
    assert d64.max().item() < 1e-4


@pytest.mark.parametrize("name", list(CONFIGS))
def test_benchmark_configs(name, hip_device):
    B, H, HV, l2 = CONFIGS[name]
    _announce(f"{name} B={B} H={H} HV={HV} l2={l2}")
    t = make_inputs(B, H, HV, seed=CONFIG_SEEDS[name])
    td = _dev(t, hip_device)
    out, new_state = gdn.run(**td, use_qk_l2norm=l2)
    torch.cuda.synchronize()
    assert torch.equal(td["state"].cpu(), t["state"]), "run() must not modify state"
    _check_against_oracle(name, t, l2, out, new_state)


@pytest.mark.parametrize("B", REF_BATCHES)
def test_reference_definition_qk4_v8(B, hip_device):
    """The reference's own decode definition (H=4, HV=8, no L2-norm)."""
    _announce(f"qk4_v8 B={B}")
    t = make_inputs(B, 4, 8, seed=2000 + B)
    td = _dev(t, hip_device)
    out = torch.empty(B, 1, 8, 128, dtype=torch.bfloat16, device=hip_device)
    new_state = torch.empty(B, 8, 128, 128, device=hip_device)
    gdn.kernel_hip(**td, output=out, new_state=new_state)
    torch.cuda.synchronize()
    _check_against_oracle(f"qk4_v8_b{B}", t, False, out, new_state)


@pytest.mark.parametrize("name", sorted(load_golden()))
def test_golden_vectors(name, hip_device):
    _announce(f"golden {name}")
    t, l2, exp_out, exp_state = load_golden()[name]
    out, new_state = gdn.run(**_dev(t, hip_device), use_qk_l2norm=l2)
    torch.cuda.synchronize()
    ref_o = torch.from_numpy(exp_out).to(torch.bfloat16)
    assert_output_close(out.cpu(), ref_o, tight_ref64=exp_out, what=name)
    assert_state_close(new_state.cpu(), torch.from_numpy(exp_state), what=name)


@pytest.mark.parametrize("H,HV", [(32, 32), (1, 32), (4, 8), (2, 64), (2, 6), (5, 15)])
def test_gva_ratios(H, HV, hip_device):
    _announce(f"gva H={H} HV={HV}")
    t = make_inputs(3, H, HV, seed=3000 + H + HV)
    out, new_state = gdn.run(**_dev(t, hip_device), use_qk_l2norm=True)
    torch.cuda.synchronize()
    _check_against_oracle(f"gva_{H}_{HV}", t, True, out, new_state)


def test_in_place_matches_out_of_place_bitwise(hip_device):
    _announce("in-place vs out-of-place")
    t = _dev(make_inputs(4, 16, 32, seed=4001), hip_device)
    out1, st1 = gdn.run(**t, use_qk_l2norm=True)
    out2 = torch.empty_like(out1)
    state = t["state"].clone()
    gdn.kernel_hip(**{**t, "state": state}, output=out2, new_state=state,
                   use_qk_l2norm=True)
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)
    assert torch.equal(st1, state)


def test_all_launch_shapes_agree_bitwise(hip_device):
    """Every (rows per lane group, waves per block, cache policy) launch gives
    the same bits: the per-row arithmetic does not depend on the mapping."""
    _announce("launch shapes")
    t = _dev(make_inputs(2, 16, 32, seed=4002), hip_device)
    ref_o, ref_s = gdn.run(**t, use_qk_l2norm=True)
    for ns, w, pol in itertools.product((1, 2, 4, 8), (1, 2, 4, 8), (0, 1, 2, 3)):
        if ns * w > 32:
            continue
        out = torch.empty_like(ref_o)
        st = torch.empty_like(ref_s)
        gdn.kernel_hip_shaped(**t, output=out, new_state=st, use_qk_l2norm=True,
                              rows_per_lane_group=ns, waves_per_block=w, cache_policy=pol)
        torch.cuda.synchronize()
        assert torch.equal(out, ref_o), (ns, w, pol)
        assert torch.equal(st, ref_s), (ns, w, pol)


def test_batch_beyond_one_launch(hip_device):
    """B = 65600 one-head sequences: more than one launch's grid-z limit
    (65535), so the host splits the batch into two launches.  Slices at the
    start, across the split and at the end match separate small calls
    bitwise (the per-row arithmetic does not depend on the launch shape)."""
    _announce("B=65600 qk1_v1, two launches")
    B, H, HV = 65600, 1, 1
    g = torch.Generator(device=hip_device).manual_seed(4100)

    def rn(*shape, scale=1.0, dtype=torch.bfloat16):
        return (torch.randn(*shape, generator=g, device=hip_device) * scale).to(dtype)

    t = dict(q=rn(B, 1, H, 128), k=rn(B, 1, H, 128), v=rn(B, 1, HV, 128),
             state=rn(B, HV, 128, 128, scale=0.05, dtype=torch.float32),
             A_log=torch.log(torch.rand(HV, generator=g, device=hip_device) * 15 + 1),
             a=rn(B, HV), dt_bias=torch.rand(HV, generator=g, device=hip_device) * 2 - 1,
             b=rn(B, HV), scale=None)
    out, st = gdn.run(**t, use_qk_l2norm=True)
    for lo, hi in ((0, 3), (65530, 65540), (B - 3, B)):
        part = {n: (x[lo:hi].contiguous() if n in ("q", "k", "v", "state", "a", "b") else x)
                for n, x in t.items()}
        o2, s2 = gdn.run(**part, use_qk_l2norm=True)
        torch.cuda.synchronize()
        assert torch.equal(out[lo:hi], o2), (lo, hi)
        assert torch.equal(st[lo:hi], s2), (lo, hi)


def test_state_none_is_zero_state(hip_device):
    _announce("state=None")
    t = make_inputs(2, 16, 32, seed=4003)
    td = _dev({**t, "state": None}, hip_device)
    out = torch.empty(2, 1, 32, 128, dtype=torch.bfloat16, device=hip_device)
    new_state = torch.full((2, 32, 128, 128), float("nan"), device=hip_device)
    gdn.kernel_hip(**td, output=out, new_state=new_state, use_qk_l2norm=True)
    torch.cuda.synchronize()
    _check_against_oracle("state_none", {**t, "state": None}, True, out, new_state)


def test_gate_edge_values(hip_device):
    """softplus above its threshold, saturated beta, no decay and full decay."""
    _announce("gate edges")
    t = make_inputs(2, 4, 8, seed=4004)
    t["a"] = torch.tensor([[[30.0, -30.0, 0.0, 19.5, 20.5, -5.0, 2.0, 8.0]],
                           [[0.0] * 8]], dtype=torch.bfloat16)
    t["b"] = torch.tensor([[[40.0, -40.0, float("inf"), float("-inf"), 0.0, 1.0, -1.0, 5.0]],
                           [[0.0] * 8]], dtype=torch.bfloat16)
    t["A_log"] = torch.tensor([0.0, 2.7, float("-inf"), -20.0, 1.0, math.log(16.0), 0.5, 0.0])
    out, new_state = gdn.run(**_dev(t, hip_device), use_qk_l2norm=True)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all() and torch.isfinite(new_state).all()
    _check_against_oracle("gate_edges", t, True, out, new_state)


def test_multi_step_in_place(hip_device):
    """Four chained in-place steps with fresh q, k, v, a, b each step."""
    _announce("multi-step")
    base = make_inputs(2, 16, 32, seed=4005)
    state_dev = base["state"].to(hip_device)
    state_ref = base["state"].clone()
    for step in range(4):
        t = make_inputs(2, 16, 32, seed=4100 + step)
        t["state"] = state_ref
        ref_o, ref_s = oracle_loop(**t, use_qk_l2norm=True)
        td = _dev({**t, "state": None}, hip_device)
        out = torch.empty(2, 1, 32, 128, dtype=torch.bfloat16, device=hip_device)
        gdn.kernel_hip(**{**td, "state": state_dev}, output=out, new_state=state_dev,
                       use_qk_l2norm=True)
        torch.cuda.synchronize()
        assert_output_close(out.cpu(), ref_o, what=f"step {step} output")
        assert_state_close(state_dev.cpu(), ref_s, what=f"step {step} state")
        state_ref = ref_s


def test_runs_on_the_callers_stream(hip_device):
    _announce("non-default stream")
    t = _dev(make_inputs(8, 16, 32, seed=4006), hip_device)
    ref_o, ref_s = gdn.run(**t, use_qk_l2norm=True)
    torch.cuda.synchronize()
    s = torch.cuda.Stream(device=hip_device)
    with torch.cuda.stream(s):
        out, st = gdn.run(**t, use_qk_l2norm=True)
    s.synchronize()
    assert torch.equal(out, ref_o) and torch.equal(st, ref_s)


def test_zero_batch(hip_device):
    t = _dev(make_inputs(0, 16, 32, seed=4007), hip_device)
    out, st = gdn.run(**t, use_qk_l2norm=True)
    assert out.shape == (0, 1, 32, 128) and st.shape == (0, 32, 128, 128)


def test_gate_tensor_shapes_agree(hip_device):
    t = _dev(make_inputs(3, 16, 32, seed=4008), hip_device)
    o1, s1 = gdn.run(**t, use_qk_l2norm=True)
    o2, s2 = gdn.run(**{**t, "a": t["a"].reshape(3, 32), "b": t["b"].reshape(3, 32)},
                     use_qk_l2norm=True)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)


def test_bf16_output_rounds_to_nearest_even(hip_device):
    """g = 1, beta = 0, scale = 1, q = e_0: o_v = state[v, 0] exactly in fp32,
    so the bf16 output must equal torch's RNE cast of the chosen values,
    including exact ties (1 + 2^-8 -> 1, 1 + 3 * 2^-8 -> 1 + 2^-6)."""
    _announce("bf16 rounding")
    vals = torch.tensor([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -(1.0 + 2.0 ** -8),
                         3.0e-3 * (1 + 2.0 ** -9), 65504.0, 1.0e-20, -7.77e5, 0.0])
    t = make_inputs(1, 1, 1, seed=4009)
    state = torch.zeros(1, 1, 128, 128)
    state[0, 0, : vals.numel(), 0] = vals
    state[0, 0, vals.numel():, 0] = torch.randn(128 - vals.numel(),
                                                generator=torch.Generator().manual_seed(5))
    q = torch.zeros(1, 1, 1, 128, dtype=torch.bfloat16)
    q[..., 0] = 1.0
    t.update(state=state, q=q, A_log=torch.tensor([float("-inf")]), scale=1.0,
             b=torch.full((1, 1, 1), float("-inf"), dtype=torch.bfloat16))
    out, new_state = gdn.run(**_dev(t, hip_device))
    torch.cuda.synchronize()
    expect = state[0, 0, :, 0].to(torch.bfloat16)
    got = out.cpu()[0, 0, 0]
    assert torch.equal(got.view(torch.int16), expect.view(torch.int16))
    assert torch.equal(new_state.cpu(), state)


def test_full_size_write_read_property(hip_device):
    """At the largest benchmark shape (B=256, qk16_v32): with beta = 1 and
    q = k the step stores v under k_hat, so S_new k_hat = v and o = scale v."""
    _announce("B=256 write/read property")
    t = make_inputs(256, 16, 32, seed=4010)
    t["k"] = t["q"].clone()
    t["b"] = torch.full_like(t["b"], float("inf"))
    td = _dev(t, hip_device)
    out, new_state = gdn.run(**td, use_qk_l2norm=True)
    k_hat = l2norm(td["k"][:, 0].float()).repeat_interleave(2, 1)      # [B, HV, K]
    read = torch.matmul(new_state, k_hat.unsqueeze(-1)).squeeze(-1)    # fp32
    v = td["v"][:, 0].float()
    torch.cuda.synchronize()
    assert (read - v).abs().max().item() < 1e-4
    o_expect = t["scale"] * v
    err = (out[:, 0].float() - o_expect).abs()
    assert bool((err <= 2.0 ** -8 * o_expect.abs() + 1e-6).all())   # within one bf16 ulp


def test_stamped_launch_matches_and_times(hip_device):
    """Event-stamped launches (hipExtLaunchKernelGGL) give the same bits as
    plain launches and a positive kernel duration."""
    import ctypes

    _announce("stamped launch")
    hip = ctypes.CDLL("libamdhip64.so.7")
    evs = [ctypes.c_void_p(), ctypes.c_void_p()]
    for ev in evs:
        assert hip.hipEventCreate(ctypes.byref(ev)) == 0
    try:
        t = _dev(make_inputs(4, 16, 32, seed=4011), hip_device)
        ref_o, ref_s = gdn.run(**t, use_qk_l2norm=True)
        out, st = torch.empty_like(ref_o), torch.empty_like(ref_s)
        gdn.kernel_hip_shaped(**t, output=out, new_state=st, use_qk_l2norm=True,
                              start_event=evs[0].value, stop_event=evs[1].value)
        assert hip.hipEventSynchronize(evs[1]) == 0
        ms = ctypes.c_float()
        assert hip.hipEventElapsedTime(ctypes.byref(ms), evs[0], evs[1]) == 0
        assert 0.0 < ms.value < 100.0
        assert torch.equal(out, ref_o) and torch.equal(st, ref_s)
    finally:
        for ev in evs:
            hip.hipEventDestroy(ev)


def test_hip_graph_capture_and_replay(hip_device):
    """The decode step captured in a HIP graph (torch.cuda.CUDAGraph on the
    capture stream) replays to the eager result, step after step, with eager
    work and synchronisations between replays."""
    _announce("hip graph capture")
    t = _dev(make_inputs(1, 16, 32, seed=4012), hip_device)
    state_g = t["state"].clone()
    state_e = t["state"].clone()
    out_g = torch.empty(1, 1, 32, 128, dtype=torch.bfloat16, device=hip_device)
    out_e = torch.empty_like(out_g)
    graph = torch.cuda.CUDAGraph()
    warm = torch.cuda.Stream(device=hip_device)
    warm.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(warm):   # warm the library up off the capture
        scratch = state_g.clone()
        gdn.kernel_hip(**{**t, "state": scratch}, output=out_g, new_state=scratch,
                       use_qk_l2norm=True)
    torch.cuda.current_stream().wait_stream(warm)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        gdn.kernel_hip(**{**t, "state": state_g}, output=out_g, new_state=state_g,
                       use_qk_l2norm=True)
    torch.cuda.synchronize()
    assert torch.equal(state_g, t["state"]), "capture must not execute the step"
    for step in range(4):
        graph.replay()
        gdn.kernel_hip(**{**t, "state": state_e}, output=out_e, new_state=state_e,
                       use_qk_l2norm=True)
        torch.cuda.synchronize()
        assert torch.equal(out_g, out_e), step
        assert torch.equal(state_g, state_e), step


@pytest.mark.parametrize("B,H,HV,l2", [(1, 16, 32, True), (1, 4, 8, False), (4, 4, 8, False)])
def test_stamped_instrument_matches_the_kernel(B, H, HV, l2, hip_device):
    """The instrumented single-token kernel (gdn_decode_step_stamped) computes
    the product kernel's bits with the same launch shape, and every
    wavefront's stamps are in order."""
    import ctypes

    _announce(f"stamped instrument B={B} H={H} HV={HV}")
    t = _dev(make_inputs(B, H, HV, seed=4100 + B + H), hip_device)
    ref_o, ref_s = gdn.run(**t, use_qk_l2norm=l2)
    ns, waves, _, blocks = _lib.launch_shape(B, HV)
    n = blocks * waves * 8
    stamps = torch.zeros(n, dtype=torch.int64, device=hip_device)
    out = torch.empty_like(ref_o)
    st = t["state"].clone()
    lib = _lib.get_lib()
    code = lib.gdn_decode_step_stamped(
        t["q"].data_ptr(), t["k"].data_ptr(), t["v"].data_ptr(), st.data_ptr(),
        t["A_log"].data_ptr(), t["a"].data_ptr(), t["dt_bias"].data_ptr(), t["b"].data_ptr(),
        t["scale"], out.data_ptr(), st.data_ptr(), B, H, HV, 128, 128, int(l2), ns, waves,
        ctypes.cast(stamps.data_ptr(), ctypes.POINTER(ctypes.c_ulonglong)), n,
        torch.cuda.current_stream().cuda_stream)
    assert code == 0
    torch.cuda.synchronize()
    assert torch.equal(out, ref_o) and torch.equal(st, ref_s)
    s = stamps.view(-1, 8).cpu()
    assert bool((s[:, 2:7] >= s[:, 1:6]).all()), "shader-clock stamps out of order"
    assert bool((s[:, 7] >= s[:, 0]).all()) and bool((s[:, 1] > 0).all())
    assert lib.gdn_decode_step_stamped(*[None] * 8, 0.1, None, None, B, H, HV, 128, 128, 0,
                                       ns, waves, None, 0, None) == 1
