"""Parity of the gfx950 prefill with the CPU oracle (needs a HIP device).

Bars, per element: output within atol = rtol = 1e-2 of the oracle loop's bf16
output (the contest's criterion, CLAUDE.md:158) and within two bf16 ulps
(2^-7 relative) + 1e-5 of the float64 chunked result; new state within
1e-3 relative + 1e-5 of the float64 result and within 1e-4 in relative
Frobenius norm.  Inputs: unit-norm q/k rows (the model's normalisation; raw
N(0,1) keys make the recurrence grow without bound), seeded on the CPU.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import flashinfer_competition_codebase_amd as gdn
from flashinfer_competition_codebase_amd import _lib
from oracle.gdn_prefill_oracle import make_prefill_inputs, prefill_chunked_fp64, prefill_loop

pytestmark = pytest.mark.gpu


def _announce(case):
    sys.stdout.write(f"[gpu case] {case}\n")
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _library_present():
    _lib.get_prefill_lib()


def _dev(t, device):
    return {n: (x.to(device) if isinstance(x, torch.Tensor) else x) for n, x in t.items()}


def _check(t, out, st, l2=False, loop=True):
    out, st = out.cpu(), st.cpu()
    o64, s64 = prefill_chunked_fp64(**t, use_qk_l2norm=l2)
    of = out.double().numpy()
    assert np.all(np.isfinite(of))
    d64 = np.abs(of - o64)
    assert np.all(d64 <= 2.0 ** -7 * np.abs(o64) + 1e-5), f"output vs fp64: max {d64.max():.3e}"
    if loop:
        ref_o, ref_s = prefill_loop(**t, use_qk_l2norm=l2)
        dl = (out.float() - ref_o.float()).abs()
        assert bool((dl <= 1e-2 + 1e-2 * ref_o.float().abs()).all()), f"output vs loop {dl.max()}"
    sd = st.double().numpy()
    ds = np.abs(sd - s64)
    assert np.all(ds <= 1e-3 * np.abs(s64) + 1e-5), f"state vs fp64: max {ds.max():.3e}"
    rel = np.linalg.norm(sd - s64) / max(np.linalg.norm(s64), 1e-30)
    assert rel <= 1e-4, rel
    return d64.max(), ds.max()


@pytest.mark.parametrize("seqlens,H,HV", [
    ([70] + [1] * 63, 4, 8),          # 64 sequences: chunk slots found in the kernels
    ([70] + [1] * 64, 4, 8),          # 65: the chunk-offsets scan
    ([70] + [1] * 99, 1, 1),          # 100: the offsets scan, then half-state scan workgroups
    ([0, 130, 0, 0, 64, 1, 0], 2, 4), # empty sequences among few
    ([6], 4, 8),                      # the size of the reference's prefill workload 0
    ([1], 4, 8),
    ([64], 4, 8),
    ([65], 4, 8),
    ([5, 70, 1, 0, 33], 4, 8),
    ([130, 3], 2, 2),
    ([100], 1, 4),
    ([200, 129], 16, 32),
    ([90, 17], 2, 6),                 # GVA ratio 3, heads not a multiple of 8
    ([77], 1, 1),                     # one head
    ([40, 64, 3], 3, 12),             # odd q/k head count, ratio 4
    ([66], 8, 64),                    # 64 v-heads
])
def test_prefill_matches_the_oracle(seqlens, H, HV, hip_device):
    _announce(f"prefill seqlens={seqlens} H={H} HV={HV}")
    t = make_prefill_inputs(seqlens, H, HV, seed=100 + sum(seqlens) + H)
    out, st = gdn.prefill_run(**_dev(t, hip_device))
    torch.cuda.synchronize()
    assert out.shape == (sum(seqlens), HV, 128) and st.shape == (len(seqlens), HV, 128, 128)
    _check(t, out, st)


def test_long_sequence_and_many_sequences(hip_device):
    _announce("prefill long + many")
    g = torch.Generator().manual_seed(3)
    lens = [int(x) for x in torch.randint(0, 160, (24,), generator=g)] + [1000]
    t = make_prefill_inputs(lens, 4, 8, seed=11)
    out, st = gdn.prefill_run(**_dev(t, hip_device))
    torch.cuda.synchronize()
    _check(t, out, st, loop=False)


@pytest.mark.parametrize("lens,H,HV,a_log_range,l2", [
    ([16384], 4, 8, None, False),     # the benchmark's prefill workloads, full size
    ([1024] * 16, 4, 8, None, False),
    ([8192], 16, 32, None, False),
    ([512] * 64, 16, 32, None, False),
    ([16384], 4, 8, (1e-3, 1e-2), False),  # slow decay (g ~ 0.993-0.9993): a long memory
    ([512] * 64, 16, 32, None, True),  # with the q/k L2-norm (raw-scale q/k)
    ([1024] * 16, 4, 8, None, True),
])
def test_bench_size_prefills_match_the_fp64_oracle(lens, H, HV, a_log_range, l2, hip_device):
    """The benchmark's prefill workloads at their full sizes against the
    float64 chunked oracle, at the bars of every other prefill test: fp32
    rounding carried through 128-256 chained chunk steps stays inside them.
    With the benchmark's gates (A_log = log U[1, 16]) a token's decay is
    e^-0.5 .. e^-11, so the state forgets within a few tokens; the last case
    draws A_log = log U[1e-3, 1e-2], so the state carries ~1000 tokens of
    history through 256 chunk steps and every step's rounding with it."""
    _announce(f"prefill bench size lens={lens[0]}x{len(lens)} H={H} HV={HV} "
              f"A_log range={a_log_range} l2={l2}")
    t = make_prefill_inputs(lens, H, HV, seed=200 + len(lens) + H, unit_qk=not l2)
    if a_log_range is not None:
        lo, hi = a_log_range
        g = torch.Generator().manual_seed(201)
        t["A_log"] = torch.log(torch.rand(HV, generator=g) * (hi - lo) + lo)
    out, st = gdn.prefill_run(**_dev(t, hip_device), use_qk_l2norm=l2)
    torch.cuda.synchronize()
    do, ds = _check(t, out, st, l2=l2, loop=False)
    _announce(f"  max |out - fp64| {do:.3e}, max |state - fp64| {ds:.3e}")


@pytest.mark.parametrize("lens,H,HV,l2,with_state", [
    ([3072], 4, 8, False, True),      # 48 chunks
    ([5000], 4, 16, False, True),     # 79 chunks: a partial last chunk and last segment
    ([4100], 1, 1, False, True),      # 65 chunks: a one-chunk last segment, one head
    ([3500], 2, 4, True, False),      # L2-norm, no initial state (segment 0 from zeros)
    ([3100], 2, 6, False, True),      # GVA ratio 3
    ([384], 4, 8, False, True),       # 6 chunks: 3 segments of 2, the fewest segmented
    ([1000], 4, 8, True, True),       # 16 chunks, the last one partial, L2-norm
    ([2048], 4, 8, False, False),     # 32 chunks, no initial state
    ([1100], 16, 32, False, True),    # 18 chunks at 32 v-heads
])
def test_segmented_long_sequence(lens, H, HV, l2, with_state, hip_device):
    """One sequence at <= 32 v-heads whose plain scan would leave most CUs
    idle runs in segments of a few chunks scanned at once (each from a zero
    start, with its 128 x 128 transition), combined, and the segments'
    outputs recomputed from their true starts: against the float64 chunked
    oracle at the prefill bars."""
    L = sum(lens)
    assert gdn.prefill.prefill_dispatches(L, 1, HV) == 4
    _announce(f"segmented prefill L={L} H={H} HV={HV} l2={l2} state={with_state}")
    t = make_prefill_inputs(lens, H, HV, seed=400 + L + HV, with_state=with_state,
                            unit_qk=not l2)
    out, st = gdn.prefill_run(**_dev(t, hip_device), use_qk_l2norm=l2)
    torch.cuda.synchronize()
    do, ds = _check(t, out, st, l2=l2, loop=False)
    _announce(f"  max |out - fp64| {do:.3e}, max |state - fp64| {ds:.3e}")


@pytest.mark.parametrize("lens,H,HV,l2,with_state", [
    ([1000, 2000, 600], 4, 8, False, True),            # slots found in the kernels
    ([5000, 4100, 6000, 3900, 5200, 4800, 5500, 4903], 4, 8, False, True),  # offsets kernel
    ([1500, 0, 700, 3000], 4, 8, True, False),         # an empty sequence, L2-norm, no state
    ([3000, 2000], 16, 32, False, True),               # 64 v-heads of work
    ([900, 20, 1300], 2, 2, False, True),              # a one-segment sequence among them
])
def test_segmented_sequences(lens, H, HV, l2, with_state, hip_device):
    """A few sequences whose plain scans would leave most CUs idle: each is
    cut into as many segments as its length needs (the plan is made for the
    mean length; the kernels count each sequence's own), against the float64
    chunked oracle at the prefill bars."""
    L, N = sum(lens), len(lens)
    assert gdn.prefill.prefill_dispatches(L, N, HV) >= 4
    _announce(f"segmented prefill lens={lens} H={H} HV={HV} l2={l2} state={with_state}")
    t = make_prefill_inputs(lens, H, HV, seed=450 + L + HV, with_state=with_state,
                            unit_qk=not l2)
    out, st = gdn.prefill_run(**_dev(t, hip_device), use_qk_l2norm=l2)
    torch.cuda.synchronize()
    do, ds = _check(t, out, st, l2=l2, loop=False)
    _announce(f"  max |out - fp64| {do:.3e}, max |state - fp64| {ds:.3e}")


def test_segmented_in_place_and_timed(hip_device):
    """Segmented path: in place equals out of place bitwise, and the timed
    entry gives the same bits with its events around the three scan-side
    launches."""
    import ctypes
    _announce("segmented prefill in place / timed")
    t = _dev(make_prefill_inputs([3200], 4, 8, seed=410), hip_device)
    ref_o, ref_s = gdn.prefill_run(**t)
    state = t["state"].clone()
    out = torch.empty_like(ref_o)
    gdn.kernel_prefill_hip(**{**t, "state": state}, output=out, new_state=state)
    torch.cuda.synchronize()
    assert torch.equal(out, ref_o) and torch.equal(state, ref_s)
    hip = ctypes.CDLL("libamdhip64.so.7")
    evs = []
    for _ in range(4):
        e = ctypes.c_void_p()
        assert hip.hipEventCreate(ctypes.byref(e)) == 0
        evs.append(e)
    try:
        out2, st2 = torch.empty_like(ref_o), torch.empty_like(ref_s)
        gdn.kernel_prefill_hip_timed(**t, output=out2, new_state=st2, events=evs)
        torch.cuda.synchronize()
        assert torch.equal(out2, ref_o) and torch.equal(st2, ref_s)
        ms = []
        for i in range(3):
            x = ctypes.c_float()
            assert hip.hipEventElapsedTime(ctypes.byref(x), evs[i], evs[i + 1]) == 0
            ms.append(x.value)
        assert ms[1] > 0.0 and ms[2] > 0.0, ms
    finally:
        for e in evs:
            hip.hipEventDestroy(e)


def test_l2norm_and_no_state(hip_device):
    _announce("prefill l2norm, state=None, raw-scale q/k")
    t = make_prefill_inputs([40, 90], 4, 8, seed=12, with_state=False, unit_qk=False)
    out, st = gdn.prefill_run(**_dev(t, hip_device), use_qk_l2norm=True)
    torch.cuda.synchronize()
    _check(t, out, st, l2=True)


@pytest.mark.parametrize("with_state", [True, False])
def test_l2norm_past_the_in_kernel_chunk_slots(with_state, hip_device):
    """65 sequences (the chunk-offsets scan and the plain scan kernel) with
    the L2-norm, whose Q row scales each wave computes for eight rows and
    shares through LDS."""
    _announce(f"prefill l2norm, 65 sequences, state={with_state}")
    t = make_prefill_inputs([70, 129] + [1] * 63, 4, 8, seed=13, with_state=with_state,
                            unit_qk=False)
    out, st = gdn.prefill_run(**_dev(t, hip_device), use_qk_l2norm=True)
    torch.cuda.synchronize()
    _check(t, out, st, l2=True)


def test_in_place_and_dps_forms_agree_bitwise(hip_device):
    _announce("prefill in place / DPS / int64 cu_seqlens")
    t = _dev(make_prefill_inputs([70, 10], 4, 8, seed=13), hip_device)
    ref_o, ref_s = gdn.prefill_run(**t)
    state = t["state"].clone()
    out = torch.empty_like(ref_o)
    gdn.kernel_prefill_hip(**{**t, "state": state, "cu_seqlens": t["cu_seqlens"].long()},
                           output=out, new_state=state)
    torch.cuda.synchronize()
    assert torch.equal(out, ref_o) and torch.equal(state, ref_s)


def test_empty_sequences_get_a_zero_state(hip_device):
    _announce("prefill empty sequences")
    t = make_prefill_inputs([0, 5, 0], 4, 8, seed=14)
    out, st = gdn.prefill_run(**_dev(t, hip_device))
    torch.cuda.synchronize()
    st = st.cpu()
    assert torch.count_nonzero(st[0]) == 0 and torch.count_nonzero(st[2]) == 0
    _check(t, out, st)
    t0 = make_prefill_inputs([0, 0], 4, 8, seed=15)          # no tokens at all
    out0, st0 = gdn.prefill_run(**_dev(t0, hip_device))
    torch.cuda.synchronize()
    assert out0.shape == (0, 8, 128) and torch.count_nonzero(st0) == 0


@pytest.mark.parametrize("cu,L", [([0], 7), ([0, 5], 10), ([0, 30, 70], 100)])
def test_tokens_outside_every_sequence_get_zero_output(cu, L, hip_device):
    """prefill_run's output for tokens that no sequence covers (no sequences
    at all, or tokens past cu_seqlens[N]) is zero, as the reference's
    zero-initialised result; the covered tokens match the oracle."""
    _announce(f"prefill uncovered tokens cu={cu} L={L}")
    N = len(cu) - 1
    lens = [cu[i + 1] - cu[i] for i in range(N)] + [L - cu[-1]]
    t = make_prefill_inputs(lens, 4, 8, seed=61)      # the last "sequence" is uncovered
    t["cu_seqlens"] = torch.tensor(cu, dtype=torch.int32)
    t["state"] = t["state"][:N].contiguous()
    out, st = gdn.prefill_run(**_dev(t, hip_device))
    torch.cuda.synchronize()
    assert out.shape == (L, 8, 128) and st.shape == (N, 8, 128, 128)
    assert torch.count_nonzero(out[cu[-1]:]) == 0
    if N:
        _check(t, out, st)


def test_prefill_equals_chained_decode_steps(hip_device):
    """A sequence's prefill equals its tokens through the decode kernel one by
    one (different algorithms: equal within the output and state bars)."""
    _announce("prefill vs chained decode")
    t = _dev(make_prefill_inputs([90], 4, 8, seed=16), hip_device)
    out, st = gdn.prefill_run(**t)
    state = t["state"].clone()
    outs = []
    for i in range(90):
        o = torch.empty(1, 1, 8, 128, dtype=torch.bfloat16, device=hip_device)
        gdn.kernel_hip(q=t["q"][i].view(1, 1, 4, 128), k=t["k"][i].view(1, 1, 4, 128),
                       v=t["v"][i].view(1, 1, 8, 128), state=state, A_log=t["A_log"],
                       a=t["a"][i].view(1, 1, 8), dt_bias=t["dt_bias"], b=t["b"][i].view(1, 1, 8),
                       scale=t["scale"], output=o, new_state=state)
        outs.append(o.view(8, 128))
    torch.cuda.synchronize()
    dec = torch.stack(outs).float().cpu()
    assert bool(((out.float().cpu() - dec).abs() <= 1e-2 + 1e-2 * dec.abs()).all())
    ds = (st.cpu() - state.cpu()).abs()
    assert bool((ds <= 1e-3 * state.cpu().abs() + 1e-5).all()), ds.max()


def test_more_than_256_sequences(hip_device):
    """Chunk offsets are scanned 256 sequences at a time: 300 short sequences
    (some empty) cross a group boundary."""
    _announce("prefill 300 sequences")
    g = torch.Generator().manual_seed(21)
    lens = [int(x) for x in torch.randint(0, 12, (300,), generator=g)] + [70]
    t = make_prefill_inputs(lens, 4, 8, seed=22)
    out, st = gdn.prefill_run(**_dev(t, hip_device))
    torch.cuda.synchronize()
    _check(t, out, st, loop=False)


def test_many_empty_sequences_past_the_token_paths_grid(hip_device):
    """65600 one-head sequences, all but five empty, 40 tokens in all: few
    enough tokens for the token-by-token path but more sequences than its
    grid holds (65535), so the chunkwise kernels run, with 257 groups of 256
    sequences in the offsets scan.  The five match the oracle; every empty
    sequence gets a zero state."""
    _announce("65600 sequences, 5 of 8 tokens, chunkwise")
    N = 65600
    picks = [0, 255, 256, 65535, N - 1]
    small = make_prefill_inputs([8] * len(picks), 1, 1, seed=77)
    lens = [0] * N
    for i in picks:
        lens[i] = 8
    cu = torch.zeros(N + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens, dtype=torch.int64), 0).to(torch.int32)
    g = torch.Generator(device=hip_device).manual_seed(78)
    state = torch.randn(N, 1, 128, 128, generator=g, device=hip_device) * 0.05
    state[picks] = small["state"].to(hip_device)
    big = {**_dev(small, hip_device), "state": state, "cu_seqlens": cu.to(hip_device)}
    assert gdn.prefill.prefill_dispatches(40, N, 1) == 3
    out, st = gdn.prefill_run(**big)
    sums = st.abs().sum(dim=(1, 2, 3))
    torch.cuda.synchronize()
    nonzero = torch.nonzero(sums).flatten().cpu().tolist()
    assert nonzero == picks
    _check(small, out, st[picks])


@pytest.mark.parametrize("cu,L", [
    ([0, 30, 5, 40, 100], 40),         # decreasing and past L; 40 tokens: the token path
    ([0, 58, 10, 60, 200, 30], 60),    # the same at 60 tokens: the one-chunk kernel
    ([0, 58] + [10, 60, 200, 30] * 20, 60),   # 81 sequences: chunkwise, the chunk-offsets scan
])
def test_malformed_cu_seqlens_stay_in_bounds(cu, L, hip_device):
    """cu_seqlens that decrease or pass L: every kernel clamps each range to
    [0, L] (and to start <= end), so the call completes with finite results;
    the first sequence, a well-formed range, gets the state that a call with
    it alone gives (bitwise: the same arithmetic on every path; past 40 tokens
    the first sequence is longer than the token-path switch, so that alone it
    runs the one-chunk kernel, the chunkwise kernels' arithmetic in one
    launch)."""
    N = len(cu) - 1
    _announce(f"malformed cu_seqlens N={N} L={L}")
    t = make_prefill_inputs([L] + [0] * (N - 1), 4, 8, seed=91)
    t["cu_seqlens"] = torch.tensor(cu, dtype=torch.int32)
    out, st = gdn.prefill_run(**_dev(t, hip_device))
    n0 = min(cu[1], L)
    alone = {**t, "q": t["q"][:n0], "k": t["k"][:n0], "v": t["v"][:n0], "a": t["a"][:n0],
             "b": t["b"][:n0], "state": t["state"][:1],
             "cu_seqlens": torch.tensor([0, n0], dtype=torch.int32)}
    _, st1 = gdn.prefill_run(**_dev(alone, hip_device))
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out.float()).all()) and bool(torch.isfinite(st).all())
    assert torch.equal(st[:1], st1)


def test_malformed_cu_seqlens_on_the_segment_path(hip_device):
    """Overlapping ranges on the segmented path (5 sequences at 8 v-heads):
    the ranges need more segments than the workspace holds for 3000 tokens,
    so every sequence is scanned as one segment; the call completes, every
    state is finite, and the first sequence (a well-formed range) ends in the
    float64 oracle's state of it alone (its output rows are shared with the
    overlapping third range, which writes them too)."""
    cu, L = [0, 1500, 200, 2600, 5000, 3000], 3000
    N = len(cu) - 1
    assert gdn.prefill.prefill_dispatches(L, N, 8) >= 4
    _announce(f"malformed cu_seqlens on the segment path N={N} L={L}")
    t = make_prefill_inputs([L] + [0] * (N - 1), 4, 8, seed=92)
    t["cu_seqlens"] = torch.tensor(cu, dtype=torch.int32)
    out, st = gdn.prefill_run(**_dev(t, hip_device))
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out.float()).all()) and bool(torch.isfinite(st).all())
    n0 = cu[1]
    alone = {**t, "q": t["q"][:n0], "k": t["k"][:n0], "v": t["v"][:n0], "a": t["a"][:n0],
             "b": t["b"][:n0], "state": t["state"][:1],
             "cu_seqlens": torch.tensor([0, n0], dtype=torch.int32)}
    _, s64 = prefill_chunked_fp64(**alone)
    sd = st[:1].cpu().double().numpy()
    ds = np.abs(sd - s64)
    assert np.all(ds <= 1e-3 * np.abs(s64) + 1e-5), f"state vs fp64: max {ds.max():.3e}"


def test_timed_entry_matches_and_times_each_kernel(hip_device):
    """gdn_prefill_timed: the same results as gdn_prefill, and its four events
    bracket the three launches (each interval non-negative, the scan's
    positive)."""
    import ctypes
    _announce("prefill timed entry")
    hip = ctypes.CDLL("libamdhip64.so.7")
    evs = []
    for _ in range(4):
        e = ctypes.c_void_p()
        assert hip.hipEventCreate(ctypes.byref(e)) == 0
        evs.append(e)
    try:
        t = _dev(make_prefill_inputs([70, 10], 4, 8, seed=23), hip_device)
        ref_o, ref_s = gdn.prefill_run(**t)
        out, st = torch.empty_like(ref_o), torch.empty_like(ref_s)
        gdn.kernel_prefill_hip_timed(**t, output=out, new_state=st, events=evs)
        torch.cuda.synchronize()
        assert torch.equal(out, ref_o) and torch.equal(st, ref_s)
        ms = []
        for i in range(3):
            x = ctypes.c_float()
            assert hip.hipEventElapsedTime(ctypes.byref(x), evs[i], evs[i + 1]) == 0
            ms.append(x.value)
        assert all(m >= 0.0 for m in ms) and ms[2] > 0.0, ms
    finally:
        for e in evs:
            hip.hipEventDestroy(e)


def test_two_thousand_short_sequences(hip_device):
    """2000 sequences of 1..8 tokens: eight groups of the offsets scan, one
    partial chunk each."""
    _announce("prefill 2000 short sequences")
    g = torch.Generator().manual_seed(31)
    lens = [int(x) for x in torch.randint(1, 9, (2000,), generator=g)]
    t = make_prefill_inputs(lens, 4, 8, seed=32)
    out, st = gdn.prefill_run(**_dev(t, hip_device))
    torch.cuda.synchronize()
    _check(t, out, st, loop=False)


def _device_prefill_inputs(lens, H, HV, device, seed):
    """Benchmark-style inputs generated on the device (unit-norm q/k rows)."""
    L, N = sum(lens), len(lens)
    g = torch.Generator(device=device).manual_seed(seed)
    f = dict(device=device)
    q = torch.randn(L, H, 128, generator=g, **f)
    k = torch.randn(L, H, 128, generator=g, **f)
    cu = torch.zeros(N + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens), 0)
    return dict(q=(q / q.norm(dim=-1, keepdim=True)).to(torch.bfloat16),
                k=(k / k.norm(dim=-1, keepdim=True)).to(torch.bfloat16),
                v=torch.randn(L, HV, 128, generator=g, **f).to(torch.bfloat16),
                state=torch.randn(N, HV, 128, 128, generator=g, **f).mul_(0.05),
                A_log=torch.log(torch.rand(HV, generator=g, **f) * 15.0 + 1.0),
                a=torch.randn(L, HV, generator=g, **f).to(torch.bfloat16),
                dt_bias=torch.rand(HV, generator=g, **f) * 2.0 - 1.0,
                b=torch.randn(L, HV, generator=g, **f).to(torch.bfloat16),
                cu_seqlens=cu.to(device), scale=None)


@pytest.mark.parametrize("lens,H,HV,cut", [
    ([1024] * 16, 16, 32, 389),       # 16 x 1024 at qk16_v32, cut off the chunk grid
    ([512] * 64, 16, 32, 200),        # the 64 x 512 qk16_v32 bench workload
    ([16384], 4, 8, 8000),            # the 1 x 16384 qk4_v8 bench workload
])
def test_split_sequences_compose_at_full_size(lens, H, HV, cut, hip_device):
    """Size-independent property of the recurrence: prefilling every sequence
    in two parts, the second starting from the first part's state, gives the
    one-shot prefill.  The parts put chunk boundaries elsewhere, so the two
    runs round differently; they must agree to the bars each meets against
    the float64 oracle: outputs within 2 bf16 ulps + 1e-5, states within
    1e-3 relative + 1e-5 per element and 1e-4 in relative Frobenius norm."""
    _announce(f"prefill split property lens={lens[0]}x{len(lens)} H={H} HV={HV} cut={cut}")
    t = _device_prefill_inputs(lens, H, HV, hip_device, seed=41)
    out, st = gdn.prefill_run(**t)
    cu = t["cu_seqlens"].cpu().tolist()
    seqs = range(len(lens))
    idx1 = torch.cat([torch.arange(cu[s], cu[s] + cut) for s in seqs]).to(hip_device)
    idx2 = torch.cat([torch.arange(cu[s] + cut, cu[s + 1]) for s in seqs]).to(hip_device)

    def part(idx, n_tok, state):
        cu_p = torch.arange(0, n_tok * len(lens) + 1, n_tok, dtype=torch.int32, device=hip_device)
        return gdn.prefill_run(q=t["q"][idx], k=t["k"][idx], v=t["v"][idx], state=state,
                               A_log=t["A_log"], a=t["a"][idx], dt_bias=t["dt_bias"],
                               b=t["b"][idx], cu_seqlens=cu_p, scale=None)

    o1, s1 = part(idx1, cut, t["state"])
    o2, s2 = part(idx2, lens[0] - cut, s1)
    torch.cuda.synchronize()
    split_out = torch.empty_like(out)
    split_out[idx1] = o1
    split_out[idx2] = o2
    ref = out.float()
    d_out = (split_out.float() - ref).abs()
    assert bool((d_out <= 2.0 ** -7 * ref.abs() + 1e-5).all()), d_out.max()
    d_st = (s2 - st).abs()
    assert bool((d_st <= 1e-3 * st.abs() + 1e-5).all()), d_st.max()
    rel = (torch.linalg.vector_norm(s2 - st) / torch.linalg.vector_norm(st)).item()
    assert rel <= 1e-4, rel


# --- prefills of at most 56 tokens: the decode kernel's variable-length mode ----

@pytest.mark.parametrize("seqlens,H,HV,l2,with_state", [
    ([56], 4, 8, False, True),            # the largest token-by-token prefill
    ([48], 4, 8, False, True),
    ([16], 4, 8, False, True),
    ([47, 1], 16, 32, True, True),        # 47 tokens: not a multiple of the 3-token loop body
    ([12] * 4, 4, 8, False, True),
    ([5, 0, 11], 4, 8, False, True),      # an empty sequence among them
    ([1] * 16, 4, 8, False, True),        # sixteen one-token sequences
    ([3, 9], 2, 8, True, True),           # GVA ratio 4, q/k L2-norm
    ([8, 8], 16, 32, False, False),       # qk16_v32, no initial state
    ([6], 1, 1, False, True),             # one head
])
def test_small_prefill_token_path(seqlens, H, HV, l2, with_state, hip_device):
    _announce(f"small prefill seqlens={seqlens} H={H} HV={HV} l2={l2} state={with_state}")
    t = make_prefill_inputs(seqlens, H, HV, seed=40 + sum(seqlens) + H, with_state=with_state)
    out, st = gdn.prefill_run(**_dev(t, hip_device), use_qk_l2norm=l2)
    torch.cuda.synchronize()
    assert out.shape == (sum(seqlens), HV, 128) and st.shape == (len(seqlens), HV, 128, 128)
    _check(t, out, st, l2=l2)


def test_small_and_chunkwise_paths_agree(hip_device):
    """The largest token-by-token prefill (one sequence of as many tokens as
    the path takes) and the same sequence followed by a 1-token one (one
    token more in all: chunkwise) agree within the output and state bars."""
    _announce("small prefill vs chunkwise")
    n = gdn.prefill.token_path_max_tokens()
    t = make_prefill_inputs([n, 1], 4, 8, seed=51)
    out_c, st_c = gdn.prefill_run(**_dev(t, hip_device))
    t_tok = {**t, "q": t["q"][:n], "k": t["k"][:n], "v": t["v"][:n], "a": t["a"][:n],
             "b": t["b"][:n], "state": t["state"][:1], "cu_seqlens": t["cu_seqlens"][:2]}
    out_t, st_t = gdn.prefill_run(**_dev(t_tok, hip_device))
    torch.cuda.synchronize()
    o_t, o_c = out_t.float().cpu(), out_c[:n].float().cpu()
    assert bool(((o_t - o_c).abs() <= 2.0 ** -7 * o_c.abs() + 1e-5).all())
    s_t, s_c = st_t.cpu(), st_c[:1].cpu()
    assert bool(((s_t - s_c).abs() <= 1e-3 * s_c.abs() + 1e-5).all())


def test_small_prefill_in_place_and_timed(hip_device):
    """Token path: in place equals out of place bitwise; the timed entry's
    first two intervals are empty steps and the third the one launch."""
    import ctypes
    _announce("small prefill in place / timed")
    t = _dev(make_prefill_inputs([7, 4], 4, 8, seed=52), hip_device)
    ref_o, ref_s = gdn.prefill_run(**t)
    state = t["state"].clone()
    out = torch.empty_like(ref_o)
    gdn.kernel_prefill_hip(**{**t, "state": state}, output=out, new_state=state)
    torch.cuda.synchronize()
    assert torch.equal(out, ref_o) and torch.equal(state, ref_s)
    hip = ctypes.CDLL("libamdhip64.so.7")
    evs = []
    for _ in range(4):
        e = ctypes.c_void_p()
        assert hip.hipEventCreate(ctypes.byref(e)) == 0
        evs.append(e)
    try:
        out2, st2 = torch.empty_like(ref_o), torch.empty_like(ref_s)
        gdn.kernel_prefill_hip_timed(**t, output=out2, new_state=st2, events=evs)
        torch.cuda.synchronize()
        assert torch.equal(out2, ref_o) and torch.equal(st2, ref_s)
        ms = []
        for i in range(3):
            x = ctypes.c_float()
            assert hip.hipEventElapsedTime(ctypes.byref(x), evs[i], evs[i + 1]) == 0
            ms.append(x.value)
        assert all(m >= 0.0 for m in ms) and ms[2] > 0.0, ms
    finally:
        for e in evs:
            hip.hipEventDestroy(e)


@pytest.mark.parametrize("seqlens,H,HV,l2", [
    ([20] * 4, 4, 8, False),          # 80 tokens: all short, the token kernel runs
    ([5] * 64, 4, 8, False),          # 64 sequences, all short
    ([56, 56], 16, 32, True),         # exactly at the limit: token kernel
    ([57, 50], 4, 8, False),          # one sequence past the limit: the chunkwise kernels
    ([150] + [3] * 10, 2, 6, False),  # one long among short ones: chunkwise
    ([0, 30, 0, 40], 4, 8, True),     # empty sequences among short ones
])
def test_batches_that_may_all_be_short(seqlens, H, HV, l2, hip_device):
    """Batches of 2..64 sequences of at most 56 tokens on average: the token
    kernel is launched first and runs only if every sequence has at most 56
    tokens (read from cu_seqlens on the device), the chunkwise kernels after
    it return at once then and run the whole batch otherwise; either way
    every output row and state matches the oracle."""
    L, N = sum(seqlens), len(seqlens)
    assert L > gdn.prefill.token_path_max_tokens()
    assert gdn.prefill.prefill_dispatches(L, N, HV) >= 3
    _announce(f"may-all-be-short batch seqlens={seqlens[:6]}.. N={N} H={H} HV={HV} l2={l2}")
    t = make_prefill_inputs(seqlens, H, HV, seed=600 + L + N)
    out = torch.full((L, HV, 128), float("nan"), dtype=torch.bfloat16, device=hip_device)
    st = torch.full((N, HV, 128, 128), float("nan"), device=hip_device)
    gdn.kernel_prefill_hip(**_dev(t, hip_device), output=out, new_state=st, use_qk_l2norm=l2)
    torch.cuda.synchronize()
    _check(t, out, st, l2=l2)


@pytest.mark.parametrize("cu,n0", [
    ([0, 30, 10, 50, 45, 90], 30),    # clamped lengths 30, 0, 40, 0, 45: the token kernel
    ([0, 60, 10, 70, 65, 90], 60),    # the first is 60 tokens: the chunkwise kernels
])
def test_malformed_cu_seqlens_when_all_may_be_short(cu, n0, hip_device):
    """Decreasing cu_seqlens in a batch that may be all short (every path
    clamps the ranges alike, so exactly one of them writes each result): the
    call completes with finite results, twice the same states (the output
    rows of overlapping ranges are written by several sequences, in no fixed
    order), and the first, well-formed sequence gets the state it gets alone
    (alone: the token kernel at 30 tokens, as in the batch; the one-chunk
    kernel at 60, which runs the chunkwise kernels' arithmetic, bit for
    bit)."""
    L = 90
    N = len(cu) - 1
    assert gdn.prefill.prefill_dispatches(L, N, 8) >= 3
    _announce(f"malformed cu_seqlens, may-all-be-short batch N={N} L={L}")
    t = make_prefill_inputs([L] + [0] * (N - 1), 4, 8, seed=93)
    t["cu_seqlens"] = torch.tensor(cu, dtype=torch.int32)
    d = _dev(t, hip_device)
    runs = []
    for _ in range(2):
        out = torch.zeros(L, 8, 128, dtype=torch.bfloat16, device=hip_device)
        st = torch.full((N, 8, 128, 128), float("nan"), device=hip_device)
        gdn.kernel_prefill_hip(**d, output=out, new_state=st)
        torch.cuda.synchronize()
        runs.append((out, st))
    out, st = runs[0]
    assert bool(torch.isfinite(out.float()).all()) and bool(torch.isfinite(st).all())
    assert bool(torch.isfinite(runs[1][0].float()).all()) and torch.equal(runs[1][1], st)
    alone = {**t, "q": t["q"][:n0], "k": t["k"][:n0], "v": t["v"][:n0], "a": t["a"][:n0],
             "b": t["b"][:n0], "state": t["state"][:1],
             "cu_seqlens": torch.tensor([0, n0], dtype=torch.int32)}
    _, st1 = gdn.prefill_run(**_dev(alone, hip_device))
    torch.cuda.synchronize()
    assert torch.equal(st[:1], st1)


@pytest.mark.parametrize("seqlens,H,HV,l2,with_state", [
    ([64], 4, 8, False, True),            # one full chunk
    ([57], 16, 32, True, True),           # just past the token path, qk16_v32, L2-norm
    ([60], 1, 1, False, False),           # one head, no initial state
    ([30, 30], 4, 8, False, True),
    ([0, 64, 0], 2, 4, True, True),       # empty sequences around a full chunk
    ([16] * 4, 16, 32, False, True),      # 4 x 32 = 128 (sequence, v-head) pairs: the most
    ([8] * 8, 4, 8, True, False),
    ([1, 63], 3, 12, False, True),        # GVA ratio 4, a one-token sequence
])
def test_one_chunk_kernel(seqlens, H, HV, l2, with_state, hip_device):
    """Prefills of 57..64 tokens in all (so every sequence is one chunk) with
    at most 128 (sequence, v-head) pairs: one launch of the one-chunk kernel,
    in which each workgroup prepares its chunk in LDS and scans it.  Against
    the oracle; in place equal to out of place bitwise; the timed entry's
    third interval is the launch."""
    import ctypes
    L, N = sum(seqlens), len(seqlens)
    assert L > gdn.prefill.token_path_max_tokens()
    assert gdn.prefill.prefill_dispatches(L, N, HV) == 1
    _announce(f"one-chunk kernel seqlens={seqlens} H={H} HV={HV} l2={l2} state={with_state}")
    t = make_prefill_inputs(seqlens, H, HV, seed=700 + L + N + H, with_state=with_state)
    td = _dev(t, hip_device)
    out, st = gdn.prefill_run(**td, use_qk_l2norm=l2)
    torch.cuda.synchronize()
    _check(t, out, st, l2=l2)
    if with_state:
        state = td["state"].clone()
        out2 = torch.empty_like(out)
        gdn.kernel_prefill_hip(**{**td, "state": state}, output=out2, new_state=state,
                               use_qk_l2norm=l2)
        torch.cuda.synchronize()
        assert torch.equal(out2, out) and torch.equal(state, st)
    hip = ctypes.CDLL("libamdhip64.so.7")
    evs = []
    for _ in range(4):
        e = ctypes.c_void_p()
        assert hip.hipEventCreate(ctypes.byref(e)) == 0
        evs.append(e)
    try:
        out3, st3 = torch.empty_like(out), torch.empty_like(st)
        gdn.kernel_prefill_hip_timed(**td, output=out3, new_state=st3, events=evs,
                                     use_qk_l2norm=l2)
        torch.cuda.synchronize()
        assert torch.equal(out3, out) and torch.equal(st3, st)
        x = ctypes.c_float()
        assert hip.hipEventElapsedTime(ctypes.byref(x), evs[2], evs[3]) == 0 and x.value > 0.0
    finally:
        for e in evs:
            hip.hipEventDestroy(e)


@pytest.mark.parametrize("l2", [False, True])
def test_one_chunk_kernel_matches_the_chunkwise_kernels_bitwise(l2, hip_device):
    """A 64-token sequence alone (the one-chunk kernel) and first in a batch
    of 64 + 65 tokens (the preparation kernel, one v-head a workgroup, and
    the half-state scan): the same bits, since the one-chunk kernel runs
    those kernels' arithmetic with the slot kept in LDS."""
    _announce(f"one-chunk kernel vs chunkwise kernels, bitwise, l2={l2}")
    t = make_prefill_inputs([64, 65], 4, 8, seed=71)
    assert gdn.prefill.prefill_dispatches(129, 2, 8) == 2
    assert gdn.prefill.prefill_dispatches(64, 1, 8) == 1
    out_c, st_c = gdn.prefill_run(**_dev(t, hip_device), use_qk_l2norm=l2)
    alone = {**t, "q": t["q"][:64], "k": t["k"][:64], "v": t["v"][:64], "a": t["a"][:64],
             "b": t["b"][:64], "state": t["state"][:1],
             "cu_seqlens": torch.tensor([0, 64], dtype=torch.int32)}
    out_1, st_1 = gdn.prefill_run(**_dev(alone, hip_device), use_qk_l2norm=l2)
    torch.cuda.synchronize()
    assert torch.equal(out_1, out_c[:64]) and torch.equal(st_1, st_c[:1])
