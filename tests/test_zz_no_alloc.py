"""gdn_prefill_noalloc: the prefill on the library's fixed per-GPU workspace,
called through the C ABI, against gdn_prefill with a caller workspace (needs
a HIP device).  Calls in a row, each smaller than the one before, each
bitwise equal to the workspace entry's result (the same kernels on the same
workspace layout): the segmented path (its segment blocks in the fixed
array), the chunk-offsets scan, slots found in the kernels, one sequence and
the token path all run on the shared array; and the entry captured in a HIP
graph replays bitwise equal to the workspace entry on new inputs."""

from __future__ import annotations

import ctypes
import sys

import pytest
import torch

import flashinfer_competition_codebase_amd as gdn
from flashinfer_competition_codebase_amd import _lib
from oracle.gdn_prefill_oracle import make_prefill_inputs

pytestmark = pytest.mark.gpu


def _announce(case):
    sys.stdout.write(f"[gpu case] {case}\n")
    sys.stdout.flush()


def _noalloc_c_abi(t, out, st, l2=False):
    """One gdn_prefill_noalloc call through ctypes on torch's current stream."""
    lib = _lib.get_prefill_lib()
    L, H = t["q"].shape[0], t["q"].shape[1]
    HV, N = t["v"].shape[1], t["cu_seqlens"].numel() - 1
    ptr = lambda x: None if x is None else x.data_ptr()  # noqa: E731
    return lib.gdn_prefill_noalloc(
        ptr(t["q"]), ptr(t["k"]), ptr(t["v"]), ptr(t["state"]), ptr(t["A_log"]), ptr(t["a"]),
        ptr(t["dt_bias"]), ptr(t["b"]), ptr(t["cu_seqlens"]), ctypes.c_float(t["scale"]),
        ptr(out), ptr(st), L, N, H, HV, 128, 128, int(l2),
        torch.cuda.current_stream().cuda_stream)


def _dev(t, device):
    return {n: (x.to(device) if isinstance(x, torch.Tensor) else x) for n, x in t.items()}


# (sequence lengths, H, HV, l2norm, with a state), each smaller than the one before
CALLS = [
    ([2048], 4, 8, False, True),                            # segments: 4 dispatches
    ([300, 70, 1] + [5] * 62 + [40], 4, 8, False, True),    # 66 sequences: offsets scan
    ([130, 64, 3], 16, 32, True, True),                     # few sequences: slots in the kernels
    ([100], 4, 8, False, False),                            # one sequence, no initial state
    ([20, 7], 4, 8, False, True),                           # 27 tokens: the token path
]


def test_noalloc_matches_the_workspace_entry_call_after_call(hip_device):
    assert gdn.prefill.prefill_dispatches(2048, 1, 8) == 4      # the first call is segmented
    for i, (lens, H, HV, l2, with_state) in enumerate(CALLS):
        _announce(f"noalloc call {i}: {len(lens)} sequences, {sum(lens)} tokens, H={H} HV={HV}")
        t = _dev(make_prefill_inputs(lens, H, HV, seed=300 + i, with_state=with_state),
                 hip_device)
        ref_o, ref_s = torch.empty_like(t["v"]), torch.empty(
            len(lens), HV, 128, 128, device=hip_device)
        gdn.kernel_prefill_hip(**t, output=ref_o, new_state=ref_s, use_qk_l2norm=l2)
        out = torch.full_like(ref_o, float("nan"))
        st = torch.full_like(ref_s, float("nan"))
        assert _noalloc_c_abi(t, out, st, l2) == 0
        torch.cuda.synchronize()
        assert torch.equal(out, ref_o), i
        assert torch.equal(st, ref_s), i


def test_noalloc_python_entry_in_place(hip_device):
    _announce("noalloc python entry, in place")
    t = _dev(make_prefill_inputs([90, 33], 4, 8, seed=310), hip_device)
    ref_o, ref_s = gdn.prefill_run(**t)
    state = t["state"].clone()
    out = torch.empty_like(ref_o)
    gdn.kernel_prefill_hip_noalloc(**{**t, "state": state}, output=out, new_state=state)
    torch.cuda.synchronize()
    assert torch.equal(out, ref_o) and torch.equal(state, ref_s)


def test_noalloc_in_a_captured_graph(hip_device):
    """The allocation-free entry inside torch.cuda.graph (one stream): after
    a warm-up call (the device's first call resolves the array's address),
    the captured segmented prefill is replayed on new q, v and gates written
    into the captured buffers, with eager work and a synchronisation between
    replays, and every replay is bitwise equal to the workspace entry on the
    same inputs."""
    _announce("noalloc captured in a graph: 1 x 2048 tokens (segments), 4 replays")
    lens, H, HV = [2048], 4, 8
    t = _dev(make_prefill_inputs(lens, H, HV, seed=330), hip_device)
    out = torch.empty_like(t["v"])
    st = torch.empty(1, HV, 128, 128, device=hip_device)
    gdn.kernel_prefill_hip_noalloc(**t, output=out, new_state=st)    # warm-up
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gdn.kernel_prefill_hip_noalloc(**t, output=out, new_state=st)
    torch.cuda.synchronize()
    ref_o, ref_s = torch.empty_like(out), torch.empty_like(st)
    for rep in range(4):
        fresh = _dev(make_prefill_inputs(lens, H, HV, seed=340 + rep), hip_device)
        for n in ("q", "v", "a", "b"):
            t[n].copy_(fresh[n])
        out.fill_(float("nan"))
        st.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        scratch = torch.randn(1 << 20, device=hip_device).sum()    # eager work between
        gdn.kernel_prefill_hip(**t, output=ref_o, new_state=ref_s)
        torch.cuda.synchronize()
        assert torch.isfinite(scratch)
        assert torch.equal(out, ref_o), rep
        assert torch.equal(st, ref_s), rep
    del graph


def test_noalloc_rejects_sizes_beyond_its_workspace(hip_device):
    """Sizes whose workspace exceeds the fixed array: the C ABI returns
    hipErrorOutOfMemory before launching anything (outputs untouched) and the
    Python entry raises ValueError naming the limit."""
    _announce("noalloc rejects oversize")
    lens, H, HV = [4096] * 5, 16, 32
    assert gdn.prefill.workspace_bytes(sum(lens), len(lens), H, HV) > \
        gdn.prefill.NOALLOC_SCRATCH_BYTES
    t = _dev(make_prefill_inputs(lens, H, HV, seed=320), hip_device)
    out = torch.zeros_like(t["v"])
    st = torch.zeros(len(lens), HV, 128, 128, device=hip_device)
    assert _noalloc_c_abi(t, out, st) == 2
    torch.cuda.synchronize()
    assert torch.count_nonzero(out) == 0 and torch.count_nonzero(st) == 0
    with pytest.raises(ValueError, match="workspace"):
        gdn.kernel_prefill_hip_noalloc(**t, output=out, new_state=st)
