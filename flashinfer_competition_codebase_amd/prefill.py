"""Python entry points of the GDN prefill, in the reference's calling forms.

Two forms, with the reference's argument names (``fn(**tensors)`` works):

* ``prefill_run(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale)`` --
  value-returning, like ``kernel_prefill_reference``
  (solution/triton/prefill_kernel.py:85-183): returns ``(output, new_state)``
  and leaves ``state`` untouched.
* ``kernel_prefill_hip(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens,
  scale, output, new_state)`` -- destination-passing, like
  ``kernel_prefill_fla_chunk`` (solution/triton/prefill_kernel.py:10-58):
  writes both outputs, returns None.  ``new_state`` may be ``state`` itself.

Both launch the gfx950 prefill of ``libgdn_prefill.so`` (chunk offsets,
per-chunk preparation, sequential scan) on the current HIP stream; there is
no CPU path.  The device workspace for the per-chunk intermediates comes
from torch's caching allocator.

Tensor contract (solution/triton/prefill_kernel.py:96-114): q, k
``[L, H, 128]`` bf16; v ``[L, HV, 128]`` bf16 with ``HV % H == 0``; state
``[N, HV, 128, 128]`` fp32 k-last or None (zeros); A_log, dt_bias ``[HV]``
fp32; a, b ``[L, HV]`` bf16; cu_seqlens ``[N + 1]`` int32 (int64 is
converted) on the same device, non-decreasing from 0 to L; scale float,
0-d tensor, None or 0 (None/0 mean ``1/sqrt(128)``); output ``[L, HV, 128]``
bf16; new_state ``[N, HV, 128, 128]`` fp32.  A sequence with no tokens gets
a zero ``new_state``, as the reference's loop leaves it
(prefill_kernel.py:147-150).  The q/k L2-norm is a keyword-only flag,
off by default as in the reference's prefill (prefill_kernel.py:45).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .kernel import K_DIM, V_DIM, _expect, _on_device, _overlap, _same_hip_device, resolve_scale

__all__ = ["prefill_run", "kernel_prefill_hip", "kernel_prefill_hip_timed",
           "kernel_prefill_hip_noalloc", "workspace_bytes", "token_path_max_tokens",
           "prefill_dispatches", "NOALLOC_SCRATCH_BYTES"]

# Size of the library's fixed per-GPU workspace (GDN_PREFILL_NOALLOC_SCRATCH_BYTES).
NOALLOC_SCRATCH_BYTES = 128 << 20


def workspace_bytes(total_seq_len: int, num_seqs: int, H: int, HV: int) -> int:
    """Device workspace bytes a prefill of this size needs."""
    n = _lib.get_prefill_lib().gdn_prefill_workspace_bytes(int(total_seq_len), int(num_seqs),
                                                          int(H), int(HV))
    if n == 0:
        raise ValueError(f"invalid prefill sizes L={total_seq_len}, N={num_seqs}, H={H}, HV={HV}")
    return n


def token_path_max_tokens() -> int:
    """Total tokens up to which a prefill is one launch of the token-by-token
    kernel instead of the chunkwise kernels."""
    return int(_lib.get_prefill_lib().gdn_prefill_token_path_max_tokens())


def prefill_dispatches(total_seq_len: int, num_seqs: int, HV: int) -> int:
    """Kernel dispatches of one prefill call over HV v-heads, as the library
    makes them (``gdn_prefill_dispatches``): 0 for no sequences, 1 for the
    token-by-token kernel or the one-chunk kernel (57..64 tokens in all, at
    most 128 (sequence, v-head) pairs); else 2 (preparation, scan) or, for a batch scanned
    in segments, 4 (preparation, two segment scans and their combine), plus
    the chunk-offsets scan first unless there is one sequence or at most 64
    with at most 2048 (slot, v-head) pairs, plus the token-by-token kernel
    first for 2..64 sequences of at most 56 tokens on average."""
    return int(_lib.get_prefill_lib().gdn_prefill_dispatches(int(total_seq_len), int(num_seqs),
                                                            int(HV)))


def check_prefill_inputs(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, output=None,
                         new_state=None):
    """Validate the prefill tensors; returns ``(L, N, H, HV)``.  Shape and dtype
    rules are the reference's (prefill_kernel.py:96-129, generalised to any
    ``HV % H == 0``); the device check comes last."""
    if not isinstance(q, torch.Tensor) or q.dim() != 3:
        raise ValueError("q must be a 3-D tensor [L, H, K]")
    if not isinstance(v, torch.Tensor) or v.dim() != 3:
        raise ValueError("v must be a 3-D tensor [L, HV, V]")
    if not isinstance(cu_seqlens, torch.Tensor) or cu_seqlens.dim() != 1 or cu_seqlens.numel() < 1:
        raise ValueError("cu_seqlens must be a 1-D tensor [N + 1]")
    if cu_seqlens.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"cu_seqlens must be int32 or int64, got {cu_seqlens.dtype}")
    L, H, K = q.shape
    HV, V = v.shape[1], v.shape[2]
    N = cu_seqlens.numel() - 1
    if K != K_DIM or V != V_DIM:
        raise ValueError(f"K and V must be {K_DIM}, got K={K}, V={V}")
    if H <= 0 or HV <= 0 or HV % H != 0:
        raise ValueError(f"v-heads must be a multiple of q/k heads, got H={H}, HV={HV}")
    if v.shape[0] != L:
        raise ValueError(f"v must have {L} tokens, got {v.shape[0]}")
    _expect(q, "q", torch.bfloat16, (L, H, K))
    _expect(k, "k", torch.bfloat16, (L, H, K))
    _expect(v, "v", torch.bfloat16, (L, HV, V))
    if state is not None:
        _expect(state, "state", torch.float32, (N, HV, V, K))
    _expect(A_log, "A_log", torch.float32, (HV,))
    _expect(dt_bias, "dt_bias", torch.float32, (HV,))
    _expect(a, "a", torch.bfloat16, (L, HV))
    _expect(b, "b", torch.bfloat16, (L, HV))
    if not cu_seqlens.is_contiguous():
        raise ValueError("cu_seqlens must be contiguous")
    if output is not None:
        _expect(output, "output", torch.bfloat16, (L, HV, V))
    if new_state is not None:
        _expect(new_state, "new_state", torch.float32, (N, HV, V, K))
    _same_hip_device(q, (k, v, A_log, a, dt_bias, b, cu_seqlens, state, output, new_state),
                     "the GDN prefill")
    if state is not None and new_state is not None and new_state is not state:
        if new_state.data_ptr() != state.data_ptr() and _overlap(new_state, state):
            raise ValueError("new_state must be state itself or not overlap it")
    return L, N, H, HV


@torch.no_grad()
def kernel_prefill_hip(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output,
                       new_state, *, use_qk_l2norm: bool = False):
    """Destination-passing prefill (reference DPS form,
    solution/triton/prefill_kernel.py:10-58): writes ``output`` and
    ``new_state``; ``new_state is state`` updates in place."""
    _launch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output, new_state,
            use_qk_l2norm, None)


@torch.no_grad()
def kernel_prefill_hip_timed(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output,
                             new_state, events, *, use_qk_l2norm: bool = False):
    """``kernel_prefill_hip`` with four ``hipEvent_t`` handles (int or
    ``ctypes.c_void_p``) recorded before the offsets, preparation and scan
    launches and after the scan (``gdn_prefill_timed``); a measurement hook,
    not part of the reference's interface."""
    if len(events) != 4:
        raise ValueError("events must be four hipEvent_t handles")
    _launch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output, new_state,
            use_qk_l2norm, events)


@torch.no_grad()
def kernel_prefill_hip_noalloc(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output,
                               new_state, *, use_qk_l2norm: bool = False):
    """``kernel_prefill_hip`` that allocates nothing (``gdn_prefill_noalloc``):
    the workspace is the library's fixed per-GPU array of
    ``NOALLOC_SCRATCH_BYTES``, so the call can sit inside HIP graph capture
    or a loop that must not allocate.  ``cu_seqlens`` must be int32 (no
    conversion copy).  Raises ValueError when these sizes need a larger
    workspace.  Calls that overlap on one GPU (different streams) race on
    that workspace; calls on one stream are ordered.  No counterpart in the
    reference."""
    if cu_seqlens.dtype != torch.int32:
        raise TypeError("kernel_prefill_hip_noalloc takes int32 cu_seqlens (no conversion copy)")
    _launch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output, new_state,
            use_qk_l2norm, None, noalloc=True)


def _launch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output, new_state,
            use_qk_l2norm, events, noalloc=False):
    if output is None or new_state is None:
        raise ValueError("kernel_prefill_hip needs preallocated output and new_state")
    L, N, H, HV = check_prefill_inputs(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens,
                                       output, new_state)
    scale = resolve_scale(scale, q.shape[-1])
    if N == 0:
        return None
    if noalloc:
        need = workspace_bytes(L, N, H, HV)
        if need > NOALLOC_SCRATCH_BYTES:
            raise ValueError(f"prefill of L={L}, N={N}, H={H}, HV={HV} needs a {need}-byte "
                             f"workspace; gdn_prefill_noalloc has {NOALLOC_SCRATCH_BYTES}")
        idx = q.get_device()
        with _on_device(idx):
            code = _lib.get_prefill_lib().gdn_prefill_noalloc(
                q.data_ptr(), k.data_ptr(), v.data_ptr(),
                None if state is None else state.data_ptr(), A_log.data_ptr(), a.data_ptr(),
                dt_bias.data_ptr(), b.data_ptr(), cu_seqlens.data_ptr(), scale,
                output.data_ptr(), new_state.data_ptr(), L, N, H, HV, K_DIM, V_DIM,
                int(bool(use_qk_l2norm)), _lib.current_stream(idx))
        _lib.check(code, "gdn_prefill_noalloc")
        return None
    if cu_seqlens.dtype != torch.int32:
        cu_seqlens = cu_seqlens.to(torch.int32)
    lib = _lib.get_prefill_lib()
    ws_bytes = workspace_bytes(L, N, H, HV)
    workspace = torch.empty(ws_bytes + 256, dtype=torch.uint8, device=q.device)
    ws_ptr = (workspace.data_ptr() + 255) & ~255
    idx = q.get_device()
    stream = _lib.current_stream(idx)
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(),
            None if state is None else state.data_ptr(),
            A_log.data_ptr(), a.data_ptr(), dt_bias.data_ptr(), b.data_ptr(),
            cu_seqlens.data_ptr(), scale, output.data_ptr(), new_state.data_ptr(),
            L, N, H, HV, K_DIM, V_DIM, int(bool(use_qk_l2norm)), ws_ptr, ws_bytes, stream)
    with _on_device(idx):
        if events is None:
            code = lib.gdn_prefill(*args)
        else:
            handles = (ctypes.c_void_p * 4)(
                *[e if isinstance(e, ctypes.c_void_p) else ctypes.c_void_p(int(e))
                  for e in events])
            code = lib.gdn_prefill_timed(*args, handles)
    _lib.check(code, "gdn_prefill_timed" if events is not None else "gdn_prefill")
    # keep the workspace (and a converted cu_seqlens) alive until the kernels ran
    workspace.record_stream(torch.cuda.current_stream(q.device))
    cu_seqlens.record_stream(torch.cuda.current_stream(q.device))
    return None


@torch.no_grad()
def prefill_run(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, *,
                use_qk_l2norm: bool = False):
    """Value-returning prefill with the reference's contract
    (``kernel_prefill_reference``, solution/triton/prefill_kernel.py:85-183):
    returns ``(output [L, HV, 128] bf16, new_state [N, HV, 128, 128] fp32)``;
    ``state`` is not modified.  Tokens that no sequence covers (all of them
    when N = 0, those past ``cu_seqlens[N]`` otherwise) get zero outputs, as
    the reference's zero-initialised result (prefill_kernel.py:135-137)."""
    L, N, H, HV = check_prefill_inputs(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens)
    output = torch.zeros((L, HV, V_DIM), dtype=torch.bfloat16, device=q.device)
    new_state = torch.empty((N, HV, V_DIM, K_DIM), dtype=torch.float32, device=q.device)
    kernel_prefill_hip(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output,
                       new_state, use_qk_l2norm=use_qk_l2norm)
    return output, new_state
