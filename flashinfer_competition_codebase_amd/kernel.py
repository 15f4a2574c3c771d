"""Python entry points of the GDN decode step, in the reference's calling forms.

Two forms, with the reference's argument names so callers can pass the
tensors as keyword arguments (``fn(**tensors)``, scripts/bench_fi_timing.py:44):

* ``run(q, k, v, state, A_log, a, dt_bias, b, scale)`` -- value-returning,
  like ``kernel_pt_reference`` (solution/triton/kernel.py:22-118): returns
  ``(output, new_state)`` and leaves ``state`` untouched.
* ``kernel_hip(q, k, v, state, A_log, a, dt_bias, b, scale, output,
  new_state)`` -- destination-passing, like ``kernel_fla_recurrent``
  (solution/triton/kernel.py:150-197) and ``kernel_cuda_v4``
  (solution/cuda/binding.py:44-60): writes both outputs and returns None.
  ``new_state`` may be ``state`` itself for an in-place update (the
  aliasing FlashInfer's entry uses, solution/triton/kernel.py:128-134).

Both run one launch of the gfx950 kernel in ``libgdn_decode.so`` on the
current HIP stream of the inputs' device; there is no CPU path.  The q/k
L2-norm is a keyword-only flag (``use_qk_l2norm``, default off as in every
reference decode entry, solution/triton/kernel.py:146), so the positional
signature is the reference's.

Tensor contract (reference shapes, solution/triton/kernel.py:33-48 and
scripts/profile_proton.py:106-110): q, k ``[B, T, H, 128]`` bf16; v
``[B, T, HV, 128]`` bf16 with ``HV % H == 0``; state ``[B, HV, 128, 128]``
k-last, fp32 or bf16, or None (zeros); A_log, dt_bias ``[HV]`` fp32; a, b
``[B, T, HV]`` bf16 (``[B, HV]`` also at T = 1); scale float, 0-d tensor,
None or 0 (None/0 mean ``1/sqrt(K)``); output ``[B, T, HV, 128]`` bf16;
new_state like state.  The reference's decode is T = 1 with an fp32 state;
T > 1 (multi-token decode: the state is read once, the T tokens are applied
in order, solution/triton/prefill_kernel.py:144-178) and a bf16 state (fp32
arithmetic, stored rounded to nearest even) are the FlashInfer decode
features the reference records (findings/fi-gdn-decode-kernel.md:11-16).
All tensors dense (contiguous) on one device.  Unlike the reference,
malformed arguments raise ``TypeError`` / ``ValueError`` before anything is
launched.
"""

from __future__ import annotations

import ctypes
import functools
import math
import weakref

import torch

from . import _lib

K_DIM = 128
V_DIM = 128

__all__ = ["run", "run_dps", "kernel_hip", "kernel_hip_shaped", "resolve_scale"]


def resolve_scale(scale, K: int = K_DIM) -> float:
    """``scale`` as a float; None or 0 mean ``1/sqrt(K)``.

    Reference: solution/triton/kernel.py:69-70 and 163-164,
    solution/cuda/binding.py:50-53 (``float(scale)`` for tensor scalars).
    """
    if scale is None:
        return 1.0 / math.sqrt(K)
    if isinstance(scale, torch.Tensor):
        if scale.numel() != 1:
            raise ValueError(f"scale must be a scalar, got shape {tuple(scale.shape)}")
        scale = scale.item()
    scale = float(scale)
    if scale == 0.0:
        return 1.0 / math.sqrt(K)
    return scale


def _expect(t, name: str, dtype: torch.dtype, shape: tuple) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if t.shape != shape:                      # torch.Size compares with a tuple
        raise ValueError(f"{name} must have shape {shape}, got {tuple(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


STATE_DTYPES = (torch.float32, torch.bfloat16)


def _gate_shape(t, B: int, T: int, HV: int) -> tuple:
    shape = tuple(t.shape) if isinstance(t, torch.Tensor) else None
    return (B, HV) if (T == 1 and shape == (B, HV)) else (B, T, HV)


def _expect_state(t, name: str, shape: tuple, dtype=None) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if t.dtype not in STATE_DTYPES:
        raise TypeError(f"{name} must be float32 or bfloat16, got {t.dtype}")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} must have the state's dtype {dtype}, got {t.dtype}")
    _expect(t, name, t.dtype, shape)


def check_inputs(q, k, v, state, A_log, a, dt_bias, b, output=None, new_state=None):
    """Validate the decode-step tensors; returns ``(B, T, H, HV)``.

    Shape and dtype rules are the reference's (solution/triton/kernel.py:
    33-48, 58-67 generalised to any ``HV % H == 0``, T >= 1 and a bf16
    state); the device check comes last so that every other rule can be
    exercised without a GPU.
    """
    if not isinstance(q, torch.Tensor) or q.dim() != 4:
        raise ValueError("q must be a 4-D tensor [B, T, H, K]")
    if not isinstance(v, torch.Tensor) or v.dim() != 4:
        raise ValueError("v must be a 4-D tensor [B, T, HV, V]")
    B, T, H, K = q.shape
    HV, V = v.shape[2], v.shape[3]
    if T < 1:
        raise ValueError(f"decode takes at least one token per sequence, got T={T}")
    if K != K_DIM or V != V_DIM:
        raise ValueError(f"K and V must be {K_DIM}, got K={K}, V={V}")
    if H <= 0 or HV <= 0 or HV % H != 0:
        raise ValueError(f"v-heads must be a multiple of q/k heads, got H={H}, HV={HV}")
    _expect(q, "q", torch.bfloat16, (B, T, H, K))
    _expect(k, "k", torch.bfloat16, (B, T, H, K))
    _expect(v, "v", torch.bfloat16, (B, T, HV, V))
    if state is not None:
        _expect_state(state, "state", (B, HV, V, K))
    _expect(A_log, "A_log", torch.float32, (HV,))
    _expect(dt_bias, "dt_bias", torch.float32, (HV,))
    _expect(a, "a", torch.bfloat16, _gate_shape(a, B, T, HV))
    _expect(b, "b", torch.bfloat16, _gate_shape(b, B, T, HV))
    if output is not None:
        _expect(output, "output", torch.bfloat16, (B, T, HV, V))
    if new_state is not None:
        _expect_state(new_state, "new_state", (B, HV, V, K),
                      None if state is None else state.dtype)
    _same_hip_device(q, (k, v, A_log, a, dt_bias, b, state, output, new_state),
                     "the GDN decode kernel")
    if state is not None and new_state is not None and new_state is not state:
        if new_state.data_ptr() != state.data_ptr() and _overlap(new_state, state):
            raise ValueError("new_state must be state itself or not overlap it")
    return B, T, H, HV


def _same_hip_device(first: torch.Tensor, others, what: str) -> int:
    """Device index of ``first``; raises unless every tensor of ``others``
    (None entries skipped) is on that device and it is a HIP device."""
    idx = first.get_device()                  # -1 off the GPU (cpu, meta, ...)
    for t in others:
        if t is not None and (t.get_device() != idx or (idx < 0 and t.device != first.device)):
            raise ValueError(f"all tensors must be on one device, got {first.device} and "
                             f"{t.device}")
    if idx < 0 or first.device.type != "cuda":
        raise ValueError(f"{what} runs on a HIP device; got tensors on {first.device}")
    return idx


def _overlap(x: torch.Tensor, y: torch.Tensor) -> bool:
    x0, y0 = x.data_ptr(), y.data_ptr()
    xn, yn = x.numel() * x.element_size(), y.numel() * y.element_size()
    return x0 < y0 + yn and y0 < x0 + xn


class _NoSwitch:
    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


_NO_SWITCH = _NoSwitch()


def _on_device(idx: int):
    """Context that makes device ``idx`` current for a launch; a no-op when
    it already is."""
    return _NO_SWITCH if torch.cuda.current_device() == idx else torch.cuda.device(idx)


def _launch(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state,
            B, T, H, HV, use_qk_l2norm, shape=None):
    lib = _lib.get_lib()
    idx = q.get_device()
    stream = _lib.current_stream(idx)
    ptrs = (q.data_ptr(), k.data_ptr(), v.data_ptr(),
            None if state is None else state.data_ptr(),
            A_log.data_ptr(), a.data_ptr(), dt_bias.data_ptr(), b.data_ptr())
    l2 = int(bool(use_qk_l2norm))
    bf16 = int(new_state.dtype == torch.bfloat16)
    # the launch goes to the inputs' device (switched to only when another is current)
    with _on_device(idx):
        if shape is not None:
            ns, waves, policy, start_event, stop_event = shape
            code = lib.gdn_decode_step_shaped(
                *ptrs, scale, output.data_ptr(), new_state.data_ptr(),
                B, T, H, HV, K_DIM, V_DIM, bf16, l2,
                int(ns), int(waves), int(policy), start_event, stop_event, stream)
            _lib.check(code, "gdn_decode_step_shaped")
        elif T == 1 and not bf16:
            code = lib.gdn_decode_step(
                *ptrs, scale, output.data_ptr(), new_state.data_ptr(),
                B, H, HV, K_DIM, V_DIM, l2, stream)
            _lib.check(code, "gdn_decode_step")
        else:
            code = lib.gdn_decode_steps(
                *ptrs, scale, output.data_ptr(), new_state.data_ptr(),
                B, T, H, HV, K_DIM, V_DIM, bf16, l2, stream)
            _lib.check(code, "gdn_decode_steps")


class _Validated:
    """A decode call that passed every check, bound once in a native plan
    (``gdn_decode_plan_create``: the same checks on the C side, the launch
    shape resolved).  It is recognised by the identities of its tensor
    objects -- while they live: a weak reference to each evicts the entry
    when that tensor is freed, so an id is never reused under a live entry
    -- and by their data pointers, compared on every call (a tensor whose
    storage was swapped in place is validated afresh).  ``run(stream)`` is
    the bound native call ``gdn_decode_plan_run(plan, 1, stream)``."""

    __slots__ = ("key", "ptrs", "device", "handle", "arr", "refs", "run", "__weakref__")

    def __init__(self, key, tensors, device, handle):
        self.key = key
        self.ptrs = _data_ptrs(*tensors)
        self.device = device
        self.handle = handle
        self.arr = (ctypes.c_void_p * 1)(handle)
        self.refs = []
        self.run = functools.partial(_lib.get_lib().gdn_decode_plan_run, self.arr, 1)

    def destroy(self) -> None:
        if self.handle is not None:
            handle, self.handle = self.handle, None
            try:
                _lib.get_lib().gdn_decode_plan_destroy(handle)
            except Exception:          # interpreter shutdown: the library may be gone
                pass


# Validated calls by the ids of their tensors, scale and flag (insertion order:
# the oldest is evicted first).  A serving loop that calls the step with a
# fixed set of buffers per layer runs every call after the first through here.
_VALIDATED: dict = {}
_VALIDATED_MAX = 256
_dp = torch.Tensor.data_ptr
_stream_of = _lib.raw_stream_accessor()


def _data_ptrs(q, k, v, state, A_log, a, dt_bias, b, output, new_state) -> tuple:
    return (_dp(q), _dp(k), _dp(v), None if state is None else _dp(state), _dp(A_log),
            _dp(a), _dp(dt_bias), _dp(b), _dp(output), _dp(new_state))


def _evict(key, _table=_VALIDATED) -> None:
    entry = _table.pop(key, None)
    if entry is not None:
        entry.destroy()


def _on_free(key):
    """Weak-reference callback that evicts ``key``; bound to its own
    references so it still works while the interpreter tears the module's
    globals down."""
    return lambda _ref, key=key, evict=_evict: evict(key)


def _bind(key, tensors, scale: float, B, T, H, HV, use_qk_l2norm) -> _Validated:
    q, k, v, state, A_log, a, dt_bias, b, output, new_state = tensors
    lib = _lib.get_lib()
    handle = ctypes.c_void_p()
    code = lib.gdn_decode_plan_create(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), None if state is None else state.data_ptr(),
        A_log.data_ptr(), a.data_ptr(), dt_bias.data_ptr(), b.data_ptr(), scale,
        output.data_ptr(), new_state.data_ptr(), B, T, H, HV, K_DIM, V_DIM,
        int(new_state.dtype == torch.bfloat16), int(bool(use_qk_l2norm)), ctypes.byref(handle))
    _lib.check(code, "gdn_decode_plan_create")
    entry = _Validated(key, tensors, q.get_device(), handle)
    if len(_VALIDATED) >= _VALIDATED_MAX:
        _evict(next(iter(_VALIDATED)))
    _VALIDATED[key] = entry
    evict = _on_free(key)
    entry.refs = [weakref.ref(t, evict) for t in tensors if t is not None]
    return entry


def kernel_hip(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state,
               *, use_qk_l2norm: bool = False):
    """Destination-passing decode step (reference DPS form,
    solution/triton/kernel.py:150-197; solution/cuda/binding.py:44-60).

    Writes ``output`` [B, T, HV, 128] bf16 and ``new_state``
    [B, HV, 128, 128] (the state's dtype).  ``new_state is state`` updates in
    place; ``state=None`` starts from zeros (solution/triton/kernel.py:83-86).

    A call with the same tensor objects (unchanged data pointers), a float or
    None scale and the same flag as an earlier validated call -- a decode
    loop's steady state -- skips the checks and launches the native plan
    bound then: one three-argument native call.  Shapes are not compared on
    that path: a tensor reshaped in place with its data pointer unchanged
    (``resize_`` within its storage, ``as_strided_``) is used with the sizes
    it was validated with; pass a new tensor object (a view) instead.
    """
    tp = type(scale)
    if scale is None or tp is float or tp is int:
        key = (id(q), id(k), id(v), id(state), id(A_log), id(a), id(dt_bias), id(b),
               id(output), id(new_state), scale, bool(use_qk_l2norm))
        entry = _VALIDATED.get(key)
        if entry is not None and entry.ptrs == (
                _dp(q), _dp(k), _dp(v), None if state is None else _dp(state), _dp(A_log),
                _dp(a), _dp(dt_bias), _dp(b), _dp(output), _dp(new_state)):
            # the plan makes its own device current for the launch
            code = entry.run(_stream_of(entry.device))
            if code:
                _lib.check(code, "gdn_decode_plan_run")
            return None
    else:
        key = None
    if output is None or new_state is None:
        raise ValueError("kernel_hip needs preallocated output and new_state")
    B, T, H, HV = check_inputs(q, k, v, state, A_log, a, dt_bias, b, output, new_state)
    scale_f = resolve_scale(scale, q.shape[-1])
    if B == 0:
        return None
    if key is not None:
        _evict(key)                    # the same objects with new storage
        with _on_device(q.get_device()):      # the plan records the current device
            entry = _bind(key, (q, k, v, state, A_log, a, dt_bias, b, output, new_state),
                          scale_f, B, T, H, HV, use_qk_l2norm)
        code = entry.run(_lib.current_stream(entry.device))
        if code:
            _lib.check(code, "gdn_decode_plan_run")
        return None
    # state=None: the kernel starts from zeros and only writes new_state
    _launch(q, k, v, state, A_log, a, dt_bias, b, scale_f, output, new_state,
            B, T, H, HV, use_qk_l2norm)
    return None


@torch.no_grad()
def kernel_hip_shaped(q, k, v, state, A_log, a, dt_bias, b, scale, output,
                      new_state, *, use_qk_l2norm: bool = False,
                      rows_per_lane_group: int = 2, waves_per_block: int = 4,
                      cache_policy: int = 1, start_event=None, stop_event=None):
    """``kernel_hip`` with an explicit launch shape, for launch-shape sweeps
    and timing.  ``start_event`` / ``stop_event`` are raw ``hipEvent_t``
    handles (ints) that the launch stamps with the kernel's own start and end
    timestamps."""
    B, T, H, HV = check_inputs(q, k, v, state, A_log, a, dt_bias, b, output, new_state)
    scale = resolve_scale(scale, q.shape[-1])
    if B == 0:
        return None
    _launch(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state,
            B, T, H, HV, use_qk_l2norm,
            shape=(rows_per_lane_group, waves_per_block, cache_policy,
                   start_event, stop_event))
    return None


@torch.no_grad()
def run(q, k, v, state, A_log, a, dt_bias, b, scale, *, use_qk_l2norm: bool = False):
    """Value-returning decode step with the reference's contract
    (``kernel_pt_reference``, solution/triton/kernel.py:22-118).

    Returns ``(output [B, T, HV, 128] bf16, new_state [B, HV, 128, 128])``,
    the new state in the state's dtype (fp32 for ``state=None``); ``state``
    is not modified.
    """
    B, T, H, HV = check_inputs(q, k, v, state, A_log, a, dt_bias, b)
    sdtype = torch.float32 if state is None else state.dtype
    output = torch.empty((B, T, HV, V_DIM), dtype=torch.bfloat16, device=q.device)
    new_state = torch.empty((B, HV, V_DIM, K_DIM), dtype=sdtype, device=q.device)
    if B > 0:
        # fresh outputs every call: launched directly, not bound for reuse
        _launch(q, k, v, state, A_log, a, dt_bias, b, resolve_scale(scale, q.shape[-1]),
                output, new_state, B, T, H, HV, use_qk_l2norm)
    return output, new_state


# The 11-argument DPS form under the name a definition's solution module
# exposes beside ``run`` (new_state may be state itself).
run_dps = kernel_hip
