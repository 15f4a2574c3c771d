"""Decode steps bound once, for serving loops: launch overhead off the path.

At B = 1 a decode step's kernel takes ~2.5-3 µs, while a call through
``kernel_hip`` costs ~12 µs of host time (argument checks, stream lookup,
the ctypes call with 18 arguments).  The reference's notes plan the two
usual cures for its own decode step: bind once and replay a CUDA graph,
or a persistent kernel (findings/potential-cuda-improvement.md:143-147,539).
Here:

* ``DecodePlan`` binds one decode call -- the same tensors and arguments as
  ``kernel_hip`` -- once: shapes, dtypes, devices and aliasing are checked
  and the launch shape is resolved in ``gdn_decode_plan_create``; ``run()``
  is then one ctypes call with three arguments and one launch.  The bound
  tensors stay fixed; the caller writes each step's q, k, v, a and b into
  them (the state is updated in place when ``new_state`` is ``state``).
* ``DecodeLayers`` holds the plans of a model's GDN layers (one state per
  layer) and runs them eagerly in one native call, or records them once in
  a HIP graph (``gdn_decode_graph_create``: stream capture on a private
  stream, no memset nodes) and replays it, one submission per model step.

Both launch on torch's current stream of the plans' device; there is no
CPU path.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .kernel import check_inputs, resolve_scale, _on_device

__all__ = ["DecodePlan", "DecodeLayers"]


class DecodePlan:
    """One decode step over fixed tensors (``kernel_hip``'s arguments,
    solution/triton/kernel.py:150-197), validated and bound once.

    ``state=None`` starts every run from zeros; ``new_state is state``
    updates the state in place, so consecutive runs continue the sequence.
    """

    def __init__(self, q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state, *,
                 use_qk_l2norm: bool = False):
        if output is None or new_state is None:
            raise ValueError("DecodePlan needs preallocated output and new_state")
        B, T, H, HV = check_inputs(q, k, v, state, A_log, a, dt_bias, b, output, new_state)
        self.device = q.get_device()
        self.shape = (B, T, H, HV)
        scale = resolve_scale(scale, q.shape[-1])
        self._lib = _lib.get_lib()
        handle = ctypes.c_void_p()
        with _on_device(self.device):          # the plan records the current device
            code = self._lib.gdn_decode_plan_create(
                q.data_ptr(), k.data_ptr(), v.data_ptr(),
                None if state is None else state.data_ptr(), A_log.data_ptr(), a.data_ptr(),
                dt_bias.data_ptr(), b.data_ptr(), scale, output.data_ptr(),
                new_state.data_ptr(), B, T, H, HV, q.shape[-1], v.shape[-1],
                int(new_state.dtype == torch.bfloat16), int(bool(use_qk_l2norm)),
                ctypes.byref(handle))
        _lib.check(code, "gdn_decode_plan_create")
        self._handle = handle
        self._one = (ctypes.c_void_p * 1)(handle)
        # the buffers the plan points at live as long as the plan
        self.tensors = dict(q=q, k=k, v=v, state=state, A_log=A_log, a=a, dt_bias=dt_bias, b=b,
                            output=output, new_state=new_state)

    @property
    def handle(self) -> ctypes.c_void_p:
        if self._handle is None:
            raise RuntimeError("the plan was closed")
        return self._handle

    def run(self) -> None:
        """One decode step on torch's current stream of the plan's device."""
        self.handle                                # raises once closed
        # the plan makes its own device current for the launch
        code = self._lib.gdn_decode_plan_run(self._one, 1, _lib.current_stream(self.device))
        if code:
            _lib.check(code, "gdn_decode_plan_run")

    def close(self) -> None:
        if self._handle is not None:
            self._lib.gdn_decode_plan_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:       # interpreter shutdown: the library may be gone
            pass


class DecodeLayers:
    """The decode steps of several layers (e.g. a model's GDN layers), each a
    ``DecodePlan``, run in order: eagerly in one native call (``run()``), or
    as one HIP graph (``capture()`` once, then ``replay()``).

    ``layers`` is a list of ``kernel_hip`` argument dicts (q, k, v, state,
    A_log, a, dt_bias, b, scale, output, new_state), one per layer, all on
    one device; each layer's buffers are fixed and rewritten by the caller
    between steps.
    """

    def __init__(self, layers, *, use_qk_l2norm: bool = False):
        if not layers:
            raise ValueError("DecodeLayers needs at least one layer")
        self.plans = [DecodePlan(**t, use_qk_l2norm=use_qk_l2norm) for t in layers]
        self.device = self.plans[0].device
        if any(p.device != self.device for p in self.plans):
            raise ValueError("all layers must be on one device")
        self._handles = (ctypes.c_void_p * len(self.plans))(*[p.handle for p in self.plans])
        self._lib = self.plans[0]._lib
        self._graph = None

    def __len__(self) -> int:
        return len(self.plans)

    def _check_open(self) -> None:
        # the native calls take the plans' raw pointers: never pass freed ones
        if self._handles is None:
            raise RuntimeError("the layers were closed")
        if any(p._handle is None for p in self.plans):
            raise RuntimeError("a layer's plan was closed")

    def run(self) -> None:
        """Every layer's step, in order, from one native call (no graph)."""
        self._check_open()
        code = self._lib.gdn_decode_plan_run(self._handles, len(self.plans),
                                             _lib.current_stream(self.device))
        if code:
            _lib.check(code, "gdn_decode_plan_run")

    def capture(self) -> None:
        """Record every layer's step, in order, in one HIP graph (replaces a
        previous one)."""
        self._check_open()
        self.release_graph()
        graph = ctypes.c_void_p()
        with _on_device(self.device):
            code = self._lib.gdn_decode_graph_create(self._handles, len(self.plans),
                                                     ctypes.byref(graph))
        _lib.check(code, "gdn_decode_graph_create")
        self._graph = graph

    def replay(self) -> None:
        """All layers' steps as one graph submission on torch's current stream."""
        self._check_open()
        if self._graph is None:
            raise RuntimeError("capture() the graph before replaying it")
        with _on_device(self.device):
            code = self._lib.gdn_decode_graph_launch(self._graph,
                                                     _lib.current_stream(self.device))
        if code:
            _lib.check(code, "gdn_decode_graph_launch")

    def release_graph(self) -> None:
        if self._graph is not None:
            self._lib.gdn_decode_graph_destroy(self._graph)
            self._graph = None

    def close(self) -> None:
        self.release_graph()
        for p in self.plans:
            p.close()
        self._handles = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
