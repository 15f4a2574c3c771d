"""The C-ABI library loads and exports exactly what include/gdn_decode.h declares.

No compute call is made: the only native calls here either query metadata or
pass arguments that the library's host-side validation rejects before any
HIP call.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from flashinfer_competition_codebase_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "gdn_decode.h"


def header_functions() -> dict:
    """name -> number of parameters, for every prototype in the header."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    protos = re.findall(r"^\s*(?:const\s+)?\w+\*?\s+(gdn_decode_\w+)\s*\(([^;]*?)\)\s*;",
                        text, flags=re.M | re.S)
    out = {}
    for name, params in protos:
        params = params.strip()
        out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_header_declares_the_abi():
    funcs = header_functions()
    assert set(funcs) == {"gdn_decode_step", "gdn_decode_steps", "gdn_decode_step_shaped",
                          "gdn_decode_launch_shape", "gdn_decode_step_stamped", "gdn_decode_plan_create",
                          "gdn_decode_plan_run", "gdn_decode_plan_destroy",
                          "gdn_decode_graph_create", "gdn_decode_graph_launch",
                          "gdn_decode_graph_destroy", "gdn_decode_error_string",
                          "gdn_decode_abi_version"}


def test_library_exports_every_declared_symbol():
    lib = _lib.get_lib()
    funcs = header_functions()
    for name, nparams in funcs.items():
        assert hasattr(lib, name), f"{name} missing from {_lib.LIB_PATH}"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
        assert len(_lib.SIGNATURES[name][1]) == nparams, name


def test_abi_version_and_error_text():
    lib = _lib.get_lib()
    assert lib.gdn_decode_abi_version() == _lib.ABI_VERSION
    assert _lib.error_string(1) == "invalid argument"


def test_launch_shape_query():
    ns, w, pol, blocks = _lib.launch_shape(1, 32)
    assert ns in (1, 2, 4, 8) and w in (1, 2, 4, 8) and pol in (0, 1, 2, 3)
    assert blocks == 32 * 128 // (4 * ns * w)
    assert _lib.launch_shape(0, 32)[3] == 0
    ns, w, pol, blocks = _lib.launch_shape(256, 32)
    assert blocks == 256 * 32 * 128 // (4 * ns * w)
    with pytest.raises(RuntimeError):
        _lib.launch_shape(-1, 32)
    with pytest.raises(RuntimeError):
        _lib.launch_shape(1, 32, T=0)


@pytest.mark.parametrize("T,bf16", [(1, False), (1, True), (2, False), (3, False),
                                    (4, False), (4, True)])
def test_launch_shape_table_stays_in_the_supported_space(T, bf16):
    """Every head count gets a shape the kernel is built for: at most 32
    rows per lane group x waves, power-of-two tiles per head, and a cache
    policy every variant has (0 or 1); or, for T = 2..4, the block kernel
    (16, 32 or 64 rows per wave, at most 128 rows per block, policy 1)."""
    for heads in (1, 7, 8, 9, 16, 32, 33, 64, 100, 128, 256, 257, 384, 512, 1000, 8192,
                  1 << 20):
        ns, w, pol, blocks = _lib.launch_shape(heads, 1, T=T, state_bf16=bf16)
        if ns in (16, 32, 64):
            assert 2 <= T <= 4 and w in (1, 2, 4, 8) and ns * w <= 128 and pol == 1
            assert blocks == heads * 128 // (ns * w)
            continue
        assert ns in (1, 2, 4, 8) and w in (1, 2, 4, 8) and ns * w <= 32
        assert pol in (0, 1)
        assert blocks == heads * 128 // (4 * ns * w)


def _step(lib, *, B=1, H=16, HV=32, K=128, V=128, ptr=None, new_state=None):
    p = ptr
    return lib.gdn_decode_step(p, p, p, p, p, p, p, p, ctypes.c_float(0.1), p,
                               new_state if new_state is not None else p,
                               B, H, HV, K, V, 1, None)


def test_validation_rejects_bad_sizes_without_launching():
    lib = _lib.get_lib()
    assert _step(lib, K=64) == 1
    assert _step(lib, V=256) == 1
    assert _step(lib, H=3) == 1          # 32 % 3 != 0
    assert _step(lib, H=0) == 1
    assert _step(lib, B=-1) == 1
    assert _step(lib) == 1               # null pointers
    assert _step(lib, B=0) == 0          # empty batch: nothing to do
    shaped = lib.gdn_decode_step_shaped
    nulls = [None] * 8
    f = ctypes.c_float(0.1)

    def sh(T, bf16, ns, w, pol, state=0x1000):
        # B = 0: a supported request returns 0 (nothing to launch), an
        # unsupported one is rejected first (nothing is dereferenced)
        args = list(nulls)
        args[3] = state
        return shaped(*args, f, None, None, 0, T, 16, 32, 128, 128, bf16, 1, ns, w, pol,
                      None, None, None)

    assert sh(1, 0, 2, 4, 1) == 0     # the B=256 fp32 shape
    assert sh(1, 0, 8, 4, 3) == 0     # 32 rows per block, nontemporal loads only
    assert sh(4, 0, 8, 1, 1) == 0     # multi-token, 8 rows per lane group
    assert sh(1, 1, 8, 2, 0) == 0     # bf16 state, 8 rows per lane group
    assert sh(1, 0, 8, 8, 0) == 1     # 8 x 8 > 32 rows per block
    assert sh(1, 0, 3, 1, 0) == 1     # not a power of two
    assert sh(1, 0, 1, 1, 4) == 1     # unknown cache policy
    assert sh(2, 0, 2, 1, 3) == 1     # multi-token kernels take cache policy 0 or 1
    assert sh(1, 1, 2, 4, 2) == 1     # bf16-state kernels take cache policy 0 or 1
    assert sh(1, 0, 2, 4, 3, state=None) == 1   # a null state runs the multi-token loop
    assert sh(0, 0, 2, 4, 1) == 1     # T < 1
    assert sh(1, 2, 2, 4, 1) == 1     # state_bf16 is 0 or 1
    # the block kernel: 16, 32 or 64 rows per wave, T = 2..4, cache policy 1
    assert sh(4, 1, 64, 2, 1) == 0
    assert sh(2, 0, 16, 8, 1) == 0
    assert sh(3, 1, 32, 4, 1, state=None) == 0
    assert sh(1, 1, 32, 2, 1) == 1    # one token: the token-by-token kernel
    assert sh(5, 1, 32, 2, 1) == 1    # more than four tokens
    assert sh(4, 1, 32, 2, 0) == 1    # ordinary stores are not built
    assert sh(4, 0, 64, 4, 1) == 1    # 256 rows per block: more than one head
    assert sh(4, 0, 48, 1, 1) == 1    # not a multiple of the 16-row tile
    steps = lib.gdn_decode_steps
    assert steps(*nulls, f, None, None, 1, 0, 16, 32, 128, 128, 0, 1, None) == 1
    assert steps(*nulls, f, None, None, 0, 4, 16, 32, 128, 128, 1, 1, None) == 0


def test_validation_rejects_misaligned_and_overlapping_state():
    """Only on hosts without a HIP device: a validation bug here would
    otherwise launch on made-up addresses."""
    import torch

    if torch.cuda.is_available():
        pytest.skip("made-up pointers are only passed where no device exists")
    lib = _lib.get_lib()
    assert _step(lib, ptr=0x100002) == 1                       # 2-byte aligned
    # H is packed in 15 bits of a kernel argument (bit 15 carries a launch flag)
    assert _step(lib, H=32768, HV=32768, ptr=0x100000) == 1
    assert _step(lib, ptr=0x100000, new_state=0x100010) == 1   # partial overlap


def test_plans_validate_once_and_run_without_checks():
    """gdn_decode_plan_create applies gdn_decode_steps' validation (nothing
    is launched; without a device the plan records none); an empty batch
    makes a plan whose runs launch nothing; plan_run and graph_create reject
    null or empty plan lists before any HIP call."""
    lib = _lib.get_lib()
    nulls = [None] * 8
    f = ctypes.c_float(0.1)
    plan = ctypes.c_void_p(1234)
    assert lib.gdn_decode_plan_create(*nulls, f, None, None, 1, 1, 16, 32, 128, 128, 0, 1,
                                      ctypes.byref(plan)) == 1
    assert plan.value is None                               # NULL on error
    assert lib.gdn_decode_plan_create(*nulls, f, None, None, 1, 1, 16, 32, 64, 128, 0, 1,
                                      ctypes.byref(plan)) == 1
    assert lib.gdn_decode_plan_create(*nulls, f, None, None, 0, 1, 16, 32, 128, 128, 0, 1,
                                      None) == 1
    assert lib.gdn_decode_plan_create(*nulls, f, None, None, 0, 1, 16, 32, 128, 128, 0, 1,
                                      ctypes.byref(plan)) == 0
    assert plan.value is not None
    arr = (ctypes.c_void_p * 2)(plan, plan)
    assert lib.gdn_decode_plan_run(arr, 2, None) == 0        # B = 0: nothing to launch
    assert lib.gdn_decode_plan_run(arr, 0, None) == 0
    assert lib.gdn_decode_plan_run(None, 1, None) == 1
    assert lib.gdn_decode_plan_run((ctypes.c_void_p * 1)(None), 1, None) == 1
    graph = ctypes.c_void_p()
    assert lib.gdn_decode_graph_create(arr, 0, ctypes.byref(graph)) == 1
    assert lib.gdn_decode_graph_create((ctypes.c_void_p * 1)(None), 1, ctypes.byref(graph)) == 1
    assert lib.gdn_decode_graph_launch(None, None) == 1
    lib.gdn_decode_plan_destroy(plan)
    lib.gdn_decode_plan_destroy(None)
    lib.gdn_decode_graph_destroy(None)


def test_serving_classes_need_a_hip_device():
    from flashinfer_competition_codebase_amd.serving import DecodeLayers, DecodePlan
    from oracle.gdn_decode_oracle import make_inputs

    t = make_inputs(1, 4, 8, seed=1)
    out = torch_empty_out(t)
    with pytest.raises(ValueError, match="HIP device"):
        DecodePlan(**t, output=out, new_state=t["state"])
    with pytest.raises(ValueError):
        DecodeLayers([])


def torch_empty_out(t):
    import torch

    B, T, HV = t["v"].shape[0], t["v"].shape[1], t["v"].shape[2]
    return torch.empty(B, T, HV, 128, dtype=torch.bfloat16)


def test_decode_layers_refuse_to_run_after_close():
    """DecodeLayers passes its plans' raw pointers to the native calls: once
    it or one of its plans is closed, run/capture/replay raise instead (no
    freed plan pointer reaches the library).  Host logic only: a stub stands
    in for the library and the plans."""
    import ctypes as ct

    from flashinfer_competition_codebase_amd.serving import DecodeLayers

    calls = []

    class StubLib:
        def gdn_decode_plan_run(self, *a):
            calls.append("run")
            return 0

        def gdn_decode_plan_destroy(self, h):
            calls.append("destroy")

        def gdn_decode_graph_destroy(self, g):
            calls.append("graph_destroy")

    class StubPlan:
        def __init__(self, lib):
            self._lib, self._handle = lib, ct.c_void_p(0x1000)

        def close(self):
            if self._handle is not None:
                self._lib.gdn_decode_plan_destroy(self._handle)
                self._handle = None

    lib = StubLib()
    layers = DecodeLayers.__new__(DecodeLayers)
    layers.plans = [StubPlan(lib), StubPlan(lib)]
    layers.device = -1
    layers._handles = (ct.c_void_p * 2)(*[p._handle for p in layers.plans])
    layers._lib = lib
    layers._graph = None

    layers.plans[1].close()                      # one plan closed on its own
    for fn in (layers.run, layers.capture, layers.replay):
        with pytest.raises(RuntimeError, match="plan was closed"):
            fn()
    layers.close()
    for fn in (layers.run, layers.capture, layers.replay):
        with pytest.raises(RuntimeError, match="layers were closed"):
            fn()
    assert "run" not in calls and calls.count("destroy") == 2
    layers.close()                               # idempotent
