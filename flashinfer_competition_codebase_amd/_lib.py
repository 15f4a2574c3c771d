"""ctypes bindings of ``libgdn_decode.so`` and ``libgdn_prefill.so`` (the C ABIs
in ``include/gdn_decode.h`` and ``include/gdn_prefill.h``).

There is no fallback: if the library is missing or fails to load, every entry
point raises ``RuntimeError`` naming the build command.  The reference builds
its native module lazily on first use (solution/cuda/binding.py:14-28); here
the library is built ahead of time, in-tree, by ``build.py``.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libgdn_decode.so"
PREFILL_LIB_PATH = Path(__file__).resolve().parent / "libgdn_prefill.so"

# Names and argument types of every exported function, in header order.
_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
SIGNATURES = {
    "gdn_decode_step": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P, _I, _I, _I, _I, _I, _I, _P],
    ),
    "gdn_decode_steps": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P] + [_I] * 8 + [_P],
    ),
    "gdn_decode_step_shaped": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P] + [_I] * 11 + [_P, _P, _P],
    ),
    "gdn_decode_step_stamped": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P] + [_I] * 8
        + [ctypes.POINTER(ctypes.c_ulonglong), ctypes.c_longlong, _P],
    ),
    "gdn_decode_launch_shape": (
        _I,
        [_I, _I, _I, _I, ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I),
         ctypes.POINTER(ctypes.c_longlong)],
    ),
    "gdn_decode_plan_create": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P] + [_I] * 8 + [ctypes.POINTER(_P)],
    ),
    "gdn_decode_plan_run": (_I, [ctypes.POINTER(_P), _I, _P]),
    "gdn_decode_plan_destroy": (None, [_P]),
    "gdn_decode_graph_create": (_I, [ctypes.POINTER(_P), _I, ctypes.POINTER(_P)]),
    "gdn_decode_graph_launch": (_I, [_P, _P]),
    "gdn_decode_graph_destroy": (None, [_P]),
    "gdn_decode_error_string": (ctypes.c_char_p, [_I]),
    "gdn_decode_abi_version": (_I, []),
}

ABI_VERSION = 6

_S = ctypes.c_size_t
PREFILL_SIGNATURES = {
    "gdn_prefill_workspace_bytes": (_S, [_I, _I, _I, _I]),
    "gdn_prefill": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P] + [_I] * 7 + [_P, _S, _P],
    ),
    "gdn_prefill_timed": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P] + [_I] * 7 + [_P, _S, _P, _P],
    ),
    "gdn_prefill_noalloc": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P] + [_I] * 7 + [_P],
    ),
    "gdn_prefill_token_path_max_tokens": (_I, []),
    "gdn_prefill_dispatches": (_I, [_I, _I, _I]),
    "gdn_prefill_abi_version": (_I, []),
}
PREFILL_ABI_VERSION = 6

_lock = threading.Lock()
_lib = None
_prefill_lib = None


def _load(path: Path, signatures: dict, version_fn: str, version: int) -> ctypes.CDLL:
    if not path.exists():
        raise RuntimeError(
            f"HIP library not found at {path}; build it with "
            "`python -m flashinfer_competition_codebase_amd.build`"
        )
    try:
        lib = ctypes.CDLL(str(path))
    except OSError as exc:
        raise RuntimeError(f"failed to load HIP library {path}: {exc}") from exc
    for name, (restype, argtypes) in signatures.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    got = getattr(lib, version_fn)()
    if got != version:
        raise RuntimeError(f"{path} has ABI version {got}, expected {version}; rebuild it")
    return lib


def load(path: Path = LIB_PATH) -> ctypes.CDLL:
    """Load the decode library at ``path`` and declare every signature."""
    return _load(path, SIGNATURES, "gdn_decode_abi_version", ABI_VERSION)


def load_prefill(path: Path = PREFILL_LIB_PATH) -> ctypes.CDLL:
    """Load the prefill library at ``path`` and declare every signature."""
    return _load(path, PREFILL_SIGNATURES, "gdn_prefill_abi_version", PREFILL_ABI_VERSION)


def get_lib() -> ctypes.CDLL:
    """Process-wide library handle, loaded on first use."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                _lib = load()
    return _lib


def get_prefill_lib() -> ctypes.CDLL:
    """Process-wide prefill library handle, loaded on first use."""
    global _prefill_lib
    if _prefill_lib is None:
        with _lock:
            if _prefill_lib is None:
                _prefill_lib = load_prefill()
    return _prefill_lib


_raw_stream = None


def raw_stream_accessor():
    """The function ``device_index -> raw hipStream_t`` of torch's current
    stream on that device (torch's raw accessor where it has one: the public
    ``current_stream`` builds a Stream object per call)."""
    global _raw_stream
    if _raw_stream is None:
        import torch
        _raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None) or (
            lambda i: torch.cuda.current_stream(i).cuda_stream)
    return _raw_stream


def current_stream(device_index: int) -> int:
    """Raw ``hipStream_t`` of torch's current stream on ``device_index``."""
    return (_raw_stream or raw_stream_accessor())(device_index)


def error_string(code: int) -> str:
    text = get_lib().gdn_decode_error_string(int(code))
    return text.decode() if text else f"error {code}"


def check(code: int, what: str) -> None:
    if code != 0:
        raise RuntimeError(f"{what} failed: {error_string(code)} (hipError_t {code})")


def launch_shape(B: int, HV: int, T: int = 1, state_bf16: bool = False
                 ) -> tuple[int, int, int, int]:
    """(rows_per_lane_group, waves_per_block, cache_policy, num_blocks)
    that gdn_decode_steps uses for B sequences of T tokens over HV v-heads."""
    ns, w, pol, nb = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_longlong()
    check(
        get_lib().gdn_decode_launch_shape(
            int(B), int(T), int(HV), int(bool(state_bf16)), ctypes.byref(ns),
            ctypes.byref(w), ctypes.byref(pol), ctypes.byref(nb)
        ),
        "gdn_decode_launch_shape",
    )
    return ns.value, w.value, pol.value, nb.value
