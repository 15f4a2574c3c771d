"""ctypes binding of ``libgdn_decode.so`` (the C ABI in ``include/gdn_decode.h``).

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
    "gdn_decode_launch_shape": (
        _I,
        [_I, _I, _I, _I, ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I),
         ctypes.POINTER(ctypes.c_longlong)],
    ),
    "gdn_decode_error_string": (ctypes.c_char_p, [_I]),
    "gdn_decode_abi_version": (_I, []),
}

ABI_VERSION = 3

_lock = threading.Lock()
_lib = None


def load(path: Path = LIB_PATH) -> ctypes.CDLL:
    """Load the library at ``path`` and declare every signature."""
    if not path.exists():
        raise RuntimeError(
            f"HIP decode library not found at {path}; build it with "
            "`python -m flashinfer_competition_codebase_amd.build`"
        )
    try:
        lib = ctypes.CDLL(str(path))
    except OSError as exc:
        raise RuntimeError(f"failed to load HIP decode library {path}: {exc}") from exc
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.gdn_decode_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(
            f"{path} has ABI version {version}, expected {ABI_VERSION}; rebuild it"
        )
    return lib


def get_lib() -> ctypes.CDLL:
    """Process-wide library handle, loaded on first use."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                _lib = load()
    return _lib


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
