"""MI355X (gfx950) Gated Delta Net decode step behind the reference's entry points.

``run`` is the value-returning form and ``kernel_hip`` the destination-passing
form of the reference's decode entry points (solution/triton/kernel.py:22-197,
solution/cuda/binding.py:35-60).  Both launch one hand-written HIP kernel from
``libgdn_decode.so``; there is no CPU or fallback path.

``ENTRY_POINTS`` and ``NO_DPS`` mirror the reference's algo registry
(scripts/shared.py:19-37): entry name -> callable, and the set of entries that
return their outputs instead of writing caller-allocated ones.
"""

from .kernel import kernel_hip, kernel_hip_shaped, resolve_scale, run

ENTRY_POINTS = {
    "hip": kernel_hip,
    "hip-run": run,
}

NO_DPS = {"hip-run"}

__all__ = ["run", "kernel_hip", "kernel_hip_shaped", "resolve_scale",
           "ENTRY_POINTS", "NO_DPS"]
