"""MI355X (gfx950) Gated Delta Net decode step and prefill behind the
reference's entry points.

``run`` is the value-returning form and ``kernel_hip`` the destination-passing
form of the reference's decode entry points (solution/triton/kernel.py:22-197,
solution/cuda/binding.py:35-60).  Both launch one hand-written HIP kernel from
``libgdn_decode.so``.  ``prefill_run`` and ``kernel_prefill_hip`` are the same
two forms of the reference's prefill entry points
(solution/triton/prefill_kernel.py:10-58, 85-183), launching the chunkwise
MFMA kernels of ``libgdn_prefill.so``.  There is no CPU or fallback path.

``ENTRY_POINTS`` and ``NO_DPS`` mirror the reference's algo registry
(scripts/shared.py:19-37, where "prefill-fla-chunk" is DPS and
"prefill-reference" value-returning): entry name -> callable, and the set of
entries that return their outputs instead of writing caller-allocated ones.
"""

from .kernel import kernel_hip, kernel_hip_shaped, resolve_scale, run, run_dps
from .serving import DecodeLayers, DecodePlan
from .prefill import (kernel_prefill_hip, kernel_prefill_hip_noalloc, kernel_prefill_hip_timed,
                      prefill_run)

ENTRY_POINTS = {
    "hip": kernel_hip,
    "hip-run": run,
    "prefill-hip": kernel_prefill_hip,
    "prefill-hip-run": prefill_run,
}

NO_DPS = {"hip-run", "prefill-hip-run"}

__all__ = ["run", "run_dps", "kernel_hip", "kernel_hip_shaped", "resolve_scale", "prefill_run",
           "kernel_prefill_hip", "kernel_prefill_hip_timed", "kernel_prefill_hip_noalloc",
           "DecodePlan", "DecodeLayers", "ENTRY_POINTS", "NO_DPS"]
