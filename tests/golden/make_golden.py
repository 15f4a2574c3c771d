"""Write the committed golden vectors for the GDN decode step.

The reference holds no golden vectors for this path (its workloads live in an
external dataset), so these fixtures are written by the float64 restatement
``oracle.gdn_decode_oracle.brute_fp64`` on seeded inputs and committed as
data: bf16 tensors as uint16 bit patterns, fp32 tensors as float32, expected
outputs as float64 (output) and float32 (new state, rounded from float64).

Run from the repository root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle.gdn_decode_oracle import brute_fp64, make_inputs  # noqa: E402

OUT = Path(__file__).resolve().parent / "gdn_decode_golden.npz"

# name -> (B, H, HV, seed, use_qk_l2norm, gate_shape)
CASES = {
    "b1_qk1_v2_l2norm": (1, 1, 2, 7001, True, "b1hv"),
    "b2_qk1_v1_raw": (2, 1, 1, 7002, False, "bhv"),
}


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def main() -> None:
    arrays = {}
    for name, (B, H, HV, seed, l2, gshape) in CASES.items():
        t = make_inputs(B, H, HV, seed=seed, gate_shape=gshape)
        out, new_state = brute_fp64(**t, use_qk_l2norm=l2)
        for key in ("q", "k", "v", "a", "b"):
            arrays[f"{name}/{key}"] = bf16_bits(t[key])
        for key in ("state", "A_log", "dt_bias"):
            arrays[f"{name}/{key}"] = t[key].numpy().astype(np.float32)
        arrays[f"{name}/scale"] = np.array(t["scale"], dtype=np.float64)
        arrays[f"{name}/use_qk_l2norm"] = np.array(l2)
        arrays[f"{name}/expected_output"] = out.astype(np.float64)
        arrays[f"{name}/expected_new_state"] = new_state.astype(np.float32)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(CASES)} cases)")


if __name__ == "__main__":
    main()
