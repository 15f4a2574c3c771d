"""Build the gfx950 decode library in-tree with hipcc.

``python -m flashinfer_competition_codebase_amd.build`` compiles
``csrc/gdn_decode.hip`` into ``libgdn_decode.so`` next to this file.  The
library is a plain C-ABI shared object (declared in ``include/gdn_decode.h``)
that the Python host side loads with ctypes.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_ROOT = PKG_DIR.parent
CSRC = PKG_DIR / "csrc" / "gdn_decode.hip"
INCLUDE_DIR = REPO_ROOT / "include"
LIB_NAME = "libgdn_decode.so"
LIB_PATH = PKG_DIR / LIB_NAME
OFFLOAD_ARCH = "gfx950"


def hipcc_path() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if found is None:
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return found


def compile_command(out: Path = LIB_PATH) -> list[str]:
    return [
        hipcc_path(),
        f"--offload-arch={OFFLOAD_ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        # Packed fp32 VALU ops stay disabled in device code.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        f"-I{INCLUDE_DIR}",
        str(CSRC),
        "-o", str(out),
    ]


def build(verbose: bool = False) -> Path:
    """Compile the library (always, even when a built copy exists)."""
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = compile_command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed with exit code {proc.returncode}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
