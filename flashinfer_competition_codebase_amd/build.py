"""Build the gfx950 libraries in-tree with hipcc.

``python -m flashinfer_competition_codebase_amd.build`` compiles, next to
this file:

* ``csrc/gdn_decode.hip`` into ``libgdn_decode.so``: the decode step, a
  plain C-ABI shared object (declared in ``include/gdn_decode.h``) that the
  Python host side loads with ctypes;
* ``csrc/gdn_prefill.hip`` into ``libgdn_prefill.so``: the variable-length
  prefill (declared in ``include/gdn_prefill.h``);
* ``csrc/calib.hip`` into ``libgdn_calib.so``: reference kernels (same-bytes
  read-modify-write, empty kernel) that only ``bench.py`` loads, to report
  the floor of the decode step's traffic.
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
CALIB_SRC = PKG_DIR / "csrc" / "calib.hip"
CALIB_PATH = PKG_DIR / "libgdn_calib.so"
PREFILL_SRC = PKG_DIR / "csrc" / "gdn_prefill.hip"
PREFILL_PATH = PKG_DIR / "libgdn_prefill.so"
# library -> source
LIBRARIES = {LIB_PATH: CSRC, PREFILL_PATH: PREFILL_SRC, CALIB_PATH: CALIB_SRC}
OFFLOAD_ARCH = "gfx950"
# Per-library extra flags.  MFMA results go to VGPRs (the VALU work that
# follows every product then reads them without a v_accvgpr_read copy; in
# the prefill's scan loop those copies were a quarter of the VALU
# instructions, in the block decode kernel a quarter of its instructions).
EXTRA_FLAGS = {PREFILL_PATH: ["-mllvm", "-amdgpu-mfma-vgpr-form"],
               LIB_PATH: ["-mllvm", "-amdgpu-mfma-vgpr-form"]}
KERNARG_PRELOAD_ARGS = int(os.environ.get("GDN_KERNARG_PRELOAD_ARGS", "8"))
# The files each library's kernels are built from (paths from the repository
# root), in the order sources_sha hashes them.
DECODE_SOURCES = ("flashinfer_competition_codebase_amd/csrc/gdn_decode_kernel.h",
                  "flashinfer_competition_codebase_amd/csrc/gdn_decode_block.h",
                  "flashinfer_competition_codebase_amd/csrc/gdn_decode.hip",
                  "flashinfer_competition_codebase_amd/build.py")
PREFILL_SOURCES = ("flashinfer_competition_codebase_amd/csrc/gdn_prefill.hip",
                   "flashinfer_competition_codebase_amd/csrc/gdn_decode_kernel.h",
                   "flashinfer_competition_codebase_amd/build.py")


def sources_sha(paths, root: Path = REPO_ROOT) -> str:
    """SHA-256 (16 hex digits) over the given source files (paths from
    ``root``), in order: the code a measurement was made on."""
    import hashlib

    h = hashlib.sha256()
    for rel in paths:
        h.update(rel.encode())
        h.update((Path(root) / rel).read_bytes())
    return h.hexdigest()[:16]


def hipcc_path() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if found is None:
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return found


def compile_command(out: Path = LIB_PATH, src: Path = CSRC,
                    extra: list[str] | None = None) -> list[str]:
    return [
        hipcc_path(),
        f"--offload-arch={OFFLOAD_ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        # Packed fp32 VALU ops stay disabled in device code.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # The decode kernel's first 8 arguments (14 dwords: the pointers and
        # sizes its first loads need) are preloaded into SGPRs at dispatch.
        "-mllvm", f"-amdgpu-kernarg-preload-count={KERNARG_PRELOAD_ARGS}",
        "-Wall",
        *(extra or []),
        f"-I{INCLUDE_DIR}",
        str(src),
        "-o", str(out),
    ]


def build(verbose: bool = False) -> Path:
    """Compile every library (always, even when built copies exist), in
    parallel; returns the decode library's path."""
    jobs = []
    for lib, src in LIBRARIES.items():
        tmp = lib.with_suffix(".so.tmp")
        cmd = compile_command(tmp, src, EXTRA_FLAGS.get(lib))
        if verbose:
            print(" ".join(cmd), flush=True)
        jobs.append((lib, tmp, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                                stderr=subprocess.STDOUT, text=True)))
    failed = []
    for lib, tmp, proc in jobs:
        out, _ = proc.communicate()
        if proc.returncode != 0:
            sys.stderr.write(out)
            failed.append(f"{lib.name} (exit code {proc.returncode})")
        else:
            os.replace(tmp, lib)
    if failed:
        raise RuntimeError("hipcc failed: " + ", ".join(failed))
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
