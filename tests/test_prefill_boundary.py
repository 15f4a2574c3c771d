"""Prefill boundary on the host: argument validation, the C ABI's exports and
its own validation (no compute call: every native call here is rejected, or
has nothing to launch, before any HIP call)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

import flashinfer_competition_codebase_amd as gdn
from tests.gdn_cases import prefill_segment_plan
from flashinfer_competition_codebase_amd import _lib
from flashinfer_competition_codebase_amd.prefill import check_prefill_inputs
from oracle.gdn_prefill_oracle import make_prefill_inputs

HEADER = Path(__file__).resolve().parents[1] / "include" / "gdn_prefill.h"


def _header_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    protos = re.findall(r"^\s*(?:const\s+)?\w+\*?\s+(gdn_prefill\w*)\s*\(([^;]*?)\)\s*;",
                        text, flags=re.M | re.S)
    return {n: (0 if p.strip() in ("", "void") else p.count(",") + 1) for n, p in protos}


def test_header_and_library_agree():
    funcs = _header_functions()
    assert set(funcs) == {"gdn_prefill_workspace_bytes", "gdn_prefill", "gdn_prefill_timed",
                          "gdn_prefill_noalloc", "gdn_prefill_token_path_max_tokens",
                          "gdn_prefill_dispatches", "gdn_prefill_abi_version"}
    lib = _lib.get_prefill_lib()
    for name, nparams in funcs.items():
        assert hasattr(lib, name)
        assert len(_lib.PREFILL_SIGNATURES[name][1]) == nparams, name
    assert lib.gdn_prefill_abi_version() == _lib.PREFILL_ABI_VERSION


def test_workspace_size_formula():
    lib = _lib.get_prefill_lib()
    # per v-head: T diag(beta) (six 16 x 32 operand blocks, bf16 hi and lo),
    # then eight rows of 64 scales
    vslot = (2 * 6 * 16 * 32 * 2 + 8 * 64 * 4)
    a256 = lambda x: (x + 255) // 256 * 256  # noqa: E731
    for L, N, H, HV in ((6, 1, 4, 8), (16384, 1, 4, 8), (1000, 37, 16, 32), (0, 3, 4, 8),
                        (100, 2, 2, 2), (40, 65600, 1, 1), (3, 10, 4, 8), (3000, 1, 4, 8),
                        (3072, 1, 4, 8), (5000, 1, 16, 16), (8192, 1, 16, 32),
                        (8192, 1, 16, 64), (2048, 1, 4, 8), (384, 1, 4, 8), (320, 1, 4, 8),
                        (1024, 1, 16, 32), (4096, 1, 16, 32), (700, 1, 2, 2),
                        (39503, 8, 4, 8), (3600, 3, 4, 8), (5000, 2, 16, 32), (8192, 8, 16, 32),
                        (20000, 64, 1, 2), (3000, 65, 1, 1), (64, 1, 4, 8), (57, 2, 16, 32),
                        (64, 4, 16, 32), (60, 5, 16, 32), (64, 16, 4, 8), (64, 17, 4, 8)):
        chunks = min((L + 63) // 64 + N, L)          # the most a well-formed batch has
        offs = a256((N + 1) * 4)
        table = a256(chunks * 16)                                        # per-chunk slot table
        want = offs + table + a256(chunks * HV * vslot)
        # segments (at most 64 sequences, N HV <= 256): S, B and M blocks for
        # the segments the workspace holds
        seg, _, nseg = prefill_segment_plan(L, N, HV)
        if seg:
            want += 3 * a256(nseg * HV * 128 * 128 * 4)
        assert lib.gdn_prefill_workspace_bytes(L, N, H, HV) == want, (L, N, H, HV)
        offsets = 0 if N == 1 or (N <= 64 and chunks * HV <= 2048) else 1
        # 2..64 sequences of at most 56 tokens on average: the token kernel first
        token = 1 if 2 <= N <= 64 and 56 < L <= 56 * N else 0
        # at most one chunk in all, half-state workgroups on at most all CUs:
        # the one-chunk kernel alone
        one_chunk = 56 < L <= 64 and 2 * N * HV <= 256
        assert lib.gdn_prefill_dispatches(L, N, HV) == (
            0 if N == 0 else 1 if (L <= 56 and N <= 65535) or one_chunk else
            token + offsets + (4 if seg else 2)), (L, N, HV)
    assert lib.gdn_prefill_workspace_bytes(-1, 1, 4, 8) == 0
    assert lib.gdn_prefill_workspace_bytes(1, 1, 4, 0) == 0
    assert lib.gdn_prefill_workspace_bytes(1, 1, 3, 8) == 0              # HV % H != 0


def test_c_side_validation_rejects_before_launching():
    lib = _lib.get_prefill_lib()
    n = [None] * 8
    f = ctypes.c_float(0.1)

    def call(L=6, N=1, H=4, HV=8, K=128, V=128, ws=None, ws_size=0, cu=None, new_state=None):
        return lib.gdn_prefill(*n, cu, f, None, new_state, L, N, H, HV, K, V, 0, ws, ws_size, None)

    assert call(N=0) == 0                     # nothing to do
    assert call(K=64) == 1
    assert call(H=3) == 1                     # 8 % 3 != 0
    assert call(L=-1) == 1
    assert call() == 1                        # null pointers
    if not torch.cuda.is_available():         # made-up pointers only where no device exists
        assert call(cu=0x1000, new_state=0x2000, ws=0x3000, ws_size=10) == 1   # short workspace
    # the timed entry validates its events before anything else
    assert lib.gdn_prefill_timed(*n, None, f, None, None, 6, 1, 4, 8, 128, 128, 0, None, 0, None,
                                 None) == 1
    ev = (ctypes.c_void_p * 4)(0x10, 0x20, None, 0x40)
    assert lib.gdn_prefill_timed(*n, None, f, None, None, 6, 1, 4, 8, 128, 128, 0, None, 0, None,
                                 ev) == 1
    # the no-allocation entry: the same validation, and sizes whose workspace
    # exceeds its fixed array rejected with hipErrorOutOfMemory before any HIP call
    assert lib.gdn_prefill_noalloc(*n, None, f, None, None, 6, 0, 4, 8, 128, 128, 0, None) == 0
    assert lib.gdn_prefill_noalloc(*n, None, f, None, None, 6, 1, 4, 8, 64, 128, 0, None) == 1
    assert lib.gdn_prefill_noalloc(*n, None, f, None, None, 6, 1, 4, 8, 128, 128, 0, None) == 1
    if not torch.cuda.is_available():         # made-up pointers only where no device exists
        fake = [0x10000 * (i + 1) for i in range(8)]
        big = 1 << 20
        assert lib.gdn_prefill_workspace_bytes(big, 1, 16, 32) > (128 << 20)
        assert lib.gdn_prefill_noalloc(*fake, 0x90000, f, 0xa0000, 0xb0000, big, 1, 16, 32, 128,
                                       128, 0, None) == 2
        # H above 32767 (the token kernel packs it in 15 bits) is refused
        assert lib.gdn_prefill(*fake, 0x90000, f, 0xa0000, 0xb0000, 6, 1, 32768, 32768, 128, 128,
                               0, 0xc0000, 1 << 30, None) == 1


def _cpu_inputs():
    return make_prefill_inputs([3, 2], 4, 8, seed=0)


def test_python_validation():
    t = _cpu_inputs()
    with pytest.raises(ValueError, match="HIP device"):
        check_prefill_inputs(**{k: v for k, v in t.items() if k != "scale"})
    bad = dict(t, q=t["q"].float())
    with pytest.raises(TypeError):
        check_prefill_inputs(**{k: v for k, v in bad.items() if k != "scale"})
    bad = dict(t, v=t["v"][:, :6].contiguous())                   # 6 % 4 != 0
    with pytest.raises(ValueError, match="multiple"):
        check_prefill_inputs(**{k: v for k, v in bad.items() if k != "scale"})
    bad = dict(t, state=t["state"][:1].contiguous())                # N mismatch
    with pytest.raises(ValueError, match="state"):
        check_prefill_inputs(**{k: v for k, v in bad.items() if k != "scale"})
    bad = dict(t, cu_seqlens=t["cu_seqlens"].float())
    with pytest.raises(TypeError, match="cu_seqlens"):
        check_prefill_inputs(**{k: v for k, v in bad.items() if k != "scale"})
    bad = dict(t, a=t["a"].unsqueeze(1))
    with pytest.raises(ValueError, match="a must have shape"):
        check_prefill_inputs(**{k: v for k, v in bad.items() if k != "scale"})


def test_entry_points_are_registered_like_the_reference():
    assert gdn.ENTRY_POINTS["prefill-hip"] is gdn.kernel_prefill_hip
    assert gdn.ENTRY_POINTS["prefill-hip-run"] is gdn.prefill_run
    assert "prefill-hip-run" in gdn.NO_DPS and "prefill-hip" not in gdn.NO_DPS
    with pytest.raises(ValueError):
        gdn.prefill_run(**_cpu_inputs())      # CPU tensors: no CPU path
