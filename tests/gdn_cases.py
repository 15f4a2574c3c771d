"""Shared shapes, tolerances and fixture loading for the decode-step tests."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

GOLDEN = Path(__file__).resolve().parent / "golden" / "gdn_decode_golden.npz"

# Benchmark shapes (B, H, HV, use_qk_l2norm), K = V = 128, T = 1.
CONFIGS = {
    "b1_qk16_v32_l2": (1, 16, 32, True),
    "b8_qk16_v32_l2": (8, 16, 32, True),
    "b64_qk16_v32_l2": (64, 16, 32, True),
    "b256_qk16_v32_l2": (256, 16, 32, True),
    "b128_qk8_v32_raw": (128, 8, 32, False),
}
CONFIG_SEEDS = {name: 1000 + i for i, name in enumerate(CONFIGS)}

# The reference's own decode definition (qk4_v8) at its workload batch sizes.
REF_BATCHES = (1, 4, 8, 16, 32, 48, 64)

# Parity bar for the bf16 output: |o - o_ref| <= ATOL + RTOL * |o_ref|.
OUT_ATOL = 1e-2
OUT_RTOL = 1e-2
# Parity bar for the fp32 state: |S - S_ref| <= STATE_RTOL * |S_ref| + STATE_ATOL.
STATE_RTOL = 1e-3
STATE_ATOL = 1e-5
# Tight bound for the output against a float64 result: within one bf16 ulp
# (2^-8 relative) plus a small absolute slack for values near zero.
OUT_TIGHT_RTOL = 2.0 ** -8
OUT_TIGHT_ATOL = 1e-6


def load_golden() -> dict:
    """Golden cases: name -> (inputs dict of CPU tensors, use_qk_l2norm,
    expected output float64 array, expected new state float32 array)."""
    data = np.load(GOLDEN, allow_pickle=False)
    names = sorted({key.split("/")[0] for key in data.files})
    cases = {}
    for name in names:
        def arr(key):
            return data[f"{name}/{key}"]
        t = {}
        for key in ("q", "k", "v", "a", "b"):
            t[key] = torch.from_numpy(arr(key).astype(np.int16)).view(torch.bfloat16)
        for key in ("state", "A_log", "dt_bias"):
            t[key] = torch.from_numpy(arr(key).astype(np.float32))
        t["scale"] = float(arr("scale"))
        cases[name] = (t, bool(arr("use_qk_l2norm")), arr("expected_output"),
                       arr("expected_new_state"))
    return cases


def assert_output_close(out, ref, *, tight_ref64=None, what="output"):
    """Stated bar against ``ref``; optional one-ulp bar against float64."""
    out = out.detach().float().cpu()
    ref = ref.detach().float().cpu()
    diff = (out - ref).abs()
    bad = diff > OUT_ATOL + OUT_RTOL * ref.abs()
    assert not bool(bad.any()), (
        f"{what}: {int(bad.sum())} elements outside atol/rtol 1e-2, "
        f"max abs diff {diff.max().item():.3e}")
    if tight_ref64 is not None:
        r64 = torch.as_tensor(np.asarray(tight_ref64), dtype=torch.float64)
        d64 = (out.double() - r64).abs()
        lim = OUT_TIGHT_ATOL + OUT_TIGHT_RTOL * r64.abs()
        badt = d64 > lim
        assert not bool(badt.any()), (
            f"{what}: {int(badt.sum())} elements more than one bf16 ulp from the "
            f"float64 result, worst excess {(d64 - lim).max().item():.3e}")


def assert_state_close(st, ref, *, what="new_state"):
    st = st.detach().cpu().double()
    ref = torch.as_tensor(np.asarray(ref) if not isinstance(ref, torch.Tensor) else ref)
    ref = ref.detach().cpu().double()
    diff = (st - ref).abs()
    bad = diff > STATE_RTOL * ref.abs() + STATE_ATOL
    assert not bool(bad.any()), (
        f"{what}: {int(bad.sum())} elements outside 1e-3 relative + 1e-5, "
        f"max abs diff {diff.max().item():.3e}")
    rel = (diff.norm() / ref.norm().clamp_min(1e-30)).item()
    assert rel <= 1e-3, f"{what}: relative Frobenius error {rel:.3e} > 1e-3"
    return rel


def prefill_segment_plan(L: int, N: int, HV: int):
    """The prefill library's segment plan, restated for the workspace-size and
    dispatch-count checks: (segmented, chunks a segment, segments the
    workspace holds).  Sequences of the mean length are cut into segments of
    the length (2 chunks or more, 3 segments or more) minimising (rounds of
    256 workgroups) x length x 5 + combine steps + 8, when that is below the
    plain scan's (rounds of N HV workgroups) x chunks x 5; at most 64
    sequences and N HV <= 256."""
    if N < 1 or N > 64 or N * HV > 256:
        return False, 0, 0
    nch = ((L + 63) // 64 + N - 1) // N

    def cost(n_len):
        n = -(-nch // n_len)
        rounds = -(-N * (2 * n - 3) * HV // 256) + -(-N * n * HV // 256)
        return rounds * n_len * 5 + (n - 2) + 8
    lens = range(2, nch // 3 + 1)
    if len(lens) == 0 or min(map(cost, lens)) >= -(-N * HV // 256) * nch * 5:
        return False, 0, 0
    seg_len = min(lens, key=cost)
    if N == 1:
        return True, seg_len, -(-((L + 63) // 64) // seg_len)
    max_slots = min((L + 63) // 64 + N, L)
    return True, seg_len, (max_slots + N * (seg_len - 1)) // seg_len
