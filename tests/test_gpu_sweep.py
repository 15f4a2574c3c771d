"""Seeded random sweeps of the decode step and the prefill on MI355X against
the oracle, across the options the named tests take one at a time: batch,
tokens per sequence, q/k heads and GVA ratio, fp32 / bf16 / no initial
state, the q/k L2-norm, the entry form (DPS in place, DPS out of place,
value-returning), the scale's forms and, for the prefill, ragged sequence
lengths with empty sequences on either side of the 56-token path switch.

Bars are those of the named tests (tests/gdn_cases.py, test_gpu_tokens.py,
test_gpu_prefill.py): outputs within 1e-2 atol/rtol of the oracle's bf16
output and one bf16 ulp of float64; bf16 states within one bf16 ulp of the
oracle's bf16 state and the round-to-nearest of the float64 state; fp32
states within 1e-3 relative of the float64 state element by element, with
the absolute floor 1e-5 scaled by the head's largest magnitude when that
exceeds 1 (raw N(0,1) keys, |k|^2 ~ 128, multiply a state's k-component by
~|1 - 128 beta| per token, so after a few tokens entries of 1e3-1e4 make
one fp32 rounding ~1e-3 and an entry that cancels to near zero cannot meet
a fixed 1e-5), and within 1e-3 in relative Frobenius norm.

Two more sweeps reach the sizes the first two keep clear of: decode batches
up to 256 (the launch-shape table's larger rows, the XCD-grouped launches,
the block kernel) at up to 8 tokens, and prefills of up to 100 sequences
(the chunk-offsets scan) and up to 1500 tokens a sequence (segments), at up
to 32 v-heads, and ragged batches of 57 to 64 tokens in all through the
one-chunk kernel, bit for bit against the chunkwise kernels.  The larger
decode sweep's keys are raw N(0, 1) rows only for single
tokens: over several tokens without the L2-norm they are scaled to unit norm
first (the normalisation the model applies before this step; raw keys grow
the state to 400-1400 within 2 to 4 tokens, where the fp32 oracle itself
misses a 1e-4 absolute bar against the float64 result), and their fp32
states meet both the oracle's bar (1e-3 relative + 1e-5) and 1e-4 absolute
against float64.
"""

from __future__ import annotations

import math
import random
import sys

import numpy as np
import pytest
import torch

import flashinfer_competition_codebase_amd as gdn
from flashinfer_competition_codebase_amd import _lib
from oracle.gdn_decode_oracle import make_inputs, oracle_loop, oracle_tokens, oracle_vec
from oracle.gdn_prefill_oracle import make_prefill_inputs, prefill_chunked_fp64, prefill_loop
from tests.gdn_cases import assert_output_close, assert_state_close

pytestmark = pytest.mark.gpu


def _announce(case):
    sys.stdout.write(f"[gpu case] {case}\n")
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _libraries_present():
    _lib.get_lib()
    _lib.get_prefill_lib()


def _dev(t, device):
    return {n: (x.to(device) if isinstance(x, torch.Tensor) else x) for n, x in t.items()}


def _assert_fp32_state(st, s64):
    sd = st.double()
    ref = torch.as_tensor(np.asarray(s64), dtype=torch.float64)
    scale = ref.abs().amax(dim=(-1, -2), keepdim=True).clamp_min(1.0)   # per head
    diff = (sd - ref).abs()
    bad = diff > 1e-3 * ref.abs() + 1e-5 * scale
    assert not bool(bad.any()), (f"{int(bad.sum())} state elements off, max diff "
                                 f"{diff.max().item():.3e} (head scale {scale.max().item():.3e})")
    rel = (diff.norm() / ref.norm().clamp_min(1e-30)).item()
    assert rel <= 1e-3, rel


def _decode_cases(n=48, seed=20261202):
    rng = random.Random(seed)
    cases = []
    for i in range(n):
        H = rng.choice([1, 2, 3, 4, 6, 8, 16])
        ratio = rng.choice([1, 2, 3, 4, 8])
        while H * ratio > 64:
            ratio //= 2
        cases.append(dict(
            i=i, B=rng.randint(1, 40), T=rng.choice([1, 1, 1, 2, 3, 5]), H=H, HV=H * ratio,
            state=rng.choices(["fp32", "bf16", "none"], weights=[6, 3, 2])[0],
            l2=rng.random() < 0.5, form=rng.choice(["inplace", "outofplace", "run"]),
            scale=rng.choice(["none", "zero", "float", "tensor"]),
            gates_bhv=rng.random() < 0.3, seed=30_000 + i))
    return cases


def _case_id(c):
    return (f"{c['i']:02d}-B{c['B']}-T{c['T']}-qk{c['H']}v{c['HV']}-{c['state']}-"
            f"{'l2' if c['l2'] else 'raw'}-{c['form']}")


def _scale_arg(kind, K=128):
    return {"none": None, "zero": 0, "float": 1.0 / math.sqrt(K),
            "tensor": torch.tensor(1.0 / math.sqrt(K))}[kind]


@pytest.mark.parametrize("c", _decode_cases(), ids=_case_id)
def test_decode_sweep(c, hip_device):
    _announce(f"decode sweep {_case_id(c)}")
    B, T, H, HV, l2 = c["B"], c["T"], c["H"], c["HV"], c["l2"]
    gate_shape = "bhv" if (c["gates_bhv"] and T == 1) else "b1hv"
    t = make_inputs(B, H, HV, seed=c["seed"], T=T, gate_shape=gate_shape)
    state_dtype = {"fp32": torch.float32, "bf16": torch.bfloat16, "none": None}[c["state"]]
    if state_dtype is None:
        t["state"] = None
    elif state_dtype == torch.bfloat16:
        t["state"] = t["state"].to(torch.bfloat16)
    t["scale"] = _scale_arg(c["scale"])
    td = _dev(t, hip_device)

    if c["form"] == "run":
        out, st = gdn.run(**td, use_qk_l2norm=l2)
        if td["state"] is not None:                 # value-returning: state untouched
            assert torch.equal(td["state"].cpu(), t["state"])
    else:
        out = torch.empty(B, T, HV, 128, dtype=torch.bfloat16, device=hip_device)
        sd = torch.float32 if state_dtype is None else state_dtype
        if c["form"] == "inplace" and td["state"] is not None:
            st = td["state"]
        else:
            st = torch.empty(B, HV, 128, 128, dtype=sd, device=hip_device)
        gdn.kernel_hip(**td, output=out, new_state=st, use_qk_l2norm=l2)
    torch.cuda.synchronize()

    tf = {**t, "state": None if t["state"] is None else t["state"].float(),
          "a": t["a"].view(B, T, HV), "b": t["b"].view(B, T, HV)}  # [B, HV] gates at T=1
    step = oracle_loop if B * HV <= 128 else oracle_vec
    ref_o, ref_s = oracle_tokens(step, **tf, use_qk_l2norm=l2,
                                 state_dtype=state_dtype or torch.float32)

    def vec64(*args, **kw):
        return oracle_vec(*args, **kw, output_fp32=True, dtype=torch.float64)

    o64, s64 = oracle_tokens(vec64, **tf, use_qk_l2norm=l2, state_dtype=None)
    assert out.shape == (B, T, HV, 128)
    assert_output_close(out.cpu(), ref_o, tight_ref64=o64, what="output")
    if state_dtype == torch.bfloat16:
        assert st.dtype == torch.bfloat16
        sc = st.cpu().double()
        d_ref = (sc - ref_s.double()).abs()
        assert bool((d_ref <= 2.0 ** -7 * ref_s.double().abs() + 1e-6).all())
        assert bool(((sc - s64).abs() <= 2.0 ** -8 * s64.abs() + 1e-6).all())
    else:
        assert st.dtype == torch.float32
        _assert_fp32_state(st.cpu(), s64)


def _prefill_cases(n=24, seed=77001):
    rng = random.Random(seed)
    cases = []
    for i in range(n):
        N = rng.randint(1, 12)
        small = rng.random() < 0.3                    # total <= 56: the token path
        if small:
            lens = [rng.randint(0, 12) for _ in range(N)]
            while sum(lens) > 56:
                lens[rng.randrange(N)] = 0
        else:
            lens = [rng.choice([0, rng.randint(1, 20), rng.randint(20, 140)]) for _ in range(N)]
            if sum(lens) <= 56:
                lens[0] += 57
        H = rng.choice([1, 2, 4, 8])
        cases.append(dict(i=i, lens=lens, H=H, HV=H * rng.choice([1, 2, 4]),
                          l2=rng.random() < 0.4, with_state=rng.random() < 0.8,
                          inplace=rng.random() < 0.5, seed=40_000 + i))
    return cases


def _pf_id(c):
    return f"{c['i']:02d}-N{len(c['lens'])}-L{sum(c['lens'])}-qk{c['H']}v{c['HV']}"


@pytest.mark.parametrize("c", _prefill_cases(), ids=_pf_id)
def test_prefill_sweep(c, hip_device):
    _announce(f"prefill sweep {_pf_id(c)} lens={c['lens']}")
    lens, H, HV, l2 = c["lens"], c["H"], c["HV"], c["l2"]
    t = make_prefill_inputs(lens, H, HV, seed=c["seed"], with_state=c["with_state"])
    td = _dev(t, hip_device)
    L, N = sum(lens), len(lens)
    if c["inplace"] and td["state"] is not None:
        out = torch.empty(L, HV, 128, dtype=torch.bfloat16, device=hip_device)
        st = td["state"]
        gdn.kernel_prefill_hip(**td, output=out, new_state=st, use_qk_l2norm=l2)
    else:
        out, st = gdn.prefill_run(**td, use_qk_l2norm=l2)
    torch.cuda.synchronize()
    out, st = out.cpu(), st.cpu()
    o64, s64 = prefill_chunked_fp64(**t, use_qk_l2norm=l2)
    of = out.double().numpy()
    assert np.all(np.isfinite(of))
    assert np.all(np.abs(of - o64) <= 2.0 ** -7 * np.abs(o64) + 1e-5)
    if L <= 400:
        ref_o, _ = prefill_loop(**t, use_qk_l2norm=l2)
        dl = (out.float() - ref_o.float()).abs()
        assert bool((dl <= 1e-2 + 1e-2 * ref_o.float().abs()).all())
    sd = st.double().numpy()
    assert np.all(np.abs(sd - s64) <= 1e-3 * np.abs(s64) + 1e-5)
    for s, n in enumerate(lens):                      # empty sequences: zero state
        if n == 0:
            assert torch.count_nonzero(st[s]) == 0


# (q/k heads, v-heads) of the larger sweeps
_HEADS = [(1, 1), (1, 4), (2, 4), (3, 12), (4, 8), (5, 15), (8, 32), (16, 32), (2, 16), (4, 4)]


def _bf16_state_ok(st, ref_s, s64):
    sc = st.cpu().double()
    d_ref = (sc - ref_s.double()).abs()
    assert bool((d_ref <= 2.0 ** -7 * ref_s.double().abs() + 1e-6).all()), "beyond one bf16 ulp"
    assert (d_ref > 0).double().mean().item() <= 1e-3, "too many elements off the oracle's"
    assert bool(((sc - s64).abs() <= 2.0 ** -8 * s64.abs() + 1e-6).all()), "not the RNE"


def _large_decode_case(i):
    r = random.Random(9100 + i)
    H, HV = r.choice(_HEADS)
    l2 = r.random() < 0.6
    T = r.choice([1, 1, 1, 2, 3, 4, 5, 8])
    bf16 = r.random() < 0.3
    B = r.choice([1, 2, 3, 5, 8, 17, 33, 64, 100, 128, 129, 200, 256])
    while B * HV > 4096:
        B //= 2
    return B, H, HV, T, l2, bf16, r.random() < 0.5


@pytest.mark.parametrize("i", range(24))
def test_decode_sweep_large_batches(i, hip_device):
    B, H, HV, T, l2, bf16, in_place = _large_decode_case(i)
    _announce(f"decode sweep, large batches {i}: B={B} H={H} HV={HV} T={T} l2={l2} "
              f"bf16={bf16} in_place={in_place}")
    t = make_inputs(B, H, HV, seed=9200 + i, T=T)
    if T > 1 and not l2:
        for n in ("q", "k"):
            x = t[n].float()
            t[n] = (x / x.norm(dim=-1, keepdim=True).clamp_min(1e-6)).to(torch.bfloat16)
    sd = torch.bfloat16 if bf16 else torch.float32
    t["state"] = t["state"].to(sd)
    td = _dev(t, hip_device)
    if in_place:
        out = torch.empty(B, T, HV, 128, dtype=torch.bfloat16, device=hip_device)
        st = td["state"].clone()
        gdn.kernel_hip(**{**td, "state": st}, output=out, new_state=st, use_qk_l2norm=l2)
    else:
        out, st = gdn.run(**td, use_qk_l2norm=l2)
    torch.cuda.synchronize()
    step = oracle_loop if B * HV <= 256 else oracle_vec
    ref_o, ref_s = oracle_tokens(step, **t, use_qk_l2norm=l2, state_dtype=sd)

    def vec64(*args, **kw):
        return oracle_vec(*args, **kw, output_fp32=True, dtype=torch.float64)

    o64, s64 = oracle_tokens(vec64, **t, use_qk_l2norm=l2, state_dtype=None)
    assert_output_close(out.cpu(), ref_o, tight_ref64=o64, what="output")
    if bf16:
        _bf16_state_ok(st, ref_s, s64)
    else:
        assert_state_close(st.cpu(), ref_s)
        assert (st.cpu().double() - s64).abs().max().item() < 1e-4


def _long_prefill_case(i):
    r = random.Random(9300 + i)
    H, HV = r.choice(_HEADS[:7] + [(2, 16)])
    N = r.choice([1, 1, 2, 3, 5, 8, 16, 40, 64, 65, 100])
    longest = r.choice([8, 56, 64, 130, 300, 1500])
    lens = [r.choice([0, 1, r.randint(1, longest)]) if r.random() < 0.2 else r.randint(1, longest)
            for _ in range(N)]
    while sum(lens) * HV > 24000:
        lens = [x // 2 for x in lens]
    return lens, H, HV, r.random() < 0.5, r.random() < 0.8


@pytest.mark.parametrize("i", range(24))
def test_prefill_sweep_many_and_long_sequences(i, hip_device):
    lens, H, HV, l2, with_state = _long_prefill_case(i)
    _announce(f"prefill sweep, many and long sequences {i}: N={len(lens)} L={sum(lens)} "
              f"longest={max(lens)} H={H} HV={HV} l2={l2} state={with_state}")
    t = make_prefill_inputs(lens, H, HV, seed=9400 + i, with_state=with_state)
    out, st = gdn.prefill_run(**_dev(t, hip_device), use_qk_l2norm=l2)
    torch.cuda.synchronize()
    out, st = out.cpu(), st.cpu()
    o64, s64 = prefill_chunked_fp64(**t, use_qk_l2norm=l2)
    of = out.double().numpy()
    assert np.all(np.isfinite(of))
    d64 = np.abs(of - o64)
    assert np.all(d64 <= 2.0 ** -7 * np.abs(o64) + 1e-5), f"output vs fp64: max {d64.max():.3e}"
    if sum(lens) * HV <= 2400:
        ref_o, _ = prefill_loop(**t, use_qk_l2norm=l2)
        dl = (out.float() - ref_o.float()).abs()
        assert bool((dl <= 1e-2 + 1e-2 * ref_o.float().abs()).all()), f"output vs loop {dl.max()}"
    sd = st.double().numpy()
    ds = np.abs(sd - s64)
    assert np.all(ds <= 1e-3 * np.abs(s64) + 1e-5), f"state vs fp64: max {ds.max():.3e}"
    rel = np.linalg.norm(sd - s64) / max(np.linalg.norm(s64), 1e-30)
    assert rel <= 1e-4, rel


@pytest.mark.parametrize("N,longest,H,HV,seed", [(1000, 20, 3, 6, 56004), (2000, 8, 4, 8, 56008)])
def test_prefill_thousands_of_sequences(N, longest, H, HV, seed, hip_device):
    """Thousands of short sequences (a tenth of them empty): the chunk-offsets
    scan over all of them and thousands of scan workgroups."""
    _announce(f"prefill of {N} sequences of at most {longest} tokens, H={H} HV={HV}")
    r = random.Random(seed)
    lens = [0 if r.random() < 0.1 else r.randint(1, longest) for _ in range(N)]
    t = make_prefill_inputs(lens, H, HV, seed=seed)
    out, st = gdn.prefill_run(**_dev(t, hip_device))
    torch.cuda.synchronize()
    o64, s64 = prefill_chunked_fp64(**t)
    of = out.cpu().double().numpy()
    d64 = np.abs(of - o64)
    assert np.all(d64 <= 2.0 ** -7 * np.abs(o64) + 1e-5), f"output vs fp64: max {d64.max():.3e}"
    sd = st.cpu().double().numpy()
    ds = np.abs(sd - s64)
    assert np.all(ds <= 1e-3 * np.abs(s64) + 1e-5), f"state vs fp64: max {ds.max():.3e}"
    for s, n in enumerate(lens):
        if n == 0:
            assert not np.any(sd[s])


def _one_chunk_case(i):
    r = random.Random(88000 + i)
    H, HV = r.choice([(1, 1), (1, 4), (2, 4), (4, 8), (3, 12), (2, 16), (8, 32), (16, 32), (1, 8)])
    while True:
        N = r.randint(1, 16)
        if 2 * N * HV <= 256:
            break
    L = r.randint(57, 64)
    cuts = sorted(r.randint(0, L) for _ in range(N - 1))
    return [b - a for a, b in zip([0] + cuts, cuts + [L])], H, HV, r.random() < 0.5, r.random() < 0.8


@pytest.mark.parametrize("i", range(24))
def test_one_chunk_sweep(i, hip_device):
    """Ragged batches of 57..64 tokens in all (empty sequences among them):
    the one-chunk kernel against the float64 oracle, and bit for bit against
    the chunkwise kernels, which run the same batch with a 65-token sequence
    appended."""
    lens, H, HV, l2, with_state = _one_chunk_case(i)
    L, N = sum(lens), len(lens)
    _announce(f"one-chunk sweep {i}: lens={lens} H={H} HV={HV} l2={l2} state={with_state}")
    assert gdn.prefill.prefill_dispatches(L, N, HV) == 1
    t = make_prefill_inputs(lens + [65], H, HV, seed=89000 + i, with_state=with_state)
    tb = {**t, "q": t["q"][:L], "k": t["k"][:L], "v": t["v"][:L], "a": t["a"][:L],
          "b": t["b"][:L], "state": None if t["state"] is None else t["state"][:N],
          "cu_seqlens": t["cu_seqlens"][:N + 1]}
    out1, st1 = gdn.prefill_run(**_dev(tb, hip_device), use_qk_l2norm=l2)
    out_c, st_c = gdn.prefill_run(**_dev(t, hip_device), use_qk_l2norm=l2)
    torch.cuda.synchronize()
    o64, s64 = prefill_chunked_fp64(**tb, use_qk_l2norm=l2)
    d64 = np.abs(out1.cpu().double().numpy() - o64)
    assert np.all(d64 <= 2.0 ** -7 * np.abs(o64) + 1e-5), f"output vs fp64: max {d64.max():.3e}"
    ds = np.abs(st1.cpu().double().numpy() - s64)
    assert np.all(ds <= 1e-3 * np.abs(s64) + 1e-5), f"state vs fp64: max {ds.max():.3e}"
    assert torch.equal(out1, out_c[:L]) and torch.equal(st1, st_c[:N])
