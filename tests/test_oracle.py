"""Pin the CPU oracle (oracle/gdn_decode_oracle.py) without the reference.

The reference ships no golden vectors for the decode step, so each part of
the oracle is pinned by what the mathematics fixes: closed forms for the
gates, a one-hot known answer for the k-last layout
(solution/triton/kernel.py:101,114), the delta rule's write/read identity,
pure decay at beta = 0, the zero-state closed form (kernel.py:83-86), the
GVA repeat-interleave invariant (kernel.py:88-89), linearity in q, scale
invariance of the L2-norm, scalar brute force on tiny shapes, and agreement
of three independent restatements.  ``test_mutants_are_caught`` plants one
plausible mistake at a time in a batched restatement and requires that at
least one of the closed-form checks rejects it.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle.gdn_decode_oracle import (
    brute_fp64, gates, l2norm, make_inputs, oracle_loop, oracle_tokens, oracle_vec,
    resolve_scale)
from tests.gdn_cases import (
    OUT_TIGHT_ATOL, OUT_TIGHT_RTOL, assert_state_close, load_golden)

NEG_INF = float("-inf")
POS_INF = float("inf")


# --------------------------------------------------------------------------
# Implementations under test: every oracle entry, returning fp32-or-better
# (output, new_state) tensors.
# --------------------------------------------------------------------------

def _loop(**t):
    return oracle_loop(**t, output_fp32=True)


def _vec(**t):
    return oracle_vec(**t, output_fp32=True)


def _vec64(**t):
    return oracle_vec(**t, output_fp32=True, dtype=torch.float64)


def _brute(**t):
    o, s = brute_fp64(**t)
    return torch.from_numpy(o), torch.from_numpy(s)


IMPLS = {"loop": _loop, "vec": _vec, "vec64": _vec64, "brute": _brute}


def _mutant(kind):
    """Batched float64 step with one planted mistake (``kind=None``: none)."""
    def impl(q, k, v, state, A_log, a, dt_bias, b, scale, *, use_qk_l2norm=False):
        B, _, H, K = q.shape
        HV, V = v.shape[2], v.shape[3]
        r = HV // H
        scale = resolve_scale(scale, K)
        g, beta = gates(A_log, a, dt_bias, b)
        g = g.reshape(B, HV).double()
        beta = beta.reshape(B, HV).double()
        if kind == "no_decay":
            g = torch.ones_like(g)
        if kind == "beta_swapped":
            beta = 1 - beta
        qf, kf, vf = q[:, 0].double(), k[:, 0].double(), v[:, 0].double()
        if use_qk_l2norm:
            qf, kf = l2norm(qf), l2norm(kf)
        if kind == "gva_tiled":
            qe, ke = qf.repeat(1, r, 1), kf.repeat(1, r, 1)
        else:
            qe, ke = qf.repeat_interleave(r, 1), kf.repeat_interleave(r, 1)
        S = torch.zeros(B, HV, V, K, dtype=torch.float64) if state is None else state.double()
        if kind == "transposed":
            S = S.transpose(-1, -2)
        Sg = g[..., None, None] * S
        old_v = (Sg @ ke[..., None])[..., 0]
        d = beta[..., None] * (vf - old_v)
        if kind == "sign":
            d = beta[..., None] * (old_v - vf)
        Sn = Sg + d[..., :, None] * ke[..., None, :]
        src = Sg if kind == "old_state_output" else Sn
        out = scale * (src @ qe[..., None])[..., 0]
        if kind == "no_scale":
            out = out / scale
        if kind == "transposed":
            Sn = Sn.transpose(-1, -2)
        return out[:, None], Sn
    return impl


MUTANTS = ["transposed", "sign", "no_decay", "beta_swapped", "gva_tiled",
           "old_state_output", "no_scale"]


# --------------------------------------------------------------------------
# Closed-form checks, each usable against any implementation.
# --------------------------------------------------------------------------

def _f64(x):
    return torch.as_tensor(x).double()


def check_layout_known_answer(impl):
    """One-hot state at storage (v=3, k=5), g = 1, beta = 0, q = e_5:
    the output is ``scale`` at v = 3 only and the state is unchanged."""
    K = V = 8
    t = make_inputs(1, 1, 1, seed=11, K=K, V=V)
    state = torch.zeros(1, 1, V, K)
    state[0, 0, 3, 5] = 1.0
    q = torch.zeros(1, 1, 1, K, dtype=torch.bfloat16)
    q[0, 0, 0, 5] = 1.0
    t.update(state=state, q=q, A_log=torch.tensor([NEG_INF]),
             b=torch.full((1, 1, 1), NEG_INF, dtype=torch.bfloat16), scale=0.5)
    out, new_state = impl(**t)
    expect = torch.zeros(V, dtype=torch.float64)
    expect[3] = 0.5
    assert torch.allclose(_f64(out).reshape(V), expect, atol=1e-7), "layout: output"
    assert torch.allclose(_f64(new_state), _f64(state), atol=1e-7), "layout: state"


def check_write_read(impl):
    """beta = 1, L2-normed q = k: the step stores v at key k, so
    ``S_new k_hat = v`` and ``o = scale * v``."""
    t = make_inputs(2, 2, 4, seed=12)
    t["k"] = t["q"].clone()
    t["b"] = torch.full_like(t["b"], POS_INF)
    out, new_state = impl(**t, use_qk_l2norm=True)
    k_hat = l2norm(t["k"][:, 0].double()).repeat_interleave(2, 1)
    v = t["v"][:, 0].double()
    read = (_f64(new_state) @ k_hat[..., None])[..., 0]
    assert torch.allclose(read, v, atol=2e-5), "write/read: S_new k != v"
    assert torch.allclose(_f64(out)[:, 0], t["scale"] * v, atol=2e-6), "write/read: o != scale v"


def check_pure_decay(impl):
    """beta = 0: ``S_new = g S`` and ``o = scale * g * S q`` with g from the
    closed form exp(-exp(A_log) * log(1 + exp(a + dt_bias)))."""
    t = make_inputs(2, 2, 4, seed=13)
    t["b"] = torch.full_like(t["b"], NEG_INF)
    out, new_state = impl(**t)
    B, HV = 2, 4
    g = torch.empty(B, HV, dtype=torch.float64)
    for bi in range(B):
        for hv in range(HV):
            x = float(t["a"][bi, 0, hv]) + float(t["dt_bias"][hv])
            sp = x if x > 20.0 else math.log1p(math.exp(x))
            g[bi, hv] = math.exp(-math.exp(float(t["A_log"][hv])) * sp)
    S = t["state"].double()
    expect_state = g[..., None, None] * S
    q = t["q"][:, 0].double().repeat_interleave(2, 1)
    expect_out = t["scale"] * (expect_state @ q[..., None])[..., 0]
    assert torch.allclose(_f64(new_state), expect_state, rtol=2e-5, atol=1e-7), "decay: state"
    assert torch.allclose(_f64(out)[:, 0], expect_out, rtol=2e-5, atol=1e-7), "decay: output"


def check_zero_state(impl):
    """state = None: ``S_new[r, :] = beta v_r k_hat`` and
    ``o_r = scale * beta * v_r * (k_hat . q_hat)``."""
    t = make_inputs(2, 2, 4, seed=14)
    t["state"] = None
    out, new_state = impl(**t, use_qk_l2norm=True)
    beta = torch.sigmoid(t["b"].double()).reshape(2, 4)
    q_hat = l2norm(t["q"][:, 0].double()).repeat_interleave(2, 1)
    k_hat = l2norm(t["k"][:, 0].double()).repeat_interleave(2, 1)
    v = t["v"][:, 0].double()
    u = beta[..., None] * v
    expect_state = u[..., :, None] * k_hat[..., None, :]
    expect_out = t["scale"] * u * (k_hat * q_hat).sum(-1, keepdim=True)
    assert torch.allclose(_f64(new_state), expect_state, rtol=1e-5, atol=1e-7), "zero: state"
    assert torch.allclose(_f64(out)[:, 0], expect_out, rtol=1e-5, atol=1e-7), "zero: output"


def check_gva(impl):
    """GVA: with HV = 2H, the step equals the step on q, k repeat-interleaved
    to HV heads (v-head hv reads q/k head hv // 2)."""
    t = make_inputs(2, 2, 4, seed=15)
    out_g, st_g = impl(**t)
    t2 = dict(t)
    t2["q"] = t["q"].repeat_interleave(2, dim=2)
    t2["k"] = t["k"].repeat_interleave(2, dim=2)
    out_e, st_e = impl(**t2)
    assert torch.allclose(_f64(out_g), _f64(out_e), atol=1e-7), "gva: output"
    assert torch.allclose(_f64(st_g), _f64(st_e), atol=1e-7), "gva: state"


CHECKS = [check_layout_known_answer, check_write_read, check_pure_decay,
          check_zero_state, check_gva]


@pytest.mark.parametrize("impl_name", list(IMPLS))
@pytest.mark.parametrize("check", CHECKS, ids=lambda c: c.__name__)
def test_oracle_passes_closed_form_checks(impl_name, check):
    check(IMPLS[impl_name])


def test_unmutated_batched_step_passes():
    for check in CHECKS:
        check(_mutant(None))


@pytest.mark.parametrize("kind", MUTANTS)
def test_mutants_are_caught(kind):
    failures = []
    for check in CHECKS:
        try:
            check(_mutant(kind))
        except AssertionError as exc:
            failures.append(f"{check.__name__}: {exc}")
    assert failures, f"no closed-form check rejects the '{kind}' mistake"


# --------------------------------------------------------------------------
# Gates, L2-norm, linearity.
# --------------------------------------------------------------------------

def test_gates_closed_forms():
    A_log = torch.tensor([0.0, math.log(16.0), NEG_INF, 1.0, -3.0])
    a = torch.tensor([[0.0, 25.0, 3.0, -30.0, 20.0]], dtype=torch.bfloat16)
    dt = torch.tensor([0.5, 0.0, 0.0, 0.25, 0.0])
    b = torch.tensor([[0.0, 40.0, -40.0, POS_INF, NEG_INF]], dtype=torch.bfloat16)
    g, beta = gates(A_log, a, dt, b)
    for i in range(5):
        x = float(a[0, i]) + float(dt[i])
        sp = x if x > 20.0 else math.log1p(math.exp(x))
        expect_g = math.exp(-math.exp(float(A_log[i])) * sp)
        assert math.isclose(float(g[0, i]), expect_g, rel_tol=2e-6, abs_tol=1e-30), i
        expect_beta = 1.0 / (1.0 + math.exp(-float(b[0, i])))
        assert math.isclose(float(beta[0, i]), expect_beta, rel_tol=1e-6, abs_tol=1e-30), i
    assert float(g[0, 2]) == 1.0          # A_log = -inf: no decay
    assert float(beta[0, 0]) == 0.5       # b = 0
    assert float(beta[0, 3]) == 1.0 and float(beta[0, 4]) == 0.0
    # softplus above the threshold is the identity: x = 25 exactly
    assert float(g[0, 1]) == pytest.approx(math.exp(-16.0 * 25.0), rel=1e-5, abs=1e-38)


def test_l2norm_closed_form_and_scale_invariance():
    x = torch.tensor([[3.0, 4.0]])
    assert torch.allclose(l2norm(x, eps=0.0), torch.tensor([[0.6, 0.8]]))
    t = make_inputs(2, 2, 4, seed=16)
    base_o, base_s = oracle_vec(**t, use_qk_l2norm=True, output_fp32=True, dtype=torch.float64)
    t2 = dict(t)
    t2["q"] = (t["q"].float() * 4.0).to(torch.bfloat16)    # powers of two: exact in bf16
    t2["k"] = (t["k"].float() * 0.25).to(torch.bfloat16)
    o2, s2 = oracle_vec(**t2, use_qk_l2norm=True, output_fp32=True, dtype=torch.float64)
    # eps / |k|^2 ~ 1e-7 is the only difference
    assert torch.allclose(o2, base_o, rtol=1e-5, atol=1e-8)
    assert torch.allclose(s2, base_s, rtol=1e-5, atol=1e-7)


def test_output_linear_in_q():
    gen = torch.Generator().manual_seed(17)
    t = make_inputs(2, 2, 4, seed=17)
    q1 = torch.randint(-2, 3, t["q"].shape, generator=gen).to(torch.bfloat16)
    q2 = torch.randint(-2, 3, t["q"].shape, generator=gen).to(torch.bfloat16)
    o1, _ = oracle_vec(**{**t, "q": q1}, output_fp32=True, dtype=torch.float64)
    o2, _ = oracle_vec(**{**t, "q": q2}, output_fp32=True, dtype=torch.float64)
    o12, _ = oracle_vec(**{**t, "q": (q1.float() + q2.float()).to(torch.bfloat16)},
                        output_fp32=True, dtype=torch.float64)
    assert torch.allclose(o12, o1 + o2, atol=1e-12)


def test_tiny_scalar_brute_force():
    """K = 3, V = 2 with plain Python floats, written from the recurrence."""
    K, V, B, H, HV = 3, 2, 1, 1, 2
    t = make_inputs(B, H, HV, seed=18, K=K, V=V)
    out, st = oracle_loop(**t, output_fp32=True)
    for hv in range(HV):
        x = float(t["a"][0, 0, hv]) + float(t["dt_bias"][hv])
        g = math.exp(-math.exp(float(t["A_log"][hv])) * math.log1p(math.exp(x)))
        beta = 1.0 / (1.0 + math.exp(-float(t["b"][0, 0, hv])))
        kv = [float(t["k"][0, 0, 0, i]) for i in range(K)]
        qv = [float(t["q"][0, 0, 0, i]) for i in range(K)]
        for r in range(V):
            srow = [g * float(t["state"][0, hv, r, i]) for i in range(K)]
            old = sum(srow[i] * kv[i] for i in range(K))
            d = beta * (float(t["v"][0, 0, hv, r]) - old)
            srow = [srow[i] + d * kv[i] for i in range(K)]
            o = t["scale"] * sum(srow[i] * qv[i] for i in range(K))
            assert math.isclose(float(out[0, 0, hv, r]), o, rel_tol=1e-5, abs_tol=1e-6)
            for i in range(K):
                assert math.isclose(float(st[0, hv, r, i]), srow[i], rel_tol=1e-5, abs_tol=1e-6)


# --------------------------------------------------------------------------
# Agreement of the restatements, contract details, golden vectors.
# --------------------------------------------------------------------------

@pytest.mark.parametrize("H,HV", [(1, 1), (2, 4), (1, 4), (4, 4)])
@pytest.mark.parametrize("l2", [False, True])
def test_restatements_agree(H, HV, l2):
    t = make_inputs(2, H, HV, seed=19 + H + HV)
    o64, s64 = brute_fp64(**t, use_qk_l2norm=l2)
    for name in ("loop", "vec"):
        o, s = IMPLS[name](**t, use_qk_l2norm=l2)
        d = (o.double() - torch.from_numpy(o64)).abs()
        assert bool((d <= 1e-6 + 1e-5 * torch.from_numpy(o64).abs()).all()), name
        assert_state_close(s, s64, what=name)
        assert (s.double() - torch.from_numpy(s64)).abs().max().item() < 2e-6, name


def test_oracle_leaves_state_untouched_and_none_is_zeros():
    t = make_inputs(1, 1, 2, seed=20)
    before = t["state"].clone()
    oracle_loop(**t)
    assert torch.equal(t["state"], before)
    o1, s1 = oracle_loop(**{**t, "state": None})
    o2, s2 = oracle_loop(**{**t, "state": torch.zeros_like(before)})
    assert torch.equal(o1, o2) and torch.equal(s1, s2)


def test_gate_shapes_equivalent_and_scale_default():
    t = make_inputs(2, 1, 2, seed=21)
    o1, s1 = oracle_loop(**t)
    o2, s2 = oracle_loop(**{**t, "a": t["a"].reshape(2, 2), "b": t["b"].reshape(2, 2)})
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
    o3, _ = oracle_loop(**{**t, "scale": None})
    o4, _ = oracle_loop(**{**t, "scale": 0.0})
    assert torch.equal(o3, o1) and torch.equal(o4, o1)   # make_inputs uses 1/sqrt(128)


def test_bf16_output_is_round_to_nearest_even_of_fp32():
    t = make_inputs(2, 2, 4, seed=22)
    ob, _ = oracle_loop(**t)
    of, _ = oracle_loop(**t, output_fp32=True)
    assert ob.dtype == torch.bfloat16
    assert torch.equal(ob, of.to(torch.bfloat16))


@pytest.mark.parametrize("name", sorted(load_golden()))
def test_golden_vectors(name):
    t, l2, exp_out, exp_state = load_golden()[name]
    for impl in (_loop, _vec):
        out, st = impl(**t, use_qk_l2norm=l2)
        r64 = torch.from_numpy(exp_out)
        d = (out.double() - r64).abs()
        assert bool((d <= OUT_TIGHT_ATOL + 1e-4 * r64.abs()).all())
        assert (st.double() - torch.from_numpy(exp_state).double()).abs().max().item() < 2e-6
    ob, _ = oracle_loop(**t, use_qk_l2norm=l2)
    d = (ob.double() - torch.from_numpy(exp_out)).abs()
    assert bool((d <= OUT_TIGHT_ATOL + OUT_TIGHT_RTOL * torch.from_numpy(exp_out).abs()).all())


# --------------------------------------------------------------------------
# Multi-token steps and the bf16 state.
# --------------------------------------------------------------------------

def _no_carry_tokens(step, q, k, v, state, A_log, a, dt_bias, b, scale, **kw):
    """Planted mistake: every token starts from the input state."""
    outs, S = [], None
    for t in range(q.shape[1]):
        sl = slice(t, t + 1)
        o, S = step(q[:, sl], k[:, sl], v[:, sl], state, A_log, a[:, sl], dt_bias,
                    b[:, sl], scale, **kw)
        outs.append(o)
    return torch.cat(outs, dim=1), S


def check_tokens_orthogonal_writes(multi):
    """Two tokens with beta = 1, g = 1 and one-hot keys e1, e2 (q = k): each
    token stores its v under its key without disturbing the other, so the
    outputs are scale*v1, scale*v2, the final state reads v1 at e1 and v2 at
    e2, and every other column is the input state's."""
    K = V = 8
    t = make_inputs(1, 1, 1, seed=31, K=K, V=V, T=2)
    k = torch.zeros(1, 2, 1, K, dtype=torch.bfloat16)
    k[0, 0, 0, 1] = 1.0
    k[0, 1, 0, 2] = 1.0
    t.update(k=k, q=k.clone(), A_log=torch.tensor([NEG_INF]), scale=0.5,
             b=torch.full((1, 2, 1), POS_INF, dtype=torch.bfloat16))
    out, S = multi(**t)
    v = t["v"][0, :, 0].double()                       # [2, V]
    S = _f64(S)[0, 0]                                  # [V, K] storage
    assert torch.allclose(_f64(out)[0, :, 0], 0.5 * v, atol=1e-6), "tokens: outputs"
    assert torch.allclose(S[:, 1], v[0], atol=1e-6), "tokens: first write lost"
    assert torch.allclose(S[:, 2], v[1], atol=1e-6), "tokens: second write"
    keep = [0] + list(range(3, K))
    assert torch.allclose(S[:, keep], t["state"].double()[0, 0][:, keep], atol=1e-7)


def _fp32_out(step):
    return lambda *args, **kw: step(*args, **kw, output_fp32=True)


def test_multi_token_known_answer_and_planted_mistake():
    for step in (_fp32_out(oracle_loop), _fp32_out(oracle_vec), brute_fp64):
        check_tokens_orthogonal_writes(
            lambda **t: oracle_tokens(step, **t, state_dtype=None))
    with pytest.raises(AssertionError):
        check_tokens_orthogonal_writes(
            lambda **t: _no_carry_tokens(_fp32_out(oracle_vec), **t))


def test_multi_token_scalar_brute_force():
    """T = 3 at K = 3, V = 2 with plain Python floats, carrying the state."""
    K, V, T = 3, 2, 3
    t = make_inputs(1, 1, 1, seed=32, K=K, V=V, T=T)
    out, st = oracle_tokens(oracle_loop, **t, output_fp32=True)
    S = [[float(t["state"][0, 0, r, i]) for i in range(K)] for r in range(V)]
    for tok in range(T):
        x = float(t["a"][0, tok, 0]) + float(t["dt_bias"][0])
        g = math.exp(-math.exp(float(t["A_log"][0])) * math.log1p(math.exp(x)))
        beta = 1.0 / (1.0 + math.exp(-float(t["b"][0, tok, 0])))
        kv = [float(t["k"][0, tok, 0, i]) for i in range(K)]
        qv = [float(t["q"][0, tok, 0, i]) for i in range(K)]
        for r in range(V):
            S[r] = [g * S[r][i] for i in range(K)]
            d = beta * (float(t["v"][0, tok, 0, r]) - sum(S[r][i] * kv[i] for i in range(K)))
            S[r] = [S[r][i] + d * kv[i] for i in range(K)]
            o = t["scale"] * sum(S[r][i] * qv[i] for i in range(K))
            assert math.isclose(float(out[0, tok, 0, r]), o, rel_tol=1e-5, abs_tol=1e-6)
    for r in range(V):
        for i in range(K):
            assert math.isclose(float(st[0, 0, r, i]), S[r][i], rel_tol=1e-5, abs_tol=1e-6)


@pytest.mark.parametrize("l2", [False, True])
def test_multi_token_restatements_agree(l2):
    t = make_inputs(2, 2, 4, seed=33, T=4)
    o64, s64 = oracle_tokens(brute_fp64, **t, use_qk_l2norm=l2, state_dtype=None)
    for step in (oracle_loop, oracle_vec):
        o, s = oracle_tokens(step, **t, use_qk_l2norm=l2, output_fp32=True)
        assert (o.double() - o64).abs().max().item() < 2e-6
        assert (s.double() - s64).abs().max().item() < 4e-6


def test_bf16_state_is_rne_of_the_fp32_result():
    t = make_inputs(2, 2, 4, seed=34, T=2)
    t["state"] = t["state"].to(torch.bfloat16)         # a bf16 state as input
    o32, s32 = oracle_tokens(oracle_loop, **t, use_qk_l2norm=True)
    o16, s16 = oracle_tokens(oracle_loop, **t, use_qk_l2norm=True,
                             state_dtype=torch.bfloat16)
    assert s16.dtype == torch.bfloat16 and torch.equal(o16, o32)
    assert torch.equal(s16, s32.to(torch.bfloat16))
