"""CPU oracle of the GDN decode step -- TEST INFRASTRUCTURE ONLY.

This module checks the gfx950 kernel; it is not part of it.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only to check or to time the reference's CPU algorithm; the
product path (``flashinfer_competition_codebase_amd``) never calls it.

It restates the reference's PyTorch decode step ``kernel_pt_reference``
(solution/triton/kernel.py:22-118) on the CPU in fp32, three ways:

* ``oracle_loop`` follows kernel.py:72-118 loop-for-loop (per-(b, hv) clone,
  transpose, decay, vec-mat, two outer products, output vec-mat, transpose
  back).  It is the CPU baseline that ``bench.py`` times.
* ``oracle_vec`` is the same arithmetic batched over (b, hv) with ``matmul``;
  fp32 for the kernel-parity tests at full sizes, fp64 on request.
* ``brute_fp64`` is an independent NumPy float64 restatement written from
  the recurrence formulas (kernel.py:50-55), used to pin the two above.

Generalisations of the reference, each off by default where it changes the
result: any ``HV % H == 0`` (the reference asserts H=4, HV=8,
kernel.py:63-67, which fails at every qk16_v32 shape), any K and V (tiny
brute-force checks; the kernel itself takes K = V = 128), gate tensors of
shape ``[B, 1, HV]`` or ``[B, HV]``, and an optional q/k L2-norm
``x * rsqrt(sum(x^2) + eps)`` with ``eps = 1e-6`` applied in fp32 before the
step (not part of ``kernel_pt_reference``; it is the normalisation the
flash-linear-attention ``l2norm`` uses, a dependency the reference names
through ``use_qk_l2norm_in_kernel`` at solution/triton/fla_prefill_code.py:1797
but does not vendor).

``oracle_tokens`` extends any of the three to T > 1 tokens per sequence: the
per-token loop of the reference's prefill oracle
(solution/triton/prefill_kernel.py:144-178, one decode step per token
against the running fp32 state, output per token) for fixed-length
sequences, optionally storing the final state in bf16 (round to nearest
even, as torch's ``.to(torch.bfloat16)``).

Pinning status (see tests/test_oracle.py for each check): gates, GVA mapping,
k-last layout, delta rule, output, state=None and the L2-norm are each pinned
by closed forms, invariants or brute force; the reference itself holds no
golden vectors for this path.  The bit-level fp32 summation order of torch's
CPU vec-mat is not pinned, and need not be at the stated tolerances.
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

L2NORM_EPS = 1e-6
SOFTPLUS_THRESHOLD = 20.0


def resolve_scale(scale, K: int) -> float:
    """None or 0 -> 1/sqrt(K) (solution/triton/kernel.py:69-70)."""
    if scale is None:
        return 1.0 / math.sqrt(K)
    scale = float(scale)
    return 1.0 / math.sqrt(K) if scale == 0.0 else scale


def gates(A_log, a, dt_bias, b):
    """fp32 decay ``g`` and update gate ``beta`` (solution/triton/kernel.py:73-75).

    ``g = exp(-exp(A_log) * softplus(a + dt_bias))`` with torch's softplus
    (threshold 20, the constant the fused kernels copy at kernel.py:299 and
    kernel.cu:135), ``beta = sigmoid(b)``.  Shapes broadcast as the
    reference's: ``a, b`` ``[B, 1, HV]`` or ``[B, HV]``, ``A_log, dt_bias``
    ``[HV]``.
    """
    x = a.float() + dt_bias.float()
    g = torch.exp(-torch.exp(A_log.float()) * F.softplus(x))
    beta = torch.sigmoid(b.float())
    return g, beta


def l2norm(x: torch.Tensor, eps: float = L2NORM_EPS) -> torch.Tensor:
    """``x * rsqrt(sum(x^2, -1) + eps)`` in the dtype of ``x``."""
    return x * torch.rsqrt((x * x).sum(dim=-1, keepdim=True) + eps)


def _prepare(q, k, v, state, A_log, a, dt_bias, b, scale, use_qk_l2norm, eps, dtype):
    B, T, H, K = q.shape
    HV, V = v.shape[2], v.shape[3]
    assert T == 1, "decode is one token per sequence"
    assert k.shape == q.shape
    assert HV % H == 0, "v-heads must be a multiple of q/k heads"
    scale = resolve_scale(scale, K)
    g, beta = gates(A_log, a, dt_bias, b)
    g = g.reshape(B, HV).to(dtype)
    beta = beta.reshape(B, HV).to(dtype)
    q_f = q.squeeze(1).to(dtype)
    k_f = k.squeeze(1).to(dtype)
    v_f = v.squeeze(1).to(dtype)
    if use_qk_l2norm:
        q_f = l2norm(q_f, eps)
        k_f = l2norm(k_f, eps)
    if state is not None:
        s_f = state.to(dtype)
    else:
        s_f = torch.zeros(B, HV, V, K, dtype=dtype, device=q.device)  # kernel.py:83-86
    r = HV // H
    q_exp = q_f.repeat_interleave(r, dim=1)  # kernel.py:88-89: v-head hv uses q/k head hv // r
    k_exp = k_f.repeat_interleave(r, dim=1)
    return B, HV, K, V, scale, g, beta, q_exp, k_exp, v_f, s_f


@torch.no_grad()
def oracle_loop(q, k, v, state, A_log, a, dt_bias, b, scale, *,
                use_qk_l2norm=False, eps=L2NORM_EPS, output_fp32=False):
    """Loop-for-loop restatement of solution/triton/kernel.py:72-118 (fp32).

    Returns ``(output [B, 1, HV, V] bf16, new_state [B, HV, V, K] fp32)``
    (``output`` stays fp32 with ``output_fp32=True``); ``state`` is not
    modified.
    """
    B, HV, K, V, scale, g_f32, beta_f32, q_exp, k_exp, v_f32, state_f32 = _prepare(
        q, k, v, state, A_log, a, dt_bias, b, scale, use_qk_l2norm, eps, torch.float32)
    new_state = torch.zeros_like(state_f32)
    output = torch.zeros(B, HV, V, dtype=torch.float32, device=q.device)
    for b_idx in range(B):                       # kernel.py:95-114
        for h_idx in range(HV):
            q_h = q_exp[b_idx, h_idx]                                    # [K]
            k_h = k_exp[b_idx, h_idx]                                    # [K]
            v_h = v_f32[b_idx, h_idx]                                    # [V]
            h_state = state_f32[b_idx, h_idx].clone().transpose(-1, -2)  # [K, V]
            g_val = g_f32[b_idx, h_idx]
            beta_val = beta_f32[b_idx, h_idx]
            old_state = g_val * h_state
            old_v = k_h @ old_state                                      # [V]
            new_v = beta_val * v_h + (1 - beta_val) * old_v
            state_remove = k_h.unsqueeze(1) @ old_v.unsqueeze(0)         # [K, V]
            state_update = k_h.unsqueeze(1) @ new_v.unsqueeze(0)
            h_state = old_state - state_remove + state_update
            output[b_idx, h_idx] = scale * (q_h @ h_state)
            new_state[b_idx, h_idx] = h_state.transpose(-1, -2)          # back to [V, K]
    output = output.unsqueeze(1)
    if not output_fp32:
        output = output.to(torch.bfloat16)        # kernel.py:117
    return output, new_state


@torch.no_grad()
def oracle_vec(q, k, v, state, A_log, a, dt_bias, b, scale, *,
               use_qk_l2norm=False, eps=L2NORM_EPS, output_fp32=False,
               dtype=torch.float32):
    """``oracle_loop``'s arithmetic batched over (b, hv) in ``dtype``.

    Same op order per head: decay, ``old_v = k . (g S)``, blend, two outer
    products, ``o = scale * q . S_new``.  Returns the new state in ``dtype``
    and the output in bf16 (or ``dtype`` with ``output_fp32=True``).
    """
    B, HV, K, V, scale, g, beta, q_exp, k_exp, v_f, s_f = _prepare(
        q, k, v, state, A_log, a, dt_bias, b, scale, use_qk_l2norm, eps, dtype)
    old_state = g[:, :, None, None] * s_f                         # [B, HV, V, K]
    old_v = torch.matmul(old_state, k_exp.unsqueeze(-1)).squeeze(-1)   # [B, HV, V]
    bt = beta.unsqueeze(-1)
    new_v = bt * v_f + (1 - bt) * old_v
    kk = k_exp.unsqueeze(-2)                                      # [B, HV, 1, K]
    new_s = old_state - old_v.unsqueeze(-1) * kk + new_v.unsqueeze(-1) * kk
    out = scale * torch.matmul(new_s, q_exp.unsqueeze(-1)).squeeze(-1)  # [B, HV, V]
    out = out.unsqueeze(1)
    if not output_fp32:
        out = out.to(torch.bfloat16)
    return out, new_s


def _np64(t) -> np.ndarray:
    return t.detach().to(torch.float64).cpu().numpy()


def brute_fp64(q, k, v, state, A_log, a, dt_bias, b, scale, *,
               use_qk_l2norm=False, eps=L2NORM_EPS):
    """Independent float64 NumPy restatement of the recurrence
    (solution/triton/kernel.py:50-55; k-last storage, kernel.py:101,114).

    Per (b, hv) with h = hv // (HV // H):  g, beta from the gate formulas;
    ``S = g * state^T`` as a [K, V] matrix; ``u = beta * (v - k^T S)``;
    ``S += k u^T``; ``o = scale * q^T S``.  Returns float64 arrays
    ``(output [B, 1, HV, V], new_state [B, HV, V, K])`` with no rounding.
    """
    qn, kn, vn = _np64(q)[:, 0], _np64(k)[:, 0], _np64(v)[:, 0]
    B, H, K = qn.shape
    HV, V = vn.shape[1], vn.shape[2]
    r = HV // H
    scale = resolve_scale(scale, K)
    A = _np64(A_log).reshape(HV)
    dt = _np64(dt_bias).reshape(HV)
    av = _np64(a).reshape(B, HV)
    bv = _np64(b).reshape(B, HV)
    S0 = np.zeros((B, HV, V, K)) if state is None else _np64(state)
    out = np.zeros((B, 1, HV, V))
    S_out = np.zeros((B, HV, V, K))
    for bi in range(B):
        for hv in range(HV):
            x = av[bi, hv] + dt[hv]
            sp = x if x > SOFTPLUS_THRESHOLD else math.log1p(math.exp(x))
            g = math.exp(-math.exp(A[hv]) * sp)
            beta = 1.0 / (1.0 + math.exp(-bv[bi, hv]))
            qh, kh = qn[bi, hv // r].copy(), kn[bi, hv // r].copy()
            if use_qk_l2norm:
                qh = qh / math.sqrt(float(qh @ qh) + eps)
                kh = kh / math.sqrt(float(kh @ kh) + eps)
            S = g * S0[bi, hv].T                  # [K, V]
            u = beta * (vn[bi, hv] - kh @ S)      # [V]
            S = S + np.outer(kh, u)
            out[bi, 0, hv] = scale * (qh @ S)
            S_out[bi, hv] = S.T
    return out, S_out


def oracle_tokens(step, q, k, v, state, A_log, a, dt_bias, b, scale, *,
                  state_dtype=torch.float32, **kw):
    """T tokens per sequence through the single-token oracle ``step``
    (``oracle_loop``, ``oracle_vec`` or ``brute_fp64``), as the reference's
    prefill oracle does for each sequence (prefill_kernel.py:144-178): token
    t's step starts from the state token t-1 left, with no rounding in
    between.  q, k ``[B, T, H, K]``, v ``[B, T, HV, V]``, a, b
    ``[B, T, HV]``.  Returns ``(output [B, T, HV, V], new_state)`` with the
    output as ``step`` gives it and the state cast to ``state_dtype`` (a
    torch dtype; ``brute_fp64`` states stay float64 NumPy when it is None).
    """
    T = q.shape[1]
    S = None if state is None else state.float()
    outs = []
    for t in range(T):
        sl = slice(t, t + 1)
        o, S = step(q[:, sl], k[:, sl], v[:, sl], S, A_log, a[:, sl], dt_bias, b[:, sl],
                    scale, **kw)
        if isinstance(S, np.ndarray):
            S = torch.from_numpy(S)
            o = torch.from_numpy(o)
        outs.append(o)
    out = torch.cat(outs, dim=1)
    if state_dtype is not None:
        S = S.to(state_dtype)
    return out, S


def make_inputs(B, H, HV, *, seed, state_std=0.05, device="cpu", K=128, V=128,
                gate_shape="b1hv", T=1):
    """Seeded decode inputs with the benchmark's distributions.

    q, k, v ~ N(0, 1) bf16 (T tokens); state ~ N(0, state_std^2) fp32; a, b
    ~ N(0, 1) bf16; A_log = log(U[1, 16]) fp32; dt_bias ~ U[-1, 1] fp32.
    ``gate_shape="bhv"`` (T = 1 only) gives a, b as ``[B, HV]``.  Generated on
    the CPU from ``torch.Generator().manual_seed(seed)`` and then moved to
    ``device``, so every device sees identical bits.
    """
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, K, generator=gen).to(torch.bfloat16)
    k = torch.randn(B, T, H, K, generator=gen).to(torch.bfloat16)
    v = torch.randn(B, T, HV, V, generator=gen).to(torch.bfloat16)
    state = torch.randn(B, HV, V, K, generator=gen) * state_std
    gshape = (B, T, HV) if gate_shape == "b1hv" else (B, HV)
    a = torch.randn(*gshape, generator=gen).to(torch.bfloat16)
    b = torch.randn(*gshape, generator=gen).to(torch.bfloat16)
    A_log = torch.log(torch.rand(HV, generator=gen) * 15.0 + 1.0)
    dt_bias = torch.rand(HV, generator=gen) * 2.0 - 1.0
    t = dict(q=q, k=k, v=v, state=state, A_log=A_log, a=a, dt_bias=dt_bias, b=b,
             scale=1.0 / math.sqrt(K))
    if device != "cpu":
        t = {n: (x.to(device) if isinstance(x, torch.Tensor) else x) for n, x in t.items()}
    return t
