"""CPU oracle of the GDN prefill -- TEST INFRASTRUCTURE ONLY.

This module checks the gfx950 prefill kernels; it is not part of them.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it; the product path never calls it.

It restates the reference's prefill ``kernel_prefill_reference``
(solution/triton/prefill_kernel.py:85-183) on the CPU:

* ``prefill_loop`` follows prefill_kernel.py:134-181 loop-for-loop in fp32:
  per sequence of ``cu_seqlens``, per token, the decode step of
  kernel.py:95-114 on all v-heads at once (decay, ``old_v = k . (g S)``,
  blend, two outer products, output) against the running state; the final
  state of each sequence goes to ``new_state``.  Generalised to any
  ``HV % H == 0`` (the reference asserts H = 4, HV = 8, prefill_kernel.py:
  126-129); ``state=None`` starts from zeros (prefill_kernel.py:152-155); a
  sequence with no tokens gets a zero ``new_state``, as in the reference
  (prefill_kernel.py:147-150 skip it and its row of the zero-initialised
  result stays zero).
* ``prefill_chunked_fp64`` is an independent float64 NumPy restatement of the
  same recurrence in chunkwise form -- the algebra the gfx950 kernels use --
  so that tests can pin that algebra against the loop:
  per chunk of C tokens with cumulative log-decay ``gamma`` and state S_0
  at the chunk start,
      A     = strict_lower(beta_i exp(gamma_i - gamma_j) k_i . k_j)
      T     = (I + A)^-1
      Delta = T diag(beta) V - T diag(beta exp(gamma)) K S_0
      O     = scale [diag(exp(gamma)) Q S_0 + (Q K^T (.) M) Delta],
              M_ij = exp(gamma_i - gamma_j) for j <= i, else 0
      S_C   = exp(gamma_C) S_0 + (diag(exp(gamma_C - gamma)) K)^T Delta
  (S in [K, V] orientation; Delta is the per-token delta-rule correction
  beta (v - g S^T k) of the loop).

Pinning: a one-token sequence is the decode step (pinned in
tests/test_oracle.py); a sequence is the decode oracle folded over its
tokens; the chunked form equals the loop for every chunk size, including
chunk boundaries inside and across sequences; planted mistakes in the
chunked form fail; empty sequences get a zero state as in the reference
(tests/test_prefill_oracle.py).
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

from oracle.gdn_decode_oracle import L2NORM_EPS, SOFTPLUS_THRESHOLD, l2norm, resolve_scale


@torch.no_grad()
def prefill_loop(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, *,
                 use_qk_l2norm=False, eps=L2NORM_EPS, output_fp32=False):
    """Loop-for-loop restatement of solution/triton/prefill_kernel.py:85-183.

    q, k ``[L, H, K]`` bf16; v ``[L, HV, V]`` bf16; state ``[N, HV, V, K]``
    fp32 (k-last) or None; A_log, dt_bias ``[HV]`` fp32; a, b ``[L, HV]``
    bf16; cu_seqlens ``[N + 1]`` int; scale float (None/0 -> 1/sqrt(K)).
    Returns ``(output [L, HV, V] bf16, new_state [N, HV, V, K] fp32)``.
    """
    L, H, K = q.shape
    HV, V = v.shape[1], v.shape[2]
    assert HV % H == 0, "v-heads must be a multiple of q/k heads"
    N = int(cu_seqlens.numel()) - 1
    scale = resolve_scale(scale, K)
    x = a.float() + dt_bias.float()                               # prefill_kernel.py:137-140
    g = torch.exp(-torch.exp(A_log.float()) * F.softplus(x))      # [L, HV]
    beta = torch.sigmoid(b.float())
    qf, kf = q.float(), k.float()
    if use_qk_l2norm:
        qf, kf = l2norm(qf, eps), l2norm(kf, eps)
    r = HV // H
    q_exp = qf.repeat_interleave(r, dim=1)                        # prefill_kernel.py:142-143
    k_exp = kf.repeat_interleave(r, dim=1)
    output = torch.zeros(L, HV, V, dtype=torch.float32)
    new_state = torch.zeros(N, HV, V, K, dtype=torch.float32)
    cu = [int(c) for c in cu_seqlens.tolist()]
    for s in range(N):                                            # prefill_kernel.py:152-181
        start, end = cu[s], cu[s + 1]
        if end - start <= 0:        # prefill_kernel.py:147-150: new_state stays zero
            continue
        if state is not None:
            S = state[s].float().clone().transpose(-1, -2)        # [HV, K, V]
        else:
            S = torch.zeros(HV, K, V)
        for t in range(start, end):
            q_t = q_exp[t].unsqueeze(1)                           # [HV, 1, K]
            k_t = k_exp[t].unsqueeze(1)
            v_t = v[t].unsqueeze(1).float()                       # [HV, 1, V]
            g_t = g[t].view(HV, 1, 1)
            b_t = beta[t].view(HV, 1, 1)
            old_S = g_t * S
            old_v = k_t @ old_S                                   # [HV, 1, V]
            new_v = b_t * v_t + (1 - b_t) * old_v
            S = old_S - k_t.transpose(-1, -2) @ old_v + k_t.transpose(-1, -2) @ new_v
            output[t] = (scale * (q_t @ S)).squeeze(1)
        new_state[s] = S.transpose(-1, -2)                        # back to [HV, V, K]
    if not output_fp32:
        output = output.to(torch.bfloat16)
    return output, new_state


def _np64(t):
    return t.detach().to(torch.float64).cpu().numpy()


def prefill_chunked_fp64(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, *,
                         chunk=64, use_qk_l2norm=False, eps=L2NORM_EPS, _mutation=None):
    """Float64 chunkwise restatement (the kernels' algebra, module docstring).

    Same arguments as ``prefill_loop``; chunks of ``chunk`` tokens start at
    each sequence's first token.  Returns float64 arrays
    ``(output [L, HV, V], new_state [N, HV, V, K])``.  ``_mutation`` plants a
    named mistake (tests only: each must be caught by the pinning checks).
    """
    qn, kn, vn = _np64(q), _np64(k), _np64(v)
    L, H, K = qn.shape
    HV, V = vn.shape[1], vn.shape[2]
    r = HV // H
    scale = resolve_scale(scale, K)
    A_log_n, dt_n = _np64(A_log), _np64(dt_bias)
    an, bn = _np64(a).reshape(L, HV), _np64(b).reshape(L, HV)
    x = an + dt_n[None, :]
    sp = np.where(x > SOFTPLUS_THRESHOLD, x, np.log1p(np.exp(np.minimum(x, SOFTPLUS_THRESHOLD))))
    logg = -np.exp(A_log_n)[None, :] * sp                         # [L, HV] log-space decay
    beta = 1.0 / (1.0 + np.exp(-bn))
    if use_qk_l2norm:
        qn = qn / np.sqrt((qn * qn).sum(-1, keepdims=True) + eps)
        kn = kn / np.sqrt((kn * kn).sum(-1, keepdims=True) + eps)
    cu = [int(c) for c in cu_seqlens.tolist()]
    N = len(cu) - 1
    out = np.zeros((L, HV, V))
    S_out = np.zeros((N, HV, V, K))
    S0_all = None if state is None else _np64(state)
    for s in range(N):
        start, end = cu[s], cu[s + 1]
        if end <= start:            # as prefill_loop: zero new_state
            continue
        for hv in range(HV):
            h = hv // r
            S = np.zeros((K, V)) if S0_all is None else S0_all[s, hv].T.copy()
            for c0 in range(start, end, chunk):
                c1 = min(c0 + chunk, end)
                Kc, Qc, Vc = kn[c0:c1, h], qn[c0:c1, h], vn[c0:c1, hv]
                bc = beta[c0:c1, hv]
                gam = np.cumsum(logg[c0:c1, hv])
                D = gam[:, None] - gam[None, :]
                n = c1 - c0
                lower = np.tril(np.ones((n, n)), -1).astype(bool)
                causal = np.tril(np.ones((n, n))).astype(bool)
                Gam = np.exp(np.where(causal, D, -np.inf))          # M, incl. diagonal
                if _mutation == "M_without_diagonal":
                    Gam = Gam * lower
                A = np.where(lower, bc[:, None] * Gam * (Kc @ Kc.T), 0.0)
                if _mutation == "A_transposed":
                    A = A.T
                T = np.linalg.inv(np.eye(n) + A)
                wdecay = np.ones(n) if _mutation == "W_without_decay" else np.exp(gam)
                W = T @ ((bc * wdecay)[:, None] * Kc)
                U = T @ (bc[:, None] * Vc)
                Delta = U - W @ S
                out[c0:c1, hv] = scale * ((np.exp(gam)[:, None] * Qc) @ S
                                          + ((Qc @ Kc.T) * Gam) @ Delta)
                last = gam[-1] if _mutation != "state_decay_from_first" else gam[0]
                S = np.exp(last) * S + (np.exp(gam[-1] - gam)[:, None] * Kc).T @ Delta
            S_out[s, hv] = S.T
    return out, S_out


def make_prefill_inputs(seqlens, H, HV, *, seed, state_std=0.05, with_state=True, K=128,
                        V=128, unit_qk=True):
    """Seeded prefill inputs for sequences of the given lengths: q, k ~ N(0, 1)
    per element, scaled to unit L2 norm per (token, head) when ``unit_qk``
    (the normalisation the model applies before this step; with raw N(0, 1)
    keys |k|^2 ~ 128 and the delta-rule factor I - beta k k^T has an
    eigenvalue 1 - 128 beta, so the recurrence grows without bound over a
    sequence), then rounded to bf16; v, a, b ~ N(0, 1) bf16; state ~
    N(0, state_std^2) fp32; A_log = log U[1, 16]; dt_bias ~ U[-1, 1];
    cu_seqlens int32; scale = 1/sqrt(K).  Drawn on the CPU."""
    gen = torch.Generator().manual_seed(seed)
    L = int(sum(seqlens))
    N = len(seqlens)
    cu = torch.zeros(N + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(seqlens, dtype=torch.int64), 0).to(torch.int32)
    q = torch.randn(L, H, K, generator=gen)
    k = torch.randn(L, H, K, generator=gen)
    if unit_qk:
        q = q / q.norm(dim=-1, keepdim=True).clamp_min(1e-6)
        k = k / k.norm(dim=-1, keepdim=True).clamp_min(1e-6)
    t = dict(
        q=q.to(torch.bfloat16),
        k=k.to(torch.bfloat16),
        v=torch.randn(L, HV, V, generator=gen).to(torch.bfloat16),
        state=(torch.randn(N, HV, V, K, generator=gen) * state_std) if with_state else None,
        A_log=torch.log(torch.rand(HV, generator=gen) * 15.0 + 1.0),
        a=torch.randn(L, HV, generator=gen).to(torch.bfloat16),
        dt_bias=torch.rand(HV, generator=gen) * 2.0 - 1.0,
        b=torch.randn(L, HV, generator=gen).to(torch.bfloat16),
        cu_seqlens=cu,
        scale=1.0 / math.sqrt(K),
    )
    return t
