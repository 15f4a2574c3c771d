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


@torch.no_grad()
def prefill_chunked_fp64(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, *,
                         chunk=64, use_qk_l2norm=False, eps=L2NORM_EPS, _mutation=None):
    """Float64 chunkwise restatement (the kernels' algebra, module docstring).

    Same arguments as ``prefill_loop``; chunks of ``chunk`` tokens start at
    each sequence's first token.  Returns float64 NumPy arrays
    ``(output [L, HV, V], new_state [N, HV, V, K])``.  Sequences of equal
    length share their chunk grid, so they and all heads are evaluated
    together as one batch (float64 CPU torch, batched BLAS products; v-head
    ``h * r + j`` of q/k head h is index ``[h, j]`` of the [H, r] head axes).
    T is not formed: W and U come from triangular solves with I + A.
    ``_mutation`` plants a named mistake (tests only: each must be caught by
    the pinning checks).
    """
    f64 = dict(dtype=torch.float64)
    qn, kn, vn = q.cpu().to(**f64), k.cpu().to(**f64), v.cpu().to(**f64)
    L, H, K = qn.shape
    HV, V = vn.shape[1], vn.shape[2]
    r = HV // H
    scale = resolve_scale(scale, K)
    A_log_n, dt_n = A_log.cpu().to(**f64), dt_bias.cpu().to(**f64)
    an, bn = a.cpu().to(**f64).reshape(L, HV), b.cpu().to(**f64).reshape(L, HV)
    x = an + dt_n[None, :]
    sp = torch.where(x > SOFTPLUS_THRESHOLD, x,
                     torch.log1p(torch.exp(torch.clamp(x, max=SOFTPLUS_THRESHOLD))))
    logg = (-torch.exp(A_log_n)[None, :] * sp).view(L, H, r)     # log-space decay
    beta = (1.0 / (1.0 + torch.exp(-bn))).view(L, H, r)
    vn = vn.view(L, H, r, V)
    if use_qk_l2norm:
        qn = qn / torch.sqrt((qn * qn).sum(-1, keepdim=True) + eps)
        kn = kn / torch.sqrt((kn * kn).sum(-1, keepdim=True) + eps)
    cu = [int(c) for c in cu_seqlens.tolist()]
    N = len(cu) - 1
    out = torch.zeros(L, H, r, V, **f64)
    S_out = torch.zeros(N, HV, V, K, **f64)
    S0_all = None if state is None else state.cpu().to(**f64)
    by_len = {}
    for s in range(N):
        if cu[s + 1] > cu[s]:       # empty sequences keep a zero new_state, as prefill_loop
            by_len.setdefault(cu[s + 1] - cu[s], []).append(s)
    neg_inf, zero = torch.tensor(-math.inf, **f64), torch.zeros((), **f64)
    for n_tok, seqs in by_len.items():
        starts = torch.tensor([cu[s] for s in seqs])
        G = len(seqs)
        # S: [G, H, r, K, V] (the k-last storage transposed)
        S = (torch.zeros(G, H, r, K, V, **f64) if S0_all is None
             else S0_all[seqs].view(G, H, r, V, K).transpose(3, 4).contiguous())
        for c0 in range(0, n_tok, chunk):
            c1 = min(c0 + chunk, n_tok)
            n = c1 - c0
            idx = starts[:, None] + torch.arange(c0, c1)[None, :]  # [G, n] token rows
            Kc = kn[idx].permute(0, 2, 1, 3).unsqueeze(2)         # [G, H, 1, n, K]
            Qc = qn[idx].permute(0, 2, 1, 3).unsqueeze(2)
            Vc = vn[idx].permute(0, 2, 3, 1, 4)                   # [G, H, r, n, V]
            bc = beta[idx].permute(0, 2, 3, 1)                    # [G, H, r, n]
            gam = torch.cumsum(logg[idx], dim=1).permute(0, 2, 3, 1)
            D = gam[..., :, None] - gam[..., None, :]
            lower = torch.tril(torch.ones(n, n, dtype=torch.bool), -1)
            causal = torch.tril(torch.ones(n, n, dtype=torch.bool))
            Gam = torch.exp(torch.where(causal, D, neg_inf))      # M, incl. diagonal
            if _mutation == "M_without_diagonal":
                Gam = Gam * lower
            A = torch.where(lower, bc[..., :, None] * Gam * (Kc @ Kc.transpose(-1, -2)), zero)
            if _mutation == "A_transposed":
                A = A.transpose(-1, -2)
            IA = torch.eye(n, **f64) + A
            wdecay = torch.ones_like(gam) if _mutation == "W_without_decay" else torch.exp(gam)
            rhs = torch.cat([((bc * wdecay)[..., None] * Kc),
                             (bc[..., None] * Vc)], dim=-1)       # [G, H, r, n, K + V]
            WU = torch.linalg.solve_triangular(IA, rhs, upper=False)
            W, U = WU[..., :K], WU[..., K:]
            Delta = U - W @ S
            o = scale * ((torch.exp(gam)[..., None] * Qc) @ S
                         + ((Qc @ Kc.transpose(-1, -2)) * Gam) @ Delta)
            out[idx] = o.permute(0, 3, 1, 2, 4)
            last = gam[..., -1] if _mutation != "state_decay_from_first" else gam[..., 0]
            S = (torch.exp(last)[..., None, None] * S
                 + (torch.exp(gam[..., -1:] - gam)[..., None] * Kc).transpose(-1, -2) @ Delta)
        S_out[seqs] = S.transpose(3, 4).reshape(G, HV, V, K)
    return out.view(L, HV, V).numpy(), S_out.numpy()


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
