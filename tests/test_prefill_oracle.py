"""Pinning the prefill oracle (CPU only).

The reference holds no prefill fixtures (its workloads live in an external
dataset, CLAUDE.md:164-168).  The loop restatement is pinned to the decode
oracle (itself pinned by closed forms, invariants and brute force in
test_oracle.py): a prefill of a sequence is the decode step folded over its
tokens.  The chunkwise float64 form -- the kernels' algebra -- is pinned to
the loop, at chunk sizes that put chunk boundaries inside sequences, and
planted mistakes in it must fail.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.gdn_decode_oracle import brute_fp64, oracle_loop, oracle_tokens
from oracle.gdn_prefill_oracle import make_prefill_inputs, prefill_chunked_fp64, prefill_loop


def _seq_as_decode(t, s):
    """Sequence s of a prefill input as T-token decode inputs (B = 1)."""
    cu = t["cu_seqlens"].tolist()
    sl = slice(cu[s], cu[s + 1])
    return dict(q=t["q"][sl].unsqueeze(0), k=t["k"][sl].unsqueeze(0), v=t["v"][sl].unsqueeze(0),
                state=None if t["state"] is None else t["state"][s:s + 1],
                A_log=t["A_log"], a=t["a"][sl].unsqueeze(0), dt_bias=t["dt_bias"],
                b=t["b"][sl].unsqueeze(0), scale=t["scale"])


@pytest.mark.parametrize("H,HV", [(4, 8), (2, 2), (1, 4)])
def test_loop_is_the_decode_step_folded_over_tokens(H, HV):
    t = make_prefill_inputs([3, 1, 5], H, HV, seed=1)
    out, st = prefill_loop(**t)
    for s in range(3):
        d = _seq_as_decode(t, s)
        o_ref, s_ref = oracle_tokens(oracle_loop, **d)
        cu = t["cu_seqlens"].tolist()
        # same fp32 arithmetic grouped per head vs batched over heads
        assert torch.allclose(out[cu[s]:cu[s + 1]].float(), o_ref[0].float(), rtol=1e-2,
                              atol=1e-5), s
        assert torch.allclose(st[s], s_ref[0], rtol=1e-5, atol=1e-6), s


def test_one_token_sequences_are_a_batched_decode_step():
    t = make_prefill_inputs([1, 1, 1, 1], 4, 8, seed=2)
    out, st = prefill_loop(**t)
    d = dict(q=t["q"].unsqueeze(1), k=t["k"].unsqueeze(1), v=t["v"].unsqueeze(1),
             state=t["state"], A_log=t["A_log"], a=t["a"], dt_bias=t["dt_bias"], b=t["b"],
             scale=t["scale"])
    o_ref, s_ref = oracle_loop(**d)
    assert torch.allclose(out.float(), o_ref[:, 0].float(), rtol=1e-2, atol=1e-5)
    assert torch.allclose(st, s_ref, rtol=1e-5, atol=1e-6)


def test_loop_against_float64_brute_force():
    t = make_prefill_inputs([4, 2], 4, 8, seed=3)
    out, st = prefill_loop(**t, output_fp32=True)
    cu = t["cu_seqlens"].tolist()
    for s in range(2):
        o64, s64 = oracle_tokens(brute_fp64, **_seq_as_decode(t, s), state_dtype=None)
        assert np.allclose(out[cu[s]:cu[s + 1]].double().numpy(), o64[0].numpy(),
                           rtol=1e-4, atol=1e-6)
        assert np.allclose(st[s].double().numpy(), s64[0].numpy(), rtol=1e-4, atol=1e-6)


def test_empty_sequences_and_no_state_follow_the_reference():
    t = make_prefill_inputs([0, 3, 0], 4, 8, seed=4)
    out, st = prefill_loop(**t)
    assert out.shape == (3, 8, 128)
    assert torch.count_nonzero(st[0]) == 0 and torch.count_nonzero(st[2]) == 0
    assert torch.count_nonzero(st[1]) > 0
    t0 = make_prefill_inputs([2], 4, 8, seed=5, with_state=False)
    out0, st0 = prefill_loop(**t0)
    z = dict(t0, state=torch.zeros(1, 8, 128, 128))
    out1, st1 = prefill_loop(**z)
    # equal up to the BLAS path (a transposed view of zeros vs fresh zeros)
    assert torch.allclose(out0.float(), out1.float(), rtol=1e-2, atol=1e-6)
    assert torch.allclose(st0, st1, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("chunk", [1, 3, 16, 64])
@pytest.mark.parametrize("l2", [False, True])
def test_chunked_form_equals_the_loop(chunk, l2):
    t = make_prefill_inputs([5, 70, 1, 0, 33], 4, 8, seed=6)
    out, st = prefill_loop(**t, use_qk_l2norm=l2, output_fp32=True)
    o64, s64 = prefill_chunked_fp64(**t, chunk=chunk, use_qk_l2norm=l2)
    assert np.allclose(out.double().numpy(), o64, rtol=1e-4, atol=2e-5)
    assert np.allclose(st.double().numpy(), s64, rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("mutation", ["M_without_diagonal", "A_transposed",
                                      "W_without_decay", "state_decay_from_first"])
def test_planted_mistakes_in_the_chunked_form_are_caught(mutation):
    t = make_prefill_inputs([70], 4, 8, seed=7)
    out, st = prefill_loop(**t, output_fp32=True)
    o64, s64 = prefill_chunked_fp64(**t, chunk=16, _mutation=mutation)
    ok_o = np.allclose(out.double().numpy(), o64, rtol=1e-4, atol=2e-5)
    ok_s = np.allclose(st.double().numpy(), s64, rtol=1e-4, atol=1e-6)
    assert not (ok_o and ok_s), mutation
