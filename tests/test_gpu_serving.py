"""The serving component (``DecodePlan`` / ``DecodeLayers``, the C ABI's
plans and HIP graph) against the CPU oracle (needs a HIP device).

A model's decode step at B = 1 (BASELINE's first config: qk16_v32, q/k
L2-norm) over several GDN layers, each with its own state updated in place:
the layers are bound once, then each model step writes fresh q, k, v, a, b
into the bound buffers and runs every layer -- replayed from one HIP graph,
or in one eager native call.  Every step of every layer is checked against
the oracle chained over the same inputs (its own state carried from step to
step), at the decode parity bars: bf16 output within atol = rtol = 1e-2 of
the oracle and one bf16 ulp of float64; fp32 state within 1e-3 relative +
1e-5 and 1e-3 in relative Frobenius norm.
"""

from __future__ import annotations

import sys

import pytest
import torch

from flashinfer_competition_codebase_amd import _lib
from flashinfer_competition_codebase_amd.serving import DecodeLayers, DecodePlan
from oracle.gdn_decode_oracle import make_inputs, oracle_loop, oracle_vec
from tests.gdn_cases import assert_output_close, assert_state_close

pytestmark = pytest.mark.gpu

INPUTS = ("q", "k", "v", "a", "b")


def _announce(case):
    sys.stdout.write(f"[gpu case] {case}\n")
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _library_present():
    _lib.get_lib()


def _bound_layers(n_layers, B, H, HV, device, seed):
    """Per layer: CPU inputs (the oracle's) and the device buffers bound once."""
    cpu, dev = [], []
    for i in range(n_layers):
        t = make_inputs(B, H, HV, seed=seed + i)
        d = {n: (x.to(device) if isinstance(x, torch.Tensor) else x) for n, x in t.items()}
        d["output"] = torch.empty(B, 1, HV, 128, dtype=torch.bfloat16, device=device)
        d["new_state"] = d["state"]                      # in place
        cpu.append(t)
        dev.append(d)
    return cpu, dev


def _check_step(case, t_cpu, d, ref_state, l2):
    """One layer's step against the oracle from ``ref_state``; returns the
    oracle's new state (the next step's starting point)."""
    t = {**t_cpu, "state": ref_state}
    ref_o, ref_s = oracle_loop(**t, use_qk_l2norm=l2)
    o64, _ = oracle_vec(**t, use_qk_l2norm=l2, output_fp32=True, dtype=torch.float64)
    assert_output_close(d["output"].cpu(), ref_o, tight_ref64=o64, what=f"{case} output")
    assert_state_close(d["state"].cpu(), ref_s, what=f"{case} state")
    return ref_s


@pytest.mark.parametrize("mode", ["graph", "eager"])
def test_layers_match_the_chained_oracle(mode, hip_device):
    n_layers, steps, l2 = 4, 3, True
    B, H, HV = 1, 16, 32
    _announce(f"DecodeLayers {mode}: {n_layers} layers x {steps} steps, B={B} qk{H}_v{HV}")
    cpu, dev = _bound_layers(n_layers, B, H, HV, hip_device, seed=5000)
    ref_states = [t["state"].clone() for t in cpu]
    layers = DecodeLayers(dev, use_qk_l2norm=l2)
    if mode == "graph":
        layers.capture()
        torch.cuda.synchronize()
        for i in range(n_layers):                       # capture runs nothing
            assert torch.equal(dev[i]["state"].cpu(), cpu[i]["state"])
    for step in range(steps):
        if step > 0:                                    # the next token's inputs
            for i in range(n_layers):
                fresh = make_inputs(B, H, HV, seed=6000 + 100 * step + i)
                for n in INPUTS:
                    cpu[i][n] = fresh[n]
                    dev[i][n].copy_(fresh[n])           # eager work between replays
        if mode == "graph":
            layers.replay()
        else:
            layers.run()
        torch.cuda.synchronize()
        for i in range(n_layers):
            ref_states[i] = _check_step(f"{mode} step {step} layer {i}", cpu[i], dev[i],
                                        ref_states[i], l2)
    layers.close()


def test_plan_runs_continue_the_sequence_and_null_state(hip_device):
    """One plan run twice continues the sequence (state in place); a plan
    without a state starts every run from zeros (the kernel's own zero
    state: new_state is only written)."""
    _announce("DecodePlan in place, and state=None")
    B, H, HV = 3, 4, 8
    t = make_inputs(B, H, HV, seed=5100)
    d = {n: (x.to(hip_device) if isinstance(x, torch.Tensor) else x) for n, x in t.items()}
    d["output"] = torch.empty(B, 1, HV, 128, dtype=torch.bfloat16, device=hip_device)
    plan = DecodePlan(**{**d, "new_state": d["state"]})
    ref = t["state"].clone()
    for step in range(2):
        plan.run()
        torch.cuda.synchronize()
        ref = _check_step(f"plan step {step}", t, d, ref, False)
    plan.close()
    with pytest.raises(RuntimeError):
        plan.run()
    out = torch.empty_like(d["output"])
    new_state = torch.full_like(d["state"], float("nan"))
    zero_plan = DecodePlan(**{**d, "state": None, "output": out, "new_state": new_state},
                           use_qk_l2norm=True)
    for _ in range(2):
        zero_plan.run()
        torch.cuda.synchronize()
        ref_o, ref_s = oracle_loop(**{**t, "state": None}, use_qk_l2norm=True)
        assert_output_close(out.cpu(), ref_o, what="null-state output")
        assert_state_close(new_state.cpu(), ref_s, what="null-state new_state")


def test_graph_of_mixed_shapes_and_the_bf16_state(hip_device):
    """A graph over layers of different batch, head layout, token count and
    state dtype replays to the same bits as the same plans run eagerly."""
    _announce("DecodeLayers mixed shapes: graph vs eager bits")
    specs = [(1, 16, 32, 1, torch.float32), (8, 4, 8, 2, torch.float32),
             (2, 16, 32, 1, torch.bfloat16), (64, 4, 8, 1, torch.float32)]
    runs = []
    for mode in ("eager", "graph"):
        layers_t = []
        for i, (B, H, HV, T, sd) in enumerate(specs):
            t = make_inputs(B, H, HV, seed=5200 + i, T=T)
            d = {n: (x.to(hip_device) if isinstance(x, torch.Tensor) else x)
                 for n, x in t.items()}
            d["state"] = d["state"].to(sd)
            d["new_state"] = d["state"]
            d["output"] = torch.empty(B, T, HV, 128, dtype=torch.bfloat16, device=hip_device)
            layers_t.append(d)
        layers = DecodeLayers(layers_t)
        if mode == "graph":
            layers.capture()
            for _ in range(2):
                layers.replay()
                torch.cuda.synchronize()
        else:
            for _ in range(2):
                layers.run()
                torch.cuda.synchronize()
        runs.append([(d["output"].clone(), d["state"].clone()) for d in layers_t])
        layers.close()
    for (o_e, s_e), (o_g, s_g) in zip(*runs):
        assert torch.equal(o_e, o_g) and torch.equal(s_e, s_g)


def test_repeat_calls_reuse_the_validated_launch(hip_device):
    """kernel_hip binds a validated call once and reruns its native plan for
    the same tensor objects: new inputs written into them between calls are
    used (each step against the oracle from the previous step's state), a
    tensor whose storage was replaced is validated and bound afresh, a
    tensor scale always takes the checked path, and freeing a bound tensor
    evicts its entry."""
    import gc

    import flashinfer_competition_codebase_amd as gdn
    from flashinfer_competition_codebase_amd import kernel as kmod

    _announce("kernel_hip repeat calls through the validated path")
    B, H, HV = 2, 4, 8
    t = make_inputs(B, H, HV, seed=5300)
    d = {n: (x.to(hip_device) if isinstance(x, torch.Tensor) else x) for n, x in t.items()}
    d["output"] = torch.empty(B, 1, HV, 128, dtype=torch.bfloat16, device=hip_device)
    d["new_state"] = d["state"]
    ref = t["state"].clone()
    sizes = []
    for step in range(4):
        fresh = make_inputs(B, H, HV, seed=5310 + step)
        for n in INPUTS:
            d[n].copy_(fresh[n].to(hip_device))
            t[n] = fresh[n]
        if step == 2:                            # same object, new storage
            d["state"].data = d["state"].clone()
            d["new_state"] = d["state"]
        gdn.kernel_hip(**d, use_qk_l2norm=True)
        torch.cuda.synchronize()
        ref = _check_step(f"repeat step {step}", t, d, ref, True)
        sizes.append(len(kmod._VALIDATED))
    assert sizes[1] == sizes[0] and sizes[3] == sizes[2], sizes   # hits add no entry
    key_count = sizes[-1]
    # a 0-d tensor scale is re-read every call: no entry for it
    gdn.kernel_hip(**{**d, "scale": torch.tensor(t["scale"])}, use_qk_l2norm=True)
    torch.cuda.synchronize()
    ref = _check_step("tensor scale", t, d, ref, True)
    assert len(kmod._VALIDATED) == key_count
    # freeing a bound tensor evicts the entry (no tensor is kept alive)
    out = d.pop("output")
    gdn.kernel_hip(**d, output=out, use_qk_l2norm=True)
    torch.cuda.synchronize()
    before = len(kmod._VALIDATED)
    del out
    gc.collect()
    assert len(kmod._VALIDATED) == before - 1
