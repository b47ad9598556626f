"""The failure path of the kernels' bounded in-kernel waits, forced from the host.

The MoE and DeltaNet-step kernels hand values between workgroups through
tagged words and wait for them with a bounded poll.  Here the host sets the
bound to zero (fk_workspace_set_poll_limit), so every wait gives up at once
and every kernel still ends normally; the checks are that the outputs are
NaN, that fk_workspace_status reports FK_ERR_DEVICE, that later calls stay
poisoned until the flag is cleared, and that after clearing the results are
again bit-identical to an untouched run.  No kernel faults or hangs: each
wait returns, it just reports failure.
"""

from __future__ import annotations

import dataclasses

import pytest
import torch

from fastkernels_amd import _lib
from fastkernels_amd import workloads as wl
from fastkernels_amd.kernels import hip
from fastkernels_amd.plan import DeltaNetStepPlan, MoeLayerPlan
from fastkernels_amd.spec import qwen36_35b_a3b_spec

pytestmark = pytest.mark.gpu

SPEC = qwen36_35b_a3b_spec()
SMALL = dataclasses.replace(SPEC, num_experts=64, expert_intermediate_size=256, hidden_size=1024)


@pytest.fixture(scope="module")
def small_moe(device):
    return wl.make_moe_weights(SMALL, seed=31, device=device)


@pytest.fixture(scope="module")
def model_moe(device):
    return wl.make_moe_weights(SPEC, seed=36, device=device)


@pytest.fixture(scope="module")
def dn_weights(device):
    return wl.make_deltanet_weights(SPEC, seed=32, device=device)


def _expect_device_error(plan):
    with pytest.raises(_lib.FastKernelsError) as info:
        plan.check_device()
    assert info.value.status == _lib.FK_ERR_DEVICE


def _outputs(plan):
    if isinstance(plan, MoeLayerPlan):
        return [plan.moe_out, plan.layer_out, plan.weights]
    return [plan.update, plan.hidden_out, plan.next_recurrent_state]


def _exercise(plan):
    plan.run()
    plan.check_device()
    good = [t.clone() for t in _outputs(plan)]
    assert all(bool(torch.isfinite(t).all()) for t in good)
    # every wait gives up at once: NaN outputs, flagged, every kernel ends
    plan.set_poll_limit(0)
    plan.run()
    torch.cuda.synchronize()
    for t in _outputs(plan):
        assert bool(torch.isnan(t).all()), "a failed wait must poison every output"
    # the flag is sticky: with the normal bound back, calls stay poisoned ...
    plan.set_poll_limit(None)
    plan.run()
    torch.cuda.synchronize()
    assert bool(torch.isnan(_outputs(plan)[0]).all())
    # ... until it is read and cleared; then results equal the untouched run
    _expect_device_error(plan)
    plan.run()
    plan.check_device()
    for a, b in zip(_outputs(plan), good):
        assert torch.equal(a, b)


@pytest.mark.parametrize("tokens", [1, 16, 300])
def test_moe_layer_wait_failure_is_poisoned_and_flagged(device, small_moe, tokens):
    # T = 1: single-launch layer; T = 16: tagged router + GEMV experts;
    # T = 300: grid-barrier router + MFMA experts
    print(f"moe wait failure tokens={tokens}", flush=True)
    plan = MoeLayerPlan(small_moe, tokens)
    plan.hidden.copy_(wl.make_hidden(tokens, SMALL.hidden_size, seed=33).to(device))
    _exercise(plan)


def test_moe_layer_model_shape_t1_wait_failure_is_poisoned_and_flagged(device, model_moe):
    # the model's shape at T = 1 takes the single launch's straight-line
    # variant (one workgroup per gate/up block, down item and row group)
    print("moe wait failure model shape T=1", flush=True)
    plan = MoeLayerPlan(model_moe, 1)
    plan.hidden.copy_(wl.make_hidden(1, SPEC.hidden_size, seed=37).to(device))
    _exercise(plan)


@pytest.mark.parametrize("tokens", [1, 8])
def test_deltanet_step_wait_failure_is_poisoned_and_flagged(device, dn_weights, tokens):
    print(f"deltanet wait failure tokens={tokens}", flush=True)
    plan = DeltaNetStepPlan(dn_weights, tokens, SPEC)
    plan.hidden.copy_(wl.make_hidden(tokens, SPEC.hidden_size, seed=34).to(device))
    _exercise(plan)


def test_operator_workspace_status_reports_and_clears(device, small_moe):
    w = small_moe
    args = (w["norm_weight"], w["router_weight"], w["expert_gate_up_weight"], w["expert_down_weight"],
            w["shared_gate_up_weight"], w["shared_down_weight"], w["shared_expert_gate_weight"])
    x = wl.make_hidden(4, SMALL.hidden_size, seed=35).to(device)
    good = hip.hip_qwen36_batched_moe_decode(x, *args, top_k=8)[0].clone()
    hip.workspace_status(device)
    # the operators' cached workspace for this stream and kind
    ws = [t for (kind, _, _), t in hip._workspaces.items() if kind == "moe"]
    assert ws
    stream = torch.cuda.current_stream(device).cuda_stream
    for t in ws:
        _lib.call("fk_workspace_set_poll_limit", t.data_ptr(), t.numel(), 0, stream)
    bad = hip.hip_qwen36_batched_moe_decode(x, *args, top_k=8)[0]
    assert bool(torch.isnan(bad).all())
    for t in ws:
        _lib.call("fk_workspace_set_poll_limit", t.data_ptr(), t.numel(), -1, stream)
    with pytest.raises(_lib.FastKernelsError) as info:
        hip.workspace_status(device)
    assert info.value.status == _lib.FK_ERR_DEVICE
    again = hip.hip_qwen36_batched_moe_decode(x, *args, top_k=8)[0]
    hip.workspace_status(device)
    assert torch.equal(again, good)


@pytest.mark.parametrize("tokens", [1, 4])
def test_attention_step_wait_failure_is_poisoned_and_flagged(device, tokens):
    # the single-launch attention step (T <= 4): every wait gives up at once
    # -> NaN update and hidden_out, the step's own cache rows NaN, the
    # position not advanced, the flag set; after clearing, the step at the
    # same position equals the untouched run bit for bit
    from fastkernels_amd.plan import AttentionStepPlan

    print(f"attention wait failure tokens={tokens}", flush=True)
    start, maxp = 21, 32
    plan = AttentionStepPlan(wl.make_attention_weights(SPEC, seed=36, device=device), tokens, SPEC,
                             max_positions=maxp, start_position=start)
    g = torch.Generator().manual_seed(37)
    plan.key_cache.copy_(torch.randn(maxp, SPEC.attention_kv_heads, SPEC.attention_head_dim, generator=g).to(device))
    plan.value_cache.copy_(torch.randn(maxp, SPEC.attention_kv_heads, SPEC.attention_head_dim, generator=g).to(device))
    plan.hidden.copy_(wl.make_hidden(tokens, SPEC.hidden_size, seed=38).to(device))
    own = slice(start, start + tokens)
    plan.run()
    plan.check_device()
    good = [plan.update.clone(), plan.hidden_out.clone(), plan.key_cache.clone()]
    assert all(bool(torch.isfinite(t).all()) for t in good)
    assert int(plan.position.item()) == start + tokens
    plan.set_poll_limit(0)
    plan.set_position(start)
    plan.run()
    torch.cuda.synchronize()
    assert bool(torch.isnan(plan.update).all()) and bool(torch.isnan(plan.hidden_out).all())
    assert bool(torch.isnan(plan.key_cache[own]).all())
    assert torch.equal(plan.key_cache[:start], good[2][:start])
    assert int(plan.position.item()) == start  # (the epoch keeper's wait failed too)
    plan.set_poll_limit(None)
    plan.run()
    torch.cuda.synchronize()
    assert bool(torch.isnan(plan.update).all())
    _expect_device_error(plan)
    plan.set_position(start)
    plan.run()
    plan.check_device()
    for a, b in zip([plan.update, plan.hidden_out, plan.key_cache], good):
        assert torch.equal(a, b)
