"""GPU parity of the Gated DeltaNet decode kernels and the DeltaNet -> MoE layer."""

from __future__ import annotations

import dataclasses

import pytest
import torch

import oracle
from fastkernels_amd import workloads as wl
from fastkernels_amd.kernels import hip
from fastkernels_amd.spec import qwen36_35b_a3b_spec
from tests.parity import assert_routing_parity, tol

pytestmark = pytest.mark.gpu

REAL = qwen36_35b_a3b_spec()
# small composite shapes of the reference layer test (tests/test_triton_moe.py:860-1008)
SMALL = dataclasses.replace(
    REAL, hidden_size=64, num_experts=16, num_routed_experts=4, expert_intermediate_size=32,
    deltanet_qk_heads=2, deltanet_value_heads=4, deltanet_head_dim=8,
)


def _dims(spec):
    return dict(qk_heads=spec.deltanet_qk_heads, value_heads=spec.deltanet_value_heads, head_dim=spec.deltanet_head_dim)


@pytest.fixture(scope="module")
def real_dn():
    return wl.make_deltanet_weights(REAL, seed=10)


def _to(d, device):
    return {k: (None if v is None else v.to(device)) for k, v in d.items()}


@pytest.mark.parametrize("spec_name,tokens", [("small", 1), ("small", 3), ("real", 1), ("real", 8)])
def test_project(device, real_dn, spec_name, tokens):
    spec = REAL if spec_name == "real" else SMALL
    w = real_dn if spec_name == "real" else wl.make_deltanet_weights(SMALL, seed=11)
    x = wl.make_hidden(tokens, spec.hidden_size, seed=12 + tokens)
    wd = _to(w, device)
    outs = hip.hip_qwen36_batched_deltanet_project(
        x.to(device), wd["input_norm_weight"], wd["in_proj_qkv_weight"], wd["in_proj_z_weight"],
        wd["in_proj_a_weight"], wd["in_proj_b_weight"],
    )
    refs = oracle.deltanet_project(x, w["input_norm_weight"], w["in_proj_qkv_weight"], w["in_proj_z_weight"],
                                   w["in_proj_a_weight"], w["in_proj_b_weight"])
    for o, r in zip(outs, refs):
        assert o.dtype == torch.float32 and o.shape == r.shape
        torch.testing.assert_close(o.cpu(), r, atol=1e-3, rtol=1e-3)


@pytest.mark.parametrize("tokens", [1, 2, 8])
@pytest.mark.parametrize("state_dtype", [torch.float32, torch.bfloat16])
def test_conv(device, tokens, state_dtype):
    g = torch.Generator().manual_seed(tokens)
    C, KS = 8192, 4
    mixed = torch.randn(tokens, C, generator=g)
    state = (0.5 * torch.randn(C, KS, generator=g)).to(state_dtype)
    w = (0.5 * torch.randn(C, 1, KS, generator=g)).to(state_dtype)
    out, nxt = hip.hip_qwen36_batched_deltanet_conv(mixed.to(device), state.to(device), w.to(device))
    r_out, r_nxt = oracle.causal_conv_update(mixed, state, w)
    torch.testing.assert_close(out.cpu(), r_out, atol=1e-5, rtol=1e-5)
    assert nxt.dtype == state_dtype
    torch.testing.assert_close(nxt.cpu().float(), r_nxt.float(), atol=0, rtol=0)


def _recurrent_inputs(spec, tokens, seed):
    g = torch.Generator().manual_seed(seed)
    Hk, Hv, D = spec.deltanet_qk_heads, spec.deltanet_value_heads, spec.deltanet_head_dim
    return dict(
        mixed_qkv=torch.randn(tokens, 2 * Hk * D + Hv * D, generator=g),
        z=torch.randn(tokens, Hv * D, generator=g),
        a_logits=torch.randn(tokens, Hv, generator=g),
        b_logits=torch.randn(tokens, Hv, generator=g),
        recurrent_state=0.1 * torch.randn(Hv, D, D, generator=g),
        out_proj_weight=(0.02 * torch.randn(spec.hidden_size, Hv * D, generator=g)).bfloat16(),
        linear_norm_weight=torch.randn(D, generator=g),
        a_log=0.02 * torch.randn(Hv, generator=g),
        dt_bias=0.02 * torch.randn(Hv, generator=g),
    )


@pytest.mark.parametrize("spec_name,tokens", [("small", 1), ("small", 4), ("small", 17), ("real", 1), ("real", 8), ("real", 20)])
def test_recurrent_output(device, spec_name, tokens):
    spec = REAL if spec_name == "real" else SMALL
    inp = _recurrent_inputs(spec, tokens, 20 + tokens)
    upd, nxt = hip.hip_qwen36_batched_deltanet_recurrent_output(*[v.to(device) for v in inp.values()], **_dims(spec))
    r_upd, r_nxt = oracle.deltanet_recurrent_output(*inp.values(), **_dims(spec))
    torch.testing.assert_close(nxt.cpu(), r_nxt, atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(upd.cpu(), r_upd, atol=2e-3, rtol=2e-3)


def test_recurrent_t_rows_equal_t_single_steps(device):
    inp = _recurrent_inputs(REAL, 4, 31)
    d = {k: v.to(device) for k, v in inp.items()}
    upd, final = hip.hip_qwen36_batched_deltanet_recurrent_output(*d.values(), **_dims(REAL))
    state = d["recurrent_state"]
    for t in range(4):
        step = dict(d)
        for key in ("mixed_qkv", "z", "a_logits", "b_logits"):
            step[key] = d[key][t : t + 1]
        step["recurrent_state"] = state
        u, state = hip.hip_qwen36_batched_deltanet_recurrent_output(*step.values(), **_dims(REAL))
        torch.testing.assert_close(u[0], upd[t], atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(state, final, atol=1e-6, rtol=1e-6)


@pytest.mark.parametrize("spec_name,tokens", [("small", 2), ("small", 17), ("real", 1), ("real", 8)])
def test_deltanet_moe_layer(device, spec_name, tokens):
    spec = REAL if spec_name == "real" else SMALL
    dn = wl.make_deltanet_weights(spec, seed=40)
    moe = wl.make_moe_weights(spec, seed=41)
    x = wl.make_hidden(tokens, spec.hidden_size, seed=42)
    dnd, moed = _to(dn, device), _to(moe, device)
    res = hip.hip_qwen36_batched_deltanet_moe_layer_decode(
        x.to(device), dnd["conv_state"], dnd["recurrent_state"], dnd["input_norm_weight"], dnd["in_proj_qkv_weight"],
        dnd["in_proj_z_weight"], dnd["in_proj_a_weight"], dnd["in_proj_b_weight"], dnd["conv1d_weight"],
        dnd["out_proj_weight"], dnd["linear_norm_weight"], dnd["a_log"], dnd["dt_bias"],
        moed["norm_weight"], moed["router_weight"], moed["expert_gate_up_weight"], moed["expert_down_weight"],
        moed["shared_gate_up_weight"], moed["shared_down_weight"], moed["shared_expert_gate_weight"],
        top_k=spec.num_routed_experts, **_dims(spec),
    )
    assert len(res) == 9
    ref = oracle.deltanet_moe_layer(x, dn["conv_state"], dn["recurrent_state"], dn, moe,
                                    top_k=spec.num_routed_experts, **_dims(spec))
    layer_hidden, dn_hidden, dn_update, moe_update, conv_state, rec_state, logits, ids, w = res
    torch.testing.assert_close(dn_update.cpu(), ref[2], **tol(torch.bfloat16))
    torch.testing.assert_close(dn_hidden.cpu(), ref[1], **tol(torch.bfloat16))
    assert conv_state.dtype == dn["conv_state"].dtype
    torch.testing.assert_close(conv_state.cpu().float(), ref[4].float(), atol=1e-2, rtol=1e-2)
    torch.testing.assert_close(rec_state.cpu(), ref[5], atol=1e-3, rtol=1e-3)
    near = assert_routing_parity(logits, ids, w, ref[6], spec.num_routed_experts)
    # experts checked under the kernel's routing (independent of near-ties)
    h = dn_hidden.cpu()
    r = oracle.routed_experts(h, ids.cpu(), w.cpu(), moe["expert_gate_up_weight"], moe["expert_down_weight"])
    r = r + oracle.shared_expert(h, moe["shared_gate_up_weight"], moe["shared_down_weight"], moe["shared_expert_gate_weight"])
    torch.testing.assert_close(moe_update.cpu(), r, **tol(torch.bfloat16))
    torch.testing.assert_close(layer_hidden.cpu(), h + r, **tol(torch.bfloat16))
    if near == 0:
        torch.testing.assert_close(layer_hidden.cpu(), ref[0], **tol(torch.bfloat16))


@pytest.mark.parametrize("tokens", [1, 2, 3, 5, 8])
def test_step_single_launch_matches_oracle(device, real_dn, tokens):
    # fk_deltanet_step at the real shapes takes the single-launch kernel:
    # VALU projections for T <= 2, MFMA projections with bf16 hi/lo
    # activations (swizzled staging, T = 3 and 5 use padded columns) above;
    # heads split over four workgroups; tagged hand-offs.
    from fastkernels_amd.plan import DeltaNetStepPlan

    x = wl.make_hidden(tokens, REAL.hidden_size, seed=60 + tokens)
    plan = DeltaNetStepPlan(_to(real_dn, device), tokens, REAL)
    plan.hidden.copy_(x.to(device))
    plan.run()
    plan.check_device()  # no bounded wait ran out (synchronises)
    update, conv, state = oracle.deltanet_update(
        x, real_dn["conv_state"], real_dn["recurrent_state"], real_dn, **_dims(REAL))
    torch.testing.assert_close(plan.update.cpu(), update, **tol(torch.bfloat16))
    torch.testing.assert_close(plan.hidden_out.cpu(), x.float() + update, **tol(torch.bfloat16))
    torch.testing.assert_close(plan.next_recurrent_state.cpu(), state, atol=1e-3, rtol=1e-3)
    torch.testing.assert_close(plan.next_conv_state.cpu().float(), conv.float(), atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("tokens", [1, 2, 5])
def test_step_single_launch_other_conv_kernel_size(device, real_dn, tokens):
    # A conv kernel size other than the model's 4 (here 3) takes the general
    # causal-conv epilogue of the single launch: at T <= 2 the window entries
    # selected through run-time compares, above from the LDS sequence.
    from fastkernels_amd.plan import DeltaNetStepPlan

    dn = dict(real_dn)
    dn["conv_state"] = real_dn["conv_state"][:, :3].contiguous()
    dn["conv1d_weight"] = real_dn["conv1d_weight"][..., :3].contiguous()
    x = wl.make_hidden(tokens, REAL.hidden_size, seed=90 + tokens)
    plan = DeltaNetStepPlan(_to(dn, device), tokens, REAL)
    plan.hidden.copy_(x.to(device))
    plan.run()
    plan.check_device()
    update, conv, state = oracle.deltanet_update(x, dn["conv_state"], dn["recurrent_state"], dn, **_dims(REAL))
    assert plan.next_conv_state.shape[1] == 3
    torch.testing.assert_close(plan.update.cpu(), update, **tol(torch.bfloat16))
    torch.testing.assert_close(plan.next_recurrent_state.cpu(), state, atol=1e-3, rtol=1e-3)
    torch.testing.assert_close(plan.next_conv_state.cpu().float(), conv.float(), atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("tokens", [1, 2, 5, 8])
def test_step_single_launch_matches_staged_kernels(device, real_dn, tokens):
    # Same step through the staged operator kernels (fp32 VALU GEMVs).
    from fastkernels_amd.plan import DeltaNetStepPlan

    x = wl.make_hidden(tokens, REAL.hidden_size, seed=70 + tokens).to(device)
    wd = _to(real_dn, device)
    plan = DeltaNetStepPlan(wd, tokens, REAL)
    plan.hidden.copy_(x)
    plan.run()
    mixed, z, a, b = hip.hip_qwen36_batched_deltanet_project(
        x, wd["input_norm_weight"], wd["in_proj_qkv_weight"], wd["in_proj_z_weight"],
        wd["in_proj_a_weight"], wd["in_proj_b_weight"])
    mixed, conv = hip.hip_qwen36_batched_deltanet_conv(mixed, wd["conv_state"], wd["conv1d_weight"])
    update, state = hip.hip_qwen36_batched_deltanet_recurrent_output(
        mixed, z, a, b, wd["recurrent_state"], wd["out_proj_weight"], wd["linear_norm_weight"], wd["a_log"],
        wd["dt_bias"], **_dims(REAL))
    torch.cuda.synchronize()
    torch.testing.assert_close(plan.update, update, atol=1e-4, rtol=1e-3)
    torch.testing.assert_close(plan.next_recurrent_state, state, atol=1e-5, rtol=1e-4)
    torch.testing.assert_close(plan.next_conv_state.float(), conv.float(), atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("tokens", [1, 2, 3])
def test_step_single_launch_narrower_hidden(device, tokens):
    # H = 1024: the single launch stages its projection tiles through the
    # MFMA path at every token count (the VALU path needs H = 2048), and its
    # LDS must be sized for that path at T <= 2 too.
    from fastkernels_amd.plan import DeltaNetStepPlan

    spec = dataclasses.replace(REAL, hidden_size=1024)
    wd = _to(wl.make_deltanet_weights(spec, seed=11), device)
    x = wl.make_hidden(tokens, spec.hidden_size, seed=75 + tokens).to(device)
    plan = DeltaNetStepPlan(wd, tokens, spec)
    plan.hidden.copy_(x)
    plan.run()
    mixed, z, a, b = hip.hip_qwen36_batched_deltanet_project(
        x, wd["input_norm_weight"], wd["in_proj_qkv_weight"], wd["in_proj_z_weight"],
        wd["in_proj_a_weight"], wd["in_proj_b_weight"])
    mixed, conv = hip.hip_qwen36_batched_deltanet_conv(mixed, wd["conv_state"], wd["conv1d_weight"])
    update, state = hip.hip_qwen36_batched_deltanet_recurrent_output(
        mixed, z, a, b, wd["recurrent_state"], wd["out_proj_weight"], wd["linear_norm_weight"], wd["a_log"],
        wd["dt_bias"], **_dims(spec))
    torch.cuda.synchronize()
    torch.testing.assert_close(plan.update, update, atol=1e-4, rtol=1e-3)
    torch.testing.assert_close(plan.next_recurrent_state, state, atol=1e-5, rtol=1e-4)
    torch.testing.assert_close(plan.next_conv_state.float(), conv.float(), atol=1e-2, rtol=1e-2)


def test_step_single_launch_repeated_calls_stay_consistent(device, real_dn):
    # The launch tag advances every launch: cycling inputs through one
    # workspace must keep reproducing each input's first result bit for bit.
    from fastkernels_amd.plan import DeltaNetStepPlan

    plan = DeltaNetStepPlan(_to(real_dn, device), 2, REAL)
    xs = [wl.make_hidden(2, REAL.hidden_size, seed=80 + i).to(device) for i in range(3)]
    first = []
    for x in xs:
        plan.hidden.copy_(x)
        plan.run()
        first.append((plan.update.clone(), plan.next_recurrent_state.clone()))
    for _ in range(4):
        for x, (u, s) in zip(xs, first):
            plan.hidden.copy_(x)
            plan.run()
            assert torch.equal(plan.update, u)
            assert torch.equal(plan.next_recurrent_state, s)
    plan.check_device()
