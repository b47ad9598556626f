"""A checkpoint on disk through the loader into the HIP kernels.

Per-expert bf16 tensors with Hugging Face names, in two safetensors shards
with an index, are packed straight onto the GPU by
`load_qwen36_moe_weights_from_safetensors`; the MoE layer computed from them
must match the CPU oracle on the same tensors packed on the host (routing
bit-exact, outputs within tests/parity.py's bf16 tolerance), and a
`MoeLayerPlan` built from the packed dataclass must give the operator's
answer.  Shapes are a reduced Qwen3.6 layer (32 experts, H = 512, I = 128,
top-8) so the shards stay a few MB.
"""

from __future__ import annotations

import dataclasses
import json

import pytest
import torch

import oracle
from fastkernels_amd import workloads as wl
from fastkernels_amd.kernels import hip
from fastkernels_amd.spec import qwen36_35b_a3b_spec
from fastkernels_amd.weights import load_qwen36_moe_weights_from_safetensors, pack_qwen36_moe_weights_from_state_dict
from tests.parity import assert_routing_parity, tol

pytestmark = pytest.mark.gpu

SPEC = dataclasses.replace(qwen36_35b_a3b_spec(), num_experts=32, hidden_size=512, expert_intermediate_size=128)
H, E, I, K = SPEC.hidden_size, SPEC.num_experts, SPEC.expert_intermediate_size, SPEC.num_routed_experts


def _checkpoint(tmp_path) -> dict[str, torch.Tensor]:
    safetensors = pytest.importorskip("safetensors.torch")
    g = torch.Generator().manual_seed(5)

    def rnd(*shape, scale=0.02):
        return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)

    p = "model.language_model.layers.0"
    t = {
        f"{p}.post_attention_layernorm.weight": rnd(H, scale=0.1),
        f"{p}.mlp.gate.weight": rnd(E, H),
        f"{p}.mlp.shared_expert.gate_proj.weight": rnd(I, H),
        f"{p}.mlp.shared_expert.up_proj.weight": rnd(I, H),
        f"{p}.mlp.shared_expert.down_proj.weight": rnd(H, I),
        f"{p}.mlp.shared_expert_gate.weight": rnd(1, H),
    }
    for e in range(E):
        t[f"{p}.mlp.experts.{e}.gate_proj.weight"] = rnd(I, H)
        t[f"{p}.mlp.experts.{e}.up_proj.weight"] = rnd(I, H)
        t[f"{p}.mlp.experts.{e}.down_proj.weight"] = rnd(H, I)
    names = sorted(t)
    shards = {"model-00001-of-00002.safetensors": names[::2], "model-00002-of-00002.safetensors": names[1::2]}
    for file, keys in shards.items():
        safetensors.save_file({k: t[k] for k in keys}, str(tmp_path / file))
    wm = {k: f for f, keys in shards.items() for k in keys}
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": wm}))
    return t


def _args(w):
    return (w.norm_weight, w.router_weight, w.expert_gate_up_weight, w.expert_down_weight, w.shared_gate_up_weight,
            w.shared_down_weight, w.shared_expert_gate_weight)


@pytest.mark.parametrize("tokens", [1, 5])
def test_checkpoint_layer_through_kernels(device, tmp_path, tokens):
    t = _checkpoint(tmp_path)
    gpu = load_qwen36_moe_weights_from_safetensors(tmp_path, 0, spec=SPEC, device=device)
    cpu = pack_qwen36_moe_weights_from_state_dict(t, 0, spec=SPEC)
    assert gpu.expert_gate_up_weight.device.type == "cuda" and gpu.expert_gate_up_weight.dtype == torch.bfloat16
    assert torch.equal(gpu.expert_gate_up_weight.cpu(), cpu.expert_gate_up_weight)
    assert torch.equal(gpu.expert_down_weight.cpu(), cpu.expert_down_weight)

    x = wl.make_hidden(tokens, H, seed=11)
    lh, moe, logits, ids, w = hip.hip_qwen36_batched_moe_layer_decode(x.to(device), *_args(gpu), top_k=K)
    o_lh, o_moe, o_logits, o_ids, o_w = oracle.moe_layer(x, *_args(cpu), top_k=K)
    near = assert_routing_parity(logits, ids, w, o_logits, K)
    if near == 0:
        assert torch.equal(ids.cpu(), o_ids)
        torch.testing.assert_close(moe.cpu(), o_moe, **tol(torch.bfloat16))
        torch.testing.assert_close(lh.cpu(), o_lh, **tol(torch.bfloat16))

    from fastkernels_amd.plan import MoeLayerPlan

    plan = MoeLayerPlan(gpu, tokens)
    plan.hidden.copy_(x.to(device))
    plan.run()
    plan.check_device()
    assert torch.equal(plan.ids, ids)
    torch.testing.assert_close(plan.layer_out, lh, atol=1e-5, rtol=1e-5)
