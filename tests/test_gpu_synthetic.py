"""GPU parity of the synthetic (tiny-spec) blocks behind the --moe-impl /
--deltanet-impl switch (reference tests/test_triton_moe.py:1112-1295)."""

from __future__ import annotations

import dataclasses

import pytest
import torch

import oracle
from fastkernels_amd.kernels import hip
from fastkernels_amd.spec import synthetic_qwen36_spec

pytestmark = pytest.mark.gpu

# reference default_tolerance (testing/tolerances.py:8-18)
TOL = {torch.float32: dict(atol=1e-4, rtol=1e-4), torch.bfloat16: dict(atol=3e-2, rtol=3e-2)}


def _layer(spec, dtype, seed):
    """Weights in the generation order of make_synthetic_qwen36_decode_weights
    (reference/qwen36_decode.py:103-137) for a DeltaNet layer."""

    g = torch.Generator().manual_seed(seed)

    def randn(*shape):
        return (0.02 * torch.randn(*shape, generator=g, dtype=dtype))

    H, E, I = spec.hidden_size, spec.num_experts, spec.expert_intermediate_size
    vw = spec.deltanet_qk_heads * spec.deltanet_value_dim_per_qk_head
    return {
        "norm_weight": torch.ones(H, dtype=dtype),
        "router_weight": randn(E, H),
        "expert_gate_up_weight": randn(E, 2 * I, H),
        "expert_down_weight": randn(E, H, I),
        "shared_gate_up_weight": randn(2 * I, H),
        "shared_down_weight": randn(H, I),
        "q_weight": randn(spec.deltanet_qk_heads * spec.deltanet_head_dim, H),
        "k_weight": randn(spec.deltanet_qk_heads * spec.deltanet_head_dim, H),
        "v_weight": randn(vw, H),
        "gate_weight": randn(vw, H),
        "out_weight": randn(H, vw),
    }


def _gpu(layer, device):
    return {k: v.to(device) for k, v in layer.items()}


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("top_k", [1, 2, 4, 8])
def test_synthetic_moe(device, dtype, top_k):
    spec = synthetic_qwen36_spec()
    spec = dataclasses.replace(spec, num_experts=max(spec.num_experts, top_k), num_routed_experts=top_k)
    layer = _layer(spec, dtype, 123)
    hidden = torch.randn(spec.hidden_size, generator=torch.Generator().manual_seed(1)).to(dtype)
    ld = _gpu(layer, device)
    out = hip.hip_synthetic_qwen36_moe_decode(
        hidden.to(device), ld["norm_weight"], ld["router_weight"], ld["expert_gate_up_weight"],
        ld["expert_down_weight"], ld["shared_gate_up_weight"], ld["shared_down_weight"], top_k=top_k,
    )
    assert out.dtype == dtype
    ref = oracle.synthetic_moe_decode(hidden, layer, top_k)
    torch.testing.assert_close(out.cpu(), ref, **TOL[dtype])


def test_synthetic_moe_256_experts(device):
    spec = dataclasses.replace(synthetic_qwen36_spec(), num_experts=256, num_routed_experts=8)
    layer = _layer(spec, torch.bfloat16, 123)
    hidden = torch.randn(spec.hidden_size, generator=torch.Generator().manual_seed(2)).bfloat16()
    ld = _gpu(layer, device)
    out = hip.hip_synthetic_qwen36_moe_decode(
        hidden.to(device), ld["norm_weight"], ld["router_weight"], ld["expert_gate_up_weight"],
        ld["expert_down_weight"], ld["shared_gate_up_weight"], ld["shared_down_weight"], top_k=8,
    )
    torch.testing.assert_close(out.cpu(), oracle.synthetic_moe_decode(hidden, layer, 8), **TOL[torch.bfloat16])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_synthetic_deltanet(device, dtype):
    spec = synthetic_qwen36_spec()
    layer = _layer(spec, dtype, 123)
    g = torch.Generator().manual_seed(3)
    hidden = torch.randn(spec.hidden_size, generator=g).to(dtype)
    state = torch.randn(spec.deltanet_state_shape(), generator=g).to(dtype)
    ld = _gpu(layer, device)
    dims = dict(qk_heads=spec.deltanet_qk_heads, head_dim=spec.deltanet_head_dim,
                value_dim_per_head=spec.deltanet_value_dim_per_qk_head)
    h, s = hip.hip_synthetic_qwen36_deltanet_decode(
        hidden.to(device), state.to(device), ld["norm_weight"], ld["q_weight"], ld["k_weight"], ld["v_weight"],
        ld["gate_weight"], ld["out_weight"], **dims,
    )
    rh, rs = oracle.synthetic_deltanet_decode(hidden, state, layer, **dims)
    torch.testing.assert_close(h.cpu(), rh, **TOL[dtype])
    torch.testing.assert_close(s.cpu(), rs, **TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_synthetic_deltanet_moe_layer(device, dtype):
    spec = synthetic_qwen36_spec()
    layer = _layer(spec, dtype, 123)
    g = torch.Generator().manual_seed(4)
    hidden = torch.randn(spec.hidden_size, generator=g).to(dtype)
    state = torch.randn(spec.deltanet_state_shape(), generator=g).to(dtype)
    dims = dict(qk_heads=spec.deltanet_qk_heads, head_dim=spec.deltanet_head_dim,
                value_dim_per_head=spec.deltanet_value_dim_per_qk_head)
    h, s = hip.hip_synthetic_qwen36_deltanet_moe_decode(
        hidden.to(device), state.to(device), _gpu(layer, device), top_k=spec.num_routed_experts, **dims
    )
    rh, rs = oracle.synthetic_deltanet_decode(hidden, state, layer, **dims)
    rh = oracle.synthetic_moe_decode(rh, layer, spec.num_routed_experts)
    torch.testing.assert_close(h.cpu(), rh, **TOL[dtype])
    torch.testing.assert_close(s.cpu(), rs, **TOL[dtype])
