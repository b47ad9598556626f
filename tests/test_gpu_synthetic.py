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


def _attn_layer(spec, dtype, seed):
    """An attention -> MoE layer of the synthetic spec (shapes of
    make_synthetic_qwen36_decode_weights, reference/qwen36_decode.py:134-147)."""

    g = torch.Generator().manual_seed(seed)

    def randn(*shape):
        return 0.3 * torch.randn(*shape, generator=g, dtype=dtype)

    H, E, I = spec.hidden_size, spec.num_experts, spec.expert_intermediate_size
    qw, kvw = spec.attention_heads * spec.attention_head_dim, spec.attention_kv_heads * spec.attention_head_dim
    return {
        "norm_weight": (1 + 0.1 * torch.randn(H, generator=g)).to(dtype),
        "router_weight": randn(E, H),
        "expert_gate_up_weight": randn(E, 2 * I, H),
        "expert_down_weight": randn(E, H, I),
        "shared_gate_up_weight": randn(2 * I, H),
        "shared_down_weight": randn(H, I),
        "q_weight": randn(qw, H),
        "k_weight": randn(kvw, H),
        "v_weight": randn(kvw, H),
        "out_weight": randn(H, qw),
    }


def _attn_inputs(spec, dtype, seed, max_positions=8):
    g = torch.Generator().manual_seed(seed)
    shape = (max_positions, spec.attention_kv_heads, spec.attention_head_dim)
    hidden = torch.randn(spec.hidden_size, generator=g).to(dtype)
    return hidden, torch.randn(*shape, generator=g).to(dtype), torch.randn(*shape, generator=g).to(dtype)


def _attn_kw(spec):
    return dict(attention_heads=spec.attention_heads, kv_heads=spec.attention_kv_heads,
                head_dim=spec.attention_head_dim, rope_dim=spec.rope_dim)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("position", [0, 2, 7])
def test_synthetic_attention(device, dtype, position):
    # reference tests/test_triton_moe.py:1189-1225
    spec = synthetic_qwen36_spec()
    layer = _attn_layer(spec, dtype, 123)
    hidden, kc, vc = _attn_inputs(spec, dtype, 7)
    ld = _gpu(layer, device)
    out, nkc, nvc = hip.hip_synthetic_qwen36_attention_decode(
        hidden.to(device), kc.to(device), vc.to(device), ld["norm_weight"], ld["q_weight"], ld["k_weight"],
        ld["v_weight"], ld["out_weight"], position=position, **_attn_kw(spec))
    r_out, r_kc, r_vc = oracle.synthetic_attention_decode(hidden, kc, vc, layer, position=position, **_attn_kw(spec))
    assert out.dtype == dtype and nkc.dtype == dtype
    torch.testing.assert_close(out.cpu(), r_out, **TOL[dtype])
    torch.testing.assert_close(nkc.cpu(), r_kc, **TOL[dtype])
    torch.testing.assert_close(nvc.cpu(), r_vc, **TOL[dtype])


def test_synthetic_attention_in_place_cache(device):
    # reference tests/test_triton_moe.py:1228-1271: copy_cache=False returns the
    # caller's caches, updated
    dtype = torch.bfloat16
    spec = synthetic_qwen36_spec()
    layer = _attn_layer(spec, dtype, 123)
    hidden, kc, vc = _attn_inputs(spec, dtype, 8)
    ld = _gpu(layer, device)
    kd, vd = kc.to(device), vc.to(device)
    out, nkc, nvc = hip.triton_synthetic_qwen36_attention_decode(
        hidden.to(device), kd, vd, ld["norm_weight"], ld["q_weight"], ld["k_weight"], ld["v_weight"],
        ld["out_weight"], position=2, copy_cache=False, **_attn_kw(spec))
    assert nkc.data_ptr() == kd.data_ptr() and nvc.data_ptr() == vd.data_ptr()
    r_out, r_kc, r_vc = oracle.synthetic_attention_decode(hidden, kc, vc, layer, position=2, **_attn_kw(spec))
    torch.testing.assert_close(out.cpu(), r_out, **TOL[dtype])
    torch.testing.assert_close(kd.cpu(), r_kc, **TOL[dtype])
    torch.testing.assert_close(vd.cpu(), r_vc, **TOL[dtype])
    # copy_cache=True (the default) leaves the caller's caches as they were
    kd2, vd2 = kc.to(device), vc.to(device)
    hip.hip_synthetic_qwen36_attention_decode(
        hidden.to(device), kd2, vd2, ld["norm_weight"], ld["q_weight"], ld["k_weight"], ld["v_weight"],
        ld["out_weight"], position=2, **_attn_kw(spec))
    assert torch.equal(kd2.cpu(), kc) and torch.equal(vd2.cpu(), vc)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_synthetic_attention_moe_layer(device, dtype):
    # reference tests/test_triton_moe.py:1299-1330, through the triton_* name
    spec = synthetic_qwen36_spec()
    layer = _attn_layer(spec, dtype, 321)
    hidden, kc, vc = _attn_inputs(spec, dtype, 9)
    out, nkc, nvc = hip.triton_synthetic_qwen36_attention_moe_decode(
        hidden.to(device), kc.to(device), vc.to(device), _gpu(layer, device), position=3,
        top_k=spec.num_routed_experts, **_attn_kw(spec))
    r_h, r_kc, r_vc = oracle.synthetic_attention_decode(hidden, kc, vc, layer, position=3, **_attn_kw(spec))
    r_h = oracle.synthetic_moe_decode(r_h, layer, spec.num_routed_experts)
    torch.testing.assert_close(out.cpu(), r_h, **TOL[dtype])
    torch.testing.assert_close(nkc.cpu(), r_kc, **TOL[dtype])
    torch.testing.assert_close(nvc.cpu(), r_vc, **TOL[dtype])


def test_reference_style_synthetic_decode_loop(device):
    """The decode loop of the reference's synthetic bench
    (bench/qwen36_decode_reference.py:65-154) with all three switches on the
    HIP blocks, called by their reference names, against the oracle's loop:
    4 layers (3 DeltaNet -> MoE, 1 attention -> MoE), 4 tokens, the DeltaNet
    states and the in-place KV caches carried from step to step.  In fp32:
    over 16 chained blocks the bf16 oracle's own rounding drifts past the
    bf16 tolerance (each bf16 block is checked on its own above)."""

    dtype = torch.float32

    from fastkernels_amd.kernels.hip import (  # the reference's names
        triton_synthetic_qwen36_attention_decode as triton_attention,
        triton_synthetic_qwen36_deltanet_decode as triton_deltanet,
        triton_synthetic_qwen36_moe_decode as triton_moe,
    )

    spec = synthetic_qwen36_spec()
    g = torch.Generator().manual_seed(77)
    H, V = spec.hidden_size, spec.vocab_size
    layers = []
    for i, kind in enumerate(spec.layer_kinds()):
        layer = _attn_layer(spec, dtype, 500 + i) if kind == "attention_moe" else _layer(spec, dtype, 500 + i)
        layer["kind"] = kind
        layers.append(layer)
    emb = (0.5 * torch.randn(V, H, generator=g)).to(dtype)
    out_norm = torch.ones(H, dtype=dtype)
    lm_head = (0.3 * torch.randn(V, H, generator=g)).to(dtype)
    n_dn = sum(k == "deltanet_moe" for k in spec.layer_kinds())
    dn_shape = (spec.deltanet_qk_heads, spec.deltanet_head_dim, spec.deltanet_value_dim_per_qk_head)
    cache_shape = (spec.context_length, spec.attention_kv_heads, spec.attention_head_dim)
    kw = dict(attention_heads=spec.attention_heads, kv_heads=spec.attention_kv_heads,
              head_dim=spec.attention_head_dim, rope_dim=spec.rope_dim)
    dkw = dict(qk_heads=spec.deltanet_qk_heads, head_dim=spec.deltanet_head_dim,
               value_dim_per_head=spec.deltanet_value_dim_per_qk_head)
    gl = [{k: (v.to(device) if torch.is_tensor(v) else v) for k, v in l.items()} for l in layers]
    st_h = [torch.zeros(dn_shape, dtype=dtype, device=device) for _ in range(n_dn)]
    kc_h, vc_h = torch.zeros(cache_shape, dtype=dtype, device=device), torch.zeros(cache_shape, dtype=dtype, device=device)
    st_o = [torch.zeros(dn_shape, dtype=dtype) for _ in range(n_dn)]
    kc_o, vc_o = torch.zeros(cache_shape, dtype=dtype), torch.zeros(cache_shape, dtype=dtype)
    for position, token in enumerate([3, 17, 5, 42]):
        print(f"synthetic decode loop dtype={dtype} position={position}", flush=True)
        h, ho, di = emb[token].to(device), emb[token], 0
        for l, lo in zip(gl, layers):
            if l["kind"] == "deltanet_moe":
                h, st_h[di] = triton_deltanet(h, st_h[di], l["norm_weight"], l["q_weight"], l["k_weight"],
                                              l["v_weight"], l["gate_weight"], l["out_weight"], **dkw)
                ho, st_o[di] = oracle.synthetic_deltanet_decode(ho, st_o[di], lo, **dkw)
                di += 1
            else:
                h, kc_h, vc_h = triton_attention(h, kc_h, vc_h, l["norm_weight"], l["q_weight"], l["k_weight"],
                                                 l["v_weight"], l["out_weight"], position=position, copy_cache=False,
                                                 **kw)
                ho, kc_o, vc_o = oracle.synthetic_attention_decode(ho, kc_o, vc_o, lo, position=position, **kw)
            h = triton_moe(h, l["norm_weight"], l["router_weight"], l["expert_gate_up_weight"],
                           l["expert_down_weight"], l["shared_gate_up_weight"], l["shared_down_weight"],
                           top_k=spec.num_routed_experts)
            ho = oracle.synthetic_moe_decode(ho, lo, spec.num_routed_experts)
        logits = oracle.rms_norm_plain(h.cpu(), out_norm) @ lm_head.transpose(0, 1)
        ref = oracle.rms_norm_plain(ho, out_norm) @ lm_head.transpose(0, 1)
        torch.testing.assert_close(logits, ref, **TOL[dtype])
        torch.testing.assert_close(kc_h.cpu(), kc_o, **TOL[dtype])
        for a, b in zip(st_h, st_o):
            torch.testing.assert_close(a.cpu(), b, **TOL[dtype])
