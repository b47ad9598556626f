"""Checkpoint -> kernel-layout weight path (fastkernels_amd.weights).

The cases follow the reference's own tests of its loader
(tests/test_qwen36_spec.py:146-366, 486-606): split per-expert Hugging Face
names, grouped expert tensors, the DeltaNet and attention layers, root
names, the full 40-layer plan, key flattening and a two-shard checkpoint
with an index.  Added here: transposed grouped tensors, a directory with no
index, lazy reads (a shard the layer does not need is never opened) and the
error messages.  Packed values are checked against the source tensors they
came from (every expert filled with its own constant, so a misplaced slice
or a swapped gate/up half fails).
"""

from __future__ import annotations

import dataclasses
import json

import pytest
import torch

from fastkernels_amd.spec import Qwen36A3BSpec, qwen36_35b_a3b_spec, synthetic_qwen36_spec
from fastkernels_amd.weights import (
    SafetensorsCheckpoint,
    flatten_qwen36_moe_weight_keys,
    load_qwen36_attention_weights_from_safetensors,
    load_qwen36_linear_attention_weights_from_safetensors,
    load_qwen36_moe_weights_from_safetensors,
    pack_qwen36_attention_weights_from_state_dict,
    pack_qwen36_linear_attention_weights_from_state_dict,
    pack_qwen36_moe_weights_from_state_dict,
    resolve_qwen36_full_weight_plan,
    resolve_qwen36_moe_weight_keys,
    resolve_qwen36_root_weight_keys,
)

SPEC = synthetic_qwen36_spec()
H, E, I = SPEC.hidden_size, SPEC.num_experts, SPEC.expert_intermediate_size


def split_moe(prefix: str) -> dict[str, torch.Tensor]:
    t = {
        f"{prefix}.post_attention_layernorm.weight": torch.arange(H, dtype=torch.float32),
        f"{prefix}.mlp.gate.weight": torch.arange(E * H, dtype=torch.float32).reshape(E, H),
        f"{prefix}.mlp.shared_expert.gate_proj.weight": torch.full((I, H), 3.0),
        f"{prefix}.mlp.shared_expert.up_proj.weight": torch.full((I, H), 4.0),
        f"{prefix}.mlp.shared_expert.down_proj.weight": torch.full((H, I), 5.0),
    }
    for e in range(E):
        t[f"{prefix}.mlp.experts.{e}.gate_proj.weight"] = torch.full((I, H), float(e + 1))
        t[f"{prefix}.mlp.experts.{e}.up_proj.weight"] = torch.full((I, H), float(e + 11))
        t[f"{prefix}.mlp.experts.{e}.down_proj.weight"] = torch.full((H, I), float(e + 21))
    return t


def grouped_moe(prefix: str, transposed: bool = False, I: int = I) -> dict[str, torch.Tensor]:
    gu = torch.arange(E * 2 * I * H, dtype=torch.float32).reshape(E, 2 * I, H)
    dn = torch.arange(E * H * I, dtype=torch.float32).reshape(E, H, I)
    return {
        f"{prefix}.post_attention_layernorm.weight": torch.ones(H),
        f"{prefix}.mlp.gate.weight": torch.ones(E, H),
        f"{prefix}.mlp.experts.gate_up_proj": gu.transpose(1, 2).contiguous() if transposed else gu,
        f"{prefix}.mlp.experts.down_proj": dn.transpose(1, 2).contiguous() if transposed else dn,
        f"{prefix}.mlp.shared_expert.gate_proj.weight": torch.full((I, H), 3.0),
        f"{prefix}.mlp.shared_expert.up_proj.weight": torch.full((I, H), 4.0),
        f"{prefix}.mlp.shared_expert.down_proj.weight": torch.full((H, I), 5.0),
        f"{prefix}.mlp.shared_expert_gate.weight": torch.full((1, H), 0.5),
    }, gu, dn


def linear_attention(prefix: str, spec: Qwen36A3BSpec = SPEC) -> dict[str, torch.Tensor]:
    vw = spec.deltanet_value_heads * spec.deltanet_head_dim
    qkw = spec.deltanet_qk_heads * spec.deltanet_head_dim
    h, hv = spec.hidden_size, spec.deltanet_value_heads
    return {
        f"{prefix}.input_layernorm.weight": torch.ones(h),
        f"{prefix}.linear_attn.in_proj_qkv.weight": torch.ones(2 * qkw + vw, h),
        f"{prefix}.linear_attn.in_proj_z.weight": torch.ones(vw, h),
        f"{prefix}.linear_attn.out_proj.weight": torch.ones(h, vw),
        f"{prefix}.linear_attn.norm.weight": torch.ones(spec.deltanet_head_dim),
        f"{prefix}.linear_attn.A_log": torch.ones(hv),
        f"{prefix}.linear_attn.dt_bias": torch.ones(hv),
        f"{prefix}.linear_attn.in_proj_a.weight": torch.ones(hv, h),
        f"{prefix}.linear_attn.in_proj_b.weight": torch.ones(hv, h),
        f"{prefix}.linear_attn.conv1d.weight": torch.ones(2 * qkw + vw, 1, 4),
        f"{prefix}.post_attention_layernorm.weight": torch.ones(h),
    }


def attention(prefix: str, spec: Qwen36A3BSpec = SPEC) -> dict[str, torch.Tensor]:
    qw = spec.attention_heads * spec.attention_head_dim
    kvw = spec.attention_kv_heads * spec.attention_head_dim
    h = spec.hidden_size
    return {
        f"{prefix}.input_layernorm.weight": torch.ones(h),
        f"{prefix}.self_attn.q_proj.weight": torch.ones(2 * qw, h),  # gated q-proj: query and gate rows
        f"{prefix}.self_attn.k_proj.weight": torch.ones(kvw, h),
        f"{prefix}.self_attn.v_proj.weight": torch.ones(kvw, h),
        f"{prefix}.self_attn.o_proj.weight": torch.ones(h, qw),
        f"{prefix}.self_attn.q_norm.weight": torch.ones(spec.attention_head_dim),
        f"{prefix}.self_attn.k_norm.weight": torch.ones(spec.attention_head_dim),
        f"{prefix}.post_attention_layernorm.weight": torch.ones(h),
    }


def test_moe_key_resolution_split_layout():
    layer = 2
    t = split_moe(f"model.layers.{layer}")
    keys = resolve_qwen36_moe_weight_keys(t, layer, spec=SPEC)
    assert keys.norm_weight == f"model.layers.{layer}.post_attention_layernorm.weight"
    assert keys.router_weight == f"model.layers.{layer}.mlp.gate.weight"
    assert keys.expert_gate_up_weight[0] == (f"model.layers.{layer}.mlp.experts.0.gate_proj.weight",
                                             f"model.layers.{layer}.mlp.experts.0.up_proj.weight")
    assert keys.expert_down_weight[-1] == f"model.layers.{layer}.mlp.experts.{E - 1}.down_proj.weight"
    assert keys.shared_gate_up_weight == (f"model.layers.{layer}.mlp.shared_expert.gate_proj.weight",
                                          f"model.layers.{layer}.mlp.shared_expert.up_proj.weight")
    assert keys.shared_expert_gate_weight is None


def test_moe_packing_split_layout_places_every_expert():
    t = split_moe("model.layers.0")
    p = pack_qwen36_moe_weights_from_state_dict(t, 0, spec=SPEC)
    assert p.expert_gate_up_weight.shape == (E, 2 * I, H)
    assert p.expert_down_weight.shape == (E, H, I)
    for e in range(E):
        assert torch.equal(p.expert_gate_up_weight[e, :I], torch.full((I, H), float(e + 1)))
        assert torch.equal(p.expert_gate_up_weight[e, I:], torch.full((I, H), float(e + 11)))
        assert torch.equal(p.expert_down_weight[e], torch.full((H, I), float(e + 21)))
    assert torch.equal(p.shared_gate_up_weight[:I], torch.full((I, H), 3.0))
    assert torch.equal(p.shared_gate_up_weight[I:], torch.full((I, H), 4.0))
    assert torch.equal(p.router_weight, t["model.layers.0.mlp.gate.weight"])


def test_moe_packing_per_expert_packed_gate_up():
    t = split_moe("model.layers.1")
    for e in range(E):
        g = t.pop(f"model.layers.1.mlp.experts.{e}.gate_proj.weight")
        u = t.pop(f"model.layers.1.mlp.experts.{e}.up_proj.weight")
        t[f"model.layers.1.mlp.experts.{e}.gate_up_proj.weight"] = torch.cat((g, u))
    p = pack_qwen36_moe_weights_from_state_dict(t, 1, spec=SPEC)
    assert torch.equal(p.expert_gate_up_weight[2, I:], torch.full((I, H), 13.0))


@pytest.mark.parametrize("transposed", [False, True])
def test_moe_packing_grouped_layout(transposed):
    # (I = 4: with the synthetic I = 8, [E, 2I, H] and [E, H, 2I] are the
    # same shape and the orientation cannot be told from it)
    spec = dataclasses.replace(SPEC, expert_intermediate_size=4)
    prefix = "model.language_model.layers.0"
    t, gu, dn = grouped_moe(prefix, transposed, I=4)
    t[f"{prefix}.mlp.shared_expert.gate_proj.weight"] = torch.full((4, H), 3.0)
    t[f"{prefix}.mlp.shared_expert.up_proj.weight"] = torch.full((4, H), 4.0)
    t[f"{prefix}.mlp.shared_expert.down_proj.weight"] = torch.full((H, 4), 5.0)
    keys = resolve_qwen36_moe_weight_keys(t, 0, spec=spec)
    p = pack_qwen36_moe_weights_from_state_dict(t, 0, spec=spec)
    assert keys.expert_gate_up_weight == f"{prefix}.mlp.experts.gate_up_proj"
    assert keys.expert_down_weight == f"{prefix}.mlp.experts.down_proj"
    assert keys.shared_expert_gate_weight == f"{prefix}.mlp.shared_expert_gate.weight"
    assert p.shared_expert_gate_weight.shape == (1, H)
    assert torch.equal(p.expert_gate_up_weight, gu) and p.expert_gate_up_weight.is_contiguous()
    assert torch.equal(p.expert_down_weight, dn) and p.expert_down_weight.is_contiguous()


def test_moe_packing_rejects_wrong_shapes_and_missing_tensors():
    t = split_moe("model.layers.0")
    t["model.layers.0.mlp.experts.1.up_proj.weight"] = torch.ones(I + 1, H)
    with pytest.raises(ValueError, match=r"experts\.1\.up_proj\.weight has shape \(9, 16\), expected \(8, 16\)"):
        pack_qwen36_moe_weights_from_state_dict(t, 0, spec=SPEC)
    t = split_moe("model.layers.0")
    del t["model.layers.0.mlp.experts.3.down_proj.weight"]
    with pytest.raises(KeyError, match="missing expert 3 down projection"):
        resolve_qwen36_moe_weight_keys(t, 0, spec=SPEC)
    t = split_moe("model.layers.0")
    t["model.layers.0.mlp.experts.2.gate_proj.weight"] = torch.ones(I, H, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="dtype"):
        pack_qwen36_moe_weights_from_state_dict(t, 0, spec=SPEC)


def test_linear_attention_and_attention_packing():
    la = linear_attention("model.language_model.layers.0")
    p = pack_qwen36_linear_attention_weights_from_state_dict(la, 0, spec=SPEC)
    vw, qkw = SPEC.deltanet_value_heads * SPEC.deltanet_head_dim, SPEC.deltanet_qk_heads * SPEC.deltanet_head_dim
    assert p.in_proj_qkv_weight.shape == (2 * qkw + vw, H)
    assert p.out_proj_weight.shape == (H, vw)
    assert p.keys.in_proj_qkv_weight == "model.language_model.layers.0.linear_attn.in_proj_qkv.weight"
    at = attention("model.language_model.layers.3")
    q = pack_qwen36_attention_weights_from_state_dict(at, 3, spec=SPEC)
    assert q.q_proj_weight.shape == (2 * SPEC.attention_heads * SPEC.attention_head_dim, H)
    assert q.keys.q_proj_weight == "model.language_model.layers.3.self_attn.q_proj.weight"
    at["model.language_model.layers.3.self_attn.k_norm.weight"] = torch.ones(3)
    with pytest.raises(ValueError, match="k_norm.weight has shape"):
        pack_qwen36_attention_weights_from_state_dict(at, 3, spec=SPEC)


def test_root_keys_and_full_plan():
    t = {"model.language_model.embed_tokens.weight": object(), "model.language_model.norm.weight": object(),
         "lm_head.weight": object()}
    roots = resolve_qwen36_root_weight_keys(t)
    assert (roots.embedding_weight, roots.output_norm_weight, roots.lm_head_weight) == (
        "model.language_model.embed_tokens.weight", "model.language_model.norm.weight", "lm_head.weight")
    tied = resolve_qwen36_root_weight_keys({"model.embed_tokens.weight": 1, "model.norm.weight": 1})
    assert tied.lm_head_weight == "model.embed_tokens.weight"
    for layer, kind in enumerate(SPEC.layer_kinds()):
        prefix = f"model.language_model.layers.{layer}"
        t.update(linear_attention(prefix) if kind == "deltanet_moe" else attention(prefix))
        t.update(grouped_moe(prefix)[0])
    plan = resolve_qwen36_full_weight_plan(t, spec=SPEC)
    assert plan.layer_counts() == {"deltanet_moe": 3, "attention_moe": 1}
    assert plan.layers[0].linear_attention is not None and plan.layers[3].attention is not None
    assert len(plan.keys()) == len(set(plan.keys()))
    assert set(plan.keys()) == set(t)  # every tensor of the checkpoint is used, none twice
    shards = plan.required_shards({k: f"shard-{i % 2}.safetensors" for i, k in enumerate(plan.keys())})
    assert shards == ("shard-0.safetensors", "shard-1.safetensors")


def test_flattened_keys_include_shared_gate():
    t = grouped_moe("model.language_model.layers.0")[0]
    flat = flatten_qwen36_moe_weight_keys(resolve_qwen36_moe_weight_keys(t, 0, spec=SPEC))
    assert "model.language_model.layers.0.mlp.experts.gate_up_proj" in flat
    assert "model.language_model.layers.0.mlp.shared_expert_gate.weight" in flat
    assert len(flat) == len(t)


def test_spec_layer_kinds_and_hf_config():
    assert qwen36_35b_a3b_spec().layer_counts() == {"deltanet_moe": 30, "attention_moe": 10}
    cfg = {"text_config": {"hidden_size": 64, "num_hidden_layers": 3, "num_experts": 8, "num_experts_per_tok": 2,
                           "moe_intermediate_size": 16, "head_dim": 32, "partial_rotary_factor": 0.25,
                           "layer_types": ["linear_attention", "full_attention", "linear_attention"],
                           "rope_parameters": {"rope_theta": 1e7}}}
    spec = Qwen36A3BSpec.from_hf_config(cfg, name="cfg")
    assert spec.layer_kinds() == ("deltanet_moe", "attention_moe", "deltanet_moe")
    assert (spec.hidden_size, spec.num_experts, spec.num_routed_experts, spec.expert_intermediate_size) == (64, 8, 2, 16)
    assert spec.rope_dim == 8 and spec.rope_theta == 1e7 and spec.deltanet_value_heads == 32


def test_spec_alias_precedence_is_per_alias_then_source():
    # reference models/qwen36.py:120-127: each alias is tried in text_config
    # and then at the top level before the next alias is looked at
    cfg = {"moe_intermediate_size": 512, "num_experts": 64,
           "text_config": {"intermediate_size": 6144, "n_routed_experts": 32, "hidden_size": 2048,
                           "num_hidden_layers": 4, "num_layers": 9}}
    spec = Qwen36A3BSpec.from_hf_config(cfg)
    assert spec.expert_intermediate_size == 512
    assert spec.num_experts == 64
    assert spec.num_layers == 4  # the first alias in text_config wins over the second
    # a None value falls through to the next source / alias
    cfg = {"text_config": {"moe_intermediate_size": None, "hidden_size": 8, "num_hidden_layers": 1,
                           "num_experts": 2, "expert_intermediate_size": 24}, "moe_intermediate_size": 40}
    assert Qwen36A3BSpec.from_hf_config(cfg).expert_intermediate_size == 40


def test_spec_positional_order_and_derived_members():
    # field order of reference models/qwen36.py:15-32: layer_types, then rope_theta
    spec = Qwen36A3BSpec("s", 64, 4, 8, 2, 1, 16, 4, 2, 8, 4, 2, 8, 4, 128, 32,
                         ("linear_attention",) * 3 + ("full_attention",), 5e5)
    assert spec.layer_types[-1] == "full_attention" and spec.rope_theta == 5e5
    assert spec.active_experts_per_token == 3
    assert spec.attention_heads_per_kv_head == 2
    shapes = spec.decode_shapes(max_positions=10)
    assert shapes["deltanet_states"] == (3, 2, 8, 16)
    assert shapes["attention_key_cache"] == (1, 10, 2, 8) == shapes["attention_value_cache"]
    assert shapes["router_logits"] == (8,) and shapes["hidden_state"] == (64,)
    assert shapes["expert_gate_up_weight"] == (8, 32, 64) and shapes["expert_down_weight"] == (8, 64, 16)
    real = qwen36_35b_a3b_spec()
    assert real.active_experts_per_token == 9 and real.attention_heads_per_kv_head == 8
    with pytest.raises(ValueError, match="divisible"):
        dataclasses.replace(real, attention_kv_heads=3).attention_heads_per_kv_head


def _save_two_shards(tmp_path, with_index: bool):
    safetensors = pytest.importorskip("safetensors.torch")
    t = split_moe("model.layers.0")
    shard_a = {k: v for k, v in t.items() if ".experts." not in k and "shared_expert" not in k}
    shard_b = {k: v for k, v in t.items() if k not in shard_a}
    other = {"model.layers.7.mlp.gate.weight": torch.ones(E, H)}  # a layer this load does not need
    safetensors.save_file(shard_a, str(tmp_path / "model-00001-of-00003.safetensors"))
    safetensors.save_file(shard_b, str(tmp_path / "model-00002-of-00003.safetensors"))
    safetensors.save_file(other, str(tmp_path / "model-00003-of-00003.safetensors"))
    if with_index:
        wm = {k: "model-00001-of-00003.safetensors" for k in shard_a}
        wm.update({k: "model-00002-of-00003.safetensors" for k in shard_b})
        wm.update({k: "model-00003-of-00003.safetensors" for k in other})
        (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": wm}))
    return t


@pytest.mark.parametrize("with_index", [True, False])
def test_safetensors_loader_reads_only_the_layers_shards(tmp_path, with_index):
    t = _save_two_shards(tmp_path, with_index)
    ckpt = SafetensorsCheckpoint(tmp_path)
    p = pack_qwen36_moe_weights_from_state_dict(ckpt, 0, spec=SPEC)
    assert sorted(ckpt._open) == ["model-00001-of-00003.safetensors", "model-00002-of-00003.safetensors"]
    assert torch.equal(p.expert_gate_up_weight[1, :I], t["model.layers.0.mlp.experts.1.gate_proj.weight"])
    assert torch.equal(p.shared_gate_up_weight[I:], t["model.layers.0.mlp.shared_expert.up_proj.weight"])
    q = load_qwen36_moe_weights_from_safetensors(tmp_path, 0, spec=SPEC)
    for f in dataclasses.fields(p):
        a, b = getattr(p, f.name), getattr(q, f.name)
        assert torch.equal(a, b) if isinstance(a, torch.Tensor) else a == b


def test_safetensors_single_file_and_mixer_loaders(tmp_path):
    safetensors = pytest.importorskip("safetensors.torch")
    t = linear_attention("model.language_model.layers.0")
    t.update(attention("model.language_model.layers.3"))
    path = tmp_path / "one.safetensors"
    safetensors.save_file(t, str(path))
    la = load_qwen36_linear_attention_weights_from_safetensors(path, 0, spec=SPEC)
    at = load_qwen36_attention_weights_from_safetensors(path, 3, spec=SPEC)
    assert torch.equal(la.conv1d_weight, t["model.language_model.layers.0.linear_attn.conv1d.weight"])
    assert at.o_proj_weight.shape == (H, SPEC.attention_heads * SPEC.attention_head_dim)
    with pytest.raises(FileNotFoundError):
        SafetensorsCheckpoint(tmp_path / "empty_dir_does_not_exist")


def test_initial_decode_state_shapes():
    from fastkernels_amd.runner import initial_qwen36_real_decode_state

    spec = qwen36_35b_a3b_spec()
    st = initial_qwen36_real_decode_state(spec, max_positions=64)
    assert len(st.deltanet_conv_states) == 30 and len(st.attention_key_cache) == 10
    assert st.deltanet_conv_states[0].shape == (8192, 4)
    assert st.deltanet_recurrent_states[0].shape == (32, 128, 128)
    assert st.attention_key_cache[0].shape == (64, 2, 256) and st.position == 0
    assert all(float(t.abs().sum()) == 0.0 for t in st.deltanet_conv_states + st.attention_value_cache)


def test_spec_summary_lines():
    # reference models/qwen36.py:97-114: the field lines, then one line per
    # token count with its routed (token, expert) rows
    from fastkernels_amd.spec import qwen36_35b_a3b_spec

    lines = qwen36_35b_a3b_spec().summary_lines()
    assert lines[0] == "model: Qwen3.6-35B-A3B"
    assert "layers: 40" in lines and "hidden_size: 2048" in lines and "experts: 256" in lines
    assert "layer pattern: deltanet_moe, deltanet_moe, deltanet_moe, attention_moe x 10" in lines
    assert "deltanet/attention layers: 30/10" in lines
    assert "routed/shared active experts: 8/1" in lines
    assert lines[-3:] == ["tokens=1: routed_expert_rows=8", "tokens=16: routed_expert_rows=128",
                          "tokens=128: routed_expert_rows=1024"]
    assert qwen36_35b_a3b_spec().summary_lines([4])[-1] == "tokens=4: routed_expert_rows=32"
