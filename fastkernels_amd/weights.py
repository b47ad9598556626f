"""Checkpoint tensors -> the layouts the kernels read.

Host side of the hot path's weight format (reference
models/qwen36_weights.py:161-716, models/qwen36_full.py:88-196): resolve the
Hugging Face tensor names of one layer, check every shape, and pack

* routed experts into ``[E, 2I, H]`` (gate rows 0..I-1, then up rows) and
  ``[E, H, I]``, whether the checkpoint stores one tensor per expert and
  projection, one ``gate_up`` tensor per expert, or grouped ``[E, ...]``
  tensors (either orientation; the ``[E, H, 2I]`` / ``[E, I, H]`` forms are
  transposed);
* the shared expert into ``[2I, H]`` and ``[H, I]``.

Loading differs from the reference in how memory is used, not in what
comes out:

* ``safetensors`` files are opened lazily (``safe_open``); only the tensors
  a layer needs are read, shard by shard, and the header's key list stands
  in for the index when a directory has none;
* packed tensors are allocated once on the target device and each source
  tensor is copied into its slice there, so a 1.6 GB bf16 MoE layer never
  exists twice in host memory (no host-side ``stack``/``cat``);
* dtypes are kept (a bf16 checkpoint stays bf16: the kernels read bf16).

Errors follow the reference: a missing tensor raises ``KeyError("missing
<what>; tried: ...")``, a wrong shape ``ValueError("<name> has shape ...,
expected ...")``.
"""

from __future__ import annotations

import json
from dataclasses import dataclass, fields
from pathlib import Path
from typing import Any, Iterable, Mapping

import torch

from .spec import Qwen36A3BSpec, qwen36_35b_a3b_spec

LAYER_PREFIXES: tuple[str, ...] = (
    "model.layers",
    "model.language_model.layers",
    "language_model.model.layers",
    "transformer.layers",
    "layers",
)
ROOT_PREFIXES: tuple[str, ...] = ("model.language_model", "model", "language_model.model", "transformer", "")

# Tensor-name alternatives of the Hugging Face Qwen3.x MoE layouts (a data
# format: the names have to match the checkpoints').
_MOE_NORM = ("post_attention_layernorm.weight", "pre_feedforward_layernorm.weight", "mlp_norm.weight",
             "input_layernorm.weight")
_ROUTER = ("mlp.gate.weight", "mlp.router.weight", "mlp.router.linear.weight")
_GROUPED_GATE_UP = ("gate_up_proj", "gate_up_proj.weight", "gate_up", "gate_up.weight", "w1", "w1.weight")
_GROUPED_DOWN = ("down_proj", "down_proj.weight", "down", "down.weight", "w2", "w2.weight")
_PACKED_GATE_UP = ("gate_up_proj.weight", "gate_up.weight", "w1.weight")
_GATE = ("gate_proj.weight", "gate.weight", "w1_gate.weight")
_UP = ("up_proj.weight", "up.weight", "w1_up.weight")
_DOWN = ("down_proj.weight", "down.weight", "w2.weight")
_SHARED = ("shared_expert", "shared_experts.0")


# ---------------------------------------------------------------------------
# Resolved names and packed tensors (field names as in the reference)
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class Qwen36MoEWeightKeys:
    """Source tensor names of one MoE layer.  Expert entries are one grouped
    name, or per expert a packed name or a (gate, up) pair."""

    norm_weight: str
    router_weight: str
    expert_gate_up_weight: tuple[tuple[str, str] | str, ...] | str
    expert_down_weight: tuple[str, ...] | str
    shared_gate_up_weight: tuple[str, str] | str
    shared_down_weight: str
    shared_expert_gate_weight: str | None = None


@dataclass(frozen=True)
class Qwen36MoEWeights:
    """Kernel-facing tensors of one MoE layer."""

    norm_weight: Any
    router_weight: Any
    expert_gate_up_weight: Any
    expert_down_weight: Any
    shared_gate_up_weight: Any
    shared_down_weight: Any
    keys: Qwen36MoEWeightKeys
    shared_expert_gate_weight: Any | None = None

    def as_dict(self) -> dict[str, Any]:
        """The tensors by field name (what `plan.MoeLayerPlan` takes)."""

        return tensor_fields(self)


@dataclass(frozen=True)
class Qwen36LinearAttentionWeightKeys:
    input_norm_weight: str
    in_proj_qkv_weight: str
    in_proj_z_weight: str
    out_proj_weight: str
    linear_norm_weight: str
    a_log: str
    dt_bias: str
    in_proj_a_weight: str
    in_proj_b_weight: str
    conv1d_weight: str
    post_attention_norm_weight: str


@dataclass(frozen=True)
class Qwen36LinearAttentionWeights:
    input_norm_weight: Any
    in_proj_qkv_weight: Any
    in_proj_z_weight: Any
    out_proj_weight: Any
    linear_norm_weight: Any
    a_log: Any
    dt_bias: Any
    in_proj_a_weight: Any
    in_proj_b_weight: Any
    conv1d_weight: Any
    post_attention_norm_weight: Any
    keys: Qwen36LinearAttentionWeightKeys

    def as_dict(self) -> dict[str, Any]:
        return tensor_fields(self)


@dataclass(frozen=True)
class Qwen36AttentionWeightKeys:
    input_norm_weight: str
    q_proj_weight: str
    k_proj_weight: str
    v_proj_weight: str
    o_proj_weight: str
    q_norm_weight: str
    k_norm_weight: str
    post_attention_norm_weight: str


@dataclass(frozen=True)
class Qwen36AttentionWeights:
    input_norm_weight: Any
    q_proj_weight: Any
    k_proj_weight: Any
    v_proj_weight: Any
    o_proj_weight: Any
    q_norm_weight: Any
    k_norm_weight: Any
    post_attention_norm_weight: Any
    keys: Qwen36AttentionWeightKeys

    def as_dict(self) -> dict[str, Any]:
        return tensor_fields(self)


@dataclass(frozen=True)
class Qwen36RootWeightKeys:
    embedding_weight: str
    output_norm_weight: str
    lm_head_weight: str


@dataclass(frozen=True)
class Qwen36LayerWeightPlan:
    layer_idx: int
    layer_kind: str
    moe: Qwen36MoEWeightKeys
    linear_attention: Qwen36LinearAttentionWeightKeys | None = None
    attention: Qwen36AttentionWeightKeys | None = None

    def keys(self) -> tuple[str, ...]:
        names: list[str] = []
        for mixer in (self.linear_attention, self.attention):
            if mixer is not None:
                names.extend(str(getattr(mixer, f.name)) for f in fields(mixer))
        names.extend(flatten_qwen36_moe_weight_keys(self.moe))
        return tuple(dict.fromkeys(names))


@dataclass(frozen=True)
class Qwen36FullWeightPlan:
    spec: Qwen36A3BSpec
    roots: Qwen36RootWeightKeys
    layers: tuple[Qwen36LayerWeightPlan, ...]

    def keys(self) -> tuple[str, ...]:
        names = [self.roots.embedding_weight, self.roots.output_norm_weight, self.roots.lm_head_weight]
        for layer in self.layers:
            names.extend(layer.keys())
        return tuple(dict.fromkeys(names))

    def required_shards(self, weight_map: Mapping[str, str]) -> tuple[str, ...]:
        return tuple(sorted({str(weight_map[k]) for k in self.keys()}))

    def layer_counts(self) -> dict[str, int]:
        kinds = [layer.layer_kind for layer in self.layers]
        return {"deltanet_moe": kinds.count("deltanet_moe"), "attention_moe": kinds.count("attention_moe")}


def tensor_fields(obj: Any) -> dict[str, Any]:
    """Field name -> value of a packed-weights dataclass, without `keys`."""

    return {f.name: getattr(obj, f.name) for f in fields(obj) if f.name != "keys"}


# ---------------------------------------------------------------------------
# Name resolution
# ---------------------------------------------------------------------------
def _bases(layer_idx: int, prefixes: tuple[str, ...]) -> list[str]:
    return [f"{p}.{layer_idx}" if p else str(layer_idx) for p in prefixes]


def _candidates(bases: Iterable[str], middles: Iterable[str], suffixes: Iterable[str]) -> list[str]:
    out = []
    for b in bases:
        for m in middles:
            for s in suffixes:
                out.append(".".join(x for x in (b, m, s) if x))
    return out


def _pick(names: Any, candidates: list[str]) -> str | None:
    for c in candidates:
        if c in names:
            return c
    return None


def _need(names: Any, candidates: list[str], label: str) -> str:
    found = _pick(names, candidates)
    if found is None:
        shown = "\n  ".join(candidates[:16])
        raise KeyError(f"missing {label}; tried:\n  {shown}")
    return found


def resolve_qwen36_moe_weight_keys(
    tensors: Any,
    layer_idx: int,
    *,
    spec: Qwen36A3BSpec | None = None,
    layer_prefixes: tuple[str, ...] = LAYER_PREFIXES,
) -> Qwen36MoEWeightKeys:
    """Tensor names of MoE layer `layer_idx` (reference qwen36_weights.py:161-348).

    `tensors` is anything with `in` over names (a state dict, a key set, a
    lazy checkpoint).  Grouped expert tensors win when both grouped names
    are present; otherwise every expert needs a packed gate/up or a gate and
    an up tensor, and a down tensor.
    """

    spec = spec or qwen36_35b_a3b_spec()
    bases = _bases(layer_idx, layer_prefixes)
    norm = _need(tensors, _candidates(bases, [""], _MOE_NORM), "MoE input norm weight")
    router = _need(tensors, _candidates(bases, [""], _ROUTER), "router weight")
    g_gu = _pick(tensors, _candidates(bases, ["mlp.experts"], _GROUPED_GATE_UP))
    g_dn = _pick(tensors, _candidates(bases, ["mlp.experts"], _GROUPED_DOWN))
    if g_gu is not None and g_dn is not None:
        gate_up: Any = g_gu
        down: Any = g_dn
    else:
        gu_items: list[tuple[str, str] | str] = []
        dn_items: list[str] = []
        for e in range(spec.num_experts):
            mid = [f"mlp.experts.{e}"]
            packed = _pick(tensors, _candidates(bases, mid, _PACKED_GATE_UP))
            if packed is not None:
                gu_items.append(packed)
            else:
                gu_items.append((_need(tensors, _candidates(bases, mid, _GATE), f"expert {e} gate projection"),
                                 _need(tensors, _candidates(bases, mid, _UP), f"expert {e} up projection")))
            dn_items.append(_need(tensors, _candidates(bases, mid, _DOWN), f"expert {e} down projection"))
        gate_up, down = tuple(gu_items), tuple(dn_items)
    shared_mid = [f"mlp.{s}" for s in _SHARED]
    s_packed = _pick(tensors, _candidates(bases, shared_mid, _PACKED_GATE_UP))
    if s_packed is not None:
        s_gate_up: Any = s_packed
    else:
        s_gate_up = (_need(tensors, _candidates(bases, shared_mid, _GATE), "shared expert gate projection"),
                     _need(tensors, _candidates(bases, shared_mid, _UP), "shared expert up projection"))
    s_down = _need(tensors, _candidates(bases, shared_mid, _DOWN), "shared expert down projection")
    s_gate = _pick(tensors, _candidates(bases, ["mlp.shared_expert_gate"], ("weight",)))
    return Qwen36MoEWeightKeys(norm, router, gate_up, down, s_gate_up, s_down, s_gate)


def flatten_qwen36_moe_weight_keys(keys: Qwen36MoEWeightKeys) -> tuple[str, ...]:
    """Every tensor name the resolved MoE keys refer to (reference qwen36_full.py:88-110)."""

    names = [keys.norm_weight, keys.router_weight, keys.shared_down_weight]
    for group in (keys.expert_gate_up_weight, keys.expert_down_weight, keys.shared_gate_up_weight):
        if isinstance(group, str):
            names.append(group)
            continue
        for item in group:
            names.extend([item] if isinstance(item, str) else item)
    if keys.shared_expert_gate_weight is not None:
        names.append(keys.shared_expert_gate_weight)
    return tuple(names)


_LINEAR_ATTENTION_NAMES = {
    "input_norm_weight": ("input_layernorm.weight", "linear-attention input norm weight"),
    "in_proj_qkv_weight": ("linear_attn.in_proj_qkv.weight", "linear-attention packed QKV projection"),
    "in_proj_z_weight": ("linear_attn.in_proj_z.weight", "linear-attention Z projection"),
    "out_proj_weight": ("linear_attn.out_proj.weight", "linear-attention output projection"),
    "linear_norm_weight": ("linear_attn.norm.weight", "linear-attention inner norm weight"),
    "a_log": ("linear_attn.A_log", "linear-attention A_log"),
    "dt_bias": ("linear_attn.dt_bias", "linear-attention dt_bias"),
    "in_proj_a_weight": ("linear_attn.in_proj_a.weight", "linear-attention A projection"),
    "in_proj_b_weight": ("linear_attn.in_proj_b.weight", "linear-attention B projection"),
    "conv1d_weight": ("linear_attn.conv1d.weight", "linear-attention conv1d weight"),
    "post_attention_norm_weight": ("post_attention_layernorm.weight", "post-attention norm weight"),
}
_ATTENTION_NAMES = {
    "input_norm_weight": ("input_layernorm.weight", "attention input norm weight"),
    "q_proj_weight": ("self_attn.q_proj.weight", "attention Q projection"),
    "k_proj_weight": ("self_attn.k_proj.weight", "attention K projection"),
    "v_proj_weight": ("self_attn.v_proj.weight", "attention V projection"),
    "o_proj_weight": ("self_attn.o_proj.weight", "attention output projection"),
    "q_norm_weight": ("self_attn.q_norm.weight", "attention Q norm"),
    "k_norm_weight": ("self_attn.k_norm.weight", "attention K norm"),
    "post_attention_norm_weight": ("post_attention_layernorm.weight", "post-attention norm weight"),
}


def _resolve_table(tensors: Any, layer_idx: int, prefixes: tuple[str, ...], table: dict, cls: type) -> Any:
    bases = _bases(layer_idx, prefixes)
    return cls(**{f: _need(tensors, _candidates(bases, [""], (suffix,)), label) for f, (suffix, label) in table.items()})


def resolve_qwen36_linear_attention_weight_keys(
    tensors: Any, layer_idx: int, *, layer_prefixes: tuple[str, ...] = LAYER_PREFIXES
) -> Qwen36LinearAttentionWeightKeys:
    """Tensor names of Gated DeltaNet layer `layer_idx` (reference qwen36_weights.py:351-382)."""

    return _resolve_table(tensors, layer_idx, layer_prefixes, _LINEAR_ATTENTION_NAMES, Qwen36LinearAttentionWeightKeys)


def resolve_qwen36_attention_weight_keys(
    tensors: Any, layer_idx: int, *, layer_prefixes: tuple[str, ...] = LAYER_PREFIXES
) -> Qwen36AttentionWeightKeys:
    """Tensor names of full-attention layer `layer_idx` (reference qwen36_weights.py:385-413)."""

    return _resolve_table(tensors, layer_idx, layer_prefixes, _ATTENTION_NAMES, Qwen36AttentionWeightKeys)


def resolve_qwen36_root_weight_keys(tensors: Any, *, prefixes: tuple[str, ...] = ROOT_PREFIXES) -> Qwen36RootWeightKeys:
    """Embedding, final norm and LM head names (reference qwen36_full.py:113-154).
    A checkpoint without an LM head ties it to the embedding."""

    def cands(suffix: str) -> list[str]:
        return [f"{p}.{suffix}" if p else suffix for p in prefixes]

    emb = _need(tensors, cands("embed_tokens.weight") + cands("wte.weight"), "token embedding weight")
    norm = _need(tensors, cands("norm.weight") + cands("final_layernorm.weight"), "final norm weight")
    head = _need(tensors, ["lm_head.weight", "model.lm_head.weight", "model.language_model.lm_head.weight",
                           "language_model.lm_head.weight", emb], "LM head weight")
    return Qwen36RootWeightKeys(emb, norm, head)


def resolve_qwen36_full_weight_plan(tensors: Any, *, spec: Qwen36A3BSpec | None = None) -> Qwen36FullWeightPlan:
    """Names of every tensor of a full decode pass, layer kinds from the spec
    (reference qwen36_full.py:157-196)."""

    spec = spec or qwen36_35b_a3b_spec()
    roots = resolve_qwen36_root_weight_keys(tensors)
    layers = []
    for i, kind in enumerate(spec.layer_kinds()):
        moe = resolve_qwen36_moe_weight_keys(tensors, i, spec=spec)
        if kind == "deltanet_moe":
            layers.append(Qwen36LayerWeightPlan(i, kind, moe,
                                                linear_attention=resolve_qwen36_linear_attention_weight_keys(tensors, i)))
        elif kind == "attention_moe":
            layers.append(Qwen36LayerWeightPlan(i, kind, moe, attention=resolve_qwen36_attention_weight_keys(tensors, i)))
        else:
            raise ValueError(f"unknown Qwen3.6 layer kind at layer {i}: {kind}")
    return Qwen36FullWeightPlan(spec, roots, tuple(layers))


# ---------------------------------------------------------------------------
# Packing
# ---------------------------------------------------------------------------
def _shape(t: Any) -> tuple[int, ...]:
    return tuple(int(d) for d in t.shape)


def _check(name: str, t: Any, expected: tuple[int, ...]) -> None:
    if _shape(t) != expected:
        raise ValueError(f"{name} has shape {_shape(t)}, expected {expected}")


def _dev(device: Any) -> torch.device | None:
    return None if device is None else torch.device(device)


def _place(t: torch.Tensor, device: Any) -> torch.Tensor:
    d = _dev(device)
    t = t if d is None else t.to(d)
    return t.contiguous()


def _grouped(t: torch.Tensor, name: str, canonical: tuple[int, ...], device: Any) -> torch.Tensor:
    """A grouped [E, a, b] tensor in canonical orientation (an [E, b, a]
    source is transposed while it is copied to the device)."""

    s = _shape(t)
    if s != canonical and s == (canonical[0], canonical[2], canonical[1]):
        t = t.transpose(1, 2)
    _check(name, t, canonical)
    return _place(t, device)


def pack_qwen36_moe_weights_from_state_dict(
    tensors: Mapping[str, Any],
    layer_idx: int,
    *,
    spec: Qwen36A3BSpec | None = None,
    layer_prefixes: tuple[str, ...] = LAYER_PREFIXES,
    device: str | torch.device | None = None,
) -> Qwen36MoEWeights:
    """Pack MoE layer `layer_idx` (reference qwen36_weights.py:416-527).

    Per-expert sources are copied straight into their slices of one
    ``[E, 2I, H]`` / ``[E, H, I]`` tensor allocated on `device` (default:
    the sources' device).  `tensors[name]` is read once per name, so a lazy
    mapping loads each tensor when it is packed.
    """

    spec = spec or qwen36_35b_a3b_spec()
    keys = resolve_qwen36_moe_weight_keys(tensors, layer_idx, spec=spec, layer_prefixes=layer_prefixes)
    E, H, I = spec.num_experts, spec.hidden_size, spec.expert_intermediate_size

    norm = tensors[keys.norm_weight]
    router = tensors[keys.router_weight]
    _check(keys.norm_weight, norm, (H,))
    _check(keys.router_weight, router, (E, H))

    def slices_into(dst_shape: tuple[int, ...], parts: Iterable[tuple[Any, str, tuple[int, ...]]]) -> torch.Tensor:
        # each source is read once: shape-checked, then copied into its slice
        dst = None
        for index, name, want in parts:
            src = tensors[name]
            _check(name, src, want)
            if dst is None:
                dst = torch.empty(dst_shape, dtype=src.dtype, device=_dev(device) or src.device)
            elif src.dtype != dst.dtype:
                raise ValueError(f"{name} has dtype {src.dtype}, expected {dst.dtype} like the layer's other experts")
            dst[index].copy_(src)
        return dst

    if isinstance(keys.expert_gate_up_weight, str):
        gate_up = _grouped(tensors[keys.expert_gate_up_weight], keys.expert_gate_up_weight, (E, 2 * I, H), device)
    else:
        parts = []
        for e, item in enumerate(keys.expert_gate_up_weight):
            if isinstance(item, str):
                parts.append(((e,), item, (2 * I, H)))
            else:
                parts.append(((e, slice(0, I)), item[0], (I, H)))
                parts.append(((e, slice(I, 2 * I)), item[1], (I, H)))
        gate_up = slices_into((E, 2 * I, H), parts)

    if isinstance(keys.expert_down_weight, str):
        down = _grouped(tensors[keys.expert_down_weight], keys.expert_down_weight, (E, H, I), device)
    else:
        down = slices_into((E, H, I), [((e,), n, (H, I)) for e, n in enumerate(keys.expert_down_weight)])

    if isinstance(keys.shared_gate_up_weight, str):
        s_gate_up = tensors[keys.shared_gate_up_weight]
        _check(keys.shared_gate_up_weight, s_gate_up, (2 * I, H))
        s_gate_up = _place(s_gate_up, device)
    else:
        g, u = keys.shared_gate_up_weight
        s_gate_up = slices_into((2 * I, H), [(slice(0, I), g, (I, H)), (slice(I, 2 * I), u, (I, H))])

    s_down = tensors[keys.shared_down_weight]
    _check(keys.shared_down_weight, s_down, (H, I))
    s_gate = None
    if keys.shared_expert_gate_weight is not None:
        s_gate = tensors[keys.shared_expert_gate_weight]
        if _shape(s_gate) not in ((H,), (1, H)):
            raise ValueError(f"{keys.shared_expert_gate_weight} has shape {_shape(s_gate)}, expected ({H},) or (1, {H})")
        s_gate = _place(s_gate, device)
    return Qwen36MoEWeights(
        norm_weight=_place(norm, device),
        router_weight=_place(router, device),
        expert_gate_up_weight=gate_up,
        expert_down_weight=down,
        shared_gate_up_weight=s_gate_up,
        shared_down_weight=_place(s_down, device),
        keys=keys,
        shared_expert_gate_weight=s_gate,
    )


def pack_qwen36_linear_attention_weights_from_state_dict(
    tensors: Mapping[str, Any],
    layer_idx: int,
    *,
    spec: Qwen36A3BSpec | None = None,
    layer_prefixes: tuple[str, ...] = LAYER_PREFIXES,
    device: str | torch.device | None = None,
) -> Qwen36LinearAttentionWeights:
    """Gated DeltaNet layer tensors, shape-checked (reference qwen36_weights.py:530-596)."""

    spec = spec or qwen36_35b_a3b_spec()
    keys = resolve_qwen36_linear_attention_weight_keys(tensors, layer_idx, layer_prefixes=layer_prefixes)
    H, Hv, D = spec.hidden_size, spec.deltanet_value_heads, spec.deltanet_head_dim
    vw, qkw = Hv * D, spec.deltanet_qk_heads * D
    conv_ch = 2 * qkw + vw
    expected = {
        "input_norm_weight": (H,), "in_proj_qkv_weight": (conv_ch, H), "in_proj_z_weight": (vw, H),
        "out_proj_weight": (H, vw), "linear_norm_weight": (D,), "a_log": (Hv,), "dt_bias": (Hv,),
        "in_proj_a_weight": (Hv, H), "in_proj_b_weight": (Hv, H), "post_attention_norm_weight": (H,),
    }
    out = {}
    for f in fields(keys):
        name = getattr(keys, f.name)
        t = tensors[name]
        if f.name == "conv1d_weight":
            if t.ndim != 3 or int(t.shape[0]) != conv_ch:
                raise ValueError(f"{name} has shape {_shape(t)}, expected ({conv_ch}, *, *)")
        else:
            _check(name, t, expected[f.name])
        out[f.name] = _place(t, device)
    return Qwen36LinearAttentionWeights(keys=keys, **out)


def pack_qwen36_attention_weights_from_state_dict(
    tensors: Mapping[str, Any],
    layer_idx: int,
    *,
    spec: Qwen36A3BSpec | None = None,
    layer_prefixes: tuple[str, ...] = LAYER_PREFIXES,
    device: str | torch.device | None = None,
) -> Qwen36AttentionWeights:
    """Full-attention layer tensors, shape-checked (reference qwen36_weights.py:599-653).
    The Q projection may carry the output gate (gated q-proj: twice the Q
    width), so only its input width is fixed; likewise the O projection's
    output width."""

    spec = spec or qwen36_35b_a3b_spec()
    keys = resolve_qwen36_attention_weight_keys(tensors, layer_idx, layer_prefixes=layer_prefixes)
    H, kvw, hd = spec.hidden_size, spec.attention_kv_heads * spec.attention_head_dim, spec.attention_head_dim
    out = {}
    for f in fields(keys):
        name = getattr(keys, f.name)
        t = tensors[name]
        if f.name == "q_proj_weight":
            if t.ndim != 2 or int(t.shape[1]) != H:
                raise ValueError(f"{name} has shape {_shape(t)}, expected (*, {H})")
        elif f.name == "o_proj_weight":
            if t.ndim != 2 or int(t.shape[0]) != H:
                raise ValueError(f"{name} has shape {_shape(t)}, expected ({H}, *)")
        else:
            want = {"input_norm_weight": (H,), "k_proj_weight": (kvw, H), "v_proj_weight": (kvw, H),
                    "q_norm_weight": (hd,), "k_norm_weight": (hd,), "post_attention_norm_weight": (H,)}[f.name]
            _check(name, t, want)
        out[f.name] = _place(t, device)
    return Qwen36AttentionWeights(keys=keys, **out)


# ---------------------------------------------------------------------------
# Lazy safetensors checkpoints
# ---------------------------------------------------------------------------
class SafetensorsCheckpoint(Mapping[str, torch.Tensor]):
    """Read-only name -> CPU tensor view of a ``.safetensors`` file or of a
    directory of shards.  Names come from ``*.safetensors.index.json``
    when present, else from the shards' headers; a tensor is read from its
    shard only when it is looked up (``safe_open``, no unpickling)."""

    def __init__(self, path: str | Path) -> None:
        try:
            from safetensors import safe_open
        except ImportError as exc:  # pragma: no cover - optional dependency
            raise RuntimeError("safetensors is required to load Qwen3.6 checkpoints") from exc
        self._safe_open = safe_open
        src = Path(path)
        self.root = src if src.is_dir() else src.parent
        self.weight_map: dict[str, str] = {}
        if src.is_dir():
            index = sorted(src.glob("*.safetensors.index.json"))
            if index:
                with index[0].open("r", encoding="utf-8") as fh:
                    wm = json.load(fh).get("weight_map", {})
                if not isinstance(wm, dict):
                    raise ValueError(f"{index[0]} does not contain a valid weight_map")
                self.weight_map = {str(k): str(v) for k, v in wm.items()}
            else:
                self._scan(sorted(src.glob("*.safetensors")))
        else:
            self._scan([src])
        if not self.weight_map:
            raise FileNotFoundError(f"no safetensors tensors found at {src}")
        self._open: dict[str, Any] = {}

    def _scan(self, files: list[Path]) -> None:
        for f in files:
            with self._safe_open(str(f), framework="pt", device="cpu") as h:
                for k in h.keys():
                    self.weight_map[k] = f.name

    def _handle(self, shard: str) -> Any:
        h = self._open.get(shard)
        if h is None:
            path = self.root / shard
            if not path.exists():
                raise FileNotFoundError(f"safetensors shard {path} named by the index does not exist")
            h = self._safe_open(str(path), framework="pt", device="cpu")
            self._open[shard] = h
        return h

    def __getitem__(self, key: str) -> torch.Tensor:
        shard = self.weight_map.get(key)
        if shard is None:
            raise KeyError(key)
        return self._handle(shard).get_tensor(key)

    def __contains__(self, key: object) -> bool:
        return key in self.weight_map

    def __iter__(self):
        return iter(self.weight_map)

    def __len__(self) -> int:
        return len(self.weight_map)

    def shards_for(self, names: Iterable[str]) -> tuple[str, ...]:
        return tuple(sorted({self.weight_map[n] for n in names}))


def load_qwen36_moe_weights_from_safetensors(
    path: str | Path,
    layer_idx: int,
    *,
    spec: Qwen36A3BSpec | None = None,
    layer_prefixes: tuple[str, ...] = LAYER_PREFIXES,
    device: str | torch.device | None = None,
) -> Qwen36MoEWeights:
    """Load and pack one MoE layer from a ``.safetensors`` file or a directory
    of shards (reference qwen36_weights.py:656-716): only that layer's
    tensors are read."""

    ckpt = SafetensorsCheckpoint(path)
    return pack_qwen36_moe_weights_from_state_dict(ckpt, layer_idx, spec=spec, layer_prefixes=layer_prefixes,
                                                   device=device)


def load_qwen36_linear_attention_weights_from_safetensors(
    path: str | Path,
    layer_idx: int,
    *,
    spec: Qwen36A3BSpec | None = None,
    layer_prefixes: tuple[str, ...] = LAYER_PREFIXES,
    device: str | torch.device | None = None,
) -> Qwen36LinearAttentionWeights:
    """Reference qwen36_weights.py:759-805."""

    ckpt = SafetensorsCheckpoint(path)
    return pack_qwen36_linear_attention_weights_from_state_dict(ckpt, layer_idx, spec=spec,
                                                                layer_prefixes=layer_prefixes, device=device)


def load_qwen36_attention_weights_from_safetensors(
    path: str | Path,
    layer_idx: int,
    *,
    spec: Qwen36A3BSpec | None = None,
    layer_prefixes: tuple[str, ...] = LAYER_PREFIXES,
    device: str | torch.device | None = None,
) -> Qwen36AttentionWeights:
    """Reference qwen36_weights.py:808-855."""

    ckpt = SafetensorsCheckpoint(path)
    return pack_qwen36_attention_weights_from_state_dict(ckpt, layer_idx, spec=spec, layer_prefixes=layer_prefixes,
                                                         device=device)
