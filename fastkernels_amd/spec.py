"""Kernel-facing shape constants of the Qwen3.6 hot path.

Mirrors the fields of `Qwen36A3BSpec` (reference models/qwen36.py:11-191)
that the MoE layer and the Gated DeltaNet step consume, plus the tiny
synthetic spec (models/qwen36.py:194-214) the synthetic switch host uses.
"""

from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class Qwen36A3BSpec:
    name: str
    hidden_size: int
    num_layers: int
    num_experts: int
    num_routed_experts: int
    num_shared_experts: int
    expert_intermediate_size: int
    deltanet_value_heads: int
    deltanet_qk_heads: int
    deltanet_head_dim: int
    attention_heads: int
    attention_kv_heads: int
    attention_head_dim: int
    rope_dim: int
    vocab_size: int
    context_length: int
    layer_types: tuple[str, ...] | None = None
    rope_theta: float = 10000.0
    # (not in the reference spec: the conv window, which the reference fixes
    # by its state shape; last so positional construction matches the reference)
    conv_kernel_size: int = 4

    @property
    def active_experts_per_token(self) -> int:
        """Routed plus shared experts each token runs (reference models/qwen36.py:34-36)."""

        return self.num_routed_experts + self.num_shared_experts

    @property
    def attention_heads_per_kv_head(self) -> int:
        """Query heads per kv head (reference models/qwen36.py:48-52)."""

        if self.attention_heads % self.attention_kv_heads:
            raise ValueError("attention_heads must be divisible by attention_kv_heads")
        return self.attention_heads // self.attention_kv_heads

    def layer_kinds(self) -> tuple[str, ...]:
        """Mixer of each layer: "deltanet_moe" or "attention_moe".  From the
        config's layer_types when given ("full_attention" -> attention),
        else three DeltaNet layers then one attention layer, repeated
        (reference models/qwen36.py:54-62)."""

        if self.layer_types is not None:
            return tuple("attention_moe" if t == "full_attention" else "deltanet_moe" for t in self.layer_types)
        cycle = ("deltanet_moe",) * 3 + ("attention_moe",)
        return tuple(cycle[i % 4] for i in range(self.num_layers))

    def attention_cache_shape(self, max_positions: int | None = None) -> tuple[int, int, int]:
        """KV cache of one attention layer: [positions, kv_heads, head_dim]."""

        return (max_positions or self.context_length, self.attention_kv_heads, self.attention_head_dim)

    def layer_counts(self) -> dict[str, int]:
        kinds = self.layer_kinds()
        return {"deltanet_moe": kinds.count("deltanet_moe"), "attention_moe": kinds.count("attention_moe")}

    def decode_shapes(self, max_positions: int | None = None) -> dict[str, tuple[int, ...]]:
        """Per-step decode tensors by name (reference models/qwen36.py:85-95):
        the stacked synthetic-layout DeltaNet states and KV caches over the
        layers of each kind, the router logits and the packed expert weights."""

        counts = self.layer_counts()
        cache = self.attention_cache_shape(max_positions)
        return {
            "hidden_state": (self.hidden_size,),
            "deltanet_states": (counts["deltanet_moe"], *self.deltanet_state_shape()),
            "attention_key_cache": (counts["attention_moe"], *cache),
            "attention_value_cache": (counts["attention_moe"], *cache),
            "router_logits": (self.num_experts,),
            "expert_gate_up_weight": (self.num_experts, self.gated_up_features, self.hidden_size),
            "expert_down_weight": (self.num_experts, self.hidden_size, self.expert_intermediate_size),
        }

    def summary_lines(self, token_counts=(1, 16, 128)) -> list[str]:
        """A text summary of the spec, one "key: value" line per field group,
        then the routed (token, expert) rows of each token count (reference
        models/qwen36.py:97-114, same lines)."""

        counts = self.layer_counts()
        kinds = self.layer_kinds()
        fields = [
            ("model", self.name),
            ("layers", self.num_layers),
            ("hidden_size", self.hidden_size),
            ("layer pattern", f"{', '.join(kinds[:4])} x {self.num_layers // 4}"),
            ("deltanet/attention layers", f"{counts['deltanet_moe']}/{counts['attention_moe']}"),
            ("deltanet qk/value heads", f"{self.deltanet_qk_heads}/{self.deltanet_value_heads}"),
            ("attention q/kv heads", f"{self.attention_heads}/{self.attention_kv_heads}"),
            ("experts", self.num_experts),
            ("routed/shared active experts", f"{self.num_routed_experts}/{self.num_shared_experts}"),
            ("expert_intermediate_size", self.expert_intermediate_size),
        ]
        return [f"{k}: {v}" for k, v in fields] + [
            f"tokens={t}: routed_expert_rows={t * self.num_routed_experts}" for t in token_counts
        ]

    @classmethod
    def from_hf_config(cls, config: dict, name: str = "hf-config") -> "Qwen36A3BSpec":
        """Spec from a Hugging Face config dict (its `text_config` when
        nested), with the reference's key aliases, their precedence and
        defaults (reference models/qwen36.py:117-161)."""

        text = config.get("text_config", config)

        # aliases in order; for each alias the text config first, then the
        # top level (an earlier alias at the top level wins over a later one
        # in text_config)
        def get(*names: str, default=None):
            for n in names:
                for src in (text, config):
                    if src.get(n) is not None:
                        return src[n]
            return default

        rope = get("rope_parameters", default={}) or {}
        partial = get("partial_rotary_factor", default=rope.get("partial_rotary_factor"))
        head_dim = int(get("attention_head_dim", "head_dim", default=256))
        rope_dim = get("rope_dim", "rotary_emb_base_dim")
        if rope_dim is None and partial is not None:
            rope_dim = int(head_dim * float(partial))
        layer_types = get("layer_types")
        return cls(
            name=name,
            hidden_size=int(get("hidden_size")),
            num_layers=int(get("num_hidden_layers", "num_layers")),
            num_experts=int(get("num_experts", "n_routed_experts")),
            num_routed_experts=int(get("num_experts_per_tok", "num_experts_per_token", default=8)),
            num_shared_experts=int(get("n_shared_experts", "num_shared_experts", default=1)),
            expert_intermediate_size=int(get("moe_intermediate_size", "expert_intermediate_size", "intermediate_size")),
            deltanet_value_heads=int(get("num_linear_attention_value_heads", "linear_num_value_heads", default=32)),
            deltanet_qk_heads=int(get("num_linear_attention_qk_heads", "linear_num_key_heads", default=16)),
            deltanet_head_dim=int(get("linear_attention_head_dim", "linear_key_head_dim", "linear_value_head_dim",
                                      default=128)),
            attention_heads=int(get("num_attention_heads", default=16)),
            attention_kv_heads=int(get("num_key_value_heads", default=2)),
            attention_head_dim=head_dim,
            rope_dim=int(rope_dim or 64),
            vocab_size=int(get("vocab_size", default=248320)),
            context_length=int(get("max_position_embeddings", "seq_length", default=262144)),
            layer_types=tuple(layer_types) if layer_types is not None else None,
            rope_theta=float(get("rope_theta", default=rope.get("rope_theta", 10000.0))),
        )

    @classmethod
    def from_json_file(cls, path, name: str | None = None) -> "Qwen36A3BSpec":
        import json
        from pathlib import Path

        p = Path(path)
        with p.open("r", encoding="utf-8") as fh:
            return cls.from_hf_config(json.load(fh), name=name or p.stem)

    @property
    def gated_up_features(self) -> int:
        return 2 * self.expert_intermediate_size

    @property
    def deltanet_value_dim_per_qk_head(self) -> int:
        if self.deltanet_value_heads % self.deltanet_qk_heads:
            raise ValueError("deltanet_value_heads must be divisible by deltanet_qk_heads")
        return (self.deltanet_value_heads // self.deltanet_qk_heads) * self.deltanet_head_dim

    @property
    def deltanet_key_dim(self) -> int:
        return self.deltanet_qk_heads * self.deltanet_head_dim

    @property
    def deltanet_value_dim(self) -> int:
        return self.deltanet_value_heads * self.deltanet_head_dim

    @property
    def deltanet_conv_dim(self) -> int:
        return 2 * self.deltanet_key_dim + self.deltanet_value_dim

    def deltanet_state_shape(self) -> tuple[int, int, int]:
        """Synthetic-path state layout `[qk_heads, head_dim, value_dim_per_qk_head]`."""

        return (self.deltanet_qk_heads, self.deltanet_head_dim, self.deltanet_value_dim_per_qk_head)

    def deltanet_recurrent_state_shape(self) -> tuple[int, int, int]:
        """Real-path recurrent state `[value_heads, head_dim, head_dim]` (fp32)."""

        return (self.deltanet_value_heads, self.deltanet_head_dim, self.deltanet_head_dim)

    def expert_bytes(self, elem_bytes: int = 2) -> int:
        """Bytes of one expert's gate/up + down weights."""

        return 3 * self.hidden_size * self.expert_intermediate_size * elem_bytes


def qwen36_35b_a3b_spec() -> Qwen36A3BSpec:
    """Qwen3.6-35B-A3B shapes (reference models/qwen36.py:170-191)."""

    return Qwen36A3BSpec(
        name="Qwen3.6-35B-A3B",
        hidden_size=2048,
        num_layers=40,
        num_experts=256,
        num_routed_experts=8,
        num_shared_experts=1,
        expert_intermediate_size=512,
        deltanet_value_heads=32,
        deltanet_qk_heads=16,
        deltanet_head_dim=128,
        attention_heads=16,
        attention_kv_heads=2,
        attention_head_dim=256,
        rope_dim=64,
        vocab_size=248320,
        context_length=262144,
        rope_theta=10000000.0,
    )


def synthetic_qwen36_spec() -> Qwen36A3BSpec:
    """Tiny spec for correctness tests (reference models/qwen36.py:194-214)."""

    return Qwen36A3BSpec(
        name="synthetic-qwen3.6-a3b",
        hidden_size=16,
        num_layers=4,
        num_experts=4,
        num_routed_experts=2,
        num_shared_experts=1,
        expert_intermediate_size=8,
        deltanet_value_heads=4,
        deltanet_qk_heads=2,
        deltanet_head_dim=4,
        attention_heads=4,
        attention_kv_heads=2,
        attention_head_dim=4,
        rope_dim=4,
        vocab_size=64,
        context_length=16,
    )
