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
    rope_theta: float = 10000.0
    conv_kernel_size: int = 4

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
