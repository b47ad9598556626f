"""Seeded synthetic inputs for the MoE / DeltaNet decode configurations, and
their algorithmic HBM byte counts.

Inputs are drawn on the CPU with a seeded `torch.Generator` in fp32, scaled,
cast to the target dtype and only then copied to the device, so a CPU check
and the GPU kernels see identical bytes (the pattern of the reference's
microbenches, e.g. bench/qwen36_real_moe_microbench.py:38-71).

Configurations (BASELINE.json `configs`):
  0  MoE layer, T=1, bf16: x ~ N(0,1); router W [E,H], experts gate/up [E,2I,H]
     and down [E,H,I], shared expert, w_g [H], all ~ N(0, 0.02); MoE norm
     weight = zeros (so the router sees RMSNorm(x) * 1).
  1  same at T=16.
  2  T=128 with a Zipf(s=1.1) router bias over a seeded expert permutation,
     bias[e] = ZIPF_ALPHA * log p_zipf(rank(e)).
  3  Gated DeltaNet step (T=1 and 8): input norm w, projections, conv1d,
     out_proj, conv_state ~ N(0, 0.02); fp32 recurrent state ~ N(0, 0.1);
     A_log, dt_bias ~ N(0, 0.02); linear_norm_weight ~ N(0, 1).
  4  40 independent config-0 layers (seed = base + layer).
"""

from __future__ import annotations

import math
from typing import Any

import torch

from .spec import Qwen36A3BSpec, qwen36_35b_a3b_spec

WEIGHT_SCALE = 0.02
STATE_SCALE = 0.1
ZIPF_S = 1.1
# Chosen so that at T=128 the hottest expert receives 20-60 tokens (40-54)
# for each of the router weights make_router_weight(seed=r), r = 0..7, with
# hidden states make_hidden(128, seed=r + 1): the weight sets bench.py
# times; tests/test_workloads.py checks it.
ZIPF_ALPHA = 0.28


def _randn(gen: torch.Generator, shape: tuple[int, ...], scale: float, dtype: torch.dtype, device: Any) -> torch.Tensor:
    t = torch.randn(*shape, generator=gen, dtype=torch.float32)
    if scale != 1.0:
        t.mul_(scale)
    return t.to(dtype).to(device)


def _randn_chunked(gen, shape, scale, dtype, device, chunk: int = 16) -> torch.Tensor:
    """Large leading-dim tensors drawn in chunks (same values as one draw) to
    bound the fp32 staging memory."""

    out = torch.empty(shape, dtype=dtype, device=device)
    for start in range(0, shape[0], chunk):
        stop = min(start + chunk, shape[0])
        out[start:stop] = _randn(gen, (stop - start, *shape[1:]), scale, dtype, "cpu").to(device)
    return out


def make_hidden(tokens: int, hidden_size: int, *, seed: int, dtype=torch.bfloat16, device: Any = "cpu") -> torch.Tensor:
    gen = torch.Generator(device="cpu").manual_seed(seed)
    return _randn(gen, (tokens, hidden_size), 1.0, dtype, device)


def make_router_weight(spec: Qwen36A3BSpec | None = None, *, seed: int, dtype=torch.bfloat16, device: Any = "cpu") -> torch.Tensor:
    """The router weight [E, H] of `make_moe_weights(seed=seed)` (its first
    draw), without drawing the experts."""

    spec = spec or qwen36_35b_a3b_spec()
    gen = torch.Generator(device="cpu").manual_seed(seed)
    return _randn(gen, (spec.num_experts, spec.hidden_size), WEIGHT_SCALE, dtype, device)


def make_moe_weights(
    spec: Qwen36A3BSpec | None = None,
    *,
    seed: int,
    dtype=torch.bfloat16,
    device: Any = "cpu",
    shared_gate: bool = True,
) -> dict[str, torch.Tensor]:
    """One MoE layer's weights, keys as in `Qwen36MoEWeights`
    (reference models/qwen36_weights.py:26-37)."""

    spec = spec or qwen36_35b_a3b_spec()
    gen = torch.Generator(device="cpu").manual_seed(seed)
    H, E, I = spec.hidden_size, spec.num_experts, spec.expert_intermediate_size
    w = {
        "norm_weight": torch.zeros(H, dtype=dtype, device=device),
        "router_weight": _randn(gen, (E, H), WEIGHT_SCALE, dtype, device),
        "expert_gate_up_weight": _randn_chunked(gen, (E, 2 * I, H), WEIGHT_SCALE, dtype, device),
        "expert_down_weight": _randn_chunked(gen, (E, H, I), WEIGHT_SCALE, dtype, device),
        "shared_gate_up_weight": _randn(gen, (2 * I, H), WEIGHT_SCALE, dtype, device),
        "shared_down_weight": _randn(gen, (H, I), WEIGHT_SCALE, dtype, device),
    }
    w["shared_expert_gate_weight"] = _randn(gen, (H,), WEIGHT_SCALE, dtype, device) if shared_gate else None
    return w


def zipf_router_bias(num_experts: int, *, seed: int, alpha: float = ZIPF_ALPHA, s: float = ZIPF_S, device: Any = "cpu") -> torch.Tensor:
    """`bias[e] = alpha * log p(rank(e))`, p(r) ∝ r^-s over a seeded permutation (fp32)."""

    gen = torch.Generator(device="cpu").manual_seed(seed + 7919)
    order = torch.randperm(num_experts, generator=gen)
    ranks = torch.empty(num_experts, dtype=torch.float64)
    ranks[order] = torch.arange(1, num_experts + 1, dtype=torch.float64)
    p = ranks.pow(-s)
    p = p / p.sum()
    return (alpha * p.log()).to(torch.float32).to(device)


def make_deltanet_weights(
    spec: Qwen36A3BSpec | None = None, *, seed: int, dtype=torch.bfloat16, device: Any = "cpu"
) -> dict[str, torch.Tensor]:
    """DeltaNet weights (keys of `Qwen36LinearAttentionWeights`,
    reference models/qwen36_weights.py:57-72) plus `conv_state` and the fp32
    `recurrent_state`."""

    spec = spec or qwen36_35b_a3b_spec()
    gen = torch.Generator(device="cpu").manual_seed(seed)
    H = spec.hidden_size
    Hk, Hv, D = spec.deltanet_qk_heads, spec.deltanet_value_heads, spec.deltanet_head_dim
    key_dim, value_dim = Hk * D, Hv * D
    conv_dim = 2 * key_dim + value_dim
    ks = spec.conv_kernel_size
    return {
        "input_norm_weight": _randn(gen, (H,), WEIGHT_SCALE, dtype, device),
        "in_proj_qkv_weight": _randn(gen, (conv_dim, H), WEIGHT_SCALE, dtype, device),
        "in_proj_z_weight": _randn(gen, (value_dim, H), WEIGHT_SCALE, dtype, device),
        "in_proj_a_weight": _randn(gen, (Hv, H), WEIGHT_SCALE, dtype, device),
        "in_proj_b_weight": _randn(gen, (Hv, H), WEIGHT_SCALE, dtype, device),
        "conv1d_weight": _randn(gen, (conv_dim, 1, ks), WEIGHT_SCALE, dtype, device),
        "out_proj_weight": _randn(gen, (H, value_dim), WEIGHT_SCALE, dtype, device),
        "linear_norm_weight": _randn(gen, (D,), 1.0, dtype, device),
        "a_log": _randn(gen, (Hv,), WEIGHT_SCALE, dtype, device),
        "dt_bias": _randn(gen, (Hv,), WEIGHT_SCALE, dtype, device),
        "conv_state": _randn(gen, (conv_dim, ks), WEIGHT_SCALE, dtype, device),
        "recurrent_state": _randn(gen, (Hv, D, D), STATE_SCALE, torch.float32, device),
    }


# ---------------------------------------------------------------------------
# Algorithmic bytes (the roofline numerator)
# ---------------------------------------------------------------------------
def moe_layer_bytes(
    tokens: int,
    distinct_experts: int,
    spec: Qwen36A3BSpec | None = None,
    *,
    weight_bytes: int = 2,
    in_bytes: int = 2,
    out_bytes: int = 4,
    outputs: int = 2,
) -> int:
    """HBM bytes a perfect MoE layer step must move.

    router W (E*H) + (U + 1) experts * 3*H*I + norm weight + w_g (H each),
    plus T*H inputs and `outputs` fp32 [T,H] results (moe update and
    layer_hidden).  `distinct_experts` (U) comes from the step's histogram.
    """

    spec = spec or qwen36_35b_a3b_spec()
    H, E, I = spec.hidden_size, spec.num_experts, spec.expert_intermediate_size
    weights = (E * H + (distinct_experts + 1) * 3 * H * I + 2 * H) * weight_bytes
    return weights + tokens * H * in_bytes + outputs * tokens * H * out_bytes


def moe_layer_flops(tokens: int, spec: Qwen36A3BSpec | None = None) -> int:
    """2*E*H router + 9 experts * 6*H*I per token."""

    spec = spec or qwen36_35b_a3b_spec()
    H, E, I = spec.hidden_size, spec.num_experts, spec.expert_intermediate_size
    return tokens * (2 * E * H + (spec.num_routed_experts + 1) * 6 * H * I)


def deltanet_step_bytes(tokens: int, spec: Qwen36A3BSpec | None = None, *, weight_bytes: int = 2) -> int:
    """Projection + conv + out-proj weights, fp32 recurrent state read and
    written, conv state read and written, and per-token inputs/outputs."""

    spec = spec or qwen36_35b_a3b_spec()
    H = spec.hidden_size
    Hk, Hv, D = spec.deltanet_qk_heads, spec.deltanet_value_heads, spec.deltanet_head_dim
    conv_dim = 2 * Hk * D + Hv * D
    ks = spec.conv_kernel_size
    weights = (conv_dim * H + Hv * D * H + 2 * Hv * H + conv_dim * ks + H * Hv * D + H + D + 2 * Hv) * weight_bytes
    state = 2 * Hv * D * D * 4
    conv_state = 2 * conv_dim * ks * weight_bytes
    io = tokens * H * weight_bytes + 2 * tokens * H * 4
    return weights + state + conv_state + io


def attention_step_bytes(tokens: int, context: int, spec: Qwen36A3BSpec | None = None, *, weight_bytes: int = 2,
                         cache_bytes: int = 4) -> int:
    """Gated attention step: Wq (query + gate rows), Wk, Wv, Wo and the norm
    weights, the cached keys and values of the `context` earlier positions
    (read once) and the new rows written, plus per-token inputs/outputs."""

    spec = spec or qwen36_35b_a3b_spec()
    H, heads, kvh, hd = spec.hidden_size, spec.attention_heads, spec.attention_kv_heads, spec.attention_head_dim
    weights = (2 * heads * hd * H + 2 * kvh * hd * H + H * heads * hd + H + 2 * hd) * weight_bytes
    cache = 2 * (context + tokens) * kvh * hd * cache_bytes
    io = tokens * H * weight_bytes + 2 * tokens * H * 4
    return weights + cache + io


def make_attention_weights(
    spec: Qwen36A3BSpec | None = None, *, seed: int, dtype=torch.bfloat16, device: Any = "cpu"
) -> dict[str, torch.Tensor]:
    """Gated-attention weights (keys of `Qwen36AttentionWeights` without the
    post-attention norm, which belongs to the MoE block)."""

    spec = spec or qwen36_35b_a3b_spec()
    gen = torch.Generator(device="cpu").manual_seed(seed)
    H, heads, kvh, hd = spec.hidden_size, spec.attention_heads, spec.attention_kv_heads, spec.attention_head_dim
    return {
        "input_norm_weight": _randn(gen, (H,), WEIGHT_SCALE, dtype, device),
        "q_proj_weight": _randn(gen, (2 * heads * hd, H), WEIGHT_SCALE, dtype, device),
        "k_proj_weight": _randn(gen, (kvh * hd, H), WEIGHT_SCALE, dtype, device),
        "v_proj_weight": _randn(gen, (kvh * hd, H), WEIGHT_SCALE, dtype, device),
        "o_proj_weight": _randn(gen, (H, heads * hd), WEIGHT_SCALE, dtype, device),
        "q_norm_weight": _randn(gen, (hd,), WEIGHT_SCALE, dtype, device),
        "k_norm_weight": _randn(gen, (hd,), WEIGHT_SCALE, dtype, device),
    }


def expected_distinct_experts(tokens: int, spec: Qwen36A3BSpec | None = None) -> float:
    spec = spec or qwen36_35b_a3b_spec()
    E, K = spec.num_experts, spec.num_routed_experts
    return E * (1.0 - math.pow(1.0 - K / E, tokens))
