"""CPU restatement of the reference oracle for the Qwen3.6 MoE + DeltaNet path.

Test infrastructure (see oracle/__init__.py).  Each function cites the
reference file:line it restates; paths are relative to
suryavanshi/fastkernels/src/fastkernels/.
"""

from __future__ import annotations

from typing import Any

import numpy as np
import torch
import torch.nn.functional as F

__all__ = [
    "rms_norm",
    "rms_norm_plain",
    "l2_norm",
    "topk_lowest_id",
    "router",
    "expert_histogram",
    "moe_align",
    "swiglu",
    "expert_mlp",
    "routed_experts",
    "shared_expert",
    "moe_update",
    "moe_layer",
    "causal_conv_update",
    "gated_rms_norm",
    "deltanet_project",
    "deltanet_recurrent",
    "deltanet_recurrent_output",
    "deltanet_update",
    "deltanet_moe_layer",
    "rope",
    "attention_update",
    "attention_moe_layer",
    "synthetic_moe_decode",
    "synthetic_deltanet_decode",
    "synthetic_attention_decode",
    "synthetic_rope",
]


# ---------------------------------------------------------------------------
# Norms
# ---------------------------------------------------------------------------
def rms_norm(hidden: Any, weight: Any, eps: float = 1e-6, offset: float = 1.0, dtype=torch.float32) -> Any:
    """`x * rsqrt(mean(x^2) + eps) * (offset + w)` in fp32.

    reference/qwen36_real.py:23-28 (offset 1); kernels/triton/qwen36_router.py:50-53
    (general `norm_offset`).
    """

    x = hidden.to(dtype)
    normed = x * torch.rsqrt((x * x).mean(dim=-1, keepdim=True) + eps)
    return normed * (offset + weight.to(dtype))


def rms_norm_plain(hidden: Any, weight: Any, eps: float = 1e-6) -> Any:
    """Synthetic-path norm `x * rsqrt(mean(x^2) + eps) * w` in the input dtype.

    reference/qwen36_decode.py:27-29.
    """

    return hidden * torch.rsqrt(hidden.pow(2).mean(dim=-1, keepdim=True) + eps) * weight


def l2_norm(hidden: Any, eps: float = 1e-6) -> Any:
    """reference/qwen36_real.py:31-35."""

    return hidden * torch.rsqrt((hidden * hidden).sum(dim=-1, keepdim=True) + eps)


# ---------------------------------------------------------------------------
# Router
# ---------------------------------------------------------------------------
def topk_lowest_id(probs: Any, k: int) -> tuple[Any, Any]:
    """Top-k along the last dim ordered by (value desc, index asc).

    Replaces `torch.topk` (reference/qwen36_real.py:336, reference/moe.py:78),
    whose tie order is unspecified, with the rule the build implements: equal
    probabilities go to the lower expert id.  A stable descending sort keeps
    equal values in ascending index order.
    """

    values, order = torch.sort(probs, dim=-1, descending=True, stable=True)
    return values[..., :k], order[..., :k]


def router(
    hidden: Any,
    norm_weight: Any,
    router_weight: Any,
    top_k: int,
    *,
    eps: float = 1e-6,
    norm_offset: float = 1.0,
    router_bias: Any | None = None,
    dtype=torch.float32,
) -> tuple[Any, Any, Any]:
    """`(logits f32[T,E], ids i64[T,K], weights f32[T,K])`.

    reference/qwen36_real.py:333-337: logits = RMSNorm(x)(1+w) @ W_r^T,
    softmax, top-k, renormalise by the sum of the selected probabilities.
    `router_bias` (an extension for skewed routing) is added to the logits.
    """

    x = hidden.reshape(-1, hidden.shape[-1])
    logits = rms_norm(x, norm_weight, eps, norm_offset, dtype) @ router_weight.to(dtype).transpose(0, 1)
    if router_bias is not None:
        logits = logits + router_bias.to(dtype).reshape(1, -1)
    probs = torch.softmax(logits, dim=-1)
    values, ids = topk_lowest_id(probs, top_k)
    weights = values / values.sum(dim=-1, keepdim=True)
    return logits, ids.to(torch.int64), weights


# ---------------------------------------------------------------------------
# Routing tables (integer work, numpy)
# ---------------------------------------------------------------------------
def expert_histogram(topk_ids: Any, num_experts: int) -> np.ndarray:
    """int32 `[E]` counts; reference/moe.py:24-30 (`bincount(minlength=E)`)."""

    ids = np.asarray(topk_ids).reshape(-1).astype(np.int64)
    if ids.size and (ids.min() < 0 or ids.max() >= num_experts):
        raise ValueError("expert ids out of range")
    return np.bincount(ids, minlength=num_experts).astype(np.int32)


def moe_align(topk_ids: Any, num_experts: int) -> tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
    """Routing tables `(counts[E], offsets[E+1], perm[P], inverse[P])`.

    The reference has no permutation (its batched path re-streams weights per
    (token, slot), kernels/triton/qwen36_expert.py:456-537); this is the
    specification the build adopts: flat pairs `j = t*K + k` sorted stably by
    expert id, so within an expert pairs keep (token, slot) order.
    `counts` equals the reference histogram (reference/moe.py:24-30).
    """

    ids = np.asarray(topk_ids).reshape(-1).astype(np.int64)
    counts = expert_histogram(ids, num_experts)
    offsets = np.zeros(num_experts + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    perm = np.argsort(ids, kind="stable").astype(np.int32)
    inverse = np.empty_like(perm)
    inverse[perm] = np.arange(perm.size, dtype=np.int32)
    return counts, offsets, perm, inverse


# ---------------------------------------------------------------------------
# Experts
# ---------------------------------------------------------------------------
def swiglu(gate_up: Any) -> Any:
    """`silu(gate) * up` over the last dim halves; reference/moe.py:16-21."""

    gate, up = gate_up.chunk(2, dim=-1)
    return F.silu(gate) * up


def expert_mlp(token: Any, gate_up_weight: Any, down_weight: Any, dtype=torch.float32) -> Any:
    """One expert on one token (reference/qwen36_real.py:343-347): the input is
    the raw (un-normalised) hidden row."""

    gate_up = gate_up_weight.to(dtype) @ token.to(dtype)
    gate, up = torch.chunk(gate_up, 2, dim=0)
    return down_weight.to(dtype) @ (F.silu(gate) * up)


def routed_experts(hidden: Any, topk_ids: Any, topk_weights: Any, gate_up: Any, down: Any, dtype=torch.float32) -> Any:
    """`out[t] = sum_k w[t,k] * expert(ids[t,k], x[t])`, fp32 `[T,H]`.

    reference/qwen36_real.py:338-347 (routed part of the token x route loop);
    ids are clamped to [0, E-1] as the reference kernels do
    (kernels/triton/qwen36_expert.py:146).
    """

    x = hidden.reshape(-1, hidden.shape[-1]).to(dtype)
    ids = topk_ids.reshape(x.shape[0], -1)
    w = topk_weights.reshape(x.shape[0], -1).to(dtype)
    num_experts = gate_up.shape[0]
    out = torch.zeros_like(x)
    for t in range(x.shape[0]):
        for k in range(ids.shape[1]):
            e = min(max(int(ids[t, k]), 0), num_experts - 1)
            out[t] += w[t, k] * expert_mlp(x[t], gate_up[e], down[e], dtype)
    return out


def shared_expert(hidden: Any, gate_up: Any, down: Any, gate_weight: Any | None = None, dtype=torch.float32) -> Any:
    """Shared expert, scaled by `sigmoid(w_g . x)` when a gate is given.

    reference/qwen36_real.py:348-353.
    """

    x = hidden.reshape(-1, hidden.shape[-1]).to(dtype)
    out = torch.stack([expert_mlp(x[t], gate_up, down, dtype) for t in range(x.shape[0])])
    if gate_weight is not None:
        g = torch.sigmoid(x @ gate_weight.to(dtype).reshape(-1))
        out = out * g.reshape(-1, 1)
    return out


def moe_update(
    hidden: Any,
    norm_weight: Any,
    router_weight: Any,
    gate_up: Any,
    down: Any,
    shared_gate_up: Any,
    shared_down: Any,
    shared_gate: Any | None = None,
    *,
    top_k: int = 8,
    eps: float = 1e-6,
    norm_offset: float = 1.0,
    router_bias: Any | None = None,
    dtype=torch.float32,
) -> tuple[Any, Any, Any, Any]:
    """Full MoE block: `(update f32[T,H], logits, ids, weights)`.

    reference/qwen36_real.py:329-354 (router on the normed x, experts on the
    raw x, shared expert with optional sigmoid gate).
    """

    x = hidden.reshape(-1, hidden.shape[-1])
    logits, ids, weights = router(
        x, norm_weight, router_weight, top_k, eps=eps, norm_offset=norm_offset, router_bias=router_bias, dtype=dtype
    )
    out = routed_experts(x, ids, weights, gate_up, down, dtype)
    out = out + shared_expert(x, shared_gate_up, shared_down, shared_gate, dtype)
    return out, logits, ids, weights


def moe_layer(hidden: Any, *args: Any, **kwargs: Any) -> tuple[Any, Any, Any, Any, Any]:
    """`(layer_hidden, moe_update, logits, ids, weights)` with
    `layer_hidden = x + update` (reference/qwen36_real.py:374-375;
    kernels/triton/qwen36_layer.py:55-106)."""

    update, logits, ids, weights = moe_update(hidden, *args, **kwargs)
    x = hidden.reshape(update.shape).to(update.dtype)
    return x + update, update, logits, ids, weights


# ---------------------------------------------------------------------------
# Gated DeltaNet
# ---------------------------------------------------------------------------
def causal_conv_update(mixed: Any, conv_state: Any, conv_weight: Any) -> tuple[Any, Any]:
    """Depthwise causal conv + SiLU with state roll.

    reference/qwen36_real.py:92-108: over `comb = [state | mixed^T]` (per
    channel), output for row t is `silu(sum_j w[c, j] * comb[c, t + 1 + j])`
    and the next state is the last `kernel_size` columns of `comb`.  Written
    as the explicit sliding sum (the reference calls conv1d).
    """

    tokens, channels = mixed.shape
    kernel_size = conv_state.shape[1]
    comb = torch.cat((conv_state.float(), mixed.float().transpose(0, 1)), dim=1)  # [C, KS + T]
    w = conv_weight.float().reshape(channels, kernel_size)
    out = torch.zeros((tokens, channels), dtype=torch.float32)
    for t in range(tokens):
        window = comb[:, t + 1 : t + 1 + kernel_size]
        out[t] = F.silu((window * w).sum(dim=1))
    next_state = comb[:, -kernel_size:].to(conv_state.dtype)
    return out, next_state


def gated_rms_norm(core: Any, gate: Any, weight: Any, eps: float = 1e-6) -> Any:
    """`o * rsqrt(mean(o^2) + eps) * w * silu(z)` (plain weight); reference/qwen36_real.py:85-89."""

    o = core.float()
    return o * torch.rsqrt((o * o).mean(dim=-1, keepdim=True) + eps) * weight.float() * F.silu(gate.float())


def deltanet_project(
    hidden: Any, norm_weight: Any, w_qkv: Any, w_z: Any, w_a: Any, w_b: Any, *, eps: float = 1e-6, norm_offset: float = 1.0
) -> tuple[Any, Any, Any, Any]:
    """RMSNorm(1+w) then the four input projections; reference/qwen36_real.py:126-130."""

    xn = rms_norm(hidden, norm_weight, eps, norm_offset)
    return tuple(xn @ w.float().transpose(0, 1) for w in (w_qkv, w_z, w_a, w_b))  # type: ignore[return-value]


def deltanet_recurrent(
    mixed_qkv: Any,
    a_logits: Any,
    b_logits: Any,
    recurrent_state: Any,
    a_log: Any,
    dt_bias: Any,
    *,
    qk_heads: int,
    value_heads: int,
    head_dim: int,
    eps: float = 1e-6,
    dtype=torch.float32,
) -> tuple[Any, Any]:
    """Gated delta rule over rows in order through one state: `(core[T, Hv*D], state')`.

    reference/qwen36_real.py:205-250.  Value head h reads qk head
    h // (Hv / Hk) (repeat_interleave, :231-234).
    """

    tokens = mixed_qkv.shape[0]
    key_dim = qk_heads * head_dim
    m = mixed_qkv.to(dtype)
    q = m[:, :key_dim].reshape(tokens, qk_heads, head_dim)
    k = m[:, key_dim : 2 * key_dim].reshape(tokens, qk_heads, head_dim)
    v = m[:, 2 * key_dim :].reshape(tokens, value_heads, head_dim)
    beta = torch.sigmoid(b_logits.to(dtype))
    g = -a_log.to(dtype).exp() * F.softplus(a_logits.to(dtype) + dt_bias.to(dtype))
    rep = value_heads // qk_heads
    q = q.repeat_interleave(rep, dim=1)
    k = k.repeat_interleave(rep, dim=1)
    q = l2_norm(q, eps) * (head_dim**-0.5)
    k = l2_norm(k, eps)
    state = recurrent_state.to(dtype)
    outs = []
    for t in range(tokens):
        state = state * g[t].exp().reshape(value_heads, 1, 1)
        delta = (v[t] - (state * k[t].unsqueeze(-1)).sum(dim=-2)) * beta[t].reshape(value_heads, 1)
        state = state + k[t].unsqueeze(-1) * delta.unsqueeze(-2)
        outs.append((state * q[t].unsqueeze(-1)).sum(dim=-2))
    core = torch.stack(outs, dim=0).reshape(tokens, value_heads * head_dim)
    return core, state


def deltanet_recurrent_output(
    mixed_qkv: Any,
    z: Any,
    a_logits: Any,
    b_logits: Any,
    recurrent_state: Any,
    out_proj_weight: Any,
    linear_norm_weight: Any,
    a_log: Any,
    dt_bias: Any,
    *,
    qk_heads: int,
    value_heads: int,
    head_dim: int,
    eps: float = 1e-6,
) -> tuple[Any, Any]:
    """`(update f32[T,H], next_state)`: recurrent rule, per-head gated RMSNorm,
    out-proj; reference/qwen36_real.py:205-260."""

    tokens = mixed_qkv.shape[0]
    core, state = deltanet_recurrent(
        mixed_qkv, a_logits, b_logits, recurrent_state, a_log, dt_bias,
        qk_heads=qk_heads, value_heads=value_heads, head_dim=head_dim, eps=eps,
    )
    normed = gated_rms_norm(
        core.reshape(tokens * value_heads, head_dim),
        z.reshape(tokens * value_heads, head_dim),
        linear_norm_weight,
        eps,
    ).reshape(tokens, value_heads * head_dim)
    update = normed @ out_proj_weight.float().transpose(0, 1)
    return update, state.to(recurrent_state.dtype)


def deltanet_update(
    hidden: Any,
    conv_state: Any,
    recurrent_state: Any,
    weights: dict[str, Any],
    *,
    qk_heads: int,
    value_heads: int,
    head_dim: int,
    eps: float = 1e-6,
) -> tuple[Any, Any, Any]:
    """`(update, next_conv_state, next_recurrent_state)`; reference/qwen36_real.py:111-148.

    `weights` keys: input_norm_weight, in_proj_qkv_weight, in_proj_z_weight,
    in_proj_a_weight, in_proj_b_weight, conv1d_weight, out_proj_weight,
    linear_norm_weight, a_log, dt_bias (models/qwen36_weights.py:57-72).
    """

    mixed, z, a, b = deltanet_project(
        hidden, weights["input_norm_weight"], weights["in_proj_qkv_weight"], weights["in_proj_z_weight"],
        weights["in_proj_a_weight"], weights["in_proj_b_weight"], eps=eps,
    )
    mixed, next_conv = causal_conv_update(mixed, conv_state, weights["conv1d_weight"])
    update, next_state = deltanet_recurrent_output(
        mixed, z, a, b, recurrent_state, weights["out_proj_weight"], weights["linear_norm_weight"],
        weights["a_log"], weights["dt_bias"], qk_heads=qk_heads, value_heads=value_heads, head_dim=head_dim, eps=eps,
    )
    return update, next_conv, next_state


def deltanet_moe_layer(
    hidden: Any,
    conv_state: Any,
    recurrent_state: Any,
    dn_weights: dict[str, Any],
    moe_weights: dict[str, Any],
    *,
    qk_heads: int,
    value_heads: int,
    head_dim: int,
    top_k: int = 8,
    eps: float = 1e-6,
    router_bias: Any | None = None,
) -> tuple[Any, ...]:
    """DeltaNet -> MoE layer, in the 9-tuple order of the reference layer wrapper
    (kernels/triton/qwen36_layer.py:236-237); maths of reference/qwen36_real.py:357-375.

    `moe_weights` keys: norm_weight, router_weight, expert_gate_up_weight,
    expert_down_weight, shared_gate_up_weight, shared_down_weight,
    shared_expert_gate_weight (optional).
    """

    update, next_conv, next_state = deltanet_update(
        hidden, conv_state, recurrent_state, dn_weights,
        qk_heads=qk_heads, value_heads=value_heads, head_dim=head_dim, eps=eps,
    )
    dn_hidden = hidden.float() + update
    layer_hidden, moe_out, logits, ids, weights = moe_layer(
        dn_hidden, moe_weights["norm_weight"], moe_weights["router_weight"], moe_weights["expert_gate_up_weight"],
        moe_weights["expert_down_weight"], moe_weights["shared_gate_up_weight"], moe_weights["shared_down_weight"],
        moe_weights.get("shared_expert_gate_weight"), top_k=top_k, eps=eps, router_bias=router_bias,
    )
    return layer_hidden, dn_hidden, update, moe_out, next_conv, next_state, logits, ids, weights


# ---------------------------------------------------------------------------
# Gated full attention
# ---------------------------------------------------------------------------
def rope(values: Any, positions: Any, rope_dim: int, theta: float, interleaved: bool = True) -> Any:
    """RoPE of the first rope_dim (rounded down to even) dims of values
    [T, heads, hd] at positions [T], angle p * theta^(-2i/rope_dim).

    interleaved: pairs (2i, 2i+1), as the reference Triton entry point
    (kernels/triton/qwen36_attention.py:270-296) and its test
    (tests/test_triton_moe.py:1011-1025); otherwise halves (i, i + rd/2),
    as the reference torch oracle (reference/qwen36_real.py:263-280).
    """

    x = values.float()
    rd = min(rope_dim, x.shape[-1])
    rd -= rd % 2
    if rd <= 0:
        return x.clone()
    inv_freq = 1.0 / (theta ** (torch.arange(0, rd, 2, dtype=torch.float32) / rd))
    ang = positions.float()[:, None] * inv_freq[None, :]  # [T, rd/2]
    cos, sin = torch.cos(ang)[:, None, :], torch.sin(ang)[:, None, :]
    out = x.clone()
    if interleaved:
        a, b = x[..., 0:rd:2], x[..., 1:rd:2]
        out[..., 0:rd:2] = a * cos - b * sin
        out[..., 1:rd:2] = a * sin + b * cos
    else:
        h = rd // 2
        a, b = x[..., :h], x[..., h:rd]
        out[..., :h] = a * cos - b * sin
        out[..., h:rd] = b * cos + a * sin
    return out


def attention_update(
    hidden: Any,
    key_cache: Any,
    value_cache: Any,
    norm_weight: Any,
    q_proj_weight: Any,
    k_proj_weight: Any,
    v_proj_weight: Any,
    out_proj_weight: Any,
    q_norm_weight: Any,
    k_norm_weight: Any,
    *,
    start_position: int,
    heads: int,
    kv_heads: int,
    head_dim: int,
    rope_dim: int,
    rope_theta: float,
    eps: float = 1e-6,
    qk_eps: float = 1e-6,
    interleaved: bool = True,
) -> tuple[Any, Any, Any]:
    """Gated attention decode (reference/qwen36_real.py:283-326; projection
    split of kernels/triton/qwen36_attention.py:507-513): `(update, key_cache',
    value_cache')`, caches [positions, kv_heads, head_dim] updated at
    start_position .. start_position + T - 1 (returned as copies)."""

    x = hidden.float()
    T = x.shape[0]
    qw = heads * head_dim
    xn = rms_norm(x, norm_weight, eps)
    qg = (xn @ q_proj_weight.float()[: 2 * qw].t()).reshape(T, heads, 2 * head_dim)
    q, gate = qg[..., :head_dim], qg[..., head_dim:]
    k = (xn @ k_proj_weight.float().t()).reshape(T, kv_heads, head_dim)
    v = (xn @ v_proj_weight.float().t()).reshape(T, kv_heads, head_dim)
    q = rms_norm(q, q_norm_weight, qk_eps)
    k = rms_norm(k, k_norm_weight, qk_eps)
    pos = torch.arange(start_position, start_position + T)
    q = rope(q, pos, rope_dim, rope_theta, interleaved)
    k = rope(k, pos, rope_dim, rope_theta, interleaved)
    kc = key_cache.clone()
    vc = value_cache.clone()
    kc[start_position : start_position + T] = k.to(kc.dtype)
    vc[start_position : start_position + T] = v.to(vc.dtype)
    keys, vals = kc.float(), vc.float()
    group = heads // kv_heads
    attended = torch.empty(T, heads, head_dim)
    for t in range(T):
        p = start_position + t
        for h in range(heads):
            j = h // group
            scores = (keys[: p + 1, j] * q[t, h]).sum(-1) * head_dim**-0.5
            attended[t, h] = (vals[: p + 1, j] * torch.softmax(scores, dim=0)[:, None]).sum(0)
    update = (attended.reshape(T, qw) * torch.sigmoid(gate.reshape(T, qw))) @ out_proj_weight.float().t()
    return update, kc, vc


def attention_moe_layer(
    hidden: Any,
    key_cache: Any,
    value_cache: Any,
    attn_weights: dict[str, Any],
    moe_weights: dict[str, Any],
    *,
    start_position: int,
    heads: int,
    kv_heads: int,
    head_dim: int,
    rope_dim: int,
    rope_theta: float,
    top_k: int = 8,
    eps: float = 1e-6,
    interleaved: bool = True,
) -> tuple[Any, ...]:
    """Attention -> MoE layer in the 9-tuple order of the reference wrapper
    (kernels/triton/qwen36_layer.py:185-201); maths of
    reference/qwen36_real.py:378-399.  `attn_weights` keys: input_norm_weight,
    q_proj_weight, k_proj_weight, v_proj_weight, o_proj_weight, q_norm_weight,
    k_norm_weight."""

    a = attn_weights
    update, kc, vc = attention_update(
        hidden, key_cache, value_cache, a["input_norm_weight"], a["q_proj_weight"], a["k_proj_weight"],
        a["v_proj_weight"], a["o_proj_weight"], a["q_norm_weight"], a["k_norm_weight"],
        start_position=start_position, heads=heads, kv_heads=kv_heads, head_dim=head_dim, rope_dim=rope_dim,
        rope_theta=rope_theta, eps=eps, interleaved=interleaved,
    )
    attn_hidden = hidden.float() + update
    layer_hidden, moe_out, logits, ids, weights = moe_layer(
        attn_hidden, moe_weights["norm_weight"], moe_weights["router_weight"], moe_weights["expert_gate_up_weight"],
        moe_weights["expert_down_weight"], moe_weights["shared_gate_up_weight"], moe_weights["shared_down_weight"],
        moe_weights.get("shared_expert_gate_weight"), top_k=top_k, eps=eps,
    )
    return layer_hidden, attn_hidden, update, moe_out, kc, vc, logits, ids, weights


# ---------------------------------------------------------------------------
# Synthetic (tiny-spec) blocks, computed in the input dtype as the reference does
# ---------------------------------------------------------------------------
def synthetic_moe_decode(hidden: Any, layer: dict[str, Any], top_k: int, eps: float = 1e-6) -> Any:
    """`hidden + routed + shared` (reference/qwen36_decode.py:212-224 with
    reference/moe.py:33-93): router on the plain-weight norm, softmax top-k
    renormalised (lower id on ties), ungated shared expert."""

    logits = rms_norm_plain(hidden, layer["norm_weight"], eps) @ layer["router_weight"].transpose(-1, -2)
    probs = torch.softmax(logits, dim=-1)
    values, ids = topk_lowest_id(probs, top_k)
    values = values / values.sum(dim=-1, keepdim=True)
    routed = torch.zeros_like(hidden)
    for k in range(top_k):
        e = int(ids[k])
        act = swiglu(layer["expert_gate_up_weight"][e] @ hidden)
        routed = routed + values[k] * (layer["expert_down_weight"][e] @ act)
    shared = layer["shared_down_weight"] @ swiglu(layer["shared_gate_up_weight"] @ hidden)
    return hidden + routed + shared


def synthetic_deltanet_decode(
    hidden: Any, state: Any, layer: dict[str, Any], *, qk_heads: int, head_dim: int, value_dim_per_head: int, eps: float = 1e-6
) -> tuple[Any, Any]:
    """Toy DeltaNet (reference/qwen36_decode.py:155-171):
    `S' = 0.95 S + k (x) v`, `out = x + W_o ((q . S') * sigmoid(W_g xn))`."""

    x = rms_norm_plain(hidden, layer["norm_weight"], eps)
    q = (x @ layer["q_weight"].transpose(-1, -2)).reshape(qk_heads, head_dim)
    k = (x @ layer["k_weight"].transpose(-1, -2)).reshape(qk_heads, head_dim)
    v = (x @ layer["v_weight"].transpose(-1, -2)).reshape(qk_heads, value_dim_per_head)
    gate = torch.sigmoid(x @ layer["gate_weight"].transpose(-1, -2)).reshape(qk_heads, value_dim_per_head)
    new_state = 0.95 * state + k.unsqueeze(-1) * v.unsqueeze(-2)
    recurrent = (q.unsqueeze(-1) * new_state).sum(dim=-2) * gate
    out = recurrent.reshape(-1) @ layer["out_weight"].transpose(-1, -2)
    return hidden + out, new_state


def synthetic_rope(values: Any, position: int, rope_dim: int) -> Any:
    """Interleaved-pair RoPE of the synthetic oracle (reference/qwen36_decode.py:37-56):
    pairs (2i, 2i + 1) of the first min(rope_dim, head_dim) (even) dims turn by
    position / 10000^(2i / r); cos and sin are cast to the values' dtype."""

    r = min(rope_dim, values.shape[-1]) if rope_dim > 0 else 0
    r -= r % 2
    if r == 0:
        return values
    ang = position / (10000.0 ** (torch.arange(0, r, 2, dtype=torch.float32) / r))
    cos, sin = torch.cos(ang).to(values.dtype), torch.sin(ang).to(values.dtype)
    out = values.clone()
    even, odd = values[..., :r:2], values[..., 1:r:2]
    out[..., :r:2] = even * cos - odd * sin
    out[..., 1:r:2] = even * sin + odd * cos
    return out


def synthetic_attention_decode(
    hidden: Any, key_cache: Any, value_cache: Any, layer: dict[str, Any], *, attention_heads: int, kv_heads: int,
    head_dim: int, rope_dim: int, position: int, eps: float = 1e-6
) -> tuple[Any, Any, Any]:
    """One-token grouped-query attention of the synthetic oracle
    (reference/qwen36_decode.py:174-209), in the input dtype: plain-weight
    RMSNorm, q/k/v projections, RoPE on q and k, the new k and v rows written
    at `position` of copies of the caches, softmax(q.k / sqrt(head_dim)) over
    rows 0..position of each query head's kv head, `hidden + W_o attended`."""

    x = rms_norm_plain(hidden, layer["norm_weight"], eps)
    q = (x @ layer["q_weight"].transpose(-1, -2)).reshape(attention_heads, head_dim)
    k = (x @ layer["k_weight"].transpose(-1, -2)).reshape(kv_heads, head_dim)
    v = (x @ layer["v_weight"].transpose(-1, -2)).reshape(kv_heads, head_dim)
    q, k = synthetic_rope(q, position, rope_dim), synthetic_rope(k, position, rope_dim)
    kc, vc = key_cache.clone(), value_cache.clone()
    kc[position] = k
    vc[position] = v
    keys, values = kc[: position + 1], vc[: position + 1]
    group = attention_heads // kv_heads
    heads = []
    for h in range(attention_heads):
        scores = (keys[:, h // group] @ q[h]) * (1.0 / head_dim**0.5)
        heads.append(torch.softmax(scores, dim=-1) @ values[:, h // group])
    attended = torch.stack(heads).reshape(-1)
    return hidden + attended @ layer["out_weight"].transpose(-1, -2), kc, vc

