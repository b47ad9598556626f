"""Pins the CPU oracle against closed forms, library routines and brute force.

Each check is chosen so that a plausible slip in the restatement (dropped
norm offset, wrong tie order, transposed weight, wrong conv window, decay
applied after the update, q/k swapped, ...) fails at least one of them.
"""

from __future__ import annotations

import collections
import itertools

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle


# ---------------------------------------------------------------------------
# RMSNorm: the reference KAT (tests/test_qwen36_spec.py:368-377)
# ---------------------------------------------------------------------------
def test_rms_norm_closed_form_kat():
    hidden = torch.tensor([[3.0, 4.0]])
    expected = hidden / torch.sqrt(torch.tensor(12.5 + 1e-6))
    torch.testing.assert_close(oracle.rms_norm(hidden, torch.zeros(2)), expected)
    torch.testing.assert_close(oracle.rms_norm(hidden, torch.ones(2)), 2.0 * expected)
    # norm_offset 0 gives the plain-weight form used by the synthetic path
    torch.testing.assert_close(oracle.rms_norm(hidden, torch.ones(2), offset=0.0), expected)
    torch.testing.assert_close(oracle.rms_norm_plain(hidden, torch.ones(2)), expected)


def test_l2_norm_unit_length():
    x = torch.randn(5, 7, generator=torch.Generator().manual_seed(3))
    torch.testing.assert_close(oracle.l2_norm(x).norm(dim=-1), torch.ones(5), atol=1e-5, rtol=0)


# ---------------------------------------------------------------------------
# Router: top-k order and renormalisation
# ---------------------------------------------------------------------------
def _brute_topk(p: list[float], k: int) -> list[int]:
    # rank(i) = #{j : p_j > p_i or (p_j == p_i and j < i)}
    ranks = {i: sum(1 for j in range(len(p)) if p[j] > p[i] or (p[j] == p[i] and j < i)) for i in range(len(p))}
    return [i for i, _ in sorted(ranks.items(), key=lambda kv: kv[1])][:k]


@pytest.mark.parametrize("seed", range(20))
def test_topk_matches_brute_force_small(seed):
    g = torch.Generator().manual_seed(seed)
    e = int(torch.randint(2, 17, (1,), generator=g))
    k = int(torch.randint(1, min(8, e) + 1, (1,), generator=g))
    # quantised values force frequent exact ties
    p = torch.randint(0, 4, (e,), generator=g).float() / 4
    values, ids = oracle.topk_lowest_id(p, k)
    assert ids.tolist() == _brute_topk(p.tolist(), k)
    assert values.tolist() == [p[i].item() for i in ids.tolist()]


def test_topk_ties_go_to_lower_id():
    p = torch.tensor([0.1, 0.3, 0.3, 0.05, 0.3, 0.25])
    _, ids = oracle.topk_lowest_id(p, 4)
    assert ids.tolist() == [1, 2, 4, 5]


def test_router_matches_torch_topk_without_ties_and_sums_to_one():
    g = torch.Generator().manual_seed(11)
    x = torch.randn(6, 64, generator=g)
    nw = 0.02 * torch.randn(64, generator=g)
    rw = 0.02 * torch.randn(16, 64, generator=g)
    logits, ids, w = oracle.router(x, nw, rw, 4)
    ref_logits = (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6) * (1 + nw)) @ rw.t()
    torch.testing.assert_close(logits, ref_logits)
    probs = torch.softmax(ref_logits, -1)
    vals, ref_ids = torch.topk(probs, 4, dim=-1)
    assert torch.equal(ids, ref_ids)
    torch.testing.assert_close(w, vals / vals.sum(-1, keepdim=True))
    torch.testing.assert_close(w.sum(-1), torch.ones(6))
    assert all(len(set(row)) == 4 for row in ids.tolist())


def test_router_bias_shifts_logits():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 32, generator=g)
    nw = torch.zeros(32)
    rw = 0.02 * torch.randn(8, 32, generator=g)
    bias = torch.zeros(8)
    bias[7] = 100.0
    logits0, _, _ = oracle.router(x, nw, rw, 2)
    logits1, ids1, _ = oracle.router(x, nw, rw, 2, router_bias=bias)
    torch.testing.assert_close(logits1 - logits0, bias.expand(2, 8))
    assert (ids1[:, 0] == 7).all()


# ---------------------------------------------------------------------------
# Histogram and permutation (integer work)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("tokens,top_k,experts", [(1, 8, 256), (16, 8, 256), (64, 8, 256), (5, 3, 4), (128, 8, 16)])
def test_histogram_matches_counter(tokens, top_k, experts):
    rng = np.random.default_rng(tokens * 1000 + experts)
    ids = rng.integers(0, experts, size=(tokens, top_k))
    counts = oracle.expert_histogram(ids, experts)
    c = collections.Counter(ids.reshape(-1).tolist())
    assert counts.tolist() == [c.get(e, 0) for e in range(experts)]
    assert counts.dtype == np.int32 and counts.sum() == tokens * top_k


def test_histogram_rejects_out_of_range():
    with pytest.raises(ValueError):
        oracle.expert_histogram(np.array([[0, 4]]), 4)


@pytest.mark.parametrize("tokens,top_k,experts", [(1, 8, 256), (3, 2, 4), (16, 8, 256), (33, 4, 8)])
def test_align_invariants_and_brute_force(tokens, top_k, experts):
    rng = np.random.default_rng(tokens + 17 * experts)
    ids = np.stack([rng.choice(experts, size=top_k, replace=False) for _ in range(tokens)])
    counts, offsets, perm, inverse = oracle.moe_align(ids, experts)
    flat = ids.reshape(-1)
    assert counts.tolist() == np.bincount(flat, minlength=experts).tolist()
    assert offsets[0] == 0 and offsets[-1] == flat.size
    assert (np.diff(offsets) == counts).all()
    assert (perm[inverse] == np.arange(flat.size)).all()
    assert (inverse[perm] == np.arange(flat.size)).all()
    # brute force: stable sort by expert id
    brute = [j for e in range(experts) for j in range(flat.size) if flat[j] == e]
    assert perm.tolist() == brute
    for e in range(experts):
        seg = perm[offsets[e] : offsets[e + 1]]
        assert (flat[seg] == e).all()
        assert (np.diff(seg) > 0).all()


# ---------------------------------------------------------------------------
# Experts: loop restatement vs a float64 dense restatement over all experts
# ---------------------------------------------------------------------------
def _dense_moe_f64(x, ids, w, gu, dn):
    """out = sum_e gate[t, e] * down_e(swiglu(gu_e x)) with one-hot gates."""

    t_count, e_count = x.shape[0], gu.shape[0]
    gates = torch.zeros(t_count, e_count, dtype=torch.float64)
    gates.scatter_add_(1, ids.long(), w.double())
    gu64, dn64, x64 = gu.double(), dn.double(), x.double()
    h = torch.einsum("eoh,th->teo", gu64, x64)
    act = F.silu(h[..., : h.shape[-1] // 2]) * h[..., h.shape[-1] // 2 :]
    y = torch.einsum("ehi,tei->teh", dn64, act)
    return (gates.unsqueeze(-1) * y).sum(1)


def test_routed_experts_match_dense_float64():
    g = torch.Generator().manual_seed(21)
    T, H, E, I, K = 3, 32, 8, 16, 3
    x = torch.randn(T, H, generator=g)
    gu = 0.1 * torch.randn(E, 2 * I, H, generator=g)
    dn = 0.1 * torch.randn(E, H, I, generator=g)
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)])
    w = torch.softmax(torch.randn(T, K, generator=g), -1)
    out = oracle.routed_experts(x, ids, w, gu, dn)
    torch.testing.assert_close(out.double(), _dense_moe_f64(x, ids, w, gu, dn), atol=1e-5, rtol=1e-5)


def test_fixed_routing_fixture_isolates_experts():
    # ids of tests/test_triton_moe.py:192 ; an expert not in the list must not matter
    g = torch.Generator().manual_seed(4)
    H, E, I = 16, 256, 8
    x = torch.randn(1, H, generator=g)
    gu = 0.1 * torch.randn(E, 2 * I, H, generator=g)
    dn = 0.1 * torch.randn(E, H, I, generator=g)
    ids = torch.tensor([[3, 17, 42, 89, 127, 199, 231, 255]])
    w = torch.full((1, 8), 1 / 8)
    out = oracle.routed_experts(x, ids, w, gu, dn)
    gu2 = gu.clone()
    gu2[0] += 1.0
    torch.testing.assert_close(out, oracle.routed_experts(x, ids, w, gu2, dn))
    torch.testing.assert_close(out.double(), _dense_moe_f64(x, ids, w, gu, dn), atol=1e-6, rtol=1e-6)


def test_shared_expert_gate_and_raw_input():
    g = torch.Generator().manual_seed(8)
    H, I = 16, 8
    x = torch.randn(2, H, generator=g)
    gu = 0.1 * torch.randn(2 * I, H, generator=g)
    dn = 0.1 * torch.randn(H, I, generator=g)
    wg = torch.randn(H, generator=g)
    ungated = oracle.shared_expert(x, gu, dn)
    gated = oracle.shared_expert(x, gu, dn, wg)
    torch.testing.assert_close(gated, ungated * torch.sigmoid(x @ wg).unsqueeze(-1))
    manual = torch.stack([dn @ (F.silu(gu[:I] @ x[t]) * (gu[I:] @ x[t])) for t in range(2)])
    torch.testing.assert_close(ungated, manual)


def test_moe_experts_use_unnormalised_hidden():
    g = torch.Generator().manual_seed(9)
    H, E, I = 16, 4, 8
    x = 3.0 * torch.randn(1, H, generator=g)
    w = {
        "nw": torch.zeros(H), "rw": 0.1 * torch.randn(E, H, generator=g),
        "gu": 0.1 * torch.randn(E, 2 * I, H, generator=g), "dn": 0.1 * torch.randn(E, H, I, generator=g),
        "sgu": 0.1 * torch.randn(2 * I, H, generator=g), "sdn": 0.1 * torch.randn(H, I, generator=g),
    }
    out, logits, ids, wts = oracle.moe_update(x, w["nw"], w["rw"], w["gu"], w["dn"], w["sgu"], w["sdn"], top_k=2)
    manual = sum(wts[0, k] * oracle.expert_mlp(x[0], w["gu"][ids[0, k]], w["dn"][ids[0, k]]) for k in range(2))
    manual = manual + oracle.expert_mlp(x[0], w["sgu"], w["sdn"])
    torch.testing.assert_close(out[0], manual)
    # scaling x scales the router input not at all (RMSNorm) but changes experts
    out2, logits2, _, _ = oracle.moe_update(2 * x, w["nw"], w["rw"], w["gu"], w["dn"], w["sgu"], w["sdn"], top_k=2)
    torch.testing.assert_close(logits2, logits, atol=1e-5, rtol=1e-5)
    assert not torch.allclose(out2, out)


# ---------------------------------------------------------------------------
# DeltaNet pieces
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("tokens", [1, 2, 5])
def test_conv_matches_torch_conv1d(tokens):
    g = torch.Generator().manual_seed(tokens)
    C, KS = 12, 4
    mixed = torch.randn(tokens, C, generator=g)
    state = torch.randn(C, KS, generator=g)
    w = torch.randn(C, 1, KS, generator=g)
    out, nxt = oracle.causal_conv_update(mixed, state, w)
    comb = torch.cat((state.unsqueeze(0), mixed.t().unsqueeze(0)), dim=-1)
    ref = F.silu(F.conv1d(comb, w, groups=C)[:, :, -tokens:]).squeeze(0).t()
    torch.testing.assert_close(out, ref)
    torch.testing.assert_close(nxt, comb[0, :, -KS:])


def test_conv_unit_last_tap_is_silu():
    C, KS = 5, 4
    mixed = torch.randn(3, C, generator=torch.Generator().manual_seed(1))
    w = torch.zeros(C, 1, KS)
    w[:, 0, KS - 1] = 1.0
    out, _ = oracle.causal_conv_update(mixed, torch.randn(C, KS), w)
    torch.testing.assert_close(out, F.silu(mixed))


def test_gated_rms_norm_constant_vector():
    core = torch.full((1, 8), 2.0)
    z = torch.zeros(1, 8)
    w = torch.ones(8)
    # silu(0) = 0
    torch.testing.assert_close(oracle.gated_rms_norm(core, z, w), torch.zeros(1, 8))
    z = torch.full((1, 8), 30.0)
    expected = torch.full((1, 8), 2.0 / (4.0 + 1e-6) ** 0.5 * 30.0 / (1 + np.exp(-30.0)))
    torch.testing.assert_close(oracle.gated_rms_norm(core, z, w), expected)


def _rand_recurrent(g, T, Hk, Hv, D):
    mixed = torch.randn(T, 2 * Hk * D + Hv * D, generator=g)
    a = torch.randn(T, Hv, generator=g)
    b = torch.randn(T, Hv, generator=g)
    state = 0.1 * torch.randn(Hv, D, D, generator=g)
    a_log = 0.1 * torch.randn(Hv, generator=g)
    dt_bias = 0.1 * torch.randn(Hv, generator=g)
    return mixed, a, b, state, a_log, dt_bias


def test_delta_rule_zero_state_closed_form():
    g = torch.Generator().manual_seed(2)
    T, Hk, Hv, D = 1, 2, 4, 8
    mixed, a, b, _, a_log, dt_bias = _rand_recurrent(g, T, Hk, Hv, D)
    core, state = oracle.deltanet_recurrent(
        mixed, a, b, torch.zeros(Hv, D, D), a_log, dt_bias, qk_heads=Hk, value_heads=Hv, head_dim=D
    )
    q = mixed[0, : Hk * D].reshape(Hk, D)
    k = mixed[0, Hk * D : 2 * Hk * D].reshape(Hk, D)
    v = mixed[0, 2 * Hk * D :].reshape(Hv, D)
    beta = torch.sigmoid(b[0])
    for h in range(Hv):
        qh = q[h // 2] / torch.sqrt((q[h // 2] ** 2).sum() + 1e-6) * D**-0.5
        kh = k[h // 2] / torch.sqrt((k[h // 2] ** 2).sum() + 1e-6)
        torch.testing.assert_close(core[0, h * D : (h + 1) * D], beta[h] * v[h] * (kh @ qh), atol=1e-6, rtol=1e-5)
        torch.testing.assert_close(state[h], torch.outer(kh, beta[h] * v[h]), atol=1e-6, rtol=1e-5)


def test_delta_rule_decay_one_is_rank_one_update():
    g = torch.Generator().manual_seed(6)
    T, Hk, Hv, D = 1, 1, 1, 4
    mixed, a, b, state, _, dt_bias = _rand_recurrent(g, T, Hk, Hv, D)
    a_log = torch.full((Hv,), -float("inf"))  # exp(A_log) = 0 -> g = 0 -> decay 1
    _, new_state = oracle.deltanet_recurrent(mixed, a, b, state, a_log, dt_bias, qk_heads=1, value_heads=1, head_dim=D)
    k = mixed[0, D : 2 * D]
    k = k / torch.sqrt((k * k).sum() + 1e-6)
    v = mixed[0, 2 * D :]
    delta = (v - state[0].t() @ k) * torch.sigmoid(b[0, 0])
    torch.testing.assert_close(new_state[0], state[0] + torch.outer(k, delta), atol=1e-6, rtol=1e-5)


def test_delta_rule_rows_are_sequential():
    g = torch.Generator().manual_seed(7)
    T, Hk, Hv, D = 3, 2, 4, 8
    mixed, a, b, state, a_log, dt_bias = _rand_recurrent(g, T, Hk, Hv, D)
    kw = dict(qk_heads=Hk, value_heads=Hv, head_dim=D)
    core, final = oracle.deltanet_recurrent(mixed, a, b, state, a_log, dt_bias, **kw)
    s = state
    for t in range(T):
        c, s = oracle.deltanet_recurrent(mixed[t : t + 1], a[t : t + 1], b[t : t + 1], s, a_log, dt_bias, **kw)
        torch.testing.assert_close(core[t], c[0])
    torch.testing.assert_close(final, s)


def test_delta_rule_matches_float64_loops():
    g = torch.Generator().manual_seed(12)
    T, Hk, Hv, D = 2, 2, 4, 8
    mixed, a, b, state, a_log, dt_bias = _rand_recurrent(g, T, Hk, Hv, D)
    core, final = oracle.deltanet_recurrent(mixed, a, b, state, a_log, dt_bias, qk_heads=Hk, value_heads=Hv, head_dim=D)
    m = mixed.double()
    S = state.double().clone()
    out = torch.zeros(T, Hv * D, dtype=torch.float64)
    for t in range(T):
        for h in range(Hv):
            hq = h // (Hv // Hk)
            q = m[t, hq * D : (hq + 1) * D]
            k = m[t, Hk * D + hq * D : Hk * D + (hq + 1) * D]
            v = m[t, 2 * Hk * D + h * D : 2 * Hk * D + (h + 1) * D]
            q = q / np.sqrt(float((q * q).sum()) + 1e-6) / np.sqrt(D)
            k = k / np.sqrt(float((k * k).sum()) + 1e-6)
            x = float(a[t, h]) + float(dt_bias[h])
            softplus = np.log1p(np.exp(x))
            decay = np.exp(-np.exp(float(a_log[h])) * softplus)
            beta = 1 / (1 + np.exp(-float(b[t, h])))
            for i, j in itertools.product(range(D), range(D)):
                S[h, i, j] *= decay
            for j in range(D):
                proj = sum(S[h, i, j] * k[i] for i in range(D))
                delta = (v[j] - proj) * beta
                for i in range(D):
                    S[h, i, j] += k[i] * delta
                out[t, h * D + j] = sum(S[h, i, j] * q[i] for i in range(D))
    torch.testing.assert_close(core.double(), out, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(final.double(), S, atol=1e-5, rtol=1e-5)


# ---------------------------------------------------------------------------
# Synthetic blocks: brute force in float64
# ---------------------------------------------------------------------------
def test_synthetic_moe_brute_force():
    g = torch.Generator().manual_seed(13)
    H, E, I, K = 16, 4, 8, 2
    layer = {
        "norm_weight": torch.ones(H), "router_weight": 0.2 * torch.randn(E, H, generator=g),
        "expert_gate_up_weight": 0.2 * torch.randn(E, 2 * I, H, generator=g),
        "expert_down_weight": 0.2 * torch.randn(E, H, I, generator=g),
        "shared_gate_up_weight": 0.2 * torch.randn(2 * I, H, generator=g),
        "shared_down_weight": 0.2 * torch.randn(H, I, generator=g),
    }
    x = torch.randn(H, generator=g)
    out = oracle.synthetic_moe_decode(x, layer, K)
    x64 = x.double()
    n = x64 / np.sqrt(float((x64 * x64).mean()) + 1e-6)
    logits = [float(n @ layer["router_weight"][e].double()) for e in range(E)]
    p = np.exp(np.array(logits) - max(logits))
    p /= p.sum()
    top = _brute_topk(p.tolist(), K)
    wsum = sum(p[e] for e in top)
    acc = x64.clone()
    for e in top:
        h = layer["expert_gate_up_weight"][e].double() @ x64
        acc += p[e] / wsum * (layer["expert_down_weight"][e].double() @ (F.silu(h[:I]) * h[I:]))
    h = layer["shared_gate_up_weight"].double() @ x64
    acc += layer["shared_down_weight"].double() @ (F.silu(h[:I]) * h[I:])
    torch.testing.assert_close(out.double(), acc, atol=1e-5, rtol=1e-5)


def test_synthetic_deltanet_brute_force():
    g = torch.Generator().manual_seed(14)
    H, Hk, D, Vd = 16, 2, 4, 8
    layer = {
        "norm_weight": torch.ones(H), "q_weight": 0.3 * torch.randn(Hk * D, H, generator=g),
        "k_weight": 0.3 * torch.randn(Hk * D, H, generator=g), "v_weight": 0.3 * torch.randn(Hk * Vd, H, generator=g),
        "gate_weight": 0.3 * torch.randn(Hk * Vd, H, generator=g), "out_weight": 0.3 * torch.randn(H, Hk * Vd, generator=g),
    }
    x = torch.randn(H, generator=g)
    state = torch.randn(Hk, D, Vd, generator=g)
    out, new_state = oracle.synthetic_deltanet_decode(x, state, layer, qk_heads=Hk, head_dim=D, value_dim_per_head=Vd)
    x64 = x.double()
    n = x64 / np.sqrt(float((x64 * x64).mean()) + 1e-6)
    q = (layer["q_weight"].double() @ n).reshape(Hk, D)
    k = (layer["k_weight"].double() @ n).reshape(Hk, D)
    v = (layer["v_weight"].double() @ n).reshape(Hk, Vd)
    gate = torch.sigmoid(layer["gate_weight"].double() @ n).reshape(Hk, Vd)
    S = torch.zeros(Hk, D, Vd, dtype=torch.float64)
    r = torch.zeros(Hk, Vd, dtype=torch.float64)
    for h, d, j in itertools.product(range(Hk), range(D), range(Vd)):
        S[h, d, j] = 0.95 * float(state[h, d, j]) + k[h, d] * v[h, j]
    for h, j in itertools.product(range(Hk), range(Vd)):
        r[h, j] = sum(q[h, d] * S[h, d, j] for d in range(D)) * gate[h, j]
    ref = x64 + layer["out_weight"].double() @ r.reshape(-1)
    torch.testing.assert_close(new_state.double(), S, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(out.double(), ref, atol=1e-5, rtol=1e-5)
