"""Pins the oracle's DeltaNet compositions and layer wiring with closed forms.

`oracle.deltanet_project` (reference/qwen36_real.py:126-130),
`oracle.deltanet_recurrent_output` (:205-260, gated norm + out-proj at
:252-259), `oracle.deltanet_update` (:111-148) and the residual wiring of
`moe_layer` / `deltanet_moe_layer` / `attention_moe_layer` (:357-375,
:378-399) are checked here against answers computed independently in
float64 numpy.  Each check is chosen so a plausible slip fails it: a norm
offset of 0 or a norm over the wrong axis, the gated RMSNorm taken over all
heads instead of per head, (1 + w) where the reference has plain w, W_out
or an input projection transposed, the z / a / b outputs swapped, z passed
through the conv, the MoE fed h instead of h + update, or the residual
dropped.
"""

from __future__ import annotations

import numpy as np
import torch

import oracle


def _rms64(x: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    return np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)


def _silu64(x: np.ndarray) -> np.ndarray:
    return x / (1.0 + np.exp(-x))


# ---------------------------------------------------------------------------
# deltanet_project: RMSNorm(1 + w) then four projections
# ---------------------------------------------------------------------------
def _one_hot_rows(rows: int, cols: int, pick: np.ndarray, scale: np.ndarray | None = None) -> torch.Tensor:
    w = np.zeros((rows, cols), dtype=np.float32)
    w[np.arange(rows), pick] = 1.0 if scale is None else scale
    return torch.from_numpy(w)


def test_deltanet_project_one_hot_rows_pick_normalised_coordinates():
    rng = np.random.default_rng(0)
    T, H, nqkv, nz, nab = 3, 24, 10, 6, 4
    x = rng.standard_normal((T, H)).astype(np.float32)
    norm_w = (0.3 * rng.standard_normal(H)).astype(np.float32)
    picks = [rng.integers(0, H, n) for n in (nqkv, nz, nab, nab)]
    scales = [rng.uniform(0.5, 2.0, n).astype(np.float32) for n in (nqkv, nz, nab, nab)]
    ws = [_one_hot_rows(n, H, p, s) for n, p, s in zip((nqkv, nz, nab, nab), picks, scales)]
    outs = oracle.deltanet_project(torch.from_numpy(x), torch.from_numpy(norm_w), *ws)
    xn = x.astype(np.float64) / _rms64(x.astype(np.float64)) * (1.0 + norm_w.astype(np.float64))
    for out, p, s, n in zip(outs, picks, scales, (nqkv, nz, nab, nab)):
        assert tuple(out.shape) == (T, n)
        np.testing.assert_allclose(out.double().numpy(), xn[:, p] * s, rtol=1e-5, atol=1e-6)


def test_deltanet_project_offset_and_weight_scale():
    g = torch.Generator().manual_seed(1)
    T, H = 2, 32
    x = torch.randn(T, H, generator=g)
    ws = [torch.randn(n, H, generator=g) for n in (12, 8, 4, 4)]
    z0 = oracle.deltanet_project(x, torch.zeros(H), *ws)
    z1 = oracle.deltanet_project(x, torch.ones(H), *ws)
    for a, b in zip(z0, z1):
        torch.testing.assert_close(b, 2.0 * a, rtol=1e-5, atol=1e-6)
    # offset 0 with w = 0 removes the input entirely
    for out in oracle.deltanet_project(x, torch.zeros(H), *ws, norm_offset=0.0):
        assert float(out.abs().max()) == 0.0
    # the norm is per token (row), not over the batch: scaling one token
    # leaves every projection unchanged
    xs = x.clone()
    xs[1] *= 37.0
    for a, b in zip(z0, oracle.deltanet_project(xs, torch.zeros(H), *ws)):
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------------------
# deltanet_recurrent_output: per-head gated RMSNorm (plain w) and W_out
# ---------------------------------------------------------------------------
def _zero_state_setup(Hk, Hv, D, head_scales, rng):
    """Inputs whose recurrent core has the closed form o_h = v_h / sqrt(D).

    With S = 0, beta = 1 (b large) and q_h, k_h along one direction,
    S' = k (x) v and o = q . S' = (q . k) v = v / sqrt(D) (q is scaled by
    D^-1/2 after the l2 norm).
    """

    T = 1
    direction = rng.standard_normal((Hk, D))
    q = direction * rng.uniform(0.5, 3.0, (Hk, 1))
    k = direction * rng.uniform(0.5, 3.0, (Hk, 1))
    v = rng.standard_normal((Hv, D)) * np.asarray(head_scales)[:, None]
    mixed = np.concatenate([q.ravel(), k.ravel(), v.ravel()])[None, :].astype(np.float32)
    b = np.full((T, Hv), 40.0, dtype=np.float32)  # sigmoid(40) == 1 in fp32
    a = rng.standard_normal((T, Hv)).astype(np.float32)
    state = np.zeros((Hv, D, D), dtype=np.float32)
    a_log = rng.standard_normal(Hv).astype(np.float32)
    dt_bias = rng.standard_normal(Hv).astype(np.float32)
    core = v.astype(np.float32).astype(np.float64) / np.sqrt(D)
    return mixed, a, b, state, a_log, dt_bias, core


def test_recurrent_output_gated_norm_is_per_head_with_plain_weight():
    rng = np.random.default_rng(2)
    Hk, Hv, D = 2, 4, 8
    scales = [1e-2, 1.0, 30.0, 300.0]  # heads at very different scales
    mixed, a, b, state, a_log, dt_bias, core = _zero_state_setup(Hk, Hv, D, scales, rng)
    z = rng.standard_normal((1, Hv * D)).astype(np.float32)
    norm_w = rng.uniform(0.2, 0.8, D).astype(np.float32)  # (1 + w) would differ by > 2x
    w_out = torch.eye(Hv * D)  # identity: the update is the normalised core itself
    update, next_state = oracle.deltanet_recurrent_output(
        torch.from_numpy(mixed), torch.from_numpy(z), torch.from_numpy(a), torch.from_numpy(b),
        torch.from_numpy(state), w_out, torch.from_numpy(norm_w), torch.from_numpy(a_log),
        torch.from_numpy(dt_bias), qk_heads=Hk, value_heads=Hv, head_dim=D,
    )
    heads = core.reshape(Hv, D)
    zz = z.astype(np.float64).reshape(Hv, D)
    expected = heads / _rms64(heads) * norm_w.astype(np.float64) * _silu64(zz)
    np.testing.assert_allclose(update.double().numpy().reshape(Hv, D), expected, rtol=1e-4, atol=1e-6)
    # every head's normalised core has RMS sqrt(ms / (ms + eps)) (1 unless the
    # head is tiny), with silu(z) and w divided out
    per_head_rms = _rms64(update.double().numpy().reshape(Hv, D) / (norm_w * _silu64(zz)), 0.0)
    ms = np.mean(heads * heads, axis=-1)
    np.testing.assert_allclose(per_head_rms.ravel(), np.sqrt(ms / (ms + 1e-6)), rtol=1e-4)
    assert per_head_rms.ravel()[1:].min() > 0.999
    # state: k_hat (x) v per value head (GQA: head h reads qk head h // 2)
    k = mixed[0, Hk * D : 2 * Hk * D].reshape(Hk, D).astype(np.float64)
    v = mixed[0, 2 * Hk * D :].reshape(Hv, D).astype(np.float64)
    for h in range(Hv):
        kh = k[h // 2] / np.sqrt((k[h // 2] ** 2).sum() + 1e-6)
        np.testing.assert_allclose(next_state[h].double().numpy(), np.outer(kh, v[h]), rtol=1e-4, atol=1e-5)


def test_recurrent_output_projection_orientation_non_square():
    rng = np.random.default_rng(3)
    Hk, Hv, D, H = 1, 2, 8, 5  # W_out [H, Hv*D] = [5, 16]: a transpose cannot even multiply
    mixed, a, b, state, a_log, dt_bias, core = _zero_state_setup(Hk, Hv, D, [0.5, 4.0], rng)
    z = rng.standard_normal((1, Hv * D)).astype(np.float32)
    norm_w = np.ones(D, dtype=np.float32)
    pick = rng.integers(0, Hv * D, H)
    coef = rng.uniform(0.5, 2.0, H).astype(np.float32)
    w_out = _one_hot_rows(H, Hv * D, pick, coef)
    update, _ = oracle.deltanet_recurrent_output(
        torch.from_numpy(mixed), torch.from_numpy(z), torch.from_numpy(a), torch.from_numpy(b),
        torch.from_numpy(state), w_out, torch.from_numpy(norm_w), torch.from_numpy(a_log),
        torch.from_numpy(dt_bias), qk_heads=Hk, value_heads=Hv, head_dim=D,
    )
    heads = core.reshape(Hv, D)
    normed = (heads / _rms64(heads) * _silu64(z.astype(np.float64).reshape(Hv, D))).ravel()
    assert tuple(update.shape) == (1, H)
    np.testing.assert_allclose(update.double().numpy()[0], normed[pick] * coef, rtol=1e-4, atol=1e-6)


# ---------------------------------------------------------------------------
# deltanet_update: the conv sits between the projections and the rule, and
# only the qkv channels go through it
# ---------------------------------------------------------------------------
def test_deltanet_update_convolves_qkv_only():
    g = torch.Generator().manual_seed(4)
    Hk, Hv, D, H = 1, 2, 4, 16
    C = 2 * Hk * D + Hv * D
    conv_w = torch.zeros(C, 1, 4)
    conv_w[:, 0, -1] = 1.0  # unit last tap: conv output = silu(current input)
    w = dict(
        input_norm_weight=0.1 * torch.randn(H, generator=g),
        in_proj_qkv_weight=torch.randn(C, H, generator=g) / 4,
        in_proj_z_weight=torch.randn(Hv * D, H, generator=g) / 4,
        in_proj_a_weight=torch.randn(Hv, H, generator=g) / 4,
        in_proj_b_weight=torch.randn(Hv, H, generator=g) / 4,
        conv1d_weight=conv_w,
        out_proj_weight=torch.randn(H, Hv * D, generator=g) / 4,
        linear_norm_weight=torch.rand(D, generator=g) + 0.5,
        a_log=0.1 * torch.randn(Hv, generator=g),
        dt_bias=0.1 * torch.randn(Hv, generator=g),
    )
    x = torch.randn(1, H, generator=g)
    conv_state = torch.randn(C, 4, generator=g)
    rec = 0.1 * torch.randn(Hv, D, D, generator=g)
    kw = dict(qk_heads=Hk, value_heads=Hv, head_dim=D)
    update, next_conv, next_rec = oracle.deltanet_update(x, conv_state, rec, w, **kw)
    mixed, z, a, b = oracle.deltanet_project(
        x, w["input_norm_weight"], w["in_proj_qkv_weight"], w["in_proj_z_weight"], w["in_proj_a_weight"],
        w["in_proj_b_weight"],
    )
    expected, expected_rec = oracle.deltanet_recurrent_output(
        torch.nn.functional.silu(mixed), z, a, b, rec, w["out_proj_weight"], w["linear_norm_weight"], w["a_log"],
        w["dt_bias"], **kw,
    )
    torch.testing.assert_close(update, expected, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(next_rec, expected_rec, rtol=1e-5, atol=1e-6)
    # the state rolls by one column and takes the new projection last
    torch.testing.assert_close(next_conv[:, :3], conv_state[:, 1:])
    torch.testing.assert_close(next_conv[:, 3], mixed[0])


# ---------------------------------------------------------------------------
# Residual wiring of the layers
# ---------------------------------------------------------------------------
def _tiny_moe(g, H):
    """One expert (E = 1, K = 1, I = 1), no shared contribution: moe(x) = d * silu(gx) * (ux)."""

    gate = torch.randn(H, generator=g)
    up = torch.randn(H, generator=g)
    d = torch.randn(H, generator=g)
    return dict(
        norm_weight=torch.zeros(H),
        router_weight=torch.randn(1, H, generator=g),
        expert_gate_up_weight=torch.stack([gate, up])[None],  # [1, 2, H]
        expert_down_weight=d.reshape(1, H, 1),
        shared_gate_up_weight=torch.zeros(2, H),
        shared_down_weight=torch.zeros(H, 1),
    )


def _tiny_moe64(mw, x: np.ndarray) -> np.ndarray:
    gu = mw["expert_gate_up_weight"][0].double().numpy()
    d = mw["expert_down_weight"][0, :, 0].double().numpy()
    return (_silu64(x @ gu[0]) * (x @ gu[1]))[:, None] * d[None, :]


def test_moe_layer_adds_the_residual():
    g = torch.Generator().manual_seed(5)
    H = 8
    mw = _tiny_moe(g, H)
    x = torch.randn(2, H, generator=g)
    layer_hidden, update, _, ids, weights = oracle.moe_layer(
        x, mw["norm_weight"], mw["router_weight"], mw["expert_gate_up_weight"], mw["expert_down_weight"],
        mw["shared_gate_up_weight"], mw["shared_down_weight"], top_k=1,
    )
    assert ids.tolist() == [[0], [0]] and weights.tolist() == [[1.0], [1.0]]
    x64 = x.double().numpy()
    np.testing.assert_allclose(update.double().numpy(), _tiny_moe64(mw, x64), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(layer_hidden.double().numpy(), x64 + _tiny_moe64(mw, x64), rtol=1e-5, atol=1e-6)


def test_deltanet_moe_layer_feeds_h_plus_update_to_the_moe():
    g = torch.Generator().manual_seed(6)
    Hk, Hv, D, H = 1, 2, 4, 8
    C = 2 * Hk * D + Hv * D
    dn = dict(
        input_norm_weight=0.1 * torch.randn(H, generator=g),
        in_proj_qkv_weight=torch.randn(C, H, generator=g) / 3,
        in_proj_z_weight=torch.randn(Hv * D, H, generator=g) / 3,
        in_proj_a_weight=torch.randn(Hv, H, generator=g) / 3,
        in_proj_b_weight=torch.randn(Hv, H, generator=g) / 3,
        conv1d_weight=torch.randn(C, 1, 4, generator=g) / 2,
        out_proj_weight=torch.randn(H, Hv * D, generator=g),
        linear_norm_weight=torch.rand(D, generator=g) + 0.5,
        a_log=0.1 * torch.randn(Hv, generator=g),
        dt_bias=0.1 * torch.randn(Hv, generator=g),
    )
    mw = _tiny_moe(g, H)
    x = torch.randn(1, H, generator=g)
    conv_state = torch.randn(C, 4, generator=g)
    rec = 0.1 * torch.randn(Hv, D, D, generator=g)
    kw = dict(qk_heads=Hk, value_heads=Hv, head_dim=D)
    out = oracle.deltanet_moe_layer(x, conv_state, rec, dn, mw, top_k=1, **kw)
    layer_hidden, dn_hidden, dn_update, moe_out = out[:4]
    ref_update, ref_conv, ref_rec = oracle.deltanet_update(x, conv_state, rec, dn, **kw)
    torch.testing.assert_close(dn_update, ref_update)
    torch.testing.assert_close(out[4], ref_conv)
    torch.testing.assert_close(out[5], ref_rec)
    h64 = x.double().numpy() + ref_update.double().numpy()
    np.testing.assert_allclose(dn_hidden.double().numpy(), h64, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(moe_out.double().numpy(), _tiny_moe64(mw, h64), rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(layer_hidden.double().numpy(), h64 + _tiny_moe64(mw, h64), rtol=1e-4, atol=1e-5)
    # the check discriminates: the MoE of the raw input is far from it
    assert np.abs(_tiny_moe64(mw, x.double().numpy()) - _tiny_moe64(mw, h64)).max() > 1e-2


def test_attention_moe_layer_feeds_h_plus_update_to_the_moe():
    g = torch.Generator().manual_seed(7)
    heads, kv_heads, hd, H = 2, 1, 4, 8
    aw = dict(
        input_norm_weight=0.1 * torch.randn(H, generator=g),
        q_proj_weight=torch.randn(2 * heads * hd, H, generator=g) / 3,
        k_proj_weight=torch.randn(kv_heads * hd, H, generator=g) / 3,
        v_proj_weight=torch.randn(kv_heads * hd, H, generator=g) / 3,
        o_proj_weight=torch.randn(H, heads * hd, generator=g),
        q_norm_weight=0.1 * torch.randn(hd, generator=g),
        k_norm_weight=0.1 * torch.randn(hd, generator=g),
    )
    mw = _tiny_moe(g, H)
    x = torch.randn(1, H, generator=g)
    kc = torch.randn(6, kv_heads, hd, generator=g)
    vc = torch.randn(6, kv_heads, hd, generator=g)
    kw = dict(start_position=3, heads=heads, kv_heads=kv_heads, head_dim=hd, rope_dim=2, rope_theta=1e4)
    out = oracle.attention_moe_layer(x, kc, vc, aw, mw, top_k=1, **kw)
    layer_hidden, attn_hidden, attn_update, moe_out = out[:4]
    ref_update, _, _ = oracle.attention_update(
        x, kc, vc, aw["input_norm_weight"], aw["q_proj_weight"], aw["k_proj_weight"], aw["v_proj_weight"],
        aw["o_proj_weight"], aw["q_norm_weight"], aw["k_norm_weight"], **kw,
    )
    torch.testing.assert_close(attn_update, ref_update)
    h64 = x.double().numpy() + ref_update.double().numpy()
    np.testing.assert_allclose(attn_hidden.double().numpy(), h64, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(moe_out.double().numpy(), _tiny_moe64(mw, h64), rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(layer_hidden.double().numpy(), h64 + _tiny_moe64(mw, h64), rtol=1e-4, atol=1e-5)
    assert np.abs(_tiny_moe64(mw, x.double().numpy()) - _tiny_moe64(mw, h64)).max() > 1e-2
