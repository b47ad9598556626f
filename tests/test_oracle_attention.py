"""Pins the attention part of the CPU oracle (oracle.rope, oracle.attention_update)
against facts that do not come from the oracle's own formulas: RoPE as
complex multiplication, its identity at position 0, norm preservation,
offset-only dot products and the permutation that links the two pairings;
the attention core against torch's scaled_dot_product_attention; a single
cached position; the cache rows a step may touch.  Shapes are the real
Qwen3.6 attention heads (16 query / 2 kv heads of 256, rope_dim 64,
theta 1e7) with a reduced hidden size.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

import oracle

HEADS, KVH, HD, RD, THETA, H = 16, 2, 256, 64, 1.0e7, 128


def _weights(seed=0):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s, sc=0.05: torch.randn(*s, generator=g) * sc  # noqa: E731
    return dict(
        norm=r(H, sc=0.2), wq=r(2 * HEADS * HD, H), wk=r(KVH * HD, H), wv=r(KVH * HD, H), wo=r(H, HEADS * HD),
        qn=r(HD, sc=0.2), kn=r(HD, sc=0.2),
    )


@pytest.mark.parametrize("interleaved", [True, False])
def test_rope_identity_at_zero_and_norm_preserving(interleaved):
    x = torch.randn(3, 4, HD, generator=torch.Generator().manual_seed(1))
    assert torch.equal(oracle.rope(x, torch.zeros(3), RD, THETA, interleaved), x)
    y = oracle.rope(x, torch.tensor([5.0, 1000.0, 123456.0]), RD, THETA, interleaved)
    assert torch.equal(y[..., RD:], x[..., RD:])  # dims past rope_dim pass through
    assert torch.allclose(y[..., :RD].norm(dim=-1), x[..., :RD].norm(dim=-1), rtol=1e-5)


def test_rope_interleaved_is_complex_multiplication():
    x = torch.randn(2, 3, HD, generator=torch.Generator().manual_seed(2), dtype=torch.float64)
    pos = torch.tensor([7.0, 300.0])
    y = oracle.rope(x, pos, RD, THETA, True)
    z = torch.complex(x[..., 0:RD:2], x[..., 1:RD:2])
    freq = THETA ** (-torch.arange(0, RD, 2, dtype=torch.float64) / RD)
    rot = torch.polar(torch.ones_like(freq), pos.double()[:, None] * freq[None, :])[:, None, :]
    w = z * rot
    torch.testing.assert_close(y[..., 0:RD:2].double(), w.real, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(y[..., 1:RD:2].double(), w.imag, atol=1e-5, rtol=1e-5)


def test_rope_pairings_differ_by_a_dim_permutation():
    # halves pairing == interleaved pairing conjugated by the permutation that
    # sends dims (0, 1, 2, 3, ..) of the interleaved layout to (0, h, 1, h+1, ..)
    x = torch.randn(2, 2, HD, generator=torch.Generator().manual_seed(3))
    pos = torch.tensor([3.0, 40.0])
    h = RD // 2
    perm = torch.arange(HD)
    perm[0:RD:2], perm[1:RD:2] = torch.arange(h), torch.arange(h, RD)
    inter = oracle.rope(x[..., perm], pos, RD, THETA, True)
    half = oracle.rope(x, pos, RD, THETA, False)
    torch.testing.assert_close(inter, half[..., perm], atol=1e-6, rtol=1e-6)


@pytest.mark.parametrize("interleaved", [True, False])
def test_rope_dot_products_depend_on_offset_only(interleaved):
    g = torch.Generator().manual_seed(4)
    q, k = torch.randn(1, 1, HD, generator=g, dtype=torch.float64), torch.randn(1, 1, HD, generator=g, dtype=torch.float64)
    d1 = (oracle.rope(q, torch.tensor([10.0]), RD, 1e4, interleaved) * oracle.rope(k, torch.tensor([3.0]), RD, 1e4, interleaved)).sum()
    d2 = (oracle.rope(q, torch.tensor([107.0]), RD, 1e4, interleaved) * oracle.rope(k, torch.tensor([100.0]), RD, 1e4, interleaved)).sum()
    assert abs(float(d1 - d2)) < 1e-4


@pytest.mark.parametrize("start,tokens", [(0, 1), (5, 3), (17, 2)])
def test_attention_update_matches_sdpa_restatement(start, tokens):
    w = _weights()
    g = torch.Generator().manual_seed(5)
    maxp = start + tokens + 2
    x = torch.randn(tokens, H, generator=g)
    kc, vc = torch.randn(maxp, KVH, HD, generator=g) * 0.5, torch.randn(maxp, KVH, HD, generator=g) * 0.5
    upd, nkc, nvc = oracle.attention_update(
        x, kc, vc, w["norm"], w["wq"], w["wk"], w["wv"], w["wo"], w["qn"], w["kn"], start_position=start, heads=HEADS,
        kv_heads=KVH, head_dim=HD, rope_dim=RD, rope_theta=THETA)
    # independent restatement: same projections, SDPA over the updated cache
    xn = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6) * (1 + w["norm"])
    qg = (xn @ w["wq"].t()).reshape(tokens, HEADS, 2 * HD)
    q, gate = qg[..., :HD], qg[..., HD:]
    hn = lambda t, wt: t * torch.rsqrt(t.pow(2).mean(-1, keepdim=True) + 1e-6) * (1 + wt)  # noqa: E731
    pos = torch.arange(start, start + tokens)
    q = oracle.rope(hn(q, w["qn"]), pos, RD, THETA, True)
    assert torch.equal(nkc[:start], kc[:start]) and torch.equal(nkc[start + tokens:], kc[start + tokens:])
    assert torch.equal(nvc[:start], vc[:start]) and torch.equal(nvc[start + tokens:], vc[start + tokens:])
    v_new = (xn @ w["wv"].t()).reshape(tokens, KVH, HD)
    torch.testing.assert_close(nvc[start:start + tokens], v_new)
    k_new = oracle.rope(hn((xn @ w["wk"].t()).reshape(tokens, KVH, HD), w["kn"]), pos, RD, THETA, True)
    torch.testing.assert_close(nkc[start:start + tokens], k_new)
    keys = nkc[: start + tokens].repeat_interleave(HEADS // KVH, dim=1).permute(1, 0, 2)  # [heads, P, hd]
    vals = nvc[: start + tokens].repeat_interleave(HEADS // KVH, dim=1).permute(1, 0, 2)
    mask = torch.arange(start + tokens)[None, :] <= pos[:, None]  # [T, P]
    att = F.scaled_dot_product_attention(q.permute(1, 0, 2), keys, vals, attn_mask=mask)  # [heads, T, hd]
    ref = (att.permute(1, 0, 2).reshape(tokens, -1) * torch.sigmoid(gate.reshape(tokens, -1))) @ w["wo"].t()
    torch.testing.assert_close(upd, ref, atol=1e-4, rtol=1e-4)


def test_attention_single_position_returns_the_value_row():
    w = _weights(1)
    x = torch.randn(1, H, generator=torch.Generator().manual_seed(6))
    kc = torch.zeros(1, KVH, HD)
    upd, nkc, nvc = oracle.attention_update(
        x, kc, kc.clone(), w["norm"], w["wq"], w["wk"], w["wv"], w["wo"], w["qn"], w["kn"], start_position=0,
        heads=HEADS, kv_heads=KVH, head_dim=HD, rope_dim=RD, rope_theta=THETA, interleaved=False)
    xn = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6) * (1 + w["norm"])
    gate = (xn @ w["wq"].t()).reshape(1, HEADS, 2 * HD)[..., HD:]
    att = nvc[0].repeat_interleave(HEADS // KVH, dim=0)[None]  # softmax over one position is 1
    ref = (att.reshape(1, -1) * torch.sigmoid(gate.reshape(1, -1))) @ w["wo"].t()
    torch.testing.assert_close(upd, ref, atol=1e-5, rtol=1e-5)


# ---------------------------------------------------------------------------
# The synthetic (tiny-spec) attention block: oracle.synthetic_rope and
# oracle.synthetic_attention_decode (reference/qwen36_decode.py:37-56,174-209)
# ---------------------------------------------------------------------------
def _complex_rope64(x, position, rope_dim):
    """Interleaved RoPE as multiplication of (even + i odd) by e^{i p theta_j},
    theta_j = 10000^(-2j / r), in float64."""

    r = min(rope_dim, x.shape[-1])
    r -= r % 2
    x = x.double()
    out = x.clone()
    if r == 0:
        return out
    z = torch.complex(x[..., :r:2], x[..., 1:r:2])
    theta = 10000.0 ** (-torch.arange(0, r, 2, dtype=torch.float64) / r)
    z = z * torch.polar(torch.ones_like(theta), position * theta)
    out[..., :r:2], out[..., 1:r:2] = z.real, z.imag
    return out


@pytest.mark.parametrize("rope_dim", [0, 3, 4, 6])
def test_synthetic_rope_is_complex_multiplication(rope_dim):
    x = torch.randn(3, 6, generator=torch.Generator().manual_seed(3))
    assert torch.equal(oracle.synthetic_rope(x, 0, rope_dim), x)
    for p in (1, 5, 77):
        torch.testing.assert_close(oracle.synthetic_rope(x, p, rope_dim).double(), _complex_rope64(x, p, rope_dim),
                                   rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("position", [0, 2, 7])
def test_synthetic_attention_decode_matches_sdpa_restatement(position):
    g = torch.Generator().manual_seed(10 + position)
    H, heads, kvh, hd, rd, P = 16, 4, 2, 4, 4, 8
    layer = dict(norm_weight=1 + 0.2 * torch.randn(H, generator=g), q_weight=0.3 * torch.randn(heads * hd, H, generator=g),
                 k_weight=0.3 * torch.randn(kvh * hd, H, generator=g), v_weight=0.3 * torch.randn(kvh * hd, H, generator=g),
                 out_weight=0.3 * torch.randn(H, heads * hd, generator=g))
    x = torch.randn(H, generator=g)
    kc, vc = torch.randn(P, kvh, hd, generator=g), torch.randn(P, kvh, hd, generator=g)
    kc0, vc0 = kc.clone(), vc.clone()
    out, nkc, nvc = oracle.synthetic_attention_decode(x, kc, vc, layer, attention_heads=heads, kv_heads=kvh,
                                                      head_dim=hd, rope_dim=rd, position=position)
    assert torch.equal(kc, kc0) and torch.equal(vc, vc0)  # the inputs are not touched
    # independent float64 restatement: RMSNorm by its formula, RoPE as complex
    # multiplication, attention by the library's SDPA over expanded kv heads
    x64 = x.double()
    xn = x64 / torch.sqrt((x64 * x64).mean() + 1e-6) * layer["norm_weight"].double()
    q = _complex_rope64((layer["q_weight"].double() @ xn).reshape(heads, hd), position, rd)
    k = _complex_rope64((layer["k_weight"].double() @ xn).reshape(kvh, hd), position, rd)
    v = (layer["v_weight"].double() @ xn).reshape(kvh, hd)
    keys, vals = kc0.double().clone(), vc0.double().clone()
    keys[position], vals[position] = k, v
    K = keys[: position + 1].permute(1, 0, 2).repeat_interleave(heads // kvh, dim=0)  # [heads, t, hd]
    V = vals[: position + 1].permute(1, 0, 2).repeat_interleave(heads // kvh, dim=0)
    att = F.scaled_dot_product_attention(q[:, None, :], K, V)[:, 0, :].reshape(-1)
    ref = x64 + layer["out_weight"].double() @ att
    torch.testing.assert_close(out.double(), ref, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(nkc[position].double(), k, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(nvc[position].double(), v, rtol=1e-5, atol=1e-5)
    rows = [t for t in range(P) if t != position]
    assert torch.equal(nkc[rows], kc0[rows]) and torch.equal(nvc[rows], vc0[rows])
