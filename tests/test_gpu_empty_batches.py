"""Batches of no tokens through the batched operators.

The reference's batched operators allocate their outputs with the token count
as the leading size and launch grids whose first dimension is that count
(e.g. qwen36_router.py:288-317, qwen36_expert.py:1096-1178,
qwen36_attention.py:448-577); at zero tokens nothing runs and the outputs
come back empty, with the caches cloned or passed through.  Its conv and
recurrent stages reject zero tokens (qwen36_deltanet.py:555-556, :789-790),
and so does the DeltaNet -> MoE layer, which calls them.  The HIP operators
match: no call of the C ABI, empty outputs of the same shapes and dtypes,
and the same ValueErrors.
"""

from __future__ import annotations

import pytest
import torch

from fastkernels_amd.kernels import hip

pytestmark = pytest.mark.gpu

H, E, I, K = 256, 16, 64, 4


def _bf(*shape, device, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * 0.05).to(torch.bfloat16).to(device)


@pytest.fixture(scope="module")
def moe(device):
    return dict(norm=_bf(H, device=device), router=_bf(E, H, device=device, seed=1),
                gu=_bf(E, 2 * I, H, device=device, seed=2), dn=_bf(E, H, I, device=device, seed=3),
                sgu=_bf(2 * I, H, device=device, seed=4), sdn=_bf(H, I, device=device, seed=5),
                sg=_bf(H, device=device, seed=6))


def _empty(t, shape, dtype):
    assert tuple(t.shape) == shape and t.dtype == dtype and t.is_cuda


def test_moe_operators_at_zero_tokens(device, moe):
    x = torch.empty((0, H), device=device, dtype=torch.bfloat16)
    logits, ids, w = hip.hip_qwen36_batched_moe_router_decode(x, moe["norm"], moe["router"], top_k=K)
    _empty(logits, (0, E), torch.float32)
    _empty(ids, (0, K), torch.int64)
    _empty(w, (0, K), torch.float32)
    out = hip.hip_qwen36_batched_routed_experts_decode(x, ids, w, moe["gu"], moe["dn"])
    _empty(out, (0, H), torch.float32)
    out = hip.hip_qwen36_batched_routed_shared_experts_decode(x, ids, w, moe["gu"], moe["dn"], moe["sgu"],
                                                               moe["sdn"], moe["sg"])
    _empty(out, (0, H), torch.float32)
    res = hip.hip_qwen36_batched_moe_decode(x, moe["norm"], moe["router"], moe["gu"], moe["dn"], moe["sgu"],
                                            moe["sdn"], moe["sg"], top_k=K)
    for t, shape, dt in zip(res, [(0, H), (0, E), (0, K), (0, K)],
                            [torch.float32, torch.float32, torch.int64, torch.float32]):
        _empty(t, shape, dt)
    res = hip.hip_qwen36_batched_moe_layer_decode(x, moe["norm"], moe["router"], moe["gu"], moe["dn"], moe["sgu"],
                                                  moe["sdn"], moe["sg"], top_k=K)
    for t, shape, dt in zip(res, [(0, H), (0, H), (0, E), (0, K), (0, K)],
                            [torch.float32, torch.float32, torch.float32, torch.int64, torch.float32]):
        _empty(t, shape, dt)
    # a following call with tokens still runs on the same workspace
    x1 = _bf(3, H, device=device, seed=9)
    logits, ids, w = hip.hip_qwen36_batched_moe_router_decode(x1, moe["norm"], moe["router"], top_k=K)
    torch.cuda.synchronize()
    assert torch.isfinite(logits).all() and torch.isfinite(w).all()
    assert ((ids >= 0) & (ids < E)).all()


def test_deltanet_operators_at_zero_tokens(device):
    qk_heads, value_heads, head_dim, ks = 2, 4, 32, 4
    key_dim, value_dim = qk_heads * head_dim, value_heads * head_dim
    conv_dim = 2 * key_dim + value_dim
    x = torch.empty((0, H), device=device, dtype=torch.bfloat16)
    wq, wz = _bf(conv_dim, H, device=device, seed=1), _bf(value_dim, H, device=device, seed=2)
    wa, wb = _bf(value_heads, H, device=device, seed=3), _bf(value_heads, H, device=device, seed=4)
    mixed, z, a, b = hip.hip_qwen36_batched_deltanet_project(x, _bf(H, device=device), wq, wz, wa, wb)
    _empty(mixed, (0, conv_dim), torch.float32)
    _empty(z, (0, value_dim), torch.float32)
    _empty(a, (0, value_heads), torch.float32)
    _empty(b, (0, value_heads), torch.float32)
    conv_state = torch.zeros(conv_dim, ks, device=device)
    conv_w = _bf(conv_dim, 1, ks, device=device, seed=5)
    with pytest.raises(ValueError, match="tokens must be positive"):
        hip.hip_qwen36_batched_deltanet_conv(mixed, conv_state, conv_w)
    state = torch.zeros(value_heads, head_dim, head_dim, device=device)
    with pytest.raises(ValueError, match="tokens must be positive"):
        hip.hip_qwen36_batched_deltanet_recurrent_output(
            mixed, z, a, b, state, _bf(H, value_dim, device=device), _bf(head_dim, device=device),
            torch.zeros(value_heads, device=device), torch.zeros(value_heads, device=device),
            qk_heads=qk_heads, value_heads=value_heads, head_dim=head_dim)


def test_attention_operators_at_zero_tokens(device, moe):
    heads, kvh, hd = 4, 2, 64
    x = torch.empty((0, H), device=device, dtype=torch.bfloat16)
    wq, wk, wv = _bf(2 * heads * hd, H, device=device, seed=1), _bf(kvh * hd, H, device=device, seed=2), \
        _bf(kvh * hd, H, device=device, seed=3)
    wo = _bf(H, heads * hd, device=device, seed=4)
    qn, kn, nw = _bf(hd, device=device, seed=5), _bf(hd, device=device, seed=6), _bf(H, device=device, seed=7)
    q, k, v = hip.hip_qwen36_batched_attention_project(x, nw, wq, wk, wv)
    _empty(q, (0, 2 * heads * hd), torch.float32)
    _empty(k, (0, kvh * hd), torch.float32)
    _empty(v, (0, kvh * hd), torch.float32)
    kc = torch.randn(8, kvh, hd, device=device)
    vc = torch.randn(8, kvh, hd, device=device)
    kw = dict(attention_heads=heads, kv_heads=kvh, head_dim=hd, rope_dim=32, start_position=5)
    upd, kc2, vc2 = hip.hip_qwen36_batched_attention_decode(x, kc, vc, nw, wq, wk, wv, wo, qn, kn, **kw)
    _empty(upd, (0, H), torch.float32)
    assert kc2.data_ptr() != kc.data_ptr() and torch.equal(kc2, kc) and torch.equal(vc2, vc)
    upd, kc3, vc3 = hip.hip_qwen36_batched_attention_decode(x, kc, vc, nw, wq, wk, wv, wo, qn, kn,
                                                            copy_cache=False, **kw)
    assert kc3.data_ptr() == kc.data_ptr() and vc3.data_ptr() == vc.data_ptr()
    res = hip.hip_qwen36_batched_attention_moe_layer_decode(
        x, kc, vc, nw, wq, wk, wv, wo, qn, kn, moe["norm"], moe["router"], moe["gu"], moe["dn"], moe["sgu"],
        moe["sdn"], moe["sg"], top_k=K, **kw)
    assert len(res) == 9
    for t, shape in zip(res[:4], [(0, H)] * 4):
        _empty(t, shape, torch.float32)
    assert torch.equal(res[4], kc) and torch.equal(res[5], vc)
    _empty(res[6], (0, E), torch.float32)
    _empty(res[7], (0, K), torch.int64)
    _empty(res[8], (0, K), torch.float32)
