"""GPU parity of the gated full-attention decode kernels against the CPU oracle.

Real Qwen3.6 attention shapes (hidden 2048, 16 query / 2 kv heads of 256,
rope_dim 64, theta 1e7), bf16 weights, caches in f32 (the reference test's
choice, tests/test_triton_moe.py:1028-1104) and bf16.  Outputs within the
bf16 tolerance of tests/parity.py; the new cache rows likewise, the other
rows bit-exact.  The Attention -> MoE layer runs a reduced MoE (32 experts,
I = 128) behind the real attention.
"""

from __future__ import annotations

import pytest
import torch

import oracle
from fastkernels_amd import _lib
from fastkernels_amd.kernels import hip
from tests.parity import assert_routing_parity, tol

pytestmark = pytest.mark.gpu

H, HEADS, KVH, HD, RD, THETA = 2048, 16, 2, 256, 64, 1.0e7
KW = dict(attention_heads=HEADS, kv_heads=KVH, head_dim=HD, rope_dim=RD, rope_theta=THETA)


@pytest.fixture(scope="module")
def attn_cpu():
    g = torch.Generator().manual_seed(21)
    r = lambda *s, sc=0.02: (torch.randn(*s, generator=g) * sc).to(torch.bfloat16)  # noqa: E731
    return dict(input_norm_weight=r(H, sc=0.5), q_proj_weight=r(2 * HEADS * HD, H), k_proj_weight=r(KVH * HD, H),
                v_proj_weight=r(KVH * HD, H), o_proj_weight=r(H, HEADS * HD), q_norm_weight=r(HD, sc=0.5),
                k_norm_weight=r(HD, sc=0.5))


@pytest.fixture(scope="module")
def attn_gpu(attn_cpu, device):
    return {k: v.to(device) for k, v in attn_cpu.items()}


def _args(w):
    return (w["input_norm_weight"], w["q_proj_weight"], w["k_proj_weight"], w["v_proj_weight"], w["o_proj_weight"],
            w["q_norm_weight"], w["k_norm_weight"])


def _inputs(tokens, start, cache_dtype, seed=3):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(tokens, H, generator=g)).to(torch.bfloat16)
    maxp = start + tokens + 3
    kc = (torch.randn(maxp, KVH, HD, generator=g) * 0.5).to(cache_dtype)
    vc = (torch.randn(maxp, KVH, HD, generator=g) * 0.5).to(cache_dtype)
    return x, kc, vc


def test_attention_project_matches_oracle(device, attn_cpu, attn_gpu):
    x = _inputs(2, 0, torch.float32)[0]
    q, k, v = hip.hip_qwen36_batched_attention_project(x.to(device), *[attn_gpu[n] for n in (
        "input_norm_weight", "q_proj_weight", "k_proj_weight", "v_proj_weight")])
    xn = oracle.rms_norm(x.float(), attn_cpu["input_norm_weight"])
    for got, w in ((q, "q_proj_weight"), (k, "k_proj_weight"), (v, "v_proj_weight")):
        torch.testing.assert_close(got.cpu(), xn @ attn_cpu[w].float().t(), **tol(torch.bfloat16))


@pytest.mark.parametrize("cache_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("tokens,start", [(1, 0), (2, 1), (5, 37), (1, 300)])
@pytest.mark.parametrize("interleaved", [True, False])
def test_attention_decode_matches_oracle(device, attn_cpu, attn_gpu, cache_dtype, tokens, start, interleaved):
    x, kc, vc = _inputs(tokens, start, cache_dtype)
    upd, nkc, nvc = hip.hip_qwen36_batched_attention_decode(
        x.to(device), kc.to(device), vc.to(device), *_args(attn_gpu), start_position=start,
        rope_interleaved=interleaved, **KW)
    o_upd, o_kc, o_vc = oracle.attention_update(
        x, kc, vc, *_args(attn_cpu), start_position=start, heads=HEADS, kv_heads=KVH, head_dim=HD, rope_dim=RD,
        rope_theta=THETA, interleaved=interleaved)
    torch.testing.assert_close(upd.cpu(), o_upd, **tol(torch.bfloat16))
    new = slice(start, start + tokens)
    torch.testing.assert_close(nkc[new].float().cpu(), o_kc[new].float(), **tol(torch.bfloat16))
    torch.testing.assert_close(nvc[new].float().cpu(), o_vc[new].float(), **tol(torch.bfloat16))
    for c, ref in ((nkc, kc), (nvc, vc)):
        assert torch.equal(c[:start].cpu(), ref[:start]) and torch.equal(c[start + tokens:].cpu(), ref[start + tokens:])


def test_attention_steps_chain_through_the_cache(device, attn_gpu):
    # three one-token calls on an in-place cache == one three-token call
    x, kc, vc = _inputs(3, 9, torch.float32, seed=8)
    kc, vc = kc.to(device), vc.to(device)
    one, k1, v1 = hip.hip_qwen36_batched_attention_decode(x.to(device), kc, vc, *_args(attn_gpu), start_position=9, **KW)
    k2, v2 = kc.clone(), vc.clone()
    ups = []
    for t in range(3):
        u, _, _ = hip.hip_qwen36_batched_attention_decode(
            x[t:t + 1].to(device), k2, v2, *_args(attn_gpu), start_position=9 + t, copy_cache=False, **KW)
        ups.append(u)
    torch.testing.assert_close(torch.cat(ups), one, atol=1e-5, rtol=1e-4)
    torch.testing.assert_close(k2, k1, atol=1e-6, rtol=1e-6)
    torch.testing.assert_close(v2, v1, atol=1e-6, rtol=1e-6)


@pytest.mark.parametrize("copy_cache", [True, False])
def test_attention_decode_more_than_32_rows(device, attn_cpu, attn_gpu, copy_cache):
    # 40 rows: two calls of the C ABI (32 + 8), the second reading the first
    # one's keys and values from the cache, against the oracle's single pass
    tokens, start = 40, 11
    x, kc, vc = _inputs(tokens, start, torch.bfloat16, seed=17)
    kd, vd = kc.to(device), vc.to(device)
    upd, nkc, nvc = hip.hip_qwen36_batched_attention_decode(
        x.to(device), kd, vd, *_args(attn_gpu), start_position=start, copy_cache=copy_cache, **KW)
    o_upd, o_kc, o_vc = oracle.attention_update(
        x, kc, vc, *_args(attn_cpu), start_position=start, heads=HEADS, kv_heads=KVH, head_dim=HD, rope_dim=RD,
        rope_theta=THETA, interleaved=True)
    torch.testing.assert_close(upd.cpu(), o_upd, **tol(torch.bfloat16))
    new = slice(start, start + tokens)
    torch.testing.assert_close(nkc[new].float().cpu(), o_kc[new].float(), **tol(torch.bfloat16))
    torch.testing.assert_close(nvc[new].float().cpu(), o_vc[new].float(), **tol(torch.bfloat16))
    assert (nkc is kd) == (not copy_cache)
    assert torch.equal(nkc[:start].cpu(), kc[:start]) and torch.equal(nvc[:start].cpu(), vc[:start])


def test_attention_moe_layer_matches_oracle(device, attn_cpu, attn_gpu):
    g = torch.Generator().manual_seed(12)
    r = lambda *s, sc=0.02: (torch.randn(*s, generator=g) * sc).to(torch.bfloat16)  # noqa: E731
    E, I, K = 32, 128, 8
    moe = dict(norm_weight=r(H, sc=0.1), router_weight=r(E, H), expert_gate_up_weight=r(E, 2 * I, H),
               expert_down_weight=r(E, H, I), shared_gate_up_weight=r(2 * I, H), shared_down_weight=r(H, I),
               shared_expert_gate_weight=r(H))
    moe_gpu = {k: v.to(device) for k, v in moe.items()}
    x, kc, vc = _inputs(2, 5, torch.float32, seed=13)
    got = hip.hip_qwen36_batched_attention_moe_layer_decode(
        x.to(device), kc.to(device), vc.to(device), *_args(attn_gpu), moe_gpu["norm_weight"],
        moe_gpu["router_weight"], moe_gpu["expert_gate_up_weight"], moe_gpu["expert_down_weight"],
        moe_gpu["shared_gate_up_weight"], moe_gpu["shared_down_weight"], moe_gpu["shared_expert_gate_weight"],
        start_position=5, top_k=K, **KW)
    want = oracle.attention_moe_layer(x, kc, vc, attn_cpu, moe, start_position=5, heads=HEADS, kv_heads=KVH,
                                      head_dim=HD, rope_dim=RD, rope_theta=THETA, top_k=K)
    layer_hidden, attn_hidden, attn_update, moe_update, nkc, nvc, logits, ids, weights = got
    for a, b in ((attn_update, want[2]), (attn_hidden, want[1]), (nkc, want[4]), (nvc, want[5])):
        torch.testing.assert_close(a.cpu(), b, **tol(torch.bfloat16))
    # the MoE half under the kernel's own routing of the kernel's attention output
    h = attn_hidden.cpu()
    ref = oracle.routed_experts(h, ids.cpu(), weights.cpu(), moe["expert_gate_up_weight"], moe["expert_down_weight"])
    ref = ref + oracle.shared_expert(h, moe["shared_gate_up_weight"], moe["shared_down_weight"],
                                     moe["shared_expert_gate_weight"])
    torch.testing.assert_close(moe_update.cpu(), ref, **tol(torch.bfloat16))
    torch.testing.assert_close(layer_hidden.cpu(), h + ref, **tol(torch.bfloat16))
    o_logits = oracle.router(h, moe["norm_weight"], moe["router_weight"], K)[0]
    if assert_routing_parity(logits, ids, weights, o_logits, K) == 0:
        assert torch.equal(ids.cpu(), want[7])


# The single-launch step (T <= 4 at these shapes) splits each token's
# positions over its attention units at run time and stages the cached rows
# in tiles of 40 per unit: long contexts take several tiles per unit, and a
# step's own positions fall in the last unit(s).
@pytest.mark.parametrize("cache_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("tokens,start", [(1, 1023), (4, 60), (3, 2000), (2, 1300)])
def test_attention_decode_long_contexts_match_oracle(device, attn_cpu, attn_gpu, cache_dtype, tokens, start):
    print(f"attention long context cache={cache_dtype} tokens={tokens} start={start}", flush=True)
    x, kc, vc = _inputs(tokens, start, cache_dtype, seed=17)
    upd, nkc, nvc = hip.hip_qwen36_batched_attention_decode(
        x.to(device), kc.to(device), vc.to(device), *_args(attn_gpu), start_position=start, **KW)
    o_upd, o_kc, o_vc = oracle.attention_update(
        x, kc, vc, *_args(attn_cpu), start_position=start, heads=HEADS, kv_heads=KVH, head_dim=HD, rope_dim=RD,
        rope_theta=THETA, interleaved=True)
    torch.testing.assert_close(upd.cpu(), o_upd, **tol(torch.bfloat16))
    new = slice(start, start + tokens)
    torch.testing.assert_close(nkc[new].float().cpu(), o_kc[new].float(), **tol(torch.bfloat16))
    torch.testing.assert_close(nvc[new].float().cpu(), o_vc[new].float(), **tol(torch.bfloat16))
    for c, ref in ((nkc, kc), (nvc, vc)):
        assert torch.equal(c[:start].cpu(), ref[:start]) and torch.equal(c[start + tokens:].cpu(), ref[start + tokens:])


def _plan(attn_gpu, tokens, max_positions, start, hidden_dtype=torch.bfloat16):
    from fastkernels_amd.plan import AttentionStepPlan
    from fastkernels_amd.spec import qwen36_35b_a3b_spec

    w = dict(attn_gpu)
    return AttentionStepPlan(w, tokens, qwen36_35b_a3b_spec(), max_positions=max_positions, start_position=start,
                             hidden_dtype=hidden_dtype)


@pytest.mark.parametrize("hidden_dtype", [torch.bfloat16, torch.float32])
def test_attention_plan_graph_replays_decode_successive_positions(device, attn_cpu, attn_gpu, hidden_dtype):
    # one captured step replayed three times == three eager steps (bit for
    # bit): the device-held position advances once per step, inside the
    # launch; the last step also matches the oracle run over the same cache
    print(f"attention plan graph replay hidden={hidden_dtype}", flush=True)
    tokens, start, maxp = 1, 37, 48
    g = torch.Generator().manual_seed(23)
    kc0 = torch.randn(maxp, KVH, HD, generator=g) * 0.5
    vc0 = torch.randn(maxp, KVH, HD, generator=g) * 0.5
    xs = [torch.randn(tokens, H, generator=g).to(hidden_dtype) for _ in range(3)]
    eager, graphed = _plan(attn_gpu, tokens, maxp, start, hidden_dtype), _plan(attn_gpu, tokens, maxp, start, hidden_dtype)
    for p in (eager, graphed):
        p.key_cache.copy_(kc0.to(device))
        p.value_cache.copy_(vc0.to(device))
    stream = torch.cuda.Stream(device)
    with torch.cuda.stream(stream):
        graphed.hidden.copy_(xs[0].to(device))
        graphed.run(stream)  # (warm: the first call sets the kernel's attributes)
        graphed.set_position(start)
        graphed.key_cache.copy_(kc0.to(device))
        graphed.value_cache.copy_(vc0.to(device))
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        graphed.run(stream)
    outs = []
    for s in range(3):
        eager.hidden.copy_(xs[s].to(device))
        eager.run()
        torch.cuda.synchronize()
        a = eager.hidden_out.clone()
        with torch.cuda.stream(stream):
            graphed.hidden.copy_(xs[s].to(device))
            graph.replay()
        stream.synchronize()
        assert torch.equal(a, graphed.hidden_out), f"step {s}"
        outs.append(a)
    assert int(graphed.position.item()) == start + 3 and int(eager.position.item()) == start + 3
    assert torch.equal(eager.key_cache, graphed.key_cache) and torch.equal(eager.value_cache, graphed.value_cache)
    # the oracle's third step over the cache the first two left
    kc, vc = kc0.clone(), vc0.clone()
    for s in range(3):
        o_upd, kc, vc = oracle.attention_update(
            xs[s], kc, vc, *_args(attn_cpu), start_position=start + s, heads=HEADS, kv_heads=KVH, head_dim=HD,
            rope_dim=RD, rope_theta=THETA, interleaved=True)
        torch.testing.assert_close(outs[s].cpu(), xs[s].float() + o_upd, **tol(torch.bfloat16))
    eager.check_device()
    graphed.check_device()


@pytest.mark.parametrize("tokens", [2, 5])
def test_attention_plan_position_past_the_cache_gives_nan(device, attn_gpu, tokens):
    # a device-held position whose step would pass the cache (T = 2: the
    # single launch, T = 5: the four launches): NaN update, caches untouched,
    # the position left where it is and the error word set (reported, then
    # cleared); a valid position afterwards decodes
    plan = _plan(attn_gpu, tokens, 8, 7)
    g = torch.Generator().manual_seed(29)
    plan.key_cache.copy_(torch.randn(8, KVH, HD, generator=g).to(device))
    plan.value_cache.copy_(torch.randn(8, KVH, HD, generator=g).to(device))
    plan.hidden.copy_(torch.randn(tokens, H, generator=g).to(torch.bfloat16).to(device))
    kc, vc = plan.key_cache.clone(), plan.value_cache.clone()
    plan.run()
    torch.cuda.synchronize()
    assert bool(torch.isnan(plan.update).all())
    assert torch.equal(plan.key_cache, kc) and torch.equal(plan.value_cache, vc)
    assert int(plan.position.item()) == 7
    with pytest.raises(_lib.FastKernelsError) as info:
        plan.check_device()
    assert info.value.status == _lib.FK_ERR_DEVICE
    assert "position" in str(info.value)
    plan.check_device()  # cleared
    plan.set_position(8 - tokens)
    plan.run()
    torch.cuda.synchronize()
    assert bool(torch.isfinite(plan.update).all())
    plan.check_device()
