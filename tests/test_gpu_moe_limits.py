"""MoE parity at the reference operators' limits, against the CPU oracle.

The reference router accepts hidden sizes up to 4096 and up to 1024 experts
(kernels/triton/qwen36_router.py:224-225, 285-286) and its expert kernels
intermediate sizes up to 1024 (qwen36_expert.py:850-851); the HIP entry
points accept the same.  These shapes reach kernels the model's own shapes
never run:
  * the grid-barrier router (moe_router_kernel) for more than 256 experts,
    hidden sizes above 2048 or more than 256 tokens, with 64-bit top-k keys
    from 512 experts on;
  * the gate/up GEMV with eight 8-element chunks per lane (H > 2048);
  * the down GEMV with two chunks per lane (I > 512);
  * hidden sizes that are multiples of 8 but not of 16 (odd chunk counts),
    through the single-launch layer, the tagged router and the GEMV experts;
  * both work-item sizes of the MFMA down kernel with both K splits.
Weights are reduced in the other dimensions so the oracle stays quick.
"""

from __future__ import annotations

import pytest
import torch

import oracle
from fastkernels_amd import workloads as wl
from fastkernels_amd.kernels import hip
from tests.parity import assert_routing_parity, histogram, tol

pytestmark = pytest.mark.gpu

K = 8


def _weights(e, h, i, seed):
    g = torch.Generator().manual_seed(seed)

    def rnd(*s, sc=0.02):
        return (torch.randn(*s, generator=g) * sc).to(torch.bfloat16)

    # norm weight, router, gate/up, down, shared gate/up, shared down, shared gate
    return [rnd(h, sc=0.1), rnd(e, h), rnd(e, 2 * i, h), rnd(e, h, i), rnd(2 * i, h), rnd(h, i), rnd(h)]


def _check(device, e, h, i, tokens, seed):
    print(f"moe limits E={e} H={h} I={i} T={tokens}", flush=True)
    w = _weights(e, h, i, seed)
    x = wl.make_hidden(tokens, h, seed=seed + 1)
    wd = [t.to(device) for t in w]
    lh, moe, logits, ids, wt = hip.hip_qwen36_batched_moe_layer_decode(x.to(device), *wd, top_k=K)
    torch.cuda.synchronize()
    o_lh, o_moe, o_logits, o_ids, _ = oracle.moe_layer(x, *w, top_k=K)
    torch.testing.assert_close(logits.cpu(), o_logits, atol=1e-4, rtol=1e-4)
    near = assert_routing_parity(logits, ids, wt, o_logits, K)
    if near == 0:
        assert torch.equal(ids.cpu(), o_ids)
        torch.testing.assert_close(moe.cpu(), o_moe, **tol(torch.bfloat16))
    # experts under the kernel's own routing (always comparable)
    ref = oracle.routed_experts(x, ids.cpu(), wt.cpu(), w[2], w[3]) + oracle.shared_expert(x, w[4], w[5], w[6])
    torch.testing.assert_close(moe.cpu(), ref, **tol(torch.bfloat16))
    torch.testing.assert_close(lh.cpu(), x.float() + ref, **tol(torch.bfloat16))
    assert hip.hip_expert_histogram(ids, e).cpu().numpy().tolist() == histogram(ids, e).tolist()
    # the router entry point alone gives the same routing
    r_logits, r_ids, r_w = hip.hip_qwen36_batched_moe_router_decode(x.to(device), wd[0], wd[1], top_k=K)
    torch.testing.assert_close(r_logits, logits, atol=1e-6, rtol=1e-6)
    assert torch.equal(r_ids, ids)
    torch.testing.assert_close(r_w, wt, atol=1e-6, rtol=1e-6)
    hip.workspace_status(device)


@pytest.mark.parametrize(
    "e,h,i,tokens",
    [
        (512, 1024, 128, 4),    # > 256 experts: grid-barrier router, 64-bit keys
        (1024, 512, 64, 3),     # the expert limit
        (64, 3072, 128, 5),     # H > 2048: 8 chunks per lane in router and gate/up
        (16, 4096, 1024, 2),    # the hidden and intermediate limits together
        (64, 1024, 1024, 1),    # I > 512 at one token: tagged router, 2 chunks per lane in down
        (64, 256, 128, 600),    # 4800 (token, expert) pairs: two calls of the C ABI (512 + 88 tokens)
    ],
)
def test_moe_layer_at_operator_limits(device, e, h, i, tokens):
    _check(device, e, h, i, tokens, seed=100 + e + h + i + tokens)


@pytest.mark.parametrize("e,h,i,tokens", [(64, 512, 64, 257), (64, 512, 256, 512)])
def test_moe_layer_beyond_256_tokens(device, e, h, i, tokens):
    # grid-barrier router for T > 256; GEMV experts (I = 64) and MFMA experts
    # (I = 256) after it; T * K = 4096 is the routing-table limit
    _check(device, e, h, i, tokens, seed=200 + tokens + i)


@pytest.mark.parametrize(
    "e,h,i,tokens",
    [
        (256, 2048, 512, 192),  # the model's shapes past 4 pairs per expert: 64-row MFMA down items
        (256, 512, 256, 100),   # I = 256 at <= 4 pairs per expert: 32-row MFMA down items, 2 steps per wavefront
    ],
)
def test_moe_layer_mfma_down_item_sizes(device, e, h, i, tokens):
    # the MFMA down kernel takes 32 output rows per work item while
    # T * K <= 4 E and 64 above; config 2 (T = 128, E = 256) covers the
    # 32-row items at the model's I = 512
    _check(device, e, h, i, tokens, seed=400 + tokens + i)


@pytest.mark.parametrize("tokens", [1, 2, 16, 64])
def test_moe_layer_hidden_not_multiple_of_16(device, tokens):
    # H = 1032 = 8 * 129: an odd number of 8-element chunks per row through
    # the single-launch layer (T = 1), the tagged router and the GEMV experts
    _check(device, 64, 1032, 128, tokens, seed=300 + tokens)


@pytest.mark.parametrize("tokens", [1, 16])
def test_router_bias_bf16_and_misaligned(device, tokens):
    # a bf16 router bias, also as a view starting 2 bytes into its storage:
    # the tagged router loads the aligned word holding each element
    e, h = 256, 2048
    w = _weights(e, h, 64, seed=400 + tokens)
    x = wl.make_hidden(tokens, h, seed=401)
    bias16 = wl.zipf_router_bias(e, seed=0).to(torch.bfloat16)
    store = torch.zeros(e + 1, dtype=torch.bfloat16, device=device)
    store[1:] = bias16.to(device)
    for bd in (bias16.to(device), store[1:]):
        logits, ids, wt = hip.hip_qwen36_batched_moe_router_decode(x.to(device), w[0].to(device), w[1].to(device),
                                                                   top_k=K, router_bias=bd)
        o_logits, _, _ = oracle.router(x, w[0], w[1], K, router_bias=bias16)
        torch.testing.assert_close(logits.cpu(), o_logits, atol=1e-4, rtol=1e-4)
        assert_routing_parity(logits, ids, wt, o_logits, K)


def test_batched_routed_experts_over_4096_pairs(device):
    # the fixed-ids expert path in calls of at most 4096 pairs (512 + 88 tokens)
    e, h, i, tokens = 32, 256, 64, 600
    w = _weights(e, h, i, seed=77)
    x = wl.make_hidden(tokens, h, seed=78)
    g = torch.Generator().manual_seed(79)
    ids = torch.stack([torch.randperm(e, generator=g)[:K] for _ in range(tokens)])
    wt = torch.softmax(torch.randn(tokens, K, generator=g), -1)
    out = hip.hip_qwen36_batched_routed_shared_experts_decode(
        x.to(device), ids.to(device), wt.to(device), *[t.to(device) for t in w[2:7]])
    ref = oracle.routed_experts(x, ids, wt, w[2], w[3]) + oracle.shared_expert(x, w[4], w[5], w[6])
    torch.testing.assert_close(out.cpu(), ref, **tol(torch.bfloat16))
