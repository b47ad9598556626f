"""GPU parity of the MoE decode layer kernels against the CPU oracle.

All inputs are generated on the CPU (seeded) and copied to the device, so the
oracle and the kernels see identical bytes.  Routing ids / histograms /
permutations are compared bit-exactly; fp32 outputs within the tolerance of
tests/parity.py.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from fastkernels_amd import workloads as wl
from fastkernels_amd.kernels import hip
from fastkernels_amd.spec import qwen36_35b_a3b_spec
from tests.parity import assert_routing_parity, histogram, tol

pytestmark = pytest.mark.gpu

SPEC = qwen36_35b_a3b_spec()
H, E, I, K = SPEC.hidden_size, SPEC.num_experts, SPEC.expert_intermediate_size, SPEC.num_routed_experts
FIXED_IDS = [3, 17, 42, 89, 127, 199, 231, 255]  # reference tests/test_triton_moe.py:192


@pytest.fixture(scope="module")
def real_cpu():
    return wl.make_moe_weights(SPEC, seed=0)


@pytest.fixture(scope="module")
def real_gpu(real_cpu, device):
    return {k: (None if v is None else v.to(device)) for k, v in real_cpu.items()}


def _moe_args(w):
    return (w["norm_weight"], w["router_weight"], w["expert_gate_up_weight"], w["expert_down_weight"],
            w["shared_gate_up_weight"], w["shared_down_weight"], w["shared_expert_gate_weight"])


# ---------------------------------------------------------------------------
# Small building blocks
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fused_swiglu(device, dtype):
    g = torch.Generator().manual_seed(0)
    gu = torch.randn(128, 1024, generator=g).to(dtype)
    out = hip.hip_fused_swiglu(gu.to(device))
    assert out.dtype == dtype
    torch.testing.assert_close(out.cpu().float(), oracle.swiglu(gu.float()), **({"atol": 3e-2, "rtol": 3e-2} if dtype == torch.bfloat16 else {"atol": 1e-5, "rtol": 1e-5}))


@pytest.mark.parametrize("idt", [torch.int32, torch.int64])
def test_expert_histogram_bit_exact(device, idt):
    g = torch.Generator().manual_seed(0)
    ids = torch.randint(0, 256, (64, 8), generator=g).to(idt)
    counts = hip.hip_expert_histogram(ids.to(device), 256)
    assert counts.dtype == torch.int32
    assert counts.cpu().numpy().tolist() == oracle.expert_histogram(ids.numpy(), 256).tolist()


@pytest.mark.parametrize(
    "tokens,top_k,experts", [(1, 8, 256), (16, 8, 256), (37, 8, 256), (128, 8, 256), (256, 8, 256), (7, 3, 5), (512, 8, 1024)]
)
def test_align_tables_bit_exact(device, tokens, top_k, experts):
    rng = np.random.default_rng(tokens * 7 + experts)
    ids = np.stack([rng.choice(experts, size=top_k, replace=False) for _ in range(tokens)])
    counts, offsets, perm, inverse = hip.hip_qwen36_moe_align(torch.from_numpy(ids).to(device), experts)
    rc, ro, rp, ri = oracle.moe_align(ids, experts)
    assert counts.cpu().numpy().tolist() == rc.tolist()
    assert offsets.cpu().numpy().tolist() == ro.tolist()
    assert perm.cpu().numpy().tolist() == rp.tolist()
    assert inverse.cpu().numpy().tolist() == ri.tolist()


# ---------------------------------------------------------------------------
# Router
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_router_real_shape(device, dtype):
    g = torch.Generator().manual_seed(1)
    x = torch.randn(H, generator=g).to(dtype)
    nw = (0.02 * torch.randn(H, generator=g)).to(dtype)
    rw = (0.02 * torch.randn(E, H, generator=g)).to(dtype)
    logits, ids, w = hip.hip_qwen36_moe_router_decode(x.to(device), nw.to(device), rw.to(device), top_k=K)
    assert logits.shape == (E,) and ids.shape == (K,) and ids.dtype == torch.int64 and w.dtype == torch.float32
    o_logits, o_ids, o_w = oracle.router(x, nw, rw, K)
    torch.testing.assert_close(logits.cpu(), o_logits[0], atol=1e-4, rtol=1e-4)
    assert_routing_parity(logits, ids, w, o_logits, K)
    torch.testing.assert_close(w.cpu(), o_w[0], atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("tokens", [1, 2, 4, 5, 8, 9, 12, 16, 17, 37, 128, 256])
def test_batched_router_and_tables(device, tokens):
    g = torch.Generator().manual_seed(2 + tokens)
    x = (0.02 * torch.randn(tokens, H, generator=g)).bfloat16()
    nw = (0.02 * torch.randn(H, generator=g)).bfloat16()
    rw = (0.02 * torch.randn(E, H, generator=g)).bfloat16()
    logits, ids, w = hip.hip_qwen36_batched_moe_router_decode(x.to(device), nw.to(device), rw.to(device), top_k=K)
    o_logits, _, _ = oracle.router(x, nw, rw, K)
    torch.testing.assert_close(logits.cpu(), o_logits, atol=1e-4, rtol=1e-4)
    near = assert_routing_parity(logits, ids, w, o_logits, K)
    assert near <= max(1, tokens // 16)
    counts = hip.hip_expert_histogram(ids, E)
    assert counts.cpu().numpy().tolist() == histogram(ids, E).tolist()


def test_router_exact_ties_go_to_lower_id(device):
    # identical router rows produce identical logits: the lower id must win
    g = torch.Generator().manual_seed(3)
    x = torch.randn(64, generator=g)
    rw = 0.05 * torch.randn(16, 64, generator=g)
    nw = torch.zeros(64)
    n = oracle.rms_norm(x, nw)
    sign = 1.0 if float(n @ rw[4]) > 0 else -1.0
    rw[4] = 4.0 * sign * rw[4]  # strong positive logit, shared by 4, 9 and 13
    rw[9] = rw[4]
    rw[13] = rw[4]
    logits, ids, w = hip.hip_qwen36_moe_router_decode(x.to(device), nw.to(device), rw.to(device), top_k=4)
    assert logits[4].item() == logits[9].item() == logits[13].item()
    o_logits, o_ids, _ = oracle.router(x, nw, rw, 4)
    assert ids.tolist()[:3] == [4, 9, 13]
    assert o_ids[0].tolist()[:3] == [4, 9, 13]
    assert_routing_parity(logits, ids, w, o_logits, 4)


@pytest.mark.parametrize("tokens,hidden", [(2, 64), (5, 64), (9, 64), (12, 64), (16, 64), (17, 64), (24, 64),
                                           (40, 256), (70, 512)])
def test_batched_router_exact_ties_go_to_lower_id(device, tokens, hidden):
    # Per token, three identical router rows give identical logits at the top
    # (the lower id first) whichever path selects: workgroup 0 for every token
    # up to 8 tokens, one workgroup per token from 9 on; from 36 tokens at a
    # hidden size that is a multiple of 256 the logits come from MFMA tiles
    # (rows 5 and 11 in one tile, 17 in the next).
    g = torch.Generator().manual_seed(30 + tokens)
    x = torch.randn(hidden, generator=g) + 0.3 * torch.randn(tokens, hidden, generator=g)  # tokens near one direction
    nw = torch.zeros(hidden)
    rw = 0.05 * torch.randn(32, hidden, generator=g)
    n = oracle.rms_norm(x, nw)
    # a row along the tokens' mean direction: the largest logit of every token
    d = n.mean(0)
    rw[5] = 4.0 * d / d.norm()
    rw[11] = rw[5]
    rw[17] = rw[5]
    # (a bf16 router weight at the MFMA shapes: the path takes bf16 rows)
    rw_dev = rw.bfloat16() if hidden % 256 == 0 else rw
    rw = rw_dev.float()
    assert bool(((n @ rw[5]) > 0.5).all())
    logits, ids, w = hip.hip_qwen36_batched_moe_router_decode(x.to(device), nw.to(device), rw_dev.to(device), top_k=4)
    o_logits, o_ids, _ = oracle.router(x, nw, rw, 4)
    for t in range(tokens):
        assert logits[t, 5].item() == logits[t, 11].item() == logits[t, 17].item()
        assert ids[t].tolist()[:3] == [5, 11, 17]
        # (the oracle's batched matmul need not round the three identical rows
        # alike, so only its set is compared; the tie rule itself is checked
        # on the kernel's own, exactly tied logits by assert_routing_parity)
        assert set(o_ids[t].tolist()[:3]) == {5, 11, 17}
    assert_routing_parity(logits, ids, w, o_logits, 4)


def test_router_bias_extension(device):
    g = torch.Generator().manual_seed(4)
    x = torch.randn(3, H, generator=g).bfloat16()
    nw = torch.zeros(H).bfloat16()
    rw = (0.02 * torch.randn(E, H, generator=g)).bfloat16()
    bias = wl.zipf_router_bias(E, seed=0)
    logits, ids, w = hip.hip_qwen36_batched_moe_router_decode(
        x.to(device), nw.to(device), rw.to(device), top_k=K, router_bias=bias.to(device)
    )
    o_logits, _, _ = oracle.router(x, nw, rw, K, router_bias=bias)
    torch.testing.assert_close(logits.cpu(), o_logits, atol=1e-4, rtol=1e-4)
    assert_routing_parity(logits, ids, w, o_logits, K)


# ---------------------------------------------------------------------------
# Expert stage with fixed routing (isolates experts from routing)
# ---------------------------------------------------------------------------
def test_single_expert_mlp(device, real_cpu):
    x = wl.make_hidden(1, H, seed=5)[0]
    gu = real_cpu["expert_gate_up_weight"][7]
    dn = real_cpu["expert_down_weight"][7]
    out = hip.hip_qwen36_single_expert_mlp_decode(x.to(device), gu.to(device), dn.to(device))
    torch.testing.assert_close(out.cpu(), oracle.expert_mlp(x, gu, dn), **tol(torch.bfloat16))


def test_expert_stage_after_other_tables_on_one_workspace(device, real_cpu):
    # The stream's workspace keeps what earlier calls of other shapes left:
    # tables of a large alignment, small integers, where a small expert
    # stage's tagged down outputs lie.  Its combine must not take them for
    # this launch's outputs.
    rng = np.random.default_rng(11)
    ids = np.stack([rng.choice(1024, size=8, replace=False) for _ in range(512)])
    hip.hip_qwen36_moe_align(torch.from_numpy(ids).to(device), 1024)
    x = wl.make_hidden(1, H, seed=5)[0]
    for e in (7, 8, 7):
        gu = real_cpu["expert_gate_up_weight"][e]
        dn = real_cpu["expert_down_weight"][e]
        out = hip.hip_qwen36_single_expert_mlp_decode(x.to(device), gu.to(device), dn.to(device))
        torch.testing.assert_close(out.cpu(), oracle.expert_mlp(x, gu, dn), **tol(torch.bfloat16))


def test_routed_shared_fixed_ids(device, real_cpu, real_gpu):
    x = wl.make_hidden(1, H, seed=6)[0]
    ids = torch.tensor(FIXED_IDS, dtype=torch.int64)
    w = torch.softmax(torch.linspace(1.0, 0.0, 8), 0)
    out = hip.hip_qwen36_routed_shared_experts_decode(
        x.to(device), ids.to(device), w.to(device), real_gpu["expert_gate_up_weight"], real_gpu["expert_down_weight"],
        real_gpu["shared_gate_up_weight"], real_gpu["shared_down_weight"], real_gpu["shared_expert_gate_weight"],
    )
    ref = oracle.routed_experts(x, ids, w, real_cpu["expert_gate_up_weight"], real_cpu["expert_down_weight"])[0]
    ref = ref + oracle.shared_expert(x, real_cpu["shared_gate_up_weight"], real_cpu["shared_down_weight"],
                                     real_cpu["shared_expert_gate_weight"])[0]
    torch.testing.assert_close(out.cpu(), ref, **tol(torch.bfloat16))
    routed = hip.hip_qwen36_routed_experts_decode(
        x.to(device), ids.to(device), w.to(device), real_gpu["expert_gate_up_weight"], real_gpu["expert_down_weight"]
    )
    ref_r = oracle.routed_experts(x, ids, w, real_cpu["expert_gate_up_weight"], real_cpu["expert_down_weight"])[0]
    torch.testing.assert_close(routed.cpu(), ref_r, **tol(torch.bfloat16))


@pytest.mark.parametrize("tokens", [2, 4, 16])
def test_batched_routed_shared_fixed_ids(device, real_cpu, real_gpu, tokens):
    x = wl.make_hidden(tokens, H, seed=7 + tokens)
    ids = torch.stack([(torch.tensor(FIXED_IDS) + 13 * t) % E for t in range(tokens)])
    w = torch.softmax(torch.randn(tokens, 8, generator=torch.Generator().manual_seed(tokens)), -1)
    out = hip.hip_qwen36_batched_routed_shared_experts_decode(
        x.to(device), ids.to(device), w.to(device), real_gpu["expert_gate_up_weight"], real_gpu["expert_down_weight"],
        real_gpu["shared_gate_up_weight"], real_gpu["shared_down_weight"], real_gpu["shared_expert_gate_weight"],
    )
    ref = oracle.routed_experts(x, ids, w, real_cpu["expert_gate_up_weight"], real_cpu["expert_down_weight"])
    ref = ref + oracle.shared_expert(x, real_cpu["shared_gate_up_weight"], real_cpu["shared_down_weight"],
                                     real_cpu["shared_expert_gate_weight"])
    torch.testing.assert_close(out.cpu(), ref, **tol(torch.bfloat16))
    routed = hip.hip_qwen36_batched_routed_experts_decode(
        x.to(device), ids.to(device), w.to(device), real_gpu["expert_gate_up_weight"], real_gpu["expert_down_weight"]
    )
    ref_r = oracle.routed_experts(x, ids, w, real_cpu["expert_gate_up_weight"], real_cpu["expert_down_weight"])
    torch.testing.assert_close(routed.cpu(), ref_r, **tol(torch.bfloat16))


def test_small_shape_fp32_weights(device):
    # the reference also exercises fp32 weights (tests/test_triton_moe.py:141)
    g = torch.Generator().manual_seed(8)
    T, Hs, Es, Is, Ks = 3, 64, 16, 32, 4
    x = torch.randn(T, Hs, generator=g)
    w = {
        "norm_weight": 0.1 * torch.randn(Hs, generator=g), "router_weight": 0.1 * torch.randn(Es, Hs, generator=g),
        "expert_gate_up_weight": 0.1 * torch.randn(Es, 2 * Is, Hs, generator=g),
        "expert_down_weight": 0.1 * torch.randn(Es, Hs, Is, generator=g),
        "shared_gate_up_weight": 0.1 * torch.randn(2 * Is, Hs, generator=g),
        "shared_down_weight": 0.1 * torch.randn(Hs, Is, generator=g),
        "shared_expert_gate_weight": 0.1 * torch.randn(Hs, generator=g),
    }
    wd = {k: v.to(device) for k, v in w.items()}
    out, logits, ids, wts = hip.hip_qwen36_batched_moe_decode(x.to(device), *_moe_args(wd), top_k=Ks)
    o_out, o_logits, o_ids, o_w = oracle.moe_update(x, *_moe_args(w), top_k=Ks)
    assert_routing_parity(logits, ids, wts, o_logits, Ks)
    # compare expert outputs under the kernel's routing
    ref = oracle.routed_experts(x, ids.cpu(), wts.cpu(), w["expert_gate_up_weight"], w["expert_down_weight"])
    ref = ref + oracle.shared_expert(x, w["shared_gate_up_weight"], w["shared_down_weight"], w["shared_expert_gate_weight"])
    torch.testing.assert_close(out.cpu(), ref, **tol(torch.float32))


# ---------------------------------------------------------------------------
# Full MoE layer at the BASELINE configs
# ---------------------------------------------------------------------------
def _check_full(device, real_cpu, real_gpu, tokens, bias=None, seed=1):
    x = wl.make_hidden(tokens, H, seed=seed)
    layer_hidden, moe, logits, ids, w = hip.hip_qwen36_batched_moe_layer_decode(
        x.to(device), *_moe_args(real_gpu), top_k=K, router_bias=None if bias is None else bias.to(device)
    )
    o_lh, o_moe, o_logits, o_ids, o_w = oracle.moe_layer(x, *_moe_args(real_cpu), top_k=K, router_bias=bias)
    torch.testing.assert_close(logits.cpu(), o_logits, atol=1e-4, rtol=1e-4)
    near = assert_routing_parity(logits, ids, w, o_logits, K)
    if near == 0:
        assert torch.equal(ids.cpu(), o_ids)
        torch.testing.assert_close(moe.cpu(), o_moe, **tol(torch.bfloat16))
        torch.testing.assert_close(layer_hidden.cpu(), o_lh, **tol(torch.bfloat16))
    # experts under the kernel's own routing (always comparable)
    ref = oracle.routed_experts(x, ids.cpu(), w.cpu(), real_cpu["expert_gate_up_weight"], real_cpu["expert_down_weight"])
    ref = ref + oracle.shared_expert(x, real_cpu["shared_gate_up_weight"], real_cpu["shared_down_weight"],
                                     real_cpu["shared_expert_gate_weight"])
    torch.testing.assert_close(moe.cpu(), ref, **tol(torch.bfloat16))
    torch.testing.assert_close(layer_hidden.cpu(), x.float() + ref, **tol(torch.bfloat16))
    counts = hip.hip_expert_histogram(ids, E).cpu().numpy()
    assert counts.tolist() == histogram(ids, E).tolist()
    return ids, counts


def test_moe_decode_t1_config0(device, real_cpu, real_gpu):
    x = wl.make_hidden(1, H, seed=1)[0]
    out, logits, ids, w = hip.hip_qwen36_moe_decode(x.to(device), *_moe_args(real_gpu), top_k=K)
    assert out.shape == (H,) and logits.shape == (E,) and ids.shape == (K,)
    o_out, o_logits, o_ids, o_w = oracle.moe_update(x, *_moe_args(real_cpu), top_k=K)
    assert_routing_parity(logits, ids, w, o_logits, K)
    torch.testing.assert_close(out.cpu(), o_out[0], **tol(torch.bfloat16))
    _check_full(device, real_cpu, real_gpu, 1)


def test_moe_layer_t16_config1(device, real_cpu, real_gpu):
    _check_full(device, real_cpu, real_gpu, 16)


def test_moe_layer_t128_zipf_config2(device, real_cpu, real_gpu):
    bias = wl.zipf_router_bias(E, seed=0)
    ids, counts = _check_full(device, real_cpu, real_gpu, 128, bias=bias)
    assert 20 <= counts.max() <= 60


def test_moe_layer_deterministic(device, real_gpu):
    x = wl.make_hidden(16, H, seed=3).to(device)
    a = hip.hip_qwen36_batched_moe_layer_decode(x, *_moe_args(real_gpu), top_k=K)
    b = hip.hip_qwen36_batched_moe_layer_decode(x, *_moe_args(real_gpu), top_k=K)
    for u, v in zip(a, b):
        assert torch.equal(u, v)


@pytest.mark.parametrize("tokens", [1, 2, 8, 64])
def test_moe_layer_fp32_hidden(device, real_cpu, real_gpu, tokens):
    # the real-weight runner feeds fp32 hidden (bench/qwen36_full_decode.py:152),
    # and a layer stack feeds each layer the previous layer's fp32 output:
    # single-launch (T = 1) and GEMV (T = 8, and T = 64: the MFMA experts take
    # bf16 hidden states only) expert paths
    x = wl.make_hidden(tokens, H, seed=9, dtype=torch.float32)
    lh, moe, logits, ids, w = hip.hip_qwen36_batched_moe_layer_decode(x.to(device), *_moe_args(real_gpu), top_k=K)
    ref = oracle.routed_experts(x, ids.cpu(), w.cpu(), real_cpu["expert_gate_up_weight"], real_cpu["expert_down_weight"])
    ref = ref + oracle.shared_expert(x, real_cpu["shared_gate_up_weight"], real_cpu["shared_down_weight"],
                                     real_cpu["shared_expert_gate_weight"])
    torch.testing.assert_close(moe.cpu(), ref, **tol(torch.bfloat16))
    torch.testing.assert_close(lh.cpu(), x + ref, **tol(torch.bfloat16))


@pytest.mark.parametrize("tokens", [1, 2, 3, 4, 16])
def test_fused_layer_matches_multi_launch(device, real_gpu, tokens):
    # fk_moe_layer takes the single-launch kernel for T <= 4; router +
    # experts take the multi-launch path.  The router arithmetic is the same
    # (ids equal, logits and weights to rounding); the expert sums are taken
    # in a different order (weights folded in before the lane reduction).
    from fastkernels_amd.plan import MoeLayerPlan

    plan = MoeLayerPlan(real_gpu, tokens)
    plan.hidden.copy_(wl.make_hidden(tokens, H, seed=70 + tokens).to(device))
    plan.run()
    fused = [t.clone() for t in (plan.layer_out, plan.moe_out, plan.logits, plan.ids, plan.weights)]
    plan.run_router()
    plan.run_experts()
    multi = (plan.layer_out, plan.moe_out, plan.logits, plan.ids, plan.weights)
    plan.check_device()  # no bounded wait ran out (synchronises)
    assert torch.equal(fused[3], multi[3])
    for a, b in zip(fused[2:], multi[2:]):
        torch.testing.assert_close(a, b, atol=1e-6, rtol=1e-6)
    for a, b in zip(fused[:2], multi[:2]):
        torch.testing.assert_close(a, b, atol=1e-5, rtol=1e-5)


def test_layer_sizes_interleaved_on_one_workspace(device, real_gpu):
    # Single-launch (T <= 4) and multi-launch (T > 4) layers, and the
    # fixed-ids expert path, share the stream's workspace: each call must
    # match a call on a fresh plan whatever ran before it.
    from fastkernels_amd.plan import MoeLayerPlan

    w = real_gpu
    args = (w["norm_weight"], w["router_weight"], w["expert_gate_up_weight"], w["expert_down_weight"],
            w["shared_gate_up_weight"], w["shared_down_weight"], w["shared_expert_gate_weight"])
    sizes = [4, 1, 8, 1, 3, 16, 2, 1]
    xs = {t: wl.make_hidden(t, H, seed=90 + t).to(device) for t in set(sizes)}
    want = {}
    for t in set(sizes):
        plan = MoeLayerPlan(w, t)
        plan.hidden.copy_(xs[t])
        plan.run()
        torch.cuda.synchronize()
        want[t] = (plan.layer_out.clone(), plan.ids.clone())
    for t in sizes:
        lh, moe, logits, ids, wts = hip.hip_qwen36_batched_moe_layer_decode(xs[t], *args, top_k=K)
        assert torch.equal(ids, want[t][1])
        torch.testing.assert_close(lh, want[t][0], atol=1e-6, rtol=1e-6)
        # fixed-ids expert stage on the same workspace after a fused call
        r = hip.hip_qwen36_batched_routed_shared_experts_decode(
            xs[t], ids, wts, w["expert_gate_up_weight"], w["expert_down_weight"], w["shared_gate_up_weight"],
            w["shared_down_weight"], w["shared_expert_gate_weight"])
        torch.testing.assert_close(r, moe, atol=1e-5, rtol=1e-5)


def test_fused_layer_repeated_calls_stay_consistent(device, real_gpu):
    # The launch tag advances every launch: many back-to-back launches
    # (rotating inputs) must keep giving the first call's answer.
    from fastkernels_amd.plan import MoeLayerPlan

    plan = MoeLayerPlan(real_gpu, 1)
    xs = [wl.make_hidden(1, H, seed=80 + i).to(device) for i in range(3)]
    ref = []
    for x in xs:
        plan.hidden.copy_(x)
        plan.run()
        ref.append(plan.layer_out.clone())
    for _ in range(5):
        for x, r in zip(xs, ref):
            plan.hidden.copy_(x)
            plan.run()
            assert torch.equal(plan.layer_out, r)
    plan.check_device()


@pytest.mark.parametrize("shape", [(32, 512, 128), (256, 2048, 128), (64, 2048, 256), (32, 2048, 512)])
@pytest.mark.parametrize("tokens", [1, 2, 5])
def test_moe_layer_reduced_shapes(device, shape, tokens):
    # Smaller expert counts and intermediate sizes through every small-T
    # path (single launch at T = 1, router + GEMV experts at T = 2 and 5).
    # I < 512 leaves lanes of the single-launch kernel's down rows idle,
    # which must not change its lane reductions.
    e, h, i = shape
    g = torch.Generator().manual_seed(5)

    def rnd(*s, sc=0.02):
        return (torch.randn(*s, generator=g) * sc).to(torch.bfloat16)

    w = [rnd(h, sc=0.1), rnd(e, h), rnd(e, 2 * i, h), rnd(e, h, i), rnd(2 * i, h), rnd(h, i), rnd(1, h)]
    x = wl.make_hidden(tokens, h, seed=11)
    lh, moe, logits, ids, wt = hip.hip_qwen36_batched_moe_layer_decode(x.to(device), *[t.to(device) for t in w], top_k=K)
    ref = oracle.routed_experts(x, ids.cpu(), wt.cpu(), w[2], w[3]) + oracle.shared_expert(x, w[4], w[5], w[6])
    torch.testing.assert_close(moe.cpu(), ref, **tol(torch.bfloat16))
    torch.testing.assert_close(lh.cpu(), x.float() + ref, **tol(torch.bfloat16))
    o_logits = oracle.moe_layer(x, *w, top_k=K)[2]
    if assert_routing_parity(logits, ids, wt, o_logits, K) == 0:
        assert torch.equal(ids.cpu(), oracle.moe_layer(x, *w, top_k=K)[3])
