"""Resident multi-layer decode runner (fastkernels_amd.runner) on the GPU.

A four-layer model in the Qwen3.6 pattern (three Gated DeltaNet layers, one
gated attention layer; real mixer shapes, a reduced MoE of 32 experts with
I = 128) decodes three steps.  Each step's output is checked against the
CPU oracle run layer by layer with the states, caches and positions carried
the same way; graph replays must reproduce eager steps bit for bit.
"""

from __future__ import annotations

import dataclasses

import pytest
import torch

import oracle
from fastkernels_amd import workloads as wl
from fastkernels_amd.runner import ResidentDecodeRunner
from fastkernels_amd.spec import qwen36_35b_a3b_spec
from tests.parity import tol

pytestmark = pytest.mark.gpu

SPEC = dataclasses.replace(qwen36_35b_a3b_spec(), num_layers=4, num_experts=32, expert_intermediate_size=128)
H, E, I, K = SPEC.hidden_size, SPEC.num_experts, SPEC.expert_intermediate_size, SPEC.num_routed_experts
HEADS, KVH, HD = SPEC.attention_heads, SPEC.attention_kv_heads, SPEC.attention_head_dim


def _moe(seed):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s, sc=0.02: (torch.randn(*s, generator=g) * sc).to(torch.bfloat16)  # noqa: E731
    return dict(norm_weight=r(H, sc=0.1), router_weight=r(E, H), expert_gate_up_weight=r(E, 2 * I, H),
                expert_down_weight=r(E, H, I), shared_gate_up_weight=r(2 * I, H), shared_down_weight=r(H, I),
                shared_expert_gate_weight=r(H))


def _attention(seed):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s, sc=0.02: (torch.randn(*s, generator=g) * sc).to(torch.bfloat16)  # noqa: E731
    return dict(input_norm_weight=r(H, sc=0.5), q_proj_weight=r(2 * HEADS * HD, H), k_proj_weight=r(KVH * HD, H),
                v_proj_weight=r(KVH * HD, H), o_proj_weight=r(H, HEADS * HD), q_norm_weight=r(HD, sc=0.5),
                k_norm_weight=r(HD, sc=0.5))


@pytest.fixture(scope="module")
def model():
    layers = []
    for i, kind in enumerate(SPEC.layer_kinds()):
        mixer = wl.make_deltanet_weights(SPEC, seed=300 + i) if kind == "deltanet_moe" else _attention(300 + i)
        layers.append((kind, mixer, _moe(400 + i)))
    return layers


def _on(device, layers):
    return [(k, {n: t.to(device) for n, t in m.items()}, {n: t.to(device) for n, t in w.items()}) for k, m, w in layers]


def test_runner_steps_match_oracle(device, model):
    tokens, steps, maxp = 2, 3, 16
    runner = ResidentDecodeRunner(_on(device, model), tokens, SPEC, max_positions=maxp)
    xs = [wl.make_hidden(tokens, H, seed=60 + s) for s in range(steps)]
    # oracle state
    st = {}
    for i, (kind, mixer, _) in enumerate(model):
        if kind == "deltanet_moe":
            st[i] = (mixer["conv_state"].clone(), mixer["recurrent_state"].clone())
        else:
            st[i] = (torch.zeros(maxp, KVH, HD), torch.zeros(maxp, KVH, HD))
    for s in range(steps):
        runner.hidden.copy_(xs[s].to(device))
        out = runner.step().cpu()
        h = xs[s]
        for i, (kind, mixer, moe) in enumerate(model):
            if kind == "deltanet_moe":
                dn = {k: v for k, v in mixer.items() if k not in ("conv_state", "recurrent_state")}
                res = oracle.deltanet_moe_layer(h, *st[i], dn, moe, qk_heads=SPEC.deltanet_qk_heads,
                                                value_heads=SPEC.deltanet_value_heads, head_dim=SPEC.deltanet_head_dim,
                                                top_k=K)
                st[i] = (res[4], res[5])
            else:
                res = oracle.attention_moe_layer(h, *st[i], mixer, moe, start_position=s * tokens, heads=HEADS,
                                                 kv_heads=KVH, head_dim=HD, rope_dim=SPEC.rope_dim,
                                                 rope_theta=SPEC.rope_theta, top_k=K)
                st[i] = (res[4], res[5])
            h = res[0]
            torch.testing.assert_close(runner.layer_outputs[i].cpu(), h, **tol(torch.bfloat16))
        torch.testing.assert_close(out, h, **tol(torch.bfloat16))
    kc, _ = runner.kv_cache(3)
    torch.testing.assert_close(kc[: steps * tokens].cpu(), st[3][0][: steps * tokens], **tol(torch.bfloat16))
    conv, rec = runner.deltanet_state(0)
    torch.testing.assert_close(rec.cpu(), st[0][1], **tol(torch.bfloat16))
    runner.check_device()


def test_runner_graph_replay_equals_eager(device, model):
    tokens = 1
    eager = ResidentDecodeRunner(_on(device, model), tokens, SPEC, max_positions=8)
    graphed = ResidentDecodeRunner(_on(device, model), tokens, SPEC, max_positions=8)
    graphed.capture()
    for s in range(4):  # both parities, twice
        x = wl.make_hidden(tokens, H, seed=90 + s).to(device)
        eager.hidden.copy_(x)
        graphed.hidden.copy_(x)
        a = eager.step().clone()
        b = graphed.replay().clone()
        torch.cuda.synchronize()
        assert torch.equal(a, b), f"step {s}"
    assert torch.equal(eager.kv_cache(3)[0], graphed.kv_cache(3)[0])
    assert torch.equal(eager.deltanet_state(1)[1], graphed.deltanet_state(1)[1])
    eager.check_device()
    graphed.check_device()


def test_runner_state_transfers_between_runners(device, model):
    # two steps on runner A, its state loaded into a fresh runner B: the
    # third step must agree bit for bit
    tokens = 1
    a = ResidentDecodeRunner(_on(device, model), tokens, SPEC, max_positions=8)
    b = ResidentDecodeRunner(_on(device, model), tokens, SPEC, max_positions=8)
    for s in range(2):
        a.hidden.copy_(wl.make_hidden(tokens, H, seed=120 + s).to(device))
        a.step()
    st = a.state()
    assert st.position == 2 and len(st.deltanet_recurrent_states) == 3 and len(st.attention_key_cache) == 1
    b.load_state(st)
    x = wl.make_hidden(tokens, H, seed=130).to(device)
    a.hidden.copy_(x)
    b.hidden.copy_(x)
    ya, yb = a.step().clone(), b.step().clone()
    assert torch.equal(ya, yb)
