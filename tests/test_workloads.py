"""Synthetic workload generators: seeds, shapes and the config-2 Zipf calibration."""

from __future__ import annotations

import dataclasses

import torch

import oracle
from fastkernels_amd import workloads as wl
from fastkernels_amd.spec import qwen36_35b_a3b_spec

SPEC = qwen36_35b_a3b_spec()


def test_router_weight_is_the_first_draw_of_the_layer_weights():
    small = dataclasses.replace(SPEC, num_experts=8, expert_intermediate_size=16, hidden_size=64)
    full = wl.make_moe_weights(small, seed=3)
    assert torch.equal(wl.make_router_weight(small, seed=3), full["router_weight"])


def test_zipf_bias_is_a_scaled_log_zipf_permutation():
    bias = wl.zipf_router_bias(SPEC.num_experts, seed=0).double()
    p = torch.exp(bias / wl.ZIPF_ALPHA)
    torch.testing.assert_close(p.sum(), torch.tensor(1.0, dtype=torch.float64), rtol=1e-5, atol=0)
    ranks = torch.arange(1, SPEC.num_experts + 1, dtype=torch.float64)
    expected = ranks.pow(-wl.ZIPF_S) / ranks.pow(-wl.ZIPF_S).sum()
    torch.testing.assert_close(torch.sort(p, descending=True).values, expected, rtol=1e-5, atol=0)


def test_zipf_calibration_puts_the_hottest_expert_in_20_to_60_tokens():
    # config 2: "hot experts receive 20-60 tokens" at T = 128, for every
    # weight set bench.py times (router seeds 0..7, hidden seeds 1..8)
    H, E = SPEC.hidden_size, SPEC.num_experts
    bias = wl.zipf_router_bias(E, seed=0)
    nw = torch.zeros(H, dtype=torch.bfloat16)
    for r in range(8):
        x = wl.make_hidden(128, H, seed=1 + r)
        _, ids, _ = oracle.router(x, nw, wl.make_router_weight(SPEC, seed=r), 8, router_bias=bias)
        hottest = int(torch.bincount(ids.reshape(-1), minlength=E).max())
        assert 20 <= hottest <= 60, (r, hottest)
