"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py):
the oracle reproduces them on the CPU, and the HIP kernels match them on the GPU."""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import oracle
from tests.golden.make_golden import DN_KEYS, MOE_KEYS, SMALL, from_np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return dict(np.load(os.path.join(GOLDEN, name)))


def _moe_inputs(d):
    w = {k: from_np(d[f"in_{k}"], bf16=True) for k in MOE_KEYS}
    return from_np(d["in_hidden"], bf16=True), w


def _dn_inputs(d):
    w = {k: from_np(d[f"in_{k}"], bf16=(k != "recurrent_state")) for k in DN_KEYS}
    return from_np(d["in_hidden"], bf16=True), w


def test_oracle_reproduces_moe_fixture():
    d = _load("moe_small.npz")
    x, w = _moe_inputs(d)
    lh, moe, logits, ids, wts = oracle.moe_layer(x, *(w[k] for k in MOE_KEYS), top_k=SMALL.num_routed_experts)
    np.testing.assert_array_equal(ids.numpy(), d["out_ids"])
    np.testing.assert_allclose(logits.numpy(), d["out_logits"], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(wts.numpy(), d["out_weights"], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(moe.numpy(), d["out_moe_update"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(lh.numpy(), d["out_layer_hidden"], rtol=1e-5, atol=1e-6)


def test_oracle_reproduces_deltanet_fixture():
    d = _load("deltanet_small.npz")
    x, w = _dn_inputs(d)
    update, conv, state = oracle.deltanet_update(
        x, w["conv_state"], w["recurrent_state"], w,
        qk_heads=SMALL.deltanet_qk_heads, value_heads=SMALL.deltanet_value_heads, head_dim=SMALL.deltanet_head_dim,
    )
    np.testing.assert_allclose(update.numpy(), d["out_update"], rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(conv.view(torch.int16).numpy().view(np.uint16), d["out_conv_state"])
    np.testing.assert_allclose(state.numpy(), d["out_recurrent_state"], rtol=1e-5, atol=1e-6)


@pytest.mark.gpu
def test_hip_moe_layer_matches_fixture(device):
    from fastkernels_amd.kernels import hip

    d = _load("moe_small.npz")
    x, w = _moe_inputs(d)
    lh, moe, logits, ids, wts = hip.hip_qwen36_batched_moe_layer_decode(
        x.to(device), *(w[k].to(device) for k in MOE_KEYS), top_k=SMALL.num_routed_experts
    )
    np.testing.assert_array_equal(ids.cpu().numpy(), d["out_ids"])
    np.testing.assert_allclose(logits.cpu().numpy(), d["out_logits"], rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(moe.cpu().numpy(), d["out_moe_update"], rtol=2e-2, atol=2e-2)
    np.testing.assert_allclose(lh.cpu().numpy(), d["out_layer_hidden"], rtol=2e-2, atol=2e-2)


@pytest.mark.gpu
def test_hip_deltanet_matches_fixture(device):
    from fastkernels_amd.kernels import hip

    d = _load("deltanet_small.npz")
    x, w = _dn_inputs(d)
    wd = {k: v.to(device) for k, v in w.items()}
    mixed, z, a, b = hip.hip_qwen36_batched_deltanet_project(
        x.to(device), wd["input_norm_weight"], wd["in_proj_qkv_weight"], wd["in_proj_z_weight"],
        wd["in_proj_a_weight"], wd["in_proj_b_weight"],
    )
    mixed, conv = hip.hip_qwen36_batched_deltanet_conv(mixed, wd["conv_state"], wd["conv1d_weight"])
    update, state = hip.hip_qwen36_batched_deltanet_recurrent_output(
        mixed, z, a, b, wd["recurrent_state"], wd["out_proj_weight"], wd["linear_norm_weight"], wd["a_log"],
        wd["dt_bias"], qk_heads=SMALL.deltanet_qk_heads, value_heads=SMALL.deltanet_value_heads,
        head_dim=SMALL.deltanet_head_dim,
    )
    np.testing.assert_allclose(update.cpu().numpy(), d["out_update"], rtol=2e-2, atol=2e-2)
    np.testing.assert_allclose(state.cpu().numpy(), d["out_recurrent_state"], rtol=1e-3, atol=1e-3)
    ref_conv = from_np(d["out_conv_state"], bf16=True).float().numpy()
    np.testing.assert_allclose(conv.cpu().float().numpy(), ref_conv, rtol=1e-2, atol=1e-2)
