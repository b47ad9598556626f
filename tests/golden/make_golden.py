"""Write the small golden fixtures under tests/golden/ from the CPU oracle.

The reference ships no golden vectors (its GPU tests are differential against
inline torch), so these fixtures are regression vectors of our own oracle,
which tests/test_oracle.py pins against closed forms, library routines and
brute force.  Inputs are seeded and stored exactly (bf16 weights as their
uint16 bit patterns); outputs are fp32.

Usage: python tests/golden/make_golden.py
"""

from __future__ import annotations

import dataclasses
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402
from fastkernels_amd import workloads as wl  # noqa: E402
from fastkernels_amd.spec import qwen36_35b_a3b_spec  # noqa: E402

SMALL = dataclasses.replace(
    qwen36_35b_a3b_spec(), hidden_size=64, num_experts=16, num_routed_experts=4, expert_intermediate_size=32,
    deltanet_qk_heads=2, deltanet_value_heads=4, deltanet_head_dim=8,
)
MOE_KEYS = ("norm_weight", "router_weight", "expert_gate_up_weight", "expert_down_weight",
            "shared_gate_up_weight", "shared_down_weight", "shared_expert_gate_weight")


def to_np(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def from_np(a: np.ndarray, bf16: bool) -> torch.Tensor:
    if bf16:
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
    return torch.from_numpy(a.copy())


def make_moe(tokens: int = 3, seed: int = 7):
    w = wl.make_moe_weights(SMALL, seed=seed)
    w["norm_weight"] = (0.1 * torch.randn(SMALL.hidden_size, generator=torch.Generator().manual_seed(seed + 1))).bfloat16()
    x = wl.make_hidden(tokens, SMALL.hidden_size, seed=seed + 2)
    lh, moe, logits, ids, wts = oracle.moe_layer(x, *(w[k] for k in MOE_KEYS), top_k=SMALL.num_routed_experts)
    data = {f"in_{k}": to_np(w[k]) for k in MOE_KEYS}
    data["in_hidden"] = to_np(x)
    data.update(out_layer_hidden=lh.numpy(), out_moe_update=moe.numpy(), out_logits=logits.numpy(),
                out_ids=ids.numpy(), out_weights=wts.numpy())
    return data


DN_KEYS = ("input_norm_weight", "in_proj_qkv_weight", "in_proj_z_weight", "in_proj_a_weight", "in_proj_b_weight",
           "conv1d_weight", "out_proj_weight", "linear_norm_weight", "a_log", "dt_bias", "conv_state", "recurrent_state")


def make_deltanet(tokens: int = 3, seed: int = 11):
    w = wl.make_deltanet_weights(SMALL, seed=seed)
    x = wl.make_hidden(tokens, SMALL.hidden_size, seed=seed + 1)
    update, conv, state = oracle.deltanet_update(
        x, w["conv_state"], w["recurrent_state"], w,
        qk_heads=SMALL.deltanet_qk_heads, value_heads=SMALL.deltanet_value_heads, head_dim=SMALL.deltanet_head_dim,
    )
    data = {f"in_{k}": to_np(w[k]) for k in DN_KEYS}
    data["in_hidden"] = to_np(x)
    data.update(out_update=update.numpy(), out_conv_state=to_np(conv), out_recurrent_state=state.numpy())
    return data


def main() -> None:
    np.savez_compressed(os.path.join(HERE, "moe_small.npz"), **make_moe())
    np.savez_compressed(os.path.join(HERE, "deltanet_small.npz"), **make_deltanet())
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
