"""Parity helpers shared by the GPU tests.

Tolerance (north star): fp32 outputs of bf16 inputs within rtol 2e-2 /
atol 2e-2 of the fp32 oracle; routing ids and histograms bit-exact.
"""

from __future__ import annotations

import numpy as np
import torch

import oracle

ATOL = 2e-2
RTOL = 2e-2
# fp32 inputs: the reference's default fp32 tolerance (testing/tolerances.py:13-14)
ATOL_F32 = 1e-4
RTOL_F32 = 1e-4


def tol(dtype: torch.dtype) -> dict[str, float]:
    if dtype == torch.float32:
        return {"atol": ATOL_F32, "rtol": RTOL_F32}
    return {"atol": ATOL, "rtol": RTOL}


def assert_routing_parity(k_logits, k_ids, k_w, o_logits, top_k: int, *, gap: float = 1e-4) -> int:
    """Routing parity at two levels.

    1. Conditional (always): the oracle's top-k applied to the kernel's own
       logits must give exactly the kernel's ids (this pins softmax / top-k /
       tie rule independent of logit rounding), except where two kernel
       probabilities are within 1e-6 relative (fp32 exp rounding).
    2. Absolute: ids equal the oracle's ids for every token whose sorted
       oracle probabilities are separated by more than `gap` (relative) at
       every position up to k; tokens with closer margins are counted and
       returned, not failed.
    """

    k_logits = k_logits.detach().float().cpu().reshape(-1, k_logits.shape[-1])
    k_ids = k_ids.detach().cpu().reshape(-1, top_k)
    k_w = k_w.detach().float().cpu().reshape(-1, top_k)
    o_logits = o_logits.detach().float().cpu().reshape(-1, o_logits.shape[-1])
    probs = torch.softmax(k_logits, dim=-1)
    c_vals, c_ids = oracle.topk_lowest_id(probs, top_k)
    for t in range(k_ids.shape[0]):
        if not torch.equal(c_ids[t], k_ids[t]):
            pk = probs[t, k_ids[t]]
            pc = probs[t, c_ids[t]]
            assert torch.allclose(pk, pc, rtol=1e-6, atol=0), f"token {t}: ids {k_ids[t].tolist()} vs {c_ids[t].tolist()}"
    torch.testing.assert_close(k_w, c_vals / c_vals.sum(-1, keepdim=True), atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(k_w.sum(-1), torch.ones(k_w.shape[0]), atol=1e-5, rtol=0)

    o_probs = torch.softmax(o_logits, dim=-1)
    sorted_p, _ = torch.sort(o_probs, dim=-1, descending=True)
    _, o_ids = oracle.topk_lowest_id(o_probs, top_k)
    near = 0
    for t in range(k_ids.shape[0]):
        margins = (sorted_p[t, :top_k] - sorted_p[t, 1 : top_k + 1]) / sorted_p[t, :top_k]
        if bool((margins > gap).all()):
            assert k_ids[t].tolist() == o_ids[t].tolist(), f"token {t}: {k_ids[t].tolist()} vs {o_ids[t].tolist()}"
        else:
            near += 1
    return near


def histogram(ids, num_experts: int) -> np.ndarray:
    return oracle.expert_histogram(ids.detach().cpu().numpy(), num_experts)
