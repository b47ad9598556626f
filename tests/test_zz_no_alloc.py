"""The allocation-free MoE layer entry point (fk_moe_layer_noalloc).

It runs fk_moe_layer's kernels with the workspace in a file-scope device
array.  Checked through the C ABI against fk_moe_layer with a caller-owned
workspace on the same inputs: two calls in a row, the second with fewer
tokens (the shared array keeps the first call's contents), across the
single-launch (T = 1), GEMV (T < 44) and MFMA (T >= 44) paths; the
results must be identical bit for bit (same kernels, same arithmetic).
Sizes beyond the array are refused before anything is launched.  The
array's error word, reached through fk_moe_noalloc_workspace, reports a
wait that ran out (forced with a wait bound of 0) and clears, after which
the results are identical again.
"""

from __future__ import annotations

import ctypes
import dataclasses

import pytest
import torch

from fastkernels_amd import _lib
from fastkernels_amd import workloads as wl
from fastkernels_amd.kernels.hip import _fcode
from fastkernels_amd.spec import qwen36_35b_a3b_spec

pytestmark = pytest.mark.gpu

SPEC = qwen36_35b_a3b_spec()
SMALL = dataclasses.replace(SPEC, num_experts=64, expert_intermediate_size=256, hidden_size=1024)
K = 8


@pytest.fixture(scope="module")
def weights(device):
    return wl.make_moe_weights(SMALL, seed=61, device=device)


def _args(w, x):
    T, H = x.shape
    E, two_i, _ = w["expert_gate_up_weight"].shape
    outs = dict(
        logits=torch.empty(T, E, device=x.device),
        ids=torch.empty(T, K, dtype=torch.int64, device=x.device),
        w=torch.empty(T, K, device=x.device),
        moe=torch.empty(T, H, device=x.device),
        layer=torch.empty(T, H, device=x.device),
    )
    sg = w["shared_expert_gate_weight"]
    head = [
        x.data_ptr(), _fcode(x, "hidden"),
        w["norm_weight"].data_ptr(), _fcode(w["norm_weight"], "norm"),
        w["router_weight"].data_ptr(), _fcode(w["router_weight"], "router"),
        None, 0,
        w["expert_gate_up_weight"].data_ptr(), w["expert_down_weight"].data_ptr(),
        _fcode(w["expert_gate_up_weight"], "experts"),
        w["shared_gate_up_weight"].data_ptr(), w["shared_down_weight"].data_ptr(),
        sg.data_ptr(), _fcode(sg, "gate"),
        T, H, two_i // 2, E, K, 1e-6, 1.0,
        outs["logits"].data_ptr(), outs["ids"].data_ptr(), outs["w"].data_ptr(),
        outs["moe"].data_ptr(), outs["layer"].data_ptr(),
    ]
    return head, outs


def _with_workspace(w, x):
    head, outs = _args(w, x)
    T, H = x.shape
    E, two_i, _ = w["expert_gate_up_weight"].shape
    nbytes = _lib.load().fk_moe_workspace_bytes(T, K, E, two_i // 2, H)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=x.device)
    stream = torch.cuda.current_stream(x.device).cuda_stream
    _lib.call("fk_moe_layer", *head, ws.data_ptr(), ws.numel(), stream)
    _lib.call("fk_workspace_status", ws.data_ptr(), ws.numel(), 0, stream)
    return outs


def _noalloc(w, x):
    head, outs = _args(w, x)
    _lib.call("fk_moe_layer_noalloc", *head, torch.cuda.current_stream(x.device).cuda_stream)
    torch.cuda.synchronize()
    return outs


@pytest.mark.parametrize("first,second", [(16, 1), (128, 2), (64, 8)])
def test_noalloc_matches_workspace_entry_point(device, weights, first, second):
    print(f"noalloc T={first} then T={second}", flush=True)
    for step, tokens in enumerate((first, second)):
        x = wl.make_hidden(tokens, SMALL.hidden_size, seed=62 + tokens).to(device)
        a = _noalloc(weights, x)
        b = _with_workspace(weights, x)
        torch.cuda.synchronize()
        assert torch.equal(a["ids"], b["ids"]), f"call {step}"
        for k in ("logits", "w", "moe", "layer"):
            assert torch.equal(a[k], b[k]), f"call {step}: {k}"
        assert bool(torch.isfinite(a["layer"]).all())


def test_noalloc_rejects_sizes_beyond_its_scratch(device, weights):
    # the smallest token count whose workspace exceeds the 16 MiB array
    lib = _lib.load()
    tokens = 1
    while lib.fk_moe_workspace_bytes(tokens, K, SMALL.num_experts, SMALL.expert_intermediate_size,
                                     SMALL.hidden_size) <= 16 << 20:
        tokens += 1
    assert tokens <= 512  # T * K within the routing-table limit, so only the size is refused
    x = torch.zeros(tokens, SMALL.hidden_size, dtype=torch.bfloat16, device=device)
    head, _ = _args(weights, x)
    status = _lib.load().fk_moe_layer_noalloc(*head, torch.cuda.current_stream(device).cuda_stream)
    assert status == _lib.FK_ERR_UNSUPPORTED
    assert "scratch" in _lib.load().fk_last_error_detail().decode()


def test_noalloc_failed_wait_is_flagged_and_clears(device, weights):
    lib = _lib.load()
    stream = torch.cuda.current_stream(device).cuda_stream
    ptr, nbytes = ctypes.c_void_p(), ctypes.c_size_t()
    _lib.call("fk_moe_noalloc_workspace", ctypes.byref(ptr), ctypes.byref(nbytes), stream)
    assert ptr.value and nbytes.value == 16 << 20
    for tokens in (1, 4):
        print(f"noalloc forced wait failure T={tokens}", flush=True)
        x = wl.make_hidden(tokens, SMALL.hidden_size, seed=70 + tokens).to(device)
        try:
            _lib.call("fk_workspace_set_poll_limit", ptr, nbytes, 0, stream)
            a = _noalloc(weights, x)
            assert bool(torch.isnan(a["layer"]).all()) and bool(torch.isnan(a["moe"]).all())
        finally:
            _lib.call("fk_workspace_set_poll_limit", ptr, nbytes, -1, stream)
        assert lib.fk_workspace_status(ptr, nbytes, 1, stream) == _lib.FK_ERR_DEVICE
        assert lib.fk_workspace_status(ptr, nbytes, 0, stream) == _lib.FK_OK
        a = _noalloc(weights, x)
        b = _with_workspace(weights, x)
        torch.cuda.synchronize()
        assert torch.equal(a["ids"], b["ids"])
        for k in ("logits", "w", "moe", "layer"):
            assert torch.equal(a[k], b[k]), k
