"""CPU-side checks of the C ABI library and the operator shim (no GPU compute)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from fastkernels_amd import _lib
from fastkernels_amd.kernels import hip

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "fastkernels_hip.h"


def _header_functions() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(fk_[a-z_0-9]+)\(", text, flags=re.M))


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _header_functions()
    assert declared, "no declarations parsed from the header"
    assert declared == set(_lib.SIGNATURES), "ctypes signatures out of sync with include/fastkernels_hip.h"
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.fk_abi_version() == 1


def test_product_library_carries_no_timeline_markers():
    # the per-phase timeline exists only in the -DFK_TIMELINE diagnostic build
    lib = _lib.load()
    for unit in ("moe_fused", "moe_router", "deltanet_step", "attn_step"):
        assert not hasattr(lib, f"fk_timeline_read_{unit}"), unit


def test_timeline_markers_have_names():
    from fastkernels_amd import timeline

    assert {k: len(v[1]) for k, v in timeline.MARKERS.items()} == {"moe": 12, "router": 6, "deltanet": 13, "attention": 15}
    assert all(len(names) <= 16 for _, names in timeline.MARKERS.values())  # kTimelineMarks


# The names of the reference operator package (fastkernels.kernels.triton
# __all__, kernels/triton/__init__.py:37-62): a host switched to this package
# finds every one of them.
REFERENCE_OPERATORS = [
    "triton_expert_histogram", "triton_fused_swiglu", "triton_qwen36_batched_attention_decode",
    "triton_qwen36_batched_attention_moe_layer_decode", "triton_qwen36_batched_attention_project",
    "triton_qwen36_batched_deltanet_conv", "triton_qwen36_batched_deltanet_moe_layer_decode",
    "triton_qwen36_batched_deltanet_project", "triton_qwen36_batched_deltanet_recurrent_output",
    "triton_qwen36_batched_moe_decode", "triton_qwen36_batched_moe_layer_decode",
    "triton_qwen36_batched_moe_router_decode", "triton_qwen36_batched_routed_experts_decode",
    "triton_qwen36_batched_routed_shared_experts_decode", "triton_qwen36_moe_decode",
    "triton_qwen36_moe_router_decode", "triton_qwen36_routed_experts_decode",
    "triton_qwen36_routed_shared_experts_decode", "triton_qwen36_single_expert_mlp_decode",
    "triton_synthetic_qwen36_attention_decode", "triton_synthetic_qwen36_attention_moe_decode",
    "triton_synthetic_qwen36_deltanet_decode", "triton_synthetic_qwen36_deltanet_moe_decode",
    "triton_synthetic_qwen36_moe_decode",
]


def test_every_reference_operator_name_is_exported():
    assert len(REFERENCE_OPERATORS) == 24
    assert set(REFERENCE_OPERATORS) == set(hip.TRITON_ALIASES)
    for name in REFERENCE_OPERATORS:
        assert getattr(hip, name) is hip.TRITON_ALIASES[name], name
    # the reference's own test module imports these names in one statement
    ns: dict = {}
    exec("from fastkernels_amd.kernels.hip import " + ", ".join(REFERENCE_OPERATORS), ns)
    assert all(name in ns for name in REFERENCE_OPERATORS)


def test_synthetic_attention_rejects_like_the_reference():
    # reference qwen36_attention.py:875-893: checked in this order, before any GPU work
    kc = torch.zeros(8, 2, 4)
    args = (torch.zeros(16), kc, kc, None, None, None, None, None)
    kw = dict(position=2, attention_heads=4, kv_heads=2, head_dim=4, rope_dim=4)
    with pytest.raises(ValueError, match="hidden must have shape"):
        hip.hip_synthetic_qwen36_attention_decode(torch.zeros(2, 16), *args[1:], **kw)
    with pytest.raises(ValueError, match="key/value caches must have shape"):
        hip.hip_synthetic_qwen36_attention_decode(args[0], torch.zeros(8, 8), kc, *args[3:], **kw)
    with pytest.raises(ValueError, match="CUDA tensors"):
        hip.hip_synthetic_qwen36_attention_decode(*args, **kw)


def test_status_strings():
    assert _lib.status_string(_lib.FK_OK) == "ok"
    assert "workspace" in _lib.status_string(_lib.FK_ERR_WORKSPACE)
    assert _lib.status_string(12345) == "unknown status"
    assert "wait" in _lib.status_string(_lib.FK_ERR_DEVICE)


def test_workspace_status_rejects_missing_workspace():
    # Host-side check: no device access for a NULL or header-less workspace.
    assert _err("fk_workspace_status", None, 0, 0, None) == _lib.FK_ERR_WORKSPACE
    assert _err("fk_workspace_status", ctypes.c_void_p(256), 32, 0, None) == _lib.FK_ERR_WORKSPACE
    assert _err("fk_workspace_set_poll_limit", None, 0, 0, None) == _lib.FK_ERR_WORKSPACE
    assert _err("fk_workspace_set_poll_limit", ctypes.c_void_p(256), 32, 0, None) == _lib.FK_ERR_WORKSPACE
    assert _err("fk_workspace_set_poll_limit", ctypes.c_void_p(256), 4096, 1 << 31, None) == _lib.FK_ERR_INVALID


def test_workspace_sizes_are_monotone():
    lib = _lib.load()
    a = lib.fk_moe_workspace_bytes(1, 8, 256, 512, 2048)
    b = lib.fk_moe_workspace_bytes(16, 8, 256, 512, 2048)
    c = lib.fk_moe_workspace_bytes(128, 8, 256, 512, 2048)
    assert 0 < a < b < c
    # per-pair activations and down outputs dominate: (T*K + T) * (I + H) * 4 bytes
    assert c >= (128 * 8 + 128) * (512 + 2048) * 4
    assert lib.fk_moe_workspace_bytes(0, 8, 256, 512, 2048) == 0
    assert lib.fk_deltanet_workspace_bytes(8, 32, 128) >= 2 * 8 * 32 * 128 * 4


def _err(fn: str, *args) -> int:
    lib = _lib.load()
    return getattr(lib, fn)(*args)


def test_entry_points_reject_bad_arguments_before_launch():
    # Validation happens on the host: NULL pointers / bad sizes return a
    # status without touching a device.
    st = _err("fk_moe_router", None, 1, None, 1, None, 1, None, 1, 1, 2048, 256, 9, 1e-6, 1.0,
              None, None, None, None, 0, None)
    assert st == _lib.FK_ERR_INVALID
    assert b"top_k" in _lib.load().fk_last_error_detail()
    st = _err("fk_moe_router", None, 1, None, 1, None, 1, None, 1, 1, 2047, 256, 8, 1e-6, 1.0,
              None, None, None, None, 0, None)
    assert st == _lib.FK_ERR_ALIGNMENT
    st = _err("fk_moe_router", None, 7, None, 1, None, 1, None, 1, 1, 2048, 256, 8, 1e-6, 1.0,
              None, None, None, None, 0, None)
    assert st == _lib.FK_ERR_DTYPE
    st = _err("fk_moe_experts", None, 1, None, None, 1, None, None, None, 0, 1, 2048, 512, 256, 8,
              None, None, None, 0, None)
    assert st == _lib.FK_ERR_INVALID
    st = _err("fk_moe_align", None, 3, None, 0, 1, 8, 256, None, 0, None, None, None, None, None)
    assert st == _lib.FK_ERR_INVALID
    st = _err("fk_moe_align", None, 0, None, 0, 1, 8, 256, None, 0, None, None, None, None, None)
    assert st == _lib.FK_ERR_DTYPE
    st = _err("fk_deltanet_conv", None, 0, None, 0, None, 0, 1, 16, 9, None, None, None)
    assert st == _lib.FK_ERR_UNSUPPORTED
    dts = (ctypes.c_int32 * 10)(*([0] * 10))
    st = _err("fk_deltanet_recurrent_output", *([None] * 10), ctypes.cast(dts, ctypes.c_void_p),
              1, 16, 32, 256, 2048, 1e-6, None, None, None, None, 0, None)
    assert st == _lib.FK_ERR_UNSUPPORTED
    st = _err("fk_synthetic_moe", None, 0, None, None, None, None, None, None, 0, 16, 4, 8, 9, 1e-6, None, 0, None)
    assert st == _lib.FK_ERR_INVALID


def test_workspace_too_small_is_reported():
    buf = (ctypes.c_uint8 * 64)()
    addr = ctypes.addressof(buf)
    addr16 = addr + (-addr % 16)
    dummy = addr16
    st = _err("fk_moe_router", dummy, 1, dummy, 1, dummy, 1, None, 1, 1, 2048, 256, 8, 1e-6, 1.0,
              dummy, dummy, dummy, dummy, 16, None)
    assert st == _lib.FK_ERR_WORKSPACE


# ---------------------------------------------------------------------------
# Shim validation mirrors the reference's ValueError rules (CPU tensors are
# rejected before any launch, as `is_cuda` checks do in the reference).
# ---------------------------------------------------------------------------
def test_router_rejects_cpu_tensors_and_bad_shapes():
    h = torch.zeros(2048)
    with pytest.raises(ValueError, match="CUDA"):
        hip.hip_qwen36_moe_router_decode(h, torch.zeros(2048), torch.zeros(256, 2048))
    with pytest.raises(ValueError, match=r"hidden must have shape \[hidden_size\]"):
        hip.hip_qwen36_moe_router_decode(torch.zeros(1, 2048), torch.zeros(2048), torch.zeros(256, 2048))
    with pytest.raises(ValueError, match="router_weight must have shape"):
        hip.hip_qwen36_moe_router_decode(h, torch.zeros(2048), torch.zeros(256, 1024))
    with pytest.raises(ValueError, match="tokens, hidden_size"):
        hip.hip_qwen36_batched_moe_router_decode(h, torch.zeros(2048), torch.zeros(256, 2048))


def test_experts_reject_missing_shared_and_bad_shapes():
    h = torch.zeros(64)
    ids = torch.zeros(4, dtype=torch.int64)
    w = torch.zeros(4)
    gu = torch.zeros(8, 32, 64)
    dn = torch.zeros(8, 64, 16)
    with pytest.raises(ValueError, match="CUDA"):
        hip.hip_qwen36_routed_experts_decode(h, ids, w, gu, dn)
    with pytest.raises(ValueError, match="same shape"):
        hip.hip_qwen36_routed_experts_decode(h, ids, torch.zeros(3), gu, dn)
    with pytest.raises(ValueError, match="experts, 2 \\* intermediate"):
        hip.hip_qwen36_routed_experts_decode(h, ids, w, gu[0], dn)


def test_deltanet_and_synthetic_validation():
    with pytest.raises(ValueError, match="mixed_qkv must have shape"):
        hip.hip_qwen36_batched_deltanet_conv(torch.zeros(8), torch.zeros(8, 4), torch.zeros(8, 1, 4))
    with pytest.raises(ValueError, match="conv_weight must have shape"):
        hip.hip_qwen36_batched_deltanet_conv(torch.zeros(1, 8), torch.zeros(8, 4), torch.zeros(8, 1, 3))
    with pytest.raises(ValueError, match="recurrent_state must have shape"):
        hip.hip_qwen36_batched_deltanet_recurrent_output(
            torch.zeros(1, 64), torch.zeros(1, 32), torch.zeros(1, 4), torch.zeros(1, 4), torch.zeros(4, 8, 4),
            torch.zeros(64, 32), torch.zeros(8), torch.zeros(4), torch.zeros(4), qk_heads=2, value_heads=4, head_dim=8,
        )
    with pytest.raises(ValueError, match="1 <= top_k <= 8"):
        hip.hip_synthetic_qwen36_moe_decode(
            torch.zeros(16), torch.zeros(16), torch.zeros(4, 16), torch.zeros(4, 16, 16), torch.zeros(4, 16, 8),
            torch.zeros(16, 16), torch.zeros(16, 8), top_k=9,
        )


def test_attention_validation():
    x, kc = torch.zeros(2, 16), torch.zeros(4, 2, 4)
    args = (torch.zeros(16), torch.zeros(32, 16), torch.zeros(8, 16), torch.zeros(8, 16), torch.zeros(16, 16),
            torch.zeros(4), torch.zeros(4))
    kw = dict(attention_heads=4, kv_heads=2, head_dim=4, rope_dim=4)
    with pytest.raises(ValueError, match="key/value caches must have shape"):
        hip.hip_qwen36_batched_attention_decode(x, torch.zeros(4, 8), kc, *args, **kw)
    with pytest.raises(ValueError, match="cache shape does not match"):
        hip.hip_qwen36_batched_attention_decode(x, torch.zeros(4, 2, 8), torch.zeros(4, 2, 8), *args, **kw)
    with pytest.raises(ValueError, match="CUDA tensors"):
        hip.hip_qwen36_batched_attention_decode(x, kc, kc.clone(), *args, **kw)
    with pytest.raises(ValueError, match="weight must have shape"):
        hip.hip_qwen36_batched_attention_project(x, torch.zeros(16), torch.zeros(32, 8), args[2], args[3])


def test_product_package_does_not_import_oracle():
    for path in (ROOT / "fastkernels_amd").rglob("*.py"):
        text = path.read_text()
        assert "import oracle" not in text and "from oracle" not in text, path


def test_poll_limit_above_the_cap_is_refused_before_any_launch():
    # refused on the host (no launch, so no GPU is needed): a failed wait must
    # still end within seconds
    lib = _lib.load()
    buf = ctypes.create_string_buffer(64)
    status = lib.fk_workspace_set_poll_limit(ctypes.addressof(buf), 64, (1 << 22) + 1, None)
    assert status == _lib.FK_ERR_INVALID
    assert "at most" in lib.fk_last_error_detail().decode()
