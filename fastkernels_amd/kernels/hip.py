"""MI355X operator API for the Qwen3.6 MoE decode layer and Gated DeltaNet step.

Every public function mirrors one entry point of the reference's
`fastkernels.kernels.triton` package (same positional/keyword signature,
same ValueError conditions, fp32 outputs where the reference returns fp32)
and runs the hand-written gfx950 kernels of libfastkernels_hip.so through
its C ABI.  Work is enqueued on the current torch stream without host
synchronisation; outputs are allocated with torch on the input's device.

Names are `hip_*`; `TRITON_ALIASES` maps each reference name
(`triton_*`) to its counterpart so callers can switch implementations by
import only (e.g. the `--moe-impl`/`--deltanet-impl` switch of
bench/qwen36_decode_reference.py).

Intentional differences from the reference (documented, not bugs):
  * top-k ties go to the lower expert id (the reference Triton kernel picks
    the higher id, qwen36_router.py:95);
  * float16 inputs are rejected (bf16 and fp32 are supported);
  * the MoE entry points take an optional keyword `router_bias` (added to
    the logits) that the reference lacks.
"""

from __future__ import annotations

import ctypes
import threading
from typing import Any

import torch

from .. import _lib

__all__ = [
    "hip_expert_histogram",
    "hip_fused_swiglu",
    "hip_qwen36_moe_router_decode",
    "hip_qwen36_batched_moe_router_decode",
    "hip_qwen36_single_expert_mlp_decode",
    "hip_qwen36_routed_experts_decode",
    "hip_qwen36_routed_shared_experts_decode",
    "hip_qwen36_batched_routed_experts_decode",
    "hip_qwen36_batched_routed_shared_experts_decode",
    "hip_qwen36_moe_decode",
    "hip_qwen36_batched_moe_decode",
    "hip_qwen36_batched_moe_layer_decode",
    "hip_qwen36_moe_align",
    "hip_qwen36_batched_deltanet_project",
    "hip_qwen36_batched_deltanet_conv",
    "hip_qwen36_batched_deltanet_recurrent_output",
    "hip_qwen36_batched_deltanet_moe_layer_decode",
    "hip_qwen36_batched_attention_project",
    "hip_qwen36_batched_attention_decode",
    "hip_qwen36_batched_attention_moe_layer_decode",
    "hip_synthetic_qwen36_moe_decode",
    "hip_synthetic_qwen36_deltanet_decode",
    "hip_synthetic_qwen36_deltanet_moe_decode",
    "hip_synthetic_qwen36_attention_decode",
    "hip_synthetic_qwen36_attention_moe_decode",
    "workspace_status",
    "TRITON_ALIASES",
]

# ---------------------------------------------------------------------------
# Plumbing
# ---------------------------------------------------------------------------
_FLOAT_CODES = {torch.float32: _lib.FK_DTYPE_F32, torch.bfloat16: _lib.FK_DTYPE_BF16}
_INDEX_CODES = {torch.int32: _lib.FK_DTYPE_I32, torch.int64: _lib.FK_DTYPE_I64}


def _fcode(t: torch.Tensor, name: str) -> int:
    try:
        return _FLOAT_CODES[t.dtype]
    except KeyError:
        raise ValueError(f"{name} must be float32 or bfloat16 (got {t.dtype})") from None


def _icode(t: torch.Tensor, name: str) -> int:
    try:
        return _INDEX_CODES[t.dtype]
    except KeyError:
        raise ValueError(f"{name} must be int32 or int64 (got {t.dtype})") from None


def _dense(t: torch.Tensor) -> torch.Tensor:
    """Contiguous and 16-byte aligned (vector loads need both)."""

    t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


_ws_lock = threading.Lock()
_workspaces: dict[tuple[str, int, int], torch.Tensor] = {}


def _workspace(kind: str, device: torch.device, nbytes: int) -> torch.Tensor:
    """Per-(kind, device, stream) workspace, zero-filled when (re)allocated.

    Kernels leave their counters at zero when they finish, so a workspace is
    reused by later calls on the same stream without clearing.
    """

    key = (kind, device.index if device.index is not None else torch.cuda.current_device(), _stream(device))
    with _ws_lock:
        ws = _workspaces.get(key)
        if ws is None or ws.numel() < nbytes:
            ws = torch.zeros(max(nbytes, 4096), dtype=torch.uint8, device=device)
            _workspaces[key] = ws
        return ws


# Workspaces whose kernels wait on other workgroups (bounded waits, error word).
_POLLING_KINDS = ("moe", "deltanet_step", "attention")


def workspace_status(device: Any = None, *, clear: bool = True) -> None:
    """Raise FastKernelsError (FK_ERR_DEVICE) if a bounded in-kernel wait of
    an operator call on `device` (any stream) ran out since the last check.

    The MoE and DeltaNet-step kernels hand values between workgroups and
    assume all workgroups of a launch are resident at once; a wait that runs
    out leaves NaN in the outputs built from incomplete inputs, and every
    later call on the same cached workspace gives NaN until this check
    clears the flag (`clear=True`).  Synchronises the workspaces' streams.
    No counterpart in the reference (its kernels never wait on each other).
    """

    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    index = dev.index if dev.index is not None else torch.cuda.current_device()
    lib = _lib.load()
    failed: list[tuple[str, int, str]] = []
    with _ws_lock:
        items = [(k, ws) for k, ws in _workspaces.items() if k[0] in _POLLING_KINDS and k[1] == index]
    for (kind, _, stream), ws in items:
        status = lib.fk_workspace_status(ws.data_ptr(), ws.numel(), 1 if clear else 0, stream)
        if status == _lib.FK_ERR_DEVICE:
            failed.append((kind, status, lib.fk_last_error_detail().decode()))
        elif status != _lib.FK_OK:
            raise _lib.FastKernelsError("fk_workspace_status", status, lib.fk_last_error_detail().decode())
    if failed:
        kind, status, detail = failed[0]
        raise _lib.FastKernelsError(f"fk_workspace_status ({kind} workspace)", status, detail)


def _require_lib() -> None:
    _lib.load()


# ---------------------------------------------------------------------------
# MoE building blocks
# ---------------------------------------------------------------------------
def hip_fused_swiglu(gate_up: Any, *, block_size: int = 256) -> Any:
    """`silu(gate) * up` for `[N, 2I]` (reference moe.py:67-84)."""

    _require_lib()
    if gate_up.ndim != 2:
        raise ValueError("gate_up must have shape [N, 2 * intermediate]")
    if gate_up.shape[1] % 2:
        raise ValueError("last dimension must be even")
    if not gate_up.is_cuda:
        raise ValueError("gate_up must be a CUDA tensor")
    gu = _dense(gate_up)
    intermediate = gu.shape[1] // 2
    out = torch.empty((gu.shape[0], intermediate), device=gu.device, dtype=gu.dtype)
    _lib.call("fk_fused_swiglu", gu.data_ptr(), _fcode(gu, "gate_up"), gu.shape[0], intermediate, out.data_ptr(), _stream(gu.device))
    return out


def hip_expert_histogram(topk_ids: Any, num_experts: int, *, block_size: int = 256) -> Any:
    """Routed-token count per expert, int32 `[E]` (reference moe.py:87-102)."""

    _require_lib()
    if topk_ids.ndim != 2:
        raise ValueError("topk_ids must have shape [tokens, top_k]")
    if not topk_ids.is_cuda:
        raise ValueError("topk_ids must be a CUDA tensor")
    ids = _dense(topk_ids)
    counts = torch.empty((num_experts,), device=ids.device, dtype=torch.int32)
    _lib.call("fk_expert_histogram", ids.data_ptr(), _icode(ids, "topk_ids"), ids.numel(), num_experts, counts.data_ptr(), _stream(ids.device))
    return counts


def hip_qwen36_moe_align(topk_ids: Any, num_experts: int, topk_weights: Any | None = None) -> tuple[Any, Any, Any, Any]:
    """Routing tables for `[T, K]` expert ids: `(counts[E], offsets[E+1], perm[T*K], inverse[T*K])`.

    `perm[p]` is the flat pair index `t*K + k` at permuted position `p`, with
    pairs sorted stably by (expert, token, slot); `inverse` is its inverse and
    `offsets` the exclusive prefix sum of `counts`.  The reference has no
    stable token permutation of its own (its expert kernels stream the
    weights per (token, slot)); `counts` equals `triton_expert_histogram`.
    """

    _require_lib()
    if topk_ids.ndim != 2:
        raise ValueError("topk_ids must have shape [tokens, top_k]")
    if not topk_ids.is_cuda:
        raise ValueError("topk_ids must be a CUDA tensor")
    ids = _dense(topk_ids)
    tokens, top_k = ids.shape
    dev = ids.device
    w = None if topk_weights is None else _dense(topk_weights)
    counts = torch.empty((num_experts,), device=dev, dtype=torch.int32)
    offsets = torch.empty((num_experts + 1,), device=dev, dtype=torch.int32)
    perm = torch.empty((tokens * top_k,), device=dev, dtype=torch.int32)
    inverse = torch.empty((tokens * top_k,), device=dev, dtype=torch.int32)
    nbytes = _lib.load().fk_moe_workspace_bytes(tokens, top_k, num_experts, 8, 8)
    ws = _workspace("moe", dev, nbytes)
    _lib.call(
        "fk_moe_align",
        ids.data_ptr(), _icode(ids, "topk_ids"), _ptr(w), _fcode(w, "topk_weights") if w is not None else 0,
        tokens, top_k, num_experts, ws.data_ptr(), ws.numel(),
        counts.data_ptr(), offsets.data_ptr(), perm.data_ptr(), inverse.data_ptr(), _stream(dev),
    )
    return counts, offsets, perm, inverse


def _router_checks(hidden: Any, norm_weight: Any, router_weight: Any, top_k: int, batched: bool) -> None:
    if batched:
        if hidden.ndim != 2:
            raise ValueError("hidden must have shape [tokens, hidden_size]")
        if norm_weight.ndim != 1 or norm_weight.shape[0] != hidden.shape[1]:
            raise ValueError("norm_weight must have shape [hidden_size]")
        if router_weight.ndim != 2 or router_weight.shape[1] != hidden.shape[1]:
            raise ValueError("router_weight must have shape [num_experts, hidden_size]")
    else:
        if hidden.ndim != 1:
            raise ValueError("hidden must have shape [hidden_size]")
        if norm_weight.shape != hidden.shape:
            raise ValueError("norm_weight must have the same shape as hidden")
        if router_weight.ndim != 2 or router_weight.shape[1] != hidden.shape[0]:
            raise ValueError("router_weight must have shape [num_experts, hidden_size]")
    if not hidden.is_cuda or not norm_weight.is_cuda or not router_weight.is_cuda:
        raise ValueError("hidden, norm_weight, and router_weight must be CUDA tensors")
    if top_k < 1 or top_k > 8:
        raise ValueError("router kernel supports 1 <= top_k <= 8")
    hidden_size = hidden.shape[-1]
    num_experts = router_weight.shape[0]
    if hidden_size > 4096 or num_experts > 1024:
        raise ValueError("router kernel currently supports hidden_size<=4096 and num_experts<=1024")
    if top_k > num_experts:
        raise ValueError("top_k must be <= number of experts")
    if hidden_size % 8:
        raise ValueError("hidden_size must be a multiple of 8 for the HIP router")


def _router_bias_checks(router_bias: Any | None, num_experts: int) -> None:
    if router_bias is None:
        return
    if not router_bias.is_cuda:
        raise ValueError("router_bias must be a CUDA tensor")
    if router_bias.numel() != num_experts:
        raise ValueError("router_bias must have num_experts elements")


# The C ABI routes at most 4096 (token, expert) pairs per call (fk_moe.hip
# kMaxPairs: one workgroup builds the routing tables in LDS).  Longer batches
# go through in consecutive calls of whole tokens on the same stream and
# workspace: every token is routed, and its experts combined, on its own, so
# the split changes no token's result beyond the kernel choice that the
# batch size makes anyway.  A batch of no tokens makes no call and returns
# empty outputs, as the reference's zero-sized launch grids do.
_MAX_PAIRS = 4096


def _token_chunks(tokens: int, top_k: int) -> list[tuple[int, int]]:
    step = max(1, _MAX_PAIRS // top_k)
    return [(s, min(tokens, s + step)) for s in range(0, tokens, step)]


def _chunk_max(chunks: list[tuple[int, int]]) -> int:
    return max((e - s for s, e in chunks), default=1)


def _run_router(hidden2d, norm_weight, router_weight, top_k, eps, norm_offset, router_bias, ws):
    tokens, hidden_size = hidden2d.shape
    num_experts = router_weight.shape[0]
    dev = hidden2d.device
    logits = torch.empty((tokens, num_experts), device=dev, dtype=torch.float32)
    ids = torch.empty((tokens, top_k), device=dev, dtype=torch.int64)
    weights = torch.empty((tokens, top_k), device=dev, dtype=torch.float32)
    nw = _dense(norm_weight)
    rb = None if router_bias is None else _dense(router_bias)
    for s, e in _token_chunks(tokens, top_k):
        _lib.call(
            "fk_moe_router",
            hidden2d[s:e].data_ptr(), _fcode(hidden2d, "hidden"),
            nw.data_ptr(), _fcode(nw, "norm_weight"),
            router_weight.data_ptr(), _fcode(router_weight, "router_weight"),
            _ptr(rb), _fcode(rb, "router_bias") if rb is not None else 0,
            e - s, hidden_size, num_experts, top_k, float(eps), float(norm_offset),
            logits[s:e].data_ptr(), ids[s:e].data_ptr(), weights[s:e].data_ptr(), ws.data_ptr(), ws.numel(), _stream(dev),
        )
    return logits, ids, weights


def hip_qwen36_moe_router_decode(
    hidden: Any,
    norm_weight: Any,
    router_weight: Any,
    *,
    top_k: int = 8,
    eps: float = 1e-6,
    norm_offset: float = 1.0,
    router_bias: Any | None = None,
) -> tuple[Any, Any, Any]:
    """One-token router: `(logits f32[E], topk_ids i64[K], topk_weights f32[K])`.

    Reference: triton_qwen36_moe_router_decode (qwen36_router.py:193-257).
    """

    _require_lib()
    _router_checks(hidden, norm_weight, router_weight, top_k, batched=False)
    _router_bias_checks(router_bias, router_weight.shape[0])
    x = _dense(hidden).reshape(1, -1)
    rw = _dense(router_weight)
    ws = _workspace("moe", x.device, _lib.load().fk_moe_workspace_bytes(1, top_k, rw.shape[0], 8, 8))
    logits, ids, weights = _run_router(x, norm_weight, rw, top_k, eps, norm_offset, router_bias, ws)
    return logits.reshape(-1), ids.reshape(-1), weights.reshape(-1)


def hip_qwen36_batched_moe_router_decode(
    hidden: Any,
    norm_weight: Any,
    router_weight: Any,
    *,
    top_k: int = 8,
    eps: float = 1e-6,
    norm_offset: float = 1.0,
    router_bias: Any | None = None,
) -> tuple[Any, Any, Any]:
    """Batched router: `(f32[T,E], i64[T,K], f32[T,K])`.

    Reference: triton_qwen36_batched_moe_router_decode (qwen36_router.py:260-319).
    """

    _require_lib()
    _router_checks(hidden, norm_weight, router_weight, top_k, batched=True)
    _router_bias_checks(router_bias, router_weight.shape[0])
    x = _dense(hidden)
    rw = _dense(router_weight)
    cmax = _chunk_max(_token_chunks(x.shape[0], top_k))
    ws = _workspace("moe", x.device, _lib.load().fk_moe_workspace_bytes(cmax, top_k, rw.shape[0], 8, 8))
    return _run_router(x, norm_weight, rw, top_k, eps, norm_offset, router_bias, ws)


def _expert_weight_checks(expert_gate_up_weight: Any, expert_down_weight: Any, hidden_size: int) -> int:
    num_experts = expert_gate_up_weight.shape[0]
    if expert_down_weight.shape[0] != num_experts:
        raise ValueError("expert gate/up and down weights must have the same number of experts")
    if expert_gate_up_weight.shape[2] != hidden_size or expert_down_weight.shape[1] != hidden_size:
        raise ValueError("expert weight hidden dimensions must match hidden")
    if expert_gate_up_weight.shape[1] % 2:
        raise ValueError("expert_gate_up_weight second dimension must be even")
    intermediate = expert_gate_up_weight.shape[1] // 2
    if expert_down_weight.shape[2] != intermediate:
        raise ValueError("expert_down_weight intermediate dimension must match gate/up weight")
    if expert_gate_up_weight.dtype != expert_down_weight.dtype:
        raise ValueError("expert gate/up and down weights must share a dtype")
    if hidden_size % 8 or intermediate % 8:
        raise ValueError("hidden_size and intermediate must be multiples of 8 for the HIP expert kernels")
    if hidden_size > 4096 or intermediate > 1024:
        raise ValueError("HIP expert kernels support hidden_size<=4096 and intermediate<=1024")
    return intermediate


def _shared_checks(shared_gate_up_weight, shared_down_weight, shared_expert_gate_weight, gu, dn, hidden_size, required):
    if shared_gate_up_weight is None or shared_down_weight is None:
        if required:
            raise ValueError("shared_gate_up_weight and shared_down_weight are required")
        return
    if not shared_gate_up_weight.is_cuda or not shared_down_weight.is_cuda:
        raise ValueError("shared expert weights must be CUDA tensors")
    if shared_gate_up_weight.shape != gu.shape[1:]:
        raise ValueError("shared_gate_up_weight must have shape [2 * intermediate, hidden_size]")
    if shared_down_weight.shape != dn.shape[1:]:
        raise ValueError("shared_down_weight must have shape [hidden_size, intermediate]")
    if shared_gate_up_weight.dtype != gu.dtype or shared_down_weight.dtype != gu.dtype:
        raise ValueError("shared expert weights must have the routed experts' dtype")
    if shared_expert_gate_weight is not None:
        if not shared_expert_gate_weight.is_cuda:
            raise ValueError("shared_expert_gate_weight must be a CUDA tensor")
        if shared_expert_gate_weight.numel() != hidden_size:
            raise ValueError("shared_expert_gate_weight must have hidden_size elements")


def _run_experts(hidden2d, gu, dn, sgu, sdn, sg, ids2d, w2d, *, layer_out=False):
    """Expert stage for `[T,H]` hidden, routing given by ids/weights (aligned
    here, in calls of at most 4096 pairs)."""

    tokens, hidden_size = hidden2d.shape
    num_experts, two_i, _ = gu.shape
    intermediate = two_i // 2
    top_k = ids2d.shape[1]
    dev = hidden2d.device
    lib = _lib.load()
    chunks = _token_chunks(tokens, top_k)
    cmax = _chunk_max(chunks)
    ws = _workspace("moe", dev, lib.fk_moe_workspace_bytes(cmax, top_k, num_experts, intermediate, hidden_size))
    stream = _stream(dev)
    ids = _dense(ids2d)
    w = _dense(w2d)
    out = torch.empty((tokens, hidden_size), device=dev, dtype=torch.float32)
    lo = torch.empty_like(out) if layer_out else None
    sgp = None if sg is None else _dense(sg)
    for s, e in chunks:
        _lib.call(
            "fk_moe_align", ids[s:e].data_ptr(), _icode(ids, "topk_ids"), w[s:e].data_ptr(), _fcode(w, "topk_weights"),
            e - s, top_k, num_experts, ws.data_ptr(), ws.numel(), None, None, None, None, stream,
        )
        _lib.call(
            "fk_moe_experts",
            hidden2d[s:e].data_ptr(), _fcode(hidden2d, "hidden"),
            gu.data_ptr(), dn.data_ptr(), _fcode(gu, "expert weights"),
            _ptr(sgu), _ptr(sdn), _ptr(sgp), _fcode(sgp, "shared_expert_gate_weight") if sgp is not None else 0,
            e - s, hidden_size, intermediate, num_experts, top_k,
            out[s:e].data_ptr(), _ptr(lo[s:e] if lo is not None else None), ws.data_ptr(), ws.numel(), stream,
        )
    return out, lo


def hip_qwen36_single_expert_mlp_decode(
    hidden: Any,
    expert_gate_up_weight: Any,
    expert_down_weight: Any,
    *,
    block_intermediate: int = 16,
    block_hidden: int = 16,
) -> Any:
    """One expert MLP for one token, f32 `[H]` (reference qwen36_expert.py:817-886)."""

    _require_lib()
    if hidden.ndim != 1:
        raise ValueError("hidden must have shape [hidden_size]")
    if expert_gate_up_weight.ndim != 2:
        raise ValueError("expert_gate_up_weight must have shape [2 * intermediate, hidden_size]")
    if expert_down_weight.ndim != 2:
        raise ValueError("expert_down_weight must have shape [hidden_size, intermediate]")
    if not hidden.is_cuda or not expert_gate_up_weight.is_cuda or not expert_down_weight.is_cuda:
        raise ValueError("hidden and expert weights must be CUDA tensors")
    hidden_size = hidden.shape[0]
    if expert_gate_up_weight.shape[1] != hidden_size or expert_down_weight.shape[0] != hidden_size:
        raise ValueError("expert weight hidden dimensions must match hidden")
    if expert_gate_up_weight.shape[0] % 2:
        raise ValueError("expert_gate_up_weight first dimension must be even")
    intermediate = expert_gate_up_weight.shape[0] // 2
    if expert_down_weight.shape[1] != intermediate:
        raise ValueError("expert_down_weight intermediate dimension must match gate/up weight")
    if hidden_size > 4096 or intermediate > 1024:
        raise ValueError("expert MLP kernel currently supports hidden_size<=4096 and intermediate<=1024")
    gu = _dense(expert_gate_up_weight).unsqueeze(0)
    dn = _dense(expert_down_weight).unsqueeze(0)
    _expert_weight_checks(gu, dn, hidden_size)
    x = _dense(hidden).reshape(1, -1)
    ids = torch.zeros((1, 1), device=x.device, dtype=torch.int32)
    w = torch.ones((1, 1), device=x.device, dtype=torch.float32)
    out, _ = _run_experts(x, gu, dn, None, None, None, ids, w)
    return out.reshape(-1)


def _routed_entry(hidden, topk_ids, topk_weights, gu_w, dn_w, sgu_w, sdn_w, sg_w, *, batched, shared, required_shared):
    _require_lib()
    if batched:
        if hidden.ndim != 2:
            raise ValueError("hidden must have shape [tokens, hidden_size]")
        if topk_ids.ndim != 2 or topk_weights.ndim != 2:
            raise ValueError("topk_ids and topk_weights must have shape [tokens, top_k]")
        if topk_ids.shape != topk_weights.shape:
            raise ValueError("topk_ids and topk_weights must have the same shape")
        if topk_ids.shape[0] != hidden.shape[0]:
            raise ValueError("topk_ids/topk_weights token dimension must match hidden")
    else:
        if hidden.ndim != 1:
            raise ValueError("hidden must have shape [hidden_size]")
        if topk_ids.ndim != 1 or topk_weights.ndim != 1:
            raise ValueError("topk_ids and topk_weights must have shape [top_k]")
        if topk_ids.shape != topk_weights.shape:
            raise ValueError("topk_ids and topk_weights must have the same shape")
    if gu_w.ndim != 3:
        raise ValueError("expert_gate_up_weight must have shape [experts, 2 * intermediate, hidden_size]")
    if dn_w.ndim != 3:
        raise ValueError("expert_down_weight must have shape [experts, hidden_size, intermediate]")
    if batched:
        tensors = [hidden, topk_ids, topk_weights, gu_w, dn_w]
        if shared and required_shared:
            tensors += [sgu_w, sdn_w]
        if not all(t is not None and t.is_cuda for t in tensors):
            raise ValueError("hidden, routing tensors, and expert weights must be CUDA tensors")
    else:
        if not hidden.is_cuda or not topk_ids.is_cuda or not topk_weights.is_cuda:
            raise ValueError("hidden, topk_ids, and topk_weights must be CUDA tensors")
        if not gu_w.is_cuda or not dn_w.is_cuda:
            raise ValueError("expert weights must be CUDA tensors")
    hidden_size = hidden.shape[-1]
    _expert_weight_checks(gu_w, dn_w, hidden_size)
    top_k = topk_ids.shape[-1]
    if top_k > 8:
        raise ValueError("routed expert path currently supports top_k <= 8")
    if shared:
        _shared_checks(sgu_w, sdn_w, sg_w, gu_w, dn_w, hidden_size, required=True)
    x = _dense(hidden).reshape(-1, hidden_size)
    ids = topk_ids.reshape(x.shape[0], top_k)
    w = topk_weights.reshape(x.shape[0], top_k)
    out, _ = _run_experts(
        x, _dense(gu_w), _dense(dn_w),
        _dense(sgu_w) if shared else None, _dense(sdn_w) if shared else None,
        sg_w if shared else None, ids, w,
    )
    return out if batched else out.reshape(-1)


def hip_qwen36_routed_experts_decode(hidden, topk_ids, topk_weights, expert_gate_up_weight, expert_down_weight):
    """Routed experts only (reference qwen36_expert.py:889-966)."""

    return _routed_entry(hidden, topk_ids, topk_weights, expert_gate_up_weight, expert_down_weight,
                         None, None, None, batched=False, shared=False, required_shared=False)


def hip_qwen36_routed_shared_experts_decode(
    hidden, topk_ids, topk_weights, expert_gate_up_weight, expert_down_weight,
    shared_gate_up_weight=None, shared_down_weight=None, shared_expert_gate_weight=None,
):
    """Routed + shared experts, one token (reference qwen36_expert.py:969-1093)."""

    return _routed_entry(hidden, topk_ids, topk_weights, expert_gate_up_weight, expert_down_weight,
                         shared_gate_up_weight, shared_down_weight, shared_expert_gate_weight,
                         batched=False, shared=True, required_shared=True)


def hip_qwen36_batched_routed_experts_decode(hidden, topk_ids, topk_weights, expert_gate_up_weight, expert_down_weight):
    """Batched routed experts only, the vLLM `fused_moe` boundary (reference qwen36_expert.py:1096-1178)."""

    return _routed_entry(hidden, topk_ids, topk_weights, expert_gate_up_weight, expert_down_weight,
                         None, None, None, batched=True, shared=False, required_shared=False)


def hip_qwen36_batched_routed_shared_experts_decode(
    hidden, topk_ids, topk_weights, expert_gate_up_weight, expert_down_weight,
    shared_gate_up_weight, shared_down_weight, shared_expert_gate_weight=None,
):
    """Batched routed + shared experts (reference qwen36_expert.py:1181-1309)."""

    return _routed_entry(hidden, topk_ids, topk_weights, expert_gate_up_weight, expert_down_weight,
                         shared_gate_up_weight, shared_down_weight, shared_expert_gate_weight,
                         batched=True, shared=True, required_shared=True)


def _moe_full(hidden2d, norm_weight, router_weight, gu_w, dn_w, sgu_w, sdn_w, sg_w, top_k, eps, norm_offset,
              router_bias, layer_out):
    hidden_size = hidden2d.shape[1]
    _router_checks(hidden2d, norm_weight, router_weight, top_k, batched=True)
    _router_bias_checks(router_bias, router_weight.shape[0])
    if gu_w.ndim != 3:
        raise ValueError("expert_gate_up_weight must have shape [experts, 2 * intermediate, hidden_size]")
    if dn_w.ndim != 3:
        raise ValueError("expert_down_weight must have shape [experts, hidden_size, intermediate]")
    tensors = (hidden2d, gu_w, dn_w, sgu_w, sdn_w)
    if not all(t is not None and t.is_cuda for t in tensors):
        raise ValueError("hidden, routing tensors, and expert weights must be CUDA tensors")
    intermediate = _expert_weight_checks(gu_w, dn_w, hidden_size)
    if router_weight.shape[0] != gu_w.shape[0]:
        raise ValueError("router_weight and expert weights disagree on the number of experts")
    _shared_checks(sgu_w, sdn_w, sg_w, gu_w, dn_w, hidden_size, required=True)
    x = _dense(hidden2d)
    tokens = x.shape[0]
    num_experts = gu_w.shape[0]
    dev = x.device
    lib = _lib.load()
    chunks = _token_chunks(tokens, top_k)
    cmax = _chunk_max(chunks)
    ws = _workspace("moe", dev, lib.fk_moe_workspace_bytes(cmax, top_k, num_experts, intermediate, hidden_size))
    rw = _dense(router_weight)
    gu, dn, sgu, sdn = _dense(gu_w), _dense(dn_w), _dense(sgu_w), _dense(sdn_w)
    nw = _dense(norm_weight)
    rb = None if router_bias is None else _dense(router_bias)
    sg = None if sg_w is None else _dense(sg_w)
    logits = torch.empty((tokens, num_experts), device=dev, dtype=torch.float32)
    ids = torch.empty((tokens, top_k), device=dev, dtype=torch.int64)
    weights = torch.empty((tokens, top_k), device=dev, dtype=torch.float32)
    out = torch.empty((tokens, hidden_size), device=dev, dtype=torch.float32)
    lo = torch.empty_like(out) if layer_out else None
    for s, e in chunks:
        _lib.call(
            "fk_moe_layer",
            x[s:e].data_ptr(), _fcode(x, "hidden"), nw.data_ptr(), _fcode(nw, "norm_weight"),
            rw.data_ptr(), _fcode(rw, "router_weight"), _ptr(rb), _fcode(rb, "router_bias") if rb is not None else 0,
            gu.data_ptr(), dn.data_ptr(), _fcode(gu, "expert weights"),
            sgu.data_ptr(), sdn.data_ptr(), _ptr(sg), _fcode(sg, "shared_expert_gate_weight") if sg is not None else 0,
            e - s, hidden_size, intermediate, num_experts, top_k, float(eps), float(norm_offset),
            logits[s:e].data_ptr(), ids[s:e].data_ptr(), weights[s:e].data_ptr(), out[s:e].data_ptr(),
            _ptr(lo[s:e] if lo is not None else None), ws.data_ptr(), ws.numel(), _stream(dev),
        )
    return out, lo, logits, ids, weights


def hip_qwen36_moe_decode(
    hidden, norm_weight, router_weight, expert_gate_up_weight, expert_down_weight,
    shared_gate_up_weight, shared_down_weight, shared_expert_gate_weight=None,
    *, top_k: int = 8, eps: float = 1e-6, router_bias: Any | None = None,
):
    """Full one-token MoE: `(out f32[H], logits, topk_ids, topk_weights)` (reference qwen36_expert.py:1312-1350)."""

    _require_lib()
    if hidden.ndim != 1:
        raise ValueError("hidden must have shape [hidden_size]")
    if norm_weight.shape != hidden.shape:
        raise ValueError("norm_weight must have the same shape as hidden")
    out, _, logits, ids, weights = _moe_full(
        hidden.reshape(1, -1), norm_weight, router_weight, expert_gate_up_weight, expert_down_weight,
        shared_gate_up_weight, shared_down_weight, shared_expert_gate_weight, top_k, eps, 1.0, router_bias, False,
    )
    return out.reshape(-1), logits.reshape(-1), ids.reshape(-1), weights.reshape(-1)


def hip_qwen36_batched_moe_decode(
    hidden, norm_weight, router_weight, expert_gate_up_weight, expert_down_weight,
    shared_gate_up_weight, shared_down_weight, shared_expert_gate_weight=None,
    *, top_k: int = 8, eps: float = 1e-6, router_bias: Any | None = None,
):
    """Batched full MoE: `(f32[T,H], f32[T,E], i64[T,K], f32[T,K])` (reference qwen36_expert.py:1353-1387)."""

    _require_lib()
    if hidden.ndim != 2:
        raise ValueError("hidden must have shape [tokens, hidden_size]")
    out, _, logits, ids, weights = _moe_full(
        hidden, norm_weight, router_weight, expert_gate_up_weight, expert_down_weight,
        shared_gate_up_weight, shared_down_weight, shared_expert_gate_weight, top_k, eps, 1.0, router_bias, False,
    )
    return out, logits, ids, weights


def hip_qwen36_batched_moe_layer_decode(
    hidden, norm_weight, router_weight, expert_gate_up_weight, expert_down_weight,
    shared_gate_up_weight, shared_down_weight, shared_expert_gate_weight=None,
    *, top_k: int = 8, eps: float = 1e-6, router_bias: Any | None = None,
):
    """MoE layer with residual: `(layer_hidden, moe_update, logits, ids, weights)` (reference qwen36_layer.py:55-106)."""

    _require_lib()
    if hidden.ndim != 2:
        raise ValueError("hidden must have shape [tokens, hidden_size]")
    if not hidden.is_cuda:
        raise ValueError("hidden must be a CUDA tensor")
    out, lo, logits, ids, weights = _moe_full(
        hidden, norm_weight, router_weight, expert_gate_up_weight, expert_down_weight,
        shared_gate_up_weight, shared_down_weight, shared_expert_gate_weight, top_k, eps, 1.0, router_bias, True,
    )
    return lo, out, logits, ids, weights


# ---------------------------------------------------------------------------
# Gated DeltaNet
# ---------------------------------------------------------------------------
def hip_qwen36_batched_deltanet_project(
    hidden, norm_weight, in_proj_qkv_weight, in_proj_z_weight, in_proj_a_weight, in_proj_b_weight,
    *, eps: float = 1e-6, norm_offset: float = 1.0, block_hidden: int = 2048,
):
    """RMSNorm(1+w) + the four input projections, f32 outputs (reference qwen36_deltanet.py:403-457)."""

    _require_lib()
    if hidden.ndim != 2:
        raise ValueError("hidden must have shape [tokens, hidden_size]")
    if norm_weight.ndim != 1 or norm_weight.shape[0] != hidden.shape[1]:
        raise ValueError("norm_weight must have shape [hidden_size]")
    weights = (in_proj_qkv_weight, in_proj_z_weight, in_proj_a_weight, in_proj_b_weight)
    for weight in weights:
        if weight.ndim != 2 or weight.shape[1] != hidden.shape[1]:
            raise ValueError("weight must have shape [out_width, hidden_size]")
    if not hidden.is_cuda or not norm_weight.is_cuda or not all(w.is_cuda for w in weights):
        raise ValueError("hidden, norm_weight, and weight must be CUDA tensors")
    tokens, hidden_size = hidden.shape
    if 1 << max(block_hidden - 1, 0).bit_length() < hidden_size:
        raise ValueError("block_hidden must be at least hidden_size")
    if in_proj_a_weight.shape[0] != in_proj_b_weight.shape[0]:
        raise ValueError("in_proj_a_weight and in_proj_b_weight must have the same number of rows")
    if len({w.dtype for w in weights}) != 1:
        raise ValueError("projection weights must share a dtype")
    x = _dense(hidden)
    nw = _dense(norm_weight)
    wq, wz, wa, wb = (_dense(w) for w in weights)
    dev = x.device
    mixed = torch.empty((tokens, wq.shape[0]), device=dev, dtype=torch.float32)
    z = torch.empty((tokens, wz.shape[0]), device=dev, dtype=torch.float32)
    a = torch.empty((tokens, wa.shape[0]), device=dev, dtype=torch.float32)
    b = torch.empty((tokens, wb.shape[0]), device=dev, dtype=torch.float32)
    if tokens == 0:
        return mixed, z, a, b
    _lib.call(
        "fk_deltanet_project",
        x.data_ptr(), _fcode(x, "hidden"), nw.data_ptr(), _fcode(nw, "norm_weight"),
        wq.data_ptr(), wz.data_ptr(), wa.data_ptr(), wb.data_ptr(), _fcode(wq, "projection weights"),
        tokens, hidden_size, wq.shape[0], wz.shape[0], wa.shape[0], float(eps), float(norm_offset),
        mixed.data_ptr(), z.data_ptr(), a.data_ptr(), b.data_ptr(), _stream(dev),
    )
    return mixed, z, a, b


def hip_qwen36_batched_deltanet_conv(mixed_qkv, conv_state, conv_weight):
    """Causal depthwise conv + SiLU + state roll (reference qwen36_deltanet.py:534-584)."""

    _require_lib()
    if mixed_qkv.ndim != 2:
        raise ValueError("mixed_qkv must have shape [tokens, channels]")
    if conv_state.ndim != 2:
        raise ValueError("conv_state must have shape [channels, kernel_size]")
    if conv_weight.ndim != 3:
        raise ValueError("conv_weight must have shape [channels, 1, kernel_size]")
    tokens, channels = mixed_qkv.shape
    if conv_state.shape[0] != channels:
        raise ValueError("mixed_qkv and conv_state disagree on channel count")
    if conv_weight.shape[0] != channels or conv_weight.shape[1] != 1 or conv_weight.shape[2] != conv_state.shape[1]:
        raise ValueError("conv_weight must have shape [channels, 1, kernel_size]")
    if not mixed_qkv.is_cuda or not conv_state.is_cuda or not conv_weight.is_cuda:
        raise ValueError("mixed_qkv, conv_state, and conv_weight must be CUDA tensors")
    if tokens < 1:
        raise ValueError("tokens must be positive")
    mixed = _dense(mixed_qkv)
    state = _dense(conv_state)
    weight = _dense(conv_weight)
    kernel_size = state.shape[1]
    conv_out = torch.empty((tokens, channels), device=mixed.device, dtype=torch.float32)
    next_state = torch.empty_like(state)
    _lib.call(
        "fk_deltanet_conv",
        mixed.data_ptr(), _fcode(mixed, "mixed_qkv"), state.data_ptr(), _fcode(state, "conv_state"),
        weight.data_ptr(), _fcode(weight, "conv_weight"), tokens, channels, kernel_size,
        conv_out.data_ptr(), next_state.data_ptr(), _stream(mixed.device),
    )
    return conv_out, next_state


def _recurrent_output(mixed_qkv, z, a_logits, b_logits, recurrent_state, out_proj_weight, linear_norm_weight,
                      a_log, dt_bias, residual, qk_heads, value_heads, head_dim, eps):
    tokens = mixed_qkv.shape[0]
    hidden_size = out_proj_weight.shape[0]
    tensors = [_dense(t) for t in (mixed_qkv, z, a_logits, b_logits, recurrent_state, out_proj_weight,
                                   linear_norm_weight, a_log, dt_bias)]
    res = None if residual is None else _dense(residual)
    names = ("mixed_qkv", "z", "a_logits", "b_logits", "recurrent_state", "out_proj_weight",
             "linear_norm_weight", "a_log", "dt_bias")
    codes = [_fcode(t, n) for t, n in zip(tensors, names)]
    codes.append(_fcode(res, "residual") if res is not None else 0)
    dtypes = (ctypes.c_int32 * 10)(*codes)
    dev = tensors[0].device
    update = torch.empty((tokens, hidden_size), device=dev, dtype=torch.float32)
    next_state = torch.empty_like(tensors[4])
    res_out = torch.empty_like(update) if res is not None else None
    lib = _lib.load()
    ws = _workspace("deltanet", dev, lib.fk_deltanet_workspace_bytes(tokens, value_heads, head_dim))
    _lib.call(
        "fk_deltanet_recurrent_output",
        *[t.data_ptr() for t in tensors], _ptr(res), ctypes.cast(dtypes, ctypes.c_void_p),
        tokens, qk_heads, value_heads, head_dim, hidden_size, float(eps),
        update.data_ptr(), next_state.data_ptr(), _ptr(res_out), ws.data_ptr(), ws.numel(), _stream(dev),
    )
    return update, next_state, res_out


def hip_qwen36_batched_deltanet_recurrent_output(
    mixed_qkv, z, a_logits, b_logits, recurrent_state, out_proj_weight, linear_norm_weight, a_log, dt_bias,
    *, qk_heads: int = 16, value_heads: int = 32, head_dim: int = 128, eps: float = 1e-6,
    block_cols: int = 8, block_value: int = 1024,
):
    """Gated delta rule + gated RMSNorm + out-proj: `(update f32[T,H], next_state)`.

    Reference: triton_qwen36_batched_deltanet_recurrent_output (qwen36_deltanet.py:744-863).
    `block_cols`/`block_value` are Triton tiling hints, accepted and ignored.
    """

    _require_lib()
    if mixed_qkv.ndim != 2:
        raise ValueError("mixed_qkv must have shape [tokens, 2*qk_width + value_width]")
    if z.ndim != 2 or a_logits.ndim != 2 or b_logits.ndim != 2:
        raise ValueError("z, a_logits, and b_logits must be batched rank-2 tensors")
    tokens, mixed_width = mixed_qkv.shape
    qk_width = qk_heads * head_dim
    value_width = value_heads * head_dim
    if mixed_width != 2 * qk_width + value_width:
        raise ValueError("mixed_qkv shape does not match qk/value head dimensions")
    if tuple(z.shape) != (tokens, value_width):
        raise ValueError("z must have shape [tokens, value_heads * head_dim]")
    if tuple(a_logits.shape) != (tokens, value_heads) or tuple(b_logits.shape) != (tokens, value_heads):
        raise ValueError("a_logits and b_logits must have shape [tokens, value_heads]")
    if tuple(recurrent_state.shape) != (value_heads, head_dim, head_dim):
        raise ValueError("recurrent_state must have shape [value_heads, head_dim, head_dim]")
    if out_proj_weight.ndim != 2 or out_proj_weight.shape[1] != value_width:
        raise ValueError("out_proj_weight must have shape [hidden_size, value_heads * head_dim]")
    if tuple(linear_norm_weight.shape) != (head_dim,):
        raise ValueError("linear_norm_weight must have shape [head_dim]")
    if tuple(a_log.shape) != (value_heads,) or tuple(dt_bias.shape) != (value_heads,):
        raise ValueError("a_log and dt_bias must have shape [value_heads]")
    tensors = (mixed_qkv, z, a_logits, b_logits, recurrent_state, out_proj_weight, linear_norm_weight, a_log, dt_bias)
    if not all(t.is_cuda for t in tensors):
        raise ValueError("all DeltaNet recurrent/output inputs must be CUDA tensors")
    if tokens < 1:
        raise ValueError("tokens must be positive")
    if value_heads % qk_heads:
        raise ValueError("value_heads must be divisible by qk_heads")
    if head_dim > 128:
        raise ValueError("HIP recurrent kernel supports head_dim <= 128")
    if value_width % 8 or value_width > 4096:
        raise ValueError("HIP output projection needs value_heads*head_dim to be a multiple of 8 and <= 4096")
    update, next_state, _ = _recurrent_output(
        mixed_qkv, z, a_logits, b_logits, recurrent_state, out_proj_weight, linear_norm_weight, a_log, dt_bias,
        None, qk_heads, value_heads, head_dim, eps,
    )
    return update, next_state


def _deltanet_step(hidden, conv_state, recurrent_state, norm_weight, w_qkv, w_z, w_a, w_b, conv1d_weight,
                   out_proj_weight, linear_norm_weight, a_log, dt_bias, qk_heads, value_heads, head_dim, eps):
    """Whole DeltaNet step + residual through fk_deltanet_step (projections with
    the conv fused in, recurrent + gated norm, out-proj)."""

    tensors = (hidden, conv_state, recurrent_state, norm_weight, w_qkv, w_z, w_a, w_b, conv1d_weight,
               out_proj_weight, linear_norm_weight, a_log, dt_bias)
    if not all(t.is_cuda for t in tensors):
        raise ValueError("all DeltaNet inputs must be CUDA tensors")
    tokens, hidden_size = hidden.shape
    key_dim, value_dim = qk_heads * head_dim, value_heads * head_dim
    conv_dim = 2 * key_dim + value_dim
    if norm_weight.ndim != 1 or norm_weight.shape[0] != hidden_size:
        raise ValueError("norm_weight must have shape [hidden_size]")
    expected = {"in_proj_qkv_weight": (w_qkv, (conv_dim, hidden_size)), "in_proj_z_weight": (w_z, (value_dim, hidden_size)),
                "in_proj_a_weight": (w_a, (value_heads, hidden_size)), "in_proj_b_weight": (w_b, (value_heads, hidden_size)),
                "out_proj_weight": (out_proj_weight, (out_proj_weight.shape[0], value_dim)),
                "recurrent_state": (recurrent_state, (value_heads, head_dim, head_dim)),
                "linear_norm_weight": (linear_norm_weight, (head_dim,)), "a_log": (a_log, (value_heads,)),
                "dt_bias": (dt_bias, (value_heads,))}
    for name, (t, shape) in expected.items():
        if tuple(t.shape) != shape:
            raise ValueError(f"{name} must have shape {list(shape)}")
    if conv_state.shape[0] != conv_dim or tuple(conv1d_weight.shape) != (conv_dim, 1, conv_state.shape[1]):
        raise ValueError("conv_state / conv1d_weight must have shapes [channels, k] / [channels, 1, k]")
    if value_heads % qk_heads:
        raise ValueError("value_heads must be divisible by qk_heads")
    if len({w_qkv.dtype, w_z.dtype, w_a.dtype, w_b.dtype}) != 1:
        raise ValueError("projection weights must share a dtype")
    x = _dense(hidden)
    ts = [_dense(t) for t in (norm_weight, w_qkv, w_z, w_a, w_b, conv_state, conv1d_weight, recurrent_state,
                              out_proj_weight, linear_norm_weight, a_log, dt_bias)]
    nw, wq, wz, wa, wb, cs, cw, rs, wo, lnw, al, dtb = ts
    codes = [_fcode(x, "hidden"), _fcode(nw, "norm_weight"), _fcode(wq, "projection weights"), _fcode(cs, "conv_state"),
             _fcode(cw, "conv1d_weight"), _fcode(rs, "recurrent_state"), _fcode(wo, "out_proj_weight"),
             _fcode(lnw, "linear_norm_weight"), _fcode(al, "a_log"), _fcode(dtb, "dt_bias")]
    dtypes = (ctypes.c_int32 * 10)(*codes)
    dev = x.device
    update = torch.empty((tokens, wo.shape[0]), device=dev, dtype=torch.float32)
    dn_hidden = torch.empty_like(update)
    next_conv = torch.empty_like(cs)
    next_rec = torch.empty_like(rs)
    lib = _lib.load()
    ws = _workspace("deltanet_step", dev, lib.fk_deltanet_step_workspace_bytes(tokens, qk_heads, value_heads, head_dim))
    _lib.call(
        "fk_deltanet_step",
        x.data_ptr(), nw.data_ptr(), wq.data_ptr(), wz.data_ptr(), wa.data_ptr(), wb.data_ptr(), cs.data_ptr(),
        cw.data_ptr(), rs.data_ptr(), wo.data_ptr(), lnw.data_ptr(), al.data_ptr(), dtb.data_ptr(),
        ctypes.cast(dtypes, ctypes.c_void_p), tokens, hidden_size, qk_heads, value_heads, head_dim, cs.shape[1],
        float(eps), update.data_ptr(), dn_hidden.data_ptr(), next_conv.data_ptr(), next_rec.data_ptr(),
        ws.data_ptr(), ws.numel(), _stream(dev),
    )
    return update, dn_hidden, next_conv, next_rec


def hip_qwen36_batched_deltanet_moe_layer_decode(
    hidden, conv_state, recurrent_state, deltanet_norm_weight, in_proj_qkv_weight, in_proj_z_weight,
    in_proj_a_weight, in_proj_b_weight, conv1d_weight, out_proj_weight, linear_norm_weight, a_log, dt_bias,
    moe_norm_weight, router_weight, expert_gate_up_weight, expert_down_weight, shared_gate_up_weight,
    shared_down_weight, shared_expert_gate_weight=None,
    *, qk_heads: int = 16, value_heads: int = 32, head_dim: int = 128, top_k: int = 8, eps: float = 1e-6,
    block_value: int = 1024, router_bias: Any | None = None,
):
    """DeltaNet -> MoE layer, returning the reference's 9-tuple
    `(layer_hidden, deltanet_hidden, deltanet_update, moe_update, conv_state,
    recurrent_state, router_logits, topk_ids, topk_weights)` (reference qwen36_layer.py:204-305)."""

    _require_lib()
    if hidden.ndim == 2 and 1 <= hidden.shape[0] <= 64 and conv_state.ndim == 2 and conv_state.shape[1] <= 8:
        dn_update, dn_hidden, next_conv, next_rec = _deltanet_step(
            hidden, conv_state, recurrent_state, deltanet_norm_weight, in_proj_qkv_weight, in_proj_z_weight,
            in_proj_a_weight, in_proj_b_weight, conv1d_weight, out_proj_weight, linear_norm_weight, a_log, dt_bias,
            qk_heads, value_heads, head_dim, eps,
        )
        layer_hidden, moe_update, logits, ids, weights = hip_qwen36_batched_moe_layer_decode(
            dn_hidden, moe_norm_weight, router_weight, expert_gate_up_weight, expert_down_weight,
            shared_gate_up_weight, shared_down_weight, shared_expert_gate_weight,
            top_k=top_k, eps=eps, router_bias=router_bias,
        )
        return layer_hidden, dn_hidden, dn_update, moe_update, next_conv, next_rec, logits, ids, weights

    mixed, z, a_l, b_l = hip_qwen36_batched_deltanet_project(
        hidden, deltanet_norm_weight, in_proj_qkv_weight, in_proj_z_weight, in_proj_a_weight, in_proj_b_weight,
        eps=eps,
    )
    mixed, next_conv = hip_qwen36_batched_deltanet_conv(mixed, conv_state, conv1d_weight)
    tokens, value_width = z.shape
    if mixed.shape[1] != 2 * qk_heads * head_dim + value_heads * head_dim:
        raise ValueError("mixed_qkv shape does not match qk/value head dimensions")
    if tuple(recurrent_state.shape) != (value_heads, head_dim, head_dim):
        raise ValueError("recurrent_state must have shape [value_heads, head_dim, head_dim]")
    if not all(t.is_cuda for t in (recurrent_state, out_proj_weight, linear_norm_weight, a_log, dt_bias)):
        raise ValueError("all DeltaNet recurrent/output inputs must be CUDA tensors")
    if value_heads % qk_heads:
        raise ValueError("value_heads must be divisible by qk_heads")
    dn_update, next_rec, dn_hidden = _recurrent_output(
        mixed, z, a_l, b_l, recurrent_state, out_proj_weight, linear_norm_weight, a_log, dt_bias,
        hidden, qk_heads, value_heads, head_dim, eps,
    )
    layer_hidden, moe_update, logits, ids, weights = hip_qwen36_batched_moe_layer_decode(
        dn_hidden, moe_norm_weight, router_weight, expert_gate_up_weight, expert_down_weight,
        shared_gate_up_weight, shared_down_weight, shared_expert_gate_weight,
        top_k=top_k, eps=eps, router_bias=router_bias,
    )
    return layer_hidden, dn_hidden, dn_update, moe_update, next_conv, next_rec, logits, ids, weights


# ---------------------------------------------------------------------------
# Gated full attention
# ---------------------------------------------------------------------------
def hip_qwen36_batched_attention_project(
    hidden, norm_weight, q_proj_weight, k_proj_weight, v_proj_weight,
    *, eps: float = 1e-6, norm_offset: float = 1.0, block_hidden: int = 2048,
):
    """RMSNorm(1+w) + the Q (query/gate pairs), K and V projections, f32
    outputs (reference qwen36_attention.py:168-211)."""

    _require_lib()
    if hidden.ndim != 2:
        raise ValueError("hidden must have shape [tokens, hidden_size]")
    if norm_weight.ndim != 1 or norm_weight.shape[0] != hidden.shape[1]:
        raise ValueError("norm_weight must have shape [hidden_size]")
    weights = (q_proj_weight, k_proj_weight, v_proj_weight)
    for weight in weights:
        if weight.ndim != 2 or weight.shape[1] != hidden.shape[1]:
            raise ValueError("weight must have shape [out_width, hidden_size]")
    if not hidden.is_cuda or not norm_weight.is_cuda or not all(w.is_cuda for w in weights):
        raise ValueError("hidden, norm_weight, and weight must be CUDA tensors")
    tokens, hidden_size = hidden.shape
    if 1 << max(block_hidden - 1, 0).bit_length() < hidden_size:
        raise ValueError("block_hidden must be at least hidden_size")
    if k_proj_weight.shape != v_proj_weight.shape:
        raise ValueError("k_proj_weight and v_proj_weight must have the same shape")
    if len({w.dtype for w in weights}) != 1:
        raise ValueError("projection weights must share a dtype")
    x, nw = _dense(hidden), _dense(norm_weight)
    wq, wk, wv = (_dense(w) for w in weights)
    dev = x.device
    q = torch.empty((tokens, wq.shape[0]), device=dev, dtype=torch.float32)
    k = torch.empty((tokens, wk.shape[0]), device=dev, dtype=torch.float32)
    v = torch.empty((tokens, wv.shape[0]), device=dev, dtype=torch.float32)
    if tokens == 0:
        return q, k, v
    _lib.call(
        "fk_attention_project",
        x.data_ptr(), _fcode(x, "hidden"), nw.data_ptr(), _fcode(nw, "norm_weight"),
        wq.data_ptr(), wk.data_ptr(), wv.data_ptr(), _fcode(wq, "projection weights"),
        tokens, hidden_size, wq.shape[0], wk.shape[0], float(eps), float(norm_offset),
        q.data_ptr(), k.data_ptr(), v.data_ptr(), _stream(dev),
    )
    return q, k, v


_MAX_ATTN_ROWS = 32  # rows per fk_attention_decode call (fk_attention.hip kAttnMaxTokens)


def _attention(hidden, key_cache, value_cache, norm_weight, q_proj_weight, k_proj_weight, v_proj_weight,
               out_proj_weight, q_norm_weight, k_norm_weight, start_position, attention_heads, kv_heads, head_dim,
               rope_dim, rope_theta, eps, qk_norm_eps, copy_cache, rope_interleaved, residual):
    if hidden.ndim != 2:
        raise ValueError("hidden must have shape [tokens, hidden_size]")
    if key_cache.ndim != 3 or value_cache.ndim != 3:
        raise ValueError("key/value caches must have shape [positions, kv_heads, head_dim]")
    if key_cache.shape != value_cache.shape:
        raise ValueError("key and value caches must have the same shape")
    if tuple(key_cache.shape[1:]) != (kv_heads, head_dim):
        raise ValueError("cache shape does not match kv_heads/head_dim")
    if not all(t.is_cuda for t in (hidden, key_cache, value_cache)):
        raise ValueError("hidden and caches must be CUDA tensors")
    if start_position < 0 or start_position + hidden.shape[0] > key_cache.shape[0]:
        raise ValueError("decode positions exceed cache length")
    q_width, kv_width = attention_heads * head_dim, kv_heads * head_dim
    hidden_size = hidden.shape[1]
    if out_proj_weight.ndim != 2 or out_proj_weight.shape[1] != q_width:
        raise ValueError("out_proj_weight must have shape [hidden_size, attention_heads * head_dim]")
    if q_proj_weight.ndim != 2 or q_proj_weight.shape[0] < 2 * q_width or q_proj_weight.shape[1] != hidden_size:
        raise ValueError("q_proj_weight must have at least 2 * attention_heads * head_dim rows")
    if tuple(k_proj_weight.shape) != (kv_width, hidden_size) or tuple(v_proj_weight.shape) != (kv_width, hidden_size):
        raise ValueError("k/v projection weights must have shape [kv_heads * head_dim, hidden_size]")
    if out_proj_weight.shape[0] != hidden_size:
        raise ValueError("out_proj_weight must have hidden_size rows")
    if key_cache.dtype != value_cache.dtype:
        raise ValueError("key and value caches must share a dtype")
    if len({w.dtype for w in (q_proj_weight, k_proj_weight, v_proj_weight, out_proj_weight)}) != 1:
        raise ValueError("projection weights must share a dtype")
    if q_norm_weight.dtype != k_norm_weight.dtype or q_norm_weight.numel() != head_dim or k_norm_weight.numel() != head_dim:
        raise ValueError("q_norm_weight and k_norm_weight must have head_dim elements and share a dtype")
    x = _dense(hidden)
    tokens = x.shape[0]
    kc = key_cache.clone() if copy_cache else key_cache
    vc = value_cache.clone() if copy_cache else value_cache
    if not kc.is_contiguous() or not vc.is_contiguous():
        raise ValueError("key/value caches must be contiguous when updated in place")
    # the query rows past 2 * q_width (if any) are not used
    wq = _dense(q_proj_weight[: 2 * q_width])
    wk, wv, wo = _dense(k_proj_weight), _dense(v_proj_weight), _dense(out_proj_weight)
    nw, qn, kn = _dense(norm_weight), _dense(q_norm_weight), _dense(k_norm_weight)
    dev = x.device
    update = torch.empty((tokens, hidden_size), device=dev, dtype=torch.float32)
    out = torch.empty_like(update) if residual else None
    # The C ABI decodes at most _MAX_ATTN_ROWS rows per call (their new keys
    # sit in LDS); longer batches go through in consecutive calls: each call
    # writes its rows' keys and values into the cache before the next one
    # reads them, which is the causal order one call keeps.
    # No rows: no call (the caches are returned as given, or copied).
    step = _MAX_ATTN_ROWS
    nbytes = _lib.load().fk_attention_workspace_bytes(min(max(tokens, 1), step), attention_heads, kv_heads, head_dim)
    ws = _workspace("attention", dev, nbytes)
    for s in range(0, tokens, step):
        e = min(tokens, s + step)
        _lib.call(
            "fk_attention_decode",
            x[s:e].data_ptr(), _fcode(x, "hidden"), nw.data_ptr(), _fcode(nw, "norm_weight"),
            wq.data_ptr(), wk.data_ptr(), wv.data_ptr(), wo.data_ptr(), _fcode(wq, "projection weights"),
            qn.data_ptr(), kn.data_ptr(), _fcode(qn, "q_norm_weight"),
            kc.data_ptr(), vc.data_ptr(), _fcode(kc, "key_cache"), kc.shape[0], int(start_position) + s, None,
            e - s, hidden_size, attention_heads, kv_heads, head_dim, int(rope_dim), float(rope_theta),
            1 if rope_interleaved else 0, float(eps), float(qk_norm_eps),
            update[s:e].data_ptr(), _ptr(out[s:e] if out is not None else None), ws.data_ptr(), ws.numel(), _stream(dev),
        )
    return update, out, kc, vc


def hip_qwen36_batched_attention_decode(
    hidden, key_cache, value_cache, norm_weight, q_proj_weight, k_proj_weight, v_proj_weight, out_proj_weight,
    q_norm_weight, k_norm_weight,
    *, start_position: int = 0, attention_heads: int = 16, kv_heads: int = 2, head_dim: int = 256,
    rope_dim: int = 64, rope_theta: float = 10000.0, eps: float = 1e-6, qk_norm_eps: float = 1e-6,
    block_hidden: int = 2048, copy_cache: bool = True, rope_interleaved: bool = True,
):
    """Gated full-attention decode of `tokens` rows at positions
    start_position.. through the KV cache: `(update, key_cache, value_cache)`
    (reference qwen36_attention.py:448-577).  RoPE pairs are interleaved
    (2i, 2i+1) like the reference entry point; `rope_interleaved=False`
    rotates halves (i, i + rope_dim/2) like the reference's torch oracle.
    With copy_cache=False the caches are updated in place."""

    _require_lib()
    update, _, kc, vc = _attention(
        hidden, key_cache, value_cache, norm_weight, q_proj_weight, k_proj_weight, v_proj_weight, out_proj_weight,
        q_norm_weight, k_norm_weight, start_position, attention_heads, kv_heads, head_dim, rope_dim, rope_theta,
        eps, qk_norm_eps, copy_cache, rope_interleaved, False,
    )
    return update, kc, vc


def hip_qwen36_batched_attention_moe_layer_decode(
    hidden, key_cache, value_cache, attention_norm_weight, q_proj_weight, k_proj_weight, v_proj_weight,
    out_proj_weight, q_norm_weight, k_norm_weight, moe_norm_weight, router_weight, expert_gate_up_weight,
    expert_down_weight, shared_gate_up_weight, shared_down_weight, shared_expert_gate_weight=None,
    *, start_position: int = 0, attention_heads: int = 16, kv_heads: int = 2, head_dim: int = 256,
    rope_dim: int = 64, rope_theta: float = 10000.0, top_k: int = 8, eps: float = 1e-6,
    qk_norm_eps: float = 1e-6, copy_cache: bool = True, rope_interleaved: bool = True,
    router_bias: Any | None = None,
):
    """Attention -> MoE layer, returning the reference's 9-tuple
    `(layer_hidden, attention_hidden, attention_update, moe_update, key_cache,
    value_cache, router_logits, topk_ids, topk_weights)` (reference
    qwen36_layer.py:109-201); the residual add is fused into the attention
    output projection."""

    _require_lib()
    update, attn_hidden, kc, vc = _attention(
        hidden, key_cache, value_cache, attention_norm_weight, q_proj_weight, k_proj_weight, v_proj_weight,
        out_proj_weight, q_norm_weight, k_norm_weight, start_position, attention_heads, kv_heads, head_dim,
        rope_dim, rope_theta, eps, qk_norm_eps, copy_cache, rope_interleaved, True,
    )
    layer_hidden, moe_update, logits, ids, weights = hip_qwen36_batched_moe_layer_decode(
        attn_hidden, moe_norm_weight, router_weight, expert_gate_up_weight, expert_down_weight,
        shared_gate_up_weight, shared_down_weight, shared_expert_gate_weight,
        top_k=top_k, eps=eps, router_bias=router_bias,
    )
    return layer_hidden, attn_hidden, update, moe_update, kc, vc, logits, ids, weights


# ---------------------------------------------------------------------------
# Synthetic (tiny-spec) blocks
# ---------------------------------------------------------------------------
def hip_synthetic_qwen36_moe_decode(
    hidden, norm_weight, router_weight, expert_gate_up_weight, expert_down_weight,
    shared_gate_up_weight, shared_down_weight, *, top_k: int, eps: float = 1e-6,
):
    """One-token synthetic MoE incl. residual, output in hidden's dtype (reference qwen36_moe.py:362-444)."""

    _require_lib()
    if top_k < 1 or top_k > 8:
        raise ValueError("prototype synthetic Qwen3.6 MoE kernel supports 1 <= top_k <= 8")
    if hidden.ndim != 1:
        raise ValueError("hidden must have shape [hidden_size]")
    if not hidden.is_cuda:
        raise ValueError("hidden must be a CUDA tensor")
    if expert_gate_up_weight.ndim != 3:
        raise ValueError("expert_gate_up_weight must have shape [experts, 2 * intermediate, hidden]")
    if expert_down_weight.ndim != 3:
        raise ValueError("expert_down_weight must have shape [experts, hidden, intermediate]")
    hidden_size = hidden.shape[0]
    num_experts = router_weight.shape[0]
    intermediate = expert_down_weight.shape[2]
    if hidden_size > 128 or intermediate > 128 or num_experts > 256:
        raise ValueError("prototype synthetic Qwen3.6 MoE kernel supports hidden/intermediate<=128 and experts<=256")
    if top_k > num_experts:
        raise ValueError("top_k must be <= number of experts")
    ws = [_dense(t) for t in (norm_weight, router_weight, expert_gate_up_weight, expert_down_weight,
                              shared_gate_up_weight, shared_down_weight)]
    if len({t.dtype for t in ws}) != 1:
        raise ValueError("synthetic MoE weights must share a dtype")
    x = _dense(hidden)
    out = torch.empty_like(x)
    _lib.call(
        "fk_synthetic_moe",
        x.data_ptr(), _fcode(x, "hidden"), *[t.data_ptr() for t in ws], _fcode(ws[0], "weights"),
        hidden_size, num_experts, intermediate, top_k, float(eps), out.data_ptr(), _fcode(out, "out"),
        _stream(x.device),
    )
    return out


def hip_synthetic_qwen36_deltanet_decode(
    hidden, state, norm_weight, q_weight, k_weight, v_weight, gate_weight, out_weight,
    *, qk_heads: int, head_dim: int, value_dim_per_head: int, eps: float = 1e-6,
):
    """One-token toy DeltaNet: `(hidden', state')` (reference qwen36_deltanet.py:966-1041)."""

    _require_lib()
    if hidden.ndim != 1:
        raise ValueError("hidden must have shape [hidden_size]")
    if state.ndim != 3:
        raise ValueError("state must have shape [qk_heads, head_dim, value_dim_per_head]")
    if not hidden.is_cuda or not state.is_cuda:
        raise ValueError("hidden and state must be CUDA tensors")
    if tuple(state.shape) != (qk_heads, head_dim, value_dim_per_head):
        raise ValueError("state shape does not match qk_heads/head_dim/value_dim_per_head")
    ws = [_dense(t) for t in (norm_weight, q_weight, k_weight, v_weight, gate_weight, out_weight)]
    if len({t.dtype for t in ws}) != 1:
        raise ValueError("synthetic DeltaNet weights must share a dtype")
    x = _dense(hidden)
    s = _dense(state)
    x_out = torch.empty_like(x)
    s_out = torch.empty_like(s)
    _lib.call(
        "fk_synthetic_deltanet",
        x.data_ptr(), _fcode(x, "hidden"), s.data_ptr(), _fcode(s, "state"), *[t.data_ptr() for t in ws],
        _fcode(ws[0], "weights"), x.shape[0], qk_heads, head_dim, value_dim_per_head, float(eps),
        x_out.data_ptr(), s_out.data_ptr(), _stream(x.device),
    )
    return x_out, s_out


def hip_synthetic_qwen36_deltanet_moe_decode(hidden, state, layer, *, qk_heads, head_dim, value_dim_per_head, top_k):
    """Synthetic DeltaNet -> MoE layer (reference qwen36_layer.py:308-343)."""

    hidden, next_state = hip_synthetic_qwen36_deltanet_decode(
        hidden, state, layer["norm_weight"], layer["q_weight"], layer["k_weight"], layer["v_weight"],
        layer["gate_weight"], layer["out_weight"],
        qk_heads=qk_heads, head_dim=head_dim, value_dim_per_head=value_dim_per_head,
    )
    hidden = hip_synthetic_qwen36_moe_decode(
        hidden, layer["norm_weight"], layer["router_weight"], layer["expert_gate_up_weight"],
        layer["expert_down_weight"], layer["shared_gate_up_weight"], layer["shared_down_weight"], top_k=top_k,
    )
    return hidden, next_state


def hip_synthetic_qwen36_attention_decode(
    hidden, key_cache, value_cache, norm_weight, q_weight, k_weight, v_weight, out_weight,
    *, position: int, attention_heads: int, kv_heads: int, head_dim: int, rope_dim: int, eps: float = 1e-6,
    fuse_project_rope: bool = False, copy_cache: bool = True,
):
    """One-token synthetic grouped-query attention: `(hidden', key_cache', value_cache')`
    (reference qwen36_attention.py:852-998).  `copy_cache=False` updates the
    caches in place and returns them; `fuse_project_rope` selects a launch
    shape in the reference and changes nothing here (one launch either way)."""

    _require_lib()
    if hidden.ndim != 1:
        raise ValueError("hidden must have shape [hidden_size]")
    if key_cache.ndim != 3 or value_cache.ndim != 3:
        raise ValueError("key/value caches must have shape [positions, kv_heads, head_dim]")
    if not hidden.is_cuda or not key_cache.is_cuda or not value_cache.is_cuda:
        raise ValueError("hidden and caches must be CUDA tensors")
    if key_cache.shape != value_cache.shape:
        raise ValueError("key and value caches must have the same shape")
    if tuple(key_cache.shape[1:]) != (kv_heads, head_dim):
        raise ValueError("cache shape does not match kv_heads/head_dim")
    if position >= key_cache.shape[0]:
        raise ValueError("position exceeds cache length")
    hidden_size = hidden.shape[0]
    q_width, kv_width, max_positions = attention_heads * head_dim, kv_heads * head_dim, key_cache.shape[0]
    if hidden_size > 128 or q_width > 128 or kv_width > 128 or max_positions > 128:
        raise ValueError("prototype synthetic Qwen3.6 attention kernel only supports tiny synthetic shapes")
    if position < 0:
        raise ValueError("position must be >= 0")
    if attention_heads % kv_heads != 0:
        raise ValueError("attention_heads must be a multiple of kv_heads")
    if key_cache.dtype != value_cache.dtype:
        raise ValueError("key and value caches must share a dtype")
    ws = [_dense(t) for t in (norm_weight, q_weight, k_weight, v_weight, out_weight)]
    if len({t.dtype for t in ws}) != 1:
        raise ValueError("synthetic attention weights must share a dtype")
    x = _dense(hidden)
    if copy_cache:
        kc, vc = key_cache.clone(), value_cache.clone()
    else:
        if not key_cache.is_contiguous() or not value_cache.is_contiguous():
            raise ValueError("copy_cache=False needs contiguous caches")
        kc, vc = key_cache, value_cache
    out = torch.empty_like(x)
    _lib.call(
        "fk_synthetic_attention",
        x.data_ptr(), _fcode(x, "hidden"), kc.data_ptr(), vc.data_ptr(), _fcode(kc, "key_cache"),
        *[t.data_ptr() for t in ws], _fcode(ws[0], "weights"), hidden_size, attention_heads, kv_heads, head_dim,
        rope_dim, position, max_positions, float(eps), out.data_ptr(), _stream(x.device),
    )
    return out, kc, vc


def hip_synthetic_qwen36_attention_moe_decode(
    hidden, key_cache, value_cache, layer, *, position: int, attention_heads: int, kv_heads: int, head_dim: int,
    rope_dim: int, top_k: int, copy_cache: bool = True,
):
    """Synthetic Attention -> MoE layer (reference qwen36_layer.py:346-384)."""

    hidden, next_key_cache, next_value_cache = hip_synthetic_qwen36_attention_decode(
        hidden, key_cache, value_cache, layer["norm_weight"], layer["q_weight"], layer["k_weight"],
        layer["v_weight"], layer["out_weight"], position=position, attention_heads=attention_heads,
        kv_heads=kv_heads, head_dim=head_dim, rope_dim=rope_dim, copy_cache=copy_cache,
    )
    hidden = hip_synthetic_qwen36_moe_decode(
        hidden, layer["norm_weight"], layer["router_weight"], layer["expert_gate_up_weight"],
        layer["expert_down_weight"], layer["shared_gate_up_weight"], layer["shared_down_weight"], top_k=top_k,
    )
    return hidden, next_key_cache, next_value_cache


# Reference name -> HIP implementation, for import-level drop-in switching.
TRITON_ALIASES = {
    "triton_" + name[len("hip_"):]: globals()[name]
    for name in __all__
    if name.startswith("hip_") and name != "hip_qwen36_moe_align"
}
globals().update(TRITON_ALIASES)
