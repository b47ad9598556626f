"""Preallocated decode-step plans over the C ABI.

A plan owns every buffer a step touches (inputs, outputs, workspace), so a
step is one or a few C-ABI calls with no torch allocation and no host sync.
That makes steps cheap to issue from a serving loop and capturable in a HIP
graph (torch.cuda.CUDAGraph), which is how bench.py times them.

  MoeLayerPlan      router + top-k + routing tables + experts + residual
                    (fk_moe_layer), or its two stages separately.
  DeltaNetStepPlan  projections + conv -> recurrent/gated-norm -> out-proj
                    (+ residual) through fk_deltanet_step, writing the next
                    conv / recurrent states.
  AttentionStepPlan gated full attention (+ residual) through
                    fk_attention_decode at a device-held position that the
                    step advances itself, with the KV
                    caches it owns updated in place.
"""

from __future__ import annotations

import ctypes
from typing import Any

import torch

from . import _lib
from .kernels.hip import _dense, _fcode
from .spec import Qwen36A3BSpec, qwen36_35b_a3b_spec


def _stream_handle(stream: torch.cuda.Stream | None, device: torch.device) -> int:
    s = stream if stream is not None else torch.cuda.current_stream(device)
    return s.cuda_stream


def _check_device(workspace: torch.Tensor, device: torch.device, stream: torch.cuda.Stream | None) -> None:
    """Raise FastKernelsError (FK_ERR_DEVICE) if a bounded in-kernel wait of
    an earlier step on this workspace ran out; clears the flag.  Synchronises
    the stream, so call it outside timed or captured regions."""

    _lib.call("fk_workspace_status", workspace.data_ptr(), workspace.numel(), 1, _stream_handle(stream, device))


def _set_poll_limit(workspace: torch.Tensor, device: torch.device, limit: int | None,
                    stream: torch.cuda.Stream | None) -> None:
    """Bound every in-kernel wait of later steps to `limit` poll rounds
    (stream-ordered; None restores the built-in bound, 0 makes every wait
    give up at once: flagged NaN outputs, every kernel still ends)."""

    _lib.call("fk_workspace_set_poll_limit", workspace.data_ptr(), workspace.numel(),
              -1 if limit is None else int(limit), _stream_handle(stream, device))


class MoeLayerPlan:
    """One MoE layer (router + experts + residual) at a fixed token count."""

    def __init__(
        self,
        weights: dict[str, Any],
        tokens: int,
        *,
        top_k: int = 8,
        eps: float = 1e-6,
        norm_offset: float = 1.0,
        router_bias: Any | None = None,
        hidden: torch.Tensor | None = None,
        hidden_dtype: torch.dtype = torch.bfloat16,
    ) -> None:
        self.lib = _lib.load()
        if hasattr(weights, "as_dict"):  # packed checkpoint tensors (weights.Qwen36MoEWeights)
            weights = weights.as_dict()
        w = {k: (None if v is None else _dense(v)) for k, v in weights.items()}
        self.w = w
        gu = w["expert_gate_up_weight"]
        self.device = gu.device
        self.num_experts, two_i, self.hidden_size = gu.shape
        self.intermediate = two_i // 2
        self.tokens = tokens
        self.top_k = top_k
        self.eps = float(eps)
        self.norm_offset = float(norm_offset)
        self.router_bias = None if router_bias is None else _dense(router_bias)
        dev = self.device
        self.hidden = hidden if hidden is not None else torch.zeros((tokens, self.hidden_size), dtype=hidden_dtype, device=dev)
        self.logits = torch.empty((tokens, self.num_experts), dtype=torch.float32, device=dev)
        self.ids = torch.empty((tokens, top_k), dtype=torch.int64, device=dev)
        self.weights = torch.empty((tokens, top_k), dtype=torch.float32, device=dev)
        self.moe_out = torch.empty((tokens, self.hidden_size), dtype=torch.float32, device=dev)
        self.layer_out = torch.empty_like(self.moe_out)
        nbytes = self.lib.fk_moe_workspace_bytes(tokens, top_k, self.num_experts, self.intermediate, self.hidden_size)
        self.workspace = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        sg = w.get("shared_expert_gate_weight")
        self._sg = sg
        self._sg_code = _fcode(sg, "shared_expert_gate_weight") if sg is not None else 0

    # The three entry points -------------------------------------------------
    def run(self, stream: torch.cuda.Stream | None = None) -> None:
        w = self.w
        rb = self.router_bias
        _lib.call(
            "fk_moe_layer",
            self.hidden.data_ptr(), _fcode(self.hidden, "hidden"),
            w["norm_weight"].data_ptr(), _fcode(w["norm_weight"], "norm_weight"),
            w["router_weight"].data_ptr(), _fcode(w["router_weight"], "router_weight"),
            None if rb is None else rb.data_ptr(), 0 if rb is None else _fcode(rb, "router_bias"),
            w["expert_gate_up_weight"].data_ptr(), w["expert_down_weight"].data_ptr(),
            _fcode(w["expert_gate_up_weight"], "experts"),
            w["shared_gate_up_weight"].data_ptr(), w["shared_down_weight"].data_ptr(),
            None if self._sg is None else self._sg.data_ptr(), self._sg_code,
            self.tokens, self.hidden_size, self.intermediate, self.num_experts, self.top_k,
            self.eps, self.norm_offset,
            self.logits.data_ptr(), self.ids.data_ptr(), self.weights.data_ptr(),
            self.moe_out.data_ptr(), self.layer_out.data_ptr(),
            self.workspace.data_ptr(), self.workspace.numel(), _stream_handle(stream, self.device),
        )

    def run_router(self, stream: torch.cuda.Stream | None = None) -> None:
        w = self.w
        rb = self.router_bias
        _lib.call(
            "fk_moe_router",
            self.hidden.data_ptr(), _fcode(self.hidden, "hidden"),
            w["norm_weight"].data_ptr(), _fcode(w["norm_weight"], "norm_weight"),
            w["router_weight"].data_ptr(), _fcode(w["router_weight"], "router_weight"),
            None if rb is None else rb.data_ptr(), 0 if rb is None else _fcode(rb, "router_bias"),
            self.tokens, self.hidden_size, self.num_experts, self.top_k, self.eps, self.norm_offset,
            self.logits.data_ptr(), self.ids.data_ptr(), self.weights.data_ptr(),
            self.workspace.data_ptr(), self.workspace.numel(), _stream_handle(stream, self.device),
        )

    def run_experts(self, stream: torch.cuda.Stream | None = None) -> None:
        """Expert stage for the routing tables left in the workspace by the
        last `run`/`run_router` of this plan."""

        w = self.w
        _lib.call(
            "fk_moe_experts",
            self.hidden.data_ptr(), _fcode(self.hidden, "hidden"),
            w["expert_gate_up_weight"].data_ptr(), w["expert_down_weight"].data_ptr(),
            _fcode(w["expert_gate_up_weight"], "experts"),
            w["shared_gate_up_weight"].data_ptr(), w["shared_down_weight"].data_ptr(),
            None if self._sg is None else self._sg.data_ptr(), self._sg_code,
            self.tokens, self.hidden_size, self.intermediate, self.num_experts, self.top_k,
            self.moe_out.data_ptr(), self.layer_out.data_ptr(),
            self.workspace.data_ptr(), self.workspace.numel(), _stream_handle(stream, self.device),
        )

    def check_device(self, stream: torch.cuda.Stream | None = None) -> None:
        _check_device(self.workspace, self.device, stream)

    def set_poll_limit(self, limit: int | None, stream: torch.cuda.Stream | None = None) -> None:
        _set_poll_limit(self.workspace, self.device, limit, stream)


class DeltaNetStepPlan:
    """One Gated DeltaNet decode step (T rows through one state) + residual,
    issued as one C-ABI call, fk_deltanet_step (one launch at the model's
    shapes and dtypes)."""

    def __init__(
        self,
        weights: dict[str, Any],
        tokens: int,
        spec: Qwen36A3BSpec | None = None,
        *,
        eps: float = 1e-6,
        hidden: torch.Tensor | None = None,
        hidden_dtype: torch.dtype = torch.bfloat16,
    ) -> None:
        self.lib = _lib.load()
        spec = spec or qwen36_35b_a3b_spec()
        self.spec = spec
        w = {k: _dense(v) for k, v in weights.items()}
        self.w = w
        dev = w["in_proj_qkv_weight"].device
        self.device = dev
        self.tokens = tokens
        self.eps = float(eps)
        H = spec.hidden_size
        self.hidden = hidden if hidden is not None else torch.zeros((tokens, H), dtype=hidden_dtype, device=dev)
        self.next_conv_state = torch.empty_like(w["conv_state"])
        self.next_recurrent_state = torch.empty_like(w["recurrent_state"])
        self.update = torch.empty((tokens, H), dtype=torch.float32, device=dev)
        self.hidden_out = torch.empty_like(self.update)
        nbytes = self.lib.fk_deltanet_step_workspace_bytes(
            tokens, spec.deltanet_qk_heads, spec.deltanet_value_heads, spec.deltanet_head_dim
        )
        self.workspace = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        order = ("input_norm_weight", "in_proj_qkv_weight", "conv_state", "conv1d_weight", "recurrent_state",
                 "out_proj_weight", "linear_norm_weight", "a_log", "dt_bias")
        codes = [_fcode(self.hidden, "hidden")] + [_fcode(w[k], k) for k in order]
        for k in ("in_proj_z_weight", "in_proj_a_weight", "in_proj_b_weight"):
            if w[k].dtype != w["in_proj_qkv_weight"].dtype:
                raise ValueError("projection weights must share a dtype")
        self._dtypes = (ctypes.c_int32 * 10)(*codes)

    def run(self, stream: torch.cuda.Stream | None = None) -> None:
        w, sp = self.w, self.spec
        _lib.call(
            "fk_deltanet_step",
            self.hidden.data_ptr(), w["input_norm_weight"].data_ptr(),
            w["in_proj_qkv_weight"].data_ptr(), w["in_proj_z_weight"].data_ptr(),
            w["in_proj_a_weight"].data_ptr(), w["in_proj_b_weight"].data_ptr(),
            w["conv_state"].data_ptr(), w["conv1d_weight"].data_ptr(), w["recurrent_state"].data_ptr(),
            w["out_proj_weight"].data_ptr(), w["linear_norm_weight"].data_ptr(), w["a_log"].data_ptr(),
            w["dt_bias"].data_ptr(), ctypes.cast(self._dtypes, ctypes.c_void_p),
            self.tokens, sp.hidden_size, sp.deltanet_qk_heads, sp.deltanet_value_heads, sp.deltanet_head_dim,
            w["conv_state"].shape[1], self.eps,
            self.update.data_ptr(), self.hidden_out.data_ptr(), self.next_conv_state.data_ptr(),
            self.next_recurrent_state.data_ptr(), self.workspace.data_ptr(), self.workspace.numel(),
            _stream_handle(stream, self.device),
        )

    def check_device(self, stream: torch.cuda.Stream | None = None) -> None:
        _check_device(self.workspace, self.device, stream)

    def set_poll_limit(self, limit: int | None, stream: torch.cuda.Stream | None = None) -> None:
        _set_poll_limit(self.workspace, self.device, limit, stream)


class AttentionStepPlan:
    """One gated full-attention decode step of `tokens` rows + residual.

    The plan owns the KV caches ([max_positions, kv_heads, head_dim]) and a
    device int32 `position`; every run decodes at that position and advances
    it by `tokens` once every workgroup has read it, so a step captured once
    in a HIP graph decodes successive positions on replay.  `set_position()`
    rewinds it.
    """

    def __init__(
        self,
        weights: Any,
        tokens: int,
        spec: Qwen36A3BSpec | None = None,
        *,
        max_positions: int,
        cache_dtype: torch.dtype = torch.float32,
        start_position: int = 0,
        eps: float = 1e-6,
        rope_interleaved: bool = True,
        hidden: torch.Tensor | None = None,
        hidden_dtype: torch.dtype = torch.bfloat16,
    ) -> None:
        self.lib = _lib.load()
        if hasattr(weights, "as_dict"):
            weights = weights.as_dict()
        spec = spec or qwen36_35b_a3b_spec()
        self.spec = spec
        w = {k: _dense(v) for k, v in weights.items() if v is not None}
        self.w = w
        dev = w["q_proj_weight"].device
        self.device = dev
        self.tokens = tokens
        self.eps = float(eps)
        self.interleaved = 1 if rope_interleaved else 0
        H, heads, kvh, hd = spec.hidden_size, spec.attention_heads, spec.attention_kv_heads, spec.attention_head_dim
        qw = heads * hd
        if w["q_proj_weight"].shape[0] < 2 * qw:
            raise ValueError("q_proj_weight must have at least 2 * attention_heads * head_dim rows")
        self._wq = w["q_proj_weight"][: 2 * qw]
        self.max_positions = max_positions
        self.hidden = hidden if hidden is not None else torch.zeros((tokens, H), dtype=hidden_dtype, device=dev)
        self.key_cache = torch.zeros((max_positions, kvh, hd), dtype=cache_dtype, device=dev)
        self.value_cache = torch.zeros_like(self.key_cache)
        self.position = torch.tensor([start_position], dtype=torch.int32, device=dev)
        self.update = torch.empty((tokens, H), dtype=torch.float32, device=dev)
        self.hidden_out = torch.empty_like(self.update)
        nbytes = self.lib.fk_attention_workspace_bytes(tokens, heads, kvh, hd)
        self.workspace = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        self._codes = (_fcode(self.hidden, "hidden"), _fcode(w["input_norm_weight"], "input_norm_weight"),
                       _fcode(self._wq, "q_proj_weight"), _fcode(w["q_norm_weight"], "q_norm_weight"),
                       _fcode(self.key_cache, "key_cache"))

    def set_position(self, position: int) -> None:
        self.position.fill_(int(position))

    def run(self, stream: torch.cuda.Stream | None = None) -> None:
        w, sp = self.w, self.spec
        s = _stream_handle(stream, self.device)
        hc, nc, wc, qc, cc = self._codes
        _lib.call(
            "fk_attention_decode",
            self.hidden.data_ptr(), hc, w["input_norm_weight"].data_ptr(), nc,
            self._wq.data_ptr(), w["k_proj_weight"].data_ptr(), w["v_proj_weight"].data_ptr(),
            w["o_proj_weight"].data_ptr(), wc, w["q_norm_weight"].data_ptr(), w["k_norm_weight"].data_ptr(), qc,
            self.key_cache.data_ptr(), self.value_cache.data_ptr(), cc, self.max_positions, 0,
            self.position.data_ptr(), self.tokens, sp.hidden_size, sp.attention_heads, sp.attention_kv_heads,
            sp.attention_head_dim, sp.rope_dim, float(sp.rope_theta), self.interleaved, self.eps, self.eps,
            self.update.data_ptr(), self.hidden_out.data_ptr(), self.workspace.data_ptr(), self.workspace.numel(), s,
        )

    def check_device(self, stream: torch.cuda.Stream | None = None) -> None:
        _check_device(self.workspace, self.device, stream)

    def set_poll_limit(self, limit: int | None, stream: torch.cuda.Stream | None = None) -> None:
        _set_poll_limit(self.workspace, self.device, limit, stream)
