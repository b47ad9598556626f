"""Preallocated decode-step plans over the C ABI.

A plan owns every buffer a step touches (inputs, outputs, workspace), so a
step is one or a few C-ABI calls with no torch allocation and no host sync.
That makes steps cheap to issue from a serving loop and capturable in a HIP
graph (torch.cuda.CUDAGraph), which is how bench.py times them.

  MoeLayerPlan      router + top-k + routing tables + experts + residual
                    (fk_moe_layer), or its two stages separately.
  DeltaNetStepPlan  projections -> conv -> recurrent/gated-norm/out-proj
                    (+ residual), writing the next conv / recurrent states.
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
        nbytes = self.lib.fk_moe_workspace_bytes(tokens, top_k, self.num_experts, self.intermediate)
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


class DeltaNetStepPlan:
    """One Gated DeltaNet decode step (T rows through one state) + residual."""

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
        self.mixed = torch.empty((tokens, w["in_proj_qkv_weight"].shape[0]), dtype=torch.float32, device=dev)
        self.z = torch.empty((tokens, w["in_proj_z_weight"].shape[0]), dtype=torch.float32, device=dev)
        self.a = torch.empty((tokens, w["in_proj_a_weight"].shape[0]), dtype=torch.float32, device=dev)
        self.b = torch.empty_like(self.a)
        self.conv_out = torch.empty_like(self.mixed)
        self.next_conv_state = torch.empty_like(w["conv_state"])
        self.next_recurrent_state = torch.empty_like(w["recurrent_state"])
        self.update = torch.empty((tokens, H), dtype=torch.float32, device=dev)
        self.hidden_out = torch.empty_like(self.update)
        nbytes = self.lib.fk_deltanet_workspace_bytes(tokens, spec.deltanet_value_heads, spec.deltanet_head_dim)
        self.workspace = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        names = ("conv_out", "z", "a", "b", "recurrent_state", "out_proj_weight", "linear_norm_weight", "a_log", "dt_bias")
        tensors = (self.conv_out, self.z, self.a, self.b, w["recurrent_state"], w["out_proj_weight"],
                   w["linear_norm_weight"], w["a_log"], w["dt_bias"])
        codes = [_fcode(t, n) for t, n in zip(tensors, names)] + [_fcode(self.hidden, "hidden")]
        self._dtypes = (ctypes.c_int32 * 10)(*codes)

    def run(self, stream: torch.cuda.Stream | None = None) -> None:
        w, sp = self.w, self.spec
        s = _stream_handle(stream, self.device)
        _lib.call(
            "fk_deltanet_project",
            self.hidden.data_ptr(), _fcode(self.hidden, "hidden"),
            w["input_norm_weight"].data_ptr(), _fcode(w["input_norm_weight"], "norm"),
            w["in_proj_qkv_weight"].data_ptr(), w["in_proj_z_weight"].data_ptr(),
            w["in_proj_a_weight"].data_ptr(), w["in_proj_b_weight"].data_ptr(), _fcode(w["in_proj_qkv_weight"], "proj"),
            self.tokens, sp.hidden_size, self.mixed.shape[1], self.z.shape[1], self.a.shape[1], self.eps, 1.0,
            self.mixed.data_ptr(), self.z.data_ptr(), self.a.data_ptr(), self.b.data_ptr(), s,
        )
        _lib.call(
            "fk_deltanet_conv",
            self.mixed.data_ptr(), _lib.FK_DTYPE_F32, w["conv_state"].data_ptr(), _fcode(w["conv_state"], "conv_state"),
            w["conv1d_weight"].data_ptr(), _fcode(w["conv1d_weight"], "conv1d"), self.tokens, self.mixed.shape[1],
            w["conv_state"].shape[1], self.conv_out.data_ptr(), self.next_conv_state.data_ptr(), s,
        )
        _lib.call(
            "fk_deltanet_recurrent_output",
            self.conv_out.data_ptr(), self.z.data_ptr(), self.a.data_ptr(), self.b.data_ptr(),
            w["recurrent_state"].data_ptr(), w["out_proj_weight"].data_ptr(), w["linear_norm_weight"].data_ptr(),
            w["a_log"].data_ptr(), w["dt_bias"].data_ptr(), self.hidden.data_ptr(),
            ctypes.cast(self._dtypes, ctypes.c_void_p),
            self.tokens, sp.deltanet_qk_heads, sp.deltanet_value_heads, sp.deltanet_head_dim, sp.hidden_size, self.eps,
            self.update.data_ptr(), self.next_recurrent_state.data_ptr(), self.hidden_out.data_ptr(),
            self.workspace.data_ptr(), self.workspace.numel(), s,
        )
