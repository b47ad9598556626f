"""Resident-weight multi-layer decode runner.

The pattern of the reference's real-shape runner (bench/qwen36_full_decode.py:
132-545) without per-step weight loads: every layer's weights stay in HBM
(a full Qwen3.6-35B-A3B stack is ~67 GB of bf16, a quarter of one MI355X),
and a decode step is each layer's mixer (Gated DeltaNet or gated full
attention) followed by its MoE block, the hidden state carried between
layers in fp32 device buffers that the plans share, with no host work
between layers.

Steps can be issued eagerly (`step`) or captured once as HIP graphs and
replayed (`capture` / `replay`).  State that a step changes lives on the
device so a captured step stays valid:
  * DeltaNet conv/recurrent states ping-pong between two buffers: two
    plans per DeltaNet layer (even / odd steps) read one pair and write the
    other, and two graphs alternate;
  * attention layers decode at a device-held position that each step
    advances (AttentionStepPlan), writing their KV caches in place.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Sequence

import torch

from .plan import AttentionStepPlan, DeltaNetStepPlan, MoeLayerPlan
from .spec import Qwen36A3BSpec, qwen36_35b_a3b_spec


@dataclass(frozen=True)
class Qwen36RealDecodeState:
    """Per-sequence decode state (reference reference/qwen36_real.py:12-20):
    DeltaNet conv and recurrent states, attention KV caches, in layer order
    within each kind, and the next position."""

    deltanet_conv_states: tuple[Any, ...]
    deltanet_recurrent_states: tuple[Any, ...]
    attention_key_cache: tuple[Any, ...]
    attention_value_cache: tuple[Any, ...]
    position: int = 0


def initial_qwen36_real_decode_state(
    spec: Qwen36A3BSpec,
    *,
    max_positions: int | None = None,
    conv_kernel_size: int = 4,
    device: Any = "cpu",
    dtype: Any = None,
) -> Qwen36RealDecodeState:
    """Zero states and caches for one sequence (reference reference/qwen36_real.py:40-80)."""

    dtype = dtype or torch.float32
    counts = spec.layer_counts()
    conv_dim = spec.deltanet_conv_dim
    rec = spec.deltanet_recurrent_state_shape()
    cache = spec.attention_cache_shape(max_positions)
    z = lambda shape: torch.zeros(shape, device=device, dtype=dtype)  # noqa: E731
    return Qwen36RealDecodeState(
        deltanet_conv_states=tuple(z((conv_dim, conv_kernel_size)) for _ in range(counts["deltanet_moe"])),
        deltanet_recurrent_states=tuple(z(rec) for _ in range(counts["deltanet_moe"])),
        attention_key_cache=tuple(z(cache) for _ in range(counts["attention_moe"])),
        attention_value_cache=tuple(z(cache) for _ in range(counts["attention_moe"])),
        position=0,
    )


def _tensors(w: Any) -> dict[str, Any]:
    return dict(w.as_dict()) if hasattr(w, "as_dict") else dict(w)


class ResidentDecodeRunner:
    """Decode steps over resident layers.

    `layers`: (kind, mixer_weights, moe_weights) per layer, kind
    "deltanet_moe" (mixer: the DeltaNet tensors plus initial `conv_state`
    and `recurrent_state`, which are copied) or "attention_moe" (mixer: the
    attention tensors; its caches start at zero).  Weights may be dicts or
    the packed dataclasses of fastkernels_amd.weights.  `hidden` ([T, H],
    hidden_dtype) is layer 0's input and `output` the last layer's fp32
    output; `layer_outputs[i]` is layer i's.
    """

    def __init__(
        self,
        layers: Sequence[tuple[str, Any, Any]],
        tokens: int,
        spec: Qwen36A3BSpec | None = None,
        *,
        max_positions: int = 4096,
        cache_dtype: torch.dtype = torch.float32,
        top_k: int | None = None,
        hidden_dtype: torch.dtype = torch.bfloat16,
        rope_interleaved: bool = True,
    ) -> None:
        spec = spec or qwen36_35b_a3b_spec()
        self.spec = spec
        self.tokens = tokens
        top_k = top_k or spec.num_routed_experts
        self.mixers: list[tuple[Any, Any]] = []
        self.moes: list[MoeLayerPlan] = []
        self.kinds: list[str] = []
        prev = None
        for i, (kind, mixer_w, moe_w) in enumerate(layers):
            mw = _tensors(mixer_w)
            if kind == "deltanet_moe":
                mw["conv_state"] = mw["conv_state"].clone()
                mw["recurrent_state"] = mw["recurrent_state"].clone()
                even = DeltaNetStepPlan(mw, tokens, spec, hidden=prev, hidden_dtype=hidden_dtype)
                odd_w = dict(even.w)
                odd_w["conv_state"] = even.next_conv_state
                odd_w["recurrent_state"] = even.next_recurrent_state
                odd = DeltaNetStepPlan(odd_w, tokens, spec, hidden=even.hidden)
                odd.next_conv_state = even.w["conv_state"]
                odd.next_recurrent_state = even.w["recurrent_state"]
                odd.update, odd.hidden_out = even.update, even.hidden_out
                pair: tuple[Any, Any] = (even, odd)
            elif kind == "attention_moe":
                att = AttentionStepPlan(mw, tokens, spec, max_positions=max_positions, cache_dtype=cache_dtype,
                                        rope_interleaved=rope_interleaved, hidden=prev, hidden_dtype=hidden_dtype)
                pair = (att, att)
            else:
                raise ValueError(f"unknown layer kind at layer {i}: {kind}")
            moe = MoeLayerPlan(_tensors(moe_w), tokens, top_k=top_k, hidden=pair[0].hidden_out)
            self.mixers.append(pair)
            self.moes.append(moe)
            self.kinds.append(kind)
            prev = moe.layer_out
        if not self.moes:
            raise ValueError("at least one layer is needed")
        self.hidden = self.mixers[0][0].hidden
        self.output = self.moes[-1].layer_out
        self.layer_outputs = [m.layer_out for m in self.moes]
        self.parity = 0
        self._graphs: list[torch.cuda.CUDAGraph] | None = None

    def _issue(self, parity: int, stream: torch.cuda.Stream | None) -> None:
        for pair, moe in zip(self.mixers, self.moes):
            pair[parity].run(stream)
            moe.run(stream)

    def step(self, stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        """One decode step over every layer, issued eagerly."""

        self._issue(self.parity, stream)
        self.parity ^= 1
        return self.output

    def capture(self, stream: torch.cuda.Stream | None = None) -> None:
        """Record one step per parity as HIP graphs (nothing executes)."""

        s = stream or torch.cuda.Stream(self.output.device)
        graphs = []
        for parity in (0, 1):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                self._issue(parity, s)
            graphs.append(g)
        self._graphs = graphs

    def replay(self) -> torch.Tensor:
        """One decode step by replaying the captured graph of this parity."""

        if self._graphs is None:
            raise RuntimeError("capture() first")
        self._graphs[self.parity].replay()
        self.parity ^= 1
        return self.output

    # state of layer i as the next step will read it
    def deltanet_state(self, i: int) -> tuple[torch.Tensor, torch.Tensor]:
        p = self.mixers[i][self.parity]
        return p.w["conv_state"], p.w["recurrent_state"]

    def kv_cache(self, i: int) -> tuple[torch.Tensor, torch.Tensor]:
        p = self.mixers[i][0]
        return p.key_cache, p.value_cache

    def state(self) -> Qwen36RealDecodeState:
        """The state the next step reads (device tensors, not copies; the
        position is read back from the device)."""

        dn = [i for i, k in enumerate(self.kinds) if k == "deltanet_moe"]
        at = [i for i, k in enumerate(self.kinds) if k == "attention_moe"]
        pos = int(self.mixers[at[0]][0].position.item()) if at else 0
        return Qwen36RealDecodeState(
            deltanet_conv_states=tuple(self.deltanet_state(i)[0] for i in dn),
            deltanet_recurrent_states=tuple(self.deltanet_state(i)[1] for i in dn),
            attention_key_cache=tuple(self.kv_cache(i)[0] for i in at),
            attention_value_cache=tuple(self.kv_cache(i)[1] for i in at),
            position=pos,
        )

    def load_state(self, state: Qwen36RealDecodeState) -> None:
        """Copy a sequence's state into the buffers the next step reads
        (caches up to the shorter of the two lengths)."""

        dn = [i for i, k in enumerate(self.kinds) if k == "deltanet_moe"]
        at = [i for i, k in enumerate(self.kinds) if k == "attention_moe"]
        if len(state.deltanet_conv_states) != len(dn) or len(state.attention_key_cache) != len(at):
            raise ValueError("state does not match the runner's layer kinds")
        for i, conv, rec in zip(dn, state.deltanet_conv_states, state.deltanet_recurrent_states):
            c, r = self.deltanet_state(i)
            c.copy_(conv)
            r.copy_(rec)
        for i, kc, vc in zip(at, state.attention_key_cache, state.attention_value_cache):
            k, v = self.kv_cache(i)
            n = min(k.shape[0], kc.shape[0])
            k[:n].copy_(kc[:n])
            v[:n].copy_(vc[:n])
        self.set_position(state.position)

    def set_position(self, position: int) -> None:
        for pair, kind in zip(self.mixers, self.kinds):
            if kind == "attention_moe":
                pair[0].set_position(position)

    def check_device(self, stream: torch.cuda.Stream | None = None) -> None:
        for pair, moe in zip(self.mixers, self.moes):
            pair[0].check_device(stream)
            if pair[1] is not pair[0]:
                pair[1].check_device(stream)
            moe.check_device(stream)
