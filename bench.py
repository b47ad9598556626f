#!/usr/bin/env python
"""Benchmark of the MI355X Qwen3.6 MoE decode layer (and the DeltaNet step).

Headline (the JSON `value`): microseconds per MoE layer decode step at batch
16, bf16 weights, weights resident in HBM.
Extra sub-results on the same line: batch 1 (config 0), batch 128 with the
Zipf router bias (config 2), the Gated DeltaNet step at batch 1 and 8
(config 3), and a stack of 40 independent resident MoE layers (64.7 GB of
weights) run 32 times at batch 1 and 8 with the residual carried from layer
to layer (config 4; cache-cold by construction).

Method: every step is one MoE layer (router + top-k + routing tables +
experts + residual) issued through the C ABI from a preallocated plan.  K
steps are captured in one HIP graph and replayed once between two HIP events
on the capture stream, after W eager warmup steps and untimed replays (the
last of them still running when the timed one is enqueued, so the GPU does
not idle while the host submits the graph).
Steps cycle through R independent weight sets (each 1.6 GB) so one step's
57.7 MB does not stay in the 256 MB last-level cache.  The expert stage
(gate/up + down kernels, 98% of the bytes) is timed the same way on its own
to give the roofline entry.  The CPU baseline is the oracle (a CPU
restatement of the reference's PyTorch path) on the same inputs.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

METRIC = "µs per MoE layer decode step at batch 1/16/128; achieved HBM TB/s vs peak"
HBM_PEAK_GBS = 8000.0  # MI355X published HBM3E bandwidth
GRAPH_WARM_REPLAYS = 2  # untimed replays of each captured graph before the timed one, at least
GRAPH_WARM_STEPS = 256  # ... and at least this many untimed steps (the memory system warms over ~100-200 steps)
REFERENCE_A100_T1_US = 181.5  # real_moe_ms 0.1815 ms, A100 (reference docs/modal.md:1053)


def parse_args() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=64)
    p.add_argument("--warmup", type=int, default=8)
    p.add_argument("--tokens", type=int, default=16, help="batch of the headline workload")
    p.add_argument("--weight-sets", type=int, default=8)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="bound on the CPU-baseline sample")
    p.add_argument("--no-extra", action="store_true", help="skip the batch-1/128 and DeltaNet sub-results")
    p.add_argument("--zipf", action="store_true", help="with --only moe: add the config-2 Zipf router bias")
    p.add_argument("--no-stack", action="store_true", help="skip the 40-layer resident stack (config 4)")
    p.add_argument("--stack-layers", type=int, default=40, help="layers of the config-4 stack")
    p.add_argument("--context", type=int, default=1024, help="with --only attention: cached positions before the step")
    p.add_argument("--only", choices=["moe", "deltanet", "copy", "stack", "attention", "model"], default=None,
                   help="run a single timing loop (for profilers) and print its line; "
                        "'copy' runs 16 device-to-device copies of 1 GiB (PMC byte-counter calibration)")
    return p.parse_args()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model_name() -> str:
    """The host CPU's model string (/proc/cpuinfo), for the CPU baseline."""

    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def copy_bandwidth_tbs(torch, dev) -> float:
    """Read + write TB/s of 16 device-to-device copies of 1 GiB."""

    nbytes = 1 << 30
    src = torch.ones(nbytes // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(16):
        dst.copy_(src)
    end.record()
    end.synchronize()
    secs = start.elapsed_time(end) * 1e-3
    del src, dst
    torch.cuda.empty_cache()
    return round(2 * nbytes * 16 / secs / 1e12, 3)


def read_bandwidth_tbs(torch, dev) -> float:
    """TB/s of fk_stream_read over 4 GiB (16-byte non-temporal loads in
    one-shot 16 KiB workgroups, the fastest read shape measured on this
    part), 8 timed passes after one warm pass."""

    from fastkernels_amd import _lib

    nbytes = 4 << 30
    src = torch.ones(nbytes // 2, dtype=torch.bfloat16, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    _lib.call("fk_stream_read", src.data_ptr(), nbytes, sink.data_ptr(), stream.cuda_stream)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(8):
        _lib.call("fk_stream_read", src.data_ptr(), nbytes, sink.data_ptr(), stream.cuda_stream)
    end.record(stream)
    end.synchronize()
    secs = start.elapsed_time(end) * 1e-3
    del src, sink
    torch.cuda.empty_cache()
    return round(nbytes * 8 / secs / 1e12, 3)


def cpu_time(fn, seconds: float, min_iters: int = 2) -> tuple[float, int]:
    """Microseconds per call of fn() after one warmup call, over >= min_iters
    calls and about `seconds` of wall time."""

    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        if n >= min_iters and time.perf_counter() - t0 > seconds:
            break
    return (time.perf_counter() - t0) / n * 1e6, n


def cpu_other_configs(oracle, torch, wl, spec, w_cpu, args_cpu, cpu_layers, K, E, H) -> dict:
    """The oracle on the other BASELINE configs (same inputs as the GPU
    runs' weight set 0), a few seconds each."""

    out = {}
    x1 = wl.make_hidden(1, H, seed=1)
    us, n = cpu_time(lambda: oracle.moe_layer(x1, *args_cpu, top_k=K), 3.0)
    out["moe_t1"] = {"us_per_layer_step": round(us, 1), "iterations": n}
    x128 = wl.make_hidden(128, H, seed=1)
    bias = wl.zipf_router_bias(E, seed=0)
    us, n = cpu_time(lambda: oracle.moe_layer(x128, *args_cpu, top_k=K, router_bias=bias), 4.0)
    out["moe_t128_zipf"] = {"us_per_layer_step": round(us, 1), "iterations": n}
    d = wl.make_deltanet_weights(spec, seed=2000)
    kw = dict(qk_heads=spec.deltanet_qk_heads, value_heads=spec.deltanet_value_heads, head_dim=spec.deltanet_head_dim)
    for tokens in (1, 8):
        x = wl.make_hidden(tokens, H, seed=50)
        us, n = cpu_time(lambda: oracle.deltanet_update(x, d["conv_state"], d["recurrent_state"], d, **kw), 3.0)
        out[f"deltanet_t{tokens}"] = {"us_per_step": round(us, 1), "iterations": n}
    if cpu_layers:
        args_l = [(w["norm_weight"], w["router_weight"], w["expert_gate_up_weight"], w["expert_down_weight"],
                   w["shared_gate_up_weight"], w["shared_down_weight"], w["shared_expert_gate_weight"])
                  for w in cpu_layers]
        for tokens in (1, 8):
            x0 = wl.make_hidden(tokens, H, seed=7)

            def two_layers():
                h = oracle.moe_layer(x0, *args_l[0], top_k=K)[0]
                oracle.moe_layer(h, *args_l[1], top_k=K)

            us, n = cpu_time(two_layers, 3.0)
            out[f"moe_stack40_t{tokens}"] = {
                "us_per_layer_step": round(us / 2, 1),
                "us_per_stack_step_extrapolated": round(us / 2 * 40, 1),
                "iterations": n,
                "sample": "layers 0 and 1 of the stack chained (fp32 hidden into layer 1); the 40-layer step "
                          "extrapolated as 40 x the per-layer time (the full stack needs 64.7 GB of host RAM)",
            }
    return out


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(
            f"bench.py measures one GPU: this build has no multi-GPU path (requested --gpus {args.gpus}). "
            "Run with --gpus 1.",
            file=sys.stderr,
        )
        return 2

    import torch

    from fastkernels_amd import workloads as wl
    from fastkernels_amd.plan import AttentionStepPlan, DeltaNetStepPlan, MoeLayerPlan
    from fastkernels_amd.spec import qwen36_35b_a3b_spec

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    if args.only == "copy":
        nbytes = 1 << 30
        src = torch.ones(nbytes // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(16):
            dst.copy_(src)
        torch.cuda.synchronize()
        secs = time.perf_counter() - t0
        print(json.dumps({"copy_bytes_per_launch": nbytes, "launches": 16, "read_plus_write_tbs": round(2 * nbytes * 16 / secs / 1e12, 3)}))
        return 0
    spec = qwen36_35b_a3b_spec()
    H, E, I, K = spec.hidden_size, spec.num_experts, spec.expert_intermediate_size, spec.num_routed_experts
    stream = torch.cuda.Stream(dev)

    # -- weight sets, generated on the device (seeded) ------------------------
    def moe_set(r: int) -> dict:
        g = torch.Generator(device=dev).manual_seed(1000 + r)

        def rnd(*shape):
            return (torch.randn(*shape, generator=g, device=dev, dtype=torch.float32) * wl.WEIGHT_SCALE).to(torch.bfloat16)

        def rnd_big(*shape):
            out = torch.empty(shape, device=dev, dtype=torch.bfloat16)
            for s in range(0, shape[0], 32):
                out[s : s + 32] = rnd(min(32, shape[0] - s), *shape[1:])
            return out

        # (the router weight comes from the CPU generator, as the tests draw
        # it, so the config-2 Zipf calibration holds for these very sets)
        return {
            "norm_weight": torch.zeros(H, device=dev, dtype=torch.bfloat16),
            "router_weight": wl.make_router_weight(spec, seed=r).to(dev),
            "expert_gate_up_weight": rnd_big(E, 2 * I, H),
            "expert_down_weight": rnd_big(E, H, I),
            "shared_gate_up_weight": rnd(2 * I, H),
            "shared_down_weight": rnd(H, I),
            "shared_expert_gate_weight": rnd(H),
        }

    R = max(1, args.weight_sets)
    log(f"generating {R} MoE weight sets on {torch.cuda.get_device_name(0)}")
    sets = [] if args.only in ("deltanet", "stack", "attention", "model") else [moe_set(r) for r in range(R)]
    torch.cuda.synchronize()

    def warm_replays(steps: int) -> int:
        return max(GRAPH_WARM_REPLAYS, -(-GRAPH_WARM_STEPS // steps))

    def timed_graph(fns, steps: int, warmup: int) -> float:
        """ms per step over exactly `steps` graph-captured steps."""

        with torch.cuda.stream(stream):
            for i in range(warmup):
                fns[i % len(fns)](stream)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(steps):
                fns[i % len(fns)](stream)
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        # replay() launches on the current stream: make it the timed stream.
        # Untimed replays first, at least GRAPH_WARM_STEPS steps of them: the
        # first uploads the graph, and a T=16 step over the 13 GB of rotating
        # weight sets runs ~4% slow until ~100-200 steps have run (measured:
        # 20-step replays after 65 steps 114.3 us, after 200 steps 108.4 us,
        # as 64-step ones), then exactly `steps` steps timed in one replay.
        # The timed replay is enqueued while one more untimed replay runs, so
        # the GPU does not wait for the host to submit the graph.
        with torch.cuda.stream(stream):
            for _ in range(warm_replays(steps)):
                graph.replay()
            stream.synchronize()
            graph.replay()
            start.record(stream)
            graph.replay()
            end.record(stream)
        end.synchronize()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps

    def moe_plans(tokens: int, bias=None, nsets: int = R) -> list:
        plans = []
        for r in range(nsets):
            p = MoeLayerPlan(sets[r], tokens, top_k=K, router_bias=bias)
            p.hidden.copy_(wl.make_hidden(tokens, H, seed=1 + r, dtype=torch.bfloat16).to(dev))
            plans.append(p)
        return plans

    def distinct(plans) -> list[int]:
        torch.cuda.synchronize()
        return [int((torch.bincount(p.ids.reshape(-1), minlength=E) > 0).sum()) for p in plans]

    def moe_result(tokens: int, bias=None, nsets: int = R, steps: int = args.steps) -> dict:
        plans = moe_plans(tokens, bias, nsets)
        fns = [p.run for p in plans]
        ms_layer = timed_graph(fns, steps, args.warmup)
        u = distinct(plans)
        # The router stage writes the routing tables that the expert stage
        # reads (the single-launch layer keeps its tables in LDS), so it runs
        # first.
        ms_router = timed_graph([p.run_router for p in plans], steps, 2)
        ms_experts = timed_graph([p.run_experts for p in plans], steps, 2)
        for p in plans:  # no bounded in-kernel wait ran out in any timed step
            p.check_device(stream)
        per_step_u = [u[i % len(u)] for i in range(steps)]
        layer_bytes = sum(wl.moe_layer_bytes(tokens, x, spec) for x in per_step_u) / steps
        expert_bytes = sum(
            (x + 1) * 3 * H * I * 2 + H * 2 + tokens * H * 2 + 2 * tokens * H * 4 for x in per_step_u
        ) / steps
        us = ms_layer * 1e3
        return {
            "tokens": tokens,
            "us_per_layer_step": round(us, 3),
            "distinct_experts_mean": round(sum(per_step_u) / steps, 2),
            "algorithmic_bytes_per_step": int(layer_bytes),
            "achieved_tbs": round(layer_bytes / (ms_layer * 1e-3) / 1e12, 3),
            "hbm_frac": round(layer_bytes / (ms_layer * 1e-3) / (HBM_PEAK_GBS * 1e9), 4),
            "expert_stage_us": round(ms_experts * 1e3, 3),
            "expert_stage_bytes": int(expert_bytes),
            "expert_stage_tbs": round(expert_bytes / (ms_experts * 1e-3) / 1e12, 3),
            "router_stage_us": round(ms_router * 1e3, 3),
            "weight_sets": nsets,
            "_plans": plans,
        }

    def deltanet_result(tokens: int, nsets: int = R) -> dict:
        dn_sets = [wl.make_deltanet_weights(spec, seed=2000 + r, device=dev) for r in range(nsets)]
        dplans = []
        for r in range(nsets):
            dp = DeltaNetStepPlan(dn_sets[r], tokens, spec)
            dp.hidden.copy_(wl.make_hidden(tokens, H, seed=50 + r).to(dev))
            dplans.append(dp)
        ms = timed_graph([p.run for p in dplans], args.steps, args.warmup)
        for p in dplans:
            p.check_device(stream)
        nbytes = wl.deltanet_step_bytes(tokens, spec)
        return {
            "tokens": tokens,
            "us_per_step": round(ms * 1e3, 3),
            "algorithmic_bytes_per_step": nbytes,
            "achieved_tbs": round(nbytes / (ms * 1e-3) / 1e12, 3),
            "hbm_frac": round(nbytes / (ms * 1e-3) / (HBM_PEAK_GBS * 1e9), 4),
        }

    def attention_result(tokens: int, context: int, nsets: int = R) -> dict:
        """Gated attention step of `tokens` rows after `context` cached
        positions (f32 caches), weights rotated over `nsets` sets."""

        aplans = []
        steps = args.steps
        for r in range(nsets):
            w = wl.make_attention_weights(spec, seed=3000 + r, device=dev)
            # every run advances the position: room for the warmup, untimed and timed replays
            ap = AttentionStepPlan(w, tokens, spec,
                                   max_positions=context + (args.warmup + (warm_replays(steps) + 2) * steps + 8) * tokens,
                                   start_position=context)
            ap.hidden.copy_(wl.make_hidden(tokens, H, seed=70 + r).to(dev))
            aplans.append(ap)
        ms = timed_graph([p.run for p in aplans], steps, args.warmup)
        for p in aplans:
            p.check_device(stream)
        nbytes = wl.attention_step_bytes(tokens, context, spec)
        return {
            "tokens": tokens,
            "context": context,
            "us_per_step": round(ms * 1e3, 3),
            "algorithmic_bytes_per_step": nbytes,
            "achieved_tbs": round(nbytes / (ms * 1e-3) / 1e12, 3),
            "hbm_frac": round(nbytes / (ms * 1e-3) / (HBM_PEAK_GBS * 1e9), 4),
        }

    def model_result(tokens: int, lsets: list, steps: int = 16) -> dict:
        """Full resident decode step: the spec's 40 layers (DeltaNet or gated
        attention mixer, then the MoE block), captured once per parity and
        replayed (fastkernels_amd.runner)."""

        from fastkernels_amd.runner import ResidentDecodeRunner

        layers = []
        for l, kind in enumerate(spec.layer_kinds()):
            if kind == "deltanet_moe":
                mixer = wl.make_deltanet_weights(spec, seed=4000 + l, device=dev)
            else:
                mixer = wl.make_attention_weights(spec, seed=4000 + l, device=dev)
            layers.append((kind, mixer, lsets[l % len(lsets)]))
        warm = 8  # decode steps (320 layer steps) before the timed ones
        runner = ResidentDecodeRunner(layers, tokens, spec, max_positions=(steps + warm + 8) * tokens)
        runner.hidden.copy_(wl.make_hidden(tokens, H, seed=8).to(dev))
        runner.capture(stream)
        with torch.cuda.stream(stream):
            for _ in range(warm - 1):
                runner.replay()
            stream.synchronize()
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            runner.replay()  # (the timed replays are enqueued while this one runs)
            start.record(stream)
            for _ in range(steps):
                runner.replay()
            end.record(stream)
        end.synchronize()
        ms = start.elapsed_time(end) / steps
        runner.check_device(stream)
        u = distinct(runner.moes)
        counts = spec.layer_counts()
        nbytes = (sum(wl.moe_layer_bytes(tokens, x, spec, in_bytes=4) for x in u)
                  + counts["deltanet_moe"] * wl.deltanet_step_bytes(tokens, spec)
                  + counts["attention_moe"] * wl.attention_step_bytes(tokens, 4 * tokens, spec))
        res = {
            "tokens": tokens,
            "layers": len(layers),
            "layer_counts": counts,
            "us_per_decode_step": round(ms * 1e3, 3),
            "tokens_per_s": round(tokens / (ms * 1e-3), 1),
            "algorithmic_bytes_per_step": int(nbytes),
            "achieved_tbs": round(nbytes / (ms * 1e-3) / 1e12, 3),
            "hbm_frac": round(nbytes / (ms * 1e-3) / (HBM_PEAK_GBS * 1e9), 4),
            "note": "graph replays of one decode step; attention context grows from 0 (bytes counted at 4 tokens)",
        }
        del runner, layers
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        return res

    def stack_result(tokens: int, layers: int, steps: int, lsets: list | None = None) -> dict:
        """Config 4: `layers` independent resident MoE layers (weights seeded
        base + layer), each step running them in order with the residual
        carried across layers: layer l reads layer l-1's fp32 layer output."""

        lsets = lsets if lsets is not None else [moe_set(100 + l) for l in range(layers)]
        lplans = []
        for l in range(layers):
            prev = lplans[-1].layer_out if lplans else None
            lp = MoeLayerPlan(lsets[l], tokens, top_k=K, hidden=prev)
            if prev is None:
                lp.hidden.copy_(wl.make_hidden(tokens, H, seed=7).to(dev))
            lplans.append(lp)

        def step(s):
            for lp in lplans:
                lp.run(s)

        ms = timed_graph([step], steps, 2)
        for lp in lplans:
            lp.check_device(stream)
        us_layer = ms * 1e3 / layers
        u = distinct(lplans)
        nbytes = sum(
            wl.moe_layer_bytes(tokens, x, spec, in_bytes=2 if l == 0 else 4) for l, x in enumerate(u)
        ) / layers
        res = {
            "tokens": tokens,
            "layers": layers,
            "steps": steps,
            "us_per_layer_step": round(us_layer, 3),
            "us_per_stack_step": round(ms * 1e3, 3),
            "distinct_experts_mean": round(sum(u) / layers, 2),
            "algorithmic_bytes_per_layer_step": int(nbytes),
            "resident_weight_bytes": int(sum(sum(t.numel() * t.element_size() for t in s.values()) for s in lsets)),
            "achieved_tbs": round(nbytes / (us_layer * 1e-6) / 1e12, 3),
            "hbm_frac": round(nbytes / (us_layer * 1e-6) / (HBM_PEAK_GBS * 1e9), 4),
            "launches_per_step": layers,
        }
        del lplans
        torch.cuda.synchronize()
        return res

    if args.only == "stack":
        print(json.dumps(stack_result(args.tokens, args.stack_layers, min(args.steps, 32))))
        return 0
    if args.only == "attention":
        print(json.dumps(attention_result(args.tokens, args.context)))
        return 0
    if args.only == "model":
        msets = [moe_set(100 + l) for l in range(spec.num_layers)]
        print(json.dumps(model_result(args.tokens, msets)))
        return 0
    if args.only == "moe":
        res = moe_result(args.tokens, bias=wl.zipf_router_bias(E, seed=0).to(dev) if args.zipf else None)
        res.pop("_plans")
        print(json.dumps(res))
        return 0
    if args.only == "deltanet":
        print(json.dumps(deltanet_result(args.tokens)))
        return 0

    # -- headline: MoE layer at batch `tokens` ---------------------------------
    log(f"timing MoE layer T={args.tokens}")
    main_res = moe_result(args.tokens)
    plans = main_res.pop("_plans")
    ms_per_step = main_res["us_per_layer_step"] / 1e3

    sub = {}
    if not args.no_extra:
        log("timing MoE layer T=1")
        r1 = moe_result(1)
        r1.pop("_plans")
        r1["reference_a100_us"] = REFERENCE_A100_T1_US
        sub["moe_t1"] = r1
        log("timing MoE layer T=128 (Zipf router bias)")
        bias = wl.zipf_router_bias(E, seed=0).to(dev)
        r128 = moe_result(128, bias=bias, nsets=min(R, 4), steps=min(args.steps, 32))
        p128 = r128.pop("_plans")
        torch.cuda.synchronize()
        r128["hottest_expert_tokens"] = [int(torch.bincount(p.ids.reshape(-1), minlength=E).max()) for p in p128]
        r128["zipf_alpha"] = wl.ZIPF_ALPHA
        # MFMA utilisation of the expert stage (dense bf16 peak 2.5 PFLOP/s):
        # useful flops are 2 per multiply-add of the (token, slot) pairs'
        # gate/up (2I x H) and down (H x I) products plus the shared expert's;
        # the kernels execute more (tokens padded to 16-column tiles, and the
        # down kernel's fp32 activations as two bf16 columns each, hi + lo).
        n_rows = 128 * K + 128
        useful = n_rows * 6 * H * I
        cnt = torch.bincount(p128[0].ids.reshape(-1), minlength=E).tolist() + [128]  # + the shared expert
        gu_cols = sum(-(-c // 16) * 16 for c in cnt)  # gate/up: 16 tokens per tile
        dn_cols = sum(-(-c // 8) * 16 for c in cnt)  # down: 8 tokens (hi + lo columns) per tile
        executed = gu_cols * 4 * H * I + dn_cols * 2 * H * I
        r128["mfma_flops_useful"] = int(useful)
        r128["mfma_flops_executed_set0"] = int(executed)
        r128["mfma_util"] = round(useful / (r128["expert_stage_us"] * 1e-6) / 2.5e15, 5)
        sub["moe_t128_zipf"] = r128
        del p128
        log("timing Gated DeltaNet step T=1 and T=8")
        for tokens in (1, 8):
            sub[f"deltanet_t{tokens}"] = deltanet_result(tokens)
        log("timing the gated attention step T=1 after 1024 cached positions")
        sub["attention_t1_ctx1024"] = attention_result(1, 1024)
    cpu_layers = None
    if not args.no_extra and not args.no_stack:
        lsets = [moe_set(100 + l) for l in range(max(args.stack_layers, spec.num_layers))]
        if not args.no_cpu_baseline:  # two config-4 layers for the CPU baseline's stack sample
            cpu_layers = [{k: v.cpu() for k, v in lsets[l].items()} for l in range(2)]
        for tokens in (1, 8):
            log(f"timing the {args.stack_layers}-layer resident stack, T={tokens} (config 4)")
            sub[f"moe_stack{args.stack_layers}_t{tokens}"] = stack_result(tokens, args.stack_layers, 32, lsets)
        log(f"timing the full {spec.num_layers}-layer decode step (DeltaNet/attention + MoE), T=1")
        sub["model_decode_t1"] = model_result(1, lsets)
        del lsets
        torch.cuda.synchronize()
        torch.cuda.empty_cache()

    # -- measured device-copy bandwidth (read + write), for the fraction of a
    # bandwidth this GPU actually reaches ---------------------------------------
    log("device copy bandwidth (1 GiB, 16 copies) and read-stream bandwidth (4 GiB, 8 passes)")
    copy_tbs = copy_bandwidth_tbs(torch, dev)
    read_tbs = read_bandwidth_tbs(torch, dev)

    # -- CPU baseline (oracle on the host cores, bounded sample) ----------------
    cpu = None
    if not args.no_cpu_baseline:
        log("CPU baseline (oracle restatement of the reference PyTorch MoE path)")
        import oracle

        torch.set_num_threads(os.cpu_count() or 1)
        w_cpu = {k: v.cpu() for k, v in sets[0].items()}
        x_cpu = plans[0].hidden.cpu()
        args_cpu = (w_cpu["norm_weight"], w_cpu["router_weight"], w_cpu["expert_gate_up_weight"],
                    w_cpu["expert_down_weight"], w_cpu["shared_gate_up_weight"], w_cpu["shared_down_weight"],
                    w_cpu["shared_expert_gate_weight"])
        oracle.moe_layer(x_cpu, *args_cpu, top_k=K)  # warmup
        n, t0 = 0, time.perf_counter()
        while True:
            oracle.moe_layer(x_cpu, *args_cpu, top_k=K)
            n += 1
            if n >= 2 and time.perf_counter() - t0 > args.cpu_seconds:
                break
        cpu_us = (time.perf_counter() - t0) / n * 1e6
        cpu = {
            "value": round(cpu_us, 1),
            "unit": "us per layer step",
            "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"MoE layer T={args.tokens} (weight set 0, same bytes as the GPU run), {n} iterations after 1 warmup",
            "cpu_model": cpu_model_name(),
            "os_cpu_count": os.cpu_count(),
        }
        if not args.no_extra:
            cpu["other_configs"] = cpu_other_configs(oracle, torch, wl, spec, w_cpu, args_cpu, cpu_layers, K, E, H)
        del w_cpu

    expert_frac = main_res["expert_stage_tbs"] * 1e12 / (HBM_PEAK_GBS * 1e9)
    # HBM bytes per expert stage from the committed rocprofv3 --pmc FETCH_SIZE /
    # WRITE_SIZE passes (profiles/moe_layer_pmc_traffic.md), when recorded.
    traffic = None
    traffic_file = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "pmc_traffic.json")
    if os.path.exists(traffic_file):
        with open(traffic_file) as fh:
            rec = json.load(fh).get(f"moe_layer_t{args.tokens}")
        if rec:
            traffic = rec["expert_stage_traffic_bytes"]
    for r in [main_res, *sub.values()]:
        if isinstance(r, dict) and "achieved_tbs" in r:
            r["frac_of_measured_copy"] = round(r["achieved_tbs"] / copy_tbs, 4) if copy_tbs else None
            r["frac_of_measured_read"] = round(r["achieved_tbs"] / read_tbs, 4) if read_tbs else None
    line = {
        "metric": METRIC,
        "value": main_res["us_per_layer_step"],
        "unit": "us",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "graph_warm_replays": GRAPH_WARM_REPLAYS,
        "graph_warm_steps": GRAPH_WARM_STEPS,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"moe_layer_t{args.tokens}",
            "tokens": args.tokens,
            "hidden": H,
            "experts": E,
            "top_k": K,
            "intermediate": I,
            "shared_expert": "sigmoid-gated",
            "weight_sets": R,
            "parallelism": "single-gpu",
        },
        "roofline": {
            "kernel": "moe_gateup_kernel + moe_down_kernel + moe_combine_kernel (expert stage)",
            "bound": "hbm",
            "achieved": round(main_res["expert_stage_tbs"] * 1e3, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(expert_frac, 4),
            "traffic": traffic,
            "traffic_source": "profiles/pmc_traffic.json: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE passes of this "
                              "workload's expert stage, scaled by a 1 GiB copy calibration (not measured in this run)"
                              if traffic is not None else None,
            "algorithmic_bytes": main_res["expert_stage_bytes"],
            "scope": "expert stage only (3 launches); the whole layer step, router included, is layer.hbm_frac",
            "frac_of_measured_copy": round(main_res["expert_stage_tbs"] / copy_tbs, 4) if copy_tbs else None,
            "frac_of_measured_read": round(main_res["expert_stage_tbs"] / read_tbs, 4) if read_tbs else None,
        },
        "copy_bandwidth_tbs": copy_tbs,
        "read_bandwidth_tbs": read_tbs,
        "measured_bandwidth_note": "copy: torch device-to-device copy of 1 GiB, read + write bytes; read: "
                                   "fk_stream_read over 4 GiB, 16-byte non-temporal loads in one-shot 16 KiB workgroups",
        "layer": main_res,
        "sub_results": sub,
        "cpu_baseline": cpu,
        "device": torch.cuda.get_device_name(0),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
