"""Per-phase timeline of the single-launch kernels (a diagnostic, not the product path).

Usage, on a GPU, after ``python -m fastkernels_amd.build --timeline``::

    python -m fastkernels_amd.timeline moe --tokens 1
    python -m fastkernels_amd.timeline deltanet --tokens 8
    python -m fastkernels_amd.timeline router --tokens 128 --zipf
    python -m fastkernels_amd.timeline attention --tokens 1 --context 1024

It loads ``libfastkernels_hip_timeline.so``: the same kernels compiled with
``-DFK_TIMELINE``, in which thread 0 of every workgroup of
``moe_fused_kernel`` (the MoE layer at T = 1), ``moe_router_tagged_kernel``
(the router stage from two tokens on; the layer's router stage alone is
timed), ``deltanet_step_kernel`` and ``attn_step_kernel`` (the attention step
after ``--context`` cached positions) keeps the wall clock (100 MHz) at each
phase boundary.  Steps run in steady
state: 16 back-to-back steps over 4 weight sets are captured as one HIP graph
and replayed; the markers are cleared and the graph replayed once more, so the
recorded step is the last of 16 that follow one another on the stream.  The
report gives, per marker, the number of workgroups that passed it and the
min / mean / max time after the earliest workgroup start, in microseconds, as
a markdown table; ``--dump PATH`` also writes every workgroup's marker
times to a CSV file (one row per workgroup), for spreads by role.  The
markers perturb the code a little (a few registers and
stores): the totals read a few tenths of a microsecond above the product
build's.
"""

from __future__ import annotations

import argparse
import ctypes
import sys

MARKERS = {
    "moe": (
        "moe_fused",
        [
            "workgroup start",
            "P1 item done (router row, shared intermediate or gate stored)",
            "logits of the token polled",
            "top-k selected",
            "routing table in LDS",
            "routed gate/up block done, down rows issued, shared activations in LDS",
            "the down item's slot activations in LDS",
            "down rows applied, y stored (wavefront 7)",
            "end: y of the K slots polled, rows written",
            "fast path: wavefront 0 issues its gate/up rows",
            "fast path: wavefront 0's gate/up rows issued",
            "fast path: wavefront 0's gate/up products done",
        ],
    ),
    "router": (
        "moe_router",
        [
            "workgroup start",
            "first tile of logits stored",
            "every tile of logits stored",
            "top-k done, ids published (workgroups < T; the others end here)",
            "workgroup 0: every id polled, epoch advanced",
            "workgroup 0: routing tables built",
        ],
    ),
    "attention": (
        "attn_step",
        [
            "workgroup start",
            "weight rows issued",
            "A: projection rows stored (started)",
            "B: attention inputs read",
            "B: chunk partial stored",
            "M: gated values stored",
            "C1: gated values read",
            "C1: partial sums stored",
            "C2: output rows written",
            "end",
            "B: q and own-key norms",
            "B: RoPE",
            "B: tile of cached rows issued (loop entered)",
            "B: softmax over the chunk done",
            "B: wavefronts merged, partials stored",
        ],
    ),
    "deltanet": (
        "deltanet_step",
        [
            "workgroup start",
            "tokens normalised and staged",
            "A: projection tiles done (stored)",
            "B: head inputs read and normalised",
            "B: recurrence done",
            "B: gated values and sums of squares stored",
            "C1: unit inputs staged",
            "C1: unit partial sums stored",
            "C2: output rows written",
            "end",
            "A: first loads issued (tokens, norm and a/b rows, state, conv taps)",
            "A: first weight tiles issued",
            "tokens in (wavefront 0's sums of squares done)",
        ],
    ),
}


def parse_args(argv=None) -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("kernel", choices=sorted(MARKERS))
    p.add_argument("--tokens", type=int, default=1)
    p.add_argument("--steps", type=int, default=16)
    p.add_argument("--weight-sets", type=int, default=4)
    p.add_argument("--zipf", action="store_true", help="router: the config-2 Zipf router bias")
    p.add_argument("--context", type=int, default=1024, help="attention: cached positions before the step")
    p.add_argument("--dump", default=None, help="also write every workgroup's marker times (µs) to this CSV file")
    return p.parse_args(argv)


def main(argv=None) -> int:
    args = parse_args(argv)
    from fastkernels_amd import _lib
    from fastkernels_amd import build as fk_build

    if not fk_build.TIMELINE_LIB_PATH.exists():
        print(f"{fk_build.TIMELINE_LIB_PATH} is missing: run `python -m fastkernels_amd.build --timeline`", file=sys.stderr)
        return 1
    _lib.LIB_PATH = fk_build.TIMELINE_LIB_PATH  # before anything loads the library
    lib = _lib.load()

    import torch

    from fastkernels_amd import workloads as wl
    from fastkernels_amd.plan import AttentionStepPlan, DeltaNetStepPlan, MoeLayerPlan
    from fastkernels_amd.spec import qwen36_35b_a3b_spec

    if not torch.cuda.is_available():
        print("the timeline needs a GPU", file=sys.stderr)
        return 1
    unit, names = MARKERS[args.kernel]
    read = getattr(lib, f"fk_timeline_read_{unit}")
    read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    clear = getattr(lib, f"fk_timeline_clear_{unit}")
    clear.argtypes = []
    dev = torch.device("cuda", 0)
    spec = qwen36_35b_a3b_spec()
    T, R = args.tokens, max(1, args.weight_sets)
    H, E, I = spec.hidden_size, spec.num_experts, spec.expert_intermediate_size

    def moe_set(r: int) -> dict:
        # drawn on the device (seeded), 32 experts at a time
        g = torch.Generator(device=dev).manual_seed(1000 + r)

        def rnd(*shape):
            out = torch.empty(shape, device=dev, dtype=torch.bfloat16)
            step = 32 if len(shape) == 3 else shape[0]
            for s in range(0, shape[0], step):
                n = min(step, shape[0] - s)
                out[s : s + n] = (torch.randn(n, *shape[1:], generator=g, device=dev) * wl.WEIGHT_SCALE).to(torch.bfloat16)
            return out

        return {
            "norm_weight": torch.zeros(H, device=dev, dtype=torch.bfloat16),
            "router_weight": rnd(E, H),
            "expert_gate_up_weight": rnd(E, 2 * I, H),
            "expert_down_weight": rnd(E, H, I),
            "shared_gate_up_weight": rnd(2 * I, H),
            "shared_down_weight": rnd(H, I),
            "shared_expert_gate_weight": rnd(H),
        }

    bias = wl.zipf_router_bias(E, seed=0).to(dev) if args.zipf else None
    plans = []
    for r in range(R):
        if args.kernel in ("moe", "router"):
            p = MoeLayerPlan(moe_set(r), T, top_k=spec.num_routed_experts, router_bias=bias)
        elif args.kernel == "attention":
            # room for every run of the warmup, the capture's replays and the marked replay
            p = AttentionStepPlan(wl.make_attention_weights(spec, seed=3000 + r, device=dev), T, spec,
                                  max_positions=args.context + (4 * args.steps + 8) * T, start_position=args.context)
        else:
            p = DeltaNetStepPlan(wl.make_deltanet_weights(spec, seed=2000 + r, device=dev), T, spec)
        p.hidden.copy_(wl.make_hidden(T, spec.hidden_size, seed=50 + r).to(dev))
        plans.append(p)
    stream = torch.cuda.Stream(dev)

    def step(p):
        if args.kernel == "router":
            p.run_router(stream)
        else:
            p.run(stream)

    with torch.cuda.stream(stream):
        for i in range(2 * R):
            step(plans[i % R])
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(args.steps):
            step(plans[i % R])
    with torch.cuda.stream(stream):
        graph.replay()
        stream.synchronize()
        if clear() != 0:
            raise RuntimeError("fk_timeline_clear failed")
        graph.replay()
        stream.synchronize()
    for p in plans:
        p.check_device(stream)
    rows, marks = 1024, 16
    buf = (ctypes.c_ulonglong * (rows * marks))()
    if read(buf, ctypes.sizeof(buf)) != 0:
        raise RuntimeError("fk_timeline_read failed")
    wgs = [list(buf[i * marks : (i + 1) * marks]) for i in range(rows) if buf[i * marks] != 0]
    if not wgs:
        print(f"no markers recorded: the {unit} kernel did not run at T={T}", file=sys.stderr)
        return 1
    t0 = min(w[0] for w in wgs)
    cmd = " ".join(["python -m fastkernels_amd.timeline", *(argv if argv is not None else sys.argv[1:])])
    print(f"Command: `{cmd}` ({len(wgs)} workgroups, {torch.cuda.get_device_name(0)})")
    print()
    print("| marker | workgroups | min µs | mean µs | max µs |")
    print("|---|---:|---:|---:|---:|")
    for k, name in enumerate(names):
        v = [(w[k] - t0) / 100.0 for w in wgs if w[k] != 0]
        if v:
            print(f"| {k}: {name} | {len(v)} | {min(v):.2f} | {sum(v) / len(v):.2f} | {max(v):.2f} |")
    if args.dump:
        with open(args.dump, "w") as fh:
            fh.write("workgroup," + ",".join(f"m{k}" for k in range(len(names))) + "\n")
            for i in range(rows):
                w = buf[i * marks : (i + 1) * marks]
                if w[0] != 0:
                    fh.write(f"{i}," + ",".join(f"{(w[k] - t0) / 100.0:.2f}" if w[k] else "" for k in range(len(names))) + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
