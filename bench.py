"""Benchmark: the L 64x8 MoE FFN layer forward at 16384 tokens on one MI355X.

A step is one forward pass of the whole MoE FFN layer (models/layers.py:596-634):
gate GEMM, router kernel, dispatch, fused gather + gate_up GEMM + SwiGLU,
down GEMM and combine, over 16384 bf16 tokens of N(0,1) with N(0, 0.02)
weights (H=1280, E=64, I=448, top-8).  Inputs stay resident in HBM.
Consecutive steps alternate between weight copies so the 256 MB
Infinity Cache cannot keep one layer's 220 MB of expert weights.

Printed (one JSON line on stdout): active TFLOP/s of the layer (6*R*H*I per
step, R = T*k) and ms per layer over the timed steps; per-op times from a
separate pass of the same workload with HIP events around every op (events
stall the stream for a few microseconds each, so they stay out of the
headline pass); the roofline of the dominant kernel (fused gate_up + SwiGLU
GEMM, from those events on its stream, with the HBM traffic of a committed
counter summary when it describes the kernel that ran) and the reference's
eager CPU path timed on the host's cores.

Pass order: at least 100 untimed layer forwards, then the per-op pass (at
least 60 forwards), then the headline pass: W warmup steps and exactly K timed
steps.  The GPU's clocks take a few tens of milliseconds of load to settle
after idling (the first 20 forwards after 5 warmup steps measured 0.67 ms per
layer, later windows 0.59-0.60 ms), so both timed passes run at the settled
clock.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1]
                       [--workload l64x8|xl_skew|xl128|decode_t{1,8,64,256}|xl128_train|l64x8_train|xl_skew_train]
       python bench.py --calibrate-copy-mb 512   (a plain copy, for scaling rocprofv3 byte counters)
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE FFN ms/layer + active TFLOP/s (% bf16 MFMA peak), L 64x8, 16k tokens"
# the same figures for the other layer-forward shapes (parity-test and comparison workloads)
LAYER_METRICS = {
    "l64x8": METRIC,
    "xl_skew": "MoE FFN ms/layer + active TFLOP/s (% bf16 MFMA peak), XL 64x8 skewed loads, 16k tokens",
    "xl128": "MoE FFN ms/layer + active TFLOP/s (% bf16 MFMA peak), XL 128x8, 32k tokens",
}
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA (published)
PEAK_HBM_GBS = 8000.0

WORKLOADS = {
    # name: (tokens, hidden, experts, inter, top_k, logit bias std)
    "l64x8": (16384, 1280, 64, 448, 8, 0.0),
    "xl_skew": (16384, 1536, 64, 512, 8, 1.5),
    "xl128": (32768, 1536, 128, 512, 8, 0.0),
    # decode steps of the XL 64x8 layer: HBM-bound weight streaming, replayed from a HIP graph
    "decode_t1": (1, 1536, 64, 512, 8, 0.0),
    "decode_t8": (8, 1536, 64, 512, 8, 0.0),
    "decode_t64": (64, 1536, 64, 512, 8, 0.0),
    "decode_t256": (256, 1536, 64, 512, 8, 0.0),
    # XL 128x8 training GEMMs: forward, dgrad and wgrad of both grouped linears
    "xl128_train": (32768, 1536, 128, 512, 8, 0.0),
    # whole-layer training steps (forward + backward) at the L and XL-skew shapes
    "l64x8_train": (16384, 1280, 64, 448, 8, 0.0),
    "xl_skew_train": (16384, 1536, 64, 512, 8, 1.5),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_layer(hrm, dev, t, h, e, i, k, bias_std, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    layer = hrm.SparseMoESwiGLU(h, i, e, k, True, implementation="grouped_triton").to(dev, torch.bfloat16)
    with torch.no_grad():
        layer.gate.weight.normal_(0.0, 0.02, generator=g)
        layer.experts.gate_up_weight.normal_(0.0, 0.02, generator=g)
        layer.experts.down_weight.normal_(0.0, 0.02, generator=g)
        x = torch.randn(t, h, device=dev, generator=g).to(torch.bfloat16)
        if bias_std > 0:
            b = torch.randn(e, device=dev, generator=g) * bias_std
            wg = layer.gate.weight.double()
            v = wg.T @ torch.linalg.solve(wg @ wg.T, b.double())
            x = (x.double() + v[None, :]).to(torch.bfloat16)
    return layer, x


class OpTimer:
    """Records HIP events around each call of the named ``hrm_moe_amd.ops`` functions.

    The layer looks its ops up on the module at call time, so wrapping the
    module attributes times the kernels the layer really launches.  Events go
    on torch's current stream, the stream every op launches on; with the GPU
    queue kept full by the timed loop, an event pair brackets exactly that
    op's kernels.
    """

    NAMES = ("router_topk", "permute", "router_topk_dispatch", "gate_up_swiglu", "grouped_gemm_nt", "combine")

    def __init__(self, ops):
        self.ops = ops
        self.orig = {n: getattr(ops, n) for n in self.NAMES}
        self.pairs = {n: [] for n in self.NAMES}
        self.active = False
        for n, f in self.orig.items():
            setattr(ops, n, self._wrap(n, f))

    def _wrap(self, name, fn):
        def timed(*a, **kw):
            if not self.active:
                return fn(*a, **kw)
            s = torch.cuda.Event(enable_timing=True)
            e = torch.cuda.Event(enable_timing=True)
            s.record()
            r = fn(*a, **kw)
            e.record()
            self.pairs[name].append((s, e))
            return r
        return timed

    def restore(self):
        for n, f in self.orig.items():
            setattr(self.ops, n, f)

    def mean_ms(self):
        return {n: (statistics.fmean(s.elapsed_time(e) for s, e in v) if v else 0.0)
                for n, v in self.pairs.items()}


def time_layers(layers, xs, steps, warmup, timer=None):
    """ms per layer over `steps` forwards after `warmup`; with `timer`, per-op events are recorded too.

    Each timed event costs the stream a few microseconds of idle time, so the
    headline layer time is taken with timer=None and the per-op times in a
    separate pass over the same workload.
    """
    with torch.no_grad():
        for s in range(warmup):
            layers[s % len(layers)](xs[s % len(xs)])
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        if timer is not None:
            timer.active = True
        start.record()
        for s in range(steps):
            layers[s % len(layers)](xs[s % len(xs)])
        end.record()
        torch.cuda.synchronize()
        if timer is not None:
            timer.active = False
        wall = time.perf_counter() - t0
    return start.elapsed_time(end) / steps, wall


def calibrate_copy(mb, reps=5):
    """A plain device copy of ``mb`` MiB, for scaling rocprofv3's FETCH_SIZE / WRITE_SIZE counters."""
    n = mb * (1 << 20)
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibrate_copy_bytes_read": n, "calibrate_copy_bytes_written": n, "reps": reps}), flush=True)


def read_traffic(name, kernel):
    """HBM traffic per launch of ``kernel`` from a committed rocprofv3 --pmc summary under profiles/.

    The summary names the kernel instantiation it measured (``kernel:`` line);
    when that is not ``kernel`` (the instantiation this run launched), the
    figures describe other code and None is returned.  Bytes are FETCH_SIZE and
    WRITE_SIZE per dispatch, scaled by what the counters read for a plain copy
    of known size; FETCH_SIZE counts L2 misses, Infinity Cache hits included.
    """
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path) or not kernel:
        return None
    fields = {}
    for line in open(path):
        key, sep, val = line.partition(":")
        if sep and key in ("kernel", "fetch_bytes_per_launch", "write_bytes_per_launch",
                           "algorithmic_bytes_per_launch", "expert_partitioned_min_bytes_per_launch"):
            fields[key] = val.strip()
    if fields.get("kernel") != kernel:
        log(f"traffic summary {name} describes {fields.get('kernel')!r}, this run launched {kernel!r}: not used")
        return None
    out = {"kernel": kernel, "source": f"profiles/{name}"}
    for key in ("fetch_bytes_per_launch", "write_bytes_per_launch", "algorithmic_bytes_per_launch",
                "expert_partitioned_min_bytes_per_launch"):
        if key in fields:
            out[key] = int(float(fields[key]))
    return out


def _cpu_layer_inputs(t, h, e, i, bias_std, dtype, seed=1234):
    """Synthetic inputs of one layer on the CPU, built like make_layer's (N(0,1) tokens, N(0, 0.02) weights)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(t, h, generator=g)
    wg = torch.randn(e, h, generator=g) * 0.02
    wgu = torch.randn(e, 2 * i, h, generator=g) * 0.02
    wdn = torch.randn(e, h, i, generator=g) * 0.02
    if bias_std > 0:
        b = torch.randn(e, generator=g, dtype=torch.float64) * bias_std
        wg64 = wg.double()
        x = (x.double() + (wg64.T @ torch.linalg.solve(wg64 @ wg64.T, b))[None, :]).float()
    return [a.to(dtype) for a in (x, wg, wgu, wdn)]


def _time_cpu_layer(t, h, e, i, k, bias_std, dtype, runs):
    """Median seconds of the reference's eager CPU layer forward (oracle.moe_forward_eager) over ``runs``."""
    from oracle import moe_oracle

    args = _cpu_layer_inputs(t, h, e, i, bias_std, dtype)
    moe_oracle.moe_forward_eager(*args, k)
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        moe_oracle.moe_forward_eager(*args, k)
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def cpu_baseline(t, h, e, i, k, bias_std=0.0, runs=5, legs=()):
    """The reference's eager CPU path on the host cores: the bench's layer at full size in bf16.

    ``legs``: more (name, T, H, E, I, k, bias, dtype) layers timed the same way,
    reported beside the headline leg (the L and XL-skew shapes in bf16 and fp32).
    """
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count()
    sec = _time_cpu_layer(t, h, e, i, k, bias_std, torch.bfloat16, runs)
    flops = 6.0 * t * k * h * i
    out = {
        "value": round(flops / sec / 1e12, 5),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"the whole layer ({t} tokens, bf16), reference eager CPU path (router, stable sort, per-expert "
                   f"F.linear, index_add_), median of {runs} runs after 1 warmup: {sec * 1e3:.1f} ms; "
                   f"torch threads {torch.get_num_threads()}, os.cpu_count()={os.cpu_count()}, affinity={affinity}"),
        "ms_per_layer": round(sec * 1e3, 3),
    }
    extra = []
    for name, lt, lh, le, li, lk, lb, ldt in legs:
        sec = _time_cpu_layer(lt, lh, le, li, lk, lb, ldt, runs)
        extra.append({"leg": name, "dtype": str(ldt).replace("torch.", ""), "tokens": lt,
                      "ms_per_layer": round(sec * 1e3, 3),
                      "tflops": round(6.0 * lt * lk * lh * li / sec / 1e12, 5)})
        log(f"cpu baseline {name} {extra[-1]['dtype']}: {sec * 1e3:.1f} ms per layer")
    if extra:
        out["legs"] = extra
    return out


def decode_gate_up_us(layers, xs, dispatches, reps):
    """Average duration (us) of the layer's gate_up kernel alone at a decode size, its instantiation, and
    whether it is the one-launch router + dispatch + gate_up kernel (one or two tokens) rather than the
    gate_up GEMM after the router.

    One HIP graph holds one launch per weight copy, back to back; HIP events on
    the replaying stream bracket ``reps`` replays.
    """
    from hrm_moe_amd import _lib, ops

    weights = [layer.experts.gate_up_weight.to(x.dtype) for layer, x in zip(layers, xs)]
    k = layers[0].top_k
    with torch.no_grad():
        logits = [torch.nn.functional.linear(x, layer.gate.weight) for layer, x in zip(layers, xs)]
        fused = ops.router_gate_up_decode_ok(logits[0], xs[0], weights[0], k)

        def body():
            for c, (x, d, w) in enumerate(zip(xs, dispatches, weights)):
                if fused:
                    ops.router_gate_up_decode(logits[c], x, w, k, True)
                else:
                    ops.gate_up_swiglu(x, d, w)

        side = torch.cuda.Stream()  # default priority
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            body()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            body()
    kernel = _lib.last_gemm_kernel(_lib.GEMM_KIND_GATE_UP)
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e3 / (reps * len(xs)), kernel, fused


def run_decode(args, hrm, dev):
    """Decode-size layer latency over weight copies that together exceed the MALL: the layers chained in one
    HIP graph (the headline), and each replayed from its own graph."""
    from hrm_moe_amd import ops

    t, h, e, i, k, _ = WORKLOADS[args.workload]
    copies = max(args.weight_copies, 8)
    layers, xs, graphs = [], [], []
    for c in range(copies):
        layer, x = make_layer(hrm, dev, t, h, e, i, k, 0.0, seed=4321 + c)
        layers.append(layer)
        xs.append(x)
        graphs.append(hrm.GraphedMoEForward(layer, x))
    # Headline: each graph's tokens already sit in its captured input buffer (a serving loop has
    # the op before write them there), so a step is the replay alone.  A second pass passes the
    # tokens from their own buffer, which adds the copy into the graph's buffer.
    def timed(inputs):
        for s in range(args.warmup):
            graphs[s % copies](inputs[s % copies])
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for s in range(args.steps):
            graphs[s % copies](inputs[s % copies])
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / args.steps * 1e3

    us_single = timed([g.static_in for g in graphs])
    us_copy = timed(xs)
    # Headline: the decode caller runs every layer of the model in one call (a whole decode step,
    # simple_inference_engine.py:337-339), so the layers are captured as a stack in one graph,
    # layer c + 1 reading layer c's output; per-layer latency = replay time / copies.
    stack_in = xs[0].clone()
    with torch.no_grad():
        side = torch.cuda.Stream()  # default priority
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                hcur = stack_in
                for layer in layers:
                    hcur = layer(hcur)
        torch.cuda.current_stream().wait_stream(side)
        stack = torch.cuda.CUDAGraph()
        with torch.cuda.graph(stack):
            hcur = stack_in
            for layer in layers:
                hcur = layer(hcur)
    reps = max(1, args.steps // copies)
    for _ in range(max(1, args.warmup // copies)):
        stack.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        stack.replay()
    end.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(end) / (reps * copies) * 1e3
    # algorithmic bytes: the touched experts' weights, the tokens in and out, the router weight
    with torch.no_grad():
        dispatches = []
        for c in range(copies):
            logits = torch.nn.functional.linear(xs[c], layers[c].gate.weight)
            dispatches.append(ops.router_topk_dispatch(logits, k, True, torch.bfloat16, want_probs=False)[3])
    distinct = [int((d.tokens_per_expert > 0).sum().item()) for d in dispatches]
    touched = statistics.fmean(distinct)
    nbytes = touched * 3 * h * i * 2 + 2 * t * h * 2 + h * e * 2
    gbs = nbytes / (us * 1e-6) / 1e9
    log(f"decode T={t}: {us:.2f} us/layer in a {copies}-layer stack graph; one graph per layer {us_single:.2f} us "
        f"({us_copy:.2f} with the input copy), {touched:.1f} experts touched, {nbytes / 1e6:.1f} MB, {gbs:.0f} GB/s")
    # dominant kernel: the fused gather + gate_up + SwiGLU, timed alone from a graph of back-to-back
    # launches over the weight copies (HIP events on the stream the graph is replayed on)
    gu_us, gu_kernel, gu_fused = decode_gate_up_us(layers, xs, dispatches, max(args.steps, 20))
    # touched experts' gate/up weights, the gathered rows and the act rows; the one-launch kernel also
    # reads the logits
    gu_bytes = (statistics.fmean(n * 2 * i * h * 2 for n in distinct) + t * k * (h + i) * 2
                + (t * e * 2 if gu_fused else 0))
    gu_gbs = gu_bytes / (gu_us * 1e-6) / 1e9
    log(f"decode T={t}: gate_up kernel {gu_kernel} {gu_us:.2f} us, {gu_bytes / 1e6:.1f} MB, {gu_gbs:.0f} GB/s")
    result = {
        "metric": f"MoE FFN decode latency, XL 64x8 (H={h}, E={e}, I={i}, top-{k}), {t} tokens",
        "value": round(us, 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"{args.workload}: {copies} MoE FFN layer forwards (each with its own weights) "
                               f"chained in one HIP graph, per layer, {t} tokens, H={h}, E={e}, I={i}, top-{k} "
                               f"(us_one_graph_per_layer: each layer replayed from its own graph, tokens in its "
                               f"input buffer; us_with_input_copy: copied in each step)",
                   "tokens": t, "hidden": h, "experts": e, "inter": i, "top_k": k, "weight_copies": copies},
        "us_one_graph_per_layer": round(us_single, 3),
        "us_with_input_copy": round(us_copy, 3),
        "layer_hbm": {"bytes_per_step": int(nbytes), "achieved_gbs": round(gbs, 1),
                      "frac": round(gbs / PEAK_HBM_GBS, 4), "experts_touched": touched},
        "roofline": {"kernel": f"{gu_kernel} ({'router, dispatch, ' if gu_fused else ''}fused gather + gate_up GEMM "
                               f"+ SwiGLU)", "bound": "hbm",
                     "achieved": round(gu_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / PEAK_HBM_GBS, 4), "traffic": None,
                     "bytes_per_launch": int(gu_bytes), "avg_launch_us": round(gu_us, 3)},
    }
    traffic = read_traffic(f"gate_up_swiglu_{args.workload}_traffic.txt", gu_kernel)
    if traffic is not None:
        result["roofline"]["traffic"] = traffic["fetch_bytes_per_launch"] + traffic["write_bytes_per_launch"]
        result["roofline"]["traffic_detail"] = traffic
    if not args.no_cpu_baseline:
        cb = cpu_baseline(t, h, e, i, k, runs=5)
        result["cpu_baseline"] = {"value": round(cb["ms_per_layer"] * 1e3, 1), "unit": "us/layer",
                                  "cores": cb["cores"], "kind": cb["kind"], "sample": cb["sample"]}
    print(json.dumps(result), flush=True)


def run_train_gemms(args, hrm, dev):
    """XL 128x8 grouped linears, forward + backward (dgrad and wgrad) through hip_grouped_linear's autograd.

    One step: gate_up = A[R,H] . W_gu[e]^T and down = act[R,I] . W_dn[e]^T
    forward, then backward with N(0,1) upstream grads.  Rows are split evenly
    over the experts (the near-uniform routing of N(0,0.02) gates).  Work per
    step: 3 x 2 x R x (H x 2I + I x H) flops.
    """
    t, h, e, i, k, _ = WORKLOADS[args.workload]
    r = t * k
    g = torch.Generator(device=dev).manual_seed(7)
    bf = torch.bfloat16
    tpe = torch.full((e,), r // e, dtype=torch.int64, device=dev)
    tpe[: r - int(tpe.sum())] += 1
    a = torch.randn(r, h, device=dev, generator=g).to(bf).requires_grad_(True)
    act = torch.randn(r, i, device=dev, generator=g).to(bf).requires_grad_(True)
    w_gu = (torch.randn(e, 2 * i, h, device=dev, generator=g) * 0.02).to(bf).requires_grad_(True)
    w_dn = (torch.randn(e, h, i, device=dev, generator=g) * 0.02).to(bf).requires_grad_(True)
    d_gu = torch.randn(r, 2 * i, device=dev, generator=g).to(bf)
    d_dn = torch.randn(r, h, device=dev, generator=g).to(bf)

    def step():
        y1 = hrm.hip_grouped_linear(a, w_gu, tpe)
        y2 = hrm.hip_grouped_linear(act, w_dn, tpe)
        torch.autograd.backward([y1, y2], [d_gu, d_dn])
        a.grad = act.grad = w_gu.grad = w_dn.grad = None

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        step()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    flops = 3 * 2.0 * r * (h * 2 * i + i * h)
    tflops = flops / (ms * 1e-3) / 1e12
    log(f"xl128 training GEMMs: {ms:.4f} ms per step, {tflops:.1f} TFLOP/s")
    print(json.dumps({
        "metric": "XL 128x8 grouped GEMMs forward + dgrad + wgrad, TFLOP/s (% bf16 MFMA peak)",
        "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"xl128_train: gate_up and down grouped linears of {r} rows, H={h}, E={e}, I={i}, "
                               f"forward + backward with N(0,1) upstream grads", "rows": r, "hidden": h,
                   "experts": e, "inter": i},
        "pct_bf16_peak": round(100 * tflops / PEAK_BF16_TFLOPS, 2),
        "flops_per_step": flops,
    }), flush=True)


def _composition_compute(experts, hidden_states, selected_experts, routing_weights, dispatch=None):
    """The reference's grouped composition (models/layers.py:311-334) under torch autograd, for comparison.

    HIP router, dispatch and grouped GEMMs (hip_grouped_linear: forward, dgrad,
    wgrad); gather, SwiGLU, weighting and index_add_ as torch ops.  Timed beside
    the fused HIP backward of the expert block; not part of the package.
    """
    import torch.nn.functional as F
    from hrm_moe_amd import hip_grouped_linear, ops

    dtype = hidden_states.dtype
    d = ops.permute(selected_experts, experts.num_experts, want_sort_idx=True)
    tok = d.sorted_token_idx.long()
    sorted_weights = routing_weights.to(dtype).reshape(-1).index_select(0, d.sort_idx)
    gate_up = hip_grouped_linear(hidden_states.index_select(0, tok), experts.gate_up_weight.to(dtype),
                                 d.tokens_per_expert)
    gate, up = gate_up.chunk(2, dim=-1)
    y = hip_grouped_linear(F.silu(gate) * up, experts.down_weight.to(dtype), d.tokens_per_expert)
    out = torch.zeros_like(hidden_states)
    out.index_add_(0, tok, (y * sorted_weights[:, None]).to(dtype))
    return out, d.tokens_per_expert


def run_layer_train(args, hrm, dev):
    """One training step of the whole MoE FFN layer: forward with the aux-loss context, then backward.

    Upstream gradient g ~ N(0,1) on the output, plus the aux loss.  Gradients reach
    the hidden states, the router weight and both expert weights.  Work per
    step counted: the expert GEMMs, 6*R*H*I forward + 12*R*H*I backward (dgrad
    and wgrad of both projections).  The same steps are also timed with the
    reference's composition under autograd (_composition_compute: torch ops
    for gather, SwiGLU, weighting and index_add_, HIP grouped GEMMs).
    """
    import types

    t, h, e, i, k, bias = WORKLOADS[args.workload]
    r = t * k
    layers, xs = [], []
    for c in range(args.weight_copies):
        layer, x = make_layer(hrm, dev, t, h, e, i, k, bias, seed=1234 + c)
        layers.append(layer)
        xs.append(x.requires_grad_(True))
    g = torch.randn(t, h, device=dev, generator=torch.Generator(device=dev).manual_seed(99)).to(torch.bfloat16)

    def step(j):
        layer = layers[j % len(layers)]
        ctx = {}
        out = layer(xs[j % len(xs)], moe_context=ctx)
        torch.autograd.backward([out, torch.stack(ctx["aux_losses"]).sum()], [g, None])
        for p in layer.parameters():
            p.grad = None
        xs[j % len(xs)].grad = None

    def timed():
        for j in range(args.warmup):
            step(j)
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for j in range(args.steps):
            step(j)
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / args.steps

    for layer in layers:  # the composition first: it also settles the clocks before the timed fused steps
        layer.experts._compute = types.MethodType(_composition_compute, layer.experts)
    try:
        ms_ref = timed()
    finally:
        for layer in layers:
            del layer.experts._compute
    ms = timed()
    flops = 18.0 * r * h * i
    tflops = flops / (ms * 1e-3) / 1e12
    log(f"{args.workload}: {ms:.4f} ms per training step ({tflops:.1f} TFLOP/s); "
        f"reference composition under autograd {ms_ref:.4f} ms")
    print(json.dumps({
        "metric": f"MoE FFN layer training step (forward + backward), H={h}, E={e}, I={i}, top-{k}, {t} tokens",
        "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"{args.workload}: MoE FFN layer forward + backward, N(0,1) output grads + aux loss, "
                               f"{t} tokens, H={h}, E={e}, I={i}, top-{k}", "tokens": t, "hidden": h, "experts": e,
                   "inter": i, "top_k": k, "weight_copies": args.weight_copies},
        "pct_bf16_peak": round(100 * tflops / PEAK_BF16_TFLOPS, 2),
        "flops_per_step": flops,
        "reference_composition_ms_per_step": round(ms_ref, 5),
    }), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="l64x8", choices=sorted(WORKLOADS))
    ap.add_argument("--weight-copies", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-cpu-legs", action="store_true", help="time only the bench's own layer on the CPU")
    ap.add_argument("--calibrate-copy-mb", type=int, default=0)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: hrm_moe_amd has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    assert torch.cuda.is_available(), "bench.py needs a ROCm GPU"
    if args.calibrate_copy_mb:
        calibrate_copy(args.calibrate_copy_mb)
        return

    import hrm_moe_amd as hrm

    hrm.load_library()
    dev = torch.device("cuda:0")
    if args.workload.startswith("decode"):
        run_decode(args, hrm, dev)
        return
    if args.workload == "xl128_train":
        run_train_gemms(args, hrm, dev)
        return
    if args.workload.endswith("_train"):
        run_layer_train(args, hrm, dev)
        return
    t, h, e, i, k, bias = WORKLOADS[args.workload]
    r = t * k
    layers, xs = [], []
    for c in range(max(1, args.weight_copies)):
        layer, x = make_layer(hrm, dev, t, h, e, i, k, bias, seed=1234 + c)
        layers.append(layer)
        xs.append(x)
    # untimed forwards first, to bring the clocks to their loaded state; then the per-op pass
    # (HIP events around every op, on the op's stream), then the headline pass
    from hrm_moe_amd import _lib

    time_layers(layers, xs, max(args.steps, 100), 0)
    timer = OpTimer(hrm.ops)
    ms_instr, _ = time_layers(layers, xs, max(args.steps, 60), 2, timer)
    timer.restore()
    gate_up_kernel = _lib.last_gemm_kernel(_lib.GEMM_KIND_GATE_UP)
    ms, wall = time_layers(layers, xs, args.steps, args.warmup)
    flops = 6.0 * r * h * i
    tflops = flops / (ms * 1e-3) / 1e12

    op_ms = timer.mean_ms()
    phases = {
        # one fused call (router + dispatch) for E <= 128 and k <= 8, else two
        "router_and_dispatch": op_ms["router_topk"] + op_ms["permute"] + op_ms["router_topk_dispatch"],
        "gate_up_swiglu": op_ms["gate_up_swiglu"],
        "down_gemm": op_ms["grouped_gemm_nt"],
        "combine": op_ms["combine"],
    }
    phases["gate_gemm_and_gaps"] = max(0.0, ms_instr - sum(phases.values()))
    gate_up_ms = phases["gate_up_swiglu"]
    gate_up_flops = 4.0 * r * h * i
    achieved = gate_up_flops / (gate_up_ms * 1e-3) / 1e12
    log("per-op means over an instrumented pass (ms): " + ", ".join(f"{n} {v:.4f}" for n, v in phases.items())
        + f"; instrumented layer {ms_instr:.4f} ms")
    log(f"layer {ms:.4f} ms ({wall / args.steps * 1e3:.4f} ms wall per step), {tflops:.1f} TFLOP/s active, "
        f"{100 * tflops / PEAK_BF16_TFLOPS:.1f}% of bf16 peak")

    result = {
        "metric": LAYER_METRICS[args.workload],
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"{args.workload}: MoE FFN layer forward, {t} tokens, H={h}, E={e}, I={i}, top-{k}, "
                        f"fp32 router" + (f", logit bias N(0,{bias})" if bias else ""),
            "tokens": t, "hidden": h, "experts": e, "inter": i, "top_k": k,
            "weight_copies": len(layers),
        },
        "ms_per_layer": round(ms, 5),
        "pct_bf16_peak": round(100 * tflops / PEAK_BF16_TFLOPS, 2),
        "phase_ms": {n: round(v, 5) for n, v in phases.items()},
        "phase_pass_ms_per_layer": round(ms_instr, 5),
        "roofline": {
            "kernel": f"{gate_up_kernel} (fused gather + gate_up GEMM + SwiGLU)",
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": None,
            "flops_per_launch": gate_up_flops,
            "avg_launch_ms": round(gate_up_ms, 5),
        },
    }
    traffic = read_traffic(f"gate_up_swiglu_{args.workload}_traffic.txt", gate_up_kernel)
    if traffic is not None:
        result["roofline"]["traffic"] = traffic["fetch_bytes_per_launch"] + traffic["write_bytes_per_launch"]
        result["roofline"]["traffic_detail"] = traffic
    if not args.no_cpu_baseline:
        legs = []
        if args.workload == "l64x8" and not args.no_cpu_legs:
            xl = WORKLOADS["xl_skew"]
            legs = [("l64x8", t, h, e, i, k, bias, torch.float32),
                    ("xl_skew", xl[0], xl[1], xl[2], xl[3], xl[4], xl[5], torch.bfloat16),
                    ("xl_skew", xl[0], xl[1], xl[2], xl[3], xl[4], xl[5], torch.float32)]
        result["cpu_baseline"] = cpu_baseline(t, h, e, i, k, bias, legs=legs)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
