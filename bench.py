"""Benchmark of the TR-MoE layer hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c2_bf16_prefill_16384]

A step is one forward of one TR-MoE layer (TRHashEngine, HIP backend) over
one batch of synthetic, seeded input already resident in HBM: route
partition (K1), routed experts (K3), shared gate|up + SwiGLU (K2), shared
down + un-permute + combine (K4).  ``value`` is tokens/s of the whole step.

Per-kernel durations are measured live with HIP events recorded on the
stream the kernels run on (torch's current stream), around every kernel of
every timed step.  ``roofline`` reports the kernel with the largest share of
the step against MI355X's published dense peak (MFMA-bound GEMMs) or HBM
bandwidth.  ``cpu_baseline`` times the CPU oracle (the reference's universal
PyTorch dispatch restated, torch fp32 on the host cores) on a bounded sample
of the same workload.  Prints one JSON line.
"""

from __future__ import annotations

import argparse
import gc
import json
import os
import statistics
import sys
import time
from pathlib import Path
from typing import Optional

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "complexity-framework_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "TR-MoE layer tokens/sec @200M shape (prefill+decode); MFMA% / HBM GB/s"
PEAK = {"bf16": 2500.0, "fp8": 2500.0, "fp32": 157.3}   # dense TFLOP/s (fp8 weights run bf16 MFMA)
HBM_PEAK = 8000.0                                         # GB/s


def _kernel_work(w, n_tokens, strategy):
    """Algorithmic FLOPs and bytes per launch of each kernel.  FLOPs count only
    the useful work of the layer (6 N H (S + k W) in total, split by kernel);
    the dense-routed kernels also execute the masked experts, which is not
    credited.  Bytes count each kernel's operands and outputs once."""
    H, S, E, k = w.hidden, w.shared, w.active_experts or w.experts, w.top_k
    Wd = w.active_width or w.width
    act = 4 if w.dtype == "fp32" else 2
    wb = {"fp32": 4, "bf16": 2, "fp8": 1}[w.dtype]
    N = n_tokens
    work = {
        "route_sort": dict(flops=0.0, bytes=8 * N + 8 * k * N * 2 + 8 * k * N),
        "routed_experts": dict(flops=6.0 * N * H * k * Wd,
                               bytes=act * k * N * H + wb * 3 * E * H * Wd + act * k * N * H),
        "shared_gate_up": dict(flops=4.0 * N * H * S, bytes=act * N * H + wb * 2 * S * H + act * N * S),
        "shared_down_combine": dict(flops=2.0 * N * S * H,
                                    bytes=act * N * S + wb * S * H + act * k * N * H + act * N * H),
    }
    if strategy == "dense":
        F = S + E * Wd
        work["dense_routed_gate_up"] = dict(flops=4.0 * N * H * (S + k * Wd),
                                            bytes=act * N * H + wb * 2 * F * H + act * N * F)
        work["shared_down_combine"] = dict(flops=2.0 * N * H * (S + k * Wd),
                                           bytes=act * N * F + wb * F * H + act * N * H)
    return work


class KernelTimer:
    """Wraps the ops entry points so every launch is bracketed by events."""

    NAMES = ("route_sort", "routed_experts", "shared_gate_up", "shared_down_combine", "combine",
             "dense_routed_gate_up")

    def __init__(self, ops, torch):
        self.ops, self.torch = ops, torch
        self.enabled = False
        self.events = {n: [] for n in self.NAMES}
        self._orig = {}
        for name in self.NAMES:
            fn = getattr(ops, name)
            self._orig[name] = fn
            setattr(ops, name, self._wrap(name, fn))

    def _wrap(self, name, fn):
        def wrapped(*a, **kw):
            if not self.enabled:
                return fn(*a, **kw)
            s = self.torch.cuda.Event(enable_timing=True)
            e = self.torch.cuda.Event(enable_timing=True)
            s.record()
            out = fn(*a, **kw)
            e.record()
            self.events[name].append((s, e))
            return out

        return wrapped

    def averages_ms(self):
        out = {}
        for name, evs in self.events.items():
            if evs:
                out[name] = sum(s.elapsed_time(e) for s, e in evs) / len(evs)
        return out

    def restore(self):
        for name, fn in self._orig.items():
            setattr(self.ops, name, fn)


def cpu_baseline(w, sample_tokens: int, reps: int = 5):
    """Oracle forward (torch fp32 CPU) on the first `sample_tokens` tokens."""
    import torch

    from complexity_amd import workloads
    from oracle import trmoe_oracle as O

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    x = workloads.make_hidden(w).reshape(1, -1, w.hidden)[:, :sample_tokens]
    ids = workloads.make_token_ids(w).reshape(1, -1)[:, :sample_tokens]
    p = workloads.make_weights(w)
    params = {k.replace(".weight", ""): v for k, v in p.items()}
    table = torch.from_numpy(O.multi_hash_table(w.vocab, w.experts, w.top_k, w.layer_index))
    if w.active_experts:
        table = torch.from_numpy(O.multi_hash_table(w.vocab, w.active_experts, w.top_k, w.layer_index))
    rw = (1.0 / w.top_k,) * w.top_k

    def run():
        return O.engine_forward(x, ids, table, params, route_weights=rw,
                                active_experts=w.active_experts, active_width=w.active_width)

    for _ in range(2):
        run()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    try:
        model = next(line.split(":", 1)[1].strip() for line in open("/proc/cpuinfo") if "model name" in line)
    except Exception:
        model = "unknown"
    return {
        "value": sample_tokens / med,
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{sample_tokens} tokens of {w.name}, fp32 torch CPU oracle (masked dense per-expert loop), "
                  f"median of {reps} after 2 warm-ups, {model}",
    }


def decode_hbm(torch, workloads, dev, w=None, layers: int = 16, steps: int = 50, warmup: int = 5,
               per_layer_tables: bool = False, block: Optional[str] = None):
    """Decode: w's tokens (C3: 64; C4: 8) through `layers` distinct weight sets
    per step (286 MB of bf16 weights > the 256 MB Infinity Cache), per-layer
    time and HBM GB/s.  per_layer_tables: layer i routes with layer_index i
    (C4's 16-layer model).

    A decode step of the stack is captured once as a HIP graph (the serving
    form of the reference's CUDA_GRAPH backend, engine.py:597-716) and
    replayed; the eager per-layer time is reported beside it.

    block: the MLP half of a decoder block instead of the bare layer,
    x + mlp(rmsnorm(x)) (block.py:271-278): "fused" runs
    forward_norm_residual (the norm inside the gate|up kernel, the residual in
    the down epilogue); "unfused" runs the norm as torch ops and then
    forward_with_residual."""
    w = w or workloads.C3
    engines = [workloads.build_engine(w, dev, backend="hip", seed=i,
                                      **({"layer_index": i} if per_layer_tables else {}))
               for i in range(layers)]
    x = workloads.make_hidden(w).to(dev).to(torch.bfloat16)
    ids = workloads.make_token_ids(w).to(dev)

    nw = (torch.rand(w.hidden, generator=torch.Generator().manual_seed(5)) + 0.5).to(dev).to(torch.bfloat16)

    def layer(e):
        if block == "fused":
            return e.forward_norm_residual(x, ids, nw, 1e-6)
        if block == "unfused":
            normed = nw * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6))
            return e.forward_with_residual(normed, ids, x)
        return e(x, ids)

    def stack():
        out = None
        for e in engines:
            out = layer(e)
        return out

    def timed(fn, n):
        torch.cuda.synchronize()
        gc.collect()
        gc.disable()
        sustain(torch, fn, 3)
        s, t = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(n):
            fn()
        t.record()
        torch.cuda.synchronize()
        gc.enable()
        return s.elapsed_time(t) / (n * layers)

    H, S, E, Wd = w.hidden, w.shared, w.experts, w.width
    weight_bytes = 2 * (3 * H * S + 3 * E * H * Wd)
    bytes_per_layer = weight_bytes + 2 * 2 * w.tokens * H + 8 * w.tokens + 8 * 2 * w.tokens

    def graphed(fn):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn()
        side.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fn()
        return graph

    with torch.no_grad():
        for _ in range(warmup):
            stack()
        eager_ms = timed(stack, steps)
        per_layer_ms = timed(graphed(stack).replay, steps)
        floor_ms = None
        if block is None:
            # the same bytes per layer in one streaming launch each (16
            # distinct buffers, as many bytes as the layers' weights), replayed
            # the same way: the gap to it is what the two kernels lose
            from complexity_amd import ops

            bufs = [torch.full(((bytes_per_layer + 15) // 16 * 4,), i, dtype=torch.int32, device=dev)
                    for i in range(layers)]
            sink = torch.empty(1024, dtype=torch.int32, device=dev)

            def streams():
                for b in bufs:
                    ops.stream_read(b, sink)

            floor_ms = timed(graphed(streams).replay, steps)
            del bufs
    gbps = bytes_per_layer / (per_layer_ms * 1e-3) / 1e9
    name = w.name if block is None else f"{w.name}_block_{block}"
    out = {
        "workload": name,
        "layers_rotated": layers,
        "mode": "hip_graph_replay",
        "ms_per_layer": per_layer_ms,
        "eager_ms_per_layer": eager_ms,
        "tokens_per_s": w.tokens / (per_layer_ms * 1e-3),
        "hbm_gbps": gbps,
        "hbm_frac": gbps / HBM_PEAK,
        "algorithmic_bytes_per_layer": bytes_per_layer,
    }
    if floor_ms is not None:
        out["stream_floor_us_per_layer"] = floor_ms * 1e3
        out["stream_floor_gbps"] = bytes_per_layer / (floor_ms * 1e-3) / 1e9
        out["kernel_loss_us_per_layer"] = (per_layer_ms - floor_ms) * 1e3
        out["roofline"] = {"bound": "hbm", "achieved": gbps, "peak": HBM_PEAK, "unit": "GB/s",
                           "frac": gbps / HBM_PEAK, "traffic": measured_traffic(w.name, "decode_layer"),
                           "kernel": "decode layer (gate|up + down launches)",
                           "algorithmic_bytes_per_launch": bytes_per_layer, "avg_us": per_layer_ms * 1e3}
    return out


def c5_layer(torch, workloads, ops, dev, steps: int = 10, warmup: int = 3):
    """C5: the fp8-e4m3 W8A16 layer at 32768 tokens (E=16, H=2048, S=5632,
    W=256), the quantised path the north star names.  The MFMAs run in bf16,
    so the roofline uses the bf16 dense peak."""
    w = workloads.C5
    engine = workloads.build_engine(w, dev, backend="hip")
    x = workloads.make_hidden(w).to(dev).to(torch.bfloat16)
    ids = workloads.make_token_ids(w).to(dev)
    timer = KernelTimer(ops, torch)
    try:
        ms, kernel_ms, _, strategy = time_engine(torch, engine, x, ids, steps, warmup, timer)
    finally:
        timer.restore()
    kernels, _, roof = kernel_report(w, kernel_ms, strategy)
    tflops = w.flops() / (ms * 1e-3) / 1e12
    out = {"workload": w.name, "ms_per_layer": ms, "tokens_per_s": w.tokens / (ms * 1e-3),
           "layer_tflops": tflops, "layer_mfma_frac": tflops / PEAK["fp8"], "strategy": strategy,
           "kernels": kernels, "roofline": roof}
    out["w8a8"] = c5_w8a8(torch, engine, w, x, ids, ops, steps, warmup)
    return out


def c5_w8a8(torch, engine, w, x, ids, ops, steps: int, warmup: int):
    """The same C5 layer with fp8_activations (W8A8; no reference counterpart,
    and not C5's W8A16 configuration, so reported beside it).  True: x
    quantized per token to e4m3 into the shared gate|up on the e4m3 MFMA,
    which writes h as e4m3 with a power-of-two scale per 32 features into
    the shared down on the scaled e4m3 MFMA.  "gate_up": the gate|up only.
    The shared ops are priced against the 5.0 PFLOP/s fp8 peak."""
    flat = x.reshape(-1, w.hidden)
    packed = engine._hip_packed()

    def ev(fn, n):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(n):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / n

    try:
        with torch.no_grad():
            gc.collect()
            gc.disable()
            engine.fp8_activations = "gate_up"
            sustain(torch, lambda: engine(x, ids), warmup)
            gate_up_only_ms = ev(lambda: engine(x, ids), steps)
            engine.fp8_activations = True
            sustain(torch, lambda: engine(x, ids), warmup)
            layer_ms = ev(lambda: engine(x, ids), steps)
            xq, xs = ops.quantize_rows_e4m3(flat)
            quant_ms = ev(lambda: ops.quantize_rows_e4m3(flat), steps)
            args = (xq, xs, packed.shared_gate_up, packed.shared_gate_up_scale, packed.shared_width)
            gemm_ms = ev(lambda: ops.shared_gate_up_a8(*args), steps)
            hq, hs = ops.shared_gate_up_a8_mx(*args)
            gemm_mx_ms = ev(lambda: ops.shared_gate_up_a8_mx(*args), steps)
            down_ms = ev(lambda: ops.shared_down_combine_a8(hq, hs, packed.shared_width, packed.shared_down,
                                                            packed.shared_down_scale, w.hidden, None, None, 2,
                                                            (0.5, 0.5), 1.0, 1.0), steps)
            gc.enable()
    finally:
        engine.fp8_activations = False
    gu_flops = 4.0 * w.tokens * w.hidden * w.shared
    down_flops = 2.0 * w.tokens * w.hidden * w.shared
    tf = lambda f, ms: f / (ms * 1e-3) / 1e12
    return {"ms_per_layer": layer_ms, "tokens_per_s": w.tokens / (layer_ms * 1e-3),
            "quantize_us": quant_ms * 1e3,
            "shared_gate_up_a8_block_h_us": gemm_mx_ms * 1e3,
            "shared_gate_up_a8_block_h_fp8_frac": tf(gu_flops, gemm_mx_ms) / 5.0e3,
            "shared_down_a8_us": down_ms * 1e3, "shared_down_a8_tflops": tf(down_flops, down_ms),
            "shared_down_a8_fp8_frac": tf(down_flops, down_ms) / 5.0e3,
            "gate_up_only": {"ms_per_layer": gate_up_only_ms, "tokens_per_s": w.tokens / (gate_up_only_ms * 1e-3),
                             "shared_gate_up_a8_us": gemm_ms * 1e3,
                             "shared_gate_up_a8_tflops": tf(gu_flops, gemm_ms),
                             "shared_gate_up_a8_fp8_frac": tf(gu_flops, gemm_ms) / 5.0e3,
                             "shared_gate_up_a8_with_quantize_fp8_frac": tf(gu_flops, gemm_ms + quant_ms) / 5.0e3}}


def c1_layer(torch, workloads, ops, dev, steps: int = 50, warmup: int = 10, cpu: bool = True):
    """C1: the fp32 layer at 2048 tokens (4 x 512, uniform ids), the
    reference's CPU-runnable case, on the HIP backend.  The fp32 GEMMs run on
    v_mfma_f32_32x32x2f32, so the roofline uses the fp32 matrix peak; the CPU
    oracle runs beside it on all 2048 tokens."""
    w = workloads.C1
    engine = workloads.build_engine(w, dev, backend="hip")
    x = workloads.make_hidden(w).to(dev)
    ids = workloads.make_token_ids(w).to(dev)
    timer = KernelTimer(ops, torch)
    try:
        ms, kernel_ms, _, strategy = time_engine(torch, engine, x, ids, steps, warmup, timer)
    finally:
        timer.restore()
    kernels, _, roof = kernel_report(w, kernel_ms, strategy)
    tflops = w.flops() / (ms * 1e-3) / 1e12
    out = {"workload": w.name, "dtype": "f32", "ms_per_layer": ms, "tokens_per_s": w.tokens / (ms * 1e-3),
           "layer_tflops": tflops, "layer_mfma_frac": tflops / PEAK["fp32"], "strategy": strategy,
           "kernels": kernels, "roofline": roof}
    if cpu:
        out["cpu_baseline"] = cpu_baseline(w, w.tokens)
    return out


def c4_e2e(torch, dev, steps: int = 128, reps: int = 3):
    """C4 end to end: the 16-layer TR-GQA 200M decoder (complexity_amd.decoder,
    random-init bf16, HIP TR-MoE layer in every block, SDPA attention).

    Prefill: 8 x 2048 Zipf(1.1) ids through every layer plus the last
    position's logits, timed with HIP events (median of `reps`).  Decode:
    `steps` greedy steps of one token per sequence (8 per step), the step
    captured once as a HIP graph and replayed.  MLP share: prefill from
    events around each block's two halves (a separate instrumented run);
    decode from a graph of the 16 MLP halves alone at the decode shape,
    against the whole step."""
    from complexity_amd import workloads
    from complexity_amd.decoder import TRGQAConfig, TRGQADecoder

    cfg = TRGQAConfig()
    model = TRGQADecoder(cfg).to(dev, torch.bfloat16).init_weights(0).eval()
    ids = workloads.zipf_ids(8 * 2048, cfg.vocab_size, 1.1, torch.Generator().manual_seed(0)).view(8, 2048).to(dev)

    def prefill():
        h = model.prefill(ids, steps + 1, return_logits=False)
        return model.logits(h[:, -1:]).argmax(dim=-1).view(-1)

    def ev():
        return torch.cuda.Event(enable_timing=True)

    with torch.no_grad():
        gc.collect()
        gc.disable()
        prefill()
        torch.cuda.synchronize()
        pre = []
        for _ in range(reps):
            s, e = ev(), ev()
            s.record()
            first = prefill()
            e.record()
            torch.cuda.synchronize()
            pre.append(s.elapsed_time(e))
        prefill_ms = statistics.median(pre)
        timings = {}
        model.prefill(ids, steps + 1, return_logits=False, timings=timings)
        torch.cuda.synchronize()
        attn_ms = sum(s.elapsed_time(e) for s, e in timings["attention"])
        mlp_ms = sum(s.elapsed_time(e) for s, e in timings["mlp"])
        model.capture_decode(8)
        model._g_ids.copy_(first)
        s, e = ev(), ev()
        s.record()
        for _ in range(steps):
            model._graph.replay()
        e.record()
        torch.cuda.synchronize()
        step_ms = s.elapsed_time(e) / steps
        # the MLP halves alone at the decode shape, one graph over 16 layers
        h = (torch.randn(8, 1, cfg.hidden_size, generator=torch.Generator().manual_seed(2)) * 0.5).to(dev, torch.bfloat16)
        tok = first.view(8, 1)

        def mlps():
            out = h
            for b in model.layers:
                n = b.post_attention_layernorm
                out = b.mlp.forward_norm_residual(out, tok, n.weight, n.eps)
            return out

        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            mlps()
        side.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            mlps()
        sustain(torch, graph.replay, 5)
        s, e = ev(), ev()
        s.record()
        for _ in range(steps):
            graph.replay()
        e.record()
        torch.cuda.synchronize()
        mlp_step_ms = s.elapsed_time(e) / steps
        gc.enable()
    return {
        "workload": "c4_tr_gqa_200m_prefill_8x2048_decode_128",
        "layers": cfg.num_layers,
        "prefill_tokens": int(ids.numel()),
        "prefill_ms": prefill_ms,
        "prefill_tokens_per_s": ids.numel() / (prefill_ms * 1e-3),
        "prefill_mlp_share": mlp_ms / (mlp_ms + attn_ms),
        "decode_steps": steps,
        "decode_mode": "hip_graph_replay",
        "decode_ms_per_step": step_ms,
        "decode_tokens_per_s": 8 / (step_ms * 1e-3),
        "decode_mlp_ms_per_step": mlp_step_ms,
        "decode_mlp_share": mlp_step_ms / step_ms,
        "attention": "torch SDPA (flash causal prefill, memory-efficient masked decode)",
    }


def train_step(torch, engine, w, x, ids, steps: int = 10, warmup: int = 3):
    """Forward + backward through autograd on the HIP backend (the layer's
    gradients of x and every weight), timed with HIP events like the forward.
    Useful backward work is twice the forward's FLOPs.  Above 128 tokens the
    forward also stores the raw gate|up outputs and the backward reads them
    back, so it executes exactly that (decode sizes recompute gate|up)."""
    from complexity_amd.tr_hash import TRHashBackend

    xg = x.detach().clone().requires_grad_(True)
    dout = (torch.randn(x.shape, device=x.device) * 0.1).to(x.dtype)

    def step():
        # a training step starts from cleared gradients (no accumulation kernels)
        engine.zero_grad(set_to_none=True)
        xg.grad = None
        out = engine(xg, ids)
        out.backward(dout)

    gc.collect()
    gc.disable()
    warm = sustain(torch, step, warmup)
    assert engine.last_backend.selected is TRHashBackend.HIP, engine.last_backend
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        step()
    stop.record()
    torch.cuda.synchronize()
    gc.enable()
    ms = start.elapsed_time(stop) / steps
    engine.zero_grad(set_to_none=True)
    return {"workload": w.name, "steps": steps, "ms_per_step_fwd_bwd": ms,
            "tokens_per_s": w.tokens / (ms * 1e-3), "useful_tflops": 3 * w.flops() / (ms * 1e-3) / 1e12, **warm}


def norm_train(torch, engine, w, x, ids, steps: int = 20, warmup: int = 5):
    """The block's MLP half under autograd (forward_norm_residual, whose
    RMSNorm runs on trmoe_rmsnorm_forward/_backward there), eager; and the
    norm alone, forward + backward: its kernels replayed as a HIP graph (their
    few tens of us would otherwise measure the host), and the reference's
    torch formula (norms.py:53-55) under autograd, eager (about ten kernels
    over the full tensors: bound by the GPU, and its backward's reductions
    are not captured into a graph here).  The norm's HBM roofline: x and y
    (forward), then x, dy and dx (backward) once each, 5 N H element bytes."""
    from complexity_amd import ops

    h = x.shape[-1]
    nw = (torch.rand(h, device=x.device) + 0.5).to(x.dtype).requires_grad_(True)
    xg = x.detach().clone().requires_grad_(True)
    dout = (torch.randn(x.shape, device=x.device) * 0.1).to(x.dtype)
    flat = xg.detach().reshape(-1, h).clone().requires_grad_(True)
    dflat = dout.reshape(-1, h)

    def block():
        engine.zero_grad(set_to_none=True)
        xg.grad = None
        nw.grad = None
        engine.forward_norm_residual(xg, ids, nw, 1e-6).backward(dout)

    def norm_hip():
        y, r = ops.rmsnorm_forward(flat.detach(), nw.detach(), 1e-6)
        ops.rmsnorm_backward(flat.detach(), nw.detach(), r, dflat)

    def norm_torch():
        flat.grad = None
        nw.grad = None
        var = flat.pow(2).mean(-1, keepdim=True)
        (nw * (flat * torch.rsqrt(var + 1e-6))).backward(dflat)

    def graphed(fn):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                fn()
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        return g.replay

    def timed(fn):
        sustain(torch, fn, warmup)
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            fn()
        stop.record()
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / steps

    out = {"workload": w.name, "steps": steps}
    gc.collect()
    gc.disable()
    out["block_ms_per_step_fwd_bwd"] = timed(block)
    out["norm_path"] = engine.last_norm
    out["norm_hip_graph_us_fwd_bwd"] = timed(graphed(norm_hip)) * 1e3
    out["norm_torch_eager_us_fwd_bwd"] = timed(norm_torch) * 1e3
    gc.enable()
    nbytes = 5 * x.numel() * x.element_size()
    out["norm_hip_hbm_frac"] = nbytes / (out["norm_hip_graph_us_fwd_bwd"] * 1e-6) / (HBM_PEAK * 1e9)
    engine.zero_grad(set_to_none=True)
    return out


# The MI355X raises its clocks over the first tens of ms of sustained load
# (measured: a C2 layer step takes 338 us right after five warm-up steps and
# 277-280 us once ~60 steps have run back to back; after 1 s idle it ramps
# again).  Every leg therefore warms up for at least W steps AND at least
# WARM_S seconds of back-to-back work before its timed region, so that the
# timed steps measure the steady state, not the ramp.
WARM_S = 0.3


def sustain(torch, fn, min_iters: int, min_s: float = WARM_S) -> dict:
    """Run fn at least min_iters times and until min_s seconds have passed;
    returns {"warmup_iters": n, "warmup_s": t}."""
    t0 = time.perf_counter()
    n = 0
    while True:
        fn()
        n += 1
        if n >= min_iters and n % 4 == 0:
            torch.cuda.synchronize()
            if time.perf_counter() - t0 >= min_s:
                break
    torch.cuda.synchronize()
    return {"warmup_iters": n, "warmup_s": time.perf_counter() - t0}


def time_engine(torch, engine, x, ids, steps, warmup, timer):
    """K timed forwards after W warm-ups, then K more with per-op HIP events
    for the kernel averages.  The step time comes from the first loop only:
    an event recorded between two kernels costs the stream ~10 us (measured),
    so the per-op events stay out of the headline figure."""
    from complexity_amd.tr_hash import TRHashBackend

    timer.events = {n: [] for n in timer.NAMES}
    with torch.no_grad():
        # a full collection of the interpreter's heap (torch's import leaves
        # millions of objects) stalls the host for ~40 ms; keep it out of the
        # timed region, as timeit does, and before the warm-up: the GPU idles
        # meanwhile and its clocks drop
        gc.collect()
        gc.disable()
        warm = sustain(torch, lambda: engine(x, ids), warmup)
        assert engine.last_backend.selected is TRHashBackend.HIP, engine.last_backend
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        start.record()
        for _ in range(steps):
            engine(x, ids)
        stop.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        timer.enabled = True
        for _ in range(steps):
            engine(x, ids)
        torch.cuda.synchronize()
        timer.enabled = False
        gc.enable()
    time_engine.last_warm = warm
    return start.elapsed_time(stop) / steps, timer.averages_ms(), wall, engine._packed.strategy


def measured_traffic(workload: str, op: str):
    """HBM bytes per launch of `op` on `workload`, as recorded from rocprofv3
    FETCH_SIZE / WRITE_SIZE runs in profiles/traffic_*.txt (each counter scaled
    by what it reads for a copy kernel of known size); None when absent."""
    for path in sorted((ROOT / "profiles").glob("traffic_*.txt")):
        fields = {}
        for line in path.read_text().splitlines():
            if " = " in line and not line.startswith("#"):
                key, val = line.split(" = ", 1)
                fields[key.strip()] = val.strip()
        if fields.get("workload") == workload and fields.get("op") == op:
            try:
                return float(fields["traffic_bytes_per_launch"])
            except (KeyError, ValueError):
                return None
    return None


def kernel_report(w, kernel_ms, strategy):
    work = _kernel_work(w, w.tokens, strategy)
    kernels = {}
    for name, ms in kernel_ms.items():
        wk = work.get(name, dict(flops=0.0, bytes=0.0))
        kernels[name] = {
            "avg_us": ms * 1e3,
            "tflops": wk["flops"] / (ms * 1e-3) / 1e12 if wk["flops"] else 0.0,
            "gbps": wk["bytes"] / (ms * 1e-3) / 1e9,
        }
    dominant = max(kernel_ms, key=kernel_ms.get)
    dwk = work[dominant]
    dms = kernel_ms[dominant]
    traffic = measured_traffic(w.name, dominant)
    if dwk["flops"]:
        achieved = dwk["flops"] / (dms * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": achieved, "peak": PEAK[w.dtype], "unit": "TFLOP/s",
                "frac": achieved / PEAK[w.dtype], "traffic": traffic, "kernel": dominant,
                "algorithmic_flops_per_launch": dwk["flops"], "algorithmic_bytes_per_launch": dwk["bytes"],
                "avg_us": dms * 1e3}
    else:
        achieved = dwk["bytes"] / (dms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK, "unit": "GB/s",
                "frac": achieved / HBM_PEAK, "traffic": traffic, "kernel": dominant,
                "algorithmic_bytes_per_launch": dwk["bytes"], "avg_us": dms * 1e3}
    return kernels, dominant, roof


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="c2_bf16_prefill_16384")
    ap.add_argument("--cpu-sample", type=int, default=4096)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-other", action="store_true", help="skip timing the second routed strategy")
    ap.add_argument("--no-train", action="store_true", help="skip the forward+backward (autograd) timing")
    ap.add_argument("--no-c4", action="store_true", help="skip the 16-layer TR-GQA decoder (C4) end to end")
    ap.add_argument("--no-c5", action="store_true", help="skip the fp8 W8A16 layer (C5)")
    ap.add_argument("--no-c1", action="store_true", help="skip the fp32 C1 layer (2048 tokens) and its CPU leg")
    ap.add_argument("--no-block", action="store_true",
                    help="skip the decode block legs (the C3 MLP half with its norm fused / unfused)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="end with three elementwise copies of MIB MiB (reference kernel for HBM counters)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(json.dumps({"error": "this build measures one GPU only: the TR-MoE layer shards by tokens "
                          "with no communication in forward, so N GPUs run N independent copies; "
                          "run with --gpus 1"}))
        sys.exit(2)

    import torch

    from complexity_amd import _native, ops, workloads
    from complexity_amd.tr_hash import TRHashBackend

    _native.load()
    dev = torch.device("cuda:0")
    w = workloads.WORKLOADS[args.workload]
    engine = workloads.build_engine(w, dev, backend="hip")
    act = torch.float32 if w.dtype == "fp32" else torch.bfloat16
    x = workloads.make_hidden(w).to(dev).to(act)
    ids = workloads.make_token_ids(w).to(dev)

    timer = KernelTimer(ops, torch)
    ms_per_step, kernel_ms, wall, strategy = time_engine(torch, engine, x, ids, args.steps, args.warmup, timer)
    head_warm = time_engine.last_warm
    kernels, dominant, roof = kernel_report(w, kernel_ms, strategy)
    secondary = {}
    other = "grouped" if strategy == "dense" and not args.no_other else None
    if other is not None:
        engine.routed_strategy = other
        ms2, kms2, _, _ = time_engine(torch, engine, x, ids, args.steps, args.warmup, timer)
        k2, _, _ = kernel_report(w, kms2, other)
        secondary = {"strategy": other, "ms_per_step": ms2, "tokens_per_s": w.tokens / (ms2 * 1e-3),
                     "kernels": k2}
        engine.routed_strategy = "auto"
    timer.restore()
    tokens = w.tokens

    layer_tflops = w.flops() / (ms_per_step * 1e-3) / 1e12
    result = {
        "metric": METRIC,
        "value": tokens / (ms_per_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_steps_run": head_warm["warmup_iters"],
        "warmup_s": head_warm["warmup_s"],
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"fp32": "f32", "bf16": "bf16", "fp8": "fp8e4m3 weights / bf16 act"}[w.dtype],
        "data": "synthetic (seeded Zipf(1.1) token ids, x~N(0,1), weights~N(0,0.02))",
        "config": {"workload": w.name, "tokens": tokens, "batch": w.batch, "seq": w.seq, "hidden": w.hidden,
                   "shared_width": w.shared, "experts": w.experts, "expert_width": w.width, "top_k": w.top_k,
                   "routing": "token_id_multi_hash", "vocab": w.vocab, "parallelism": "single_gpu"},
        "layer_tflops": layer_tflops,
        "layer_mfma_frac": layer_tflops / PEAK[w.dtype],
        "wall_s_timed": wall,
        "strategy": strategy,
        "kernels": kernels,
        "roofline": roof,
        "other_strategy": secondary,
        "backend": engine.last_backend.selected.value,
        "device": torch.cuda.get_device_name(0),
    }
    if not args.no_train and w.dtype != "fp8":
        train = train_step(torch, engine, w, x, ids)
        train["backward_ms"] = train["ms_per_step_fwd_bwd"] - ms_per_step
        result["train"] = train
        result["train_block"] = norm_train(torch, engine, w, x, ids)
    if not args.no_decode:
        result["decode"] = decode_hbm(torch, workloads, dev)
        result["decode_c4"] = decode_hbm(torch, workloads, dev, w=workloads.C4_DECODE, per_layer_tables=True)
        if not args.no_block:
            # the block's MLP half with the post-attention RMSNorm and residual
            # fused (F2) and unfused, C3
            fused = decode_hbm(torch, workloads, dev, block="fused")
            unfused = decode_hbm(torch, workloads, dev, block="unfused")
            result["decode_block"] = {
                "workload": workloads.C3.name,
                "fused_us_per_layer": fused["ms_per_layer"] * 1e3,
                "unfused_us_per_layer": unfused["ms_per_layer"] * 1e3,
            }
    if not args.no_c4:
        result["c4_e2e"] = c4_e2e(torch, dev)
    if not args.no_c1 and w.name != workloads.C1.name:
        result["c1"] = c1_layer(torch, workloads, ops, dev, cpu=not args.no_cpu)
    if not args.no_c5 and w.name != workloads.C5.name:
        result["c5"] = c5_layer(torch, workloads, ops, dev)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(w, min(args.cpu_sample, tokens))
    if args.calibrate_copy:
        n = args.calibrate_copy << 20
        src = torch.ones(n // 2, dtype=torch.bfloat16, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        result["calibration_copy_bytes"] = n
    print(json.dumps(result))


if __name__ == "__main__":
    main()
