#!/usr/bin/env python3
"""MoE layer throughput on one MI355X at the Gemma 4 26B-A4B shape (hidden 2816, 128 experts, top-8,
expert FFN 704).

    python bench.py [--steps K] [--warmup W] [--config C] [--configs 2,3,4] [--eager] [--no-cpu]

A step is one MoE layer over one batch of synthetic tokens, from router logits to the combined [T, H]
output, exactly the calls Gemma 4's fused decoder makes (flide/backbones/gemma4/fused.py:236-240):
moe.route(logits, k, scale) -> moe.experts(x, w, top, ids, GeGLU) -> moe.combine_norm(y, dense, w1, w2).
The layer is captured once into a HIP graph and replayed, as the reference serves it
(flide/backbones/gemma4/graphs.py:193-215); --eager launches it op by op instead.

Prints one JSON line. Its top level is the headline workload (--config, default 1: decode, 64 tokens):
tokens/s of the whole step (inputs resident in HBM), the roofline of the dominant kernel (the gate/up
grouped product with GeGLU fused, timed with HIP events on the stream it runs on), and the reference's
CPU torch path timed on this host's cores on a bounded sample. `configs` holds the same measurements for
the other BASELINE workloads (--configs, default 2,3,4: prefill bf16, FP8, skewed), each with its layer
step, its gate/up and down products against their rooflines.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

HBM_PEAK = 8.0e12          # bytes/s, MI355X HBM3E
MFMA_PEAK = {"bf16": 2.5e15, "fp8": 5.0e15}   # dense FLOP/s


def _usable_cores() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    try:   # cgroup v2 quota
        q, p = open("/sys/fs/cgroup/cpu.max").read().split()
        if q != "max":
            n = min(n, max(1, int(int(q) / int(p))))
    except (OSError, ValueError):
        pass
    return max(1, n)


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


class Layer:
    """One workload's tensors on the GPU, its layer step and its two expert products launched alone."""

    def __init__(self, cfg, dev, weights_on_device: bool):
        import torch

        from flide_amd import workloads
        from flide_amd.kernels import moe

        self.cfg, self.dev = cfg, dev
        self.fp8 = cfg.dtype == "fp8"
        if weights_on_device:
            d = workloads.make_inputs(cfg, seed=0, with_weights=False)
            d.update(workloads.device_weights(cfg, dev, seed=0))
        else:
            d = workloads.make_inputs(cfg, seed=0)
        self.host = d
        self.logits = d["logits"].to(dev)
        self.x = d["x"].to(dev)
        w = {"experts": d["w_gu"].to(dev), "experts_down": d["w_d"].to(dev), "inter": cfg.I, "topk": cfg.k}
        if self.fp8:
            w["experts_scale"] = d["w_gu_scale"].to(dev)
            w["experts_down_scale"] = d["w_d_scale"].to(dev)
        self.w = w
        self.scale = torch.ones(cfg.E, dtype=torch.bfloat16, device=dev)   # Gemma per_expert_scale
        self.dense = self.x.clone()                                          # the dense MLP branch's output
        self.w1 = torch.ones(cfg.H, dtype=torch.bfloat16, device=dev)
        self.w2 = torch.ones(cfg.H, dtype=torch.bfloat16, device=dev)

        # the two products alone, on this routing, for the kernel timings
        top, ids = moe.route(self.logits, cfg.k, self.scale)
        self.bm = moe.tile(cfg.pairs, self.fp8)[0]
        self.rows, self.blocks, self.used = moe.align(ids, cfg.E, self.bm)
        counts = torch.bincount(ids.flatten().long(), minlength=cfg.E)
        self.n_hit = int((counts > 0).sum().item())
        self.top = top
        self.act = torch.empty(cfg.pairs, cfg.I, dtype=self.x.dtype, device=dev)
        self.y = torch.empty(cfg.pairs, cfg.H, dtype=self.x.dtype if self.fp8 else torch.float32, device=dev)
        if self.fp8:
            from flide_amd.kernels.fp8 import quantize_tokens
            self.qx, self.sx = quantize_tokens(self.x)
        self.gate_up()
        if self.fp8:
            self.qa, self.sa = quantize_tokens(self.act)

    def step(self):
        from flide_amd.kernels import moe
        from flide_amd.kernels import pointwise as pw

        def act(gu, n):   # Gemma's activation callable (flide/backbones/gemma4/fused.py:238)
            return pw.geglu(gu[:, :n], gu[:, n:])

        cfg = self.cfg
        top, ids = moe.route(self.logits, cfg.k, self.scale)
        y = moe.experts(self.x, self.w, top, ids, act)
        return moe.combine_norm(y, self.dense, self.w1, self.w2, cfg.k, 1e-6)

    def _grouped(self, a, sa, w, ws, N, K, out, out_dtype, weights, by_token, act):
        from flide_amd import _hip

        c, st = self.cfg, _hip.stream(self.dev)
        if self.fp8:
            _hip.call("flide_moe_grouped_fp8", a.data_ptr(), a.stride(0), sa.data_ptr(), w.data_ptr(), w.stride(0),
                      w.stride(1), ws.data_ptr(), ws.stride(0), N, K, out.data_ptr(), out.stride(0), out_dtype,
                      _hip.ptr(weights), self.rows.data_ptr(), self.blocks.data_ptr(), self.used.data_ptr(),
                      c.pairs, self.blocks.shape[0], c.k, by_token, act, self.bm, 0, st)
        else:
            _hip.call("flide_moe_grouped", a.data_ptr(), a.stride(0), _hip.BF16, w.data_ptr(), w.stride(0),
                      w.stride(1), N, K, out.data_ptr(), out.stride(0), out_dtype, _hip.ptr(weights),
                      self.rows.data_ptr(), self.blocks.data_ptr(), self.used.data_ptr(), c.pairs,
                      self.blocks.shape[0], c.k, by_token, act, self.bm, 0, st)

    def gate_up(self):
        from flide_amd import _hip

        c, w = self.cfg, self.w
        a, sa = (self.qx, self.sx) if self.fp8 else (self.x, None)
        self._grouped(a, sa, w["experts"], w.get("experts_scale"), 2 * c.I, c.H, self.act, _hip.BF16, None, 1,
                      _hip.ACT_GEGLU)

    def down(self):
        from flide_amd import _hip

        c, w = self.cfg, self.w
        a, sa = (self.qa, self.sa) if self.fp8 else (self.act, None)
        self._grouped(a, sa, w["experts_down"], w.get("experts_down_scale"), c.H, c.I, self.y,
                      _hip.BF16 if self.fp8 else _hip.F32, self.top.reshape(-1), 0, _hip.ACT_NONE)

    # ---- timings ------------------------------------------------------------------------------------
    def time_steps(self, steps: int, warmup: int, eager: bool) -> float:
        """Seconds per layer step: W warmup steps, then K steps between two synchronisations."""
        import torch

        for _ in range(max(1, warmup)):
            self.step()
        torch.cuda.synchronize()
        graph = None
        if not eager:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self.step()
            for _ in range(max(1, warmup)):
                graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            if graph is not None:
                graph.replay()
            else:
                self.step()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps

    def time_kernel(self, fn, reps: int) -> float:
        """Average seconds of one launch of `fn`, timed in layer context: each rep runs a whole layer
        step, then `fn` once between two HIP events on the stream both launch on (torch's current stream),
        so the kernel runs at the clock the layer sustains."""
        import torch

        for _ in range(3):
            fn()
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
        torch.cuda.synchronize()
        for ev0, ev1 in evs:
            self.step()
            ev0.record()
            fn()
            ev1.record()
        torch.cuda.synchronize()
        return sum(ev0.elapsed_time(ev1) for ev0, ev1 in evs) / 1e3 / len(evs)

    # ---- algorithmic work ---------------------------------------------------------------------------
    def bytes_gate_up(self) -> int:
        c, bw = self.cfg, 1 if self.fp8 else 2
        return self.n_hit * 2 * c.I * c.H * bw + c.T * c.H * bw + c.pairs * c.I * 2

    def bytes_down(self) -> int:
        c, bw = self.cfg, 1 if self.fp8 else 2
        return self.n_hit * c.H * c.I * bw + c.pairs * c.I * bw + c.pairs * c.H * (2 if self.fp8 else 4)

    def flops_gate_up(self) -> int:
        return self.cfg.pairs * 2 * self.cfg.H * 2 * self.cfg.I

    def flops_down(self) -> int:
        return self.cfg.pairs * 2 * self.cfg.I * self.cfg.H


def _roofline(layer: Layer, k_s: float, flops: int, nbytes: int, bound: str, kernel: str) -> dict:
    if bound == "hbm":
        roof = {"bound": "hbm", "achieved": nbytes / k_s / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s"}
    else:
        peak = MFMA_PEAK["fp8" if layer.fp8 else "bf16"]
        roof = {"bound": "mfma", "achieved": flops / k_s / 1e12, "peak": peak / 1e12, "unit": "TFLOP/s"}
    roof["frac"] = roof["achieved"] / roof["peak"]
    if bound == "mfma":   # the other roofline of the same launch, on its algorithmic bytes
        roof["hbm_frac"] = nbytes / k_s / HBM_PEAK
    roof["kernel"] = kernel
    roof["kernel_us"] = k_s * 1e6
    roof["algorithmic_bytes"] = nbytes
    return roof


def measure(layer: Layer, steps: int, warmup: int, eager: bool, reps: int) -> dict:
    """The layer step and both products of one workload."""
    from flide_amd.rocprof import traffic_for

    cfg = layer.cfg
    step_s = layer.time_steps(steps, warmup, eager)
    bound = "hbm" if cfg.idx == 1 else "mfma"
    prec = "fp8" if layer.fp8 else "bf16"
    gu = _roofline(layer, layer.time_kernel(layer.gate_up, reps), layer.flops_gate_up(), layer.bytes_gate_up(),
                   bound, f"grouped gate/up + GeGLU ({prec}, bm {layer.bm})")
    gu["traffic"] = traffic_for(cfg.name)
    dn = _roofline(layer, layer.time_kernel(layer.down, reps), layer.flops_down(), layer.bytes_down(), bound,
                   f"grouped down x weight ({prec}, bm {layer.bm})")
    dn["traffic"] = traffic_for(cfg.name, "down")
    # the whole layer against the same peak: for decode the bytes it must read (every hit expert's weights
    # and the activations; the timed step starts at the logits, so the router's table is not among them),
    # for prefill the expert FLOPs
    if bound == "hbm":
        lb = layer.n_hit * 3 * cfg.I * cfg.H * (1 if layer.fp8 else 2) + cfg.T * cfg.H * 2
        gu["layer"] = {"achieved": lb / step_s / 1e9, "frac": lb / step_s / HBM_PEAK, "bytes": lb}
    else:
        gu["layer"] = {"achieved": cfg.flops / step_s / 1e12, "frac": cfg.flops / step_s / gu["peak"] / 1e12}
    return {"step_s": step_s, "roofline": gu, "down": dn}


def cpu_baseline(layer: Layer, seconds: float) -> dict:
    """The reference's CPU torch path (fp32) on this host's cores, on a bounded sample of the workload."""
    import torch

    from oracle import cpu_path

    cfg, d = layer.cfg, layer.host
    ncores = _usable_cores()
    torch.set_num_threads(ncores)
    lg, xc = d["logits"].float(), d["x"].float()
    if layer.fp8:
        wgu = d["w_gu"].float() * d["w_gu_scale"].unsqueeze(-1)
        wd = d["w_d"].float() * d["w_d_scale"].unsqueeze(-1)
    else:
        wgu, wd = d["w_gu"].float(), d["w_d"].float()
    wgu, wd = wgu.cpu(), wd.cpu()
    Tc = min(cfg.T, 512)   # whole layers for small T, else the first Tc tokens of the same batch
    lg, xc = lg[:Tc], xc[:Tc]
    cpu_path.layer_cpu(lg, xc, wgu, wd, cfg.k)        # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < seconds and len(times) < 50):
        t1 = time.perf_counter()
        cpu_path.layer_cpu(lg, xc, wgu, wd, cfg.k)
        times.append(time.perf_counter() - t1)
    times.sort()
    med = times[len(times) // 2]
    return {"value": Tc / med, "unit": "tokens/s", "cores": ncores, "kind": "port",
            "sample": f"{len(times)} runs (median) of route+experts on {Tc} of the {cfg.T} tokens, fp32, "
                      f"torch CPU (transformers' eager Gemma 4 experts loop restated), {_cpu_model()}"}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=1, help="BASELINE config of the headline line (1 = decode)")
    ap.add_argument("--configs", default="2,3,4", help="other BASELINE configs reported in the same line")
    ap.add_argument("--config-steps", type=int, default=50, help="timed layer steps for each of --configs")
    ap.add_argument("--eager", action="store_true", help="launch op by op instead of replaying a HIP graph")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline sample budget")
    ap.add_argument("--kernel-reps", type=int, default=50)
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this build's MoE layer keeps all experts on one MI355X (no "
              "expert-parallel path is built); run it with --gpus 1", file=sys.stderr)
        return 2

    import torch

    from flide_amd import _hip, workloads

    extra = [int(c) for c in args.configs.split(",") if c.strip()]
    if any(workloads.CONFIGS[c].dtype == "fp32" for c in [args.config] + extra):
        print("config 0 is the CPU plumbing case; the GPU bench runs configs 1-4", file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    _hip.load()

    cfg = workloads.CONFIGS[args.config]
    head = Layer(cfg, dev, weights_on_device=True)
    m = measure(head, args.steps, args.warmup, args.eager, args.kernel_reps)
    step_s = m["step_s"]
    cpu = None
    if not args.no_cpu and int(os.environ.get("RANK", "0")) == 0:
        cpu = cpu_baseline(head, args.cpu_seconds)
    n_hit = head.n_hit
    del head
    torch.cuda.empty_cache()

    configs = {}
    for c in extra:
        if c == args.config:
            continue
        ccfg = workloads.CONFIGS[c]
        lay = Layer(ccfg, dev, weights_on_device=True)
        mc = measure(lay, args.config_steps, 5, args.eager, max(5, args.kernel_reps // 5))
        configs[ccfg.name] = {
            "tokens": ccfg.T, "dtype": ccfg.dtype, "bm": lay.bm, "hit_experts": lay.n_hit,
            "value": ccfg.T / mc["step_s"], "unit": "tokens/s", "ms_per_step": mc["step_s"] * 1e3,
            "steps": args.config_steps, "layer_tflops": ccfg.flops / mc["step_s"] / 1e12,
            "roofline": mc["roofline"], "down": mc["down"]}
        del lay
        torch.cuda.empty_cache()

    rec = {
        "metric": "MoE layer tokens/s @ 26B-A4B shape, bf16 & FP8; % of HBM/MFMA peak",
        "value": cfg.T / step_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_s * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8" if cfg.dtype == "fp8" else "bf16",
        "data": "synthetic: seeded N(0,1) logits/activations drawn on the host (config 4: Zipf-biased logits), "
                "random-init N(0,0.02) expert weights drawn on the GPU",
        "config": {"workload": cfg.name, "tokens": cfg.T, "hidden": cfg.H, "experts": cfg.E, "topk": cfg.k,
                   "expert_ffn": cfg.I, "hit_experts": n_hit, "graph": not args.eager,
                   "layer_tflops": cfg.flops / step_s / 1e12},
        "roofline": m["roofline"],
        "down": m["down"],
        "cpu_baseline": cpu,
        "configs": configs,
    }
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
