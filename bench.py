#!/usr/bin/env python3
"""MoE layer throughput on one MI355X at the Gemma 4 26B-A4B shape (hidden 2816, 128 experts, top-8,
expert FFN 704).

    python bench.py [--steps K] [--warmup W] [--config C] [--eager] [--no-cpu]

A step is one MoE layer over one batch of synthetic tokens, from router logits to the combined [T, H]
output, exactly the calls Gemma 4's fused decoder makes (flide/backbones/gemma4/fused.py:236-240):
moe.route(logits, k, scale) -> moe.experts(x, w, top, ids, GeGLU) -> moe.combine_norm(y, dense, w1, w2).
The layer is captured once into a HIP graph and replayed, as the reference serves it
(flide/backbones/gemma4/graphs.py:193-215); --eager launches it op by op instead.

Prints one JSON line: tokens/s of the whole step (inputs resident in HBM), the roofline of the dominant
kernel (the gate/up grouped product with GeGLU fused, timed alone with HIP events on the stream it runs
on), and the reference's CPU torch path timed on this host's cores on a bounded sample.
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


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=1, help="BASELINE config index (1 = decode, the headline)")
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
    from flide_amd.kernels import moe
    from flide_amd.kernels import pointwise as pw

    cfg = workloads.CONFIGS[args.config]
    if cfg.dtype == "fp32":
        print("config 0 is the CPU plumbing case; the GPU bench runs configs 1-4", file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    _hip.load()

    d = workloads.make_inputs(cfg, seed=0)
    fp8 = cfg.dtype == "fp8"
    logits = d["logits"].to(dev)
    x = d["x"].to(dev)
    w = {"experts": d["w_gu"].to(dev), "experts_down": d["w_d"].to(dev), "inter": cfg.I, "topk": cfg.k}
    if fp8:
        w["experts_scale"] = d["w_gu_scale"].to(dev)
        w["experts_down_scale"] = d["w_d_scale"].to(dev)
    scale = torch.ones(cfg.E, dtype=torch.bfloat16, device=dev)        # Gemma per_expert_scale
    dense = x.clone()                                                  # the dense MLP branch's output
    w1 = torch.ones(cfg.H, dtype=torch.bfloat16, device=dev)
    w2 = torch.ones(cfg.H, dtype=torch.bfloat16, device=dev)
    eps = 1e-6

    def act(gu, n):   # Gemma's activation callable (flide/backbones/gemma4/fused.py:238)
        return pw.geglu(gu[:, :n], gu[:, n:])

    def layer():
        top, ids = moe.route(logits, cfg.k, scale)
        y = moe.experts(x, w, top, ids, act)
        return moe.combine_norm(y, dense, w1, w2, cfg.k, eps)

    for _ in range(max(1, args.warmup)):
        out = layer()
    torch.cuda.synchronize()
    graph = None
    if not args.eager:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = layer()
        for _ in range(max(1, args.warmup)):
            graph.replay()
        torch.cuda.synchronize()

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        if graph is not None:
            graph.replay()
        else:
            out = layer()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    step_s = elapsed / args.steps
    tokens_per_s = cfg.T / step_s

    # ---- dominant kernel alone: gate/up grouped product with GeGLU fused -----------------------------
    top, ids = moe.route(logits, cfg.k, scale)
    bm = moe.tile(cfg.pairs, fp8)[0]
    rows, blocks, used = moe.align(ids, cfg.E, bm)
    counts = torch.bincount(ids.flatten().long(), minlength=cfg.E)
    n_hit = int((counts > 0).sum().item())
    actbuf = torch.empty(cfg.pairs, cfg.I, dtype=x.dtype, device=dev)
    if fp8:
        from flide_amd.kernels.fp8 import quantize_tokens
        qx, sx = quantize_tokens(x)

    def gate_up():
        if fp8:
            _hip.call("flide_moe_grouped_fp8", qx.data_ptr(), qx.stride(0), sx.data_ptr(), w["experts"].data_ptr(),
                      w["experts"].stride(0), w["experts"].stride(1), w["experts_scale"].data_ptr(),
                      w["experts_scale"].stride(0), 2 * cfg.I, cfg.H, actbuf.data_ptr(), actbuf.stride(0),
                      _hip.BF16, None, rows.data_ptr(), blocks.data_ptr(), used.data_ptr(), cfg.pairs,
                      blocks.shape[0], cfg.k, 1, _hip.ACT_GEGLU, bm, 0, _hip.stream(dev))
        else:
            moe.grouped(x, w["experts"], actbuf, rows, blocks, used, cfg.k, True, tile=(bm, 128, 4, 2),
                        act=_hip.ACT_GEGLU)

    for _ in range(3):
        gate_up()
    # Timed in layer context: each rep runs a whole layer, then this product once more between two HIP
    # events on the stream both launch on (torch's current stream). The kernel then runs at the clock the
    # layer sustains; back-to-back launches of the prefill product alone run it up to 20% slower.
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.kernel_reps)]
    torch.cuda.synchronize()
    for ev0, ev1 in evs:
        layer()
        ev0.record()
        gate_up()
        ev1.record()
    torch.cuda.synchronize()
    k_s = sum(ev0.elapsed_time(ev1) for ev0, ev1 in evs) / 1e3 / len(evs)
    bpw = 1 if fp8 else 2
    gu_bytes = n_hit * 2 * cfg.I * cfg.H * bpw + cfg.T * cfg.H * (1 if fp8 else 2) + cfg.pairs * cfg.I * 2
    gu_flops = cfg.pairs * 2 * cfg.H * 2 * cfg.I
    if cfg.idx == 1:
        roof = {"bound": "hbm", "achieved": gu_bytes / k_s / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s"}
    else:
        peak = MFMA_PEAK["fp8" if fp8 else "bf16"]
        roof = {"bound": "mfma", "achieved": gu_flops / k_s / 1e12, "peak": peak / 1e12, "unit": "TFLOP/s"}
    roof["frac"] = roof["achieved"] / roof["peak"]
    if roof["bound"] == "mfma":   # the other roofline of the same launch, on its algorithmic bytes
        roof["hbm_frac"] = gu_bytes / k_s / HBM_PEAK
    # HBM bytes per dispatch of this kernel at this workload, from the committed rocprofv3 --pmc summary
    # (FETCH_SIZE + WRITE_SIZE scaled by a copy kernel of known size); None when not profiled
    from flide_amd.rocprof import traffic_for
    roof["traffic"] = traffic_for(cfg.name)
    roof["algorithmic_bytes"] = gu_bytes
    # the whole layer against the same peak: its algorithmic bytes (all hit experts' weights, x and the
    # router table) for the HBM-bound decode case, its expert FLOPs otherwise; per step of the timed loop
    if roof["bound"] == "hbm":
        layer_bytes = n_hit * 3 * cfg.I * cfg.H * bpw + cfg.T * cfg.H * 2 + cfg.E * cfg.H * 2
        roof["layer"] = {"achieved": layer_bytes / step_s / 1e9, "frac": layer_bytes / step_s / HBM_PEAK,
                         "bytes": layer_bytes}
    else:
        roof["layer"] = {"achieved": cfg.flops / step_s / 1e12, "frac": cfg.flops / step_s / roof["peak"] / 1e12}
    roof["kernel"] = "grouped gate/up + GeGLU (" + ("fp8" if fp8 else "bf16") + f", bm {bm})"
    roof["kernel_us"] = k_s * 1e6

    # ---- CPU baseline: the reference's CPU torch path, fp32, on this host's cores ------------------
    cpu = None
    if not args.no_cpu and int(os.environ.get("RANK", "0")) == 0:
        from oracle import cpu_path

        ncores = _usable_cores()
        torch.set_num_threads(ncores)
        lg, xc = d["logits"].float(), d["x"].float()
        if fp8:
            wgu = d["w_gu"].float() * d["w_gu_scale"].unsqueeze(-1)
            wd = d["w_d"].float() * d["w_d_scale"].unsqueeze(-1)
        else:
            wgu, wd = d["w_gu"].float(), d["w_d"].float()
        # bounded sample: whole layers for small T, else the first Tc tokens of the same batch
        Tc = min(cfg.T, 512)
        lg, xc = lg[:Tc], xc[:Tc]
        cpu_path.layer_cpu(lg, xc, wgu, wd, cfg.k)        # warm-up
        times = []
        t_start = time.perf_counter()
        while len(times) < 3 or (time.perf_counter() - t_start < args.cpu_seconds and len(times) < 50):
            t1 = time.perf_counter()
            cpu_path.layer_cpu(lg, xc, wgu, wd, cfg.k)
            times.append(time.perf_counter() - t1)
        times.sort()
        med = times[len(times) // 2]
        cpu = {"value": Tc / med, "unit": "tokens/s", "cores": ncores, "kind": "port",
               "sample": f"{len(times)} runs (median) of route+experts on {Tc} of the {cfg.T} tokens, fp32, "
                         f"torch CPU (transformers' eager Gemma 4 experts loop restated), {_cpu_model()}"}

    rec = {
        "metric": "MoE layer tokens/s @ 26B-A4B shape, bf16 & FP8; % of HBM/MFMA peak",
        "value": tokens_per_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_s * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8" if fp8 else "bf16",
        "data": "synthetic (seeded N(0,1) logits/activations, N(0,0.02) random-init expert weights)",
        "config": {"workload": cfg.name, "tokens": cfg.T, "hidden": cfg.H, "experts": cfg.E, "topk": cfg.k,
                   "expert_ffn": cfg.I, "hit_experts": n_hit, "graph": graph is not None,
                   "layer_tflops": cfg.flops / step_s / 1e12},
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
