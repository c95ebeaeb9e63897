"""Timing of the steps on either side of the MoE layer at the Gemma 4 shape (H 2816, E 128, top-8, bf16):
in front, the router, rms_norm, the reference's three-call glue (rms_norm -> router, rms_norm;
flide/backbones/gemma4/fused.py:234-237) and the fused router_norm, with torch.mm (hipBLASLt) beside the router
for scale; behind, combine_norm alone and fused with the post-norm step (combine_norm_sandwich, fused.py:215,224),
and Qwen's combine (moe.py:256-277) at the same shape.

Each entry is the mean over 20 replays of a HIP graph holding 20 calls, so one launch of a small kernel
(about 4-5 us) is part of every figure, as it is inside a captured layer. Prints one JSON line per batch size.

    python -m flide_amd.bench_router [--tokens 64 1025 4096 8192]
    python <repo>/flide_amd/bench_router.py                 # by path, e.g. under rocprofv3 from /tmp
"""
from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

import torch

if __package__ in (None, ""):   # run by path: make the package importable
    sys.path.insert(0, str(Path(__file__).resolve().parent.parent))

from flide_amd.kernels import moe  # noqa: E402
from flide_amd.kernels import pointwise as pw  # noqa: E402

H, E, EPS = 2816, 128, 1e-6


def _graph_us(fn, reps: int = 20, replays: int = 20) -> float:
    for _ in range(3):
        fn()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / replays / reps * 1e3


def run(tokens) -> list[dict]:
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(0)
    out = []
    for T in tokens:
        h = torch.randn(T, H, device=dev, generator=gen).to(torch.bfloat16)
        nw = torch.rand(H, device=dev, generator=gen) * 0.1
        wr = (torch.randn(E, H, device=dev, generator=gen) * 0.02).to(torch.bfloat16)
        n2 = torch.rand(H, device=dev, generator=gen).to(torch.bfloat16)
        r = pw.rms_norm(h, nw, EPS, offset=False)

        def three():
            logits, _ = moe.router(pw.rms_norm(h, nw, EPS, offset=False), wr)
            return logits, pw.rms_norm(h, n2, EPS, offset=False)

        y = torch.randn(T * 8, H, device=dev, generator=gen)
        dense = torch.randn(T, H, device=dev, generator=gen).to(torch.bfloat16)
        w1, w2, wp, wn = (torch.rand(H, device=dev, generator=gen).to(torch.bfloat16) + 0.5 for _ in range(4))
        sc = torch.tensor([0.75], device=dev, dtype=torch.bfloat16)
        gl = torch.randn(T, 1, device=dev, generator=gen)

        row = {"tokens": T, "unit": "us per call",
               "router": _graph_us(lambda: moe.router(r, wr)),
               "torch_mm_bf16": _graph_us(lambda: torch.mm(r, wr.t())),
               "rms_norm": _graph_us(lambda: pw.rms_norm(h, nw, EPS, offset=False)),
               "three_calls": _graph_us(three),
               "router_norm": _graph_us(lambda: moe.router_norm(h, nw, wr, EPS, n2)),
               "combine_norm": _graph_us(lambda: moe.combine_norm(y, dense, w1, w2, 8, EPS)),
               "combine_norm_sandwich": _graph_us(
                   lambda: moe.combine_norm_sandwich(y, dense, w1, w2, 8, EPS, h, wp, sc, wn)),
               "combine_qwen": _graph_us(lambda: moe.combine(y, dense, gl, 8))}
        del y
        row = {k: (round(v, 2) if isinstance(v, float) else v) for k, v in row.items()}
        print(json.dumps(row), flush=True)
        out.append(row)
    return out


def main(argv=None) -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--tokens", type=int, nargs="+", default=[64, 1025, 4096, 8192])
    a = ap.parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("bench_router needs a GPU")
    run(a.tokens)


if __name__ == "__main__":
    main()
