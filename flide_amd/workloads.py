"""Seeded synthetic workloads for the five BASELINE configurations of the MoE layer.

Everything is drawn on the CPU with torch.Generator().manual_seed(seed), in the order logits, x, w_gu,
w_d (then the router weight for config 0), so the CPU baseline, the parity checks and the GPU see the
same bits. Weights are N(0, 0.02) float32 masters, cast to the config's dtype (bf16), or quantised per
output row to e4m3fn for the FP8 config. No checkpoints: the shapes are Gemma 4 26B-A4B's MoE block
(hidden 2816, 128 experts, top-8, expert FFN 704).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class Config:
    idx: int
    name: str
    T: int
    H: int
    E: int
    k: int
    I: int
    dtype: str        # "fp32" (CPU plumbing), "bf16" or "fp8" (e4m3 experts, bf16 activations)
    logits: str       # "router" (x . W_r), "normal" (N(0,1) drawn directly), "zipf" (skewed)

    @property
    def pairs(self) -> int:
        return self.T * self.k

    @property
    def flops(self) -> int:
        """Algorithmic expert FLOPs: T*k pairs x (2*H*2I + 2*I*H); no padding, router excluded."""
        return self.pairs * (2 * self.H * 2 * self.I + 2 * self.I * self.H)


CONFIGS = {
    0: Config(0, "cfg0_cpu_fp32", 256, 1024, 16, 2, 512, "fp32", "router"),
    1: Config(1, "cfg1_decode_bf16", 64, 2816, 128, 8, 704, "bf16", "normal"),
    2: Config(2, "cfg2_prefill_bf16", 8192, 2816, 128, 8, 704, "bf16", "normal"),
    3: Config(3, "cfg3_fp8", 4096, 2816, 128, 8, 704, "fp8", "normal"),
    4: Config(4, "cfg4_skewed_bf16", 16384, 2816, 128, 8, 704, "bf16", "zipf"),
}

# Skewed routing (config 4): a Zipf(s=1.2) popularity over a seeded permutation of the experts,
# bias_e = ZIPF_C * log(pmf(rank_e)) = -ZIPF_C * s * log(rank_e) + const, with the ZIPF_EMPTY
# lowest-ranked experts outside the Zipf support (bias -1e4: never picked). ZIPF_C was calibrated once
# (seed 0) so the busiest expert takes ~10x the mean load; the support cut leaves 10 experts empty.
ZIPF_S = 1.2
ZIPF_C = 0.44
ZIPF_EMPTY = 10


def zipf_bias(E: int, g: torch.Generator) -> torch.Tensor:
    perm = torch.randperm(E, generator=g)
    rank = torch.empty(E)
    rank[perm] = torch.arange(1, E + 1, dtype=torch.float32)
    bias = -ZIPF_C * ZIPF_S * torch.log(rank)
    bias[rank > E - ZIPF_EMPTY] = -1e4
    return bias


def make_inputs(cfg: Config | int, seed: int = 0, T: int | None = None, with_weights: bool = True) -> dict:
    """CPU tensors for `cfg` (T overrides the token count for smaller parity cases):
    logits f32 [T,E], x [T,H], w_gu [E,2I,H], w_d [E,H,I] (in the config dtype; fp8 configs also carry
    the float32 masters' per-row scales w_gu_scale [E,2I], w_d_scale [E,H] and e4m3 weights), and for
    config 0 the router weight w_r [E,H]."""
    if isinstance(cfg, int):
        cfg = CONFIGS[cfg]
    T = cfg.T if T is None else T
    g = torch.Generator().manual_seed(seed)
    out: dict = {"cfg": cfg, "T": T}
    if cfg.logits in ("normal", "zipf"):
        logits = torch.randn(T, cfg.E, generator=g)
        if cfg.logits == "zipf":
            logits = logits + zipf_bias(cfg.E, g)
        out["logits"] = logits
    x = torch.randn(T, cfg.H, generator=g)
    if with_weights:
        w_gu = torch.randn(cfg.E, 2 * cfg.I, cfg.H, generator=g) * 0.02
        w_d = torch.randn(cfg.E, cfg.H, cfg.I, generator=g) * 0.02
    if cfg.logits == "router":
        w_r = torch.randn(cfg.E, cfg.H, generator=g) * 0.02
        out["w_r"] = w_r
        out["logits"] = (x.double() @ w_r.double().T).float()
    if cfg.dtype == "fp32":
        out["x"] = x
        if with_weights:
            out["w_gu"], out["w_d"] = w_gu, w_d
    else:
        out["x"] = x.to(torch.bfloat16)
        if with_weights:
            if cfg.dtype == "fp8":
                out["w_gu"], out["w_gu_scale"] = quantize_rows_cpu(w_gu)
                out["w_d"], out["w_d_scale"] = quantize_rows_cpu(w_d)
            else:
                out["w_gu"], out["w_d"] = w_gu.to(torch.bfloat16), w_d.to(torch.bfloat16)
    return out


def quantize_rows_cpu(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """[E, N, K] float32 masters -> (e4m3fn [E, N, K], float32 scales [E, N]) with flide/kernels/fp8.py:
    22-26's formula (scale = max(amax_row, 1e-12) / 448; q = clamp(w / scale, +-448) cast to e4m3fn).
    Used to build the FP8 workload's weights on the host, in slices to bound memory."""
    E, N, K = w.shape
    q = torch.empty(E, N, K, dtype=torch.float8_e4m3fn)
    s = torch.empty(E, N, dtype=torch.float32)
    for e in range(E):
        we = w[e].float()
        sc = we.abs().amax(dim=1, keepdim=True).clamp(min=1e-12) * (1.0 / 448.0)
        q[e] = (we / sc).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
        s[e] = sc[:, 0]
    return q, s


def device_weights(cfg: Config | int, device, seed: int = 0) -> dict:
    """Expert weights of `cfg`'s shape drawn on the GPU (N(0, 0.02) float32 masters from a device
    generator seeded with `seed`, then bf16, or quantised per row to e4m3fn by this library's own
    quantize_experts for the FP8 config): the benchmark's fast path, seconds instead of the CPU draw's
    tens of seconds. Same distributions as make_inputs, not the same bits."""
    from .kernels import moe

    if isinstance(cfg, int):
        cfg = CONFIGS[cfg]
    g = torch.Generator(device=device).manual_seed(seed)
    out = {}
    for name, shape in (("w_gu", (cfg.E, 2 * cfg.I, cfg.H)), ("w_d", (cfg.E, cfg.H, cfg.I))):
        w = (torch.randn(*shape, generator=g, device=device) * 0.02).to(torch.bfloat16)
        if cfg.dtype == "fp8":
            out[name], out[name + "_scale"] = moe.quantize_experts(w)
        else:
            out[name] = w
        del w
    return out
