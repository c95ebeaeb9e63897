"""The reference's CPU torch path for the MoE layer, restated in torch -- TEST/BASELINE INFRASTRUCTURE.

Only tests/ and bench.py's cpu_baseline leg import this. It restates what Flide runs on the CPU for a
Gemma 4 MoE block (flide/backbones/gemma4/__init__.py:260-262,284-288 hand fp32 MoE to transformers'
eager modules): transformers' Gemma4TextRouter.forward (modeling_gemma4.py:1335-1356: softmax in float32,
top-k, renormalise, times per_expert_scale) and Gemma4TextExperts.forward (:1295-1319: for each hit
expert, gather its tokens, linear -> chunk(2) -> gelu_tanh(gate) * up -> linear -> times the routing
weight -> index_add_). Routing is taken from the logits with the lower-id tie rule (torch.topk's tie
order is unspecified), so it agrees with the GPU path bit-for-bit.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def route_cpu(logits: torch.Tensor, k: int, scale: torch.Tensor | None = None):
    """softmax(fp32) -> top-k (descending, lower id on ties) -> renormalise -> * scale[ids]."""
    probs = torch.softmax(logits.float(), dim=-1)
    order = torch.sort(logits.float(), dim=-1, descending=True, stable=True).indices[:, :k]
    top = torch.gather(probs, 1, order)
    top = top / top.sum(dim=-1, keepdim=True)
    if scale is not None:
        top = top * scale.float()[order]
    return top, order


def experts_cpu(x: torch.Tensor, w_gu: torch.Tensor, w_d: torch.Tensor, top: torch.Tensor, ids: torch.Tensor,
                act: str = "geglu") -> torch.Tensor:
    """Gemma4TextExperts.forward's loop over hit experts (modeling_gemma4.py:1300-1319), float32: the
    [T, H] weighted sum of each token's experts."""
    out = torch.zeros_like(x)
    E = w_gu.shape[0]
    mask = F.one_hot(ids.long(), num_classes=E).permute(2, 1, 0)   # [E, k, T]
    hit = torch.greater(mask.sum(dim=(-1, -2)), 0).nonzero()
    for e in hit[:, 0].tolist():
        slot, tok = torch.where(mask[e])
        cur = x[tok]
        gate, up = F.linear(cur, w_gu[e]).chunk(2, dim=-1)
        if act == "geglu":
            h = F.gelu(gate, approximate="tanh") * up
        else:
            h = F.silu(gate) * up
        h = F.linear(h, w_d[e]) * top[tok, slot, None]
        out.index_add_(0, tok, h.to(out.dtype))
    return out


def layer_cpu(logits, x, w_gu, w_d, k: int, scale=None, act: str = "geglu") -> torch.Tensor:
    """route -> experts: the MoE branch of one Gemma 4 layer on the CPU, float32."""
    top, ids = route_cpu(logits, k, scale)
    return experts_cpu(x, w_gu, w_d, top, ids, act)
