"""Write the golden fixtures under tests/golden/ (run from the repo root: python tests/golden/make_golden.py).

The vectors come from the CPU oracle (oracle/moe_oracle.py), which tests/test_oracle.py pins against
transformers' eager Gemma 4 modules, torch's number-format casts and brute force. Before writing, this
script cross-checks the experts fixture once more against transformers' Gemma4TextExperts (the
reference's CPU torch path) so a fixture can never silently encode a drifted oracle. Inputs are seeded
and small (every file well under 1 MB).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from oracle import moe_oracle as orc  # noqa: E402


def bf16(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).float().numpy()


def route_cases():
    g = torch.Generator().manual_seed(101)
    logits = torch.randn(96, 64, generator=g)
    logits[:32] = torch.randint(-2, 3, (32, 64), generator=g).float()   # exact ties
    logits[32] = 0.0                                                     # all equal
    scale = (torch.rand(64, generator=g) + 0.5).numpy()
    w, ids = orc.route(logits.numpy(), 6, scale)
    return {"logits": logits.numpy(), "scale": scale, "k": np.array(6), "w": w, "ids": ids}


def align_cases():
    rng = np.random.default_rng(102)
    T, E, k = 300, 24, 4
    pool = [e for e in range(E) if e != 7]              # expert 7 stays empty
    ids = []
    for _ in range(T):
        first = 3 if rng.random() < 0.6 else int(rng.choice(pool))   # skew towards expert 3
        rest = rng.permutation([e for e in pool if e != first])[:k - 1]
        ids.append([first, *rest])
    ids = np.array(ids, np.int32)
    out = {"ids": ids, "E": np.array(E)}
    for bm in (16, 64):
        al = orc.align(ids, E, bm)
        out[f"rows_bm{bm}"] = al["rows"]
        out[f"blocks_bm{bm}"] = al["blocks"]
        out[f"used_bm{bm}"] = al["used"]
    out["counts"] = orc.align(ids, E, 16)["counts"]
    return out


def experts_case():
    g = torch.Generator().manual_seed(103)
    T, H, E, k, I = 32, 128, 6, 2, 64
    logits = torch.randn(T, E, generator=g)
    x = bf16(torch.randn(T, H, generator=g))
    w_gu = bf16(torch.randn(E, 2 * I, H, generator=g) * 0.05)
    w_d = bf16(torch.randn(E, H, I, generator=g) * 0.05)
    dense = bf16(torch.randn(T, H, generator=g))
    w1 = bf16(torch.rand(H, generator=g) + 0.5)
    w2 = bf16(torch.rand(H, generator=g) + 0.5)
    top, ids = orc.route(logits.numpy(), k)
    y = orc.experts(x, w_gu, w_d, top, ids, I, "geglu", "bf16")
    out = orc.combine_norm(y, dense, w1, w2, k, 1e-6, "bf16")
    # cross-check against the reference's CPU torch path (fp32, no 16-bit roundings in between)
    from transformers.models.gemma4.configuration_gemma4 import Gemma4TextConfig
    from transformers.models.gemma4.modeling_gemma4 import Gemma4TextExperts

    cfg = Gemma4TextConfig(hidden_size=H, intermediate_size=2 * I, num_hidden_layers=1, num_attention_heads=2,
                           num_key_value_heads=1, head_dim=16, vocab_size=64, enable_moe_block=True,
                           num_experts=E, top_k_experts=k, moe_intermediate_size=I,
                           hidden_activation="gelu_pytorch_tanh")
    ex = Gemma4TextExperts(cfg).float()
    with torch.no_grad():
        ex.gate_up_proj.copy_(torch.from_numpy(w_gu))
        ex.down_proj.copy_(torch.from_numpy(w_d))
        ref = ex(torch.from_numpy(x), torch.from_numpy(ids).long(), torch.from_numpy(top)).numpy()
    got = orc.combine_sum(y, k, "fp32")
    err = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert err < 1e-2, f"oracle experts drifted from transformers' Gemma4TextExperts: {err:.2e}"
    return {"logits": logits.numpy(), "x": x, "w_gu": w_gu, "w_d": w_d, "dense": dense, "w1": w1, "w2": w2,
            "k": np.array(k), "inter": np.array(I), "top": top, "ids": ids, "y": y, "out": out}


def fp8_case():
    g = torch.Generator().manual_seed(104)
    T, H, E, k, I = 24, 128, 4, 2, 64
    logits = torch.randn(T, E, generator=g)
    x = bf16(torch.randn(T, H, generator=g))
    q_gu, s_gu = orc.quantize_experts(torch.randn(E, 2 * I, H, generator=g).numpy() * 0.02)
    q_d, s_d = orc.quantize_experts(torch.randn(E, H, I, generator=g).numpy() * 0.02)
    top, ids = orc.route(logits.numpy(), k)
    y = orc.experts_fp8(x, q_gu, s_gu, q_d, s_d, top, ids, I, "geglu")
    qx, sx = orc.quantize_tokens(x)
    return {"logits": logits.numpy(), "x": x, "q_gu": orc.e4m3fn_encode(q_gu), "s_gu": s_gu,
            "q_d": orc.e4m3fn_encode(q_d), "s_d": s_d, "k": np.array(k), "inter": np.array(I), "top": top,
            "ids": ids, "y": y, "qx": orc.e4m3fn_encode(qx), "sx": sx}


def main():
    for name, fn in (("route", route_cases), ("align", align_cases), ("experts_bf16", experts_case),
                     ("experts_fp8", fp8_case)):
        path = HERE / f"{name}.npz"
        np.savez_compressed(path, **fn())
        print(f"wrote {path.relative_to(ROOT)} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
