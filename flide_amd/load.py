"""Routed-expert weights for the MoE layer straight from a safetensors checkpoint, in the layout
`moe.experts` takes: 16-bit `experts` [E, 2I, H] and `experts_down` [E, H, I], or for the FP8 path float8
(e4m3fn) tensors of those shapes with float32 per-row scales `experts_scale` [E, 2I] and
`experts_down_scale` [E, H].

This is the expert side of the reference's direct loader (flide/backbones/load.py:1-30, 186-250):
- A float8 tensor is taken as stored, bytes and scale, never quantised again. Its per-output-row scale is
  the tensor `<name>_scale` (compressed-tensors' `weight_scale` beside `weight`), which may sit in another
  shard than the weight: the index names its shard (load.py:190-197; tests/test_load_split_scale.py).
- A 16-bit tensor read for the FP8 path is quantised on the device as it is read
  (`flide_moe_quantize_rows`, fp8.py:22-26's amax / 448 per row), so device memory holds the float8 copy.
- A float8 tensor read for the 16-bit path is expanded through its scale (load.py:252-255).

Two checkpoint layouts:
- fused, as transformers' Gemma 4 experts store them: `<prefix>.gate_up_proj` [E, 2I, H] (gate rows then
  up rows) and `<prefix>.down_proj` [E, H, I];
- per expert, as Qwen3.5-MoE and most float8 exports do: `<prefix>.<j>.gate_proj.weight` [I, H],
  `.up_proj.weight` [I, H] and `.down_proj.weight` [H, I], stacked here (gate rows first).

Only the reading runs on the host: the quantisation is the library's HIP kernel, so the FP8 path from a
16-bit checkpoint needs a GPU device.
"""
from __future__ import annotations

import json
import re
from pathlib import Path

import torch

FP8 = torch.float8_e4m3fn


def checkpoint_files(model_dir: str) -> list[Path]:
    """The checkpoint's safetensors shards: those its index lists, else model.safetensors, else every
    *.safetensors file (load.py:35-47)."""
    d = Path(model_dir)
    index = d / "model.safetensors.index.json"
    if index.is_file():
        return [d / f for f in sorted(set(json.loads(index.read_text())["weight_map"].values()))]
    if (d / "model.safetensors").is_file():
        return [d / "model.safetensors"]
    found = sorted(d.glob("*.safetensors"))
    if not found:
        raise FileNotFoundError(f"no safetensors weights in {model_dir}")
    return found


class Checkpoint:
    """Name -> tensor over all shards of a safetensors checkpoint, each tensor read alone onto `device`."""

    def __init__(self, model_dir: str, device: str | torch.device = "cpu"):
        from safetensors import safe_open

        self._open = safe_open
        self.device = str(device)
        self.where: dict[str, Path] = {}
        for path in checkpoint_files(model_dir):   # what each shard holds, whatever the index says
            with safe_open(str(path), framework="pt", device="cpu") as f:
                for k in f.keys():
                    self.where[k] = path

    def __contains__(self, name: str) -> bool:
        return name in self.where

    def dtype(self, name: str) -> str:
        with self._open(str(self._path(name)), framework="pt", device="cpu") as f:
            return f.get_slice(name).get_dtype()

    def get(self, name: str) -> torch.Tensor:
        with self._open(str(self._path(name)), framework="pt", device=self.device) as f:
            return f.get_tensor(name)

    def _path(self, name: str) -> Path:
        if name not in self.where:
            raise KeyError(f"{name} is not in the checkpoint")
        return self.where[name]


def _row_scale(ck: Checkpoint, name: str, rows: tuple[int, ...]) -> torch.Tensor:
    """The float32 per-row scale of float8 tensor `name` with leading shape `rows` ([.., N]): stored as
    [.., N], [.., N, 1], or one value for the whole tensor."""
    key = name + "_scale"
    if key not in ck:
        raise KeyError(f"{name} is stored in float8 but the checkpoint has no {key}")
    s = ck.get(key).float()
    n = 1
    for r in rows:
        n *= r
    if s.numel() == n:
        return s.reshape(rows).contiguous()
    if s.numel() == 1:
        return s.reshape(()).expand(rows).contiguous()
    raise ValueError(f"{key}: {tuple(s.shape)} is not a per-row scale of {name} (rows {rows}); block scales "
                     "are not supported")


def read(ck: Checkpoint, name: str, fp8: bool, dtype: torch.dtype = torch.bfloat16):
    """Tensor `name` [.., N, K] for the FP8 path ((float8, float32 scale [.., N])) or the 16-bit path
    (a `dtype` tensor)."""
    if "F8" in ck.dtype(name):
        q = ck.get(name)
        if q.dtype != FP8:
            raise TypeError(f"{name}: float8 format {q.dtype} is not e4m3fn")
        s = _row_scale(ck, name, tuple(q.shape[:-1]))
        if fp8:
            return q, s.to(q.device)
        return (q.float() * s.to(q.device).unsqueeze(-1)).to(dtype)
    w = ck.get(name).to(dtype)
    if not fp8:
        return w
    from .kernels.fp8 import quantize_rows

    lead = tuple(w.shape[:-1])
    q, s = quantize_rows(w.reshape(-1, w.shape[-1]))
    return q.reshape(w.shape), s.reshape(lead)


def _stack(parts):
    """[(tensor or (q, s)), ...] per expert -> one stacked tensor, or (q, s) stacked."""
    if isinstance(parts[0], tuple):
        return torch.stack([p[0] for p in parts]), torch.stack([p[1] for p in parts])
    return torch.stack(parts)


def _cat_rows(a, b):
    if isinstance(a, tuple):
        return torch.cat([a[0], b[0]]), torch.cat([a[1], b[1]])
    return torch.cat([a, b])


def experts(model_dir: str, prefix: str, device: str | torch.device, fp8: bool,
            dtype: torch.dtype = torch.bfloat16) -> dict:
    """The routed experts under `prefix` (e.g. `model.language_model.layers.3.experts` or
    `model.layers.3.mlp.experts`) as the entries of the layer's weight dict that `moe.experts` reads:
    `experts`, `experts_down`, `inter`, and with `fp8` also `experts_scale` and `experts_down_scale`.
    The layout (fused or per expert) is found from the names in the checkpoint."""
    ck = Checkpoint(model_dir, device)
    if f"{prefix}.gate_up_proj" in ck:
        gu = read(ck, f"{prefix}.gate_up_proj", fp8, dtype)
        dn = read(ck, f"{prefix}.down_proj", fp8, dtype)
    else:
        ids = sorted({int(m.group(1)) for k in ck.where
                      for m in [re.match(re.escape(prefix) + r"\.(\d+)\.gate_proj\.weight$", k)] if m})
        if not ids or ids != list(range(len(ids))):
            raise KeyError(f"no routed experts under {prefix} (fused gate_up_proj or <j>.gate_proj.weight)")
        gu = _stack([_cat_rows(read(ck, f"{prefix}.{j}.gate_proj.weight", fp8, dtype),
                               read(ck, f"{prefix}.{j}.up_proj.weight", fp8, dtype)) for j in ids])
        dn = _stack([read(ck, f"{prefix}.{j}.down_proj.weight", fp8, dtype) for j in ids])
    w = {}
    if fp8:
        w["experts"], w["experts_scale"] = gu
        w["experts_down"], w["experts_down_scale"] = dn
    else:
        w["experts"], w["experts_down"] = gu, dn
    E, N2, H = w["experts"].shape
    if N2 % 2 or tuple(w["experts_down"].shape) != (E, H, N2 // 2):
        raise ValueError(f"{prefix}: gate/up {tuple(w['experts'].shape)} and down "
                         f"{tuple(w['experts_down'].shape)} do not make one expert FFN")
    w["inter"] = N2 // 2
    return w
