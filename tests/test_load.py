"""flide_amd.load: routed experts read from safetensors checkpoints in both layouts, float8 tensors taken as
stored with their per-row scales from any shard (the case of the reference's tests/test_load_split_scale.py),
float8 expanded for the 16-bit path (CPU only; the quantising read is a GPU test)."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from flide_amd import load

E, I, H = 3, 4, 16


def _fp8(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * 50).to(torch.float8_e4m3fn)


def _write(d: Path, shards: list[dict], index: bool = True) -> str:
    wm = {}
    for i, t in enumerate(shards):
        name = f"model-{i + 1:05d}-of-{len(shards):05d}.safetensors"
        save_file(t, str(d / name))
        wm.update({k: name for k in t})
    if index:
        (d / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": wm}))
    return str(d)


def _same_bytes(a: torch.Tensor, b: torch.Tensor) -> bool:
    return torch.equal(a.view(torch.uint8), b.view(torch.uint8))


def test_fused_float8_scale_in_another_shard(tmp_path):
    p = "model.language_model.layers.0.experts"
    gu, dn = _fp8((E, 2 * I, H), 1), _fp8((E, H, I), 2)
    sg, sd = torch.rand(E, 2 * I, 1) + 0.5, torch.rand(E, H) + 0.5
    d = _write(tmp_path, [{f"{p}.gate_up_proj": gu, f"{p}.down_proj_scale": sd},
                          {f"{p}.down_proj": dn, f"{p}.gate_up_proj_scale": sg}])
    w = load.experts(d, p, "cpu", fp8=True)
    assert _same_bytes(w["experts"], gu) and _same_bytes(w["experts_down"], dn)
    assert torch.equal(w["experts_scale"], sg.reshape(E, 2 * I)) and torch.equal(w["experts_down_scale"], sd)
    assert w["experts_scale"].dtype == torch.float32 and w["inter"] == I


def test_per_expert_float8_stacked_gate_rows_first(tmp_path):
    p = "model.layers.2.mlp.experts"
    t, ref = {}, {"gate": [], "up": [], "down": []}
    for j in range(E):
        for n, (shape, seed) in (("gate", ((I, H), 10 + j)), ("up", ((I, H), 20 + j)), ("down", ((H, I), 30 + j))):
            q = _fp8(shape, seed)
            s = torch.rand(shape[0], 1) + 0.25
            t[f"{p}.{j}.{n}_proj.weight"], t[f"{p}.{j}.{n}_proj.weight_scale"] = q, s
            ref[n].append((q, s.reshape(-1)))
    d = _write(tmp_path, [t], index=False)
    w = load.experts(d, p, "cpu", fp8=True)
    for j in range(E):
        assert _same_bytes(w["experts"][j, :I], ref["gate"][j][0]) and _same_bytes(w["experts"][j, I:], ref["up"][j][0])
        assert torch.equal(w["experts_scale"][j], torch.cat([ref["gate"][j][1], ref["up"][j][1]]))
        assert _same_bytes(w["experts_down"][j], ref["down"][j][0])
        assert torch.equal(w["experts_down_scale"][j], ref["down"][j][1])


def test_float8_expanded_for_the_16bit_path(tmp_path):
    p = "experts"
    gu, dn = _fp8((E, 2 * I, H), 3), _fp8((E, H, I), 4)
    sg, sd = torch.rand(E, 2 * I) + 0.5, torch.rand(E, H, 1) + 0.5
    d = _write(tmp_path, [{f"{p}.gate_up_proj": gu, f"{p}.gate_up_proj_scale": sg, f"{p}.down_proj": dn,
                           f"{p}.down_proj_scale": sd}])
    w = load.experts(d, p, "cpu", fp8=False, dtype=torch.float32)
    np.testing.assert_array_equal(w["experts"].numpy(), (gu.float() * sg.unsqueeze(-1)).numpy())
    np.testing.assert_array_equal(w["experts_down"].numpy(), (dn.float() * sd).numpy())
    assert "experts_scale" not in w


def test_16bit_checkpoint_for_the_16bit_path_and_tensor_scale(tmp_path):
    p = "experts"
    gu = torch.randn(E, 2 * I, H).to(torch.bfloat16)
    dn = _fp8((E, H, I), 5)
    d = _write(tmp_path, [{f"{p}.gate_up_proj": gu, f"{p}.down_proj": dn, f"{p}.down_proj_scale": torch.tensor([0.5])}])
    w = load.experts(d, p, "cpu", fp8=False)
    assert torch.equal(w["experts"], gu)
    assert torch.equal(w["experts_down"], (dn.float() * 0.5).to(torch.bfloat16))   # one scale for the tensor


def test_refusals(tmp_path):
    p = "experts"
    a = tmp_path / "a"
    a.mkdir()
    d = _write(a, [{f"{p}.gate_up_proj": _fp8((E, 2 * I, H), 6), f"{p}.down_proj": _fp8((E, H, I), 7),
                    f"{p}.down_proj_scale": torch.ones(E, H)}])
    with pytest.raises(KeyError, match="gate_up_proj_scale"):
        load.experts(d, p, "cpu", fp8=True)
    b = tmp_path / "b"
    b.mkdir()
    d = _write(b, [{f"{p}.gate_up_proj": _fp8((E, 2 * I, H), 6), f"{p}.gate_up_proj_scale": torch.ones(E, 2, 2),
                    f"{p}.down_proj": _fp8((E, H, I), 7), f"{p}.down_proj_scale": torch.ones(E, H)}])
    with pytest.raises(ValueError, match="block scales"):
        load.experts(d, p, "cpu", fp8=True)
    with pytest.raises(KeyError, match="no routed experts"):
        load.experts(d, "model.nothing", "cpu", fp8=True)
