"""Shared test helpers: seeded workloads (cached per process), tensor <-> numpy, tolerance checks."""
from __future__ import annotations

import functools

import numpy as np
import torch

from flide_amd import workloads


@functools.lru_cache(maxsize=2)
def inputs(cfg: int, seed: int = 0, T: int | None = None) -> dict:
    return workloads.make_inputs(cfg, seed=seed, T=T)


@functools.lru_cache(maxsize=8)
def logits_only(cfg: int, seed: int = 0, T: int | None = None) -> dict:
    """The same logits (and x) as inputs(), without drawing the weights."""
    return workloads.make_inputs(cfg, seed=seed, T=T, with_weights=False)


def np32(t: torch.Tensor) -> np.ndarray:
    """Any float tensor (bf16/f16/f32/e4m3) -> float32 numpy, exactly."""
    return t.detach().float().cpu().numpy()


def to_dev(d: dict, keys, dev="cuda") -> dict:
    return {k: d[k].to(dev) for k in keys}


def rel_err(got, ref) -> float:
    """||got - ref|| / ||ref|| over finite reference entries."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    m = np.isfinite(ref)
    den = np.linalg.norm(ref[m])
    return float(np.linalg.norm(got[m] - ref[m]) / (den if den > 0 else 1.0))


def assert_close(got, ref, rel: float, what: str = "") -> None:
    """Relative L2 error within `rel`, and every element within rel * max|ref| (+ rel * |ref|)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    m = np.isfinite(ref)
    assert np.isfinite(got[m]).all(), f"{what}: non-finite output"
    e = rel_err(got, ref)
    assert e <= rel, f"{what}: relative L2 error {e:.3e} > {rel}"
    scale = np.abs(ref[m]).max() if m.any() else 1.0
    worst = np.abs(got[m] - ref[m]) - rel * np.abs(ref[m])
    assert worst.max(initial=0.0) <= rel * scale, f"{what}: max elementwise excess {worst.max():.3e}"
