"""Row-wise pieces on the MoE path: flide/kernels/pointwise.py's rms_norm (no residual), geglu and
swiglu, on HIP. Arithmetic in float32 from load to store, rounded once at the output."""
from __future__ import annotations

import torch

from .. import _hip


def rms_norm(x, w, eps: float, residual=None, offset: bool = True, dtype=None):
    """y = RMSNorm(x) with weight (1 + w) when `offset`, else w; y in `dtype` (x's by default)
    (flide/kernels/pointwise.py:39-49). The residual-add form is not on the MoE path."""
    if residual is not None:
        raise NotImplementedError("rms_norm with a residual is outside the MoE path")
    dev = _hip.require_gpu(x, w)
    T, N = x.shape
    if x.stride(-1) != 1:
        x = x.contiguous()
    w = w.contiguous()
    y = torch.empty(T, N, device=dev, dtype=x.dtype if dtype is None else dtype)
    if T:
        _hip.call("flide_moe_rms_norm", x.data_ptr(), x.stride(0), _hip.dtype_code(x.dtype), w.data_ptr(),
                  _hip.dtype_code(w.dtype), y.data_ptr(), y.stride(0), _hip.dtype_code(y.dtype), T, N,
                  float(eps), int(bool(offset)), _hip.stream(dev))
    return y


def _gated(a, b, act: int):
    dev = _hip.require_gpu(a, b)
    T, n = a.shape
    if a.stride(-1) != 1 or b.stride(-1) != 1:
        raise ValueError("gated activations take views with a contiguous last dimension")
    out = torch.empty(T, n, device=dev, dtype=a.dtype)
    if T:
        _hip.call("flide_moe_gated_act", a.data_ptr(), a.stride(0), b.data_ptr(), b.stride(0), out.data_ptr(),
                  out.stride(0), _hip.dtype_code(a.dtype), T, n, act, _hip.stream(dev))
    return out


def geglu(a, b):
    """GELU-tanh(a) * b for a, b [t, n] (row-strided views, contiguous last dimension) -> [t, n]
    (flide/kernels/pointwise.py:260-268)."""
    return _gated(a, b, _hip.ACT_GEGLU)


def swiglu(gu, n: int):
    """silu(gu[:, :n]) * gu[:, n:] (flide/kernels/pointwise.py:62-69)."""
    return _gated(gu[:, :n], gu[:, n:2 * n], _hip.ACT_SWIGLU)


geglu.flide_act = "geglu_pair"
swiglu.flide_act = "swiglu"
