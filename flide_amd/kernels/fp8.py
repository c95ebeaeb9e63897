"""8-bit floating point helpers of the MoE path: flide/kernels/fp8.py:14-53 on HIP.

quantize_rows  weights [N, K] -> e4m3fn [N, K] and float32 scales [N, 1] (amax / 448 per row)
quantize_tokens activations [M, K] (unit stride along K) -> e4m3fn [M, K] and float32 [M, 1]

Both run the same HIP kernel (flide_moe_quantize_rows): scale = max(amax, 1e-12) * (1/448), q =
e4m3fn(clamp(x / scale, +-448)) with a correctly rounded division and round-to-nearest-even. An all-zero
row keeps the tiny scale and stays zero. The format is OCP e4m3fn (max 448), which gfx950's MFMA reads.
"""
from __future__ import annotations

import torch

from .. import _hip

FP8 = torch.float8_e4m3fn
FP8_MAX = 448.0


def supported(device) -> bool:
    """gfx950 (MI355X) runs e4m3fn natively; any HIP device this library was built for does."""
    return torch.cuda.is_available()


def _quantize(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    dev = _hip.require_gpu(x)
    if x.stride(-1) != 1:
        x = x.contiguous()
    M, K = x.shape
    q = torch.empty(M, K, device=dev, dtype=FP8)
    s = torch.empty(M, 1, device=dev, dtype=torch.float32)
    if M:
        _hip.call("flide_moe_quantize_rows", x.data_ptr(), x.stride(0), M, K, _hip.dtype_code(x.dtype),
                  q.data_ptr(), q.stride(0), s.data_ptr(), _hip.stream(dev))
    return q, s


def quantize_rows(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(N, K) weight -> (N, K) float8 and (N, 1) float32 scale with w ~ q * scale (fp8.py:22-26)."""
    return _quantize(w)


def quantize_tokens(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(M, K) activations -> float8 [M, K] and a [M, 1] float32 scale per token (fp8.py:46-53)."""
    return _quantize(x)
