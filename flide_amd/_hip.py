"""ctypes binding of libflide_moe.so (include/flide_moe.h).

The library is loaded after torch, so its libamdhip64.so.7 dependency resolves to the HIP runtime torch
already loaded (same SONAME): one runtime, one set of streams. Every entry point returns an int status;
`call` raises RuntimeError naming the entry point and the error on anything but 0. There is no CPU
fallback: without the built library every GPU entry point raises.
"""
from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_longlong, c_size_t, c_void_p
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime the library binds to)

LIB_PATH = Path(__file__).resolve().with_name("libflide_moe.so")

F32, BF16, F16, E4M3 = 0, 1, 2, 3
ACT_NONE, ACT_GEGLU, ACT_SWIGLU = 0, 1, 2

_P = c_void_p
_L = c_longlong
_I = c_int

# name -> argument types (every function returns int unless listed in _RESTYPES)
SIGNATURES: dict[str, list] = {
    "flide_moe_strerror": [_I],
    "flide_moe_version": [],
    "flide_moe_router": [_P, _L, _I, _I, _I, _P, _L, _I, _P, _P, _L, _P, _P],
    "flide_moe_router_norm": [_P, _L, _I, _I, _I, _P, _P, _L, _I, c_float, _P, _L, _P, _I, _P, _L, _P],
    "flide_moe_route": [_P, _L, _I, _I, _I, _P, _I, _P, _P, _P],
    "flide_moe_align_workspace": [_I, _I],
    "flide_moe_align": [_P, _I, _I, _I, _P, _P, _P, _P, _P, c_size_t, _P],
    "flide_moe_grouped": [_P, _L, _I, _P, _L, _L, _I, _I, _P, _L, _I, _P, _P, _P, _P, _I, _I, _I, _I,
                          _I, _I, _I, _P],
    "flide_moe_grouped_fp8": [_P, _L, _P, _P, _L, _L, _P, _L, _I, _I, _P, _L, _I, _P, _P, _P, _P, _I,
                              _I, _I, _I, _I, _I, _I, _P],
    "flide_moe_quantize_rows": [_P, _L, _I, _I, _I, _P, _L, _P, _P],
    "flide_moe_combine_norm": [_P, _I, _P, _L, _P, _P, _I, _P, _L, _I, _I, _I, _I, c_float, _P],
    "flide_moe_combine_norm_sandwich": [_P, _I, _P, _L, _P, _P, _P, _L, _P, _P, _I, _P, _P, _L, _P, _L, _I, _I, _I,
                                        c_float, _P],
    "flide_moe_combine": [_P, _I, _P, _P, _P, _I, _I, _I, _I, _P],
    "flide_moe_rms_norm": [_P, _L, _I, _P, _I, _P, _L, _I, _I, _I, c_float, _I, _P],
    "flide_moe_gated_act": [_P, _L, _P, _L, _P, _L, _I, _I, _I, _I, _P],
    "flide_moe_experts_workspace": [_I, _I, _I, _I, _I, _I, _I],
    "flide_moe_experts": [_P, _L, _I, _I, _I, _P, _P, _I, _P, _P, _P, _P, _I, _I, _P, _I, _I, _I, _P,
                          c_size_t, _P],
    "flide_moe_experts_noalloc": [_P, _L, _I, _I, _I, _P, _P, _I, _P, _P, _P, _P, _I, _I, _P, _I, _I, _I, _P],
}
_RESTYPES = {
    "flide_moe_strerror": ctypes.c_char_p,
    "flide_moe_version": ctypes.c_char_p,
    "flide_moe_align_workspace": c_size_t,
    "flide_moe_experts_workspace": c_size_t,
}

_lib = None


def load() -> ctypes.CDLL:
    """The loaded library (raises if it was never built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH.name} is not built: run `python -m flide_amd.build` "
                               "(or __graft_entry__.build()) first; there is no CPU fallback")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, c_int)
        _lib = lib
    return _lib


def call(name: str, *args) -> None:
    rc = getattr(load(), name)(*args)
    if rc != 0:
        msg = load().flide_moe_strerror(rc).decode()
        raise RuntimeError(f"{name} failed: {msg} (code {rc})")


def query(name: str, *args):
    return getattr(load(), name)(*args)


def stream(device: torch.device) -> int:
    """The current HIP stream of `device` as a raw handle."""
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return BF16
    if dt == torch.float16:
        return F16
    if dt == torch.float32:
        return F32
    if dt == torch.float8_e4m3fn:
        return E4M3
    raise TypeError(f"unsupported dtype {dt}")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def require_gpu(*tensors: torch.Tensor) -> torch.device:
    """The common device of `tensors`, which must be a HIP device: the product path has no CPU branch."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(f"flide_amd kernels run on the GPU only; got a tensor on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise RuntimeError("no tensor arguments")
    return dev
