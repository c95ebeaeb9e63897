"""flide_moe_experts_noalloc (the allocation-free entry point, static per-GPU scratch) against
flide_moe_experts with a caller workspace, through the C ABI: the same bits on two calls in a row, the
second smaller than the first (the scratch keeps the first call's contents), for 16-bit and float8
experts; a problem past the scratch is refused before any launch."""
from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _experts_args(x, top, ids, w, act, bm):
    from flide_amd import _hip

    T, H = x.shape
    k = ids.shape[1]
    E, I = w["gu"].shape[0], w["d"].shape[2]
    fp8 = "sgu" in w
    y = torch.full((T * k, H), float("nan"), device=DEV, dtype=x.dtype if fp8 else torch.float32)
    head = [x.data_ptr(), x.stride(0), _hip.dtype_code(x.dtype), T, H, top.data_ptr(), ids.data_ptr(), k,
            w["gu"].data_ptr(), w["d"].data_ptr(), _hip.ptr(w.get("sgu")), _hip.ptr(w.get("sd")), E, I,
            y.data_ptr(), act, bm, 0]
    return y, head, (T, k, E, H, I, bm, int(fp8))


def _run_both(x, top, ids, w, bm):
    """(y from flide_moe_experts with a fresh workspace, y from flide_moe_experts_noalloc)."""
    from flide_amd import _hip

    lib = _hip.load()
    st = _hip.stream(torch.device(DEV))
    y_ref, head, q = _experts_args(x, top, ids, w, _hip.ACT_GEGLU, bm)
    nbytes = lib.flide_moe_experts_workspace(*q)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    assert lib.flide_moe_experts(*head, ws.data_ptr(), nbytes, st) == 0
    y_na, head, _ = _experts_args(x, top, ids, w, _hip.ACT_GEGLU, bm)
    assert lib.flide_moe_experts_noalloc(*head, st) == 0
    torch.cuda.synchronize()
    return y_ref, y_na


def _weights(E, H, I, fp8, g):
    from flide_amd.kernels import moe

    w = {"gu": (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16).to(DEV),
         "d": (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16).to(DEV)}
    if fp8:
        w["gu"], w["sgu"] = moe.quantize_experts(w["gu"])
        w["d"], w["sd"] = moe.quantize_experts(w["d"])
    return w


@pytest.mark.parametrize("fp8", [False, True])
def test_noalloc_matches_workspace_entry_point(fp8):
    from flide_amd.kernels import moe

    print(f"noalloc experts fp8={fp8}", flush=True)
    g = torch.Generator().manual_seed(60 + fp8)
    E, H, I, k = 32, 2816, 704, 8
    w = _weights(E, H, I, fp8, g)
    for T in (600, 37):   # the second call smaller, on scratch holding the first call's rows and blocks
        x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(DEV)
        top, ids = moe.route(torch.randn(T, E, generator=g).to(DEV), k)
        bm = moe.tile(T * k, fp8)[0]
        print(f"  T={T} bm={bm}", flush=True)
        y_ref, y_na = _run_both(x, top, ids, w, bm)
        assert not torch.isnan(y_ref.float()).any()
        assert torch.equal(y_na, y_ref), f"T={T}: the allocation-free call differs from the workspace call"


def test_noalloc_refuses_past_its_scratch():
    from flide_amd import _hip

    print("noalloc scratch limit", flush=True)
    lib = _hip.load()
    lim = 16 << 20
    T = 4096   # 16-bit experts at the Gemma shape: act rows alone are 46 MB
    assert lib.flide_moe_experts_workspace(T, 8, 128, 2816, 704, 128, 0) > lim
    null = None
    rc = lib.flide_moe_experts_noalloc(null, 2816, _hip.BF16, T, 2816, null, null, 8, null, null, null, null, 128,
                                       704, null, _hip.ACT_GEGLU, 128, 0, null)
    assert rc == 4
    assert b"static scratch" in lib.flide_moe_strerror(rc)
    assert lib.flide_moe_experts_workspace(1400, 8, 128, 2816, 704, 32, 0) <= lim
