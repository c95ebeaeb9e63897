"""GPU parity: the HIP path (through the C ABI, via flide_amd.kernels) against the CPU oracle on the same
seeded inputs. Routing ids, counts and the permutation are compared bit-exactly; outputs within 1e-2
relative for 16-bit experts and 3e-2 for FP8 experts."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe_oracle as orc
from tests.helpers import assert_close, inputs, logits_only, np32

pytestmark = pytest.mark.gpu

DEV = "cuda"
REL_BF16 = 1e-2
REL_FP8 = 3e-2


def _moe():
    from flide_amd.kernels import moe

    return moe


def _hip_mod():
    from flide_amd import _hip

    return _hip


def _gelu_act(gu, n):
    from flide_amd.kernels import pointwise as pw

    return pw.geglu(gu[:, :n], gu[:, n:])


# --------------------------------------------------------------------------------------------------
# routing
# --------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("T,E,k", [(1, 16, 2), (64, 128, 8), (300, 96, 6), (257, 1000, 4), (8, 8, 8), (33, 5, 1),
                                   (2048, 16, 2), (2500, 96, 6), (2049, 128, 16), (3001, 5, 1), (4096, 33, 3)])
def test_route_matches_oracle(T, E, k):
    print(f"route T={T} E={E} k={k}", flush=True)
    g = torch.Generator().manual_seed(T * 7 + E)
    logits = torch.randn(T, E, generator=g)
    scale = torch.rand(E, generator=g) + 0.5
    w, ids = _moe().route(logits.to(DEV), k, scale.to(DEV))
    rw, rids = orc.route(logits.numpy(), k, scale.numpy())
    np.testing.assert_array_equal(ids.cpu().numpy(), rids)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("T", [512, 4096])
def test_route_ties_go_to_lower_id(T):
    """Both route kernels (one token per wave below 2048 tokens, four per wave from there)."""
    print(f"route ties T={T}", flush=True)
    g = torch.Generator().manual_seed(5)
    logits = torch.randint(-3, 3, (T, 128), generator=g).float()   # heavy exact ties
    logits[0] = 0.0                                                   # all equal: ids 0..k-1, weights 1/k
    w, ids = _moe().route(logits.to(DEV), 8)
    rw, rids = orc.route(logits.numpy(), 8)
    np.testing.assert_array_equal(ids.cpu().numpy(), rids)
    np.testing.assert_array_equal(ids.cpu().numpy()[0], np.arange(8))
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(w.cpu().numpy()[0], np.full(8, 1 / 8), rtol=1e-6)


@pytest.mark.parametrize("cfg", [1, 2, 3, 4])
def test_route_configs_exact(cfg):
    print(f"route cfg{cfg}", flush=True)
    d = logits_only(cfg)
    c = d["cfg"]
    w, ids = _moe().route(d["logits"].to(DEV), c.k)
    rw, rids = orc.route(d["logits"].numpy(), c.k)
    np.testing.assert_array_equal(ids.cpu().numpy(), rids)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-5, atol=1e-7)


# --------------------------------------------------------------------------------------------------
# align
# --------------------------------------------------------------------------------------------------
def _check_align(ids_np, E, bm):
    moe = _moe()
    ids = torch.from_numpy(ids_np.astype(np.int32)).to(DEV)
    counts = torch.full((E,), -7, dtype=torch.int32, device=DEV)
    rows, blocks, used = moe.align(ids, E, bm, counts=counts)
    ref = orc.align(ids_np, E, bm)
    u = int(used.item())
    assert u == int(ref["used"][0])
    assert rows.shape[0] == ref["total"] and blocks.shape[0] == ref["total"] // bm
    np.testing.assert_array_equal(rows.cpu().numpy()[:u], ref["rows"][:u])
    np.testing.assert_array_equal(blocks.cpu().numpy()[:u // bm], ref["blocks"][:u // bm])
    np.testing.assert_array_equal(counts.cpu().numpy(), ref["counts"])


@pytest.mark.parametrize("T,E,k,bm", [(64, 128, 8, 16), (256, 16, 2, 64), (5000, 128, 8, 128), (3, 7, 2, 1),
                                      (1000, 1000, 4, 32), (2048, 128, 8, 128), (512, 128, 8, 48),
                                      (700, 60, 3, 24), (1, 128, 8, 128), (513, 128, 8, 32)])
def test_align_random(T, E, k, bm):
    print(f"align T={T} E={E} k={k} bm={bm}", flush=True)
    rng = np.random.default_rng(T + E)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)])
    _check_align(ids, E, bm)


def test_align_skewed_and_empty():
    print("align skew", flush=True)
    rng = np.random.default_rng(3)
    ids = np.zeros((4099, 4), np.int64)
    ids[:, 0] = 5                                    # one expert takes every token
    ids[:, 1:] = rng.integers(6, 9, (4099, 3))       # experts 0..4 and 9.. stay empty
    _check_align(ids, 16, 64)


@pytest.mark.parametrize("cfg", [1, 2, 3, 4])
def test_align_configs_exact(cfg):
    """Every config's routing at the tile its experts call pads with (cfg3: the float8 tile)."""
    d = logits_only(cfg)
    c = d["cfg"]
    _, rids = orc.route(d["logits"].numpy(), c.k)
    bm = _moe().tile(c.pairs, c.dtype == "fp8")[0]
    print(f"align cfg{cfg} bm={bm}", flush=True)
    _check_align(rids, c.E, bm)


# --------------------------------------------------------------------------------------------------
# grouped products and the experts
# --------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("bm", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("by_token,mul_w,out32", [(True, False, False), (False, True, True)])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_grouped_bf16(bm, by_token, mul_w, out32, dt):
    """Plain grouped products (16-bit rows and experts, 16-bit or float32 out) on every tile."""
    print(f"grouped bm={bm} by_token={by_token} {dt}", flush=True)
    moe = _moe()
    g = torch.Generator().manual_seed(bm)
    T, E, k, N, K = 96, 12, 3, 200, 136
    logits = torch.randn(T, E, generator=g)
    _, ids = orc.route(logits.numpy(), k)
    rows_in = T if by_token else T * k
    a = torch.randn(rows_in, K, generator=g).to(dt)
    w = (torch.randn(E, N, K, generator=g) * 0.05).to(dt)
    wts = torch.rand(T * k, generator=g)
    rows, blocks, used = moe.align(torch.from_numpy(ids).to(DEV), E, bm)
    out = torch.full((T * k, N), float("nan"), device=DEV, dtype=torch.float32 if out32 else dt)
    moe.grouped(a.to(DEV), w.to(DEV), out, rows, blocks, used, k, by_token, wts.to(DEV) if mul_w else None,
                tile=(bm, 128, 4, 2))
    al = orc.align(ids, E, bm)
    odt = "fp32" if out32 else ("bf16" if dt == torch.bfloat16 else "f16")
    ref = orc.grouped(np32(a), np32(w), al["rows"], al["blocks"], al["used"], T * k, k, by_token,
                      wts.numpy() if mul_w else None, bm=bm, out_dtype=odt)
    assert_close(np32(out), ref, REL_BF16 if not out32 else 1e-5, "grouped")


@pytest.mark.parametrize("bm", [32, 64, 128])
@pytest.mark.parametrize("layout", ["tail", "strided"])
@pytest.mark.parametrize("mul_w", [True, False])
def test_grouped_f32_out_layouts(bm, layout, mul_w):
    """Float32 outputs of the plain product in the layouts its epilogue treats differently: 4 columns
    per lane when out and its row stride are 4-float aligned (here with N % 4 != 0, so the last group of
    each row is partial), one column per lane otherwise (a view one float into a row of stride 203).
    Columns outside the view stay untouched."""
    print(f"grouped f32 out bm={bm} {layout} mul_w={mul_w}", flush=True)
    moe = _moe()
    g = torch.Generator().manual_seed(300 + bm)
    T, E, k, K = 80, 10, 3, 200
    N, width, c0 = (202, 204, 0) if layout == "tail" else (200, 203, 1)
    logits = torch.randn(T, E, generator=g)
    _, ids = orc.route(logits.numpy(), k)
    a = torch.randn(T, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(E, N, K, generator=g) * 0.05).to(torch.bfloat16)
    wts = torch.rand(T * k, generator=g)
    rows, blocks, used = moe.align(torch.from_numpy(ids).to(DEV), E, bm)
    buf = torch.full((T * k, width), float("nan"), device=DEV, dtype=torch.float32)
    out = buf[:, c0:c0 + N]
    moe.grouped(a.to(DEV), w.to(DEV), out, rows, blocks, used, k, True, wts.to(DEV) if mul_w else None,
                tile=(bm, 128, 4, 2))
    al = orc.align(ids, E, bm)
    ref = orc.grouped(np32(a), np32(w), al["rows"], al["blocks"], al["used"], T * k, k, True,
                      wts.numpy() if mul_w else None, bm=bm, out_dtype="fp32")
    assert_close(np32(out), ref, 1e-5, f"f32 out {layout}")
    rest = torch.cat([buf[:, :c0], buf[:, c0 + N:]], 1)
    assert torch.isnan(rest).all(), "a store landed outside the output view"


@pytest.mark.parametrize("bm", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("act", ["geglu", "swiglu"])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_grouped_gated_tails(bm, act, dt):
    """The fused gate/up epilogue on every tile with tails in both directions: half = 100 output columns
    (not a multiple of any tile's column count) and K = 200 (not a multiple of any stage width)."""
    print(f"grouped gated bm={bm} {act}", flush=True)
    from flide_amd import _hip

    moe = _moe()
    g = torch.Generator().manual_seed(100 + bm)
    T, E, k, half, K = 80, 6, 2, 100, 200
    _, ids = orc.route(torch.randn(T, E, generator=g).numpy(), k)
    x = torch.randn(T, K, generator=g).to(dt)
    w = (torch.randn(E, 2 * half, K, generator=g) * 0.08).to(dt)
    rows, blocks, used = moe.align(torch.from_numpy(ids).to(DEV), E, bm)
    out = torch.full((T * k, half), float("nan"), device=DEV, dtype=dt)
    code = _hip.ACT_GEGLU if act == "geglu" else _hip.ACT_SWIGLU
    moe.grouped(x.to(DEV), w.to(DEV), out, rows, blocks, used, k, True, tile=(bm, 128, 4, 2), act=code)
    al = orc.align(ids, E, bm)
    odt = "bf16" if dt == torch.bfloat16 else "f16"
    gu = orc.grouped(np32(x), np32(w), al["rows"], al["blocks"], al["used"], T * k, k, True, bm=bm, out_dtype=odt)
    ref = orc.geglu(gu[:, :half], gu[:, half:], odt) if act == "geglu" else orc.swiglu(gu, half, odt)
    assert not np.isnan(np32(out)).any(), "a valid pair's row was not written"
    assert_close(np32(out), ref, REL_BF16, f"gated bm={bm} {act}")


@pytest.mark.parametrize("bm", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("act", ["geglu", "swiglu"])
@pytest.mark.parametrize("odt", [torch.bfloat16, torch.float16])
def test_grouped_fp8_gated_tails(bm, act, odt):
    """The fused float8 gate/up epilogue on every tile (bm 128 is what 4096-16384 tokens run: 8 waves,
    BN 256, 3 stages) against the dequantised computation: half = 300 output columns (three column
    tiles of 128 and a tail of 44 at BN 256), K = 400 (three 128-wide stages and a 16-wide tail, long
    enough for every tile's ring), experts holding 1-3 blocks, rows by token. The oracle rounds gu to
    the output type before the activation, as the reference stores gu (moe.py:345-350)."""
    print(f"grouped fp8 gated bm={bm} {act} {odt}", flush=True)
    from flide_amd import _hip

    moe = _moe()
    g = torch.Generator().manual_seed(300 + bm)
    T, E, k, half, K = 700, 6, 2, 300, 400
    _, ids = orc.route(torch.randn(T, E, generator=g).numpy(), k)
    x = torch.randn(T, K, generator=g).to(odt)
    w = (torch.randn(E, 2 * half, K, generator=g) * 0.05).to(torch.bfloat16)
    qw, sw = orc.quantize_experts(np32(w))
    qx, sx = orc.quantize_tokens(np32(x))
    wq = torch.from_numpy(orc.e4m3fn_encode(qw)).view(torch.float8_e4m3fn).to(DEV)
    rows, blocks, used = moe.align(torch.from_numpy(ids).to(DEV), E, bm)
    out = torch.full((T * k, half), float("nan"), device=DEV, dtype=odt)
    code = _hip.ACT_GEGLU if act == "geglu" else _hip.ACT_SWIGLU
    moe.grouped_fp8(x.to(DEV), wq, torch.from_numpy(sw).to(DEV), out, rows, blocks, used, k, True,
                    tile=(bm, 128, 4, 2), act=code)
    al = orc.align(ids, E, bm)
    odn = "bf16" if odt == torch.bfloat16 else "f16"
    gu = orc.grouped(qx * sx, qw * sw[:, :, None], al["rows"], al["blocks"], al["used"], T * k, k, True, bm=bm,
                     out_dtype=odn)
    ref = orc.geglu(gu[:, :half], gu[:, half:], odn) if act == "geglu" else orc.swiglu(gu, half, odn)
    assert not np.isnan(np32(out)).any(), "a valid pair's row was not written"
    assert_close(np32(out), ref, REL_BF16, f"fp8 gated bm={bm} {act}")


@pytest.mark.parametrize("bm", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("fp8,K", [(False, 8), (False, 40), (True, 16), (True, 48)])
def test_grouped_short_k(bm, fp8, K):
    """K shorter than every tile's stage ring: each tile has to fall back to a kernel without one."""
    print(f"grouped short K bm={bm} fp8={fp8} K={K}", flush=True)
    moe = _moe()
    g = torch.Generator().manual_seed(7 * bm + K)
    T, E, k, N = 72, 5, 2, 96
    _, ids = orc.route(torch.randn(T, E, generator=g).numpy(), k)
    x = torch.randn(T, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(E, N, K, generator=g) * 0.1).to(torch.bfloat16)
    rows, blocks, used = moe.align(torch.from_numpy(ids).to(DEV), E, bm)
    out = torch.full((T * k, N), float("nan"), device=DEV, dtype=torch.bfloat16)
    al = orc.align(ids, E, bm)
    if fp8:
        qw, sw = orc.quantize_experts(np32(w))
        qx, sx = orc.quantize_tokens(np32(x))
        wq = torch.from_numpy(orc.e4m3fn_encode(qw)).view(torch.float8_e4m3fn).to(DEV)
        moe.grouped_fp8(x.to(DEV), wq, torch.from_numpy(sw).to(DEV), out, rows, blocks, used, k, True,
                        tile=(bm, 128, 4, 2))
        a_ref, w_ref = qx * sx, qw * sw[:, :, None]   # the dequantised computation
    else:
        moe.grouped(x.to(DEV), w.to(DEV), out, rows, blocks, used, k, True, tile=(bm, 128, 4, 2))
        a_ref, w_ref = np32(x), np32(w)
    ref = orc.grouped(a_ref, w_ref, al["rows"], al["blocks"], al["used"], T * k, k, True, bm=bm, out_dtype="bf16")
    assert not np.isnan(np32(out)).any(), "a valid pair's row was not written"
    assert_close(np32(out), ref, REL_BF16, f"short K bm={bm}")


@pytest.mark.parametrize("T,E,k,N,K,odt,mul_w,by_token", [
    (1200, 128, 8, 2816, 704, torch.bfloat16, True, False),    # the Gemma down product
    (1100, 16, 4, 2000, 208, torch.float32, False, False),     # K and N tails
    (700, 8, 2, 333, 768, torch.float16, True, True),          # longest K, rows by token
    (2048, 64, 8, 512, 144, torch.bfloat16, False, True),
])
def test_grouped_fp8_plain_bm128(T, E, k, N, K, odt, mul_w, by_token):
    """The FP8 plain product at bm 128 with K <= 768 (activation rows resident in LDS, weight tiles
    streamed across column tiles) against the dequantised computation."""
    print(f"grouped fp8 plain bm128 T={T} N={N} K={K} {odt}", flush=True)
    moe = _moe()
    g = torch.Generator().manual_seed(T + K)
    _, ids = orc.route(torch.randn(T, E, generator=g).numpy(), k)
    x = torch.randn(T if by_token else T * k, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(E, N, K, generator=g) * 0.05).to(torch.bfloat16)
    wts = torch.rand(T * k, generator=g)
    rows, blocks, used = moe.align(torch.from_numpy(ids).to(DEV), E, 128)
    out = torch.full((T * k, N), float("nan"), device=DEV, dtype=odt)
    qw, sw = orc.quantize_experts(np32(w))
    qx, sx = orc.quantize_tokens(np32(x))
    wq = torch.from_numpy(orc.e4m3fn_encode(qw)).view(torch.float8_e4m3fn).to(DEV)
    moe.grouped_fp8(x.to(DEV), wq, torch.from_numpy(sw).to(DEV), out, rows, blocks, used, k, by_token,
                    wts.to(DEV) if mul_w else None, tile=(128, 128, 4, 2))
    al = orc.align(ids, E, 128)
    odn = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "fp32"}[odt]
    ref = orc.grouped(qx * sx, qw * sw[:, :, None], al["rows"], al["blocks"], al["used"], T * k, k, by_token,
                      wts.numpy() if mul_w else None, bm=128, out_dtype=odn)
    assert not np.isnan(np32(out)).any(), "a valid pair's row was not written"
    # float32 out: fp32 accumulation against the oracle's float64 (the FP8 bar is 3e-2)
    assert_close(np32(out), ref, REL_BF16 if odt != torch.float32 else 1e-4, "fp8 plain bm128")


@pytest.mark.parametrize("layout", ["tail", "offset"])
def test_grouped_fp8_plain_out_views(layout):
    """16-bit outputs of the FP8 plain product at bm 128 in the two layouts its epilogue treats
    differently: rows of 8-element-aligned stride staged and stored 8 columns per lane, here with
    N % 8 != 0 so the last group is partial ("tail"); and a view one element into the row, which takes
    the per-column stores ("offset"). Columns outside the view stay untouched."""
    print(f"grouped fp8 plain out view {layout}", flush=True)
    moe = _moe()
    T, E, k, K = 900, 12, 4, 704
    N, width, c0 = (700, 704, 0) if layout == "tail" else (512, 520, 1)
    g = torch.Generator().manual_seed(N + c0)
    _, ids = orc.route(torch.randn(T, E, generator=g).numpy(), k)
    x = torch.randn(T * k, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(E, N, K, generator=g) * 0.05).to(torch.bfloat16)
    wts = torch.rand(T * k, generator=g)
    rows, blocks, used = moe.align(torch.from_numpy(ids).to(DEV), E, 128)
    buf = torch.full((T * k, width), float("nan"), device=DEV, dtype=torch.bfloat16)
    out = buf[:, c0:c0 + N]
    qw, sw = orc.quantize_experts(np32(w))
    qx, sx = orc.quantize_tokens(np32(x))
    wq = torch.from_numpy(orc.e4m3fn_encode(qw)).view(torch.float8_e4m3fn).to(DEV)
    moe.grouped_fp8(x.to(DEV), wq, torch.from_numpy(sw).to(DEV), out, rows, blocks, used, k, False,
                    wts.to(DEV), tile=(128, 128, 4, 2))
    al = orc.align(ids, E, 128)
    ref = orc.grouped(qx * sx, qw * sw[:, :, None], al["rows"], al["blocks"], al["used"], T * k, k, False,
                      wts.numpy(), bm=128, out_dtype="bf16")
    assert not np.isnan(np32(out)).any(), "a valid pair's row was not written"
    assert_close(np32(out), ref, REL_BF16, f"fp8 plain out {layout}")
    rest = torch.cat([buf[:, :c0], buf[:, c0 + N:]], 1)
    assert torch.isnan(rest.float()).all(), "a store landed outside the output view"


@pytest.mark.parametrize("shape", ["long_runs", "few_items"])
@pytest.mark.parametrize("kind", ["bf16_geglu", "f16_swiglu", "fp8_geglu", "bf16_plain_w", "f16_plain"])
def test_grouped_persistent_edges(kind, shape):
    """The persistent bm-128 products (one workgroup per CU walking its XCD's items; gated 16-bit and
    float8 with 16-bit out, plain 16-bit with float32 out) at K of exactly 10 stages, the fewest they
    take (640 for 16-bit, 1280 for float8), in the two places their work order departs from the bench
    shapes: two experts holding ~80 blocks each ("long_runs": an expert's run of blocks reaches past
    the 64-entry window on both sides) and ~16 items for 256 workgroups ("few_items": most workgroups
    own no item). Output views narrower than their row stride (a partial last column tile); columns
    outside the view stay untouched."""
    print(f"grouped persistent {kind} {shape}", flush=True)
    from flide_amd import _hip

    moe = _moe()
    fp8, gated = kind.startswith("fp8"), not kind.endswith(("plain", "plain_w"))
    dt = torch.float16 if kind.startswith("f16") else torch.bfloat16
    T, E, k = (20000, 2, 1) if shape == "long_runs" else (300, 4, 2)
    K = 1280 if fp8 else 640
    cols, width = (196, 200) if gated else (298, 300)
    N = 2 * cols if gated else cols
    by_token = gated
    mul_w = kind.endswith("_w")
    g = torch.Generator().manual_seed(T + K + len(kind))
    _, ids = orc.route(torch.randn(T, E, generator=g).numpy(), k)
    x = torch.randn(T if by_token else T * k, K, generator=g).to(dt)
    w = (torch.randn(E, N, K, generator=g) * 0.03).to(torch.bfloat16 if fp8 else dt)
    wts = torch.rand(T * k, generator=g)
    rows, blocks, used = moe.align(torch.from_numpy(ids).to(DEV), E, 128)
    al = orc.align(ids, E, 128)
    if shape == "long_runs":
        nb = int(np.asarray(al["used"]).reshape(-1)[0]) // 128
        assert np.bincount(al["blocks"][:nb]).min() > 64, "each expert should hold more than 64 blocks"
    odt = dt if gated else torch.float32
    odn = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "fp32"}[odt]
    buf = torch.full((T * k, width), float("nan"), device=DEV, dtype=odt)
    out = buf[:, :cols]
    act = (_hip.ACT_GEGLU if "geglu" in kind else _hip.ACT_SWIGLU) if gated else _hip.ACT_NONE
    wd = wts.to(DEV) if mul_w else None
    if fp8:
        qw, sw = orc.quantize_experts(np32(w))
        qx, sx = orc.quantize_tokens(np32(x))
        wq = torch.from_numpy(orc.e4m3fn_encode(qw)).view(torch.float8_e4m3fn).to(DEV)
        moe.grouped_fp8(x.to(DEV), wq, torch.from_numpy(sw).to(DEV), out, rows, blocks, used, k, by_token, wd,
                        tile=(128, 128, 4, 2), act=act)
        a_ref, w_ref = qx * sx, qw * sw[:, :, None]
    else:
        moe.grouped(x.to(DEV), w.to(DEV), out, rows, blocks, used, k, by_token, wd, tile=(128, 128, 4, 2), act=act)
        a_ref, w_ref = np32(x), np32(w)
    gu = orc.grouped(a_ref, w_ref, al["rows"], al["blocks"], al["used"], T * k, k, by_token,
                     wts.numpy() if mul_w else None, bm=128, out_dtype=odn)
    if gated:
        ref = orc.geglu(gu[:, :cols], gu[:, cols:], odn) if "geglu" in kind else orc.swiglu(gu, cols, odn)
    else:
        ref = gu
    assert not np.isnan(np32(out)).any(), "a valid pair's row was not written"
    # float32 out: fp32 accumulation against the oracle's float64
    assert_close(np32(out), ref, REL_BF16 if gated else 1e-5, f"persistent {kind} {shape}")
    assert torch.isnan(buf[:, cols:].float()).all(), "a store landed outside the output view"


def _experts_case(cfg, T=None, pairs_subset=None, fp8=False):
    moe = _moe()
    d = inputs(cfg, 0, T)
    c = d["cfg"]
    T = d["T"]
    top, ids = moe.route(d["logits"].to(DEV), c.k)
    w = {"experts": d["w_gu"].to(DEV), "experts_down": d["w_d"].to(DEV), "inter": c.I}
    if fp8:
        w["experts_scale"] = d["w_gu_scale"].to(DEV)
        w["experts_down_scale"] = d["w_d_scale"].to(DEV)
    y = moe.experts(d["x"].to(DEV), w, top, ids, _gelu_act)
    torch.cuda.synchronize()
    rtop, rids = orc.route(d["logits"].numpy(), c.k)
    np.testing.assert_array_equal(ids.cpu().numpy(), rids)
    if fp8:
        ref = orc.experts_fp8(np32(d["x"]), np32(d["w_gu"]), d["w_gu_scale"].numpy(), np32(d["w_d"]),
                              d["w_d_scale"].numpy(), rtop, rids, c.I, "geglu", pairs=pairs_subset)
    else:
        ref = orc.experts(np32(d["x"]), np32(d["w_gu"]), np32(d["w_d"]), rtop, rids, c.I, "geglu", "bf16",
                          pairs=pairs_subset)
    sel = slice(None) if pairs_subset is None else pairs_subset
    return np32(y)[sel], ref[sel], y


def test_experts_cfg1_decode():
    print("experts cfg1", flush=True)
    got, ref, _ = _experts_case(1)
    assert_close(got, ref, REL_BF16, "experts cfg1")


def test_experts_cfg1_shape_other_tiles():
    """T = 512 .. 8192 at the Gemma shape run the bm 32 / 64 / 128 kernels (bm 16 and 256: test_grouped_bf16)."""
    for T in (512, 2048, 4096, 8192):
        print(f"experts cfg1 T={T}", flush=True)
        sub = np.random.default_rng(T).choice(T * 8, 256, replace=False)
        got, ref, _ = _experts_case(1, T=T, pairs_subset=np.sort(sub))
        assert_close(got, ref, REL_BF16, f"experts T={T}")


@pytest.mark.parametrize("T,E,H,I,dt", [(40, 16, 2816, 704, torch.bfloat16), (700, 12, 1008, 320, torch.float16),
                                       (1100, 16, 2816, 704, torch.bfloat16)])
def test_experts_fp8_matches_call_sequence(T, E, H, I, dt):
    """The FP8 experts call quantizes the token rows inside its placement launch (align_one below 4096 pairs,
    align_place above): bit-identical to the reference's sequence align -> grouped_fp8 (gate/up, quantizing
    x) -> grouped_fp8 (down, x weight) on the same tiles (moe.py:336-353)."""
    print(f"experts fp8 vs call sequence T={T} E={E} H={H} I={I} {dt}", flush=True)
    moe = _moe()
    k = 8
    g = torch.Generator(device=DEV).manual_seed(T + H)
    logits = torch.randn(T, E, generator=g, device=DEV)
    x = torch.randn(T, H, generator=g, device=DEV).to(dt)
    q_gu, s_gu = moe.quantize_experts((torch.randn(E, 2 * I, H, generator=g, device=DEV) * 0.02).to(dt))
    q_d, s_d = moe.quantize_experts((torch.randn(E, H, I, generator=g, device=DEV) * 0.02).to(dt))
    top, ids = moe.route(logits, k)
    w = {"experts": q_gu, "experts_down": q_d, "inter": I, "experts_scale": s_gu, "experts_down_scale": s_d}
    y = moe.experts(x, w, top, ids, _gelu_act)
    tl = moe.tile(T * k, True)
    rows, blocks, used = moe.align(ids, E, tl[0])
    act = torch.empty(T * k, I, dtype=dt, device=DEV)
    moe.grouped_fp8(x, q_gu, s_gu, act, rows, blocks, used, k, True, tile=tl, act=_hip_mod().ACT_GEGLU)
    ref = torch.full((T * k, H), float("nan"), dtype=dt, device=DEV)
    moe.grouped_fp8(act, q_d, s_d, ref, rows, blocks, used, k, False, top.reshape(-1), tile=tl)
    torch.cuda.synchronize()
    assert not torch.isnan(ref.float()).any()
    assert torch.equal(y, ref), f"{(y != ref).sum().item()} of {y.numel()} values differ"


@pytest.mark.parametrize("T,E,H,I,dt", [(2100, 16, 1408, 320, torch.bfloat16), (3000, 24, 2816, 704, torch.float16)])
def test_experts_matches_call_sequence(T, E, H, I, dt):
    """The 16-bit experts call at the bm-128 tile (persistent products) against the reference's sequence
    align -> grouped (gate/up with the activation) -> grouped (down, x weight, float32 rows) on the same
    tiles: the same bits (moe.py:336-353)."""
    print(f"experts vs call sequence T={T} E={E} H={H} I={I} {dt}", flush=True)
    moe = _moe()
    k = 8
    g = torch.Generator(device=DEV).manual_seed(T + H)
    logits = torch.randn(T, E, generator=g, device=DEV)
    x = torch.randn(T, H, generator=g, device=DEV).to(dt)
    w_gu = (torch.randn(E, 2 * I, H, generator=g, device=DEV) * 0.02).to(dt)
    w_d = (torch.randn(E, H, I, generator=g, device=DEV) * 0.02).to(dt)
    top, ids = moe.route(logits, k)
    tl = moe.tile(T * k, False)
    assert tl[0] == 128
    y = moe.experts(x, {"experts": w_gu, "experts_down": w_d, "inter": I}, top, ids, _gelu_act)
    rows, blocks, used = moe.align(ids, E, tl[0])
    act = torch.empty(T * k, I, dtype=dt, device=DEV)
    moe.grouped(x, w_gu, act, rows, blocks, used, k, True, tile=tl, act=_hip_mod().ACT_GEGLU)
    ref = torch.full((T * k, H), float("nan"), dtype=torch.float32, device=DEV)
    moe.grouped(act, w_d, ref, rows, blocks, used, k, False, top.reshape(-1), tile=tl)
    torch.cuda.synchronize()
    assert not torch.isnan(ref).any()
    assert torch.equal(y, ref), f"{(y != ref).sum().item()} of {y.numel()} values differ"


def test_experts_cfg3_fp8_subset():
    print("experts cfg3 fp8 T=512", flush=True)
    sub = np.sort(np.random.default_rng(0).choice(512 * 8, 512, replace=False))
    got, ref, _ = _experts_case(3, T=512, pairs_subset=sub, fp8=True)
    assert_close(got, ref, REL_FP8, "experts fp8")


def test_experts_cfg3_fp8_decode_tile():
    print("experts cfg3 fp8 T=64", flush=True)
    got, ref, _ = _experts_case(3, T=64, fp8=True)
    assert_close(got, ref, REL_FP8, "experts fp8 T=64")


# --------------------------------------------------------------------------------------------------
# combine, quantize, router, norms
# --------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("T,H,k,ydt", [(37, 2816, 8, torch.float32), (29, 1024, 2, torch.float32),
                                       (19, 2048 + 64, 3, torch.bfloat16), (11, 4096, 5, torch.float32),
                                       (7, 1000, 1, torch.bfloat16), (5, 2816, 4, torch.bfloat16)])
def test_combine_norm(T, H, k, ydt):
    """The vector kernel at every per-lane load count (k up to 2, 4 and 8), ragged H, f32 and bf16 y."""
    print(f"combine_norm T={T} H={H} k={k} y {ydt}", flush=True)
    moe = _moe()
    g = torch.Generator().manual_seed(11)
    y = torch.randn(T * k, H, generator=g).to(ydt)
    dense = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w1 = (torch.rand(H, generator=g) + 0.5).to(torch.bfloat16)
    w2 = (torch.rand(H, generator=g) + 0.5).to(torch.bfloat16)
    out = moe.combine_norm(y.to(DEV), dense.to(DEV), w1.to(DEV), w2.to(DEV), k, 1e-6)
    ref = orc.combine_norm(np32(y), np32(dense), np32(w1), np32(w2), k, 1e-6)
    assert_close(np32(out), ref, 1e-2, "combine_norm")
    # one bf16 rounding: at most 1 ulp from the float64 reference
    np.testing.assert_allclose(np32(out), ref, rtol=2 ** -7, atol=1e-6)


@pytest.mark.parametrize("ydt,scale,nxt", [(torch.float32, True, True), (torch.bfloat16, False, True),
                                            (torch.float32, True, False)])
def test_combine_norm_sandwich(ydt, scale, nxt):
    """combine_norm and Gemma's following post-norm step (pointwise.sandwich) in one launch."""
    print(f"combine_norm_sandwich y {ydt} scale={scale} next={nxt}", flush=True)
    moe = _moe()
    g = torch.Generator().manual_seed(13)
    T, H, k, eps = 37, 2816, 8, 1e-6
    y = torch.randn(T * k, H, generator=g).to(ydt)
    dense = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w1, w2, wp, wn = ((torch.rand(H, generator=g) + 0.5).to(torch.bfloat16) for _ in range(4))
    h = (torch.randn(T, H, generator=g) * 3).to(torch.bfloat16)
    s = torch.tensor([0.75], dtype=torch.bfloat16)
    dev = [t.to(DEV) for t in (y, dense, w1, w2, h, wp, s, wn)]
    h_out, x_out = moe.combine_norm_sandwich(dev[0], dev[1], dev[2], dev[3], k, eps, dev[4], dev[5],
                                             dev[6] if scale else None, dev[7] if nxt else None)
    assert (x_out is None) == (not nxt)
    # the oracle end to end: combine_norm rounded to bf16 (as the reference stores d), then sandwich
    d = orc.combine_norm(np32(y), np32(dense), np32(w1), np32(w2), k, eps)
    rh, rx = orc.sandwich(d, np32(h), np32(wp), eps, np32(s) if scale else None, np32(wn) if nxt else None)
    np.testing.assert_allclose(np32(h_out), rh, rtol=2 ** -7, atol=2 ** -7)
    if nxt:
        np.testing.assert_allclose(np32(x_out), rx, rtol=2 ** -6, atol=2 ** -7)
    # the second phase alone: the oracle's sandwich of this library's own combine_norm output, to one ulp
    dg = np32(moe.combine_norm(dev[0], dev[1], dev[2], dev[3], k, eps))
    gh, gx = orc.sandwich(dg, np32(h), np32(wp), eps, np32(s) if scale else None, np32(wn) if nxt else None)
    np.testing.assert_allclose(np32(h_out), gh, rtol=2 ** -7, atol=1e-6)
    if nxt:
        np.testing.assert_allclose(np32(x_out), gx, rtol=2 ** -6, atol=1e-6)


@pytest.mark.parametrize("ydt,H,k", [(torch.float32, 2048 + 64, 4), (torch.bfloat16, 2048, 8),
                                     (torch.float32, 4100, 3), (torch.float32, 2048, 10)])
def test_combine_qwen(ydt, H, k):
    """The vector kernel (f32 and bf16 y), and the scalar one for H past 4096 or k past 8."""
    print(f"combine y {ydt} H={H} k={k}", flush=True)
    moe = _moe()
    g = torch.Generator().manual_seed(12)
    T = 19
    y = torch.randn(T * k, H, generator=g).to(ydt)
    shared = torch.randn(T, H, generator=g).to(torch.bfloat16)
    gate = torch.randn(T, 1, generator=g)
    out = moe.combine(y.to(DEV), shared.to(DEV), gate.to(DEV), k)
    ref = orc.combine(np32(y), np32(shared), gate.numpy(), k)
    np.testing.assert_allclose(np32(out), ref, rtol=2 ** -7, atol=1e-6)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("K", [704, 2816, 136])
def test_quantize_rows_bit_exact(dt, K):
    """Scales and e4m3 bytes bit-exact: 16-bit rows take the one-wave-per-row vector kernel (K = 136 and
    704 and 2816 use 1, 2 and 8 register pieces per lane), float32 rows the per-element kernel."""
    print(f"quantize {dt} K={K}", flush=True)
    from flide_amd.kernels import fp8

    g = torch.Generator().manual_seed(13)
    scale = torch.logspace(-6, 3, 97) if dt != torch.float16 else torch.logspace(-3, 3, 97)
    x = torch.randn(97, K, generator=g) * scale.unsqueeze(1)
    x[3] = 0.0
    x[5, :10] = torch.tensor([448.0, -448.0, 1e-30, -1e-30, 0.0, -0.0, 3.0, 5e-3, 1e-8, 2.0])
    x = x.to(dt)
    q, s = fp8.quantize_tokens(x.to(DEV))
    rq, rs = orc.quantize_rows(np32(x))
    np.testing.assert_array_equal(s.cpu().numpy(), rs)
    np.testing.assert_array_equal(q.cpu().view(torch.uint8).numpy(), orc.e4m3fn_encode(rq))


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("K", [704, 2816])
def test_quantize_rows_vec_matches_division(dt, K):
    """The 16-bit kernel's quotient (x * (1/s) and one fma correction) against the float32 kernel's true
    division on the same values, byte for byte: rows of 16-bit bit patterns drawn uniformly below a random
    amax (log-uniform magnitudes, so exact e4m3 ties, subnormals and values under the smallest code are
    common), and rows holding +-inf or NaN (an inf scale takes the division in both kernels)."""
    print(f"quantize vec vs division {dt} K={K}", flush=True)
    from flide_amd.kernels import fp8

    g = np.random.default_rng(21)
    M = 256
    finite_max = 0x7F7F if dt == torch.bfloat16 else 0x7BFF
    amax_bits = g.integers(1, finite_max, M)
    bits = (g.random((M, K)) * amax_bits[:, None]).astype(np.int64)
    bits[:, 0] = amax_bits
    bits |= np.where(g.random((M, K)) < 0.5, 0x8000, 0)   # sign
    x = torch.from_numpy(bits.astype(np.uint16).view(np.int16)).view(dt)
    inf, nan = float("inf"), float("nan")
    x[0, :4] = torch.tensor([inf, 1.0, -0.0, -3.0])
    x[1, 5], x[2, 7], x[3, 9] = -inf, nan, nan
    x[4] = 0.0
    x[4, 3] = -0.0
    q, s = fp8.quantize_tokens(x.to(DEV))
    qf, sf = fp8.quantize_tokens(x.float().to(DEV))
    np.testing.assert_array_equal(s.cpu().numpy(), sf.cpu().numpy())
    np.testing.assert_array_equal(q.cpu().view(torch.uint8).numpy(), qf.cpu().view(torch.uint8).numpy())


def test_quantize_experts_matches_rows():
    print("quantize_experts", flush=True)
    moe = _moe()
    g = torch.Generator().manual_seed(14)
    w = (torch.randn(4, 64, 256, generator=g) * 0.02).to(torch.bfloat16)
    q, s = moe.quantize_experts(w.to(DEV))
    rq, rs = orc.quantize_experts(np32(w))
    np.testing.assert_array_equal(s.cpu().numpy(), rs)
    np.testing.assert_array_equal(q.cpu().view(torch.uint8).numpy(), orc.e4m3fn_encode(rq))


@pytest.mark.parametrize("T,H,E", [(77, 2816, 128), (1100, 2816, 200), (5, 200, 64), (40, 40, 128)])
def test_router_logits(T, H, E):
    """Both router tiles (16 x 32 up to 1024 tokens, 64 x 64 above), a partial expert tile (E = 200), fewer
    32-wide K steps than waves (H = 200: 7 steps over 8 waves) and a partial last step (H = 40)."""
    print(f"router T={T} H={H} E={E}", flush=True)
    moe = _moe()
    g = torch.Generator().manual_seed(15 + T)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    wr = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16)
    wg = (torch.randn(H, generator=g) * 0.02).to(torch.bfloat16)
    logits, gate = moe.router(x.to(DEV), wr.to(DEV), wg.to(DEV))
    rl, rg = orc.router(np32(x), np32(wr), np32(wg))
    np.testing.assert_allclose(logits.cpu().numpy(), rl, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(gate.cpu().numpy(), rg, rtol=1e-5, atol=1e-5)


def test_router_batch_invariant():
    """A token's logits are the same bits whichever batch it is routed in: the K split over waves is fixed,
    only the tile changes with T (77 tokens: small tiles; 1100: large tiles), for both router forms."""
    print("router batch invariance", flush=True)
    moe = _moe()
    g = torch.Generator().manual_seed(23)
    T, H, E = 1100, 2816, 128
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(DEV)
    wr = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    nw = (torch.rand(H, generator=g) * 0.1).to(DEV)
    n2 = (torch.rand(H, generator=g) + 0.5).to(torch.bfloat16).to(DEV)
    big, _ = moe.router(x, wr)
    for a, b in ((0, 77), (500, 577), (1090, 1100)):
        small, _ = moe.router(x[a:b], wr)
        assert torch.equal(small, big[a:b]), (a, b)
    bl, bx = moe.router_norm(x, nw, wr, 1e-6, n2)
    sl, sx = moe.router_norm(x[500:577], nw, wr, 1e-6, n2)
    assert torch.equal(sl, bl[500:577]) and torch.equal(sx, bx[500:577])


@pytest.mark.parametrize("T,E,dt,n2dt", [(77, 128, torch.bfloat16, "same"), (77, 200, torch.bfloat16, "same"),
                                         (77, 128, torch.float16, "same"), (1100, 200, torch.bfloat16, "same"),
                                         (5000, 128, torch.bfloat16, torch.float32), (77, 128, torch.bfloat16, None)])
def test_router_norm_fused(T, E, dt, n2dt):
    """Gemma's router input fused into the router: logits of rms_norm(h, norm_w) against the router weight,
    and the experts' input rms_norm(h, norm2_w), from one launch. E = 200: a partial expert tile; T = 1100
    and 5000: the larger tiles; a float32 norm2 weight; no x2 at all."""
    print(f"router_norm T={T} E={E} {dt} norm2 {n2dt}", flush=True)
    moe = _moe()
    g = torch.Generator().manual_seed(17 + E + T)
    H, eps = 2816, 1e-6
    h = (torch.randn(T, H, generator=g) * 3).to(dt)
    norm_w = torch.rand(H, generator=g) * 0.1 + 0.01                 # float32, as Gemma folds its router scale
    wr = (torch.randn(E, H, generator=g) * 0.02).to(dt)
    norm2_w = (torch.rand(H, generator=g) + 0.5).to(dt if n2dt == "same" else (n2dt or dt))
    logits, x2 = moe.router_norm(h.to(DEV), norm_w.to(DEV), wr.to(DEV), eps, norm2_w.to(DEV) if n2dt else None)
    odt = "bf16" if dt == torch.bfloat16 else "f16"
    r = orc.rms_norm(np32(h), norm_w.numpy(), eps, offset=False, dtype=odt)
    rl, _ = orc.router(r, np32(wr))
    # r may differ from the float64 statistic's rounding by one ulp in a few elements: |dlogit| < 1e-3
    np.testing.assert_allclose(logits.cpu().numpy(), rl, rtol=1e-3, atol=1e-3)
    if n2dt is None:
        assert x2 is None
    else:
        rx = orc.rms_norm(np32(h), np32(norm2_w), eps, offset=False, dtype=odt)
        np.testing.assert_allclose(np32(x2), rx, rtol=2 ** -7 if dt == torch.bfloat16 else 2 ** -10, atol=1e-7)
    # and the same as the three separate calls the glue makes today, to the same bar
    from flide_amd.kernels import pointwise as pw
    l3, _ = moe.router(pw.rms_norm(h.to(DEV), norm_w.to(DEV), eps, offset=False), wr.to(DEV))
    np.testing.assert_allclose(logits.cpu().numpy(), l3.cpu().numpy(), rtol=1e-3, atol=1e-3)


_NAME = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


@pytest.mark.parametrize("xdt,wdt,N,offset,ydt,pad", [
    (torch.bfloat16, torch.float32, 2816, False, None, 0),     # Gemma's router norm: the vector kernel
    (torch.bfloat16, torch.bfloat16, 2816, True, None, 0),     # Qwen's zero-centred weight
    (torch.float16, torch.float16, 704, False, None, 0),
    (torch.bfloat16, torch.bfloat16, 8192, False, None, 24),   # 16 chunks per lane, strided rows
    (torch.bfloat16, torch.float32, 8200, False, None, 0),     # wider than the vector kernel: scalar kernel
    (torch.bfloat16, torch.float32, 100, False, None, 0),      # N % 8 != 0: scalar kernel
    (torch.bfloat16, torch.float32, 2816, False, torch.float32, 0),   # another output type: scalar kernel
])
def test_rms_norm(xdt, wdt, N, offset, ydt, pad):
    print(f"rms_norm {xdt} w {wdt} N={N} offset={offset} y {ydt} pad={pad}", flush=True)
    from flide_amd.kernels import pointwise as pw

    g = torch.Generator().manual_seed(N + pad)
    xf = (torch.randn(45, N + pad, generator=g) * 2).to(xdt)
    x = xf[:, :N]
    w = (torch.rand(N, generator=g) * 0.5 - (0.25 if offset else -0.01)).to(wdt)
    y = pw.rms_norm(x.to(DEV) if not pad else xf.to(DEV)[:, :N], w.to(DEV), 1e-6, offset=offset, dtype=ydt)
    ref = orc.rms_norm(np32(x), np32(w), 1e-6, offset=offset, dtype=_NAME[ydt or xdt])
    tol = {torch.bfloat16: 2 ** -7, torch.float16: 2 ** -10, torch.float32: 1e-5}[ydt or xdt]
    np.testing.assert_allclose(np32(y), ref, rtol=tol, atol=1e-6)


def test_rms_norm_and_geglu():
    print("rms_norm/geglu", flush=True)
    from flide_amd.kernels import pointwise as pw

    g = torch.Generator().manual_seed(16)
    h = torch.randn(33, 2816, generator=g).to(torch.bfloat16)
    wn = torch.rand(2816, generator=g) * 0.05
    y = pw.rms_norm(h.to(DEV), wn.to(DEV), 1e-6, offset=False)
    ref = orc.rms_norm(np32(h), wn.numpy(), 1e-6, offset=False)
    np.testing.assert_allclose(np32(y), ref, rtol=2 ** -7, atol=1e-7)
    gu = (torch.randn(50, 2 * 704, generator=g) * 2).to(torch.bfloat16)
    a = pw.geglu(gu[:, :704].to(DEV), gu[:, 704:].to(DEV))
    ra = orc.geglu(np32(gu[:, :704]), np32(gu[:, 704:]))
    # one bf16 ulp (the float math differs from float64 by a few float ulps); absolute floor 1e-5 near 0
    np.testing.assert_allclose(np32(a), ra, rtol=2 ** -7, atol=1e-5)


# --------------------------------------------------------------------------------------------------
# whole layer
# --------------------------------------------------------------------------------------------------
def test_moe_qwen_end_to_end():
    """Qwen3.5-MoE's feed-forward through moe.moe (moe.py:356-369): router with the shared-expert gate,
    route, experts with SwiGLU fused, the backbone's own products for the shared expert, combine."""
    print("moe qwen", flush=True)
    from flide_amd.kernels import pointwise as pw

    moe = _moe()
    g = torch.Generator().manual_seed(21)
    T, H, E, k, I, SI = 33, 2048, 64, 8, 512, 512
    bf = torch.bfloat16
    x = torch.randn(T, H, generator=g).to(bf)
    w = {"router": (torch.randn(E, H, generator=g) * 0.05).to(bf), "shared_gate": (torch.randn(1, H, generator=g) * 0.05).to(bf),
         "experts": (torch.randn(E, 2 * I, H, generator=g) * 0.03).to(bf),
         "experts_down": (torch.randn(E, H, I, generator=g) * 0.03).to(bf),
         "shared_gate_up": (torch.randn(2 * SI, H, generator=g) * 0.03).to(bf),
         "shared_down": (torch.randn(H, SI, generator=g) * 0.03).to(bf)}
    wd = {kk: v.to(DEV) for kk, v in w.items()}
    wd.update({"topk": k, "inter": I, "shared_inter": SI})

    def mm(a, b):   # the backbone's product: a [T, in] x b [out, in]^T
        return torch.matmul(a, b.t().contiguous())

    out = moe.moe(x.to(DEV), wd, mm, pw.swiglu)
    # the same steps, each checked on its own
    logits, gate = moe.router(x.to(DEV), wd["router"], wd["shared_gate"].reshape(-1))
    top, ids = moe.route(logits, k)
    rtop, rids = orc.route(logits.cpu().numpy(), k)
    np.testing.assert_array_equal(ids.cpu().numpy(), rids)
    shared = mm(pw.swiglu(mm(x.to(DEV), wd["shared_gate_up"]), SI), wd["shared_down"])
    ry = orc.experts(np32(x), np32(w["experts"]), np32(w["experts_down"]), rtop, rids, I, "swiglu", "bf16")
    ref = orc.combine(ry, np32(shared), gate.cpu().numpy(), k)
    assert_close(np32(out), ref, REL_BF16, "moe qwen")


def test_load_experts_fp8(tmp_path):
    """Expert weights from checkpoints into the FP8 path: a 16-bit checkpoint is quantised on the device as
    it is read (the same bytes and scales as quantize_experts and the oracle); a float8 checkpoint in the
    per-expert layout, with scales in another shard, is taken as stored and runs through experts()."""
    print("load experts fp8", flush=True)
    from safetensors.torch import save_file

    from flide_amd import load

    moe = _moe()
    g = torch.Generator().manual_seed(31)
    E, I, H, T, k = 8, 192, 512, 40, 4
    gu16 = (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(torch.bfloat16)
    dn16 = (torch.randn(E, H, I, generator=g) * 0.05).to(torch.bfloat16)
    a = tmp_path / "bf16"
    a.mkdir()
    save_file({"e.gate_up_proj": gu16, "e.down_proj": dn16}, str(a / "model.safetensors"))
    w = load.experts(str(a), "e", DEV, fp8=True)
    q, sc = moe.quantize_experts(gu16.to(DEV))
    assert torch.equal(w["experts"].view(torch.uint8), q.view(torch.uint8)) and torch.equal(w["experts_scale"], sc)
    rq, rs = orc.quantize_experts(np32(dn16))
    np.testing.assert_array_equal(w["experts_down_scale"].cpu().numpy(), rs)
    np.testing.assert_array_equal(w["experts_down"].cpu().view(torch.uint8).numpy(), orc.e4m3fn_encode(rq))

    b = tmp_path / "fp8"
    b.mkdir()
    sh1, sh2 = {}, {}
    for j in range(E):   # as a float8 export stores them: per expert, the scales in the first shard
        for n, qt, st in (("gate", w["experts"][j, :I], w["experts_scale"][j, :I]),
                          ("up", w["experts"][j, I:], w["experts_scale"][j, I:]),
                          ("down", w["experts_down"][j], w["experts_down_scale"][j])):
            sh2[f"m.experts.{j}.{n}_proj.weight"] = qt.cpu().contiguous()
            sh1[f"m.experts.{j}.{n}_proj.weight_scale"] = st.cpu().reshape(-1, 1).contiguous()
    save_file(sh1, str(b / "model-00001-of-00002.safetensors"))
    save_file(sh2, str(b / "model-00002-of-00002.safetensors"))
    w8 = load.experts(str(b), "m.experts", DEV, fp8=True)
    assert torch.equal(w8["experts"].view(torch.uint8), w["experts"].view(torch.uint8))
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    top, ids = moe.route(torch.randn(T, E, generator=g).to(DEV), k)
    y = moe.experts(x.to(DEV), w8, top, ids, _gelu_act)
    ref = orc.experts_fp8(np32(x), np32(w8["experts"]), w8["experts_scale"].cpu().numpy(), np32(w8["experts_down"]),
                          w8["experts_down_scale"].cpu().numpy(), top.cpu().numpy(), ids.cpu().numpy(), I, "geglu")
    assert_close(np32(y), ref, REL_FP8, "experts from a float8 checkpoint")


@pytest.mark.parametrize("T", [48, 2100])
@pytest.mark.parametrize("fp8", [False, True])
def test_graph_replays_match_eager(fp8, T):
    """The Gemma layer captured once into a HIP graph (fused router_norm -> route -> experts ->
    combine_norm_sandwich), replayed three times on new inputs written between replays by eager work: every
    replay gives the bits of an eager run on the same inputs. 48 tokens run the decode tiles, 2100 tokens
    (8400 pairs) the bm-128 prefill kernels, at H = 1408 the persistent gate/up product."""
    print(f"graph replays fp8={fp8} T={T}", flush=True)
    moe = _moe()
    g = torch.Generator().manual_seed(41)
    H, E, k, I, eps = (512 if T < 100 else 1408), 16, 4, 128, 1e-6
    assert T < 100 or moe.tile(T * k, fp8)[0] == 128
    bf = torch.bfloat16
    w = {"experts": (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(bf).to(DEV),
         "experts_down": (torch.randn(E, H, I, generator=g) * 0.05).to(bf).to(DEV), "inter": I, "topk": k}
    if fp8:
        w["experts"], w["experts_scale"] = moe.quantize_experts(w["experts"])
        w["experts_down"], w["experts_down_scale"] = moe.quantize_experts(w["experts_down"])
    wr = (torch.randn(E, H, generator=g) * 0.05).to(bf).to(DEV)
    nw = (torch.rand(H, generator=g) * 0.1).to(DEV)
    n1, n2, n3, n4, n5 = ((torch.rand(H, generator=g) + 0.5).to(bf).to(DEV) for _ in range(5))
    scale = (torch.rand(E, generator=g) + 0.5).to(bf).to(DEV)
    ls = torch.tensor([0.8], dtype=bf, device=DEV)
    h = torch.empty(T, H, dtype=bf, device=DEV)
    dense = torch.empty(T, H, dtype=bf, device=DEV)

    def layer():
        logits, x2 = moe.router_norm(h, nw, wr, eps, n1)
        top, ids = moe.route(logits, k, scale)
        y = moe.experts(x2, w, top, ids, _gelu_act)
        return moe.combine_norm_sandwich(y, dense, n2, n3, k, eps, h, n4, ls, n5)

    def new_inputs(seed):
        gg = torch.Generator().manual_seed(seed)
        h.copy_((torch.randn(T, H, generator=gg) * 2).to(bf))
        dense.copy_(torch.randn(T, H, generator=gg).to(bf))

    new_inputs(0)
    layer()   # outside capture first (the activation callable is recognised here)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_h, out_x = layer()
    for rep in range(1, 4):
        new_inputs(rep)
        graph.replay()
        torch.cuda.synchronize()
        got_h, got_x = out_h.clone(), out_x.clone()
        ref_h, ref_x = layer()
        torch.cuda.synchronize()
        assert torch.equal(got_h, ref_h) and torch.equal(got_x, ref_x), f"replay {rep}"


def test_graph_replays_match_eager_qwen():
    """Qwen's moe() (torch products for the shared expert inside) under the same capture and replay check."""
    print("graph replays qwen", flush=True)
    from flide_amd.kernels import pointwise as pw

    moe = _moe()
    g = torch.Generator().manual_seed(42)
    T, H, E, k, I, SI = 40, 512, 16, 4, 128, 128
    bf = torch.bfloat16
    w = {"router": (torch.randn(E, H, generator=g) * 0.05).to(bf), "shared_gate": (torch.randn(1, H, generator=g) * 0.05).to(bf),
         "experts": (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(bf),
         "experts_down": (torch.randn(E, H, I, generator=g) * 0.05).to(bf),
         "shared_gate_up": (torch.randn(2 * SI, H, generator=g) * 0.05).to(bf),
         "shared_down": (torch.randn(H, SI, generator=g) * 0.05).to(bf)}
    w = {kk: v.to(DEV) for kk, v in w.items()}
    w.update({"topk": k, "inter": I, "shared_inter": SI})
    x = torch.empty(T, H, dtype=bf, device=DEV)

    def mm(a, b):
        return torch.matmul(a, b.t().contiguous())

    x.copy_(torch.randn(T, H, generator=g).to(bf))
    moe.moe(x, w, mm, pw.swiglu)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = moe.moe(x, w, mm, pw.swiglu)
    for rep in range(3):
        x.copy_(torch.randn(T, H, generator=g).to(bf))
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        ref = moe.moe(x, w, mm, pw.swiglu)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"replay {rep}"


def test_empty_batches():
    """T = 0 through every entry point on the path: empty outputs of the right shapes, no launch."""
    print("empty batches", flush=True)
    from flide_amd.kernels import pointwise as pw

    moe = _moe()
    H, E, k, bf = 256, 16, 4, torch.bfloat16
    x = torch.empty(0, H, dtype=bf, device=DEV)
    wr = torch.randn(E, H, device=DEV).to(bf)
    nw = torch.rand(H, device=DEV)
    wb = torch.rand(H, device=DEV).to(bf)
    logits, gate = moe.router(x, wr, wb)
    assert logits.shape == (0, E) and gate.shape == (0, 1)
    lg, x2 = moe.router_norm(x, nw, wr, 1e-6, wb)
    assert lg.shape == (0, E) and x2.shape == (0, H)
    top, ids = moe.route(lg, k)
    assert top.shape == (0, k) and ids.shape == (0, k)
    assert pw.rms_norm(x, wb, 1e-6, offset=False).shape == (0, H)
    y = torch.empty(0, H, device=DEV)
    assert moe.combine_norm(y, x, wb, wb, k, 1e-6).shape == (0, H)
    ho, xo = moe.combine_norm_sandwich(y, x, wb, wb, k, 1e-6, x, wb, None, wb)
    assert ho.shape == (0, H) and xo.shape == (0, H)


def test_layer_cfg1_route_experts_combine():
    print("layer cfg1", flush=True)
    moe = _moe()
    d = inputs(1)
    c = d["cfg"]
    top, ids = moe.route(d["logits"].to(DEV), c.k)
    w = {"experts": d["w_gu"].to(DEV), "experts_down": d["w_d"].to(DEV), "inter": c.I}
    y = moe.experts(d["x"].to(DEV), w, top, ids, _gelu_act)
    dense = d["x"].to(DEV)
    ones = torch.ones(c.H, dtype=torch.bfloat16, device=DEV)
    out = moe.combine_norm(y, dense, ones, ones, c.k, 1e-6)
    rtop, rids = orc.route(d["logits"].numpy(), c.k)
    ry = orc.experts(np32(d["x"]), np32(d["w_gu"]), np32(d["w_d"]), rtop, rids, c.I, "geglu", "bf16")
    ref = orc.combine_norm(ry, np32(d["x"]), np.ones(c.H), np.ones(c.H), c.k, 1e-6)
    assert_close(np32(out), ref, REL_BF16, "layer cfg1")
