"""GPU parity at BASELINE's configurations and through the Gemma 4 call sequence.

  * cfg0 (256 tokens, hidden 1024, 16 experts, top-2, FFN 512): router logits x . W_r through the HIP
    router, then route, experts and combine_norm, bf16 operands, against the oracle on the same
    (bf16-rounded) inputs and against the reference's float32 CPU path;
  * cfg3 (FP8, 4096 tokens): the experts at full size, at the tile the layer runs (bm 128), against the
    dequantised computation on sampled pairs;
  * cfg4 (skewed, 16384 tokens): the experts on the Zipf routing, sampled to include the busiest
    expert's last block and the experts next to empty ones;
  * Gemma 4's FusedDecoder._moe (flide/backbones/gemma4/fused.py:231-240) call for call, and with the
    fused router_norm, against oracle.gemma_moe.
Routing ids compare bit-exactly; outputs within 1e-2 relative (bf16) and 3e-2 (FP8)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import cpu_path
from oracle import moe_oracle as orc
from tests.helpers import assert_close, inputs, np32

pytestmark = pytest.mark.gpu

DEV = "cuda"
REL_BF16 = 1e-2
REL_FP8 = 3e-2


def _moe():
    from flide_amd.kernels import moe

    return moe


def _geglu(a, b):
    """The Gemma backbone's activation helper (fused.py:28-34): pointwise.geglu on the two halves."""
    from flide_amd.kernels import pointwise as pw

    return pw.geglu(a, b)


def probe_pairs(ids: np.ndarray, E: int, bm: int, n_random: int, seed: int) -> np.ndarray:
    """Pair indices to check: n_random at random, every expert's first and last pair, all pairs of the
    busiest expert's last block (a partial block at the end of the longest segment), and every pair of
    the experts whose neighbour id holds no pair (segments next to empty ones)."""
    flat = ids.reshape(-1)
    rng = np.random.default_rng(seed)
    sel = [rng.choice(flat.size, min(n_random, flat.size), replace=False)]
    counts = np.bincount(flat, minlength=E)
    for e in range(E):
        p = np.flatnonzero(flat == e)
        if p.size == 0:
            continue
        sel.append(p[[0, -1]])
        empty_next = (e > 0 and counts[e - 1] == 0) or (e + 1 < E and counts[e + 1] == 0)
        if empty_next:
            sel.append(p[:bm])
    hot = int(np.argmax(counts))
    p = np.flatnonzero(flat == hot)
    last = p.size % bm or bm
    sel.append(p[-last:])
    return np.unique(np.concatenate(sel))


# --------------------------------------------------------------------------------------------------
# cfg0: the CPU plumbing case through the HIP path
# --------------------------------------------------------------------------------------------------
def test_cfg0_router_route_experts_combine():
    print("cfg0 router -> route -> experts -> combine_norm", flush=True)
    moe = _moe()
    d = inputs(0)
    c = d["cfg"]
    bf = torch.bfloat16
    x, wr, wgu, wd = (d[n].to(bf) for n in ("x", "w_r", "w_gu", "w_d"))
    logits, _ = moe.router(x.to(DEV), wr.to(DEV))
    top, ids = moe.route(logits, c.k)
    w = {"experts": wgu.to(DEV), "experts_down": wd.to(DEV), "inter": c.I}
    y = moe.experts(x.to(DEV), w, top, ids, lambda gu, n: _geglu(gu[:, :n], gu[:, n:]))
    ones = torch.ones(c.H, dtype=bf, device=DEV)
    out = moe.combine_norm(y, x.to(DEV), ones, ones, c.k, 1e-6)
    torch.cuda.synchronize()

    # the oracle on the same bf16 operands
    rl, _ = orc.router(np32(x), np32(wr))
    np.testing.assert_allclose(logits.cpu().numpy(), rl, rtol=1e-5, atol=1e-5)
    rtop, rids = orc.route(rl, c.k)
    np.testing.assert_array_equal(ids.cpu().numpy(), rids)
    np.testing.assert_allclose(top.cpu().numpy(), rtop, rtol=1e-5, atol=1e-7)
    ry = orc.experts(np32(x), np32(wgu), np32(wd), rtop, rids, c.I, "geglu", "bf16")
    assert_close(np32(y), ry, REL_BF16, "cfg0 experts")
    ref = orc.combine_norm(ry, np32(x), np.ones(c.H), np.ones(c.H), c.k, 1e-6)
    assert_close(np32(out), ref, REL_BF16, "cfg0 combine_norm")

    # the reference's float32 CPU path on the float32 inputs: the same routing wherever bf16 operands
    # cannot reorder the logits, and the weighted expert sums within the bf16 bar there
    l32 = d["logits"]
    ctop, cids = cpu_path.route_cpu(l32, c.k)
    ysum = cpu_path.experts_cpu(d["x"], d["w_gu"], d["w_d"], ctop, cids).numpy()
    same = (cids.numpy() == ids.cpu().numpy()).all(1)
    # where the two differ, the float32 logits of the two experts swapped are closer than the bf16
    # operands' rounding can move a logit (|dl| <= sum_h |x w| * 2^-8)
    bound = (np.abs(d["x"].numpy()) @ np.abs(d["w_r"].numpy()).T) * 2.0 ** -8
    srt = np.sort(l32.numpy(), 1)[:, ::-1]
    gap = np.minimum(srt[:, c.k - 1] - srt[:, c.k], np.min(srt[:, :c.k - 1] - srt[:, 1:c.k], 1, initial=np.inf))
    assert (gap[~same] <= 2 * bound.max(1)[~same]).all(), "a routing difference that bf16 rounding cannot explain"
    assert same.sum() >= 240, f"only {same.sum()} of 256 tokens route alike"
    gsum = np32(y).reshape(c.T, c.k, c.H).sum(1)
    assert_close(gsum[same], ysum[same], REL_BF16, "cfg0 against the float32 CPU path")


# --------------------------------------------------------------------------------------------------
# cfg3 and cfg4 at full size
# --------------------------------------------------------------------------------------------------
def _experts_full(cfg: int, fp8: bool, n_random: int):
    moe = _moe()
    d = inputs(cfg)
    c = d["cfg"]
    T = d["T"]
    top, ids = moe.route(d["logits"].to(DEV), c.k)
    w = {"experts": d["w_gu"].to(DEV), "experts_down": d["w_d"].to(DEV), "inter": c.I}
    if fp8:
        w["experts_scale"] = d["w_gu_scale"].to(DEV)
        w["experts_down_scale"] = d["w_d_scale"].to(DEV)
    y = moe.experts(d["x"].to(DEV), w, top, ids, lambda gu, n: _geglu(gu[:, :n], gu[:, n:]))
    torch.cuda.synchronize()
    rtop, rids = orc.route(d["logits"].numpy(), c.k)
    np.testing.assert_array_equal(ids.cpu().numpy(), rids)
    bm = moe.tile(T * c.k, fp8)[0]
    pairs = probe_pairs(rids, c.E, bm, n_random, cfg)
    print(f"cfg{cfg}: T={T} bm={bm}, checking {pairs.size} pairs", flush=True)
    if fp8:
        ref = orc.experts_fp8(np32(d["x"]), np32(d["w_gu"]), d["w_gu_scale"].numpy(), np32(d["w_d"]),
                              d["w_d_scale"].numpy(), rtop, rids, c.I, "geglu", pairs=pairs)
    else:
        ref = orc.experts(np32(d["x"]), np32(d["w_gu"]), np32(d["w_d"]), rtop, rids, c.I, "geglu", "bf16",
                          pairs=pairs)
    got = y[torch.from_numpy(pairs).to(DEV)].float().cpu().numpy()
    return got, ref[pairs], bm


def test_experts_cfg3_fp8_full_size():
    """4096 tokens select the 128-row float8 tiles: the gated 8-wave gate/up kernel and the resident
    down kernel, the tiles the FP8 layer runs."""
    print("experts cfg3 fp8 T=4096", flush=True)
    got, ref, bm = _experts_full(3, True, 1024)
    assert bm == 128
    assert_close(got, ref, REL_FP8, "experts cfg3 fp8")


def test_experts_cfg4_skewed_full_size():
    """16384 tokens on the Zipf routing (the busiest expert ~10x the mean, ten experts empty)."""
    print("experts cfg4 skewed T=16384", flush=True)
    d = inputs(4)
    counts = np.bincount(orc.route(d["logits"].numpy(), 8)[1].reshape(-1), minlength=128)
    assert (counts == 0).sum() >= 8 and counts.max() >= 8 * counts.mean()
    got, ref, bm = _experts_full(4, False, 1024)
    assert_close(got, ref, REL_BF16, "experts cfg4 skewed")


# --------------------------------------------------------------------------------------------------
# Gemma 4's _moe, call for call
# --------------------------------------------------------------------------------------------------
def _gemma_weights(T: int, seed: int):
    """Gemma 4 26B-A4B-shaped MoE weights as FusedDecoder holds them (fused.py:122-127): a float32
    router_norm (the router's scale times hidden^-1/2), a bf16 per_expert_scale, bf16 experts, and the
    layer's three bf16 norm weights."""
    g = torch.Generator().manual_seed(seed)
    H, E, k, I = 2816, 128, 8, 704
    bf = torch.bfloat16
    h = (torch.randn(T, H, generator=g) * 2).to(bf)
    dense = torch.randn(T, H, generator=g).to(bf)
    wd = {"router": (torch.randn(E, H, generator=g) * 0.02).to(bf),
          "router_norm": ((torch.rand(H, generator=g) + 0.5) * H ** -0.5).float(),
          "expert_scale": (torch.rand(E, generator=g) + 0.5).to(bf),
          "experts": (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(bf),
          "experts_down": (torch.randn(E, H, I, generator=g) * 0.02).to(bf),
          "inter": I, "topk": k}
    norms = {n: (torch.rand(H, generator=g) + 0.5).to(bf) for n in ("pre_norm_2", "post_norm_1", "post_norm_2")}
    return h, dense, wd, norms


def near_tied(logits: np.ndarray, k: int, bound: np.ndarray) -> np.ndarray:
    """Tokens whose top k (in order, and the k-th against the (k+1)-th) hold two logits within
    2 * bound[token] of each other: only there can logits that each moved by at most bound reorder."""
    srt = np.sort(logits, 1)[:, ::-1]
    gaps = srt[:, :k] - srt[:, 1:k + 1]
    return (gaps <= 2 * bound[:, None]).any(1)


@pytest.mark.parametrize("T", [64, 4096])
@pytest.mark.parametrize("fused_router", [False, True])
def test_gemma_moe_call_sequence(T, fused_router):
    """FusedDecoder._moe's six calls through flide_amd (rms_norm with the float32 router_norm, router,
    route with per_expert_scale, rms_norm, experts with the backbone's GeGLU lambda, combine_norm), and the
    same with the fused router_norm replacing the first three, against oracle.gemma_moe."""
    print(f"gemma _moe T={T} fused_router={fused_router}", flush=True)
    from flide_amd.kernels import pointwise as pw

    moe = _moe()
    eps = 1e-6
    h, dense, wd, norms = _gemma_weights(T, 50 + T)
    k = wd["topk"]
    w = {kk: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for kk, v in wd.items()}
    n = {kk: v.to(DEV) for kk, v in norms.items()}
    hd, dd = h.to(DEV), dense.to(DEV)
    if fused_router:
        logits, x2 = moe.router_norm(hd, w["router_norm"], w["router"], eps, n["pre_norm_2"])
        top, ids = moe.route(logits, k, w["expert_scale"])
    else:   # fused.py:234-237 in order
        r = pw.rms_norm(hd, w["router_norm"], eps, offset=False)
        logits, _ = moe.router(r, w["router"])
        top, ids = moe.route(logits, k, w["expert_scale"])
        x2 = pw.rms_norm(hd, n["pre_norm_2"], eps, offset=False)
    y = moe.experts(x2, w, top, ids, lambda gu, nn: _geglu(gu[:, :nn], gu[:, nn:]))
    out = moe.combine_norm(y, dd, n["post_norm_1"], n["post_norm_2"], k, eps)
    torch.cuda.synchronize()

    # the oracle's routing chain over the whole batch (what gemma_moe runs first); the unfused chain's
    # normed router input within one bf16 ulp of it
    scale = np32(wd["expert_scale"])
    r_ref = orc.rms_norm(np32(h), wd["router_norm"].numpy(), eps)
    if not fused_router:
        np.testing.assert_allclose(np32(r), r_ref, rtol=2 ** -7, atol=1e-7)
    l_ref, _ = orc.router(r_ref, np32(wd["router"]))
    _, ids_ref = orc.route(l_ref, k, scale)
    gl, gids = logits.cpu().numpy(), ids.cpu().numpy()
    np.testing.assert_allclose(gl, l_ref, rtol=1e-3, atol=1e-4)
    # bit-exact: the GPU's ids are the oracle's route of the GPU's own logits
    np.testing.assert_array_equal(gids, orc.route(gl, k, scale)[1])
    # and the oracle's whole chain wherever it can be: with every logit within delta of the oracle's
    # (delta from a one-ulp difference in the normed router input), two experts can only trade places
    # where their oracle logits lie within 2 * delta
    delta = np.abs(gl - l_ref).max(1)
    differ = (gids != ids_ref).any(1)
    assert not (differ & ~near_tied(l_ref, k, delta)).any(), "routing differs away from a near tie"
    assert differ.sum() <= max(2, T // 256), f"{differ.sum()} tokens route differently"
    np.testing.assert_allclose(np32(x2), orc.rms_norm(np32(h), np32(norms["pre_norm_2"]), eps),
                               rtol=2 ** -7, atol=1e-6)
    agree = np.flatnonzero(~differ)
    tokens = agree if T <= 64 else np.sort(np.random.default_rng(T).choice(agree, 96, replace=False))
    o = {kk: (np32(v) if isinstance(v, torch.Tensor) else v) for kk, v in wd.items()}
    o.update({kk: np32(v) for kk, v in norms.items()})
    ref = orc.gemma_moe(np32(h), np32(dense), o, eps, "bf16", tokens=tokens)
    assert_close(np32(out)[tokens], ref, REL_BF16, f"gemma _moe T={T}")
