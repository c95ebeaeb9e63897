"""Pins of the CPU oracle (oracle/moe_oracle.py, oracle/cpu_path.py) -- no GPU.

The reference's own tests hold no golden vectors for the MoE path (flide's tests/ never touch
flide/kernels/moe.py), so the oracle is pinned by what fixes each piece independently of its code:
  * number formats against torch's bfloat16 / float8_e4m3fn casts (a separate implementation);
  * routing and align against brute force (Python sorting and loops) and closed forms;
  * experts, routing weights and norms against transformers' eager Gemma 4 modules, which are the
    reference's CPU torch path (Gemma4TextRouter, Gemma4TextExperts, Gemma4RMSNorm);
  * the FP8 experts against the dequantised float32 computation done with torch ops;
  * the activations against torch.nn.functional.
A planted mistake in any oracle function (a dropped term, a transposed operand, a wrong tie rule or
rounding) fails at least one of these."""
from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import cpu_path
from oracle import moe_oracle as orc

# --------------------------------------------------------------------------------------------------
# number formats
# --------------------------------------------------------------------------------------------------


def test_bf16_round_matches_torch():
    g = torch.Generator().manual_seed(0)
    x = torch.cat([torch.randn(200000, generator=g) * 10,
                   torch.tensor([0.0, -0.0, 1.0, 3.4e38, -3.4e38, 1e-40, -1e-40, float("inf"), -float("inf")]),
                   # exact ties between two bfloat16 values: lsb even and odd
                   torch.tensor([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8)])])
    got = orc.bf16_round(x.numpy())
    ref = x.to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(got, ref)
    assert np.isnan(orc.bf16_round(np.array([np.nan], np.float32))).all()


def test_f16_round_matches_torch():
    g = torch.Generator().manual_seed(1)
    x = torch.cat([torch.randn(200000, generator=g) * 30,
                   torch.tensor([0.0, -0.0, 65504.0, 65520.0, -70000.0, 6e-8, 3e-8, -1e-9]),
                   # exact ties between two half values: lsb even and odd
                   torch.tensor([1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, -(1.0 + 2 ** -11)])])
    np.testing.assert_array_equal(orc.f16_round(x.numpy()), x.half().float().numpy())


def test_e4m3fn_round_matches_torch():
    g = torch.Generator().manual_seed(1)
    codes = torch.arange(256, dtype=torch.uint8)
    reps = codes.view(torch.float8_e4m3fn).float()
    reps = reps[torch.isfinite(reps)]
    # midpoints between neighbouring representable values exercise ties-to-even
    srt = torch.sort(reps.unique()).values
    mids = (srt[1:] + srt[:-1]) / 2
    vals = torch.cat([reps, mids, (torch.randn(100000, generator=g) * 40).clamp(-448, 448),
                      torch.randn(20000, generator=g) * 2 ** -8, torch.tensor([-0.0, 2 ** -10, -2 ** -10])])
    got = orc.e4m3fn_round(vals.numpy())
    ref = vals.to(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(orc.e4m3fn_encode(got), vals.to(torch.float8_e4m3fn).view(torch.uint8).numpy())


def test_e4m3fn_decode_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    got = orc.e4m3fn_decode(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    np.testing.assert_array_equal(got[~np.isnan(got)], ref[~np.isnan(ref)])
    assert got[0x7E] == 448.0 and got[0x01] == 2.0 ** -9


def _torch_quantize_rows(w: torch.Tensor):
    # the reference's quantize_rows with torch's own ops (flide/kernels/fp8.py:25-26)
    scale = w.float().abs().amax(dim=1, keepdim=True).clamp(min=1e-12) * (1.0 / 448.0)
    return (w.float() / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn), scale


def test_quantize_rows_against_torch_and_invariants():
    g = torch.Generator().manual_seed(2)
    w = torch.randn(64, 300, generator=g) * torch.logspace(-8, 4, 64).unsqueeze(1)
    w[7] = 0.0
    w[9, 3] = 1e-30
    q, s = orc.quantize_rows(w.numpy())
    tq, ts = _torch_quantize_rows(w)
    np.testing.assert_array_equal(s, ts.numpy())
    np.testing.assert_array_equal(orc.e4m3fn_encode(q), tq.view(torch.uint8).numpy())
    # invariants: the row's amax lands on 448, a zero row stays zero with the floor scale
    nz = np.abs(w.numpy()).max(1) > 0
    assert np.all(np.abs(q[nz]).max(1) == 448.0)
    assert np.all(q[7] == 0) and s[7, 0] == np.float32(1e-12) * np.float32(1 / 448)
    # dequantised error within half an e4m3 quantum (2^-4 relative) above the subnormal range
    deq = q * s
    big = np.abs(q) >= 2 ** -6
    assert np.all(np.abs(deq - w.numpy())[big] <= np.abs(w.numpy())[big] * 2 ** -4 * 1.0001)


# --------------------------------------------------------------------------------------------------
# routing
# --------------------------------------------------------------------------------------------------
def _brute_ids(logits: np.ndarray, k: int) -> np.ndarray:
    return np.array([sorted(range(len(r)), key=lambda e: (-float(r[e]), e))[:k] for r in logits], np.int32)


@pytest.mark.parametrize("E,k", [(5, 1), (8, 3), (16, 2), (13, 13), (128, 8)])
def test_route_ids_brute_force(E, k):
    rng = np.random.default_rng(E * 10 + k)
    logits = rng.integers(-2, 3, (200, E)).astype(np.float32)       # many exact ties
    logits[:50] = rng.standard_normal((50, E)).astype(np.float32)
    w, ids = orc.route(logits, k)
    np.testing.assert_array_equal(ids, _brute_ids(logits, k))
    np.testing.assert_allclose(w.sum(1), 1.0, rtol=1e-6)


def test_route_closed_forms():
    E, k = 12, 4
    eq = np.zeros((3, E), np.float32)
    w, ids = orc.route(eq, k)
    np.testing.assert_array_equal(ids, np.tile(np.arange(k), (3, 1)))
    np.testing.assert_allclose(w, 1 / k, rtol=1e-7)
    rng = np.random.default_rng(0)
    logits = rng.standard_normal((50, E)).astype(np.float32)
    w1, ids1 = orc.route(logits, 1)
    np.testing.assert_allclose(w1, 1.0)
    np.testing.assert_array_equal(ids1[:, 0], logits.argmax(1))
    scale = rng.random(E).astype(np.float32) + 0.5
    ws, idss = orc.route(logits, k, scale)
    w0, ids0 = orc.route(logits, k)
    np.testing.assert_array_equal(idss, ids0)
    np.testing.assert_allclose(ws, w0 * scale[ids0], rtol=1e-6)
    # weights are the renormalised softmax of the chosen logits
    p = torch.softmax(torch.from_numpy(logits).double(), -1).numpy()
    top = np.take_along_axis(p, ids0.astype(np.int64), 1)
    np.testing.assert_allclose(w0, top / top.sum(1, keepdims=True), rtol=1e-6)


def _tiny_gemma_config(H=64, E=16, k=2, I=32):
    from transformers.models.gemma4.configuration_gemma4 import Gemma4TextConfig

    return Gemma4TextConfig(hidden_size=H, intermediate_size=2 * I, num_hidden_layers=1, num_attention_heads=2,
                            num_key_value_heads=1, head_dim=16, vocab_size=64, enable_moe_block=True,
                            num_experts=E, top_k_experts=k, moe_intermediate_size=I,
                            hidden_activation="gelu_pytorch_tanh")


def test_route_matches_transformers_router():
    from transformers.models.gemma4.modeling_gemma4 import Gemma4TextRouter

    torch.manual_seed(0)
    cfg = _tiny_gemma_config(H=64, E=16, k=4)
    r = Gemma4TextRouter(cfg).float()
    with torch.no_grad():
        r.proj.weight.normal_(0, 0.3)
        r.scale.uniform_(0.5, 1.5)
        r.per_expert_scale.uniform_(0.5, 1.5)
    h = torch.randn(100, 64)
    with torch.no_grad():
        _, tw, ti = r(h)
        normed = r.norm(h) * r.scale * r.scalar_root_size
        logits = r.proj(normed)
    w, ids = orc.route(logits.numpy(), 4, r.per_expert_scale.detach().numpy())
    np.testing.assert_array_equal(ids, ti.numpy())
    np.testing.assert_allclose(w, tw.numpy(), rtol=1e-5, atol=1e-7)


# --------------------------------------------------------------------------------------------------
# align
# --------------------------------------------------------------------------------------------------
def _brute_align(ids: np.ndarray, E: int, bm: int):
    flat = ids.reshape(-1).tolist()
    n = len(flat)
    rows, blocks = [], []
    for e in range(E):
        mine = [p for p in range(n) if flat[p] == e]
        padded = -(-len(mine) // bm) * bm
        seg = mine + [n] * (padded - len(mine))
        rows += seg
        blocks += [e] * (padded // bm)
    return np.array(rows, np.int64), np.array(blocks, np.int64), len(rows)


@pytest.mark.parametrize("T,E,k,bm", [(10, 4, 2, 4), (33, 7, 3, 1), (64, 16, 2, 16), (5, 30, 5, 8), (0, 4, 2, 4)])
def test_align_brute_force(T, E, k, bm):
    rng = np.random.default_rng(T + E)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]) if T else np.zeros((0, k), np.int64)
    al = orc.align(ids, E, bm)
    rows, blocks, used = _brute_align(ids, E, bm)
    assert int(al["used"][0]) == used
    np.testing.assert_array_equal(al["rows"][:used], rows)
    np.testing.assert_array_equal(al["blocks"][:used // bm], blocks)
    assert al["total"] == -(-(T * k + E * (bm - 1)) // bm) * bm >= used
    np.testing.assert_array_equal(al["counts"], np.bincount(ids.reshape(-1), minlength=E))
    np.testing.assert_array_equal(al["perm"], np.argsort(ids.reshape(-1), kind="stable"))


# --------------------------------------------------------------------------------------------------
# activations, experts, norms against torch / transformers
# --------------------------------------------------------------------------------------------------
def test_activations_match_torch():
    g = torch.Generator().manual_seed(3)
    a = torch.randn(64, 100, generator=g, dtype=torch.float64) * 3
    b = torch.randn(64, 100, generator=g, dtype=torch.float64)
    np.testing.assert_allclose(orc.geglu(a.numpy(), b.numpy(), "fp32"),
                               (F.gelu(a, approximate="tanh") * b).numpy(), rtol=1e-6, atol=1e-7)
    gu = torch.cat([a, b], 1)
    np.testing.assert_allclose(orc.swiglu(gu.numpy(), 100, "fp32"), (F.silu(a) * b).numpy(), rtol=1e-6, atol=1e-7)


def test_experts_match_transformers_gemma4():
    from transformers.models.gemma4.modeling_gemma4 import Gemma4TextExperts

    torch.manual_seed(1)
    H, E, k, I, T = 64, 8, 2, 32, 40
    cfg = _tiny_gemma_config(H=H, E=E, k=k, I=I)
    ex = Gemma4TextExperts(cfg).float()
    with torch.no_grad():
        ex.gate_up_proj.normal_(0, 0.1)
        ex.down_proj.normal_(0, 0.1)
    x = torch.randn(T, H)
    logits = torch.randn(T, E)
    w, ids = orc.route(logits.numpy(), k)
    with torch.no_grad():
        ref = ex(x, torch.from_numpy(ids).long(), torch.from_numpy(w)).numpy()
    y = orc.experts(x.numpy(), ex.gate_up_proj.detach().numpy(), ex.down_proj.detach().numpy(), w, ids, I, "geglu",
                    "fp32")
    np.testing.assert_allclose(orc.combine_sum(y, k, "fp32"), ref, rtol=1e-4, atol=1e-5)
    # and the torch CPU path the bench times
    cp = cpu_path.experts_cpu(x, ex.gate_up_proj.detach(), ex.down_proj.detach(), torch.from_numpy(w),
                              torch.from_numpy(ids))
    np.testing.assert_allclose(cp.numpy(), ref, rtol=1e-5, atol=1e-6)


def test_combine_norm_matches_gemma4_rmsnorm():
    from transformers.models.gemma4.modeling_gemma4 import Gemma4RMSNorm

    torch.manual_seed(2)
    T, H, k, eps = 9, 48, 3, 1e-6
    n1, n2 = Gemma4RMSNorm(H, eps=eps), Gemma4RMSNorm(H, eps=eps)
    with torch.no_grad():
        n1.weight.uniform_(0.5, 1.5)
        n2.weight.uniform_(0.5, 1.5)
    y = torch.randn(T * k, H)
    dense = torch.randn(T, H)
    with torch.no_grad():
        ref = (n1(dense) + n2(y.reshape(T, k, H).sum(1))).numpy()
    got = orc.combine_norm(y.numpy(), dense.numpy(), n1.weight.detach().numpy(), n2.weight.detach().numpy(), k, eps,
                           "fp32")
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6)
    # rms_norm (no offset) is the same norm
    rn = orc.rms_norm(dense.numpy(), n1.weight.detach().numpy(), eps, offset=False, dtype="fp32")
    with torch.no_grad():
        np.testing.assert_allclose(rn, n1(dense).numpy(), rtol=1e-5, atol=1e-6)


def test_sandwich_matches_gemma4_decoder_layer():
    """pointwise.sandwich is the tail of transformers' Gemma4TextDecoderLayer (no per-layer input):
    (residual + post_feedforward_layernorm(d)) * layer_scalar, then the next layer's input_layernorm."""
    from transformers.models.gemma4.modeling_gemma4 import Gemma4RMSNorm

    torch.manual_seed(5)
    T, H, eps = 7, 40, 1e-6
    post, nxt = Gemma4RMSNorm(H, eps=eps), Gemma4RMSNorm(H, eps=eps)
    with torch.no_grad():
        post.weight.uniform_(0.5, 1.5)
        nxt.weight.uniform_(0.5, 1.5)
    d, h, s = torch.randn(T, H), torch.randn(T, H) * 3, torch.tensor([0.7])
    with torch.no_grad():
        ref_h = (h + post(d)) * s
        ref_x = nxt(ref_h)
    got_h, got_x = orc.sandwich(d.numpy(), h.numpy(), post.weight.detach().numpy(), eps, s.numpy(),
                                nxt.weight.detach().numpy(), "fp32")
    np.testing.assert_allclose(got_h, ref_h.numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(got_x, ref_x.numpy(), rtol=1e-5, atol=1e-6)


def test_sandwich_invariants():
    rng = np.random.default_rng(6)
    T, H = 5, 64
    d = rng.standard_normal((T, H))
    h = orc.bf16_round(rng.standard_normal((T, H)).astype(np.float32))
    w1, w2 = rng.uniform(0.5, 1.5, H), rng.uniform(0.5, 1.5, H)
    # RMS(d) is scale-free: with eps = 0, d and 2 d give the same bits
    a = orc.sandwich(d, h, w1, 0.0, None, w2)
    b = orc.sandwich(2 * d, h, w1, 0.0, None, w2)
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])
    # a zero post-norm weight leaves the (bf16) residual exactly; the layer scalar multiplies it
    np.testing.assert_array_equal(orc.sandwich(d, h, np.zeros(H), 1e-6)[0], h)
    np.testing.assert_array_equal(orc.sandwich(d, h, np.zeros(H), 1e-6, np.array([2.0]))[0], 2 * h)
    # the next norm with unit weight has unit RMS up to one bf16 rounding
    _, x = orc.sandwich(d, h, w1, 1e-12, None, np.ones(H))
    rms = np.sqrt((x.astype(np.float64) ** 2).mean(-1))
    np.testing.assert_allclose(rms, 1.0, atol=2 ** -8)
    assert orc.sandwich(d, h, w1, 1e-6)[1] is None


def test_combine_qwen_closed_form():
    rng = np.random.default_rng(4)
    T, H, k = 5, 16, 3
    y = rng.standard_normal((T * k, H)).astype(np.float32)
    sh = rng.standard_normal((T, H)).astype(np.float32)
    g = rng.standard_normal((T, 1)).astype(np.float32)
    got = orc.combine(y, sh, g, k, "fp32")
    ref = torch.from_numpy(y).double().reshape(T, k, H).sum(1) + torch.from_numpy(sh).double() * torch.sigmoid(
        torch.from_numpy(g).double())
    np.testing.assert_allclose(got, ref.numpy(), rtol=1e-6, atol=1e-6)


def test_experts_fp8_is_the_dequantised_computation():
    g = torch.Generator().manual_seed(5)
    T, H, E, k, I = 24, 64, 6, 2, 32
    x = (torch.randn(T, H, generator=g)).to(torch.bfloat16).float()
    wgu = torch.randn(E, 2 * I, H, generator=g) * 0.02
    wd = torch.randn(E, H, I, generator=g) * 0.02
    qgu, sgu = zip(*[_torch_quantize_rows(wgu[e]) for e in range(E)])
    qd, sd = zip(*[_torch_quantize_rows(wd[e]) for e in range(E)])
    qgu, qd = torch.stack(qgu).float(), torch.stack(qd).float()
    sgu, sd = torch.stack(sgu)[..., 0], torch.stack(sd)[..., 0]
    logits = torch.randn(T, E, generator=g)
    w, ids = orc.route(logits.numpy(), k)
    y = orc.experts_fp8(x.numpy(), qgu.numpy(), sgu.numpy(), qd.numpy(), sd.numpy(), w, ids, I)
    # the same computation written with torch ops: quantise rows, dequantise, float32 products
    qx, sx = _torch_quantize_rows(x)
    deq_x = qx.float() * sx
    ref = torch.empty(T * k, H)
    for p in range(T * k):
        t, e = p // k, int(ids.reshape(-1)[p])
        gu = (deq_x[t] @ (qgu[e] * sgu[e][:, None]).T).to(torch.bfloat16).float()
        a = (F.gelu(gu[:I], approximate="tanh") * gu[I:]).to(torch.bfloat16).float()
        qa, sa = _torch_quantize_rows(a[None])
        ref[p] = ((qa.float() * sa)[0] @ (qd[e] * sd[e][:, None]).T * float(w.reshape(-1)[p])).to(
            torch.bfloat16).float()
    np.testing.assert_allclose(y, ref.numpy(), rtol=2e-2, atol=2e-4)


def test_gemma_layer_composition():
    """gemma_moe = rms_norm -> router -> route -> rms_norm -> experts -> combine_norm (fused.py:231-240)."""
    rng = np.random.default_rng(6)
    T, H, E, k, I = 12, 32, 6, 2, 16
    h = rng.standard_normal((T, H)).astype(np.float32)
    wd = {"router_norm": np.full(H, H ** -0.5, np.float32), "router": rng.standard_normal((E, H)).astype(np.float32),
          "expert_scale": np.ones(E, np.float32), "topk": k, "inter": I,
          "pre_norm_2": np.ones(H, np.float32), "experts": rng.standard_normal((E, 2 * I, H)).astype(np.float32) * 0.1,
          "experts_down": rng.standard_normal((E, H, I)).astype(np.float32) * 0.1,
          "post_norm_1": np.ones(H, np.float32), "post_norm_2": np.ones(H, np.float32)}
    dense = rng.standard_normal((T, H)).astype(np.float32)
    out = orc.gemma_moe(h, dense, wd, 1e-6, "fp32")
    # by hand with torch
    ht = torch.from_numpy(h).double()
    r = ht * torch.rsqrt(ht.pow(2).mean(-1, keepdim=True) + 1e-6) * H ** -0.5
    logits = (r @ torch.from_numpy(wd["router"]).double().T).float()
    w, ids = orc.route(logits.numpy(), k)
    x2 = ht * torch.rsqrt(ht.pow(2).mean(-1, keepdim=True) + 1e-6)
    y = cpu_path.experts_cpu(x2.float(), torch.from_numpy(wd["experts"]), torch.from_numpy(wd["experts_down"]),
                             torch.from_numpy(w), torch.from_numpy(ids)).double()
    dn = torch.from_numpy(dense).double()
    ref = dn * torch.rsqrt(dn.pow(2).mean(-1, keepdim=True) + 1e-6) + y * torch.rsqrt(y.pow(2).mean(-1, keepdim=True)
                                                                                      + 1e-6)
    np.testing.assert_allclose(out, ref.numpy(), rtol=1e-4, atol=1e-5)


def test_cpu_path_route_matches_oracle():
    rng = np.random.default_rng(7)
    logits = rng.integers(-3, 3, (300, 32)).astype(np.float32)
    scale = (rng.random(32) + 0.5).astype(np.float32)
    w, ids = orc.route(logits, 6, scale)
    tw, tids = cpu_path.route_cpu(torch.from_numpy(logits), 6, torch.from_numpy(scale))
    np.testing.assert_array_equal(tids.numpy(), ids)
    np.testing.assert_allclose(tw.numpy(), w, rtol=1e-6)


@pytest.mark.parametrize("perm", list(itertools.permutations(range(3))))
def test_route_invariant_to_expert_relabelling(perm):
    """Relabelling experts permutes the chosen ids accordingly when there are no ties."""
    rng = np.random.default_rng(8)
    logits = rng.standard_normal((40, 3)).astype(np.float32)
    p = np.array(perm)
    _, ids = orc.route(logits, 2)
    _, ids_p = orc.route(logits[:, p], 2)
    np.testing.assert_array_equal(p[ids_p], ids)


# --------------------------------------------------------------------------------------------------
# grouped, the router's shared-expert gate, the zero-centred norm and Qwen's layer
# --------------------------------------------------------------------------------------------------
def _grouped_brute(a, w, ids, topk, by_token, weights, dtype):
    """out[p] for every pair p, one dot product at a time in Python floats (float64, K in order), the
    expert taken straight from the ids (not from align's blocks), times weights[p], rounded once."""
    flat = np.asarray(ids).reshape(-1)
    n, N = flat.size, w.shape[1]
    out = np.empty((n, N), np.float32)
    for p in range(n):
        src = p // topk if by_token else p
        e = int(flat[p])
        for c in range(N):
            s = 0.0
            for kk in range(a.shape[1]):
                s += float(a[src, kk]) * float(w[e, c, kk])
            if weights is not None:
                s *= float(weights[p])
            out[p, c] = s
    return orc._round(out, dtype)


@pytest.mark.parametrize("bm,by_token,mul_w,dtype", [(4, True, False, "bf16"), (8, False, True, "fp32"),
                                                    (3, True, True, "f16"), (16, False, False, "bf16")])
def test_grouped_brute_force(bm, by_token, mul_w, dtype):
    """grouped over align's padded layout equals a per-pair loop that never looks at the layout: every
    pair's row, every padding row untouched, any tile."""
    rng = np.random.default_rng(bm + 10 * by_token)
    T, E, k, N, K = 23, 5, 2, 7, 12
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)])
    ids[:6] = [3, 1]                    # one expert busier than a block, expert 4 rare
    a = orc.bf16_round(rng.standard_normal((T if by_token else T * k, K)).astype(np.float32))
    w = orc.bf16_round(rng.standard_normal((E, N, K)).astype(np.float32))
    wts = rng.random(T * k).astype(np.float32) if mul_w else None
    al = orc.align(ids, E, bm)
    got = orc.grouped(a, w, al["rows"], al["blocks"], al["used"], T * k, k, by_token, wts, bm=bm, out_dtype=dtype)
    ref = _grouped_brute(a, w, ids, k, by_token, wts, dtype)
    np.testing.assert_allclose(got, ref, rtol=2 ** -22, atol=0)
    # a row no pair names (past n_pairs) is never written
    out = np.full((T * k + 3, N), np.nan, np.float32)
    orc.grouped(a, w, al["rows"], al["blocks"], al["used"], T * k, k, by_token, wts, bm=bm, out_dtype=dtype, out=out)
    assert np.isnan(out[T * k:]).all() and not np.isnan(out[:T * k]).any()


@pytest.mark.parametrize("act", ["geglu", "swiglu"])
@pytest.mark.parametrize("bm", [4, 16])
def test_grouped_composition_is_experts(act, bm):
    """align -> grouped(gate/up, by token) -> act -> grouped(down, x weight) -- the reference's experts()
    (moe.py:336-353) -- gives orc.experts' bits (which transformers' Gemma4TextExperts pins)."""
    rng = np.random.default_rng(20 + bm)
    T, E, k, H, I = 31, 6, 3, 40, 24
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)])
    logits = rng.standard_normal((T, E)).astype(np.float32)
    top, ids = orc.route(logits, k)
    x = orc.bf16_round(rng.standard_normal((T, H)).astype(np.float32))
    wgu = orc.bf16_round((rng.standard_normal((E, 2 * I, H)) * 0.2).astype(np.float32))
    wd = orc.bf16_round((rng.standard_normal((E, H, I)) * 0.2).astype(np.float32))
    al = orc.align(ids, E, bm)
    gu = orc.grouped(x, wgu, al["rows"], al["blocks"], al["used"], T * k, k, True, bm=bm, out_dtype="bf16")
    a = orc.geglu(gu[:, :I], gu[:, I:], "bf16") if act == "geglu" else orc.swiglu(gu, I, "bf16")
    y = orc.grouped(a, wd, al["rows"], al["blocks"], al["used"], T * k, k, False, top.reshape(-1), bm=bm,
                    out_dtype="fp32")
    ref = orc.experts(x, wgu, wd, top, ids, I, act, "bf16")
    np.testing.assert_array_equal(y, ref)


def test_router_gate_term_matches_linear():
    """router's logits and its shared-expert gate logit (moe.py:152-169) against torch's F.linear in
    float64 (Qwen3_5MoeTopKRouter and shared_expert_gate are both F.linear)."""
    rng = np.random.default_rng(30)
    x = rng.standard_normal((17, 96)).astype(np.float32)
    wr = rng.standard_normal((12, 96)).astype(np.float32)
    wg = rng.standard_normal(96).astype(np.float32)
    logits, gate = orc.router(x, wr, wg)
    xt = torch.from_numpy(x).double()
    np.testing.assert_allclose(logits, F.linear(xt, torch.from_numpy(wr).double()).float().numpy(), rtol=1e-6)
    np.testing.assert_allclose(gate, F.linear(xt, torch.from_numpy(wg).double()[None]).float().numpy(), rtol=1e-6)
    assert gate.shape == (17, 1) and orc.router(x, wr)[1] is None


def test_rms_norm_offset_matches_qwen():
    """rms_norm(offset=True), the zero-centred weight (pointwise.py:21-49), against transformers'
    Qwen3_5MoeRMSNorm (float32 math, (1 + w), rounded to the input's dtype): within one bf16 rounding of
    each other (float32 vs float64 intermediates), and equal almost everywhere."""
    from transformers.models.qwen3_5_moe.modeling_qwen3_5_moe import Qwen3_5MoeRMSNorm

    torch.manual_seed(31)
    N = 256
    m = Qwen3_5MoeRMSNorm(N, eps=1e-6)
    with torch.no_grad():
        m.weight.copy_(torch.randn(N) * 0.3)
    x = (torch.randn(50, N) * 3).to(torch.bfloat16)
    with torch.no_grad():
        ref = m(x).float().numpy()
    got = orc.rms_norm(x.float().numpy(), m.weight.detach().numpy(), 1e-6, offset=True, dtype="bf16")
    np.testing.assert_allclose(got, ref, rtol=2 ** -7, atol=1e-6)
    assert (got == ref).mean() > 0.99
    # offset=False is a different formula: it must not pass for this weight
    plain = orc.rms_norm(x.float().numpy(), m.weight.detach().numpy(), 1e-6, offset=False, dtype="bf16")
    assert not np.allclose(plain, ref, rtol=1e-2)


def test_qwen_moe_matches_transformers_block():
    """qwen_moe (moe.py:356-369) against transformers' Qwen3_5MoeSparseMoeBlock in float32: router and
    softmax top-k, the SwiGLU experts loop, the shared expert and its sigmoid gate."""
    from transformers.models.qwen3_5_moe.configuration_qwen3_5_moe import Qwen3_5MoeTextConfig
    from transformers.models.qwen3_5_moe.modeling_qwen3_5_moe import Qwen3_5MoeSparseMoeBlock

    torch.manual_seed(32)
    H, E, k, I, SI, T = 64, 8, 2, 32, 48, 30
    cfg = Qwen3_5MoeTextConfig(hidden_size=H, num_experts=E, num_experts_per_tok=k, moe_intermediate_size=I,
                               shared_expert_intermediate_size=SI, hidden_act="silu")
    blk = Qwen3_5MoeSparseMoeBlock(cfg).float()
    with torch.no_grad():
        for p in blk.parameters():
            p.normal_(0, 0.2)
    x = torch.randn(1, T, H)
    with torch.no_grad():
        ref = blk(x)[0].numpy()
    se = blk.shared_expert
    wd = {"topk": k, "inter": I, "shared_inter": SI,
          "router": blk.gate.weight.detach().numpy(), "shared_gate": blk.shared_expert_gate.weight.detach().numpy(),
          "experts": blk.experts.gate_up_proj.detach().numpy(), "experts_down": blk.experts.down_proj.detach().numpy(),
          "shared_gate_up": torch.cat([se.gate_proj.weight, se.up_proj.weight]).detach().numpy(),
          "shared_down": se.down_proj.weight.detach().numpy()}
    got = orc.qwen_moe(x[0].numpy(), wd, "fp32")
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)
