"""Mixture-of-experts feed-forward on MI355X: the public functions of flide/kernels/moe.py with the same
signatures, backed by hand-written HIP kernels for gfx950 (libflide_moe.so, include/flide_moe.h).

Semantics kept from the reference:
  * router logits (and the shared-expert gate logit) summed and stored in float32 (moe.py:152-169);
  * routing: the top k of the softmax in descending order, ties to the lower expert id, renormalised,
    times per_expert_scale when given (moe.py:172-204). The selection runs on the float32 logits, whose
    order the softmax keeps, so it is exact and does not depend on how exp rounds;
  * align: the pair indices t*k + j sorted by expert, ascending within an expert, each expert padded to
    a multiple of bm with the sentinel T*k; `used` stays on the device (moe.py:207-253);
  * grouped products with float32 accumulation in one fixed K order, so a row's bits do not depend on
    the tile or the batch (moe.py:32-37); 16-bit experts return float32 rows to the combine, FP8
    experts return rows in the activation dtype (moe.py:336-353);
  * combine / combine_norm: the token's k rows summed in slot order in float32, rounded once.
Every shape is fixed by T, k and E, nothing reads the device on the host and nothing synchronises, so
every function can be captured into a HIP graph (torch.cuda.graph).

Differences by design: the gate/up activation (GeGLU or SwiGLU) runs inside the gate/up product's
epilogue when `experts` recognises `act`; `tile` returns MI355X tiles. Tensors must live on the GPU:
there is no CPU branch (the reference has none either).
"""
from __future__ import annotations

import torch

from .. import _hip
from . import pointwise

BM, BN, BK = 64, 128, 64
BK8 = 128


def tile(pairs: int, fp8: bool, device=None) -> tuple[int, int, int, int, int]:
    """(block rows, block columns, waves, stages, row blocks per group) for a layer of `pairs` pairs.
    Block rows are what `align` pads each expert to. 32 rows (decode) stream each expert's weights through
    LDS in whole 128-byte lines; 16 rows stream them straight into MFMA registers (kept for callers that
    ask for it); 64 and 128 rows are the prefill tiles. The K order is the same for every tile, so the
    bits do not change with the choice. The switch points are where the two products' summed time
    crosses on MI355X at the Gemma shape: 16-bit 32 -> 128 rows between 2048 and 3072 pairs (64 rows
    is never the fastest); float8 32 -> 64 rows past 512 pairs, 64 -> 128 past 8192."""
    if fp8:
        bm = 32 if pairs <= 512 else 64 if pairs <= 8192 else 128
    else:
        bm = 32 if pairs <= 2048 else 128
    return bm, BN, 4, 2, 0


def _tile(t: tuple | None) -> tuple[int, int, int, int, int]:
    t = tuple(t or (BM, BN, 4, 2))
    return t + (0,) * (5 - len(t))


def router(x: torch.Tensor, wr: torch.Tensor, wg: torch.Tensor | None = None):
    """Scores every expert for each token: returns float32 logits [T, E] = x @ wr^T and, when `wg` [H] is
    given, the shared-expert gate logit x @ wg as [T, 1] (else None). Both sums stay in float32 end to end
    (moe.py:152-169)."""
    dev = _hip.require_gpu(x, wr, wg)
    if x.stride(-1) != 1:
        x = x.contiguous()
    if wr.stride(-1) != 1:
        wr = wr.contiguous()
    if wr.dtype != x.dtype or (wg is not None and wg.dtype != x.dtype):
        raise TypeError(f"router weights must match x's dtype {x.dtype}")
    T, H = x.shape
    E = wr.shape[0]
    logits = torch.empty(T, E, device=dev, dtype=torch.float32)
    gate = torch.empty(T, 1, device=dev, dtype=torch.float32) if wg is not None else None
    if T:
        wgc = wg.contiguous() if wg is not None else None
        _hip.call("flide_moe_router", x.data_ptr(), x.stride(0), T, H, _hip.dtype_code(x.dtype), wr.data_ptr(),
                  wr.stride(0), E, _hip.ptr(wgc), logits.data_ptr(), logits.stride(0), _hip.ptr(gate),
                  _hip.stream(dev))
    return logits, gate


ROUTER_NORM_MAX_H = 8192   # flide_moe_router_norm's limit (include/flide_moe.h)


def router_norm(h: torch.Tensor, norm_w: torch.Tensor, wr: torch.Tensor, eps: float,
                norm2_w: torch.Tensor | None = None):
    """Gemma 4's router input fused into the router (an extension; flide/backbones/gemma4/fused.py:234-237
    runs it as three calls): (logits f32 [T, E], x2 [T, H] or None) for the residual stream h [T, H], with
    logits = router(rms_norm(h, norm_w), wr) and x2 = rms_norm(h, norm2_w) (pointwise.py:21-49, no offset,
    rounded to h's dtype). Both norms share one statistic per token, computed once."""
    dev = _hip.require_gpu(h, norm_w, wr, norm2_w)
    T, H = h.shape
    E = wr.shape[0]
    if H > ROUTER_NORM_MAX_H:   # the fused kernel stages both weights in LDS: the three calls instead
        from flide_amd.kernels import pointwise as pw
        logits, _ = router(pw.rms_norm(h, norm_w, eps, offset=False), wr)
        return logits, (pw.rms_norm(h, norm2_w, eps, offset=False) if norm2_w is not None else None)
    if h.stride(-1) != 1:
        h = h.contiguous()
    wr = wr.contiguous()
    nw = norm_w.float().contiguous()
    logits = torch.empty(T, E, device=dev, dtype=torch.float32)
    x2 = torch.empty_like(h) if norm2_w is not None else None
    n2 = norm2_w.contiguous() if norm2_w is not None else None
    if T:
        _hip.call("flide_moe_router_norm", h.data_ptr(), h.stride(0), T, H, _hip.dtype_code(h.dtype), nw.data_ptr(),
                  wr.data_ptr(), wr.stride(0), E, float(eps), logits.data_ptr(), logits.stride(0), _hip.ptr(n2),
                  _hip.dtype_code(n2.dtype) if n2 is not None else 0, _hip.ptr(x2),
                  x2.stride(0) if x2 is not None else 0, _hip.stream(dev))
    return logits, x2


def route(logits: torch.Tensor, k: int, scale: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(weights [T, k] float32, experts [T, k] int32) from router logits [T, E]: the top k in descending
    order (ties to the lower id), renormalised to sum to one, times each expert's `scale` [E] when given
    (moe.py:195-204)."""
    dev = _hip.require_gpu(logits, scale)
    if logits.dtype != torch.float32:
        raise TypeError("route takes float32 logits")
    if logits.stride(-1) != 1:
        logits = logits.contiguous()
    T, E = logits.shape
    w = torch.empty(T, k, device=dev, dtype=torch.float32)
    ids = torch.empty(T, k, device=dev, dtype=torch.int32)
    if T:
        sc = scale.contiguous() if scale is not None else None
        _hip.call("flide_moe_route", logits.data_ptr(), logits.stride(0), T, E, k, _hip.ptr(sc),
                  _hip.dtype_code(sc.dtype) if sc is not None else 0, w.data_ptr(), ids.data_ptr(),
                  _hip.stream(dev))
    return w, ids


def align(ids: torch.Tensor, experts: int, bm: int = BM, counts: torch.Tensor | None = None):
    """(rows, expert of each block, rows in use) for top-k ids [T, k] (moe.py:237-253). `counts`, when
    given (int32 [experts]), also receives the pairs per expert."""
    dev = _hip.require_gpu(ids)
    if ids.dtype != torch.int32:
        raise TypeError("align takes int32 expert ids")
    T, K = ids.shape
    n = T * K
    flat = ids.reshape(-1).contiguous()
    total = -(-(n + experts * (bm - 1)) // bm) * bm
    rows = torch.empty(total, dtype=torch.int32, device=dev)
    blocks = torch.empty(total // bm, dtype=torch.int32, device=dev)
    used = torch.empty(1, dtype=torch.int32, device=dev)
    nbytes = _hip.query("flide_moe_align_workspace", n, experts)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    _hip.call("flide_moe_align", flat.data_ptr(), n, experts, bm, rows.data_ptr(), blocks.data_ptr(),
              used.data_ptr(), _hip.ptr(counts), ws.data_ptr(), nbytes, _hip.stream(dev))
    return rows, blocks, used


def _grouped_common(a, w, out, rows, blocks, used, weights, bm):
    if rows.numel() != blocks.numel() * bm:
        raise ValueError(f"rows ({rows.numel()}) must hold blocks ({blocks.numel()}) x the tile's {bm} rows: "
                         "pass the tile align padded with")
    if rows.dtype != torch.int32 or blocks.dtype != torch.int32 or used.dtype != torch.int32:
        raise TypeError("rows, blocks and used are align's int32 outputs")
    if w.stride(-1) != 1:
        w = w.contiguous()
    if a.stride(-1) != 1:
        a = a.contiguous()
    if weights is not None:
        weights = weights.contiguous()
        if weights.dtype != torch.float32:
            weights = weights.float()
    if out.stride(-1) != 1:
        raise ValueError("out needs a contiguous last dimension")
    return a, w, weights


def grouped(a: torch.Tensor, w: torch.Tensor, out: torch.Tensor, rows, blocks, used, topk: int, by_token: bool,
            weights: torch.Tensor | None = None, tile: tuple | None = None, act: int = _hip.ACT_NONE) -> torch.Tensor:
    """For every pair p that `align` placed: out[p] = a[r] @ w[e].T with e the block's expert and r the
    pair's token (by_token) or p itself, scaled by weights[p] when weights are given (moe.py:286-299).
    `tile[0]` must equal the bm passed to `align`. `act` (an extension) applies GeGLU or SwiGLU to the gate
    and up halves inside the epilogue, so out has w.shape[1] // 2 columns."""
    dev = _hip.require_gpu(a, w, out, rows, blocks, used, weights)
    bm, bn = _tile(tile)[:2]
    a, w, weights = _grouped_common(a, w, out, rows, blocks, used, weights, bm)
    n_pairs = out.shape[0]
    N, KD = w.shape[1], w.shape[2]
    _hip.call("flide_moe_grouped", a.data_ptr(), a.stride(0), _hip.dtype_code(a.dtype), w.data_ptr(), w.stride(0),
              w.stride(1), N, KD, out.data_ptr(), out.stride(0), _hip.dtype_code(out.dtype), _hip.ptr(weights),
              rows.data_ptr(), blocks.data_ptr(), used.data_ptr(), n_pairs, blocks.shape[0], topk,
              int(bool(by_token)), act, bm, bn, _hip.stream(dev))
    return out


def grouped_fp8(a: torch.Tensor, w: torch.Tensor, w_scale: torch.Tensor, out: torch.Tensor, rows, blocks, used,
                topk: int, by_token: bool, weights: torch.Tensor | None = None, tile: tuple | None = None,
                act: int = _hip.ACT_NONE) -> torch.Tensor:
    """`grouped` with float8 experts w [E, N, K] (scales [E, N]) and the rows going in scaled to float8 per
    row (moe.py:302-318)."""
    from .fp8 import quantize_tokens

    dev = _hip.require_gpu(a, w, w_scale, out, rows, blocks, used, weights)
    bm, bn = _tile(tile)[:2]
    if a.dtype == torch.float8_e4m3fn:
        raise TypeError("grouped_fp8 quantises its input itself; pass the 16-bit rows")
    a, w, weights = _grouped_common(a, w, out, rows, blocks, used, weights, bm)
    aq, sa = quantize_tokens(a)
    w_scale = w_scale.contiguous()
    n_pairs = out.shape[0]
    N, KD = w.shape[1], w.shape[2]
    _hip.call("flide_moe_grouped_fp8", aq.data_ptr(), aq.stride(0), sa.data_ptr(), w.data_ptr(), w.stride(0),
              w.stride(1), w_scale.data_ptr(), w_scale.stride(0), N, KD, out.data_ptr(), out.stride(0),
              _hip.dtype_code(out.dtype), _hip.ptr(weights), rows.data_ptr(), blocks.data_ptr(), used.data_ptr(),
              n_pairs, blocks.shape[0], topk, int(bool(by_token)), act, bm, bn, _hip.stream(dev))
    return out


@torch.no_grad()
def quantize_experts(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantises expert weights [E, N, K] row by row: float8 codes [E, N, K] and float32 scales [E, N]
    (each row's amax / 448), so that q * scale approximates w; every expert goes through one launch
    (moe.py:321-333)."""
    from .fp8 import quantize_rows

    E, N, K = w.shape
    q, s = quantize_rows(w.reshape(E * N, K))
    return q.reshape(E, N, K), s.reshape(E, N)


# --- recognising the activation between the two products -----------------------------------------
_ACT_CACHE: dict = {}
_ACT_CACHE_MAX = 256


def _guess_act(act) -> int:
    kind = getattr(act, "flide_act", None)
    if kind == "swiglu":
        return _hip.ACT_SWIGLU
    code = getattr(act, "__code__", None)
    # names the callable calls: globals (co_names) and closure variables (co_freevars)
    names = set(code.co_names) | set(code.co_freevars) if code is not None else set()
    names.add(getattr(act, "__name__", ""))
    if names & {"_geglu", "geglu"}:
        return _hip.ACT_GEGLU
    if names & {"swiglu", "_swiglu"}:
        return _hip.ACT_SWIGLU
    return _hip.ACT_NONE


def _act_key(act):
    """(key, objects the key names by id) for an activation callable: its code object, what its closure
    cells hold and what the globals it names resolve to. Two closures of one code over different
    callables or constants get different keys; a fresh lambda over the same helper (Gemma builds one per
    call) gets the same key. The objects are kept alive beside the verdict, so their ids stay unique."""
    code = getattr(act, "__code__", None)
    if code is None:
        return ("obj", id(act)), (act,)
    held = [c.cell_contents for c in (act.__closure__ or ()) if _cell_full(c)]
    glb = getattr(act, "__globals__", {})
    held += [glb[n] for n in code.co_names if n in glb]
    held += list(act.__defaults__ or ())
    return (code, tuple(id(o) for o in held)), tuple(held)


def _cell_full(cell) -> bool:
    try:
        cell.cell_contents
    except ValueError:
        return False
    return True


def _act_kind(act, device, dtype) -> int:
    """FLIDE_ACT_GEGLU when act(gu, n) is GELU-tanh(gu[:, :n]) * gu[:, n:], FLIDE_ACT_SWIGLU when it is
    silu(gu[:, :n]) * gu[:, n:], else FLIDE_ACT_NONE (the callable then runs between the products).
    A guess from the names the callable calls is confirmed, outside graph capture, by running it next to
    the fused formula on a probe (values up to +-40, within one 16-bit rounding of the formula); the
    verdict is cached per _act_key. During capture an unconfirmed callable runs unfused (that path
    captures too)."""
    key, held = _act_key(act)
    hit = _ACT_CACHE.get(key)
    if hit is not None:
        return hit[0]
    guess = _guess_act(act)
    if guess == _hip.ACT_NONE or torch.cuda.is_current_stream_capturing():
        return _hip.ACT_NONE
    g = torch.Generator(device="cpu").manual_seed(1234)
    gu = torch.randn(16, 64, generator=g) * 3
    gu[0, :32] = torch.linspace(-40, 40, 32)
    gu[1, 32:] = torch.linspace(-40, 40, 32)
    gu = gu.to(device=device, dtype=dtype)
    try:
        got = act(gu, 32)
    except Exception:  # noqa: BLE001 - a callable that cannot take the probe is not one we fuse
        got = None
    ok = False
    if isinstance(got, torch.Tensor) and tuple(got.shape) == (16, 32):
        ref = pointwise._gated(gu[:, :32], gu[:, 32:], guess).float()
        ok = bool(torch.allclose(got.float(), ref, rtol=2 ** -7, atol=1e-5))
    kind = guess if ok else _hip.ACT_NONE
    if len(_ACT_CACHE) >= _ACT_CACHE_MAX:
        _ACT_CACHE.clear()
    _ACT_CACHE[key] = (kind, held)
    return kind


def experts(x: torch.Tensor, w: dict, top: torch.Tensor, ids: torch.Tensor, act) -> torch.Tensor:
    """The routed experts' rows for x [T, hidden] on the routing (top, ids) [T, k]: [T * k, hidden], each the
    expert's output times its weight, in float32 for 16-bit experts and in the activation dtype for float8
    ones (moe.py:336-353). `act(gu, inter)` is the activation of the gate and up halves; GeGLU and SwiGLU
    run fused in the gate/up product, anything else runs as given between two grouped products."""
    dev = _hip.require_gpu(x, top, ids)
    if ids.dtype != torch.int32 or top.dtype != torch.float32:
        raise TypeError(f"experts takes route's float32 weights and int32 ids; got {top.dtype} and {ids.dtype}")
    if top.shape != ids.shape or top.shape[0] != x.shape[0]:
        raise ValueError(f"routing shapes {tuple(top.shape)}, {tuple(ids.shape)} do not match x {tuple(x.shape)}")
    T, H = x.shape
    K, I = top.shape[1], w["inter"]
    wgu, wd = w["experts"], w["experts_down"]
    E = wgu.shape[0]
    fp8 = "experts_scale" in w
    t = tile(T * K, fp8, dev)
    out_dtype = x.dtype if fp8 else torch.float32
    y = torch.empty(T * K, H, device=dev, dtype=out_dtype)
    if T == 0:
        return y
    if x.stride(-1) != 1:
        x = x.contiguous()
    kind = _act_kind(act, dev, x.dtype)
    if kind != _hip.ACT_NONE:
        wgu, wd = wgu.contiguous(), wd.contiguous()
        top_c, ids_c = top.contiguous(), ids.contiguous()
        sgu = w["experts_scale"].contiguous() if fp8 else None
        sd = w["experts_down_scale"].contiguous() if fp8 else None
        nbytes = _hip.query("flide_moe_experts_workspace", T, K, E, H, I, t[0], int(fp8))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        _hip.call("flide_moe_experts", x.data_ptr(), x.stride(0), _hip.dtype_code(x.dtype), T, H, top_c.data_ptr(),
                  ids_c.data_ptr(), K, wgu.data_ptr(), wd.data_ptr(), _hip.ptr(sgu), _hip.ptr(sd), E, I,
                  y.data_ptr(), kind, t[0], t[1], ws.data_ptr(), nbytes, _hip.stream(dev))
        return y
    rows, blocks, used = align(ids.contiguous(), E, t[0])
    if fp8:
        gu = grouped_fp8(x, wgu, w["experts_scale"], x.new_empty(T * K, 2 * I), rows, blocks, used, K, True, tile=t)
        return grouped_fp8(act(gu, I), wd, w["experts_down_scale"], y, rows, blocks, used, K, False,
                           top.reshape(-1), tile=t)
    gu = grouped(x, wgu, x.new_empty(T * K, 2 * I), rows, blocks, used, K, True, tile=t)
    return grouped(act(gu, I), wd, y, rows, blocks, used, K, False, top.reshape(-1), tile=t)


def combine(y: torch.Tensor, shared: torch.Tensor, gate: torch.Tensor, k: int) -> torch.Tensor:
    """Qwen's combine: out[t] = sum_j y[t*k + j] + sigmoid(gate[t]) * shared[t] for y [T*k, H], shared
    [T, H] and gate logits [T, 1]; float32 arithmetic, one rounding to shared's dtype (moe.py:269-277)."""
    dev = _hip.require_gpu(y, shared, gate)
    T, H = shared.shape
    shared = shared.contiguous()
    out = torch.empty_like(shared)
    if T:
        y = y.contiguous()
        g = gate.contiguous().float()
        _hip.call("flide_moe_combine", y.data_ptr(), _hip.dtype_code(y.dtype), shared.data_ptr(), g.data_ptr(),
                  out.data_ptr(), _hip.dtype_code(out.dtype), T, H, k, _hip.stream(dev))
    return out


def moe(x: torch.Tensor, w: dict, mm, swiglu) -> torch.Tensor:
    """The feed-forward of a Qwen3.5 MoE layer for rows x [T, hidden]: the routed experts' weighted sum plus
    the shared expert scaled by its sigmoid gate (moe.py:356-369). `mm` and `swiglu` are the backbone's
    own product and activation."""
    K = w["topk"]
    wr, wg = w["router"], w["shared_gate"]
    if isinstance(wr, torch.Tensor) and isinstance(wg, torch.Tensor):
        logits, gate = router(x, wr, wg)
    else:   # LoRA-wrapped weights are not plain tensors: the backbone's mm computes them
        logits, gate = mm(x, wr), mm(x, wg)
    top, ids = route(logits, K)
    y = experts(x, w, top, ids, swiglu)
    shared = mm(swiglu(mm(x, w["shared_gate_up"]), w["shared_inter"]), w["shared_down"])
    return combine(y, shared, gate, K)


def combine_norm_sandwich(y: torch.Tensor, dense: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, k: int,
                          eps: float, h: torch.Tensor, w_post: torch.Tensor, scale: torch.Tensor | None = None,
                          w_next: torch.Tensor | None = None):
    """Gemma 4's combine and the post-feed-forward step in one launch (an extension; the reference runs
    moe.combine_norm then pointwise.sandwich, flide/backbones/gemma4/fused.py:215,224-225):
    (h_out, x_out or None) = sandwich(combine_norm(y, dense, w1, w2, k, eps), h, w_post, eps, scale, w_next),
    with combine_norm's output rounded to bf16 in between as the reference stores it (moe.py:372-395,
    pointwise.py:214-245). bf16 activations and weights, H <= 4096, k <= 8."""
    dev = _hip.require_gpu(y, dense, w1, w2, h, w_post, scale, w_next)
    T, H = dense.shape
    for t in (dense, h, w1, w2, w_post) + ((w_next,) if w_next is not None else ()):
        if t.dtype != torch.bfloat16:
            raise TypeError("combine_norm_sandwich takes bf16 activations and norm weights")
    h_out = torch.empty_like(h)
    x_out = torch.empty_like(h) if w_next is not None else None
    if T:
        if dense.stride(-1) != 1:
            dense = dense.contiguous()
        if h.stride(-1) != 1:
            h = h.contiguous()
        y = y.contiguous()
        w1, w2, w_post = w1.contiguous(), w2.contiguous(), w_post.contiguous()
        wn = w_next.contiguous() if w_next is not None else None
        _hip.call("flide_moe_combine_norm_sandwich", y.data_ptr(), _hip.dtype_code(y.dtype), dense.data_ptr(),
                  dense.stride(0), w1.data_ptr(), w2.data_ptr(), h.data_ptr(), h.stride(0), w_post.data_ptr(),
                  _hip.ptr(scale), _hip.dtype_code(scale.dtype) if scale is not None else 0, _hip.ptr(wn),
                  h_out.data_ptr(), h_out.stride(0), _hip.ptr(x_out), x_out.stride(0) if x_out is not None else 0,
                  T, H, k, float(eps), _hip.stream(dev))
    return h_out, x_out


def combine_norm(y: torch.Tensor, dense: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, k: int,
                 eps: float) -> torch.Tensor:
    """Joins Gemma 4's dense-MLP output and its experts: out[t] = RMS(dense[t]) * w1 + RMS(s[t]) * w2 with
    s[t] = sum_j y[t*k + j] taken in slot order; float32 arithmetic, rounded once to dense's dtype
    (moe.py:386-395)."""
    dev = _hip.require_gpu(y, dense, w1, w2)
    T, H = dense.shape
    out = torch.empty_like(dense)
    if T:
        if dense.stride(-1) != 1:
            dense = dense.contiguous()
        y = y.contiguous()
        w1, w2 = w1.contiguous(), w2.contiguous()
        if w2.dtype != w1.dtype:
            w2 = w2.to(w1.dtype)
        _hip.call("flide_moe_combine_norm", y.data_ptr(), _hip.dtype_code(y.dtype), dense.data_ptr(), dense.stride(0),
                  w1.data_ptr(), w2.data_ptr(), _hip.dtype_code(w1.dtype), out.data_ptr(), out.stride(0),
                  _hip.dtype_code(out.dtype), T, H, k, float(eps), _hip.stream(dev))
    return out
