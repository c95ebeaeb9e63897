"""numpy restatement of Flide's MoE hot path -- TEST INFRASTRUCTURE (the parity oracle), NOT PRODUCT CODE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only as
the checker. Every function cites the reference line it restates (paths are relative to the reference
checkout `flide` 0.1.18).

Arithmetic: products and sums in float64 (the reference sums in float32 inside tl.dot, in an order the
contract does not fix), rounded to float32 where the reference keeps float32, and to bfloat16 (round to
nearest even) where the reference stores x.dtype. FP8 is OCP e4m3fn (max 448), rounded to nearest even.

Pins (tests/test_oracle.py): route/align against brute force and torch.sort/bincount/argsort; experts and
the layer against transformers' eager Gemma4TextRouter/Gemma4TextExperts/Gemma4RMSNorm (the reference's
CPU torch path); GeGLU/SwiGLU against torch.nn.functional; the e4m3fn rounding against torch's
float8_e4m3fn cast; quantize_* against their closed forms. Routing selection is defined on the float32
logits (ties to the lower expert id), which is the reference's selection on softmax probabilities
(flide/kernels/moe.py:182-187) wherever exp rounding does not merge two distinct logits into one
probability.
"""
from __future__ import annotations

import numpy as np

FP8_MAX = 448.0
_F32 = np.float32


# ----------------------------------------------------------------------------------------------------
# number formats
# ----------------------------------------------------------------------------------------------------
def bf16_round(x) -> np.ndarray:
    """float32 -> nearest bfloat16 (ties to even), returned as float32; NaN stays NaN."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, out)


def e4m3fn_round(x) -> np.ndarray:
    """float32 (|x| <= 448) -> nearest OCP e4m3fn value (ties to even), as float32. Normal numbers have a
    quantum of 2^(e-3); below 2^-6 the subnormal quantum is 2^-9."""
    x = np.asarray(x, dtype=np.float64)
    a = np.abs(x)
    _, ex = np.frexp(a)                      # a = m * 2^ex, m in [0.5, 1)
    e = np.maximum(ex - 1, -6)               # unbiased exponent, floored at the subnormal range
    q = np.ldexp(np.rint(np.ldexp(a, -(e - 3))), e - 3)
    q = np.where(a == 0, 0.0, q)
    return np.copysign(q, x).astype(np.float32)


def e4m3fn_encode(v) -> np.ndarray:
    """exact e4m3fn values -> their byte codes (S EEEE MMM, bias 7)."""
    v = np.asarray(v, dtype=np.float64)
    a = np.abs(v)
    sign = np.signbit(v).astype(np.uint8) << 7
    _, ex = np.frexp(np.where(a == 0, 1.0, a))
    e = ex - 1
    sub = a < 2.0 ** -6
    mant_sub = np.rint(a / 2.0 ** -9).astype(np.int64)
    mant_norm = np.rint((a / np.ldexp(1.0, e) - 1.0) * 8).astype(np.int64)
    exp_field = np.where(sub, 0, e + 7)
    mant = np.where(sub, mant_sub, mant_norm)
    code = (exp_field.astype(np.int64) << 3) | mant
    return (sign | code.astype(np.uint8)).astype(np.uint8)


def e4m3fn_decode(code) -> np.ndarray:
    """e4m3fn byte codes -> float32 values (0x7F/0xFF are NaN)."""
    c = np.asarray(code, dtype=np.uint8).astype(np.int64)
    s = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 7
    v = np.where(e == 0, m * 2.0 ** -9, (1 + m / 8.0) * np.ldexp(1.0, e - 7))
    v = np.where((c & 0x7F) == 0x7F, np.nan, v)
    return (s * v).astype(np.float32)


def f16_round(x) -> np.ndarray:
    """Round to IEEE binary16 (numpy's cast: round to nearest even, overflow to inf) and back to float32."""
    with np.errstate(over="ignore"):   # overflow to inf is the defined result
        return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def _round(x, dtype: str) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    if dtype == "bf16":
        return bf16_round(x)
    return f16_round(x) if dtype == "f16" else x


# ----------------------------------------------------------------------------------------------------
# pointwise pieces on the path
# ----------------------------------------------------------------------------------------------------
def rms_norm(x, w, eps: float, offset: bool = False, dtype: str = "bf16") -> np.ndarray:
    """flide/kernels/pointwise.py:21-49: y = x * rsqrt(mean(x^2) + eps) * (1 + w if offset else w), in
    float32 arithmetic, rounded once to `dtype`."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    inv = 1.0 / np.sqrt((x * x).sum(-1, keepdims=True) / x.shape[-1] + eps)
    return _round(x * inv * ((1.0 + w) if offset else w), dtype)


def gelu_tanh(a) -> np.ndarray:
    """0.5 a (1 + tanh(sqrt(2/pi) (a + 0.044715 a^3))) in float64 (flide/kernels/pointwise.py:254-256)."""
    a = np.asarray(a, np.float64)
    return 0.5 * a * (1.0 + np.tanh(0.7978845608028654 * (a + 0.044715 * a * a * a)))


def geglu(a, b, dtype: str = "bf16") -> np.ndarray:
    """flide/kernels/pointwise.py:248-268: GELU-tanh(a) * b, float32 math, rounded once."""
    return _round(gelu_tanh(a) * np.asarray(b, np.float64), dtype)


def swiglu(gu, n: int, dtype: str = "bf16") -> np.ndarray:
    """flide/kernels/pointwise.py:52-69: silu(gu[:, :n]) * gu[:, n:], rounded once."""
    a = np.asarray(gu[:, :n], np.float64)
    b = np.asarray(gu[:, n:2 * n], np.float64)
    return _round(a / (1.0 + np.exp(-a)) * b, dtype)


# ----------------------------------------------------------------------------------------------------
# router, route, align
# ----------------------------------------------------------------------------------------------------
def router(x, wr, wg=None):
    """flide/kernels/moe.py:128-169: float32 logits [T, E] = x . wr^T (and the shared-expert gate logit
    [T, 1] = x . wg when given), summed without rounding to 16 bits."""
    x = np.asarray(x, np.float64)
    logits = (x @ np.asarray(wr, np.float64).T).astype(np.float32)
    gate = None if wg is None else (x @ np.asarray(wg, np.float64).reshape(-1, 1)).astype(np.float32)
    return logits, gate


def topk_ids(logits, k: int) -> np.ndarray:
    """The k largest logits per row in descending order, the lower expert id first on equal values
    (flide/kernels/moe.py:182-187). A stable sort of -logits keeps lower ids first among equals."""
    logits = np.asarray(logits, np.float32)
    order = np.argsort(-logits, axis=-1, kind="stable")
    return order[:, :k].astype(np.int32)


def route(logits, k: int, scale=None):
    """flide/kernels/moe.py:172-204: (w [T, k] float32, ids [T, k] int32). Softmax over all E in float32,
    the top k, renormalised to sum to one, times scale[id] when given (Gemma 4 per_expert_scale)."""
    logits = np.asarray(logits, np.float32)
    ids = topk_ids(logits, k)
    l64 = logits.astype(np.float64)
    p = np.exp(l64 - l64.max(-1, keepdims=True))
    p = p / p.sum(-1, keepdims=True)
    top = np.take_along_axis(p, ids.astype(np.int64), -1)
    w = top / top.sum(-1, keepdims=True)
    if scale is not None:
        w = w * np.asarray(scale, np.float64)[ids]
    return w.astype(np.float32), ids


def align(ids, experts: int, bm: int = 64):
    """flide/kernels/moe.py:207-253 as a closed form. Returns a dict with
      rows    int32 [total]: per expert its pair indices (t*k + j) ascending, then the sentinel n = T*k up
              to a multiple of bm; entries past `used` are -1 here (the reference leaves them unset)
      blocks  int32 [total // bm]: the expert of each bm-row block (-1 past `used`, unset in the reference)
      used    int32 [1]: the padded row count
      counts  int32 [E], offsets int32 [E] (exclusive prefix of counts), perm int32 [n] (stable argsort)
    where total = ceil((n + E (bm - 1)) / bm) * bm is the static upper bound (moe.py:249)."""
    ids = np.asarray(ids, np.int64)
    n = ids.size
    flat = ids.reshape(-1)
    counts = np.bincount(flat, minlength=experts)[:experts]
    padded = (counts + bm - 1) // bm * bm
    ends = np.cumsum(padded)
    starts = ends - padded
    total = -(-(n + experts * (bm - 1)) // bm) * bm
    rows = np.full(total, -1, np.int64)
    blocks = np.full(total // bm, -1, np.int64)
    perm = np.argsort(flat, kind="stable")
    off = np.concatenate([[0], np.cumsum(counts)[:-1]])
    for e in range(experts):
        s, c, p = starts[e], counts[e], padded[e]
        rows[s:s + c] = perm[off[e]:off[e] + c]
        rows[s + c:s + p] = n
        blocks[s // bm:(s + p) // bm] = e
    used = int(ends[-1]) if experts else 0
    return {"rows": rows.astype(np.int32), "blocks": blocks.astype(np.int32),
            "used": np.array([used], np.int32), "counts": counts.astype(np.int32),
            "offsets": off.astype(np.int32), "perm": perm.astype(np.int32), "total": total}


# ----------------------------------------------------------------------------------------------------
# grouped products and the experts orchestration
# ----------------------------------------------------------------------------------------------------
def grouped(a, w, rows, blocks, used, n_pairs: int, topk: int, by_token: bool, weights=None,
            bm: int = 64, out_dtype: str = "fp32", out=None):
    """flide/kernels/moe.py:46-83,286-299: out[pair] = a[pair // topk if by_token else pair] @ w[e]^T,
    times weights[pair] when given, for every valid pair of every block below `used`. Rows of `out` not
    named by a valid pair are left as they were (NaN in a fresh output)."""
    a = np.asarray(a, np.float64)
    N = w.shape[1]
    if out is None:
        out = np.full((n_pairs, N), np.nan, np.float32)
    used = int(np.asarray(used).reshape(-1)[0])
    for b in range(used // bm):
        e = int(blocks[b])
        pairs = np.asarray(rows[b * bm:(b + 1) * bm], np.int64)
        pairs = pairs[pairs < n_pairs]
        if pairs.size == 0:
            continue
        src = pairs // topk if by_token else pairs
        acc = a[src] @ np.asarray(w[e], np.float64).T
        if weights is not None:
            acc = acc * np.asarray(weights, np.float64)[pairs][:, None]
        out[pairs] = _round(acc, out_dtype)
    return out


def experts(x, w_gu, w_d, top, ids, inter: int, act: str = "geglu", dtype: str = "bf16", pairs=None):
    """flide/kernels/moe.py:336-353 for 16-bit (or float32) experts: [T*k, H] float32 rows
       gu[p] = round_D(x[p // k] @ w_gu[e_p]^T)      (w_gu rows 0..I-1 gate, I..2I-1 up)
       a[p]  = round_D(act(gu[p, :I], gu[p, I:]))
       y[p]  = (a[p] @ w_d[e_p]^T) * top[p]           (float32, rounded once at the layer's sum)
    `pairs` restricts the computation to a subset of pair indices (other rows are NaN)."""
    x = np.asarray(x, np.float32)
    T, H = x.shape
    k = ids.shape[1]
    flat = np.asarray(ids, np.int64).reshape(-1)
    wts = np.asarray(top, np.float64).reshape(-1)
    y = np.full((T * k, w_d.shape[1]), np.nan, np.float32)
    sel = np.arange(T * k) if pairs is None else np.asarray(pairs, np.int64)
    for e in np.unique(flat[sel]):
        p = sel[flat[sel] == e]
        gu = _round(x[p // k].astype(np.float64) @ np.asarray(w_gu[e], np.float64).T, dtype)
        if act == "geglu":
            a = geglu(gu[:, :inter], gu[:, inter:2 * inter], dtype)
        elif act == "swiglu":
            a = swiglu(gu, inter, dtype)
        else:
            raise ValueError(act)
        y[p] = (a.astype(np.float64) @ np.asarray(w_d[e], np.float64).T * wts[p][:, None]).astype(np.float32)
    return y


# ----------------------------------------------------------------------------------------------------
# FP8
# ----------------------------------------------------------------------------------------------------
def quantize_rows(w):
    """flide/kernels/fp8.py:22-26: scale = max(amax_row, 1e-12) * (1/448) in float32; q = e4m3fn(clamp(w /
    scale, +-448)). Returns (q values as float32 [N, K], scale float32 [N, 1])."""
    w = np.asarray(w, np.float32)
    amax = np.abs(w).max(axis=1, keepdims=True) if w.shape[1] else np.zeros((w.shape[0], 1), np.float32)
    scale = np.maximum(amax, _F32(1e-12)) * _F32(1.0 / FP8_MAX)
    q = np.clip(w / scale, -FP8_MAX, FP8_MAX).astype(np.float32)
    return e4m3fn_round(q), scale.astype(np.float32)


def quantize_tokens(x):
    """flide/kernels/fp8.py:29-53: per row s = max(amax, 1e-12) * (1/448); q = e4m3fn(clamp(x / s, +-448))
    with a correctly rounded division. Returns (q float32 values [M, K], s float32 [M, 1])."""
    return quantize_rows(x)


def quantize_experts(w):
    """flide/kernels/moe.py:321-333: per expert quantize_rows; scales [E, N]."""
    w = np.asarray(w, np.float32)
    qs, ss = zip(*(quantize_rows(w[e]) for e in range(w.shape[0]))) if w.shape[0] else ((), ())
    q = np.stack(qs) if qs else np.zeros(w.shape, np.float32)
    s = np.stack([s[:, 0] for s in ss]) if ss else np.zeros(w.shape[:2], np.float32)
    return q, s


def experts_fp8(x, q_gu, s_gu, q_d, s_d, top, ids, inter: int, act: str = "geglu", pairs=None):
    """flide/kernels/moe.py:86-125,302-318,345-349 with float8 experts: activations quantised per token
    (gate/up) and per pair (down); acc = sum_k q_a q_w in float64 (the reference: float32), then
    * s_a[row] * s_w[e, col] (* top[pair]); both products stored in bfloat16 (x.dtype)."""
    x = np.asarray(x, np.float32)
    T, H = x.shape
    k = ids.shape[1]
    flat = np.asarray(ids, np.int64).reshape(-1)
    wts = np.asarray(top, np.float64).reshape(-1)
    qx, sx = quantize_tokens(x)
    y = np.full((T * k, q_d.shape[1]), np.nan, np.float32)
    sel = np.arange(T * k) if pairs is None else np.asarray(pairs, np.int64)
    for e in np.unique(flat[sel]):
        p = sel[flat[sel] == e]
        t = p // k
        acc = qx[t].astype(np.float64) @ np.asarray(q_gu[e], np.float64).T
        gu = bf16_round(acc * sx[t].astype(np.float64) * np.asarray(s_gu[e], np.float64)[None, :])
        if act == "geglu":
            a = geglu(gu[:, :inter], gu[:, inter:2 * inter], "bf16")
        else:
            a = swiglu(gu, inter, "bf16")
        qa, sa = quantize_tokens(a)
        acc = qa.astype(np.float64) @ np.asarray(q_d[e], np.float64).T
        y[p] = bf16_round(acc * sa.astype(np.float64) * np.asarray(s_d[e], np.float64)[None, :] * wts[p][:, None])
    return y


# ----------------------------------------------------------------------------------------------------
# combine
# ----------------------------------------------------------------------------------------------------
def combine_norm(y, dense, w1, w2, k: int, eps: float, dtype: str = "bf16") -> np.ndarray:
    """flide/kernels/moe.py:372-395: RMS(dense[t]) * w1 + RMS(sum_j y[t*k + j]) * w2, float32 math with the
    expert rows summed in slot order, rounded once to dense's dtype."""
    d = np.asarray(dense, np.float64)
    T, H = d.shape
    s = np.asarray(y, np.float64).reshape(T, k, H).sum(1)
    a = d / np.sqrt((d * d).sum(-1, keepdims=True) / H + eps) * np.asarray(w1, np.float64)
    b = s / np.sqrt((s * s).sum(-1, keepdims=True) / H + eps) * np.asarray(w2, np.float64)
    return _round(a + b, dtype)


def sandwich(d, h, w1, eps: float, scale=None, w2=None, dtype: str = "bf16"):
    """flide/kernels/pointwise.py:213-245 (Gemma 4's post-norm step): h_out = (h + RMS(d) * w1) * scale,
    rounded once to `dtype`; with w2, x = RMS(h_out) * w2 of the rounded h_out, rounded once. Returns
    (h_out, x or None)."""
    d = np.asarray(d, np.float64)
    N = d.shape[-1]
    r = np.asarray(h, np.float64) + d / np.sqrt((d * d).sum(-1, keepdims=True) / N + eps) * np.asarray(w1, np.float64)
    if scale is not None:
        r = r * float(np.asarray(scale, np.float64).reshape(-1)[0])
    hb = _round(r, dtype)
    if w2 is None:
        return hb, None
    hf = hb.astype(np.float64)
    return hb, _round(hf / np.sqrt((hf * hf).sum(-1, keepdims=True) / N + eps) * np.asarray(w2, np.float64), dtype)


def combine(y, shared, gate, k: int, dtype: str = "bf16") -> np.ndarray:
    """flide/kernels/moe.py:256-277: sum_j y[t*k + j] + shared[t] * sigmoid(gate[t]), rounded once."""
    sh = np.asarray(shared, np.float64)
    T, H = sh.shape
    s = np.asarray(y, np.float64).reshape(T, k, H).sum(1)
    g = np.asarray(gate, np.float64).reshape(T, 1)
    return _round(s + sh / (1.0 + np.exp(-g)), dtype)


def combine_sum(y, k: int, dtype: str = "bf16") -> np.ndarray:
    """The weighted combine alone: sum_j y[t*k + j] in slot order, rounded once."""
    y = np.asarray(y, np.float64)
    return _round(y.reshape(-1, k, y.shape[-1]).sum(1), dtype)


# ----------------------------------------------------------------------------------------------------
# whole layers
# ----------------------------------------------------------------------------------------------------
def gemma_moe(h, dense, wd: dict, eps: float, dtype: str = "bf16", tokens=None, parts: dict | None = None):
    """flide/backbones/gemma4/fused.py:231-240 (FusedDecoder._moe): rms_norm -> router -> route(scale)
    -> rms_norm -> experts(GeGLU) -> combine_norm. `tokens` (ascending indices) restricts the expert
    products and the combine to those tokens' rows (routing still runs over the whole batch) and the
    result to those rows. `parts`, when given, receives the intermediate logits, top, ids and x2."""
    r = rms_norm(h, wd["router_norm"], eps, dtype=dtype)
    logits, _ = router(r, wd["router"])
    k = wd["topk"]
    top, ids = route(logits, k, wd["expert_scale"])
    x2 = rms_norm(h, wd["pre_norm_2"], eps, dtype=dtype)
    if parts is not None:
        parts.update(logits=logits, top=top, ids=ids, x2=x2)
    tok = np.arange(h.shape[0]) if tokens is None else np.asarray(tokens, np.int64)
    pairs = (tok[:, None] * k + np.arange(k)[None, :]).reshape(-1)
    y = experts(x2, wd["experts"], wd["experts_down"], top, ids, wd["inter"], "geglu", dtype, pairs=pairs)
    return combine_norm(y[pairs], np.asarray(dense)[tok], wd["post_norm_1"], wd["post_norm_2"], k, eps, dtype)


def qwen_moe(x, wd: dict, dtype: str = "bf16") -> np.ndarray:
    """flide/kernels/moe.py:356-369: router (+ shared gate) -> route -> experts(SwiGLU) -> shared expert
    (swiglu(x @ shared_gate_up^T) @ shared_down^T) -> combine."""
    k = wd["topk"]
    logits, gate = router(x, wd["router"], wd["shared_gate"])
    top, ids = route(logits, k)
    y = experts(x, wd["experts"], wd["experts_down"], top, ids, wd["inter"], "swiglu", dtype)
    x64 = np.asarray(x, np.float64)
    sgu = _round(x64 @ np.asarray(wd["shared_gate_up"], np.float64).T, dtype)
    sa = swiglu(sgu, wd["shared_inter"], dtype)
    shared = _round(sa.astype(np.float64) @ np.asarray(wd["shared_down"], np.float64).T, dtype)
    return combine(y, shared, gate, k, dtype)
