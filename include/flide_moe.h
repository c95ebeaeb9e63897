/*
 * flide_moe.h -- C ABI of the MI355X (gfx950) mixture-of-experts layer.
 *
 * Each entry point replaces one function of the reference's MoE hot path
 * (flide 0.1.18, flide/kernels/moe.py, fp8.py, pointwise.py) and is what that module's Python
 * wrappers would bind through ctypes. Conventions shared by every entry point:
 *   - plain device pointers, element strides (not bytes) for rows, sizes as int;
 *   - the last dimension of every matrix is contiguous (stride 1);
 *   - work is enqueued on `stream` and never synchronised; no device memory is read on the host,
 *     so every call can be captured into a HIP graph;
 *   - scratch memory comes from the caller (a `workspace` of the size the matching *_workspace call
 *     returns); nothing here allocates;
 *   - the return value is 0 on success or a FLIDE_MOE_ERR_* code (flide_moe_strerror names it).
 * Element type codes (the `*_dtype` arguments): FLIDE_F32, FLIDE_BF16, FLIDE_F16, FLIDE_E4M3.
 */
#ifndef FLIDE_MOE_H
#define FLIDE_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* flide_stream_t; /* a hipStream_t */

enum {
  FLIDE_F32 = 0,
  FLIDE_BF16 = 1,
  FLIDE_F16 = 2,
  FLIDE_E4M3 = 3, /* OCP float8 e4m3fn, max 448 */
};

enum {
  FLIDE_ACT_NONE = 0,
  FLIDE_ACT_GEGLU = 1, /* GELU-tanh(gate) * up, flide/kernels/pointwise.py:248-268 */
  FLIDE_ACT_SWIGLU = 2, /* silu(gate) * up, flide/kernels/pointwise.py:52-69 */
};

enum {
  FLIDE_MOE_OK = 0,
  FLIDE_MOE_ERR_ARG = 1,       /* a size, stride, pointer alignment or dtype the kernels do not take */
  FLIDE_MOE_ERR_WORKSPACE = 2, /* workspace smaller than the *_workspace query returned */
  FLIDE_MOE_ERR_TILE = 3,      /* a tile shape with no compiled kernel */
  FLIDE_MOE_ERR_SCRATCH = 4,   /* larger than flide_moe_experts_noalloc's static scratch */
  FLIDE_MOE_ERR_HIP_BASE = 1000 /* + hipError_t of a failed launch */
};

/* Human-readable name of a return code. */
const char* flide_moe_strerror(int rc);

/* Library version and the gfx target it was built for, e.g. "flide_moe 0.1 gfx950". */
const char* flide_moe_version(void);

/*
 * Router logits. Replaces moe.router + _router_kernel (flide/kernels/moe.py:128-169).
 * logits[t, e] = sum_h x[t, h] * wr[e, h] and, when wg != NULL, gate[t] = sum_h x[t, h] * wg[h], both
 * summed and stored in float32. x: [T, H] (x_dtype BF16 or F16, row stride sx); wr: [E, H] (same dtype,
 * row stride swr); wg: [H] or NULL; logits: [T, E] float32 (row stride sl); gate: [T] float32.
 * The K sum's order does not depend on T, so a token's logits are the same bits in any batch.
 */
int flide_moe_router(const void* x, long long sx, int T, int H, int x_dtype, const void* wr,
                     long long swr, int E, const void* wg, float* logits, long long sl, float* gate,
                     flide_stream_t stream);

/*
 * Router logits with the router's RMSNorm fused in. Replaces the Gemma 4 glue
 *   r = pointwise.rms_norm(h, router_norm); logits = moe.router(r, W_r);
 *   x2 = pointwise.rms_norm(h, pre_feedforward_layernorm_2.weight)
 * (flide/backbones/gemma4/fused.py:234-237; pointwise.py:21-49 without offset or residual) in one
 * launch. With inv = rsqrt(mean_h(h^2) + eps) per token: r = round((h * inv) * norm_w), logits = r @ wr^T
 * summed in float32, and, when x2 != NULL, x2 = round((h * inv) * norm2_w), rounded to h's type.
 * h: [T, H] (h_dtype BF16 or F16, row stride sh); norm_w: [H] float32; wr: [E, H] (h's type, row stride
 * swr); logits: [T, E] float32 (row stride sl); norm2_w: [H] (norm2_dtype F32, BF16 or F16) or NULL;
 * x2: [T, H] in h's type (row stride sx2) or NULL. H <= 8192; H, sh, swr and sx2 multiples of 8; h, wr,
 * norm_w, norm2_w and x2 16-byte aligned. A token's logits are the same bits whatever T (as
 * flide_moe_router's, which sums K in the same order).
 */
int flide_moe_router_norm(const void* h, long long sh, int T, int H, int h_dtype, const float* norm_w,
                          const void* wr, long long swr, int E, float eps, float* logits, long long sl,
                          const void* norm2_w, int norm2_dtype, void* x2, long long sx2,
                          flide_stream_t stream);

/*
 * Routing. Replaces moe.route + _route_kernel (flide/kernels/moe.py:172-204).
 * For each token: the k largest logits in descending order (ties to the lower expert id), weights
 * w = softmax(logits)[ids] / sum(softmax(logits)[ids]) in float32, times scale[ids] when scale != NULL.
 * logits: [T, E] float32 (row stride sl); scale: [E] (scale_dtype F32, BF16 or F16) or NULL;
 * w: [T, k] float32; ids: [T, k] int32 (both contiguous). Needs 1 <= k <= E <= 1024.
 */
int flide_moe_route(const float* logits, long long sl, int T, int E, int k, const void* scale,
                    int scale_dtype, float* w, int* ids, flide_stream_t stream);

/*
 * Workspace bytes flide_moe_align needs for n = T*k pairs over E experts.
 */
size_t flide_moe_align_workspace(int n, int E);

/*
 * Sort and pad. Replaces moe.align + _count_kernel + _place_kernel (flide/kernels/moe.py:207-253).
 * ids: [n] int32 expert ids (ids out of [0, E) are dropped). Outputs, with total = ceil((n + E*(bm-1))
 * / bm) * bm:
 *   rows [total]      per expert its pair indices in ascending order, then the sentinel n up to a
 *                     multiple of bm; entries past *used are left unset
 *   blocks [total/bm] the expert of each bm-row block below *used (the rest unset)
 *   used [1]          rows in use (sum of the padded counts)
 *   counts [E]        pairs per expert (may be NULL)
 */
int flide_moe_align(const int* ids, int n, int E, int bm, int* rows, int* blocks, int* used,
                    int* counts, void* workspace, size_t workspace_bytes, flide_stream_t stream);

/*
 * Grouped product in 16 bits. Replaces moe.grouped + _grouped_kernel (flide/kernels/moe.py:46-83,
 * 286-299), with the gate/up activation optionally fused into the epilogue.
 *   act == FLIDE_ACT_NONE:  out[p, n] = (a[row(p)] . w[e(p), n]) (* weights[p]),  n < N
 *   act != FLIDE_ACT_NONE:  out[p, n] = act(gu[p, n], gu[p, n + N/2]),            n < N/2
 *                           where gu = a[row(p)] . w[e(p)]^T rounded to a_dtype (gate rows first)
 * for every pair p = rows[i] < n_pairs of every bm-row block i / bm below *used, e(p) = blocks[i/bm],
 * row(p) = p / topk when by_token else p. a: [*, K] (a_dtype BF16 or F16, row stride sa); w: [E, N, K]
 * same dtype (strides sbe, sbn); out: [n_pairs, N or N/2] (out_dtype F32 or a_dtype, row stride sc);
 * weights: [n_pairs] float32 or NULL. nbm = total / bm is the static block count (grid bound).
 * bm must be the value align padded with; bn selects the column tile (0 = default).
 * K must be a multiple of 8 and rows 16-byte aligned. The last a row a pair names and the last row of
 * one expert's weights must each end within 4 GiB of their base (the kernels use 32-bit byte offsets);
 * larger operands return FLIDE_MOE_ERR_ARG.
 */
int flide_moe_grouped(const void* a, long long sa, int a_dtype, const void* w, long long sbe,
                      long long sbn, int N, int K, void* out, long long sc, int out_dtype,
                      const float* weights, const int* rows, const int* blocks, const int* used,
                      int n_pairs, int nbm, int topk, int by_token, int act, int bm, int bn,
                      flide_stream_t stream);

/*
 * Grouped product in float8. Replaces moe.grouped_fp8 + _grouped_fp8_kernel (flide/kernels/moe.py:
 * 86-125, 302-318) after its quantize_tokens call: a is already e4m3 with per-row scales a_scale.
 *   out[p, n] = (sum_k a[row(p), k] * w[e, n, k]) * a_scale[row(p)] * w_scale[e, n] (* weights[p])
 * with the same fused-activation option as flide_moe_grouped (the activation reads gu rounded to
 * out_dtype). a: [*, K] e4m3 (row stride sa); a_scale: [*] float32; w: [E, N, K] e4m3 (strides sbe,
 * sbn); w_scale: [E, N] float32 (row stride sse); out: out_dtype BF16, F16 or F32. K % 16 == 0.
 * The same 4 GiB operand limit as flide_moe_grouped.
 */
int flide_moe_grouped_fp8(const void* a, long long sa, const float* a_scale, const void* w,
                          long long sbe, long long sbn, const float* w_scale, long long sse, int N,
                          int K, void* out, long long sc, int out_dtype, const float* weights,
                          const int* rows, const int* blocks, const int* used, int n_pairs, int nbm,
                          int topk, int by_token, int act, int bm, int bn, flide_stream_t stream);

/*
 * Per-row float8 quantization. Replaces fp8.quantize_tokens + _quantize_tokens (flide/kernels/
 * fp8.py:29-53) and, row by row, fp8.quantize_rows (fp8.py:22-26) under moe.quantize_experts
 * (moe.py:321-333): s[r] = max(amax_k |x[r, k]|, 1e-12) * (1/448); q[r, k] = e4m3fn(clamp(x[r, k] /
 * s[r], +-448)), round to nearest even. x: [M, K] (x_dtype F32, BF16 or F16, row stride sx);
 * q: [M, K] e4m3 (row stride sq); s: [M] float32.
 */
int flide_moe_quantize_rows(const void* x, long long sx, int M, int K, int x_dtype, void* q,
                            long long sq, float* s, flide_stream_t stream);

/*
 * Gemma 4 combine. Replaces moe.combine_norm + _combine_norm_kernel (flide/kernels/moe.py:372-395):
 * out[t] = RMS(dense[t]) * w1 + RMS(sum_{j<k} y[t*k + j]) * w2, RMS(v) = v * rsqrt(mean(v^2) + eps),
 * float32 math, the k rows summed in slot order, rounded once to out_dtype. y: [T*k, H] (y_dtype F32,
 * BF16 or F16, contiguous rows of H); dense: [T, H] (dtype = out_dtype, row stride sd); w1, w2: [H]
 * (w_dtype); out: [T, H] (row stride so).
 */
int flide_moe_combine_norm(const void* y, int y_dtype, const void* dense, long long sd,
                           const void* w1, const void* w2, int w_dtype, void* out, long long so,
                           int out_dtype, int T, int H, int k, float eps, flide_stream_t stream);

/*
 * Gemma 4 combine fused with the step after it. Replaces
 *   d = moe.combine_norm(y, dense, w1, w2, k, eps)                              (moe.py:372-395)
 *   h_out, x_out = pointwise.sandwich(d, h, w_post, eps, scale=s, w2=w_next)   (pointwise.py:214-245)
 * as called at flide/backbones/gemma4/fused.py:215,224-225, in one launch: d is rounded to bf16 as the
 * reference stores it but never written; h_out = round((h + RMS(d) * w_post) * s) (s = *scale, or no
 * multiply when scale is NULL); with w_next, x_out = round(RMS(h_out) * w_next). float32 math.
 * y: [T*k, H] F32 or BF16 (contiguous, 16-byte aligned); dense, h, h_out, x_out: [T, H] bf16 (row
 * strides sd, sh, sho, sxo, multiples of 4); w1, w2, w_post, w_next: [H] bf16; scale: one element of
 * scale_dtype or NULL; w_next and x_out both NULL to skip x_out. H % 4 == 0, H <= 4096, k <= 8; bf16
 * arrays 8-byte aligned.
 */
int flide_moe_combine_norm_sandwich(const void* y, int y_dtype, const void* dense, long long sd,
                                    const void* w1, const void* w2, const void* h, long long sh,
                                    const void* w_post, const void* scale, int scale_dtype,
                                    const void* w_next, void* h_out, long long sho, void* x_out,
                                    long long sxo, int T, int H, int k, float eps, flide_stream_t stream);

/*
 * Qwen3.5 combine. Replaces moe.combine + _combine_kernel (flide/kernels/moe.py:256-277):
 * out[t] = sum_{j<k} y[t*k + j] + shared[t] * sigmoid(gate[t]), float32 math, rounded once.
 * y: [T*k, H] (y_dtype); shared: [T, H] contiguous (out_dtype); gate: [T] float32; out: [T, H].
 */
int flide_moe_combine(const void* y, int y_dtype, const void* shared, const float* gate, void* out,
                      int out_dtype, int T, int H, int k, flide_stream_t stream);

/*
 * RMSNorm on the path's inputs. Replaces pointwise.rms_norm without residual (flide/kernels/
 * pointwise.py:21-49): y[t] = x[t] * rsqrt(mean(x[t]^2) + eps) * (offset ? 1 + w : w), float32 math,
 * rounded once to y_dtype. x: [T, N] (x_dtype, row stride sx); w: [N] (w_dtype); y: [T, N] (sy).
 */
int flide_moe_rms_norm(const void* x, long long sx, int x_dtype, const void* w, int w_dtype,
                       void* y, long long sy, int y_dtype, int T, int N, float eps, int offset,
                       flide_stream_t stream);

/*
 * Gated activations. Replace pointwise.geglu (flide/kernels/pointwise.py:248-268) and
 * pointwise.swiglu (pointwise.py:52-69): out[t, c] = act(a[t, c], b[t, c]) for c < n, float32 math,
 * rounded once. a, b: [T, n] row-strided views (dtype, strides sa, sb); out: [T, n] (stride so).
 */
int flide_moe_gated_act(const void* a, long long sa, const void* b, long long sb, void* out,
                        long long so, int dtype, int T, int n, int act, flide_stream_t stream);

/*
 * Workspace bytes flide_moe_experts needs.
 */
size_t flide_moe_experts_workspace(int T, int k, int E, int H, int I, int bm, int fp8);

/*
 * The routed experts in one call. Replaces moe.experts (flide/kernels/moe.py:336-353) for the fused
 * activations: align, then the gate/up grouped product with the activation in its epilogue, then the
 * down grouped product times the routing weight.
 * x: [T, H] (x_dtype BF16 or F16, row stride sx); top: [T, k] float32; ids: [T, k] int32 (contiguous).
 * 16-bit experts (w_scale_gu == NULL): w_gu [E, 2I, H], w_d [E, H, I] in x_dtype, contiguous;
 *   y: [T*k, H] float32.
 * float8 experts: w_gu, w_d e4m3 with w_scale_gu [E, 2I], w_scale_d [E, H] float32; activations are
 *   quantised per token (gate/up) and per pair (down); y: [T*k, H] in x_dtype.
 * act: FLIDE_ACT_GEGLU or FLIDE_ACT_SWIGLU. bm, bn: the tile (bm as align pads; bn 0 = default).
 */
int flide_moe_experts(const void* x, long long sx, int x_dtype, int T, int H, const float* top,
                      const int* ids, int k, const void* w_gu, const void* w_d, const float* w_scale_gu,
                      const float* w_scale_d, int E, int I, void* y, int act, int bm, int bn,
                      void* workspace, size_t workspace_bytes, flide_stream_t stream);

/*
 * Bytes of device memory flide_moe_experts_noalloc keeps per GPU (a static array, resident from the
 * library's load until the process ends).
 */
#define FLIDE_MOE_NOALLOC_SCRATCH_BYTES (16u << 20)

/*
 * flide_moe_experts without a workspace argument: its scratch is a static device array of
 * FLIDE_MOE_NOALLOC_SCRATCH_BYTES per GPU, so the call allocates nothing at all (no hipMalloc, no
 * allocating library call). No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid allocation). Same arguments,
 * kernels and output bits as flide_moe_experts. A problem whose flide_moe_experts_workspace exceeds the
 * scratch returns FLIDE_MOE_ERR_SCRATCH (at the Gemma 4 26B-A4B shape: about 1480 tokens with 16-bit
 * experts, about 840 with float8 ones). Every call on one GPU uses that GPU's one array: calls that
 * overlap on a GPU (on different streams, or from different threads) race and must be ordered by the
 * caller. The array's contents carry over between calls; nothing in it needs to start zeroed.
 */
int flide_moe_experts_noalloc(const void* x, long long sx, int x_dtype, int T, int H, const float* top,
                              const int* ids, int k, const void* w_gu, const void* w_d,
                              const float* w_scale_gu, const float* w_scale_d, int E, int I, void* y,
                              int act, int bm, int bn, flide_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FLIDE_MOE_H */
