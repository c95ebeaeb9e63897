// Router logits and routing: flide/kernels/moe.py:128-204 re-designed for CDNA4.
//
// router: a plain [T, H] x [E, H]^T product with float32 output, its K split over the 8 waves of a
//   workgroup (below); fragments are read straight from global memory (the router weight, 0.7 MB at the
//   Gemma shape, stays in L2).
// route: one wave64 per token. The token's E logits sit in registers (E/64 per lane); k rounds of a
//   wave argmax (larger logit, then lower expert id) pick the experts, so the selection is exact and
//   independent of how exp rounds; the softmax weights follow the reference's formula.
#include <float.h>
#include <limits.h>

#include "routing.hpp"

namespace {

// Router product split over K inside the workgroup. The 8 waves of a workgroup share one tile of 16*MB
// tokens x 16*NB experts; wave w sums the 32-wide K steps [w*S/8, (w+1)*S/8) of the S = ceil(H/32)
// steps with v_mfma_f32_16x16x32 (U steps' loads in flight at once), and the 8 partial tiles are added
// in wave order through LDS. The K split does not depend on the tile, so a token's logits are the same
// bits whatever T and whichever tile the host picks (batch invariant), and at 64 tokens the product
// runs on 256 waves. The cost at every size is the load instructions per CU (16 rows x 64 bytes each),
// not the MFMAs, so the loops keep loads unconditional and let the compiler issue a group at once.
constexpr int RS_WAVES = 8;
constexpr int RS_HOLD = 12;   // K steps per wave held in registers by the norm-fused form
constexpr int RN_MAX_H = 8192;   // the norm-fused form stages 2 x H float32 weights in LDS

template <typename T, int MB, int NB, int U, bool NORM, int N2DT = FLIDE_F32>
__global__ __launch_bounds__(RS_WAVES * 64) void router_split_kernel(
    const u16* __restrict__ x, long long sx, int T_, int H, const u16* __restrict__ wr, long long swr,
    int E, float* __restrict__ logits, long long sl, const float* __restrict__ norm_w, float eps,
    const void* norm2_w, u16* __restrict__ x2, long long sx2) {
  constexpr int TM = 16 * MB, TE = 16 * NB, RP = TE + 4;   // +4: the 4 row groups land on distinct banks
  __shared__ float red[RS_WAVES][16][RP];
  __shared__ float s_ss[RS_WAVES][TM];
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63, r = l & 15, g = l >> 4;
  const int S = (H + 31) >> 5, s0 = wave * S / RS_WAVES, s1 = (wave + 1) * S / RS_WAVES;
  // Workgroup b runs on XCD b % 8. XCD j takes the j-th contiguous run of the token-major list of
  // (token tile, expert tile) items, so the workgroups sharing a token tile share one XCD's L2 and x is
  // read from HBM once, not once per expert tile.
  const int ne = (E + TE - 1) / TE, items = gridDim.x, q = items / 8, rem = items % 8;
  const int xj = blockIdx.x % 8, xi = blockIdx.x / 8;
  const int item = xj * q + (xj < rem ? xj : rem) + xi;
  const int et = item % ne;
  const int t0 = (item / ne) * TM, e0 = et * TE;
  // rows past T or E read row 0 (their results are never stored), so every load below is in bounds
  const u16* xp[MB];
  bool tv[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int t = t0 + mb * 16 + r;
    tv[mb] = t < T_;
    xp[mb] = x + (long long)(tv[mb] ? t : 0) * sx;
  }
  const u16* wp[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int e = e0 + nb * 16 + r;
    wp[nb] = wr + (long long)(e < E ? e : 0) * swr;
  }
  // This lane's 8 K-values of step s are s*32 + g*8 .. +8 (H % 8 == 0: all in or all out). Steps past the
  // wave's range re-read its last step and lanes past H read H - 8; both are zeroed before use, so every
  // load is in bounds and a wave issues the same loads whatever its range (exact load-counter waits).
  auto kof = [&](int st) {
    const int sc = st < s1 ? st : s1 - 1;   // a wave with no steps (H < 256) reads step 0, uses nothing
    const int k = (sc > 0 ? sc : 0) * 32 + g * 8;
    return k < H ? k : H - 8;
  };
  // steps out of range and lanes past H take zero fragments of both operands (0 * 0: no 0 * inf)
  auto kin = [&](int st) { return st < s1 && st * 32 + g * 8 < H; };
  f32x4_t acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto mma = [&](const u32x4_t (&a)[MB], const u32x4_t (&b)[NB]) {   // acc += a b^T
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = Mfma16<T>::mma(a[mb], b[nb], acc[mb][nb]);
  };

  if constexpr (!NORM) {
    for (int st = s0; st < s1; st += U) {
      u32x4_t a[U][MB], b[U][NB];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int k = kof(st + u);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) a[u][mb] = *(const u32x4_t*)(xp[mb] + k);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) b[u][nb] = *(const u32x4_t*)(wp[nb] + k);
      }
      // no branch on the step: a branch would let the compiler sink each step's loads next to its MFMAs
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool in = kin(st + u);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) a[u][mb] = in ? a[u][mb] : u32x4_t{0, 0, 0, 0};
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) b[u][nb] = in ? b[u][nb] : u32x4_t{0, 0, 0, 0};
        mma(a[u], b[u]);
      }
    }
  } else {
    // Gemma's router input fused in front (flide/backbones/gemma4/fused.py:234-237): both of the layer's
    // norms of h share one statistic, inv = rsqrt(mean(h^2) + eps), each wave summing the squares of its
    // own K range. The wave's first RS_HOLD steps of h stay in registers from the statistic to the
    // MFMAs (Gemma's and Qwen's H need at most 11); steps beyond are read again. Both norm weights are
    // staged once per workgroup in LDS as float32 (nw: [H], n2: [H]).
    extern __shared__ float s_w[];
    float* s_nw = s_w;
    float* s_n2 = s_w + H;
    for (int i = threadIdx.x * 4; i < H; i += RS_WAVES * 64 * 4) {
      *(float4*)(s_nw + i) = *(const float4*)(norm_w + i);
      if (x2) {
        if constexpr (N2DT == FLIDE_F32) {
          *(float4*)(s_n2 + i) = *(const float4*)((const float*)norm2_w + i);
        } else {
          const uint2 v = *(const uint2*)((const u16*)norm2_w + i);
          const u16 hv[4] = {(u16)(v.x & 0xffff), (u16)(v.x >> 16), (u16)(v.y & 0xffff), (u16)(v.y >> 16)};
#pragma unroll
          for (int j = 0; j < 4; ++j) s_n2[i + j] = N2DT == FLIDE_BF16 ? bf16_to_f32(hv[j]) : f16_to_f32(hv[j]);
        }
      }
    }
    u32x4_t hr[RS_HOLD][MB];
#pragma unroll
    for (int j = 0; j < RS_HOLD; ++j)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) hr[j][mb] = *(const u32x4_t*)(xp[mb] + kof(s0 + j));
    auto ldb = [&](u32x4_t (&b)[U][NB], int st) {
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) b[u][nb] = *(const u32x4_t*)(wp[nb] + kof(st + u));
    };
    u32x4_t b0[U][NB];
    ldb(b0, s0);   // the first router-weight loads do not wait for the statistic
    float ss[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) ss[mb] = 0.f;
    auto sq = [&](const u32x4_t (&v)[MB], bool in) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float f = in ? Mfma16<T>::to_f32((u16)(v[mb][j >> 1] >> (16 * (j & 1)))) : 0.f;
          ss[mb] += f * f;
        }
    };
#pragma unroll
    for (int j = 0; j < RS_HOLD; ++j) sq(hr[j], kin(s0 + j));
    for (int st = s0 + RS_HOLD; st < s1; ++st) {
      u32x4_t v[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) v[mb] = *(const u32x4_t*)(xp[mb] + kof(st));
      sq(v, kin(st));
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      ss[mb] += __shfl_xor(ss[mb], 16);
      ss[mb] += __shfl_xor(ss[mb], 32);
      if (g == 0) s_ss[wave][mb * 16 + r] = ss[mb];
    }
    __syncthreads();   // also orders the weight staging above
    float inv[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < RS_WAVES; ++w) t += s_ss[w][mb * 16 + r];
      inv[mb] = rsqrtf(t / H + eps);
    }
    // r = round((h * inv) * norm_w) into the MFMAs (no round trip of r through memory); the workgroups of
    // the first expert tile also write the experts' input x2 = round((h * inv) * norm2_w)
    // (pointwise.py:21-36)
    const bool wx2 = x2 && et == 0;
    auto step = [&](u32x4_t (&a)[MB], u32x4_t (&b)[NB], int st) {
      const bool in = kin(st);
      const int k = kof(st);
      const float4 w0 = *(const float4*)(s_nw + k), w1 = *(const float4*)(s_nw + k + 4);
      const float4 v0 = *(const float4*)(s_n2 + k), v1 = *(const float4*)(s_n2 + k + 4);
      const float nw[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
      const float n2[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        u32x4_t o = {0, 0, 0, 0}, o2 = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float hn = Mfma16<T>::to_f32((u16)(a[mb][j >> 1] >> (16 * (j & 1)))) * inv[mb];
          o[j >> 1] |= (uint32_t)Mfma16<T>::from_f32(hn * nw[j]) << (16 * (j & 1));
          o2[j >> 1] |= (uint32_t)Mfma16<T>::from_f32(hn * n2[j]) << (16 * (j & 1));
        }
        a[mb] = in ? o : u32x4_t{0, 0, 0, 0};
        if (wx2 && tv[mb] && in) *(u32x4_t*)(x2 + (long long)(t0 + mb * 16 + r) * sx2 + k) = o2;
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) b[nb] = in ? b[nb] : u32x4_t{0, 0, 0, 0};
      mma(a, b);
    };
#pragma unroll
    for (int j0 = 0; j0 < RS_HOLD; j0 += U) {   // no branch on the step (see above)
      u32x4_t b[U][NB];
      if (j0 == 0) {
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) b[u][nb] = b0[u][nb];
      } else {
        ldb(b, s0 + j0);
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (j0 + u < RS_HOLD) step(hr[j0 + u], b[u], s0 + j0 + u);
    }
    for (int st = s0 + RS_HOLD; st < s1; ++st) {
      const int k = kof(st);
      u32x4_t a[MB], b[NB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) a[mb] = *(const u32x4_t*)(xp[mb] + k);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) b[nb] = *(const u32x4_t*)(wp[nb] + k);
      step(a, b, st);
    }
  }

  // D[(l/16)*4 + i][l%16] of each fragment: rows are tokens, columns experts
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    if (mb) __syncthreads();   // the previous block's sums have been read
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[wave][g * 4 + i][nb * 16 + r] = acc[mb][nb][i];
    __syncthreads();
    for (int o = threadIdx.x; o < 16 * TE; o += RS_WAVES * 64) {
      const int row = o / TE, col = o % TE;
      float v = red[0][row][col];
#pragma unroll
      for (int w = 1; w < RS_WAVES; ++w) v += red[w][row][col];
      const int t = t0 + mb * 16 + row, e = e0 + col;
      if (t < T_ && e < E) logits[(long long)t * sl + e] = v;
    }
  }
}

// Tile by batch size (measured on MI355X at H = 2816, E = 128). Small tiles spread small batches over
// many workgroups; large tiles cut the router weight's re-reads from L2 at prefill sizes. Every tile sums
// K the same way, so the choice never changes a logit's bits.
template <typename T, int MB, int NB, int U, bool NORM, int N2DT>
void launch_tile(const u16* x, long long sx, int T_, int H, const u16* wr, long long swr, int E, float* logits,
                 long long sl, const float* norm_w, float eps, const void* norm2_w, u16* x2, long long sx2,
                 hipStream_t st) {
  const size_t lds = NORM ? 2 * (size_t)H * sizeof(float) : 0;   // the norm weights, staged as float32
  const dim3 grid(((E + 16 * NB - 1) / (16 * NB)) * ((T_ + 16 * MB - 1) / (16 * MB)));
  router_split_kernel<T, MB, NB, U, NORM, N2DT><<<grid, RS_WAVES * 64, lds, st>>>(
      x, sx, T_, H, wr, swr, E, logits, sl, norm_w, eps, norm2_w, x2, sx2);
}

template <typename T, bool NORM, int N2DT = FLIDE_F32>
void launch_router(const u16* x, long long sx, int T_, int H, const u16* wr, long long swr, int E,
                   float* logits, long long sl, const float* norm_w, float eps, const void* norm2_w,
                   u16* x2, long long sx2, hipStream_t st) {
#define RT_TILE(MB, NB, U) launch_tile<T, MB, NB, U, NORM, N2DT>(x, sx, T_, H, wr, swr, E, logits, sl, norm_w, \
                                                               eps, norm2_w, x2, sx2, st)
  if constexpr (NORM) {   // 16 tokens: h stays in registers between the statistic and the MFMAs
    if (T_ <= 512) RT_TILE(1, 1, 2);
    else if (T_ <= 4096) RT_TILE(1, 4, 1);
    else RT_TILE(1, 8, 1);
  } else {
    if (T_ <= 768) RT_TILE(1, 1, 4);
    else if (T_ <= 3072) RT_TILE(2, 2, 2);
    else RT_TILE(4, 4, 1);
  }
#undef RT_TILE
}

// shared-expert gate logit: one wave per token, float32 sum of bf16/f16 products
template <typename T>
__global__ __launch_bounds__(256) void gate_kernel(const u16* __restrict__ x, long long sx, int T_,
                                                   int H, const u16* __restrict__ wg,
                                                   float* __restrict__ gate) {
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T_) return;
  const u16* xp = x + (long long)t * sx;
  float s = 0.f;
  for (int h = l; h < H; h += 64) s += Mfma16<T>::to_f32(xp[h]) * Mfma16<T>::to_f32(wg[h]);
  s = wave_sum(s);
  if (l == 0) gate[t] = s;
}

template <int EPL>
__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ logits, long long sl,
                                                    int T_, int E, int k, const void* scale,
                                                    int scale_dtype, float* __restrict__ w,
                                                    int* __restrict__ ids) {
  const long long t = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T_) return;
  float v[EPL], sc[EPL];
  routing::load_logits<EPL>(logits + t * sl, E, v);
  routing::load_scales<EPL>(scale, scale_dtype, E, sc);
  routing::route_select<EPL>(v, sc, E, k, w + t * k, ids + t * k, nullptr);
}

// Up to 128 experts and k <= 16: four tokens per wave, 16 lanes per token, lane u holding the logits of
// experts u + 16 i. A selection round is a local scan of EPL16 values and a 16-lane argmax (four DPP
// steps), so one wave's instructions select four tokens at once: at 8192 tokens the one-token-per-wave
// kernel issues about 600 VALU instructions per token and is bound by that (13.1 -> 8.2 us; 4096 tokens
// 8.9 -> 7.5 us). The same selection rule (larger logit, then lower id) and the same sums as
// route_select, in a 16-lane layout (the float sums round differently: weights within 1e-5).
template <int EPL16>
__global__ __launch_bounds__(256) void route16_kernel(const float* __restrict__ logits, long long sl, int T_, int E,
                                                      int k, const void* scale, int scale_dtype,
                                                      float* __restrict__ w, int* __restrict__ ids) {
  const int l = lane_id(), u = l & 15, row0 = l & ~15;
  const long long t0 = ((long long)blockIdx.x * 4 + (threadIdx.x >> 6)) * 4;
  if (t0 >= T_) return;   // the wave's four tokens all lie past the batch
  const long long t = t0 + (l >> 4);
  const bool live = t < T_;   // a dead token's lanes take part in the shuffles and store nothing
  float v[EPL16], sc[EPL16];
#pragma unroll
  for (int i = 0; i < EPL16; ++i) v[i] = live && u + 16 * i < E ? logits[t * sl + u + 16 * i] : -INFINITY;
  {
    uint32_t raw[EPL16];
    if (scale_dtype == FLIDE_F32) {
#pragma unroll
      for (int i = 0; i < EPL16; ++i)
        raw[i] = scale && u + 16 * i < E ? ((const uint32_t*)scale)[u + 16 * i] : 0x3f800000u;
    } else {
      const uint32_t one = scale_dtype == FLIDE_BF16 ? 0x3f80u : 0x3c00u;
#pragma unroll
      for (int i = 0; i < EPL16; ++i) raw[i] = scale && u + 16 * i < E ? ((const u16*)scale)[u + 16 * i] : one;
    }
#pragma unroll
    for (int i = 0; i < EPL16; ++i)
      sc[i] = scale_dtype == FLIDE_F32 ? __uint_as_float(raw[i])
              : scale_dtype == FLIDE_BF16 ? bf16_to_f32((u16)raw[i]) : f16_to_f32((u16)raw[i]);
  }
  float m = v[0];
#pragma unroll
  for (int i = 1; i < EPL16; ++i) m = fmaxf(m, v[i]);
  m = row16_max(m);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < EPL16; ++i)
    if (u + 16 * i < E) s += expf(v[i] - m);
  s = row16_sum(s);
  unsigned taken = 0;
  float my_v = -INFINITY;   // lane u < k: the u-th selected logit and its id
  int my_id = 0;
  for (int j = 0; j < k; ++j) {
    float bv = -INFINITY;
    int bi = INT_MAX;
#pragma unroll
    for (int i = 0; i < EPL16; ++i) {
      const int e = u + 16 * i;
      const bool free_ = e < E && !((taken >> i) & 1u);
      // a lane's ids ascend with i, so a strict > keeps the lower id among equal local values
      if (free_ && (v[i] > bv || bi == INT_MAX)) {
        bv = v[i];
        bi = e;
      }
    }
    row16_argmax(bv, bi);
    if (bi != INT_MAX && (bi & 15) == u) taken |= 1u << (bi >> 4);
    if (u == j) {
      my_v = bv;
      my_id = bi;
    }
  }
  float my_sc = 1.f;
  const int src = row0 | (my_id & 15);
#pragma unroll
  for (int i = 0; i < EPL16; ++i) {
    const float c = __shfl(sc[i], src);
    if ((my_id >> 4) == i) my_sc = c;
  }
  const float my_p = u < k ? expf(my_v - m) / s : 0.f;
  float topsum = 0.f;   // in slot order
  for (int j = 0; j < k; ++j) topsum += __shfl(my_p, row0 | j);
  if (live && u < k) {
    w[t * k + u] = my_p / topsum * my_sc;
    ids[t * k + u] = my_id;
  }
}

}  // namespace

extern "C" int flide_moe_router(const void* x, long long sx, int T, int H, int x_dtype,
                                const void* wr, long long swr, int E, const void* wg, float* logits,
                                long long sl, float* gate, flide_stream_t stream) {
  if (T < 0 || H <= 0 || E <= 0 || H % 8 || sx % 8 || swr % 8) return FLIDE_MOE_ERR_ARG;
  if (x_dtype != FLIDE_BF16 && x_dtype != FLIDE_F16) return FLIDE_MOE_ERR_ARG;
  if (((uintptr_t)x | (uintptr_t)wr) & 15) return FLIDE_MOE_ERR_ARG;
  if (T == 0) return FLIDE_MOE_OK;
  hipStream_t st = (hipStream_t)stream;
  if (x_dtype == FLIDE_BF16)
    launch_router<__bf16, false>((const u16*)x, sx, T, H, (const u16*)wr, swr, E, logits, sl, nullptr, 0.f,
                                 nullptr, nullptr, 0, st);
  else
    launch_router<_Float16, false>((const u16*)x, sx, T, H, (const u16*)wr, swr, E, logits, sl, nullptr, 0.f,
                                   nullptr, nullptr, 0, st);
  FLIDE_CHECK_LAUNCH();
  if (wg) {
    dim3 g2((T + 3) / 4);
    if (x_dtype == FLIDE_BF16)
      gate_kernel<__bf16><<<g2, 256, 0, st>>>((const u16*)x, sx, T, H, (const u16*)wg, gate);
    else
      gate_kernel<_Float16><<<g2, 256, 0, st>>>((const u16*)x, sx, T, H, (const u16*)wg, gate);
    FLIDE_CHECK_LAUNCH();
  }
  return FLIDE_MOE_OK;
}

extern "C" int flide_moe_router_norm(const void* h, long long sh, int T, int H, int h_dtype,
                                     const float* norm_w, const void* wr, long long swr, int E, float eps,
                                     float* logits, long long sl, const void* norm2_w, int norm2_dtype,
                                     void* x2, long long sx2, flide_stream_t stream) {
  if (T < 0 || H <= 0 || E <= 0 || H % 8 || sh % 8 || swr % 8 || !norm_w) return FLIDE_MOE_ERR_ARG;
  if (h_dtype != FLIDE_BF16 && h_dtype != FLIDE_F16) return FLIDE_MOE_ERR_ARG;
  if (H > RN_MAX_H) return FLIDE_MOE_ERR_ARG;   // both norm weights are staged in 64 KB of LDS
  if (x2 && (!norm2_w || (norm2_dtype != FLIDE_F32 && norm2_dtype != FLIDE_BF16 && norm2_dtype != FLIDE_F16)))
    return FLIDE_MOE_ERR_ARG;
  if (((uintptr_t)h | (uintptr_t)wr | (uintptr_t)norm_w | (uintptr_t)norm2_w | (uintptr_t)x2) & 15 ||
      (x2 && sx2 % 8))
    return FLIDE_MOE_ERR_ARG;
  if (T == 0) return FLIDE_MOE_OK;
  hipStream_t st = (hipStream_t)stream;
#define RN_LAUNCH(TT, N2) launch_router<TT, true, N2>((const u16*)h, sh, T, H, (const u16*)wr, swr, E, logits, sl, \
                                                    norm_w, eps, norm2_w, (u16*)x2, sx2, st)
  const int n2 = x2 ? norm2_dtype : FLIDE_F32;   // no x2: the kernel's norm2 loads read norm_w
  if (h_dtype == FLIDE_BF16) {
    if (n2 == FLIDE_F32) RN_LAUNCH(__bf16, FLIDE_F32);
    else if (n2 == FLIDE_BF16) RN_LAUNCH(__bf16, FLIDE_BF16);
    else RN_LAUNCH(__bf16, FLIDE_F16);
  } else {
    if (n2 == FLIDE_F32) RN_LAUNCH(_Float16, FLIDE_F32);
    else if (n2 == FLIDE_BF16) RN_LAUNCH(_Float16, FLIDE_BF16);
    else RN_LAUNCH(_Float16, FLIDE_F16);
  }
#undef RN_LAUNCH
  FLIDE_CHECK_LAUNCH();
  return FLIDE_MOE_OK;
}

extern "C" int flide_moe_route(const float* logits, long long sl, int T, int E, int k,
                               const void* scale, int scale_dtype, float* w, int* ids,
                               flide_stream_t stream) {
  if (T < 0 || E < 1 || E > 1024 || k < 1 || k > E || k > 64) return FLIDE_MOE_ERR_ARG;
  if (scale && scale_dtype != FLIDE_F32 && scale_dtype != FLIDE_BF16 && scale_dtype != FLIDE_F16)
    return FLIDE_MOE_ERR_ARG;
  if (T == 0) return FLIDE_MOE_OK;
  hipStream_t st = (hipStream_t)stream;
  // four tokens per wave once the batch is large enough for the one-token-per-wave kernel to be bound by
  // its instruction count (at 64 tokens that kernel's shorter chain wins: 3.5 against 7 us)
  if (E <= 128 && k <= 16 && T >= 2048) {
    const dim3 g16((T + 15) / 16);
#define ROUTE16(N) route16_kernel<N><<<g16, 256, 0, st>>>(logits, sl, T, E, k, scale, scale_dtype, w, ids)
    if (E <= 16) ROUTE16(1);
    else if (E <= 32) ROUTE16(2);
    else if (E <= 64) ROUTE16(4);
    else ROUTE16(8);
#undef ROUTE16
    FLIDE_CHECK_LAUNCH();
    return FLIDE_MOE_OK;
  }
  dim3 grid((T + 3) / 4);
  int epl = (E + 63) / 64;
#define ROUTE_CASE(N)                                                                          \
  case N:                                                                                      \
    route_kernel<N><<<grid, 256, 0, st>>>(logits, sl, T, E, k, scale, scale_dtype, w, ids); \
    break;
  switch (epl <= 1 ? 1 : epl <= 2 ? 2 : epl <= 4 ? 4 : epl <= 8 ? 8 : 16) {
    ROUTE_CASE(1)
    ROUTE_CASE(2)
    ROUTE_CASE(4)
    ROUTE_CASE(8)
    ROUTE_CASE(16)
  }
#undef ROUTE_CASE
  FLIDE_CHECK_LAUNCH();
  return FLIDE_MOE_OK;
}
