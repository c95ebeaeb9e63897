// Router logits and routing: flide/kernels/moe.py:128-204 re-designed for CDNA4.
//
// router: a plain [T, H] x [E, H]^T product with float32 output. One workgroup of 4 waves computes a
//   32-token x 128-expert tile; each wave a 16 x 64 slab with v_mfma_f32_16x16x32 fragments read
//   straight from global memory (the router weight, 0.7 MB at the Gemma shape, stays in L2).
// route: one wave64 per token. The token's E logits sit in registers (E/64 per lane); k rounds of a
//   wave argmax (larger logit, then lower expert id) pick the experts, so the selection is exact and
//   independent of how exp rounds; the softmax weights follow the reference's formula.
#include <float.h>
#include <limits.h>

#include "common.hpp"

namespace {

constexpr int RT_TOK = 32;   // router tile: tokens
constexpr int RT_EXP = 128;  // router tile: experts

template <typename T>
__global__ __launch_bounds__(256) void router_kernel(const u16* __restrict__ x, long long sx, int T_,
                                                     int H, const u16* __restrict__ wr, long long swr,
                                                     int E, float* __restrict__ logits, long long sl) {
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int wm = wave & 1, wn = wave >> 1;
  const int t0 = blockIdx.x * RT_TOK + wm * 16;
  const int e0 = blockIdx.y * RT_EXP + wn * 64;
  const int r = l & 15, g = l >> 4;
  const int trow = t0 + r;
  const bool tvalid = trow < T_;
  const u16* xp = x + (long long)(tvalid ? trow : 0) * sx;
  const u16* wp[4];
  bool evalid[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) {
    int e = e0 + nb * 16 + r;
    evalid[nb] = e < E;
    wp[nb] = wr + (long long)(evalid[nb] ? e : 0) * swr;
  }
  f32x4_t acc[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) acc[nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < H; k0 += 64) {
    // this lane's K-values of the two 32-wide MFMA steps: k0 + s*32 + g*8 .. +8
    const int kk = k0 + g * 8;
    u32x4_t a0 = {0, 0, 0, 0}, a1 = {0, 0, 0, 0};
    if (tvalid && kk < H) a0 = *(const u32x4_t*)(xp + kk);
    if (tvalid && kk + 32 < H) a1 = *(const u32x4_t*)(xp + kk + 32);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      u32x4_t b0 = {0, 0, 0, 0}, b1 = {0, 0, 0, 0};
      if (evalid[nb] && kk < H) b0 = *(const u32x4_t*)(wp[nb] + kk);
      if (evalid[nb] && kk + 32 < H) b1 = *(const u32x4_t*)(wp[nb] + kk + 32);
      acc[nb] = Mfma16<T>::mma(a0, b0, acc[nb]);
      acc[nb] = Mfma16<T>::mma(a1, b1, acc[nb]);
    }
  }
  // D[(l/16)*4 + i][l%16]: rows are tokens, columns experts
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) {
    int e = e0 + nb * 16 + r;
    if (e >= E) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int t = t0 + g * 4 + i;
      if (t < T_) logits[(long long)t * sl + e] = acc[nb][i];
    }
  }
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

FLIDE_DEV float load_scalar(const void* p, int dtype, int i) {
  if (dtype == FLIDE_F32) return ((const float*)p)[i];
  if (dtype == FLIDE_BF16) return bf16_to_f32(((const u16*)p)[i]);
  return f16_to_f32(((const u16*)p)[i]);
}

template <int EPL>
__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ logits, long long sl,
                                                    int T_, int E, int k, const void* scale,
                                                    int scale_dtype, float* __restrict__ w,
                                                    int* __restrict__ ids) {
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  const long long t = (long long)blockIdx.x * 4 + wave;
  if (t >= T_) return;
  const float* row = logits + t * sl;
  float v[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    int e = l + 64 * i;
    v[i] = e < E ? row[e] : -INFINITY;
  }
  float m = v[0];
#pragma unroll
  for (int i = 1; i < EPL; ++i) m = fmaxf(m, v[i]);
  m = wave_max(m);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < EPL; ++i)
    if (l + 64 * i < E) s += expf(v[i] - m);
  s = wave_sum(s);
  unsigned taken = 0;
  float my_v = -INFINITY;   // lane j < k: the j-th selected logit and its id
  int my_id = 0;
  for (int j = 0; j < k; ++j) {
    float bv = -INFINITY;
    int bi = INT_MAX;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      int e = l + 64 * i;
      bool free_ = e < E && !((taken >> i) & 1u);
      // lanes hold ascending ids, so a strict > keeps the lower id among equal local values
      if (free_ && (v[i] > bv || bi == INT_MAX)) {
        bv = v[i];
        bi = e;
      }
    }
    wave_argmax(bv, bi);
    if (bi != INT_MAX && (bi & 63) == l) taken |= 1u << (bi >> 6);
    if (l == j) {
      my_v = bv;
      my_id = bi;
    }
  }
  // probabilities of the selected experts, summed in slot order (lane reads of lanes 0..k-1)
  const float my_p = l < k ? expf(my_v - m) / s : 0.f;
  float topsum = 0.f;
  for (int j = 0; j < k; ++j) topsum += __shfl(my_p, j);
  if (l < k) {
    float ww = my_p / topsum;
    if (scale) ww *= load_scalar(scale, scale_dtype, my_id);
    w[t * k + l] = ww;
    ids[t * k + l] = my_id;
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
  dim3 grid((T + RT_TOK - 1) / RT_TOK, (E + RT_EXP - 1) / RT_EXP);
  if (x_dtype == FLIDE_BF16)
    router_kernel<__bf16><<<grid, 256, 0, st>>>((const u16*)x, sx, T, H, (const u16*)wr, swr, E,
                                                 logits, sl);
  else
    router_kernel<_Float16><<<grid, 256, 0, st>>>((const u16*)x, sx, T, H, (const u16*)wr, swr, E,
                                                   logits, sl);
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

extern "C" int flide_moe_route(const float* logits, long long sl, int T, int E, int k,
                               const void* scale, int scale_dtype, float* w, int* ids,
                               flide_stream_t stream) {
  if (T < 0 || E < 1 || E > 1024 || k < 1 || k > E || k > 64) return FLIDE_MOE_ERR_ARG;
  if (scale && scale_dtype != FLIDE_F32 && scale_dtype != FLIDE_BF16 && scale_dtype != FLIDE_F16)
    return FLIDE_MOE_ERR_ARG;
  if (T == 0) return FLIDE_MOE_OK;
  hipStream_t st = (hipStream_t)stream;
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
