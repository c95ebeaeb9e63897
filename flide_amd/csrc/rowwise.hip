// Row-wise kernels on the MoE path: combine_norm / combine (flide/kernels/moe.py:256-277,372-395),
// per-row float8 quantization (flide/kernels/fp8.py:22-53), RMSNorm (flide/kernels/pointwise.py:21-49)
// and the unfused gated activations (pointwise.py:52-69,248-268).
//
// One workgroup of 256 threads per row for the reductions. Rows are read with 16-byte vector loads
// when the row length and stride allow it (every Gemma/Qwen shape does), else element by element.
// All arithmetic is float32, rounded once at the store.
#include <type_traits>

#include "common.hpp"
#include "quantize.hpp"

namespace {

constexpr int RW_THREADS = 256;

FLIDE_DEV float load_any(const void* p, int dtype, long long i) {
  if (dtype == FLIDE_F32) return ((const float*)p)[i];
  if (dtype == FLIDE_BF16) return bf16_to_f32(((const u16*)p)[i]);
  return f16_to_f32(((const u16*)p)[i]);
}

FLIDE_DEV void store_any(void* p, int dtype, long long i, float v) {
  if (dtype == FLIDE_F32) ((float*)p)[i] = v;
  else if (dtype == FLIDE_BF16) ((u16*)p)[i] = f32_to_bf16(v);
  else ((u16*)p)[i] = f32_to_f16(v);
}

// block-wide float sum (256 threads = 4 waves); every thread gets the total
FLIDE_DEV float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) red[wave] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

FLIDE_DEV float block_max(float v, float* red) {
  v = wave_max(v);
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) red[wave] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// ---------------------------------------------------------------------------------------------------
// combine_norm: one workgroup per token; the token's k rows summed in slot order into registers
// ---------------------------------------------------------------------------------------------------
constexpr int CN_MAXV = 8;  // up to 256 * 8 * 4 = 8192 columns with float4 pieces

template <int YDT>
__global__ __launch_bounds__(RW_THREADS) void combine_norm_kernel(const void* __restrict__ y,
                                                                  const void* __restrict__ dense,
                                                                  long long sd, const void* w1,
                                                                  const void* w2, int w_dtype,
                                                                  void* __restrict__ out, long long so,
                                                                  int out_dtype, int H, int k,
                                                                  float eps) {
  __shared__ float red[4];
  const long long t = blockIdx.x;
  const int nv = H / 4;  // float4 pieces (H % 4 == 0 checked on the host)
  float4 acc[CN_MAXV];
  float ss = 0.f;
#pragma unroll
  for (int v = 0; v < CN_MAXV; ++v) {
    const int c4 = threadIdx.x + v * RW_THREADS;
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    if (c4 < nv) {
      for (int j = 0; j < k; ++j) {
        const long long row = (t * k + j) * (long long)H;
        float4 yv;
        if constexpr (YDT == FLIDE_F32) {
          yv = ((const float4*)((const float*)y + row))[c4];
        } else {
          uint2 raw = ((const uint2*)((const u16*)y + row))[c4];
          if constexpr (YDT == FLIDE_BF16) {
            yv = make_float4(bf16_to_f32(raw.x & 0xffff), bf16_to_f32(raw.x >> 16),
                             bf16_to_f32(raw.y & 0xffff), bf16_to_f32(raw.y >> 16));
          } else {
            yv = make_float4(f16_to_f32(raw.x & 0xffff), f16_to_f32(raw.x >> 16),
                             f16_to_f32(raw.y & 0xffff), f16_to_f32(raw.y >> 16));
          }
        }
        s.x += yv.x; s.y += yv.y; s.z += yv.z; s.w += yv.w;
      }
      ss += s.x * s.x + s.y * s.y + s.z * s.z + s.w * s.w;
    }
    acc[v] = s;
  }
  float dd = 0.f;
  for (int c = threadIdx.x; c < H; c += RW_THREADS) {
    float d = load_any(dense, out_dtype, t * sd + c);
    dd += d * d;
  }
  const float sum_ss = block_sum(ss, red);
  const float sum_dd = block_sum(dd, red);
  const float inv_b = rsqrtf(sum_ss / H + eps);
  const float inv_a = rsqrtf(sum_dd / H + eps);
#pragma unroll
  for (int v = 0; v < CN_MAXV; ++v) {
    const int c4 = threadIdx.x + v * RW_THREADS;
    if (c4 >= nv) continue;
    const float vals[4] = {acc[v].x, acc[v].y, acc[v].z, acc[v].w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = c4 * 4 + q;
      const float d = load_any(dense, out_dtype, t * sd + c);
      const float a = d * inv_a * load_any(w1, w_dtype, c);
      const float b = vals[q] * inv_b * load_any(w2, w_dtype, c);
      store_any(out, out_dtype, t * so + c, a + b);
    }
  }
}

// combine_norm, vectorised for the common dtypes (y f32 or bf16; dense, out, w1, w2 bf16) and
// H <= 4096: every load of the token (k rows of y, dense, both weights) is issued before any sum.
// With SW, Gemma's next step follows in the same pass (pointwise.sandwich, pointwise.py:214-231): the
// rounded output d stays in registers and h_out = round((h + d * rsqrt(mean(d^2) + eps) * wp) * s), then,
// with wn, x_out = round(h_out * rsqrt(mean(h_out^2) + eps) * wn); d itself is not stored.
struct SandwichArgs {
  const u16* h;           // the residual stream [T, H]
  long long sh;
  const u16* wp;          // post-feed-forward norm weight [H]
  const void* scale;      // the layer scalar (one element) or null
  int scale_dtype;
  const u16* wn;          // next layer's input norm weight [H] or null
  u16* h_out;
  long long sho;
  u16* x_out;
  long long sxo;
};

// Both sums of a token's two norms, from one pair of barriers; each sum is the one block_sum gives.
FLIDE_DEV float2 block_sum2(float a, float b, float* red) {
  a = wave_sum(a);
  b = wave_sum(b);
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) {
    red[wave] = a;
    red[4 + wave] = b;
  }
  __syncthreads();
  return make_float2(red[0] + red[1] + red[2] + red[3], red[4] + red[5] + red[6] + red[7]);
}

// The float32 sum of a token's y rows for one group of four columns, in slot order.
template <typename YT> struct YGroup;
template <> struct YGroup<float> {
  typedef float raw __attribute__((ext_vector_type(4)));
  // y is read exactly once: float32 rows with non-temporal loads, which keep them from evicting what the
  // other wavefronts' rows still need (combine_norm at 8192 tokens: 153 -> 134 us, 6.2 TB/s)
  static FLIDE_DEV raw load(const float* row, int c4) { return __builtin_nontemporal_load((const raw*)row + c4); }
  static FLIDE_DEV float4 f32(raw r) { return make_float4(r[0], r[1], r[2], r[3]); }
};
template <> struct YGroup<u16> {
  typedef uint32_t raw __attribute__((ext_vector_type(2)));
  // 16-bit rows with plain loads: faster for them when y comes from HBM (4096 tokens, bf16 y: 53 -> 40 us;
  // no difference right after the down product, whose y the next read finds in the last-level cache)
  static FLIDE_DEV raw load(const u16* row, int c4) { return *((const raw*)row + c4); }
  static FLIDE_DEV float4 f32(raw r) {
    return make_float4(bf16_to_f32(r[0] & 0xffff), bf16_to_f32(r[0] >> 16), bf16_to_f32(r[1] & 0xffff),
                       bf16_to_f32(r[1] >> 16));
  }
};

FLIDE_DEV float4 bf16x4_f32(uint2 r) {
  return make_float4(bf16_to_f32(r.x & 0xffff), bf16_to_f32(r.x >> 16), bf16_to_f32(r.y & 0xffff),
                     bf16_to_f32(r.y >> 16));
}

// Every load of the token is issued before the first one is used: the k rows of y, dense, both norm
// weights and, with SW, h and the two sandwich weights. The loads stay unconditional so that nothing
// waits between them (a load under a per-lane or per-slot branch is followed by a wait for all loads in
// flight: three round trips per token, 4.9 us at 64 tokens): a lane past the row's end loads the row's
// last group and slots k .. KMAX - 1 load slot k - 1 again, and neither value is used.
template <typename YT, int KMAX, bool SW = false>
__global__ __launch_bounds__(RW_THREADS) void combine_norm_bf16_kernel(const YT* __restrict__ y,
                                                                       const u16* __restrict__ dense,
                                                                       long long sd, const u16* __restrict__ w1,
                                                                       const u16* __restrict__ w2,
                                                                       u16* __restrict__ out, long long so,
                                                                       int H, int k, float eps,
                                                                       SandwichArgs sw = {}) {
  constexpr int V = 4;  // float4 groups per thread: H <= 256 * 4 * 4
  typedef YGroup<YT> G;
  __shared__ float red[8];
  const long long t = blockIdx.x;
  const int nv = H / 4;
  typename G::raw yr[V][KMAX];
  uint2 draw[V], a1r[V], a2r[V], hr[V], wpr[V], wnr[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    if (v * RW_THREADS >= nv) break;   // the same for every lane
    const int c4 = min((int)threadIdx.x + v * RW_THREADS, nv - 1);
#pragma unroll
    for (int j = 0; j < KMAX; ++j) yr[v][j] = G::load(y + (t * k + (j < k ? j : k - 1)) * (long long)H, c4);
    draw[v] = ((const uint2*)(dense + t * sd))[c4];
    a1r[v] = ((const uint2*)w1)[c4];
    a2r[v] = ((const uint2*)w2)[c4];
    if constexpr (SW) {
      hr[v] = ((const uint2*)(sw.h + t * sw.sh))[c4];
      wpr[v] = ((const uint2*)sw.wp)[c4];
      if (sw.wn) wnr[v] = ((const uint2*)sw.wn)[c4];
    }
  }
  float sc = 1.f;
  if constexpr (SW) {
    if (sw.scale) sc = load_any(sw.scale, sw.scale_dtype, 0);
  }
  float4 acc[V], dv[V];
  float ss = 0.f, dd = 0.f;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    acc[v] = make_float4(0.f, 0.f, 0.f, 0.f);
    dv[v] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (v * RW_THREADS >= nv) break;
    if ((int)threadIdx.x + v * RW_THREADS >= nv) continue;
    dv[v] = bf16x4_f32(draw[v]);
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {   // slot order
      if (j >= k) break;
      const float4 yv = G::f32(yr[v][j]);
      acc[v].x += yv.x; acc[v].y += yv.y; acc[v].z += yv.z; acc[v].w += yv.w;
    }
    ss += acc[v].x * acc[v].x + acc[v].y * acc[v].y + acc[v].z * acc[v].z + acc[v].w * acc[v].w;
    dd += dv[v].x * dv[v].x + dv[v].y * dv[v].y + dv[v].z * dv[v].z + dv[v].w * dv[v].w;
  }
  const float2 sums = block_sum2(ss, dd, red);
  const float inv_b = rsqrtf(sums.x / H + eps);
  const float inv_a = rsqrtf(sums.y / H + eps);
#pragma unroll
  for (int v = 0; v < V; ++v) {
    if (v * RW_THREADS >= nv) break;
    const int c4 = threadIdx.x + v * RW_THREADS;
    if (c4 >= nv) continue;
    const uint2 a1 = a1r[v], a2 = a2r[v];
    const float o0 = dv[v].x * inv_a * bf16_to_f32(a1.x & 0xffff) + acc[v].x * inv_b * bf16_to_f32(a2.x & 0xffff);
    const float o1 = dv[v].y * inv_a * bf16_to_f32(a1.x >> 16) + acc[v].y * inv_b * bf16_to_f32(a2.x >> 16);
    const float o2 = dv[v].z * inv_a * bf16_to_f32(a1.y & 0xffff) + acc[v].z * inv_b * bf16_to_f32(a2.y & 0xffff);
    const float o3 = dv[v].w * inv_a * bf16_to_f32(a1.y >> 16) + acc[v].w * inv_b * bf16_to_f32(a2.y >> 16);
    uint2 o;
    o.x = (uint32_t)f32_to_bf16(o0) | ((uint32_t)f32_to_bf16(o1) << 16);
    o.y = (uint32_t)f32_to_bf16(o2) | ((uint32_t)f32_to_bf16(o3) << 16);
    if constexpr (SW) {
      dv[v] = bf16x4_f32(o);   // d, rounded as the reference stores it
    } else {
      ((uint2*)(out + t * so))[c4] = o;
    }
  }
  if constexpr (SW) {
    float d2 = 0.f;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      if (v * RW_THREADS >= nv) break;
      if ((int)threadIdx.x + v * RW_THREADS >= nv) continue;
      d2 += dv[v].x * dv[v].x + dv[v].y * dv[v].y + dv[v].z * dv[v].z + dv[v].w * dv[v].w;
    }
    const float inv_d = rsqrtf(block_sum(d2, red) / H + eps);
    float h2 = 0.f;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      if (v * RW_THREADS >= nv) break;
      const int c4 = threadIdx.x + v * RW_THREADS;
      if (c4 >= nv) continue;
      const float dq[4] = {dv[v].x, dv[v].y, dv[v].z, dv[v].w};
      const uint32_t hu[2] = {hr[v].x, hr[v].y}, wu[2] = {wpr[v].x, wpr[v].y};
      float hb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float hh = bf16_to_f32((hu[i >> 1] >> (16 * (i & 1))) & 0xffff);
        const float ww = bf16_to_f32((wu[i >> 1] >> (16 * (i & 1))) & 0xffff);
        float r = hh + dq[i] * inv_d * ww;
        if (sw.scale) r *= sc;
        hb[i] = bf16_round(r);
        h2 += hb[i] * hb[i];
      }
      dv[v] = make_float4(hb[0], hb[1], hb[2], hb[3]);
      uint2 o;
      o.x = (uint32_t)f32_to_bf16(hb[0]) | ((uint32_t)f32_to_bf16(hb[1]) << 16);
      o.y = (uint32_t)f32_to_bf16(hb[2]) | ((uint32_t)f32_to_bf16(hb[3]) << 16);
      ((uint2*)(sw.h_out + t * sw.sho))[c4] = o;
    }
    if (sw.wn) {
      const float inv_h = rsqrtf(block_sum(h2, red) / H + eps);
#pragma unroll
      for (int v = 0; v < V; ++v) {
        if (v * RW_THREADS >= nv) break;
        const int c4 = threadIdx.x + v * RW_THREADS;
        if (c4 >= nv) continue;
        const uint2 wr = wnr[v];
        uint2 o;
        o.x = (uint32_t)f32_to_bf16(dv[v].x * inv_h * bf16_to_f32(wr.x & 0xffff)) |
              ((uint32_t)f32_to_bf16(dv[v].y * inv_h * bf16_to_f32(wr.x >> 16)) << 16);
        o.y = (uint32_t)f32_to_bf16(dv[v].z * inv_h * bf16_to_f32(wr.y & 0xffff)) |
              ((uint32_t)f32_to_bf16(dv[v].w * inv_h * bf16_to_f32(wr.y >> 16)) << 16);
        ((uint2*)(sw.x_out + t * sw.sxo))[c4] = o;
      }
    }
  }
}

// KMAX: the loads a lane issues per group of columns (k rounded up to 2, 4 or 8)
template <typename YT, bool SW>
void launch_combine_norm_vec(const YT* y, const u16* dense, long long sd, const u16* w1, const u16* w2, u16* out,
                             long long so, int T, int H, int k, float eps, SandwichArgs sw, hipStream_t st) {
#define CN(KM) combine_norm_bf16_kernel<YT, KM, SW><<<T, RW_THREADS, 0, st>>>(y, dense, sd, w1, w2, out, so, H, k, eps, sw)
  if (k <= 2) CN(2);
  else if (k <= 4) CN(4);
  else CN(8);
#undef CN
}

// combine (Qwen), vectorised for y float32 or bf16 with bf16 shared and out, H % 4 == 0, H <= 4096 and
// k <= 8: one workgroup per token, the k rows summed in slot order in registers, y read non-temporally
// (each element is read once), then + shared * sigmoid(gate) and one rounding (moe.py:256-277).
template <typename YT>
__global__ __launch_bounds__(RW_THREADS) void combine_vec_kernel(const YT* __restrict__ y,
                                                                 const u16* __restrict__ shared,
                                                                 const float* __restrict__ gate,
                                                                 u16* __restrict__ out, int H, int k) {
  constexpr int V = 4, KMAX = 8;
  const long long t = blockIdx.x;
  const int nv = H / 4;
  const float sg = 1.0f / (1.0f + expf(-gate[t]));
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int c4 = threadIdx.x + v * RW_THREADS;
    if (c4 >= nv) continue;
    float4 yv[KMAX];
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      if (j >= k) break;
      const long long row = (t * k + j) * (long long)H;
      if constexpr (std::is_same<YT, float>::value) {
        typedef float f32x4v __attribute__((ext_vector_type(4)));
        const f32x4v q = __builtin_nontemporal_load((const f32x4v*)(y + row) + c4);
        yv[j] = make_float4(q[0], q[1], q[2], q[3]);
      } else {
        typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
        const u32x2v raw = *((const u32x2v*)(y + row) + c4);   // 16-bit rows: plain loads (as combine_norm)
        yv[j] = make_float4(bf16_to_f32(raw[0] & 0xffff), bf16_to_f32(raw[0] >> 16), bf16_to_f32(raw[1] & 0xffff),
                            bf16_to_f32(raw[1] >> 16));
      }
    }
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {   // slot order
      if (j >= k) break;
      acc.x += yv[j].x; acc.y += yv[j].y; acc.z += yv[j].z; acc.w += yv[j].w;
    }
    const uint2 sr = ((const uint2*)(shared + t * H))[c4];
    uint2 o;
    o.x = (uint32_t)f32_to_bf16(acc.x + bf16_to_f32(sr.x & 0xffff) * sg) |
          ((uint32_t)f32_to_bf16(acc.y + bf16_to_f32(sr.x >> 16) * sg) << 16);
    o.y = (uint32_t)f32_to_bf16(acc.z + bf16_to_f32(sr.y & 0xffff) * sg) |
          ((uint32_t)f32_to_bf16(acc.w + bf16_to_f32(sr.y >> 16) * sg) << 16);
    ((uint2*)(out + t * H))[c4] = o;
  }
}

// combine (Qwen): sum of the k rows + shared * sigmoid(gate); one workgroup per (token, 1024 columns)
template <int YDT>
__global__ __launch_bounds__(RW_THREADS) void combine_kernel(const void* __restrict__ y,
                                                             const void* __restrict__ shared,
                                                             const float* __restrict__ gate,
                                                             void* __restrict__ out, int out_dtype,
                                                             int H, int k) {
  const long long t = blockIdx.x;
  const float gt = gate[t];
  const float sg = 1.0f / (1.0f + expf(-gt));
  for (int c = blockIdx.y * 1024 + threadIdx.x; c < min(H, (int)(blockIdx.y + 1) * 1024);
       c += RW_THREADS) {
    float s = 0.f;
    for (int j = 0; j < k; ++j) s += load_any(y, YDT, (t * k + j) * (long long)H + c);
    const float sh = load_any(shared, out_dtype, t * H + c);
    store_any(out, out_dtype, t * H + c, s + sh * sg);
  }
}

// ---------------------------------------------------------------------------------------------------
// per-row e4m3 quantization: s = max(amax, 1e-12) * (1/448); q = e4m3(clamp(x / s, +-448))
// ---------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(RW_THREADS) void quantize_rows_kernel(const void* __restrict__ x,
                                                                   long long sx, int K, int x_dtype,
                                                                   u8* __restrict__ q, long long sq,
                                                                   float* __restrict__ s) {
  __shared__ float red[4];
  const long long row = blockIdx.x;
  float amax = 0.f;
  for (int c = threadIdx.x; c < K; c += RW_THREADS)
    amax = fmaxf(amax, fabsf(load_any(x, x_dtype, row * sx + c)));
  amax = block_max(amax, red);
  const float sc = fmaxf(amax, 1e-12f) * (1.0f / 448.0f);
  if (threadIdx.x == 0) s[row] = sc;
  for (int c = threadIdx.x; c < K; c += RW_THREADS) {
    float v = load_any(x, x_dtype, row * sx + c) / sc;  // correctly rounded division
    v = fminf(fmaxf(v, -448.0f), 448.0f);
    q[row * sq + c] = f32_to_e4m3fn(v);
  }
}

// 16-bit rows, K % 8 == 0, K <= NV * 512: one wave per row (4 rows per workgroup), quant::quantize_row16.
template <int NV, bool BF16>
__global__ __launch_bounds__(RW_THREADS) void quantize_rows_vec_kernel(const u16* __restrict__ x, long long sx,
                                                                       int K, int M, u8* __restrict__ q,
                                                                       long long sq, float* __restrict__ s) {
  const long long row = (long long)blockIdx.x * (RW_THREADS / 64) + (threadIdx.x >> 6);
  if (row >= M) return;
  quant::quantize_row16<NV, BF16>(x, sx, K, row, q, sq, s);
}

// ---------------------------------------------------------------------------------------------------
// RMSNorm without residual
// ---------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(RW_THREADS) void rms_norm_kernel(const void* __restrict__ x, long long sx,
                                                              int x_dtype, const void* w, int w_dtype,
                                                              void* __restrict__ yout, long long sy,
                                                              int y_dtype, int N, float eps,
                                                              int offset) {
  __shared__ float red[4];
  const long long row = blockIdx.x;
  float ss = 0.f;
  for (int c = threadIdx.x; c < N; c += RW_THREADS) {
    float v = load_any(x, x_dtype, row * sx + c);
    ss += v * v;
  }
  ss = block_sum(ss, red);
  const float inv = rsqrtf(ss / N + eps);
  for (int c = threadIdx.x; c < N; c += RW_THREADS) {
    float v = load_any(x, x_dtype, row * sx + c);
    float wv = load_any(w, w_dtype, c);
    if (offset) wv = 1.0f + wv;
    store_any(yout, y_dtype, row * sy + c, v * inv * wv);
  }
}

template <int ACT>
__global__ __launch_bounds__(RW_THREADS) void gated_act_kernel(const void* __restrict__ a,
                                                               long long sa,
                                                               const void* __restrict__ b,
                                                               long long sb, void* __restrict__ out,
                                                               long long so, int dtype, int n) {
  const long long row = blockIdx.x;
  for (int c = blockIdx.y * 1024 + threadIdx.x; c < min(n, (int)(blockIdx.y + 1) * 1024);
       c += RW_THREADS) {
    const float av = load_any(a, dtype, row * sa + c);
    const float bv = load_any(b, dtype, row * sb + c);
    store_any(out, dtype, row * so + c, act_f32<ACT>(av, bv));
  }
}

bool dtype_ok(int d) { return d == FLIDE_F32 || d == FLIDE_BF16 || d == FLIDE_F16; }

}  // namespace

extern "C" int flide_moe_combine_norm(const void* y, int y_dtype, const void* dense, long long sd,
                                      const void* w1, const void* w2, int w_dtype, void* out,
                                      long long so, int out_dtype, int T, int H, int k, float eps,
                                      flide_stream_t stream) {
  if (T < 0 || H <= 0 || k <= 0 || H % 4 || H > 4 * RW_THREADS * CN_MAXV) return FLIDE_MOE_ERR_ARG;
  if (!dtype_ok(y_dtype) || !dtype_ok(w_dtype) || !dtype_ok(out_dtype)) return FLIDE_MOE_ERR_ARG;
  if ((uintptr_t)y & 15) return FLIDE_MOE_ERR_ARG;
  if (T == 0) return FLIDE_MOE_OK;
  hipStream_t st = (hipStream_t)stream;
  const bool vec = out_dtype == FLIDE_BF16 && w_dtype == FLIDE_BF16 && H <= 4 * 4 * RW_THREADS && k <= 8 &&
                   sd % 4 == 0 && so % 4 == 0 && !(((uintptr_t)dense | (uintptr_t)out | (uintptr_t)w1 | (uintptr_t)w2) & 7);
  if (vec && y_dtype == FLIDE_F32) {
    launch_combine_norm_vec<float, false>((const float*)y, (const u16*)dense, sd, (const u16*)w1, (const u16*)w2,
                                          (u16*)out, so, T, H, k, eps, {}, st);
    FLIDE_CHECK_LAUNCH();
    return FLIDE_MOE_OK;
  }
  if (vec && y_dtype == FLIDE_BF16) {
    launch_combine_norm_vec<u16, false>((const u16*)y, (const u16*)dense, sd, (const u16*)w1, (const u16*)w2,
                                        (u16*)out, so, T, H, k, eps, {}, st);
    FLIDE_CHECK_LAUNCH();
    return FLIDE_MOE_OK;
  }
  if (y_dtype == FLIDE_F32)
    combine_norm_kernel<FLIDE_F32><<<T, RW_THREADS, 0, st>>>(y, dense, sd, w1, w2, w_dtype, out, so,
                                                              out_dtype, H, k, eps);
  else if (y_dtype == FLIDE_BF16)
    combine_norm_kernel<FLIDE_BF16><<<T, RW_THREADS, 0, st>>>(y, dense, sd, w1, w2, w_dtype, out, so,
                                                               out_dtype, H, k, eps);
  else
    combine_norm_kernel<FLIDE_F16><<<T, RW_THREADS, 0, st>>>(y, dense, sd, w1, w2, w_dtype, out, so,
                                                              out_dtype, H, k, eps);
  FLIDE_CHECK_LAUNCH();
  return FLIDE_MOE_OK;
}

extern "C" int flide_moe_combine(const void* y, int y_dtype, const void* shared, const float* gate,
                                 void* out, int out_dtype, int T, int H, int k,
                                 flide_stream_t stream) {
  if (T < 0 || H <= 0 || k <= 0 || !dtype_ok(y_dtype) || !dtype_ok(out_dtype))
    return FLIDE_MOE_ERR_ARG;
  if (T == 0) return FLIDE_MOE_OK;
  hipStream_t st = (hipStream_t)stream;
  if (out_dtype == FLIDE_BF16 && (y_dtype == FLIDE_F32 || y_dtype == FLIDE_BF16) && H % 4 == 0 &&
      H <= 4 * 4 * RW_THREADS && k <= 8 && !((uintptr_t)y & 15) && !(((uintptr_t)shared | (uintptr_t)out) & 7)) {
    if (y_dtype == FLIDE_F32)
      combine_vec_kernel<float><<<T, RW_THREADS, 0, st>>>((const float*)y, (const u16*)shared, gate, (u16*)out, H, k);
    else
      combine_vec_kernel<u16><<<T, RW_THREADS, 0, st>>>((const u16*)y, (const u16*)shared, gate, (u16*)out, H, k);
    FLIDE_CHECK_LAUNCH();
    return FLIDE_MOE_OK;
  }
  dim3 grid(T, (H + 1023) / 1024);
  if (y_dtype == FLIDE_F32)
    combine_kernel<FLIDE_F32><<<grid, RW_THREADS, 0, st>>>(y, shared, gate, out, out_dtype, H, k);
  else if (y_dtype == FLIDE_BF16)
    combine_kernel<FLIDE_BF16><<<grid, RW_THREADS, 0, st>>>(y, shared, gate, out, out_dtype, H, k);
  else
    combine_kernel<FLIDE_F16><<<grid, RW_THREADS, 0, st>>>(y, shared, gate, out, out_dtype, H, k);
  FLIDE_CHECK_LAUNCH();
  return FLIDE_MOE_OK;
}

extern "C" int flide_moe_quantize_rows(const void* x, long long sx, int M, int K, int x_dtype,
                                       void* q, long long sq, float* s, flide_stream_t stream) {
  if (M < 0 || K < 0 || !dtype_ok(x_dtype)) return FLIDE_MOE_ERR_ARG;
  if (M == 0) return FLIDE_MOE_OK;
  hipStream_t st = (hipStream_t)stream;
  if (quant::row16_ok(x, sx, K, x_dtype, q, sq)) {
    const int nv = quant::row16_nv(K);
    const dim3 grid((M + 3) / 4);
#define QV(NV)                                                                                            \
  do {                                                                                                     \
    if (x_dtype == FLIDE_BF16)                                                                             \
      quantize_rows_vec_kernel<NV, true><<<grid, RW_THREADS, 0, st>>>((const u16*)x, sx, K, M, (u8*)q, sq, s); \
    else                                                                                                   \
      quantize_rows_vec_kernel<NV, false><<<grid, RW_THREADS, 0, st>>>((const u16*)x, sx, K, M, (u8*)q, sq, s); \
  } while (0)
    if (nv == 1) QV(1);
    else if (nv == 2) QV(2);
    else if (nv == 4) QV(4);
    else if (nv == 8) QV(8);
    else QV(16);
#undef QV
    FLIDE_CHECK_LAUNCH();
    return FLIDE_MOE_OK;
  }
  quantize_rows_kernel<<<M, RW_THREADS, 0, st>>>(x, sx, K, x_dtype, (u8*)q, sq, s);
  FLIDE_CHECK_LAUNCH();
  return FLIDE_MOE_OK;
}

// RMSNorm of 16-bit rows into the same type (flide/kernels/pointwise.py:21-36): one wave per row, the
// row held in registers between the two passes (NV 16-byte chunks per lane), so x is read from memory once.
template <bool BF16, int WDT, int NV>
__global__ __launch_bounds__(RW_THREADS) void rms_norm_vec_kernel(const u16* __restrict__ x, long long sx,
                                                                  const void* __restrict__ w,
                                                                  u16* __restrict__ y, long long sy, int N,
                                                                  int T, float eps, int offset) {
  const int l = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * (RW_THREADS / 64) + (threadIdx.x >> 6);
  if (row >= T) return;
  const int nv = N / 8;
  const uint4* xr = (const uint4*)(x + row * sx);
  uint4 raw[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int c = l + v * 64;
    raw[v] = c < nv ? xr[c] : make_uint4(0, 0, 0, 0);
  }
  auto val = [](uint32_t u, int hi) {
    const u16 h = hi ? (u16)(u >> 16) : (u16)(u & 0xffff);
    return BF16 ? bf16_to_f32(h) : f16_to_f32(h);
  };
  auto rnd = [](float f) -> uint32_t { return BF16 ? f32_to_bf16(f) : f32_to_f16(f); };
  float ss = 0.f;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const uint32_t u[4] = {raw[v].x, raw[v].y, raw[v].z, raw[v].w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float f = val(u[i >> 1], i & 1);
      ss += f * f;
    }
  }
  ss = wave_sum(ss);
  const float inv = rsqrtf(ss / N + eps);
  uint4* yr = (uint4*)(y + row * sy);
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int c = l + v * 64;
    if (c >= nv) continue;
    float wv[8];
    if constexpr (WDT == FLIDE_F32) {
      const float4 w0 = ((const float4*)w)[2 * c], w1 = ((const float4*)w)[2 * c + 1];
      wv[0] = w0.x; wv[1] = w0.y; wv[2] = w0.z; wv[3] = w0.w;
      wv[4] = w1.x; wv[5] = w1.y; wv[6] = w1.z; wv[7] = w1.w;
    } else {
      const uint4 wr = ((const uint4*)w)[c];
      const uint32_t u[4] = {wr.x, wr.y, wr.z, wr.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const u16 h = (i & 1) ? (u16)(u[i >> 1] >> 16) : (u16)(u[i >> 1] & 0xffff);
        wv[i] = WDT == FLIDE_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
      }
    }
    const uint32_t u[4] = {raw[v].x, raw[v].y, raw[v].z, raw[v].w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float w0 = offset ? 1.0f + wv[2 * i] : wv[2 * i], w1 = offset ? 1.0f + wv[2 * i + 1] : wv[2 * i + 1];
      o[i] = rnd(val(u[i], 0) * inv * w0) | (rnd(val(u[i], 1) * inv * w1) << 16);
    }
    yr[c] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

template <bool BF16, int WDT>
void launch_rms_norm_vec(const void* x, long long sx, const void* w, void* y, long long sy, int T, int N,
                         float eps, int offset, hipStream_t st) {
  const int per_lane = (N / 8 + 63) / 64;
  const dim3 grid((T + RW_THREADS / 64 - 1) / (RW_THREADS / 64));
#define RV(NV) rms_norm_vec_kernel<BF16, WDT, NV><<<grid, RW_THREADS, 0, st>>>( \
    (const u16*)x, sx, w, (u16*)y, sy, N, T, eps, offset)
  if (per_lane <= 1) RV(1);
  else if (per_lane <= 2) RV(2);
  else if (per_lane <= 4) RV(4);
  else if (per_lane <= 6) RV(6);
  else if (per_lane <= 8) RV(8);
  else RV(16);
#undef RV
}

extern "C" int flide_moe_combine_norm_sandwich(const void* y, int y_dtype, const void* dense, long long sd,
                                               const void* w1, const void* w2, const void* h, long long sh,
                                               const void* w_post, const void* scale, int scale_dtype,
                                               const void* w_next, void* h_out, long long sho, void* x_out,
                                               long long sxo, int T, int H, int k, float eps,
                                               flide_stream_t stream) {
  if (T < 0 || H <= 0 || k <= 0 || k > 8 || H % 4 || H > 4 * 4 * RW_THREADS) return FLIDE_MOE_ERR_ARG;
  if (y_dtype != FLIDE_F32 && y_dtype != FLIDE_BF16) return FLIDE_MOE_ERR_ARG;
  if (scale && !dtype_ok(scale_dtype)) return FLIDE_MOE_ERR_ARG;
  if (!dense || !w1 || !w2 || !h || !w_post || !h_out || (w_next && !x_out)) return FLIDE_MOE_ERR_ARG;
  if (sd % 4 || sh % 4 || sho % 4 || (w_next && sxo % 4)) return FLIDE_MOE_ERR_ARG;
  if (((uintptr_t)y & 15) || (((uintptr_t)dense | (uintptr_t)w1 | (uintptr_t)w2 | (uintptr_t)h | (uintptr_t)w_post |
                               (uintptr_t)w_next | (uintptr_t)h_out | (uintptr_t)x_out) & 7))
    return FLIDE_MOE_ERR_ARG;
  if (T == 0) return FLIDE_MOE_OK;
  const SandwichArgs sw{(const u16*)h, sh, (const u16*)w_post, scale, scale_dtype, (const u16*)w_next,
                        (u16*)h_out, sho, (u16*)x_out, sxo};
  hipStream_t st = (hipStream_t)stream;
  if (y_dtype == FLIDE_F32)
    launch_combine_norm_vec<float, true>((const float*)y, (const u16*)dense, sd, (const u16*)w1, (const u16*)w2,
                                         nullptr, 0, T, H, k, eps, sw, st);
  else
    launch_combine_norm_vec<u16, true>((const u16*)y, (const u16*)dense, sd, (const u16*)w1, (const u16*)w2,
                                       nullptr, 0, T, H, k, eps, sw, st);
  FLIDE_CHECK_LAUNCH();
  return FLIDE_MOE_OK;
}

extern "C" int flide_moe_rms_norm(const void* x, long long sx, int x_dtype, const void* w,
                                  int w_dtype, void* y, long long sy, int y_dtype, int T, int N,
                                  float eps, int offset, flide_stream_t stream) {
  if (T < 0 || N <= 0 || !dtype_ok(x_dtype) || !dtype_ok(w_dtype) || !dtype_ok(y_dtype))
    return FLIDE_MOE_ERR_ARG;
  if (T == 0) return FLIDE_MOE_OK;
  hipStream_t st = (hipStream_t)stream;
  // 16-bit rows into their own type, 16-byte aligned, at most 8192 wide: the vector kernel
  if (x_dtype != FLIDE_F32 && y_dtype == x_dtype && N % 8 == 0 && N <= 64 * 8 * 16 && sx % 8 == 0 &&
      sy % 8 == 0 && !(((uintptr_t)x | (uintptr_t)y | (uintptr_t)w) & 15)) {
#define RN(BF, WD) launch_rms_norm_vec<BF, WD>(x, sx, w, y, sy, T, N, eps, offset, st)
    const bool bf = x_dtype == FLIDE_BF16;
    if (w_dtype == FLIDE_F32) { if (bf) RN(true, FLIDE_F32); else RN(false, FLIDE_F32); }
    else if (w_dtype == FLIDE_BF16) { if (bf) RN(true, FLIDE_BF16); else RN(false, FLIDE_BF16); }
    else { if (bf) RN(true, FLIDE_F16); else RN(false, FLIDE_F16); }
#undef RN
    FLIDE_CHECK_LAUNCH();
    return FLIDE_MOE_OK;
  }
  rms_norm_kernel<<<T, RW_THREADS, 0, st>>>(x, sx, x_dtype, w, w_dtype, y, sy, y_dtype, N, eps, offset);
  FLIDE_CHECK_LAUNCH();
  return FLIDE_MOE_OK;
}

extern "C" int flide_moe_gated_act(const void* a, long long sa, const void* b, long long sb,
                                   void* out, long long so, int dtype, int T, int n, int act,
                                   flide_stream_t stream) {
  if (T < 0 || n < 0 || !dtype_ok(dtype)) return FLIDE_MOE_ERR_ARG;
  if (T == 0 || n == 0) return FLIDE_MOE_OK;
  dim3 grid(T, (n + 1023) / 1024);
  hipStream_t st = (hipStream_t)stream;
  if (act == ACT_GEGLU)
    gated_act_kernel<ACT_GEGLU><<<grid, RW_THREADS, 0, st>>>(a, sa, b, sb, out, so, dtype, n);
  else if (act == ACT_SWIGLU)
    gated_act_kernel<ACT_SWIGLU><<<grid, RW_THREADS, 0, st>>>(a, sa, b, sb, out, so, dtype, n);
  else
    return FLIDE_MOE_ERR_ARG;
  FLIDE_CHECK_LAUNCH();
  return FLIDE_MOE_OK;
}
