// Grouped expert products on CDNA4 MFMA: flide/kernels/moe.py:46-125,286-318 re-designed for gfx950.
//
// Work unit: one bm-row block of pairs (all of one expert, as align padded them) times one column tile
// of that expert's weight [N, K] (K contiguous). Rows are gathered on the fly (row = pair / topk for the
// gate/up product, pair for the down product); the padding sentinel n_pairs reads as zeros and is never
// stored. Blocks at or past *used exit at once, so the static grid (total / bm blocks) never needs the
// host to read the device.
//
// Two kernel families, one arithmetic:
//  * lds    (bm 64/128, prefill): 4 waves, the block's rows and the weight tile staged through LDS in
//           64-wide K chunks, double buffered, with the next chunk's global loads in flight during the
//           current chunk's MFMAs.
//  * stream (bm 16/32, decode): no LDS; each wave streams its own weight rows from HBM straight into
//           MFMA operand registers, several chunks in flight, and reads the block's few rows from L2.
// Both use the fixed K assignment of common.hpp, so a pair's sums are the same bits whichever kernel
// or tile runs it (the reference's batch-invariance promise, flide/kernels/moe.py:5-8,35-37).
//
// Fused gate/up activation (act != ACT_NONE): the weight tile holds BN/2 gate rows and the BN/2 up
// rows of the same output columns (rows c and c + N/2), each wave holds matching gate and up
// fragments, and the epilogue rounds both to the 16-bit type (as the reference stores gu) before
// act(gate, up) is applied and rounded once. gu is never written to memory.
#include <stdlib.h>

#include "grouped_common.hpp"

// weight loads of the streaming kernels are ordinary loads: they measured faster than non-temporal
// ones on MI355X for this pattern (5.6 vs 4.75 TB/s at the decode shape)
#define FLIDE_WLOAD(p) (*(p))

namespace {
using namespace grouped_detail;

// ---------------------------------------------------------------------------------------------------
// LDS-tiled 16-bit kernel (prefill)
// ---------------------------------------------------------------------------------------------------
template <typename T, typename OutT, int ACT, int BM, int BN, int WAVES_M, int WAVES_N>
__global__ __launch_bounds__(WAVES_M* WAVES_N * 64) void grouped_lds16(GroupArgs p) {
  constexpr int NT = WAVES_M * WAVES_N * 64;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int FM = WM / 16, FN = WN / 16;
  constexpr int CA = (BM * 8 + NT - 1) / NT;  // 16-byte chunks per thread, A tile
  constexpr int CB = (BN * 8 + NT - 1) / NT;  // B tile
  static_assert(ACT == ACT_NONE || FN % 2 == 0, "gated tiles pair gate and up fragments");

  __shared__ __attribute__((aligned(16))) u16 As[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) u16 Bs[2][BN * LDK];
  __shared__ int s_pairs[BM];

  const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63;
  const int pm = blockIdx.x / p.ntn, pn = blockIdx.x % p.ntn;
  if (pm * BM >= *p.used) return;
  const long long e = p.blocks[pm];
  for (int r = tid; r < BM; r += NT) s_pairs[r] = p.rows[pm * BM + r];
  __syncthreads();

  const u16* A = (const u16*)p.a;
  const u16* B = (const u16*)p.w + e * p.sbe;
  const int K = p.K;
  const int half = p.N / 2;

  // global source of each of this thread's chunks
  const u16* a_src[CA];
  int a_dst[CA];
  bool a_ok[CA];
#pragma unroll
  for (int i = 0; i < CA; ++i) {
    int q = tid + i * NT;
    int row = q >> 3, kc = q & 7;
    a_ok[i] = q < BM * 8;
    int pair = a_ok[i] ? s_pairs[row] : p.n_pairs;
    a_ok[i] = a_ok[i] && pair < p.n_pairs;
    long long src = p.by_token ? pair / p.topk : pair;
    a_src[i] = A + (a_ok[i] ? src * p.sa : 0) + kc * 8;
    a_dst[i] = row * LDK + kc * 8;
  }
  const u16* b_src[CB];
  int b_dst[CB];
  bool b_ok[CB];
#pragma unroll
  for (int i = 0; i < CB; ++i) {
    int q = tid + i * NT;
    int row = q >> 3, kc = q & 7;
    bool in = q < BN * 8;
    long long n;
    if constexpr (ACT == ACT_NONE) {
      n = (long long)pn * BN + row;
      b_ok[i] = in && n < p.N;
    } else {
      int c = pn * (BN / 2) + (row < BN / 2 ? row : row - BN / 2);
      b_ok[i] = in && c < half;
      n = row < BN / 2 ? c : c + half;
    }
    b_src[i] = B + (b_ok[i] ? n * p.sbn : 0) + kc * 8;
    b_dst[i] = row * LDK + kc * 8;
  }

  u32x4_t ra[CA], rb[CB];
  auto load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      int kk = k0 + (a_dst[i] % LDK);
      ra[i] = (a_ok[i] && kk < K) ? *(const u32x4_t*)(a_src[i] + k0) : u32x4_t{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      int kk = k0 + (b_dst[i] % LDK);
      rb[i] = (b_ok[i] && kk < K) ? *(const u32x4_t*)(b_src[i] + k0) : u32x4_t{0, 0, 0, 0};
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < CA; ++i)
      if (tid + i * NT < BM * 8) *(u32x4_t*)(&As[buf][a_dst[i]]) = ra[i];
#pragma unroll
    for (int i = 0; i < CB; ++i)
      if (tid + i * NT < BN * 8) *(u32x4_t*)(&Bs[buf][b_dst[i]]) = rb[i];
  };

  const int wm = wave % WAVES_M, wn = wave / WAVES_M;
  const int r = l & 15, g = l >> 4;
  int brow[FN];
#pragma unroll
  for (int fn = 0; fn < FN; ++fn) {
    if constexpr (ACT == ACT_NONE) {
      brow[fn] = wn * WN + fn * 16;
    } else {
      constexpr int H2 = FN / 2;
      brow[fn] = fn < H2 ? wn * (WN / 2) + fn * 16 : BN / 2 + wn * (WN / 2) + (fn - H2) * 16;
    }
  }

  f32x4_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int nk = (K + 63) / 64;
  load(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load((kt + 1) * 64);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      u32x4_t af[FM], bfr[FN];
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
        af[fm] = *(const u32x4_t*)(&As[buf][(wm * WM + fm * 16 + r) * LDK + s * 32 + g * 8]);
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
        bfr[fn] = *(const u32x4_t*)(&Bs[buf][(brow[fn] + r) * LDK + s * 32 + g * 8]);
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) acc[fm][fn] = Mfma16<T>::mma(af[fm], bfr[fn], acc[fm][fn]);
    }
    if (kt + 1 < nk) store(buf ^ 1);
    __syncthreads();
  }

  const float ones[4] = {1.f, 1.f, 1.f, 1.f};
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
    const int row0 = wm * WM + fm * 16;
    if constexpr (ACT == ACT_NONE) {
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const int col = pn * BN + wn * WN + fn * 16 + r;
        store_frag<OutT, ACT, T>(p, s_pairs, row0, col, acc[fm][fn], acc[fm][fn], 1.f, 1.f, ones,
                                 col < p.N);
      }
    } else {
#pragma unroll
      for (int fn = 0; fn < FN / 2; ++fn) {
        const int col = pn * (BN / 2) + wn * (WN / 2) + fn * 16 + r;
        store_frag<OutT, ACT, T>(p, s_pairs, row0, col, acc[fm][fn], acc[fm][fn + FN / 2], 1.f, 1.f,
                                 ones, col < half);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------------
// streaming 16-bit kernel (decode): weights straight from HBM into MFMA operands
// ---------------------------------------------------------------------------------------------------
// Block: FM*16 rows; each of the 4 waves owns NF weight fragments of 16 rows (gated: NF/2 gate and the
// NF/2 matching up fragments). Column tile of the workgroup: 4 * NF * 16 weight rows.
template <typename T, typename OutT, int ACT, int FM, int NF, int U>
__global__ __launch_bounds__(256) void grouped_stream16(GroupArgs p) {
  constexpr int BM = FM * 16;
  constexpr int BNW = 4 * NF * 16;  // weight rows per workgroup
  __shared__ int s_pairs[BM];
  const int tid = threadIdx.x, l = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int pm = blockIdx.x / p.ntn, pn = blockIdx.x % p.ntn;
  // `used` and the block's expert load together; the weight stream starts before the block's pair ids
  // are known, so their latency overlaps the first weight loads
  const int used = *p.used;
  const long long e = p.blocks[pm];
  if (pm * BM >= used) return;

  const int r = l & 15, g = l >> 4;
  const int K = p.K, half = p.N / 2;
  const u16* B = (const u16*)p.w + e * p.sbe;
  const u16* b_src[NF];
  bool b_ok[NF];
  int colv[NF];
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    long long n;
    if constexpr (ACT == ACT_NONE) {
      n = (long long)pn * BNW + (wave * NF + f) * 16 + r;
      b_ok[f] = n < p.N;
      colv[f] = (int)n;
    } else {
      constexpr int H2 = NF / 2;
      int ff = f < H2 ? f : f - H2;
      int c = pn * (BNW / 2) + (wave * H2 + ff) * 16 + r;
      b_ok[f] = c < half;
      n = f < H2 ? c : c + half;
      colv[f] = c;
    }
    b_src[f] = B + (b_ok[f] ? n * p.sbn : 0) + g * 8;
  }
  const int nk = (K + 63) / 64;
  // weight chunks of one group of U 64-wide K chunks: [u][frag][MFMA step]
  auto load_w = [&](int c0, u32x4_t (&bb)[U][NF][2]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = (c0 + u) * 64 + g * 8;
      const bool kin0 = (c0 + u) < nk && k < K, kin1 = (c0 + u) < nk && k + 32 < K;
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        bb[u][f][0] = (b_ok[f] && kin0) ? FLIDE_WLOAD((const u32x4_t*)(b_src[f] + (c0 + u) * 64)) : u32x4_t{0, 0, 0, 0};
        bb[u][f][1] = (b_ok[f] && kin1) ? FLIDE_WLOAD((const u32x4_t*)(b_src[f] + (c0 + u) * 64 + 32))
                                        : u32x4_t{0, 0, 0, 0};
      }
    }
  };
  u32x4_t bb[U][NF][2];
  load_w(0, bb);

  // the block's pair ids: straight from global for the operand rows, through LDS for the epilogue
  const u16* A = (const u16*)p.a;
  const u16* a_src[FM];
  bool a_ok[FM];
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
    const int pair = p.rows[pm * BM + fm * 16 + r];
    a_ok[fm] = pair < p.n_pairs;
    const long long src = p.by_token ? pair / p.topk : pair;
    a_src[fm] = A + (a_ok[fm] ? src * p.sa : 0) + g * 8;
  }
  if (tid < BM) s_pairs[tid] = p.rows[pm * BM + tid];

  f32x4_t acc[FM][NF];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < NF; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int c0 = 0; c0 < nk; c0 += U) {
    u32x4_t aa[U][FM][2];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = (c0 + u) * 64 + g * 8;
      const bool kin0 = (c0 + u) < nk && k < K, kin1 = (c0 + u) < nk && k + 32 < K;
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        aa[u][fm][0] = (a_ok[fm] && kin0) ? *(const u32x4_t*)(a_src[fm] + (c0 + u) * 64) : u32x4_t{0, 0, 0, 0};
        aa[u][fm][1] = (a_ok[fm] && kin1) ? *(const u32x4_t*)(a_src[fm] + (c0 + u) * 64 + 32) : u32x4_t{0, 0, 0, 0};
      }
    }
    // the next group's weights go out before this group's MFMAs
    u32x4_t nb[U][NF][2];
    if (c0 + U < nk) load_w(c0 + U, nb);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
#pragma unroll
          for (int f = 0; f < NF; ++f) acc[fm][f] = Mfma16<T>::mma(aa[u][fm][s], bb[u][f][s], acc[fm][f]);
    if (c0 + U < nk) {
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int f = 0; f < NF; ++f) {
          bb[u][f][0] = nb[u][f][0];
          bb[u][f][1] = nb[u][f][1];
        }
    }
  }
  __syncthreads();   // s_pairs for the epilogue

  const float ones[4] = {1.f, 1.f, 1.f, 1.f};
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
    if constexpr (ACT == ACT_NONE) {
#pragma unroll
      for (int f = 0; f < NF; ++f)
        store_frag<OutT, ACT, T>(p, s_pairs, fm * 16, colv[f], acc[fm][f], acc[fm][f], 1.f, 1.f, ones,
                                 b_ok[f]);
    } else {
#pragma unroll
      for (int f = 0; f < NF / 2; ++f)
        store_frag<OutT, ACT, T>(p, s_pairs, fm * 16, colv[f], acc[fm][f], acc[fm][f + NF / 2], 1.f,
                                 1.f, ones, b_ok[f]);
    }
  }
}

// ---------------------------------------------------------------------------------------------------
// float8 kernels: e4m3 x e4m3 -> float32 with v_mfma_f32_16x16x128_f8f6f4, then * a_scale[row] *
// w_scale[e, col] (* weight). 128-wide K chunks; lane group g holds k = g*32 + [0, 32).
// ---------------------------------------------------------------------------------------------------
template <typename OutT, int ACT, int BM, int BN, int WAVES_M, int WAVES_N>
__global__ __launch_bounds__(WAVES_M* WAVES_N * 64) void grouped_lds8(GroupArgs p) {
  constexpr int NT = WAVES_M * WAVES_N * 64;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int FM = WM / 16, FN = WN / 16;
  constexpr int CA = (BM * 8 + NT - 1) / NT;  // 16-byte chunks per thread (8 per 128-byte row)
  constexpr int CB = (BN * 8 + NT - 1) / NT;
  static_assert(ACT == ACT_NONE || FN % 2 == 0, "gated tiles pair gate and up fragments");

  __shared__ __attribute__((aligned(16))) u8 As[2][BM * LDK8];
  __shared__ __attribute__((aligned(16))) u8 Bs[2][BN * LDK8];
  __shared__ int s_pairs[BM];
  __shared__ float s_ascale[BM];

  const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63;
  const int pm = blockIdx.x / p.ntn, pn = blockIdx.x % p.ntn;
  if (pm * BM >= *p.used) return;
  const long long e = p.blocks[pm];
  for (int rr = tid; rr < BM; rr += NT) {
    int pair = p.rows[pm * BM + rr];
    s_pairs[rr] = pair;
    long long src = p.by_token ? pair / p.topk : pair;
    s_ascale[rr] = pair < p.n_pairs ? p.a_scale[src] : 0.f;
  }
  __syncthreads();

  const u8* A = (const u8*)p.a;
  const u8* B = (const u8*)p.w + e * p.sbe;
  const int K = p.K;
  const int half = p.N / 2;

  const u8* a_src[CA];
  int a_dst[CA];
  bool a_ok[CA];
#pragma unroll
  for (int i = 0; i < CA; ++i) {
    int q = tid + i * NT;
    int row = q >> 3, kc = q & 7;
    a_ok[i] = q < BM * 8;
    int pair = a_ok[i] ? s_pairs[row] : p.n_pairs;
    a_ok[i] = a_ok[i] && pair < p.n_pairs;
    long long src = p.by_token ? pair / p.topk : pair;
    a_src[i] = A + (a_ok[i] ? src * p.sa : 0) + kc * 16;
    a_dst[i] = row * LDK8 + kc * 16;
  }
  const u8* b_src[CB];
  int b_dst[CB];
  bool b_ok[CB];
#pragma unroll
  for (int i = 0; i < CB; ++i) {
    int q = tid + i * NT;
    int row = q >> 3, kc = q & 7;
    bool in = q < BN * 8;
    long long n;
    if constexpr (ACT == ACT_NONE) {
      n = (long long)pn * BN + row;
      b_ok[i] = in && n < p.N;
    } else {
      int c = pn * (BN / 2) + (row < BN / 2 ? row : row - BN / 2);
      b_ok[i] = in && c < half;
      n = row < BN / 2 ? c : c + half;
    }
    b_src[i] = B + (b_ok[i] ? n * p.sbn : 0) + kc * 16;
    b_dst[i] = row * LDK8 + kc * 16;
  }

  u32x4_t ra[CA], rb[CB];
  auto load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      int kk = k0 + (a_dst[i] % LDK8);
      ra[i] = (a_ok[i] && kk < K) ? *(const u32x4_t*)(a_src[i] + k0) : u32x4_t{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      int kk = k0 + (b_dst[i] % LDK8);
      rb[i] = (b_ok[i] && kk < K) ? *(const u32x4_t*)(b_src[i] + k0) : u32x4_t{0, 0, 0, 0};
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < CA; ++i)
      if (tid + i * NT < BM * 8) *(u32x4_t*)(&As[buf][a_dst[i]]) = ra[i];
#pragma unroll
    for (int i = 0; i < CB; ++i)
      if (tid + i * NT < BN * 8) *(u32x4_t*)(&Bs[buf][b_dst[i]]) = rb[i];
  };

  const int wm = wave % WAVES_M, wn = wave / WAVES_M;
  const int r = l & 15, g = l >> 4;
  int brow[FN];
#pragma unroll
  for (int fn = 0; fn < FN; ++fn) {
    if constexpr (ACT == ACT_NONE) {
      brow[fn] = wn * WN + fn * 16;
    } else {
      constexpr int H2 = FN / 2;
      brow[fn] = fn < H2 ? wn * (WN / 2) + fn * 16 : BN / 2 + wn * (WN / 2) + (fn - H2) * 16;
    }
  }

  f32x4_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int nk = (K + 127) / 128;
  load(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load((kt + 1) * 128);
    i32x8_t af[FM], bfr[FN];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const u8* src = &As[buf][(wm * WM + fm * 16 + r) * LDK8 + g * 16];
      u32x4_t lo = *(const u32x4_t*)src, hi = *(const u32x4_t*)(src + 64);
      af[fm] = i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    }
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
      const u8* src = &Bs[buf][(brow[fn] + r) * LDK8 + g * 16];
      u32x4_t lo = *(const u32x4_t*)src, hi = *(const u32x4_t*)(src + 64);
      bfr[fn] = i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    }
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) acc[fm][fn] = mfma_fp8(af[fm], bfr[fn], acc[fm][fn]);
    if (kt + 1 < nk) store(buf ^ 1);
    __syncthreads();
  }

  const float* ws = p.w_scale + e * p.sse;
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
    const int row0 = wm * WM + fm * 16;
    float rs[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) rs[i] = s_ascale[row0 + g * 4 + i];
    if constexpr (ACT == ACT_NONE) {
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const int col = pn * BN + wn * WN + fn * 16 + r;
        const bool ok = col < p.N;
        store_frag<OutT, ACT, typename OutRound<OutT>::type>(p, s_pairs, row0, col, acc[fm][fn], acc[fm][fn],
                                      ok ? ws[col] : 0.f, 0.f, rs, ok);
      }
    } else {
#pragma unroll
      for (int fn = 0; fn < FN / 2; ++fn) {
        const int col = pn * (BN / 2) + wn * (WN / 2) + fn * 16 + r;
        const bool ok = col < half;
        store_frag<OutT, ACT, typename OutRound<OutT>::type>(p, s_pairs, row0, col, acc[fm][fn], acc[fm][fn + FN / 2],
                                      ok ? ws[col] : 0.f, ok ? ws[col + half] : 0.f, rs, ok);
      }
    }
  }
}

template <typename OutT, int ACT, int FM, int NF, int U>
__global__ __launch_bounds__(256) void grouped_stream8(GroupArgs p) {
  constexpr int BM = FM * 16;
  constexpr int BNW = 4 * NF * 16;
  __shared__ int s_pairs[BM];
  __shared__ float s_ascale[BM];
  const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63;
  const int pm = blockIdx.x / p.ntn, pn = blockIdx.x % p.ntn;
  if (pm * BM >= *p.used) return;
  const long long e = p.blocks[pm];
  if (tid < BM) {
    int pair = p.rows[pm * BM + tid];
    s_pairs[tid] = pair;
    long long src = p.by_token ? pair / p.topk : pair;
    s_ascale[tid] = pair < p.n_pairs ? p.a_scale[src] : 0.f;
  }
  __syncthreads();

  const int r = l & 15, g = l >> 4;
  const int K = p.K, half = p.N / 2;
  const u8* A = (const u8*)p.a;
  const u8* B = (const u8*)p.w + e * p.sbe;

  const u8* a_src[FM];
  bool a_ok[FM];
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
    int pair = s_pairs[fm * 16 + r];
    a_ok[fm] = pair < p.n_pairs;
    long long src = p.by_token ? pair / p.topk : pair;
    a_src[fm] = A + (a_ok[fm] ? src * p.sa : 0) + g * 16;
  }
  const u8* b_src[NF];
  bool b_ok[NF];
  int colv[NF];
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    long long n;
    if constexpr (ACT == ACT_NONE) {
      n = (long long)pn * BNW + (wave * NF + f) * 16 + r;
      b_ok[f] = n < p.N;
      colv[f] = (int)n;
    } else {
      constexpr int H2 = NF / 2;
      int ff = f < H2 ? f : f - H2;
      int c = pn * (BNW / 2) + (wave * H2 + ff) * 16 + r;
      b_ok[f] = c < half;
      n = f < H2 ? c : c + half;
      colv[f] = c;
    }
    b_src[f] = B + (b_ok[f] ? n * p.sbn : 0) + g * 16;
  }

  f32x4_t acc[FM][NF];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < NF; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int nk = (K + 127) / 128;
  for (int c0 = 0; c0 < nk; c0 += U) {
    u32x4_t bb[U][NF][2], aa[U][FM][2];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = (c0 + u) * 128 + g * 16;
      const bool kin0 = (c0 + u) < nk && k < K, kin1 = (c0 + u) < nk && k + 64 < K;
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        bb[u][f][0] = (b_ok[f] && kin0) ? __builtin_nontemporal_load((const u32x4_t*)(b_src[f] + (c0 + u) * 128))
                                        : u32x4_t{0, 0, 0, 0};
        bb[u][f][1] = (b_ok[f] && kin1) ? __builtin_nontemporal_load((const u32x4_t*)(b_src[f] + (c0 + u) * 128 + 64))
                                        : u32x4_t{0, 0, 0, 0};
      }
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        aa[u][fm][0] = (a_ok[fm] && kin0) ? *(const u32x4_t*)(a_src[fm] + (c0 + u) * 128) : u32x4_t{0, 0, 0, 0};
        aa[u][fm][1] = (a_ok[fm] && kin1) ? *(const u32x4_t*)(a_src[fm] + (c0 + u) * 128 + 64) : u32x4_t{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        i32x8_t av = i32x8_t{(int)aa[u][fm][0][0], (int)aa[u][fm][0][1], (int)aa[u][fm][0][2], (int)aa[u][fm][0][3],
                             (int)aa[u][fm][1][0], (int)aa[u][fm][1][1], (int)aa[u][fm][1][2], (int)aa[u][fm][1][3]};
#pragma unroll
        for (int f = 0; f < NF; ++f) {
          i32x8_t bv = i32x8_t{(int)bb[u][f][0][0], (int)bb[u][f][0][1], (int)bb[u][f][0][2], (int)bb[u][f][0][3],
                               (int)bb[u][f][1][0], (int)bb[u][f][1][1], (int)bb[u][f][1][2], (int)bb[u][f][1][3]};
          acc[fm][f] = mfma_fp8(av, bv, acc[fm][f]);
        }
      }
  }

  const float* ws = p.w_scale + e * p.sse;
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
    float rs[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) rs[i] = s_ascale[fm * 16 + g * 4 + i];
    if constexpr (ACT == ACT_NONE) {
#pragma unroll
      for (int f = 0; f < NF; ++f)
        store_frag<OutT, ACT, typename OutRound<OutT>::type>(p, s_pairs, fm * 16, colv[f], acc[fm][f], acc[fm][f],
                                      b_ok[f] ? ws[colv[f]] : 0.f, 0.f, rs, b_ok[f]);
    } else {
#pragma unroll
      for (int f = 0; f < NF / 2; ++f)
        store_frag<OutT, ACT, typename OutRound<OutT>::type>(p, s_pairs, fm * 16, colv[f], acc[fm][f], acc[fm][f + NF / 2],
                                      b_ok[f] ? ws[colv[f]] : 0.f, b_ok[f] ? ws[colv[f] + half] : 0.f,
                                      rs, b_ok[f]);
    }
  }
}

// ---------------------------------------------------------------------------------------------------
// dispatch
// ---------------------------------------------------------------------------------------------------
// Compiled tiles: bm 32/64/128/256 -> direct-to-LDS kernels (grouped_dma.hip); bm 16, and bm 32 when K is
// too short for their ring -> stream kernels (4 waves x NF fragments); bm 64/128/256 with K too short
// for the ring -> the register-staged LDS kernels above.
constexpr int STREAM_NF = 2;       // 16-row weight fragments per wave (gated products)
constexpr int STREAM_NF_DOWN = 2;  // ... and for the plain (down) products
constexpr int STREAM_U = 4;        // K chunks in flight per wave

template <typename T, typename OutT, int ACT>
int launch16(GroupArgs& p, int bm, hipStream_t st) {
  dim3 block(256);
  if (bm == 32) {   // the direct-to-LDS kernel streams whole lines (grouped_dma.hip)
    const int out_dtype = std::is_same<OutT, float>::value ? FLIDE_F32
                          : std::is_same<OutT, Bf16Out>::value ? FLIDE_BF16 : FLIDE_F16;
    const int rc = dma_dispatch16(p, std::is_same<T, __bf16>::value, out_dtype, ACT, bm, st);
    if (rc != FLIDE_MOE_ERR_TILE) return rc;   // else K is too short for the ring: the stream kernel
  }
  if (bm == 16 || bm == 32) {
    constexpr int NF = ACT == ACT_NONE ? STREAM_NF_DOWN : STREAM_NF;
    constexpr int BNW = 4 * NF * 16;
    const int cols = ACT == ACT_NONE ? p.N : p.N / 2;
    const int per = ACT == ACT_NONE ? BNW : BNW / 2;
    p.ntn = (cols + per - 1) / per;
    dim3 grid(p.nbm * p.ntn);
    if (bm == 16) grouped_stream16<T, OutT, ACT, 1, NF, STREAM_U><<<grid, block, 0, st>>>(p);
    else grouped_stream16<T, OutT, ACT, 2, NF, STREAM_U><<<grid, block, 0, st>>>(p);
    return FLIDE_MOE_OK;
  }
  if (bm == 64 || bm == 128 || bm == 256) {
    const int out_dtype = std::is_same<OutT, float>::value ? FLIDE_F32
                          : std::is_same<OutT, Bf16Out>::value ? FLIDE_BF16 : FLIDE_F16;
    const int rc = dma_dispatch16(p, std::is_same<T, __bf16>::value, out_dtype, ACT, bm, st);
    if (rc != FLIDE_MOE_ERR_TILE) return rc;   // else K is too short for the ring: the LDS kernel below
  }
  if (bm == 64 || bm == 128 || bm == 256) {
    constexpr int BN = 128;
    const int cols = ACT == ACT_NONE ? p.N : p.N / 2;
    const int per = ACT == ACT_NONE ? BN : BN / 2;
    p.ntn = (cols + per - 1) / per;
    dim3 grid(p.nbm * p.ntn);
    if (bm == 64) grouped_lds16<T, OutT, ACT, 64, BN, 2, 2><<<grid, block, 0, st>>>(p);
    else if (bm == 128) grouped_lds16<T, OutT, ACT, 128, BN, 2, 2><<<grid, block, 0, st>>>(p);
    else grouped_lds16<T, OutT, ACT, 256, BN, 2, 2><<<grid, block, 0, st>>>(p);
    return FLIDE_MOE_OK;
  }
  return FLIDE_MOE_ERR_TILE;
}

template <typename OutT, int ACT>
int launch8(GroupArgs& p, int bm, hipStream_t st) {
  dim3 block(256);
  if (bm == 32) {
    const int out_dtype = std::is_same<OutT, float>::value ? FLIDE_F32
                          : std::is_same<OutT, Bf16Out>::value ? FLIDE_BF16 : FLIDE_F16;
    const int rc = dma_dispatch8(p, out_dtype, ACT, bm, st);
    if (rc != FLIDE_MOE_ERR_TILE) return rc;   // else K is too short for the ring: the stream kernel
  }
  if (bm == 16 || bm == 32) {
    constexpr int NF = ACT == ACT_NONE ? STREAM_NF_DOWN : STREAM_NF;
    constexpr int BNW = 4 * NF * 16;
    const int cols = ACT == ACT_NONE ? p.N : p.N / 2;
    const int per = ACT == ACT_NONE ? BNW : BNW / 2;
    p.ntn = (cols + per - 1) / per;
    dim3 grid(p.nbm * p.ntn);
    if (bm == 16) grouped_stream8<OutT, ACT, 1, NF, STREAM_U><<<grid, block, 0, st>>>(p);
    else grouped_stream8<OutT, ACT, 2, NF, STREAM_U><<<grid, block, 0, st>>>(p);
    return FLIDE_MOE_OK;
  }
  if (bm == 64 || bm == 128 || bm == 256) {
    const int out_dtype = std::is_same<OutT, float>::value ? FLIDE_F32
                          : std::is_same<OutT, Bf16Out>::value ? FLIDE_BF16 : FLIDE_F16;
    const int rc = dma_dispatch8(p, out_dtype, ACT, bm, st);
    if (rc != FLIDE_MOE_ERR_TILE) return rc;   // else K is too short for the ring: the LDS kernel below
  }
  if (bm == 64 || bm == 128 || bm == 256) {
    constexpr int BN = 128;
    const int cols = ACT == ACT_NONE ? p.N : p.N / 2;
    const int per = ACT == ACT_NONE ? BN : BN / 2;
    p.ntn = (cols + per - 1) / per;
    dim3 grid(p.nbm * p.ntn);
    if (bm == 64) grouped_lds8<OutT, ACT, 64, BN, 2, 2><<<grid, block, 0, st>>>(p);
    else if (bm == 128) grouped_lds8<OutT, ACT, 128, BN, 2, 2><<<grid, block, 0, st>>>(p);
    else grouped_lds8<OutT, ACT, 256, BN, 2, 2><<<grid, block, 0, st>>>(p);
    return FLIDE_MOE_OK;
  }
  return FLIDE_MOE_ERR_TILE;
}

template <typename T>
int dispatch16(GroupArgs& p, int out_dtype, int act, int bm, hipStream_t st) {
  const bool out16 = (out_dtype == FLIDE_BF16 && std::is_same<T, __bf16>::value) ||
                     (out_dtype == FLIDE_F16 && std::is_same<T, _Float16>::value);
  typedef typename std::conditional<std::is_same<T, __bf16>::value, Bf16Out, F16Out>::type O16;
  if (act == ACT_NONE) {
    if (out_dtype == FLIDE_F32) return launch16<T, float, ACT_NONE>(p, bm, st);
    if (out16) return launch16<T, O16, ACT_NONE>(p, bm, st);
    return FLIDE_MOE_ERR_ARG;
  }
  if (!out16) return FLIDE_MOE_ERR_ARG;
  if (act == ACT_GEGLU) return launch16<T, O16, ACT_GEGLU>(p, bm, st);
  if (act == ACT_SWIGLU) return launch16<T, O16, ACT_SWIGLU>(p, bm, st);
  return FLIDE_MOE_ERR_ARG;
}

int dispatch8(GroupArgs& p, int out_dtype, int act, int bm, hipStream_t st) {
  if (act == ACT_NONE) {
    if (out_dtype == FLIDE_F32) return launch8<float, ACT_NONE>(p, bm, st);
    if (out_dtype == FLIDE_BF16) return launch8<Bf16Out, ACT_NONE>(p, bm, st);
    if (out_dtype == FLIDE_F16) return launch8<F16Out, ACT_NONE>(p, bm, st);
    return FLIDE_MOE_ERR_ARG;
  }
  if (out_dtype == FLIDE_BF16) {
    if (act == ACT_GEGLU) return launch8<Bf16Out, ACT_GEGLU>(p, bm, st);
    if (act == ACT_SWIGLU) return launch8<Bf16Out, ACT_SWIGLU>(p, bm, st);
  }
  if (out_dtype == FLIDE_F16) {
    if (act == ACT_GEGLU) return launch8<F16Out, ACT_GEGLU>(p, bm, st);
    if (act == ACT_SWIGLU) return launch8<F16Out, ACT_SWIGLU>(p, bm, st);
  }
  return FLIDE_MOE_ERR_ARG;
}

// The prefill and decode kernels address the gathered activation rows and one expert's weight rows as
// 32-bit byte offsets from uniform 64-bit bases: the last row a pair can name (row max_row of a, row
// N - 1 of an expert) must end below 4 GiB from its base.
bool offsets_fit_32(long long sa, long long max_row, long long sbn, int N, int K, int eb) {
  const long long lim = 0xFFFFFFFFLL;
  return (max_row * sa + K) * eb <= lim && ((long long)(N - 1) * sbn + K) * eb <= lim;
}

}  // namespace

extern "C" int flide_moe_grouped(const void* a, long long sa, int a_dtype, const void* w,
                                 long long sbe, long long sbn, int N, int K, void* out,
                                 long long sc, int out_dtype, const float* weights,
                                 const int* rows, const int* blocks, const int* used, int n_pairs,
                                 int nbm, int topk, int by_token, int act, int bm, int bn,
                                 flide_stream_t stream) {
  (void)bn;
  if (N <= 0 || K <= 0 || K % 8 || sa % 8 || sbn % 8 || sbe % 8 || n_pairs < 0 || nbm < 0 ||
      topk <= 0)
    return FLIDE_MOE_ERR_ARG;
  if (act != ACT_NONE && N % 2) return FLIDE_MOE_ERR_ARG;
  if (((uintptr_t)a | (uintptr_t)w) & 15) return FLIDE_MOE_ERR_ARG;
  if (nbm == 0 || n_pairs == 0) return FLIDE_MOE_OK;
  if (!offsets_fit_32(sa, by_token ? (n_pairs - 1) / topk : n_pairs - 1, sbn, N, K, 2))
    return FLIDE_MOE_ERR_ARG;
  GroupArgs p{};
  p.a = a; p.sa = sa; p.w = w; p.sbe = sbe; p.sbn = sbn;
  p.N = N; p.K = K; p.out = out; p.sc = sc; p.weights = weights;
  p.rows = rows; p.blocks = blocks; p.used = used;
  p.n_pairs = n_pairs; p.nbm = nbm; p.topk = topk; p.by_token = by_token;
  hipStream_t st = (hipStream_t)stream;
  int rc;
  if (a_dtype == FLIDE_BF16) rc = dispatch16<__bf16>(p, out_dtype, act, bm, st);
  else if (a_dtype == FLIDE_F16) rc = dispatch16<_Float16>(p, out_dtype, act, bm, st);
  else return FLIDE_MOE_ERR_ARG;
  if (rc) return rc;
  FLIDE_CHECK_LAUNCH();
  return FLIDE_MOE_OK;
}

extern "C" int flide_moe_grouped_fp8(const void* a, long long sa, const float* a_scale,
                                     const void* w, long long sbe, long long sbn,
                                     const float* w_scale, long long sse, int N, int K, void* out,
                                     long long sc, int out_dtype, const float* weights,
                                     const int* rows, const int* blocks, const int* used,
                                     int n_pairs, int nbm, int topk, int by_token, int act, int bm,
                                     int bn, flide_stream_t stream) {
  (void)bn;
  if (N <= 0 || K <= 0 || K % 16 || sa % 16 || sbn % 16 || sbe % 16 || n_pairs < 0 || nbm < 0 ||
      topk <= 0 || !a_scale || !w_scale)
    return FLIDE_MOE_ERR_ARG;
  if (act != ACT_NONE && N % 2) return FLIDE_MOE_ERR_ARG;
  if (((uintptr_t)a | (uintptr_t)w) & 15) return FLIDE_MOE_ERR_ARG;
  if (nbm == 0 || n_pairs == 0) return FLIDE_MOE_OK;
  if (!offsets_fit_32(sa, by_token ? (n_pairs - 1) / topk : n_pairs - 1, sbn, N, K, 1))
    return FLIDE_MOE_ERR_ARG;
  GroupArgs p{};
  p.a = a; p.sa = sa; p.w = w; p.sbe = sbe; p.sbn = sbn;
  p.a_scale = a_scale; p.w_scale = w_scale; p.sse = sse;
  p.N = N; p.K = K; p.out = out; p.sc = sc; p.weights = weights;
  p.rows = rows; p.blocks = blocks; p.used = used;
  p.n_pairs = n_pairs; p.nbm = nbm; p.topk = topk; p.by_token = by_token;
  int rc = dispatch8(p, out_dtype, act, bm, (hipStream_t)stream);
  if (rc) return rc;
  FLIDE_CHECK_LAUNCH();
  return FLIDE_MOE_OK;
}
