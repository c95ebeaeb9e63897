// Pieces shared by the grouped-product kernels: the argument block, output conversions and the
// epilogue that turns MFMA accumulators into stored rows (optionally through the fused activation).
#pragma once
#include <type_traits>

#include "common.hpp"

namespace grouped_detail {

constexpr int LDK = 64 + 8;      // LDS row pitch (u16) for the 16-bit kernels: 144 bytes
constexpr int LDK8 = 128 + 16;   // LDS row pitch (bytes) for the float8 kernels

template <typename OutT> FLIDE_DEV OutT cvt_out(float v);
template <> FLIDE_DEV float cvt_out<float>(float v) { return v; }

struct Bf16Out { u16 v; };
struct F16Out { u16 v; };

template <typename OutT> struct OutTraits;
template <> struct OutTraits<float> {
  typedef float storage;
  static FLIDE_DEV float conv(float v) { return v; }
  static FLIDE_DEV float round16(float v) { return v; }
};
template <> struct OutTraits<Bf16Out> {
  typedef u16 storage;
  static FLIDE_DEV u16 conv(float v) { return f32_to_bf16(v); }
};
template <> struct OutTraits<F16Out> {
  typedef u16 storage;
  static FLIDE_DEV u16 conv(float v) { return f32_to_f16(v); }
};

// rounding of gu to the activation dtype before the fused activation
template <typename T> FLIDE_DEV float round_in(float v);
template <> FLIDE_DEV float round_in<__bf16>(float v) { return bf16_to_f32(f32_to_bf16(v)); }
template <> FLIDE_DEV float round_in<_Float16>(float v) { return f16_to_f32(f32_to_f16(v)); }

struct GroupArgs {
  const void* a;       // activations [*, K]
  long long sa;
  const void* w;       // weights [E, N, K]
  long long sbe, sbn;
  const float* a_scale;  // fp8: per-row scales of a
  const float* w_scale;  // fp8: [E, N]
  long long sse;
  int N, K;
  void* out;
  long long sc;
  const float* weights;
  const int* rows;
  const int* blocks;
  const int* used;
  int n_pairs, nbm, topk, by_token;
  int ntn;             // column tiles
  int pack_f32;        // float outputs with out and sc 4-float aligned: store_frag_f32x4 may be used
};

// ---------------------------------------------------------------------------------------------------
// shared epilogue: one 16x16 fragment pair (or single fragment) of a block
// ---------------------------------------------------------------------------------------------------
// Row of the tile that output register i of lane l holds: (l / 16) * 4 + i; column: l % 16.
// s_wt: the tile rows' routing weights staged in LDS (p.weights[pair], 1 for padding), or null to read
// p.weights directly.
template <typename OutT, int ACT, typename T>
FLIDE_DEV void store_frag(const GroupArgs& p, const int* s_pairs, int row0, int col, const f32x4_t& g,
                          const f32x4_t& u, float colscale_g, float colscale_u, const float* rowscale,
                          bool col_ok, const float* s_wt = nullptr) {
  typedef typename OutTraits<OutT>::storage S;
  const int l = lane_id();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int tr = row0 + (l >> 4) * 4 + i;
    const int pair = s_pairs[tr];
    if (pair >= p.n_pairs || !col_ok) continue;
    float v;
    if constexpr (ACT == ACT_NONE) {
      v = g[i] * rowscale[i] * colscale_g;
      if (p.weights) v *= s_wt ? s_wt[tr] : p.weights[pair];
    } else {
      float gg = round_in<T>(g[i] * rowscale[i] * colscale_g);
      float uu = round_in<T>(u[i] * rowscale[i] * colscale_u);
      v = act_f32<ACT>(gg, uu);
      if (p.weights) v *= p.weights[pair];
    }
    ((S*)p.out)[(long long)pair * p.sc + col] = OutTraits<OutT>::conv(v);
  }
}

// 4 x 4 transpose across the lanes of each quad (lanes 4q .. 4q + 3), for wide epilogue stores. On
// entry lane L holds v[i] = M[i][L & 3] of its quad's 4 x 4 block (in an MFMA 16 x 16 fragment: rows
// (L / 16) * 4 + i, column L % 16); on exit it holds v[j] = M[L & 3][j], 4 consecutive columns of one
// row. Two DPP quad permutations: lanes L and L ^ 1 trade the rows of the other parity, then lanes L
// and L ^ 2 trade the halves of the row the other one keeps. Every lane of the wave must be active.
template <int CTRL> FLIDE_DEV float dpp_quad_perm(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
FLIDE_DEV void quad_transpose(float v[4]) {
  const int L = lane_id();
  const bool b = L & 1, h = (L >> 1) & 1;
  // lanes L, L ^ 1 (quad_perm [1, 0, 3, 2]): keep rows b and b + 2, send rows 1 - b and 3 - b
  const float ra = dpp_quad_perm<0xB1>(b ? v[0] : v[1]);
  const float rb = dpp_quad_perm<0xB1>(b ? v[2] : v[3]);
  const float r0[2] = {b ? ra : v[0], b ? v[1] : ra};   // row b, quad columns (L & 2) + 0, 1
  const float r2[2] = {b ? rb : v[2], b ? v[3] : rb};   // row b + 2
  // lanes L, L ^ 2 (quad_perm [2, 3, 0, 1]): keep row b + 2h, send row b + 2(1 - h)
  const float k0 = h ? r2[0] : r0[0], k1 = h ? r2[1] : r0[1];
  const float q0 = dpp_quad_perm<0x4E>(h ? r0[0] : r2[0]);
  const float q1 = dpp_quad_perm<0x4E>(h ? r0[1] : r2[1]);
  v[0] = h ? q0 : k0;
  v[1] = h ? q1 : k1;
  v[2] = h ? k0 : q0;
  v[3] = h ? k1 : q1;
}

// Plain-product fragment with float outputs, stored 4 columns per lane (one 16-byte store per lane
// and fragment instead of four 4-byte ones): the same values as store_frag<float, ACT_NONE>, computed
// in the same order before the transpose. Needs out and sc 4-float aligned (GroupArgs::pack_f32).
// Measured on the 16-bit down product, which is bound by the vector memory pipe: 582 -> 503 us at
// 8192 tokens, 1147 -> 980 us at 16384 (with 16-bit outputs, 8-byte stores measured slower).
FLIDE_DEV void store_frag_f32x4(const GroupArgs& p, const int* s_pairs, const float* s_wt, int row0,
                                int colbase, const f32x4_t& acc, const float* rowscale, float colscale) {
  const int l = lane_id();
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[i] = acc[i] * rowscale[i] * colscale;
    if (p.weights) v[i] *= s_wt[row0 + (l >> 4) * 4 + i];
  }
  quad_transpose(v);
  const int pair = s_pairs[row0 + (l >> 4) * 4 + (l & 3)];
  const int col0 = colbase + (l & 12);
  if (pair >= p.n_pairs || col0 >= p.N) return;
  float* o = (float*)p.out + (long long)pair * p.sc + col0;
  if (col0 + 4 <= p.N) {
    *(f32x4_t*)o = f32x4_t{v[0], v[1], v[2], v[3]};
  } else {
#pragma unroll
    for (int j = 0; j < 3; ++j)
      if (col0 + j < p.N) o[j] = v[j];
  }
}

// rounding type of gu before a fused activation, from the output type
template <typename OutT> struct OutRound { typedef __bf16 type; };
template <> struct OutRound<F16Out> { typedef _Float16 type; };

// direct-to-LDS kernels for the 64/128-row tiles (grouped_dma.hip)
int dma_dispatch16(GroupArgs& p, bool is_bf16, int out_dtype, int act, int bm, hipStream_t st);
int dma_dispatch8(GroupArgs& p, int out_dtype, int act, int bm, hipStream_t st);

}  // namespace grouped_detail
