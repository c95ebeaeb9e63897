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
};

// ---------------------------------------------------------------------------------------------------
// shared epilogue: one 16x16 fragment pair (or single fragment) of a block
// ---------------------------------------------------------------------------------------------------
// Row of the tile that output register i of lane l holds: (l / 16) * 4 + i; column: l % 16.
template <typename OutT, int ACT, typename T>
FLIDE_DEV void store_frag(const GroupArgs& p, const int* s_pairs, int row0, int col, const f32x4_t& g,
                          const f32x4_t& u, float colscale_g, float colscale_u, const float* rowscale,
                          bool col_ok) {
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
      if (p.weights) v *= p.weights[pair];
    } else {
      float gg = round_in<T>(g[i] * rowscale[i] * colscale_g);
      float uu = round_in<T>(u[i] * rowscale[i] * colscale_u);
      v = act_f32<ACT>(gg, uu);
      if (p.weights) v *= p.weights[pair];
    }
    ((S*)p.out)[(long long)pair * p.sc + col] = OutTraits<OutT>::conv(v);
  }
}

// rounding type of gu before a fused activation, from the output type
template <typename OutT> struct OutRound { typedef __bf16 type; };
template <> struct OutRound<F16Out> { typedef _Float16 type; };

// direct-to-LDS kernels for the 64/128-row tiles (grouped_dma.hip)
int dma_dispatch16(GroupArgs& p, bool is_bf16, int out_dtype, int act, int bm, hipStream_t st);
int dma_dispatch8(GroupArgs& p, int out_dtype, int act, int bm, hipStream_t st);

}  // namespace grouped_detail
