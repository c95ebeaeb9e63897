// The per-row float8 quantizer of 16-bit rows, one wave per row (flide/kernels/fp8.py:29-53): s = max(amax,
// 1e-12) / 448 and the row's e4m3fn bytes. Shared by rowwise.hip (quantize_rows) and align.hip (the experts
// call's placement launch, which quantizes the token rows in its spare workgroups).
#pragma once
#include "common.hpp"

namespace quant {

// The row's pieces (already in registers) to e4m3 bytes.
template <int NV, bool BF16, bool FINITE>
FLIDE_DEV void quantize_pieces(const uint4 (&raw)[NV], int l, int nv, float sc, uint2* __restrict__ qr) {
  const float rinv = 1.0f / sc, nrinv = -rinv;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int c = l + v * 64;
    if (c >= nv) continue;
    qr[c] = quantize_piece8<BF16, FINITE>(raw[v], sc, rinv, nrinv);
  }
}

// Row `row` of x (16-bit, K % 8 == 0, K <= NV * 512) by the calling wave: the row is loaded once in 16-byte
// pieces and kept in registers between the amax and the quantization; each lane stores 8 quantized bytes at
// a time. The same bytes as the per-element kernel (its true float32 division, made here by div_markstein,
// or by the division for a row holding an inf).
template <int NV, bool BF16>
FLIDE_DEV void quantize_row16(const u16* __restrict__ x, long long sx, int K, long long row, u8* __restrict__ q,
                              long long sq, float* __restrict__ s) {
  const int l = threadIdx.x & 63;
  const int nv = K / 8;
  const uint4* xr = (const uint4*)(x + row * sx);
  uint4 raw[NV];
  float amax = 0.f;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int c = l + v * 64;
    raw[v] = c < nv ? xr[c] : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int v = 0; v < NV; ++v) amax = piece8_amax<BF16>(raw[v], amax);
  // every lane holds the row's amax after the reduction; taking lane 0's makes the branch below uniform
  amax = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(wave_max(amax))));
  const float sc = fmaxf(amax, 1e-12f) * (1.0f / 448.0f);
  if (l == 0) s[row] = sc;
  uint2* qr = (uint2*)(q + row * sq);
  if (sc < INFINITY)
    quantize_pieces<NV, BF16, true>(raw, l, nv, sc, qr);
  else
    quantize_pieces<NV, BF16, false>(raw, l, nv, sc, qr);
}

// Whether quantize_row16 takes these rows: 16-bit, whole 16-byte pieces, at most 16 pieces per lane.
inline bool row16_ok(const void* x, long long sx, int K, int x_dtype, const void* q, long long sq) {
  return (x_dtype == FLIDE_BF16 || x_dtype == FLIDE_F16) && K % 8 == 0 && K <= 16 * 512 && sx % 8 == 0 &&
         sq % 8 == 0 && !((uintptr_t)x & 15) && !((uintptr_t)q & 7);
}

// quantize_row16's NV for K: 16-byte pieces per lane, rounded up to 1, 2, 4, 8 or 16
inline int row16_nv(int K) {
  const int per_lane = (K / 8 + 63) / 64;
  return per_lane <= 1 ? 1 : per_lane <= 2 ? 2 : per_lane <= 4 ? 4 : per_lane <= 8 ? 8 : 16;
}

}  // namespace quant
