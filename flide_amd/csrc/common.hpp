// Shared device helpers for the MoE kernels: number formats, wave64 reductions and the CDNA4 MFMA
// fragments every grouped product uses. gfx950 only.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/flide_moe.h"

typedef uint16_t u16;
typedef uint8_t u8;
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

#define FLIDE_DEV __device__ __forceinline__

// ---------------------------------------------------------------------------------------------------
// number formats
// ---------------------------------------------------------------------------------------------------
FLIDE_DEV float bf16_to_f32(u16 v) { return __uint_as_float((uint32_t)v << 16); }

// float32 -> bfloat16 bits, round to nearest even; NaN stays a quiet NaN. A __bf16 conversion compiles
// to gfx950's v_cvt_pk_bf16_f32 (one instruction, two values when the compiler pairs them), which was
// checked on the GPU against the integer form, (u + 0x7fff + lsb) >> 16 and (u >> 16) | 0x40 for NaN,
// over all 2^32 inputs: identical, NaN payloads and subnormals included. The integer form with an early
// return for NaN compiled to exec-mask branches around every conversion of an epilogue.
FLIDE_DEV u16 f32_to_bf16(float f) { return __builtin_bit_cast(u16, (__bf16)f); }

FLIDE_DEV float f16_to_f32(u16 v) { return (float)__builtin_bit_cast(_Float16, v); }
FLIDE_DEV u16 f32_to_f16(float f) { return __builtin_bit_cast(u16, (_Float16)f); }

FLIDE_DEV float bf16_round(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// float32 with |x| <= 448 -> OCP e4m3fn byte (S EEEE MMM, bias 7), round to nearest even. Normal
// numbers keep 3 mantissa bits; below 2^-6 the quantum is 2^-9 (subnormals). Inputs above 448 in
// magnitude saturate to 448 (callers clamp first, as flide/kernels/fp8.py:42 does).
FLIDE_DEV u8 f32_to_e4m3fn(float x) {
  uint32_t u = __float_as_uint(x);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (u8)(sign | 0x7fu);           // NaN
  if (a >= 0x43e00000u) return (u8)(sign | 0x7eu);          // >= 448: saturate
  int e = (int)(a >> 23) - 127;                             // unbiased exponent of |x|
  if (e < -6) {
    // subnormal range of e4m3fn: value = m * 2^-9, m in [0, 8]; 8 means the smallest normal 2^-6
    float q = __uint_as_float(a) * 512.0f;                  // exact scaling by 2^9
    float r = __builtin_rintf(q);                           // ties to even (default rounding mode)
    uint32_t m = (uint32_t)r;
    return (u8)(sign | m);                                  // m == 8 encodes exponent field 1, mantissa 0
  }
  // normal: keep 3 mantissa bits of the float32 mantissa with round to nearest even
  uint32_t mant = a & 0x7fffffu;
  uint32_t lsb = (mant >> 20) & 1u;
  uint32_t rounded = a + 0x7ffffu + lsb;                    // may carry into the exponent
  int e2 = (int)(rounded >> 23) - 127;
  uint32_t m3 = (rounded >> 20) & 7u;
  uint32_t code = ((uint32_t)(e2 + 7) << 3) | m3;
  if (code > 0x7eu) code = 0x7eu;
  return (u8)(sign | code);
}

FLIDE_DEV float e4m3fn_to_f32(u8 c) {
  uint32_t s = (c & 0x80u) << 24;
  uint32_t e = (c >> 3) & 0xfu;
  uint32_t m = c & 7u;
  if ((c & 0x7fu) == 0x7fu) return __uint_as_float(0x7fc00000u | s);
  if (e == 0) return __uint_as_float(s) + (s ? -1.0f : 1.0f) * (float)m * 0.001953125f;
  return __uint_as_float(s | ((e + 120u) << 23) | (m << 20));
}

// x / sc with the bits of the correctly rounded float32 division, in three operations instead of the
// division's ten: q0 = x * (1/sc) is within about an ulp of the quotient, and one correction from the
// exact residual x - q0*sc (an fma) rounds to the correctly rounded quotient (Markstein's theorem for a
// correctly rounded reciprocal and a faithful first quotient). The residual is x - q0*sc negated so that
// x = -0 keeps its sign (nrinv = -1/sc). For 16-bit x and the scales the quantiser makes (sc from a
// 16-bit amax) the result was compared with the division on every (x, amax) pair of bfloat16 and of
// float16: identical wherever |x / sc| > 2^-11, and elsewhere the same sign (both encode to +-0 in
// e4m3). sc must be finite: an inf in the row makes sc inf and the residual NaN, which the caller handles
// with the division.
FLIDE_DEV float div_markstein(float x, float sc, float rinv, float nrinv) {
  const float q0 = x * rinv;
  return __builtin_fmaf(__builtin_fmaf(q0, sc, -x), nrinv, q0);
}

// One 16-byte piece of a 16-bit row (8 values, bf16 or f16) quantized by the row's scale sc: x / sc
// (div_markstein when sc is finite, else the division), clamped to +-448, rounded to e4m3fn bytes by
// gfx950's packed conversion (round to nearest even; on clamped inputs it gives f32_to_e4m3fn's bytes,
// checked on every code, every tie and its neighbours). rinv = 1 / sc, nrinv = -rinv.
template <bool BF16, bool FINITE>
FLIDE_DEV uint2 quantize_piece8(const uint4& raw, float sc, float rinv, float nrinv) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
  float t[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const u16 h = (i & 1) ? (u16)(w[i >> 1] >> 16) : (u16)(w[i >> 1] & 0xffff);
    const float xv = BF16 ? bf16_to_f32(h) : f16_to_f32(h);
    t[i] = FINITE ? div_markstein(xv, sc, rinv, nrinv) : xv / sc;
    t[i] = fminf(fmaxf(t[i], -448.0f), 448.0f);
  }
  uint32_t lo = __builtin_amdgcn_cvt_pk_fp8_f32(t[0], t[1], 0u, false);
  lo = __builtin_amdgcn_cvt_pk_fp8_f32(t[2], t[3], lo, true);
  uint32_t hi = __builtin_amdgcn_cvt_pk_fp8_f32(t[4], t[5], 0u, false);
  hi = __builtin_amdgcn_cvt_pk_fp8_f32(t[6], t[7], hi, true);
  return make_uint2(lo, hi);
}

// The largest |value| of a 16-byte piece of 16-bit values.
template <bool BF16> FLIDE_DEV float piece8_amax(const uint4& raw, float amax) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const u16 h = (i & 1) ? (u16)(w[i >> 1] >> 16) : (u16)(w[i >> 1] & 0xffff);
    amax = fmaxf(amax, fabsf(BF16 ? bf16_to_f32(h) : f16_to_f32(h)));
  }
  return amax;
}

// ---------------------------------------------------------------------------------------------------
// wave64 reductions
// ---------------------------------------------------------------------------------------------------
// All-reductions in registers: two DPP butterflies inside each quad (quad_perm [1,0,3,2] and [2,3,0,1]),
// row_half_mirror and row_mirror inside each row of 16 lanes, then gfx950's v_permlane16_swap and
// v_permlane32_swap across rows (no LDS round trip). Each step combines a lane's value with its partner's
// by a commutative operation, so every lane ends with the same bits, and the two outputs of a swap (the
// lane's own value and its partner's, in an order that depends on the lane) need no select. All 64 lanes
// must be active.
FLIDE_DEV int dpp_xor1(int v) { return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true); }
FLIDE_DEV int dpp_xor2(int v) { return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true); }
FLIDE_DEV int dpp_half_mirror(int v) { return __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, true); }
FLIDE_DEV int dpp_mirror(int v) { return __builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, true); }

template <typename Op> FLIDE_DEV float wave_reduce(float v, Op op) {
  v = op(v, __int_as_float(dpp_xor1(__float_as_int(v))));
  v = op(v, __int_as_float(dpp_xor2(__float_as_int(v))));
  v = op(v, __int_as_float(dpp_half_mirror(__float_as_int(v))));
  v = op(v, __int_as_float(dpp_mirror(__float_as_int(v))));
  const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false);
  v = op(__int_as_float(s16[0]), __int_as_float(s16[1]));
  const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
  return op(__int_as_float(s32[0]), __int_as_float(s32[1]));
}

FLIDE_DEV float wave_max(float v) {
  return wave_reduce(v, [](float a, float b) { return fmaxf(a, b); });
}

FLIDE_DEV float wave_sum(float v) {
  return wave_reduce(v, [](float a, float b) { return a + b; });
}

// (value, index) argmax over the wave: larger value wins, the lower index on equal values (a total
// order, so the combination is commutative). Lanes with nothing left carry value -inf and index
// INT_MAX, so they never win over a real entry.
FLIDE_DEV void wave_argmax(float& v, int& i) {
  // `|` and `&`, not `||` and `&&`: the short-circuit forms compile to exec-mask branches, three per
  // step, and a top-8 selection runs 48 steps in one dependent chain (route: 6.3 -> 3.5 us at 64 tokens)
  auto pick = [](float& v, int& i, float ov, int oi) {
    const bool take = (ov > v) | ((ov == v) & (oi < i));
    v = take ? ov : v;
    i = take ? oi : i;
  };
  pick(v, i, __int_as_float(dpp_xor1(__float_as_int(v))), dpp_xor1(i));
  pick(v, i, __int_as_float(dpp_xor2(__float_as_int(v))), dpp_xor2(i));
  pick(v, i, __int_as_float(dpp_half_mirror(__float_as_int(v))), dpp_half_mirror(i));
  pick(v, i, __int_as_float(dpp_mirror(__float_as_int(v))), dpp_mirror(i));
  {
    const auto sv = __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false);
    const auto si = __builtin_amdgcn_permlane16_swap(i, i, false, false);
    v = __int_as_float(sv[0]);
    i = si[0];
    pick(v, i, __int_as_float(sv[1]), si[1]);
  }
  {
    const auto sv = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
    const auto si = __builtin_amdgcn_permlane32_swap(i, i, false, false);
    v = __int_as_float(sv[0]);
    i = si[0];
    pick(v, i, __int_as_float(sv[1]), si[1]);
  }
}

// The same reductions inside each row of 16 lanes (the four DPP steps above): every lane ends with its
// row's result, so a wave can carry four independent 16-lane groups.
FLIDE_DEV float row16_max(float v) {
  v = fmaxf(v, __int_as_float(dpp_xor1(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp_xor2(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp_half_mirror(__float_as_int(v))));
  return fmaxf(v, __int_as_float(dpp_mirror(__float_as_int(v))));
}

FLIDE_DEV float row16_sum(float v) {
  v += __int_as_float(dpp_xor1(__float_as_int(v)));
  v += __int_as_float(dpp_xor2(__float_as_int(v)));
  v += __int_as_float(dpp_half_mirror(__float_as_int(v)));
  return v + __int_as_float(dpp_mirror(__float_as_int(v)));
}

FLIDE_DEV void row16_argmax(float& v, int& i) {
  auto pick = [](float& v, int& i, float ov, int oi) {
    const bool take = (ov > v) | ((ov == v) & (oi < i));
    v = take ? ov : v;
    i = take ? oi : i;
  };
  pick(v, i, __int_as_float(dpp_xor1(__float_as_int(v))), dpp_xor1(i));
  pick(v, i, __int_as_float(dpp_xor2(__float_as_int(v))), dpp_xor2(i));
  pick(v, i, __int_as_float(dpp_half_mirror(__float_as_int(v))), dpp_half_mirror(i));
  pick(v, i, __int_as_float(dpp_mirror(__float_as_int(v))), dpp_mirror(i));
}

FLIDE_DEV int lane_id() { return (int)__lane_id(); }

// ---------------------------------------------------------------------------------------------------
// MFMA fragments (gfx950)
//
// v_mfma_f32_16x16x32_{bf16,f16}: lane l holds 8 K-values of row (l % 16) of A and of column (l % 16)
// of B, and 4 outputs D[(l / 16) * 4 + i][l % 16], i = 0..3. Which 8 K-values a lane holds only has
// to agree between A and B. Every 16-bit product here uses the same fixed assignment: for each 32-wide
// K step c (in ascending order, one MFMA each), lane group g = l / 16 holds k = c*32 + g*8 + [0, 8).
// The sums therefore do not depend on the kernel, the tile shape or the number of rows in a batch.
//
// v_mfma_f32_16x16x128_f8f6f4 (e4m3 x e4m3): lane l holds 32 bytes of row (l % 16) of A and of column
// (l % 16) of B; here lane group g holds k = g*16 + [0, 16) and 64 + g*16 + [0, 16) of each 128-wide
// K chunk (two 16-byte pieces whose LDS reads are bank-conflict-free), chunks in ascending K.
// ---------------------------------------------------------------------------------------------------
template <typename T> struct Mfma16;

template <> struct Mfma16<__bf16> {
  static FLIDE_DEV f32x4_t mma(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
  static FLIDE_DEV float to_f32(u16 v) { return bf16_to_f32(v); }
  static FLIDE_DEV u16 from_f32(float f) { return f32_to_bf16(f); }
};

template <> struct Mfma16<_Float16> {
  static FLIDE_DEV f32x4_t mma(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
  static FLIDE_DEV float to_f32(u16 v) { return f16_to_f32(v); }
  static FLIDE_DEV u16 from_f32(float f) { return f32_to_f16(f); }
};

FLIDE_DEV f32x4_t mfma_fp8(const i32x8_t& a, const i32x8_t& b, const f32x4_t& c) {
  // format 0 = e4m3 for both operands; zero scale operands select the unscaled instruction
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// ---------------------------------------------------------------------------------------------------
// activations between the two grouped products (flide/kernels/pointwise.py:52-59,248-257)
// ---------------------------------------------------------------------------------------------------
// GELU-tanh(a) * b. 0.5 a (1 + tanh z) with z = sqrt(2/pi) (a + 0.044715 a^3) equals a / (1 + e^{-2z}),
// evaluated with the hardware reciprocal (v_rcp_f32, 1 ulp) instead of an IEEE division (about ten
// instructions with its scaling and fix-up): an epilogue evaluates this for every output of a gated tile.
// Large negative a: e^{-2z} overflows to inf, the reciprocal gives 0 and so does the product.
FLIDE_DEV float geglu_f32(float a, float b) {
  const float y = -1.5957691216057308f * (a + 0.044715f * a * a * a);   // -2z
  return a * __builtin_amdgcn_rcpf(1.0f + __expf(y)) * b;
}

// SiLU(a) * b = a / (1 + e^{-a}) * b, with the same reciprocal
FLIDE_DEV float swiglu_f32(float a, float b) { return a * __builtin_amdgcn_rcpf(1.0f + __expf(-a)) * b; }

enum { ACT_NONE = 0, ACT_GEGLU = 1, ACT_SWIGLU = 2 };

template <int ACT> FLIDE_DEV float act_f32(float g, float u) {
  if constexpr (ACT == ACT_GEGLU) return geglu_f32(g, u);
  else return swiglu_f32(g, u);
}

// status helpers for the C ABI
#define FLIDE_CHECK_LAUNCH()                                         \
  do {                                                               \
    hipError_t _e = hipGetLastError();                               \
    if (_e != hipSuccess) return FLIDE_MOE_ERR_HIP_BASE + (int)_e;   \
  } while (0)
