// Device pieces of routing: the per-token top-k selection (flide/kernels/moe.py:172-204, route.hip)
// and the constants of the placement of pairs into per-expert segments (moe.py:207-253, align.hip).
#pragma once
#include <limits.h>

#include "common.hpp"

namespace routing {

constexpr int ALIGN_PER_WAVE = 256;   // pairs one wave places per chunk (two-launch path)
constexpr int ALIGN_MAX_E = 1024;

FLIDE_DEV float load_scalar(const void* p, int dtype, int i) {
  if (dtype == FLIDE_F32) return ((const float*)p)[i];
  if (dtype == FLIDE_BF16) return bf16_to_f32(((const u16*)p)[i]);
  return f16_to_f32(((const u16*)p)[i]);
}

// Per-lane inputs of one token's routing: the token's logits at experts l + 64 i (lane l; -inf past E).
template <int EPL> FLIDE_DEV void load_logits(const float* __restrict__ row, int E, float (&v)[EPL]) {
  const int l = lane_id();
#pragma unroll
  for (int i = 0; i < EPL; ++i) v[i] = l + 64 * i < E ? row[l + 64 * i] : -INFINITY;
}

// The per-expert scale at experts l + 64 i (1 without a scale), loaded once per wave. The raw bits of
// every element are loaded before any is converted: a conversion inside the dtype branch puts a wait
// for all of the wave's loads (the logits' too) between one element's load and the next.
template <int EPL> FLIDE_DEV void load_scales(const void* scale, int dtype, int E, float (&sc)[EPL]) {
  const int l = lane_id();
  uint32_t raw[EPL];
  if (dtype == FLIDE_F32) {
#pragma unroll
    for (int i = 0; i < EPL; ++i)
      raw[i] = scale && l + 64 * i < E ? ((const uint32_t*)scale)[l + 64 * i] : 0x3f800000u;
  } else {
    const uint32_t one = dtype == FLIDE_BF16 ? 0x3f80u : 0x3c00u;
#pragma unroll
    for (int i = 0; i < EPL; ++i) raw[i] = scale && l + 64 * i < E ? ((const u16*)scale)[l + 64 * i] : one;
  }
#pragma unroll
  for (int i = 0; i < EPL; ++i)
    sc[i] = dtype == FLIDE_F32 ? __uint_as_float(raw[i])
            : dtype == FLIDE_BF16 ? bf16_to_f32((u16)raw[i]) : f16_to_f32((u16)raw[i]);
}

// One token's routing by one wave from its logits v: the k largest of E in descending order, ties to
// the lower expert id, and their softmax probabilities renormalised over the k, times the expert's
// scale (sc, as load_scales holds it). Lane j < k writes slot j: wout[j], idout[j] (and idlds[j] when
// idlds != nullptr).
template <int EPL>
FLIDE_DEV void route_select(const float (&v)[EPL], const float (&sc)[EPL], int E, int k, float* __restrict__ wout,
                            int* __restrict__ idout, int* idlds) {
  const int l = lane_id();
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
  // the scale of this lane's expert, from the lane that holds it (every lane takes part in the shuffles)
  float my_sc = 1.f;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const float c = __shfl(sc[i], my_id & 63);
    if ((my_id >> 6) == i) my_sc = c;
  }
  // probabilities of the selected experts, summed in slot order (lane reads of lanes 0..k-1)
  const float my_p = l < k ? expf(my_v - m) / s : 0.f;
  float topsum = 0.f;
  for (int j = 0; j < k; ++j) topsum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_p), j));
  if (l < k) {
    const float ww = my_p / topsum;
    wout[l] = ww * my_sc;
    idout[l] = my_id;
    if (idlds) idlds[l] = my_id;
  }
}

// The experts call's float8 form of flide_moe_align (align.hip): the same placement (counts not written),
// with the token rows x [M, K] quantized per row into q / s by the placement launch's spare workgroups.
// FLIDE_MOE_ERR_TILE when the rows do not suit the vector quantizer (the caller then runs the two apart).
int align_quantizing(const int* ids, int n, int E, int bm, int* rows, int* blocks, int* used, void* workspace,
                     size_t workspace_bytes, const void* x, long long sx, int M, int K, int x_dtype, void* q,
                     long long sq, float* s, hipStream_t st);

}  // namespace routing
