// Device pieces of routing: the per-token top-k selection (flide/kernels/moe.py:172-204, route.hip)
// and the chunked placement of pairs into per-expert segments (moe.py:207-253, align.hip).
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

template <int NW> struct AlignShared {
  int start[ALIGN_MAX_E];    // padded start of each expert's segment
  int before[ALIGN_MAX_E];   // this expert's pairs in earlier chunks
  int cnt[ALIGN_MAX_E];      // total pairs per expert
  int wcur[NW][ALIGN_MAX_E];
  int scan_tmp[NW];
};

// Placement of chunk c of the two-launch path by one workgroup of NW waves.
template <int NW>
FLIDE_DEV void align_place_wg(const int* __restrict__ ids, int n, int E, int bm, int c, int nchunks,
                              const int* __restrict__ hist, int* __restrict__ rows,
                              int* __restrict__ blocks, int* __restrict__ used, int* __restrict__ counts,
                              AlignShared<NW>& S) {
  constexpr int ALIGN_THREADS = NW * 64, ALIGN_WAVES = NW, ALIGN_CHUNK = NW * ALIGN_PER_WAVE;
  int* const start = S.start;
  int* const before = S.before;
  int* const cnt = S.cnt;
  int (*const wcur)[ALIGN_MAX_E] = S.wcur;
  int* const scan_tmp = S.scan_tmp;
  const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63;

  const int cbase = c * ALIGN_CHUNK;
  // this wave's pairs: 1/NW of the chunk, in pair order
  const int wper = ALIGN_PER_WAVE;
  const int wbase = cbase + wave * wper;
  const int wend = min(n, wbase + wper);
  // per-expert totals and the share of earlier chunks
  for (int e = tid; e < E; e += ALIGN_THREADS) {
    int b = 0, tot = 0;
#pragma unroll 8
    for (int j = 0; j < nchunks; ++j) {
      int v = hist[(long long)j * E + e];
      if (j < c) b += v;
      tot += v;
    }
    before[e] = b;
    cnt[e] = tot;
  }
  __syncthreads();
  // exclusive scan of the padded counts over experts: each thread owns a run of ceil(E / 256); a
  // shuffle scan inside each wave, then the waves' totals
  const int per = (E + ALIGN_THREADS - 1) / ALIGN_THREADS;
  int run = 0;
  for (int j = 0; j < per; ++j) {
    int e = tid * per + j;
    if (e < E) run += (cnt[e] + bm - 1) / bm * bm;
  }
  int incl = run;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int v = __shfl_up(incl, o);
    if (l >= o) incl += v;
  }
  if (l == 63) scan_tmp[wave] = incl;
  __syncthreads();
  int acc = incl - run;
  for (int w = 0; w < wave; ++w) acc += scan_tmp[w];
  for (int j = 0; j < per; ++j) {
    int e = tid * per + j;
    if (e < E) {
      start[e] = acc;
      acc += (cnt[e] + bm - 1) / bm * bm;
    }
  }
  __syncthreads();

  // each wave's quarter of the chunk: its own histogram first, so waves place in pair order
  for (int e = l; e < E; e += 64) wcur[wave][e] = 0;
  __syncthreads();
  for (int i = wbase + l; i < wend; i += 64) {
    int e = ids[i];
    if ((unsigned)e < (unsigned)E) atomicAdd(&wcur[wave][e], 1);
  }
  __syncthreads();
  // wcur[w][e] <- start[e] + before[e] + pairs of waves < w in this chunk
  for (int e = tid; e < E; e += ALIGN_THREADS) {
    int a = start[e] + before[e];
    for (int w = 0; w < ALIGN_WAVES; ++w) {
      int v = wcur[w][e];
      wcur[w][e] = a;
      a += v;
    }
  }
  __syncthreads();

  int nbits = 1;
  while ((1 << nbits) <= E) ++nbits;  // ids and the sentinel E fit in nbits
  const unsigned long long lt = (l == 0) ? 0ull : (~0ull >> (64 - l));
  for (int i0 = wbase; i0 < wend; i0 += 64) {
    const int i = i0 + l;
    int e = i < wend ? ids[i] : E;
    if ((unsigned)e >= (unsigned)E) e = E;
    unsigned long long same = ~0ull;
    for (int b = 0; b < nbits; ++b) {
      unsigned long long bal = __ballot((e >> b) & 1);
      same &= ((e >> b) & 1) ? bal : ~bal;
    }
    if (e < E) {
      const int rank = __popcll(same & lt);
      const int old = wcur[wave][e];
      rows[old + rank] = i;
      if (rank == 0) wcur[wave][e] = old + __popcll(same);
    }
  }

  // chunk 0: sentinels, block map, counts, used
  if (c == 0) {
    for (int e = tid; e < E; e += ALIGN_THREADS) {
      const int s = start[e], ce = cnt[e];
      const int p = (ce + bm - 1) / bm * bm;
      for (int r = s + ce; r < s + p; ++r) rows[r] = n;
      for (int b = s / bm; b < (s + p) / bm; ++b) blocks[b] = e;
      if (counts) counts[e] = ce;
      if (e == E - 1) used[0] = s + p;
    }
  }
}


}  // namespace routing
