// Sort and pad the (token, slot) pairs by expert: flide/kernels/moe.py:207-253 re-designed.
//
// The reference runs one program per expert, each scanning all n pairs (O(E n)). Here two launches do
// O(n) work in total:
//   align_count  chunk c of ALIGN_CHUNK pairs -> an LDS histogram -> hist[c][E] in the workspace
//                (skipped up to ALIGN_FUSED_MAX pairs: one align_place<true> then counts them itself)
//   align_place  every chunk sums the histograms before it (and all of them, for the padded expert
//                offsets), then places its pairs in pair order: each wave walks its quarter of the
//                chunk 64 pairs at a time; lanes with the same expert find each other with log2(E+1)
//                ballots, rank themselves by lane order and bump the wave's LDS counter once.
//                Chunk 0's workgroup also writes the padding sentinels, the block -> expert map,
//                `used` and the counts.
// The result is the reference's layout exactly: per expert its pairs in ascending pair order, then the
// sentinel n up to a multiple of bm.
#include "common.hpp"

namespace {

constexpr int ALIGN_THREADS = 256;
constexpr int ALIGN_WAVES = ALIGN_THREADS / 64;
constexpr int ALIGN_PER_WAVE = 256;   // pairs one wave places per chunk (two-launch path)
constexpr int ALIGN_CHUNK = ALIGN_WAVES * ALIGN_PER_WAVE;
constexpr int ALIGN_FUSED_MAX = 4096;  // up to this many pairs one workgroup counts and places all
constexpr int ALIGN_MAX_E = 1024;

__global__ __launch_bounds__(ALIGN_THREADS) void align_count(const int* __restrict__ ids, int n,
                                                             int E, int* __restrict__ hist) {
  __shared__ int h[ALIGN_MAX_E];
  for (int e = threadIdx.x; e < E; e += ALIGN_THREADS) h[e] = 0;
  __syncthreads();
  const int base = blockIdx.x * ALIGN_CHUNK;
  const int end = min(n, base + ALIGN_CHUNK);
  for (int i = base + threadIdx.x; i < end; i += ALIGN_THREADS) {
    int e = ids[i];
    if ((unsigned)e < (unsigned)E) atomicAdd(&h[e], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += ALIGN_THREADS) hist[(long long)blockIdx.x * E + e] = h[e];
}

template <bool FUSED>
__global__ __launch_bounds__(ALIGN_THREADS) void align_place(const int* __restrict__ ids, int n, int E,
                                                             int bm, int nchunks,
                                                             const int* __restrict__ hist,
                                                             int* __restrict__ rows,
                                                             int* __restrict__ blocks,
                                                             int* __restrict__ used,
                                                             int* __restrict__ counts) {
  __shared__ int start[ALIGN_MAX_E];   // padded start of each expert's segment
  __shared__ int before[ALIGN_MAX_E];  // this expert's pairs in earlier chunks
  __shared__ int cnt[ALIGN_MAX_E];     // total pairs per expert
  __shared__ int wcur[ALIGN_WAVES][ALIGN_MAX_E];
  __shared__ int scan_tmp[ALIGN_WAVES];
  const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63;
  const int c = blockIdx.x;

  const int cbase = c * ALIGN_CHUNK;
  // this wave's pairs: a quarter of the chunk (FUSED: of all n pairs, in 64-pair steps), in pair order
  const int wper = FUSED ? (n + ALIGN_WAVES * 64 - 1) / (ALIGN_WAVES * 64) * 64 : ALIGN_PER_WAVE;
  const int wbase = cbase + wave * wper;
  const int wend = min(n, wbase + wper);
  if constexpr (FUSED) {
    // one chunk holds every pair: count them here (per wave, which the placement needs anyway)
    for (int e = l; e < E; e += 64) wcur[wave][e] = 0;
    __syncthreads();
    for (int i = wbase + l; i < wend; i += 64) {
      int e = ids[i];
      if ((unsigned)e < (unsigned)E) atomicAdd(&wcur[wave][e], 1);
    }
    __syncthreads();
    for (int e = tid; e < E; e += ALIGN_THREADS) {
      int tot = 0;
      for (int w = 0; w < ALIGN_WAVES; ++w) tot += wcur[w][e];
      before[e] = 0;
      cnt[e] = tot;
    }
  } else {
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
  if constexpr (!FUSED) {
    for (int e = l; e < E; e += 64) wcur[wave][e] = 0;
    __syncthreads();
    for (int i = wbase + l; i < wend; i += 64) {
      int e = ids[i];
      if ((unsigned)e < (unsigned)E) atomicAdd(&wcur[wave][e], 1);
    }
    __syncthreads();
  }
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

}  // namespace

// chunks of the two-launch path (1 when one workgroup handles every pair)
int align_chunks(int n) { return n <= ALIGN_FUSED_MAX ? 1 : (n + ALIGN_CHUNK - 1) / ALIGN_CHUNK; }

extern "C" size_t flide_moe_align_workspace(int n, int E) {
  if (n < 0 || E <= 0) return 0;
  return (size_t)align_chunks(n) * (size_t)E * sizeof(int);
}

extern "C" int flide_moe_align(const int* ids, int n, int E, int bm, int* rows, int* blocks,
                               int* used, int* counts, void* workspace, size_t workspace_bytes,
                               flide_stream_t stream) {
  if (n < 0 || E <= 0 || E > ALIGN_MAX_E || bm <= 0) return FLIDE_MOE_ERR_ARG;
  if (workspace_bytes < flide_moe_align_workspace(n, E)) return FLIDE_MOE_ERR_WORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  const int nchunks = align_chunks(n);
  int* hist = (int*)workspace;
  if (nchunks == 1) {   // one workgroup counts and places every pair
    align_place<true><<<1, ALIGN_THREADS, 0, st>>>(ids, n, E, bm, 1, hist, rows, blocks, used, counts);
    FLIDE_CHECK_LAUNCH();
    return FLIDE_MOE_OK;
  }
  align_count<<<nchunks, ALIGN_THREADS, 0, st>>>(ids, n, E, hist);
  FLIDE_CHECK_LAUNCH();
  align_place<false><<<nchunks, ALIGN_THREADS, 0, st>>>(ids, n, E, bm, nchunks, hist, rows, blocks, used,
                                                        counts);
  FLIDE_CHECK_LAUNCH();
  return FLIDE_MOE_OK;
}
