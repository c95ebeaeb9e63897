// Sort and pad the (token, slot) pairs by expert: flide/kernels/moe.py:207-253 re-designed.
//
// The reference runs one program per expert, each scanning all n pairs (O(E n)). Here the work is O(n):
// up to ALIGN_FUSED_MAX pairs one launch of one workgroup (align_one, below); beyond that two launches:
//   align_count  chunk c of ALIGN_CHUNK pairs -> an LDS histogram -> hist[c][E] in the workspace
//   align_place  every chunk sums the histograms before it (and all of them, for the padded expert
//                offsets), then places its pairs in pair order: each wave walks its quarter of the
//                chunk 64 pairs at a time; lanes with the same expert find each other with log2(E+1)
//                ballots, rank themselves by lane order and bump the wave's LDS counter once.
//                Chunk c also writes, for experts e = c, c + nchunks, ..., the padding sentinels,
//                the block -> expert map and the counts (and `used` with the last expert).
// The result is the reference's layout exactly: per expert its pairs in ascending pair order, then the
// sentinel n up to a multiple of bm.
#include "quantize.hpp"
#include "routing.hpp"

namespace {
using namespace routing;

constexpr int ALIGN_THREADS = 256;
constexpr int ALIGN_WAVES = ALIGN_THREADS / 64;
constexpr int ALIGN_CHUNK = ALIGN_WAVES * ALIGN_PER_WAVE;
constexpr int ALIGN_FUSED_MAX = 4096;  // up to this many pairs one workgroup counts and places all

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

// Chunk c's placement by one workgroup of ALIGN_THREADS (the body of align_place).
FLIDE_DEV void align_place_chunk(int c, const int* __restrict__ ids, int n, int E, int bm, int nchunks,
                                 const int* __restrict__ hist, int* __restrict__ rows, int* __restrict__ blocks,
                                 int* __restrict__ used, int* __restrict__ counts) {
  constexpr int PL = ALIGN_PER_WAVE / 64;   // pairs per lane
  __shared__ int start[ALIGN_MAX_E];    // padded start of each expert's segment
  __shared__ int before[ALIGN_MAX_E];   // this expert's pairs in earlier chunks
  __shared__ int cnt[ALIGN_MAX_E];      // total pairs per expert
  __shared__ int wcnt[ALIGN_WAVES][ALIGN_MAX_E];   // per wave: its pairs per expert, then its base
  __shared__ int scan_tmp[ALIGN_WAVES];
  const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63;
  // the wave's pairs [wbase, wbase + 256), 4 per lane in 64-pair groups, loaded once and held in registers
  const int wbase = c * ALIGN_CHUNK + wave * ALIGN_PER_WAVE;
  int e_g[PL];
#pragma unroll
  for (int g = 0; g < PL; ++g) e_g[g] = ids[min(wbase + g * 64 + l, n - 1)];   // in bounds; past n dropped below
  // per-expert totals and the share of earlier chunks: the whole histogram matrix [nchunks][E], read by
  // every thread in a strided share with 16 loads in flight (issued with the ids), added into LDS
  const int total = nchunks * E;
  int hv[16];
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const int i = tid + u * ALIGN_THREADS;
    hv[u] = i < total ? hist[i] : 0;
  }
  for (int e = tid; e < E; e += ALIGN_THREADS) {
    before[e] = 0;
    cnt[e] = 0;
#pragma unroll
    for (int w = 0; w < ALIGN_WAVES; ++w) wcnt[w][e] = 0;
  }
  __syncthreads();
  for (int i0 = tid;; ) {
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      if (hv[u] == 0) continue;
      const int i = i0 + u * ALIGN_THREADS, j = i / E, e = i - j * E;
      atomicAdd(&cnt[e], hv[u]);
      if (j < c) atomicAdd(&before[e], hv[u]);
    }
    i0 += ALIGN_THREADS * 16;
    if (i0 >= total) break;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int i = i0 + u * ALIGN_THREADS;
      hv[u] = i < total ? hist[i] : 0;
    }
  }
  // the wave's own pairs per expert, and each lane's offset among the wave's pairs of its expert: lanes
  // of a 64-pair group with the same expert find each other with log2(E+1) ballots; the lowest adds the
  // group's count (every lane reads the counter before the lowest one writes it)
  int nbits = 1;
  while ((1 << nbits) <= E) ++nbits;  // ids and the stand-in E fit in nbits
  const unsigned long long lt = (l == 0) ? 0ull : (~0ull >> (64 - l));
  int off_g[PL];
#pragma unroll
  for (int g = 0; g < PL; ++g) {
    int e = e_g[g];
    if (wbase + g * 64 + l >= n || (unsigned)e >= (unsigned)E) e = E;
    e_g[g] = e;
    unsigned long long same = ~0ull;
    for (int b = 0; b < nbits; ++b) {
      const unsigned long long bal = __ballot((e >> b) & 1);
      same &= ((e >> b) & 1) ? bal : ~bal;
    }
    off_g[g] = 0;
    if (e < E) {
      const int rank = __popcll(same & lt);
      const int old = wcnt[wave][e];
      off_g[g] = old + rank;
      if (rank == 0) wcnt[wave][e] = old + __popcll(same);
    }
  }
  __syncthreads();
  // exclusive scan of the padded counts over experts: each thread owns a run of ceil(E / 256); a
  // shuffle scan inside each wave, then the waves' totals
  const int per = (E + ALIGN_THREADS - 1) / ALIGN_THREADS;
  int run = 0;
  for (int j = 0; j < per; ++j) {
    const int e = tid * per + j;
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
    const int e = tid * per + j;
    if (e < E) {
      start[e] = acc;
      // wcnt[w][e] <- start[e] + before[e] + pairs of waves < w in this chunk
      int a = acc + before[e];
#pragma unroll
      for (int w = 0; w < ALIGN_WAVES; ++w) {
        const int v = wcnt[w][e];
        wcnt[w][e] = a;
        a += v;
      }
      acc += (cnt[e] + bm - 1) / bm * bm;
    }
  }
  __syncthreads();
#pragma unroll
  for (int g = 0; g < PL; ++g)
    if (e_g[g] < E) rows[wcnt[wave][e_g[g]] + off_g[g]] = wbase + g * 64 + l;

  // experts c, c + nchunks, ...: sentinels after the pairs, the block -> expert map, the counts; every
  // thread of the workgroup takes a stride of each expert's rows and blocks
  for (int e = c; e < E; e += nchunks) {
    const int s = start[e], ce = cnt[e];
    const int p = (ce + bm - 1) / bm * bm;
    for (int r = s + ce + tid; r < s + p; r += ALIGN_THREADS) rows[r] = n;
    for (int b = s / bm + tid; b < (s + p) / bm; b += ALIGN_THREADS) blocks[b] = e;
    if (tid == 0) {
      if (counts) counts[e] = ce;
      if (e == E - 1) used[0] = s + p;
    }
  }
}

__global__ __launch_bounds__(ALIGN_THREADS) void align_place(const int* __restrict__ ids, int n, int E, int bm,
                                                             int nchunks, const int* __restrict__ hist,
                                                             int* __restrict__ rows, int* __restrict__ blocks,
                                                             int* __restrict__ used, int* __restrict__ counts) {
  align_place_chunk(blockIdx.x, ids, n, E, bm, nchunks, hist, rows, blocks, used, counts);
}

// Up to ALIGN_FUSED_MAX pairs: one workgroup of 8 waves, one pass over the ids. Wave w owns the pairs
// [w * wper, (w + 1) * wper), up to 8 per lane in 64-pair groups, held in registers from one load.
//   1. each group's lanes with the same expert find each other with ballots; the lowest one adds the
//      group's count to the wave's LDS counter for that expert, and every lane keeps its offset among
//      the wave's pairs of that expert (counter before the group + rank in the group);
//   2. one thread per expert: the total over waves, an exclusive scan of the padded totals (the
//      segments' starts), the waves' bases inside the segment and the segment's blocks in an LDS
//      block -> expert map;
//   3. each pair's row is base + offset; the padding rows (the sentinel n) and the block map are written
//      by all threads in strides, so no thread loops over an expert's padding alone.
// 64 tokens x 8: 6.1 us for the two-pass form with 4 waves (ids loaded twice, an expert's padding
// written by one thread).
constexpr int ALIGN1_WAVES = 8;
constexpr int ALIGN1_THREADS = ALIGN1_WAVES * 64;
constexpr int ALIGN1_PER_LANE = ALIGN_FUSED_MAX / ALIGN1_THREADS;
constexpr int ALIGN1_MAX_BLOCKS = ALIGN_FUSED_MAX + ALIGN_MAX_E;   // >= ceil((n + E (bm - 1)) / bm)

FLIDE_DEV void align_one_body(const int* __restrict__ ids, int n, int E, int bm, int* __restrict__ rows,
                              int* __restrict__ blocks, int* __restrict__ used, int* __restrict__ counts) {
  __shared__ int wcnt[ALIGN1_WAVES][ALIGN_MAX_E];   // per wave: pairs per expert, then its base
  __shared__ int start[ALIGN_MAX_E], cnt[ALIGN_MAX_E];
  __shared__ int bexp[ALIGN1_MAX_BLOCKS];
  __shared__ int scan_tmp[ALIGN1_WAVES];
  __shared__ int s_used;
  const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63;
  const int wper = (n + ALIGN1_THREADS - 1) / ALIGN1_THREADS * 64;   // pairs per wave, whole groups
  const int ng = wper / 64;                                          // groups per wave (<= 8)
  const int wbase = wave * wper;

  int e_g[ALIGN1_PER_LANE];
#pragma unroll
  for (int g = 0; g < ALIGN1_PER_LANE; ++g) {
    if (g >= ng) break;
    e_g[g] = ids[min(wbase + g * 64 + l, n - 1)];   // in bounds; a lane past n is dropped below
  }
  for (int w = 0; w < ALIGN1_WAVES; ++w)
    for (int e = tid; e < E; e += ALIGN1_THREADS) wcnt[w][e] = 0;
  __syncthreads();

  int nbits = 1;
  while ((1 << nbits) <= E) ++nbits;  // ids and the stand-in E fit in nbits
  const unsigned long long lt = (l == 0) ? 0ull : (~0ull >> (64 - l));
  int off_g[ALIGN1_PER_LANE];
#pragma unroll
  for (int g = 0; g < ALIGN1_PER_LANE; ++g) {
    if (g >= ng) break;
    int e = e_g[g];
    if (wbase + g * 64 + l >= n || (unsigned)e >= (unsigned)E) e = E;
    e_g[g] = e;
    unsigned long long same = ~0ull;
    for (int b = 0; b < nbits; ++b) {
      const unsigned long long bal = __ballot((e >> b) & 1);
      same &= ((e >> b) & 1) ? bal : ~bal;
    }
    off_g[g] = 0;
    if (e < E) {
      const int rank = __popcll(same & lt);
      const int old = wcnt[wave][e];   // every lane reads before the group's lowest lane writes
      off_g[g] = old + rank;
      if (rank == 0) wcnt[wave][e] = old + __popcll(same);
    }
  }
  __syncthreads();

  // one thread per expert (E <= 1024 = 2 per thread): totals, padded exclusive scan, wave bases
  const bool pow2 = (bm & (bm - 1)) == 0;
  const int sh = 31 - __clz(bm);
  auto pad = [&](int c) { return pow2 ? (c + bm - 1) & ~(bm - 1) : (c + bm - 1) / bm * bm; };
  constexpr int PER = ALIGN_MAX_E / ALIGN1_THREADS;
  int tot[PER], run = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = tid * PER + j;
    tot[j] = 0;
    if (e < E)
      for (int w = 0; w < ALIGN1_WAVES; ++w) tot[j] += wcnt[w][e];
    run += pad(tot[j]);
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
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = tid * PER + j;
    if (e >= E) break;
    const int s = acc, p = pad(tot[j]);
    start[e] = s;
    cnt[e] = tot[j];
    int a = s;
    for (int w = 0; w < ALIGN1_WAVES; ++w) {
      const int v = wcnt[w][e];
      wcnt[w][e] = a;
      a += v;
    }
    for (int b = pow2 ? s >> sh : s / bm, b1 = pow2 ? (s + p) >> sh : (s + p) / bm; b < b1; ++b) bexp[b] = e;
    if (counts) counts[e] = tot[j];
    if (e == E - 1) {
      used[0] = s + p;
      s_used = s + p;
    }
    acc += p;
  }
  __syncthreads();

#pragma unroll
  for (int g = 0; g < ALIGN1_PER_LANE; ++g) {
    if (g >= ng) break;
    const int e = e_g[g];
    if (e < E) rows[wcnt[wave][e] + off_g[g]] = wbase + g * 64 + l;
  }
  const int u = s_used;
  for (int r = tid; r < u; r += ALIGN1_THREADS) {
    const int e = bexp[pow2 ? r >> sh : r / bm];
    if (r >= start[e] + cnt[e]) rows[r] = n;
  }
  const int nb = pow2 ? u >> sh : u / bm;
  for (int b = tid; b < nb; b += ALIGN1_THREADS) blocks[b] = bexp[b];
}

__global__ __launch_bounds__(ALIGN1_THREADS) void align_one(const int* __restrict__ ids, int n, int E, int bm,
                                                            int* __restrict__ rows, int* __restrict__ blocks,
                                                            int* __restrict__ used, int* __restrict__ counts) {
  align_one_body(ids, n, E, bm, rows, blocks, used, counts);
}

// The experts call's float8 form: the placement launch's spare workgroups quantize the token rows x [M, K]
// (quant::quantize_row16, one wave per row), which do not depend on the placement; one launch less and the
// two overlap. Workgroups below `nplace` place pairs, the others quantize ROWS rows each.
template <int NV, bool BF16>
__global__ __launch_bounds__(ALIGN_THREADS) void align_place_quant(const int* __restrict__ ids, int n, int E, int bm,
                                                                   int nchunks, const int* __restrict__ hist,
                                                                   int* __restrict__ rows, int* __restrict__ blocks,
                                                                   int* __restrict__ used, const u16* __restrict__ x,
                                                                   long long sx, int K, int M, u8* __restrict__ q,
                                                                   long long sq, float* __restrict__ s) {
  if ((int)blockIdx.x < nchunks) {
    align_place_chunk(blockIdx.x, ids, n, E, bm, nchunks, hist, rows, blocks, used, nullptr);
    return;
  }
  const long long row = (long long)(blockIdx.x - nchunks) * (ALIGN_THREADS / 64) + (threadIdx.x >> 6);
  if (row < M) quant::quantize_row16<NV, BF16>(x, sx, K, row, q, sq, s);
}

template <int NV, bool BF16>
__global__ __launch_bounds__(ALIGN1_THREADS) void align_one_quant(const int* __restrict__ ids, int n, int E, int bm,
                                                                  int* __restrict__ rows, int* __restrict__ blocks,
                                                                  int* __restrict__ used, const u16* __restrict__ x,
                                                                  long long sx, int K, int M, u8* __restrict__ q,
                                                                  long long sq, float* __restrict__ s) {
  if (blockIdx.x == 0) {
    align_one_body(ids, n, E, bm, rows, blocks, used, nullptr);
    return;
  }
  const long long row = (long long)(blockIdx.x - 1) * ALIGN1_WAVES + (threadIdx.x >> 6);
  if (row < M) quant::quantize_row16<NV, BF16>(x, sx, K, row, q, sq, s);
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
    align_one<<<1, ALIGN1_THREADS, 0, st>>>(ids, n, E, bm, rows, blocks, used, counts);
    FLIDE_CHECK_LAUNCH();
    return FLIDE_MOE_OK;
  }
  align_count<<<nchunks, ALIGN_THREADS, 0, st>>>(ids, n, E, hist);
  FLIDE_CHECK_LAUNCH();
  align_place<<<nchunks, ALIGN_THREADS, 0, st>>>(ids, n, E, bm, nchunks, hist, rows, blocks, used, counts);
  FLIDE_CHECK_LAUNCH();
  return FLIDE_MOE_OK;
}

namespace routing {

int align_quantizing(const int* ids, int n, int E, int bm, int* rows, int* blocks, int* used, void* workspace,
                     size_t workspace_bytes, const void* x, long long sx, int M, int K, int x_dtype, void* q,
                     long long sq, float* s, hipStream_t st) {
  if (n <= 0 || E <= 0 || E > ALIGN_MAX_E || bm <= 0 || M <= 0 || !quant::row16_ok(x, sx, K, x_dtype, q, sq))
    return FLIDE_MOE_ERR_TILE;
  if (workspace_bytes < flide_moe_align_workspace(n, E)) return FLIDE_MOE_ERR_WORKSPACE;
  const int nchunks = align_chunks(n);
  int* hist = (int*)workspace;
  const bool bf = x_dtype == FLIDE_BF16;
  const int nv = quant::row16_nv(K);
  const u16* xx = (const u16*)x;
  u8* qq = (u8*)q;
#define AQ(NV)                                                                                                   \
  do {                                                                                                           \
    if (nchunks == 1) {                                                                                          \
      const dim3 g(1 + (M + ALIGN1_WAVES - 1) / ALIGN1_WAVES);                                                  \
      if (bf) align_one_quant<NV, true><<<g, ALIGN1_THREADS, 0, st>>>(ids, n, E, bm, rows, blocks, used, xx, sx, K, M, qq, sq, s); \
      else align_one_quant<NV, false><<<g, ALIGN1_THREADS, 0, st>>>(ids, n, E, bm, rows, blocks, used, xx, sx, K, M, qq, sq, s); \
    } else {                                                                                                     \
      align_count<<<nchunks, ALIGN_THREADS, 0, st>>>(ids, n, E, hist);                                           \
      const dim3 g(nchunks + (M + ALIGN_WAVES - 1) / ALIGN_WAVES);                                              \
      if (bf) align_place_quant<NV, true><<<g, ALIGN_THREADS, 0, st>>>(ids, n, E, bm, nchunks, hist, rows, blocks, used, xx, sx, K, M, qq, sq, s); \
      else align_place_quant<NV, false><<<g, ALIGN_THREADS, 0, st>>>(ids, n, E, bm, nchunks, hist, rows, blocks, used, xx, sx, K, M, qq, sq, s); \
    }                                                                                                            \
  } while (0)
  if (nv == 1) AQ(1);
  else if (nv == 2) AQ(2);
  else if (nv == 4) AQ(4);
  else if (nv == 8) AQ(8);
  else AQ(16);
#undef AQ
  FLIDE_CHECK_LAUNCH();
  return FLIDE_MOE_OK;
}

}  // namespace routing
