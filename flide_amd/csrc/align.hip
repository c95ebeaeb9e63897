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

template <bool FUSED>
__global__ __launch_bounds__(ALIGN_THREADS) void align_place(const int* __restrict__ ids, int n, int E,
                                                             int bm, int nchunks,
                                                             const int* __restrict__ hist,
                                                             int* __restrict__ rows,
                                                             int* __restrict__ blocks,
                                                             int* __restrict__ used,
                                                             int* __restrict__ counts) {
  __shared__ AlignShared<ALIGN_WAVES> S;
  align_place_wg<FUSED, ALIGN_WAVES>(ids, n, E, bm, blockIdx.x, nchunks, hist, rows, blocks, used, counts, S);
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
