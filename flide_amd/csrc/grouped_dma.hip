// Prefill-shaped grouped products: direct-to-LDS loads, a multi-stage ring and large MFMA tiles.
//
// One workgroup (4 or 8 waves) computes a BM-row block of pairs (one expert, as align padded
// it) against a BN-row tile of that expert's weight. Per K stage it moves (BM + BN) rows of 128 bytes
// straight from global memory into LDS with global_load_lds_dwordx4 (gfx950): no VGPR staging, no LDS
// write instructions. NS stages are in flight: while the MFMAs consume stage kt, the loads of stages
// kt+1 .. kt+NS-1 are outstanding; a wave waits only for its own loads of stage kt (vmcnt) and one
// barrier per stage publishes everyone's.
//
// LDS layout: rows of 8 x 16-byte chunks, chunk c of row r stored at position c ^ (r & 7). Measured on
// gfx950 (SQ_LDS_BANK_CONFLICT), this makes every MFMA operand read here conflict-free: a 16-row
// fragment read of chunk c (16-bit steps: c = s*4 + g; float8: c = g and g + 4) runs at the full
// 256 bytes per clock, where unswizzled rows or chunk pairs (2g, 2g + 1) take twice as long.
// A direct load writes 64 lanes x 16 bytes contiguously, so each lane fetches the global chunk that
// belongs at its LDS position under that swizzle.
//
// Padding rows (the sentinel pair) and weight rows past N load real but unused data (row 0 / the last
// valid row): MFMA rows and columns never mix, and the epilogue stores neither. K tails read a 16-byte
// block of zeros. Work items are ordered so each XCD (workgroup b runs on XCD b % 8) walks a contiguous
// range of (block, column tile) items: the block's rows and the expert's weight tiles are reused from
// that XCD's L2.
//
// Arithmetic is the same as every other grouped kernel here (common.hpp): 16-bit products in 32-wide
// K steps with lane group g holding k = c*32 + g*8 + [0, 8); float8 in 128-wide steps with lane group g
// holding k = g*16 + [0, 16) and 64 + g*16 + [0, 16).
#include "dma_common.hpp"

namespace {
using namespace grouped_detail;

//
// NLD > 0 splits the roles: the WAVES_M x WAVES_N compute waves only read LDS, issue MFMAs and run the
// epilogue, and NLD loader waves only issue the stage ring's loads and wait for them (a wave's vmcnt counts
// its own loads, so no compute wave ever waits on a load). The per-stage barrier then publishes a stage
// the loaders waited for and frees the slot the compute waves read last. The float8 gated bm-128 product
// at 4096 tokens: 256 -> 241 us; 16-bit products gain nothing or lose (the 16-bit down product 4%).
template <typename T, typename OutT, int ACT, int BM, int BN, int WAVES_M, int WAVES_N, int NS, int ROWB, int OCC,
          int XCD_CHUNK_BLOCKS, bool NTW, int NLD = 0>
__global__ __launch_bounds__((WAVES_M * WAVES_N + NLD) * 64, OCC) void grouped_dma(GroupArgs p) {
  constexpr bool FP8 = std::is_same<T, Fp8Tag>::value;
  constexpr int EB = DmaElem<T>::BYTES;
  constexpr int KS = ROWB / EB;                // K values per stage
  constexpr int CPR = ROWB / 16;               // 16-byte chunks per stage row
  constexpr int RPI = 64 / CPR;                // rows one 1 KB load instruction fills
  constexpr int STEPS = FP8 ? 1 : ROWB / 64;   // MFMA K steps per stage
  constexpr int A_BYTES = BM * ROWB, B_BYTES = BN * ROWB, STAGE = A_BYTES + B_BYTES;
  constexpr int NW = WAVES_M * WAVES_N;                      // compute waves per workgroup
  constexpr int NLW = NLD > 0 ? NLD : NW;                    // waves that issue loads
  constexpr int LA = BM / (NLW * RPI), LB = BN / (NLW * RPI);  // 1 KB loads per loading wave per stage
  static_assert(!FP8 || ROWB == 128, "float8 stages hold one 128-wide MFMA step");
  static_assert(BM % (NLW * RPI) == 0 && BN % (NLW * RPI) == 0, "tile rows split over the loading waves");
  static_assert(NLD == 0 || BM >= 64, "split roles only for the prefill tiles");
  constexpr int L = LA + LB;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int FM = WM / 16, FN = WN / 16;
  static_assert(NW == 4 || NW == 8, "4 or 8 waves");
  static_assert(BM % 32 == 0 && BN % 32 == 0, "tile rows come in 32s");
  static_assert(ACT == ACT_NONE || FN % 2 == 0, "gated tiles pair gate and up fragments");
  static_assert((NS - 1) * L < 64, "loads in flight must fit vmcnt");

  // one LDS object per ring slot: distinct objects let the compiler see that reading slot s does not
  // alias the loads still landing in the other slots (it would otherwise wait for all of them)
  __shared__ __attribute__((aligned(1024))) char lds0[STAGE];
  __shared__ __attribute__((aligned(1024))) char lds1[STAGE];
  __shared__ __attribute__((aligned(1024))) char lds2[NS > 2 ? STAGE : 16];
  __shared__ __attribute__((aligned(1024))) char lds3[NS > 3 ? STAGE : 16];
  __shared__ int s_pairs[BM];
  __shared__ float s_ascale[FP8 ? BM : 1];
  __shared__ float s_wt[ACT == ACT_NONE ? BM : 1];   // plain products: the rows' routing weights

  const int tid = threadIdx.x, l = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform, in an SGPR
  const bool loads = NLD == 0 || wave >= NW;                   // this wave issues loads
  const int lw = NLD > 0 ? wave - NW : wave;                   // its index among the loading waves
  // Workgroup b runs on XCD b % 8.
  int pm, pn;
  long long e;   // the block's expert
  if constexpr (BM >= 64) {
    // Prefill tiles: the items (block, column tile) in use, ordered by expert, are split into 8
    // contiguous ranges, range x for the workgroups of XCD x. An expert's blocks and all its column
    // tiles then run on one XCD at about the same time, so each weight tile comes from HBM about once
    // and is shared in that XCD's L2. Inside an expert the gated (gate/up) products run column-tile
    // major, so the expert's blocks load each weight tile together (HBM fetch of the 16-bit gate/up
    // product at 8192 tokens 3.1 -> 2.1 GB; gate/up 4-11% faster at 4096-16384 tokens than the XCD
    // chunks below); the plain (down) products run block major, measured 2-3% faster for them.
    const int nused = *p.used / BM;
    const long long R = (long long)nused * p.ntn;
    const int x = blockIdx.x & 7;
    const long long it = R * x / 8 + (blockIdx.x >> 3);
    if (it >= R * (x + 1) / 8) return;
    const int blk = (int)(it / p.ntn);   // a block of the item's expert
    int s0, s1;
    e = expert_run(p.blocks, blk, nused, l, s0, s1);
    s0 = __builtin_amdgcn_readfirstlane(s0);
    const int local = (int)(it - (long long)s0 * p.ntn);
    if constexpr (ACT != ACT_NONE) {
      const int nb = __builtin_amdgcn_readfirstlane(s1) - s0;
      pn = local / nb;
      pm = s0 + local % nb;
    } else {
      pm = s0 + local / p.ntn;
      pn = local % p.ntn;
    }
  } else {
    // Decode tiles: items are cut into chunks of CH items (a few blocks of one expert and all their
    // column tiles) and chunk c goes to XCD c % 8, so each XCD's workgroups reuse the chunk's rows and
    // weight tiles from that XCD's L2, and the dead items at the end of the static grid spread over all
    // XCDs (the host rounds the grid to a multiple of 8 * CH). Inside a chunk the gated (gate/up)
    // products run column-tile major, so the blocks that share a weight tile start back to back; the
    // plain (down) products run block major.
    const int CH = p.ntn * XCD_CHUNK_BLOCKS;
    const int b = blockIdx.x;
    const int j = b >> 3;
    const int chunk = (j / CH) * 8 + (b & 7), within = j % CH;
    if constexpr (ACT != ACT_NONE) {
      pm = chunk * XCD_CHUNK_BLOCKS + within % XCD_CHUNK_BLOCKS;
      pn = within / XCD_CHUNK_BLOCKS;
    } else {
      const int widx = chunk * CH + within;
      pm = widx / p.ntn;
      pn = widx % p.ntn;
    }
    if (pm >= p.nbm || pm * BM >= *p.used) return;
    e = __builtin_amdgcn_readfirstlane(p.blocks[pm]);
  }
  const int K = p.K;
  const int half = p.N / 2;
  const char* A = (const char*)p.a;
  const char* B = (const char*)p.w + e * p.sbe * EB;
  // full stages load through buffer resources over the activation rows and the expert's weight rows
  const long long a_rows = p.by_token ? (p.n_pairs + p.topk - 1) / p.topk : p.n_pairs;
  const __amdgpu_buffer_rsrc_t rsA = buf_rsrc(A, ((a_rows - 1) * p.sa + K) * EB);
  const __amdgpu_buffer_rsrc_t rsB = buf_rsrc(B, ((long long)(p.N - 1) * p.sbn + K) * EB);
  const int kc = ((l % CPR) ^ swz<CPR>(l / CPR)) * (16 / EB);
  uint32_t b_off32[LB];
#pragma unroll
  for (int i = 0; i < LB; ++i) {
    const int row = (lw * LB + i) * RPI + l / CPR;
    long long n;
    if constexpr (ACT == ACT_NONE) {
      n = (long long)pn * BN + row;
      if (n >= p.N) n = p.N - 1;
    } else {
      int cc = pn * (BN / 2) + (row < BN / 2 ? row : row - BN / 2);
      if (cc >= half) cc = half - 1;
      n = row < BN / 2 ? cc : cc + half;
    }
    b_off32[i] = (uint32_t)((n * p.sbn + kc) * EB);
  }
  // The weight rows' offsets depend only on the expert and the column tile, so the weight parts of the
  // first NS - 1 stages go in flight before the block's pairs are read (their activation parts follow
  // in the K loop's prologue, which then waits for both): the workgroup's start-up keeps the memory
  // pipe busy (the plain product at 8192 tokens 1.5% faster, no change elsewhere).
  if (loads) {
    char* const slots[4] = {lds0, lds1, lds2, lds3};
#pragma unroll
    for (int st = 0; st < NS - 1; ++st) {
      FLIDE_LDS_AS char* sb = (FLIDE_LDS_AS char*)slots[st];
#pragma unroll
      for (int i = 0; i < LB; ++i)
        dma16b<NTW ? 2 : 0>(rsB, b_off32[i], (uint32_t)(st * KS * EB), sb + A_BYTES + (lw * LB + i) * 1024);
    }
  }
  // The rows' activation scales (float8) and routing weights (plain products) are read only by the
  // epilogue. With one row per thread in whole waves, their loads (which need the pair loads) go straight
  // to LDS and stay in flight: loading waves wait for them with their first stages (the K loop's
  // prologue waits for every load), compute waves of the split roles after the K loop.
  constexpr bool DEFER = (NW + NLD) * 64 >= BM && BM % 64 == 0;
  constexpr bool POST_WAIT = DEFER && NLD > 0 && (FP8 || ACT == ACT_NONE);   // compute waves issued some
  for (int r = tid; r < BM; r += (NW + NLD) * 64) {
    const int pair = p.rows[pm * BM + r];
    s_pairs[r] = pair;
    const bool ok = pair < p.n_pairs;
    if constexpr (FP8) {
      const long long src = p.by_token ? pair / p.topk : pair;
      if constexpr (DEFER)
        dma4(ok ? (const void*)(p.a_scale + src) : (const void*)g_zero16, (FLIDE_LDS_AS char*)s_ascale + (r & ~63) * 4);
      else s_ascale[r] = ok ? p.a_scale[src] : 0.f;
    }
    if constexpr (ACT == ACT_NONE) {
      if constexpr (DEFER)
        dma4(ok && p.weights ? (const void*)(p.weights + pair) : (const void*)&g_one, (FLIDE_LDS_AS char*)s_wt + (r & ~63) * 4);
      else s_wt[r] = p.weights && ok ? p.weights[pair] : 1.f;
    }
  }
  lds_barrier();   // the weight loads of the first stages stay in flight

  // This lane's global source for each of its loads: tile row (instr * RPI + l / CPR) and logical chunk
  // c = (l % CPR) ^ swz(row). Instruction rows start at multiples of RPI, so swz(row) and therefore c
  // (and the chunk's K offset kc) depend on the lane only.
  // Per-lane 32-bit byte offsets from the operands' uniform bases (A rows are gathered pairs, B rows
  // the expert's weight rows); a full stage's load is buffer resource (SGPRs) + offset (one VGPR) +
  // the stage's K offset (one SGPR). Both tensors stay below 4 GB.
  uint32_t a_off32[LA];
#pragma unroll
  for (int i = 0; i < LA; ++i) {
    const int row = (lw * LA + i) * RPI + l / CPR;
    const int pair = s_pairs[row];
    const long long src = pair < p.n_pairs ? (p.by_token ? pair / p.topk : pair) : 0;
    a_off32[i] = (uint32_t)((src * p.sa + kc) * EB);
  }
  if constexpr (NLD > 0) {
    if (wave >= NW) {   // loader waves: the stage ring's loads, one barrier per stage
      const int nk = (K + KS - 1) / KS, nfull = K / KS;
      auto slot_at = [&](int kt) -> char* {
        const int sl = kt % NS;
        return sl == 0 ? lds0 : sl == 1 ? lds1 : sl == 2 ? lds2 : lds3;
      };
      auto issue = [&](int kt) {
        FLIDE_LDS_AS char* sb = (FLIDE_LDS_AS char*)slot_at(kt);
        if (kt < nfull) {
          const uint32_t kb = (uint32_t)(kt * KS * EB);
#pragma unroll
          for (int i = 0; i < LA; ++i) dma16b<0>(rsA, a_off32[i], kb, sb + (lw * LA + i) * 1024);
#pragma unroll
          for (int i = 0; i < LB; ++i) dma16b<NTW ? 2 : 0>(rsB, b_off32[i], kb, sb + A_BYTES + (lw * LB + i) * 1024);
        } else {   // the partial last stage: chunks past K read a 16-byte block of zeros
          const long long kb = (long long)kt * KS * EB;
          const bool in = kt * KS + kc < K;
#pragma unroll
          for (int i = 0; i < LA; ++i)
            dma16(in ? (const void*)(A + kb + a_off32[i]) : (const void*)g_zero16, sb + (lw * LA + i) * 1024);
#pragma unroll
          for (int i = 0; i < LB; ++i)
            dma16w<NTW>(in ? (const void*)(B + kb + b_off32[i]) : (const void*)g_zero16,
                        sb + A_BYTES + (lw * LB + i) * 1024);
        }
      };
      // the weight parts of stages 0 .. NS - 2 are in flight already (the host guarantees NS - 1 full stages)
#pragma unroll
      for (int st = 0; st < NS - 1; ++st) {
        FLIDE_LDS_AS char* sb = (FLIDE_LDS_AS char*)slot_at(st);
#pragma unroll
        for (int i = 0; i < LA; ++i) dma16b<0>(rsA, a_off32[i], (uint32_t)(st * KS * EB), sb + (lw * LA + i) * 1024);
      }
      wait_vmcnt<0>();
      for (int kt = 0; kt < nk; ++kt) {
        wait_stage<NS, L>(min(NS - 2, nk - 1 - kt));
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (kt + NS - 1 < nk) issue(kt + NS - 1);
      }
      return;
    }
  }
  const int wm = wave % WAVES_M, wn = wave / WAVES_M;
  const int r = l & 15, g = l >> 4;
  // LDS byte offset of this lane's chunk j within a 16-row fragment (16-bit: logical chunk s*4 + g for
  // MFMA step s; float8: chunks g and g + 4 of one step). Fragments start at multiples of 16 rows, so
  // the swizzle depends on r only: a fragment at tile row R adds the constant R * ROWB.
  int lane_off[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) lane_off[j] = r * ROWB + ((((j * 4 + g) % CPR) ^ swz<CPR>(r)) << 4);
  auto a_off = [&](int fm, int j) { return (wm * WM + fm * 16) * ROWB + lane_off[j]; };
  bool m_live[FM];
#pragma unroll
  for (int fm = 0; fm < FM; ++fm)   // a block's valid pairs come first: a fragment whose first row is padding is all padding
    m_live[fm] = __builtin_amdgcn_readfirstlane(s_pairs[wm * WM + fm * 16]) < p.n_pairs;
  int brow[FN], colbase[FN];
#pragma unroll
  for (int fn = 0; fn < FN; ++fn) {
    if constexpr (ACT == ACT_NONE) {
      brow[fn] = wn * WN + fn * 16;
      colbase[fn] = pn * BN + brow[fn];
    } else {
      constexpr int H2 = FN / 2;
      const int f = fn < H2 ? fn : fn - H2;
      brow[fn] = (fn < H2 ? 0 : BN / 2) + wn * (WN / 2) + f * 16;
      colbase[fn] = pn * (BN / 2) + wn * (WN / 2) + f * 16;
    }
  }
  auto b_off = [&](int fn, int j) { return A_BYTES + brow[fn] * ROWB + lane_off[j]; };
  const int ncols = ACT == ACT_NONE ? p.N : half;
  // gated float8 tiles: the gate and up column scales of this lane's output columns, loaded now so that the
  // epilogue does not start with a round trip (1 for 16-bit weights)
  float cs_g[FN / 2 > 0 ? FN / 2 : 1], cs_u[FN / 2 > 0 ? FN / 2 : 1];
#pragma unroll
  for (int fn = 0; fn < FN / 2; ++fn) {
    const int col = colbase[fn] + r;
    const bool ok = col < half;
    cs_g[fn] = FP8 && ACT != ACT_NONE && ok ? p.w_scale[e * p.sse + col] : (FP8 ? 0.f : 1.f);
    cs_u[fn] = FP8 && ACT != ACT_NONE && ok ? p.w_scale[e * p.sse + col + half] : (FP8 ? 0.f : 1.f);
  }
  const bool wave_live = __builtin_amdgcn_readfirstlane(colbase[0]) < ncols && m_live[0];   // stores anything

  f32x4_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // The K loop runs inside a lambda whose ring-slot pointers are __restrict__: after inlining, every
  // LDS access carries alias-scope metadata, which lets the compiler's wait-count pass see that reading
  // slot s does not alias the loads still landing in the other slots. The steady-state loop is also
  // branch-free (unconditional loads, a constant wait count): control-flow joins make that pass fall
  // back to waiting for every outstanding load before each LDS read, collapsing the ring to one stage.
  const int nk = (K + KS - 1) / KS;
  // FMA: fragment rows this wave computes: all FM, or fewer when its trailing fragments are padding
  // (1 x 4 waves span the whole block and skip in steps of 4 fragments; 2 x 2 waves skip per fragment)
  auto kloop = [&](auto fma_tag, char* __restrict__ s0, char* __restrict__ s1, char* __restrict__ s2,
                   char* __restrict__ s3) {
    constexpr int FMA = decltype(fma_tag)::value;
    auto slot_ptr = [&](int slot) -> char* { return slot == 0 ? s0 : slot == 1 ? s1 : slot == 2 ? s2 : s3; };
    // loads of a full stage kt (k0 + KS <= K) into ring slot `slot`: uniform base + lane offset
    auto issue = [&](int kt, int slot) {
      FLIDE_LDS_AS char* sb = (FLIDE_LDS_AS char*)slot_ptr(slot);
      const uint32_t kb = (uint32_t)(kt * KS * EB);
#pragma unroll
      for (int i = 0; i < LA; ++i) dma16b<0>(rsA, a_off32[i], kb, sb + (lw * LA + i) * 1024);
#pragma unroll
      for (int i = 0; i < LB; ++i) dma16b<NTW ? 2 : 0>(rsB, b_off32[i], kb, sb + A_BYTES + (lw * LB + i) * 1024);
    };
    // the partial last stage (K % KS != 0): chunks past K read a 16-byte block of zeros
    auto issue_tail = [&](int kt, int slot) {
      FLIDE_LDS_AS char* sb = (FLIDE_LDS_AS char*)slot_ptr(slot);
      const int k0 = kt * KS;
      const long long kb = (long long)k0 * EB;
      const bool in = k0 + kc < K;
#pragma unroll
      for (int i = 0; i < LA; ++i)
        dma16(in ? (const void*)(A + kb + a_off32[i]) : (const void*)g_zero16, sb + (lw * LA + i) * 1024);
#pragma unroll
      for (int i = 0; i < LB; ++i)
        dma16w<NTW>(in ? (const void*)(B + kb + b_off32[i]) : (const void*)g_zero16,
              sb + A_BYTES + (lw * LB + i) * 1024);
    };
    auto compute = [&](int slot) {
      const char* sbase = slot_ptr(slot);
      if constexpr (FMA == 0) {
        (void)sbase;   // every row of this wave is padding: loads and barriers only
      } else if constexpr (FP8) {
        i32x8_t af[FMA], bfr[FN];
#pragma unroll
        for (int fm = 0; fm < FMA; ++fm) {
          const u32x4_t lo = *(const u32x4_t*)(sbase + a_off(fm, 0));
          const u32x4_t hi = *(const u32x4_t*)(sbase + a_off(fm, 1));
          af[fm] = i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        }
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
          const u32x4_t lo = *(const u32x4_t*)(sbase + b_off(fn, 0));
          const u32x4_t hi = *(const u32x4_t*)(sbase + b_off(fn, 1));
          bfr[fn] = i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        }
#pragma unroll
        for (int fm = 0; fm < FMA; ++fm)
#pragma unroll
          for (int fn = 0; fn < FN; ++fn) acc[fm][fn] = mfma_fp8(af[fm], bfr[fn], acc[fm][fn]);
      } else {
#pragma unroll
        for (int s = 0; s < STEPS; ++s) {
          u32x4_t af[FMA], bfr[FN];
#pragma unroll
          for (int fm = 0; fm < FMA; ++fm) af[fm] = *(const u32x4_t*)(sbase + a_off(fm, s));
#pragma unroll
          for (int fn = 0; fn < FN; ++fn) bfr[fn] = *(const u32x4_t*)(sbase + b_off(fn, s));
#pragma unroll
          for (int fm = 0; fm < FMA; ++fm)
#pragma unroll
            for (int fn = 0; fn < FN; ++fn) acc[fm][fn] = Mfma16<T>::mma(af[fm], bfr[fn], acc[fm][fn]);
        }
      }
    };
    const int nfull = K / KS;
    if constexpr (NLD > 0) {
      // Compute waves of the split roles. The barrier that publishes stage kt + 1 sits in the middle of
      // stage kt's MFMAs: the fragment rows [0, H1) run first, which frees their A fragments; after the
      // barrier those are read again from stage kt + 1 under the MFMAs of rows [H1, FMA), and the B
      // fragments and the remaining A fragments follow. A wave thus enters every barrier with MFMA work
      // whose operands are in registers, instead of all waves reading the stage at once behind it
      // (compute half alone: 1474 -> 1219 cycles per float8 stage of a 128 x 256 tile; same registers).
      // A fragment is two 16-byte LDS reads: lo/hi K halves of one float8 step, or two 16-bit steps.
      static_assert(FP8 || STEPS == 2, "two 16-byte reads per fragment");
      (void)nfull;
      if constexpr (FMA == 0) {
        for (int kt = 0; kt < nk; ++kt) ring_barrier();
        return;
      } else {
        constexpr int H1 = FMA < 2 ? FMA : 2;
        u32x4_t af[FMA][2], bfr[FN][2];
        auto read_a = [&](const char* sb, int fm) {
          af[fm][0] = *(const u32x4_t*)(sb + a_off(fm, 0));
          af[fm][1] = *(const u32x4_t*)(sb + a_off(fm, 1));
        };
        auto read_b = [&](const char* sb, int fn) {
          bfr[fn][0] = *(const u32x4_t*)(sb + b_off(fn, 0));
          bfr[fn][1] = *(const u32x4_t*)(sb + b_off(fn, 1));
        };
        auto rows = [&](auto lo_tag, auto hi_tag) {   // the MFMAs of fragment rows [LO, HI) of one stage
#pragma unroll
          for (int fm = decltype(lo_tag)::value; fm < decltype(hi_tag)::value; ++fm)
#pragma unroll
            for (int fn = 0; fn < FN; ++fn) {
              if constexpr (FP8) {
                const u32x4_t *a = af[fm], *b = bfr[fn];
                acc[fm][fn] = mfma_fp8(i32x8_t{(int)a[0][0], (int)a[0][1], (int)a[0][2], (int)a[0][3], (int)a[1][0], (int)a[1][1], (int)a[1][2], (int)a[1][3]},
                                       i32x8_t{(int)b[0][0], (int)b[0][1], (int)b[0][2], (int)b[0][3], (int)b[1][0], (int)b[1][1], (int)b[1][2], (int)b[1][3]},
                                       acc[fm][fn]);
              } else {
                acc[fm][fn] = Mfma16<T>::mma(af[fm][0], bfr[fn][0], acc[fm][fn]);
                acc[fm][fn] = Mfma16<T>::mma(af[fm][1], bfr[fn][1], acc[fm][fn]);
              }
            }
        };
        auto read_rest = [&](const char* sb) {
#pragma unroll
          for (int fn = 0; fn < FN; ++fn) read_b(sb, fn);
#pragma unroll
          for (int fm = H1; fm < FMA; ++fm) read_a(sb, fm);
        };
        ring_barrier();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int fm = 0; fm < H1; ++fm) read_a(slot_ptr(0), fm);
        read_rest(slot_ptr(0));
        int slot = 0;
        // every iteration but the last publishes and reads the next stage (branch-free, see above)
        for (int kt = 0; kt + 1 < nk; ++kt) {
          const int nxt = slot + 1 == NS ? 0 : slot + 1;
          rows(std::integral_constant<int, 0>{}, std::integral_constant<int, H1>{});
          __builtin_amdgcn_sched_barrier(0);   // those MFMAs issue before the barrier, not after it
          ring_barrier();
          asm volatile("" ::: "memory");
          const char* sb = slot_ptr(nxt);
#pragma unroll
          for (int fm = 0; fm < H1; ++fm) read_a(sb, fm);
          rows(std::integral_constant<int, H1>{}, std::integral_constant<int, FMA>{});
          read_rest(sb);
          slot = nxt;
        }
        rows(std::integral_constant<int, 0>{}, std::integral_constant<int, FMA>{});
        return;
      }
    }
    // prologue: the host guarantees NS - 1 full stages, so these loads are unconditional (a conditional
    // load here would again make the wait-count pass conservative at the loop header); the weight parts
    // went out first, so the stage counts of wait_stage do not hold until everything has landed
#pragma unroll
    for (int st = 0; st < NS - 1; ++st) {   // activation parts; the weight parts are in flight already
      FLIDE_LDS_AS char* sb = (FLIDE_LDS_AS char*)slot_ptr(st);
#pragma unroll
      for (int i = 0; i < LA; ++i) dma16b<0>(rsA, a_off32[i], (uint32_t)(st * KS * EB), sb + (lw * LA + i) * 1024);
    }
    wait_vmcnt<0>();
    // steady state: stage kt computes while stages kt+1 .. kt+NS-1 load; every stage it issues is full
    const int nmain = nfull - (NS - 1);   // iterations that issue a full stage
    int kt0 = 0;
    for (; kt0 + NS <= nmain; kt0 += NS) {
#pragma unroll
      for (int slot = 0; slot < NS; ++slot) {
        wait_stage<NS, L>(NS - 2);
        ring_barrier();
        issue(kt0 + slot + NS - 1, (slot + NS - 1) % NS);
        compute(slot);
      }
    }
    // drain: the remaining issuing iterations (fewer than NS, plus the partial stage if any) and the
    // last NS - 1 stages
#pragma unroll
    for (int i = 0; i < 2 * NS - 1; ++i) {
      const int kt = kt0 + i;
      if (kt < nk) {
        wait_stage<NS, L>(min(NS - 2, nk - 1 - kt));
        ring_barrier();
        const int ks = kt + NS - 1;
        if (ks < nfull) issue(ks, (i + NS - 1) % NS);
        else if (ks < nk) issue_tail(ks, (i + NS - 1) % NS);
        compute(i % NS);
      }
    }
  };
  // a wave whose columns all lie past N (the last column tile) computes nothing either
  const bool col_live = __builtin_amdgcn_readfirstlane(colbase[0]) < ncols;
  if constexpr (WAVES_M == 1 && FM == 16) {
    int nlive = 0;   // live fragment rows (a block's valid pairs come first)
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) nlive += m_live[fm] ? 1 : 0;
    if (!col_live) kloop(std::integral_constant<int, 0>{}, lds0, lds1, lds2, lds3);
    else if (nlive <= 4) kloop(std::integral_constant<int, 4>{}, lds0, lds1, lds2, lds3);
    else if (nlive <= 8) kloop(std::integral_constant<int, 8>{}, lds0, lds1, lds2, lds3);
    else if (nlive <= 12) kloop(std::integral_constant<int, 12>{}, lds0, lds1, lds2, lds3);
    else kloop(std::integral_constant<int, 16>{}, lds0, lds1, lds2, lds3);
  } else if constexpr (WAVES_M > 1 && FM == 4) {
    // each wave skips its trailing padding fragments (waves of the lower half of a partly filled
    // block, or all of them, see padding only); the loads and barriers are the same in every variant
    int nlive = 0;
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) nlive += m_live[fm] ? 1 : 0;
    if (!col_live) nlive = 0;
    if (nlive == 0) kloop(std::integral_constant<int, 0>{}, lds0, lds1, lds2, lds3);
    else if (nlive == 1) kloop(std::integral_constant<int, 1>{}, lds0, lds1, lds2, lds3);
    else if (nlive == 2) kloop(std::integral_constant<int, 2>{}, lds0, lds1, lds2, lds3);
    else if (nlive == 3) kloop(std::integral_constant<int, 3>{}, lds0, lds1, lds2, lds3);
    else kloop(std::integral_constant<int, 4>{}, lds0, lds1, lds2, lds3);
  } else {
    kloop(std::integral_constant<int, FM>{}, lds0, lds1, lds2, lds3);
  }

  if constexpr (POST_WAIT) {
    wait_vmcnt<0>();
    ring_barrier();   // the scales are in LDS, and every compute wave is done reading the ring
  }
  typedef typename std::conditional<FP8, typename OutRound<OutT>::type, T>::type RT;   // gu rounding
  const float* ws = FP8 ? p.w_scale + e * p.sse : nullptr;
  if constexpr (BM == 128 && ACT != ACT_NONE && sizeof(typename OutTraits<OutT>::storage) == 2) {
    // Gated bm-128 products with 16-bit outputs in rows of 16-byte pieces: the tile's BM x BN/2 activation
    // values are staged in ring slot 0 (free once every compute wave is past the K loop), then each lane
    // stores 8 columns of a row, so a store instruction writes whole 256-byte row segments instead of
    // 2-byte values scattered over 4 rows (float8 gate/up at 4096 tokens 247 -> 232 us, 16-bit gate/up at
    // 8192 tokens 655 -> 627 us, 16384 tokens on skewed routing 1219 -> 1161 us; same values)
    if (!p.weights && ((uintptr_t)p.out & 15) == 0 && p.sc % 8 == 0) {
      typedef typename OutTraits<OutT>::storage S;
      constexpr int TC = BN / 2;
      static_assert(BM * TC * 2 <= STAGE, "the staged tile fits a ring slot");
      S* tile = (S*)lds0;
      if constexpr (!POST_WAIT) ring_barrier();   // every compute wave is done reading the ring
      if (wave_live) {
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) {
          if (!m_live[fm]) continue;
          const int row0 = wm * WM + fm * 16;
          float rs[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) rs[i] = FP8 ? s_ascale[row0 + g * 4 + i] : 1.f;
#pragma unroll
          for (int fn = 0; fn < FN / 2; ++fn) {
            const int col = colbase[fn] + r;
            const int lc = col - pn * TC;
#pragma unroll
            for (int i = 0; i < 4; ++i) {   // the values store_frag computes, in the same order
              const float gg = round_in<RT>(acc[fm][fn][i] * rs[i] * cs_g[fn]);
              const float uu = round_in<RT>(acc[fm][fn + FN / 2][i] * rs[i] * cs_u[fn]);
              tile[(row0 + g * 4 + i) * TC + lc] = OutTraits<OutT>::conv(act_f32<ACT>(gg, uu));
            }
          }
        }
      }
      ring_barrier();
      constexpr int LPR = TC / 8;        // lanes per row, 8 columns each
      constexpr int RPP = NW * 64 / LPR;   // rows per pass
      const int c8 = (tid % LPR) * 8;
      const int col0 = pn * TC + c8;
      for (int rr = tid / LPR; rr < BM; rr += RPP) {
        const int pair = s_pairs[rr];
        if (pair >= p.n_pairs || col0 >= half) continue;
        const uint4 q = *(const uint4*)(tile + rr * TC + c8);
        S* o = (S*)p.out + (long long)pair * p.sc + col0;
        if (col0 + 8 <= half) {
          *(uint4*)o = q;
        } else {
          const S ev[8] = {(S)(q.x & 0xffff), (S)(q.x >> 16), (S)(q.y & 0xffff), (S)(q.y >> 16),
                           (S)(q.z & 0xffff), (S)(q.z >> 16), (S)(q.w & 0xffff), (S)(q.w >> 16)};
#pragma unroll
          for (int j = 0; j < 7; ++j)
            if (col0 + j < half) o[j] = ev[j];
        }
      }
      return;
    }
  }
  if (!wave_live) return;
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
    if (!m_live[fm]) continue;
    const int row0 = wm * WM + fm * 16;
    float rs[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) rs[i] = FP8 ? s_ascale[row0 + g * 4 + i] : 1.f;
    if constexpr (ACT == ACT_NONE && !FP8 && std::is_same<OutT, float>::value) {
      if (p.pack_f32) {
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) store_frag_f32x4(p, s_pairs, s_wt, row0, colbase[fn], acc[fm][fn], rs, 1.f);
      } else {
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
          const int col = colbase[fn] + r;
          store_frag<OutT, ACT, RT>(p, s_pairs, row0, col, acc[fm][fn], acc[fm][fn], 1.f, 1.f, rs, col < p.N, s_wt);
        }
      }
    } else if constexpr (ACT == ACT_NONE) {
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const int col = colbase[fn] + r;
        const bool ok = col < p.N;
        store_frag<OutT, ACT, RT>(p, s_pairs, row0, col, acc[fm][fn], acc[fm][fn],
                                  FP8 ? (ok ? ws[col] : 0.f) : 1.f, 1.f, rs, ok, s_wt);
      }
    } else {
#pragma unroll
      for (int fn = 0; fn < FN / 2; ++fn) {
        const int col = colbase[fn] + r;
        const bool ok = col < half;
        store_frag<OutT, ACT, RT>(p, s_pairs, row0, col, acc[fm][fn], acc[fm][fn + FN / 2], cs_g[fn], cs_u[fn],
                                  rs, ok);
      }
    }
  }
}

// The current device's CUs, rounded down to a multiple of 8 (0 if unknown).
int cu_count() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cus[dev] = n / 8 * 8;
  }
  return cus[dev];
}

// Float8 plain (down) products with short rows (K <= 768, the 704-wide down product): the block's
// activation rows stay resident in LDS and NLD loader waves stream the expert's weight tiles through a
// ring, continuously over several column tiles. With K this short, the per-tile kernel above spends
// most of a block's life filling and draining its ring (6 stages per tile); here the ring runs across
// tile boundaries and the activation rows are read once per block, not once per tile.
//
// Roles: waves 0-7 (2 x 4, each 64 rows x 32 columns of a 128 x 128 tile) load the activation rows
// once, then only read LDS, issue MFMAs and store; waves 8 .. 8 + NLD - 1 only issue direct-to-LDS
// weight loads and wait for them. A wave's vmcnt counts its own memory operations, so the compute
// waves' epilogue stores never hold up the loads' waits (in a single-role kernel every wait after a
// store would wait for that store too). One barrier per stage: at stage s the loaders have waited for
// stage s and the compute waves have finished stage s - 1, whose ring slot the loaders refill right
// after it. Each loader issues 1 / NLD of a stage's weight rows: one wave issuing them all measured
// as the bound of this kernel (the float8 down product at 4096 tokens 247 us with one loader wave,
// 204 with two, 190 with four; eight need more waves per SIMD than the compute waves' registers allow).
// The column scales of tile t travel with every stage of tile t (BN / 64 loads of 256 bytes, issued by
// loaders 0 .. BN / 64 - 1, so each loader's stages hold the same number of loads) into s_ws[t & 1],
// read by the tile's epilogue.
//
// Arithmetic: the same 128-wide K steps, lane mapping, MFMA and epilogue order as grouped_dma, so the
// output bits are the same.
template <typename OutT, int NS, int BN, int KT_MAX, int XB, int NLD, bool WIDE, bool AREG = false>
__global__ __launch_bounds__((8 + NLD) * 64, 1) void grouped_fp8_resident(GroupArgs p, int tpb, int nch, int cus) {
  constexpr int BM = 128, ROWB = 128;
  // compute waves: WIDE (16-bit outputs, aligned): 8 x 1 waves of 16 rows x BN columns, each wave owning
  // whole output row segments of the tile; else 2 x 4 waves of 64 x BN / 4
  constexpr int WAVES_M = WIDE ? 8 : 2, WM = BM / WAVES_M, WN = BN / (8 / WAVES_M), FM = WM / 16, FN = WN / 16;
  constexpr int A_KT = BM * ROWB, B_BYTES = BN * ROWB;
  constexpr int LB = BN / 8, LW = BN / 64;   // loads per stage: weight rows, scales
  constexpr int LBW = LB / NLD;               // weight loads per loader wave and stage
  static_assert(LB % NLD == 0 && (NLD == 1 || LW <= NLD), "loaders split the stage evenly");
  static_assert((NS - 1) * (LBW + LW) < 64 && 2 * KT_MAX < 64, "loads in flight must fit vmcnt");
  static_assert(NS >= 3 && NS <= 7 && BN % 64 == 0 && FN >= 1, "ring of 3..7 slots, 64-row multiples");
  static_assert(!AREG || (WIDE && FM == 1), "operand rows in registers: one 16-row fragment per wave");

  __shared__ __attribute__((aligned(1024))) char s_a[AREG ? 16 : KT_MAX * A_KT];
  __shared__ __attribute__((aligned(1024))) char s_b[NS * B_BYTES];
  __shared__ __attribute__((aligned(16))) float s_ws[2][BN];
  __shared__ int s_pairs[BM];
  __shared__ float s_ascale[BM];
  __shared__ float s_wt[BM];
  // WIDE epilogue: each wave turns 4 output rows at a time into row-major 16-bit values here
  __shared__ __attribute__((aligned(16))) uint16_t s_stage[WIDE ? 8 : 1][WIDE ? 4 * BN : 8];

  const int tid = threadIdx.x, l = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // items (block, column chunk), chunked per XCD as in grouped_dma
  const int CH = nch * XB;
  const int b = blockIdx.x;
  const int j = b >> 3;
  const int widx = ((j / CH) * 8 + (b & 7)) * CH + j % CH;
  const int ntn = (p.N + BN - 1) / BN;
  int pm, c, t0, nt;
  if (cus > 0) {
    // Halves of the column tiles (nch = 2), except that the last m blocks, whose items the grid
    // dispatches last, are cut in thirds, with m such that the items fill whole rounds of the CUs:
    // the last round then runs items of 8 tiles instead of 11 (at 4096 tokens 648 items, 2.5 rounds,
    // become 768)
    const int nused = *p.used / BM;
    const int m = max(0, min(nused, (2 * nused + cus - 1) / cus * cus - 2 * nused));
    const int nh = 2 * (nused - m);   // items of the halved blocks
    if (widx >= nh + 3 * m) return;
    const int tpb3 = (ntn + 2) / 3;
    if (widx < nh) {
      pm = widx / 2, c = widx % 2;
      t0 = c * tpb;
      nt = min(t0 + tpb, ntn) - t0;
    } else {
      pm = nused - m + (widx - nh) / 3, c = (widx - nh) % 3;
      t0 = c * tpb3;
      nt = min(t0 + tpb3, ntn) - t0;
    }
  } else {
    pm = widx / nch, c = widx % nch;
    if (pm >= p.nbm || pm * BM >= *p.used) return;
    t0 = c * tpb;
    nt = min(t0 + tpb, ntn) - t0;
  }
  if (nt <= 0) return;
  const int K = p.K, KT = (K + ROWB - 1) / ROWB;
  const int S = nt * KT;
  const long long e = p.blocks[pm];
  for (int r = tid; r < BM; r += (8 + NLD) * 64) {
    const int pair = p.rows[pm * BM + r];
    s_pairs[r] = pair;
    const bool ok = pair < p.n_pairs;
    const long long src = p.by_token ? pair / p.topk : pair;
    s_ascale[r] = ok ? p.a_scale[src] : 0.f;
    s_wt[r] = ok && p.weights ? p.weights[pair] : 1.f;
  }
  __syncthreads();
  // lane l of a 1 KB load fills row l / 8 (of 8) at chunk position l % 8, which holds logical chunk
  // (l % 8) ^ (row & 7); rows start at multiples of 8, so the chunk's byte offset depends on l only
  const int kc = ((l & 7) ^ (l >> 3)) * 16;

  if (wave >= 8) {   // ---------------- loaders ----------------
    const int li = wave - 8;
    const char* B = (const char*)p.w + e * p.sbe;
    const float* WS = p.w_scale + e * p.sse;
    auto issue = [&](int s) {
      const int t = t0 + s / KT, kt = s % KT, slot = s % NS;
      FLIDE_LDS_AS char* sb = (FLIDE_LDS_AS char*)(s_b + slot * B_BYTES);
      const int k0 = kt * ROWB;
      const bool in = k0 + kc < K;
#pragma unroll
      for (int i = 0; i < LBW; ++i) {   // rows (li * LBW + i) * 8 .. + 7 of the tile
        const int ii = li * LBW + i;
        const int n = min(t * BN + ii * 8 + (l >> 3), p.N - 1);
        dma16(in ? (const void*)(B + (long long)n * p.sbn + k0 + kc) : (const void*)g_zero16, sb + ii * 1024);
      }
      for (int q = li; q < LW; q += NLD) {
        const int col = min(t * BN + q * 64 + l, p.N - 1);
        __builtin_amdgcn_global_load_lds((const FLIDE_GLOBAL_AS void*)(WS + col),
                                         (FLIDE_LDS_AS void*)&s_ws[t & 1][q * 64], 4, 0, 0);
      }
    };
    // LPS: this loader's loads per stage (its weight rows, plus a scale load for loaders below LW)
    auto loop = [&](auto lps_tag) {
      constexpr int LPS = decltype(lps_tag)::value;
      for (int s = 0; s < NS - 1 && s < S; ++s) issue(s);
      for (int s = 0; s < S; ++s) {
        const int ahead = min(NS - 2, S - 1 - s);   // stages after s already in flight
        if (NS > 6 && ahead >= 5) wait_vmcnt<(NS > 6 ? 5 : 0) * LPS>();
        else if (NS > 5 && ahead >= 4) wait_vmcnt<(NS > 5 ? 4 : 0) * LPS>();
        else if (NS > 4 && ahead >= 3) wait_vmcnt<(NS > 4 ? 3 : 0) * LPS>();
        else if (NS > 3 && ahead >= 2) wait_vmcnt<(NS > 3 ? 2 : 0) * LPS>();
        else if (ahead >= 1) wait_vmcnt<LPS>();
        else wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (s + NS - 1 < S) issue(s + NS - 1);
      }
    };
    if constexpr (NLD == 1) loop(std::integral_constant<int, LBW + LW>{});
    else if (li < LW) loop(std::integral_constant<int, LBW + 1>{});
    else loop(std::integral_constant<int, LBW>{});
    return;
  }

  // ---------------- compute waves ----------------
  if constexpr (!AREG) {
    const char* A = (const char*)p.a;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int row = (wave * 2 + q) * 8 + (l >> 3);
      const int pair = s_pairs[row];
      const long long src = pair < p.n_pairs ? (p.by_token ? pair / p.topk : pair) : 0;
      const char* ar = A + src * p.sa;
      for (int kt = 0; kt < KT; ++kt) {
        const bool in = kt * ROWB + kc < K;
        dma16(in ? (const void*)(ar + kt * ROWB + kc) : (const void*)g_zero16,
              (FLIDE_LDS_AS char*)(s_a + kt * A_KT) + (wave * 2 + q) * 1024);
      }
    }
    wait_vmcnt<0>();
  }
  const int wm = wave % WAVES_M, wn = wave / WAVES_M;
  const int r = l & 15, g = l >> 4;
  int lane_off[2];
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) lane_off[jj] = r * ROWB + ((((jj * 4 + g) % 8) ^ (r & 7)) << 4);
  int nlive = 0;
#pragma unroll
  for (int fm = 0; fm < FM; ++fm)
    nlive += __builtin_amdgcn_readfirstlane(s_pairs[wm * WM + fm * 16]) < p.n_pairs ? 1 : 0;
  typedef typename OutTraits<OutT>::storage St;

  auto run = [&](auto fma_tag) {
    constexpr int FMA = decltype(fma_tag)::value;
    f32x4_t acc[FM][FN];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) acc[fm][fn] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // the wave's rows are the same for every tile: their pair, activation scale and routing weight
    // stay in registers (row wm * WM + fm * 16 + g * 4 + i of output register i)
    constexpr int FR = FMA > 0 ? FMA : 1;
    int prow[FR][4];
    float rsc[FR][4], rwt[FR][4];
#pragma unroll
    for (int fm = 0; fm < FR; ++fm)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = wm * WM + fm * 16 + g * 4 + i;
        prow[fm][i] = s_pairs[row];
        rsc[fm][i] = s_ascale[row];
        rwt[fm][i] = s_wt[row];
      }
    const bool mulw = p.weights != nullptr;
    int kt = 0, slot = 0, t = t0;
    for (int s = 0; s < S; ++s) {
      ring_barrier();
      asm volatile("" ::: "memory");
      if constexpr (FMA > 0) {
        const char* sa_ = s_a + kt * A_KT + wm * WM * ROWB;
        const char* sb_ = s_b + slot * B_BYTES + wn * WN * ROWB;
        i32x8_t af[FMA], bfr[FN];
#pragma unroll
        for (int fm = 0; fm < FMA; ++fm) {
          const u32x4_t lo = *(const u32x4_t*)(sa_ + fm * 16 * ROWB + lane_off[0]);
          const u32x4_t hi = *(const u32x4_t*)(sa_ + fm * 16 * ROWB + lane_off[1]);
          af[fm] = i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        }
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
          const u32x4_t lo = *(const u32x4_t*)(sb_ + fn * 16 * ROWB + lane_off[0]);
          const u32x4_t hi = *(const u32x4_t*)(sb_ + fn * 16 * ROWB + lane_off[1]);
          bfr[fn] = i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        }
#pragma unroll
        for (int fm = 0; fm < FMA; ++fm)
#pragma unroll
          for (int fn = 0; fn < FN; ++fn) acc[fm][fn] = mfma_fp8(af[fm], bfr[fn], acc[fm][fn]);
        if (WIDE && kt == KT - 1) {   // epilogue of tile t, 4 rows at a time through LDS (see the launcher)
          float cs[FN];
#pragma unroll
          for (int fn = 0; fn < FN; ++fn) cs[fn] = s_ws[t & 1][wn * WN + fn * 16 + r];
          uint16_t* stg = s_stage[wave];
          const int c8 = (l & 15) * 8;   // this lane's 8 columns of the staged row l / 16 (= g)
          const int col0 = t * BN + c8;
#pragma unroll
          for (int i = 0; i < 4; ++i) {   // output register i: rows g * 4 + i (one per lane group g)
#pragma unroll
            for (int fn = 0; fn < FN; ++fn) {
              float v = acc[0][fn][i] * rsc[0][i] * cs[fn];
              if (mulw) v *= rwt[0][i];
              stg[g * BN + fn * 16 + r] = OutTraits<OutT>::conv(v);
            }
            __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): the wave's staging writes are done
            const uint4 q = *(const uint4*)(stg + g * BN + c8);
            const int pair = prow[0][i];
            if (pair < p.n_pairs && col0 < p.N) {
              uint16_t* o = (uint16_t*)p.out + (long long)pair * p.sc + col0;
              if (col0 + 8 <= p.N) {
                *(uint4*)o = q;
              } else {
                const uint16_t e[8] = {(uint16_t)(q.x & 0xffff), (uint16_t)(q.x >> 16), (uint16_t)(q.y & 0xffff),
                                       (uint16_t)(q.y >> 16), (uint16_t)(q.z & 0xffff), (uint16_t)(q.z >> 16),
                                       (uint16_t)(q.w & 0xffff), (uint16_t)(q.w >> 16)};
#pragma unroll
                for (int j = 0; j < 7; ++j)
                  if (col0 + j < p.N) o[j] = e[j];
              }
            }
          }
#pragma unroll
          for (int fn = 0; fn < FN; ++fn) acc[0][fn] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        } else if (!WIDE && kt == KT - 1) {   // epilogue of tile t: out = acc * s_a[row] * s_w[col] (* routing weight)
          float cs[FN];
#pragma unroll
          for (int fn = 0; fn < FN; ++fn) cs[fn] = s_ws[t & 1][wn * WN + fn * 16 + r];
#pragma unroll
          for (int fm = 0; fm < FMA; ++fm) {
#pragma unroll
            for (int fn = 0; fn < FN; ++fn) {
              const int col = t * BN + wn * WN + fn * 16 + r;
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const int pair = prow[fm][i];
                if (pair < p.n_pairs && col < p.N) {
                  float v = acc[fm][fn][i] * rsc[fm][i] * cs[fn];
                  if (mulw) v *= rwt[fm][i];
                  ((St*)p.out)[(long long)pair * p.sc + col] = OutTraits<OutT>::conv(v);
                }
              }
              acc[fm][fn] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            }
          }
        }
      }
      if (++slot == NS) slot = 0;
      if (++kt == KT) { kt = 0; ++t; }
    }
  };
  // AREG (the WIDE layout): lane (r, g) of wave w holds row 16 w + r's K chunks g and g + 4 of every
  // 128-wide k-tile, the MFMA's A operand for that k-tile, loaded once per block straight from global
  // memory into registers. The LDS then holds only the weight ring, deep enough (7 slots: six 16 KB
  // stages in flight per CU instead of two) that the weight stream is no longer bound by the bytes a
  // CU keeps in flight.
  auto run_areg = [&](auto fma_tag) {
    constexpr int FMA = decltype(fma_tag)::value;
    i32x8_t areg[KT_MAX];
    if constexpr (FMA > 0) {
      const int pair = s_pairs[wave * 16 + r];
      const long long src = pair < p.n_pairs ? (p.by_token ? pair / p.topk : pair) : 0;
      const char* ar = (const char*)p.a + src * p.sa;
#pragma unroll
      for (int kt = 0; kt < KT_MAX; ++kt) {   // chunks past K are zeros
        const int k0 = kt * ROWB + g * 16, k1 = k0 + 64;
        uint4 lo = make_uint4(0u, 0u, 0u, 0u), hi = lo;
        if (k0 < K) lo = *(const uint4*)(ar + k0);
        if (k1 < K) hi = *(const uint4*)(ar + k1);
        areg[kt] = i32x8_t{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
      }
    }
    f32x4_t acc[FN];
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) acc[fn] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    int prow[4];
    float rsc[4], rwt[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {   // output register i: row 16 w + g * 4 + i
      const int row = wave * 16 + g * 4 + i;
      prow[i] = s_pairs[row];
      rsc[i] = s_ascale[row];
      rwt[i] = s_wt[row];
    }
    const bool mulw = p.weights != nullptr;
    int slot = 0;
    for (int t = t0; t < t0 + nt; ++t) {
#pragma unroll
      for (int kt = 0; kt < KT_MAX; ++kt) {
        if (kt < KT) {
          ring_barrier();
          asm volatile("" ::: "memory");
          if constexpr (FMA > 0) {
            const char* sb_ = s_b + slot * B_BYTES;
#pragma unroll
            for (int h = 0; h < 2; ++h) {   // the tile's columns in two halves (registers)
              i32x8_t bfr[FN / 2];
#pragma unroll
              for (int fn = 0; fn < FN / 2; ++fn) {
                const char* fb = sb_ + (h * (FN / 2) + fn) * 16 * ROWB;
                const u32x4_t lo = *(const u32x4_t*)(fb + lane_off[0]);
                const u32x4_t hi = *(const u32x4_t*)(fb + lane_off[1]);
                bfr[fn] = i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
              }
#pragma unroll
              for (int fn = 0; fn < FN / 2; ++fn)
                acc[h * (FN / 2) + fn] = mfma_fp8(areg[kt], bfr[fn], acc[h * (FN / 2) + fn]);
            }
          }
          if (++slot == NS) slot = 0;
        }
      }
      if constexpr (FMA > 0) {   // epilogue of tile t, 4 rows at a time through LDS, as the WIDE layout above
        float cs[FN];
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) cs[fn] = s_ws[t & 1][fn * 16 + r];
        uint16_t* stg = s_stage[wave];
        const int c8 = (l & 15) * 8;
        const int col0 = t * BN + c8;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int fn = 0; fn < FN; ++fn) {
            float v = acc[fn][i] * rsc[i] * cs[fn];
            if (mulw) v *= rwt[i];
            stg[g * BN + fn * 16 + r] = OutTraits<OutT>::conv(v);
          }
          __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): the wave's staging writes are done
          const uint4 q = *(const uint4*)(stg + g * BN + c8);
          const int pair = prow[i];
          if (pair < p.n_pairs && col0 < p.N) {
            uint16_t* o = (uint16_t*)p.out + (long long)pair * p.sc + col0;
            if (col0 + 8 <= p.N) {
              *(uint4*)o = q;
            } else {
              const uint16_t e[8] = {(uint16_t)(q.x & 0xffff), (uint16_t)(q.x >> 16), (uint16_t)(q.y & 0xffff),
                                     (uint16_t)(q.y >> 16), (uint16_t)(q.z & 0xffff), (uint16_t)(q.z >> 16),
                                     (uint16_t)(q.w & 0xffff), (uint16_t)(q.w >> 16)};
#pragma unroll
              for (int j = 0; j < 7; ++j)
                if (col0 + j < p.N) o[j] = e[j];
            }
          }
        }
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) acc[fn] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
    }
  };
  if constexpr (AREG) {
    if (nlive == 0) run_areg(std::integral_constant<int, 0>{});
    else run_areg(std::integral_constant<int, 1>{});
  } else if constexpr (FM == 1) {
    if (nlive == 0) run(std::integral_constant<int, 0>{});
    else run(std::integral_constant<int, 1>{});
  } else {
    if (nlive == 0) run(std::integral_constant<int, 0>{});
    else if (nlive == 1) run(std::integral_constant<int, 1>{});
    else if (nlive == 2) run(std::integral_constant<int, 2>{});
    else if (nlive == 3) run(std::integral_constant<int, 3>{});
    else run(std::integral_constant<int, 4>{});
  }
}

// grouped_fp8_resident for a float8 plain product with 128-row blocks: K of 129..768 (whole 16-byte
// chunks). Column tiles are split into chunks so that the grid holds at least about 640 items
// (2.5 per CU at one workgroup per CU); returns FLIDE_MOE_ERR_TILE when the shape does not fit.
template <typename OutT, int NS = 3, int BN = 128, int NLD = 4>
int launch_fp8_resident(GroupArgs& p, hipStream_t st) {
  constexpr int KT_MAX = 6, XB = 4;
  // s_ws[t & 1] is refilled for tile t + 2 from stage (t + 2) * KT - (NS - 1) on, which must come after
  // tile t's epilogue (stage (t + 1) * KT - 1): KT >= NS - 1 stages of K
  if (p.K <= (NS - 2) * 128 || p.K > KT_MAX * 128 || p.K % 16) return FLIDE_MOE_ERR_TILE;
  const int ntn = (p.N + BN - 1) / BN;
  int nch = (640 + p.nbm - 1) / max(p.nbm, 1);
  nch = max(1, min(nch, ntn));
  const int tpb = (ntn + nch - 1) / nch;
  nch = (ntn + tpb - 1) / tpb;
  p.ntn = ntn;
  // two chunks per block: the last blocks' items may be cut in thirds (see the kernel), up to 3 per block
  const int cus = nch == 2 ? cu_count() : 0;
  const int items = p.nbm * (cus > 0 ? 3 : nch);
  const int round = 8 * nch * XB;
  dim3 grid((items + round - 1) / round * round), block((8 + NLD) * 64);
  // 16-bit outputs whose rows take 16-byte stores: the WIDE layout, where each store instruction writes
  // 4 rows x 256 bytes (whole lines) instead of 64 scattered 2-byte values
  typedef typename OutTraits<OutT>::storage S;
  if constexpr (sizeof(S) == 2) {
    if (p.sc % 8 == 0 && (uintptr_t)p.out % 16 == 0) {
      // K of 641..768 (six k-tiles, as the 704-wide down product) with 16-byte aligned activation rows:
      // the rows in registers and a 7-slot weight ring (its column scales need KT >= 6 slots of lead)
      if ((p.K + 127) / 128 == KT_MAX && p.sa % 16 == 0 && (uintptr_t)p.a % 16 == 0) {
        grouped_fp8_resident<OutT, 7, BN, KT_MAX, XB, NLD, true, true><<<grid, block, 0, st>>>(p, tpb, nch, cus);
        return FLIDE_MOE_OK;
      }
      grouped_fp8_resident<OutT, NS, BN, KT_MAX, XB, NLD, true><<<grid, block, 0, st>>>(p, tpb, nch, cus);
      return FLIDE_MOE_OK;
    }
  }
  grouped_fp8_resident<OutT, NS, BN, KT_MAX, XB, NLD, false><<<grid, block, 0, st>>>(p, tpb, nch, cus);
  return FLIDE_MOE_OK;
}

// Tiles (default BN = 256 weight rows). Two waves per SIMD matter more than deeper rings or larger
// tiles here (measured: variants with one wave per SIMD lose 15-40% on gfx950; rings of 4-6 stages
// were slower too): either two 4-wave workgroups per CU, or one 8-wave workgroup:
//  bm 256 (16-bit): 1 x 4 waves of 256 x 64, 64-byte stage rows, 4 stages = 128 KB, one workgroup per CU;
//     the waves share all 256 rows, so a block's padded tail costs no MFMA time
//  bm 128 (16-bit): 2 x 4 waves of 64 x 64 in one 512-thread workgroup, 3 stages. Gated (gate/up):
//     128-byte stage rows (144 KB), 4-10% faster than two workgroups of 2 x 2 waves with 64-byte rows
//     at 4096-16384 tokens; plain (down): 64-byte rows (72 KB; 645 -> 598 us against 2 x 2 waves)
//  bm 64  (16-bit): 128-byte stage rows, 3 stages. Gated: 1 x 4 waves of 64 x 32, BN = 128 (72 KB, two
//     workgroups per CU); plain: 2 x 4 waves of 32 x 64 (120 KB). At 1024-2048 tokens 12-15% (gate/up)
//     and 3-7% (down) faster than 1 x 4 waves with 64-byte rows
//  float8 (128-byte stage rows, one 128-wide MFMA step): bm 64 with BN = 128 and 2 stages (48 KB, three
//     workgroups per CU); bm 128 in 8-wave workgroups: the plain (down) product 64 x 32 per wave, 2
//     stages (375 -> 290 us at 4096 tokens; with K <= 768 grouped_fp8_resident replaces it, 180 us),
//     the gated (gate/up) product 64 x 64 per wave with BN = 256
//     and 3 stages (144 KB; 5-10% faster than 2 x 2 waves of BN 128 at 4096-16384 tokens), its loads
//     issued by 4 more waves (split roles: 256 -> 241 us at 4096 tokens); bm 256:
//     2 stages = 128 KB
//  bm 32 (decode): 128-byte stage rows, 3 stages. 16-bit: BN = 64 (gated 2 x 2 waves, plain 1 x 4),
//     36 KB, three workgroups per CU; float8: 1 x 4 waves, BN = 128, 60 KB. Weight-streaming bound:
//     whole 128-byte lines per row and stage read measurably faster than the half-line pairs of the
//     register-streaming kernel (gate/up 180 -> 170 us, down 112 -> 94 us at 64 tokens; fp8 110 ->
//     95 / 61 -> 52 us)
// ---------------------------------------------------------------------------------------------------
// Persistent products: bm 128, BN 256, split roles (gated: float8 or 16-bit, staged epilogue; plain:
// 16-bit weights with float32 outputs)
// ---------------------------------------------------------------------------------------------------
// At 4096 tokens the per-tile kernel spends about a third of a float8 gate/up tile's life outside its K
// loop: the start-up chain (the item's expert, its pairs, the first stages) and the epilogue, while the
// CU's load pipe idles. Here one workgroup per CU walks the items of its XCD's range (items j, j + W,
// j + 2W, ... of the range for the W workgroups of that XCD, the order in which the per-tile launch's
// workgroups are dispatched) and the stage ring runs on across items. During an item's K loop, compute
// wave 0 finds the next item's block, column tile and expert, waves 0-1 bring its pairs and activation
// scales into the other half of double-buffered LDS, and every compute wave loads its column scales; the
// loader waves build the next item's operand offsets and switch to them two stages before the item
// ends, so its first stages land during this item's last MFMAs and epilogue. The next item's metadata
// moves only through LDS, written after one stage barrier and read after a later one (see act()).
// Barriers per item, for every wave: the item's nk stage barriers, then two in the epilogue.
// The arithmetic is grouped_dma's (K steps, MFMA order, epilogue), so the bits are too. 16-bit weights:
// 64 K per 128-byte stage row as two 32-wide MFMA steps, no scales. Plain (down) products: items in
// grouped_dma's block-major order, the rows' routing weights in place of the activation scales, and
// the float32 epilogue of 16-byte stores from registers (no staging, no epilogue barriers).
template <typename T, typename OutT, int ACT>
__global__ __launch_bounds__(12 * 64, 1) void grouped_persist(GroupArgs p) {
  constexpr bool FP8 = std::is_same<T, Fp8Tag>::value;
  constexpr bool GATED = ACT != ACT_NONE;
  constexpr int EPB = GATED ? 2 : 0;   // barriers in an item's epilogue
  constexpr int EB = DmaElem<T>::BYTES;
  constexpr int BM = 128, BN = 256, NS = 3, ROWB = 128, NW = 8, NLD = 4, WAVES_M = 2;
  constexpr int CPR = 8, RPI = 8, KS = ROWB / EB;   // K per 128-byte stage row
  constexpr int A_BYTES = BM * ROWB, STAGE = A_BYTES + BN * ROWB;
  constexpr int LA = BM / (NLD * RPI), LB = BN / (NLD * RPI), L = LA + LB;
  constexpr int WM = BM / WAVES_M, WN = BN / (NW / WAVES_M), FM = WM / 16, FN = WN / 16, TC = BN / 2;
  static_assert(FM == 4 && FN == 4 && (NS - 1) * L < 64, "2 x 4 waves of 64 x 64, loads in flight fit vmcnt");
  typedef typename OutTraits<OutT>::storage S;
  typedef typename std::conditional<FP8, typename OutRound<OutT>::type, T>::type RT;   // gate/up rounding
  static_assert(GATED ? sizeof(S) == 2 : (!FP8 && std::is_same<OutT, float>::value),
                "gated: 16-bit outputs; plain: 16-bit weights, float32 outputs");
  __shared__ __attribute__((aligned(1024))) char lds0[STAGE];
  __shared__ __attribute__((aligned(1024))) char lds1[STAGE];
  __shared__ __attribute__((aligned(1024))) char lds2[STAGE];
  __shared__ int s_pairs[2][BM];
  __shared__ float s_ascale[2][BM];   // the rows' activation scales (gated float8) or routing weights (plain)
  __shared__ int s_meta[2][4];   // the item's block, column tile and expert

  const int tid = threadIdx.x, l = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int K = p.K, half = p.N / 2, nk = K / KS;
  const int ncols = GATED ? half : p.N;
  // this workgroup's items: XCD x's range of the items in use, every W-th from j
  const int nused = *p.used / BM;
  const long long R = (long long)nused * p.ntn;
  const int x = blockIdx.x & 7, W = gridDim.x >> 3, j = blockIdx.x >> 3;
  const long long it0 = R * x / 8 + j, it_end = R * (x + 1) / 8;
  const int n_items = it0 < it_end ? (int)((it_end - it0 + W - 1) / W) : 0;
  if (n_items == 0) return;

  // item -> (block, column tile, expert) in grouped_dma's prefill order (column-tile major inside an
  // expert for the gated products, block major for the plain ones), by one wave: expert_run's window
  // loads, issued apart from their use
  int wlo = 0, whi = 0;
  auto window = [&](long long it) {
    const int blk = (int)(it / p.ntn);
    const int li = blk - 63 + l, hi = blk + l;
    wlo = li >= 0 ? p.blocks[li] : -1;
    whi = hi < nused ? p.blocks[hi] : -1;
  };
  auto resolve = [&](long long it, int* meta) {
    const int blk = (int)(it / p.ntn);
    const int e = __builtin_amdgcn_readfirstlane(whi);   // lane 0 read blocks[blk]
    const unsigned long long ml = __ballot(wlo != e), mh = __ballot(whi != e);
    const int s0 = __builtin_amdgcn_readfirstlane(
        ml ? blk - 63 + (63 - __builtin_clzll(ml)) + 1 : expert_first_block(p.blocks, blk - 64, e, l));
    const int s1 = __builtin_amdgcn_readfirstlane(
        mh ? blk + __builtin_ctzll(mh) : expert_end_block(p.blocks, blk + 64, e, nused, l));
    const int local = (int)(it - (long long)s0 * p.ntn), nb = s1 - s0;
    if (l == 0) {
      meta[0] = GATED ? s0 + local % nb : s0 + local / p.ntn;
      meta[1] = GATED ? local / nb : local % p.ntn;
      meta[2] = e;
    }
  };
  auto scale_of = [&](int pair) {   // the row value the epilogue reads: activation scale or routing weight
    if constexpr (!GATED) return p.weights && pair < p.n_pairs ? p.weights[pair] : 1.f;
    if constexpr (!FP8) return 1.f;
    return pair < p.n_pairs ? p.a_scale[p.by_token ? pair / p.topk : pair] : 0.f;
  };

  // start-up: the first item's metadata, pairs and scales
  if (wave == 0) {
    window(it0);
    resolve(it0, s_meta[0]);
  }
  lds_barrier();
  if (tid < BM) {
    const int pair = p.rows[s_meta[0][0] * BM + tid];
    s_pairs[0][tid] = pair;
    s_ascale[0][tid] = scale_of(pair);
  }
  lds_barrier();

  if (wave >= NW) {   // ---------------- loaders ----------------
    const int lw = wave - NW;
    const int kc = ((l % CPR) ^ swz<CPR>(l / CPR)) * 16;   // this lane's chunk's K offset (bytes)
    const long long a_rows = p.by_token ? (p.n_pairs + p.topk - 1) / p.topk : p.n_pairs;
    const __amdgpu_buffer_rsrc_t rsA = buf_rsrc(p.a, ((a_rows - 1) * p.sa + K) * EB);
    __amdgpu_buffer_rsrc_t rsB[2];
    uint32_t b_off[2][LB], a_off[2][LA];   // [item parity]
    auto set_ops = [&](int buf) {   // the operands of the item whose metadata is in buffer buf
      const int pn = __builtin_amdgcn_readfirstlane(s_meta[buf][1]);
      const long long e = __builtin_amdgcn_readfirstlane(s_meta[buf][2]);
      rsB[buf] = buf_rsrc((const char*)p.w + e * p.sbe * EB, ((long long)(p.N - 1) * p.sbn + K) * EB);
#pragma unroll
      for (int i = 0; i < LB; ++i) {
        const int row = (lw * LB + i) * RPI + l / CPR;
        long long n;
        if constexpr (GATED) {
          int cc = pn * TC + (row < TC ? row : row - TC);
          if (cc >= half) cc = half - 1;
          n = row < TC ? cc : cc + half;
        } else {
          n = min(pn * BN + row, p.N - 1);
        }
        b_off[buf][i] = (uint32_t)(n * p.sbn * EB + kc);
      }
#pragma unroll
      for (int i = 0; i < LA; ++i) {
        const int pair = s_pairs[buf][(lw * LA + i) * RPI + l / CPR];
        const long long src = pair < p.n_pairs ? (p.by_token ? pair / p.topk : pair) : 0;
        a_off[buf][i] = (uint32_t)(src * p.sa * EB + kc);
      }
    };
    auto issue = [&](int slot, int kt, int buf) {   // stage kt of the item in buffer buf, into ring slot
      FLIDE_LDS_AS char* sb = (FLIDE_LDS_AS char*)(slot == 0 ? lds0 : slot == 1 ? lds1 : lds2);
      const uint32_t kb = (uint32_t)(kt * ROWB);
#pragma unroll
      for (int i = 0; i < LA; ++i) dma16b<0>(rsA, a_off[buf][i], kb, sb + (lw * LA + i) * 1024);
#pragma unroll
      for (int i = 0; i < LB; ++i) dma16b<0>(rsB[buf], b_off[buf][i], kb, sb + A_BYTES + (lw * LB + i) * 1024);
    };
    set_ops(0);
#pragma unroll
    for (int st = 0; st < NS - 1; ++st) issue(st, st, 0);
    const int S_all = n_items * nk;
    int g = 0;   // global stage
    for (int n = 0; n < n_items; ++n) {
      const int buf = n & 1;
      const bool has_next = n + 1 < n_items;
      for (int kt = 0; kt < nk; ++kt, ++g) {
        wait_stage<NS, L>(min(NS - 2, S_all - 1 - g));
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (kt == 6 && has_next) set_ops(buf ^ 1);   // the compute waves placed its pairs at stage 5
        const int ks = kt + NS - 1;
        if (ks < nk) issue((g + NS - 1) % NS, ks, buf);
        else if (has_next) issue((g + NS - 1) % NS, ks - nk, buf ^ 1);
      }
#pragma unroll
      for (int eb = 0; eb < EPB; ++eb) __builtin_amdgcn_s_barrier();   // the epilogue's barriers
    }
    return;
  }

  // ---------------- compute waves ----------------
  const int wm = wave % WAVES_M, wn = wave / WAVES_M;
  const int r = l & 15, g = l >> 4;
  int lane_off[2];
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) lane_off[jj] = r * ROWB + ((((jj * 4 + g) % CPR) ^ swz<CPR>(r)) << 4);
  auto a_off = [&](int fm, int jj) { return (wm * WM + fm * 16) * ROWB + lane_off[jj]; };
  auto brow = [&](int fn) {   // gated: gate fragments first, then the matching up fragments
    if constexpr (!GATED) return wn * WN + fn * 16;
    const int f = fn < FN / 2 ? fn : fn - FN / 2;
    return (fn < FN / 2 ? 0 : TC) + wn * (WN / 2) + f * 16;
  };
  auto b_off = [&](int fn, int jj) { return A_BYTES + brow(fn) * ROWB + lane_off[jj]; };
  f32x4_t acc[FM][FN];
  int g_stage = 0;
  int pair_next = 0;
  float scale_next = 0.f;
  for (int n = 0; n < n_items; ++n) {
    const int buf = n & 1, nbuf = buf ^ 1;
    const bool has_next = n + 1 < n_items;
    const long long it_next = it0 + (long long)(n + 1) * W;
    // the next item's metadata, after this item's stage barrier k (nk >= 10)
    auto act = [&](int k) {
      if (!has_next) return;
      if (k == 0 && wave == 0) window(it_next);
      if (k == 2 && wave == 0) resolve(it_next, s_meta[nbuf]);
      if (k == 3 && tid < BM) pair_next = p.rows[s_meta[nbuf][0] * BM + tid];   // s_meta written before barrier 3
      if (k == 5 && tid < BM) {   // the loaders read the pairs after barrier 6
        s_pairs[nbuf][tid] = pair_next;
        scale_next = scale_of(pair_next);
      }
      if (k == 8 && tid < BM) s_ascale[nbuf][tid] = scale_next;   // read by that item's epilogue
    };
    const int pn = __builtin_amdgcn_readfirstlane(s_meta[buf][1]);
    // this lane's columns' gate and up scales, read by the epilogue
    float cs_g[FN / 2], cs_u[FN / 2];
    {
      const long long e = __builtin_amdgcn_readfirstlane(s_meta[buf][2]);
#pragma unroll
      for (int f = 0; f < FN / 2; ++f) {
        const int col = pn * TC + wn * (WN / 2) + f * 16 + r;
        const bool ok = col < half;
        cs_g[f] = !FP8 || !GATED ? 1.f : ok ? p.w_scale[e * p.sse + col] : 0.f;
        cs_u[f] = !FP8 || !GATED ? 1.f : ok ? p.w_scale[e * p.sse + col + half] : 0.f;
      }
    }
    bool m_live[FM];
    int nlive = 0;
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      m_live[fm] = __builtin_amdgcn_readfirstlane(s_pairs[buf][wm * WM + fm * 16]) < p.n_pairs;
      nlive += m_live[fm] ? 1 : 0;
    }
    const int colbase0 = GATED ? pn * TC + wn * (WN / 2) : pn * BN + wn * WN;
    const bool wave_live = colbase0 < ncols && m_live[0];
    if (colbase0 >= ncols) nlive = 0;
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) acc[fm][fn] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // the item's K loop, barrier in mid-stage as in grouped_dma's split roles
    auto kloop = [&](auto fma_tag, char* __restrict__ s0, char* __restrict__ s1, char* __restrict__ s2) {
      constexpr int FMA = decltype(fma_tag)::value;
      auto slot_ptr = [&](int slot) -> char* { return slot == 0 ? s0 : slot == 1 ? s1 : s2; };
      if constexpr (FMA == 0) {
        for (int k = 0; k < nk; ++k) {
          ring_barrier();
          asm volatile("" ::: "memory");
          act(k);
        }
      } else {
        constexpr int H1 = FMA < 2 ? FMA : 2;
        u32x4_t af[FMA][2], bfr[FN][2];
        auto read_a = [&](const char* sb, int fm) {
          af[fm][0] = *(const u32x4_t*)(sb + a_off(fm, 0));
          af[fm][1] = *(const u32x4_t*)(sb + a_off(fm, 1));
        };
        auto read_rest = [&](const char* sb) {
#pragma unroll
          for (int fn = 0; fn < FN; ++fn) {
            bfr[fn][0] = *(const u32x4_t*)(sb + b_off(fn, 0));
            bfr[fn][1] = *(const u32x4_t*)(sb + b_off(fn, 1));
          }
#pragma unroll
          for (int fm = H1; fm < FMA; ++fm) read_a(sb, fm);
        };
        auto rows = [&](auto lo_tag, auto hi_tag) {
#pragma unroll
          for (int fm = decltype(lo_tag)::value; fm < decltype(hi_tag)::value; ++fm)
#pragma unroll
            for (int fn = 0; fn < FN; ++fn) {
              const u32x4_t *a = af[fm], *b = bfr[fn];
              if constexpr (FP8) {
                acc[fm][fn] = mfma_fp8(i32x8_t{(int)a[0][0], (int)a[0][1], (int)a[0][2], (int)a[0][3], (int)a[1][0], (int)a[1][1], (int)a[1][2], (int)a[1][3]},
                                       i32x8_t{(int)b[0][0], (int)b[0][1], (int)b[0][2], (int)b[0][3], (int)b[1][0], (int)b[1][1], (int)b[1][2], (int)b[1][3]},
                                       acc[fm][fn]);
              } else {   // two 32-wide K steps, in order
                acc[fm][fn] = Mfma16<T>::mma(a[0], b[0], acc[fm][fn]);
                acc[fm][fn] = Mfma16<T>::mma(a[1], b[1], acc[fm][fn]);
              }
            }
        };
        int slot = g_stage % NS;
        ring_barrier();
        asm volatile("" ::: "memory");
        act(0);
#pragma unroll
        for (int fm = 0; fm < H1; ++fm) read_a(slot_ptr(slot), fm);
        read_rest(slot_ptr(slot));
        for (int kt = 0; kt + 1 < nk; ++kt) {
          const int nxt = slot + 1 == NS ? 0 : slot + 1;
          rows(std::integral_constant<int, 0>{}, std::integral_constant<int, H1>{});
          __builtin_amdgcn_sched_barrier(0);   // those MFMAs issue before the barrier
          ring_barrier();
          asm volatile("" ::: "memory");
          act(kt + 1);
          const char* sb = slot_ptr(nxt);
#pragma unroll
          for (int fm = 0; fm < H1; ++fm) read_a(sb, fm);
          rows(std::integral_constant<int, H1>{}, std::integral_constant<int, FMA>{});
          read_rest(sb);
          slot = nxt;
        }
        rows(std::integral_constant<int, 0>{}, std::integral_constant<int, FMA>{});
      }
    };
    if (nlive == 0) kloop(std::integral_constant<int, 0>{}, lds0, lds1, lds2);
    else if (nlive == 1) kloop(std::integral_constant<int, 1>{}, lds0, lds1, lds2);
    else if (nlive == 2) kloop(std::integral_constant<int, 2>{}, lds0, lds1, lds2);
    else if (nlive == 3) kloop(std::integral_constant<int, 3>{}, lds0, lds1, lds2);
    else kloop(std::integral_constant<int, 4>{}, lds0, lds1, lds2);
    const int last = (g_stage + nk - 1) % NS;   // the ring slot of the item's last stage
    g_stage += nk;
    if constexpr (!GATED) {   // float32 rows, 16 bytes per lane after the quad transpose (store_frag_f32x4)
      if (wave_live) {   // the ring slot is refilled only after every wave's next stage barrier
        const float ones[4] = {1.f, 1.f, 1.f, 1.f};
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) {
          if (!m_live[fm]) continue;
#pragma unroll
          for (int fn = 0; fn < FN; ++fn)
            store_frag_f32x4(p, s_pairs[buf], s_ascale[buf], wm * WM + fm * 16, colbase0 + fn * 16, acc[fm][fn], ones, 1.f);
        }
      }
      continue;
    }

    // epilogue: the BM x TC activation tile staged in the last stage's slot (the loaders refill it only
    // after the next item's first barrier), then 16-byte row pieces
    wait_vmcnt<0>();   // the column scales, the next item's pair and scale loads
    ring_barrier();    // every compute wave is done reading the ring
    S* tile = (S*)(last == 0 ? lds0 : last == 1 ? lds1 : lds2);
    if (wave_live) {
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        if (!m_live[fm]) continue;
        const int row0 = wm * WM + fm * 16;
        float rs[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) rs[i] = FP8 ? s_ascale[buf][row0 + g * 4 + i] : 1.f;
#pragma unroll
        for (int f = 0; f < FN / 2; ++f) {
          const int lc = wn * (WN / 2) + f * 16 + r;
#pragma unroll
          for (int i = 0; i < 4; ++i) {   // the values store_frag computes, in the same order
            const float gg = round_in<RT>(acc[fm][f][i] * rs[i] * cs_g[f]);
            const float uu = round_in<RT>(acc[fm][f + FN / 2][i] * rs[i] * cs_u[f]);
            tile[(row0 + g * 4 + i) * TC + lc] = OutTraits<OutT>::conv(act_f32<ACT>(gg, uu));
          }
        }
      }
    }
    ring_barrier();
    constexpr int LPR = TC / 8;          // lanes per row, 8 columns each
    constexpr int RPP = NW * 64 / LPR;   // rows per pass
    const int c8 = (tid % LPR) * 8;
    const int col0 = pn * TC + c8;
    for (int rr = tid / LPR; rr < BM; rr += RPP) {
      const int pair = s_pairs[buf][rr];
      if (pair >= p.n_pairs || col0 >= half) continue;
      const uint4 q = *(const uint4*)(tile + rr * TC + c8);
      S* o = (S*)p.out + (long long)pair * p.sc + col0;
      if (col0 + 8 <= half) {
        *(uint4*)o = q;
      } else {
        const S ev[8] = {(S)(q.x & 0xffff), (S)(q.x >> 16), (S)(q.y & 0xffff), (S)(q.y >> 16),
                         (S)(q.z & 0xffff), (S)(q.z >> 16), (S)(q.w & 0xffff), (S)(q.w >> 16)};
#pragma unroll
        for (int jj = 0; jj < 7; ++jj)
          if (col0 + jj < half) o[jj] = ev[jj];
      }
    }
  }
}

// the persistent kernel where it applies: gated products with 16-bit outputs in 16-byte aligned rows and
// no routing weights, plain 16-bit products with float32 outputs in 16-byte aligned rows; K a whole
// number of stages, at least 10 (the next item's metadata needs stages 0-8 of the current one); one
// workgroup per CU, a multiple of 8
template <typename T, typename OutT, int ACT>
int launch_persist(GroupArgs& p, hipStream_t st) {
  constexpr int KS = 128 / DmaElem<T>::BYTES;
  constexpr bool FP8 = std::is_same<T, Fp8Tag>::value;
  typedef typename OutTraits<OutT>::storage S;
  if constexpr (ACT != ACT_NONE ? sizeof(S) != 2 : (FP8 || !std::is_same<OutT, float>::value)) {
    return FLIDE_MOE_ERR_TILE;
  } else {
    if ((ACT != ACT_NONE && p.weights) || p.sc % (16 / sizeof(S)) || (uintptr_t)p.out % 16 || p.K % KS ||
        p.K / KS < 10)
      return FLIDE_MOE_ERR_TILE;
    const int cus = cu_count();
    if (cus < 8) return FLIDE_MOE_ERR_TILE;
    p.ntn = ACT != ACT_NONE ? (p.N / 2 + 127) / 128 : (p.N + 255) / 256;
    p.pack_f32 = ACT == ACT_NONE;
    grouped_persist<T, OutT, ACT><<<dim3(cus), dim3(12 * 64), 0, st>>>(p);
    return FLIDE_MOE_OK;
  }
}

constexpr int DMA_BN = 256;

template <typename T, typename OutT, int ACT, int BM, int WM_, int WN_, int NS, int ROWB, int OCC, int XB,
          int BN = DMA_BN, int NLD = 0>
int launch_one(GroupArgs& p, hipStream_t st) {
  constexpr int KS = ROWB / DmaElem<T>::BYTES;
  if (p.K < (NS - 1) * KS) return FLIDE_MOE_ERR_TILE;   // the ring needs NS - 1 full stages
  const int cols = ACT == ACT_NONE ? p.N : p.N / 2;
  const int per = ACT == ACT_NONE ? BN : BN / 2;
  p.ntn = (cols + per - 1) / per;
  const int items = p.nbm * p.ntn;
  p.pack_f32 = std::is_same<OutT, float>::value && p.sc % 4 == 0 && (uintptr_t)p.out % 16 == 0;
  // decode tiles: whole XCD chunks; prefill tiles: eight equal ranges of the static item count (each
  // XCD's range of the items in use is at most that long)
  const int round = BM >= 64 ? 8 : 8 * p.ntn * XB;
  dim3 grid((items + round - 1) / round * round), block((WM_ * WN_ + NLD) * 64);
  // Non-temporal weight loads (dma16w / dma16b<2>) for every 32-row (decode) product and for the gated products of
  // larger tiles while padding fills at least half the blocks (most experts then hold one block, so each
  // weight tile is read once); the plain (down) products of larger tiles measured slower with them. Only
  // for weight rows of whole 128-byte lines: a row that ends mid-line (float8 down rows of 704 bytes)
  // shares that line with the next row, which an `nt` load drops from L2 before it is read again.
  constexpr int EB = DmaElem<T>::BYTES;
  const bool lines = (p.sbn * EB) % 128 == 0 && (p.sbe * EB) % 128 == 0 && ((uintptr_t)p.w & 127) == 0;
  bool nt = false;
  if constexpr (BM == 32) nt = lines;
  else if constexpr (ACT != ACT_NONE) nt = lines && 2LL * p.n_pairs <= (long long)p.nbm * BM;
  if constexpr (BM == 32 || ACT != ACT_NONE) {
    if (nt) {
      grouped_dma<T, OutT, ACT, BM, BN, WM_, WN_, NS, ROWB, OCC, XB, true, NLD><<<grid, block, 0, st>>>(p);
      return FLIDE_MOE_OK;
    }
  }
  grouped_dma<T, OutT, ACT, BM, BN, WM_, WN_, NS, ROWB, OCC, XB, false, NLD><<<grid, block, 0, st>>>(p);
  return FLIDE_MOE_OK;
}

template <typename T, typename OutT, int ACT>
int launch_dma(GroupArgs& p, int bm, hipStream_t st) {
  constexpr bool FP8 = std::is_same<T, Fp8Tag>::value;
  if constexpr (FP8) {
    if (bm == 32) return launch_one<T, OutT, ACT, 32, 1, 4, 3, 128, 2, 8, 128>(p, st);
    if (bm == 256) return launch_one<T, OutT, ACT, 256, 1, 4, 2, 128, 1, 2>(p, st);
    if (bm == 128) {   // 8 waves: down 64 x 32 each (BN 128; K <= 768: grouped_fp8_resident), gate/up 64 x 64 each (BN 256, 3 stages)
      if constexpr (ACT == ACT_NONE) {
        if (launch_fp8_resident<OutT>(p, st) == FLIDE_MOE_OK) return FLIDE_MOE_OK;
        return launch_one<T, OutT, ACT, 128, 2, 4, 2, 128, 2, 4, 128>(p, st);
      }
      else {
        if (launch_persist<T, OutT, ACT>(p, st) == FLIDE_MOE_OK) return FLIDE_MOE_OK;
        return launch_one<T, OutT, ACT, 128, 2, 4, 3, 128, 1, 4, 256, 4>(p, st);   // + 4 loader waves
      }
    }
    if (bm == 64) return launch_one<T, OutT, ACT, 64, 1, 4, 2, 128, 2, 8, 128>(p, st);
  } else {
    if (bm == 32) {   // 64-row weight tiles: finer work units shorten the last round of workgroups
      if constexpr (ACT == ACT_NONE) return launch_one<T, OutT, ACT, 32, 1, 4, 3, 128, 3, 4, 64>(p, st);
      else return launch_one<T, OutT, ACT, 32, 2, 2, 3, 128, 3, 4, 64>(p, st);
    }
    if (bm == 256) return launch_one<T, OutT, ACT, 256, 1, 4, 4, 64, 1, 2>(p, st);
    if (bm == 128) {   // 8 waves of 64 x 64, two per SIMD within one workgroup
      if constexpr (ACT == ACT_NONE) {
        if (launch_persist<T, OutT, ACT>(p, st) == FLIDE_MOE_OK) return FLIDE_MOE_OK;
        return launch_one<T, OutT, ACT, 128, 2, 4, 3, 64, 1, 4>(p, st);
      } else {
        if (launch_persist<T, OutT, ACT>(p, st) == FLIDE_MOE_OK) return FLIDE_MOE_OK;
        return launch_one<T, OutT, ACT, 128, 2, 4, 3, 128, 1, 4>(p, st);
      }
    }
    if (bm == 64) {   // 128-byte stage rows: down in 8 waves, gate/up in two 4-wave workgroups of BN 128
      if constexpr (ACT == ACT_NONE) return launch_one<T, OutT, ACT, 64, 2, 4, 3, 128, 1, 8>(p, st);
      else return launch_one<T, OutT, ACT, 64, 1, 4, 3, 128, 2, 8, 128>(p, st);
    }
  }
  return FLIDE_MOE_ERR_TILE;
}

}  // namespace

namespace grouped_detail {

int dma_dispatch16(GroupArgs& p, bool is_bf16, int out_dtype, int act, int bm, hipStream_t st) {
  if (is_bf16) {
    if (act == ACT_NONE && out_dtype == FLIDE_F32) return launch_dma<__bf16, float, ACT_NONE>(p, bm, st);
    if (out_dtype != FLIDE_BF16) return FLIDE_MOE_ERR_ARG;
    if (act == ACT_NONE) return launch_dma<__bf16, Bf16Out, ACT_NONE>(p, bm, st);
    if (act == ACT_GEGLU) return launch_dma<__bf16, Bf16Out, ACT_GEGLU>(p, bm, st);
    if (act == ACT_SWIGLU) return launch_dma<__bf16, Bf16Out, ACT_SWIGLU>(p, bm, st);
    return FLIDE_MOE_ERR_ARG;
  }
  if (act == ACT_NONE && out_dtype == FLIDE_F32) return launch_dma<_Float16, float, ACT_NONE>(p, bm, st);
  if (out_dtype != FLIDE_F16) return FLIDE_MOE_ERR_ARG;
  if (act == ACT_NONE) return launch_dma<_Float16, F16Out, ACT_NONE>(p, bm, st);
  if (act == ACT_GEGLU) return launch_dma<_Float16, F16Out, ACT_GEGLU>(p, bm, st);
  if (act == ACT_SWIGLU) return launch_dma<_Float16, F16Out, ACT_SWIGLU>(p, bm, st);
  return FLIDE_MOE_ERR_ARG;
}

int dma_dispatch8(GroupArgs& p, int out_dtype, int act, int bm, hipStream_t st) {
  if (act == ACT_NONE) {
    if (out_dtype == FLIDE_F32) return launch_dma<Fp8Tag, float, ACT_NONE>(p, bm, st);
    if (out_dtype == FLIDE_BF16) return launch_dma<Fp8Tag, Bf16Out, ACT_NONE>(p, bm, st);
    if (out_dtype == FLIDE_F16) return launch_dma<Fp8Tag, F16Out, ACT_NONE>(p, bm, st);
    return FLIDE_MOE_ERR_ARG;
  }
  if (out_dtype == FLIDE_BF16) {
    if (act == ACT_GEGLU) return launch_dma<Fp8Tag, Bf16Out, ACT_GEGLU>(p, bm, st);
    if (act == ACT_SWIGLU) return launch_dma<Fp8Tag, Bf16Out, ACT_SWIGLU>(p, bm, st);
  }
  if (out_dtype == FLIDE_F16) {
    if (act == ACT_GEGLU) return launch_dma<Fp8Tag, F16Out, ACT_GEGLU>(p, bm, st);
    if (act == ACT_SWIGLU) return launch_dma<Fp8Tag, F16Out, ACT_SWIGLU>(p, bm, st);
  }
  return FLIDE_MOE_ERR_ARG;
}

}  // namespace grouped_detail
