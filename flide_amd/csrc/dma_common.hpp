// Pieces of the direct-to-LDS grouped kernels (grouped_dma.hip): global -> LDS loads
// (global_load_lds_dwordx4 and buffer_load_dwordx4 ... lds, gfx950), vmcnt waits, the LDS chunk
// swizzle, element traits and the expert-major work order's segment search. Each including file gets its own copies (anonymous namespace).
#pragma once
#include "grouped_common.hpp"

#define FLIDE_GLOBAL_AS __attribute__((address_space(1)))
#define FLIDE_LDS_AS __attribute__((address_space(3)))

namespace {
using namespace grouped_detail;

__device__ __attribute__((aligned(16))) const uint32_t g_zero16[4] = {0, 0, 0, 0};
__device__ const float g_one = 1.0f;

template <int N> FLIDE_DEV void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  // s_waitcnt: vmcnt[3:0] bits 3:0, vmcnt[5:4] bits 15:14; expcnt (6:4) and lgkmcnt (11:8) left open
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

FLIDE_DEV void dma16(const void* src, FLIDE_LDS_AS void* dst) {
  __builtin_amdgcn_global_load_lds((const FLIDE_GLOBAL_AS void*)src, dst, 16, 0, 0);
}

// 4 bytes per lane (global_load_lds_dword): lane l's value lands at dst + 4 l
FLIDE_DEV void dma4(const void* src, FLIDE_LDS_AS void* dst) {
  __builtin_amdgcn_global_load_lds((const FLIDE_GLOBAL_AS void*)src, dst, 4, 0, 0);
}

// The same load through a raw buffer resource (buffer_load_dwordx4 ... lds): the per-lane offset is a
// 32-bit VGPR and the stage's K offset an SGPR, so a full stage needs no per-lane 64-bit address
// arithmetic and each load keeps one VGPR instead of two (the 16-bit gated product at 8192 tokens 4%
// faster, the float8 one's registers 212 -> 182). Word 3 0x00020000: 32-bit data format, the value
// for gfx9-family raw buffers. num_records bounds the resource at the operand's extent (the callers
// check that every offset fits in 32 bits).
FLIDE_DEV __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, long long bytes) {
  const int n = bytes > 0x7fffffffLL ? -1 : (int)bytes;   // -1: 0xffffffff, the whole 32-bit range
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}
template <int AUX> FLIDE_DEV void dma16b(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                         FLIDE_LDS_AS void* dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, (int)voff, (int)soff, 0, AUX);
}

// The weight loads: non-temporal (`nt`, cache-policy bit 1 on gfx950) when NT, i.e. when every weight
// byte is read by one block only (an expert's pairs fill one block). They then stop displacing the
// activation rows that the block's column tiles share in L2: at 64 tokens gate/up streams 6.5 TB/s
// instead of 5.7 (down 6.1 instead of 5.2); at 512-1024 tokens the bm-128 gate/up gains 4-6%. Where
// several blocks share a weight tile (prefill) the same loads are 15-60% slower, so they stay plain.
template <bool NT> FLIDE_DEV void dma16w(const void* src, FLIDE_LDS_AS void* dst) {
  __builtin_amdgcn_global_load_lds((const FLIDE_GLOBAL_AS void*)src, dst, 16, 0, NT ? 2 : 0);
}

// chunk swizzle of a row with CPR 16-byte chunks (8 for 128-byte rows, 4 for 64-byte rows); both
// measured bank-conflict-free for the fragment reads below
template <int CPR> FLIDE_DEV int swz(int row) { return CPR == 8 ? (row & 7) : ((row >> 1) & 3); }

// The barrier of a stage ring, taken by every wave that reads the ring: its own LDS reads complete
// first. gfx950's s_barrier does not wait for outstanding memory operations, and the compiler leaves
// reads of the slot consumed last in flight across it (the MFMAs that use them follow the barrier),
// while the loads issued right after the barrier refill that very slot: without the wait, another
// wave's direct-to-LDS write could land before such a read is served.
FLIDE_DEV void ring_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0); vmcnt (bits 3:0, 15:14) and expcnt (6:4) open
  __builtin_amdgcn_s_barrier();
}

// Waits until at most `ahead` (0 .. NS-2) stages of this wave's loads are still in flight (each stage =
// L loads).
template <int NS, int L> FLIDE_DEV void wait_stage(int ahead) {
  static_assert(NS >= 2 && NS <= 4, "stage ring of 2..4");
  if constexpr (NS >= 4) {
    if (ahead >= 2) { wait_vmcnt<2 * L>(); return; }
  }
  if constexpr (NS >= 3) {
    if (ahead >= 1) { wait_vmcnt<L>(); return; }
  }
  wait_vmcnt<0>();
}

// Element type traits of the two kernel families: 16-bit (2 bytes, 64 K per 128-byte stage row, two
// 32-wide MFMA steps) and float8 (1 byte, 128 K per stage row, one 128-wide MFMA step).
template <typename T> struct DmaElem {
  static constexpr int BYTES = 2;
};
struct Fp8Tag {};
template <> struct DmaElem<Fp8Tag> {
  static constexpr int BYTES = 1;
};

// First block of the run of blocks holding expert e that contains block blk (blocks[blk] == e; align
// writes each expert's blocks contiguously): the wave looks 64 entries back at a time until an entry
// differs. Entries below blk are all in use, and a lane below 0 reads -1, so the loop ends.
FLIDE_DEV int expert_first_block(const int* blocks, int blk, int e, int l) {
  int base = blk;
  for (;;) {
    const int idx = base - 63 + l;
    const int v = idx >= 0 ? blocks[idx] : -1;
    const unsigned long long m = __ballot(v != e);
    if (m) return base - 63 + (63 - __builtin_clzll(m)) + 1;
    base -= 64;
  }
}

// One past the last block of that run, looking forward 64 entries at a time; entries at or past
// nused (unset by align) are never read.
FLIDE_DEV int expert_end_block(const int* blocks, int blk, int e, int nused, int l) {
  int base = blk;
  for (;;) {
    const int idx = base + l;
    const int v = idx < nused ? blocks[idx] : -1;
    const unsigned long long m = __ballot(v != e);
    if (m) return base + __builtin_ctzll(m);
    base += 64;
  }
}

// The expert e = blocks[blk] and the run [first, end) of its blocks. One pair of loads covers blocks
// blk - 63 .. blk + 63, so a run of up to 64 blocks on either side costs one round trip (the searches
// above need one for blocks[blk] and one more each); longer runs continue with those searches.
FLIDE_DEV int expert_run(const int* blocks, int blk, int nused, int l, int& first, int& end) {
  const int lo_idx = blk - 63 + l, hi_idx = blk + l;
  const int lo = lo_idx >= 0 ? blocks[lo_idx] : -1;
  const int hi = hi_idx < nused ? blocks[hi_idx] : -1;
  const int e = __builtin_amdgcn_readfirstlane(hi);   // lane 0 read blocks[blk]
  const unsigned long long ml = __ballot(lo != e), mh = __ballot(hi != e);
  first = ml ? blk - 63 + (63 - __builtin_clzll(ml)) + 1 : expert_first_block(blocks, blk - 64, e, l);
  end = mh ? blk + __builtin_ctzll(mh) : expert_end_block(blocks, blk + 64, e, nused, l);
  return e;
}

// Workgroup barrier for LDS data only: waits for this wave's LDS accesses but not for its global loads
// (loads into the stage ring stay in flight), and keeps the compiler from moving memory accesses across.
FLIDE_DEV void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

}  // namespace
