// moe.experts in one C call (flide/kernels/moe.py:336-353): align, gate/up product with the fused
// activation, down product times the routing weight; plus the float8 variant with its two
// per-row quantizations (flide/kernels/moe.py:345-349, fp8.py:29-53). All scratch lives in the
// caller's workspace, carved in the fixed order below, so the call allocates nothing and can be
// captured into a HIP graph. flide_moe_experts_noalloc carves the same layout out of a static device
// array instead, for callers that cannot allocate at all.
#include <mutex>

#include "routing.hpp"

namespace {

size_t align_up(size_t v) { return (v + 255) & ~(size_t)255; }

struct ExpertsLayout {
  size_t hist, rows, blocks, used, act, qx, sx, qa, sa, total;
};

ExpertsLayout layout(int T, int k, int E, int H, int I, int bm, int fp8) {
  ExpertsLayout L{};
  const long long n = (long long)T * k;
  const long long total = (n + (long long)E * (bm - 1) + bm - 1) / bm * bm;
  size_t off = 0;
  L.hist = off;   off = align_up(off + flide_moe_align_workspace((int)n, E));
  L.rows = off;   off = align_up(off + (size_t)total * 4);
  L.blocks = off; off = align_up(off + (size_t)(total / bm) * 4);
  L.used = off;   off = align_up(off + 4);
  L.act = off;    off = align_up(off + (size_t)n * I * 2);
  if (fp8) {
    L.qx = off; off = align_up(off + (size_t)T * H);
    L.sx = off; off = align_up(off + (size_t)T * 4);
    L.qa = off; off = align_up(off + (size_t)n * I);
    L.sa = off; off = align_up(off + (size_t)n * 4);
  }
  L.total = off;
  return L;
}

}  // namespace

extern "C" const char* flide_moe_strerror(int rc) {
  switch (rc) {
    case FLIDE_MOE_OK: return "ok";
    case FLIDE_MOE_ERR_ARG: return "invalid argument (size, stride, alignment or dtype)";
    case FLIDE_MOE_ERR_WORKSPACE: return "workspace too small";
    case FLIDE_MOE_ERR_TILE: return "no kernel compiled for this tile shape";
    case FLIDE_MOE_ERR_SCRATCH:
      return "problem larger than the allocation-free entry point's static scratch "
             "(FLIDE_MOE_NOALLOC_SCRATCH_BYTES): call flide_moe_experts with a workspace";
    default:
      if (rc >= FLIDE_MOE_ERR_HIP_BASE) return hipGetErrorString((hipError_t)(rc - FLIDE_MOE_ERR_HIP_BASE));
      return "unknown error";
  }
}

extern "C" const char* flide_moe_version(void) { return "flide_moe 0.1 gfx950"; }

extern "C" size_t flide_moe_experts_workspace(int T, int k, int E, int H, int I, int bm, int fp8) {
  if (T < 0 || k <= 0 || E <= 0 || H <= 0 || I <= 0 || bm <= 0) return 0;
  return layout(T, k, E, H, I, bm, fp8).total;
}

namespace {

bool experts_args_ok(int T, int H, int k, int E, int I, int bm, int x_dtype, int act, const float* w_scale_gu,
                     const float* w_scale_d) {
  return T >= 0 && H > 0 && k > 0 && E > 0 && I > 0 && bm > 0 && (x_dtype == FLIDE_BF16 || x_dtype == FLIDE_F16) &&
         (act == ACT_GEGLU || act == ACT_SWIGLU) && ((w_scale_gu != nullptr) == (w_scale_d != nullptr));
}

// The two products on align's layout (rows, blocks, used in the workspace `ws` carved by `L`).
int run_products(const void* x, long long sx, int x_dtype, int T, int H, const float* top, int k,
                 const void* w_gu, const void* w_d, const float* w_scale_gu, const float* w_scale_d, int E, int I,
                 void* y, int act, int bm, int bn, char* ws, const ExpertsLayout& L, bool x_quantized,
                 flide_stream_t stream) {
  const int fp8 = w_scale_gu != nullptr;
  int* rows = (int*)(ws + L.rows);
  int* blocks = (int*)(ws + L.blocks);
  int* used = (int*)(ws + L.used);
  void* actbuf = ws + L.act;
  const int n = T * k;
  const long long total = ((long long)n + (long long)E * (bm - 1) + bm - 1) / bm * bm;
  const int nbm = (int)(total / bm);
  int rc;
  if (!fp8) {
    rc = flide_moe_grouped(x, sx, x_dtype, w_gu, (long long)2 * I * H, H, 2 * I, H, actbuf, I,
                           x_dtype, nullptr, rows, blocks, used, n, nbm, k, 1, act, bm, bn, stream);
    if (rc) return rc;
    return flide_moe_grouped(actbuf, I, x_dtype, w_d, (long long)H * I, I, H, I, y, H, FLIDE_F32,
                             top, rows, blocks, used, n, nbm, k, 0, ACT_NONE, bm, bn, stream);
  }
  u8* qx = (u8*)(ws + L.qx);
  float* sxs = (float*)(ws + L.sx);
  u8* qa = (u8*)(ws + L.qa);
  float* sas = (float*)(ws + L.sa);
  if (!x_quantized) {
    rc = flide_moe_quantize_rows(x, sx, T, H, x_dtype, qx, H, sxs, stream);
    if (rc) return rc;
  }
  rc = flide_moe_grouped_fp8(qx, H, sxs, w_gu, (long long)2 * I * H, H, w_scale_gu, 2 * I, 2 * I, H,
                             actbuf, I, x_dtype, nullptr, rows, blocks, used, n, nbm, k, 1, act, bm,
                             bn, stream);
  if (rc) return rc;
  rc = flide_moe_quantize_rows(actbuf, I, n, I, x_dtype, qa, I, sas, stream);
  if (rc) return rc;
  return flide_moe_grouped_fp8(qa, I, sas, w_d, (long long)H * I, I, w_scale_d, H, H, I, y, H,
                               x_dtype, top, rows, blocks, used, n, nbm, k, 0, ACT_NONE, bm, bn,
                               stream);
}

// flide_moe_experts and its allocation-free twin: arguments checked, then `ws` (ws_bytes >=
// layout().total) carved, align run and the products enqueued. Nothing in the layout needs to start
// zeroed: align writes its histograms before reading them, and the products write every row they
// later read.
int run_experts(const void* x, long long sx, int x_dtype, int T, int H, const float* top, const int* ids,
                int k, const void* w_gu, const void* w_d, const float* w_scale_gu, const float* w_scale_d,
                int E, int I, void* y, int act, int bm, int bn, char* ws, size_t ws_bytes,
                flide_stream_t stream) {
  if (!experts_args_ok(T, H, k, E, I, bm, x_dtype, act, w_scale_gu, w_scale_d)) return FLIDE_MOE_ERR_ARG;
  if (T == 0) return FLIDE_MOE_OK;
  const ExpertsLayout L = layout(T, k, E, H, I, bm, w_scale_gu != nullptr);
  if (ws_bytes < L.total) return FLIDE_MOE_ERR_WORKSPACE;
  int* rows = (int*)(ws + L.rows);
  int* blocks = (int*)(ws + L.blocks);
  int* used = (int*)(ws + L.used);
  // float8 experts: the token rows are quantized by the placement launch's spare workgroups where the
  // vector quantizer takes them (one launch less; the two overlap), else by their own launch below
  bool xq = false;
  int rc;
  if (w_scale_gu != nullptr) {
    rc = routing::align_quantizing(ids, T * k, E, bm, rows, blocks, used, ws + L.hist, L.rows - L.hist, x, sx, T,
                                   H, x_dtype, ws + L.qx, H, (float*)(ws + L.sx), (hipStream_t)stream);
    if (rc == FLIDE_MOE_OK) xq = true;
    else if (rc != FLIDE_MOE_ERR_TILE) return rc;
  }
  if (!xq) {
    rc = flide_moe_align(ids, T * k, E, bm, rows, blocks, used, nullptr, ws + L.hist, L.rows - L.hist, stream);
    if (rc) return rc;
  }
  return run_products(x, sx, x_dtype, T, H, top, k, w_gu, w_d, w_scale_gu, w_scale_d, E, I, y, act, bm, bn, ws,
                      L, xq, stream);
}

// The allocation-free entry point's scratch: one copy of this array per device, resident from module
// load until the process ends. Host code never passes `scratch` itself (on the host it names a
// stand-in, not device memory): each device's address comes from hipGetSymbolAddress, taken once per
// device with that device current, and only that address reaches the kernels.
static __device__ __align__(256) char scratch[FLIDE_MOE_NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch[MAX_DEVICES];

// this device's address of `scratch` (the stream's device, or the current one for the null stream)
int scratch_for(hipStream_t st, char** out) {
  int cur = 0, dev = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return FLIDE_MOE_ERR_HIP_BASE + (int)e;
  dev = cur;
  if (st != nullptr) {
    e = hipStreamGetDevice(st, &dev);
    if (e != hipSuccess) return FLIDE_MOE_ERR_HIP_BASE + (int)e;
  }
  if (dev < 0 || dev >= MAX_DEVICES) return FLIDE_MOE_ERR_ARG;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) return FLIDE_MOE_ERR_HIP_BASE + (int)e;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    const hipError_t back = dev != cur ? hipSetDevice(cur) : hipSuccess;
    if (e != hipSuccess) return FLIDE_MOE_ERR_HIP_BASE + (int)e;
    if (back != hipSuccess) return FLIDE_MOE_ERR_HIP_BASE + (int)back;
    if (p == nullptr) return FLIDE_MOE_ERR_HIP_BASE + (int)hipErrorInvalidSymbol;
    g_scratch[dev] = p;
  }
  *out = (char*)g_scratch[dev];
  return FLIDE_MOE_OK;
}

}  // namespace

extern "C" int flide_moe_experts(const void* x, long long sx, int x_dtype, int T, int H,
                                 const float* top, const int* ids, int k, const void* w_gu,
                                 const void* w_d, const float* w_scale_gu, const float* w_scale_d,
                                 int E, int I, void* y, int act, int bm, int bn, void* workspace,
                                 size_t workspace_bytes, flide_stream_t stream) {
  return run_experts(x, sx, x_dtype, T, H, top, ids, k, w_gu, w_d, w_scale_gu, w_scale_d, E, I, y, act,
                     bm, bn, (char*)workspace, workspace_bytes, stream);
}

extern "C" int flide_moe_experts_noalloc(const void* x, long long sx, int x_dtype, int T, int H,
                                         const float* top, const int* ids, int k, const void* w_gu,
                                         const void* w_d, const float* w_scale_gu,
                                         const float* w_scale_d, int E, int I, void* y, int act,
                                         int bm, int bn, flide_stream_t stream) {
  if (T < 0 || H <= 0 || k <= 0 || E <= 0 || I <= 0 || bm <= 0) return FLIDE_MOE_ERR_ARG;
  if (T == 0) return FLIDE_MOE_OK;
  const size_t need = layout(T, k, E, H, I, bm, w_scale_gu != nullptr).total;
  if (need > FLIDE_MOE_NOALLOC_SCRATCH_BYTES) return FLIDE_MOE_ERR_SCRATCH;
  char* ws = nullptr;
  const int rc = scratch_for((hipStream_t)stream, &ws);
  if (rc) return rc;
  return run_experts(x, sx, x_dtype, T, H, top, ids, k, w_gu, w_d, w_scale_gu, w_scale_d, E, I, y, act,
                     bm, bn, ws, FLIDE_MOE_NOALLOC_SCRATCH_BYTES, stream);
}
