// Internal definitions shared by the host translation units of libcdclq_hip.so: the context
// object behind the opaque `cdclq_ctx` of include/cdclq.h, its grow-only device workspace and the
// error / timing helpers. Not part of the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <string>
#include <vector>

#include "cdclq.h"

namespace cdclq {

struct DevBuf {
  void* p = nullptr;
  size_t cap = 0;
};

struct TimedRegion {
  int phase;
  hipEvent_t a, b;
};

}  // namespace cdclq

struct cdclq_ctx {
  int device = 0;
  hipStream_t st = nullptr;
  hipStream_t st2 = nullptr;  // side stream of the factorisation's look-ahead (default priority)
  hipEvent_t ev_col = nullptr, ev_panel = nullptr;
  std::string err;
  // workspace (grow-only)
  using DevBuf = cdclq::DevBuf;
  DevBuf w_in, h_in, m_in, x_in, y_in, h64_in, u_out, codes_o, scales_o, zeros_o;
  DevBuf wp, wwork, wq, ebuf, gbits_d, perm_d, deadp_d, dead_d, diag_d, colsq_d, invd, colloss_d;
  DevBuf G, part, rlog, rcnt, clog, ccnt, sel_d, ld_d, mp, t1, t2, a64, y64, tbuf, tpart, status_d, rtiles_d,
      tiles_d, proxy_p, cs_d, gemm_part, mid_d;
  // one-entry PrepCache (src/engine.rs:207-223): key, perm, damping and the device factors
  bool cache_valid = false;
  std::string cache_key;
  std::vector<uint32_t> cache_perm;
  size_t cache_n = 0;
  double cache_damp = 0.0;
  DevBuf cache_u, cache_h32;
  // packed-container workspace (container.cpp)
  DevBuf pk_in[4], pk_out[4], pk_tab[3], pk_flag;
  bool pk_layout_valid = false;  // pk_tab[0] holds the tables of this layout
  size_t pk_layout_n = 0, pk_layout_g = 0;
  std::vector<uint8_t> pk_layout_wid;
  // device address of this GPU's fixed scratch (allocation-free Gram entry point), or null with
  // the lookup's error
  void* gram_scratch = nullptr;
  hipError_t gram_scratch_err = hipSuccess;
  // near-midpoint accounting of the last quantize_layer call
  cdclq_midpoint_counts mid_last = {};
  // timing
  bool timing = false;
  // pinned host staging of the repair loop's per-pass transfers (grows; freed with the context)
  void* pin = nullptr;
  size_t pin_size = 0;
  std::vector<cdclq::TimedRegion> pending;
  std::vector<hipEvent_t> event_pool;  // recycled timing events (creating one per region is slow)
  uint32_t pk_epoch = 0;               // tags this call's device flags (no per-call clearing)
  double ms[CDCLQ_PHASE_COUNT] = {};
  uint64_t launches[CDCLQ_PHASE_COUNT] = {};
};

namespace cdclq {

inline int fail(cdclq_ctx* ctx, int code, const std::string& msg) {
  ctx->err = msg;
  return code;
}

#define HIPCK(expr)                                                                                   \
  do {                                                                                                \
    hipError_t e_ = (expr);                                                                           \
    if (e_ != hipSuccess)                                                                             \
      return fail(ctx, CDCLQ_DEVICE, std::string("HIP error '") + hipGetErrorString(e_) + "' in " #expr); \
  } while (0)
#define CK(expr)                       \
  do {                                 \
    int rc_ = (expr);                  \
    if (rc_ != CDCLQ_OK) return rc_;   \
  } while (0)

inline int ensure(cdclq_ctx* ctx, DevBuf& b, size_t bytes) {
  if (bytes == 0) bytes = 256;
  if (b.cap >= bytes) return CDCLQ_OK;
  if (b.p) {
    hipError_t e = hipFree(b.p);
    b.p = nullptr;
    b.cap = 0;
    if (e != hipSuccess) return fail(ctx, CDCLQ_DEVICE, std::string("hipFree failed: ") + hipGetErrorString(e));
  }
  hipError_t e = hipMalloc(&b.p, bytes);
  if (e != hipSuccess) {
    b.p = nullptr;
    (void)hipGetLastError();
    return fail(ctx, CDCLQ_OOM, "device allocation of " + std::to_string(bytes) + " bytes failed (" +
                                    hipGetErrorString(e) + ")");
  }
  b.cap = bytes;
  return CDCLQ_OK;
}

template <class T>
inline T* P(DevBuf& b) {
  return static_cast<T*>(b.p);
}

inline void free_buf(DevBuf& b) {
  if (b.p) (void)hipFree(b.p);
  b.p = nullptr;
  b.cap = 0;
}

inline hipEvent_t pooled_event(cdclq_ctx* ctx) {
  if (!ctx->event_pool.empty()) {
    hipEvent_t e = ctx->event_pool.back();
    ctx->event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  return hipEventCreate(&e) == hipSuccess ? e : nullptr;
}

struct PhaseScope {
  cdclq_ctx* ctx;
  int phase;
  hipEvent_t a = nullptr;
  PhaseScope(cdclq_ctx* c, int ph) : ctx(c), phase(ph) {
    if (ctx->timing && (a = pooled_event(ctx)) != nullptr) (void)hipEventRecord(a, ctx->st);
  }
  ~PhaseScope() {
    if (!ctx->timing || !a) return;
    hipEvent_t b = pooled_event(ctx);
    if (b) {
      (void)hipEventRecord(b, ctx->st);
      ctx->pending.push_back({phase, a, b});
    } else {
      ctx->event_pool.push_back(a);
    }
  }
};

}  // namespace cdclq
