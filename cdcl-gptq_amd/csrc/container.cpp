// C-ABI entry points of the packed container cdclq-v1 (include/cdclq.h): validation, the layout
// tables shared by every row, host staging, and the k_pack.hip launches.
//
// Layout tables (row-independent, built on the host from gbits in O(d_in + row_bytes)):
//   coff[j]   bit offset of code j in a row (coff[d_in] = bits per row), cwid[j] its width,
//   wfirst[w] first code whose 8-bit window [coff[j], coff[j] + 8) reaches bit 32 w (the OR of a
//             whole u8 code can reach 8 bits past its offset, src/quant.rs:120).
#include <hip/hip_runtime.h>

#include <cstring>
#include <string>
#include <vector>

#include "cdclq.h"
#include "ctx.h"
#include "kernels.h"

namespace {

using namespace cdclq;

constexpr size_t kMaxDin = (size_t)1 << 17;  // a row of u8 codes (+ padding) fits one workgroup's LDS

struct Layout {
  size_t rb = 0;
  std::vector<uint32_t> coff;
  std::vector<uint8_t> cwid;
  std::vector<int> wfirst;
  std::vector<uint32_t> rdesc;  // runs of 8 columns: byte offset << 4 | width (when they share widths)
};

// Checks the conditions under which the reference indexes in bounds (group > 0, a width for every
// column's group) plus this build's limits; returns "" when the layout is usable.
std::string check_layout(size_t d_in, size_t group, const uint8_t* gbits, size_t ngroups, bool need_widths) {
  if (d_in == 0) return "";
  if (d_in > kMaxDin) return "d_in " + std::to_string(d_in) + " exceeds this build's limit of 131072 columns";
  if (group == 0) return "group size must be > 0";
  const size_t used = (d_in + group - 1) / group;
  if (ngroups < used)
    return "ngroups " + std::to_string(ngroups) + " is smaller than ceil(d_in / group) = " + std::to_string(used);
  if (need_widths) {
    if (!gbits) return "gbits is null";
    for (size_t gi = 0; gi < used; ++gi)
      if (gbits[gi] < 1 || gbits[gi] > 8)
        return "gbits[" + std::to_string(gi) + "] = " + std::to_string(gbits[gi]) + " is outside 1..=8";
  }
  return "";
}

size_t row_bytes_of(size_t d_in, size_t group, const uint8_t* gbits) {
  size_t bits = 0;
  for (size_t j = 0; j < d_in; j += group) bits += (size_t)gbits[j / group] * std::min(group, d_in - j);
  return (bits + 7) / 8;
}

Layout build_layout(size_t n, size_t g, const uint8_t* gbits) {
  Layout L;
  L.coff.resize(n + 1);
  L.cwid.resize(n);
  uint32_t off = 0;
  for (size_t j = 0; j < n; ++j) {
    L.coff[j] = off;
    L.cwid[j] = gbits[j / g];
    off += L.cwid[j];
  }
  L.coff[n] = off;
  L.rb = ((size_t)off + 7) / 8;
  const size_t wpr = (L.rb + 3) / 4;
  L.wfirst.resize(wpr);
  size_t j = 0;
  for (size_t w = 0; w < wpr; ++w) {
    while (j < n && (size_t)L.coff[j] + 8 <= 32 * w) ++j;
    L.wfirst[w] = (int)j;
  }
  L.rdesc.resize((n + 7) / 8);
  for (size_t k = 0; k < L.rdesc.size(); ++k) L.rdesc[k] = ((L.coff[8 * k] >> 3) << 4) | L.cwid[8 * k];
  return L;
}

struct LayoutDev {
  uint32_t* coff;
  int* wfirst;
  uint8_t* cwid;
  uint32_t* rdesc;
};

// Uploads the tables into ctx->pk_tab[0] as one block: coff (n+1 u32) | wfirst (wpr i32) |
// rdesc (runs u32) | cwid (n u8). The block stays valid for later calls with the same layout (every
// call ends with a stream synchronisation, so no kernel still reads it when it is replaced).
int upload_layout(cdclq_ctx* ctx, const Layout& L, size_t g, LayoutDev* D) {
  const size_t n = L.cwid.size();
  const size_t a = (L.coff.size() * 4 + 255) & ~(size_t)255;
  const size_t b = (L.wfirst.size() * 4 + 255) & ~(size_t)255;
  const size_t c = (L.rdesc.size() * 4 + 255) & ~(size_t)255;
  char* base;
  const bool hit = ctx->pk_layout_valid && ctx->pk_layout_n == n && ctx->pk_layout_g == g &&
                   ctx->pk_layout_wid == L.cwid && ctx->pk_tab[0].p != nullptr;
  if (!hit) {
    ctx->pk_layout_valid = false;
    std::vector<char> blob(a + b + c + n + 16, 0);
    std::memcpy(blob.data(), L.coff.data(), L.coff.size() * 4);
    if (!L.wfirst.empty()) std::memcpy(blob.data() + a, L.wfirst.data(), L.wfirst.size() * 4);
    if (!L.rdesc.empty()) std::memcpy(blob.data() + a + b, L.rdesc.data(), L.rdesc.size() * 4);
    if (n) std::memcpy(blob.data() + a + b + c, L.cwid.data(), n);
    CK(ensure(ctx, ctx->pk_tab[0], blob.size()));
    HIPCK(hipMemcpy(ctx->pk_tab[0].p, blob.data(), blob.size(), hipMemcpyHostToDevice));
    ctx->pk_layout_valid = true;
    ctx->pk_layout_n = n;
    ctx->pk_layout_g = g;
    ctx->pk_layout_wid = L.cwid;
  }
  base = P<char>(ctx->pk_tab[0]);
  D->coff = reinterpret_cast<uint32_t*>(base);
  D->wfirst = reinterpret_cast<int*>(base + a);
  D->rdesc = reinterpret_cast<uint32_t*>(base + a + b);
  D->cwid = reinterpret_cast<uint8_t*>(base + a + b + c);
  return CDCLQ_OK;
}

// Device flags: [0] bad perm entry, [1] pack spill. Zeroed once at allocation; afterwards each call
// compares them against its own epoch number.
int flags(cdclq_ctx* ctx) {
  if (ctx->pk_flag.p) return CDCLQ_OK;
  CK(ensure(ctx, ctx->pk_flag, 256));
  HIPCK(hipMemset(ctx->pk_flag.p, 0, 256));
  return CDCLQ_OK;
}

// Epoch of a call (never 0, the flags' initial value).
uint32_t next_epoch(cdclq_ctx* ctx) {
  if (++ctx->pk_epoch == 0) ++ctx->pk_epoch;
  return ctx->pk_epoch;
}

size_t dtype_size(int dtype) { return dtype == CDCLQ_DTYPE_F32 ? 4 : 2; }

int check_dtype(cdclq_ctx* ctx, int dtype) {
  if (dtype != CDCLQ_DTYPE_F32 && dtype != CDCLQ_DTYPE_F16 && dtype != CDCLQ_DTYPE_BF16)
    return fail(ctx, CDCLQ_INVALID_ARG, "unsupported output dtype " + std::to_string(dtype) + " (need F32/F16/BF16)");
  return CDCLQ_OK;
}

int pack_device(cdclq_ctx* ctx, size_t d_out, size_t n, size_t g, const uint8_t* gbits, size_t ng,
                const uint8_t* codes, const float* scales, const float* zeros, const uint32_t* perm, uint8_t* qweight,
                size_t qweight_bytes, uint16_t* s16, uint8_t* qz, int32_t* p32) {
  if (d_out == 0 || n == 0) return CDCLQ_OK;
  const std::string why = check_layout(n, g, gbits, ng, true);
  if (!why.empty()) return fail(ctx, CDCLQ_INVALID_ARG, why);
  if (!codes || !scales || !zeros || !perm || !qweight || !s16 || !qz || !p32)
    return fail(ctx, CDCLQ_INVALID_ARG, "null buffer argument");
  const Layout L = build_layout(n, g, gbits);
  if (qweight_bytes < d_out * L.rb)
    return fail(ctx, CDCLQ_INVALID_ARG, "qweight holds " + std::to_string(qweight_bytes) + " bytes, the layer needs " +
                                            std::to_string(d_out * L.rb));
  HIPCK(hipSetDevice(ctx->device));
  LayoutDev D;
  CK(upload_layout(ctx, L, g, &D));
  CK(flags(ctx));
  uint32_t* spill = P<uint32_t>(ctx->pk_flag) + 1;
  const uint32_t epoch = next_epoch(ctx);
  // runs of 8 columns share one width when group boundaries fall on multiples of 8
  const bool runs = (g % 8 == 0) || (n <= g);
  {
    PhaseScope ps(ctx, CDCLQ_PHASE_PACK);
    if (runs) {
      HIPCK(pack_runs(ctx->st, (long)d_out, (int)n, (int)L.rb, codes, D.rdesc, qweight, spill, epoch));
      // a code wider than its group's width spills into the next run: then the general kernel,
      // which follows the reference's unmasked OR, redoes the layer (a no-op launch otherwise)
      HIPCK(pack_rows(ctx->st, (long)d_out, (int)n, (int)L.rb, codes, D.coff, D.wfirst, qweight, spill, epoch));
    } else {
      HIPCK(pack_rows(ctx->st, (long)d_out, (int)n, (int)L.rb, codes, D.coff, D.wfirst, qweight, nullptr, 0));
    }
    HIPCK(pack_meta(ctx->st, (long)(d_out * ng), scales, zeros, s16, qz));
  }
  HIPCK(hipMemcpyAsync(p32, perm, n * 4, hipMemcpyDeviceToDevice, ctx->st));  // `p as i32`: same bits
  HIPCK(hipStreamSynchronize(ctx->st));
  return CDCLQ_OK;
}

// Enqueues the output column map into ctx->pk_tab[1]; a perm entry outside 0..n sets the flag
// that finish_dequant() reads (entries outside the range are skipped, never written through).
int map_columns(cdclq_ctx* ctx, size_t n, size_t g, bool packed, const uint32_t* perm, const uint32_t* coff,
                const uint8_t* cwid, uint32_t** cdesc, int** cgrp) {
  const size_t a = (n * 4 + 255) & ~(size_t)255;
  CK(ensure(ctx, ctx->pk_tab[1], 3 * a));
  CK(flags(ctx));
  char* base = P<char>(ctx->pk_tab[1]);
  int* last = reinterpret_cast<int*>(base);
  *cdesc = reinterpret_cast<uint32_t*>(base + a);
  *cgrp = reinterpret_cast<int*>(base + 2 * a);
  const uint32_t epoch = next_epoch(ctx);
  HIPCK(column_map(ctx->st, (int)n, (int)g, packed, perm, coff, cwid, last, *cdesc, *cgrp, P<uint32_t>(ctx->pk_flag),
                   epoch));
  return CDCLQ_OK;
}

// Waits for the dequantization and reports a perm entry outside 0..n (the reference panics on its
// out-of-bounds scatter; here the output is unspecified and the call fails).
int finish_dequant(cdclq_ctx* ctx, size_t n) {
  uint32_t bad = 0;
  HIPCK(hipMemcpyAsync(&bad, ctx->pk_flag.p, 4, hipMemcpyDeviceToHost, ctx->st));
  HIPCK(hipStreamSynchronize(ctx->st));
  if (bad == ctx->pk_epoch)
    return fail(ctx, CDCLQ_INVALID_ARG, "perm has an entry outside 0..d_in (" + std::to_string(n) + ")");
  return CDCLQ_OK;
}

int dequant_packed_device(cdclq_ctx* ctx, size_t d_out, size_t n, size_t g, const uint8_t* gbits, size_t ng,
                          const uint8_t* qweight, size_t qweight_bytes, const uint16_t* s16, const uint8_t* qz,
                          const int32_t* p32, int dtype, void* out) {
  CK(check_dtype(ctx, dtype));
  if (d_out == 0 || n == 0) return CDCLQ_OK;
  const std::string why = check_layout(n, g, gbits, ng, true);
  if (!why.empty()) return fail(ctx, CDCLQ_INVALID_ARG, why);
  if (!qweight || !s16 || !qz || !p32 || !out) return fail(ctx, CDCLQ_INVALID_ARG, "null buffer argument");
  const Layout L = build_layout(n, g, gbits);
  if (qweight_bytes < d_out * L.rb)
    return fail(ctx, CDCLQ_INVALID_ARG, "qweight holds " + std::to_string(qweight_bytes) + " bytes, the layer needs " +
                                            std::to_string(d_out * L.rb));
  HIPCK(hipSetDevice(ctx->device));
  LayoutDev D;
  CK(upload_layout(ctx, L, g, &D));
  uint32_t* cdesc;
  int* cgrp;
  CK(map_columns(ctx, n, g, true, reinterpret_cast<const uint32_t*>(p32), D.coff, D.cwid, &cdesc, &cgrp));
  {
    PhaseScope ps(ctx, CDCLQ_PHASE_DEQUANT);
    HIPCK(dequant_rows(ctx->st, true, dtype, (long)d_out, (int)n, (int)ng, (int)L.rb, qweight, cdesc, cgrp, s16, qz,
                       out));
  }
  return finish_dequant(ctx, n);
}

int dequant_layer_device(cdclq_ctx* ctx, size_t d_out, size_t n, size_t g, size_t ng, const uint8_t* codes,
                         const float* scales, const float* zeros, const uint32_t* perm, int dtype, void* out) {
  CK(check_dtype(ctx, dtype));
  if (d_out == 0 || n == 0) return CDCLQ_OK;
  const std::string why = check_layout(n, g, nullptr, ng, false);
  if (!why.empty()) return fail(ctx, CDCLQ_INVALID_ARG, why);
  if (!codes || !scales || !zeros || !perm || !out) return fail(ctx, CDCLQ_INVALID_ARG, "null buffer argument");
  HIPCK(hipSetDevice(ctx->device));
  uint32_t* cdesc;
  int* cgrp;
  CK(map_columns(ctx, n, g, false, perm, nullptr, nullptr, &cdesc, &cgrp));
  {
    PhaseScope ps(ctx, CDCLQ_PHASE_DEQUANT);
    HIPCK(dequant_rows(ctx->st, false, dtype, (long)d_out, (int)n, (int)ng, (int)n, codes, cdesc, cgrp, scales,
                       zeros, out));
  }
  return finish_dequant(ctx, n);
}

template <class T>
int stage_in(cdclq_ctx* ctx, DevBuf& b, const T* src, size_t count, const T** dst) {
  CK(ensure(ctx, b, count * sizeof(T)));
  if (count) HIPCK(hipMemcpyAsync(b.p, src, count * sizeof(T), hipMemcpyHostToDevice, ctx->st));
  *dst = static_cast<const T*>(b.p);
  return CDCLQ_OK;
}

}  // namespace

extern "C" {

int cdclq_row_bytes(size_t d_in, size_t group, const uint8_t* gbits, size_t ngroups, size_t* row_bytes) {
  if (!row_bytes) return CDCLQ_INVALID_ARG;
  *row_bytes = 0;
  if (!check_layout(d_in, group, gbits, ngroups, true).empty()) return CDCLQ_INVALID_ARG;
  if (d_in) *row_bytes = row_bytes_of(d_in, group, gbits);
  return CDCLQ_OK;
}

int cdclq_pack_layer_device(cdclq_ctx* ctx, size_t d_out, size_t d_in, size_t group, const uint8_t* gbits,
                            size_t ngroups, const uint8_t* codes, const float* scales, const float* zeros,
                            const uint32_t* perm, uint8_t* qweight, size_t qweight_bytes, uint16_t* scales_f16,
                            uint8_t* qzeros, int32_t* perm_i32) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  return pack_device(ctx, d_out, d_in, group, gbits, ngroups, codes, scales, zeros, perm, qweight, qweight_bytes,
                     scales_f16, qzeros, perm_i32);
}

int cdclq_pack_layer(cdclq_ctx* ctx, size_t d_out, size_t d_in, size_t group, const uint8_t* gbits, size_t ngroups,
                     const uint8_t* codes, const float* scales, const float* zeros, const uint32_t* perm,
                     uint8_t* qweight, size_t qweight_bytes, uint16_t* scales_f16, uint8_t* qzeros, int32_t* perm_i32) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  if (d_out == 0 || d_in == 0) return CDCLQ_OK;
  const std::string why = check_layout(d_in, group, gbits, ngroups, true);
  if (!why.empty()) return fail(ctx, CDCLQ_INVALID_ARG, why);
  if (!codes || !scales || !zeros || !perm || !qweight || !scales_f16 || !qzeros || !perm_i32)
    return fail(ctx, CDCLQ_INVALID_ARG, "null buffer argument");
  const size_t rb = row_bytes_of(d_in, group, gbits), qb = d_out * rb, nm = d_out * ngroups;
  if (qweight_bytes < qb)
    return fail(ctx, CDCLQ_INVALID_ARG,
                "qweight holds " + std::to_string(qweight_bytes) + " bytes, the layer needs " + std::to_string(qb));
  HIPCK(hipSetDevice(ctx->device));
  const uint8_t* dc;
  const float *ds, *dz;
  const uint32_t* dp;
  CK(stage_in(ctx, ctx->pk_in[0], codes, d_out * d_in, &dc));
  CK(stage_in(ctx, ctx->pk_in[1], scales, nm, &ds));
  CK(stage_in(ctx, ctx->pk_in[2], zeros, nm, &dz));
  CK(stage_in(ctx, ctx->pk_in[3], perm, d_in, &dp));
  CK(ensure(ctx, ctx->pk_out[0], qb));
  CK(ensure(ctx, ctx->pk_out[1], nm * 2));
  CK(ensure(ctx, ctx->pk_out[2], nm));
  CK(ensure(ctx, ctx->pk_out[3], d_in * 4));
  CK(pack_device(ctx, d_out, d_in, group, gbits, ngroups, dc, ds, dz, dp, P<uint8_t>(ctx->pk_out[0]), qb,
                 P<uint16_t>(ctx->pk_out[1]), P<uint8_t>(ctx->pk_out[2]), P<int32_t>(ctx->pk_out[3])));
  HIPCK(hipMemcpyAsync(qweight, ctx->pk_out[0].p, qb, hipMemcpyDeviceToHost, ctx->st));
  HIPCK(hipMemcpyAsync(scales_f16, ctx->pk_out[1].p, nm * 2, hipMemcpyDeviceToHost, ctx->st));
  HIPCK(hipMemcpyAsync(qzeros, ctx->pk_out[2].p, nm, hipMemcpyDeviceToHost, ctx->st));
  HIPCK(hipMemcpyAsync(perm_i32, ctx->pk_out[3].p, d_in * 4, hipMemcpyDeviceToHost, ctx->st));
  HIPCK(hipStreamSynchronize(ctx->st));
  return CDCLQ_OK;
}

int cdclq_dequantize_packed_device(cdclq_ctx* ctx, size_t d_out, size_t d_in, size_t group, const uint8_t* gbits,
                                   size_t ngroups, const uint8_t* qweight, size_t qweight_bytes,
                                   const uint16_t* scales_f16, const uint8_t* qzeros, const int32_t* perm_i32,
                                   int dtype, void* out) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  return dequant_packed_device(ctx, d_out, d_in, group, gbits, ngroups, qweight, qweight_bytes, scales_f16, qzeros,
                               perm_i32, dtype, out);
}

int cdclq_dequantize_packed(cdclq_ctx* ctx, size_t d_out, size_t d_in, size_t group, const uint8_t* gbits,
                            size_t ngroups, const uint8_t* qweight, size_t qweight_bytes, const uint16_t* scales_f16,
                            const uint8_t* qzeros, const int32_t* perm_i32, int dtype, void* out) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  CK(check_dtype(ctx, dtype));
  if (d_out == 0 || d_in == 0) return CDCLQ_OK;
  const std::string why = check_layout(d_in, group, gbits, ngroups, true);
  if (!why.empty()) return fail(ctx, CDCLQ_INVALID_ARG, why);
  if (!qweight || !scales_f16 || !qzeros || !perm_i32 || !out)
    return fail(ctx, CDCLQ_INVALID_ARG, "null buffer argument");
  const size_t rb = row_bytes_of(d_in, group, gbits), qb = d_out * rb, nm = d_out * ngroups;
  if (qweight_bytes < qb)
    return fail(ctx, CDCLQ_INVALID_ARG,
                "qweight holds " + std::to_string(qweight_bytes) + " bytes, the layer needs " + std::to_string(qb));
  HIPCK(hipSetDevice(ctx->device));
  const uint8_t *dq, *dz;
  const uint16_t* ds;
  const int32_t* dp;
  CK(stage_in(ctx, ctx->pk_in[0], qweight, qb, &dq));
  CK(stage_in(ctx, ctx->pk_in[1], scales_f16, nm, &ds));
  CK(stage_in(ctx, ctx->pk_in[2], qzeros, nm, &dz));
  CK(stage_in(ctx, ctx->pk_in[3], perm_i32, d_in, &dp));
  const size_t ob = d_out * d_in * dtype_size(dtype);
  CK(ensure(ctx, ctx->pk_out[0], ob));
  CK(dequant_packed_device(ctx, d_out, d_in, group, gbits, ngroups, dq, qb, ds, dz, dp, dtype, ctx->pk_out[0].p));
  HIPCK(hipMemcpyAsync(out, ctx->pk_out[0].p, ob, hipMemcpyDeviceToHost, ctx->st));
  HIPCK(hipStreamSynchronize(ctx->st));
  return CDCLQ_OK;
}

int cdclq_dequantize_layer_device(cdclq_ctx* ctx, size_t d_out, size_t d_in, size_t group, size_t ngroups,
                                  const uint8_t* codes, const float* scales, const float* zeros, const uint32_t* perm,
                                  int dtype, void* out) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  return dequant_layer_device(ctx, d_out, d_in, group, ngroups, codes, scales, zeros, perm, dtype, out);
}

int cdclq_dequantize_layer(cdclq_ctx* ctx, size_t d_out, size_t d_in, size_t group, size_t ngroups,
                           const uint8_t* codes, const float* scales, const float* zeros, const uint32_t* perm,
                           int dtype, void* out) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  CK(check_dtype(ctx, dtype));
  if (d_out == 0 || d_in == 0) return CDCLQ_OK;
  const std::string why = check_layout(d_in, group, nullptr, ngroups, false);
  if (!why.empty()) return fail(ctx, CDCLQ_INVALID_ARG, why);
  if (!codes || !scales || !zeros || !perm || !out) return fail(ctx, CDCLQ_INVALID_ARG, "null buffer argument");
  const size_t nm = d_out * ngroups;
  HIPCK(hipSetDevice(ctx->device));
  const uint8_t* dc;
  const float *ds, *dz;
  const uint32_t* dp;
  CK(stage_in(ctx, ctx->pk_in[0], codes, d_out * d_in, &dc));
  CK(stage_in(ctx, ctx->pk_in[1], scales, nm, &ds));
  CK(stage_in(ctx, ctx->pk_in[2], zeros, nm, &dz));
  CK(stage_in(ctx, ctx->pk_in[3], perm, d_in, &dp));
  const size_t ob = d_out * d_in * dtype_size(dtype);
  CK(ensure(ctx, ctx->pk_out[0], ob));
  CK(dequant_layer_device(ctx, d_out, d_in, group, ngroups, dc, ds, dz, dp, dtype, ctx->pk_out[0].p));
  HIPCK(hipMemcpyAsync(out, ctx->pk_out[0].p, ob, hipMemcpyDeviceToHost, ctx->st));
  HIPCK(hipStreamSynchronize(ctx->st));
  return CDCLQ_OK;
}

}  // extern "C"
