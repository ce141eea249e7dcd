// Host side of the MI355X engine: the control flow of engine::quantize_layer
// (src/engine.rs:690-799), build_prepared (:320-342) and process_chunk (:366-674), driving the
// gfx950 kernels, plus the C-ABI entry points declared in include/cdclq.h.
//
// Only scalar bookkeeping runs on the host -- validation, the column permutation sort, the
// damping mean, sub-block selection and the per-chunk convergence test -- with the reference's
// exact f64 operation order. Every per-weight operation runs on the GPU.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdint>
#include <cstring>
#include <string>
#include <type_traits>
#include <vector>

#include "cdclq.h"
#include "cdclq_dev.h"
#include "ctx.h"
#include "kernels.h"

namespace {

using namespace cdclq;

double now_secs() {
  using namespace std::chrono;
  return duration<double>(steady_clock::now().time_since_epoch()).count();
}

// Rust's `{:e}` (LowerExp) of an f64: shortest round-trip digits, exponent without '+'/padding.
std::string rust_lower_exp(double d) {
  if (std::isnan(d)) return "NaN";
  if (std::isinf(d)) return d < 0 ? "-inf" : "inf";
  char buf[64];
  for (int p = 0; p < 17; ++p) {
    std::snprintf(buf, sizeof buf, "%.*e", p, d);
    if (std::strtod(buf, nullptr) == d) break;
  }
  char* e = std::strchr(buf, 'e');
  const int ex = std::atoi(e + 1);
  *e = 0;
  return std::string(buf) + "e" + std::to_string(ex);
}


void drain_timing(cdclq_ctx* ctx) {
  for (auto& r : ctx->pending) {
    float ms = 0.0f;
    if (hipEventSynchronize(r.b) == hipSuccess && hipEventElapsedTime(&ms, r.a, r.b) == hipSuccess) {
      ctx->ms[r.phase] += ms;
      ctx->launches[r.phase] += 1;
    }
    ctx->event_pool.push_back(r.a);
    ctx->event_pool.push_back(r.b);
  }
  ctx->pending.clear();
}

size_t effective_group(const cdclq_config* cfg, size_t n) {
  return (cfg->group == 0 || cfg->group >= n) ? n : (size_t)cfg->group;
}

// src/engine.rs:240-258 (same messages)
int validate(cdclq_ctx* ctx, const cdclq_config* cfg, size_t n) {
  if (cfg->bits < 2 || cfg->bits > 8 || cfg->skeleton_bits < 2 || cfg->skeleton_bits > 8)
    return fail(ctx, CDCLQ_INVALID_ARG, "bits and skeleton_bits must be in 2..=8");
  if (cfg->block == 0 || cfg->sub_block == 0) return fail(ctx, CDCLQ_INVALID_ARG, "block and sub_block must be > 0");
  const size_t g = effective_group(cfg, n);
  if (g < n && cfg->block % g != 0 && g % cfg->block != 0)
    return fail(ctx, CDCLQ_INVALID_ARG,
                "group size " + std::to_string(g) + " must divide the block size " + std::to_string(cfg->block) +
                    " (or be a multiple of it)");
  if (cfg->skeleton_pct > 0.0 && g >= n) return fail(ctx, CDCLQ_INVALID_ARG, "the skeleton needs a finite group size");
  if (!(cfg->refine_frac >= 0.0 && cfg->refine_frac <= 1.0))
    return fail(ctx, CDCLQ_INVALID_ARG, "refine_frac must be in [0, 1]");
  return CDCLQ_OK;
}

// Rust `sort_by(|a, b| key[b].partial_cmp(&key[a]).unwrap_or(Equal).then(a.cmp(&b)))`
void sort_desc_index(std::vector<size_t>& idx, const std::vector<double>& key) {
  std::stable_sort(idx.begin(), idx.end(), [&](size_t a, size_t b) {
    const double ka = key[a], kb = key[b];
    if (kb < ka) return true;
    if (kb > ka) return false;
    return a < b;
  });
}

// Blocks of the Cholesky applied per deferred trailing pass (see factor()).
constexpr int kCholDefer = 4;
// Blocks of phase 1 applied per deferred lazy-update pass (see quantize_device()).
constexpr int kLazyDefer = 4;

// U from the flipped matrix `a` (n x n f64, overwritten by L): blocked Cholesky, triangular inverse
// of L into y, then U_ij = (f32) y[n-1-i][n-1-j] (src/linalg.rs:362-375).
int factor(cdclq_ctx* ctx, int n, double* a, double* y, float* u) {
  const int NB = 96;
  hipStream_t st = ctx->st;
  CK(ensure(ctx, ctx->status_d, 16));
  int* status = P<int>(ctx->status_d);
  double* pivot = reinterpret_cast<double*>(P<char>(ctx->status_d) + 8);
  HIPCK(hipMemsetAsync(ctx->status_d.p, 0, 16, st));
  // Blocked Cholesky with deferred trailing updates. Block columns are taken in periods of
  // kCholDefer blocks. Before block c is factored, the earlier blocks of its period are applied to
  // its block column (rows c.., in block order). At the end of a period its blocks are applied, in
  // order, to every column beyond it: to the next period's block columns on the main stream,
  // then to the rest on the side stream, which runs while the next period is factored and is
  // waited for before the next period's own pass touches the same columns. Each block's update
  // is still one k = 96 chain folded into the element (src/linalg.rs:243-270), and every element
  // receives the blocks' updates in block order; only the grouping of launches differs.
  hipStream_t st2 = ctx->st2;
  const int nb = (n + NB - 1) / NB;
  bool side_pending = false;
  for (int c = 0; c < nb; ++c) {
    const int kc = c * NB, kb = std::min(NB, n - kc), kend = kc + kb;
    const int g0 = (c / kCholDefer) * kCholDefer, kg = g0 * NB;
    if (c > g0)  // blocks g0 .. c - 1 applied to block column c
      HIPCK(chol_update(st, n - kc, kb, kc - kg, a + (long)kc * n + kg, n, a + (long)kc * n + kc, n));
    HIPCK(chol_diag(st, n, a, kc, kb, status, pivot));
    if (kend < n) HIPCK(chol_panel(st, n, a, kc, kb, status));
    const bool period_end = (c - g0 == kCholDefer - 1) || c + 1 == nb;
    if (!period_end || kend >= n) continue;
    const int c2 = std::min(n, kend + kCholDefer * NB);  // end of the next period's block columns
    if (side_pending) HIPCK(hipStreamWaitEvent(st, ctx->ev_panel, 0));  // it wrote columns >= kend
    side_pending = false;
    HIPCK(chol_update(st, n - kend, c2 - kend, kend - kg, a + (long)kend * n + kg, n, a + (long)kend * n + kend, n));
    if (c2 < n) {
      HIPCK(hipEventRecord(ctx->ev_col, st));
      HIPCK(hipStreamWaitEvent(st2, ctx->ev_col, 0));
      HIPCK(chol_update(st2, n - c2, n - c2, kend - kg, a + (long)c2 * n + kg, n, a + (long)c2 * n + c2, n));
      HIPCK(hipEventRecord(ctx->ev_panel, st2));
      side_pending = true;
    }
  }
  if (side_pending) HIPCK(hipStreamWaitEvent(st, ctx->ev_panel, 0));
  struct {
    int status;
    int pad;
    double pivot;
  } hs;
  HIPCK(hipMemcpyAsync(&hs, ctx->status_d.p, 16, hipMemcpyDeviceToHost, st));
  HIPCK(hipStreamSynchronize(st));
  if (hs.status) {
    return fail(ctx, CDCLQ_NOT_PD,
                "matrix is not positive definite (pivot " + std::to_string(hs.status - 1) + " = " +
                    rust_lower_exp(hs.pivot) + "); increase --damp or check the Hessian");
  }
  HIPCK(fill_zero_f64(st, y, (size_t)n * n));
  HIPCK(trinv_diag(st, n, a, y, status));
  if (n > NB && n % 2 == 0) {
    // Triangular inverse, right-looking (src/linalg.rs:284-346 with the same per-element
    // operations): block row s needs t_s = L[s:e, 0:s] Y[0:s, 0:s], i.e. per element the chains of
    // the KC panels [0, 256), [256, 512), ... of k < s folded in order, then Y[s:e, 0:s] =
    // -Y_ss t_s. All block rows' t live in T (zeroed: the fold's first C' is 0), and as soon as
    // Y's rows [256 p, 256 p + 256) are final, one GEMM folds panel p's chains into every block
    // row that has the whole panel (block start >= 256 (p + 1)); a block row then folds only its
    // last, partial panel [256 floor(s / 256), s) itself. Every element of t receives its panels'
    // chains in panel order, as in the reference's pgemm_f64. Y[k][j] = 0 for k < j, so the
    // columns past a panel's last row add +0 chains to a +0 accumulator and are skipped.
    CK(ensure(ctx, ctx->tbuf, (size_t)n * n * sizeof(double)));
    double* T = P<double>(ctx->tbuf);
    HIPCK(fill_zero_f64(st, T + (size_t)NB * n, (size_t)(n - NB) * n));
    int done = 0;  // panels folded into every block row that has them
    for (int s = NB; s < n; s += NB) {
      const int e = std::min(s + NB, n), w = e - s, full = s / CDCLQ_KC, kp = full * CDCLQ_KC;
      for (; done < full; ++done) {
        const int k0 = done * CDCLQ_KC, c1 = k0 + CDCLQ_KC;
        const int r0 = (c1 + NB - 1) / NB * NB;  // first block row holding the whole panel
        HIPCK(inv_acc(st, n - r0, c1, CDCLQ_KC, a + (long)r0 * n + k0, n, y + (long)k0 * n, n, T + (long)r0 * n, n));
      }
      if (s > kp)  // the last, partial panel [kp, s)
        HIPCK(inv_acc(st, w, s, s - kp, a + (long)s * n + kp, n, y + (long)kp * n, n, T + (long)s * n, n));
      if (inv_gemm_eligible(w, s, w, y + (long)s * n + s, n, T + (long)s * n, n))
        HIPCK(inv_gemm(st, w, s, w, -1.0, y + (long)s * n + s, n, T + (long)s * n, n, y + (long)s * n, n));
      else
        HIPCK(gemm_chain<double>(st, w, s, w, -1.0, 0, y + (long)s * n + s, n, 1, T + (long)s * n, n, 1,
                                 y + (long)s * n, n, 1, false, (double*)nullptr));
    }
  } else if (n > NB) {  // odd n (rows not 16-byte aligned): per block row, panels split and folded
    CK(ensure(ctx, ctx->tbuf, (size_t)NB * n * sizeof(double)));
    CK(ensure(ctx, ctx->tpart, gemm_partials_elems(NB, n, n) * sizeof(double)));
    for (int s = NB; s < n; s += NB) {
      const int e = std::min(s + NB, n), w = e - s;
      double* t = P<double>(ctx->tbuf);
      // t = L[s:e, 0:s] Y[0:s, 0:s]; Y[s:e, 0:s] = -Y_ss t  (src/linalg.rs:307-343)
      double* tp = s > 256 ? P<double>(ctx->tpart) : nullptr;
      HIPCK(gemm_chain<double>(st, w, s, s, 1.0, 0, a + (long)s * n, n, 1, y, n, 1, t, s, 1, false, tp,
                               /*b_lower_tri=*/true));
      HIPCK(gemm_chain<double>(st, w, s, w, -1.0, 0, y + (long)s * n + s, n, 1, t, s, 1, y + (long)s * n, n, 1, false,
                               (double*)nullptr));
    }
  }
  HIPCK(scatter_u(st, n, y, u));
  return CDCLQ_OK;
}

// Pinned host staging of at least `bytes` (kept by the context; a larger request replaces it
// after the stream has drained, since earlier copies may still read it).
int ensure_pinned(cdclq_ctx* ctx, size_t bytes) {
  if (ctx->pin_size >= bytes) return CDCLQ_OK;
  if (ctx->pin) {
    HIPCK(hipStreamSynchronize(ctx->st));
    HIPCK(hipHostFree(ctx->pin));
    ctx->pin = nullptr;
    ctx->pin_size = 0;
  }
  HIPCK(hipHostMalloc(&ctx->pin, bytes, hipHostMallocDefault));
  ctx->pin_size = bytes;
  return CDCLQ_OK;
}

// The G = E H[:, c0:c0+wd] GEMM of phase 2 (src/engine.rs:548, :608): per-panel chains into
// ctx->part, then folded in panel order into ctx->G.
int grad_gemm(cdclq_ctx* ctx, int rows, int n, int c0, int wd, const float* e, const float* h32, const int* rtiles,
              int ntiles) {
  hipError_t err = panel_gemm(ctx->st, rows, wd, n, e, n, h32 + c0, n, P<float>(ctx->part), rtiles, ntiles);
  if (err == hipSuccess)
    err = fold_panels(ctx->st, rows, wd, (n + 255) / 256, P<float>(ctx->part), P<float>(ctx->G), rtiles, ntiles);
  return err == hipSuccess ? CDCLQ_OK : fail(ctx, CDCLQ_DEVICE, std::string("gradient GEMM: ") + hipGetErrorString(err));
}

// Dead columns, column order and the factor cache entry (U, damped permuted h32) for (hkey, perm):
// src/engine.rs:708-723 with build_prepared (:320-342). A cache entry that matches is reused.
static int prepare(cdclq_ctx* ctx, const float* w, int d_out, int n, const float* h, const char* hkey,
                   const cdclq_config* cfg, int g, std::vector<uint32_t>& perm, std::vector<uint8_t>& dead,
                   size_t& nskel) {
  hipStream_t st = ctx->st;
  const size_t n_ = (size_t)n;
  // ---- dead columns and column order (src/engine.rs:708-717, :271-304)
  CK(ensure(ctx, ctx->diag_d, (size_t)n * 4));
  HIPCK(diag_extract(st, n, h, P<float>(ctx->diag_d)));
  std::vector<float> hd32(n);
  HIPCK(hipMemcpyAsync(hd32.data(), ctx->diag_d.p, (size_t)n * 4, hipMemcpyDeviceToHost, st));
  HIPCK(hipStreamSynchronize(st));
  std::vector<double> hdiag(n);
  dead.assign(n, 0);
  for (int j = 0; j < n; ++j) {
    hdiag[j] = (double)hd32[j];
    dead[j] = hdiag[j] == 0.0;
  }
  nskel = 0;
  perm.clear();
  perm.reserve(n);
  std::vector<uint8_t> in_skel(n, 0);
  if (cfg->skeleton_pct > 0.0 && g < n) {
    const size_t full_groups = (size_t)n / g;
    const double v = std::round(cfg->skeleton_pct / 100.0 * (double)n / (double)g);
    const size_t want = v > 0.0 ? (size_t)v : 0;
    const size_t capg = full_groups > 0 ? full_groups - 1 : 0;
    nskel = std::min(want, capg);
    if (nskel > 0) {
      CK(ensure(ctx, ctx->dead_d, (size_t)n));
      CK(ensure(ctx, ctx->colsq_d, (size_t)n * 8));
      HIPCK(hipMemcpyAsync(ctx->dead_d.p, dead.data(), n, hipMemcpyHostToDevice, st));
      HIPCK(colsq(st, d_out, n, w, P<uint8_t>(ctx->dead_d), P<double>(ctx->colsq_d)));
      std::vector<double> cs(n);
      HIPCK(hipMemcpyAsync(cs.data(), ctx->colsq_d.p, (size_t)n * 8, hipMemcpyDeviceToHost, st));
      HIPCK(hipStreamSynchronize(st));
      std::vector<double> sal(n);
      for (int j = 0; j < n; ++j) sal[j] = hdiag[j] * cs[j];
      std::vector<size_t> idx(n);
      for (int j = 0; j < n; ++j) idx[j] = j;
      sort_desc_index(idx, sal);
      for (size_t t = 0; t < nskel * g; ++t) {
        in_skel[idx[t]] = 1;
        perm.push_back((uint32_t)idx[t]);
      }
    }
  }
  {
    std::vector<size_t> rest;
    rest.reserve(n);
    for (int j = 0; j < n; ++j)
      if (!in_skel[j]) rest.push_back(j);
    if (cfg->act_order) sort_desc_index(rest, hdiag);
    for (size_t j : rest) perm.push_back((uint32_t)j);
  }

  // ---- factor cache (src/engine.rs:718-723) and build_prepared (:320-342)
  const std::string key = hkey ? hkey : "";
  const bool reuse = ctx->cache_valid && ctx->cache_key == key && ctx->cache_n == n_ && ctx->cache_perm == perm;
  CK(ensure(ctx, ctx->perm_d, (size_t)n * 4));
  HIPCK(hipMemcpyAsync(ctx->perm_d.p, perm.data(), (size_t)n * 4, hipMemcpyHostToDevice, st));
  if (!reuse) {
    ctx->cache_valid = false;
    double mean_diag = 0.0;
    for (int i = 0; i < n; ++i) {
      double v = hdiag[perm[i]];
      if (v == 0.0) v = 1.0;
      mean_diag += v;
    }
    mean_diag /= (double)n;
    const double damp_val = cfg->damp * mean_diag;
    CK(ensure(ctx, ctx->cache_h32, (size_t)n * n * 4));
    CK(ensure(ctx, ctx->cache_u, (size_t)n * n * 4));
    CK(ensure(ctx, ctx->a64, (size_t)n * n * 8));
    CK(ensure(ctx, ctx->y64, (size_t)n * n * 8));
    {
      PhaseScope ps(ctx, CDCLQ_PHASE_FACTOR);
      HIPCK(build_flipped(st, n, h, P<uint32_t>(ctx->perm_d), damp_val, P<double>(ctx->a64), P<float>(ctx->cache_h32)));
      CK(factor(ctx, n, P<double>(ctx->a64), P<double>(ctx->y64), P<float>(ctx->cache_u)));
    }
    ctx->cache_valid = true;
    ctx->cache_key = key;
    ctx->cache_perm = perm;
    ctx->cache_n = n_;
    ctx->cache_damp = damp_val;
  }
  return CDCLQ_OK;
}

int quantize_device(cdclq_ctx* ctx, const float* w, size_t d_out_, size_t n_, const float* h, const float* m,
                    const char* hkey, const cdclq_config* cfg, size_t nthreads, uint8_t* codes, float* scales,
                    float* zeros, uint32_t* perm_out, uint8_t* gbits_out, cdclq_layer_stats* stats) {
  if (!cfg) return fail(ctx, CDCLQ_INVALID_ARG, "cfg is null");
  if (!w || !h || !codes || !scales || !zeros || !perm_out || !gbits_out)
    return fail(ctx, CDCLQ_INVALID_ARG, "null buffer argument");
  if (d_out_ == 0 || n_ == 0) return fail(ctx, CDCLQ_INVALID_ARG, "empty layer (d_out and d_in must be > 0)");
  if (n_ > 65535 || d_out_ > (size_t)1 << 20 || d_out_ * n_ > ((size_t)1 << 31) - 1)
    return fail(ctx, CDCLQ_INVALID_ARG, "layer too large for this build (d_in <= 65535, d_out*d_in < 2^31)");
  CK(validate(ctx, cfg, n_));
  ctx->mid_last = cdclq_midpoint_counts{};
  const int d_out = (int)d_out_, n = (int)n_;
  const int g = (int)effective_group(cfg, n_);
  const int ng = (n + g - 1) / g;
  const int bsz = (int)std::min<uint64_t>(cfg->block, (uint64_t)n);
  const int sbw = (int)std::min<uint64_t>(cfg->sub_block, (uint64_t)n);
  hipStream_t st = ctx->st;
  HIPCK(hipSetDevice(ctx->device));
  const double t0 = now_secs();

  std::vector<uint32_t> perm;
  std::vector<uint8_t> dead;
  size_t nskel = 0;
  CK(prepare(ctx, w, d_out, n, h, hkey, cfg, g, perm, dead, nskel));
  const float* U = P<float>(ctx->cache_u);
  const float* H32 = P<float>(ctx->cache_h32);

  // ---- permuted (and optionally target-adjusted) weights (src/engine.rs:726-755)
  std::vector<uint8_t> dead_perm(n);
  for (int j = 0; j < n; ++j) dead_perm[j] = dead[perm[j]];
  CK(ensure(ctx, ctx->deadp_d, (size_t)n));
  HIPCK(hipMemcpyAsync(ctx->deadp_d.p, dead_perm.data(), n, hipMemcpyHostToDevice, st));
  const size_t wn = (size_t)d_out * n;
  CK(ensure(ctx, ctx->wp, wn * 4));
  float* wp = P<float>(ctx->wp);
  HIPCK(permute_w(st, d_out, n, w, P<uint32_t>(ctx->perm_d), P<uint8_t>(ctx->deadp_d), wp));
  if (m) {
    PhaseScope ps(ctx, CDCLQ_PHASE_TARGET);
    CK(ensure(ctx, ctx->mp, (size_t)n * n * 4));
    CK(ensure(ctx, ctx->t1, wn * 4));
    CK(ensure(ctx, ctx->t2, wn * 4));
    float* mp = P<float>(ctx->mp);
    HIPCK(permute_m(st, n, m, P<uint32_t>(ctx->perm_d), (float)ctx->cache_damp, mp));
    float* t1 = P<float>(ctx->t1);
    float* t2 = P<float>(ctx->t2);
    if (chain_gemm_tiles_ok(d_out, n, n, wp, n, mp, n, t1, n)) {
      // matrix cores, panels folded in registers; U^T staged row-major in the factorisation's f64
      // work buffer (free once U is built), so the second GEMM reads B row by row
      CK(ensure(ctx, ctx->a64, (size_t)n * n * 8));
      float* ut = P<float>(ctx->a64);
      HIPCK(transpose_f32(st, n, U, ut));
      HIPCK(chain_gemm_tiles(st, d_out, n, n, wp, n, mp, n, t1, n, 0));
      HIPCK(chain_gemm_tiles(st, d_out, n, n, t1, n, ut, n, t2, n, 2));  // B = U^T, zero above its diagonal
      HIPCK(chain_gemm_tiles(st, d_out, n, n, t2, n, U, n, wp, n, 1));   // B = U, zero below its diagonal
    } else {
      HIPCK(gemm_chain<float>(st, d_out, n, n, 1.0f, 0, wp, n, 1, mp, n, 1, t1, n, 1, false, nullptr));
      HIPCK(gemm_chain<float>(st, d_out, n, n, 1.0f, 0, t1, n, 1, U, 1, n, t2, n, 1, false, nullptr));
      HIPCK(gemm_chain<float>(st, d_out, n, n, 1.0f, 0, t2, n, 1, U, n, 1, wp, n, 1, false, nullptr));
    }
  }
  HIPCK(hipStreamSynchronize(st));
  const double secs_prepare = now_secs() - t0;

  // ---- per-group widths and row chunks (src/engine.rs:760, :768-770)
  std::vector<uint8_t> gbits(ng);
  for (int gi = 0; gi < ng; ++gi) gbits[gi] = (uint8_t)((size_t)gi < nskel ? cfg->skeleton_bits : cfg->bits);
  CK(ensure(ctx, ctx->gbits_d, (size_t)ng));
  HIPCK(hipMemcpyAsync(ctx->gbits_d.p, gbits.data(), ng, hipMemcpyHostToDevice, st));
  const size_t nt = nthreads ? nthreads : 1;
  size_t rcz;
  if (cfg->row_chunk > 0) {
    rcz = cfg->row_chunk;
  } else {
    rcz = (d_out_ + nt - 1) / nt;
    rcz = std::min<size_t>(std::max<size_t>(rcz, 32), 256);
  }
  rcz = std::max<size_t>(std::min(rcz, d_out_), 1);
  const int rc = (int)rcz;
  const int nchunks = (d_out + rc - 1) / rc;

  const double t1 = now_secs();
  // near-midpoint counters (MID_SLOTS u64) and the per-row descent evaluation counts (d_out u32)
  CK(ensure(ctx, ctx->mid_d, MID_SLOTS * 8 + (size_t)d_out * 4));
  unsigned long long* mid = P<unsigned long long>(ctx->mid_d);
  uint32_t* cd_evals = reinterpret_cast<uint32_t*>(mid + MID_SLOTS);
  HIPCK(zero_words(st, reinterpret_cast<int*>(mid), 2 * MID_SLOTS + d_out));
  // ---- phase 1: blocked GPTQ with lazy updates (src/engine.rs:397-479)
  CK(ensure(ctx, ctx->wwork, wn * 4));
  CK(ensure(ctx, ctx->wq, wn * 4));
  CK(ensure(ctx, ctx->ebuf, wn * 4));
  CK(ensure(ctx, ctx->invd, (size_t)n * 4));
  CK(ensure(ctx, ctx->colloss_d, (size_t)nchunks * n * 8));
  float* wwork = P<float>(ctx->wwork);
  float* wq = P<float>(ctx->wq);
  float* eb = P<float>(ctx->ebuf);
  std::vector<double> loss_gptq(nchunks, 0.0);
  std::vector<double> colloss((size_t)nchunks * n);
  {
    PhaseScope ps(ctx, CDCLQ_PHASE_GPTQ);
    HIPCK(hipMemcpyAsync(wwork, wp, wn * 4, hipMemcpyDeviceToDevice, st));
    HIPCK(inv_diag(st, n, U, P<float>(ctx->invd)));
    // Lazy update of W's columns [c0, c1) by blocks b0 .. b1 - 1 (full blocks of bsz columns), in
    // block order, each W -= E[:, block] U[block, c0:c1] as its own chain (src/engine.rs:452-471).
    auto lazy = [&](hipStream_t s, int c0, int c1, int b0, int b1) -> int {
      if (c1 <= c0 || b1 <= b0) return CDCLQ_OK;
      const int k0 = b0 * bsz, k = (b1 - b0) * bsz;
      if (chain_gemm_mfma_ok(d_out, c1 - c0, k, eb + k0, n, U + (long)k0 * n + c0, n, bsz)) {
        HIPCK(chain_gemm_mfma(s, d_out, c1 - c0, k, -1.0f, 1, eb + k0, n, U + (long)k0 * n + c0, n, wwork + c0, n,
                              bsz));
        return CDCLQ_OK;
      }
      for (int b = b0; b < b1; ++b)
        HIPCK(gemm_chain<float>(s, d_out, c1 - c0, bsz, -1.0f, 1, eb + (long)b * bsz, n, 1,
                                U + (long)b * bsz * n + c0, n, 1, wwork + c0, n, 1, false, nullptr));
      return CDCLQ_OK;
    };
    // Blocks are taken in periods of kLazyDefer. Before block b's sweep, the earlier blocks of its
    // period are applied to its columns; at a period's end its blocks are applied to the next
    // period's columns (main stream) and to the rest (side stream, overlapping the next period's
    // sweeps and waited for before the next period's pass reaches the same columns). Every column
    // still receives the blocks' updates in block order. This needs groups that stay inside a
    // block (the group grid reads no column past the block) and blocks of at most one KC panel;
    // otherwise every block's update follows its sweep.
    const int nb = (n + bsz - 1) / bsz;
    const bool in_block = bsz % g == 0;  // groups never reach past their block
    const int defer = (in_block && bsz <= CDCLQ_KC) ? kLazyDefer : 1;
    bool side_pending = false;
    for (int b = 0; b < nb; ++b) {
      const int i1 = b * bsz, i2 = std::min(i1 + bsz, n), cnt = i2 - i1;
      const int p0 = (b / defer) * defer;
      if (b > p0) CK(lazy(st, i1, i2, p0, b));
      HIPCK(gptq_block(st, d_out, n, i1, cnt, g, ng, wwork, U, P<float>(ctx->invd), P<uint8_t>(ctx->gbits_d),
                       cfg->mse_grid, scales, zeros, codes, wq, eb, mid, in_block));
      if ((b - p0 != defer - 1 && b + 1 != nb) || i2 >= n) continue;
      // with groups reaching past a block, the next sweep reads W beyond its block: no overlap
      const int c2 = in_block ? std::min(n, i2 + defer * bsz) : n;
      if (side_pending) HIPCK(hipStreamWaitEvent(st, ctx->ev_panel, 0));  // it wrote columns >= i2
      side_pending = false;
      CK(lazy(st, i2, c2, p0, b + 1));
      if (c2 < n) {
        HIPCK(hipEventRecord(ctx->ev_col, st));
        HIPCK(hipStreamWaitEvent(ctx->st2, ctx->ev_col, 0));
        CK(lazy(ctx->st2, c2, n, p0, b + 1));
        HIPCK(hipEventRecord(ctx->ev_panel, ctx->st2));
        side_pending = true;
      }
    }
    if (side_pending) HIPCK(hipStreamWaitEvent(st, ctx->ev_panel, 0));
    HIPCK(cdclq::colloss(st, d_out, n, rc, eb, P<double>(ctx->colloss_d)));
  }
  HIPCK(hipMemcpyAsync(colloss.data(), ctx->colloss_d.p, colloss.size() * 8, hipMemcpyDeviceToHost, st));
  HIPCK(hipStreamSynchronize(st));
  for (int c = 0; c < nchunks; ++c) {
    double s = 0.0;
    for (int j = 0; j < n; ++j) s += colloss[(size_t)c * n + j];
    loss_gptq[c] = s;
  }

  // ---- phase 2: conflict selection + repair (src/engine.rs:488-671)
  const int n_sb = (n + sbw - 1) / sbw;
  std::vector<double> ld(nchunks, 0.0);
  std::vector<uint64_t> updates(nchunks, 0), refined(nchunks, 0);
  const bool do_cd = cfg->refine_frac > 0.0 && cfg->cd_sweeps > 0 && cfg->passes > 0;
  const bool do_refit = cfg->refit_scales && g <= 1024;
  if (cfg->method == CDCLQ_METHOD_CDCL && (do_cd || do_refit)) {
    PhaseScope ps(ctx, CDCLQ_PHASE_REPAIR);
    std::vector<uint8_t> sel((size_t)nchunks * n_sb, 0);
    if (do_cd) {
      const double kf = std::ceil(cfg->refine_frac * (double)n_sb);
      size_t kk = kf > 0.0 ? (size_t)kf : 0;
      kk = std::min<size_t>(std::max<size_t>(kk, 1), n_sb);
      std::vector<double> sums(n_sb);
      std::vector<size_t> order(n_sb);
      for (int c = 0; c < nchunks; ++c) {
        for (int s = 0; s < n_sb; ++s) {
          const int c0 = s * sbw, c1 = std::min((s + 1) * sbw, n);
          double acc = 0.0;
          for (int j = c0; j < c1; ++j) acc += colloss[(size_t)c * n + j];
          sums[s] = acc;
          order[s] = s;
        }
        sort_desc_index(order, sums);
        for (size_t t = 0; t < kk; ++t) sel[(size_t)c * n_sb + order[t]] = 1;
        refined[c] = kk;
      }
    }
    CK(ensure(ctx, ctx->sel_d, sel.size()));
    HIPCK(hipMemcpyAsync(ctx->sel_d.p, sel.data(), sel.size(), hipMemcpyHostToDevice, st));
    HIPCK(sub_f32(st, wn, wp, wq, eb));  // e = W - W_hat (src/engine.rs:516-519)
    const int wdmax = std::max(do_cd ? sbw : 1, do_refit ? g : 1);
    CK(ensure(ctx, ctx->part, panel_partials_elems(d_out, wdmax, n) * 4));
    CK(ensure(ctx, ctx->G, (size_t)d_out * wdmax * 4));
    // Per-pass logs of accepted deltas (folded into the chunk losses in the reference's order).
    const int cap = std::max(1, do_cd ? sbw * (int)cfg->cd_sweeps : 1);
    CK(ensure(ctx, ctx->rlog, (size_t)ng * d_out * 8));
    CK(ensure(ctx, ctx->rcnt, (size_t)ng * d_out * 4));
    if (do_cd) {
      CK(ensure(ctx, ctx->clog, (size_t)n_sb * d_out * cap * 8));
      CK(ensure(ctx, ctx->ccnt, (size_t)n_sb * d_out * 4));
    }
    double* rlog = P<double>(ctx->rlog);
    uint32_t* rcnt = P<uint32_t>(ctx->rcnt);
    double* clog = do_cd ? P<double>(ctx->clog) : nullptr;
    uint32_t* ccnt = do_cd ? P<uint32_t>(ctx->ccnt) : nullptr;
    // Per-pass transfers, each one copy through pinned memory: down, the chunk losses and update
    // counts (ld_d = [ld f64 | upd u64]); up, the active flags and the tile lists (rtiles_d =
    // [active u8, padded to 16 bytes | tile lists i32]).
    CK(ensure(ctx, ctx->ld_d, (size_t)nchunks * 16));
    double* ldd = P<double>(ctx->ld_d);
    uint64_t* updd = reinterpret_cast<uint64_t*>(ldd + nchunks);
    HIPCK(hipMemsetAsync(ldd, 0, (size_t)nchunks * 8, st));
    std::vector<uint8_t> act(nchunks, 1);
    std::vector<double> prev(nchunks, 0.0);
    std::vector<uint64_t> upd(nchunks);
    // The gradient GEMM runs only over the 128-row tiles that hold rows of a chunk still being
    // repaired: list 0 for the refit steps (active chunks), list 1 + s for CD sub-block s (active
    // chunks that selected it). A null list means every tile (the final refit).
    const int rt = panel_row_tile(), ntile = (d_out + rt - 1) / rt;
    std::vector<int> tl((size_t)(1 + n_sb) * ntile), tcnt(1 + n_sb);
    const size_t apad = ((size_t)nchunks + 15) / 16 * 16, up_bytes = apad + tl.size() * sizeof(int);
    CK(ensure(ctx, ctx->rtiles_d, up_bytes));
    uint8_t* active = P<uint8_t>(ctx->rtiles_d);
    int* rtiles = reinterpret_cast<int*>(P<char>(ctx->rtiles_d) + apad);
    CK(ensure_pinned(ctx, up_bytes + (size_t)nchunks * 16));
    char* pin_up = static_cast<char*>(ctx->pin);
    char* pin_down = pin_up + up_bytes;
    auto upload_pass = [&]() -> int {  // the previous upload has finished: every pass ends in a sync
      std::memcpy(pin_up, act.data(), nchunks);
      std::memcpy(pin_up + apad, tl.data(), tl.size() * sizeof(int));
      HIPCK(hipMemcpyAsync(ctx->rtiles_d.p, pin_up, up_bytes, hipMemcpyHostToDevice, st));
      return CDCLQ_OK;
    };
    auto download_pass = [&]() -> int {
      HIPCK(hipMemcpyAsync(pin_down, ldd, (size_t)nchunks * 16, hipMemcpyDeviceToHost, st));
      HIPCK(hipStreamSynchronize(st));
      std::memcpy(ld.data(), pin_down, (size_t)nchunks * 8);
      std::memcpy(upd.data(), pin_down + (size_t)nchunks * 8, (size_t)nchunks * 8);
      return CDCLQ_OK;
    };
    auto build_tiles = [&]() -> int {
      for (int l = 0; l <= n_sb; ++l) {
        int cnt = 0;
        for (int t = 0; t < ntile; ++t) {
          const int c_lo = (t * rt) / rc, c_hi = (std::min((t + 1) * rt, d_out) - 1) / rc;
          bool need = false;
          for (int c = c_lo; c <= c_hi && !need; ++c)
            need = act[c] && (l == 0 || sel[(size_t)c * n_sb + (l - 1)]);
          if (need) tl[(size_t)l * ntile + cnt++] = t;
        }
        tcnt[l] = cnt;
      }
      return upload_pass();
    };
    CK(build_tiles());
    bool all_tiles = false;
    auto refit_all = [&]() -> int {
      HIPCK(hipMemsetAsync(rcnt, 0, (size_t)ng * d_out * 4, st));
      for (int gi = 0; gi < ng; ++gi) {
        const int c0 = gi * g, wd = std::min(c0 + g, n) - c0;
        const int* tl0 = all_tiles ? nullptr : rtiles;
        const int nt0 = all_tiles ? ntile : tcnt[0];
        // the refit kernel folds the per-panel chains itself where it can (one launch less)
        const bool fused = refit_folds_chains(wd);
        if (fused)
          HIPCK(panel_gemm(st, d_out, wd, n, eb, n, H32 + c0, n, P<float>(ctx->part), tl0, nt0));
        else
          CK(grad_gemm(ctx, d_out, n, c0, wd, eb, H32, tl0, nt0));
        HIPCK(refit_group(st, d_out, n, ng, g, gi, rc, P<float>(ctx->G), H32, codes, scales, zeros, wq, eb,
                          active, rlog + (size_t)gi * d_out, rcnt + (size_t)gi * d_out,
                          fused ? P<float>(ctx->part) : nullptr, fused ? (n + 255) / 256 : 0));
      }
      return CDCLQ_OK;
    };
    const uint64_t npass = cfg->passes > 0 ? cfg->passes : 1;
    for (uint64_t pass = 0; pass < npass; ++pass) {
      HIPCK(hipMemsetAsync(updd, 0, (size_t)nchunks * 8, st));
      if (do_refit) CK(refit_all());
      if (do_cd) {
        HIPCK(hipMemsetAsync(ccnt, 0, (size_t)n_sb * d_out * 4, st));
        for (int s = 0; s < n_sb; ++s) {
          bool any = false;
          for (int c = 0; c < nchunks && !any; ++c) any = act[c] && sel[(size_t)c * n_sb + s];
          if (!any) continue;
          const int c0 = s * sbw, wd = std::min(c0 + sbw, n) - c0;
          const int* tl_s = rtiles + (size_t)(1 + s) * ntile;
          // the descent kernel folds the per-panel chains itself where it can (one launch less)
          const bool fused = cd_folds_chains(wd);
          if (fused)
            HIPCK(panel_gemm(st, d_out, wd, n, eb, n, H32 + c0, n, P<float>(ctx->part), tl_s, tcnt[1 + s]));
          else
            CK(grad_gemm(ctx, d_out, n, c0, wd, eb, H32, tl_s, tcnt[1 + s]));
          HIPCK(cd_subblock(st, d_out, n, ng, g, c0, wd, s, n_sb, rc, (int)cfg->cd_sweeps, P<float>(ctx->G), H32,
                            P<uint8_t>(ctx->gbits_d), scales, zeros, codes, wq, eb, active,
                            P<uint8_t>(ctx->sel_d), clog + (size_t)s * d_out * cap, ccnt + (size_t)s * d_out, cap,
                            mid, cd_evals, fused ? P<float>(ctx->part) : nullptr, fused ? (n + 255) / 256 : 0));
        }
      }
      HIPCK(pass_accum(st, d_out, rc, nchunks, do_refit ? ng : 0, rlog, rcnt, do_cd ? n_sb : 0, cap, clog, ccnt,
                       active, ldd, updd));
      CK(download_pass());
      bool any_active = false;
      for (int c = 0; c < nchunks; ++c) {
        if (!act[c]) continue;
        updates[c] += upd[c];
        const double gain = prev[c] - ld[c];
        prev[c] = ld[c];
        if (upd[c] == 0 || gain < cfg->tol * (loss_gptq[c] + ld[c]))
          act[c] = 0;  // converged (src/engine.rs:663-665)
        else
          any_active = true;
      }
      if (!any_active) break;
      CK(build_tiles());
    }
    if (do_refit) {  // final refit (src/engine.rs:668-670)
      std::fill(act.begin(), act.end(), 1);
      all_tiles = true;
      CK(upload_pass());
      HIPCK(hipMemsetAsync(updd, 0, (size_t)nchunks * 8, st));
      CK(refit_all());
      HIPCK(pass_accum(st, d_out, rc, nchunks, ng, rlog, rcnt, 0, cap, clog, ccnt, active, ldd, updd));
      CK(download_pass());
      for (int c = 0; c < nchunks; ++c) updates[c] += upd[c];
    }
  }
  HIPCK(hipStreamSynchronize(st));
  const double secs_quant = now_secs() - t1;
  {
    std::vector<unsigned long long> mh(MID_SLOTS);
    std::vector<uint32_t> ev(d_out);
    HIPCK(hipMemcpyAsync(mh.data(), mid, MID_SLOTS * 8, hipMemcpyDeviceToHost, st));
    HIPCK(hipMemcpyAsync(ev.data(), cd_evals, (size_t)d_out * 4, hipMemcpyDeviceToHost, st));
    HIPCK(hipStreamSynchronize(st));
    cdclq_midpoint_counts mc{};
    mc.code_decisions = (uint64_t)d_out * n;
    mc.code_near = mh[MID_CODE_NEAR];
    mc.zero_decisions = (uint64_t)d_out * ng;
    mc.zero_near = mh[MID_ZERO_NEAR];
    for (uint32_t v : ev) mc.cd_decisions += v;
    mc.cd_near = mh[MID_CD_NEAR];
    ctx->mid_last = mc;
  }

  std::memcpy(perm_out, perm.data(), (size_t)n * 4);
  std::memcpy(gbits_out, gbits.data(), (size_t)ng);
  if (stats) {
    cdclq_layer_stats s{};
    for (int c = 0; c < nchunks; ++c) {
      s.loss_gptq += loss_gptq[c];
      s.loss_final += loss_gptq[c] + ld[c];
      s.subblocks_total += (uint64_t)n_sb;
      s.subblocks_refined += refined[c];
      s.code_updates += updates[c];
    }
    s.skeleton_groups = nskel;
    size_t row_bits = 0;
    for (int j = 0; j < n; ++j) row_bits += gbits[j / g];
    s.bits_codes = (double)row_bits / (double)n;
    s.bits_total = s.bits_codes + 24.0 / (double)g;
    s.secs_prepare = secs_prepare;
    s.secs_quant = secs_quant;
    *stats = s;
  }
  return CDCLQ_OK;
}

// One launch of the matrix-core Gram kernel over several (X, Y, H) jobs (src/linalg.rs:388-418).
// The status words and the job / tile lists live in the context's grow-only workspace, or, when
// `fixed` is set (the allocation-free entry point), in that GPU's fixed scratch memory
// (kGramScratchBytes: 256 B of status, 256 B for the job record, then the tiles).
int gram_batch_device(cdclq_ctx* ctx, int count, const float* const* xs, const float* const* ys, const size_t* ts,
                      const size_t* ns, double* const* hs, char* fixed = nullptr) {
  if (count <= 0) return CDCLQ_OK;
  if (!xs || !ys || !ts || !ns || !hs) return fail(ctx, CDCLQ_INVALID_ARG, "null buffer argument");
  HIPCK(hipSetDevice(ctx->device));
  hipStream_t st = ctx->st;
  std::vector<GramJob> jobs;
  std::vector<int> syms;
  bool vec4 = true;
  for (int i = 0; i < count; ++i) {
    if (!xs[i] || !ys[i] || !hs[i]) return fail(ctx, CDCLQ_INVALID_ARG, "null buffer argument");
    if (ns[i] == 0 || ts[i] == 0) continue;
    if (ns[i] > 65535 || ts[i] > ((size_t)1 << 31) - 4096)
      return fail(ctx, CDCLQ_INVALID_ARG, "gram_accumulate: n <= 65535 and t < 2^31 in this build");
    jobs.push_back(GramJob{xs[i], ys[i], hs[i], (int)ns[i], (int)ts[i]});
    vec4 = vec4 && (ns[i] % 4 == 0) && ((uintptr_t)xs[i] % 16 == 0) && ((uintptr_t)ys[i] % 16 == 0);
  }
  if (jobs.empty()) return CDCLQ_OK;
  if (fixed && (jobs.size() != 1 || 16 * (jobs.size() + 1) > 256 || sizeof(GramJob) > 256))
    return fail(ctx, CDCLQ_INVALID_ARG, "gram_accumulate: the allocation-free path takes one accumulation");
  // Mirrored (upper-triangle-only) tiles need Y == X and a bitwise-symmetric incoming H.
  int* status;
  if (fixed) {
    status = reinterpret_cast<int*>(fixed);
  } else {
    CK(ensure(ctx, ctx->status_d, 16 * (jobs.size() + 1)));
    status = P<int>(ctx->status_d);
  }
  HIPCK(zero_words(st, status, (int)(4 * (jobs.size() + 1))));
  for (size_t i = 0; i < jobs.size(); ++i)
    if (jobs[i].x == jobs[i].y) HIPCK(sym_check(st, jobs[i].n, jobs[i].h, status + 4 * i));
  std::vector<int> flags(4 * jobs.size());
  HIPCK(hipMemcpyAsync(flags.data(), status, flags.size() * 4, hipMemcpyDeviceToHost, st));
  HIPCK(hipStreamSynchronize(st));
  // Jobs whose tiles are all interior go to the direct-to-LDS kernel, the rest to k_gram_mfma.
  std::vector<int4> tiles[2];
  for (size_t i = 0; i < jobs.size(); ++i) {
    const bool sym = jobs[i].x == jobs[i].y && flags[4 * i] == 0;
    if (gram_dma_eligible(jobs[i].n, jobs[i].t, jobs[i].x, jobs[i].y))
      gram_dma_tiles((int)i, jobs[i].n, sym, tiles[1]);
    else
      gram_mfma_tiles((int)i, jobs[i].n, sym, tiles[0]);
  }
  // XCD-aware order: workgroup w runs on XCD w % 8. The direct-to-LDS tiles go in gangs of 4 x 8
  // neighbouring tiles, one gang per XCD at a time (the gang's 32 workgroups share 4 X and 8 Y
  // stripes in that XCD's L2); the others in a contiguous run per XCD (sharing X stripes).
  gram_dma_order(tiles[1]);
  {
    auto& tl = tiles[0];
    const size_t nx = 8, m = tl.size();
    std::vector<int4> ord(m);
    const size_t per = (m + nx - 1) / nx;
    size_t w = 0;
    for (size_t k = 0; k < per; ++k)
      for (size_t x = 0; x < nx; ++x) {
        const size_t src = x * per + k;
        if (src < m) ord[w++] = tl[src];
      }
    tl.swap(ord);
  }
  const size_t ntile = tiles[0].size() + tiles[1].size();
  GramJob* djobs;
  int4* dtiles;
  int* prog = nullptr;  // gang pacing words, one per tile slot (none on the allocation-free path)
  if (fixed) {
    if (ntile > kGramScratchTiles)
      return fail(ctx, CDCLQ_INVALID_ARG, "gram_accumulate: tile list exceeds the allocation-free scratch");
    djobs = reinterpret_cast<GramJob*>(fixed + 256);
    dtiles = reinterpret_cast<int4*>(fixed + 512);
  } else {
    CK(ensure(ctx, ctx->tiles_d, jobs.size() * sizeof(GramJob) + 64 + ntile * (sizeof(int4) + sizeof(int))));
    char* base = P<char>(ctx->tiles_d);
    djobs = reinterpret_cast<GramJob*>(base);
    dtiles = reinterpret_cast<int4*>(base + ((jobs.size() * sizeof(GramJob) + 63) / 64) * 64);
    prog = reinterpret_cast<int*>(dtiles + ntile);
    HIPCK(zero_words(st, prog, (int)ntile));
  }
  HIPCK(hipMemcpyAsync(djobs, jobs.data(), jobs.size() * sizeof(GramJob), hipMemcpyHostToDevice, st));
  HIPCK(hipMemcpyAsync(dtiles, tiles[0].data(), tiles[0].size() * sizeof(int4), hipMemcpyHostToDevice, st));
  HIPCK(hipMemcpyAsync(dtiles + tiles[0].size(), tiles[1].data(), tiles[1].size() * sizeof(int4),
                       hipMemcpyHostToDevice, st));
  {
    PhaseScope ps(ctx, CDCLQ_PHASE_GRAM);
    HIPCK(gram_mfma(st, djobs, dtiles, (int)tiles[0].size(), vec4));
    HIPCK(gram_dma(st, djobs, dtiles + tiles[0].size(), (int)tiles[1].size(), prog));
  }
  HIPCK(hipStreamSynchronize(st));
  return CDCLQ_OK;
}

// linalg::sgemm / dgemm and pgemm_f32 / pgemm_f64 (src/linalg.rs:56-184) on device memory: C = alpha A B
// + beta C with arbitrary strides, in matrixmultiply's per-element order. Row-major f32 products
// with alpha 1 and beta 0 (the shape of the asymmetric target) run on the matrix cores, panels
// folded in registers; the rest on the chain GEMMs (panels split over workgroups when k spans
// several, then folded in order).
template <typename T>
int gemm_device(cdclq_ctx* ctx, size_t m, size_t k, size_t n, T alpha, const T* a, ptrdiff_t rsa, ptrdiff_t csa,
                const T* b, ptrdiff_t rsb, ptrdiff_t csb, T beta, T* c, ptrdiff_t rsc, ptrdiff_t csc) {
  if (m == 0 || n == 0) return CDCLQ_OK;
  if (!c || (k > 0 && (!a || !b))) return fail(ctx, CDCLQ_INVALID_ARG, "null buffer argument");
  if (m > (size_t)INT32_MAX / 2 || n > (size_t)INT32_MAX / 2 || k > (size_t)INT32_MAX / 2)
    return fail(ctx, CDCLQ_INVALID_ARG, "gemm: m, k and n must be below 2^30 in this build");
  HIPCK(hipSetDevice(ctx->device));
  const int mi = (int)m, ki = (int)k, ni = (int)n;
  if constexpr (std::is_same<T, float>::value) {
    if (alpha == 1.0f && beta == 0.0f && csa == 1 && csb == 1 && csc == 1 &&
        chain_gemm_tiles_ok(mi, ni, ki, a, rsa, b, rsb, c, rsc)) {
      HIPCK(chain_gemm_tiles(ctx->st, mi, ni, ki, a, rsa, b, rsb, c, rsc, 0));
      HIPCK(hipStreamSynchronize(ctx->st));
      return CDCLQ_OK;
    }
  }
  T* part = nullptr;
  if (k > (size_t)CDCLQ_KC) {
    CK(ensure(ctx, ctx->gemm_part, gemm_partials_elems(mi, ni, ki) * sizeof(T)));
    part = P<T>(ctx->gemm_part);
  }
  HIPCK(gemm_chain<T>(ctx->st, mi, ni, ki, alpha, beta, a, rsa, csa, b, rsb, csb, c, rsc, csc, false, part));
  HIPCK(hipStreamSynchronize(ctx->st));
  return CDCLQ_OK;
}

int gram_device(cdclq_ctx* ctx, const float* x, const float* y, size_t t, size_t n, double* h) {
  if (!x || !y || !h) return fail(ctx, CDCLQ_INVALID_ARG, "null buffer argument");
  return gram_batch_device(ctx, 1, &x, &y, &t, &n, &h);
}

int uchol_device(cdclq_ctx* ctx, const double* h, size_t n_, float* u) {
  if (!h || !u) return fail(ctx, CDCLQ_INVALID_ARG, "null buffer argument");
  if (n_ == 0) return CDCLQ_OK;
  if (n_ > 65535) return fail(ctx, CDCLQ_INVALID_ARG, "n > 65535 is not supported in this build");
  HIPCK(hipSetDevice(ctx->device));
  const int n = (int)n_;
  CK(ensure(ctx, ctx->a64, (size_t)n * n * 8));
  CK(ensure(ctx, ctx->y64, (size_t)n * n * 8));
  {
    PhaseScope ps(ctx, CDCLQ_PHASE_FACTOR);
    HIPCK(build_flipped_f64(ctx->st, n, h, P<double>(ctx->a64)));
    CK(factor(ctx, n, P<double>(ctx->a64), P<double>(ctx->y64), u));
  }
  HIPCK(hipStreamSynchronize(ctx->st));
  return CDCLQ_OK;
}

}  // namespace

// ====================================================================== C ABI
extern "C" {

int cdclq_abi_version(void) { return CDCLQ_ABI_VERSION; }
size_t cdclq_sizeof_config(void) { return sizeof(cdclq_config); }
size_t cdclq_sizeof_stats(void) { return sizeof(cdclq_layer_stats); }

void cdclq_default_config(cdclq_config* c) {
  if (!c) return;
  std::memset(c, 0, sizeof(*c));
  c->bits = 3;
  c->group = 128;
  c->block = 128;
  c->damp = 0.01;
  c->act_order = 1;
  c->skeleton_pct = 0.0;
  c->skeleton_bits = 8;
  c->mse_grid = 0;
  c->method = CDCLQ_METHOD_CDCL;
  c->refine_frac = 1.0;
  c->sub_block = 64;
  c->cd_sweeps = 1;
  c->passes = 10;
  c->tol = 1e-3;
  c->refit_scales = 1;
  c->row_chunk = 0;
}

size_t cdclq_num_groups(const cdclq_config* cfg, size_t d_in) {
  if (!cfg || d_in == 0) return 0;
  const size_t g = effective_group(cfg, d_in);
  return (d_in + g - 1) / g;
}

int cdclq_ctx_create(int device, cdclq_ctx** out) {
  if (!out) return CDCLQ_INVALID_ARG;
  *out = nullptr;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) return CDCLQ_DEVICE;
  if (hipSetDevice(device) != hipSuccess) return CDCLQ_DEVICE;
  cdclq_ctx* ctx = new (std::nothrow) cdclq_ctx();
  if (!ctx) return CDCLQ_OOM;
  ctx->device = device;
  if (hipStreamCreateWithFlags(&ctx->st, hipStreamNonBlocking) != hipSuccess ||
      hipStreamCreateWithFlags(&ctx->st2, hipStreamNonBlocking) != hipSuccess ||
      hipEventCreateWithFlags(&ctx->ev_col, hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&ctx->ev_panel, hipEventDisableTiming) != hipSuccess) {
    for (hipEvent_t e : {ctx->ev_col, ctx->ev_panel})
      if (e) (void)hipEventDestroy(e);
    for (hipStream_t q : {ctx->st2, ctx->st})
      if (q) (void)hipStreamDestroy(q);
    delete ctx;
    return CDCLQ_DEVICE;
  }
  // this GPU's fixed scratch of the allocation-free Gram entry point (looked up once per device)
  ctx->gram_scratch_err = gram_scratch(device, &ctx->gram_scratch);
  *out = ctx;
  return CDCLQ_OK;
}

void cdclq_ctx_destroy(cdclq_ctx* ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->st);
  (void)hipStreamSynchronize(ctx->st2);
  drain_timing(ctx);
  DevBuf* bufs[] = {&ctx->w_in, &ctx->h_in, &ctx->m_in, &ctx->x_in, &ctx->y_in, &ctx->h64_in, &ctx->u_out,
                    &ctx->codes_o, &ctx->scales_o, &ctx->zeros_o, &ctx->wp, &ctx->wwork, &ctx->wq, &ctx->ebuf,
                    &ctx->gbits_d, &ctx->perm_d, &ctx->deadp_d, &ctx->dead_d, &ctx->diag_d, &ctx->colsq_d,
                    &ctx->invd, &ctx->colloss_d, &ctx->G, &ctx->part, &ctx->rlog, &ctx->rcnt, &ctx->clog, &ctx->ccnt, &ctx->rtiles_d,
                    &ctx->sel_d, &ctx->ld_d, &ctx->mp, &ctx->t1, &ctx->t2, &ctx->a64, &ctx->y64,
                    &ctx->tbuf, &ctx->tpart, &ctx->status_d, &ctx->tiles_d, &ctx->proxy_p, &ctx->cs_d, &ctx->gemm_part, &ctx->mid_d,
                    &ctx->cache_u, &ctx->cache_h32, &ctx->pk_flag};
  for (DevBuf* b : bufs) free_buf(*b);
  for (DevBuf& b : ctx->pk_in) free_buf(b);
  for (DevBuf& b : ctx->pk_out) free_buf(b);
  for (DevBuf& b : ctx->pk_tab) free_buf(b);
  for (hipEvent_t e : ctx->event_pool) (void)hipEventDestroy(e);
  if (ctx->pin) (void)hipHostFree(ctx->pin);
  (void)hipEventDestroy(ctx->ev_col);
  (void)hipEventDestroy(ctx->ev_panel);
  (void)hipStreamDestroy(ctx->st2);
  (void)hipStreamDestroy(ctx->st);
  delete ctx;
}

const char* cdclq_last_error(const cdclq_ctx* ctx) { return ctx ? ctx->err.c_str() : "null context"; }

int cdclq_ctx_clear_cache(cdclq_ctx* ctx) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->cache_valid = false;
  ctx->cache_key.clear();
  ctx->cache_perm.clear();
  return CDCLQ_OK;
}

int cdclq_quantize_layer_device(cdclq_ctx* ctx, const float* w, size_t d_out, size_t d_in, const float* h,
                                const float* m, const char* hkey, const cdclq_config* cfg, size_t nthreads,
                                uint8_t* codes, float* scales, float* zeros, uint32_t* perm, uint8_t* gbits,
                                cdclq_layer_stats* stats) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  return quantize_device(ctx, w, d_out, d_in, h, m, hkey, cfg, nthreads, codes, scales, zeros, perm, gbits, stats);
}

int cdclq_prepare_layer_device(cdclq_ctx* ctx, const float* w, size_t d_out, size_t d_in, const float* h,
                               const char* hkey, const cdclq_config* cfg) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  if (!cfg) return fail(ctx, CDCLQ_INVALID_ARG, "cfg is null");
  if (!w || !h) return fail(ctx, CDCLQ_INVALID_ARG, "null buffer argument");
  if (d_out == 0 || d_in == 0) return fail(ctx, CDCLQ_INVALID_ARG, "empty layer (d_out and d_in must be > 0)");
  if (d_in > 65535 || d_out > (size_t)1 << 20 || d_out * d_in > ((size_t)1 << 31) - 1)
    return fail(ctx, CDCLQ_INVALID_ARG, "layer too large for this build (d_in <= 65535, d_out*d_in < 2^31)");
  CK(validate(ctx, cfg, d_in));
  HIPCK(hipSetDevice(ctx->device));
  std::vector<uint32_t> perm;
  std::vector<uint8_t> dead;
  size_t nskel = 0;
  CK(prepare(ctx, w, (int)d_out, (int)d_in, h, hkey, cfg, (int)effective_group(cfg, d_in), perm, dead, nskel));
  HIPCK(hipStreamSynchronize(ctx->st));
  return CDCLQ_OK;
}

int cdclq_quantize_layer(cdclq_ctx* ctx, const float* w, size_t d_out, size_t d_in, const float* h, const float* m,
                         const char* hkey, const cdclq_config* cfg, size_t nthreads, uint8_t* codes, float* scales,
                         float* zeros, uint32_t* perm, uint8_t* gbits, cdclq_layer_stats* stats) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  if (!cfg) return fail(ctx, CDCLQ_INVALID_ARG, "cfg is null");
  if (!w || !h || !codes || !scales || !zeros || !perm || !gbits)
    return fail(ctx, CDCLQ_INVALID_ARG, "null buffer argument");
  if (d_out == 0 || d_in == 0) return fail(ctx, CDCLQ_INVALID_ARG, "empty layer (d_out and d_in must be > 0)");
  CK(validate(ctx, cfg, d_in));
  HIPCK(hipSetDevice(ctx->device));
  const size_t ng = cdclq_num_groups(cfg, d_in);
  const size_t wn = d_out * d_in, hn = d_in * d_in;
  CK(ensure(ctx, ctx->w_in, wn * 4));
  CK(ensure(ctx, ctx->h_in, hn * 4));
  CK(ensure(ctx, ctx->codes_o, wn));
  CK(ensure(ctx, ctx->scales_o, d_out * ng * 4));
  CK(ensure(ctx, ctx->zeros_o, d_out * ng * 4));
  HIPCK(hipMemcpyAsync(ctx->w_in.p, w, wn * 4, hipMemcpyHostToDevice, ctx->st));
  HIPCK(hipMemcpyAsync(ctx->h_in.p, h, hn * 4, hipMemcpyHostToDevice, ctx->st));
  if (m) {
    CK(ensure(ctx, ctx->m_in, hn * 4));
    HIPCK(hipMemcpyAsync(ctx->m_in.p, m, hn * 4, hipMemcpyHostToDevice, ctx->st));
  }
  CK(quantize_device(ctx, P<float>(ctx->w_in), d_out, d_in, P<float>(ctx->h_in), m ? P<float>(ctx->m_in) : nullptr,
                     hkey, cfg, nthreads, P<uint8_t>(ctx->codes_o), P<float>(ctx->scales_o), P<float>(ctx->zeros_o),
                     perm, gbits, stats));
  HIPCK(hipMemcpyAsync(codes, ctx->codes_o.p, wn, hipMemcpyDeviceToHost, ctx->st));
  HIPCK(hipMemcpyAsync(scales, ctx->scales_o.p, d_out * ng * 4, hipMemcpyDeviceToHost, ctx->st));
  HIPCK(hipMemcpyAsync(zeros, ctx->zeros_o.p, d_out * ng * 4, hipMemcpyDeviceToHost, ctx->st));
  HIPCK(hipStreamSynchronize(ctx->st));
  return CDCLQ_OK;
}

int cdclq_gram_accumulate_device(cdclq_ctx* ctx, const float* x, const float* y, size_t t, size_t n, double* h) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  return gram_device(ctx, x, y, t, n, h);
}

int cdclq_gram_accumulate_device_noalloc(cdclq_ctx* ctx, const float* x, const float* y, size_t t, size_t n,
                                        double* h) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  if (!x || !y || !h) return fail(ctx, CDCLQ_INVALID_ARG, "null buffer argument");
  if (n == 0 || t == 0) return CDCLQ_OK;
  if (n > (size_t)kGramNoAllocMaxN)
    return fail(ctx, CDCLQ_INVALID_ARG, "gram_accumulate_device_noalloc: n = " + std::to_string(n) +
                                            " exceeds the allocation-free limit of " +
                                            std::to_string(kGramNoAllocMaxN) + " columns");
  if (!ctx->gram_scratch)
    return fail(ctx, CDCLQ_DEVICE, std::string("allocation-free scratch unavailable on this device (") +
                                       hipGetErrorString(ctx->gram_scratch_err) + ")");
  return gram_batch_device(ctx, 1, &x, &y, &t, &n, &h, static_cast<char*>(ctx->gram_scratch));
}

int cdclq_ctx_last_midpoint_counts(const cdclq_ctx* ctx, cdclq_midpoint_counts* out) {
  if (!ctx || !out) return CDCLQ_INVALID_ARG;
  *out = ctx->mid_last;
  return CDCLQ_OK;
}

int cdclq_sgemm_device(cdclq_ctx* ctx, size_t m, size_t k, size_t n, float alpha, const float* a, ptrdiff_t rsa,
                       ptrdiff_t csa, const float* b, ptrdiff_t rsb, ptrdiff_t csb, float beta, float* c, ptrdiff_t rsc,
                       ptrdiff_t csc) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  return gemm_device<float>(ctx, m, k, n, alpha, a, rsa, csa, b, rsb, csb, beta, c, rsc, csc);
}

int cdclq_dgemm_device(cdclq_ctx* ctx, size_t m, size_t k, size_t n, double alpha, const double* a, ptrdiff_t rsa,
                       ptrdiff_t csa, const double* b, ptrdiff_t rsb, ptrdiff_t csb, double beta, double* c,
                       ptrdiff_t rsc, ptrdiff_t csc) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  return gemm_device<double>(ctx, m, k, n, alpha, a, rsa, csa, b, rsb, csb, beta, c, rsc, csc);
}

int cdclq_gram_accumulate_batch_device(cdclq_ctx* ctx, int count, const float* const* xs, const float* const* ys,
                                       const size_t* ts, const size_t* ns, double* const* hs) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  return gram_batch_device(ctx, count, xs, ys, ts, ns, hs);
}

int cdclq_gram_accumulate(cdclq_ctx* ctx, const float* x, const float* y, size_t t, size_t n, double* h) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  if (!x || !y || !h) return fail(ctx, CDCLQ_INVALID_ARG, "null buffer argument");
  if (n == 0 || t == 0) return CDCLQ_OK;
  HIPCK(hipSetDevice(ctx->device));
  const bool sym = (x == y);
  CK(ensure(ctx, ctx->x_in, t * n * 4));
  CK(ensure(ctx, ctx->h64_in, n * n * 8));
  HIPCK(hipMemcpyAsync(ctx->x_in.p, x, t * n * 4, hipMemcpyHostToDevice, ctx->st));
  if (!sym) {
    CK(ensure(ctx, ctx->y_in, t * n * 4));
    HIPCK(hipMemcpyAsync(ctx->y_in.p, y, t * n * 4, hipMemcpyHostToDevice, ctx->st));
  }
  HIPCK(hipMemcpyAsync(ctx->h64_in.p, h, n * n * 8, hipMemcpyHostToDevice, ctx->st));
  CK(gram_device(ctx, P<float>(ctx->x_in), sym ? P<float>(ctx->x_in) : P<float>(ctx->y_in), t, n,
                 P<double>(ctx->h64_in)));
  HIPCK(hipMemcpyAsync(h, ctx->h64_in.p, n * n * 8, hipMemcpyDeviceToHost, ctx->st));
  HIPCK(hipStreamSynchronize(ctx->st));
  return CDCLQ_OK;
}

int cdclq_hessian_accumulate_device(cdclq_ctx* ctx, const float* x, const float* y, const float* token_w, size_t t,
                                    size_t n, double* acc) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  if (!x || !y || !acc) return fail(ctx, CDCLQ_INVALID_ARG, "null buffer argument");
  if (t == 0 || n == 0) return CDCLQ_OK;
  if (!token_w) return gram_device(ctx, x, y, t, n, acc);
  // weighted tokens: both operands scaled by sqrt(w_t), then the plain accumulation
  HIPCK(hipSetDevice(ctx->device));
  CK(ensure(ctx, ctx->x_in, t * n * 4));
  HIPCK(token_scale(ctx->st, (long)t, (int)n, x, token_w, P<float>(ctx->x_in)));
  const float* ys = P<float>(ctx->x_in);
  if (y != x) {
    CK(ensure(ctx, ctx->y_in, t * n * 4));
    HIPCK(token_scale(ctx->st, (long)t, (int)n, y, token_w, P<float>(ctx->y_in)));
    ys = P<float>(ctx->y_in);
  }
  return gram_device(ctx, P<float>(ctx->x_in), ys, t, n, acc);
}

int cdclq_hessian_finalize_device(cdclq_ctx* ctx, const double* acc, size_t n, uint64_t tokens, float* h) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  if (!acc || !h) return fail(ctx, CDCLQ_INVALID_ARG, "null buffer argument");
  if (tokens == 0) return fail(ctx, CDCLQ_INVALID_ARG, "no calibration token was accumulated");
  HIPCK(hipSetDevice(ctx->device));
  HIPCK(normalize_acc(ctx->st, (long)(n * n), acc, (double)tokens, h));
  HIPCK(hipStreamSynchronize(ctx->st));
  return CDCLQ_OK;
}

int cdclq_upper_chol_of_inverse_device(cdclq_ctx* ctx, const double* h, size_t n, float* u) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  return uchol_device(ctx, h, n, u);
}

int cdclq_upper_chol_of_inverse(cdclq_ctx* ctx, const double* h, size_t n, float* u) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  if (!h || !u) return fail(ctx, CDCLQ_INVALID_ARG, "null buffer argument");
  if (n == 0) return CDCLQ_OK;
  HIPCK(hipSetDevice(ctx->device));
  CK(ensure(ctx, ctx->h64_in, n * n * 8));
  CK(ensure(ctx, ctx->u_out, n * n * 4));
  HIPCK(hipMemcpyAsync(ctx->h64_in.p, h, n * n * 8, hipMemcpyHostToDevice, ctx->st));
  CK(uchol_device(ctx, P<double>(ctx->h64_in), n, P<float>(ctx->u_out)));
  HIPCK(hipMemcpyAsync(u, ctx->u_out.p, n * n * 4, hipMemcpyDeviceToHost, ctx->st));
  HIPCK(hipStreamSynchronize(ctx->st));
  return CDCLQ_OK;
}

int cdclq_proxy_loss(cdclq_ctx* ctx, const float* w_t, const float* w_hat, size_t rows, size_t n, const float* h,
                     double* out) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  if (!w_t || !w_hat || !h || !out) return fail(ctx, CDCLQ_INVALID_ARG, "null buffer argument");
  *out = 0.0;
  if (rows == 0 || n == 0) return CDCLQ_OK;
  HIPCK(hipSetDevice(ctx->device));
  const size_t wn = rows * n;
  CK(ensure(ctx, ctx->w_in, wn * 4));
  CK(ensure(ctx, ctx->t1, wn * 4));
  CK(ensure(ctx, ctx->t2, wn * 4));
  CK(ensure(ctx, ctx->h_in, n * n * 4));
  HIPCK(hipMemcpyAsync(ctx->w_in.p, w_t, wn * 4, hipMemcpyHostToDevice, ctx->st));
  HIPCK(hipMemcpyAsync(ctx->t2.p, w_hat, wn * 4, hipMemcpyHostToDevice, ctx->st));
  HIPCK(hipMemcpyAsync(ctx->h_in.p, h, n * n * 4, hipMemcpyHostToDevice, ctx->st));
  HIPCK(sub_f32(ctx->st, wn, P<float>(ctx->w_in), P<float>(ctx->t2), P<float>(ctx->t1)));  // e
  HIPCK(gemm_chain<float>(ctx->st, (int)rows, (int)n, (int)n, 1.0f, 0, P<float>(ctx->t1), (long)n, 1,
                          P<float>(ctx->h_in), (long)n, 1, P<float>(ctx->t2), (long)n, 1, false, nullptr));
  const int nb = 1024;
  CK(ensure(ctx, ctx->proxy_p, nb * 8));
  HIPCK(proxy_reduce(ctx->st, wn, P<float>(ctx->t1), P<float>(ctx->t2), P<double>(ctx->proxy_p), nb));
  std::vector<double> part(nb);
  HIPCK(hipMemcpyAsync(part.data(), ctx->proxy_p.p, nb * 8, hipMemcpyDeviceToHost, ctx->st));
  HIPCK(hipStreamSynchronize(ctx->st));
  double s = 0.0;
  for (double v : part) s += v;
  *out = s;
  return CDCLQ_OK;
}

int cdclq_device_alloc(cdclq_ctx* ctx, size_t bytes, void** ptr) {
  if (!ctx || !ptr) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  HIPCK(hipSetDevice(ctx->device));
  *ptr = nullptr;
  hipError_t e = hipMalloc(ptr, bytes ? bytes : 256);
  if (e != hipSuccess) {
    *ptr = nullptr;
    (void)hipGetLastError();
    return fail(ctx, CDCLQ_OOM, "device allocation of " + std::to_string(bytes) + " bytes failed");
  }
  return CDCLQ_OK;
}

int cdclq_device_free(cdclq_ctx* ctx, void* ptr) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  if (!ptr) return CDCLQ_OK;
  HIPCK(hipSetDevice(ctx->device));
  HIPCK(hipStreamSynchronize(ctx->st));
  HIPCK(hipFree(ptr));
  return CDCLQ_OK;
}

int cdclq_memcpy_h2d(cdclq_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  HIPCK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->st));
  HIPCK(hipStreamSynchronize(ctx->st));
  return CDCLQ_OK;
}

int cdclq_memcpy_d2h(cdclq_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  HIPCK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->st));
  HIPCK(hipStreamSynchronize(ctx->st));
  return CDCLQ_OK;
}

int cdclq_memset_device(cdclq_ctx* ctx, void* dst, int value, size_t bytes) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  HIPCK(hipMemsetAsync(dst, value, bytes, ctx->st));
  HIPCK(hipStreamSynchronize(ctx->st));
  return CDCLQ_OK;
}

int cdclq_synth_normal_device(cdclq_ctx* ctx, uint64_t seed, uint64_t offset, size_t count, float sigma, float* out) {
  if (!ctx || (!out && count)) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  HIPCK(synth_normal(ctx->st, seed, offset, count, sigma, out));
  HIPCK(hipStreamSynchronize(ctx->st));
  return CDCLQ_OK;
}

int cdclq_synth_outlier_scales(uint64_t seed, size_t n, double frac, float factor, float* scales) {
  if (!scales && n) return CDCLQ_INVALID_ARG;
  size_t k = (size_t)std::round(frac * (double)n);
  if (k > n) k = n;
  std::vector<size_t> idx(n);
  for (size_t j = 0; j < n; ++j) {
    idx[j] = j;
    scales[j] = 1.0f;
  }
  for (size_t i = 0; i < k; ++i) {
    const size_t j = i + (size_t)(mix64(seed + (i + 1) * 0x9E3779B97F4A7C15ULL) % (uint64_t)(n - i));
    std::swap(idx[i], idx[j]);
  }
  for (size_t i = 0; i < k; ++i) scales[idx[i]] = factor;
  return CDCLQ_OK;
}

int cdclq_synth_tokens_heavy_device(cdclq_ctx* ctx, uint64_t seed, uint64_t row0, size_t t, size_t n,
                                    const float* ch_scale, const uint8_t* heavy, float* x) {
  if (!ctx || (!x && t && n)) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  // channel scales (n f32) and the heavy-tail mask (n u8) staged in one buffer
  const size_t off = (n * 4 + 255) & ~(size_t)255;
  CK(ensure(ctx, ctx->cs_d, off + n));
  const float* cs = nullptr;
  const uint8_t* hv = nullptr;
  if (ch_scale) {
    HIPCK(hipMemcpyAsync(ctx->cs_d.p, ch_scale, n * 4, hipMemcpyHostToDevice, ctx->st));
    cs = P<float>(ctx->cs_d);
  }
  if (heavy) {
    HIPCK(hipMemcpyAsync(P<char>(ctx->cs_d) + off, heavy, n, hipMemcpyHostToDevice, ctx->st));
    hv = reinterpret_cast<const uint8_t*>(P<char>(ctx->cs_d) + off);
  }
  HIPCK(synth_tokens(ctx->st, seed, row0, t, n, cs, hv, x));
  HIPCK(hipStreamSynchronize(ctx->st));
  return CDCLQ_OK;
}

int cdclq_synth_tokens_device(cdclq_ctx* ctx, uint64_t seed, uint64_t row0, size_t t, size_t n, const float* ch_scale,
                              float* x) {
  return cdclq_synth_tokens_heavy_device(ctx, seed, row0, t, n, ch_scale, nullptr, x);
}

int cdclq_synth_perturb_device(cdclq_ctx* ctx, uint64_t seed, uint64_t offset, size_t count, float sigma,
                               const float* x, float* out) {
  if (!ctx || ((!x || !out) && count)) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  HIPCK(synth_perturb(ctx->st, seed, offset, count, sigma, x, out));
  HIPCK(hipStreamSynchronize(ctx->st));
  return CDCLQ_OK;
}

int cdclq_synth_lognormal_scales(uint64_t seed, size_t n, float sigma, float* scales) {
  if (!scales && n) return CDCLQ_INVALID_ARG;
  for (size_t j = 0; j < n; ++j) scales[j] = (float)std::exp((double)sigma * (double)synth_normal_at(seed, j));
  return CDCLQ_OK;
}

int cdclq_f64_to_f32_device(cdclq_ctx* ctx, const double* h64, size_t count, float* h32) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  HIPCK(f64_to_f32(ctx->st, count, h64, h32));
  HIPCK(hipStreamSynchronize(ctx->st));
  return CDCLQ_OK;
}

int cdclq_ctx_set_timing(cdclq_ctx* ctx, int enable) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->timing = enable != 0;
  return CDCLQ_OK;
}

int cdclq_ctx_reset_timing(cdclq_ctx* ctx) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  drain_timing(ctx);
  for (int i = 0; i < CDCLQ_PHASE_COUNT; ++i) {
    ctx->ms[i] = 0.0;
    ctx->launches[i] = 0;
  }
  return CDCLQ_OK;
}

int cdclq_ctx_get_timing(cdclq_ctx* ctx, int phase, uint64_t* launches, double* ms) {
  if (!ctx || phase < 0 || phase >= CDCLQ_PHASE_COUNT) return CDCLQ_INVALID_ARG;
  drain_timing(ctx);
  if (launches) *launches = ctx->launches[phase];
  if (ms) *ms = ctx->ms[phase];
  return CDCLQ_OK;
}

}  // extern "C"
