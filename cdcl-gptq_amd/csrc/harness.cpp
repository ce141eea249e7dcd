// The synthetic-layer benchmark of the reference (src/bench.rs, `cdclq bench`) on the GPU engine:
// the same generator stream, the same method variants and the same report, with round-to-nearest,
// quantization and the held-out output error computed on the device. Also the C-ABI entry points
// of the evaluation pieces themselves (engine::rtn_layer, engine::proxy_loss on device memory,
// bench::rel_err).
//
// The generator (splitmix64 + Box-Muller, src/rng.rs:22-57) runs on the host in the reference's
// exact draw order with the platform's f32 logf / sinf / cosf (what Rust's f32::ln / sin / cos
// call); every GEMM (the low-rank activation product, the output-error products) is the bit-exact
// chain GEMM on the device, so W, X and H are bit-identical to the reference's.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "cdclq.h"
#include "ctx.h"
#include "kernels.h"

namespace {

using namespace cdclq;

// rng::Rng (src/rng.rs:22-57)
struct Rng {
  uint64_t s;
  bool has_spare = false;
  float spare = 0.0f;
  explicit Rng(uint64_t seed) : s(seed + 0x9E3779B97F4A7C15ULL) {}
  uint64_t next_u64() {
    s += 0x9E3779B97F4A7C15ULL;
    uint64_t z = s;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
  }
  float uniform() { return ((float)(next_u64() >> 40) + 0.5f) / (float)(1ULL << 24); }
  float normal() {
    if (has_spare) {
      has_spare = false;
      return spare;
    }
    const float u1 = uniform(), u2 = uniform();
    const float r = sqrtf(-2.0f * logf(u1));
    const float th = 6.28318548f * u2;  // 2 * std::f32::consts::PI, exact in f32
    spare = r * sinf(th);
    has_spare = true;
    return r * cosf(th);
  }
};

double now_secs() {
  using namespace std::chrono;
  return duration<double>(steady_clock::now().time_since_epoch()).count();
}

struct Dev {
  void* p = nullptr;
  Dev() = default;
  Dev(const Dev&) = delete;
  Dev& operator=(const Dev&) = delete;
  ~Dev() {
    if (p) (void)hipFree(p);
  }
  hipError_t alloc(size_t bytes) {
    if (p) (void)hipFree(p);
    p = nullptr;
    return hipMalloc(&p, bytes ? bytes : 256);
  }
  template <class T>
  T* as() const {
    return static_cast<T*>(p);
  }
};

// ---- Rust formatting (std::fmt) of the report's numbers
// {:.Ne}: mantissa with N decimals, exponent without sign padding ("6.1946e-3", "1.0000e0")
std::string rust_exp(double v, int prec) {
  if (std::isnan(v)) return "NaN";
  if (std::isinf(v)) return v < 0 ? "-inf" : "inf";
  char buf[64];
  std::snprintf(buf, sizeof buf, "%.*e", prec, v);
  char* e = std::strchr(buf, 'e');
  const int ex = std::atoi(e + 1);
  *e = 0;
  return std::string(buf) + "e" + std::to_string(ex);
}
std::string fixed(double v, const char* fmt) {
  char buf[64];
  std::snprintf(buf, sizeof buf, fmt, v);
  return buf;
}
// Display of an f64 / f32: the shortest digits that read back to the value, no exponent ("0.01", "5")
std::string rust_display(double v, bool is_f32) {
  if (std::isnan(v)) return "NaN";
  if (std::isinf(v)) return v < 0 ? "-inf" : "inf";
  if (v == 0.0) return std::signbit(v) ? "-0" : "0";
  char buf[64];
  int p = 0;
  for (; p < 17; ++p) {
    std::snprintf(buf, sizeof buf, "%.*e", p, v);
    if (is_f32 ? (std::strtof(buf, nullptr) == (float)v) : (std::strtod(buf, nullptr) == v)) break;
  }
  std::string s(buf);
  const bool neg = s[0] == '-';
  if (neg) s = s.substr(1);
  const size_t epos = s.find('e');
  const int ex = std::atoi(s.c_str() + epos + 1);
  std::string digits;
  for (size_t i = 0; i < epos; ++i)
    if (s[i] != '.') digits += s[i];
  std::string out;
  const int point = ex + 1;  // digits before the decimal point
  if (point <= 0) {
    out = "0." + std::string(-point, '0') + digits;
  } else if ((size_t)point >= digits.size()) {
    out = digits + std::string(point - digits.size(), '0');
  } else {
    out = digits.substr(0, point) + "." + digits.substr(point);
  }
  return (neg ? "-" : "") + out;
}

struct Row {
  std::string name;
  double loss, calib, test, secs, bpw;
};

// bench::table (src/bench.rs:129-154)
std::string table(const std::string& title, const std::vector<Row>& rows, size_t base) {
  std::string s = "\n### " + title + "\n\n";
  s += "| method | proxy loss | calib err | held-out err | vs GPTQ (held-out) | bits/weight | time (s) |\n";
  s += "|---|---:|---:|---:|---:|---:|---:|\n";
  for (size_t i = 0; i < rows.size(); ++i) {
    const Row& r = rows[i];
    const std::string vs = (i == base || rows[base].test == 0.0)
                               ? std::string("-")
                               : fixed(100.0 * (r.test / rows[base].test - 1.0), "%+.1f") + "%";
    s += "| " + r.name + " | " + (r.loss > 0.0 ? rust_exp(r.loss, 4) : std::string("-")) + " | " +
         rust_exp(r.calib, 4) + " | " + rust_exp(r.test, 4) + " | " + vs + " | " + fixed(r.bpw, "%.3f") + " | " +
         fixed(r.secs, "%.2f") + " |\n";
  }
  return s;
}

int fail_msg(cdclq_ctx* ctx, int code, const std::string& m) { return fail(ctx, code, m); }

// ActGen (src/bench.rs:41-80) with the low-rank product and the per-element step on the device.
struct ActGen {
  size_t n, rank;
  Dev a;  // rank x n
  std::vector<float> scale;
  Dev scale_d;
};

int actgen_new(cdclq_ctx* ctx, Rng& rng, size_t n, ActGen& g) {
  g.n = n;
  g.rank = std::max<size_t>(n / 8, 8);
  std::vector<float> a(g.rank * n);
  const float rs = sqrtf((float)g.rank);
  for (auto& v : a) v = rng.normal() / rs;
  g.scale.resize(n);
  for (auto& v : g.scale) v = expf(0.6f * rng.normal());
  for (auto& v : g.scale)
    if (rng.uniform() < 0.005f) v *= 20.0f + 40.0f * rng.uniform();
  HIPCK(g.a.alloc(a.size() * 4));
  HIPCK(hipMemcpy(g.a.p, a.data(), a.size() * 4, hipMemcpyHostToDevice));
  HIPCK(g.scale_d.alloc(n * 4));
  HIPCK(hipMemcpy(g.scale_d.p, g.scale.data(), n * 4, hipMemcpyHostToDevice));
  return CDCLQ_OK;
}

// ActGen::sample (src/bench.rs:66-79): x (device, tokens x n)
int actgen_sample(cdclq_ctx* ctx, ActGen& g, Rng& rng, size_t tokens, float* x) {
  const size_t n = g.n, rank = g.rank;
  std::vector<float> z(tokens * rank);
  for (auto& v : z) v = rng.normal();
  std::vector<float> noise(tokens * n), massive(tokens);
  for (size_t t = 0; t < tokens; ++t) {
    massive[t] = rng.uniform() < 0.02f ? 4.0f : 1.0f;
    float* row = noise.data() + t * n;
    for (size_t j = 0; j < n; ++j) row[j] = 0.3f * rng.normal();
  }
  Dev zd, nd, md;
  HIPCK(zd.alloc(z.size() * 4));
  HIPCK(nd.alloc(noise.size() * 4));
  HIPCK(md.alloc(tokens * 4));
  HIPCK(hipMemcpy(zd.p, z.data(), z.size() * 4, hipMemcpyHostToDevice));
  HIPCK(hipMemcpy(nd.p, noise.data(), noise.size() * 4, hipMemcpyHostToDevice));
  HIPCK(hipMemcpy(md.p, massive.data(), tokens * 4, hipMemcpyHostToDevice));
  HIPCK(gemm_chain<float>(ctx->st, (int)tokens, (int)n, (int)rank, 1.0f, 0, zd.as<float>(), (long)rank, 1,
                          g.a.as<float>(), (long)n, 1, x, (long)n, 1, false, nullptr));
  HIPCK(act_scale(ctx->st, (long)tokens, (int)n, nd.as<float>(), g.scale_d.as<float>(), md.as<float>(), x));
  HIPCK(hipStreamSynchronize(ctx->st));
  return CDCLQ_OK;
}

int rel_err_device(cdclq_ctx* ctx, const float* w, const float* wq, const float* x, const float* xt, size_t rows,
                   size_t n, size_t t, double* out) {
  Dev o1, o2, part;
  const int nb = 1024;
  HIPCK(o1.alloc(rows * t * 4));
  HIPCK(o2.alloc(rows * t * 4));
  HIPCK(part.alloc(2 * nb * 8));
  // o = W x^T (rows x t): B[k][j] = x[j][k]
  HIPCK(gemm_chain<float>(ctx->st, (int)rows, (int)t, (int)n, 1.0f, 0, w, (long)n, 1, x, 1, (long)n, o1.as<float>(),
                          (long)t, 1, false, nullptr));
  HIPCK(gemm_chain<float>(ctx->st, (int)rows, (int)t, (int)n, 1.0f, 0, wq, (long)n, 1, xt, 1, (long)n, o2.as<float>(),
                          (long)t, 1, false, nullptr));
  HIPCK(err_reduce(ctx->st, rows * t, o1.as<float>(), o2.as<float>(), part.as<double>(), nb));
  std::vector<double> h(2 * nb);
  HIPCK(hipMemcpyAsync(h.data(), part.p, h.size() * 8, hipMemcpyDeviceToHost, ctx->st));
  HIPCK(hipStreamSynchronize(ctx->st));
  double num = 0.0, den = 0.0;
  for (int b = 0; b < nb; ++b) {
    num += h[2 * b];
    den += h[2 * b + 1];
  }
  *out = num / den;
  return CDCLQ_OK;
}

size_t eff_group(const cdclq_config& c, size_t n) { return (c.group == 0 || c.group >= n) ? n : (size_t)c.group; }

int check_bench_args(cdclq_ctx* ctx, const cdclq_bench_args* a) {
  if (!a) return fail_msg(ctx, CDCLQ_INVALID_ARG, "args is null");
  if (a->rows == 0 || a->cols == 0 || a->tokens == 0 || a->test_tokens == 0)
    return fail_msg(ctx, CDCLQ_INVALID_ARG, "rows, cols, tokens and test_tokens must be > 0");
  if (a->cols > 65536 || a->rows * a->cols > ((size_t)1 << 31) - 1 || a->tokens * a->cols > ((size_t)1 << 34))
    return fail_msg(ctx, CDCLQ_INVALID_ARG, "benchmark layer too large for this build");
  return CDCLQ_OK;
}

}  // namespace

extern "C" {

int cdclq_rtn_layer_device(cdclq_ctx* ctx, const float* w, size_t d_out, size_t n, const cdclq_config* cfg,
                           float* out) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  if (!cfg) return fail(ctx, CDCLQ_INVALID_ARG, "cfg is null");
  if (cfg->bits > 31) return fail(ctx, CDCLQ_INVALID_ARG, "bits must be < 32");
  if (d_out == 0 || n == 0) return CDCLQ_OK;
  if (!w || !out) return fail(ctx, CDCLQ_INVALID_ARG, "null buffer argument");
  HIPCK(hipSetDevice(ctx->device));
  HIPCK(rtn_rows(ctx->st, (long)d_out, (int)n, (int)eff_group(*cfg, n), (int)cfg->bits, cfg->mse_grid, w, out));
  HIPCK(hipStreamSynchronize(ctx->st));
  return CDCLQ_OK;
}

int cdclq_rtn_layer(cdclq_ctx* ctx, const float* w, size_t d_out, size_t n, const cdclq_config* cfg, float* out) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  if (!cfg) return fail(ctx, CDCLQ_INVALID_ARG, "cfg is null");
  if (d_out == 0 || n == 0) return CDCLQ_OK;
  if (!w || !out) return fail(ctx, CDCLQ_INVALID_ARG, "null buffer argument");
  HIPCK(hipSetDevice(ctx->device));
  Dev wd, od;
  HIPCK(wd.alloc(d_out * n * 4));
  HIPCK(od.alloc(d_out * n * 4));
  HIPCK(hipMemcpy(wd.p, w, d_out * n * 4, hipMemcpyHostToDevice));
  CK(cdclq_rtn_layer_device(ctx, wd.as<float>(), d_out, n, cfg, od.as<float>()));
  HIPCK(hipMemcpy(out, od.p, d_out * n * 4, hipMemcpyDeviceToHost));
  return CDCLQ_OK;
}

int cdclq_rel_err_device(cdclq_ctx* ctx, const float* w, const float* w_hat, const float* x, const float* x_t,
                         size_t rows, size_t n, size_t t, double* out) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  if (!w || !w_hat || !x || !x_t || !out) return fail(ctx, CDCLQ_INVALID_ARG, "null buffer argument");
  if (rows == 0 || n == 0 || t == 0) return fail(ctx, CDCLQ_INVALID_ARG, "rows, n and t must be > 0");
  HIPCK(hipSetDevice(ctx->device));
  return rel_err_device(ctx, w, w_hat, x, x_t, rows, n, t, out);
}

int cdclq_rel_err(cdclq_ctx* ctx, const float* w, const float* w_hat, const float* x, const float* x_t, size_t rows,
                  size_t n, size_t t, double* out) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  if (!w || !w_hat || !x || !x_t || !out) return fail(ctx, CDCLQ_INVALID_ARG, "null buffer argument");
  if (rows == 0 || n == 0 || t == 0) return fail(ctx, CDCLQ_INVALID_ARG, "rows, n and t must be > 0");
  HIPCK(hipSetDevice(ctx->device));
  Dev a, b, c, d;
  HIPCK(a.alloc(rows * n * 4));
  HIPCK(b.alloc(rows * n * 4));
  HIPCK(c.alloc(t * n * 4));
  HIPCK(hipMemcpy(a.p, w, rows * n * 4, hipMemcpyHostToDevice));
  HIPCK(hipMemcpy(b.p, w_hat, rows * n * 4, hipMemcpyHostToDevice));
  HIPCK(hipMemcpy(c.p, x, t * n * 4, hipMemcpyHostToDevice));
  const float* xt = c.as<float>();
  if (x_t != x) {
    HIPCK(d.alloc(t * n * 4));
    HIPCK(hipMemcpy(d.p, x_t, t * n * 4, hipMemcpyHostToDevice));
    xt = d.as<float>();
  }
  return rel_err_device(ctx, a.as<float>(), b.as<float>(), c.as<float>(), xt, rows, n, t, out);
}

int cdclq_proxy_loss_device(cdclq_ctx* ctx, const float* w_t, const float* w_hat, size_t rows, size_t n,
                            const float* h, double* out) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  if (!w_t || !w_hat || !h || !out) return fail(ctx, CDCLQ_INVALID_ARG, "null buffer argument");
  *out = 0.0;
  if (rows == 0 || n == 0) return CDCLQ_OK;
  HIPCK(hipSetDevice(ctx->device));
  const size_t wn = rows * n;
  Dev e, eh, part;
  const int nb = 1024;
  HIPCK(e.alloc(wn * 4));
  HIPCK(eh.alloc(wn * 4));
  HIPCK(part.alloc(nb * 8));
  HIPCK(sub_f32(ctx->st, wn, w_t, w_hat, e.as<float>()));
  HIPCK(gemm_chain<float>(ctx->st, (int)rows, (int)n, (int)n, 1.0f, 0, e.as<float>(), (long)n, 1, h, (long)n, 1,
                          eh.as<float>(), (long)n, 1, false, nullptr));
  HIPCK(proxy_reduce(ctx->st, wn, e.as<float>(), eh.as<float>(), part.as<double>(), nb));
  std::vector<double> p(nb);
  HIPCK(hipMemcpyAsync(p.data(), part.p, nb * 8, hipMemcpyDeviceToHost, ctx->st));
  HIPCK(hipStreamSynchronize(ctx->st));
  double s = 0.0;
  for (double v : p) s += v;
  *out = s;
  return CDCLQ_OK;
}

int cdclq_bench_run(cdclq_ctx* ctx, const cdclq_bench_args* a, cdclq_bench_row* rows_out, size_t max_rows,
                    size_t* nrows, char* report, size_t report_cap, size_t* report_len) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  CK(check_bench_args(ctx, a));
  HIPCK(hipSetDevice(ctx->device));
  const size_t rows = a->rows, n = a->cols, T = a->tokens, TT = a->test_tokens;
  const size_t nthreads = a->nthreads ? a->nthreads : 1;
  Rng rng(a->seed);
  ActGen gen;
  CK(actgen_new(ctx, rng, n, gen));
  // gen_weights (src/bench.rs:82-97)
  std::vector<float> w(rows * n);
  for (size_t r = 0; r < rows; ++r) {
    const float sigma = 0.02f * expf(0.3f * rng.normal());
    for (size_t j = 0; j < n; ++j) {
      float v = rng.normal() * sigma;
      if (rng.uniform() < 0.001f) v *= 8.0f;
      w[r * n + j] = v;
    }
  }
  Dev wd, xd, xte, h64, h32, wq, codes, scales, zeros, permd;
  HIPCK(wd.alloc(rows * n * 4));
  HIPCK(hipMemcpy(wd.p, w.data(), rows * n * 4, hipMemcpyHostToDevice));
  HIPCK(xd.alloc(T * n * 4));
  HIPCK(xte.alloc(TT * n * 4));
  CK(actgen_sample(ctx, gen, rng, T, xd.as<float>()));
  CK(actgen_sample(ctx, gen, rng, TT, xte.as<float>()));
  HIPCK(h64.alloc(n * n * 8));
  HIPCK(h32.alloc(n * n * 4));
  HIPCK(hipMemsetAsync(h64.p, 0, n * n * 8, ctx->st));
  CK(cdclq_gram_accumulate_device(ctx, xd.as<float>(), xd.as<float>(), T, n, h64.as<double>()));
  CK(cdclq_f64_to_f32_device(ctx, h64.as<double>(), n * n, h32.as<float>()));
  const size_t ncal = std::min<size_t>(T, 4096);

  const size_t ngmax = n;  // group >= 1
  HIPCK(wq.alloc(rows * n * 4));
  HIPCK(codes.alloc(rows * n));
  HIPCK(scales.alloc(rows * ngmax * 4));
  HIPCK(zeros.alloc(rows * ngmax * 4));
  HIPCK(permd.alloc(n * 4));

  std::string rep;
  {
    char buf[512];
    std::snprintf(buf, sizeof buf,
                  "## Synthetic layer %zux%zu, %zu calibration tokens, %zu held-out tokens, %zu threads\n\nbits=%u "
                  "group=%llu damp=%s act_order=%s mse_grid=%s sub_block=%llu cd_sweeps=%llu\n",
                  rows, n, T, TT, nthreads, a->cfg.bits, (unsigned long long)a->cfg.group,
                  rust_display(a->cfg.damp, false).c_str(), a->cfg.act_order ? "true" : "false",
                  a->cfg.mse_grid ? "true" : "false", (unsigned long long)a->cfg.sub_block,
                  (unsigned long long)a->cfg.cd_sweeps);
    rep += buf;
  }

  // evaluation on (calibration, held-out) tokens with the given inputs of the quantized layer
  auto eval = [&](const float* wqd, const float* xc, const float* xtc, const float* xh, const float* xth, double* c,
                  double* t) -> int {
    CK(rel_err_device(ctx, wd.as<float>(), wqd, xc, xtc, rows, n, ncal, c));
    CK(rel_err_device(ctx, wd.as<float>(), wqd, xh, xth, rows, n, TT, t));
    return CDCLQ_OK;
  };
  auto run_one = [&](const std::string& name, const cdclq_config& cfg, const float* hh, const float* m,
                     const float* xc, const float* xtc, const float* xh, const float* xth, Row* out) -> int {
    CK(cdclq_ctx_clear_cache(ctx));  // every run starts from an empty PrepCache (src/bench.rs:199)
    const size_t ng = cdclq_num_groups(&cfg, n);
    std::vector<uint32_t> perm(n);
    std::vector<uint8_t> gbits(ng);
    cdclq_layer_stats st;
    const double t0 = now_secs();
    CK(cdclq_quantize_layer_device(ctx, wd.as<float>(), rows, n, hh, m, "bench", &cfg, nthreads, codes.as<uint8_t>(),
                                   scales.as<float>(), zeros.as<float>(), perm.data(), gbits.data(), &st));
    const double secs = now_secs() - t0;
    HIPCK(hipMemcpy(permd.p, perm.data(), n * 4, hipMemcpyHostToDevice));
    CK(cdclq_dequantize_layer_device(ctx, rows, n, eff_group(cfg, n), ng, codes.as<uint8_t>(), scales.as<float>(),
                                     zeros.as<float>(), permd.as<uint32_t>(), CDCLQ_DTYPE_F32, wq.as<float>()));
    double c, t;
    CK(eval(wq.as<float>(), xc, xtc, xh, xth, &c, &t));
    *out = Row{name, st.loss_final, c, t, secs, st.bits_total};
    return CDCLQ_OK;
  };
  const float* X = xd.as<float>();
  const float* XTE = xte.as<float>();
  const float* H = h32.as<float>();

  cdclq_config base = a->cfg;
  base.skeleton_pct = 0.0;
  cdclq_config gptq = base;
  gptq.method = CDCLQ_METHOD_GPTQ;
  cdclq_config rtn_cfg = base;
  rtn_cfg.act_order = 0;
  std::vector<Row> out;
  {
    const double t0 = now_secs();
    CK(cdclq_rtn_layer_device(ctx, wd.as<float>(), rows, n, &rtn_cfg, wq.as<float>()));
    const double secs = now_secs() - t0;
    double c, t;
    CK(eval(wq.as<float>(), X, X, XTE, XTE, &c, &t));
    const double g = (double)eff_group(rtn_cfg, n);
    out.push_back(Row{"RTN (no compensation)", 0.0, c, t, secs, (double)rtn_cfg.bits + 24.0 / g});
  }
  Row r;
  CK(run_one("GPTQ", gptq, H, nullptr, X, X, XTE, XTE, &r));
  out.push_back(r);
  struct Variant {
    const char* name;
    double frac;
    uint64_t sweeps, passes;
    int refit;
  };
  const Variant variants[4] = {{"ablation: scale refit only (3 passes)", 0.0, 1, 3, 1},
                               {"ablation: coordinate descent only (4 passes)", 1.0, 1, 4, 0},
                               {"CDCL-GPTQ fast (50% sub-blocks, 2 passes)", 0.5, 1, 2, 1},
                               {"CDCL-GPTQ balanced (all sub-blocks, 4 passes)", 1.0, 1, 4, 1}};
  for (const Variant& v : variants) {
    cdclq_config c = base;
    c.method = CDCLQ_METHOD_CDCL;
    c.refine_frac = v.frac;
    c.cd_sweeps = v.sweeps;
    c.passes = v.passes;
    c.refit_scales = v.refit;
    c.tol = 0.0;
    CK(run_one(v.name, c, H, nullptr, X, X, XTE, XTE, &r));
    out.push_back(r);
  }
  {
    cdclq_config c = base;
    c.method = CDCLQ_METHOD_CDCL;
    const std::string name = "CDCL-GPTQ default (up to " + std::to_string(c.passes) + " passes, tol " +
                             rust_display(c.tol, false) + ")";
    CK(run_one(name, c, H, nullptr, X, X, XTE, XTE, &r));
    out.push_back(r);
  }
  rep += table("Equal-bits comparison (same grid, ordering, damping)", out, 1);
  std::vector<Row> all = out;

  if (a->cfg.skeleton_pct > 0.0) {  // src/bench.rs:243-263
    cdclq_config g2 = gptq, c2 = base;
    g2.skeleton_pct = a->cfg.skeleton_pct;
    c2.skeleton_pct = a->cfg.skeleton_pct;
    c2.method = CDCLQ_METHOD_CDCL;
    std::vector<Row> sk;
    sk.push_back(Row{out[1].name + " (no skeleton, for reference)", out[1].loss, out[1].calib, out[1].test,
                     out[1].secs, out[1].bpw});
    CK(run_one("GPTQ + skeleton", g2, H, nullptr, X, X, XTE, XTE, &r));
    sk.push_back(r);
    CK(run_one("CDCL-GPTQ + skeleton", c2, H, nullptr, X, X, XTE, XTE, &r));
    sk.push_back(r);
    rep += table("Protected skeleton (" + rust_display(a->cfg.skeleton_pct, false) + "% of input columns at " +
                     std::to_string(a->cfg.skeleton_bits) + " bits) - note the higher bits/weight",
                 sk, 1);
    all.insert(all.end(), sk.begin() + 1, sk.end());
  }

  if (a->asym_noise > 0.0f) {  // src/bench.rs:265-311
    Dev rms, nd, xt, xte_t, ht64, m64, ht, mm;
    HIPCK(rms.alloc(n * 4));
    HIPCK(channel_rms(ctx->st, (long)T, (int)n, X, rms.as<float>()));
    HIPCK(xt.alloc(T * n * 4));
    HIPCK(xte_t.alloc(TT * n * 4));
    {
      std::vector<float> nrm(T * n);
      for (auto& v : nrm) v = rng.normal();
      HIPCK(nd.alloc(nrm.size() * 4));
      HIPCK(hipMemcpy(nd.p, nrm.data(), nrm.size() * 4, hipMemcpyHostToDevice));
      HIPCK(add_noise(ctx->st, (long)T, (int)n, a->asym_noise, rms.as<float>(), nd.as<float>(), X, xt.as<float>()));
      HIPCK(hipStreamSynchronize(ctx->st));
      std::vector<float> nrm2(TT * n);
      for (auto& v : nrm2) v = rng.normal();
      HIPCK(hipMemcpy(nd.p, nrm2.data(), nrm2.size() * 4, hipMemcpyHostToDevice));
      HIPCK(add_noise(ctx->st, (long)TT, (int)n, a->asym_noise, rms.as<float>(), nd.as<float>(), XTE,
                      xte_t.as<float>()));
      HIPCK(hipStreamSynchronize(ctx->st));
    }
    HIPCK(ht64.alloc(n * n * 8));
    HIPCK(m64.alloc(n * n * 8));
    HIPCK(ht.alloc(n * n * 4));
    HIPCK(mm.alloc(n * n * 4));
    HIPCK(hipMemsetAsync(ht64.p, 0, n * n * 8, ctx->st));
    HIPCK(hipMemsetAsync(m64.p, 0, n * n * 8, ctx->st));
    CK(cdclq_gram_accumulate_device(ctx, xt.as<float>(), xt.as<float>(), T, n, ht64.as<double>()));
    CK(cdclq_gram_accumulate_device(ctx, X, xt.as<float>(), T, n, m64.as<double>()));
    CK(cdclq_f64_to_f32_device(ctx, ht64.as<double>(), n * n, ht.as<float>()));
    CK(cdclq_f64_to_f32_device(ctx, m64.as<double>(), n * n, mm.as<float>()));
    const float* XT = xt.as<float>();
    const float* XTET = xte_t.as<float>();
    std::vector<Row> ar;
    double c, t;
    CK(eval(wd.as<float>(), X, XT, XTE, XTET, &c, &t));
    ar.push_back(Row{"FP weights on noisy inputs (floor)", 0.0, c, t, 0.0, 16.0});
    CK(run_one("GPTQ, symmetric target (H~ only)", gptq, ht.as<float>(), nullptr, X, XT, XTE, XTET, &r));
    ar.push_back(r);
    CK(run_one("GPTQ, asymmetric target (W* = W M H~^-1)", gptq, ht.as<float>(), mm.as<float>(), X, XT, XTE, XTET,
               &r));
    ar.push_back(r);
    cdclq_config c3 = base;
    c3.method = CDCLQ_METHOD_CDCL;
    CK(run_one("CDCL-GPTQ, asymmetric target", c3, ht.as<float>(), mm.as<float>(), X, XT, XTE, XTET, &r));
    ar.push_back(r);
    rep += table("Quantized-input calibration (relative input noise " + rust_display(a->asym_noise, true) +
                     "): error is ||W x - W_hat x~||",
                 ar, 1);
    all.insert(all.end(), ar.begin(), ar.end());
  }

  if (nrows) *nrows = all.size();
  if (rows_out) {
    for (size_t i = 0; i < all.size() && i < max_rows; ++i) {
      cdclq_bench_row& o = rows_out[i];
      std::memset(o.name, 0, sizeof o.name);
      std::strncpy(o.name, all[i].name.c_str(), sizeof o.name - 1);
      o.loss = all[i].loss;
      o.calib = all[i].calib;
      o.test = all[i].test;
      o.secs = all[i].secs;
      o.bpw = all[i].bpw;
    }
  }
  if (report_len) *report_len = rep.size();
  if (report && report_cap) {
    const size_t k = std::min(report_cap - 1, rep.size());
    std::memcpy(report, rep.data(), k);
    report[k] = 0;
  }
  return CDCLQ_OK;
}

}  // extern "C"
