/*
 * cdclq.h -- C ABI of the MI355X-native (gfx950) CDCL-GPTQ per-layer quantization engine.
 *
 * Drop-in boundary for the reference Rust crate `cdclq` 1.0.1 (tailot/CDCL-GPTQ): each entry
 * point below names the reference function it replaces (path:line in that crate). Plain
 * pointers and sizes only; no GPU runtime types appear in any signature.
 *
 * Conventions
 *  - Matrices are row-major. `*_device` entry points take pointers to device (HBM) memory of the
 *    context's GPU; the others take host memory and stage it through the device themselves.
 *  - Every call is synchronous (returns after the device work finished), like the reference.
 *  - Status codes: CDCLQ_OK on success; on failure cdclq_last_error(ctx) holds the message. For
 *    conditions the reference reports with anyhow::bail! the text is the reference's text.
 *  - A context is thread-compatible, not thread-safe: one context per host thread and GPU.
 *    It owns the device workspace and the one-entry factor cache (PrepCache).
 *  - No call aborts the process.
 */
#ifndef CDCLQ_H
#define CDCLQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CDCLQ_ABI_VERSION 1

typedef enum cdclq_status {
  CDCLQ_OK = 0,
  CDCLQ_INVALID_ARG = 1, /* src/engine.rs:240-258 validate(), shape/size errors */
  CDCLQ_NOT_PD = 2,      /* src/linalg.rs:215-219 non-positive / non-finite pivot */
  CDCLQ_NON_FINITE = 3,  /* reserved: non-finite input scan (src/io.rs:205-212) */
  CDCLQ_DEVICE = 4,      /* HIP runtime error */
  CDCLQ_OOM = 5          /* device allocation failed */
} cdclq_status;

/* engine::Method (src/engine.rs:83-88) */
typedef enum cdclq_method { CDCLQ_METHOD_GPTQ = 0, CDCLQ_METHOD_CDCL = 1 } cdclq_method;

/* engine::Config (src/engine.rs:94-144); defaults via cdclq_default_config
 * (src/engine.rs:146-167). Booleans are 0/1. */
typedef struct cdclq_config {
  uint32_t bits;          /* 2..=8 */
  uint32_t skeleton_bits; /* 2..=8 */
  uint64_t group;         /* 0 = one group per row */
  uint64_t block;
  uint64_t sub_block;
  uint64_t cd_sweeps;
  uint64_t passes;
  uint64_t row_chunk; /* 0 = automatic from nthreads (src/engine.rs:768-770) */
  double damp;
  double skeleton_pct;
  double refine_frac;
  double tol;
  int32_t act_order;
  int32_t mse_grid;
  int32_t method; /* cdclq_method */
  int32_t refit_scales;
} cdclq_config;

/* engine::LayerStats (src/engine.rs:174-199) */
typedef struct cdclq_layer_stats {
  double loss_gptq;
  double loss_final;
  uint64_t subblocks_total;
  uint64_t subblocks_refined;
  uint64_t code_updates;
  uint64_t skeleton_groups;
  double bits_codes;
  double bits_total;
  double secs_prepare;
  double secs_quant;
} cdclq_layer_stats;

typedef struct cdclq_ctx cdclq_ctx;

int cdclq_abi_version(void);
size_t cdclq_sizeof_config(void);
size_t cdclq_sizeof_stats(void);

/* Config::default() (src/engine.rs:146-167) */
void cdclq_default_config(cdclq_config* cfg);

/* Number of groups for a layer of width d_in: ceil(d_in / effective_group)
 * (src/engine.rs:227-233, :705). */
size_t cdclq_num_groups(const cdclq_config* cfg, size_t d_in);

/* Context on GPU `device`: owns a HIP stream, the device workspace and the PrepCache
 * (src/engine.rs:220-223, created as `None` by every reference caller). */
int cdclq_ctx_create(int device, cdclq_ctx** out);
void cdclq_ctx_destroy(cdclq_ctx* ctx);
/* Message of the last failed call on ctx ("" if none). Valid until the next call on ctx. */
const char* cdclq_last_error(const cdclq_ctx* ctx);
/* Drops the cached factorisation (`*cache = None`, src/engine.rs:720). */
int cdclq_ctx_clear_cache(cdclq_ctx* ctx);

/*
 * engine::quantize_layer (src/engine.rs:690-799).
 *   w      d_out x d_in f32, original column order
 *   h      d_in x d_in f32 calibration Hessian
 *   m      optional d_in x d_in cross-covariance (NULL = symmetric target)
 *   hkey   Hessian identity for the factor cache (src/engine.rs:718)
 *   nthreads  stands in for rayon::current_num_threads() when cfg->row_chunk == 0
 * Outputs (caller-allocated): codes[d_out*d_in] u8 in permuted column order, scales[d_out*ng],
 * zeros[d_out*ng] (f32, f16-exact / integer-valued), perm[d_in] (perm[j] = original column at
 * permuted position j), gbits[ng], stats (may be NULL). ng = cdclq_num_groups(cfg, d_in).
 */
int cdclq_quantize_layer(cdclq_ctx* ctx, const float* w, size_t d_out, size_t d_in, const float* h, const float* m,
                         const char* hkey, const cdclq_config* cfg, size_t nthreads, uint8_t* codes, float* scales,
                         float* zeros, uint32_t* perm, uint8_t* gbits, cdclq_layer_stats* stats);
/* Same contract; w, h, m, codes, scales, zeros are device pointers; perm, gbits, stats host. */
int cdclq_quantize_layer_device(cdclq_ctx* ctx, const float* w, size_t d_out, size_t d_in, const float* h,
                                const float* m, const char* hkey, const cdclq_config* cfg, size_t nthreads,
                                uint8_t* codes, float* scales, float* zeros, uint32_t* perm, uint8_t* gbits,
                                cdclq_layer_stats* stats);

/* The factor cache fill that cdclq_quantize_layer[_device] performs first (src/engine.rs:708-723,
 * build_prepared :320-342), on its own: the column order for (w, h, cfg) and, unless ctx's cache
 * already holds it, U and the damped permuted H for (hkey, that order). A following
 * cdclq_quantize_layer[_device] on ctx with the same hkey, h and cfg (and, with the skeleton, the
 * same w) reuses the entry, exactly as a second reference call through the same PrepCache does.
 * No reference counterpart: it lets a caller run the factorisations of several contexts ahead of
 * their other work. w, h: device pointers. Synchronous. */
int cdclq_prepare_layer_device(cdclq_ctx* ctx, const float* w, size_t d_out, size_t d_in, const float* h,
                               const char* hkey, const cdclq_config* cfg);

/* Near-midpoint accounting of the last cdclq_quantize_layer[_device] call on ctx (no reference
 * counterpart: the parity contract's record of rounding decisions an implementation with another
 * operation order could legitimately resolve differently). A decision clamp(round(a / b) + z, 0,
 * maxq) is near a midpoint when a / b evaluated in f64 from the same f32 operands lies within 1e-9
 * of k + 1/2 and the two candidates differ after clamping. Counted: the phase-1 codes
 * (src/quant.rs:92-95, d_out x d_in decisions), the group zero points of the chosen grid
 * (src/quant.rs:59, d_out x ngroups), and the coordinate-descent evaluations in the reference's
 * visit order (src/engine.rs:626-636). */
typedef struct cdclq_midpoint_counts {
  uint64_t code_decisions;
  uint64_t code_near;
  uint64_t zero_decisions;
  uint64_t zero_near;
  uint64_t cd_decisions;
  uint64_t cd_near;
} cdclq_midpoint_counts;
int cdclq_ctx_last_midpoint_counts(const cdclq_ctx* ctx, cdclq_midpoint_counts* out);

/* linalg::gram_accumulate (src/linalg.rs:388-418): h (n x n, f64) += x^T y, x and y token-major
 * t x n f32. y == x selects the symmetric Hessian path. */
int cdclq_gram_accumulate(cdclq_ctx* ctx, const float* x, const float* y, size_t t, size_t n, double* h);
int cdclq_gram_accumulate_device(cdclq_ctx* ctx, const float* x, const float* y, size_t t, size_t n, double* h);
/* Allocation-free variant of cdclq_gram_accumulate_device, with no counterpart in the reference:
 * for callers that cannot allocate device memory (calibration hooks in a tight forward loop,
 * harnesses that forbid hipMalloc). Same arguments, same result bit for bit. It calls no hipMalloc
 * / hipFree: its status words and tile list live in a fixed array of about 2 MiB per GPU, held
 * until the process ends. Like the other entry points it is synchronous: it reads the symmetry
 * check's flag back to the host to choose the tile list, copies that list from host memory and
 * waits for its stream, so it cannot be recorded into a HIP graph. Limit: n <= 32768 (larger n
 * returns CDCLQ_INVALID_ARG before any device work). Every call on a GPU shares that GPU's array,
 * so calls that overlap on one GPU (several contexts or threads at once) race; calls in sequence
 * do not. */
int cdclq_gram_accumulate_device_noalloc(cdclq_ctx* ctx, const float* x, const float* y, size_t t, size_t n,
                                        double* h);
/* `count` independent accumulations in one launch (device pointers): hs[i] += xs[i]^T ys[i] with
 * ts[i] tokens of width ns[i]. Each result equals a separate gram_accumulate call; batching only
 * lets the inputs of one decoder layer (q/k/v, o, gate/up, down) share the GPU. The reference's
 * capture script accumulates all of a layer's Hessians in the same forward pass
 * (scripts/capture_hessians.py:233-245). */
int cdclq_gram_accumulate_batch_device(cdclq_ctx* ctx, int count, const float* const* xs, const float* const* ys,
                                       const size_t* ts, const size_t* ns, double* const* hs);

/* Calibration capture (scripts/capture_hessians.py:233-245, :266), device memory: acc (n x n f64)
 * += sum_t w_t x_t y_t^T over t tokens (token-major t x n f32). The token weight is applied as the
 * reference does, x_t * sqrt(w_t) in f32 on both operands; token_w NULL = all 1. y == x gives the
 * Hessian; y = the quantized model's layer input gives the cross-covariance M of the asymmetric
 * target (src/engine.rs:690-699), which the reference's capture does not produce. Each call's
 * tokens are summed exactly as cdclq_gram_accumulate (f32 chains over 2048-token chunks, f64 sums). */
int cdclq_hessian_accumulate_device(cdclq_ctx* ctx, const float* x, const float* y, const float* token_w, size_t t,
                                    size_t n, double* acc);
/* The 1/N normalisation (scripts/capture_hessians.py:266): h = (f32)(acc / tokens), rounded once. */
int cdclq_hessian_finalize_device(cdclq_ctx* ctx, const double* acc, size_t n, uint64_t tokens, float* h);

/* linalg::upper_chol_of_inverse (src/linalg.rs:362-375): u (n x n f32, upper) with
 * h^-1 = u^T u. h is not modified. */
int cdclq_upper_chol_of_inverse(cdclq_ctx* ctx, const double* h, size_t n, float* u);
int cdclq_upper_chol_of_inverse_device(cdclq_ctx* ctx, const double* h, size_t n, float* u);

/* linalg::sgemm / dgemm (src/linalg.rs:56-99) and pgemm_f32 / pgemm_f64 (:101-184), device memory:
 * C = alpha A B + beta C for A m x k, B k x n, C m x n with arbitrary element strides (rs* = row
 * stride, cs* = column stride, in elements). The result is matrixmultiply 0.3.8's: per element a
 * fused multiply-add chain over each 256-wide panel of k, started from 0 and folded in panel order,
 * C = fma(alpha, chain, C'), with C' = beta C before the first panel (C unread when beta == 0);
 * k == 0 gives C = beta C (0 when beta == 0). C must not alias A or B. */
int cdclq_sgemm_device(cdclq_ctx* ctx, size_t m, size_t k, size_t n, float alpha, const float* a, ptrdiff_t rsa,
                       ptrdiff_t csa, const float* b, ptrdiff_t rsb, ptrdiff_t csb, float beta, float* c, ptrdiff_t rsc,
                       ptrdiff_t csc);
int cdclq_dgemm_device(cdclq_ctx* ctx, size_t m, size_t k, size_t n, double alpha, const double* a, ptrdiff_t rsa,
                       ptrdiff_t csa, const double* b, ptrdiff_t rsb, ptrdiff_t csb, double beta, double* c,
                       ptrdiff_t rsc, ptrdiff_t csc);

/* engine::proxy_loss (src/engine.rs:808-815): sum_rows e H e^T with e = w_t - w_hat. */
int cdclq_proxy_loss(cdclq_ctx* ctx, const float* w_t, const float* w_hat, size_t rows, size_t n, const float* h,
                     double* out);

/* ---- Packed container "cdclq-v1" (src/io.rs:227-293, src/quant.rs:98-236) ----
 * A packed layer is six tensors: .qweight u8 [d_out, row_bytes] (each row the codes of that row in
 * permuted column order, appended low bit first with the width of their group, last byte
 * zero-filled), .scales f16 [d_out, ngroups], .qzeros u8 [d_out, ngroups], .perm i32 [d_in],
 * .gbits u8 [ngroups], .gsize i32 [1]. Column j of the permuted order belongs to group j / group.
 * Group widths must be in 1..=8 (the engine writes 2..=8) and ngroups >= ceil(d_in / group). */
typedef enum cdclq_dtype { CDCLQ_DTYPE_F32 = 0, CDCLQ_DTYPE_F16 = 1, CDCLQ_DTYPE_BF16 = 2 } cdclq_dtype;

/* quant::row_bytes (src/quant.rs:102-104): ceil(sum over j < d_in of gbits[j / group] / 8). */
int cdclq_row_bytes(size_t d_in, size_t group, const uint8_t* gbits, size_t ngroups, size_t* row_bytes);

/* io::packed_tensors (src/io.rs:244-264) with QLayer::pack / pack_row (src/quant.rs:207-214,
 * :113-131): the bytes of .qweight (qweight_bytes >= d_out * row_bytes), .scales (f16 bit
 * patterns, half::f16::from_f32), .qzeros (`zero as u8`) and .perm (`perm as i32`) for one layer.
 * codes d_out x d_in (permuted order), scales / zeros d_out x ngroups f32, perm d_in. */
int cdclq_pack_layer(cdclq_ctx* ctx, size_t d_out, size_t d_in, size_t group, const uint8_t* gbits, size_t ngroups,
                     const uint8_t* codes, const float* scales, const float* zeros, const uint32_t* perm,
                     uint8_t* qweight, size_t qweight_bytes, uint16_t* scales_f16, uint8_t* qzeros, int32_t* perm_i32);
/* Same contract; every array except gbits is device memory (codes never leave the GPU). */
int cdclq_pack_layer_device(cdclq_ctx* ctx, size_t d_out, size_t d_in, size_t group, const uint8_t* gbits,
                            size_t ngroups, const uint8_t* codes, const float* scales, const float* zeros,
                            const uint32_t* perm, uint8_t* qweight, size_t qweight_bytes, uint16_t* scales_f16,
                            uint8_t* qzeros, int32_t* perm_i32);

/* The `cdclq dequant` expansion of one layer: io::read_packed_layer (src/io.rs:270-293), i.e.
 * QLayer::from_packed (src/quant.rs:219-236) + QLayer::dequantize (src/quant.rs:189-202), then
 * io::f32_to_bytes (src/io.rs:50-57) into `dtype` (cdclq_dtype). out is d_out x d_in in the
 * original column order: 4-byte floats for F32, 16-bit patterns for F16 / BF16 (bit-identical to
 * the reference for every non-NaN value; a NaN stays a NaN, its payload is platform-defined as in
 * the reference). Every perm entry must be in 0..d_in (the reference panics otherwise); a repeated
 * entry keeps the reference's scatter result (the later column wins, unwritten columns are 0). */
int cdclq_dequantize_packed(cdclq_ctx* ctx, size_t d_out, size_t d_in, size_t group, const uint8_t* gbits,
                            size_t ngroups, const uint8_t* qweight, size_t qweight_bytes, const uint16_t* scales_f16,
                            const uint8_t* qzeros, const int32_t* perm_i32, int dtype, void* out);
int cdclq_dequantize_packed_device(cdclq_ctx* ctx, size_t d_out, size_t d_in, size_t group, const uint8_t* gbits,
                                   size_t ngroups, const uint8_t* qweight, size_t qweight_bytes,
                                   const uint16_t* scales_f16, const uint8_t* qzeros, const int32_t* perm_i32,
                                   int dtype, void* out);
/* QLayer::dequantize (src/quant.rs:189-202) + io::f32_to_bytes (src/io.rs:50-57) on the engine's
 * unpacked output (the pipeline's dequant/ tensors, src/pipeline.rs:153-162): codes d_out x d_in,
 * scales / zeros d_out x ngroups f32, perm d_in. */
int cdclq_dequantize_layer(cdclq_ctx* ctx, size_t d_out, size_t d_in, size_t group, size_t ngroups,
                           const uint8_t* codes, const float* scales, const float* zeros, const uint32_t* perm,
                           int dtype, void* out);
int cdclq_dequantize_layer_device(cdclq_ctx* ctx, size_t d_out, size_t d_in, size_t group, size_t ngroups,
                                  const uint8_t* codes, const float* scales, const float* zeros, const uint32_t* perm,
                                  int dtype, void* out);

/* ---- Evaluation and the synthetic benchmark (src/engine.rs:808-838, src/bench.rs) ---- */
/* engine::rtn_layer (src/engine.rs:822-838): round-to-nearest on each group's find_params grid,
 * no compensation, original column order; out is d_out x n f32 (dequantized values). Uses
 * cfg->bits, cfg->group and cfg->mse_grid. */
int cdclq_rtn_layer(cdclq_ctx* ctx, const float* w, size_t d_out, size_t n, const cdclq_config* cfg, float* out);
int cdclq_rtn_layer_device(cdclq_ctx* ctx, const float* w, size_t d_out, size_t n, const cdclq_config* cfg,
                           float* out);
/* engine::proxy_loss (src/engine.rs:808-815) on device memory. */
int cdclq_proxy_loss_device(cdclq_ctx* ctx, const float* w_t, const float* w_hat, size_t rows, size_t n,
                            const float* h, double* out);
/* bench::rel_err (src/bench.rs:106-121): ||W x - W_hat x~||^2 / ||W x||^2 over t tokens; x and x_t
 * are t x n token-major (pass x for x_t to measure the weight error alone). The f32 products are the
 * reference's chains; the two f64 sums run in parallel (not in element order). */
int cdclq_rel_err(cdclq_ctx* ctx, const float* w, const float* w_hat, const float* x, const float* x_t, size_t rows,
                  size_t n, size_t t, double* out);
int cdclq_rel_err_device(cdclq_ctx* ctx, const float* w, const float* w_hat, const float* x, const float* x_t,
                         size_t rows, size_t n, size_t t, double* out);

/* bench::BenchArgs (src/bench.rs:19-32); nthreads stands in for rayon::current_num_threads() (the
 * automatic row chunk and the report header). md / dump outputs are the caller's (the report text
 * is returned). */
typedef struct cdclq_bench_args {
  size_t rows;
  size_t cols;
  size_t tokens;
  size_t test_tokens;
  uint64_t seed;
  float asym_noise;
  uint32_t nthreads;
  cdclq_config cfg;
} cdclq_bench_args;
/* One row of the report (src/bench.rs:124-128). */
typedef struct cdclq_bench_row {
  char name[96];
  double loss;  /* proxy loss after the repair (0: not reported) */
  double calib; /* relative output error on the first min(tokens, 4096) calibration tokens */
  double test;  /* relative output error on the held-out tokens */
  double secs;
  double bpw;
} cdclq_bench_row;
/* bench::run (src/bench.rs:164-340) on the GPU: the same generator stream, method variants and
 * markdown report (times are this GPU's). rows_out receives up to max_rows rows in report order
 * (equal-bits table, then the skeleton rows, then the asymmetric rows); *nrows the total. report
 * (may be NULL) receives the markdown, truncated to report_cap - 1 bytes; *report_len its length. */
int cdclq_bench_run(cdclq_ctx* ctx, const cdclq_bench_args* args, cdclq_bench_row* rows_out, size_t max_rows,
                    size_t* nrows, char* report, size_t report_cap, size_t* report_len);

/* ---- Model pipeline (src/pipeline.rs) ---- */
/* pipeline::QuantOpts (src/pipeline.rs:24-40): shard and Hessian safetensors paths, output
 * directory, config, --only / --skip substrings, the two outputs; nthreads stands in for
 * rayon::current_num_threads() (automatic row chunks); verbose prints the reference's per-layer
 * progress line on stderr. */
typedef struct cdclq_quant_opts {
  const char* const* weights;
  size_t n_weights;
  const char* const* hessians;
  size_t n_hessians;
  const char* out_dir;
  cdclq_config cfg;
  const char* const* only;
  size_t n_only;
  const char* const* skip;
  size_t n_skip;
  int32_t emit_packed;
  int32_t emit_dequant;
  uint32_t nthreads;
  int32_t verbose;
} cdclq_quant_opts;
/* pipeline::quantize_model (src/pipeline.rs:79-227): every 2-D `*.weight` tensor that passes the
 * filters and has a Hessian (directly or through the store's aliases) is quantized on the GPU, jobs
 * ordered by (Hessian owner, layer) so q/k/v and gate/up share one factorisation; everything else is
 * passed through. Writes <out_dir>/dequant/<shard> (checkpoint dtypes), <out_dir>/packed/<shard>
 * (cdclq-v1; metadata quantization, orig_dtype, bits) and <out_dir>/report.json, whose text is also
 * returned (truncated to report_cap - 1; *report_len = full length). Error texts follow
 * src/io.rs / src/pipeline.rs (missing Hessian, non-square or non-finite H, width mismatch). */
int cdclq_quantize_model(cdclq_ctx* ctx, const cdclq_quant_opts* opts, char* report_json, size_t report_cap,
                         size_t* report_len);
/* pipeline::dequantize_packed (src/pipeline.rs:239-275): every `X.qweight` layer of a packed shard
 * becomes `X.weight` (original column order) in `dtype` (cdclq_dtype; -1 = the header's orig_dtype,
 * else F16); other tensors pass through. *nlayers = layers expanded. */
int cdclq_dequantize_model(cdclq_ctx* ctx, const char* input, const char* output, int dtype, size_t* nlayers);

/* ---- Device memory staging for callers without their own GPU runtime binding. ---- */
int cdclq_device_alloc(cdclq_ctx* ctx, size_t bytes, void** ptr);
int cdclq_device_free(cdclq_ctx* ctx, void* ptr);
int cdclq_memcpy_h2d(cdclq_ctx* ctx, void* dst, const void* src, size_t bytes);
int cdclq_memcpy_d2h(cdclq_ctx* ctx, void* dst, const void* src, size_t bytes);
int cdclq_memset_device(cdclq_ctx* ctx, void* dst, int value, size_t bytes);

/* ---- Synthetic calibration inputs generated in HBM (benchmark harness support; no reference
 * counterpart -- the reference's bench generator is src/bench.rs:41-97). Counter-based:
 * value i of stream `seed` = Box-Muller(splitmix64 draws 2i, 2i+1), identical on host and device. */
int cdclq_synth_normal_device(cdclq_ctx* ctx, uint64_t seed, uint64_t offset, size_t count, float sigma, float* out);
/* Host array of n channel scales: exactly round(frac * n) channels (seeded partial Fisher-Yates on
 * the same counter stream) get `factor`, the rest 1. */
int cdclq_synth_outlier_scales(uint64_t seed, size_t n, double frac, float factor, float* scales);
/* x[r][j] = normal(seed, (row0 + r) * n + j) * ch_scale[j]; ch_scale is a host array of n. */
int cdclq_synth_tokens_device(cdclq_ctx* ctx, uint64_t seed, uint64_t row0, size_t t, size_t n,
                              const float* ch_scale, float* x);
/* As cdclq_synth_tokens_device, with heavy-tailed channels: where heavy[j] != 0 (host array of n,
 * may be NULL) channel j draws Student-t with 3 degrees of freedom, Z / sqrt(chi2_3 / 3), from the
 * same counter stream (plus a second stream for chi2_3), identical on host and device. */
int cdclq_synth_tokens_heavy_device(cdclq_ctx* ctx, uint64_t seed, uint64_t row0, size_t t, size_t n,
                                    const float* ch_scale, const uint8_t* heavy, float* x);
/* out[i] = x[i] + sigma * normal(seed, offset + i) (device memory; out may equal x). */
int cdclq_synth_perturb_device(cdclq_ctx* ctx, uint64_t seed, uint64_t offset, size_t count, float sigma,
                               const float* x, float* out);
/* Host array of n log-normal channel scales: scales[j] = exp(sigma * normal(seed, j)). */
int cdclq_synth_lognormal_scales(uint64_t seed, size_t n, float sigma, float* scales);
/* h32[i] = (float)h64[i] (the cast at src/bench.rs:177). */
int cdclq_f64_to_f32_device(cdclq_ctx* ctx, const double* h64, size_t count, float* h32);

/* ---- Per-phase device timing (HIP events on the context's stream), for the harness. ---- */
enum {
  CDCLQ_PHASE_GRAM = 0,     /* H-accumulation kernels */
  CDCLQ_PHASE_FACTOR = 1,   /* permute/damp + Cholesky + triangular inverse -> U */
  CDCLQ_PHASE_GPTQ = 2,     /* phase 1: block sweeps + lazy GEMM */
  CDCLQ_PHASE_REPAIR = 3,   /* phase 2: refit + coordinate descent */
  CDCLQ_PHASE_TARGET = 4,   /* asymmetric target GEMMs */
  CDCLQ_PHASE_PACK = 5,     /* packed container: bit-packing and metadata kernels */
  CDCLQ_PHASE_DEQUANT = 6,  /* packed container: dequantization kernel */
  CDCLQ_PHASE_COUNT = 7
};
int cdclq_ctx_set_timing(cdclq_ctx* ctx, int enable);
int cdclq_ctx_reset_timing(cdclq_ctx* ctx);
/* Accumulated device milliseconds and number of timed launches of `phase` since the reset. */
int cdclq_ctx_get_timing(cdclq_ctx* ctx, int phase, uint64_t* launches, double* ms);

#ifdef __cplusplus
}
#endif
#endif
