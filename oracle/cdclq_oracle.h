/*
 * CPU oracle for the CDCL-GPTQ per-layer quantization engine.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference Rust crate
 * (tailot/CDCL-GPTQ, `cdclq` 1.0.1) used as the parity checker for the HIP library and as the
 * timed CPU baseline. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it. The product (libcdclq_hip.so) never links or calls it.
 *
 * Every function cites the reference file:line it restates. Arithmetic follows the reference
 * op for op: IEEE f32/f64, no contraction of a*b+c (build with -ffp-contract=off), Rust's
 * f32::round = C roundf (half away from zero), and the GEMMs of the `matrixmultiply` 0.3.8
 * dependency restated as per-element fused-multiply-add chains in k order, split into KC = 256
 * panels that are combined in panel order (C = fma(alpha, chain_p, C)).
 *
 * Pinning status (what checks each function; see tests/test_oracle_*.py):
 *   round_f16          exhaustive over all 2^32 f32 patterns vs numpy float16 (IEEE RNE)
 *   pack/unpack/dequant  the reference's own round trip (src/quant.rs:262-275, Rng(9) codes),
 *                      an independent big-integer / numpy.packbits bit-stream formulation,
 *                      numpy float32 dequantization; f16/bf16 narrowing vs numpy float16 and
 *                      torch bfloat16 (non-NaN), NaN rule by construction only
 *   find_params/quant  closed form + brute force + src/quant.rs:279-286 properties
 *   gram_accumulate    f64 brute force, exact symmetry, chunk edges (T = 2047/2048/2049)
 *   cholesky/tri_inv   numpy/scipy Cholesky and inverse; src/linalg.rs:447-504 properties
 *   quantize_layer     the reference's own engine tests (src/engine.rs:890-988), an independent
 *                      f64 per-column GPTQ (scripts/ref_gptq_check.py:25-64 algorithm),
 *                      brute-force optimality of every repair move on tiny inputs
 *   sgemm/dgemm chains parity UNPINNED against the Rust binary: matrixmultiply 0.3.8 is not in
 *                      /root/reference and cannot be built here; its FMA-chain/KC=256 order is
 *                      an assumption checked only against f64 brute force (tolerance) and the
 *                      reference's parallel == serial property (src/linalg.rs:510-541).
 */
#ifndef CDCLQ_ORACLE_H
#define CDCLQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same field layout as cdclq_config in include/cdclq.h (checked by a test). Mirrors
 * `engine::Config` (src/engine.rs:94-144). method: 0 = Gptq, 1 = Cdcl. */
typedef struct orc_config {
  uint32_t bits;
  uint32_t skeleton_bits;
  uint64_t group;
  uint64_t block;
  uint64_t sub_block;
  uint64_t cd_sweeps;
  uint64_t passes;
  uint64_t row_chunk;
  double damp;
  double skeleton_pct;
  double refine_frac;
  double tol;
  int32_t act_order;
  int32_t mse_grid;
  int32_t method;
  int32_t refit_scales;
} orc_config;

/* `engine::LayerStats` (src/engine.rs:174-199). */
typedef struct orc_layer_stats {
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
} orc_layer_stats;

enum { ORC_OK = 0, ORC_INVALID_ARG = 1, ORC_NOT_PD = 2 };

size_t orc_sizeof_config(void);
size_t orc_sizeof_stats(void);
void orc_default_config(orc_config* cfg);

/* src/quant.rs:20-26 */
float orc_round_f16(float x);
void orc_round_f16_array(const float* x, float* y, size_t n);
/* src/quant.rs:40-83 */
void orc_find_params(const float* vals, size_t len, uint32_t bits, int mse, float* scale, float* zero);
/* src/quant.rs:92-95 */
float orc_quant_code(float x, float scale, float zero, float maxq, uint8_t* code);

/* src/linalg.rs:56-99 (matrixmultiply semantics, see header comment) */
void orc_sgemm(size_t m, size_t k, size_t n, float alpha, const float* a, ptrdiff_t rsa, ptrdiff_t csa, const float* b,
               ptrdiff_t rsb, ptrdiff_t csb, float beta, float* c, ptrdiff_t rsc, ptrdiff_t csc);
void orc_dgemm(size_t m, size_t k, size_t n, double alpha, const double* a, ptrdiff_t rsa, ptrdiff_t csa, const double* b,
               ptrdiff_t rsb, ptrdiff_t csb, double beta, double* c, ptrdiff_t rsc, ptrdiff_t csc);

/* src/linalg.rs:200-276. Returns ORC_NOT_PD with the reference's message in err. */
int orc_cholesky_lower(double* a, size_t n, char* err, size_t errlen);
/* src/linalg.rs:284-347 */
void orc_tri_inverse_lower(const double* l, size_t n, double* y);
/* src/linalg.rs:362-375 (h is copied, not consumed) */
int orc_upper_chol_of_inverse(const double* h, size_t n, float* u, char* err, size_t errlen);
/* src/linalg.rs:388-418 */
void orc_gram_accumulate(const float* x, const float* y, size_t t, size_t n, double* h);

/* One-entry PrepCache (src/engine.rs:207-223). */
typedef struct orc_cache orc_cache;
orc_cache* orc_cache_new(void);
void orc_cache_free(orc_cache* c);

/* engine::quantize_layer (src/engine.rs:690-799). Outputs: codes[d_out*d_in] (permuted order),
 * scales/zeros[d_out*ng], perm[d_in], gbits[ng]. nthreads plays rayon::current_num_threads()
 * for the automatic row chunk (src/engine.rs:768-770). m may be NULL. */
int orc_quantize_layer(const float* w, size_t d_out, size_t d_in, const float* h, const float* m, const char* hkey,
                       const orc_config* cfg, size_t nthreads, orc_cache* cache, uint8_t* codes, float* scales,
                       float* zeros, uint32_t* perm, uint8_t* gbits, orc_layer_stats* st, char* err, size_t errlen);
size_t orc_num_groups(const orc_config* cfg, size_t n);

/* engine::proxy_loss (src/engine.rs:808-815); f64 reduction in index order. */
double orc_proxy_loss(const float* w_t, const float* w_hat, size_t rows, size_t n, const float* h);
/* engine::rtn_layer (src/engine.rs:822-838) */
void orc_rtn_layer(const float* w, size_t d_out, size_t n, const orc_config* cfg, float* out);
/* QLayer::dequantize (src/quant.rs:189-202) */
void orc_dequantize(size_t d_out, size_t n, size_t g, const uint32_t* perm, size_t ng, const uint8_t* codes,
                    const float* scales, const float* zeros, float* out);

/* Packed container cdclq-v1. dtype: 0 = F32, 1 = F16, 2 = BF16.
 * half 2.4.1 conversions (IEEE RNE narrowing; NaN keeps sign and upper payload, quiet bit set). */
uint16_t orc_f32_to_f16_bits(float x);
float orc_f16_bits_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16_bits(float x);
/* io::f32_to_bytes (src/io.rs:50-57) */
void orc_narrow(const float* v, size_t count, int dtype, void* out);
/* quant::row_bytes (src/quant.rs:102-104) */
size_t orc_row_bytes(size_t n, size_t g, const uint8_t* gbits);
/* quant::pack_row / unpack_row (src/quant.rs:113-151) */
void orc_pack_row(const uint8_t* codes, size_t n, size_t g, const uint8_t* gbits, uint8_t* out);
void orc_unpack_row(const uint8_t* data, size_t n, size_t g, const uint8_t* gbits, uint8_t* codes);
/* io::packed_tensors + QLayer::pack (src/io.rs:244-264, src/quant.rs:207-214) */
void orc_pack_layer(size_t d_out, size_t n, size_t g, const uint8_t* gbits, size_t ng, const uint8_t* codes,
                    const float* scales, const float* zeros, const uint32_t* perm, uint8_t* qweight, uint16_t* scales16,
                    uint8_t* qzeros, int32_t* perm32);
/* io::read_packed_layer + QLayer::dequantize + f32_to_bytes (src/io.rs:270-293, src/quant.rs:189-236) */
void orc_dequantize_packed(size_t d_out, size_t n, size_t g, const uint8_t* gbits, size_t ng, const uint8_t* qweight,
                           const uint16_t* scales16, const uint8_t* qzeros, const int32_t* perm32, int dtype,
                           void* out);

/* Synthetic benchmark inputs (src/bench.rs:41-97, :275-295) from Rng(seed) in the reference's draw
 * order; xt / xte_t (asymmetric-noise copies) may be NULL when asym_noise == 0. */
void orc_bench_inputs(uint64_t seed, size_t rows, size_t n, size_t tokens, size_t test_tokens, float asym_noise,
                      float* w, float* x, float* xte, float* xt, float* xte_t);
/* bench::rel_err (src/bench.rs:106-121) */
double orc_rel_err(const float* w, const float* wq, const float* x, const float* xt, size_t rows, size_t n,
                   size_t t);

/* rng.rs restatement (src/rng.rs:22-57). normal() uses the platform libm (glibc logf/sinf/cosf). */
typedef struct orc_rng {
  uint64_t s;
  int32_t has_spare;
  float spare;
} orc_rng;
void orc_rng_new(orc_rng* r, uint64_t seed);
uint64_t orc_rng_next_u64(orc_rng* r);
float orc_rng_uniform(orc_rng* r);
float orc_rng_normal(orc_rng* r);

/* Counter-based synthetic generator shared (as an algorithm) with the device generator in the
 * HIP library, so both sides consume identical bytes. f64 log / cos written from basic IEEE ops.
 *   normal_at(seed, i): splitmix64 at counters 2i, 2i+1 -> Box-Muller cos branch, f32. */
float orc_synth_normal_at(uint64_t seed, uint64_t i);
void orc_synth_normal(uint64_t seed, uint64_t offset, size_t n, float sigma, float* out);
/* Per-channel scale vector: exactly round(frac*n) channels (seeded Fisher-Yates) get `factor`. */
void orc_synth_outlier_scales(uint64_t seed, size_t n, double frac, float factor, float* scales);
void orc_synth_lognormal_scales(uint64_t seed, size_t n, float sigma, float* scales);
/* X (t x n, token-major): x[r][j] = normal_at(seed, (row0 + r)*n + j) * ch_scale[j]. */
void orc_synth_tokens(uint64_t seed, uint64_t row0, size_t t, size_t n, const float* ch_scale, float* x);
float orc_synth_student3_at(uint64_t seed, uint64_t i);
/* Near-midpoint accounting of the last orc_quantize_layer call: code decisions, near; zero-point
 * decisions, near; descent evaluations, near (same definitions as cdclq_midpoint_counts). */
void orc_last_midpoint_counts(uint64_t* out);
/* d_out x n map of near-midpoint decisions filled by the next orc_quantize_layer calls (NULL: off):
 * bit 0 phase-1 code, bit 1 a descent evaluation, bit 2 the group's zero point. */
void orc_set_midpoint_map(uint8_t* map);
void orc_synth_tokens_heavy(uint64_t seed, uint64_t row0, size_t t, size_t n, const float* ch_scale,
                            const uint8_t* heavy, float* x);
double orc_synth_log(double x);
double orc_synth_cos2pi(double u);

/* Test hook: plant a known mistake (0 = none). Used only by tests that check the pinning
 * checks catch it. */
void orc_set_mutation(int id);

/* Threads used by the oracle's OpenMP regions (0 = OpenMP default). */
void orc_set_threads(int nthreads);

#ifdef __cplusplus
}
#endif
#endif
