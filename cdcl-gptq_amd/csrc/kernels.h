// Host-side launchers of the gfx950 kernels (one translation unit per kernel family).
// All launchers enqueue on `st` and return hipGetLastError() of the launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <vector>

namespace cdclq {

// ---- k_gemm.hip: bit-exact chain GEMMs (matrixmultiply 0.3.8 order, see k_gemm.hip)
// C = alpha * A * B + beta * C in the matrixmultiply order: per panel, C = fma(alpha, chain, C')
// with C' = beta * C before the first panel (0 when beta == 0, C unread). `lower` computes only
// tiles that intersect the lower triangle (i >= j) of C. When k spans several KC panels and
// `partials` is non-null, panels run in parallel into partials[npanel][m][n] and are combined in
// panel order.
template <typename T>
hipError_t gemm_chain(hipStream_t st, int m, int n, int k, T alpha, T beta, const T* A, long rsa, long csa,
                      const T* B, long rsb, long csb, T* C, long rsc, long csc, bool lower, T* partials,
                      bool b_lower_tri = false);
size_t gemm_partials_elems(int m, int n, int k);
// Cholesky trailing update of the lower tiles of C (m x n) by k / 96 consecutive 96-column blocks
// of L rows P (m x k, row stride ldp; P's first n rows are also the right operand, transposed):
// for each block b in order, C = fma(-1, chain_b, C) with chain_b the 96-step FMA chain of
// P[:, b] P[0:n, b]^T (src/linalg.rs:243-270, one dgemm per block).
hipError_t chol_update(hipStream_t st, int m, int n, int k, const double* P, long ldp, double* C, long ldc);
// The triangular inverse's product Y[s:e, 0:s] = alpha Y_ss t (beta = 0, m <= 96 rows, k <= KC: one
// panel; A along k, B along n; src/linalg.rs:330-343) on the pipelined kernel. inv_gemm_eligible
// lists the requirements (else use gemm_chain).
bool inv_gemm_eligible(int m, int n, int k, const double* A, long lda, const double* B, long ldb);
hipError_t inv_gemm(hipStream_t st, int m, int n, int k, double alpha, const double* A, long lda, const double* B,
                    long ldb, double* C, long ldc);

// C = fma(1, chain, C) for one k range of at most one KC panel (A along k, B along j): a panel's
// contribution to the triangular inverse's block-row products, applied right-looking to every
// block row below it, or a block row's last, partial panel (src/linalg.rs:307-321).
// inv_acc_eligible lists the requirements.
bool inv_acc_eligible(int m, int n, int k, const double* A, long lda, const double* B, long ldb);
hipError_t inv_acc(hipStream_t st, int m, int n, int k, const double* A, long lda, const double* B, long ldb,
                   double* C, long ldc);

// ---- k_gram.hip: H (n x n, f64) += X^T Y over 2048-token chunks on the matrix cores.
struct GramJob {
  const float* x;  // t x n, token-major
  const float* y;  // t x n (== x for a Hessian)
  double* h;       // n x n accumulator
  int n;
  int t;
};
// Appends the workgroup tiles of job `job` (int4: job, row block of 128, col block of 64,
// mirror flag). `sym`: Y == X and the incoming H is symmetric.
void gram_mfma_tiles(int job, int n, bool sym, std::vector<int4>& out);
// direct-to-LDS gram for jobs that satisfy gram_dma_eligible (all tiles interior, T % 64 == 0), on
// 128 x 128 tiles (int4: job, row block of 128, col block of 128, flags: mirror in bit 0, gang
// size in bits 1-6, position in the gang in bits 7-11, gang in bits 12-30; job -1: an empty slot).
// prog: one zeroed int per tile slot for the gang pacing, or null (no pacing).
hipError_t gram_dma(hipStream_t st, const GramJob* jobs, const int4* tiles, int ntiles, int* prog);
void gram_dma_tiles(int job, int n, bool sym, std::vector<int4>& out);
// Reorders a gram_dma_tiles list (jobs contiguous) into gangs of 32 neighbouring tiles (each job in
// Morton order of (row block, col block): an aligned gang is a 4 x 8 block of tiles, 12 stripes of
// X and Y instead of up to 33 for a run of one row), gang g on XCD g % 8 in round g / 8: slot
// (32 round + position) * 8 + XCD (workgroup w runs on XCD w % 8), empty slots after the last
// tile. Sets the gang fields of the flags.
void gram_dma_order(std::vector<int4>& tiles);
bool gram_dma_eligible(int n, int t, const void* x, const void* y);
hipError_t gram_mfma(hipStream_t st, const GramJob* jobs, const int4* tiles, int ntiles, bool vec4);
hipError_t sym_check(hipStream_t st, int n, const double* h, int* flag);
// p[0..count) = 0 (a kernel, not a memset node)
hipError_t zero_words(hipStream_t st, int* p, int count);
// Fixed device memory of the allocation-free Gram entry point: status words (256 B), the job
// record (256 B), then the tile list of one job with n <= kGramNoAllocMaxN (non-symmetric worst
// case: ceil(n/128) * ceil(n/64) tiles of 16 bytes).
constexpr int kGramNoAllocMaxN = 32768;
constexpr size_t kGramScratchTiles = (size_t)(kGramNoAllocMaxN / 128) * (kGramNoAllocMaxN / 64);
constexpr size_t kGramScratchBytes = 512 + kGramScratchTiles * 16;
// Device address of this GPU's copy of that memory; `device` must be the current device. Looked
// up once per device (hipGetSymbolAddress) and kept for the life of the process.
hipError_t gram_scratch(int device, void** ptr);

// ---- k_factor.hip: damping, Cholesky, triangular inverse, U
hipError_t build_flipped(hipStream_t st, int n, const float* h, const uint32_t* perm, double damp_val, double* a,
                         float* h32);
hipError_t build_flipped_f64(hipStream_t st, int n, const double* h, double* a);
hipError_t chol_diag(hipStream_t st, int n, double* a, int k, int kb, int* status, double* pivot);
hipError_t chol_panel(hipStream_t st, int n, double* a, int k, int kb, const int* status);
hipError_t trinv_diag(hipStream_t st, int n, const double* l, double* y, const int* status);
hipError_t scatter_u(hipStream_t st, int n, const double* y, float* u);
hipError_t fill_zero_f64(hipStream_t st, double* p, size_t count);

// ---- k_engine.hip: phase 1 / phase 2 sweeps and helpers
hipError_t permute_w(hipStream_t st, int d_out, int n, const float* w, const uint32_t* perm, const uint8_t* dead_perm,
                     float* wp);
hipError_t permute_m(hipStream_t st, int n, const float* m, const uint32_t* perm, float damp32, float* mp);
hipError_t diag_extract(hipStream_t st, int n, const float* h, float* diag);
hipError_t colsq(hipStream_t st, int d_out, int n, const float* w, const uint8_t* dead, double* out);
hipError_t inv_diag(hipStream_t st, int n, const float* u, float* invd);
// Phase-1 sweep of block [i1, i1 + cnt) for all rows. groups_in_block: every group grid of the
// block reads only columns of the block (the block width is a multiple of the group size), which
// allows the lanes-per-row kernel.
hipError_t gptq_block(hipStream_t st, int rows, int n, int i1, int cnt, int g, int ng, float* w, const float* u,
                      const float* invd, const uint8_t* gbits, int mse, float* scales, float* zeros, uint8_t* codes,
                      float* wq, float* err, unsigned long long* mid, bool groups_in_block);
hipError_t colloss(hipStream_t st, int rows, int n, int rc, const float* err, double* out);
hipError_t sub_f32(hipStream_t st, size_t count, const float* a, const float* b, float* out);
// ---- k_repair.hip: phase 2
// P[p][r][c] = chain over panel p of A[r][k] B[k][c] (r < m, c < wd)
size_t panel_partials_elems(int m, int wd, int k);
// Repair gradient: per-panel chains of G = A B into P (np x m x wd), for the listed 128-row tiles
// of A (all tiles when rtiles is null), then their ordered fold into G (d_out x wd).
int panel_row_tile();
hipError_t panel_gemm(hipStream_t st, int m, int wd, int k, const float* A, long lda, const float* B, long ldb,
                      float* P, const int* rtiles, int ntiles);
hipError_t fold_panels(hipStream_t st, int m, int wd, int np, const float* P, float* G, const int* rtiles,
                       int ntiles);
// f32 chain GEMM on the matrix cores folding one chain per kfold steps of k straight into C:
// starting from beta_one ? C : 0, C = fma(alpha, chain_b, C) for b = 0 .. k / kfold - 1 in order
// (kfold = 0: one chain over all of k). A m x k (row stride lda), B k x n (row stride ldb),
// kfold <= 256 (one KC panel) and kfold % 32 == 0; the _ok test lists every requirement (else use
// gemm_chain). One block of the GPTQ lazy update per chain (src/engine.rs:452-471).
bool chain_gemm_mfma_ok(int m, int n, int k, const float* A, long lda, const float* B, long ldb, int kfold = 0);
hipError_t chain_gemm_mfma(hipStream_t st, int m, int n, int k, float alpha, int beta_one, const float* A, long lda,
                           const float* B, long ldb, float* C, long ldc, int kfold = 0);
// ---- k_gemm_wide.hip: multi-panel f32 chain GEMM C = A B (alpha 1, beta 0) on the matrix cores,
// panels folded in registers (the asymmetric target's three GEMMs). tri: 0 dense B, 1 B upper
// triangular (B[k][j] = 0 for k > j), 2 B lower triangular (B[k][j] = 0 for k < j).
bool chain_gemm_tiles_ok(int m, int n, int k, const float* A, long lda, const float* B, long ldb, const float* C,
                         long ldc);
hipError_t chain_gemm_tiles(hipStream_t st, int m, int n, int k, const float* A, long lda, const float* B, long ldb,
                            float* C, long ldc, int tri);
hipError_t transpose_f32(hipStream_t st, int n, const float* src, float* dst);
// Scale refit of group gi from its gradient: G (rows x wd), or, with P, the np per-panel chains of
// panel_gemm (P[p][rows][wd]) folded in panel order by the kernel itself (no separate fold
// launch); refit_folds_chains(wd) says whether that form is available.
hipError_t refit_group(hipStream_t st, int rows, int n, int ng, int g, int gi, int rc, const float* G,
                       const float* h32, const uint8_t* codes, float* scales, const float* zeros, float* wq, float* e,
                       const uint8_t* active, double* dlog, uint32_t* dcnt, const float* P = nullptr, int np = 0);
bool refit_folds_chains(int wd);
// Coordinate descent over one sub-block. The gradient comes from G, or, when P is non-null, from
// the np per-panel chains of panel_gemm (P[p][rows][wd]), folded in panel order by the kernel
// itself (no separate fold launch); cd_folds_chains(wd) says whether that form is available.
bool cd_folds_chains(int wd);
hipError_t cd_subblock(hipStream_t st, int rows, int n, int ng, int g, int c0, int wd, int sb, int nsb, int rc,
                       int sweeps, float* G, const float* h32, const uint8_t* gbits, const float* scales,
                       const float* zeros, uint8_t* codes, float* wq, float* e, const uint8_t* active,
                       const uint8_t* sel, double* dlog, uint32_t* dcnt, int cap, unsigned long long* mid,
                       uint32_t* evals, const float* P = nullptr, int np = 0);
// Folds one pass's logged deltas into the per-chunk loss (exact reference order); nref refit
// steps (rlog/rcnt: [nref][rows]) then ncd CD steps (clog: [ncd][rows][cap], ccnt: [ncd][rows]).
hipError_t pass_accum(hipStream_t st, int rows, int rc, int nchunks, int nref, const double* rlog,
                      const uint32_t* rcnt, int ncd, int cap, const double* clog, const uint32_t* ccnt,
                      const uint8_t* active, double* ld, uint64_t* upd);
// ---- k_pack.hip: packed container cdclq-v1 (bit streams LSB first, per-group widths)
// qw (d_out x rb) from codes (d_out x n); coff[j] = bit offset of code j (coff[n] = total bits),
// wfirst[w] = first code whose 8-bit window reaches bit 32 w of a row. With only_if non-null the
// launch does nothing unless *only_if == epoch.
hipError_t pack_rows(hipStream_t st, long d_out, int n, int rb, const uint8_t* codes, const uint32_t* coff,
                     const int* wfirst, uint8_t* qw, const uint32_t* only_if, uint32_t epoch);
// fast path when every run of 8 columns lies in one group (rdesc[k] = byte offset of run k << 4 |
// width); *spill is set to epoch if a code exceeds its width (then pack_rows redoes the layer)
hipError_t pack_runs(hipStream_t st, long d_out, int n, int rb, const uint8_t* codes, const uint32_t* rdesc,
                     uint8_t* qw, uint32_t* spill, uint32_t epoch);
hipError_t pack_meta(hipStream_t st, long count, const float* scales, const float* zeros, uint16_t* s16, uint8_t* z8);
// output column map: last[c] = max j with perm[j] == c (-1: none), cdesc[c] = bit offset << 4 |
// width (packed) or last[c] (unpacked), cgrp[c] = last[c] / g; *bad is set to epoch if some
// perm[j] >= n.
hipError_t column_map(hipStream_t st, int n, int g, bool packed, const uint32_t* perm, const uint32_t* coff,
                      const uint8_t* cwid, int* last, uint32_t* cdesc, int* cgrp, uint32_t* bad, uint32_t epoch);
// out (d_out x n, dtype) from packed rows (srcb = row bytes) or u8 code rows (srcb = n)
hipError_t dequant_rows(hipStream_t st, bool packed, int dtype, long d_out, int n, int ng, int srcb,
                        const uint8_t* src, const uint32_t* cdesc, const int* cgrp, const void* scales,
                        const void* zeros, void* out);

// ---- k_eval.hip: benchmark-harness evaluation
// out (d_out x n) = engine::rtn_layer of w with group g
hipError_t rtn_rows(hipStream_t st, long d_out, int n, int g, int bits, int mse, const float* w, float* out);
// partial[2b] = sum (o1 - o2)^2, partial[2b+1] = sum o1^2 over block b's share (f64)
hipError_t err_reduce(hipStream_t st, size_t count, const float* o1, const float* o2, double* partial, int nblocks);
// x = (x + noise) * scale[j] * massive[t]
hipError_t act_scale(hipStream_t st, long tokens, int n, const float* noise, const float* scale, const float* massive,
                     float* x);
// rms[j] = sqrt(sum_t x[t][j]^2 / tokens), f32 sums in token order
hipError_t channel_rms(hipStream_t st, long tokens, int n, const float* x, float* rms);
// xt = x + a * rms[j] * nrm
hipError_t add_noise(hipStream_t st, long tokens, int n, float a, const float* rms, const float* nrm, const float* x,
                     float* xt);

// io::tensor_to_f32 (dtype: CDCLQ_DTYPE_*) and io's first non-finite element (*first must start at
// a value >= count; it ends at the smallest non-finite index, if any)
hipError_t decode_to_f32(hipStream_t st, long count, int dtype, const void* src, float* out);
hipError_t first_non_finite(hipStream_t st, long count, const float* x, unsigned long long* first);

// out = x * sqrt(w[t]) per token row; h = (float)(acc / tokens)
hipError_t token_scale(hipStream_t st, long t, int n, const float* x, const float* w, float* out);
hipError_t normalize_acc(hipStream_t st, long count, const double* acc, double tokens, float* h);

hipError_t synth_normal(hipStream_t st, uint64_t seed, uint64_t offset, size_t count, float sigma, float* out);
// x[r][j] = (heavy[j] ? student3 : normal)(seed, (row0 + r) n + j) * ch_scale[j] (null arrays: none / 1)
hipError_t synth_tokens(hipStream_t st, uint64_t seed, uint64_t row0, size_t t, size_t n, const float* ch_scale,
                        const uint8_t* heavy, float* x);
hipError_t synth_perturb(hipStream_t st, uint64_t seed, uint64_t offset, size_t count, float sigma, const float* x,
                         float* out);
hipError_t f64_to_f32(hipStream_t st, size_t count, const double* a, float* b);
hipError_t proxy_reduce(hipStream_t st, size_t count, const float* e, const float* eh, double* partial, int nblocks);

}  // namespace cdclq
