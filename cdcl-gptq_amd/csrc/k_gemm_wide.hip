// Multi-panel f32 chain GEMM on the matrix cores, C = A B (alpha 1, beta 0), with the
// matrixmultiply 0.3.8 order of the reference (src/linalg.rs:56-184): per C element a fused chain
// over each KC = 256 panel of k, started from 0, and the panels folded in order,
// C = fma(1, chain_p, C) with C = 0 before the first panel. It serves the three GEMMs of the
// asymmetric calibration target W* = ((W M') U^T) U (src/engine.rs:737-755), where k = n and the
// output is as wide as k, so the output tiles alone fill the GPU and no panel runs apart from the
// others: each workgroup folds the panels of its tile in registers and writes C once.
//
// Chains: v_mfma_f32_32x32x1_2b_f32 (K = 1, one rounding per product, bit-identical to fmaf), as in
// the repair gradient and the lazy update. Tile 128 x 128, 8 waves (wave w: rows 32 (w & 3) .. +31,
// columns 64 (w >> 2) .. +63); 32-k stages filled with global_load_lds_dwordx4 into a ring of three
// (two stages in flight behind the one being multiplied), the stage layout and load plan of the
// lazy update's 128 x 128 tile.
//
// Triangular B (the factor U is upper triangular):
//   TRI_UPPER (B = U, B[k][j] = 0 for k > j): every product past column j of the tile is
//   fma(a, 0, c) = c exactly, so the tile stops at k = its last column + 1; the panels it skips are
//   all-zero chains (+0), and C + (+0) = C.
//   TRI_LOWER (B = U^T, B[k][j] = 0 for k < j): panels that end before the tile's first column hold
//   only zero products; their chains are +0 and fold into C = +0, so the tile starts at the panel
//   holding its first column, where the leading zero products leave the chain at +0.
// Both are exact for finite A; an infinite or NaN entry of A inside a skipped zero block would
// make the reference's chain NaN there and not this one.
#include "cdclq_dev.h"
#include "kernels.h"

namespace cdclq {
namespace {

typedef float v32f __attribute__((ext_vector_type(32)));

constexpr int TM = 128, TN = 128, SK = 32, NBUF = 3;
constexpr int STAGE = SK * TM + SK * TN;  // floats per stage: A [128 rows][8 slots][4], B [32 k][128 cols]
constexpr int LPW = STAGE / 512 / 4;      // 1 KB loads per wave and stage (4: two of A, two of B)
// tiles per XCD block: 4 row tiles x 8 column tiles run together on one XCD and share their A and B
// stages through its L2
constexpr int XB_R = 4, XB_C = 8, XB = XB_R * XB_C;

__device__ __forceinline__ v32f mfma32(float a, float b, v32f c) {
  return __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, c, 0, 0, 0);
}

template <int TRI>
__global__ __launch_bounds__(512) void k_chain_gemm_tiles(int m, int n, int k, const float* __restrict__ A, long lda,
                                                          const float* __restrict__ B, long ldb, float* __restrict__ C,
                                                          long ldc) {
  __shared__ float R[NBUF][STAGE];
  // Workgroup b runs on XCD b % 8. Slot i = b / 8 of an XCD belongs to block (i / 32) * 8 + xcd;
  // a block is 4 x 8 tiles, row tiles outer.
  const int ntr = (m + TM - 1) / TM, ntc = (n + TN - 1) / TN;
  const int nbc = (ntc + XB_C - 1) / XB_C;
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const int blk = (slot / XB) * 8 + xcd, pos = slot % XB;
  const int tr = (blk / nbc) * XB_R + pos / XB_C, tc = (blk % nbc) * XB_C + pos % XB_C;
  if (tr >= ntr || tc >= ntc) return;
  const int r0 = tr * TM, cb = tc * TN;
  int kbeg = 0, kend = k;
  if (TRI == 1) kend = min(k, cb + TN);
  if (TRI == 2) kbeg = (cb / CDCLQ_KC) * CDCLQ_KC;
  const int nst = (kend - kbeg) / SK;
  if (nst <= 0) {  // no nonzero product reaches this tile (only possible with TRI): C = +0
    const int tid = threadIdx.x;
    for (int e = tid; e < TM * TN; e += 512) {
      const int row = r0 + e / TN, col = cb + e % TN;
      if (row < m && col < n) C[(long)row * ldc + col] = 0.0f;
    }
    return;
  }
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = wv & 3, wc = wv >> 2;
  // per-lane source offsets (relative to A + r0 * lda + ks and B + ks * ldb): loads 0..15 fill the
  // A stage (8 rows each, k-quad (lane & 7) ^ (row & 7) into slot lane & 7), loads 16..31 the B
  // stage (2 k rows each); rows past m and columns past n read clamped addresses whose values only
  // reach outputs that are never stored
  int off[LPW];
#pragma unroll
  for (int q = 0; q < LPW; ++q) {
    const int ins = wv + 8 * q;
    if (q < 2) {
      const int rl = 8 * ins + (lane >> 3);
      off[q] = (min(r0 + rl, m - 1) - r0) * (int)lda + 4 * ((lane & 7) ^ (rl & 7));
    } else {
      off[q] = (2 * (ins - 16) + (lane >> 5)) * (int)ldb + min(cb + 4 * (lane & 31), n - 4);
    }
  }
  const uint32_t lds0 = lds_offset(&R[0][0]);
  const float* a_base = A + (long)r0 * lda;
  int fi = 0;  // stages issued
  auto issue = [&]() {
    if (fi >= nst) return;
    const uint32_t buf = lds0 + (uint32_t)((fi % NBUF) * STAGE * 4);
    const int ks = kbeg + fi * SK;
    const float* ea = a_base + ks;
    const float* hb = B + (long)ks * ldb;
#pragma unroll
    for (int q = 0; q < LPW; ++q) {
      const int ins = wv + 8 * q;
      dma16_untracked((q < 2 ? ea : hb) + off[q], buf + 1024u * (uint32_t)ins);
    }
    ++fi;
  };
  issue();
  issue();
  const int er = 32 * wr + (lane & 31);
  v32f acc = {};
  float c[32];
#pragma unroll
  for (int r = 0; r < 32; ++r) c[r] = 0.0f;
  for (int fc = 0; fc < nst; ++fc) {
    // this wave's part of stage fc has landed once at most the next stage's loads are outstanding
    if (fi - fc >= 2)
      wait_vmcnt<LPW>();
    else
      wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();  // all parts of stage fc visible; every read of stage fc - 1 done
    issue();                       // stage fc + 2, into the slot of stage fc - 1
    const float* buf = &R[fc % NBUF][0];
    const float* es = buf + 32 * er;
    const float* hs = buf + SK * TM + 64 * wc + lane;
#pragma unroll
    for (int q = 0; q < SK / 4; ++q) {
      const float4 a = *reinterpret_cast<const float4*>(es + 4 * (q ^ (er & 7)));
      acc = mfma32(a.x, hs[(4 * q + 0) * TN], acc);
      acc = mfma32(a.y, hs[(4 * q + 1) * TN], acc);
      acc = mfma32(a.z, hs[(4 * q + 2) * TN], acc);
      acc = mfma32(a.w, hs[(4 * q + 3) * TN], acc);
    }
    const int knext = kbeg + (fc + 1) * SK;
    if (knext % CDCLQ_KC == 0 || knext == kend) {  // a panel (or the tile's k range) ends here
#pragma unroll
      for (int r = 0; r < 32; ++r) c[r] = __builtin_fmaf(1.0f, acc[r], c[r]);
      acc = v32f{};
    }
  }
  // block b = r >> 4 (cols 32b..), row i = (r & 3) + 8 * ((r & 15) >> 2) + 4 * (lane >> 5), col j = lane & 31
#pragma unroll
  for (int r = 0; r < 32; ++r) {
    const int row = r0 + 32 * wr + (r & 3) + 8 * ((r & 15) >> 2) + 4 * (lane >> 5);
    const int col = cb + 64 * wc + 32 * (r >> 4) + (lane & 31);
    if (row < m && col < n) C[(long)row * ldc + col] = c[r];
  }
}

// dst = src^T for an n x n matrix: 64 x 64 tiles through LDS (padded rows), coalesced both ways.
__global__ __launch_bounds__(256) void k_transpose(int n, const float* __restrict__ src, float* __restrict__ dst) {
  __shared__ float t[64][65];
  const int bi = blockIdx.y * 64, bj = blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4) {
    const int i = bi + r, j = bj + tx;
    if (i < n && j < n) t[r][tx] = src[(long)i * n + j];
  }
  __syncthreads();
  for (int r = ty; r < 64; r += 4) {
    const int i = bj + r, j = bi + tx;  // dst[i][j] = src[j][i]
    if (i < n && j < n) dst[(long)i * n + j] = t[tx][r];
  }
}

}  // namespace

hipError_t transpose_f32(hipStream_t st, int n, const float* src, float* dst) {
  if (n <= 0) return hipSuccess;
  const unsigned nb = (unsigned)((n + 63) / 64);
  hipLaunchKernelGGL(k_transpose, dim3(nb, nb), dim3(256), 0, st, n, src, dst);
  return hipGetLastError();
}

bool chain_gemm_tiles_ok(int m, int n, int k, const float* A, long lda, const float* B, long ldb, const float* C,
                         long ldc) {
  return m > 0 && n >= 4 && k > 0 && k % SK == 0 && n % 4 == 0 && lda % 4 == 0 && ldb % 4 == 0 && lda >= k &&
         ldb >= n && ldc >= n && (uintptr_t)A % 16 == 0 && (uintptr_t)B % 16 == 0 && (uintptr_t)C % 4 == 0 &&
         (long)m * lda < (1L << 31) && (long)k * ldb < (1L << 31);
}

hipError_t chain_gemm_tiles(hipStream_t st, int m, int n, int k, const float* A, long lda, const float* B, long ldb,
                            float* C, long ldc, int tri) {
  const int ntr = (m + TM - 1) / TM, ntc = (n + TN - 1) / TN;
  const long nblk = (long)((ntr + XB_R - 1) / XB_R) * ((ntc + XB_C - 1) / XB_C);
  const long grid = ((nblk + 7) / 8) * 8 * XB;  // every XCD gets the same number of block slots
  if (grid > 0x7fffffffL) return hipErrorInvalidValue;
  if (tri == 1)
    hipLaunchKernelGGL(k_chain_gemm_tiles<1>, dim3((unsigned)grid), dim3(512), 0, st, m, n, k, A, lda, B, ldb, C, ldc);
  else if (tri == 2)
    hipLaunchKernelGGL(k_chain_gemm_tiles<2>, dim3((unsigned)grid), dim3(512), 0, st, m, n, k, A, lda, B, ldb, C, ldc);
  else
    hipLaunchKernelGGL(k_chain_gemm_tiles<0>, dim3((unsigned)grid), dim3(512), 0, st, m, n, k, A, lda, B, ldb, C, ldc);
  return hipGetLastError();
}

}  // namespace cdclq
