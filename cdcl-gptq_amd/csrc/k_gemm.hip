// Bit-exact chain GEMMs for gfx950.
//
// The reference computes every GEMM through matrixmultiply 0.3.8 (src/linalg.rs:56-184). Its FMA
// micro-kernels give each C element one sequential fused-multiply-add chain over k, restarted at
// every KC = 256 panel, and fold the panel results in order: C = fma(alpha, chain_p, C'), with
// C' = beta*C for the first panel (C unread when beta == 0) and C afterwards. These kernels keep
// exactly that per-element operation sequence -- which makes them bit-identical to the
// reference -- and are free in everything else: tile shapes, thread mapping, and running the
// panels of one element in parallel (the ordered fold then happens in k_combine).
#include <cstdint>
#include <type_traits>

#include "cdclq_dev.h"
#include "kernels.h"

namespace cdclq {
namespace {

constexpr int BM = 64, BN = 64, KT = 16;

__device__ __forceinline__ float fma_t(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
__device__ __forceinline__ double fma_t(double a, double b, double c) { return __builtin_fma(a, b, c); }

// 64x64 output tile per 256-thread workgroup, 4x4 per thread, k staged through LDS in steps of
// KT (KT divides KC, so panel ends coincide with stage ends).
//
// b_tri: B is lower triangular (B[k][c] = +0 for k < c). Every product before the first nonzero
// row of the tile's columns is fma(a, +0, +0) = +0 on a chain that is still +0, and a panel made
// only of such products folds to +0, so the tile starts its k loop at its first column (rounded
// down to a stage, which keeps the panel ends on stage ends) with identical results.
template <typename T, bool SPLIT, bool LOWER>
__global__ __launch_bounds__(256) void k_gemm(int m, int n, int k, T alpha, T beta, const T* __restrict__ A,
                                              long rsa, long csa, const T* __restrict__ B, long rsb, long csb,
                                              T* __restrict__ C, long rsc, long csc, T* __restrict__ P, int b_tri) {
  __shared__ T As[KT][BM + 4];
  __shared__ T Bs[KT][BN + 4];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int i0 = blockIdx.y * BM, j0 = blockIdx.x * BN;
  if (LOWER && j0 > i0 + BM - 1) return;  // tile strictly above the diagonal
  int kbeg = 0, kend = k;
  if (SPLIT) {
    kbeg = blockIdx.z * CDCLQ_KC;
    kend = min(k, kbeg + CDCLQ_KC);
  }
  // the k loop starts at kfirst; the panel bookkeeping still counts from kbeg
  const int kfirst = b_tri ? max(kbeg, (j0 / KT) * KT) : kbeg;
  T acc[4][4], cv[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      acc[a][b] = T(0);
      cv[a][b] = T(0);
    }
  if (!SPLIT && beta != T(0)) {  // C' = beta * C (C is not read when beta == 0)
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int gi = i0 + ty * 4 + a, gj = j0 + tx * 4 + b;
        if (gi < m && gj < n) cv[a][b] = beta * C[(long)gi * rsc + (long)gj * csc];
      }
  }
  for (int k0 = kfirst; k0 < kend; k0 += KT) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = tid + 256 * q;
      int ii, kk;
      if (csa == 1) {
        kk = e & (KT - 1);
        ii = e >> 4;
      } else {
        ii = e & (BM - 1);
        kk = e >> 6;
      }
      const int gi = i0 + ii, gk = k0 + kk;
      // past the end of k: A = -0, B = +0, so the padded step fma(-0, +0, c) = c + (-0) = c is exact
      // for every c, -0 included (a chain can reach -0 through underflow)
      As[kk][ii] = (gi < m && gk < kend) ? A[(long)gi * rsa + (long)gk * csa] : T(-0.0);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = tid + 256 * q;
      int jj, kk;
      if (csb == 1) {
        jj = e & (BN - 1);
        kk = e >> 6;
      } else {
        kk = e & (KT - 1);
        jj = e >> 4;
      }
      const int gj = j0 + jj, gk = k0 + kk;
      Bs[kk][jj] = (gj < n && gk < kend) ? B[(long)gk * rsb + (long)gj * csb] : T(0);
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) {
      T av[4], bv[4];
#pragma unroll
      for (int a = 0; a < 4; ++a) av[a] = As[kk][ty * 4 + a];
#pragma unroll
      for (int b = 0; b < 4; ++b) bv[b] = Bs[kk][tx * 4 + b];
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = fma_t(av[a], bv[b], acc[a][b]);
    }
    __syncthreads();
    if (!SPLIT) {
      const int kn = k0 + KT;
      if ((kn % CDCLQ_KC) == 0 || kn >= kend) {
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            cv[a][b] = fma_t(alpha, acc[a][b], cv[a][b]);
            acc[a][b] = T(0);
          }
      }
    }
  }
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int gi = i0 + ty * 4 + a, gj = j0 + tx * 4 + b;
      if (gi < m && gj < n) {
        if (SPLIT)
          P[((long)blockIdx.z * m + gi) * n + gj] = acc[a][b];
        else
          C[(long)gi * rsc + (long)gj * csc] = cv[a][b];
      }
    }
}

// f64 chains on the matrix cores. v_mfma_f64_16x16x4f64 advances every element of a 16 x 16 block
// by four chain steps, c = fma(a3, b3, fma(a2, b2, fma(a1, b1, fma(a0, b0, c)))) in k order, each
// fma rounded once: a probe over 2^20 elements with operands spread over 2^+-60 (where the reverse
// order differs in a third of the cases) matched that sequence bit for bit. Operand layout: lane l
// supplies A[l % 16][l / 16] and B[l / 16][l % 16]; D[i][j] is register r of lane j + 16 (i % 4)
// with i = l / 16 + 4 r. Slots past the end of k hold A = -0, B = +0, whose step c + (-0) = c is
// exact. Workgroup tile BM x 64 (BM = 64, or 96 for the triangular inverse's 96-row block rows,
// which a 64-row tile would cover with a quarter of its rows idle); wave (wi, wj) owns rows
// (BM / 2) wi.., cols 32 wj.. as (BM / 32) x 2 blocks; k is staged 16 at a time through
// double-buffered LDS. Operand loads are 16-byte pairs along the contiguous dimension when the
// host found it aligned (mode 1: along k, mode 2: along i / j). Without SPLIT the chain restarts
// and is folded into C every `kfold` steps of k: KC for a GEMM, the 96-column block width for
// the Cholesky's deferred trailing updates (several blocks' updates, each folded in order).
typedef double v4d __attribute__((ext_vector_type(4)));
typedef double v2d __attribute__((ext_vector_type(2)));
constexpr int DBM = 64, DBN = 64, DKT = 16, DPAD = 16;

template <bool SPLIT, bool LOWER, int BM = DBM>
__global__ __launch_bounds__(256) void k_dgemm_mfma(int m, int n, int k, double alpha, double beta,
                                                    const double* __restrict__ A, long rsa, long csa, int amode,
                                                    const double* __restrict__ B, long rsb, long csb, int bmode,
                                                    double* __restrict__ C, long rsc, long csc, double* __restrict__ P,
                                                    int b_tri, int kfold) {
  static_assert(BM == 64 || BM == 96, "64- or 96-row tiles");
  constexpr int WR = BM / 2;        // rows per wave
  constexpr int NBI = WR / 16;      // 16-row blocks per wave
  constexpr int QA = BM * DKT / 512;  // A pairs per thread and stage
  constexpr int PA = BM / 2;        // A pairs per k row (mode 2)
  __shared__ double As[2][DKT][BM + DPAD];   // As[.][k][i]
  __shared__ double Bs[2][DKT][DBN + DPAD];  // Bs[.][k][j]
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wi = wv >> 1, wj = wv & 1;
  const int i0 = blockIdx.y * BM, j0 = blockIdx.x * DBN;
  if (LOWER && j0 > i0 + BM - 1) return;  // tile strictly above the diagonal
  int kbeg = 0, kend = k;
  if (SPLIT) {
    kbeg = blockIdx.z * CDCLQ_KC;
    kend = min(k, kbeg + CDCLQ_KC);
  }
  const int kfirst = b_tri ? max(kbeg, (j0 / DKT) * DKT) : kbeg;
  v2d ra[QA], rb[2];
  // pair p = tid + 256 q of the A tile (BM x 16) / B tile (16 x 64); 2 doubles each
  auto a_at = [&](int i, int kk) -> double {
    return (i < m && kk < kend) ? A[(long)i * rsa + (long)kk * csa] : -0.0;
  };
  auto b_at = [&](int kk, int j) -> double {
    return (kk < kend && j < n) ? B[(long)kk * rsb + (long)j * csb] : 0.0;
  };
  auto gload = [&](int k0) {
#pragma unroll
    for (int q = 0; q < QA; ++q) {
      const int pr = tid + 256 * q;
      if (amode == 2) {  // along i
        const int kk = pr / PA, i = (pr % PA) * 2, gi = i0 + i, gk = k0 + kk;
        if (gi + 1 < m && gk < kend)
          ra[q] = *reinterpret_cast<const v2d*>(A + (long)gi * rsa + (long)gk * csa);
        else
          ra[q] = v2d{a_at(gi, gk), a_at(gi + 1, gk)};
      } else {  // along k (vector when amode == 1)
        const int i = pr >> 3, kk = (pr & 7) * 2, gi = i0 + i, gk = k0 + kk;
        if (amode == 1 && gi < m && gk + 1 < kend)
          ra[q] = *reinterpret_cast<const v2d*>(A + (long)gi * rsa + (long)gk * csa);
        else
          ra[q] = v2d{a_at(gi, gk), a_at(gi, gk + 1)};
      }
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int pr = tid + 256 * q;
      if (bmode == 2) {  // along j
        const int kk = pr >> 5, j = (pr & 31) * 2, gj = j0 + j, gk = k0 + kk;
        if (gj + 1 < n && gk < kend)
          rb[q] = *reinterpret_cast<const v2d*>(B + (long)gk * rsb + (long)gj * csb);
        else
          rb[q] = v2d{b_at(gk, gj), b_at(gk, gj + 1)};
      } else {  // along k (vector when bmode == 1)
        const int j = pr >> 3, kk = (pr & 7) * 2, gj = j0 + j, gk = k0 + kk;
        if (bmode == 1 && gj < n && gk + 1 < kend)
          rb[q] = *reinterpret_cast<const v2d*>(B + (long)gk * rsb + (long)gj * csb);
        else
          rb[q] = v2d{b_at(gk, gj), b_at(gk + 1, gj)};
      }
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int q = 0; q < QA; ++q) {
      const int pr = tid + 256 * q;
      if (amode == 2) {
        const int kk = pr / PA, i = (pr % PA) * 2;
        As[buf][kk][i] = ra[q].x;
        As[buf][kk][i + 1] = ra[q].y;
      } else {
        const int i = pr >> 3, kk = (pr & 7) * 2;
        As[buf][kk][i] = ra[q].x;
        As[buf][kk + 1][i] = ra[q].y;
      }
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int pr = tid + 256 * q;
      if (bmode == 2) {
        const int kk = pr >> 5, j = (pr & 31) * 2;
        Bs[buf][kk][j] = rb[q].x;
        Bs[buf][kk][j + 1] = rb[q].y;
      } else {
        const int j = pr >> 3, kk = (pr & 7) * 2;
        Bs[buf][kk][j] = rb[q].x;
        Bs[buf][kk + 1][j] = rb[q].y;
      }
    }
  };
  v4d acc[NBI][2], cv[NBI][2];
#pragma unroll
  for (int bi = 0; bi < NBI; ++bi)
#pragma unroll
    for (int bj = 0; bj < 2; ++bj)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        acc[bi][bj][r] = 0.0;
        cv[bi][bj][r] = 0.0;
        if (!SPLIT && beta != 0.0) {
          const int gi = i0 + WR * wi + 16 * bi + (lane >> 4) + 4 * r, gj = j0 + 32 * wj + 16 * bj + (lane & 15);
          if (gi < m && gj < n) cv[bi][bj][r] = beta * C[(long)gi * rsc + (long)gj * csc];
        }
      }
  const int nst = kend > kfirst ? (kend - kfirst + DKT - 1) / DKT : 0;
  if (nst > 0) {
    gload(kfirst);
    lstore(0);
    __syncthreads();
  }
  for (int s = 0; s < nst; ++s) {
    const int buf = s & 1, k0 = kfirst + s * DKT;
    if (s + 1 < nst) gload(k0 + DKT);
#pragma unroll
    for (int k4 = 0; k4 < DKT; k4 += 4) {
      double a[NBI], b[2];
#pragma unroll
      for (int x = 0; x < NBI; ++x) a[x] = As[buf][k4 + (lane >> 4)][WR * wi + 16 * x + (lane & 15)];
#pragma unroll
      for (int x = 0; x < 2; ++x) b[x] = Bs[buf][k4 + (lane >> 4)][32 * wj + 16 * x + (lane & 15)];
#pragma unroll
      for (int bi = 0; bi < NBI; ++bi)
#pragma unroll
        for (int bj = 0; bj < 2; ++bj)
          acc[bi][bj] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[bi], b[bj], acc[bi][bj], 0, 0, 0);
    }
    if (s + 1 < nst) lstore(buf ^ 1);
    __syncthreads();
    if (!SPLIT) {
      const int kn = k0 + DKT;
      if ((kn % kfold) == 0 || kn >= kend) {
#pragma unroll
        for (int bi = 0; bi < NBI; ++bi)
#pragma unroll
          for (int bj = 0; bj < 2; ++bj)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              cv[bi][bj][r] = __builtin_fma(alpha, acc[bi][bj][r], cv[bi][bj][r]);
              acc[bi][bj][r] = 0.0;
            }
      }
    }
  }
#pragma unroll
  for (int bi = 0; bi < NBI; ++bi)
#pragma unroll
    for (int bj = 0; bj < 2; ++bj)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int gi = i0 + WR * wi + 16 * bi + (lane >> 4) + 4 * r, gj = j0 + 32 * wj + 16 * bj + (lane & 15);
        if (gi < m && gj < n) {
          if (SPLIT)
            P[((long)blockIdx.z * m + gi) * n + gj] = acc[bi][bj][r];
          else
            C[(long)gi * rsc + (long)gj * csc] = cv[bi][bj][r];
        }
      }
}

// Pipelined f64 chain GEMM for the factorisation's large products (same per-element sequence as
// k_dgemm_mfma: chains of v_mfma_f64_16x16x4f64 restarted and folded every `kfold` steps of k).
// Requirements (checked by the host): A rows run along k (A[i][k], k contiguous); B either along
// k (BT: B[k][j] = Bt[j][k]) or along j (B[k][j]); every row start 16-byte aligned; k, the k range
// of every tile and kfold multiples of DMK; n even when B runs along j. Workgroup tile BM x 128
// (BM = 128: the Cholesky's trailing updates; 64: its left-looking block-column updates; 96: the
// inverse's block rows), BM / 32 x 2 waves,
// wave (wr, wc) owning rows 32 wr .. +31 and columns 64 wc .. +63 as 2 x 4 blocks of 16 x 16.
// Stages of DMK = 16 k are filled with global_load_lds_dwordx4 into a ring of DMS, DMS - 1 stages
// in flight, one bare barrier per stage. A k-contiguous operand is staged as [row][8 slots of 16 B]
// with k-pair p of row r in slot p ^ ((r >> 1) & 7), so the 16 rows a matrix-core fragment reads
// at one k fall on distinct banks; B along j is staged as [k][128]. Rows and columns past the
// matrix are read from clamped addresses and only reach outputs that are never stored. b_tri
// (B lower triangular, beta == 0) starts each tile's k loop at its first column, as in k_dgemm_mfma.
constexpr int DMK = 16, DMS = 4, DMN = 128;
constexpr long kDmmWide = 512;  // 128-row tiles from two full rounds of one workgroup per CU (256 CUs)
template <int BM, bool BT, bool SPLIT>
__global__ __launch_bounds__(BM * 4) void k_dmm(int m, int n, int k, double alpha, double beta,
                                               const double* __restrict__ A, long lda, const double* __restrict__ B,
                                               long ldb, double* __restrict__ C, long ldc, double* __restrict__ P,
                                               int kfold, int lower, int b_tri) {
  constexpr int NW = BM / 16;                    // waves: BM / 32 row groups x 2 column groups
  constexpr int ABYTES = BM * DMK * 8;           // A part of a stage
  constexpr int SBYTES = ABYTES + DMN * DMK * 8;  // stage
  constexpr int NI = SBYTES / 1024;              // 1 KB load instructions per stage
  constexpr int LMAX = (NI + NW - 1) / NW, LMIN = NI / NW;
  __shared__ double R[DMS * SBYTES / 8];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = wv >> 1, wc = wv & 1;
  const int i0 = blockIdx.y * BM, j0 = blockIdx.x * DMN;
  if (lower && j0 > i0 + BM - 1) return;  // tile strictly above the diagonal
  int kbeg = 0, kend = k;
  if (SPLIT) {
    kbeg = blockIdx.z * CDCLQ_KC;
    kend = min(k, kbeg + CDCLQ_KC);
  }
  const int kfirst = b_tri ? max(kbeg, (j0 / DMK) * DMK) : kbeg;
  const int nst = kend > kfirst ? (kend - kfirst) / DMK : 0;
  const int nload = (NI - wv + NW - 1) / NW;  // this wave's loads per stage (LMIN or LMAX)
  // per-lane source offsets of this wave's loads, relative to the stage's k0
  const double* src[LMAX];
  uint32_t dst[LMAX];
#pragma unroll
  for (int q = 0; q < LMAX; ++q) {
    const int ins = min(wv + NW * q, NI - 1);
    dst[q] = (uint32_t)ins * 1024u;
    if (ins < BM / 8) {  // A rows 8 ins .. +7
      const int r = 8 * ins + (lane >> 3), pr = (lane & 7) ^ ((r >> 1) & 7);
      src[q] = A + (long)min(i0 + r, m - 1) * lda + 2 * pr;
    } else if (BT) {  // Bt rows (B columns) 8 (ins - BM / 8) .. +7
      const int r = 8 * (ins - BM / 8) + (lane >> 3), pr = (lane & 7) ^ ((r >> 1) & 7);
      src[q] = B + (long)min(j0 + r, n - 1) * ldb + 2 * pr;
    } else {  // B k row ins - BM / 8, columns 2 lane, 2 lane + 1
      src[q] = B + (long)(ins - BM / 8) * ldb + min(j0 + 2 * lane, n - 2);
    }
  }
  const uint32_t lds0 = lds_offset(&R[0]);
  auto issue = [&](int st) {  // stage st (k0 = kfirst + DMK st) into ring slot st % DMS
    const long koff = (long)(kfirst + DMK * st);
    const uint32_t base = lds0 + (uint32_t)((st % DMS) * SBYTES);
#pragma unroll
    for (int q = 0; q < LMAX; ++q) {
      if (q >= nload) continue;  // uniform
      const int ins = wv + NW * q;
      const double* g = src[q];
      if (ins < BM / 8 || BT)
        g += koff;  // along k within the row
      else
        g += koff * ldb;  // k rows
      dma16_untracked(reinterpret_cast<const float*>(g), base + dst[q]);
    }
  };
  v4d acc[2][4], cv[2][4];
#pragma unroll
  for (int bi = 0; bi < 2; ++bi)
#pragma unroll
    for (int bj = 0; bj < 4; ++bj)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        acc[bi][bj][r] = 0.0;
        cv[bi][bj][r] = 0.0;
      }
  for (int st = 0; st < DMS - 1 && st < nst; ++st) issue(st);
  // Element (bi, bj, r) of a lane lies at a uniform offset from the lane's first one, so a whole
  // tile (a uniform test) loads and stores C from one address per lane.
  const bool whole = i0 + BM <= m && j0 + DMN <= n;
  const long cbase = (long)(i0 + 32 * wr + (lane >> 4)) * ldc + j0 + 64 * wc + (lane & 15);
  auto coff = [&](int bi, int bj, int r) { return (long)(16 * bi + 4 * r) * ldc + 16 * bj; };
  if (!SPLIT && beta != 0.0) {  // C' = beta * C; 1 * C is C itself
    if (whole) {
#pragma unroll
      for (int bi = 0; bi < 2; ++bi)
#pragma unroll
        for (int bj = 0; bj < 4; ++bj)
#pragma unroll
          for (int r = 0; r < 4; ++r) cv[bi][bj][r] = C[cbase + coff(bi, bj, r)];
    } else {
#pragma unroll
      for (int bi = 0; bi < 2; ++bi)
#pragma unroll
        for (int bj = 0; bj < 4; ++bj)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int gi = min(i0 + 32 * wr + 16 * bi + (lane >> 4) + 4 * r, m - 1);
            const int gj = min(j0 + 64 * wc + 16 * bj + (lane & 15), n - 1);
            cv[bi][bj][r] = C[(long)gi * ldc + gj];
          }
    }
    // one wait here (with the first stages in flight) instead of one the compiler would place at
    // every fold inside the loop, where it would also drain the stage ring
    wait_vmcnt<0>();
    if (beta != 1.0) {
#pragma unroll
      for (int bi = 0; bi < 2; ++bi)
#pragma unroll
        for (int bj = 0; bj < 4; ++bj)
#pragma unroll
          for (int r = 0; r < 4; ++r) cv[bi][bj][r] = beta * cv[bi][bj][r];
    }
  }
  // LDS element offsets (doubles) of this lane's fragment reads within a stage, for k-step 0
  int aoff[2], boff[4];
#pragma unroll
  for (int bi = 0; bi < 2; ++bi) aoff[bi] = (32 * wr + 16 * bi + (lane & 15)) * DMK;
#pragma unroll
  for (int bj = 0; bj < 4; ++bj) boff[bj] = BT ? ABYTES / 8 + (64 * wc + 16 * bj + (lane & 15)) * DMK
                                              : ABYTES / 8 + (lane >> 4) * DMN + 64 * wc + 16 * bj + (lane & 15);
  for (int st = 0; st < nst; ++st) {
    // this wave's loads of stage st have landed once at most those of the later stages in flight
    // remain; the barrier then publishes every wave's part and retires all reads of stage st - 1
    const int later = min(DMS - 2, nst - 1 - st);
    if (later >= 2) {
      if (nload == LMAX) wait_vmcnt<2 * LMAX>(); else wait_vmcnt<2 * LMIN>();
    } else if (later == 1) {
      if (nload == LMAX) wait_vmcnt<LMAX>(); else wait_vmcnt<LMIN>();
    } else {
      wait_vmcnt<0>();
    }
    __builtin_amdgcn_s_barrier();
    if (st + DMS - 1 < nst) issue(st + DMS - 1);  // into the slot of stage st - 1
    const double* S = &R[(st % DMS) * (SBYTES / 8)];
#pragma unroll
    for (int k4 = 0; k4 < DMK; k4 += 4) {
      const int kk = k4 + (lane >> 4);
      double a[2], b[4];
#pragma unroll
      for (int bi = 0; bi < 2; ++bi) {
        const int r = 32 * wr + 16 * bi + (lane & 15);
        a[bi] = S[aoff[bi] + 2 * ((kk >> 1) ^ ((r >> 1) & 7)) + (kk & 1)];
      }
#pragma unroll
      for (int bj = 0; bj < 4; ++bj) {
        if (BT) {
          const int r = 64 * wc + 16 * bj + (lane & 15);
          b[bj] = S[boff[bj] + 2 * ((kk >> 1) ^ ((r >> 1) & 7)) + (kk & 1)];
        } else {
          b[bj] = S[boff[bj] + k4 * DMN];
        }
      }
#pragma unroll
      for (int bi = 0; bi < 2; ++bi)
#pragma unroll
        for (int bj = 0; bj < 4; ++bj)
          acc[bi][bj] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[bi], b[bj], acc[bi][bj], 0, 0, 0);
    }
    if (!SPLIT) {
      const int kn = kfirst + DMK * (st + 1);
      if ((kn % kfold) == 0 || kn >= kend) {
#pragma unroll
        for (int bi = 0; bi < 2; ++bi)
#pragma unroll
          for (int bj = 0; bj < 4; ++bj)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              cv[bi][bj][r] = __builtin_fma(alpha, acc[bi][bj][r], cv[bi][bj][r]);
              acc[bi][bj][r] = 0.0;
            }
      }
    }
  }
  if (!SPLIT && whole) {
#pragma unroll
    for (int bi = 0; bi < 2; ++bi)
#pragma unroll
      for (int bj = 0; bj < 4; ++bj)
#pragma unroll
        for (int r = 0; r < 4; ++r) C[cbase + coff(bi, bj, r)] = cv[bi][bj][r];
    return;
  }
#pragma unroll
  for (int bi = 0; bi < 2; ++bi)
#pragma unroll
    for (int bj = 0; bj < 4; ++bj)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int gi = i0 + 32 * wr + 16 * bi + (lane >> 4) + 4 * r, gj = j0 + 64 * wc + 16 * bj + (lane & 15);
        if (gi < m && gj < n) {
          if (SPLIT)
            P[((long)blockIdx.z * m + gi) * n + gj] = acc[bi][bj][r];
          else
            C[(long)gi * ldc + gj] = cv[bi][bj][r];
        }
      }
}

// operand load mode for k_dgemm_mfma from the strides along k and along the other index:
// 1 = 16-byte pairs along k, 2 = pairs along the other index, 0 = scalar loads
inline int dmode(const double* p, long k_stride, long other_stride) {
  if ((uintptr_t)p % 16 != 0) return 0;
  if (k_stride == 1 && other_stride % 2 == 0) return 1;
  if (other_stride == 1 && k_stride % 2 == 0) return 2;
  return 0;
}

// Ordered fold of per-panel chains: C = fma(alpha, P_p, C') for p = 0, 1, ... (see file header).
template <typename T>
__global__ __launch_bounds__(256) void k_combine(int m, int n, int np, T alpha, T beta, const T* __restrict__ P,
                                                 T* __restrict__ C, long rsc, long csc) {
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long)m * n) return;
  const int i = (int)(idx / n), j = (int)(idx % n);
  T* c = C + (long)i * rsc + (long)j * csc;
  T cv = beta != T(0) ? beta * *c : T(0);
  const T* src = P + (long)i * n + j;
  const long ps = (long)m * n;
  int p = 0;
  for (; p + 8 <= np; p += 8) {  // 8 panel loads in flight, folded in order
    T v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = src[(long)(p + u) * ps];
#pragma unroll
    for (int u = 0; u < 8; ++u) cv = fma_t(alpha, v[u], cv);
  }
  for (; p < np; ++p) cv = fma_t(alpha, src[(long)p * ps], cv);
  *c = cv;
}

}  // namespace

size_t gemm_partials_elems(int m, int n, int k) {
  const size_t np = (size_t)((k + CDCLQ_KC - 1) / CDCLQ_KC);
  return np * (size_t)m * (size_t)n;
}

template <typename T>
hipError_t gemm_chain(hipStream_t st, int m, int n, int k, T alpha, T beta, const T* A, long rsa, long csa,
                      const T* B, long rsb, long csb, T* C, long rsc, long csc, bool lower, T* partials,
                      bool b_lower_tri) {
  // the zero-prefix skip relies on C starting at +0, i.e. beta == 0
  const int bt = (b_lower_tri && beta == T(0)) ? 1 : 0;
  if (m <= 0 || n <= 0) return hipSuccess;
  if (k <= 0) {
    // k == 0: C = beta * C, or 0 when beta == 0, untouched when beta == 1 (src/linalg.rs:79-92)
    if (beta != T(1)) {
      hipLaunchKernelGGL((k_combine<T>), dim3((unsigned)(((long)m * n + 255) / 256)), dim3(256), 0, st, m, n, 0, alpha,
                         beta, (const T*)nullptr, C, rsc, csc);
    }
    return hipGetLastError();
  }
  const dim3 grid((n + BN - 1) / BN, (m + BM - 1) / BM, 1);
  const int np = (k + CDCLQ_KC - 1) / CDCLQ_KC;
  if constexpr (std::is_same<T, double>::value) {
    static_assert(DBM == BM && DBN == BN, "same tiling as the VALU kernel");
    const int am = dmode(A, csa, rsa), bm = dmode(B, rsb, csb);
    if (np > 1 && partials != nullptr && !lower) {
      dim3 g3 = grid;
      g3.z = np;
      if (m == 96) {  // the triangular inverse's block rows: one 96-row tile
        g3.y = 1;
        hipLaunchKernelGGL((k_dgemm_mfma<true, false, 96>), g3, dim3(256), 0, st, m, n, k, alpha, beta, A, rsa,
                           csa, am, B, rsb, csb, bm, C, rsc, csc, partials, bt, CDCLQ_KC);
      } else {
        hipLaunchKernelGGL((k_dgemm_mfma<true, false>), g3, dim3(256), 0, st, m, n, k, alpha, beta, A, rsa, csa,
                           am, B, rsb, csb, bm, C, rsc, csc, partials, bt, CDCLQ_KC);
      }
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
      hipLaunchKernelGGL((k_combine<T>), dim3((unsigned)(((long)m * n + 255) / 256)), dim3(256), 0, st, m, n, np,
                         alpha, beta, (const T*)partials, C, rsc, csc);
      return hipGetLastError();
    }
    if (lower)
      hipLaunchKernelGGL((k_dgemm_mfma<false, true>), grid, dim3(256), 0, st, m, n, k, alpha, beta, A, rsa, csa,
                         am, B, rsb, csb, bm, C, rsc, csc, (double*)nullptr, bt, CDCLQ_KC);
    else
      hipLaunchKernelGGL((k_dgemm_mfma<false, false>), grid, dim3(256), 0, st, m, n, k, alpha, beta, A, rsa, csa,
                         am, B, rsb, csb, bm, C, rsc, csc, (double*)nullptr, bt, CDCLQ_KC);
    return hipGetLastError();
  }
  if (np > 1 && partials != nullptr && !lower) {
    dim3 g3 = grid;
    g3.z = np;
    hipLaunchKernelGGL((k_gemm<T, true, false>), g3, dim3(256), 0, st, m, n, k, alpha, beta, A, rsa, csa, B, rsb,
                       csb, C, rsc, csc, partials, bt);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((k_combine<T>), dim3((unsigned)(((long)m * n + 255) / 256)), dim3(256), 0, st, m, n, np, alpha,
                       beta, (const T*)partials, C, rsc, csc);
    return hipGetLastError();
  }
  if (lower)
    hipLaunchKernelGGL((k_gemm<T, false, true>), grid, dim3(256), 0, st, m, n, k, alpha, beta, A, rsa, csa, B,
                       rsb, csb, C, rsc, csc, (T*)nullptr, bt);
  else
    hipLaunchKernelGGL((k_gemm<T, false, false>), grid, dim3(256), 0, st, m, n, k, alpha, beta, A, rsa, csa, B,
                       rsb, csb, C, rsc, csc, (T*)nullptr, bt);
  return hipGetLastError();
}

namespace {
bool aligned16(const void* p) { return (uintptr_t)p % 16 == 0; }
}  // namespace

hipError_t chol_update(hipStream_t st, int m, int n, int k, const double* P, long ldp, double* C, long ldc) {
  if (m <= 0 || n <= 0 || k <= 0) return hipSuccess;
  if (n >= 64 && m >= 2 && k % DMK == 0 && aligned16(P) && ldp % 2 == 0) {  // the pipelined tiles
    // 64-row tiles (twice the workgroups) where 128-row ones would fill the device less than twice:
    // the left-looking updates and a period's main-stream pass
    if ((long)((n + DMN - 1) / DMN) * ((m + 127) / 128) < kDmmWide) {
      const dim3 grid((n + DMN - 1) / DMN, (m + 63) / 64, 1);
      hipLaunchKernelGGL((k_dmm<64, true, false>), grid, dim3(256), 0, st, m, n, k, -1.0, 1.0, P, ldp, P, ldp, C,
                         ldc, (double*)nullptr, 96, 1, 0);
    } else {
      const dim3 grid((n + DMN - 1) / DMN, (m + 127) / 128, 1);
      hipLaunchKernelGGL((k_dmm<128, true, false>), grid, dim3(512), 0, st, m, n, k, -1.0, 1.0, P, ldp, P, ldp, C,
                         ldc, (double*)nullptr, 96, 1, 0);
    }
    return hipGetLastError();
  }
  const dim3 grid((n + DBN - 1) / DBN, (m + DBM - 1) / DBM, 1);
  const int pm = dmode(P, 1, ldp);  // both operands run along k = the rows of P
  hipLaunchKernelGGL((k_dgemm_mfma<false, true>), grid, dim3(256), 0, st, m, n, k, -1.0, 1.0, P, ldp, 1L, pm, P,
                     1L, ldp, pm, C, ldc, 1L, (double*)nullptr, 0, 96);
  return hipGetLastError();
}

bool inv_gemm_eligible(int m, int n, int k, const double* A, long lda, const double* B, long ldb) {
  return m > 0 && m <= 96 && n >= 2 && n % 2 == 0 && k > 0 && k % DMK == 0 && aligned16(A) && lda % 2 == 0 &&
         aligned16(B) && ldb % 2 == 0;
}

hipError_t inv_gemm(hipStream_t st, int m, int n, int k, double alpha, const double* A, long lda, const double* B,
                    long ldb, double* C, long ldc) {
  if (m <= 0 || n <= 0 || k <= 0) return hipSuccess;
  if (!inv_gemm_eligible(m, n, k, A, lda, B, ldb) || k > CDCLQ_KC) return hipErrorInvalidValue;
  const dim3 grid((n + DMN - 1) / DMN, 1, 1);
  hipLaunchKernelGGL((k_dmm<96, false, false>), grid, dim3(384), 0, st, m, n, k, alpha, 0.0, A, lda, B, ldb, C, ldc,
                     (double*)nullptr, CDCLQ_KC, 0, 0);
  return hipGetLastError();
}

bool inv_acc_eligible(int m, int n, int k, const double* A, long lda, const double* B, long ldb) {
  return m > 0 && n >= 2 && n % 2 == 0 && k > 0 && k <= CDCLQ_KC && k % DMK == 0 && aligned16(A) && lda % 2 == 0 &&
         aligned16(B) && ldb % 2 == 0;
}

hipError_t inv_acc(hipStream_t st, int m, int n, int k, const double* A, long lda, const double* B, long ldb,
                   double* C, long ldc) {
  if (m <= 0 || n <= 0 || k <= 0) return hipSuccess;
  if (!inv_acc_eligible(m, n, k, A, lda, B, ldb)) return hipErrorInvalidValue;
  if (m > 96 && (long)((n + DMN - 1) / DMN) * ((m + 127) / 128) >= kDmmWide) {  // the rows below a panel
    const dim3 grid((n + DMN - 1) / DMN, (m + 127) / 128, 1);
    hipLaunchKernelGGL((k_dmm<128, false, false>), grid, dim3(512), 0, st, m, n, k, 1.0, 1.0, A, lda, B, ldb, C, ldc,
                       (double*)nullptr, CDCLQ_KC, 0, 0);
  } else if (m > 96) {  // a panel whose 128-row tiles would fill the device less than twice
    const dim3 grid((n + DMN - 1) / DMN, (m + 63) / 64, 1);
    hipLaunchKernelGGL((k_dmm<64, false, false>), grid, dim3(256), 0, st, m, n, k, 1.0, 1.0, A, lda, B, ldb, C, ldc,
                       (double*)nullptr, CDCLQ_KC, 0, 0);
  } else {  // one block row
    const dim3 grid((n + DMN - 1) / DMN, 1, 1);
    hipLaunchKernelGGL((k_dmm<96, false, false>), grid, dim3(384), 0, st, m, n, k, 1.0, 1.0, A, lda, B, ldb, C, ldc,
                       (double*)nullptr, CDCLQ_KC, 0, 0);
  }
  return hipGetLastError();
}

template hipError_t gemm_chain<float>(hipStream_t, int, int, int, float, float, const float*, long, long, const float*,
                                      long, long, float*, long, long, bool, float*, bool);
template hipError_t gemm_chain<double>(hipStream_t, int, int, int, double, double, const double*, long, long,
                                       const double*, long, long, double*, long, long, bool, double*, bool);

}  // namespace cdclq
