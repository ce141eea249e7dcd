// f64 factorisation kernels: U with H^-1 = U^T U (src/linalg.rs:200-375, src/engine.rs:320-342).
//
// Blocking follows the reference's NB = 96 block columns because the block boundaries fix the
// floating-point operation sequence of every element:
//   * diagonal block: unblocked left-looking Cholesky with separate multiply/subtract roundings;
//   * panel solve below it: for each column j of the block, s = a_ij - sum_t x_t l_jt in t order;
//   * trailing update: a_ij = fma(-1, chain_t(p_it p_jt), a_ij) per block (k_gemm.hip, lower tiles);
//   * inverse of every diagonal block by columns (mul/add roundings), then per block row two
//     chained GEMMs (k_gemm.hip).
// The panel solve gives a row four lanes (its columns interleaved over them): column t is
// finalised at step t and immediately subtracted from every later column, which performs the
// reference's per-element subtraction sequence in the same order.
#include "cdclq_dev.h"
#include "kernels.h"

namespace cdclq {
namespace {

constexpr int NBC = 96;  // src/linalg.rs:202, :285

// hp = perm(H) in f64, dead diagonal -> 1, + damp on the diagonal; h32 = (f32)hp; a = flip(hp).
__global__ __launch_bounds__(256) void k_build_flipped(int n, const float* __restrict__ h,
                                                       const uint32_t* __restrict__ perm, double damp_val,
                                                       double* __restrict__ a, float* __restrict__ h32) {
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long)n * n) return;
  const int p = (int)(idx / n), q = (int)(idx % n);
  double v = (double)h[(long)perm[p] * n + perm[q]];
  if (p == q) {
    if (v == 0.0) v = 1.0;
    v = v + damp_val;
  }
  h32[idx] = (float)v;
  a[(long)(n - 1 - p) * n + (n - 1 - q)] = v;
}

__global__ __launch_bounds__(256) void k_build_flipped_f64(int n, const double* __restrict__ h, double* __restrict__ a) {
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  const long nn = (long)n * n;
  if (idx >= nn) return;
  a[idx] = h[nn - 1 - idx];
}

// Unblocked factorisation of the diagonal block (src/linalg.rs:209-229). The reference works by
// columns (left-looking): d = a_jj - sum_{t<j} l_jt l_jt, l_jj = sqrt(d), then
// l_ij = (a_ij - sum_{t<j} l_it l_jt) / l_jj, every term a separate multiply and subtract in t
// order. Applying the subtraction of column t to the whole trailing triangle as soon as column t
// is final (right-looking) performs exactly the same operations on every element in the same
// order, with the trailing triangle updated in parallel.
//
// One wavefront, no barriers: the lanes form an 8 x 8 grid and element (i, j) lives in register
// slot (i / 8, j / 8) of lane (i % 8, j % 8) for the whole factorisation (2-D cyclic, so every
// step's trailing triangle is spread over all lanes; 12 x 12 slots, the lower 78 of them used).
// Step t: the lanes holding column t publish it (updated through step t - 1) to LDS, every lane
// divides one or two of its entries by l_tt and publishes column t of L, and every lane applies
// that column to its slots. LDS accesses of one wavefront complete in order, so a read issued
// after a write sees it. Slot columns left of t's are skipped; the registers of finished columns
// (and of the upper triangle) that are still updated are never read again.
// Step t first updates the slot column that holds column t + 1 and publishes it, then runs
// column t + 1's pivot (read from the register of the lane that holds it), square root and
// divisions, applies column t to the rest of its slots, and stores column t + 1 of L and reads it
// back for step t + 1. Every element still receives the same operations in the same order. The
// block's time is this per-column chain (the square root, the divisions, two LDS round trips):
// spreading the slots over four wavefronts measured no faster. A failing pivot is recorded (the
// first one) and reported at the end; the remaining steps run on with values that are discarded
// with the error.
constexpr int DGL = 8;           // lane grid side
constexpr int DSL = NBC / DGL;   // row / column slots per lane

__device__ __forceinline__ double readlane_f64(double v, int l) {  // l uniform
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_readlane((int)(b & 0xffffffffLL), l);
  const int hi = __builtin_amdgcn_readlane((int)(b >> 32), l);
  return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

__global__ __launch_bounds__(64) void k_chol_diag(int n, double* __restrict__ a, int k, int kb, int* status,
                                                  double* pivot) {
  __shared__ double pre[NBC + 64];  // column t with all earlier columns applied; + a discard slot per lane
  __shared__ double col[NBC + 32];  // column t of L (zero above row t); + discard slots for lanes 32..63
  if (*status) return;
  const int lane = threadIdx.x, tr = lane >> 3, tc = lane & 7;
  double v[DSL][DSL];
#pragma unroll
  for (int r = 0; r < DSL; ++r)
#pragma unroll
    for (int c = 0; c <= r; ++c) {
      const int i = DGL * r + tr, j = DGL * c + tc;
      v[r][c] = a[(long)(k + min(i, kb - 1)) * n + k + min(j, kb - 1)];
    }
  int fail_t = -1;
  double fail_d = 0.0;
  double c0 = 0.0, c1 = 0.0;  // this lane's entries (rows lane, lane + 64) of the latest column of L
  // column tn (slot column ctn, lanes tc == ltn) to LDS; the other lanes write their discard slot
  auto publish = [&](int ctn, int ltn) {
    const bool own = tc == ltn;
#pragma unroll
    for (int r = ctn; r < DSL; ++r) pre[own ? DGL * r + tr : NBC + lane] = v[r][ctn];
  };
  // pivot d of column tn (read by the caller from the register of its owner lane, so that the
  // square root starts without an LDS round trip), its square root and the divided column of L
  // into LDS; both dividends are read before the square root (values past kb are computed from
  // clamped reads and never stored)
  auto divide = [&](int tn, double d) {
    const double p0 = pre[lane], p1 = pre[min(lane + 64, NBC - 1)];
    const bool rec = (!(d > 0.0) || !isfinite(d)) && fail_t < 0 && tn < kb;
    fail_d = rec ? d : fail_d;
    fail_t = rec ? tn : fail_t;
    const double ltt = sqrt(d);
    const double q0 = p0 / ltt, q1 = p1 / ltt;
    c0 = (lane == tn) ? ltt : ((lane > tn && lane < kb) ? q0 : 0.0);
    c1 = (lane + 64 == tn) ? ltt : ((lane + 64 > tn && lane + 64 < kb) ? q1 : 0.0);
    col[lane] = c0;
    col[lane < 32 ? lane + 64 : NBC + lane - 32] = c1;
  };
  auto store_col = [&](int tn) {
    if (lane >= tn && lane < kb) a[(long)(k + lane) * n + k + tn] = c0;
    if (lane + 64 >= tn && lane + 64 < kb) a[(long)(k + lane + 64) * n + k + tn] = c1;
  };
  double ci[DSL], cj[DSL];  // column t of L at rows DGL q + tr (ci) and DGL q + tc (cj)
  publish(0, 0);
  divide(0, readlane_f64(v[0][0], 0));
  store_col(0);
#pragma unroll
  for (int q = 0; q < DSL; ++q) {
    ci[q] = col[DGL * q + tr];
    cj[q] = col[DGL * q + tc];
  }
#pragma unroll
  for (int ct = 0; ct < DSL; ++ct) {
    const int nlt = min(DGL, kb - DGL * ct);  // uniform; <= 0 past the block
    for (int lt = 0; lt < nlt; ++lt) {
      const int t = DGL * ct + lt;  // ci / cj hold column t of L
      if (lt + 1 < DGL) {           // column t + 1 lives in slot column ct
#pragma unroll
        for (int r = ct; r < DSL; ++r) v[r][ct] = v[r][ct] - ci[r] * cj[ct];
        publish(ct, lt + 1);
        divide(t + 1, readlane_f64(v[ct][ct], (DGL + 1) * (lt + 1)));  // l_{t+1,t+1}: lane 9 ((t + 1) % 8)
#pragma unroll
        for (int r = ct + 1; r < DSL; ++r)
#pragma unroll
          for (int c = ct + 1; c <= r; ++c) v[r][c] = v[r][c] - ci[r] * cj[c];
        if (t + 1 < kb) store_col(t + 1);
#pragma unroll
        for (int q = ct; q < DSL; ++q) {
          ci[q] = col[DGL * q + tr];
          cj[q] = col[DGL * q + tc];
        }
      } else if (ct + 1 < DSL) {  // column t + 1 starts slot column ct + 1; slot column ct is finished
#pragma unroll
        for (int r = ct + 1; r < DSL; ++r) v[r][ct + 1] = v[r][ct + 1] - ci[r] * cj[ct + 1];
        publish(ct + 1, 0);
        divide(t + 1, readlane_f64(v[ct + 1][ct + 1], 0));
#pragma unroll
        for (int r = ct + 2; r < DSL; ++r)
#pragma unroll
          for (int c = ct + 2; c <= r; ++c) v[r][c] = v[r][c] - ci[r] * cj[c];
        if (t + 1 < kb) store_col(t + 1);
#pragma unroll
        for (int q = ct + 1; q < DSL; ++q) {
          ci[q] = col[DGL * q + tr];
          cj[q] = col[DGL * q + tc];
        }
      }
    }
  }
  if (lane == 0 && fail_t >= 0) {
    *status = k + fail_t + 1;
    *pivot = fail_d;
  }
}

// Panel solve X L_kk^T = A_panel for all rows below the block (src/linalg.rs:233-241): for each
// row, x_j = (a_j - sum_{t<j} x_t l_jt) / l_jj, every product and difference rounded separately,
// t ascending. Four lanes per row, 16 rows per wavefront: lane 4 r + g holds columns
// j = 4 q + g (q < 24) of row r, so the columns still open at any step are spread evenly over the
// row's lanes. Step t: the lane holding column t divides it by l_tt (all lanes run the division;
// the others' quotients are discarded), a quad permutation hands the quotient to the row's four
// lanes, and each lane subtracts x_t l_jt from its columns j > t. Column j thus receives the
// reference's subtractions in the reference's order (right-looking instead of a dot product per
// column), and finished columns are never touched again. The lower part of L_kk is staged in LDS
// as LP[t][g][q] = l_{4q+g, t} (zero on and above the diagonal and past the block), so a lane reads
// the factors of its columns for step t as consecutive pairs; the diagonal is staged separately.
constexpr int PQ = NBC / 4;  // columns per lane

template <int C>
__device__ __forceinline__ double quad_bcast(double v) {  // lane 4 r + C's value to lanes 4 r .. 4 r + 3
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_mov_dpp((int)(b & 0xffffffffLL), C * 85, 0xf, 0xf, false);
  const int hi = __builtin_amdgcn_mov_dpp((int)(b >> 32), C * 85, 0xf, 0xf, false);
  return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

// Step T of the panel solve for one lane (see k_chol_panel); templated on T so that every index
// into the lane's columns is a constant. On entry `xo` is column T divided by its pivot (valid in
// the lanes holding column T), `cur` this step's factors l_{4q+g, T} (q >= T / 4) and `dn` the
// next pivot l_{T+1, T+1}, read from LDS a step ahead so that their latency hides behind the
// previous step. The step finalises column T, updates column T + 1 first and starts its division,
// so that the division's latency overlaps the step's other updates (a division started for a
// column past the block, T + 1 = kb, divides by the pivot 1 staged there and is never used).
template <int T>
__device__ __forceinline__ void chol_panel_step(double (&s)[PQ], const double (&cur)[PQ], double xo, double dn,
                                                int g, int kb, const double* lp0, const double* dg) {
  constexpr int qt = T >> 2, gt = T & 3, T1 = T + 1, q1 = T1 >> 2;
  if (T >= kb) return;  // uniform; a real branch, which also bounds the scheduler's reach
  double nxt[PQ], dn2 = 1.0;
  if constexpr (T1 < NBC) {
    const double* lp = lp0 + (T1 * 4 + g) * PQ;  // LP[T + 1][g][.]
#pragma unroll
    for (int q = q1; q < PQ; ++q) nxt[q] = lp[q];
    if constexpr (T1 + 1 < NBC) dn2 = dg[T1 + 1];
  }
  const double x = quad_bcast<gt>(xo);
  double up = s[qt] - x * cur[qt];
  asm volatile("" : "+v"(up));  // computed in every lane, so that the select below is no branch
  const double keep = s[qt];
  const double upd = g > gt ? up : keep;
  s[qt] = g == gt ? xo : upd;
  if constexpr (T1 < NBC) {
    if constexpr (q1 != qt) s[q1] = s[q1] - x * cur[q1];
    double xo1 = s[q1] / dn;
    asm volatile("" : "+v"(xo1));  // the division starts here, before the step's other updates
#pragma unroll
    for (int q = q1 + 1; q < PQ; ++q) s[q] = s[q] - x * cur[q];
    chol_panel_step<T1>(s, nxt, xo1, dn2, g, kb, lp0, dg);
  }
}

__global__ __launch_bounds__(256) void k_chol_panel(int n, double* __restrict__ a, int k, int kb,
                                                    const int* status) {
  __shared__ double LP[NBC][4][PQ];
  __shared__ double dg[NBC];
  if (*status) return;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  {  // stage the block with all of a thread's loads in flight at once (clamped addresses)
    constexpr int PER = NBC * NBC / 256;
    double v[PER];
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const int x = tid + 256 * e, j = x / NBC, t = x % NBC;
      v[e] = a[(long)(k + min(j, kb - 1)) * n + k + min(t, kb - 1)];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const int x = tid + 256 * e, j = x / NBC, t = x % NBC;
      LP[t][j & 3][j >> 2] = (t < j && j < kb) ? v[e] : 0.0;
      if (t == j) dg[t] = t < kb ? v[e] : 1.0;
    }
  }
  __syncthreads();
  const int g = lane & 3;
  const int row = k + kb + (blockIdx.x * 4 + wv) * 16 + (lane >> 2);
  const double* src = a + (long)min(row, n - 1) * n + k;  // rows past the end: computed, never stored
  double s[PQ];
#pragma unroll
  for (int q = 0; q < PQ; ++q) s[q] = src[min(4 * q + g, kb - 1)];
  double f0[PQ];
#pragma unroll
  for (int q = 0; q < PQ; ++q) f0[q] = LP[0][g][q];
  chol_panel_step<0>(s, f0, s[0] / dg[0], dg[1], g, kb, &LP[0][0][0], dg);
  if (row < n) {
    double* dst = a + (long)row * n + k;
#pragma unroll
    for (int q = 0; q < PQ; ++q)
      if (4 * q + g < kb) dst[4 * q + g] = s[q];
  }
}

// Explicit inverse of every NB x NB diagonal block of L (src/linalg.rs:291-306), one column per
// thread: yii_cc = 1/l_cc, yii_ic = -(sum_{t=c}^{i-1} l_it yii_tc) / l_ii with mul/add roundings.
__global__ __launch_bounds__(128) void k_trinv_diag(int n, const double* __restrict__ l, double* __restrict__ y,
                                                    const int* status) {
  __shared__ double Y[NBC][NBC + 1];
  if (*status) return;
  const int s = blockIdx.x * NBC;
  const int w = min(NBC, n - s);
  const int c = threadIdx.x;
  if (c < w) {
    Y[c][c] = 1.0 / l[(long)(s + c) * n + s + c];
    for (int i = c + 1; i < w; ++i) {
      double acc = 0.0;
      const double* li = l + (long)(s + i) * n + s;
      for (int t = c; t < i; ++t) acc = acc + li[t] * Y[t][c];
      Y[i][c] = -acc / li[i];
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < w * w; e += blockDim.x) {
    const int i = e / w, j = e % w;
    if (j <= i) y[(long)(s + i) * n + s + j] = Y[i][j];
  }
}

// U_ij = (f32) y[n-1-i][n-1-j] for j >= i, 0 below (src/linalg.rs:368-373).
__global__ __launch_bounds__(256) void k_scatter_u(int n, const double* __restrict__ y, float* __restrict__ u) {
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long)n * n) return;
  const int i = (int)(idx / n), j = (int)(idx % n);
  u[idx] = (j >= i) ? (float)y[(long)(n - 1 - i) * n + (n - 1 - j)] : 0.0f;
}

__global__ __launch_bounds__(256) void k_fill_zero_f64(double* p, long count) {
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx < count) p[idx] = 0.0;
}

inline unsigned nblk(long count) { return (unsigned)((count + 255) / 256); }

}  // namespace

hipError_t build_flipped(hipStream_t st, int n, const float* h, const uint32_t* perm, double damp_val, double* a,
                         float* h32) {
  hipLaunchKernelGGL(k_build_flipped, dim3(nblk((long)n * n)), dim3(256), 0, st, n, h, perm, damp_val, a, h32);
  return hipGetLastError();
}

hipError_t build_flipped_f64(hipStream_t st, int n, const double* h, double* a) {
  hipLaunchKernelGGL(k_build_flipped_f64, dim3(nblk((long)n * n)), dim3(256), 0, st, n, h, a);
  return hipGetLastError();
}

hipError_t chol_diag(hipStream_t st, int n, double* a, int k, int kb, int* status, double* pivot) {
  hipLaunchKernelGGL(k_chol_diag, dim3(1), dim3(64), 0, st, n, a, k, kb, status, pivot);
  return hipGetLastError();
}

hipError_t chol_panel(hipStream_t st, int n, double* a, int k, int kb, const int* status) {
  const int rows = n - (k + kb);
  if (rows <= 0) return hipSuccess;
  const int per_wg = 64;  // 4 wavefronts of 16 rows
  hipLaunchKernelGGL(k_chol_panel, dim3((rows + per_wg - 1) / per_wg), dim3(256), 0, st, n, a, k, kb, status);
  return hipGetLastError();
}

hipError_t trinv_diag(hipStream_t st, int n, const double* l, double* y, const int* status) {
  hipLaunchKernelGGL(k_trinv_diag, dim3((n + NBC - 1) / NBC), dim3(128), 0, st, n, l, y, status);
  return hipGetLastError();
}

hipError_t scatter_u(hipStream_t st, int n, const double* y, float* u) {
  hipLaunchKernelGGL(k_scatter_u, dim3(nblk((long)n * n)), dim3(256), 0, st, n, y, u);
  return hipGetLastError();
}

hipError_t fill_zero_f64(hipStream_t st, double* p, size_t count) {
  if (!count) return hipSuccess;
  hipLaunchKernelGGL(k_fill_zero_f64, dim3(nblk((long)count)), dim3(256), 0, st, p, (long)count);
  return hipGetLastError();
}

}  // namespace cdclq
