// f64 factorisation kernels: U with H^-1 = U^T U (src/linalg.rs:200-375, src/engine.rs:320-342).
//
// Blocking follows the reference's NB = 96 block columns because the block boundaries fix the
// floating-point operation sequence of every element:
//   * diagonal block: unblocked left-looking Cholesky with separate multiply/subtract roundings;
//   * panel solve below it: for each column j of the block, s = a_ij - sum_t x_t l_jt in t order;
//   * trailing update: a_ij = fma(-1, chain_t(p_it p_jt), a_ij) per block (k_gemm.hip, lower tiles);
//   * inverse of every diagonal block by columns (mul/add roundings), then per block row two
//     chained GEMMs (k_gemm.hip).
// The panel solve runs one wave per row with the block's columns spread over lanes: column t is
// finalised at step t and immediately subtracted from every later column, which performs the
// reference's per-element subtraction sequence in the same order.
#include "cdclq_dev.h"
#include "kernels.h"

namespace cdclq {
namespace {

constexpr int NBC = 96;  // src/linalg.rs:202, :285

__device__ __forceinline__ double readlane_f64(double v, int lane) {
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_readlane((int)(b & 0xffffffffLL), lane);
  const int hi = __builtin_amdgcn_readlane((int)(b >> 32), lane);
  return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

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
// The steps are software-pipelined: step t first updates the slot column that holds column t + 1
// and publishes it, then runs column t + 1's pivot, square root and divisions while it applies
// column t to the rest of its slots (no branch between them, so the two interleave), then stores
// column t + 1 of L and reads it back for step t + 1. Every element still receives the same
// operations in the same order. A failing pivot is recorded (the first one) and reported at the
// end; the remaining steps run on with values that are discarded with the error.
constexpr int DGL = 8;           // lane grid side
constexpr int DSL = NBC / DGL;   // row / column slots per lane
__global__ __launch_bounds__(64) void k_chol_diag(int n, double* __restrict__ a, int k, int kb, int* status,
                                                  double* pivot) {
  __shared__ double pre[NBC + 64];  // column t with all earlier columns applied; + a discard slot per lane
  __shared__ double col[NBC];       // column t of L (zero above row t)
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
  // pivot of column tn and the divided column of L into LDS (values past kb are computed from
  // clamped reads and never stored)
  auto divide = [&](int tn) {
    const double d = pre[tn];
    const bool rec = (!(d > 0.0) || !isfinite(d)) && fail_t < 0 && tn < kb;
    fail_d = rec ? d : fail_d;
    fail_t = rec ? tn : fail_t;
    const double ltt = sqrt(d);
    const double q0 = pre[lane] / ltt, q1 = pre[min(lane + 64, NBC - 1)] / ltt;
    c0 = (lane == tn) ? ltt : ((lane > tn && lane < kb) ? q0 : 0.0);
    c1 = (lane + 64 == tn) ? ltt : ((lane + 64 > tn && lane + 64 < kb) ? q1 : 0.0);
    col[lane] = c0;
    if (lane + 64 < NBC) col[lane + 64] = c1;
  };
  auto store_col = [&](int tn) {
    if (lane >= tn && lane < kb) a[(long)(k + lane) * n + k + tn] = c0;
    if (lane + 64 >= tn && lane + 64 < kb) a[(long)(k + lane + 64) * n + k + tn] = c1;
  };
  double ci[DSL], cj[DSL];  // column t of L at rows DGL q + tr (ci) and DGL q + tc (cj)
  publish(0, 0);
  divide(0);
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
        divide(t + 1);
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
        divide(t + 1);
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

// Panel solve X L_kk^T = A_panel for all rows below the block (src/linalg.rs:233-241). One wave
// advances PANEL_RPW rows together (columns over lanes), so the LDS reads of L and the long
// divisions of the rows overlap. The strict lower part of L is staged transposed with zeros on
// and above the diagonal (the diagonal separately), so step t applies x_t to every lane without
// predication: lanes at or before t, already final, take -x_t * 0 into a copy that is no longer
// read; each final value is kept in f0 / f1 when its step comes. Columns 0..63 (held in s0) and
// 64.. (s1) run as two loops, so the lane holding column t is known without a select.
constexpr int PANEL_RPW = 4;  // rows per wave
__global__ __launch_bounds__(256) void k_chol_panel(int n, double* __restrict__ a, int k, int kb,
                                                    const int* status) {
  __shared__ double LT[NBC][NBC + 1];  // LT[t][j] = L[j][t] for t < j < kb, else 0
  __shared__ double dg[NBC];           // L[t][t]
  if (*status) return;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  {  // stage the block with all of a thread's loads in flight at once
    constexpr int PER = NBC * NBC / 256;
    double v[PER];
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int e = tid + 256 * q, j = e / NBC, t = e % NBC;
      v[q] = a[(long)(k + min(j, kb - 1)) * n + k + min(t, kb - 1)];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int e = tid + 256 * q, j = e / NBC, t = e % NBC;
      LT[t][j] = (t < j && j < kb) ? v[q] : 0.0;
      if (t == j) dg[t] = v[q];
    }
  }
  __syncthreads();
  const int kend = k + kb;
  const int i0 = kend + (blockIdx.x * 4 + wv) * PANEL_RPW;
  double s0[PANEL_RPW], s1[PANEL_RPW], f0[PANEL_RPW], f1[PANEL_RPW];
#pragma unroll
  for (int q = 0; q < PANEL_RPW; ++q) {
    const int i = min(i0 + q, n - 1);  // rows past the end are computed but never stored
    const double* row = a + (long)i * n + k;
    s0[q] = (lane < kb) ? row[lane] : 0.0;
    s1[q] = (lane + 64 < kb) ? row[lane + 64] : 0.0;
    f0[q] = 0.0;
    f1[q] = 0.0;
  }
  const int kb0 = min(kb, 64);
  for (int t = 0; t < kb0; ++t) {  // column t in s0 (lane t)
    const double ltt = dg[t];
    const double l0 = LT[t][lane], l1 = (lane + 64 < NBC) ? LT[t][lane + 64] : 0.0;
#pragma unroll
    for (int q = 0; q < PANEL_RPW; ++q) {
      const double xt = readlane_f64(s0[q], t) / ltt;
      f0[q] = (lane == t) ? xt : f0[q];
      s0[q] = s0[q] - xt * l0;
      s1[q] = s1[q] - xt * l1;
    }
  }
  for (int t = 64; t < kb; ++t) {  // column t in s1 (lane t - 64); columns 0..63 are final
    const double ltt = dg[t];
    const double l1 = (lane + 64 < NBC) ? LT[t][lane + 64] : 0.0;
#pragma unroll
    for (int q = 0; q < PANEL_RPW; ++q) {
      const double xt = readlane_f64(s1[q], t - 64) / ltt;
      f1[q] = (lane + 64 == t) ? xt : f1[q];
      s1[q] = s1[q] - xt * l1;
    }
  }
#pragma unroll
  for (int q = 0; q < PANEL_RPW; ++q) {
    const int i = i0 + q;
    if (i >= n) break;
    double* row = a + (long)i * n + k;
    if (lane < kb) row[lane] = f0[q];
    if (lane + 64 < kb) row[lane + 64] = f1[q];
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
  const int per_wg = 4 * PANEL_RPW;
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
