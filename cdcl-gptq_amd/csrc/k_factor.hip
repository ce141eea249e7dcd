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

// Unblocked factorisation of the diagonal block (src/linalg.rs:209-229).
__global__ __launch_bounds__(256) void k_chol_diag(int n, double* __restrict__ a, int k, int kb, int* status,
                                                   double* pivot) {
  __shared__ double L[NBC][NBC + 1];
  __shared__ int fail;
  if (*status) return;
  const int tid = threadIdx.x;
  for (int e = tid; e < kb * kb; e += 256) {
    const int i = e / kb, j = e % kb;
    L[i][j] = (j <= i) ? a[(long)(k + i) * n + k + j] : 0.0;
  }
  if (tid == 0) fail = 0;
  __syncthreads();
  for (int j = 0; j < kb; ++j) {
    if (tid == 0) {
      double d = L[j][j];
      for (int t = 0; t < j; ++t) {
        const double v = L[j][t];
        d = d - v * v;
      }
      if (!(d > 0.0) || !isfinite(d)) {
        fail = 1;
        *status = k + j + 1;
        *pivot = d;
      } else {
        L[j][j] = sqrt(d);
      }
    }
    __syncthreads();
    if (fail) return;
    const double dj = L[j][j];
    for (int i = j + 1 + tid; i < kb; i += 256) {
      double s = L[i][j];
      for (int t = 0; t < j; ++t) s = s - L[i][t] * L[j][t];
      L[i][j] = s / dj;
    }
    __syncthreads();
  }
  for (int e = tid; e < kb * kb; e += 256) {
    const int i = e / kb, j = e % kb;
    if (j <= i) a[(long)(k + i) * n + k + j] = L[i][j];
  }
}

// Panel solve X L_kk^T = A_panel for all rows below the block (src/linalg.rs:233-241).
constexpr int PANEL_RPW = 4;  // rows per wave
__global__ __launch_bounds__(256) void k_chol_panel(int n, double* __restrict__ a, int k, int kb,
                                                    const int* status) {
  __shared__ double LT[NBC][NBC + 1];  // LT[t][j] = L[j][t]
  if (*status) return;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  for (int e = tid; e < kb * kb; e += 256) {
    const int j = e / kb, t = e % kb;
    LT[t][j] = (t <= j) ? a[(long)(k + j) * n + k + t] : 0.0;
  }
  __syncthreads();
  const int kend = k + kb;
  for (int q = 0; q < PANEL_RPW; ++q) {
    const int i = kend + (blockIdx.x * PANEL_RPW + q) * 4 + wv;
    if (i >= n) break;
    double* row = a + (long)i * n + k;
    double s0 = (lane < kb) ? row[lane] : 0.0;
    double s1 = (lane + 64 < kb) ? row[lane + 64] : 0.0;
    for (int t = 0; t < kb; ++t) {
      const double st = (t < 64) ? readlane_f64(s0, t) : readlane_f64(s1, t - 64);
      const double xt = st / LT[t][t];
      if (lane == t) s0 = xt;
      if (lane + 64 == t) s1 = xt;
      if (lane > t && lane < kb) s0 = s0 - xt * LT[t][lane];
      if (lane + 64 > t && lane + 64 < kb) s1 = s1 - xt * LT[t][lane + 64];
    }
    if (lane < kb) row[lane] = s0;
    if (lane + 64 < kb) row[lane + 64] = s1;
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
  hipLaunchKernelGGL(k_chol_diag, dim3(1), dim3(256), 0, st, n, a, k, kb, status, pivot);
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
