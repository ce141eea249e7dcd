// Per-row sweep kernels of the quantization engine (src/engine.rs:366-674) and small helpers.
//
// Rows are independent in both phases (src/engine.rs:9-15), so every sweep kernel gives one
// 64-lane wavefront to one row: the row's columns of the current block / group / sub-block live in
// VGPRs spread over the lanes, the column loop runs in wave-uniform control flow, the value of the
// current column is broadcast with v_readlane, and updates of the not-yet-visited columns are
// lane-parallel. Each element therefore sees exactly the reference's sequence of roundings.
#include <algorithm>

#include "cdclq_dev.h"
#include "kernels.h"

namespace cdclq {
namespace {

inline unsigned nblk(long count) { return (unsigned)((count + 255) / 256); }
// Grid of a grid-stride launch over `count` elements: at most 2^20 workgroups of 256, so the
// dispatch stays far below 2^32 work-items whatever the element count (a 524,288-token input of
// width 8192 alone has 2^32 elements).
inline unsigned gs_blocks(long count) { return (unsigned)std::min<long>((count + 255) / 256, 1L << 20); }

__device__ __forceinline__ int readlane_i(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }

// ---------------------------------------------------------------- preparation helpers
__global__ __launch_bounds__(256) void k_diag_extract(int n, const float* __restrict__ h, float* __restrict__ d) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j < n) d[j] = h[(long)j * n + j];
}

// wp[r][j] = w0[r][perm[j]], where w0 has dead columns zeroed (src/engine.rs:708-716, :726-731).
__global__ __launch_bounds__(256) void k_permute_w(int d_out, int n, const float* __restrict__ w,
                                                   const uint32_t* __restrict__ perm,
                                                   const uint8_t* __restrict__ dead_perm, float* __restrict__ wp) {
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long)d_out * n) return;
  const int r = (int)(idx / n), j = (int)(idx % n);
  wp[idx] = dead_perm[j] ? 0.0f : w[(long)r * n + perm[j]];
}

// mp = perm(M) with the f32 ridge on the diagonal (src/engine.rs:739-746).
__global__ __launch_bounds__(256) void k_permute_m(int n, const float* __restrict__ m,
                                                   const uint32_t* __restrict__ perm, float damp32,
                                                   float* __restrict__ mp) {
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long)n * n) return;
  const int i = (int)(idx / n), j = (int)(idx % n);
  float v = m[(long)perm[i] * n + perm[j]];
  if (i == j) v += damp32;
  mp[idx] = v;
}

// colsq[j] = sum_r (f64 w0_rj)^2 in row order (src/engine.rs:279-285).
__global__ __launch_bounds__(256) void k_colsq(int d_out, int n, const float* __restrict__ w,
                                               const uint8_t* __restrict__ dead, double* __restrict__ out) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= n) return;
  double s = 0.0;
  if (!dead[j]) {
    // the sum stays sequential over the rows; the loads go out CS_BATCH rows ahead of the adds
    constexpr int CS_BATCH = 32;
    for (int r0 = 0; r0 < d_out; r0 += CS_BATCH) {
      float v[CS_BATCH];
#pragma unroll
      for (int q = 0; q < CS_BATCH; ++q) v[q] = w[(long)min(r0 + q, d_out - 1) * n + j];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int q = 0; q < CS_BATCH; ++q) {
        if (r0 + q < d_out) {
          const double x = (double)v[q];
          s = s + x * x;
        }
      }
    }
  }
  out[j] = s;
}

__global__ __launch_bounds__(256) void k_inv_diag(int n, const float* __restrict__ u, float* __restrict__ invd) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j < n) invd[j] = 1.0f / u[(long)j * n + j];
}

// ---------------------------------------------------------------- phase 1 (src/engine.rs:397-473)
// One block [i1, i1+cnt) for all rows; NPL = values per lane (cnt <= 64*NPL), one wave per row,
// GB_ROWS rows per workgroup. For blocks of at most 128 columns the workgroup stages the block of
// U (rows and columns i1..i1+cnt) and 1/U_jj in LDS first, so the column steps, each of which
// needs row j of the block, read it from LDS instead of a round trip to L2.
constexpr int GB_ROWS = 8;
template <int NPL>
__global__ __launch_bounds__(64 * GB_ROWS) void k_gptq_block(int rows, int n, int i1, int cnt, int g, int ng,
                                                    const float* __restrict__ w, const float* __restrict__ u,
                                                    const float* __restrict__ invd, const uint8_t* __restrict__ gbits,
                                                    int mse, float* __restrict__ scales, float* __restrict__ zeros,
                                                    uint8_t* __restrict__ codes, float* __restrict__ wq,
                                                    float* __restrict__ err, unsigned long long* __restrict__ mid) {
  constexpr bool STAGE = NPL <= 2;
  constexpr int UB = STAGE ? 64 * NPL : 1;  // staged block width
  __shared__ float ub[UB * UB];
  __shared__ float idv[UB];
  const int lane = threadIdx.x & 63;
  if constexpr (STAGE) {  // clamped addresses: every load is unconditional, a batch in flight at once
    constexpr int PER = UB * UB / (64 * GB_ROWS), BATCH = PER < 16 ? PER : 16;
#pragma unroll
    for (int b = 0; b < PER; b += BATCH) {
      float v[BATCH];
#pragma unroll
      for (int q = 0; q < BATCH; ++q) {
        const int x = threadIdx.x + 64 * GB_ROWS * (b + q), i = x / UB, c = x % UB;
        v[q] = u[(long)(i1 + min(i, cnt - 1)) * n + i1 + min(c, cnt - 1)];
      }
#pragma unroll
      for (int q = 0; q < BATCH; ++q) {
        const int x = threadIdx.x + 64 * GB_ROWS * (b + q), i = x / UB, c = x % UB;
        ub[x] = (i < cnt && c < cnt) ? v[q] : 0.0f;
      }
    }
    if (threadIdx.x < UB) idv[threadIdx.x] = invd[i1 + min((int)threadIdx.x, cnt - 1)];
    __syncthreads();
  }
  const int r = __builtin_amdgcn_readfirstlane(blockIdx.x * GB_ROWS + (threadIdx.x >> 6));
  if (r >= rows) return;
  const int i2 = i1 + cnt;
  const float* wr = w + (long)r * n;
  float x[NPL], mq[NPL], mwq[NPL], me[NPL];
#pragma unroll
  for (int s = 0; s < NPL; ++s) {
    const int c = s * 64 + lane;
    x[s] = (c < cnt) ? wr[i1 + c] : 0.0f;
    mq[s] = 0.0f;
    mwq[s] = 0.0f;
    me[s] = 0.0f;
  }
  // A block that starts inside a group (block < group) continues with the stored grid.
  float sc = 0.0f, zr = 0.0f, maxq = 0.0f;
  // near-midpoint decisions of this row (wave-uniform: every lane evaluates the same column)
  unsigned near_codes = 0, near_zeros = 0;
  if (i1 % g != 0) {
    const int gi = i1 / g;
    sc = scales[(long)r * ng + gi];
    zr = zeros[(long)r * ng + gi];
    maxq = (float)((1u << gbits[gi]) - 1u);
  }
#pragma unroll
  for (int s = 0; s < NPL; ++s) {
    for (int ii = 0; ii < 64; ++ii) {
      const int i = s * 64 + ii;
      if (i >= cnt) break;
      const int j = i1 + i;
      if (j % g == 0) {
        // group grid from the weights current at this column (src/engine.rs:410-423):
        // columns < i2 from the in-block values, columns >= i2 from the full-width buffer.
        const int gi = j / g;
        const int gend = min(j + g, n);
        maxq = (float)((1u << gbits[gi]) - 1u);
        float lmin = INFINITY, lmax = -INFINITY;
#pragma unroll
        for (int s2 = 0; s2 < NPL; ++s2) {
          const int col = i1 + s2 * 64 + lane;
          if (col < i2 && col >= j && col < gend) {
            lmin = rs_minf(lmin, x[s2]);
            lmax = rs_maxf(lmax, x[s2]);
          }
        }
        for (int col = i2 + lane; col < gend; col += 64) {
          const float v = wr[col];
          lmin = rs_minf(lmin, v);
          lmax = rs_maxf(lmax, v);
        }
        float xmin = rs_minf(0.0f, wave_min(lmin));
        float xmax = rs_maxf(0.0f, wave_max(lmax));
        if (xmin == 0.0f && xmax == 0.0f) {
          xmin = -1.0f;
          xmax = 1.0f;
        }
        grid_mk(xmin, xmax, maxq, &sc, &zr);
        float lo_used = xmin;  // the lower end of the grid chosen below, for the zero's accounting
        if (mse) {
          // 24 clip ratios, one per lane; each lane runs its candidate's sequential error sum over
          // the group in column order (src/quant.rs:65-81), then the first minimum wins.
          const int cand = lane < 24 ? lane : 0;
          const float p = 1.0f - 0.02f * (float)cand;
          float cs, cz;
          grid_mk(p * xmin, p * xmax, maxq, &cs, &cz);
          float errs = 0.0f;
#pragma unroll
          for (int s2 = 0; s2 < NPL; ++s2) {
            for (int jj = 0; jj < 64; ++jj) {
              const int col = i1 + s2 * 64 + jj;
              if (col >= i2 || col >= gend) break;
              if (col < j) continue;
              const float v = readlane(x[s2], jj);
              float qq;
              const float d = quant_dq(v, cs, cz, maxq, &qq);
              const float ee = d - v;
              errs = errs + ee * ee;
            }
          }
          for (int col = i2 > j ? i2 : j; col < gend; ++col) {
            const float v = wr[col];
            float qq;
            const float d = quant_dq(v, cs, cz, maxq, &qq);
            const float ee = d - v;
            errs = errs + ee * ee;
          }
          float be = (lane < 24 && errs == errs) ? errs : INFINITY;
          int bc = (lane < 24) ? lane : (1 << 20);
#pragma unroll
          for (int o = 32; o > 0; o >>= 1) {
            const float oe = __shfl_xor(be, o, 64);
            const int oc = __shfl_xor(bc, o, 64);
            if (oe < be || (oe == be && oc < bc)) {
              be = oe;
              bc = oc;
            }
          }
          bc = readlane_i(bc, 0);
          sc = readlane(cs, bc);
          zr = readlane(cz, bc);
          lo_used = (1.0f - 0.02f * (float)bc) * xmin;
        }
        near_zeros += near_midpoint(-lo_used, sc, 0.0f, maxq) ? 1u : 0u;
        if (lane == 0) {
          scales[(long)r * ng + gi] = sc;
          zeros[(long)r * ng + gi] = zr;
        }
      }
      // With the block staged, row i of U and 1/U_ii are read before the column's quantization,
      // so the LDS latency overlaps the division instead of following it (unconditional reads
      // inside the staged block; lanes outside the update discard them).
      float uv[NPL], di = 0.0f;
      if constexpr (STAGE) {
        di = idv[i];
#pragma unroll
        for (int s2 = 0; s2 < NPL; ++s2) uv[s2] = ub[i * UB + s2 * 64 + lane];
      }
      const float xv = readlane(x[s], ii);
      float q;
      const float dq = quant_dq(xv, sc, zr, maxq, &q);
      near_codes += near_midpoint(xv, sc, zr, maxq) ? 1u : 0u;
      const float e = (xv - dq) * (STAGE ? di : invd[j]);
      if (lane == ii) {
        mq[s] = q;
        mwq[s] = dq;
        me[s] = e;
      }
      const float* urow = u + (long)j * n + i1;
#pragma unroll
      for (int s2 = s; s2 < NPL; ++s2) {
        const int c = s2 * 64 + lane;
        if constexpr (STAGE)  // lanes at or before column i (already quantized) and past cnt take
          x[s2] = x[s2] - e * uv[s2];  // garbage that is never read: no predicate
        else if (c > i && c < cnt)
          x[s2] = x[s2] - e * urow[c];
      }
    }
  }
#pragma unroll
  for (int s = 0; s < NPL; ++s) {
    const int c = s * 64 + lane;
    if (c < cnt) {
      const long o = (long)r * n + i1 + c;
      codes[o] = code_of(mq[s]);
      wq[o] = mwq[s];
      err[o] = me[s];
    }
  }
  if (lane == 0 && (near_codes | near_zeros)) {  // rare: counted with one atomic per row and kind
    if (near_codes) atomicAdd(&mid[MID_CODE_NEAR], (unsigned long long)near_codes);
    if (near_zeros) atomicAdd(&mid[MID_ZERO_NEAR], (unsigned long long)near_zeros);
  }
}

// Phase-1 block sweep with L lanes per row (64 / L rows per wavefront), for blocks of at most 128
// columns whose groups lie inside the block, without the MSE grid. Per column the wave-per-row
// kernel above runs the quantization of one value on all 64 lanes; here L lanes share it, so the
// redundant part of every column step shrinks 64 / L times while the update of the later columns
// (the row's working values, VPL = 128 / L per lane, lane ll holding columns VPL ll .. +VPL - 1)
// stays lane-parallel. Column i's value comes from its owner lane by a shuffle inside the row's
// lane group; the group grid reduces min / max over the same L lanes. Each element sees exactly
// the reference's operations in the reference's order (src/engine.rs:397-451); the registers of
// columns already quantized keep taking updates that are never read. W wavefronts per workgroup
// share the staged block of U (64 KB, so two workgroups per CU).
template <int L, int W>
__global__ __launch_bounds__(64 * W) void k_gptq_rows(int rows, int n, int i1, int cnt, int g, int ng,
                                                   const float* __restrict__ w, const float* __restrict__ u,
                                                   const float* __restrict__ invd,
                                                   const uint8_t* __restrict__ gbits, float* __restrict__ scales,
                                                   float* __restrict__ zeros, uint8_t* __restrict__ codes,
                                                   float* __restrict__ wq, float* __restrict__ err,
                                                   unsigned long long* __restrict__ mid) {
  constexpr int VPL = 128 / L;  // columns per lane
  constexpr int R = 64 / L;     // rows per wavefront
  __shared__ float ub[128 * 128];
  __shared__ float idv[128];
  {  // stage the block of U (zero outside cnt x cnt) and 1 / U_ii: clamped, unconditional loads
    constexpr int NT = 64 * W, PER = 128 * 128 / NT, BATCH = PER < 16 ? PER : 16;
#pragma unroll
    for (int b = 0; b < PER; b += BATCH) {
      float v[BATCH];
#pragma unroll
      for (int q = 0; q < BATCH; ++q) {
        const int x = threadIdx.x + NT * (b + q), i = x >> 7, c = x & 127;
        v[q] = u[(long)(i1 + min(i, cnt - 1)) * n + i1 + min(c, cnt - 1)];
      }
#pragma unroll
      for (int q = 0; q < BATCH; ++q) {
        const int x = threadIdx.x + NT * (b + q), i = x >> 7, c = x & 127;
        ub[x] = (i < cnt && c < cnt) ? v[q] : 0.0f;
      }
    }
    if (threadIdx.x < 128) idv[threadIdx.x] = invd[i1 + min((int)threadIdx.x, cnt - 1)];
    __syncthreads();
  }
  const int lane = threadIdx.x & 63;
  const int rr = lane / L, ll = lane % L;
  const int r = (blockIdx.x * W + (threadIdx.x >> 6)) * R + rr;
  if (__builtin_amdgcn_readfirstlane(r - rr) >= rows) return;  // the wave's first row
  const bool live = r < rows;
  const float* wr = w + (long)min(r, rows - 1) * n + i1;
  // the owned columns' results; with 16 columns per lane the codes are kept one byte each (the
  // registers then allow four wavefronts per SIMD)
  constexpr bool PACK = VPL >= 16;
  float x[VPL], mwq[VPL], me[VPL], mq[PACK ? 1 : VPL];
  uint32_t mcode[PACK ? VPL / 4 : 1];
#pragma unroll
  for (int t = 0; t < VPL; ++t) {
    const int c = VPL * ll + t;
    x[t] = (c < cnt) ? wr[c] : 0.0f;
    mwq[t] = 0.0f;
    me[t] = 0.0f;
    if constexpr (PACK) {
      if ((t & 3) == 0) mcode[t >> 2] = 0u;
    } else {
      mq[t] = 0.0f;
    }
  }
  float sc = 0.0f, zr = 0.0f, maxq = 0.0f;
  unsigned near_codes = 0, near_zeros = 0;  // zero points: counted once per row, by its lane 0
  // With at most 8 columns per lane (the launcher keeps g a multiple of 8 here) a lane's columns lie
  // in one group, so each lane tests its own columns' code decisions for a near midpoint after the
  // sweep, from the value each had when it was decided (xs) and its group's grid (gsc, gzr, gmq),
  // instead of the row's lane 0 testing every column inside the sweep's dependent chain.
  constexpr bool DEFER = VPL <= 8;
  float xs[DEFER ? VPL : 1];
  float gsc = 0.0f, gzr = 0.0f, gmq = 0.0f;
  const int base = rr * L;                  // the row group's first lane
  for (int oi = 0; oi < L; ++oi) {          // owner lane of the columns VPL oi .. +VPL - 1
#pragma unroll
    for (int t = 0; t < VPL; ++t) {
      const int i = VPL * oi + t;
      if (i < cnt) {  // uniform
        const int j = i1 + i;
        if (j % g == 0) {  // group grid over the group's columns, all inside the block
          const int gi = j / g, gend = min(i + g, cnt);
          maxq = (float)((1u << gbits[gi]) - 1u);
          float lmin = INFINITY, lmax = -INFINITY;
#pragma unroll
          for (int t2 = 0; t2 < VPL; ++t2) {
            const int c = VPL * ll + t2;
            if (c >= i && c < gend) {
              lmin = rs_minf(lmin, x[t2]);
              lmax = rs_maxf(lmax, x[t2]);
            }
          }
#pragma unroll
          for (int o = L / 2; o > 0; o >>= 1) {
            lmin = rs_minf(lmin, __shfl_xor(lmin, o, 64));
            lmax = rs_maxf(lmax, __shfl_xor(lmax, o, 64));
          }
          float xmin = rs_minf(0.0f, lmin), xmax = rs_maxf(0.0f, lmax);
          if (xmin == 0.0f && xmax == 0.0f) {
            xmin = -1.0f;
            xmax = 1.0f;
          }
          grid_mk(xmin, xmax, maxq, &sc, &zr);
          if constexpr (DEFER) {
            if (VPL * ll >= i && VPL * ll < i + g) {  // this lane's columns are in the group
              gsc = sc;
              gzr = zr;
              gmq = maxq;
            }
          }
          if (ll == 0) {
            near_zeros += near_midpoint(-xmin, sc, 0.0f, maxq) ? 1u : 0u;
            if (live) {
              scales[(long)r * ng + gi] = sc;
              zeros[(long)r * ng + gi] = zr;
            }
          }
        }
        float uv[VPL];
#pragma unroll
        for (int t2 = 0; t2 < VPL; ++t2) uv[t2] = ub[i * 128 + VPL * ll + t2];
        const float di = idv[i];
        float xv;  // column i of the row: lane base + oi's x[t]
        if constexpr (L >= 32) {
          // read from each row group's owner lane (uniform lane indices) and selected by row group:
          // a few cycles, against a cross-lane permute through the LDS unit on the step's chain
          // (with four or more row groups per wavefront the extra instructions cost more than the
          // permute's latency in these issue-bound sweeps)
          xv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x[t]), oi));
#pragma unroll
          for (int q = 1; q < R; ++q) {
            const float sq = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x[t]), q * L + oi));
            xv = rr == q ? sq : xv;
          }
        } else {
          xv = __shfl(x[t], base + oi, 64);
        }
        float q;
        const float dq = quant_dq(xv, sc, zr, maxq, &q);
        if constexpr (!DEFER) {
          if (ll == 0) near_codes += near_midpoint(xv, sc, zr, maxq) ? 1u : 0u;
        }
        const float e = (xv - dq) * di;
        if (ll == oi) {
          if constexpr (DEFER) xs[t] = xv;
          if constexpr (PACK)
            mcode[t >> 2] = (mcode[t >> 2] & ~(0xffu << (8 * (t & 3)))) | ((uint32_t)code_of(q) << (8 * (t & 3)));
          else
            mq[t] = q;
          mwq[t] = dq;
          me[t] = e;
        }
#pragma unroll
        for (int t2 = 0; t2 < VPL; ++t2) x[t2] = x[t2] - e * uv[t2];
      }
    }
  }
  if (live) {
#pragma unroll
    for (int t = 0; t < VPL; ++t) {
      const int c = VPL * ll + t;
      if (c < cnt) {
        const long o = (long)r * n + i1 + c;
        if constexpr (PACK)
          codes[o] = (uint8_t)(mcode[t >> 2] >> (8 * (t & 3)));
        else
          codes[o] = code_of(mq[t]);
        wq[o] = mwq[t];
        err[o] = me[t];
        if constexpr (DEFER) near_codes += near_midpoint(xs[t], gsc, gzr, gmq) ? 1u : 0u;
      }
    }
    if (near_codes) atomicAdd(&mid[MID_CODE_NEAR], (unsigned long long)near_codes);
    if (near_zeros) atomicAdd(&mid[MID_ZERO_NEAR], (unsigned long long)near_zeros);
  }
}

// Phase-1 block sweep for blocks wider than 1024 columns (the register kernel above holds at most
// 16 values per lane). Same per-element operations and order; the block's working values live in
// the row of w itself (columns i1..i2, dead after the block: the lazy update reads only columns
// >= i2), and each column step reads what the previous steps wrote. One wavefront per row, four
// rows per workgroup. A lane's stores are ordered before the wave's next loads by a workgroup-scope
// fence (all lanes of a wave share the CU's vector cache).
__global__ __launch_bounds__(256) void k_gptq_block_mem(int rows, int n, int i1, int cnt, int g, int ng,
                                                        float* __restrict__ w, const float* __restrict__ u,
                                                        const float* __restrict__ invd,
                                                        const uint8_t* __restrict__ gbits, int mse,
                                                        float* __restrict__ scales, float* __restrict__ zeros,
                                                        uint8_t* __restrict__ codes, float* __restrict__ wq,
                                                        float* __restrict__ err, unsigned long long* __restrict__ mid) {
  const int lane = threadIdx.x & 63;
  const int r = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
  if (r >= rows) return;
  float* wr = w + (long)r * n;
  float sc = 0.0f, zr = 0.0f, maxq = 0.0f;
  unsigned near_codes = 0, near_zeros = 0;
  if (i1 % g != 0) {
    const int gi = i1 / g;
    sc = scales[(long)r * ng + gi];
    zr = zeros[(long)r * ng + gi];
    maxq = (float)((1u << gbits[gi]) - 1u);
  }
  for (int i = 0; i < cnt; ++i) {
    const int j = i1 + i;
    if (j % g == 0) {
      // group grid from the current values of columns j..gend: in-block columns hold the working
      // values, columns >= i2 the full-width values (src/engine.rs:410-423)
      const int gi = j / g;
      const int gend = min(j + g, n);
      maxq = (float)((1u << gbits[gi]) - 1u);
      float lmin = INFINITY, lmax = -INFINITY;
      for (int col = j + lane; col < gend; col += 64) {
        const float v = wr[col];
        lmin = rs_minf(lmin, v);
        lmax = rs_maxf(lmax, v);
      }
      float xmin = rs_minf(0.0f, wave_min(lmin));
      float xmax = rs_maxf(0.0f, wave_max(lmax));
      if (xmin == 0.0f && xmax == 0.0f) {
        xmin = -1.0f;
        xmax = 1.0f;
      }
      grid_mk(xmin, xmax, maxq, &sc, &zr);
      float lo_used = xmin;
      if (mse) {  // one candidate per lane, sequential error sum in column order (src/quant.rs:65-81)
        const int cand = lane < 24 ? lane : 0;
        const float p = 1.0f - 0.02f * (float)cand;
        float cs, cz;
        grid_mk(p * xmin, p * xmax, maxq, &cs, &cz);
        float errs = 0.0f;
        for (int col = j; col < gend; ++col) {
          const float v = wr[col];
          float qq;
          const float d = quant_dq(v, cs, cz, maxq, &qq);
          const float ee = d - v;
          errs = errs + ee * ee;
        }
        float be = (lane < 24 && errs == errs) ? errs : INFINITY;
        int bc = (lane < 24) ? lane : (1 << 20);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
          const float oe = __shfl_xor(be, o, 64);
          const int oc = __shfl_xor(bc, o, 64);
          if (oe < be || (oe == be && oc < bc)) {
            be = oe;
            bc = oc;
          }
        }
        bc = readlane_i(bc, 0);
        sc = readlane(cs, bc);
        zr = readlane(cz, bc);
        lo_used = (1.0f - 0.02f * (float)bc) * xmin;
      }
      near_zeros += near_midpoint(-lo_used, sc, 0.0f, maxq) ? 1u : 0u;
      if (lane == 0) {
        scales[(long)r * ng + gi] = sc;
        zeros[(long)r * ng + gi] = zr;
      }
    }
    const float xv = wr[j];
    float q;
    const float dq = quant_dq(xv, sc, zr, maxq, &q);
    near_codes += near_midpoint(xv, sc, zr, maxq) ? 1u : 0u;
    const float e = (xv - dq) * invd[j];
    if (lane == 0) {
      const long o = (long)r * n + j;
      codes[o] = code_of(q);
      wq[o] = dq;
      err[o] = e;
    }
    const float* urow = u + (long)j * n;
    for (int c = j + 1 + lane; c < i1 + cnt; c += 64) wr[c] = wr[c] - e * urow[c];
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  }
  if (lane == 0 && (near_codes | near_zeros)) {
    if (near_codes) atomicAdd(&mid[MID_CODE_NEAR], (unsigned long long)near_codes);
    if (near_zeros) atomicAdd(&mid[MID_ZERO_NEAR], (unsigned long long)near_zeros);
  }
}

// colloss[chunk][j] = sum over the chunk's rows, in row order, of (f64)(eps*eps) (src/engine.rs:438).
__global__ __launch_bounds__(256) void k_colloss(int rows, int n, int rc, const float* __restrict__ err,
                                                 double* __restrict__ out) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  const int c = blockIdx.y;
  if (j >= n) return;
  const int r0 = c * rc, r1 = min(rows, r0 + rc);
  double s = 0.0;
  for (int r = r0; r < r1; ++r) {
    const float e = err[(long)r * n + j];
    s = s + (double)(e * e);
  }
  out[(long)c * n + j] = s;
}

__global__ __launch_bounds__(256) void k_sub(long count, const float* __restrict__ a, const float* __restrict__ b,
                                             float* __restrict__ o) {
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx < count) o[idx] = a[idx] - b[idx];
}

// Per-chunk loss bookkeeping of one pass, in the reference's order (src/engine.rs:583, :640):
// steps in execution order (refit groups, then CD sub-blocks), within a step rows ascending,
// within a row its accepted deltas in the order they were made. One workgroup per chunk. The
// (step, row) entries of the chunk are taken ACC_ENT at a time in that order: each thread loads
// the counts of ACC_ENT / 256 consecutive entries, one workgroup scan gives every entry its first
// position in the fold order, and the deltas are gathered into LDS ACC_LDS positions at a time
// (every position finds its entry by binary search over the offsets, so all loads are
// independent). Waves 1-3 gather the next ACC_LDS positions while wave 0 folds the current ones
// sequentially in f64, so the fold's add chain sets the time.
constexpr int ACC_LDS = 4096;
constexpr int ACC_ENT = 4096;
constexpr int ACC_PER = ACC_ENT / 256;
__global__ __launch_bounds__(256) void k_pass_accum(int rows, int rc, int nref, const double* __restrict__ rlog,
                                                    const uint32_t* __restrict__ rcnt, int ncd, int cap,
                                                    const double* __restrict__ clog,
                                                    const uint32_t* __restrict__ ccnt,
                                                    const uint8_t* __restrict__ active, double* __restrict__ ld,
                                                    uint64_t* __restrict__ upd) {
  __shared__ double vals[2][ACC_LDS + 32];  // padding: wave 0 reads up to 32 past the batch's end
  __shared__ uint32_t offs[ACC_ENT + 1];  // exclusive offsets of the batch's entries; offs[ne] = total
  __shared__ uint32_t wsum[4];
  const int c = blockIdx.x;
  if (!active[c]) return;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int r0 = c * rc, nr = min(rows, r0 + rc) - r0;
  const long nent = (long)(nref + ncd) * nr;  // entries (step, row) of this chunk, fold order
  double acc = ld[c];                          // meaningful in wave 0
  uint64_t u = upd[c];
  // entry e -> (step e / nr, row r0 + e % nr)
  auto entry_cnt = [&](long e) -> uint32_t {
    const int step = (int)(e / nr), row = r0 + (int)(e % nr);
    return step < nref ? rcnt[(long)step * rows + row] : ccnt[(long)(step - nref) * rows + row];
  };
  auto value_at = [&](long e, uint32_t k) -> double {
    const int step = (int)(e / nr), row = r0 + (int)(e % nr);
    return step < nref ? rlog[(long)step * rows + row] : clog[((long)(step - nref) * rows + row) * cap + k];
  };
  for (long eb = 0; eb < nent; eb += ACC_ENT) {
    const int ne = (int)min((long)ACC_ENT, nent - eb);
    // counts of this thread's ACC_PER consecutive entries, all loads in flight at once
    uint32_t k[ACC_PER];
#pragma unroll
    for (int q = 0; q < ACC_PER; ++q) {
      const int e = tid * ACC_PER + q;
      k[q] = e < ne ? entry_cnt(eb + e) : 0u;
    }
    uint32_t tsum = 0;
#pragma unroll
    for (int q = 0; q < ACC_PER; ++q) tsum += k[q];
    uint32_t incl = tsum;  // workgroup exclusive scan of the thread sums
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t v = __shfl_up(incl, o, 64);
      if (lane >= o) incl += v;
    }
    if (lane == 63) wsum[wv] = incl;
    __syncthreads();
    uint32_t run = incl - tsum;
    for (int w = 0; w < wv; ++w) run += wsum[w];
    const uint32_t total = wsum[0] + wsum[1] + wsum[2] + wsum[3];
#pragma unroll
    for (int q = 0; q < ACC_PER; ++q) {
      const int e = tid * ACC_PER + q;
      if (e < ne) offs[e] = run;
      run += k[q];
    }
    if (tid == 0) offs[ne] = total;
    __syncthreads();
    if (total == 0) continue;  // uniform
    u += total;
    // gather positions [done, done + m) into vals[buf]; threads [t0, t0 + nthr) take part
    auto gather = [&](uint32_t done, int buf, int t0, int nthr) {
      const uint32_t m = min((uint32_t)ACC_LDS, total - done);
      for (uint32_t i = tid - t0; i < m; i += nthr) {
        const uint32_t pos = done + i;
        int lo = 0, hi = ne;  // largest e in [0, ne) with offs[e] <= pos
        while (hi - lo > 1) {
          const int mid = (lo + hi) >> 1;
          if (offs[mid] <= pos) lo = mid; else hi = mid;
        }
        vals[buf][i] = value_at(eb + lo, pos - offs[lo]);
      }
    };
    gather(0, 0, 0, 256);
    __syncthreads();
    int buf = 0;
    for (uint32_t done = 0; done < total; done += ACC_LDS) {
      const uint32_t m = min((uint32_t)ACC_LDS, total - done);
      if (wv == 0) {
        // Three register batches of 8 rotate: each is read two batches before it is added, so
        // the adds never wait on the most recent reads. Reads past m (inside the padding) are
        // never added.
        const double* vb = &vals[buf][0];
        const uint32_t m8 = m & ~7u;
        double va[8], vb8[8], vc[8];
        auto rd = [&](uint32_t at, double* d) {
#pragma unroll
          for (int q = 0; q < 8; ++q) d[q] = vb[at + q];
          asm volatile("" : "+v"(acc) : : "memory");  // the reads stay ahead of the adds that follow
        };
        auto add = [&](const double* d) {
#pragma unroll
          for (int q = 0; q < 8; ++q) acc = acc + d[q];
        };
        rd(0, va);
        rd(8, vb8);
        uint32_t i = 0;
        for (; i + 24 <= m8; i += 24) {
          rd(i + 16, vc);
          add(va);
          rd(i + 24, va);
          add(vb8);
          rd(i + 32, vb8);
          add(vc);
        }
        if (i < m8) {  // at most two batches left, already in va and vb8
          add(va);
          i += 8;
          if (i < m8) {
            add(vb8);
            i += 8;
          }
        }
        for (; i < m; ++i) acc = acc + vb[i];
      } else if (done + ACC_LDS < total) {
        gather(done + ACC_LDS, buf ^ 1, 64, 192);
      }
      __syncthreads();
      buf ^= 1;
    }
  }
  if (tid == 0) {
    ld[c] = acc;
    upd[c] = u;
  }
}

// ---------------------------------------------------------------- synthetic inputs
__global__ __launch_bounds__(256) void k_synth_normal(uint64_t seed, uint64_t offset, long count, float sigma,
                                                      float* __restrict__ out) {
  for (long idx = (long)blockIdx.x * 256 + threadIdx.x; idx < count; idx += (long)gridDim.x * 256)
    out[idx] = synth_normal_at(seed, offset + (uint64_t)idx) * sigma;
}

__global__ __launch_bounds__(256) void k_synth_tokens(uint64_t seed, uint64_t row0, long t, int n,
                                                      const float* __restrict__ cs, const uint8_t* __restrict__ heavy,
                                                      float* __restrict__ x) {
  const long count = t * (long)n;
  for (long idx = (long)blockIdx.x * 256 + threadIdx.x; idx < count; idx += (long)gridDim.x * 256) {
    const long r = idx / n;
    const int j = (int)(idx % n);
    const uint64_t i = (row0 + (uint64_t)r) * (uint64_t)n + (uint64_t)j;
    const float v = (heavy && heavy[j]) ? synth_student3_at(seed, i) : synth_normal_at(seed, i);
    x[idx] = v * (cs ? cs[j] : 1.0f);
  }
}

// out = x + sigma * normal(seed, offset + i)
__global__ __launch_bounds__(256) void k_synth_perturb(uint64_t seed, uint64_t offset, long count, float sigma,
                                                       const float* __restrict__ x, float* __restrict__ out) {
  for (long idx = (long)blockIdx.x * 256 + threadIdx.x; idx < count; idx += (long)gridDim.x * 256)
    out[idx] = x[idx] + synth_normal_at(seed, offset + (uint64_t)idx) * sigma;
}

__global__ __launch_bounds__(256) void k_f64_to_f32(long count, const double* __restrict__ a, float* __restrict__ b) {
  for (long idx = (long)blockIdx.x * 256 + threadIdx.x; idx < count; idx += (long)gridDim.x * 256)
    b[idx] = (float)a[idx];
}

// Block partial sums of (f64)e * (f64)eh for proxy_loss (src/engine.rs:814).
__global__ __launch_bounds__(256) void k_proxy_reduce(long count, const float* __restrict__ e,
                                                      const float* __restrict__ eh, double* __restrict__ partial) {
  __shared__ double red[256];
  double s = 0.0;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < count; i += (long)gridDim.x * 256)
    s += (double)e[i] * (double)eh[i];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) partial[blockIdx.x] = red[0];
}

}  // namespace

hipError_t diag_extract(hipStream_t st, int n, const float* h, float* diag) {
  hipLaunchKernelGGL(k_diag_extract, dim3(nblk(n)), dim3(256), 0, st, n, h, diag);
  return hipGetLastError();
}
hipError_t permute_w(hipStream_t st, int d_out, int n, const float* w, const uint32_t* perm, const uint8_t* dead_perm,
                     float* wp) {
  hipLaunchKernelGGL(k_permute_w, dim3(nblk((long)d_out * n)), dim3(256), 0, st, d_out, n, w, perm, dead_perm, wp);
  return hipGetLastError();
}
hipError_t permute_m(hipStream_t st, int n, const float* m, const uint32_t* perm, float damp32, float* mp) {
  hipLaunchKernelGGL(k_permute_m, dim3(nblk((long)n * n)), dim3(256), 0, st, n, m, perm, damp32, mp);
  return hipGetLastError();
}
hipError_t colsq(hipStream_t st, int d_out, int n, const float* w, const uint8_t* dead, double* out) {
  hipLaunchKernelGGL(k_colsq, dim3(nblk(n)), dim3(256), 0, st, d_out, n, w, dead, out);
  return hipGetLastError();
}
hipError_t inv_diag(hipStream_t st, int n, const float* u, float* invd) {
  hipLaunchKernelGGL(k_inv_diag, dim3(nblk(n)), dim3(256), 0, st, n, u, invd);
  return hipGetLastError();
}

static int npl_for(int cnt) {
  if (cnt <= 64) return 1;
  if (cnt <= 128) return 2;
  if (cnt <= 256) return 4;
  if (cnt <= 512) return 8;
  if (cnt <= 1024) return 16;
  return 0;
}

hipError_t gptq_block(hipStream_t st, int rows, int n, int i1, int cnt, int g, int ng, float* w, const float* u,
                      const float* invd, const uint8_t* gbits, int mse, float* scales, float* zeros, uint8_t* codes,
                      float* wq, float* err, unsigned long long* mid, bool groups_in_block) {
  // Lanes per row: as few as keep about two wavefronts per SIMD busy (1024 SIMDs), at least 8.
  // Two 64 KB workgroups per CU, every row resident at once up to 32768 rows: 32 lanes per row
  // and 4 wavefronts per workgroup up to 4096 rows (at most 2 wavefronts per SIMD), 16 lanes and
  // 8 wavefronts up to 16384 (at most 4 per SIMD), 8 lanes and 8 wavefronts above. With 32 or 16
  // lanes a lane's 4 or 8 columns must lie in one group (g a multiple of 8), for the deferred
  // near-midpoint test; other groups take k_gptq_block.
  if (groups_in_block && !mse && cnt <= 128 && i1 % g == 0 && rows >= 2048 && (g % 8 == 0 || rows > 16384)) {
    if (rows > 16384)
      hipLaunchKernelGGL((k_gptq_rows<8, 8>), dim3((rows + 63) / 64), dim3(512), 0, st, rows, n, i1, cnt, g, ng, w, u,
                         invd, gbits, scales, zeros, codes, wq, err, mid);
    else if (rows > 4096)
      hipLaunchKernelGGL((k_gptq_rows<16, 8>), dim3((rows + 31) / 32), dim3(512), 0, st, rows, n, i1, cnt, g, ng, w,
                         u, invd, gbits, scales, zeros, codes, wq, err, mid);
    else
      hipLaunchKernelGGL((k_gptq_rows<32, 4>), dim3((rows + 7) / 8), dim3(256), 0, st, rows, n, i1, cnt, g, ng, w, u,
                         invd, gbits, scales, zeros, codes, wq, err, mid);
    return hipGetLastError();
  }
  const dim3 grid((rows + GB_ROWS - 1) / GB_ROWS), blk(64 * GB_ROWS);
#define GPTQ_CASE(N)                                                                                                   \
  case N:                                                                                                              \
    hipLaunchKernelGGL(k_gptq_block<N>, grid, blk, 0, st, rows, n, i1, cnt, g, ng, w, u, invd, gbits, mse, scales,    \
                       zeros, codes, wq, err, mid);                                                                    \
    break;
  switch (npl_for(cnt)) {
    GPTQ_CASE(1)
    GPTQ_CASE(2)
    GPTQ_CASE(4)
    GPTQ_CASE(8)
    GPTQ_CASE(16)
    default:  // wider than 1024 columns: the working values stay in w
      hipLaunchKernelGGL(k_gptq_block_mem, dim3((rows + 3) / 4), dim3(256), 0, st, rows, n, i1, cnt, g, ng, w, u, invd,
                         gbits, mse, scales, zeros, codes, wq, err, mid);
      break;
  }
#undef GPTQ_CASE
  return hipGetLastError();
}

hipError_t colloss(hipStream_t st, int rows, int n, int rc, const float* err, double* out) {
  const int nchunks = (rows + rc - 1) / rc;
  hipLaunchKernelGGL(k_colloss, dim3(nblk(n), nchunks), dim3(256), 0, st, rows, n, rc, err, out);
  return hipGetLastError();
}

hipError_t sub_f32(hipStream_t st, size_t count, const float* a, const float* b, float* out) {
  hipLaunchKernelGGL(k_sub, dim3(nblk((long)count)), dim3(256), 0, st, (long)count, a, b, out);
  return hipGetLastError();
}

hipError_t pass_accum(hipStream_t st, int rows, int rc, int nchunks, int nref, const double* rlog,
                      const uint32_t* rcnt, int ncd, int cap, const double* clog, const uint32_t* ccnt,
                      const uint8_t* active, double* ld, uint64_t* upd) {
  hipLaunchKernelGGL(k_pass_accum, dim3(nchunks), dim3(256), 0, st, rows, rc, nref, rlog, rcnt, ncd, cap, clog, ccnt,
                     active, ld, upd);
  return hipGetLastError();
}

hipError_t synth_normal(hipStream_t st, uint64_t seed, uint64_t offset, size_t count, float sigma, float* out) {
  if (!count) return hipSuccess;
  hipLaunchKernelGGL(k_synth_normal, dim3(gs_blocks((long)count)), dim3(256), 0, st, seed, offset, (long)count, sigma, out);
  return hipGetLastError();
}

hipError_t synth_tokens(hipStream_t st, uint64_t seed, uint64_t row0, size_t t, size_t n, const float* ch_scale,
                        const uint8_t* heavy, float* x) {
  if (!t || !n) return hipSuccess;
  hipLaunchKernelGGL(k_synth_tokens, dim3(gs_blocks((long)(t * n))), dim3(256), 0, st, seed, row0, (long)t, (int)n, ch_scale,
                     heavy, x);
  return hipGetLastError();
}
hipError_t synth_perturb(hipStream_t st, uint64_t seed, uint64_t offset, size_t count, float sigma, const float* x,
                         float* out) {
  if (!count) return hipSuccess;
  hipLaunchKernelGGL(k_synth_perturb, dim3(gs_blocks((long)count)), dim3(256), 0, st, seed, offset, (long)count, sigma, x,
                     out);
  return hipGetLastError();
}

hipError_t f64_to_f32(hipStream_t st, size_t count, const double* a, float* b) {
  if (!count) return hipSuccess;
  hipLaunchKernelGGL(k_f64_to_f32, dim3(gs_blocks((long)count)), dim3(256), 0, st, (long)count, a, b);
  return hipGetLastError();
}

hipError_t proxy_reduce(hipStream_t st, size_t count, const float* e, const float* eh, double* partial, int nblocks) {
  hipLaunchKernelGGL(k_proxy_reduce, dim3(nblocks), dim3(256), 0, st, (long)count, e, eh, partial);
  return hipGetLastError();
}

}  // namespace cdclq
