// Phase-2 kernels (src/engine.rs:534-670): the repair gradient G = E H[:, c0:c0+wd] on the matrix
// cores, and the refit / coordinate-descent sweeps that consume it.
//
// Gradient. The reference computes G with matrixmultiply (k = n): per element a fused chain over
// each KC = 256 panel of k, panels folded in order. k_panel_gemm computes every panel's chain in
// parallel with v_mfma_f32_32x32x1_2b_f32 (K = 1, single rounding per product, bit-identical to
// fmaf) and stores the per-panel values; k_fold then folds them in panel order, one thread per
// element. Workgroup: 128 rows x 64 cols x one panel, E and the panel of H staged in
// double-buffered LDS.
//
// Sweeps. The refit of a group of at most 128 columns computes U H_CC for 64 rows on the matrix
// cores from H_CC staged in LDS (wider groups: one wavefront per row, H_CC from L2). The descent
// runs one wavefront per row, columns over lanes: it evaluates all columns of a sub-block at once
// and touches a row of H_sb only when a code moves, reading it from L2.
#include <algorithm>
#include <atomic>
#include <cstdint>
#include <type_traits>

#include "cdclq_dev.h"
#include "kernels.h"

namespace cdclq {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

typedef float v32f __attribute__((ext_vector_type(32)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int PR = 128;  // rows per panel-GEMM workgroup (32 per wave)
constexpr int PC = 64;   // cols per panel-GEMM workgroup

__device__ __forceinline__ v32f mfma32(float a, float b, v32f c) {
  return __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, c, 0, 0, 0);
}

// Work unit: 128 rows x 64 cols x one KC panel. Wave w owns rows 32w..32w+31 as one
// v_mfma_f32_32x32x1_2b accumulator whose two blocks are the column halves: lanes i and 32 + i
// supply A row i, lane L supplies B column L. SK = k per LDS stage; the E stage is row-major with
// a padded stride (16-byte aligned rows, conflict-free b128 reads), the B stage is k-major.
//
// The grid is sized to the resident workgroup slots and each workgroup walks a contiguous range
// of units (panels fastest, so consecutive units continue along the same E rows). The stage
// pipeline runs across unit boundaries: the first stage of the next unit is loaded while the last
// stage of the current one is multiplied, and the accumulator is written out and cleared between
// them, so no workgroup pays a cold start per panel.
template <int SK, bool VEC4>
__global__ __launch_bounds__(256) void k_panel_gemm(int m, int wd, int k, const float* __restrict__ A, long lda,
                                                    const float* __restrict__ B, long ldb, float* __restrict__ P,
                                                    int nunits, const int* __restrict__ rtiles, int nrt) {
  constexpr int ES = SK + 4;
  constexpr int EQ = PR * SK / 4 / 256;  // float4 of E per thread per stage
  constexpr int HQ = SK * PC / 4 / 256;  // float4 of B per thread per stage
  constexpr int K4 = SK / 4;             // float4 per E row per stage
  static_assert(EQ >= 1 && HQ >= 1, "stage too small for the workgroup");
  __shared__ float Es[2][PR * ES];
  __shared__ float Hs[2][SK * PC];
  const int np = (k + CDCLQ_KC - 1) / CDCLQ_KC;
  const int u0 = (int)((long)blockIdx.x * nunits / gridDim.x);
  const int u1 = (int)((long)(blockIdx.x + 1) * nunits / gridDim.x);
  if (u0 >= u1) return;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  struct Unit {
    int r0, cb, p, k0, kc, nst;
  };
  auto unit = [&](int u) {
    Unit t;
    const int ct = u / (nrt * np), rem = u % (nrt * np);
    t.r0 = (rtiles ? rtiles[rem / np] : rem / np) * PR;
    t.p = rem % np;
    t.cb = ct * PC;
    t.k0 = t.p * CDCLQ_KC;
    t.kc = min(CDCLQ_KC, k - t.k0);
    t.nst = (t.kc + SK - 1) / SK;
    return t;
  };
  float4 pe[EQ], ph[HQ];
  // VEC4: unconditional 16-byte loads from clamped addresses (rows >= m only feed outputs that are
  // never stored; k slots past the panel are replaced below); otherwise guarded scalar loads.
  auto gload = [&](const Unit& t, int ks) {
#pragma unroll
    for (int q = 0; q < EQ; ++q) {
      const int e = tid + 256 * q;
      const int r = t.r0 + e / K4, kk = ks + (e % K4) * 4;
      if (VEC4) {
        pe[q] = *reinterpret_cast<const float4*>(A + (long)min(r, m - 1) * lda + t.k0 + min(kk, t.kc - 4));
      } else {
        float4 v = make_float4(-0.f, -0.f, -0.f, -0.f);
        if (r < m) {
          const float* src = A + (long)r * lda + t.k0 + kk;
          if (kk < t.kc) v.x = src[0];
          if (kk + 1 < t.kc) v.y = src[1];
          if (kk + 2 < t.kc) v.z = src[2];
          if (kk + 3 < t.kc) v.w = src[3];
        }
        pe[q] = v;
      }
    }
#pragma unroll
    for (int q = 0; q < HQ; ++q) {
      const int e = tid + 256 * q;  // kk = e >> 4, c4 = (e & 15) * 4
      const int kk = ks + (e >> 4), c = t.cb + (e & 15) * 4;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (kk < t.kc) {
        const float* src = B + (long)(t.k0 + kk) * ldb + c;
        if (c < wd) v.x = src[0];
        if (c + 1 < wd) v.y = src[1];
        if (c + 2 < wd) v.z = src[2];
        if (c + 3 < wd) v.w = src[3];
      }
      ph[q] = v;
    }
  };
  auto lstore = [&](int buf, const Unit& t, int ks) {
#pragma unroll
    for (int q = 0; q < EQ; ++q) {
      const int e = tid + 256 * q;
      float4 v = pe[q];
      // k is a multiple of 4 under VEC4, so a slot is either wholly inside the panel or wholly past
      // its end (then the clamped load read other data). Past the end, E is -0 and B is +0: the
      // step fma(-0, +0, c) = c + (-0) = c leaves every chain value unchanged, -0 included.
      if (VEC4 && ks + (e % K4) * 4 >= t.kc) v = make_float4(-0.f, -0.f, -0.f, -0.f);
      *reinterpret_cast<float4*>(&Es[buf][(e / K4) * ES + (e % K4) * 4]) = v;
    }
#pragma unroll
    for (int q = 0; q < HQ; ++q) {
      const int e = tid + 256 * q;
      *reinterpret_cast<float4*>(&Hs[buf][(e >> 4) * PC + (e & 15) * 4]) = ph[q];
    }
  };
  v32f acc = {};
  auto compute = [&](int buf) {
    const float* es = &Es[buf][(32 * wv + (lane & 31)) * ES];
    const float* hs = &Hs[buf][lane];
#pragma unroll
    for (int k4 = 0; k4 < SK; k4 += 4) {
      const float4 a = *reinterpret_cast<const float4*>(es + k4);
      acc = mfma32(a.x, hs[(k4 + 0) * PC], acc);
      acc = mfma32(a.y, hs[(k4 + 1) * PC], acc);
      acc = mfma32(a.z, hs[(k4 + 2) * PC], acc);
      acc = mfma32(a.w, hs[(k4 + 3) * PC], acc);
    }
  };
  int u = u0, s = 0, buf = 0;
  Unit cur = unit(u);
  gload(cur, 0);
  lstore(0, cur, 0);
  __syncthreads();
  while (true) {
    // the stage after (u, s) in this workgroup's sequence
    int un = u, sn = s + 1;
    Unit nxt = cur;
    if (sn >= cur.nst) {
      un = u + 1;
      sn = 0;
      if (un < u1) nxt = unit(un);
    }
    const bool more = un < u1;
    if (more) gload(nxt, sn * SK);
    compute(buf);
    if (sn == 0) {  // (u, s) was the unit's last stage: write its chains and start the next
      // block b = r >> 4 (cols 32b..), row i = (r & 3) + 8 * ((r & 15) >> 2) + 4 * (lane >> 5), col j = lane & 31
#pragma unroll
      for (int r = 0; r < 32; ++r) {
        const int row = cur.r0 + 32 * wv + (r & 3) + 8 * ((r & 15) >> 2) + 4 * (lane >> 5);
        const int col = cur.cb + 32 * (r >> 4) + (lane & 31);
        if (row < m && col < wd) P[((long)cur.p * m + row) * wd + col] = acc[r];
      }
      acc = v32f{};
    }
    if (!more) break;
    lstore(buf ^ 1, nxt, sn * SK);
    __syncthreads();
    buf ^= 1;
    u = un;
    s = sn;
    cur = nxt;
  }
}

// Direct-to-LDS variant of k_panel_gemm, used when k % 32 == 0, wd % 4 == 0 and the rows of E and
// H are 16-byte aligned. Stages are filled with global_load_lds_dwordx4 into a ring of three, two
// stages in flight behind the one being multiplied, one bare barrier per stage; units, the MFMA
// mapping and the outputs are those of k_panel_gemm. Stage layout: E as [128 rows][8 slots][4],
// slot s of row r holding k-quad s ^ (r & 7) (load i: lane l -> row 8 i + (l >> 3), so each load
// reads eight whole 128-byte row segments, and the XOR keeps the b128 reads of 32 rows free of bank
// conflicts), then B as [32 k][64 cols] (load j: lane l -> k row 4 j + (l >> 4), columns
// 4 (l & 15) .. +3). Rows past m and columns past wd are read from clamped addresses and only
// reach outputs that are never stored. The per-panel chains are written with nontemporal stores
// (and k_fold reads them with nontemporal loads): they are used once, and cached they would evict
// E, which the next step streams again and which fits the last-level cache on its own.
constexpr int DSK = 32;
constexpr int DNB = 3;
constexpr int DSTAGE = DSK * PR + DSK * PC;  // floats per stage (E 4096 + B 2048)
constexpr int DPW = DSTAGE / 256 / 4;        // 1 KB loads per wave and stage (6)

// DIRECT (C != null: the GPTQ lazy trailing update): the unit covers all of k, one chain per
// kfold steps (kfold <= 256: one KC panel), each folded straight into the C values held in
// registers in k order, C = fma(alpha, chain, C), starting from beta_one ? C : 0 -- one block's
// update (src/engine.rs:452-471) per kfold, several consecutive blocks per launch.
// Otherwise (the repair gradient) the chains go to P.
template <bool DIRECT>
__global__ __launch_bounds__(256) void k_panel_dma(int m, int wd, int k, const float* __restrict__ A, long lda,
                                                   const float* __restrict__ B, long ldb, float* __restrict__ P,
                                                   int nunits, const int* __restrict__ rtiles, int nrt,
                                                   float* __restrict__ C, long ldc, float alpha, int beta_one,
                                                   int kfold) {
  __shared__ float R[DNB][DSTAGE];
  const int np = k / CDCLQ_KC + (k % CDCLQ_KC != 0);
  // With a full grid (two workgroups per CU), workgroups j and j + G/2 end up on the same CU: the
  // first half fills every CU once and the second half pairs up with it in dispatch order. They
  // take adjacent unit ranges 2j and 2j + 1, whose sizes (floor and ceiling of units / G) add up
  // to the CU's fair share when units / G is not whole.
  const int G = gridDim.x, j = blockIdx.x;
  const int v = (G & 1) ? j : (j < G / 2 ? 2 * j : 2 * (j - G / 2) + 1);
  const int u0 = (int)((long)v * nunits / G);
  const int u1 = (int)((long)(v + 1) * nunits / G);
  if (u0 >= u1) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  struct Unit {
    int r0, cb, p, k0, nst;
  };
  auto unit = [&](int u) {
    Unit t;
    if (DIRECT) {  // all of k; column tiles fastest, so consecutive units share their E tile
      const int nct = (wd + PC - 1) / PC;
      t.r0 = (u / nct) * PR;
      t.cb = (u % nct) * PC;
      t.p = 0;
      t.k0 = 0;
      t.nst = k / DSK;
    } else {
      const int ct = u / (nrt * np), rem = u % (nrt * np);
      t.r0 = (rtiles ? rtiles[rem / np] : rem / np) * PR;
      t.p = rem % np;
      t.cb = ct * PC;
      t.k0 = t.p * CDCLQ_KC;
      t.nst = min(CDCLQ_KC, k - t.k0) / DSK;
    }
    return t;
  };
  const uint32_t lds0 = lds_offset(&R[0][0]);
  // Issue cursor (unit iu_idx, stage is; ring slot fi % DNB). Per-lane source offsets are fixed for
  // a unit (relative to a uniform base), so a stage's loads cost one address add each.
  int iu_idx = u0, is = 0, fi = 0;
  Unit iu = unit(u0);
  bool ivalid = true;
  int off[DPW];
  auto unit_offsets = [&]() {
#pragma unroll
    for (int q = 0; q < DPW; ++q) {
      const int ins = wv + 4 * q;  // loads 0..15 are E (q < 4), 16..23 are B (q >= 4)
      if (q < 4) {  // E rows 8 ins .. 8 ins + 7, relative to row r0 and column k0 + ks
        const int rl = 8 * ins + (lane >> 3);
        off[q] = (min(iu.r0 + rl, m - 1) - iu.r0) * (int)lda + 4 * ((lane & 7) ^ (rl & 7));
      } else {  // B k rows 4 j .. 4 j + 3, relative to row k0 + ks and column 0
        off[q] = (4 * (ins - 16) + (lane >> 4)) * (int)ldb + min(iu.cb + 4 * (lane & 15), wd - 4);
      }
    }
  };
  unit_offsets();
  auto issue_next = [&]() {
    if (!ivalid) return;
    const uint32_t buf = lds0 + (uint32_t)((fi % DNB) * DSTAGE * 4);
    const int ks = iu.k0 + is * DSK;
    const float* ea = A + (long)iu.r0 * lda + ks;
    const float* hb = B + (long)ks * ldb;
#pragma unroll
    for (int q = 0; q < DPW; ++q) {
      const int ins = wv + 4 * q;  // each load fills 1 KB: stage slot 256 ins (floats)
      dma16_untracked((q < 4 ? ea : hb) + off[q], buf + 1024u * (uint32_t)ins);
    }
    ++fi;
    if (++is >= iu.nst) {
      if (++iu_idx < u1) {
        iu = unit(iu_idx);
        is = 0;
        unit_offsets();
      } else {
        ivalid = false;
      }
    }
  };
  issue_next();
  issue_next();
  const int er = 32 * wv + (lane & 31);
  // Vector memory operations complete in issue order, so "at most the newest DPW outstanding"
  // means everything older -- stage fc and any stores issued before stage fc + 1's loads -- is
  // done. With C, at a unit's last stage the next load is issued after the unit's C stores, so the
  // wait that follows does not also hold back the stage after. Without C, a unit's chains stay in
  // acc until the next unit's first stage has landed and are stored there, before that stage's
  // load is issued: the stores then have the whole stage to complete before the next wait.
  int fc = 0;
  v32f acc = {};
  Unit pu = iu;  // without C: the unit whose chains acc holds
  // Register r of the accumulator holds row (r & 3) + 8 ((r & 15) >> 2) + 4 (lane >> 5) of the
  // wave's 32 rows and column 32 (r >> 4) + (lane & 31): relative to the lane's first element its
  // offset is uniform, so a whole tile (the common case, a uniform test) needs one address per lane.
  auto roff = [](int r, long ld) { return ((r & 3) + 8 * ((r & 15) >> 2)) * ld + 32 * (r >> 4); };
  auto store_p = [&](const Unit& t) {
    if (t.r0 + PR <= m && t.cb + PC <= wd) {
      float* q = P + ((long)t.p * m + t.r0 + 32 * wv + 4 * (lane >> 5)) * wd + t.cb + (lane & 31);
#pragma unroll
      for (int r = 0; r < 32; ++r) __builtin_nontemporal_store(acc[r], q + roff(r, wd));
      return;
    }
    // block b = r >> 4 (cols 32b..), row i = (r & 3) + 8 * ((r & 15) >> 2) + 4 * (lane >> 5), col j = lane & 31
#pragma unroll
    for (int r = 0; r < 32; ++r) {
      const int row = t.r0 + 32 * wv + (r & 3) + 8 * ((r & 15) >> 2) + 4 * (lane >> 5);
      const int col = t.cb + 32 * (r >> 4) + (lane & 31);
      if (row < m && col < wd) __builtin_nontemporal_store(acc[r], &P[((long)t.p * m + row) * wd + col]);
    }
  };
  for (int cu_idx = u0; cu_idx < u1; ++cu_idx) {
    const Unit cu = unit(cu_idx);
    float cv[32];  // with C: the unit's C values, loaded while its stages are multiplied
    for (int cs = 0; cs < cu.nst; ++cs) {
      // this wave's part of stage fc has landed once at most the next stage's loads are outstanding
      if (fi - fc >= 2)
        wait_vmcnt<DPW>();
      else
        wait_vmcnt<0>();
      __builtin_amdgcn_s_barrier();  // publishes all parts; all reads of stage fc - 1 are done
      if (!DIRECT && cs == 0 && cu_idx > u0) {
        store_p(pu);
        acc = v32f{};
      }
      // C is loaded before the stage after next, so the next stage's wait (everything but the
      // newest stage's loads) covers it rather than also holding back that stage.
      if (DIRECT && cs == 0) {
        if (!beta_one) {
#pragma unroll
          for (int r = 0; r < 32; ++r) cv[r] = 0.0f;
        } else if (cu.r0 + PR <= m && cu.cb + PC <= wd) {
          const float* q = C + (long)(cu.r0 + 32 * wv + 4 * (lane >> 5)) * ldc + cu.cb + (lane & 31);
#pragma unroll
          for (int r = 0; r < 32; ++r) cv[r] = q[roff(r, ldc)];
        } else {
#pragma unroll
          for (int r = 0; r < 32; ++r) {  // clamped addresses; values outside m x wd are never used
            const int row = min(cu.r0 + 32 * wv + (r & 3) + 8 * ((r & 15) >> 2) + 4 * (lane >> 5), m - 1);
            const int col = min(cu.cb + 32 * (r >> 4) + (lane & 31), wd - 1);
            cv[r] = C[(long)row * ldc + col];
          }
        }
      }
      if (!DIRECT || cs + 1 < cu.nst) issue_next();  // into the slot of stage fc - 1
      const float* buf = &R[fc % DNB][0];
      const float* es = buf + 32 * er;
      const float* hs = buf + DSK * PR + lane;
#pragma unroll
      for (int q = 0; q < DSK / 4; ++q) {
        const float4 a = *reinterpret_cast<const float4*>(es + 4 * (q ^ (er & 7)));
        acc = mfma32(a.x, hs[(4 * q + 0) * PC], acc);
        acc = mfma32(a.y, hs[(4 * q + 1) * PC], acc);
        acc = mfma32(a.z, hs[(4 * q + 2) * PC], acc);
        acc = mfma32(a.w, hs[(4 * q + 3) * PC], acc);
      }
      ++fc;
      if (DIRECT && cs + 1 < cu.nst && ((cs + 1) * DSK) % kfold == 0) {  // a block's chain is complete
#pragma unroll
        for (int r = 0; r < 32; ++r) cv[r] = __builtin_fmaf(alpha, acc[r], cv[r]);
        acc = v32f{};
      }
    }
    if (DIRECT) {
      if (cu.r0 + PR <= m && cu.cb + PC <= wd) {
        float* q = C + (long)(cu.r0 + 32 * wv + 4 * (lane >> 5)) * ldc + cu.cb + (lane & 31);
#pragma unroll
        for (int r = 0; r < 32; ++r) q[roff(r, ldc)] = __builtin_fmaf(alpha, acc[r], cv[r]);
      } else {
#pragma unroll
        for (int r = 0; r < 32; ++r) {
          const int row = cu.r0 + 32 * wv + (r & 3) + 8 * ((r & 15) >> 2) + 4 * (lane >> 5);
          const int col = cu.cb + 32 * (r >> 4) + (lane & 31);
          if (row < m && col < wd) C[(long)row * ldc + col] = __builtin_fmaf(alpha, acc[r], cv[r]);
        }
      }
      acc = v32f{};
      issue_next();  // the load deferred at the unit's last stage
    } else {
      pu = cu;
    }
  }
  if (!DIRECT) store_p(pu);
}

// The lazy trailing update C = fma(alpha, A B, C) (k <= 256, one panel) on 128 x 128 tiles: 8
// waves, wave w rows 32 (w & 3) .. +31 and columns 64 (w >> 2) .. +63, one E tile read per 128
// columns; the stages, load plan and per-element chain are those of k_panel_dma<true> (B stage
// [32 k][128 cols], 2 k rows per load). Used when there are enough 128 x 128 tiles to give
// every CU one. Without C (DIRECT false) the same tile computes the repair gradient's 128-column
// per-panel chains (units (row tile, panel)), stored to P as k_panel_dma<false> stores them, when
// there are at least four units per workgroup.
constexpr int LPC = 128;
constexpr int LSTAGE = DSK * PR + DSK * LPC;   // 8192 floats = 32 KB
constexpr int LDPW = LSTAGE / 512 / 4;         // 4 loads per wave and stage
template <bool DIRECT>
__global__ __launch_bounds__(512) void k_lazy_wide(int m, int wd, int k, const float* __restrict__ A, long lda,
                                                   const float* __restrict__ B, long ldb, float* __restrict__ C,
                                                   long ldc, float alpha, int nunits, float* __restrict__ P,
                                                   const int* __restrict__ rtiles, int kfold) {
  // With C a ring of two stages (64 KB), so that a narrow update's workgroup (72 KB) fits beside
  // this one on each CU: this kernel runs on a side stream while the main stream updates and
  // sweeps the next blocks. Without C the ring of three.
  constexpr int NB = DIRECT ? 2 : DNB;
  __shared__ float R[NB][LSTAGE];
  const int nct = (wd + LPC - 1) / LPC;
  const int np = k / CDCLQ_KC + (k % CDCLQ_KC != 0);
  const int u0 = (int)((long)blockIdx.x * nunits / gridDim.x);
  const int u1 = (int)((long)(blockIdx.x + 1) * nunits / gridDim.x);
  if (u0 >= u1) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = wv & 3, wc = wv >> 2;
  struct Unit {
    int r0, cb, p, k0, nst;
  };
  auto unit = [&](int u) {
    Unit t;
    if (DIRECT) {  // all of k (chains folded every kfold), column tiles fastest
      t.r0 = (u / nct) * PR;
      t.cb = (u % nct) * LPC;
      t.p = 0;
      t.k0 = 0;
      t.nst = k / DSK;
    } else {  // the repair gradient, wd == 128: (row tile, panel), panels fastest
      t.r0 = (rtiles ? rtiles[u / np] : u / np) * PR;
      t.cb = 0;
      t.p = u % np;
      t.k0 = t.p * CDCLQ_KC;
      t.nst = min(CDCLQ_KC, k - t.k0) / DSK;
    }
    return t;
  };
  const uint32_t lds0 = lds_offset(&R[0][0]);
  int iu_idx = u0, is = 0, fi = 0;
  Unit iu = unit(u0);
  bool ivalid = true;
  int off[LDPW];
  auto unit_offsets = [&]() {
#pragma unroll
    for (int q = 0; q < LDPW; ++q) {
      const int ins = wv + 8 * q;
      if (q < 2) {
        const int rl = 8 * ins + (lane >> 3);
        off[q] = (min(iu.r0 + rl, m - 1) - iu.r0) * (int)lda + 4 * ((lane & 7) ^ (rl & 7));
      } else {
        off[q] = (2 * (ins - 16) + (lane >> 5)) * (int)ldb + min(iu.cb + 4 * (lane & 31), wd - 4);
      }
    }
  };
  unit_offsets();
  auto issue_next = [&]() {
    if (!ivalid) return;
    const uint32_t buf = lds0 + (uint32_t)((fi % NB) * LSTAGE * 4);
    const int ks = iu.k0 + is * DSK;
    const float* ea = A + (long)iu.r0 * lda + ks;
    const float* hb = B + (long)ks * ldb;
#pragma unroll
    for (int q = 0; q < LDPW; ++q) {
      const int ins = wv + 8 * q;
      dma16_untracked((q < 2 ? ea : hb) + off[q], buf + 1024u * (uint32_t)ins);
    }
    ++fi;
    if (++is >= iu.nst) {
      if (++iu_idx < u1) {
        iu = unit(iu_idx);
        is = 0;
        unit_offsets();
      } else {
        ivalid = false;
      }
    }
  };
  issue_next();
  if (NB == 3) issue_next();
  const int er = 32 * wr + (lane & 31);
  // Without C, ordering as in k_panel_dma: the chains are stored (nontemporal) at the next unit's
  // first stage. With C (ring of two) each stage waits for everything issued before it -- its own
  // loads, issued one stage ahead, the unit's C loads and the previous unit's C stores -- and the
  // next stage's loads are issued after the barrier that retires the reads of its slot.
  int fc = 0;
  v32f acc = {};
  Unit pu = iu;
  // as in k_panel_dma: a whole tile stores from one address per lane plus uniform offsets
  auto roff = [](int r, long ld) { return ((r & 3) + 8 * ((r & 15) >> 2)) * ld + 32 * (r >> 4); };
  auto store_p = [&](const Unit& t) {
    if (t.r0 + PR <= m && LPC <= wd) {
      float* q = P + ((long)t.p * m + t.r0 + 32 * wr + 4 * (lane >> 5)) * wd + 64 * wc + (lane & 31);
#pragma unroll
      for (int r = 0; r < 32; ++r) __builtin_nontemporal_store(acc[r], q + roff(r, wd));
      return;
    }
#pragma unroll
    for (int r = 0; r < 32; ++r) {
      const int row = t.r0 + 32 * wr + (r & 3) + 8 * ((r & 15) >> 2) + 4 * (lane >> 5);
      const int col = 64 * wc + 32 * (r >> 4) + (lane & 31);
      if (row < m && col < wd) __builtin_nontemporal_store(acc[r], &P[((long)t.p * m + row) * wd + col]);
    }
  };
  for (int cu_idx = u0; cu_idx < u1; ++cu_idx) {
    const Unit cu = unit(cu_idx);
    float cv[32];
    for (int cs = 0; cs < cu.nst; ++cs) {
      if (!DIRECT && fi - fc >= 2)
        wait_vmcnt<LDPW>();
      else
        wait_vmcnt<0>();
      __builtin_amdgcn_s_barrier();
      if (!DIRECT && cs == 0 && cu_idx > u0) {
        store_p(pu);
        acc = v32f{};
      }
      if (DIRECT && cs == 0) {
        if (cu.r0 + PR <= m && cu.cb + LPC <= wd) {
          const float* q = C + (long)(cu.r0 + 32 * wr + 4 * (lane >> 5)) * ldc + cu.cb + 64 * wc + (lane & 31);
#pragma unroll
          for (int r = 0; r < 32; ++r) cv[r] = q[roff(r, ldc)];
        } else {
#pragma unroll
          for (int r = 0; r < 32; ++r) {
            const int row = min(cu.r0 + 32 * wr + (r & 3) + 8 * ((r & 15) >> 2) + 4 * (lane >> 5), m - 1);
            const int col = min(cu.cb + 64 * wc + 32 * (r >> 4) + (lane & 31), wd - 1);
            cv[r] = C[(long)row * ldc + col];
          }
        }
      }
      issue_next();
      const float* buf = &R[fc % NB][0];
      const float* es = buf + 32 * er;
      const float* hs = buf + DSK * PR + 64 * wc + lane;
#pragma unroll
      for (int q = 0; q < DSK / 4; ++q) {
        const float4 a = *reinterpret_cast<const float4*>(es + 4 * (q ^ (er & 7)));
        acc = mfma32(a.x, hs[(4 * q + 0) * LPC], acc);
        acc = mfma32(a.y, hs[(4 * q + 1) * LPC], acc);
        acc = mfma32(a.z, hs[(4 * q + 2) * LPC], acc);
        acc = mfma32(a.w, hs[(4 * q + 3) * LPC], acc);
      }
      ++fc;
      if (DIRECT && cs + 1 < cu.nst && ((cs + 1) * DSK) % kfold == 0) {  // a block's chain is complete
#pragma unroll
        for (int r = 0; r < 32; ++r) cv[r] = __builtin_fmaf(alpha, acc[r], cv[r]);
        acc = v32f{};
      }
    }
    if (DIRECT) {
      if (cu.r0 + PR <= m && cu.cb + LPC <= wd) {
        float* q = C + (long)(cu.r0 + 32 * wr + 4 * (lane >> 5)) * ldc + cu.cb + 64 * wc + (lane & 31);
#pragma unroll
        for (int r = 0; r < 32; ++r) q[roff(r, ldc)] = __builtin_fmaf(alpha, acc[r], cv[r]);
      } else {
#pragma unroll
        for (int r = 0; r < 32; ++r) {
          const int row = cu.r0 + 32 * wr + (r & 3) + 8 * ((r & 15) >> 2) + 4 * (lane >> 5);
          const int col = cu.cb + 64 * wc + 32 * (r >> 4) + (lane & 31);
          if (row < m && col < wd) C[(long)row * ldc + col] = __builtin_fmaf(alpha, acc[r], cv[r]);
        }
      }
      acc = v32f{};
    } else {
      pu = cu;
    }
  }
  if (!DIRECT) store_p(pu);
}

// G[r][c] = ordered fold of the panel chains (alpha 1, beta 0): C = fma(1, P_p, C) for p = 0, 1, ...
// One thread per element of the listed 128-row tiles, panel loads unrolled so many are in flight.
// The kernel streams the chains from HBM at 5-6 TB/s; keeping 32 loads in flight per thread
// instead of 8 measured no faster.
__global__ __launch_bounds__(256) void k_fold(int m, int wd, int np, const int* __restrict__ rtiles, long count,
                                              const float* __restrict__ P, float* __restrict__ G) {
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= count) return;
  const long tw = (long)PR * wd;
  const int t = (int)(idx / tw), within = (int)(idx % tw);
  const int row = (rtiles ? rtiles[t] : t) * PR + within / wd;
  if (row >= m) return;
  const long g = (long)row * wd + within % wd;
  const long pstride = (long)m * wd;
  const float* src = P + g;
  float acc = 0.0f;
  int p = 0;
  for (; p + 8 <= np; p += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = __builtin_nontemporal_load(src + (long)(p + u) * pstride);
#pragma unroll
    for (int u = 0; u < 8; ++u) acc = __builtin_fmaf(1.0f, v[u], acc);
  }
  for (; p < np; ++p) acc = __builtin_fmaf(1.0f, __builtin_nontemporal_load(src + (long)p * pstride), acc);
  G[g] = acc;
}

// Closed-form f16 scale refit of group gi (src/engine.rs:543-587) for groups wider than 128
// columns (narrower ones take k_refit_mfma). One wavefront per row, columns over lanes; H_CC is
// read from L2.
template <int NPL>
__global__ __launch_bounds__(256) void k_refit(int rows, int n, int ng, int g, int gi, int rc, const float* __restrict__ G,
                                               const float* __restrict__ h32,
                                               const uint8_t* __restrict__ codes, float* __restrict__ scales,
                                               const float* __restrict__ zeros, float* __restrict__ wq,
                                               float* __restrict__ e, const uint8_t* __restrict__ active,
                                               double* __restrict__ dlog, uint32_t* __restrict__ dcnt) {
  constexpr int RW = 1;
  const int c0 = gi * g, wd = min(c0 + g, n) - c0;
  const int lane = threadIdx.x & 63;
  const int rbase = __builtin_amdgcn_readfirstlane((blockIdx.x * 4 + (threadIdx.x >> 6)) * RW);
  bool live[RW];
  bool any = false;
#pragma unroll
  for (int q = 0; q < RW; ++q) {
    const int r = rbase + q;
    live[q] = r < rows && active[r / rc];
    any = any || live[q];
    if (r < rows && !live[q] && lane == 0) dcnt[r] = 0;
  }
  if (!any) return;

  float uu[RW][NPL], gg[RW][NPL], acc[RW][NPL], cvh[RW][NPL];
#pragma unroll
  for (int q = 0; q < RW; ++q) {
    const int r = rbase + q;
    const float z = live[q] ? zeros[(long)r * ng + gi] : 0.0f;
#pragma unroll
    for (int s = 0; s < NPL; ++s) {
      const int k = s * 64 + lane;
      const bool in = live[q] && k < wd;
      uu[q][s] = in ? (float)codes[(long)r * n + c0 + k] - z : 0.0f;
      gg[q][s] = in ? G[(long)r * wd + k] : 0.0f;
      acc[q][s] = 0.0f;
      cvh[q][s] = 0.0f;
    }
  }
  // hu[k2] = sum_k uu[k] * H[c0+k][c0+k2] (sgemm at src/engine.rs:560: fma chain per KC panel)
  auto hu_step = [&](int k, int s1, int kl) {
    float h[NPL];
#pragma unroll
    for (int s2 = 0; s2 < NPL; ++s2) {
      const int k2 = s2 * 64 + lane;
      h[s2] = k2 < wd ? h32[(long)(c0 + k) * n + c0 + k2] : 0.0f;
    }
#pragma unroll
    for (int q = 0; q < RW; ++q) {
      const float uk = readlane(uu[q][s1], kl);
#pragma unroll
      for (int s2 = 0; s2 < NPL; ++s2) acc[q][s2] = __builtin_fmaf(uk, h[s2], acc[q][s2]);
    }
  };
#pragma unroll
  for (int s1 = 0; s1 < NPL; ++s1) {
    const int kb = s1 * 64;
    if (kb >= wd) break;
    const int cnt = min(64, wd - kb);
    if (cnt == 64) {
#pragma unroll 16
      for (int kl = 0; kl < 64; ++kl) hu_step(kb + kl, s1, kl);
    } else {
      for (int kl = 0; kl < cnt; ++kl) hu_step(kb + kl, s1, kl);
    }
    if (((kb + 64) % CDCLQ_KC) == 0 || kb + cnt == wd) {  // panel end: C = fma(1, chain, C)
#pragma unroll
      for (int q = 0; q < RW; ++q)
#pragma unroll
        for (int s2 = 0; s2 < NPL; ++s2) {
          cvh[q][s2] = __builtin_fmaf(1.0f, acc[q][s2], cvh[q][s2]);
          acc[q][s2] = 0.0f;
        }
    }
  }
  // num = sum_k u_k g_k, den = sum_k u_k hu_k, sequential in k (src/engine.rs:562-566). The
  // products are rounded on their own before each add, so every lane forms its column's products
  // at once and the sequential part is one broadcast and one add per term.
#pragma unroll
  for (int q = 0; q < RW; ++q)
#pragma unroll
    for (int s = 0; s < NPL; ++s) {
      gg[q][s] = uu[q][s] * gg[q][s];    // u_k g_k
      cvh[q][s] = uu[q][s] * cvh[q][s];  // u_k hu_k
    }
  float num[RW], den[RW];
#pragma unroll
  for (int q = 0; q < RW; ++q) num[q] = den[q] = 0.0f;
  auto nd_step = [&](int s1, int kl) {
#pragma unroll
    for (int q = 0; q < RW; ++q) {
      num[q] = num[q] + readlane(gg[q][s1], kl);
      den[q] = den[q] + readlane(cvh[q][s1], kl);
    }
  };
#pragma unroll
  for (int s1 = 0; s1 < NPL; ++s1) {
    const int kb = s1 * 64;
    if (kb >= wd) break;
    const int cnt = min(64, wd - kb);
    if (cnt == 64) {
#pragma unroll 16
      for (int kl = 0; kl < 64; ++kl) nd_step(s1, kl);
    } else {
      for (int kl = 0; kl < cnt; ++kl) nd_step(s1, kl);
    }
  }
#pragma unroll
  for (int q = 0; q < RW; ++q) {
    if (!live[q]) continue;
    const int r = rbase + q;
    const float s_old = scales[(long)r * ng + gi];
    uint32_t moved = 0;
    if (den[q] > 1e-30f) {
      const float s_new = rs_maxf(round_f16(s_old + num[q] / den[q]), CDCLQ_F16_MIN_NORMAL);
      const float d = s_new - s_old;
      const float dl32 = (-2.0f * d) * num[q] + (d * d) * den[q];
      if ((double)dl32 < 0.0) {
        if (lane == 0) {
          scales[(long)r * ng + gi] = s_new;
          dlog[r] = (double)dl32;
        }
#pragma unroll
        for (int s = 0; s < NPL; ++s) {
          const int k = s * 64 + lane;
          if (k < wd) {
            const long o = (long)r * n + c0 + k;
            const float ndq = s_new * uu[q][s];
            e[o] = e[o] + (wq[o] - ndq);
            wq[o] = ndq;
          }
        }
        moved = 1;
      }
    }
    if (lane == 0) dcnt[r] = moved;
  }
}

// Matrix-core refit for groups of at most 128 columns, RF_ROWS rows per workgroup, same results as
// k_refit. hu = U H_CC (U = codes - zero, one row per row of the group) is a K = 1 chain per
// element in k order (one KC panel), so a K = 1 MFMA computes it as the sgemm does. 64 rows:
// v_mfma_f32_32x32x1_2b_f32, wave w takes rows 32 (w >> 1) .. +31 and columns 64 (w & 1) .. +63.
// 32 and 16 rows (two resident workgroups per CU, for matrices whose rows fit that way in one
// round): v_mfma_f32_16x16x1_4b_f32, its four 16 x 16 blocks side by side, half the chain latency
// of the 32 x 32 form; wave w takes rows 16 (w >> 1) .. +15 (32 rows; with 16 rows only waves 0
// and 1) and columns 64 (w & 1) .. +63 (lane l supplies A = u of row 16 (w >> 1) + l % 16 and
// B = H_CC column 64 (w & 1) + l; D register r of lane l is row 16 (w >> 1) + 4 (l >> 4) + (r & 3),
// column 64 (w & 1) + 16 (r >> 2) + (l & 15)). A = u is read from the codes
// staged in LDS, B = H_CC staged in LDS. The products u_k hu_k and u_k g_k are then formed in
// parallel into LDS, the sequential sums num = sum u_k g_k and den = sum u_k hu_k run one lane per
// row, and the accepted rows' e and W_hat are updated by the whole workgroup along the columns.
constexpr int RF_CS = 132;  // byte stride of a staged code row (33 dwords: conflict-free by row)
constexpr int RF_PS = 129;  // float stride of a staged product row (odd: conflict-free by row)

__device__ __forceinline__ v16f mfma16(float a, float b, v16f c) {
  return __builtin_amdgcn_mfma_f32_16x16x1f32(a, b, c, 0, 0, 0);
}

template <int RF_ROWS>
__global__ __launch_bounds__(256) void k_refit_mfma(int rows, int n, int ng, int g, int gi, int rc,
                                                    const float* __restrict__ G, const float* __restrict__ h32,
                                                    const uint8_t* __restrict__ codes, float* __restrict__ scales,
                                                    const float* __restrict__ zeros, float* __restrict__ wq,
                                                    float* __restrict__ e, const uint8_t* __restrict__ active,
                                                    double* __restrict__ dlog, uint32_t* __restrict__ dcnt,
                                                    const float* __restrict__ P, int np) {
  // H_CC (zero outside wd x wd), then the products: PH = S[0 ..], PG = S[RF_ROWS * RF_PS ..]
  __shared__ float S[2 * RF_ROWS * RF_PS > 128 * 128 ? 2 * RF_ROWS * RF_PS : 128 * 128];
  __shared__ uint32_t CB[RF_ROWS * RF_CS / 4];
  __shared__ float zrow[RF_ROWS], snew[RF_ROWS];
  __shared__ int mv[RF_ROWS];
  __shared__ int nlive;
  const int c0 = gi * g, wd = min(c0 + g, n) - c0;
  const int r0 = blockIdx.x * RF_ROWS;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  if (tid == 0) nlive = 0;
  __syncthreads();
  if (tid < RF_ROWS) {
    const int r = r0 + tid;
    const bool live = r < rows && active[r / rc];
    if (r < rows && !live) dcnt[r] = 0;
    if (live) atomicAdd(&nlive, 1);
    zrow[tid] = zeros[(long)min(r, rows - 1) * ng + gi];
  }
  __syncthreads();
  if (nlive == 0) return;
  // Whole groups fold the GEMM's per-panel chains with 16-byte loads (below); the first batch of
  // FB0 panels is issued here, so that its latency overlaps the H_CC staging and the hu chains
  // (not in the 64-row form, whose registers would then allow one workgroup per CU).
  constexpr int PER4 = RF_ROWS * 32 / 256;
  constexpr int FB4 = PER4 == 2 ? 16 : (PER4 == 4 ? 8 : 4);
  constexpr int FB0 = RF_ROWS == 64 ? 0 : FB4;
  const bool fvec = P && wd == 128 && (reinterpret_cast<uintptr_t>(P) & 15) == 0;
  const long pstride4 = (long)rows * 128;
  v4f v0[FB0 ? FB0 : 1][PER4];
  auto issue_v0 = [&]() {
    if (FB0) {
#pragma unroll
      for (int u = 0; u < FB0; ++u) {
        const long po = (long)min(u, np - 1) * pstride4;
#pragma unroll
        for (int i = 0; i < PER4; ++i) {
          const int x = tid + 256 * i, rl = x >> 5, k4 = x & 31;
          v0[u][i] = __builtin_nontemporal_load(
              reinterpret_cast<const v4f*>(P + po + (long)min(r0 + rl, rows - 1) * 128 + 4 * k4));
        }
      }
    }
  };
  // whole, 16-byte aligned rows, with chains to fold (the engine always passes them here)
  const bool vec = fvec && (n & 3) == 0 && (c0 & 3) == 0;
  if (vec) {  // stage H_CC with 16-byte loads (16 per thread, all in flight) and the codes by words
    // (issued before the fold's first batch, unconditionally in this branch: vector loads complete
    // in order, so the LDS stores then wait for these loads only)
    v4f hq[16];
    uint32_t cw[RF_ROWS * 32 / 256];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int x = tid + 256 * u;  // float4 slot: row x >> 5, columns 4 (x & 31) ..
      hq[u] = *reinterpret_cast<const v4f*>(h32 + (long)(c0 + (x >> 5)) * n + c0 + 4 * (x & 31));
    }
#pragma unroll
    for (int u = 0; u < RF_ROWS * 32 / 256; ++u) {
      const int x = tid + 256 * u, rl = x >> 5, k4 = x & 31;
      const int r = min(r0 + rl, rows - 1);
      cw[u] = *reinterpret_cast<const uint32_t*>(codes + (long)r * n + c0 + 4 * k4);
    }
    __builtin_amdgcn_sched_barrier(0);
    issue_v0();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 16; ++u) *reinterpret_cast<v4f*>(&S[4 * (tid + 256 * u)]) = hq[u];
#pragma unroll
    for (int u = 0; u < RF_ROWS * 32 / 256; ++u) {
      const int x = tid + 256 * u, rl = x >> 5, k4 = x & 31;
      CB[rl * (RF_CS / 4) + k4] = cw[u];
    }
  } else {  // clamped scalar loads, zero padding outside wd
    if (fvec) issue_v0();
    constexpr int PER = 128 * 128 / 256, BATCH = 16;
#pragma unroll
    for (int b = 0; b < PER; b += BATCH) {
      float v[BATCH];
#pragma unroll
      for (int u = 0; u < BATCH; ++u) {
        const int x = tid + 256 * (b + u);
        v[u] = h32[(long)(c0 + min(x >> 7, wd - 1)) * n + c0 + min(x & 127, wd - 1)];
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < BATCH; ++u) {
        const int x = tid + 256 * (b + u);
        S[x] = ((x >> 7) < wd && (x & 127) < wd) ? v[u] : 0.0f;
      }
    }
    uint8_t* cb = reinterpret_cast<uint8_t*>(CB);
#pragma unroll 8
    for (int i = 0; i < RF_ROWS * 128 / 256; ++i) {
      const int x = tid + 256 * i, rl = x >> 7, k = x & 127;
      const int r = min(r0 + rl, rows - 1);
      cb[rl * RF_CS + k] = k < wd ? codes[(long)r * n + c0 + k] : 0;
    }
  }
  __syncthreads();
  // hu chains on the matrix cores
  constexpr bool R64 = RF_ROWS == 64;
  static_assert(RF_ROWS == 64 || RF_ROWS == 32 || RF_ROWS == 16, "64-, 32- or 16-row workgroups");
  const int wr = RF_ROWS == 16 ? 0 : wv >> 1, wc = wv & 1;
  const bool mwave = RF_ROWS != 16 || wv < 2;
  const int arow = R64 ? 32 * wr + (lane & 31) : 16 * wr + (lane & 15);
  const float za = zrow[arow];
  const uint32_t* crow = CB + arow * (RF_CS / 4);
  const float* hcol = S + 64 * (wc & 1) + lane;
  typedef typename std::conditional<R64, v32f, v16f>::type acc_t;
  acc_t acc = {};
  auto step = [&](float a, float b) {
    if constexpr (R64)
      acc = mfma32(a, b, acc);
    else
      acc = mfma16(a, b, acc);
  };
  if (mwave) {
    int k0 = 0;
    for (; k0 + 8 <= wd; k0 += 8) {
      const uint32_t w0 = crow[k0 >> 2], w1 = crow[(k0 >> 2) + 1];
      float hb[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) hb[j] = hcol[(k0 + j) * 128];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t w = j < 4 ? w0 : w1;
        step((float)((w >> (8 * (j & 3))) & 0xffu) - za, hb[j]);
      }
    }
    for (; k0 < wd; ++k0) {
      const uint32_t w = crow[k0 >> 2];
      step((float)((w >> (8 * (k0 & 3))) & 0xffu) - za, hcol[k0 * 128]);
    }
  }
  __syncthreads();  // every wave is done with H_CC
  const uint8_t* cb = reinterpret_cast<const uint8_t*>(CB);
  float* PH = S;
  float* PG = S + RF_ROWS * RF_PS;
  if (mwave) {
#pragma unroll
    for (int r = 0; r < (R64 ? 32 : 16); ++r) {  // panel end C = fma(1, chain, 0), then u_k * hu_k
      const int row = R64 ? 32 * wr + (r & 3) + 8 * ((r & 15) >> 2) + 4 * (lane >> 5)
                          : 16 * wr + 4 * (lane >> 4) + (r & 3);
      const int col = R64 ? 64 * wc + 32 * (r >> 4) + (lane & 31) : 64 * wc + 16 * (r >> 2) + (lane & 15);
      const float u = (float)cb[row * RF_CS + col] - zrow[row];
      PH[row * RF_PS + col] = u * __builtin_fmaf(1.0f, acc[r], 0.0f);
    }
  }
  if (fvec) {
    // u_k * g_k for whole groups: the same ordered fold with 16-byte loads. Slot x = tid + 256 i
    // covers row x >> 5, columns 4 (x & 31) .. + 3, so a batch of FB4 panels is FB4 * PER4
    // loads a thread (at most 40 in flight, below the wave's 63 outstanding vector loads) and the
    // 56 panels of a 14336-wide input take 3 batches instead of 7.
    const long pstride = pstride4;
    v4f acc4[PER4];
#pragma unroll
    for (int i = 0; i < PER4; ++i) acc4[i] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < FB0; ++u) {
      if (u < np) {  // uniform
#pragma unroll
        for (int i = 0; i < PER4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc4[i][j] = __builtin_fmaf(1.0f, v0[u][i][j], acc4[i][j]);
      }
    }
    for (int p = FB0; p < np; p += FB4) {
      v4f v[FB4][PER4];
#pragma unroll
      for (int u = 0; u < FB4; ++u) {
        const long po = (long)min(p + u, np - 1) * pstride;
#pragma unroll
        for (int i = 0; i < PER4; ++i) {
          const int x = tid + 256 * i, rl = x >> 5, k4 = x & 31;
          v[u][i] = __builtin_nontemporal_load(
              reinterpret_cast<const v4f*>(P + po + (long)min(r0 + rl, rows - 1) * 128 + 4 * k4));
        }
      }
      __builtin_amdgcn_sched_barrier(0);  // every load of the batch is issued before the first add
#pragma unroll
      for (int u = 0; u < FB4; ++u) {
        if (p + u < np) {  // uniform
#pragma unroll
          for (int i = 0; i < PER4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc4[i][j] = __builtin_fmaf(1.0f, v[u][i][j], acc4[i][j]);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < PER4; ++i) {
      const int x = tid + 256 * i, rl = x >> 5, k4 = x & 31;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int k = 4 * k4 + j;
        PG[rl * RF_PS + k] = ((float)cb[rl * RF_CS + k] - zrow[rl]) * acc4[i][j];
      }
    }
  } else {  // u_k * g_k: all of a thread's G loads in flight at once (clamped addresses)
    constexpr int PER = RF_ROWS * 128 / 256;
    float gv[PER];
    if (P) {
      // G folded here from the gradient GEMM's per-panel chains (P[p][row][col], rows x wd per
      // panel), in panel order from 0 as k_fold does: C = fma(1, P_p, C). FB panels of every
      // element are loaded at once; the last batch is predicated. A workgroup that got here holds
      // a live row, and its 16-64 rows lie in one 128-row tile, which the GEMM therefore computed.
      constexpr int FB = PER <= 8 ? 8 : (PER <= 16 ? 4 : 2);
      const long pstride = (long)rows * wd;
#pragma unroll
      for (int i = 0; i < PER; ++i) gv[i] = 0.0f;
      for (int p = 0; p < np; p += FB) {
        float v[FB][PER];
#pragma unroll
        for (int u = 0; u < FB; ++u) {
          const long po = (long)min(p + u, np - 1) * pstride;
#pragma unroll
          for (int i = 0; i < PER; ++i) {
            const int x = tid + 256 * i, rl = x >> 7, k = x & 127;
            v[u][i] = __builtin_nontemporal_load(P + po + (long)min(r0 + rl, rows - 1) * wd + min(k, wd - 1));
          }
        }
        __builtin_amdgcn_sched_barrier(0);  // every load of the batch is issued before the first add
#pragma unroll
        for (int u = 0; u < FB; ++u) {
          if (p + u < np) {  // uniform
#pragma unroll
            for (int i = 0; i < PER; ++i) gv[i] = __builtin_fmaf(1.0f, v[u][i], gv[i]);
          }
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int x = tid + 256 * i, rl = x >> 7, k = x & 127;
        gv[i] = G[(long)min(r0 + rl, rows - 1) * wd + min(k, wd - 1)];
      }
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int x = tid + 256 * i, rl = x >> 7, k = x & 127;
      if (k < wd) PG[rl * RF_PS + k] = ((float)cb[rl * RF_CS + k] - zrow[rl]) * gv[i];
    }
  }
  __syncthreads();
  // num = sum_k u_k g_k, den = sum_k u_k hu_k, sequential in k (src/engine.rs:562-566); then the
  // closed-form f16 scale and its acceptance test (:567-587)
  if (wv == 0 && lane < RF_ROWS) {
    const int r = r0 + lane;
    const bool live = r < rows && active[r / rc];
    int moved = 0;
    float s_new = 0.0f;
    if (live) {
      const float* pg = PG + lane * RF_PS;
      const float* ph = PH + lane * RF_PS;
      float num = 0.0f, den = 0.0f;
      int k = 0;
      for (; k + 8 <= wd; k += 8) {
        float a[8], b[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          a[j] = pg[k + j];
          b[j] = ph[k + j];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          num = num + a[j];
          den = den + b[j];
        }
      }
      for (; k < wd; ++k) {
        num = num + pg[k];
        den = den + ph[k];
      }
      const float s_old = scales[(long)r * ng + gi];
      if (den > 1e-30f) {
        s_new = rs_maxf(round_f16(s_old + num / den), CDCLQ_F16_MIN_NORMAL);
        const float d = s_new - s_old;
        const float dl32 = (-2.0f * d) * num + (d * d) * den;
        if ((double)dl32 < 0.0) {
          scales[(long)r * ng + gi] = s_new;
          dlog[r] = (double)dl32;
          moved = 1;
        }
      }
      dcnt[r] = moved;
    }
    mv[lane] = moved;
    snew[lane] = s_new;
  }
  __syncthreads();
  // e += W_hat - ndq, W_hat = ndq on the accepted rows. Whole, aligned groups: 16-byte accesses,
  // slot x = tid + 256 i covering row x >> 5, columns 4 (x & 31) .. + 3, all loads in flight.
  if (vec && ((reinterpret_cast<uintptr_t>(e) | reinterpret_cast<uintptr_t>(wq)) & 15) == 0) {
    v4f ev[PER4], qv[PER4];
#pragma unroll
    for (int i = 0; i < PER4; ++i) {
      const int x = tid + 256 * i, rl = x >> 5, k4 = x & 31;
      if (mv[rl]) {
        const long o = (long)(r0 + rl) * n + c0 + 4 * k4;
        ev[i] = *reinterpret_cast<const v4f*>(e + o);
        qv[i] = *reinterpret_cast<const v4f*>(wq + o);
      }
    }
#pragma unroll
    for (int i = 0; i < PER4; ++i) {
      const int x = tid + 256 * i, rl = x >> 5, k4 = x & 31;
      if (mv[rl]) {
        const long o = (long)(r0 + rl) * n + c0 + 4 * k4;
        const uint32_t cw = *reinterpret_cast<const uint32_t*>(cb + rl * RF_CS + 4 * k4);
        v4f ne, nq;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          nq[j] = snew[rl] * ((float)((cw >> (8 * j)) & 0xffu) - zrow[rl]);
          ne[j] = ev[i][j] + (qv[i][j] - nq[j]);
        }
        *reinterpret_cast<v4f*>(e + o) = ne;
        *reinterpret_cast<v4f*>(wq + o) = nq;
      }
    }
    return;
  }
  // otherwise in two halves of 16 elements per thread with all of a half's loads in flight at once
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    constexpr int PER = RF_ROWS * 128 / 256 / 2;
    float ev[PER], qv[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int x = tid + 256 * (PER * h + i), rl = x >> 7, k = x & 127;
      if (k < wd && mv[rl]) {
        const long o = (long)(r0 + rl) * n + c0 + k;
        ev[i] = e[o];
        qv[i] = wq[o];
      }
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int x = tid + 256 * (PER * h + i), rl = x >> 7, k = x & 127;
      if (k < wd && mv[rl]) {
        const long o = (long)(r0 + rl) * n + c0 + k;
        const float ndq = snew[rl] * ((float)cb[rl * RF_CS + k] - zrow[rl]);
        e[o] = ev[i] + (qv[i] - ndq);
        wq[o] = ndq;
      }
    }
  }
}

// Coordinate-descent sweeps over sub-block [c0, c0+wd) (src/engine.rs:600-658); one wave per row,
// one column per lane. The reference visits the columns one after another and a column's decision
// depends on the gradient left by the moves before it. Every lane evaluates its own column's
// decision with the current gradient (the same IEEE operations the sequential visit would do);
// the lowest column at or after the cursor whose code changes is the next move of the sequential
// order, since the columns before it saw exactly this gradient and kept their codes. The move is
// applied (gradient update over the whole sub-block, wave-parallel), the cursor jumps past it and
// the columns after it are evaluated again. A sweep therefore costs one round per move plus one.
// NPL elements of one row of G = E H[:, c0:c0+wd] (columns 64 s + lane) from the per-panel chains
// of the gradient GEMM (P[p][row][col], stride pstride between panels): the ordered fold of
// k_fold, C = fma(1, P_p, C) for p = 0, 1, ... from C = 0. Loads go out in batches of B panels
// for every column (NPL * B loads in flight); the last batch is predicated, not split into
// single loads, and only loaded panels are added.
template <int NPL, int B>
__device__ __forceinline__ void fold_chains(const float* __restrict__ src, long pstride, int np, int wd, int lane,
                                            float (&gg)[NPL]) {
  float acc[NPL];
#pragma unroll
  for (int s = 0; s < NPL; ++s) acc[s] = 0.0f;
  for (int p = 0; p < np; p += B) {
    float v[NPL][B];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int pu = min(p + u, np - 1);
#pragma unroll
      for (int s = 0; s < NPL; ++s)
        v[s][u] = __builtin_nontemporal_load(src + (long)pu * pstride + min(s * 64 + lane, wd - 1));
    }
    __builtin_amdgcn_sched_barrier(0);  // every load of the batch is issued before the first add
#pragma unroll
    for (int u = 0; u < B; ++u) {
      if (p + u < np) {  // uniform
#pragma unroll
        for (int s = 0; s < NPL; ++s) acc[s] = __builtin_fmaf(1.0f, v[s][u], acc[s]);
      }
    }
  }
#pragma unroll
  for (int s = 0; s < NPL; ++s) gg[s] = s * 64 + lane < wd ? acc[s] : 0.0f;
}

template <int NPL, int FBW = 0>
// The 64-column form asks for 8 wavefronts per SIMD: the unrolled panel addresses of its fold would
// otherwise take enough scalar registers to cap it at 7. FBW (64-column form only) widens the
// fold's batches to FBW panels for gradients of many panels, at 6 wavefronts per SIMD.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NPL == 1 ? (FBW ? 6 : 8) : 1))) void k_cd(
    int rows, int n, int ng, int g, int c0, int wd, int sb, int nsb, int rc, int sweeps, const float* __restrict__ G,
    const float* __restrict__ h32, const uint8_t* __restrict__ gbits, const float* __restrict__ scales,
    const float* __restrict__ zeros, uint8_t* __restrict__ codes, float* __restrict__ wq, float* __restrict__ e,
    const uint8_t* __restrict__ active, const uint8_t* __restrict__ sel, double* __restrict__ dlog,
    uint32_t* __restrict__ dcnt, int cap, unsigned long long* __restrict__ mid, uint32_t* __restrict__ evals,
    const float* __restrict__ P, int np) {
  // Sub-blocks of up to 64 columns keep H_CC (the sub-block's rows and columns of h32, 16 KB) in
  // LDS, shared by the workgroup's rows: the gradient update after a move reads its row from there.
  constexpr int HW = NPL * 64;
  constexpr bool HLDS = NPL == 1;
  __shared__ float hs[HLDS ? HW * HW : 1];
  const int lane = threadIdx.x & 63;
  const int r = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
  // The H_CC loads go out with the row's selection test and are written to LDS after the fold.
  constexpr int HPER = HLDS ? HW * HW / 256 : 1;
  float hv[HPER];
  if (HLDS) {  // clamped addresses; entries outside wd x wd are never read
#pragma unroll
    for (int q = 0; q < HPER; ++q) {
      const int x = threadIdx.x + 256 * q, i = x / HW, c = x % HW;
      hv[q] = h32[(long)(c0 + min(i, wd - 1)) * n + c0 + min(c, wd - 1)];
    }
  }
  const int chunk = min(r, rows - 1) / rc;
  uint32_t act = active[chunk], pick = sel[(long)chunk * nsb + sb];
  asm volatile("" : "+v"(act), "+v"(pick));  // both loads issued before either is tested
  const bool live = r < rows && act && pick;
  // per-column state and parameters, one column per lane and slice; the gradient is either G or,
  // with P, folded here from the GEMM's per-panel chains (P[p][row][col], rows x wd per panel)
  float gg[NPL], mwq[NPL], me[NPL], hd[NPL], sc[NPL], zz[NPL], mq[NPL];
  int mc[NPL];
  uint8_t gb[NPL];
  if (live) {
    // unconditional clamped loads; lanes past wd are never selected or stored
#pragma unroll
    for (int s = 0; s < NPL; ++s) {
      const int j = c0 + min(s * 64 + lane, wd - 1);
      const long o = (long)r * n + j;
      const int gi = j / g;
      mwq[s] = wq[o];
      me[s] = e[o];
      mc[s] = (int)codes[o];
      hd[s] = h32[(long)j * n + j];
      sc[s] = scales[(long)r * ng + gi];
      zz[s] = zeros[(long)r * ng + gi];
      gb[s] = gbits[gi];
    }
    if (P) {
      fold_chains<NPL, (FBW ? FBW : (NPL <= 2 ? 16 / NPL : 2))>(P + (long)r * wd, (long)rows * wd, np, wd, lane, gg);
    } else {
#pragma unroll
      for (int s = 0; s < NPL; ++s) gg[s] = s * 64 + lane < wd ? G[(long)r * wd + s * 64 + lane] : 0.0f;
    }
#pragma unroll
    for (int s = 0; s < NPL; ++s) {
      const bool in = s * 64 + lane < wd;
      mwq[s] = in ? mwq[s] : 0.0f;
      me[s] = in ? me[s] : 0.0f;
      mc[s] = in ? mc[s] : 0;
      mq[s] = (float)((1u << gb[s]) - 1u);
    }
  }
  if (HLDS) {
#pragma unroll
    for (int q = 0; q < HPER; ++q) hs[threadIdx.x + 256 * q] = hv[q];
    __syncthreads();
  }
  if (!live) {
    if (r < rows && lane == 0) dcnt[r] = 0;
    return;
  }
  uint32_t moves = 0, nevals = 0, nnear = 0;
  double* dl = dlog + (long)r * cap;
  for (int sw = 0; sw < sweeps; ++sw) {
    bool changed = false;
#pragma unroll
    for (int s = 0; s < NPL; ++s) {
      const bool in = s * 64 + lane < wd;
      const uint64_t inmask = __ballot(in);
      int start = 0;
      while (start < 64) {
        // this lane's column, visited now: target = w_hat_j + g_j / H_jj (src/engine.rs:626-640)
        const float target = mwq[s] + gg[s] / hd[s];
        float qv;
        const float newdq = quant_dq(target, sc[s], zz[s], mq[s], &qv);
        const int qc = (int)code_of(qv);
        const uint64_t mask = __ballot(in && lane >= start && qc != mc[s]);
        // the sequential visit evaluated columns start .. (the move, or the slice's end) with this gradient
        const int last = mask ? (int)__builtin_ctzll(mask) : 63;
        const uint64_t seen = (~0ull << start) & (last == 63 ? ~0ull : ((1ull << (last + 1)) - 1ull)) & inmask;
        nevals += (uint32_t)__builtin_popcountll(seen);
        nnear += (uint32_t)__builtin_popcountll(__ballot(near_midpoint(target, sc[s], zz[s], mq[s])) & seen);
        if (mask == 0) break;
        const int jl = __builtin_amdgcn_readfirstlane(__builtin_ctzll(mask));
        const float cur = readlane(mwq[s], jl);
        const float nd = readlane(newdq, jl);
        const float gj = readlane(gg[s], jl);
        const float hjj = readlane(hd[s], jl);
        const float de = cur - nd;
        const float d32 = (2.0f * de) * gj + (de * de) * hjj;
        if (lane == 0) dl[moves] = (double)d32;
        ++moves;
        const float* hrow = HLDS ? &hs[(s * 64 + jl) * HW] : h32 + (long)(c0 + s * 64 + jl) * n + c0;
#pragma unroll
        for (int s2 = 0; s2 < NPL; ++s2) {  // lanes past wd (never selected, never stored) take
          const int k = s2 * 64 + lane;       // garbage: no predicate, clamped address
          gg[s2] = gg[s2] + de * hrow[min(k, wd - 1)];
        }
        if (lane == jl) {
          mwq[s] = nd;
          mc[s] = qc;
          me[s] = me[s] + de;
        }
        changed = true;
        start = jl + 1;
      }
    }
    if (!changed) break;
  }
#pragma unroll
  for (int s = 0; s < NPL; ++s) {
    const int k = s * 64 + lane;
    if (k < wd) {
      const long o = (long)r * n + c0 + k;
      wq[o] = mwq[s];
      e[o] = me[s];
      codes[o] = (uint8_t)mc[s];
    }
  }
  if (lane == 0) {
    dcnt[r] = moves;
    evals[r] += nevals;  // one wave per row: no other writer in this launch
    if (nnear) atomicAdd(&mid[MID_CD_NEAR], (unsigned long long)nnear);
  }
}

// Coordinate descent for sub-blocks wider than 1024 columns (k_cd keeps at most 16 columns per
// lane). Same decisions, order and accounting as k_cd; the row's gradient lives in G (this step's
// buffer, updated in place) and the per-column state in wq / e / codes, visited 64 columns at a
// time. After a move the whole gradient row is updated in memory and the current slice reloaded;
// a workgroup-scope fence orders the wave's stores before its next loads.
__global__ __launch_bounds__(256) void k_cd_mem(int rows, int n, int ng, int g, int c0, int wd, int sb, int nsb,
                                                int rc, int sweeps, float* __restrict__ G,
                                                const float* __restrict__ h32, const uint8_t* __restrict__ gbits,
                                                const float* __restrict__ scales, const float* __restrict__ zeros,
                                                uint8_t* __restrict__ codes, float* __restrict__ wq,
                                                float* __restrict__ e, const uint8_t* __restrict__ active,
                                                const uint8_t* __restrict__ sel, double* __restrict__ dlog,
                                                uint32_t* __restrict__ dcnt, int cap,
                                                unsigned long long* __restrict__ mid, uint32_t* __restrict__ evals) {
  const int lane = threadIdx.x & 63;
  const int r = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
  if (r >= rows) return;
  const int chunk = r / rc;
  if (!active[chunk] || !sel[(long)chunk * nsb + sb]) {
    if (lane == 0) dcnt[r] = 0;
    return;
  }
  float* gr = G + (long)r * wd;
  uint32_t moves = 0, nevals = 0, nnear = 0;
  double* dl = dlog + (long)r * cap;
  for (int sw = 0; sw < sweeps; ++sw) {
    bool changed = false;
    for (int s0 = 0; s0 < wd; s0 += 64) {
      const int k = s0 + lane;
      const bool in = k < wd;
      const int j = c0 + min(k, wd - 1);
      const long o = (long)r * n + j;
      const int gi = j / g;
      const float hd = h32[(long)j * n + j], sc = scales[(long)r * ng + gi], zz = zeros[(long)r * ng + gi];
      const float mq = (float)((1u << gbits[gi]) - 1u);
      float mwq = in ? wq[o] : 0.0f, me = in ? e[o] : 0.0f;
      int mc = in ? (int)codes[o] : 0;
      float gg = in ? gr[k] : 0.0f;
      const uint64_t inmask = __ballot(in);
      int start = 0;
      while (start < 64) {
        const float target = mwq + gg / hd;
        float qv;
        const float newdq = quant_dq(target, sc, zz, mq, &qv);
        const int qc = (int)code_of(qv);
        const uint64_t mask = __ballot(in && lane >= start && qc != mc);
        const int last = mask ? (int)__builtin_ctzll(mask) : 63;
        const uint64_t seen = (~0ull << start) & (last == 63 ? ~0ull : ((1ull << (last + 1)) - 1ull)) & inmask;
        nevals += (uint32_t)__builtin_popcountll(seen);
        nnear += (uint32_t)__builtin_popcountll(__ballot(near_midpoint(target, sc, zz, mq)) & seen);
        if (mask == 0) break;
        const int jl = __builtin_amdgcn_readfirstlane(__builtin_ctzll(mask));
        const float cur = readlane(mwq, jl);
        const float nd = readlane(newdq, jl);
        const float gj = readlane(gg, jl);
        const float hjj = readlane(hd, jl);
        const float de = cur - nd;
        const float d32 = (2.0f * de) * gj + (de * de) * hjj;
        if (lane == 0) dl[moves] = (double)d32;
        ++moves;
        if (lane == jl) {
          mwq = nd;
          mc = qc;
          me = me + de;
          wq[o] = mwq;
          e[o] = me;
          codes[o] = (uint8_t)mc;
        }
        // g_k = g_k + de * H[j, c0 + k] over the whole sub-block row (src/engine.rs:641-646)
        const float* hrow = h32 + (long)(c0 + s0 + jl) * n + c0;
        for (int k2 = lane; k2 < wd; k2 += 64) gr[k2] = gr[k2] + de * hrow[k2];
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
        gg = in ? gr[k] : 0.0f;
        changed = true;
        start = jl + 1;
      }
    }
    if (!changed) break;
  }
  if (lane == 0) {
    dcnt[r] = moves;
    evals[r] += nevals;
    if (nnear) atomicAdd(&mid[MID_CD_NEAR], (unsigned long long)nnear);
  }
}

int npl_for(int cnt) {
  if (cnt <= 64) return 1;
  if (cnt <= 128) return 2;
  if (cnt <= 256) return 4;
  if (cnt <= 512) return 8;
  if (cnt <= 1024) return 16;
  return 0;
}

}  // namespace

size_t panel_partials_elems(int m, int wd, int k) {
  return (size_t)((k + CDCLQ_KC - 1) / CDCLQ_KC) * (size_t)m * (size_t)wd;
}

int panel_row_tile() { return PR; }

// compute units of the current device (cached per process)
static hipError_t cu_count(int* out) {
  static std::atomic<int> cached{0};
  int v = cached.load(std::memory_order_relaxed);
  if (v == 0) {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err == hipSuccess) err = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev);
    if (err != hipSuccess) return err;
    v = std::max(1, v);
    cached.store(v, std::memory_order_relaxed);
  }
  *out = v;
  return hipSuccess;
}

// resident workgroups of k_panel_dma on the whole device (cached per process)
static hipError_t dma_slots(int* out) {
  static std::atomic<int> cached{0};
  int v = cached.load(std::memory_order_relaxed);
  if (v == 0) {
    int dev = 0, cus = 0, per = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err == hipSuccess) err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (err == hipSuccess) err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, k_panel_dma<false>, 256, 0);
    if (err != hipSuccess) return err;
    v = std::max(1, cus * std::max(1, per));
    cached.store(v, std::memory_order_relaxed);
  }
  *out = v;
  return hipSuccess;
}

// resident k_lazy_wide<DIRECT> workgroups on the whole device (cached per process)
template <bool DIRECT>
static hipError_t wide_slots(int* out) {
  static std::atomic<int> cached{0};
  int v = cached.load(std::memory_order_relaxed);
  if (v == 0) {
    int dev = 0, cus = 0, per = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err == hipSuccess) err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (err == hipSuccess) err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, k_lazy_wide<DIRECT>, 512, 0);
    if (err != hipSuccess) return err;
    v = std::max(1, cus * std::max(1, per));
    cached.store(v, std::memory_order_relaxed);
  }
  *out = v;
  return hipSuccess;
}

hipError_t panel_gemm(hipStream_t st, int m, int wd, int k, const float* A, long lda, const float* B, long ldb,
                      float* P, const int* rtiles, int ntiles) {
  if (m <= 0 || wd <= 0 || k <= 0) return hipSuccess;
  if (!rtiles) ntiles = (m + PR - 1) / PR;
  if (ntiles <= 0) return hipSuccess;
  const bool vec4 = (lda % 4 == 0) && ((uintptr_t)A % 16 == 0) && k % 4 == 0;
  constexpr int SK = 32;
  const long nunits = (long)ntiles * ((k + CDCLQ_KC - 1) / CDCLQ_KC) * ((wd + PC - 1) / PC);
  if (nunits > INT32_MAX) return hipErrorInvalidValue;
  // one workgroup per resident slot (occupancy is a property of the kernel, cached per process;
  // concurrent first calls compute the same value)
  static std::atomic<int> slots[2] = {0, 0};
  std::atomic<int>& sl = slots[vec4 ? 1 : 0];
  if (sl.load(std::memory_order_relaxed) == 0) {
    int dev = 0, cus = 0, per = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err == hipSuccess) err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (err == hipSuccess)
      err = vec4 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, k_panel_gemm<SK, true>, 256, 0)
                 : hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, k_panel_gemm<SK, false>, 256, 0);
    if (err != hipSuccess) return err;
    sl.store(std::max(1, cus * std::max(1, per)), std::memory_order_relaxed);
  }
  const int grid = (int)std::min<long>(nunits, sl.load(std::memory_order_relaxed));
  const bool dma = vec4 && k % DSK == 0 && wd % 4 == 0 && wd >= 4 && ldb % 4 == 0 && (uintptr_t)B % 16 == 0;
  if (dma) {
    if (wd == LPC) {  // 128-column gradients of tall enough matrices: one E tile read per unit
      int ws = 0;
      const hipError_t e2 = wide_slots<false>(&ws);
      if (e2 != hipSuccess) return e2;
      const long wunits = (long)ntiles * ((k + CDCLQ_KC - 1) / CDCLQ_KC);
      if (wunits >= 4L * ws) {
        hipLaunchKernelGGL(k_lazy_wide<false>, dim3(ws), dim3(512), 0, st, m, wd, k, A, lda, B, ldb, (float*)nullptr,
                           0L, 0.0f, (int)wunits, P, rtiles, CDCLQ_KC);
        return hipGetLastError();
      }
    }
    int dslots = 0;
    const hipError_t err = dma_slots(&dslots);
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(k_panel_dma<false>, dim3((int)std::min<long>(nunits, dslots)), dim3(256), 0, st, m, wd, k, A, lda,
                       B, ldb, P, (int)nunits, rtiles, ntiles, (float*)nullptr, 0L, 0.0f, 0, CDCLQ_KC);
    return hipGetLastError();
  }
  if (vec4)
    hipLaunchKernelGGL((k_panel_gemm<SK, true>), dim3(grid), dim3(256), 0, st, m, wd, k, A, lda, B, ldb, P,
                       (int)nunits, rtiles, ntiles);
  else
    hipLaunchKernelGGL((k_panel_gemm<SK, false>), dim3(grid), dim3(256), 0, st, m, wd, k, A, lda, B, ldb, P,
                       (int)nunits, rtiles, ntiles);
  return hipGetLastError();
}

bool chain_gemm_mfma_ok(int m, int n, int k, const float* A, long lda, const float* B, long ldb, int kfold) {
  const int kf = kfold > 0 ? kfold : k;
  return m > 0 && n >= 4 && k > 0 && kf <= CDCLQ_KC && kf % DSK == 0 && k % kf == 0 && n % 4 == 0 &&
         lda % 4 == 0 && ldb % 4 == 0 && (uintptr_t)A % 16 == 0 && (uintptr_t)B % 16 == 0;
}

hipError_t chain_gemm_mfma(hipStream_t st, int m, int n, int k, float alpha, int beta_one, const float* A, long lda,
                           const float* B, long ldb, float* C, long ldc, int kfold) {
  if (!chain_gemm_mfma_ok(m, n, k, A, lda, B, ldb, kfold)) return hipErrorInvalidValue;
  const int kf = kfold > 0 ? kfold : k;
  int ws = 0;
  const hipError_t e2 = wide_slots<true>(&ws);
  if (e2 != hipSuccess) return e2;
  const long wunits = (long)((m + PR - 1) / PR) * ((n + LPC - 1) / LPC);
  if (beta_one && wunits >= ws && wunits <= INT32_MAX) {
    hipLaunchKernelGGL(k_lazy_wide<true>, dim3(ws), dim3(512), 0, st, m, n, k, A, lda, B, ldb, C, ldc, alpha,
                       (int)wunits, (float*)nullptr, (const int*)nullptr, kf);
    return hipGetLastError();
  }
  int dslots = 0;
  const hipError_t err = dma_slots(&dslots);
  if (err != hipSuccess) return err;
  const int ntiles = (m + PR - 1) / PR;
  const long nunits = (long)ntiles * ((n + PC - 1) / PC);
  hipLaunchKernelGGL(k_panel_dma<true>, dim3((int)std::min<long>(nunits, dslots)), dim3(256), 0, st, m, n, k, A, lda, B, ldb,
                     (float*)nullptr, (int)nunits, (const int*)nullptr, ntiles, C, ldc, alpha, beta_one, kf);
  return hipGetLastError();
}

hipError_t fold_panels(hipStream_t st, int m, int wd, int np, const float* P, float* G, const int* rtiles,
                       int ntiles) {
  if (!rtiles) ntiles = (m + PR - 1) / PR;
  const long count = (long)ntiles * PR * wd;
  if (count <= 0 || m <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_fold, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, st, m, wd, np, rtiles, count, P, G);
  return hipGetLastError();
}

bool refit_folds_chains(int wd) { return wd > 0 && wd <= 128; }  // the matrix-core k_refit_mfma

hipError_t refit_group(hipStream_t st, int rows, int n, int ng, int g, int gi, int rc, const float* G,
                       const float* h32, const uint8_t* codes, float* scales, const float* zeros, float* wq, float* e,
                       const uint8_t* active, double* dlog, uint32_t* dcnt, const float* P, int np) {
  const int wd = std::min(gi * g + g, n) - gi * g;
  if (P && !refit_folds_chains(wd)) return hipErrorInvalidValue;
  if (wd <= 128) {
    // the smallest workgroups (shortest chains) whose count still fits two per CU, so that all
    // rows are resident in one round; 64-row ones beyond that
    int cus = 0;
    const hipError_t err = cu_count(&cus);
    if (err != hipSuccess) return err;
    if ((rows + 15) / 16 <= 2 * cus)
      hipLaunchKernelGGL(k_refit_mfma<16>, dim3((rows + 15) / 16), dim3(256), 0, st, rows, n, ng, g, gi, rc, G, h32,
                         codes, scales, zeros, wq, e, active, dlog, dcnt, P, np);
    else if ((rows + 31) / 32 <= 2 * cus)
      hipLaunchKernelGGL(k_refit_mfma<32>, dim3((rows + 31) / 32), dim3(256), 0, st, rows, n, ng, g, gi, rc, G, h32,
                         codes, scales, zeros, wq, e, active, dlog, dcnt, P, np);
    else
      hipLaunchKernelGGL(k_refit_mfma<64>, dim3((rows + 63) / 64), dim3(256), 0, st, rows, n, ng, g, gi, rc, G, h32,
                         codes, scales, zeros, wq, e, active, dlog, dcnt, P, np);
    return hipGetLastError();
  }
#define REFIT_CASE(N)                                                                                                  \
  hipLaunchKernelGGL((k_refit<N>), dim3((rows + 3) / 4), dim3(256), 0, st, rows, n, ng, g, gi, rc, G, h32, codes,      \
                     scales, zeros, wq, e, active, dlog, dcnt)
  switch (npl_for(wd)) {
    case 4: REFIT_CASE(4); break;
    case 8: REFIT_CASE(8); break;
    case 16: REFIT_CASE(16); break;
    default: return hipErrorInvalidValue;
  }
#undef REFIT_CASE
  return hipGetLastError();
}

bool cd_folds_chains(int wd) { return wd > 0 && wd <= 1024; }  // the register-resident k_cd<NPL>

hipError_t cd_subblock(hipStream_t st, int rows, int n, int ng, int g, int c0, int wd, int sb, int nsb, int rc,
                       int sweeps, float* G, const float* h32, const uint8_t* gbits, const float* scales,
                       const float* zeros, uint8_t* codes, float* wq, float* e, const uint8_t* active,
                       const uint8_t* sel, double* dlog, uint32_t* dcnt, int cap, unsigned long long* mid,
                       uint32_t* evals, const float* P, int np) {
  const dim3 grid((rows + 3) / 4), blk(256);
  if (P && !cd_folds_chains(wd)) return hipErrorInvalidValue;
#define CD_CASE(N)                                                                                                     \
  hipLaunchKernelGGL((k_cd<N>), grid, blk, 0, st, rows, n, ng, g, c0, wd, sb, nsb, rc, sweeps, G, h32, gbits, scales,  \
                     zeros, codes, wq, e, active, sel, dlog, dcnt, cap, mid, evals, P, np)
  switch (npl_for(wd)) {
    case 1:
      if (P && np > 16)  // many panels: fewer, wider fold batches
        hipLaunchKernelGGL((k_cd<1, 32>), grid, blk, 0, st, rows, n, ng, g, c0, wd, sb, nsb, rc, sweeps, G, h32, gbits,
                           scales, zeros, codes, wq, e, active, sel, dlog, dcnt, cap, mid, evals, P, np);
      else
        CD_CASE(1);
      break;
    case 2: CD_CASE(2); break;
    case 4: CD_CASE(4); break;
    case 8: CD_CASE(8); break;
    case 16: CD_CASE(16); break;
    default:  // wider than 1024 columns: gradient row and column state in memory
      hipLaunchKernelGGL(k_cd_mem, grid, blk, 0, st, rows, n, ng, g, c0, wd, sb, nsb, rc, sweeps, G,
                         h32, gbits, scales, zeros, codes, wq, e, active, sel, dlog, dcnt, cap, mid, evals);
      break;
  }
#undef CD_CASE
  return hipGetLastError();
}

}  // namespace cdclq
