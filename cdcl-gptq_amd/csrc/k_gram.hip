// H += X^T Y on the matrix cores (src/linalg.rs:388-418), bit-exact.
//
// The reference's order per element: for each 2048-token chunk, tmp = fold over KC = 256-token
// panels of a fused-multiply-add chain in token order (first panel: tmp = chain; later panels:
// tmp = tmp + chain), then h += (f64)tmp. v_mfma_f32_32x32x1_2b_f32 has K = 1: every instruction
// adds exactly one product to each accumulator element with a single rounding, which the
// day-0 probe showed to be bit-identical to fmaf (including denormals). A chain of these
// instructions over the tokens of a panel is therefore the reference's chain.
//
// Work split: a 256-thread workgroup owns a 128 (rows) x 64 (cols) tile of one H; wave w owns
// rows [64*(w>>1), +64) x cols [32*(w&1), +32) as one 2-block accumulator (block b = rows
// 32b..32b+31). Tokens are staged 32 at a time through double-buffered LDS (row-major, so each
// lane reads its row/col of the current token with a conflict-free ds_read_b32). The chunk sum
// (f32) and the running H value (f64) stay in VGPRs for the whole token range, so H is read and
// written once.
//
// A launch walks a list of tiles that may belong to several Hessians (GramJob), so the four
// inputs of a decoder layer fill the GPU together. For symmetric jobs only tiles of the upper
// 128x128 super-tile triangle are listed and off-diagonal results are also written transposed
// (exact: fma(a, b, c) == fma(b, a, c)); this requires the incoming H to be symmetric, which the
// host checks.
#include <algorithm>
#include <climits>
#include <mutex>

#include "cdclq_dev.h"
#include "kernels.h"

namespace cdclq {
namespace {

// Device memory of the allocation-free entry point (cdclq_gram_accumulate_device_noalloc): the
// symmetry status words, the job record and the tile list of one accumulation with n <= 32768.
// Each GPU holds its own copy for the life of the process. Host code never uses this name as an
// address (it is a host-side stand-in there): gram_scratch() looks up the device address.
static __device__ __align__(256) unsigned char scratch[kGramScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

typedef float v32f __attribute__((ext_vector_type(32)));
typedef __attribute__((address_space(1))) const float gfloat;
typedef float f4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const f4v gf4v;

constexpr int TI = 128, TJ = 64, KT = 32;

__device__ __forceinline__ v32f mfma32(float a, float b, v32f c) {
  return __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, c, 0, 0, 0);
}

template <bool VEC4>
__global__ __launch_bounds__(256, 2) void k_gram_mfma(const GramJob* __restrict__ jobs,
                                                      const int4* __restrict__ tiles) {
  __shared__ float Xs[2][KT][TI];
  __shared__ float Ys[2][KT][TJ];
  const int4 tl = tiles[blockIdx.x];
  const GramJob jb = jobs[tl.x];
  const int n = jb.n, T = jb.t;
  const float* __restrict__ X = jb.x;
  const float* __restrict__ Y = jb.y;
  __attribute__((address_space(1))) double* H = (__attribute__((address_space(1))) double*)jb.h;
  const int i0 = tl.y * TI, j0 = tl.z * TJ;
  const bool mirror = tl.w != 0;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wi = wv >> 1, wj = wv & 1;

  // Per-lane output coordinates of accumulator register r (probe-verified layout):
  // block b = r >> 4, i = 8*((r&15)>>2) + 4*(lane>>5) + (r&3), j = lane & 31.
  const int rbase = i0 + 64 * wi + 4 * (lane >> 5);
  const int col = j0 + 32 * wj + (lane & 31);
  double h[32];
#pragma unroll
  for (int r = 0; r < 32; ++r) {
    const int row = rbase + 32 * (r >> 4) + 8 * ((r & 15) >> 2) + (r & 3);
    h[r] = (row < n && col < n) ? H[(long)row * n + col] : 0.0;
  }

  // Stage loader: Xs = X[t0:t0+KT, i0:i0+TI], Ys = Y[t0:t0+KT, j0:j0+TJ] (zero outside). The job's
  // pointers come from memory, so they are cast to the global address space explicitly: generic
  // (flat) loads would share the LDS wait counter and stall every LDS read behind them.
  const gfloat* Xg = (const gfloat*)X;
  const gfloat* Yg = (const gfloat*)Y;
  f4v px[4], py[2];
  unsigned okm = 0;  // bit q (X) / 4 + q (Y): the slot lies inside the matrix
  // VEC4 (n % 4 == 0): every thread always issues its 16-byte loads, from an address clamped into
  // the matrix, and slots outside are zeroed only when written to LDS; no branches or selects sit
  // between the loads and the matrix-core loop, so the prefetch of the next stage stays in flight.
  auto ld4 = [&](const gfloat* base, int t, int c, int bit, float pad) -> f4v {
    if (VEC4) {
      okm |= (t < T && c < n) ? (1u << bit) : 0u;
      return *(const gf4v*)(base + (long)min(t, T - 1) * n + min(c, n - 4));
    }
    f4v v = {pad, pad, pad, pad};
    if (t < T) {
      const gfloat* p = base + (long)t * n + c;
      if (c < n) v.x = p[0];
      if (c + 1 < n) v.y = p[1];
      if (c + 2 < n) v.z = p[2];
      if (c + 3 < n) v.w = p[3];
    }
    return v;
  };
  // Interior tiles with whole stages (all of config 4) take a lean path: a uniform stage base plus
  // per-lane offsets fixed for the whole launch, so a stage's six loads cost no vector ALU work.
  const bool interior = VEC4 && i0 + TI <= n && j0 + TJ <= n;
  int offx[4], offy[2];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int e = tid + 256 * q;
    offx[q] = (e >> 5) * n + i0 + (e & 31) * 4;
  }
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int e = tid + 256 * q;
    offy[q] = (e >> 4) * n + j0 + (e & 15) * 4;
  }
  auto gload = [&](int t0) {
    if (interior && t0 + KT <= T) {
      okm = 0x3f;
      const gfloat* xst = Xg + (long)t0 * n;
      const gfloat* yst = Yg + (long)t0 * n;
#pragma unroll
      for (int q = 0; q < 4; ++q) px[q] = *(const gf4v*)(xst + offx[q]);
#pragma unroll
      for (int q = 0; q < 2; ++q) py[q] = *(const gf4v*)(yst + offy[q]);
      return;
    }
    okm = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = tid + 256 * q;  // 0..1023 float4 slots of the 32 x 128 tile
      px[q] = ld4(Xg, t0 + (e >> 5), i0 + (e & 31) * 4, q, -0.0f);
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int e = tid + 256 * q;  // 0..511 float4 slots of the 32 x 64 tile
      py[q] = ld4(Yg, t0 + (e >> 4), j0 + (e & 15) * 4, 4 + q, 0.0f);
    }
  };
  // Slots outside the matrix: X is -0 and Y is +0, so a padded token adds fma(-0, +0, c) = c + (-0),
  // which leaves every chain value unchanged (a chain can reach -0 through underflow).
  auto keep = [&](f4v v, int bit, float pad) -> f4v {
    if (!VEC4 || ((okm >> bit) & 1u)) return v;
    return f4v{pad, pad, pad, pad};
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = tid + 256 * q;
      *reinterpret_cast<f4v*>(&Xs[buf][e >> 5][(e & 31) * 4]) = keep(px[q], q, -0.0f);
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int e = tid + 256 * q;
      *reinterpret_cast<f4v*>(&Ys[buf][e >> 4][(e & 15) * 4]) = keep(py[q], 4 + q, 0.0f);
    }
  };

  const int nstage = (T + KT - 1) / KT;
  gload(0);
  lstore(0);
  __syncthreads();
  v32f acc = {};
  float tmp[32];
#pragma unroll
  for (int r = 0; r < 32; ++r) tmp[r] = 0.0f;
  const float* xa = &Xs[0][0][64 * wi + lane];
  const float* yb = &Ys[0][0][32 * wj + (lane & 31)];
  for (int s = 0; s < nstage; ++s) {
    const int buf = s & 1;
    const int t0 = s * KT;
    if (s + 1 < nstage) gload(t0 + KT);
    const float* xs = xa + buf * (KT * TI);
    const float* ys = yb + buf * (KT * TJ);
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) acc = mfma32(xs[kk * TI], ys[kk * TJ], acc);
    const int tn = t0 + KT;
    if ((tn % CDCLQ_KC) == 0 || tn >= T) {  // panel end: tmp = fma(1, chain, tmp)
#pragma unroll
      for (int r = 0; r < 32; ++r) tmp[r] = __builtin_fmaf(1.0f, acc[r], tmp[r]);
      acc = v32f{};
      if ((tn % 2048) == 0 || tn >= T) {  // chunk end: h += (f64) tmp
#pragma unroll
        for (int r = 0; r < 32; ++r) {
          h[r] += (double)tmp[r];
          tmp[r] = 0.0f;
        }
      }
    }
    if (s + 1 < nstage) lstore(buf ^ 1);
    __syncthreads();
  }
#pragma unroll
  for (int r = 0; r < 32; ++r) {
    const int row = rbase + 32 * (r >> 4) + 8 * ((r & 15) >> 2) + (r & 3);
    if (row < n && col < n) {
      H[(long)row * n + col] = h[r];
      if (mirror) H[(long)col * n + row] = h[r];
    }
  }
}

// Direct-to-LDS variant for jobs whose tiles are all interior and whose token count is a multiple
// of DKT (n % 128 == 0, T % 64 == 0, 16-byte aligned rows; every config-4 input). A 512-thread
// workgroup owns a 128 x 128 tile (one per CU): wave w holds rows 64 (w >> 2) .. +63 x columns
// 32 (w & 3) .. +31 as one 2-block K=1 accumulator, two waves per SIMD. Stages of 64 tokens are
// filled with global_load_lds_dwordx4 (lane L's 16 bytes land at the instruction's LDS base + 16 L),
// so no registers hold prefetched data and no LDS stores are issued; two stages (128 KB) alternate,
// the next one loading while the current one is multiplied, one bare barrier per stage. Within a
// stage each wave reads its operands two token pairs ahead of the matrix core (the issue order is
// pinned, so an LDS read's latency hides behind the two MFMA pairs before its use). The wider tile
// streams X once per 128 x 128 outputs instead of per 128 x 64 (a third less traffic per flop than
// k_gram_mfma's tiles). Arithmetic, per-element operation order, panel and chunk folds are those of
// k_gram_mfma.
constexpr int DTJ = 128;                  // tile columns
constexpr int DKT = 64;                   // tokens per stage
constexpr int DSTAGE = DKT * (TI + DTJ);  // floats per stage: X [64][128], Y [64][128]
constexpr int DPW = DSTAGE / 512 / 4;     // 1 KB load instructions per wave and stage (8)
constexpr int DLA = 2;                    // token pairs read ahead of the matrix core
constexpr int GANG_LAG = 4;               // stages a gang member may run ahead of its slowest one
constexpr int GANG_SPIN = 100;            // polls before a member stops pacing (≈ 0.2 ms)

__global__ __launch_bounds__(512, 1) void k_gram_dma(const GramJob* __restrict__ jobs,
                                                     const int4* __restrict__ tiles, int* __restrict__ prog) {
  __shared__ float R[2][DSTAGE];
  const int4 tl = tiles[blockIdx.x];
  if (tl.x < 0) return;  // an empty slot of a short gang (gram_dma_order)
  const GramJob jb = jobs[tl.x];
  const int n = jb.n, T = jb.t;
  __attribute__((address_space(1))) double* H = (__attribute__((address_space(1))) double*)jb.h;
  const int i0 = tl.y * TI, j0 = tl.z * DTJ;
  const bool mirror = (tl.w & 1) != 0;
  const int gsz = (tl.w >> 1) & 63, gpos = (tl.w >> 7) & 31, gid = tl.w >> 12;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wr = wv >> 2, wc = wv & 3;
  const int rbase = i0 + 64 * wr + 4 * (lane >> 5);
  const int col = j0 + 32 * wc + (lane & 31);
  double h[32];
#pragma unroll
  for (int r = 0; r < 32; ++r) h[r] = H[(long)(rbase + 32 * (r >> 4) + 8 * ((r & 15) >> 2) + (r & 3)) * n + col];
  // Stage layout: X [64 tokens][128 rows] (instructions 0..31), then Y [64][128 cols]
  // (instructions 32..63); instruction q: lane -> token 2 (q & 31) + (lane >> 5), columns
  // 4 (lane & 31). Wave w issues instructions w, w + 8, ..., w + 56.
  const float* src[DPW];
  int dst[DPW];
#pragma unroll
  for (int q = 0; q < DPW; ++q) {
    const int ins = wv + 8 * q;
    const int tok = 2 * (ins & 31) + (lane >> 5);
    src[q] = (ins < 32 ? jb.x + i0 : jb.y + j0) + (long)tok * n + 4 * (lane & 31);
    dst[q] = 256 * ins;
  }
  const int nstage = T / DKT;
  auto issue = [&](int s) {
    float* buf = &R[s & 1][0];
    const long t0n = (long)s * DKT * n;
#pragma unroll
    for (int q = 0; q < DPW; ++q) dma16(src[q] + t0n, buf + dst[q]);
  };
  issue(0);
  // Gang pacing (prog != null). The 32 tiles of a gang run on one XCD at the same time and share 4
  // X and 8 Y stripes in its L2 only while they stay within a few stages of each other. Wave 0
  // publishes the stage its workgroup has reached in prog[32 gang + position] (INT_MAX once done)
  // and loads the others' stages; before the next stage's barrier, if any member is more than
  // GANG_LAG stages behind, it polls until none is, or gives up pacing after GANG_SPIN polls (a
  // member that is not resident). Pacing only delays; the arithmetic is untouched.
  int* const gp = (prog != nullptr && gsz > 1) ? prog + 32 * gid : nullptr;
  bool pace = gp != nullptr && __builtin_amdgcn_readfirstlane(wv) == 0;
  int seen = INT_MAX;  // lane < gsz: the stage member `lane` had published, loaded a stage earlier
  v32f acc = {};
  float tmp[32];
#pragma unroll
  for (int r = 0; r < 32; ++r) tmp[r] = 0.0f;
  for (int s = 0; s < nstage; ++s) {
    // this wave's part of stage s has landed; the barrier publishes every wave's part and retires
    // all reads of stage s - 1, whose buffer the next stage's loads then fill
    wait_vmcnt<0>();
    if (pace) {
      if (__builtin_amdgcn_ballot_w64(lane < gsz && s - seen > GANG_LAG)) {
        int polls = 0;
        do {
          __builtin_amdgcn_s_sleep(8);
          if (lane < gsz) seen = __hip_atomic_load(gp + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } while (__builtin_amdgcn_ballot_w64(lane < gsz && s - seen > GANG_LAG) && ++polls < GANG_SPIN);
        pace = polls < GANG_SPIN;
      }
      if (lane == 0) __hip_atomic_store(gp + gpos, s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (lane < gsz) seen = __hip_atomic_load(gp + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_barrier();
    if (s + 1 < nstage) issue(s + 1);
    const float* xs = &R[s & 1][64 * wr + lane];
    const float* ys = &R[s & 1][DKT * TI + 32 * wc + (lane & 31)];
    float a0[DKT / 2], a1[DKT / 2], b0[DKT / 2], b1[DKT / 2];
    auto ld = [&](int p) {
      a0[p] = xs[(2 * p) * TI];
      a1[p] = xs[(2 * p + 1) * TI];
      b0[p] = ys[(2 * p) * DTJ];
      b1[p] = ys[(2 * p + 1) * DTJ];
    };
#pragma unroll
    for (int p = 0; p < DLA; ++p) ld(p);
#pragma unroll
    for (int p = 0; p < DKT / 2; ++p) {
      if (p + DLA < DKT / 2) ld(p + DLA);
      acc = mfma32(a0[p], b0[p], acc);
      acc = mfma32(a1[p], b1[p], acc);
    }
    // issue order: the first DLA pairs' reads, then per pair the reads DLA ahead and its 2 MFMAs
#pragma unroll
    for (int p = 0; p < DLA; ++p) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
    for (int p = 0; p < DKT / 2; ++p) {
      if (p + DLA < DKT / 2) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    }
    const int tn = (s + 1) * DKT;
    if ((tn % CDCLQ_KC) == 0 || tn >= T) {  // panel end: tmp = fma(1, chain, tmp)
#pragma unroll
      for (int r = 0; r < 32; ++r) tmp[r] = __builtin_fmaf(1.0f, acc[r], tmp[r]);
      acc = v32f{};
      if ((tn % 2048) == 0 || tn >= T) {  // chunk end: h += (f64) tmp
#pragma unroll
        for (int r = 0; r < 32; ++r) {
          h[r] += (double)tmp[r];
          tmp[r] = 0.0f;
        }
      }
    }
  }
  if (gp != nullptr && tid == 0) __hip_atomic_store(gp + gpos, INT_MAX, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
  for (int r = 0; r < 32; ++r) {
    const int row = rbase + 32 * (r >> 4) + 8 * ((r & 15) >> 2) + (r & 3);
    H[(long)row * n + col] = h[r];
    if (mirror) H[(long)col * n + row] = h[r];
  }
}

// flag |= (h not bitwise symmetric)
__global__ __launch_bounds__(256) void k_sym_check(int n, const double* __restrict__ h, int* flag) {
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long)n * n) return;
  const int i = (int)(idx / n), j = (int)(idx % n);
  if (j <= i) return;
  const unsigned long long a = __double_as_longlong(h[idx]);
  const unsigned long long b = __double_as_longlong(h[(long)j * n + i]);
  if (a != b) atomicOr(flag, 1);
}

// A fill kernel rather than hipMemsetAsync, so the clear stays an ordinary kernel node when a
// caller records the stream into a HIP graph.
__global__ __launch_bounds__(256) void k_zero_words(int* __restrict__ p, int count) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < count) p[i] = 0;
}

}  // namespace

void gram_mfma_tiles(int job, int n, bool sym, std::vector<int4>& out) {
  const int ni = (n + TI - 1) / TI;
  const int nj = (n + TJ - 1) / TJ;
  if (!sym) {
    for (int I = 0; I < ni; ++I)
      for (int J = 0; J < nj; ++J) out.push_back(make_int4(job, I, J, 0));
    return;
  }
  // upper triangle of 128x128 super-tiles; each super-tile = two 128x64 workgroup tiles
  for (int I = 0; I < ni; ++I)
    for (int S = I; S < ni; ++S)
      for (int h = 0; h < 2; ++h) {
        const int J = 2 * S + h;
        if (J >= nj) continue;
        out.push_back(make_int4(job, I, J, S != I ? 1 : 0));
      }
}

hipError_t gram_mfma(hipStream_t st, const GramJob* jobs, const int4* tiles, int ntiles, bool vec4) {
  if (ntiles <= 0) return hipSuccess;
  if (vec4)
    hipLaunchKernelGGL(k_gram_mfma<true>, dim3(ntiles), dim3(256), 0, st, jobs, tiles);
  else
    hipLaunchKernelGGL(k_gram_mfma<false>, dim3(ntiles), dim3(256), 0, st, jobs, tiles);
  return hipGetLastError();
}

hipError_t gram_dma(hipStream_t st, const GramJob* jobs, const int4* tiles, int ntiles, int* prog) {
  if (ntiles <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_gram_dma, dim3(ntiles), dim3(512), 0, st, jobs, tiles, prog);
  return hipGetLastError();
}

// Morton index of tile (I, J), the column bit lowest: 32 consecutive indices are a 4 x 8 block
static uint64_t tile_morton(int I, int J) {
  uint64_t k = 0;
  for (int b = 0; b < 24; ++b) k |= (uint64_t)((J >> b) & 1) << (2 * b) | (uint64_t)((I >> b) & 1) << (2 * b + 1);
  return k;
}

void gram_dma_order(std::vector<int4>& tl) {
  // each job's tiles in Morton order, jobs one after another
  for (size_t i = 0; i < tl.size();) {
    size_t j = i;
    while (j < tl.size() && tl[j].x == tl[i].x) ++j;
    std::stable_sort(tl.begin() + i, tl.begin() + j,
                     [](const int4& a, const int4& b) { return tile_morton(a.y, a.z) < tile_morton(b.y, b.z); });
    i = j;
  }
  // gangs of 32 consecutive tiles (one may span two jobs), so the launch takes no more rounds of
  // 256 workgroups than the tiles need; the gang fields stay 0 (no pacing) past 2^19 gangs
  const size_t m = tl.size(), ng = (m + 31) / 32, rounds = (ng + 7) / 8;
  const bool fields = ng < (size_t(1) << 19);
  std::vector<int4> out(rounds * 8 * 32, make_int4(-1, 0, 0, 0));
  for (size_t t = 0; t < m; ++t) {
    const size_t g = t / 32, p = t % 32;
    int4 v = tl[t];
    const int gs = (int)std::min<size_t>(32, m - 32 * g);
    v.w = (v.w & 1) | (fields ? (gs << 1) | ((int)p << 7) | ((int)g << 12) : 0);
    out[(32 * (g / 8) + p) * 8 + g % 8] = v;
  }
  tl.swap(out);
}

void gram_dma_tiles(int job, int n, bool sym, std::vector<int4>& out) {
  const int nb = n / TI;  // n % 128 == 0 for these jobs
  for (int I = 0; I < nb; ++I)
    for (int J = sym ? I : 0; J < nb; ++J) out.push_back(make_int4(job, I, J, (sym && J != I) ? 1 : 0));
}

bool gram_dma_eligible(int n, int t, const void* x, const void* y) {
  return n % 128 == 0 && t % DKT == 0 && t > 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)y % 16 == 0;
}

hipError_t gram_scratch(int device, void** ptr) {
  *ptr = nullptr;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return e;
    if (cur != device) return hipErrorInvalidDevice;  // the caller makes `device` current
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch_ptr[device] = p;
  }
  *ptr = g_scratch_ptr[device];
  return hipSuccess;
}

hipError_t zero_words(hipStream_t st, int* p, int count) {
  if (count <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_zero_words, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, st, p, count);
  return hipGetLastError();
}

hipError_t sym_check(hipStream_t st, int n, const double* h, int* flag) {
  const long nn = (long)n * n;
  hipLaunchKernelGGL(k_sym_check, dim3((unsigned)((nn + 255) / 256)), dim3(256), 0, st, n, h, flag);
  return hipGetLastError();
}

}  // namespace cdclq
