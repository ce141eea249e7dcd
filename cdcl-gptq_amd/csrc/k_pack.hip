// Packed container cdclq-v1 on the device: bit-packing of code rows, the f16 / u8 / i32 companion
// tensors, and dequantization (packed or unpacked codes -> original column order, narrowed to the
// checkpoint dtype once).
//
// Narrowing of dequantized values (F16 / BF16 outputs) is bit-identical to half 2.4.1 for every
// finite and infinite value; a NaN result stays a NaN with the hardware's payload (the reference's
// own NaN payloads are those of x86, e.g. its default NaN for inf * 0).
//
// Row layout (src/quant.rs:113-131): the codes of a row, in permuted column order, appended low bit
// first into one bit stream with the width of each code's group; the last partial byte is written.
// Code j occupies bits [off_j, off_j + width) with off_j = sum of the widths of codes 0..j-1. The
// reference ORs each whole u8 code into its accumulator without masking, so an out-of-range code
// spills into the bits that follow; byte o of a row is therefore the OR of (code_j << off_j) over
// all j, restricted to bits [8 o, 8 o + 8). Every kernel here follows that definition, which is
// what the reference's accumulator loop computes for any input.
//
// All tables that depend only on the column layout (bit offsets, widths, the first code reaching
// each output word, the output column -> source column map) are built once per call and shared by
// every row; they stay in L2.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "cdclq.h"
#include "cdclq_dev.h"
#include "kernels.h"

namespace cdclq {
namespace {

// half 2.4.1 f16::from_f32: IEEE binary16, round to nearest even, overflow to infinity; NaN keeps
// its sign and the upper 10 payload bits and gets the quiet bit (src/io.rs:261).
__device__ __forceinline__ uint16_t f32_to_f16_bits(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t exp = (u >> 23) & 0xffu;
  uint32_t man = u & 0x7fffffu;
  if (exp == 0xffu) return (uint16_t)(man ? (sign | 0x7e00u | (man >> 13)) : (sign | 0x7c00u));
  const int e = (int)exp - 112;  // rebias 127 -> 15
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {  // binary16 subnormal or zero
    if (e < -10) return (uint16_t)sign;
    man |= 0x800000u;
    const int sh = 14 - e;
    uint32_t q = man >> sh;
    const uint32_t rem = man & ((1u << sh) - 1u), half = 1u << (sh - 1);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
  }
  uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
  const uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;  // a carry into the exponent is correct
  return (uint16_t)h;
}

// half 2.4.1 f16::to_f32: exact widening; NaN payload kept with the quiet bit set (src/io.rs:286).
__device__ __forceinline__ float f16_bits_to_f32(uint16_t hb) {
  const uint32_t h = hb;
  const uint32_t sign = (h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t u;
  if (exp == 0x1fu) {
    u = sign | 0x7f800000u | (man << 13) | (man ? 0x400000u : 0u);
  } else if (exp == 0) {
    if (man == 0) {
      u = sign;
    } else {  // subnormal: normalise (value man * 2^-24 is exact in f32)
      const int lz = __clz((int)man) - 21;  // 10 - (index of the top set bit)
      man = (man << lz) & 0x3ffu;
      u = sign | ((uint32_t)(113 - lz) << 23) | (man << 13);
    }
  } else {
    u = sign | ((exp + 112u) << 23) | (man << 13);
  }
  return __uint_as_float(u);
}

// Rust `z as u8`: truncation toward zero, saturating at 0 and 255, NaN -> 0 (src/io.rs:258).
__device__ __forceinline__ uint8_t f32_as_u8(float z) {
  if (!(z > 0.0f)) return 0;
  if (z >= 255.0f) return 255;
  return (uint8_t)z;
}

// One thread per 4-byte word of a row: word w holds row bits [32 w, 32 w + 32). `coff[j]` is
// off_j (j <= n, coff[n] = total bits); `wfirst[w]` the first code whose 8-bit window
// [off_j, off_j + 8) reaches bit 32 w.
// With `only_if` set the kernel does nothing unless *only_if == epoch (the fast path's spill flag
// of this call), so the fallback can be enqueued without a host round trip.
__global__ __launch_bounds__(256) void k_pack_rows(long d_out, int n, int rb, int wpr, const uint8_t* __restrict__ codes,
                                                   const uint32_t* __restrict__ coff,
                                                   const int* __restrict__ wfirst, uint8_t* __restrict__ qw,
                                                   const uint32_t* __restrict__ only_if, uint32_t epoch) {
  if (only_if && *only_if != epoch) return;
  for (long t = (long)blockIdx.x * 256 + threadIdx.x; t < d_out * wpr; t += (long)gridDim.x * 256) {
  const long r = t / wpr;
  const int w = (int)(t - r * wpr);
  const uint8_t* cr = codes + r * n;
  const int bit0 = 32 * w;
  uint64_t v = 0;
  for (int j = wfirst[w]; j < n; ++j) {
    const int off = (int)coff[j];
    if (off >= bit0 + 32) break;
    const uint32_t c = cr[j];
    const int s = off - bit0;
    v |= s >= 0 ? ((uint64_t)c << s) : (uint64_t)(c >> (-s));
  }
  uint8_t* dst = qw + r * rb + 4 * w;
  if (4 * w + 4 <= rb && ((uintptr_t)dst & 3u) == 0) {
    *reinterpret_cast<uint32_t*>(dst) = (uint32_t)v;
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (4 * w + k < rb) dst[k] = (uint8_t)(v >> (8 * k));
  }
  }
}

// .scales (f16 bits) and .qzeros (u8) of io::packed_tensors (src/io.rs:250-256).
__global__ __launch_bounds__(256) void k_pack_meta(long count, const float* __restrict__ scales,
                                                   const float* __restrict__ zeros, uint16_t* __restrict__ s16,
                                                   uint8_t* __restrict__ z8) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= count) return;
  s16[i] = f32_to_f16_bits(scales[i]);
  z8[i] = f32_as_u8(zeros[i]);
}

// Inverse column map with the reference's scatter semantics (`row[perm[j]] = ...`, later j wins,
// columns nobody writes stay 0): last[c] = max j with perm[j] == c. A perm entry >= n (as u32)
// sets *bad to this call's epoch instead of writing (the reference panics there). Flags carry the
// epoch of the call that set them, so they never need clearing.
__global__ __launch_bounds__(256) void k_fill_i32(int count, int v, int* __restrict__ p) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < count) p[i] = v;
}

__global__ __launch_bounds__(256) void k_invert_perm(int n, const uint32_t* __restrict__ perm, int* __restrict__ last,
                                                     uint32_t* __restrict__ bad, uint32_t epoch) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= n) return;
  const uint32_t c = perm[j];
  if (c >= (uint32_t)n) {
    atomicExch(bad, epoch);
    return;
  }
  atomicMax(&last[c], j);
}

// Per output column c, in the form the dequantization consumes: cdesc[c] = byte offset in a staged
// row of the aligned 64-bit word holding the first bit of column last[c]'s code (bits 0-19), the
// bit position in that word (bits 20-25) and the code width (bits 26-29); unpacked rows hold one
// byte per code, so there it is the byte offset last[c] with width 8. cgrp[c] = byte offset of the
// column's (scale, zero) pair in a staged row's pairs. Bit 31 of cdesc marks a column that no j
// writes.
__global__ __launch_bounds__(256) void k_col_desc(int n, int g, int packed, const int* __restrict__ last,
                                                  const uint32_t* __restrict__ coff, const uint8_t* __restrict__ cwid,
                                                  uint32_t* __restrict__ cdesc, int* __restrict__ cgrp) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= n) return;
  const int j = last[c];
  if (j < 0) {
    cdesc[c] = 0x80000000u;
    cgrp[c] = 0;
    return;
  }
  if (packed) {
    const uint32_t off = coff[j];
    cdesc[c] = ((off >> 6) * 8u) | ((off & 63u) << 20) | ((uint32_t)cwid[j] << 26);
  } else {
    cdesc[c] = (uint32_t)j | (8u << 26);
  }
  cgrp[c] = (j / g) * 8;
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Two floats narrowed to a packed pair with v_cvt_pk_f16_f32 / v_cvt_pk_bf16_f32 (round to nearest
// even, f32 denormals kept): identical to half 2.4.1 for every finite and infinite input; a NaN
// stays a NaN, its payload is the hardware's.
template <int DT>
__device__ __forceinline__ uint32_t narrow2(float a, float b) {
  const f32x2 v = {a, b};
  if (DT == CDCLQ_DTYPE_F16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

template <int DT>
__device__ __forceinline__ void store4(void* out, long idx, int cnt, const float* v) {
  if (DT == CDCLQ_DTYPE_F32) {
    float* o = static_cast<float*>(out) + idx;
    if (cnt == 4 && (reinterpret_cast<uintptr_t>(o) & 15u) == 0) {
      *reinterpret_cast<float4*>(o) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (k < cnt) o[k] = v[k];
    }
  } else {
    const uint32_t lo = narrow2<DT>(v[0], v[1]), hi = narrow2<DT>(v[2], v[3]);
    uint16_t* o = static_cast<uint16_t*>(out) + idx;
    if (cnt == 4 && (reinterpret_cast<uintptr_t>(o) & 7u) == 0) {
      *reinterpret_cast<uint2*>(o) = make_uint2(lo, hi);
    } else {
      const uint16_t h[4] = {(uint16_t)lo, (uint16_t)(lo >> 16), (uint16_t)hi, (uint16_t)(hi >> 16)};
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (k < cnt) o[k] = h[k];
    }
  }
}

// One workgroup per `rpb` consecutive rows. The rows' source bytes (packed bit streams, or one u8
// code per column) and their (scale, zero) pairs are staged in LDS; each thread then takes 4
// consecutive output columns, reads their map entries once, and produces those columns for every
// staged row:
//   out[r][c] = scale * ((f32)code - zero) for the column j = last[c] (src/quant.rs:189-202),
// narrowed once to DT (src/io.rs:50-57). PACKED reads f16 scales and u8 zeros (src/io.rs:283-285);
// otherwise f32 scales and zeros as the engine produced them.
template <bool PACKED, int DT>
__global__ __launch_bounds__(256) void k_dequant_rows(long d_out, int rpb, int n, int ng, int srcb, int sstride,
                                                      const uint8_t* __restrict__ src,
                                                      const uint32_t* __restrict__ cdesc,
                                                      const int* __restrict__ cgrp, const void* __restrict__ sc,
                                                      const void* __restrict__ zr, void* __restrict__ out) {
  extern __shared__ __align__(16) uint8_t lds[];
  float2* sz = reinterpret_cast<float2*>(lds + (long)rpb * sstride);  // [rpb][ng] (scale, zero)
  const long r0 = (long)blockIdx.x * rpb;
  const int nr = (int)min((long)rpb, d_out - r0);
  const int tid = threadIdx.x;
  const bool v16 = (srcb & 15) == 0 && (reinterpret_cast<uintptr_t>(src) & 15u) == 0;
  const bool v4 = (srcb & 3) == 0 && (reinterpret_cast<uintptr_t>(src) & 3u) == 0;
  if (v16) {  // the staged rows are contiguous in HBM: 16-byte pieces, four loads in flight per thread
    const int per = srcb / 16, total = nr * per;
    const uint4* s = reinterpret_cast<const uint4*>(src + r0 * (long)srcb);
    for (int i0 = tid; i0 < total; i0 += 1024) {
      uint4 t[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) t[q] = s[min(i0 + 256 * q, total - 1)];  // clamped: loads never branch
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int i = i0 + 256 * q;
        if (i < total) {
          const int rr = i / per;
          reinterpret_cast<uint4*>(lds + rr * sstride)[i - rr * per] = t[q];
        }
      }
    }
  } else {
    for (int rr = 0; rr < nr; ++rr) {
      const uint8_t* s = src + (r0 + rr) * (long)srcb;
      uint8_t* d = lds + rr * sstride;
      if (v4) {
        for (int i = tid; i < srcb / 4; i += 256)
          reinterpret_cast<uint32_t*>(d)[i] = reinterpret_cast<const uint32_t*>(s)[i];
      } else {
        for (int i = tid; i < srcb; i += 256) d[i] = s[i];
      }
    }
  }
  if (tid < 16 * nr) lds[(tid >> 4) * sstride + srcb + (tid & 15)] = 0;  // the word after a row's end is read
  for (int i = tid; i < nr * ng; i += 256) {
    const long e = r0 * ng + i;
    float scale, zero;
    if (PACKED) {
      scale = f16_bits_to_f32(static_cast<const uint16_t*>(sc)[e]);
      zero = (float)static_cast<const uint8_t*>(zr)[e];
    } else {
      scale = static_cast<const float*>(sc)[e];
      zero = static_cast<const float*>(zr)[e];
    }
    sz[i] = make_float2(scale, zero);
  }
  __syncthreads();
  const bool mapv = (reinterpret_cast<uintptr_t>(cdesc) & 15u) == 0 && (reinterpret_cast<uintptr_t>(cgrp) & 15u) == 0;
  for (int c0 = 4 * tid; c0 < n; c0 += 1024) {
    const int cnt = min(4, n - c0);
    uint32_t dsc[4] = {0x80000000u, 0x80000000u, 0x80000000u, 0x80000000u};
    uint32_t so[4] = {0, 0, 0, 0};
    if (cnt == 4 && mapv) {
      const uint4 dv = *reinterpret_cast<const uint4*>(cdesc + c0);
      const uint4 gv = *reinterpret_cast<const uint4*>(cgrp + c0);
      dsc[0] = dv.x, dsc[1] = dv.y, dsc[2] = dv.z, dsc[3] = dv.w;
      so[0] = gv.x, so[1] = gv.y, so[2] = gv.z, so[3] = gv.w;
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (k < cnt) {
          dsc[k] = cdesc[c0 + k];
          so[k] = (uint32_t)cgrp[c0 + k];
        }
    }
    // Unpacked once per column for all staged rows. A column written by no j reads slot 0 and is
    // forced to +0 below, so the row loop has no per-element branches.
    uint32_t wo[4], sh[4], msk[4];
    bool ok[4], cross[4];
    bool anycross = false;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      ok[k] = (dsc[k] >> 31) == 0;
      const uint32_t b = (dsc[k] >> 26) & 15u;
      wo[k] = dsc[k] & 0xfffffu;
      sh[k] = (dsc[k] >> 20) & 63u;
      msk[k] = (1u << b) - 1u;
      cross[k] = PACKED && sh[k] + b > 64u;
      anycross |= cross[k];
    }
    for (int rr = 0; rr < nr; ++rr) {
      const uint8_t* row = lds + rr * sstride;
      const uint8_t* rsz = reinterpret_cast<const uint8_t*>(sz + rr * ng);
      uint32_t code[4];
      float2 q[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if (PACKED)
          code[k] = (uint32_t)(*reinterpret_cast<const uint64_t*>(row + wo[k]) >> sh[k]);
        else
          code[k] = row[wo[k]];
        q[k] = *reinterpret_cast<const float2*>(rsz + so[k]);
      }
      if (PACKED && anycross) {
#pragma unroll
        for (int k = 0; k < 4; ++k)
          if (cross[k]) code[k] |= (uint32_t)(*reinterpret_cast<const uint64_t*>(row + wo[k] + 8) << (64u - sh[k]));
      }
      float v[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float x = q[k].x * ((float)(code[k] & msk[k]) - q[k].y);
        v[k] = ok[k] ? x : 0.0f;
      }
      store4<DT>(out, (r0 + rr) * (long)n + c0, cnt, v);
    }
  }
}

// Fast path of the packing when every run of 8 columns (j = 8k .. 8k+7) lies in one group (group
// size a multiple of 8, or a single group): such a run has one width b, starts on a byte boundary
// and fills exactly b bytes (the row's last, shorter run ends in the zero-filled partial byte).
// One thread per run. A code wider than its group's width would spill into the next run's bits
// (the reference ORs whole u8 codes); such a row is flagged in *spill and the caller re-packs the
// layer with k_pack_rows, which follows the reference for any input.
// rdesc[k] = (byte offset of run k) << 4 | its width.
__global__ __launch_bounds__(256) void k_pack_runs(long d_out, int n, int rb, int runs, const uint8_t* __restrict__ codes,
                                                   const uint32_t* __restrict__ rdesc, uint8_t* __restrict__ qw,
                                                   uint32_t* __restrict__ spill, uint32_t epoch) {
  const long t = (long)blockIdx.x * 256 + threadIdx.x;
  if (t >= d_out * runs) return;
  const long r = t / runs;
  const int j0 = 8 * (int)(t - r * runs);
  const int m = min(8, n - j0);
  const uint8_t* cr = codes + r * n + j0;
  uint64_t c8 = 0;
  if (m == 8 && (reinterpret_cast<uintptr_t>(cr) & 7u) == 0) {
    c8 = *reinterpret_cast<const uint64_t*>(cr);
  } else {
    for (int i = 0; i < m; ++i) c8 |= (uint64_t)cr[i] << (8 * i);
  }
  const uint32_t rd = rdesc[j0 >> 3], b = rd & 15u;
  uint64_t acc = 0;
  uint32_t over = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t c = (uint32_t)(c8 >> (8 * i)) & 0xffu;  // zero past the row end
    acc |= (uint64_t)c << (i * b);
    over |= c >> b;
  }
  if (over) atomicExch(spill, epoch);
  const int nb = (m * (int)b + 7) / 8;
  uint8_t* dst = qw + r * rb + (rd >> 4);
  const uintptr_t a = reinterpret_cast<uintptr_t>(dst);
  if (nb == 8 && (a & 7u) == 0) {
    *reinterpret_cast<uint64_t*>(dst) = acc;
  } else if (nb == 4 && (a & 3u) == 0) {
    *reinterpret_cast<uint32_t*>(dst) = (uint32_t)acc;
  } else if (nb == 2 && (a & 1u) == 0) {
    *reinterpret_cast<uint16_t*>(dst) = (uint16_t)acc;
  } else {
    for (int i = 0; i < nb; ++i) dst[i] = (uint8_t)(acc >> (8 * i));
  }
}

}  // namespace

hipError_t pack_rows(hipStream_t st, long d_out, int n, int rb, const uint8_t* codes, const uint32_t* coff,
                     const int* wfirst, uint8_t* qw, const uint32_t* only_if, uint32_t epoch) {
  const int wpr = (rb + 3) / 4;
  const long total = d_out * wpr;
  if (total <= 0) return hipSuccess;
  const long blocks = std::min<long>((total + 255) / 256, 2048);
  hipLaunchKernelGGL(k_pack_rows, dim3((unsigned)blocks), dim3(256), 0, st, d_out, n, rb, wpr, codes, coff, wfirst, qw,
                     only_if, epoch);
  return hipGetLastError();
}

hipError_t pack_meta(hipStream_t st, long count, const float* scales, const float* zeros, uint16_t* s16, uint8_t* z8) {
  if (count <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_pack_meta, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, st, count, scales, zeros, s16,
                     z8);
  return hipGetLastError();
}

hipError_t column_map(hipStream_t st, int n, int g, bool packed, const uint32_t* perm, const uint32_t* coff,
                      const uint8_t* cwid, int* last, uint32_t* cdesc, int* cgrp, uint32_t* bad, uint32_t epoch) {
  const dim3 grid((unsigned)((n + 255) / 256));
  hipLaunchKernelGGL(k_fill_i32, grid, dim3(256), 0, st, n, -1, last);
  hipLaunchKernelGGL(k_invert_perm, grid, dim3(256), 0, st, n, perm, last, bad, epoch);
  hipLaunchKernelGGL(k_col_desc, grid, dim3(256), 0, st, n, g, packed ? 1 : 0, last, coff, cwid, cdesc, cgrp);
  return hipGetLastError();
}

hipError_t pack_runs(hipStream_t st, long d_out, int n, int rb, const uint8_t* codes, const uint32_t* rdesc,
                     uint8_t* qw, uint32_t* spill, uint32_t epoch) {
  const int runs = (n + 7) / 8;
  const long total = d_out * runs;
  if (total > 0)
    hipLaunchKernelGGL(k_pack_runs, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, d_out, n, rb, runs,
                       codes, rdesc, qw, spill, epoch);
  return hipGetLastError();
}

// LDS per staged row: its source bytes + 16 bytes of padding (16-byte aligned) + ng (scale, zero)
static int dequant_sstride(int srcb) { return (srcb + 16 + 15) & ~15; }

static int dequant_rows_per_block(long d_out, int srcb, int ng) {
  const long per_row = dequant_sstride(srcb) + 8L * ng;
  // up to 8 rows share each column's map entries; <= 40 KiB of LDS; >= 512 workgroups
  const long r = std::min<long>(40960 / per_row, d_out / 512);
  return (int)std::max<long>(1, std::min<long>(8, r));
}

static size_t dequant_lds_bytes(int srcb, int ng, int rpb) { return (size_t)rpb * (dequant_sstride(srcb) + 8 * (size_t)ng); }

hipError_t dequant_rows(hipStream_t st, bool packed, int dtype, long d_out, int n, int ng, int srcb,
                        const uint8_t* src, const uint32_t* cdesc, const int* cgrp, const void* scales,
                        const void* zeros, void* out) {
  if (d_out <= 0 || n <= 0) return hipSuccess;
  const int rpb = dequant_rows_per_block(d_out, srcb, ng);
  const int sstride = dequant_sstride(srcb);
  const size_t lds = dequant_lds_bytes(srcb, ng, rpb);
  const unsigned grid = (unsigned)((d_out + rpb - 1) / rpb);
  auto go = [&](auto kern) -> hipError_t {
    if (lds > 65536) {
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kern, dim3(grid), dim3(256), lds, st, d_out, rpb, n, ng, srcb, sstride, src, cdesc, cgrp,
                       scales, zeros, out);
    return hipGetLastError();
  };
  if (packed) {
    if (dtype == CDCLQ_DTYPE_F32) return go(k_dequant_rows<true, CDCLQ_DTYPE_F32>);
    if (dtype == CDCLQ_DTYPE_F16) return go(k_dequant_rows<true, CDCLQ_DTYPE_F16>);
    return go(k_dequant_rows<true, CDCLQ_DTYPE_BF16>);
  }
  if (dtype == CDCLQ_DTYPE_F32) return go(k_dequant_rows<false, CDCLQ_DTYPE_F32>);
  if (dtype == CDCLQ_DTYPE_F16) return go(k_dequant_rows<false, CDCLQ_DTYPE_F16>);
  return go(k_dequant_rows<false, CDCLQ_DTYPE_BF16>);
}

}  // namespace cdclq
