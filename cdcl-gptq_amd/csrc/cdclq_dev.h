// Device-side helpers shared by the gfx950 kernels: IEEE grid arithmetic, Rust-semantics
// min/max/clamp, wave-level reductions and the counter-based synthetic generator.
//
// Every function here must produce exactly the f32/f64 bits the reference produces, so the
// whole library is compiled with -ffp-contract=off (no silent a*b+c fusion) and with
// correctly-rounded f32 division/sqrt (hipcc's default). Fused operations are written out as
// __builtin_fmaf / __builtin_fma where the reference's matrixmultiply kernels fuse.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define CDCLQ_F16_MIN_NORMAL 6.103515625e-5f  // 2^-14, src/quant.rs:20
#define CDCLQ_KC 256                          // matrixmultiply 0.3.8 KC panel width

namespace cdclq {

// Rust f32::min / f32::max (a NaN argument yields the other one) and f32::clamp.
__device__ __host__ __forceinline__ float rs_minf(float a, float b) { return (b < a) ? b : (a != a ? b : a); }
__device__ __host__ __forceinline__ float rs_maxf(float a, float b) { return (b > a) ? b : (a != a ? b : a); }
__device__ __host__ __forceinline__ float rs_clampf(float x, float lo, float hi) {
  if (x < lo) x = lo;
  if (x > hi) x = hi;
  return x;
}

// half 2.4.1 f16::from_f32(x).to_f32(): IEEE binary16 round-to-nearest-even (src/quant.rs:24-26).
// v_cvt_f16_f32 rounds to nearest even in the default mode; any f16-subnormal result is floored to
// 2^-14 by every caller, and overflow goes to +-inf as in the reference.
__device__ __forceinline__ float round_f16(float x) { return (float)(_Float16)x; }

// quant::quant_code (src/quant.rs:92-95). Returns the dequantized value, the code in *q.
__device__ __forceinline__ float quant_dq(float x, float scale, float zero, float maxq, float* q) {
  float v = rs_clampf(__builtin_roundf(x / scale) + zero, 0.0f, maxq);
  *q = v;
  return scale * (v - zero);
}

__device__ __forceinline__ uint8_t code_of(float q) { return (q == q) ? (uint8_t)q : (uint8_t)0; }

// Near-midpoint test of one rounding decision clamp(round(num / den) + zero, 0, maxq) (the
// accounting of the parity contract): the pre-round value in f64 from the same f32 operands lies
// within 1e-9 of k + 1/2, and the two candidate results differ after clamping. The f32 quotient is
// then exactly k + 1/2 (half an f32 ulp of any |v| >= 1/2 exceeds 1e-9), which screens out all but
// those cases before the f64 division.
__device__ __forceinline__ bool near_midpoint(float num, float den, float zero, float maxq) {
  const float q = num / den;
  const float fl = __builtin_floorf(q);
  if (q - fl != 0.5f) return false;
  const double v = (double)num / (double)den;
  if (__builtin_fabs(v - (__builtin_floor(v) + 0.5)) > 1e-9) return false;
  return rs_clampf(fl + zero, 0.0f, maxq) != rs_clampf(fl + 1.0f + zero, 0.0f, maxq);
}

// Slots of the device counters of one quantize_layer call (unsigned long long each).
enum { MID_CODE_NEAR = 0, MID_ZERO_NEAR = 1, MID_CD_NEAR = 2, MID_SLOTS = 8 };

// find_params' `mk` closure (src/quant.rs:54-61).
__device__ __forceinline__ void grid_mk(float lo, float hi, float maxq, float* s, float* z) {
  float scale = round_f16((hi - lo) / maxq);
  if (scale < CDCLQ_F16_MIN_NORMAL) scale = CDCLQ_F16_MIN_NORMAL;
  *s = scale;
  *z = rs_clampf(__builtin_roundf(-lo / scale), 0.0f, maxq);
}

// ---- wave64 reductions (all lanes receive the result)
__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = rs_minf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = rs_maxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ int wave_or(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v |= __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float readlane(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// ---- counter-based synthetic generator (same algorithm as the host copy in engine.cpp)
__device__ __host__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}
__device__ __host__ __forceinline__ double u01_at(uint64_t seed, uint64_t k) {
  uint64_t z = mix64(seed + (k + 1) * 0x9E3779B97F4A7C15ULL);
  return ((double)(z >> 12) + 0.5) * (1.0 / 4503599627370496.0);
}
// ln(x) for x in (0, 1]: exponent split + 2*atanh series, basic IEEE operations only.
__device__ __host__ __forceinline__ double synth_log(double x) {
  uint64_t b = __builtin_bit_cast(uint64_t, x);
  int e = (int)((b >> 52) & 0x7ff) - 1023;
  double mm = __builtin_bit_cast(double, (b & 0xfffffffffffffULL) | (1023ULL << 52));
  if (mm > 1.4142135623730951) {
    mm = mm * 0.5;
    e += 1;
  }
  double s = (mm - 1.0) / (mm + 1.0);
  double s2 = s * s;
  double p = 0.043478260869565216;
  p = p * s2 + 0.047619047619047616;
  p = p * s2 + 0.05263157894736842;
  p = p * s2 + 0.058823529411764705;
  p = p * s2 + 0.06666666666666667;
  p = p * s2 + 0.07692307692307693;
  p = p * s2 + 0.09090909090909091;
  p = p * s2 + 0.1111111111111111;
  p = p * s2 + 0.14285714285714285;
  p = p * s2 + 0.2;
  p = p * s2 + 0.3333333333333333;
  p = p * s2 + 1.0;
  return (double)e * 0.6931471805599453 + 2.0 * s * p;
}
// cos(2*pi*u): reduction to [0, pi/2] by symmetry, Taylor series to x^22.
__device__ __host__ __forceinline__ double synth_cos2pi(double u) {
  double w = u - floor(u + 0.5);
  if (w < 0.0) w = -w;
  double sign = 1.0;
  if (w > 0.25) {
    w = 0.5 - w;
    sign = -1.0;
  }
  double x = w * 6.283185307179586;
  double x2 = x * x;
  double p = 8.896791392450574e-22;
  p = p * x2 - 4.110317623312165e-19;
  p = p * x2 + 1.5619206968586225e-16;
  p = p * x2 - 4.779477332387385e-14;
  p = p * x2 + 1.1470745597729725e-11;
  p = p * x2 - 2.08767569878681e-09;
  p = p * x2 + 2.755731922398589e-07;
  p = p * x2 - 2.48015873015873e-05;
  p = p * x2 + 0.001388888888888889;
  p = p * x2 - 0.041666666666666664;
  p = p * x2 + 0.5;
  p = 1.0 - p * x2;
  return sign * p;
}
__device__ __host__ __forceinline__ float synth_normal_at(uint64_t seed, uint64_t i) {
  double u1 = u01_at(seed, 2 * i);
  double u2 = u01_at(seed, 2 * i + 1);
  double r = sqrt(-2.0 * synth_log(u1));
  return (float)(r * synth_cos2pi(u2));
}
// Student-t with 3 degrees of freedom, Z / sqrt(chi2_3 / 3): Z = normal i of `seed`, chi2_3 the sum
// of squares of normals 3i, 3i+1, 3i+2 of a second stream; f64 basic operations, rounded once.
__device__ __host__ __forceinline__ float synth_student3_at(uint64_t seed, uint64_t i) {
  const uint64_t s2 = mix64(seed ^ 0x7F4A7C159E3779B9ULL);
  const double z = (double)synth_normal_at(seed, i);
  const double a = (double)synth_normal_at(s2, 3 * i), b = (double)synth_normal_at(s2, 3 * i + 1),
               c = (double)synth_normal_at(s2, 3 * i + 2);
  const double chi = a * a + b * b + c * c;
  return (float)(z * sqrt(3.0 / chi));
}

// ---- direct-to-LDS loads
// global_load_lds_dwordx4: every lane reads 16 bytes at its own global address; lane L's bytes land
// at lds + 16 L (lds is wave-uniform). Completion is counted by vmcnt like any vector load.
__device__ __forceinline__ void dma16(const float* g, float* lds) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)g,
                                   (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

// The same load issued from inline assembly: the compiler then tracks no LDS write for it and adds
// no wait of its own before later LDS reads (it would wait for every load in flight); the caller
// orders the data with wait_vmcnt and a barrier. The memory clobber keeps the compiler from moving
// LDS accesses across it; s_nop 0 covers the M0-write to LDS-DMA wait state. M0 is clobbered:
// only for kernels whose compiled code does not otherwise keep a value in M0 (checked for
// k_panel_dma and k_lazy_wide, where these blocks are M0's only writers and nothing else reads it).
__device__ __forceinline__ void dma16_untracked(const float* g, uint32_t lds_byte_offset) {
  const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds_byte_offset);
  uint32_t m0out;  // M0 is written by the block: declared as an output so the compiler knows
  asm volatile("s_mov_b32 %0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               : "={m0}"(m0out)
               : "v"(g), "s"(m0v)
               : "memory");
  (void)m0out;
}

// LDS byte offset of a generic pointer into LDS (the low 32 bits of a generic address in the LDS
// aperture are the offset).
__device__ __forceinline__ uint32_t lds_offset(const void* p) { return (uint32_t)(uintptr_t)p; }

// s_waitcnt vmcnt(N) with expcnt / lgkmcnt unconstrained (gfx9 encoding)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

}  // namespace cdclq
