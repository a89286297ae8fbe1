// Device helpers shared by the gfx950 kernels: IEEE-exact float steps,
// the reference's activation quantiser, exp and binary16 rounding.
//
// Every float operation that must reproduce the reference's order is written
// with __fadd_rn / __fmul_rn / __fdiv_rn so that no multiply-add is ever
// contracted (the library is also compiled with -ffp-contract=off).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fah {

constexpr int kWave = 64;

__device__ __forceinline__ float fadd(float a, float b) { return __fadd_rn(a, b); }
__device__ __forceinline__ float fmul(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float fdiv(float a, float b) { return __fdiv_rn(a, b); }

__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }

// Correctly rounded single-precision square root for positive normal inputs:
// hardware estimate (within 1 ulp) corrected by the sign of the fma residual
// of its two neighbours.
__device__ __forceinline__ float sqrt_rn(float x) {
  float s = __builtin_amdgcn_sqrtf(x);
  float down = u2f(f2u(s) - 1u);
  float up = u2f(f2u(s) + 1u);
  float r_down = __builtin_fmaf(-down, s, x);
  float r_up = __builtin_fmaf(-up, s, x);
  if (r_down <= 0.0f) s = down;
  else if (r_up > 0.0f) s = up;
  return s;
}

// exp as the reference's x64 ExpAvx (src/FunAsrNet/TensorMath.ExpAvx.cs:83-116):
// clamp to +-104 (NaN passes), x = n ln2 + r in double, degree-8 Taylor
// polynomial in fma form, scale by 2^n, narrow to float.
__device__ __forceinline__ float exp_ref(float value) {
  if (value != value) return value;
  float c = value < -104.0f ? -104.0f : (value > 104.0f ? 104.0f : value);
  double x = (double)c;
  double n = __builtin_rint(x * 1.4426950408889634074);
  double r = __builtin_fma(n, -0.6931471805599453094, x);
  double square = r * r;
  double fourth = square * square;
  double p23 = __builtin_fma(r, 1.0 / 6, 0.5);
  double p45 = __builtin_fma(r, 1.0 / 120, 1.0 / 24);
  double p67 = __builtin_fma(r, 1.0 / 5040, 1.0 / 720);
  double low = __builtin_fma(square, p23, 1.0 + r);
  double high = __builtin_fma(square, __builtin_fma(square, 1.0 / 40320, p67), p45);
  double e = __builtin_fma(fourth, high, low);
  long long biased = (long long)(int)n + 1023;
  double scale = __longlong_as_double(biased << 52);
  return (float)(e * scale);
}

// binary16 round trip of src/FunAsrNet/TensorMath.Half.cs:18-53
// (round to nearest even, overflow to infinity, subnormals kept).
__device__ __forceinline__ _Float16 to_half(float f) { return (_Float16)f; }
__device__ __forceinline__ float from_half(_Float16 h) { return (float)h; }

// One 32-value block of TensorMath.Quantize (src/FunAsrNet/TensorMath.cs:397-411,
// TensorMath.QuantizeAvx.cs:15-72): d = amax/127f; inv = d==0 ? 0 : 1f/d;
// q = clamp(round_half_away(x*inv), -127, 127) with .NET's saturating
// float->int conversion (NaN -> 0). The amax is the integer maximum of the
// absolute bit patterns (NaN above infinity), as the AVX path takes it.
__device__ __forceinline__ int8_t quantize_value(float x, float inverse) {
  // Branch-free: selects instead of divergent returns.
  const float v = fmul(x, inverse);
  const float t = __builtin_truncf(v);
  const float frac = __builtin_fabsf(fadd(v, -t));
  float r = frac >= 0.5f ? fadd(t, v < 0.0f ? -1.0f : 1.0f) : t;
  r = __builtin_fminf(__builtin_fmaxf(r, -127.0f), 127.0f);
  return v != v ? (int8_t)0 : (int8_t)(int)r;
}

__device__ __forceinline__ float block_scale(uint32_t max_abs_bits, float* inverse) {
  float d = fdiv(u2f(max_abs_bits), 127.0f);
  *inverse = d == 0.0f ? 0.0f : fdiv(1.0f, d);
  return d;
}

// Cross-lane moves within rows of 16 lanes (DPP): quad_perm [1,0,3,2] and
// [2,3,0,1], row_half_mirror (lane i <- 7-i of its 8) and row_mirror
// (lane i <- 15-i). All 64 lanes must be active.
constexpr int kDppQuadXor1 = 0xB1, kDppQuadXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

template <int Ctrl>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, Ctrl, 0xF, 0xF, false);
}
template <int Ctrl>
__device__ __forceinline__ double dpp_double(double v) {
  const unsigned long long u = (unsigned long long)__double_as_longlong(v);
  const uint32_t lo = dpp_u32<Ctrl>((uint32_t)u), hi = dpp_u32<Ctrl>((uint32_t)(u >> 32));
  return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}
__device__ __forceinline__ double readlane_double(double v, int lane) {
  const unsigned long long u = (unsigned long long)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), lane);
  return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

// Maximum over each aligned group of 8 lanes, in all 8 lanes.
__device__ __forceinline__ uint32_t max8_u32(uint32_t m) {
  uint32_t o = dpp_u32<kDppQuadXor1>(m);
  m = o > m ? o : m;
  o = dpp_u32<kDppQuadXor2>(m);
  m = o > m ? o : m;
  o = dpp_u32<kDppHalfMirror>(m);
  return o > m ? o : m;
}

// Wave-wide double sum (64 lanes, all active), the same value in every lane:
// pairwise within rows of 16 by DPP, then the four row sums.
__device__ __forceinline__ double wave_sum_double(double v) {
  v += dpp_double<kDppQuadXor1>(v);
  v += dpp_double<kDppQuadXor2>(v);
  v += dpp_double<kDppHalfMirror>(v);
  v += dpp_double<kDppMirror>(v);
  return (readlane_double(v, 0) + readlane_double(v, 16)) + (readlane_double(v, 32) + readlane_double(v, 48));
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  for (int m = 32; m >= 1; m >>= 1) {
    uint32_t o = __shfl_xor(v, m, kWave);
    v = o > v ? o : v;
  }
  return v;
}
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
  for (int m = 32; m >= 1; m >>= 1) {
    unsigned long long o = __shfl_xor(v, m, kWave);
    v = o > v ? o : v;
  }
  return v;
}

// Key that orders logits as QwenDecoder.Greedy does (QwenDecoder.cs:278-326):
// larger value wins, equal values keep the smaller index, -0 equals +0, NaN
// never wins (key 0).
__device__ __forceinline__ unsigned long long greedy_key(float v, uint32_t index) {
  if (v != v) return 0ull;
  if (v == 0.0f) v = 0.0f;
  uint32_t u = f2u(v);
  uint32_t ordered = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)ordered << 32) | (unsigned long long)(0xffffffffu - index);
}
__device__ __forceinline__ uint32_t greedy_index(unsigned long long key) {
  return 0xffffffffu - (uint32_t)(key & 0xffffffffull);
}

}  // namespace fah
