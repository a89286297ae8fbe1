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

// round(q * k) for an F16 k, as one mixed-precision fma with a +0 addend
// (no separate conversion): equal to fmul(q, (float)k) except that a -0
// product comes out +0. Callers only add it to sums that start at +0 and so
// are never -0 (x + -0 = x + +0 for every x but -0), which are unchanged.
__device__ __forceinline__ float mulh(float q, _Float16 k) { return __builtin_fmaf(q, (float)k, 0.0f); }

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


// ---- shared by the decode, persistent and prefill kernels ----------------

// Workgroup barrier that orders LDS only. __syncthreads() also fences global
// memory, which makes the compiler wait for every outstanding global load
// (vmcnt(0)) before the barrier -- that would drain the weight stream the
// GEMV issues ahead of its activation prologue.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Block-wide sum of one double per thread (256 threads, 4 waves).
__device__ __forceinline__ double block_sum_double(double v, double* scratch) {
  v = wave_sum_double(v);
  int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (lane == 0) scratch[wave] = v;
  lds_barrier();
  double total = 0.0;
  int waves = (blockDim.x + kWave - 1) / kWave;
  for (int i = 0; i < waves; ++i) total += scratch[i];
  return total;
}

// The reference's square sum of an RMSNorm row
// (src/FunAsrNet/TensorMath.Elementwise.cs:58-76 with mean 0): four double
// chains j = 0..3 over x[4i + j] in index order (the lanes of its two
// Vector128<double> accumulators), combined as (s0 + s2) + (s1 + s3), then
// the tail one value at a time. x(k) returns value k as a float. One thread
// does the whole sum (the rare path of rms_mean below).
template <class Read>
__device__ __forceinline__ double sum_sq_reference(Read x, int width) {
  double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
  int k = 0;
  for (; k + 4 <= width; k += 4) {
    const double a = x(k), b = x(k + 1), c = x(k + 2), d = x(k + 3);
    s0 = s0 + a * a;
    s1 = s1 + b * b;
    s2 = s2 + c * c;
    s3 = s3 + d * d;
  }
  double r = (s0 + s2) + (s1 + s3);
  for (; k < width; ++k) {
    const double z = x(k);
    r = r + z * z;
  }
  return r;
}

// The float mean (float)(S / width) of the reference's ordered square sum S,
// from `tree`, the same squares summed in another order. The squares are
// exact in double and nonnegative, so the reference's sum lies within
// (width/4 + 1) u S of the exact sum and a tree of depth D within D u S
// (u = 2^-53, recursive summation bounds): for any tree depth below
// width/4 + 78 the two means differ by less than 2 (width/4 + 40) ulps of the
// double mean m = tree / width (plus half an ulp where the division rounds).
// Rounding to float only changes at the midpoints between floats, where the
// 29 bits of m below the float mantissa read 2^28. When m is further than
// that margin from a midpoint and at least 2^-126 (a normal float), S rounds
// to the same float as m. Otherwise (about one row in 10^6, an all-zero row,
// or a sum below 2^-126) the reference's sum is formed in its own order.
// Infinite and NaN sums are infinite and NaN in any order.
__device__ __forceinline__ bool rms_mean_unsettled(double m, int width) {
  const uint64_t bits = (uint64_t)__double_as_longlong(m);
  const uint32_t low = (uint32_t)bits & 0x1fffffffu, high = (uint32_t)(bits >> 32);
  const uint32_t margin = 2u * (uint32_t)(width / 4 + 40) + 2u;
  return low + margin - (1u << 28) <= 2u * margin || high < (897u << 20);
}

// RMSNorm inverse of src/FunAsrNet/TensorMath.Elementwise.cs:58-78 (rms),
// 1f / MathF.Sqrt((float)(S / width) + eps), from the tree's sum, and
// whether the reference's S might give another one (rms_mean_unsettled).
// Latency-bound callers use the inverse at once and redo their step with
// rms_inverse_reference in the rare case, testing the flag afterwards, so
// that no branch sits between the sum and the loads that follow it.
struct RmsGuess {
  float inverse;
  bool unsettled;
};
__device__ __forceinline__ RmsGuess rms_inverse_guess(double tree, int width, float eps) {
  const double m = tree / (double)width;
  return RmsGuess{fdiv(1.0f, sqrt_rn(fadd((float)m, eps))), rms_mean_unsettled(m, width)};
}
template <class Read>
__device__ __forceinline__ float rms_inverse_reference(int width, float eps, Read x) {
  return fdiv(1.0f, sqrt_rn(fadd((float)(sum_sq_reference(x, width) / (double)width), eps)));
}
// A wave-uniform flag (every lane holds the same `tree`): one scalar test.
__device__ __forceinline__ bool wave_any(bool flag) { return __builtin_amdgcn_ballot_w64(flag) != 0; }

// The reference's inverse directly (x(k) returns value k of the row).
template <class Read>
__device__ __forceinline__ float rms_inverse(double tree, int width, float eps, Read x) {
  const RmsGuess g = rms_inverse_guess(tree, width, eps);
  if (__builtin_expect(wave_any(g.unsettled), 0)) return rms_inverse_reference(width, eps, x);
  return g.inverse;
}

// QK-norm (+ RoPE) of one 128-channel head vector held by a whole wave
// (QwenDecoder.cs:188-194, Rope.cs:14-55): lane c holds channels c and
// c + 64, the rotation partners; nw the norm weights, cs the position's 64
// cosines followed by its 64 sines (unused without ROPE). The square sum is
// the two 64-channel wave trees added low half first; the rare
// reference-order path reads the channels across the wave and redoes the
// step. Returns the (c, c + 64) pair, rotated with ROPE.
template <bool ROPE>
__device__ __forceinline__ float2 head_norm_rope(float lo, float hi, const float* nw, const float* cs, float eps) {
  const int c = threadIdx.x & (kWave - 1);
  const double sq = wave_sum_double((double)lo * (double)lo) + wave_sum_double((double)hi * (double)hi);
  const RmsGuess g = rms_inverse_guess(sq, 128, eps);
  const float w0 = nw[c], w1 = nw[64 + c];
  const float co = ROPE ? cs[c] : 1.0f, sn = ROPE ? cs[64 + c] : 0.0f;
  auto step = [&](float inverse) {
    const float nlo = fmul(fmul(lo, inverse), w0), nhi = fmul(fmul(hi, inverse), w1);
    if (!ROPE) return make_float2(nlo, nhi);
    return make_float2(fadd(fmul(nlo, co), -fmul(nhi, sn)), fadd(fmul(nlo, sn), fmul(nhi, co)));
  };
  float2 r = step(g.inverse);
  if (__builtin_expect(wave_any(g.unsettled), 0))
    r = step(rms_inverse_reference(128, eps, [&](int k) { return __shfl(k < 64 ? lo : hi, k & 63, kWave); }));
  return r;
}

// Quantise four consecutive values held by this lane; the 32-value block is
// spread over 8 consecutive lanes (shuffle max of the absolute bit patterns).
// Returns the four int8 codes packed little-endian; *scale gets the block's d.
__device__ __forceinline__ int quantize4(float v0, float v1, float v2, float v3, float* scale) {
  uint32_t m = f2u(v0) & 0x7fffffffu;
  uint32_t t = f2u(v1) & 0x7fffffffu;
  m = t > m ? t : m;
  t = f2u(v2) & 0x7fffffffu;
  m = t > m ? t : m;
  t = f2u(v3) & 0x7fffffffu;
  m = t > m ? t : m;
#pragma unroll
  for (int s = 1; s < 8; s <<= 1) {
    uint32_t o = __shfl_xor(m, s, 8);
    m = o > m ? o : m;
  }
  float inverse;
  *scale = block_scale(m, &inverse);
  uint32_t packed = (uint32_t)(uint8_t)quantize_value(v0, inverse) | ((uint32_t)(uint8_t)quantize_value(v1, inverse) << 8) |
                    ((uint32_t)(uint8_t)quantize_value(v2, inverse) << 16) |
                    ((uint32_t)(uint8_t)quantize_value(v3, inverse) << 24);
  return (int)packed;
}

// One 16-byte piece of a K row (8 F16 channels 8i..8i+7) into the eight
// channel-strided accumulators: acc[j] += q[8i+j] * k[8i+j].
__device__ __forceinline__ void score8(float* acc, const uint4& kk, const float4& q0, const float4& q1) {
  const uint32_t w[4] = {kk.x, kk.y, kk.z, kk.w};
  _Float16 k[8];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    k[2 * m] = __builtin_bit_cast(_Float16, (uint16_t)(w[m] & 0xffffu));
    k[2 * m + 1] = __builtin_bit_cast(_Float16, (uint16_t)(w[m] >> 16));
  }
  // The accumulators start at +0 (mulh's condition).
  acc[0] = fadd(acc[0], mulh(q0.x, k[0]));
  acc[1] = fadd(acc[1], mulh(q0.y, k[1]));
  acc[2] = fadd(acc[2], mulh(q0.z, k[2]));
  acc[3] = fadd(acc[3], mulh(q0.w, k[3]));
  acc[4] = fadd(acc[4], mulh(q1.x, k[4]));
  acc[5] = fadd(acc[5], mulh(q1.y, k[5]));
  acc[6] = fadd(acc[6], mulh(q1.z, k[6]));
  acc[7] = fadd(acc[7], mulh(q1.w, k[7]));
}
__device__ __forceinline__ void score8(float* acc, const uint4& kk, const float* q) {
  score8(acc, kk, *reinterpret_cast<const float4*>(q), *reinterpret_cast<const float4*>(q + 4));
}

__device__ __forceinline__ float nan_max_p(float a, float b) {
  // Selects, not branches: a if a is NaN, else b if b is NaN, else the larger.
  const float larger = b > a ? b : a;
  const float r = b != b ? b : larger;
  return a != a ? a : r;
}

// nan_max_p over the 64 lanes of a wave (all active), in every lane.
__device__ __forceinline__ float wave_max_nan(float m) {
  m = nan_max_p(m, u2f(dpp_u32<kDppQuadXor1>(f2u(m))));
  m = nan_max_p(m, u2f(dpp_u32<kDppQuadXor2>(f2u(m))));
  m = nan_max_p(m, u2f(dpp_u32<kDppHalfMirror>(f2u(m))));
  m = nan_max_p(m, u2f(dpp_u32<kDppMirror>(f2u(m))));
  const float r0 = u2f((uint32_t)__builtin_amdgcn_readlane((int)f2u(m), 0));
  const float r1 = u2f((uint32_t)__builtin_amdgcn_readlane((int)f2u(m), 16));
  const float r2 = u2f((uint32_t)__builtin_amdgcn_readlane((int)f2u(m), 32));
  const float r3 = u2f((uint32_t)__builtin_amdgcn_readlane((int)f2u(m), 48));
  return nan_max_p(nan_max_p(r0, r1), nan_max_p(r2, r3));
}

// Part of the time-ordered value sum of channel c = 2 * lane + HI: acc =
// acc + p[t] * v[t][c] in order (the reference's value loop) over
// positions [t0, t0 + count), whose V rows sit at 256 B per position from
// `base`. The dword at byte 4 * lane of a V row holds channels 2 * lane (low
// half) and 2 * lane + 1 (high half). Blocks of 16 positions: 8 paired
// reads and 4 probability reads, the next block's issued before the
// current block is added.
template <bool HI>
__device__ __forceinline__ void value_region(const char* base, const float* p, int t0, int count, float& acc) {
  const int lane = threadIdx.x & (kWave - 1);
  auto half = [](uint32_t d) { return __builtin_bit_cast(_Float16, (uint16_t)(HI ? d >> 16 : d)); };
  // Drain earlier scalar loads: with none pending, the waits inside the
  // block loop can count LDS reads instead of draining them all.
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  {
    const char* vr = base + 4 * lane;
    // The probabilities through a per-lane pointer, so that their block loads
    // take immediate offsets from one VGPR and issue with the value loads.
    using lds_float = __attribute__((address_space(3))) const float;
    lds_float* pl = (lds_float*)(p + t0);
    asm volatile("" : "+v"(pl));
    auto one = [&](int i) { acc = fadd(acc, mulh(p[t0 + i], half(*reinterpret_cast<const uint32_t*>(vr + (size_t)i * 256)))); };
    int i = 0;
    for (; i < count && ((t0 + i) & 3) != 0; ++i) one(i);
    auto fetch = [&](uint32_t* v, float4* pq, int i0) {
#pragma unroll
      for (int k = 0; k < 16; ++k) v[k] = *reinterpret_cast<const uint32_t*>(vr + (size_t)(i0 + k) * 256);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        typedef float f4 __attribute__((ext_vector_type(4)));
        using lds_f4 = __attribute__((address_space(3))) const f4;
        const f4 v = *reinterpret_cast<lds_f4*>(pl + i0 + 4 * k);
        pq[k] = make_float4(v.x, v.y, v.z, v.w);
      }
    };
    // The sixteen products first, then the in-order adds: each add then
    // finds its product long finished instead of waiting for the mixed
    // multiply issued just before it.
    auto add16 = [&](const uint32_t* v, const float4* pq) {
      float m[16];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        m[4 * k] = mulh(pq[k].x, half(v[4 * k]));
        m[4 * k + 1] = mulh(pq[k].y, half(v[4 * k + 1]));
        m[4 * k + 2] = mulh(pq[k].z, half(v[4 * k + 2]));
        m[4 * k + 3] = mulh(pq[k].w, half(v[4 * k + 3]));
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int k = 0; k < 16; ++k) acc = fadd(acc, m[k]);
    };
    if (i + 16 <= count) {
      uint32_t va[16], vb[16];
      float4 pa[4], pb[4];
      // sched_barrier keeps each block's loads ahead of the previous block's
      // adds (the scheduler would otherwise sink them next to their use).
      fetch(va, pa, i);
      for (; i + 48 <= count; i += 32) {
        fetch(vb, pb, i + 16);
        __builtin_amdgcn_sched_barrier(0);
        add16(va, pa);
        __builtin_amdgcn_sched_barrier(0);
        fetch(va, pa, i + 32);
        __builtin_amdgcn_sched_barrier(0);
        add16(vb, pb);
        __builtin_amdgcn_sched_barrier(0);
      }
      // va holds [i, i + 16); i + 16 <= count here.
      if (i + 32 <= count) {
        fetch(vb, pb, i + 16);
        __builtin_amdgcn_sched_barrier(0);
        add16(va, pa);
        add16(vb, pb);
        i += 32;
      } else {
        add16(va, pa);
        i += 16;
      }
    }
    for (; i < count; ++i) one(i);
  }
}

}  // namespace fah
