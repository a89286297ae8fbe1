// Lock-step sessions step in one launch: the decoder layers of up to 16
// sessions, one new token each, in one grid of one workgroup per CU
// (FunAsr.cs:122-190 runs these steps one session at a time; every session's
// arithmetic here is that of its own decode step).
//
// Every workgroup owns a fixed slice of every projection's rows and computes
// them for all sessions at once, so each weight byte is read once per step
// for the whole batch. The phases of a layer hand their outputs over through
// global memory as tagged words (the value and its generation in one 64-bit
// word, written with one relaxed device-scope store), so a consumer sees data
// and readiness in the same load and no grid barrier is needed:
//
//   norm      one workgroup per session row: RMSNorm + Q8_0 of the row
//   q/k/v     all workgroups: their q/k/v rows for every session
//   attention one workgroup per (session, query head): QK-norm, RoPE, the
//             new K/V row, exact softmax and time-ordered value sums over
//             the session's cache (V rows staged in LDS), Q8_0 output
//   o         all workgroups: their o rows + the residual (kept in registers
//             by the same workgroup, which also owns those rows of down)
//   norm      one workgroup per session row (ffn norm)
//   gate/up   16 pairs of gate and up rows per workgroup: SwiGLU, then the
//             Q8_0 block of 32 ffn values, whose two halves swap their
//             maxima so that both use the block's scale
//   down      all workgroups: their down rows + the residual
//
// Quantised rows travel as Q8_0 words (four int8 codes, the block scale's
// halves in the side bits of words 0 and 1) in word-major order: word j of
// block b at j B + b, so that the product lanes of consecutive blocks read
// consecutive LDS words. After the last layer the norm workgroups write the
// output-normalised rows in Q8_0 for the lm_head. Every wait is bounded: a
// missing generation sets the error word and the workgroup leaves, so a
// broken launch ends.
#include <algorithm>

#include "fah_device.h"
#include "fah_internal.h"

namespace fah {
namespace {

using u64 = unsigned long long;
using lds_ptr = __attribute__((address_space(3))) void*;

constexpr int kSG = 256;                      // workgroups, all co-resident (one per CU)
constexpr int kST = 256;                      // threads per workgroup (four waves)
constexpr int kSLds = 160 * 1024;             // dynamic LDS per workgroup
constexpr int kSPositions = 320;              // bound on an attention unit's position + 1
constexpr int kVArea = kSPositions * 256;     // V rows of the unit's earlier positions
constexpr int kSmall = kSLds - 8 * 1024;      // small attention and exchange buffers
constexpr int kPhases = 8;                    // exchanges per layer
constexpr long kSSpin = 1L << 21;             // bounded polls per wait (~1-2 s)
constexpr uint32_t kQMask = 0xFFFF0000u;      // quantised words: 16-bit tags
constexpr int kGuPairs = 32;                  // gate/up pairs per workgroup (one Q8_0 block)

// Small area offsets (bytes from kSmall).
constexpr int kPOff = 0;                            // probabilities [kSPositions]
constexpr int kQOff = kPOff + kSPositions * 4;      // q, then value sums [128]
constexpr int kKcOff = kQOff + 512;                 // this position's K row (F16) [128]
constexpr int kVcOff = kKcOff + 256;                // this position's V row (F16) [128]
constexpr int kYOff = kVcOff + 256;                 // normalised q and k [2][128]
constexpr int kTagOff = kYOff + 1024;               // q, k, v words [3][128]
constexpr int kRedOff = kTagOff + 3 * 128 * 8;      // doubles [8]
constexpr int kLaneOff = kRedOff + 64;              // doubles [8]
constexpr int kChainOff = kLaneOff + 64;            // doubles [8]
constexpr int kMaxOff = kChainOff + 64;             // floats [4]
constexpr int kExactOff = kMaxOff + 16;             // ints [4]
constexpr int kInvOff = kExactOff + 16;             // float
constexpr int kOkOff = kInvOff + 16;                // ints [4]
static_assert(kOkOff + 16 <= 8 * 1024, "small area");
static_assert(kTagOff % 16 == 0, "16-byte LDS destinations");

// A load through a global-address-space pointer: unlike a generic (flat)
// load it cannot alias LDS, so it need not wait for the direct-to-LDS loads
// in flight.
// A store through a global-address-space pointer: a generic (flat) store
// might write LDS, so a workgroup barrier after it would wait for it.
__device__ __forceinline__ void gstore(_Float16* p, _Float16 v) { *(__attribute__((address_space(1))) _Float16*)p = v; }
__device__ __forceinline__ float gload(const float* p) { return *(const __attribute__((address_space(1))) float*)p; }
__device__ __forceinline__ uint4 gload(const uint4* p) {
  typedef unsigned int v4 __attribute__((ext_vector_type(4)));
  const v4 v = *(const __attribute__((address_space(1))) v4*)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float4 gload(const float4* p) {
  typedef float v4 __attribute__((ext_vector_type(4)));
  const v4 v = *(const __attribute__((address_space(1))) v4*)p;
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ unsigned err_load(const unsigned* e) {
  return __hip_atomic_load(e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void err_raise(unsigned* e) {
  __hip_atomic_fetch_or(e, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void put_word(u64* p, uint32_t gen, uint32_t bits) {
  __hip_atomic_store(p, ((u64)gen << 32) | (u64)bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Quantised word: 16-bit tag and 16 side bits (the block scale's halves in
// words 0 and 1 of a block) above four int8 codes.
__device__ __forceinline__ void put_qword(u64* p, uint32_t gen, uint32_t side, uint32_t codes) {
  __hip_atomic_store(p, ((u64)((gen << 16) | (side & 0xFFFFu)) << 32) | (u64)codes, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t qside(int k, float d) {
  return k == 0 ? (f2u(d) & 0xFFFFu) : (k == 1 ? f2u(d) >> 16 : 0u);
}
// Position of word wi (values 4 wi .. 4 wi + 3, block wi / 8) in a
// word-major row of B blocks.
__device__ __forceinline__ int word_major(int wi, int B) { return (wi & 7) * B + (wi >> 3); }
__device__ __forceinline__ bool current(const uint4& t, uint32_t want, uint32_t mask) {
  return (t.y & mask) == want && (t.w & mask) == want;
}

// One wave: tagged words src[128 first, 128 total) into tag (same offsets)
// until all carry the generation (high words equal `want` under `mask`).
// The last chunk's last 64 bytes are polled first (two reads in flight), so
// that an early consumer costs one small read per round trip; then rounds
// over the chunks not yet current. The loads are device-coherent (sc1).
// False after the spin bound or when another workgroup reported an error.
__device__ bool gather_words(const u64* src, u64* tag, int first, int total, uint32_t want, uint32_t mask,
                             unsigned* error) {
  const int lane = threadIdx.x & (kWave - 1);
  if (total <= first) return true;
  long spin = 0;
  {
    const u64* s = src + (size_t)(total - 1) * 128 + 120;
    u64* d = tag + (size_t)(total - 1) * 128 + 120;
    if (lane < 4) __builtin_amdgcn_global_load_lds(s + 2 * lane, (lds_ptr)d, 16, 0, 16);
    for (;; ++spin) {
      if (lane < 4) __builtin_amdgcn_global_load_lds(s + 2 * lane, (lds_ptr)d, 16, 0, 16);
      __builtin_amdgcn_s_waitcnt(1 | (7 << 4) | (15 << 8));  // vmcnt <= 1: the older poll is in
      const uint4 t = lane < 4 ? *reinterpret_cast<const uint4*>(d + 2 * lane) : make_uint4(0, want, 0, want);
      if (__all(current(t, want, mask))) break;
      if (spin > kSSpin || ((spin & 63) == 63 && err_load(error))) {
        if (lane == 0) err_raise(error);
        __builtin_amdgcn_s_waitcnt(0);
        return false;
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
  }
  const int n = total - first;
  u64 pending = n >= 64 ? ~0ull : ((1ull << n) - 1ull);
  for (;; ++spin) {
    for (u64 m = pending; m; m &= m - 1) {
      const int k = first + __builtin_ctzll(m);
      __builtin_amdgcn_global_load_lds(src + (size_t)k * 128 + 2 * lane, (lds_ptr)(tag + (size_t)k * 128), 16, 0, 16);
    }
    __builtin_amdgcn_s_waitcnt(0);
    for (u64 m = pending; m; m &= m - 1) {
      const int j = __builtin_ctzll(m);
      const uint4 t = *reinterpret_cast<const uint4*>(tag + (size_t)(first + j) * 128 + 2 * lane);
      if (__all(current(t, want, mask))) pending &= ~(1ull << j);
    }
    if (!pending) return true;
    if (spin > kSSpin || ((spin & 63) == 63 && err_load(error))) {
      if (lane == 0) err_raise(error);
      return false;
    }
  }
}

// One wave: two 128-word chunks at a, b into tag[0, 256), polled whole in
// rounds of two reads, two rounds in flight.
__device__ bool gather2(const u64* a, const u64* b, u64* tag, uint32_t gen, unsigned* error) {
  const int lane = threadIdx.x & (kWave - 1);
  auto round = [&] {
    __builtin_amdgcn_global_load_lds(a + 2 * lane, (lds_ptr)(tag), 16, 0, 16);
    __builtin_amdgcn_global_load_lds(b + 2 * lane, (lds_ptr)(tag + 128), 16, 0, 16);
  };
  round();
  for (long spin = 0;; ++spin) {
    round();
    __builtin_amdgcn_s_waitcnt(2 | (7 << 4) | (15 << 8));  // vmcnt <= 2: the older round is in
    bool all = true;
#pragma unroll
    for (int k = 0; k < 2; ++k) all = all && __all(current(*reinterpret_cast<const uint4*>(tag + 128 * k + 2 * lane), gen, ~0u));
    if (all) {
      __builtin_amdgcn_s_waitcnt(0);  // the newer round writes the same current words
      return true;
    }
    if (spin > kSSpin || ((spin & 63) == 63 && err_load(error))) {
      if (lane == 0) err_raise(error);
      __builtin_amdgcn_s_waitcnt(0);
      return false;
    }
  }
}

// One wave: 16 tagged words at src into tag, two polls in flight.
__device__ bool gather16(const u64* src, u64* tag, uint32_t gen, unsigned* error) {
  const int lane = threadIdx.x & (kWave - 1);
  auto poll = [&] {
    if (lane < 8) __builtin_amdgcn_global_load_lds(src + 2 * lane, (lds_ptr)tag, 16, 0, 16);
  };
  poll();
  for (long spin = 0;; ++spin) {
    poll();
    __builtin_amdgcn_s_waitcnt(1 | (7 << 4) | (15 << 8));
    const uint4 t = lane < 8 ? *reinterpret_cast<const uint4*>(tag + 2 * lane) : make_uint4(0, gen, 0, gen);
    if (__all(current(t, gen, ~0u))) {
      __builtin_amdgcn_s_waitcnt(0);
      return true;
    }
    if (spin > kSSpin || ((spin & 63) == 63 && err_load(error))) {
      if (lane == 0) err_raise(error);
      __builtin_amdgcn_s_waitcnt(0);
      return false;
    }
  }
}

// Whether every wave's part succeeded (two barriers, so the flags can be
// written again by the next call).
__device__ __forceinline__ bool all_waves(bool ok, int* ok_s) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & (kWave - 1);
  if (lane == 0) ok_s[wave] = ok ? 1 : 0;
  lds_barrier();
  const bool r = (ok_s[0] & ok_s[1] & ok_s[2] & ok_s[3]) != 0;
  lds_barrier();
  return r;
}

// The score of one position whose K row (16 pieces of 8 F16 channels) is in
// registers: the eight channel-strided accumulators and their pairwise tree
// (AttentionAvx.cs:74-118), divided by the divisor. q is read from LDS in
// blocks of 16 channels, the next block's reads issued before the current
// block's products, so that a wave waits for one LDS round trip per score
// rather than one per 8 channels.
__device__ __forceinline__ float score_regs(const uint4* k, const float* q, float divisor) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  using lds_f4 = __attribute__((address_space(3))) const f4;
  // No scalar loads pending: the block waits can count LDS reads alone.
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  lds_f4* ql = (lds_f4*)q;
  asm volatile("" : "+v"(ql));
  float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  f4 qa[4], qb[4];
  auto fetch = [&](f4* d, int blk) {
#pragma unroll
    for (int j = 0; j < 4; ++j) d[j] = ql[4 * blk + j];
  };
  auto use = [&](const f4* d, int blk) {
    score8(acc, k[2 * blk], make_float4(d[0].x, d[0].y, d[0].z, d[0].w), make_float4(d[1].x, d[1].y, d[1].z, d[1].w));
    score8(acc, k[2 * blk + 1], make_float4(d[2].x, d[2].y, d[2].z, d[2].w), make_float4(d[3].x, d[3].y, d[3].z, d[3].w));
  };
  fetch(qa, 0);
#pragma unroll
  for (int blk = 0; blk < 8; blk += 2) {
    fetch(qb, blk + 1);
    __builtin_amdgcn_sched_barrier(0);
    use(qa, blk);
    __builtin_amdgcn_sched_barrier(0);
    if (blk + 2 < 8) fetch(qa, blk + 2);
    __builtin_amdgcn_sched_barrier(0);
    use(qb, blk + 1);
    __builtin_amdgcn_sched_barrier(0);
  }
  const float sc = fadd(fadd(fadd(acc[0], acc[4]), fadd(acc[1], acc[5])), fadd(fadd(acc[2], acc[6]), fadd(acc[3], acc[7])));
  return fdiv(sc, divisor);
}

typedef int v4i __attribute__((ext_vector_type(4)));

// One wave's 16-row tile of a projection for up to 16 sessions on the matrix
// cores, in q8_head_mfma16_kernel's operand layout: lane (r, q) = (lane % 16,
// lane / 16) keeps weight bytes 8q .. 8q + 7 of every block of tile row r and
// the row's block scales; per block one v_mfma_i32_16x16x32_i8 forms the
// exact int32 block dots of the 16 rows with 16 sessions' codes (session r
// as operand A), and lane (r, q) adds the terms ((float)dot * w_scale) *
// x_scale of sessions 4q .. 4q + 3 in block order -- the few-frame kernel's
// arithmetic and order.
template <int K>
struct MfmaTile {
  static constexpr int B = K / 32;
  static constexpr int APS = 65;  // u64 per block in the packed operands (64 + 1: no bank conflicts)
  long wv[B];
  float wsv[B];

  template <class RowOf>
  __device__ __forceinline__ void load(const int8_t* w, const _Float16* s, RowOf row_of) {
    const int lane = threadIdx.x & (kWave - 1), r = lane & 15, q = lane >> 4;
    const int sr = row_of(r);
    const int8_t* wrow = w + (size_t)sr * K + 8 * q;
#pragma unroll
    for (int b = 0; b < B; ++b) {
      wv[b] = *(const __attribute__((address_space(1))) long*)(wrow + 32 * b);
      wsv[b] = (float)s[(size_t)sr * B + b];
    }
  }

  // All threads: the sessions' gathered words (stage: [S][K / 4], word j of
  // block b at j B + b) into the packed A operands apack[b][q * 16 + r] and
  // the session scales xs[b][16] (sessions past S: zero).
  __device__ __forceinline__ static void pack(const u64* stage, int S, u64* apack, float* xs) {
    const int tid = threadIdx.x, r = tid >> 4, m = tid & 15;
    for (int b = m; b < B; b += 16) {
      uint32_t lo[8];
      uint32_t s01 = 0;
      if (r < S) {
        const u64* src = stage + (size_t)r * (K / 4) + b;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const u64 v = src[(size_t)j * B];
          lo[j] = (uint32_t)v;
          if (j == 0) s01 = (uint32_t)(v >> 32) & 0xFFFFu;
          if (j == 1) s01 |= ((uint32_t)(v >> 32) & 0xFFFFu) << 16;
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) lo[j] = 0u;
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) apack[(size_t)b * APS + q * 16 + r] = (u64)lo[2 * q] | ((u64)lo[2 * q + 1] << 32);
      xs[b * 16 + r] = u2f(s01);
    }
  }

  // This wave's sums: acc[j] = row r, session 4q + j. The next block's dots
  // are issued before this block's terms are added (and its operand read
  // before that), so the adds do not wait for the matrix core.
  __device__ __forceinline__ void sums(const u64* apack, const float* xs, float* acc) const {
    const int lane = threadIdx.x & (kWave - 1), q = lane >> 4;
    const v4i zero4 = {0, 0, 0, 0};
    acc[0] = acc[1] = acc[2] = acc[3] = 0.0f;
    long an = (long)apack[lane];
    v4i dc = __builtin_amdgcn_mfma_i32_16x16x32_i8(an, wv[0], zero4, 0, 0, 0);
    if (B > 1) an = (long)apack[(size_t)APS + lane];
    float4 xn = *reinterpret_cast<const float4*>(xs + 4 * q);
#pragma unroll
    for (int b = 0; b < B; ++b) {
      v4i dn = dc;
      const float4 xv = xn;
      if (b + 1 < B) {
        dn = __builtin_amdgcn_mfma_i32_16x16x32_i8(an, wv[b + 1], zero4, 0, 0, 0);
        xn = *reinterpret_cast<const float4*>(xs + (b + 1) * 16 + 4 * q);
      }
      if (b + 2 < B) an = (long)apack[(size_t)(b + 2) * APS + lane];
      __builtin_amdgcn_sched_barrier(0);
      acc[0] = fadd(acc[0], fmul(fmul((float)dc[0], wsv[b]), xv.x));
      acc[1] = fadd(acc[1], fmul(fmul((float)dc[1], wsv[b]), xv.y));
      acc[2] = fadd(acc[2], fmul(fmul((float)dc[2], wsv[b]), xv.z));
      acc[3] = fadd(acc[3], fmul(fmul((float)dc[3], wsv[b]), xv.w));
      __builtin_amdgcn_sched_barrier(0);
      dc = dn;
    }
  }
};

// A workgroup's rows of one projection (K inputs, SLOTS storage rows) for
// every session, as q8_gemm_few_kernel forms them: lane = (row step, block)
// keeps its rows' 32-byte weight blocks and block scales in registers; for
// each session's quantised input block it forms the exact int32 block dot
// (v_dot4_i32_i8 x 8) and the term ((float)dot * w_scale) * x_scale into
// LDS; then one lane per (row, session) adds the terms in block order.
template <int K, int SLOTS>
struct Slice {
  static constexpr int B = K / 32, RS = kST / B, P = (SLOTS + RS - 1) / RS, TB = B + 4, KW = K / 4;
  uint4 w0[P], w1[P];
  float ws[P];

  template <class RowOf>
  __device__ __forceinline__ void load(const int8_t* w, const _Float16* s, RowOf row_of) {
    const int tid = threadIdx.x, lrow = tid / B, b = tid - lrow * B;
    const bool active = lrow < RS;
#pragma unroll
    for (int k = 0; k < P; ++k) {
      // Unconditional loads (row clamped into the matrix); rows past the
      // slice are never summed.
      const int i = lrow + RS * k;
      const int sr = active && i < SLOTS ? row_of(i) : 0;
      const uint4* wp = reinterpret_cast<const uint4*>(w + (size_t)sr * K + 32 * b);
      w0[k] = wp[0];
      w1[k] = wp[1];
      ws[k] = (float)s[(size_t)sr * B + b];
    }
  }

  // stage: the sessions' quantised rows as gathered words [S][KW] in
  // word-major order (word j of block b at j B + b, so that the lanes of
  // consecutive blocks read consecutive words); terms: [SLOTS][S][TB] floats.
  __device__ __forceinline__ void products(const u64* stage, int S, float* terms) const {
    const int tid = threadIdx.x, lrow = tid / B, b = tid - lrow * B;
    if (lrow >= RS) return;
    // Two sessions' blocks in flight: the next one is read while this one is
    // formed, the buffers alternating (no register copies).
    auto fetch = [&](uint2* u, int f) {
      const uint2* xp = reinterpret_cast<const uint2*>(stage + (size_t)f * KW + b);
#pragma unroll
      for (int j = 0; j < 8; ++j) u[j] = xp[j * B];
    };
    auto form = [&](const uint2* u, int f) {
      const float xsv = u2f((u[0].y & 0xFFFFu) | ((u[1].y & 0xFFFFu) << 16));
#pragma unroll
      for (int k = 0; k < P; ++k) {
        const int i = lrow + RS * k;
        if (i < SLOTS) {
          // One chain of eight (integer sums: exact in any order; the P
          // rows' chains interleave).
          int dot = 0;
          dot = __builtin_amdgcn_sdot4((int)w0[k].x, (int)u[0].x, dot, false);
          dot = __builtin_amdgcn_sdot4((int)w0[k].y, (int)u[1].x, dot, false);
          dot = __builtin_amdgcn_sdot4((int)w0[k].z, (int)u[2].x, dot, false);
          dot = __builtin_amdgcn_sdot4((int)w0[k].w, (int)u[3].x, dot, false);
          dot = __builtin_amdgcn_sdot4((int)w1[k].x, (int)u[4].x, dot, false);
          dot = __builtin_amdgcn_sdot4((int)w1[k].y, (int)u[5].x, dot, false);
          dot = __builtin_amdgcn_sdot4((int)w1[k].z, (int)u[6].x, dot, false);
          dot = __builtin_amdgcn_sdot4((int)w1[k].w, (int)u[7].x, dot, false);
          terms[((size_t)i * S + f) * TB + b] = fmul(fmul((float)dot, ws[k]), xsv);
        }
      }
    };
    uint2 ua[8], ub[8];
    fetch(ua, 0);
    int f = 0;
    for (; f + 2 <= S; f += 2) {
      fetch(ub, f + 1);
      form(ua, f);
      if (f + 2 < S) fetch(ua, f + 2);
      form(ub, f + 1);
    }
    if (f < S) form(ua, f);
  }

  __device__ __forceinline__ static float row_sum(const float* terms, int i, int f, int S) {
    const float* t = terms + ((size_t)i * S + f) * TB;
    float sum = 0.0f;
#pragma unroll 4
    for (int b = 0; b < B; b += 4) {
      const float4 v = *reinterpret_cast<const float4*>(t + b);
      sum = fadd(sum, v.x);
      sum = fadd(sum, v.y);
      sum = fadd(sum, v.z);
      sum = fadd(sum, v.w);
    }
    return sum;
  }
  static constexpr size_t stage_bytes(int S) { return (size_t)S * KW * 8; }
};

// Gathers the sessions' quantised rows ([S][KW] words) on all four waves.
template <int KW>
__device__ __forceinline__ bool gather_rows(const u64* src, u64* stage, int S, uint32_t gen, unsigned* error, int* ok_s) {
  const int wave = threadIdx.x >> 6;
  const int n = S * KW / 128;
  const bool ok = gather_words(src, stage, wave * n / 4, (wave + 1) * n / 4, gen << 16, kQMask, error);
  return all_waves(ok, ok_s);
}

// RMSNorm + Q8_0 of one W-value row, norm_quantize_rows_kernel's arithmetic:
// thread t holds values 4t + 1024c; the square sum in any tree order with
// the reference order where the mean is unsettled (rms_inverse). read(k)
// returns value k. Each thread's 4 codes and (every 8th thread) the block
// scale go to emit(e, codes, d).
template <int W>
struct NormWeights {
  static constexpr int NC = (W + 1023) / 1024;
  float4 v[NC];
  // Thread t's weights 4t + 1024c .. + 3, loaded ahead of the row's gather
  // (a wave's loads complete in order: a load issued after the gather's
  // weight loads would wait for them).
  __device__ __forceinline__ void load(const float* norm_w) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int e = c * 1024 + 4 * (int)threadIdx.x;
      v[c] = e < W ? gload(reinterpret_cast<const float4*>(norm_w + e)) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  }
};

template <int W, class Read, class Emit>
__device__ __forceinline__ void norm_row(Read read, const NormWeights<W>& nwt, float eps, double* red_s, Emit emit) {
  constexpr int NC = NormWeights<W>::NC;
  const int tid = threadIdx.x;
  float4 v[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int e = c * 1024 + 4 * tid;
    v[c] = e < W ? make_float4(read(e), read(e + 1), read(e + 2), read(e + 3)) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  double sq = 0.0;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    sq += (double)v[c].x * (double)v[c].x + (double)v[c].y * (double)v[c].y;
    sq += (double)v[c].z * (double)v[c].z + (double)v[c].w * (double)v[c].w;
  }
  const float inverse = rms_inverse(block_sum_double(sq, red_s), W, eps, read);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int e = c * 1024 + 4 * tid;
    if (e < W) {
      const float4 w = nwt.v[c];
      const float x0 = fmul(fmul(v[c].x, inverse), w.x), x1 = fmul(fmul(v[c].y, inverse), w.y);
      const float x2 = fmul(fmul(v[c].z, inverse), w.z), x3 = fmul(fmul(v[c].w, inverse), w.w);
      float d;
      const int packed = quantize4(x0, x1, x2, x3, &d);
      emit(e, packed, d);
    }
  }
}

template <int W, int H, int KVH, int FF>
__global__ __launch_bounds__(kST) void session_step_kernel(SessionStepArgs a) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  constexpr int HS = 128, G = H / KVH, QW = H * HS, KVW = KVH * HS, NQKV = QW + 2 * KVW;
  // o and down: kOGroups groups of sessions, each workgroup R2 rows of one
  // group (fewer sessions a workgroup: less of the exchanged vectors to read,
  // more weight rows, which are requested before the wait).
  constexpr int kOGroups = 4, kOSessions = 16 / kOGroups;
  // q/k/v: kQGroups groups of sessions likewise; gate/up: kGuGroups groups,
  // kGuPairs pairs (one Q8_0 block of the ffn vector) a workgroup.
  constexpr int kQGroups = 2, kQSessions = 16 / kQGroups, kGuGroups = 2, kGuSessions = 16 / kGuGroups;
  constexpr int R1 = NQKV * kQGroups / kSG, R2 = W * kOGroups / kSG, NGU = FF / kGuPairs * kGuGroups;
  static_assert(NQKV % kSG == 0 && W % kSG == 0 && FF % 32 == 0 && NGU <= kSG && NGU % 2 == 0, "shape");
  using QkvSlice = Slice<W, R1>;
  using OSlice = Slice<QW, R2>;
  using GuTile = MfmaTile<W>;
  static_assert(2 * kGuPairs == 64, "four 16-row gate/up tiles, one a wave");
  using DownSlice = Slice<FF, R2>;
  static_assert(QkvSlice::stage_bytes(kQSessions) + (size_t)R1 * kQSessions * QkvSlice::TB * 4 <= (size_t)(kSmall - kVArea),
                "q/k/v area");
  static_assert(OSlice::stage_bytes(kOSessions) + (size_t)R2 * kOSessions * OSlice::TB * 4 <= (size_t)kSmall, "o area");
  // Gate/up LDS: the gathered rows, then from kGuPackOff the packed operands,
  // session scales, sums and SwiGLU values.
  constexpr int kGuPackOff = kGuSessions * (W / 4) * 8;
  static_assert(kGuPackOff + (size_t)GuTile::B * GuTile::APS * 8 + GuTile::B * 16 * 4 + 2 * kGuPairs * 16 * 4 +
                    kGuPairs * kGuSessions * 4 <=
                    (size_t)kSmall, "gate/up area");
  static_assert(DownSlice::stage_bytes(kOSessions) + (size_t)R2 * kOSessions * DownSlice::TB * 4 <= (size_t)kSmall,
                "down area");

  const int w = blockIdx.x, tid = threadIdx.x, wave = tid >> 6, lane = tid & (kWave - 1);
  const int S = a.S, L = a.layers;
  if (err_load(a.error)) return;
  const uint32_t g0 = __hip_atomic_load(a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) *
                          (uint32_t)(kPhases * L + 1) + 1u;
  auto gen = [&](int l, int p) { return g0 + (uint32_t)(l * kPhases + p - 1); };

  char* small = lds + kSmall;
  float* p_s = reinterpret_cast<float*>(small + kPOff);
  float* q_s = reinterpret_cast<float*>(small + kQOff);
  _Float16* kcur_s = reinterpret_cast<_Float16*>(small + kKcOff);
  _Float16* vcur_s = reinterpret_cast<_Float16*>(small + kVcOff);
  float* y_s = reinterpret_cast<float*>(small + kYOff);
  u64* qkv_tag = reinterpret_cast<u64*>(small + kTagOff);
  double* red_s = reinterpret_cast<double*>(small + kRedOff);
  double* lane_s = reinterpret_cast<double*>(small + kLaneOff);
  double* chain_s = reinterpret_cast<double*>(small + kChainOff);
  float* tmax_s = reinterpret_cast<float*>(small + kMaxOff);
  int* exact_s = reinterpret_cast<int*>(small + kExactOff);
  float* inv_s = reinterpret_cast<float*>(small + kInvOff);
  int* ok_s = reinterpret_cast<int*>(small + kOkOff);

  // Roles. The norm rows of session s on workgroup 192 + s + 16 (s % 4):
  // past the gate/up workgroups (their ffn norm does not delay a gate/up
  // share), one XCD per session row mod 8. Attention unit w is (session
  // w / H, query head w % H).
  static_assert(NGU <= 192, "norm workgroups hold no gate/up share");
  const int nr = w - 192, ns = (nr >= 0 && (nr & 15) + 16 * ((nr & 15) & 3) == nr && (nr & 15) < S) ? (nr & 15) : -1;
  const int us = w / H, uh = w % H, kh = uh / G;
  const bool unit = us < S;
  int pos = 0, cap = 0;
  const float *rcos = nullptr, *rsin = nullptr;
  _Float16 *kbase = nullptr, *vbase = nullptr;
  if (unit) {
    const SessionRef& ss = a.sessions[us];
    pos = min(*ss.position, a.max_positions - 1);
    cap = ss.capacity;
    rcos = ss.rope_cos;
    rsin = ss.rope_sin;
    kbase = ss.kcache;
    vbase = ss.vcache;
  }
  const int nv = pos, n = pos + 1;  // earlier positions read from the cache; this one is local
  // Exchange words per layer.
  const size_t LX = (size_t)S * W, LQ = (size_t)S * (W / 4), LQKV = (size_t)S * NQKV, LATT = (size_t)S * (QW / 4),
               LH = (size_t)S * (FF / 4);

  // o/down share: rows R2 (w / kOGroups) .. of sessions f0 .. f0 + Sg - 1
  // (group w % kOGroups). Their residual: lane t < R2 Sg holds (row
  // R2 (w / kOGroups) + t / Sg, session f0 + t % Sg).
  // A batch below 16 sessions is split evenly over the groups (ceil(S /
  // groups) sessions a group), so that every group has work.
  const int on = (S + kOGroups - 1) / kOGroups, qn = (S + kQGroups - 1) / kQGroups, gn = (S + kGuGroups - 1) / kGuGroups;
  const int f0 = on * (w % kOGroups), Sg = max(0, min(on, S - f0)), orow0 = R2 * (w / kOGroups);
  // q/k/v share: rows qrow0 .. of sessions qf0 .. qf0 + Sq - 1; gate/up
  // share: pairs gp0 .. of sessions gf0 .. gf0 + Sgu - 1.
  const int qf0 = qn * (w % kQGroups), Sq = max(0, min(qn, S - qf0)), qrow0 = R1 * (w / kQGroups);
  const int gf0 = gn * (w % kGuGroups), Sgu = max(0, min(gn, S - gf0)), gp0 = kGuPairs * (w / kGuGroups);
  float xres = 0.0f, ares = 0.0f;
  const int ri = tid / max(Sg, 1), rf = f0 + tid - ri * max(Sg, 1), rrow = orow0 + ri;
  const bool rlane = tid < R2 * Sg;
  if (rlane) xres = a.x_in[(size_t)rf * W + rrow];

  for (int l = 0; l < L; ++l) {
    const PersistentLayer& lw = a.layer_table[l];
    // This layer's exchange words (each layer has its own: a slow reader of
    // one layer's words never meets the next layer's).
    u64* const tx = a.tx + (size_t)l * LX;
    u64* const txq = a.txq + (size_t)l * LQ;
    u64* const tqkv = a.tqkv + (size_t)l * LQKV;
    u64* const tattq = a.tattq + (size_t)l * LATT;
    u64* const ta = a.ta + (size_t)l * LX;
    u64* const taq = a.taq + (size_t)l * LQ;
    u64* const thq = a.thq + (size_t)l * LH;
    // ---- attention unit: this layer's earlier K rows (one a thread, in
    // registers) and V rows (to LDS), requested at the start of the layer --
    // by a norm workgroup once it has gathered its q/k/v input, so that
    // neither of its gathers waits behind them -- and used after q/k/v.
    const _Float16* kc = unit ? kbase + ((size_t)l * KVH + kh) * (size_t)cap * HS : nullptr;
    const _Float16* vc = unit ? vbase + ((size_t)l * KVH + kh) * (size_t)cap * HS : nullptr;
    uint4 k0[16];
    auto kv_loads = [&]() __attribute__((always_inline)) {
      const char* src = reinterpret_cast<const char*>(vc);
      const int bytes = nv * HS * 2;
      for (int c = wave * 1024; c < bytes; c += 4 * 1024)
        if (c + 16 * lane < bytes) __builtin_amdgcn_global_load_lds(src + c + 16 * lane, (lds_ptr)(lds + c), 16, 0, 0);
      if (tid < nv) {
        const uint4* row = reinterpret_cast<const uint4*>(kc + (size_t)tid * HS);
#pragma unroll
        for (int i = 0; i < 16; ++i) k0[i] = gload(row + i);
      }
    };
    // The unit's QK-norm weight and RoPE factors of its channel (thread t:
    // channel t % 128 of q (t < 128) or k), requested first.
    float qk_nw = 0.0f, qk_cs = 0.0f, qk_sn = 0.0f;
    if (unit) {
      const int c = tid & (HS - 1), half = HS / 2;
      qk_nw = gload((tid < HS ? lw.q_norm : lw.k_norm) + c);
      qk_cs = gload(rcos + (size_t)pos * half + (c & (half - 1)));
      qk_sn = gload(rsin + (size_t)pos * half + (c & (half - 1)));
    }
    if (unit && ns < 0) kv_loads();

    // The q/k/v weight slice: requested now, or by a norm workgroup once its
    // row is gathered (its polls would wait behind the loads), so that its
    // products do not start later than the others'.
    QkvSlice qsl;
    auto qkv_weights = [&]() __attribute__((always_inline)) { qsl.load(lw.wqkv, lw.sqkv, [&](int i) { return qrow0 + i; }); };
    if (ns < 0) qkv_weights();

    // ---- attention norm of session row ns (norm workgroups)
    u64* qstage = reinterpret_cast<u64*>(lds + kVArea);  // q/k/v phase: staging, then terms
    if (ns >= 0) {
      NormWeights<W> nwt;
      nwt.load(lw.attn_norm);
      u64* dst = txq + (size_t)ns * (W / 4);
      auto emit = [&](int e, int packed, float d) {
        put_qword(dst + word_major(e / 4, W / 32), gen(l, 1), qside((e / 4) & 7, d), (uint32_t)packed);
      };
      if (l == 0) {
        qkv_weights();
        const float* row = a.x_in + (size_t)ns * W;
        norm_row<W>([&](int k) { return row[k]; }, nwt, a.eps, red_s, emit);
      } else {
        const bool ok = gather_words(a.tx + (size_t)(l - 1) * LX + (size_t)ns * W, qstage, wave * (W / 128) / 4, (wave + 1) * (W / 128) / 4,
                                     gen(l - 1, 8), ~0u, a.error);
        if (!all_waves(ok, ok_s)) return;
        qkv_weights();
        norm_row<W>([&](int k) { return u2f((uint32_t)qstage[k]); }, nwt, a.eps, red_s, emit);
      }
      lds_barrier();
      if (unit && Sq == 0) kv_loads();
    }

    // ---- q/k/v rows qrow0 .. of sessions qf0 ..
    if (Sq > 0) {
      if (!gather_rows<W / 4>(txq + (size_t)qf0 * (W / 4), qstage, Sq, gen(l, 1), a.error, ok_s)) return;
      if (unit && ns >= 0) kv_loads();
      float* terms = reinterpret_cast<float*>(lds + kVArea + QkvSlice::stage_bytes(Sq));
      qsl.products(qstage, Sq, terms);
      lds_barrier();
      for (int t = tid; t < R1 * Sq; t += kST) {
        const int i = t / Sq, f = t - i * Sq;
        put_word(tqkv + (size_t)(qf0 + f) * NQKV + qrow0 + i, gen(l, 2), f2u(QkvSlice::row_sum(terms, i, f, Sq)));
      }
    }

    // ---- attention of (session us, query head uh)
    if (unit) {
      bool ok = true;
      const u64* base = tqkv + (size_t)us * NQKV;
      if (wave == 0) ok = gather2(base + uh * HS, base + QW + kh * HS, qkv_tag, gen(l, 2), a.error);
      if (!all_waves(ok, ok_s)) return;
      // QK-norm and RoPE of q (threads 0-127) and k (128-255)
      // (QwenDecoder.cs:186-203, Rope.cs:14-55); the first query head of the
      // pair writes the K row. The v row is gathered during the value sums.
      {
        const int part = tid >> 7, c = tid & 127, half = HS / 2;
        const float v = u2f((uint32_t)qkv_tag[128 * part + c]);
        const float nw = qk_nw, cs = qk_cs, sn = qk_sn;
        const double sq = wave_sum_double((double)v * (double)v);
        if (lane == 0) red_s[wave] = sq;
        lds_barrier();
        const float inverse = rms_inverse(red_s[2 * part] + red_s[2 * part + 1], HS, a.eps,
                                          [&](int k) { return u2f((uint32_t)qkv_tag[128 * part + k]); });
        y_s[part * 128 + c] = fmul(fmul(v, inverse), nw);
        lds_barrier();
        const float* y = y_s + part * 128;
        float r;
        if (c < half) r = fadd(fmul(y[c], cs), -fmul(y[c + half], sn));
        else r = fadd(fmul(y[c - half], sn), fmul(y[c], cs));
        if (part == 0) {
          q_s[c] = r;
        } else {
          const _Float16 k16 = to_half(r);
          kcur_s[c] = k16;
          if (uh % G == 0) gstore(const_cast<_Float16*>(kc) + (size_t)pos * HS + c, k16);
        }
      }
      lds_barrier();
      // Scores: one position per thread, its K row in registers (thread nv,
      // this position when it is below kST, copies its row from LDS), eight
      // channel-strided accumulators and their pairwise tree
      // (AttentionAvx.cs:74-118); positions from kST on read their rows here.
      if (tid == nv) {
#pragma unroll
        for (int i = 0; i < 16; ++i) k0[i] = reinterpret_cast<const uint4*>(kcur_s)[i];
      }
      // Each thread also takes the maximum of its own scores (the softmax's
      // first step, SoftmaxAvx.cs:11-58, order-free), so that one barrier
      // serves both.
      float m = -__builtin_inff();
      if (tid < n) {
        const float sc = score_regs(k0, q_s, a.divisor);
        p_s[tid] = sc;
        m = sc;
      }
      for (int s = tid + kST; s < n; s += kST) {
        float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
        if (s < nv) {
          const uint4* row = reinterpret_cast<const uint4*>(kc + (size_t)s * HS);
#pragma unroll
          for (int i0 = 0; i0 < 16; i0 += 4) {
            uint4 kk[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) kk[i] = row[i0 + i];
#pragma unroll
            for (int i = 0; i < 4; ++i) score8(acc, kk[i], q_s + 8 * (i0 + i));
          }
        } else {
#pragma unroll
          for (int i = 0; i < 16; ++i) score8(acc, reinterpret_cast<const uint4*>(kcur_s)[i], q_s + 8 * i);
        }
        const float sc = fdiv(fadd(fadd(fadd(acc[0], acc[4]), fadd(acc[1], acc[5])), fadd(fadd(acc[2], acc[6]), fadd(acc[3], acc[7]))),
                              a.divisor);
        p_s[s] = sc;
        m = nan_max_p(m, sc);
      }
      // Exact softmax (SoftmaxAvx.cs:11-58): the maximum, the numerators, the
      // double denominator -- as wave trees when every numerator is 0 or in
      // [2^-17, 1] (then every partial sum is exact), the reference's
      // residue chains otherwise. (A thread's numerators come from its own
      // scores; the value sums read all of them after a later barrier.)
      m = wave_max_nan(m);
      if (lane == 0) tmax_s[wave] = m;
      lds_barrier();
      const float mx = nan_max_p(nan_max_p(tmax_s[0], tmax_s[1]), nan_max_p(tmax_s[2], tmax_s[3]));
      double dpart = 0.0;
      bool dexact = true;
      for (int s = tid; s < n; s += kST) {
        const float ev = exp_ref(fadd(p_s[s], -mx));
        p_s[s] = ev;
        dpart += (double)ev;
        dexact = dexact && (ev == 0.0f || (ev >= 0x1p-17f && ev <= 1.0f));
      }
      dpart = wave_sum_double(dpart);
      const bool wexact = __all(dexact);
      if (lane == 0) {
        lane_s[wave] = dpart;
        exact_s[wave] = wexact ? 1 : 0;
      }
      lds_barrier();
      float inverse;
      if (exact_s[0] & exact_s[1] & exact_s[2] & exact_s[3]) {
        inverse = (float)(1.0 / (((lane_s[0] + lane_s[1]) + lane_s[2]) + lane_s[3]));
      } else {  // (every thread takes the same branch)
        const int full = n & ~7;
        if (tid < 8) {
          double acc = 0.0;
          int s = tid;
          for (; s + 56 < full; s += 64) {
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = p_s[s + 8 * k];
#pragma unroll
            for (int k = 0; k < 8; ++k) acc = acc + (double)v[k];
          }
          for (; s < full; s += 8) acc = acc + (double)p_s[s];
          chain_s[tid] = acc;
        }
        lds_barrier();
        if (tid == 0) {
          double sum = ((chain_s[0] + chain_s[4]) + (chain_s[1] + chain_s[5])) + ((chain_s[2] + chain_s[6]) + (chain_s[3] + chain_s[7]));
          for (int s = full; s < n; ++s) sum = sum + (double)p_s[s];
          inv_s[0] = (float)(1.0 / sum);
        }
        lds_barrier();
        inverse = inv_s[0];
      }
      for (int s = tid; s < n; s += kST) p_s[s] = fmul(p_s[s], inverse);
      __builtin_amdgcn_s_waitcnt(0);  // this wave's V rows are in LDS
      lds_barrier();
      // Time-ordered value sums (AttentionAvx.cs:120-171): channel 2 lane + w
      // on wave w < 2, in blocks of 16 positions, the next block's LDS reads
      // issued before the current block is added. Meanwhile wave 2 gathers
      // this position's v row (rounded to F16; QwenDecoder.cs:195-203), which
      // the first query head of the pair writes to the cache, and which
      // gives the last term.
      float vacc = 0.0f;
      bool vok = true;
      if (wave < 2) {
        if (wave == 0) value_region<false>(lds, p_s, 0, nv, vacc);
        else value_region<true>(lds, p_s, 0, nv, vacc);
      } else if (wave == 2) {
        vok = gather_words(tqkv + (size_t)us * NQKV + QW + KVW + kh * HS, qkv_tag + 256, 0, 1, gen(l, 2), ~0u, a.error);
        if (vok) {
#pragma unroll
          for (int k = 0; k < 2; ++k) {
            const int c = lane + 64 * k;
            const _Float16 v16 = to_half(u2f((uint32_t)qkv_tag[256 + c]));
            vcur_s[c] = v16;
            if (uh % G == 0) gstore(const_cast<_Float16*>(vc) + (size_t)pos * HS + c, v16);
          }
        }
      }
      if (!all_waves(vok, ok_s)) return;
      if (wave < 2) {
        const int c = 2 * lane + wave;
        q_s[c] = fadd(vacc, mulh(p_s[pos], vcur_s[c]));
      }
      lds_barrier();
      if (tid < HS / 4) {
        const float4 v4 = *reinterpret_cast<const float4*>(q_s + 4 * tid);
        float d;
        const int packed = quantize4(v4.x, v4.y, v4.z, v4.w, &d);
        put_qword(tattq + (size_t)us * (QW / 4) + word_major(uh * (HS / 4) + tid, QW / 32), gen(l, 3), qside(tid & 7, d),
                  (uint32_t)packed);
      }
    }
    lds_barrier();

    // ---- o rows orow0 .. of sessions f0 .. + the residual
    if (Sg > 0) {
      OSlice sl;
      sl.load(lw.wo, lw.so, [&](int i) { return orow0 + i; });
      u64* stage = reinterpret_cast<u64*>(lds);
      if (!gather_rows<QW / 4>(tattq + (size_t)f0 * (QW / 4), stage, Sg, gen(l, 3), a.error, ok_s)) return;
      float* terms = reinterpret_cast<float*>(lds + OSlice::stage_bytes(Sg));
      sl.products(stage, Sg, terms);
      lds_barrier();
      if (rlane) {
        ares = fadd(OSlice::row_sum(terms, ri, rf - f0, Sg), xres);
        put_word(ta + (size_t)rf * W + rrow, gen(l, 4), f2u(ares));
      }
      lds_barrier();
    }

    // ---- ffn norm of session row ns
    if (ns >= 0) {
      NormWeights<W> nwt;
      nwt.load(lw.ffn_norm);
      u64* stage = reinterpret_cast<u64*>(lds);
      const bool ok = gather_words(ta + (size_t)ns * W, stage, wave * (W / 128) / 4, (wave + 1) * (W / 128) / 4,
                                   gen(l, 4), ~0u, a.error);
      if (!all_waves(ok, ok_s)) return;
      u64* dst = taq + (size_t)ns * (W / 4);
      norm_row<W>([&](int k) { return u2f((uint32_t)stage[k]); }, nwt, a.eps, red_s,
                  [&](int e, int packed, float d) {
                    put_qword(dst + word_major(e / 4, W / 32), gen(l, 5), qside((e / 4) & 7, d), (uint32_t)packed);
                  });
      lds_barrier();
    }

    // ---- gate/up pairs gp0 .. (one Q8_0 block of the ffn vector) of
    // sessions gf0 ..: SwiGLU, then the block's Q8_0 words
    if (w < NGU && Sgu > 0) {
      // Wave v: slots 16 v .. 16 v + 15 (gate rows of pairs 0-31, then up).
      GuTile sl;
      sl.load(lw.wgu, lw.sgu, [&](int r) {
        const int i = 16 * wave + r;
        const int p = gp0 + (i < kGuPairs ? i : i - kGuPairs), kind = i < kGuPairs ? 0 : 1;
        if (a.gu_map) return a.gu_map[2 * p + kind];
        // Tiles of `base` (the first `extra` of them base + 1) gate rows,
        // then the same count of up rows.
        const int base = a.gu_base, big = a.gu_extra * (base + 1);
        int r0, count;
        if (p < big) {
          r0 = p / (base + 1) * (base + 1);
          count = base + 1;
        } else {
          r0 = big + (p - big) / base * base;
          count = base;
        }
        return 2 * r0 + kind * count + (p - r0);
      });
      u64* stage = reinterpret_cast<u64*>(lds);
      if (!gather_rows<W / 4>(taq + (size_t)gf0 * (W / 4), stage, Sgu, gen(l, 5), a.error, ok_s)) return;
      u64* apack = reinterpret_cast<u64*>(lds + kGuPackOff);
      float* xs_s = reinterpret_cast<float*>(lds + kGuPackOff + (size_t)GuTile::B * GuTile::APS * 8);
      float* sum_s = xs_s + GuTile::B * 16;   // [2 kGuPairs][16]
      float* h_s = sum_s + 2 * kGuPairs * 16;  // [Sgu][kGuPairs]
      GuTile::pack(stage, Sgu, apack, xs_s);
      lds_barrier();
      {
        float acc[4];
        sl.sums(apack, xs_s, acc);
        const int r = lane & 15, q = lane >> 4;
        *reinterpret_cast<float4*>(sum_s + (16 * wave + r) * 16 + 4 * q) = make_float4(acc[0], acc[1], acc[2], acc[3]);
      }
      lds_barrier();
      for (int t = tid; t < kGuPairs * Sgu; t += kST) {
        const int i = t / Sgu, f = t - i * Sgu;
        // SwiGLU (Elementwise.cs:167-196).
        const float g = sum_s[i * 16 + f], u = sum_s[(kGuPairs + i) * 16 + f];
        h_s[f * kGuPairs + i] = fmul(fdiv(g, fadd(1.0f, exp_ref(-g))), u);
      }
      lds_barrier();
      // The block of each session: eight lanes, four values each (quantize4).
      if (tid < 8 * Sgu) {
        const int f = tid >> 3, j = tid & 7;
        const float4 v4 = *reinterpret_cast<const float4*>(h_s + f * kGuPairs + 4 * j);
        float d;
        const int packed = quantize4(v4.x, v4.y, v4.z, v4.w, &d);
        put_qword(thq + (size_t)(gf0 + f) * (FF / 4) + j * (FF / 32) + gp0 / 32, gen(l, 7), qside(j, d), (uint32_t)packed);
      }
      lds_barrier();
    }

    // ---- down rows orow0 .. of sessions f0 .. + the residual
    if (Sg > 0) {
      DownSlice sl;
      sl.load(lw.wd, lw.sd, [&](int i) { return orow0 + i; });
      u64* stage = reinterpret_cast<u64*>(lds);
      if (!gather_rows<FF / 4>(thq + (size_t)f0 * (FF / 4), stage, Sg, gen(l, 7), a.error, ok_s)) return;
      float* terms = reinterpret_cast<float*>(lds + DownSlice::stage_bytes(Sg));
      sl.products(stage, Sg, terms);
      lds_barrier();
      if (rlane) {
        xres = fadd(DownSlice::row_sum(terms, ri, rf - f0, Sg), ares);
        put_word(tx + (size_t)rf * W + rrow, gen(l, 8), f2u(xres));
      }
      lds_barrier();
    }
  }

  // ---- output norm of session row ns, as Q8_0 rows for the lm_head
  if (ns >= 0) {
    NormWeights<W> nwt;
    nwt.load(a.output_norm);
    u64* stage = reinterpret_cast<u64*>(lds);
    const bool ok = gather_words(a.tx + (size_t)(L - 1) * LX + (size_t)ns * W, stage, wave * (W / 128) / 4, (wave + 1) * (W / 128) / 4,
                                 gen(L - 1, 8), ~0u, a.error);
    if (!all_waves(ok, ok_s)) return;
    int8_t* xq = a.xq_out + (size_t)ns * W;
    float* xs = a.xs_out + (size_t)ns * (W / 32);
    norm_row<W>([&](int k) { return u2f((uint32_t)stage[k]); }, nwt, a.eps, red_s, [&](int e, int packed, float d) {
      *reinterpret_cast<int*>(xq + e) = packed;
      if ((tid & 7) == 0) xs[e >> 5] = d;
    });
    // Every workgroup has read the epoch (each published its last down
    // rows, which this gather waited for): the next launch's generations.
    if (ns == 0 && tid == 0) *a.epoch = *a.epoch + 1;
  }
}

template <int W, int H, int KVH, int FF>
hipError_t launch_shape(const SessionStepArgs& a, hipStream_t s) {
  static const hipError_t raised = hipFuncSetAttribute(reinterpret_cast<const void*>(session_step_kernel<W, H, KVH, FF>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, kSLds);
  if (raised != hipSuccess) return raised;
  session_step_kernel<W, H, KVH, FF><<<kSG, kST, kSLds, s>>>(a);
  return hipGetLastError();
}

template <int W, int H, int KVH, int FF>
int blocks_per_cu() {
  int b = 0;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(session_step_kernel<W, H, KVH, FF>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, kSLds) != hipSuccess)
    return 0;
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, session_step_kernel<W, H, KVH, FF>, kST, kSLds) == hipSuccess
             ? b
             : 0;
}

}  // namespace

// Shapes with an instantiation: Qwen3-0.6B and the reduced Qwen3-shaped
// decoder of the quick parity runs.
bool session_step_supported(int width, int heads, int kv_heads, int head_size, int ffn) {
  if (head_size != 128) return false;
  return (width == 1024 && heads == 16 && kv_heads == 8 && ffn == 3072) ||
         (width == 512 && heads == 4 && kv_heads == 2 && ffn == 1024);
}

int session_step_positions() { return kSPositions; }
int session_step_groups() { return kSG; }

int session_step_blocks_per_cu(int width) {
  return width == 1024 ? blocks_per_cu<1024, 16, 8, 3072>() : blocks_per_cu<512, 4, 2, 1024>();
}

hipError_t launch_session_step(const SessionStepArgs& a, hipStream_t s) {
  if (!session_step_supported(a.width, a.heads, a.kv_heads, a.head_size, a.ffn)) return hipErrorInvalidValue;
  if (a.S < 1 || a.S > 16 || a.S * a.heads > kSG || a.max_positions < 1 || a.max_positions > kSPositions || a.layers < 1)
    return hipErrorInvalidValue;
  if (a.width == 1024) return launch_shape<1024, 16, 8, 3072>(a, s);
  return launch_shape<512, 4, 2, 1024>(a, s);
}

}  // namespace fah
