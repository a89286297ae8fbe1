// FP32 kernels of the encoder-side seam and the original-precision decoder
// projections: linear projections y = x W^T + b (optionally ReLU), and
// non-causal multi-head attention.
//
// These paths have no bit-exact counterpart: the reference's CPU kernels
// already differ in float order between paths (TensorMath.cs:79-200: packed
// AVX/FMA for 16+ frames, FloatRows4Avx below 4, a generic row loop), and
// its device backend checks against a tolerance (2e-4 relative for linear
// projections, 5e-5 for attention, tools/FunAsrNet.Benchmarks
// FloatGpuChecks.cs, AttentionGpuChecks.cs). What is exact here is what the
// reference's checks require to be exact: a projection gives the same bits
// alone, in a group, or as either half of a ReLU chain (one kernel, one
// order per shape).
#include "fah_device.h"
#include "fah_internal.h"

#include <algorithm>
#include <cstdint>

namespace fah {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

// ---- GEMM on fp32 MFMA --------------------------------------------------------
// out[f][n] = sum_k x[f][k] * w[n][k] (+ bias[n]) (ReLU), any M (frames), N,
// K with K % 4 == 0 and 16-byte aligned rows. Four waves in a 2 x 2 grid,
// each a (16 BI) x (16 BJ) tile of v_mfma_f32_16x16x4f32 blocks; workgroup
// tile (32 BI) x (32 BJ); K in tiles of GK staged in two LDS buffers as
// row-major [row][GK + 4] (16-byte loads and stores; the next tile's global
// loads sit in registers while the current one is multiplied, then go to
// the other buffer, one barrier per tile). Lane layout of 16x16x4: A[i][k]
// from lane i + 16k, B[k][j] from lane j + 16k, D[4q + r][j] in lane j + 16q
// (r < 4). In substep s of a K tile, lane group q multiplies k =
// (GK / 4) q + s, so each lane reads its GK / 4 values of a row as 16-byte
// LDS reads. One order per shape: the same bits whichever entry point runs it.
#ifndef FAH_GK
#define FAH_GK 64
#endif
constexpr int kGK = FAH_GK;

template <int BI, int BJ, bool RELU>
__global__ __launch_bounds__(256) void f32_gemm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                       const float* __restrict__ bias, float* __restrict__ out, int M,
                                                       int N, int K) {
  constexpr int TM = 32 * BI, TN = 32 * BJ;              // workgroup tile
  constexpr int ROW = kGK + 4, KQ = kGK / 4;              // LDS row (floats); k values per lane group
  constexpr int PER_ROW = kGK / 4, ROWS = 256 / PER_ROW;  // 16-byte loads per row; rows per pass
  constexpr int LA = TM / ROWS, LB = TN / ROWS;           // 16-byte loads per thread and operand
  static_assert(LA >= 1 && LB >= 1 && TM % ROWS == 0 && TN % ROWS == 0, "whole load passes");
  __shared__ __attribute__((aligned(16))) float a_s[2][TM * ROW];
  __shared__ __attribute__((aligned(16))) float b_s[2][TN * ROW];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int f0 = blockIdx.y * TM, n0 = blockIdx.x * TN;
  const int wm = (wave >> 1) * 16 * BI, wn = (wave & 1) * 16 * BJ;
  const int li = lane & 15, lq = lane >> 4;
  floatx4 acc[BI][BJ];
#pragma unroll
  for (int i = 0; i < BI; ++i)
#pragma unroll
    for (int j = 0; j < BJ; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  // Global loads: thread t takes row t / PER_ROW (+ ROWS per further load),
  // the 16 bytes at k = 4 (t % PER_ROW) of the tile; rows past the edge and
  // k past K read as zero.
  const int lr = tid / PER_ROW, lc = 4 * (tid % PER_ROW);
  float4 ra[LA], rb[LB];
  auto fetch = [&](int k0) {
    const int k = k0 + lc;
#pragma unroll
    for (int u = 0; u < LA; ++u) {
      const int f = f0 + lr + ROWS * u;
      ra[u] = (f < M && k < K) ? *reinterpret_cast<const float4*>(x + (size_t)f * K + k) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < LB; ++u) {
      const int n = n0 + lr + ROWS * u;
      rb[u] = (n < N && k < K) ? *reinterpret_cast<const float4*>(w + (size_t)n * K + k) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int u = 0; u < LA; ++u) *reinterpret_cast<float4*>(&a_s[buf][(lr + ROWS * u) * ROW + lc]) = ra[u];
#pragma unroll
    for (int u = 0; u < LB; ++u) *reinterpret_cast<float4*>(&b_s[buf][(lr + ROWS * u) * ROW + lc]) = rb[u];
  };
  fetch(0);
  stage(0);
  __syncthreads();
  int buf = 0;
  for (int k0 = 0; k0 < K; k0 += kGK) {
    const bool more = k0 + kGK < K;
    if (more) fetch(k0 + kGK);
#pragma unroll
    for (int h = 0; h < KQ / 4; ++h) {
      float4 av[BI], bv[BJ];
#pragma unroll
      for (int i = 0; i < BI; ++i)
        av[i] = *reinterpret_cast<const float4*>(&a_s[buf][(wm + 16 * i + li) * ROW + KQ * lq + 4 * h]);
#pragma unroll
      for (int j = 0; j < BJ; ++j)
        bv[j] = *reinterpret_cast<const float4*>(&b_s[buf][(wn + 16 * j + li) * ROW + KQ * lq + 4 * h]);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int i = 0; i < BI; ++i)
#pragma unroll
          for (int j = 0; j < BJ; ++j) {
            const float a = e == 0 ? av[i].x : e == 1 ? av[i].y : e == 2 ? av[i].z : av[i].w;
            const float b = e == 0 ? bv[j].x : e == 1 ? bv[j].y : e == 2 ? bv[j].z : bv[j].w;
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[i][j], 0, 0, 0);
          }
    }
    if (more) {
      stage(buf ^ 1);
      __syncthreads();
      buf ^= 1;
    }
  }
#pragma unroll
  for (int j = 0; j < BJ; ++j) {
    const int n = n0 + wn + 16 * j + li;
    if (n >= N) continue;
    const float b = bias ? bias[n] : 0.0f;
#pragma unroll
    for (int i = 0; i < BI; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int f = f0 + wm + 16 * i + 4 * lq + r;
        if (f < M) {
          float v = acc[i][j][r] + b;
          if (RELU) v = v < 0.0f ? 0.0f : v;  // (-0 and NaN pass, as the reference's `v < 0 ? 0 : v`)
          out[(size_t)f * N + n] = v;
        }
      }
  }
}

// The same product for grids of at most one workgroup per CU: each of the
// four waves covers the whole 32 x 64 tile (2 x 4 blocks, eight
// accumulators in flight) over its quarter of every K tile (lane group q of
// wave w takes k = 16 w + 4 q .. + 3), and the four partial tiles are added
// in wave order in LDS at the end.
template <bool RELU>
__global__ __launch_bounds__(256) void f32_gemm_wavek_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                             const float* __restrict__ bias, float* __restrict__ out,
                                                             int M, int N, int K) {
  constexpr int GK = 64, TM = 32, TN = 64, ROW = GK + 4;
  constexpr int PER_ROW = GK / 4, ROWS = 256 / PER_ROW, LA = TM / ROWS, LB = TN / ROWS;
  __shared__ __attribute__((aligned(16))) float a_s[2][TM * ROW];
  __shared__ __attribute__((aligned(16))) float b_s[2][TN * ROW];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int f0 = blockIdx.y * TM, n0 = blockIdx.x * TN;
  const int li = lane & 15, lq = lane >> 4;
  floatx4 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  const int lr = tid / PER_ROW, lc = 4 * (tid % PER_ROW);
  float4 ra[LA], rb[LB];
  auto fetch = [&](int k0) {
    const int k = k0 + lc;
#pragma unroll
    for (int u = 0; u < LA; ++u) {
      const int f = f0 + lr + ROWS * u;
      ra[u] = (f < M && k < K) ? *reinterpret_cast<const float4*>(x + (size_t)f * K + k) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < LB; ++u) {
      const int n = n0 + lr + ROWS * u;
      rb[u] = (n < N && k < K) ? *reinterpret_cast<const float4*>(w + (size_t)n * K + k) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int u = 0; u < LA; ++u) *reinterpret_cast<float4*>(&a_s[buf][(lr + ROWS * u) * ROW + lc]) = ra[u];
#pragma unroll
    for (int u = 0; u < LB; ++u) *reinterpret_cast<float4*>(&b_s[buf][(lr + ROWS * u) * ROW + lc]) = rb[u];
  };
  fetch(0);
  stage(0);
  __syncthreads();
  int buf = 0;
  const int kl = 16 * wave + 4 * lq;
  for (int k0 = 0; k0 < K; k0 += GK) {
    const bool more = k0 + GK < K;
    if (more) fetch(k0 + GK);
    float4 av[2], bv[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) av[i] = *reinterpret_cast<const float4*>(&a_s[buf][(16 * i + li) * ROW + kl]);
#pragma unroll
    for (int j = 0; j < 4; ++j) bv[j] = *reinterpret_cast<const float4*>(&b_s[buf][(16 * j + li) * ROW + kl]);
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float a = e == 0 ? av[i].x : e == 1 ? av[i].y : e == 2 ? av[i].z : av[i].w;
          const float b = e == 0 ? bv[j].x : e == 1 ? bv[j].y : e == 2 ? bv[j].z : bv[j].w;
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[i][j], 0, 0, 0);
        }
    if (more) {
      stage(buf ^ 1);
      __syncthreads();
      buf ^= 1;
    }
  }
  // Partial tiles into LDS (the staging buffers, free once every wave is
  // past its last reads): part[w][f][n], then summed in wave order.
  __syncthreads();
  float* part = &a_s[0][0];
  static_assert(4 * TM * TN <= 2 * TM * ROW + 2 * TN * ROW, "partials fit the staging buffers");
  float* part_b = &b_s[0][0];
  auto slot = [&](int wv, int f, int n) -> float& {
    const int e = (wv * TM + f) * TN + n;
    return e < 2 * TM * ROW ? part[e] : part_b[e - 2 * TM * ROW];
  };
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) slot(wave, 16 * i + 4 * lq + r, 16 * j + li) = acc[i][j][r];
  __syncthreads();
  for (int e = tid; e < TM * TN; e += 256) {
    const int f = e / TN, n = e % TN;
    if (f0 + f >= M || n0 + n >= N) continue;
    float v = ((slot(0, f, n) + slot(1, f, n)) + slot(2, f, n)) + slot(3, f, n);
    v = v + (bias ? bias[n0 + n] : 0.0f);
    if (RELU) v = v < 0.0f ? 0.0f : v;
    out[(size_t)(f0 + f) * N + n0 + n] = v;
  }
}

// Any K and alignment: 64 x 64 tiles, K in steps of 32 staged in LDS one
// float per thread and row, four waves of 2 x 2 v_mfma_f32_16x16x4f32 blocks.
constexpr int kGT = 64, kGA = 32, kGPad = kGA + 1;

template <bool RELU>
__global__ __launch_bounds__(256) void f32_gemm_any_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                           const float* __restrict__ bias, float* __restrict__ out,
                                                           int M, int N, int K) {
  __shared__ float a_s[kGT][kGPad];  // frames x k
  __shared__ float b_s[kGT][kGPad];  // rows x k
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int f0 = blockIdx.y * kGT, n0 = blockIdx.x * kGT;
  const int fm = (wave >> 1) * 32, rn = (wave & 1) * 32;
  floatx4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  // Staging: thread t loads rows t / 32 + 8 s (s < 8), column t % 32.
  const int lr = tid >> 5, lc = tid & 31;
  for (int k0 = 0; k0 < K; k0 += kGA) {
    const int k = k0 + lc;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int r = lr + 8 * s;
      const int f = f0 + r, n = n0 + r;
      a_s[r][lc] = (f < M && k < K) ? x[(size_t)f * K + k] : 0.0f;
      b_s[r][lc] = (n < N && k < K) ? w[(size_t)n * K + k] : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < kGA; ks += 4) {
      const int kk = ks + (lane >> 4), ii = lane & 15;
      const float a0 = a_s[fm + ii][kk], a1 = a_s[fm + 16 + ii][kk];
      const float b0 = b_s[rn + ii][kk], b1 = b_s[rn + 16 + ii][kk];
      acc[0][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b0, acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b1, acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b0, acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b1, acc[1][1], 0, 0, 0);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + rn + 16 * j + (lane & 15);
      if (n >= N) continue;
      const float b = bias ? bias[n] : 0.0f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int f = f0 + fm + 16 * i + 4 * (lane >> 4) + r;
        if (f < M) {
          float v = acc[i][j][r] + b;
          if (RELU) v = v < 0.0f ? 0.0f : v;
          out[(size_t)f * N + n] = v;
        }
      }
    }
}

// ---- GEMV (few frames, weight-bandwidth bound) ------------------------------
// Each wave takes RW consecutive weight rows at a time (their loads all in
// flight together), every lane a strided share of each row (four floats per
// lane per step when rows are 16-byte aligned), the frames' inputs in LDS,
// then a wave reduction per row and frame.
constexpr int kVMaxFrames = 4, kVMaxK = 4096;

template <bool RELU, bool VEC, int kVRows>
__global__ __launch_bounds__(256) void f32_gemv_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                       const float* __restrict__ bias, float* __restrict__ out, int M,
                                                       int N, int K) {
  __shared__ __attribute__((aligned(16))) float x_s[kVMaxFrames * kVMaxK];
  const int tid = threadIdx.x, lane = tid & 63;
  for (int i = tid; i < M * K; i += 256) x_s[i] = x[i];
  __syncthreads();
  const int waves = gridDim.x * 4;
  for (int n0 = (blockIdx.x * 4 + (tid >> 6)) * kVRows; n0 < N; n0 += waves * kVRows) {
    float acc[kVRows][kVMaxFrames];
#pragma unroll
    for (int r = 0; r < kVRows; ++r)
#pragma unroll
      for (int f = 0; f < kVMaxFrames; ++f) acc[r][f] = 0.0f;
    // Rows past N re-read row N - 1 (never stored).
    const float* rows[kVRows];
#pragma unroll
    for (int r = 0; r < kVRows; ++r) rows[r] = w + (size_t)min(n0 + r, N - 1) * K;
    if (VEC) {
      for (int k = 4 * lane; k < K; k += 256) {
        float4 v[kVRows];
#pragma unroll
        for (int r = 0; r < kVRows; ++r) v[r] = *reinterpret_cast<const float4*>(rows[r] + k);
#pragma unroll
        for (int f = 0; f < kVMaxFrames; ++f)
          if (f < M) {
            const float4 u = *reinterpret_cast<const float4*>(x_s + f * K + k);
#pragma unroll
            for (int r = 0; r < kVRows; ++r) {
              acc[r][f] = __builtin_fmaf(v[r].x, u.x, acc[r][f]);
              acc[r][f] = __builtin_fmaf(v[r].y, u.y, acc[r][f]);
              acc[r][f] = __builtin_fmaf(v[r].z, u.z, acc[r][f]);
              acc[r][f] = __builtin_fmaf(v[r].w, u.w, acc[r][f]);
            }
          }
      }
    } else {
      for (int k = lane; k < K; k += 64) {
        float v[kVRows];
#pragma unroll
        for (int r = 0; r < kVRows; ++r) v[r] = rows[r][k];
#pragma unroll
        for (int f = 0; f < kVMaxFrames; ++f)
          if (f < M) {
            const float u = x_s[f * K + k];
#pragma unroll
            for (int r = 0; r < kVRows; ++r) acc[r][f] = __builtin_fmaf(v[r], u, acc[r][f]);
          }
      }
    }
#pragma unroll
    for (int r = 0; r < kVRows; ++r) {
      const int n = n0 + r;
#pragma unroll
      for (int f = 0; f < kVMaxFrames; ++f) {
        if (f >= M) break;
        float s = acc[r][f];
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m, 64);
        if (lane == 0 && n < N) {
          float v = s + (bias ? bias[n] : 0.0f);
          if (RELU) v = v < 0.0f ? 0.0f : v;
          out[(size_t)f * N + n] = v;
        }
      }
    }
  }
}

// ---- Non-causal multi-head attention ------------------------------------------
// One workgroup per (head, 16 query rows); keys in blocks of 32 staged in
// LDS with their values; online softmax (running maximum, rescaled sums),
// outputs in registers (thread t: rows 4 (t / 64) .. +3, channels t % 64,
// t % 64 + 64, ...).
constexpr int kAQ = 16, kAK = 32, kAMaxS = 256;

__global__ __launch_bounds__(256) void f32_attention_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                            const float* __restrict__ v, float* __restrict__ out,
                                                            int frames, int width, int S, float divisor) {
  __shared__ float q_s[kAQ][kAMaxS + 1];
  __shared__ float k_s[kAK][kAMaxS + 1];
  __shared__ float v_s[kAK][kAMaxS];
  __shared__ float p_s[kAQ][kAK + 1];
  __shared__ float scale_s[kAQ];
  const int tid = threadIdx.x, head = blockIdx.x, t0 = blockIdx.y * kAQ;
  const int hoff = head * S;
  for (int i = tid; i < kAQ * S; i += 256) {
    const int r = i / S, c = i - r * S;
    q_s[r][c] = t0 + r < frames ? q[(size_t)(t0 + r) * width + hoff + c] : 0.0f;
  }
  constexpr int kCh = kAMaxS / 64;  // channel slots per thread
  const int orow = 4 * (tid >> 6), oc = tid & 63;
  float o[4][kCh];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int j = 0; j < kCh; ++j) o[r][j] = 0.0f;
  // Per query row (threads 0..15 keep them): running maximum and sum.
  float run_max = -__builtin_inff(), run_sum = 0.0f;
  for (int s0 = 0; s0 < frames; s0 += kAK) {
    __syncthreads();
    for (int i = tid; i < kAK * S; i += 256) {
      const int r = i / S, c = i - r * S;
      const bool in = s0 + r < frames;
      k_s[r][c] = in ? k[(size_t)(s0 + r) * width + hoff + c] : 0.0f;
      v_s[r][c] = in ? v[(size_t)(s0 + r) * width + hoff + c] : 0.0f;
    }
    __syncthreads();
    // Scores: thread t -> (query row t / 16, keys t % 16 and t % 16 + 16).
    {
      const int qr = tid >> 4, kc = tid & 15;
      float d0 = 0.0f, d1 = 0.0f;
      for (int c = 0; c < S; ++c) {
        const float qv = q_s[qr][c];
        d0 = __builtin_fmaf(qv, k_s[kc][c], d0);
        d1 = __builtin_fmaf(qv, k_s[kc + 16][c], d1);
      }
      p_s[qr][kc] = s0 + kc < frames ? d0 / divisor : -__builtin_inff();
      p_s[qr][kc + 16] = s0 + kc + 16 < frames ? d1 / divisor : -__builtin_inff();
    }
    __syncthreads();
    // Softmax update per query row (16 threads).
    if (tid < kAQ) {
      float m = run_max;
      for (int j = 0; j < kAK; ++j) m = fmaxf(m, p_s[tid][j]);
      // The earlier blocks' sums rescaled to the new maximum (none before
      // the first block).
      const float scale = run_max == -__builtin_inff() ? 0.0f : expf(run_max - m);
      float sum = 0.0f;
      for (int j = 0; j < kAK; ++j) {
        const float e = p_s[tid][j] == -__builtin_inff() ? 0.0f : expf(p_s[tid][j] - m);
        p_s[tid][j] = e;
        sum += e;
      }
      run_sum = run_sum * scale + sum;
      scale_s[tid] = scale;
      run_max = m;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float sc = scale_s[orow + r];
#pragma unroll
      for (int j = 0; j < kCh; ++j) {
        const int c = oc + 64 * j;
        if (c < S) {
          float acc = o[r][j] * sc;
          for (int kk = 0; kk < kAK; ++kk) acc = __builtin_fmaf(p_s[orow + r][kk], v_s[kk][c], acc);
          o[r][j] = acc;
        }
      }
    }
  }
  __syncthreads();
  if (tid < kAQ) scale_s[tid] = 1.0f / run_sum;
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = t0 + orow + r;
    if (t >= frames) continue;
    const float inv = scale_s[orow + r];
#pragma unroll
    for (int j = 0; j < kCh; ++j) {
      const int c = oc + 64 * j;
      if (c < S) out[(size_t)t * width + hoff + c] = o[r][j] * inv;
    }
  }
}

// ---- Non-causal multi-head attention on fp32 MFMA (head size HS, 64 or 128) ----
// One workgroup per (head, 16 query rows); wave w takes key blocks (16 keys)
// w, w + 4, ... and keeps its own running maximum, sum and outputs; the four
// partial results are merged in LDS at the end. Per key block the scores
// come transposed, S^T = K Q^T (16 keys x 16 queries, HS / 4 MFMAs with key
// rows and query rows both read as contiguous 16-byte pieces: in substep t
// lane group g multiplies channel g HS/4 + t), so that lane (query j, group
// g) holds the probabilities of keys 4g .. 4g + 3 for query j, which is
// exactly the A operand of P V when substep u takes key 4g + u.
template <int HS>
__global__ __launch_bounds__(256) void f32_attention_mfma_kernel(const float* __restrict__ q,
                                                                 const float* __restrict__ k,
                                                                 const float* __restrict__ v, float* __restrict__ out,
                                                                 int frames, int width, float divisor) {
  constexpr int CB = HS / 16, KQ = HS / 4;  // channel blocks; channels per lane group
  __shared__ __attribute__((aligned(16))) float o_s[4][16][HS];
  __shared__ float m_s[4][16], l_s[4][16];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 15, g = lane >> 4;
  const int head = blockIdx.x, t0 = blockIdx.y * 16, hoff = head * HS;
  // This lane's query channels g KQ .. g KQ + KQ - 1 of query t0 + j (zero past the end).
  float qv[KQ];
  {
    const bool in = t0 + j < frames;
    const float* src = q + (size_t)(t0 + j) * width + hoff + g * KQ;
#pragma unroll
    for (int c = 0; c < KQ; c += 4) {
      const float4 x4 = in ? *reinterpret_cast<const float4*>(src + c) : make_float4(0.f, 0.f, 0.f, 0.f);
      qv[c] = x4.x;
      qv[c + 1] = x4.y;
      qv[c + 2] = x4.z;
      qv[c + 3] = x4.w;
    }
  }
  floatx4 o[CB];
#pragma unroll
  for (int c = 0; c < CB; ++c) o[c] = floatx4{0.f, 0.f, 0.f, 0.f};
  float run_m = -__builtin_inff(), run_l = 0.0f;  // of query j
  const int blocks = (frames + 15) / 16;
  float kv[KQ];
  auto load_k = [&](int kb) {
    const int key = kb * 16 + j;
    const bool in = key < frames;
    const float* src = k + (size_t)key * width + hoff + g * KQ;
#pragma unroll
    for (int c = 0; c < KQ; c += 4) {
      const float4 x4 = in ? *reinterpret_cast<const float4*>(src + c) : make_float4(0.f, 0.f, 0.f, 0.f);
      kv[c] = x4.x;
      kv[c + 1] = x4.y;
      kv[c + 2] = x4.z;
      kv[c + 3] = x4.w;
    }
  };
  if (wave < blocks) load_k(wave);
  for (int kb = wave; kb < blocks; kb += 4) {
    // Scores S^T[key 4g + r][query j].
    floatx4 st = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < KQ; ++t) st = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[t], qv[t], st, 0, 0, 0);
    // V values of keys 4g + u, channel 16c + j (zero past the end), and the
    // next block's keys, in flight during the softmax.
    float vv[CB][4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int key = kb * 16 + 4 * g + u;
      const bool in = key < frames;
      const float* src = v + (size_t)key * width + hoff + j;
#pragma unroll
      for (int c = 0; c < CB; ++c) vv[c][u] = in ? src[16 * c] : 0.0f;
    }
    if (kb + 4 < blocks) load_k(kb + 4);
    float sc[4], bm = -__builtin_inff();
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int key = kb * 16 + 4 * g + r;
      sc[r] = key < frames ? st[r] / divisor : -__builtin_inff();
      bm = fmaxf(bm, sc[r]);
    }
    bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
    bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
    const float nm = fmaxf(run_m, bm);
    float p[4], bl = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p[r] = sc[r] == -__builtin_inff() ? 0.0f : expf(sc[r] - nm);
      bl += p[r];
    }
    bl += __shfl_xor(bl, 16, 64);
    bl += __shfl_xor(bl, 32, 64);
    const float alpha = run_m == -__builtin_inff() ? 0.0f : expf(run_m - nm);
    run_l = run_l * alpha + bl;
    run_m = nm;
    // Output rows are queries 4g + r: their rescale factors from lanes 4g + r.
    float ar[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) ar[r] = __shfl(alpha, 4 * g + r, 64);
#pragma unroll
    for (int c = 0; c < CB; ++c) {
#pragma unroll
      for (int r = 0; r < 4; ++r) o[c][r] *= ar[r];
#pragma unroll
      for (int u = 0; u < 4; ++u) o[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[u], vv[c][u], o[c], 0, 0, 0);
    }
  }
  // Merge the four waves' partials: out = sum_w e^(m_w - M) O_w / sum_w e^(m_w - M) l_w.
  if (g == 0) {
    m_s[wave][j] = run_m;
    l_s[wave][j] = run_l;
  }
#pragma unroll
  for (int c = 0; c < CB; ++c)
#pragma unroll
    for (int r = 0; r < 4; ++r) o_s[wave][4 * g + r][16 * c + j] = o[c][r];
  __syncthreads();
  for (int e = tid; e < 16 * HS; e += 256) {
    const int row = e / HS, ch = e % HS;
    if (t0 + row >= frames) continue;
    float mx = -__builtin_inff();
#pragma unroll
    for (int w2 = 0; w2 < 4; ++w2) mx = fmaxf(mx, m_s[w2][row]);
    float num = 0.0f, den = 0.0f;
#pragma unroll
    for (int w2 = 0; w2 < 4; ++w2) {
      const float f = m_s[w2][row] == -__builtin_inff() ? 0.0f : expf(m_s[w2][row] - mx);
      num += f * o_s[w2][row][ch];
      den += f * l_s[w2][row];
    }
    out[(size_t)(t0 + row) * width + hoff + ch] = num / den;
  }
}

}  // namespace

bool f32_attention_supported(int frames, int width, int heads) {
  return frames >= 1 && frames <= 4096 && heads >= 1 && heads <= 65535 && width >= heads && width % heads == 0 &&
         width / heads <= kAMaxS;
}

hipError_t launch_f32_linear(const float* x, const float* w, const float* bias, float* out, int M, int N, int K,
                             bool relu, hipStream_t s) {
  if (M < 1 || N < 1 || K < 1) return hipErrorInvalidValue;
  if (M <= kVMaxFrames && K <= kVMaxK) {
    // Four rows per wave when that still leaves 512+ workgroups, else one.
    const bool wide = N >= 4 * 4 * 512;
    const int per = wide ? 16 : 4;
    const int groups = std::min((N + per - 1) / per, 2048);
    const bool vec = K % 4 == 0;
#define FAH_GEMV(R, V, RW) f32_gemv_kernel<R, V, RW><<<groups, 256, 0, s>>>(x, w, bias, out, M, N, K)
    if (wide) {
      if (relu) vec ? FAH_GEMV(true, true, 4) : FAH_GEMV(true, false, 4);
      else vec ? FAH_GEMV(false, true, 4) : FAH_GEMV(false, false, 4);
    } else {
      if (relu) vec ? FAH_GEMV(true, true, 1) : FAH_GEMV(true, false, 1);
      else vec ? FAH_GEMV(false, true, 1) : FAH_GEMV(false, false, 1);
    }
#undef FAH_GEMV
    return hipGetLastError();
  }
  const bool aligned = K % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0;
  if (!aligned) {
    const dim3 grid((N + kGT - 1) / kGT, (M + kGT - 1) / kGT);
    if (relu) f32_gemm_any_kernel<true><<<grid, 256, 0, s>>>(x, w, bias, out, M, N, K);
    else f32_gemm_any_kernel<false><<<grid, 256, 0, s>>>(x, w, bias, out, M, N, K);
    return hipGetLastError();
  }
  // The tile whose grid loads the CUs most evenly: rounds of 256
  // workgroups times the tile's area, the larger tile on a tie; a grid of at
  // most one 32 x 64 workgroup per CU splits K over its waves.
  const int big = ((M + 63) / 64) * ((N + 63) / 64), small = ((M + 31) / 32) * ((N + 63) / 64);
  const int64_t big_cost = (int64_t)((big + 255) / 256) * 2, small_cost = (small + 255) / 256;
  if (big_cost <= small_cost) {
    const dim3 grid((N + 63) / 64, (M + 63) / 64);
    if (relu) f32_gemm_kernel<2, 2, true><<<grid, 256, 0, s>>>(x, w, bias, out, M, N, K);
    else f32_gemm_kernel<2, 2, false><<<grid, 256, 0, s>>>(x, w, bias, out, M, N, K);
  } else {
    const dim3 grid((N + 63) / 64, (M + 31) / 32);
    if (small <= 256 && K >= 256) {
      if (relu) f32_gemm_wavek_kernel<true><<<grid, 256, 0, s>>>(x, w, bias, out, M, N, K);
      else f32_gemm_wavek_kernel<false><<<grid, 256, 0, s>>>(x, w, bias, out, M, N, K);
    } else {
      if (relu) f32_gemm_kernel<1, 2, true><<<grid, 256, 0, s>>>(x, w, bias, out, M, N, K);
      else f32_gemm_kernel<1, 2, false><<<grid, 256, 0, s>>>(x, w, bias, out, M, N, K);
    }
  }
  return hipGetLastError();
}

hipError_t launch_f32_attention(const float* q, const float* k, const float* v, float* out, int frames, int width,
                                int heads, hipStream_t s) {
  if (!f32_attention_supported(frames, width, heads)) return hipErrorInvalidValue;
  const int S = width / heads;
  const float divisor = sqrtf((float)S);
  const bool aligned = width % 4 == 0 && (reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k)) % 16 == 0;
  if (aligned && (S == 64 || S == 128)) {
    const dim3 grid(heads, (frames + 15) / 16);
    if (S == 128) f32_attention_mfma_kernel<128><<<grid, 256, 0, s>>>(q, k, v, out, frames, width, divisor);
    else f32_attention_mfma_kernel<64><<<grid, 256, 0, s>>>(q, k, v, out, frames, width, divisor);
    return hipGetLastError();
  }
  const dim3 grid(heads, (frames + kAQ - 1) / kAQ);
  f32_attention_kernel<<<grid, 256, 0, s>>>(q, k, v, out, frames, width, S, divisor);
  return hipGetLastError();
}

}  // namespace fah
