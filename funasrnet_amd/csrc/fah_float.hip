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

namespace fah {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

// ---- GEMM on fp32 MFMA --------------------------------------------------------
// out[f][n] = sum_k x[f][k] * w[n][k] (+ bias[n]) (ReLU), any M (frames), N,
// K. Workgroup tile 64 frames x 64 rows, K in steps of 32 staged in LDS
// (zero-padded past the edges); four waves, each a 32 x 32 quarter as 2 x 2
// v_mfma_f32_16x16x4f32 blocks. Lane layout of 16x16x4: A[i][k] from lane
// i + 16k, B[k][j] from lane j + 16k, D[4q + r][j] in lane j + 16q, r < 4.
constexpr int kGT = 64, kGK = 32, kGPad = kGK + 1;

template <bool RELU>
__global__ __launch_bounds__(256) void f32_gemm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                       const float* __restrict__ bias, float* __restrict__ out, int M,
                                                       int N, int K) {
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
  for (int k0 = 0; k0 < K; k0 += kGK) {
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
    for (int ks = 0; ks < kGK; ks += 4) {
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
          if (RELU) v = v < 0.0f ? 0.0f : v;  // (-0 and NaN pass, as the reference's `v < 0 ? 0 : v`)
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
  const dim3 grid((N + kGT - 1) / kGT, (M + kGT - 1) / kGT);
  if (relu) f32_gemm_kernel<true><<<grid, 256, 0, s>>>(x, w, bias, out, M, N, K);
  else f32_gemm_kernel<false><<<grid, 256, 0, s>>>(x, w, bias, out, M, N, K);
  return hipGetLastError();
}

hipError_t launch_f32_attention(const float* q, const float* k, const float* v, float* out, int frames, int width,
                                int heads, hipStream_t s) {
  if (!f32_attention_supported(frames, width, heads)) return hipErrorInvalidValue;
  const int S = width / heads;
  const float divisor = sqrtf((float)S);
  const dim3 grid(heads, (frames + kAQ - 1) / kAQ);
  f32_attention_kernel<<<grid, 256, 0, s>>>(q, k, v, out, frames, width, S, divisor);
  return hipGetLastError();
}

}  // namespace fah
