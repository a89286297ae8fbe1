// gfx950 kernels for the Qwen3 Q8_0 decoder step.
//
// Q8_0 GEMV (q8_gemv_kernel): one workgroup owns `group_rows` consecutive
// weight rows and all of K. Its 256 lanes stream the rows' 32-byte blocks
// with two 128-bit loads each (one lane = one (row, block) pair, contiguous
// across lanes), take the exact int32 block dot with v_dot4_i32_i8 against
// the quantised activation held in LDS, scale it as ((float)dot * w_scale) *
// x_scale, and park the product in LDS. One lane per row then adds the
// products in block order from 0f -- the float order of the reference's x64
// kernels (src/FunAsrNet/TensorMath.QuantizedRowsAvx.cs:27-58), so results
// are bit-identical. Weight loads are issued before the activation prologue
// (quantise / RMSNorm+quantise in LDS) so HBM latency overlaps it.
#include "fah_device.h"
#include "fah_internal.h"

namespace fah {

constexpr int kThreads = 256;
constexpr int kMaxK = 4096;

struct ScaleHalf {
  using type = _Float16;
  static __device__ __forceinline__ float get(type v) { return (float)v; }
};
struct ScaleFloat {
  using type = float;
  static __device__ __forceinline__ float get(type v) { return v; }
};

// Block-wide sum of one double per thread (256 threads, 4 waves).
__device__ __forceinline__ double block_sum_double(double v, double* scratch) {
  v = wave_sum_double(v);
  int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  double total = 0.0;
  int waves = (blockDim.x + kWave - 1) / kWave;
  for (int i = 0; i < waves; ++i) total += scratch[i];
  __syncthreads();
  return total;
}

// RMSNorm inverse of src/FunAsrNet/TensorMath.Elementwise.cs:58-78 (rms):
// 1f / sqrtf((float)(sum_sq / width) + eps). The double sum is a tree here;
// the reference's sequential lane order only changes double rounding, which
// reaches the float result with probability ~1e-7 per row.
__device__ __forceinline__ float rms_inverse(double sum_sq, int width, float eps) {
  float mean = (float)(sum_sq / (double)width);
  return fdiv(1.0f, sqrt_rn(fadd(mean, eps)));
}

// Quantise K fp32 values staged in LDS (fx) into xq/xs (LDS); one thread per
// 32-value block.
__device__ __forceinline__ void quantize_lds(const float* fx, int K, int8_t* xq, float* xs) {
  int blocks = K >> 5;
  for (int b = threadIdx.x; b < blocks; b += blockDim.x) {
    const float* v = fx + b * 32;
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      uint32_t a = f2u(v[i]) & 0x7fffffffu;
      m = a > m ? a : m;
    }
    float inverse;
    xs[b] = block_scale(m, &inverse);
    int words[8];
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      uint32_t packed = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) packed |= (uint32_t)(uint8_t)quantize_value(v[w * 4 + k], inverse) << (8 * k);
      words[w] = (int)packed;
    }
    int4* dst = reinterpret_cast<int4*>(xq + b * 32);
    dst[0] = make_int4(words[0], words[1], words[2], words[3]);
    dst[1] = make_int4(words[4], words[5], words[6], words[7]);
  }
}

template <typename Scale, int IN, int OUT, int PAIRS>
__global__ __launch_bounds__(kThreads) void q8_gemv_kernel(GemvArgs a) {
  __shared__ int4 xq_words[kMaxK / 16];
  __shared__ float xs_s[kMaxK / 32];
  __shared__ float fx_s[kMaxK];
  __shared__ float prod_s[kThreads * PAIRS + 64];
  __shared__ float sums_s[kThreads];
  __shared__ double red_s[kThreads / kWave];
  __shared__ unsigned long long key_s[kThreads / kWave];
  int8_t* xq_s = reinterpret_cast<int8_t*>(xq_words);

  const int tid = threadIdx.x;
  const int K = a.K, B = K >> 5;
  const int frame = blockIdx.y;
  const int row0 = blockIdx.x * a.group_rows;
  const int nrows = min(a.group_rows, a.rows - row0);
  const int npairs = nrows * B;
  const int stride = B + 1;

  // 1. Weight stream for this group: issued first, consumed after the prologue.
  int4 wv[PAIRS][2];
  typename Scale::type sv[PAIRS];
  const int8_t* wbase = a.w + (size_t)row0 * K;
  const typename Scale::type* sbase = reinterpret_cast<const typename Scale::type*>(a.ws) + (size_t)row0 * B;
#pragma unroll
  for (int i = 0; i < PAIRS; ++i) {
    int j = tid + i * kThreads;
    if (j < npairs) {
      const int4* p = reinterpret_cast<const int4*>(wbase + (size_t)j * 32);
      wv[i][0] = p[0];
      wv[i][1] = p[1];
      sv[i] = sbase[j];
    }
  }

  // 2. Activation prologue into LDS.
  if (IN == kInputQuantized) {
    const int4* src = reinterpret_cast<const int4*>(a.xq + (size_t)frame * K);
    for (int i = tid; i < K / 16; i += kThreads) xq_words[i] = src[i];
    for (int i = tid; i < B; i += kThreads) xs_s[i] = a.xs[(size_t)frame * B + i];
  } else {
    const float* x = a.x + (size_t)frame * K;
    double sq = 0.0;
    for (int i = tid; i < K; i += kThreads) {
      float v = x[i];
      fx_s[i] = v;
      if (IN == kInputNorm) sq += (double)v * (double)v;
    }
    if (IN == kInputNorm) {
      double total = block_sum_double(sq, red_s);
      float inverse = rms_inverse(total, K, a.eps);
      for (int i = tid; i < K; i += kThreads) fx_s[i] = fmul(fmul(fx_s[i], inverse), a.norm_w[i]);
    }
    __syncthreads();
    quantize_lds(fx_s, K, xq_s, xs_s);
  }
  __syncthreads();

  // 3. Exact block dots and scaled products.
#pragma unroll
  for (int i = 0; i < PAIRS; ++i) {
    int j = tid + i * kThreads;
    if (j < npairs) {
      int r = j / B, b = j - r * B;
      const int4* xv = reinterpret_cast<const int4*>(xq_s + b * 32);
      int4 x0 = xv[0], x1 = xv[1];
      int dot = 0;
      dot = __builtin_amdgcn_sdot4(wv[i][0].x, x0.x, dot, false);
      dot = __builtin_amdgcn_sdot4(wv[i][0].y, x0.y, dot, false);
      dot = __builtin_amdgcn_sdot4(wv[i][0].z, x0.z, dot, false);
      dot = __builtin_amdgcn_sdot4(wv[i][0].w, x0.w, dot, false);
      dot = __builtin_amdgcn_sdot4(wv[i][1].x, x1.x, dot, false);
      dot = __builtin_amdgcn_sdot4(wv[i][1].y, x1.y, dot, false);
      dot = __builtin_amdgcn_sdot4(wv[i][1].z, x1.z, dot, false);
      dot = __builtin_amdgcn_sdot4(wv[i][1].w, x1.w, dot, false);
      prod_s[r * stride + b] = fmul(fmul((float)dot, Scale::get(sv[i])), xs_s[b]);
    }
  }
  __syncthreads();

  // 4. Ordered block sum, one lane per row.
  float sum = 0.0f;
  if (tid < nrows) {
    const float* pr = prod_s + tid * stride;
    for (int b = 0; b < B; ++b) sum = fadd(sum, pr[b]);
  }

  // 5. Epilogue.
  float* out = a.out + (size_t)frame * a.out_rows;
  if (OUT == kOutPlain) {
    if (tid < nrows) out[row0 + tid] = a.bias ? fadd(a.bias[row0 + tid], sum) : sum;
  } else if (OUT == kOutResidual) {
    if (tid < nrows) out[row0 + tid] = fadd(sum, a.resid[(size_t)frame * a.out_rows + row0 + tid]);
  } else if (OUT == kOutSwiGLU) {
    // Rows of a group: group_rows/2 gate rows, then the matching up rows
    // (src/FunAsrNet/TensorMath.Elementwise.cs:167-196: g / (1 + exp(-g)) * up).
    if (tid < nrows) sums_s[tid] = sum;
    __syncthreads();
    int half = a.group_rows >> 1;
    if (tid < half) {
      float g = sums_s[tid], u = sums_s[half + tid];
      float silu = fdiv(g, fadd(1.0f, exp_ref(-g)));
      out[blockIdx.x * half + tid] = fmul(silu, u);
    }
  } else if (OUT == kOutGreedy) {
    unsigned long long key = 0ull;
    if (tid < nrows) {
      out[row0 + tid] = sum;
      key = greedy_key(sum, (uint32_t)(row0 + tid));
    }
    key = wave_max_u64(key);
    if (tid % kWave == 0) key_s[tid / kWave] = key;
    __syncthreads();
    if (tid == 0) {
      unsigned long long best = key_s[0];
      for (int w = 1; w < kThreads / kWave; ++w) best = key_s[w] > best ? key_s[w] : best;
      a.partial_keys[(size_t)frame * gridDim.x + blockIdx.x] = best;
    }
  }
}

// Greedy over the lm_head's per-group maxima (QwenDecoder.Greedy semantics,
// with the NaN-first rule: logits[0] NaN -> 0). Also records the token and
// advances the decoder position when asked.
__global__ __launch_bounds__(1024) void greedy_reduce_kernel(const unsigned long long* keys, int count,
                                                             const float* logits, int* token) {
  __shared__ unsigned long long part[1024 / kWave];
  unsigned long long best = 0ull;
  for (int i = threadIdx.x; i < count; i += blockDim.x) best = keys[i] > best ? keys[i] : best;
  best = wave_max_u64(best);
  if (threadIdx.x % kWave == 0) part[threadIdx.x / kWave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < (int)(blockDim.x / kWave); ++w) best = part[w] > best ? part[w] : best;
    float first = logits[0];
    *token = (first != first || best == 0ull) ? 0 : (int)greedy_index(best);
  }
}

// Embedding row of QwenDecoder.Embed (Gguf.cs:340-344): (float)q * scale.
// The token comes from device memory; it is also appended to the history.
template <typename Scale>
__global__ __launch_bounds__(kThreads) void embed_kernel(const int8_t* q, const void* scales, int K, int vocab,
                                                         const int* token, float* x, int* history,
                                                         int* history_count) {
  int t = *token;
  if (t < 0 || t >= vocab) t = 0;
  const typename Scale::type* s = reinterpret_cast<const typename Scale::type*>(scales);
  for (int j = threadIdx.x; j < K; j += blockDim.x) {
    size_t at = (size_t)t * K + j;
    x[j] = fmul((float)q[at], Scale::get(s[at / 32]));
  }
  if (history && threadIdx.x == 0) {
    int n = *history_count;
    history[n] = t;
    *history_count = n + 1;
  }
}

// Per-head QK RMSNorm + RoPE (QwenDecoder.cs:188-194, Rope.cs:14-55) and the
// F16 KV write (QwenDecoder.cs:195-203, Half.cs:18-53). Workgroups
// [0, heads) prepare query heads; [heads, heads+kv_heads) key/value heads.
// 128 threads = one per channel (head_size 128).
__global__ __launch_bounds__(128) void qk_prepare_kernel(QkArgs a) {
  __shared__ double red_s[2];
  __shared__ float y_s[128];
  const int c = threadIdx.x;
  const int pos = *a.position;
  const int hs = a.head_size, half = hs >> 1;
  const bool is_q = blockIdx.x < a.heads;
  const int head = is_q ? blockIdx.x : blockIdx.x - a.heads;
  const float* src = is_q ? a.qkv + head * hs : a.qkv + a.q_width + head * hs;
  const float* w = is_q ? a.q_norm : a.k_norm;
  float v = src[c];
  double sq = wave_sum_double((double)v * (double)v);
  if (c % kWave == 0) red_s[c / kWave] = sq;
  __syncthreads();
  float inverse = rms_inverse(red_s[0] + red_s[1], hs, a.eps);
  y_s[c] = fmul(fmul(v, inverse), w[c]);
  __syncthreads();
  float r;
  const float* cosine = a.rope_cos + (size_t)pos * half;
  const float* sine = a.rope_sin + (size_t)pos * half;
  if (c < half) {
    float x0 = y_s[c], x1 = y_s[c + half];
    r = fadd(fmul(x0, cosine[c]), -fmul(x1, sine[c]));
  } else {
    float x0 = y_s[c - half], x1 = y_s[c];
    r = fadd(fmul(x0, sine[c - half]), fmul(x1, cosine[c - half]));
  }
  if (is_q) {
    a.q_out[head * hs + c] = r;
  } else {
    size_t row = ((size_t)head * a.capacity + pos) * hs + c;
    a.kcache[row] = to_half(r);
    a.vcache[row] = to_half(a.qkv[a.q_width + a.kv_width + head * hs + c]);
  }
}

// Attention scores of one query head over positions [0, pos]: eight lane
// accumulators (channel c -> lane c % 8) of product-then-add, folded as
// ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)), divided by sqrtf(head_size)
// (TensorMath.AttentionAvx.cs:74-160, AudioKernels.cs:94-147).
// Grid (heads, G): each workgroup walks chunks of 32 positions.
__global__ __launch_bounds__(kThreads) void attn_scores_kernel(AttnArgs a) {
  const int head = blockIdx.x, kh = head / (a.heads / a.kv_heads);
  const int hs = a.head_size;
  const int n = *a.position + 1;
  const int j = threadIdx.x & 7, local = threadIdx.x >> 3;
  const float* q = a.q + head * hs;
  float qv[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) qv[i] = q[8 * i + j];
  const _Float16* kbase = a.kcache + (size_t)kh * a.capacity * hs;
  for (int t0 = blockIdx.y * 32; t0 < n; t0 += gridDim.y * 32) {
    int t = t0 + local;
    float acc = 0.0f;
    if (t < n) {
      const _Float16* k = kbase + (size_t)t * hs;
#pragma unroll
      for (int i = 0; i < 16; ++i) acc = fadd(acc, fmul(qv[i], from_half(k[8 * i + j])));
    }
    float s = fadd(acc, __shfl_xor(acc, 4, 8));
    s = fadd(s, __shfl_xor(s, 1, 8));
    s = fadd(s, __shfl_xor(s, 2, 8));
    if (t < n && j == 0) a.scores[(size_t)head * a.capacity + t] = fdiv(s, a.divisor);
  }
}

// Softmax (TensorMath.SoftmaxAvx.cs:11-58) and the value sum of one query
// head: out[c] = sum over t of v[t][c] * p[t], in time order from 0f
// (TensorMath.AttentionAvx.cs:173-224). One thread per channel.
__global__ __launch_bounds__(128) void attn_values_kernel(AttnArgs a) {
  extern __shared__ float p_s[];
  __shared__ float max_s[2];
  __shared__ double lane_s[8];
  __shared__ float inv_s;
  const int head = blockIdx.x, kh = head / (a.heads / a.kv_heads);
  const int hs = a.head_size;
  const int n = *a.position + 1;
  const int tid = threadIdx.x;
  const float* scores = a.scores + (size_t)head * a.capacity;
  float m = -__builtin_inff();
  for (int t = tid; t < n; t += blockDim.x) {
    float v = scores[t];
    p_s[t] = v;
    m = (v != v || m != m) ? (v != v ? v : m) : (v > m ? v : m);
  }
  for (int s = 32; s >= 1; s >>= 1) {
    float o = __shfl_xor(m, s, kWave);
    m = (o != o || m != m) ? (o != o ? o : m) : (o > m ? o : m);
  }
  if (tid % kWave == 0) max_s[tid / kWave] = m;
  __syncthreads();
  float mx = max_s[0], m1 = max_s[1];
  mx = (m1 != m1 || mx != mx) ? (m1 != m1 ? m1 : mx) : (m1 > mx ? m1 : mx);
  for (int t = tid; t < n; t += blockDim.x) p_s[t] = exp_ref(fadd(p_s[t], -mx));
  __syncthreads();
  const int full = n & ~7;
  if (tid < 8) {
    double l = 0.0;
    for (int t = tid; t < full; t += 8) l = l + (double)p_s[t];
    lane_s[tid] = l;
  }
  __syncthreads();
  if (tid == 0) {
    double sum = ((lane_s[0] + lane_s[4]) + (lane_s[1] + lane_s[5])) + ((lane_s[2] + lane_s[6]) + (lane_s[3] + lane_s[7]));
    for (int t = full; t < n; ++t) sum = sum + (double)p_s[t];
    inv_s = (float)(1.0 / sum);
  }
  __syncthreads();
  const float inverse = inv_s;
  for (int t = tid; t < n; t += blockDim.x) p_s[t] = fmul(p_s[t], inverse);
  __syncthreads();
  const _Float16* v = a.vcache + (size_t)kh * a.capacity * hs + tid;
  float acc = 0.0f;
  int t = 0;
  for (; t + 4 <= n; t += 4) {
    float v0 = from_half(v[(size_t)(t + 0) * hs]);
    float v1 = from_half(v[(size_t)(t + 1) * hs]);
    float v2 = from_half(v[(size_t)(t + 2) * hs]);
    float v3 = from_half(v[(size_t)(t + 3) * hs]);
    acc = fadd(acc, fmul(v0, p_s[t + 0]));
    acc = fadd(acc, fmul(v1, p_s[t + 1]));
    acc = fadd(acc, fmul(v2, p_s[t + 2]));
    acc = fadd(acc, fmul(v3, p_s[t + 3]));
  }
  for (; t < n; ++t) acc = fadd(acc, fmul(from_half(v[(size_t)t * hs]), p_s[t]));
  a.out[head * hs + tid] = acc;
}

__global__ void advance_kernel(int* position, int frames) {
  if (threadIdx.x == 0) *position += frames;
}

// Standalone quantiser: one thread per 32-value block.
__global__ __launch_bounds__(kThreads) void quantize_kernel(const float* x, int64_t blocks, int8_t* q, float* s) {
  int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= blocks) return;
  const float* v = x + b * 32;
  float vals[32];
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    vals[i] = v[i];
    uint32_t u = f2u(vals[i]) & 0x7fffffffu;
    m = u > m ? u : m;
  }
  float inverse;
  s[b] = block_scale(m, &inverse);
#pragma unroll
  for (int i = 0; i < 32; ++i) q[b * 32 + i] = quantize_value(vals[i], inverse);
}

// Exact int32 block dots of one activation row against every weight row.
__global__ __launch_bounds__(kThreads) void block_dots_kernel(const int8_t* x, const int8_t* w, int rows, int K,
                                                              int* dots) {
  int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int B = K >> 5;
  if (j >= (int64_t)rows * B) return;
  int64_t r = j / B;
  int b = (int)(j - r * B);
  const int4* wp = reinterpret_cast<const int4*>(w + r * K + b * 32);
  const int4* xp = reinterpret_cast<const int4*>(x + b * 32);
  int4 w0 = wp[0], w1 = wp[1], x0 = xp[0], x1 = xp[1];
  int dot = 0;
  dot = __builtin_amdgcn_sdot4(w0.x, x0.x, dot, false);
  dot = __builtin_amdgcn_sdot4(w0.y, x0.y, dot, false);
  dot = __builtin_amdgcn_sdot4(w0.z, x0.z, dot, false);
  dot = __builtin_amdgcn_sdot4(w0.w, x0.w, dot, false);
  dot = __builtin_amdgcn_sdot4(w1.x, x1.x, dot, false);
  dot = __builtin_amdgcn_sdot4(w1.y, x1.y, dot, false);
  dot = __builtin_amdgcn_sdot4(w1.z, x1.z, dot, false);
  dot = __builtin_amdgcn_sdot4(w1.w, x1.w, dot, false);
  dots[j] = dot;
}

// ---------------------------------------------------------------------------
// Host-side launchers
// ---------------------------------------------------------------------------

template <typename Scale, int IN, int OUT>
static hipError_t launch_gemv_pairs(const GemvArgs& a, int frames, int pairs_per_thread, hipStream_t s) {
  dim3 grid((a.rows + a.group_rows - 1) / a.group_rows, frames);
  switch (pairs_per_thread) {
    case 1: q8_gemv_kernel<Scale, IN, OUT, 1><<<grid, kThreads, 0, s>>>(a); break;
    case 2: q8_gemv_kernel<Scale, IN, OUT, 2><<<grid, kThreads, 0, s>>>(a); break;
    case 3: q8_gemv_kernel<Scale, IN, OUT, 3><<<grid, kThreads, 0, s>>>(a); break;
    case 4: q8_gemv_kernel<Scale, IN, OUT, 4><<<grid, kThreads, 0, s>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename Scale, int IN>
static hipError_t launch_gemv_out(const GemvArgs& a, int out, int frames, int ppt, hipStream_t s) {
  switch (out) {
    case kOutPlain: return launch_gemv_pairs<Scale, IN, kOutPlain>(a, frames, ppt, s);
    case kOutResidual: return launch_gemv_pairs<Scale, IN, kOutResidual>(a, frames, ppt, s);
    case kOutSwiGLU: return launch_gemv_pairs<Scale, IN, kOutSwiGLU>(a, frames, ppt, s);
    case kOutGreedy: return launch_gemv_pairs<Scale, IN, kOutGreedy>(a, frames, ppt, s);
  }
  return hipErrorInvalidValue;
}

template <typename Scale>
static hipError_t launch_gemv_in(const GemvArgs& a, int in, int out, int frames, int ppt, hipStream_t s) {
  switch (in) {
    case kInputQuantized: return launch_gemv_out<Scale, kInputQuantized>(a, out, frames, ppt, s);
    case kInputFloat: return launch_gemv_out<Scale, kInputFloat>(a, out, frames, ppt, s);
    case kInputNorm: return launch_gemv_out<Scale, kInputNorm>(a, out, frames, ppt, s);
  }
  return hipErrorInvalidValue;
}

int gemv_max_k() { return kMaxK; }

int gemv_pairs_per_thread(int group_rows, int K) {
  int pairs = group_rows * (K >> 5);
  return (pairs + kThreads - 1) / kThreads;
}

hipError_t launch_gemv(const GemvArgs& a, bool half_scales, int in, int out, int frames, hipStream_t s) {
  if (a.K % 32 != 0 || a.K > kMaxK || a.group_rows < 1 || a.group_rows > 64 || a.rows < 1) return hipErrorInvalidValue;
  if (out == kOutSwiGLU && (a.group_rows % 2 != 0 || a.rows % a.group_rows != 0)) return hipErrorInvalidValue;
  int ppt = gemv_pairs_per_thread(a.group_rows, a.K);
  if (ppt < 1 || ppt > 4) return hipErrorInvalidValue;
  return half_scales ? launch_gemv_in<ScaleHalf>(a, in, out, frames, ppt, s)
                     : launch_gemv_in<ScaleFloat>(a, in, out, frames, ppt, s);
}

hipError_t launch_greedy_reduce(const unsigned long long* keys, int count, const float* logits, int* token,
                                hipStream_t s) {
  greedy_reduce_kernel<<<1, 1024, 0, s>>>(keys, count, logits, token);
  return hipGetLastError();
}

hipError_t launch_embed(const int8_t* q, const void* scales, bool half_scales, int K, int vocab, const int* token,
                        float* x, int* history, int* history_count, hipStream_t s) {
  if (half_scales)
    embed_kernel<ScaleHalf><<<1, kThreads, 0, s>>>(q, scales, K, vocab, token, x, history, history_count);
  else
    embed_kernel<ScaleFloat><<<1, kThreads, 0, s>>>(q, scales, K, vocab, token, x, history, history_count);
  return hipGetLastError();
}

hipError_t launch_qk_prepare(const QkArgs& a, hipStream_t s) {
  if (a.head_size != 128) return hipErrorInvalidValue;
  qk_prepare_kernel<<<a.heads + a.kv_heads, 128, 0, s>>>(a);
  return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs& a, int score_groups, hipStream_t s) {
  if (a.head_size != 128) return hipErrorInvalidValue;
  attn_scores_kernel<<<dim3(a.heads, score_groups), kThreads, 0, s>>>(a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  attn_values_kernel<<<a.heads, 128, sizeof(float) * a.capacity, s>>>(a);
  return hipGetLastError();
}

hipError_t launch_advance(int* position, int frames, hipStream_t s) {
  advance_kernel<<<1, 64, 0, s>>>(position, frames);
  return hipGetLastError();
}

hipError_t launch_quantize(const float* x, int64_t n, int8_t* q, float* scales, hipStream_t s) {
  int64_t blocks = n / 32;
  if (blocks == 0) return hipSuccess;
  quantize_kernel<<<(unsigned)((blocks + kThreads - 1) / kThreads), kThreads, 0, s>>>(x, blocks, q, scales);
  return hipGetLastError();
}

hipError_t launch_block_dots(const int8_t* x, const int8_t* w, int rows, int K, int* dots, hipStream_t s) {
  int64_t n = (int64_t)rows * (K / 32);
  if (n == 0) return hipSuccess;
  block_dots_kernel<<<(unsigned)((n + kThreads - 1) / kThreads), kThreads, 0, s>>>(x, w, rows, K, dots);
  return hipGetLastError();
}

}  // namespace fah
