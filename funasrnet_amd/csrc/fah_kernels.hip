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
using lds_ptr = __attribute__((address_space(3))) void*;
constexpr int kMaxK = 4096;       // K held in registers in 4 chunks (the decoder's projections)
constexpr int kMaxKLarge = 16384; // wider inputs (larger models' down projection): 16 chunks

struct ScaleHalf {
  using type = _Float16;
  static __device__ __forceinline__ float get(type v) { return (float)v; }
};
struct ScaleFloat {
  using type = float;
  static __device__ __forceinline__ float get(type v) { return v; }
};

// CH: chunks of 4 * kThreads values, K <= CH * 1024.
template <typename Scale, int IN, int OUT, int PAIRS, int CH>
__global__ __launch_bounds__(kThreads) void q8_gemv_kernel(GemvArgs a) {
  constexpr int kMaxChunks = CH;
  __shared__ int xq_s[kMaxChunks * kThreads];
  __shared__ float xs_s[kMaxChunks * kThreads / 8];
  __shared__ float prod_s[kThreads * PAIRS];  // [block][row]
  __shared__ float sums_s[64];
  __shared__ double red_s[kThreads / kWave];

  const int tid = threadIdx.x;
  const int K = a.K, B = K >> 5;
  const int frame = blockIdx.y;
  const int R = a.group_rows;
  const int row0 = blockIdx.x * R;
  const int nrows = min(R, a.rows - row0);
  const int npairs = nrows * B;

  // 1. Activation, norm-weight and residual loads first: waiting for them
  //    later does not wait for the weight stream issued after them.
  float4 xv[kMaxChunks];
  float4 nw[kMaxChunks];
  int xw[kMaxChunks];
  // Block scales of a quantised input: B = K/32 of them, two per lane past
  // 256 blocks (K > 8192).
  float xsv = 0.0f, xsv2 = 0.0f, rv = 0.0f;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    int e = c * 4 * kThreads + 4 * tid;
    if (e < K) {
      if (IN == kInputQuantized) {
        xw[c] = *reinterpret_cast<const int*>(a.xq + (size_t)frame * K + e);
      } else {
        xv[c] = *reinterpret_cast<const float4*>(a.x + (size_t)frame * K + e);
        if (IN == kInputNorm) nw[c] = *reinterpret_cast<const float4*>(a.norm_w + e);
      }
    }
  }
  if (IN == kInputQuantized && tid < B) xsv = a.xs[(size_t)frame * B + tid];
  if (IN == kInputQuantized && kMaxChunks > 8 && kThreads + tid < B) xsv2 = a.xs[(size_t)frame * B + kThreads + tid];
  if (OUT == kOutResidual && tid < nrows) rv = a.resid[(size_t)frame * a.out_rows + row0 + tid];
  if (OUT == kOutPlain && a.bias && tid < nrows) rv = a.bias[row0 + tid];

  // 2. Weight stream for this group: one lane per (row, block) pair.
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

  // 3. Activation prologue into LDS.
  if (IN == kInputQuantized) {
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) {
      int e = c * 4 * kThreads + 4 * tid;
      if (e < K) xq_s[e >> 2] = xw[c];
    }
    if (tid < B) xs_s[tid] = xsv;
    if (kMaxChunks > 8 && kThreads + tid < B) xs_s[kThreads + tid] = xsv2;
  } else {
    float inverse = 1.0f;
    if (IN == kInputNorm) {
      double sq = 0.0;
#pragma unroll
      for (int c = 0; c < kMaxChunks; ++c) {
        int e = c * 4 * kThreads + 4 * tid;
        if (e < K) {
          sq += (double)xv[c].x * (double)xv[c].x + (double)xv[c].y * (double)xv[c].y;
          sq += (double)xv[c].z * (double)xv[c].z + (double)xv[c].w * (double)xv[c].w;
        }
      }
      const float* row = a.x + (size_t)frame * K;
      inverse = rms_inverse(block_sum_double(sq, red_s), K, a.eps, [&](int k) { return row[k]; });
    }
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) {
      int e = c * 4 * kThreads + 4 * tid;
      if (e < K) {
        float4 v = xv[c];
        if (IN == kInputNorm) {
          v.x = fmul(fmul(v.x, inverse), nw[c].x);
          v.y = fmul(fmul(v.y, inverse), nw[c].y);
          v.z = fmul(fmul(v.z, inverse), nw[c].z);
          v.w = fmul(fmul(v.w, inverse), nw[c].w);
        }
        float d;
        xq_s[e >> 2] = quantize4(v.x, v.y, v.z, v.w, &d);
        if ((tid & 7) == 0) xs_s[e >> 5] = d;
      }
    }
  }
  lds_barrier();

  // 4. Exact block dots and scaled products, stored block-major.
#pragma unroll
  for (int i = 0; i < PAIRS; ++i) {
    int j = tid + i * kThreads;
    if (j < npairs) {
      int r = j / B, b = j - r * B;
      const int4* xp = reinterpret_cast<const int4*>(xq_s + b * 8);
      int4 x0 = xp[0], x1 = xp[1];
      int dot = 0;
      dot = __builtin_amdgcn_sdot4(wv[i][0].x, x0.x, dot, false);
      dot = __builtin_amdgcn_sdot4(wv[i][0].y, x0.y, dot, false);
      dot = __builtin_amdgcn_sdot4(wv[i][0].z, x0.z, dot, false);
      dot = __builtin_amdgcn_sdot4(wv[i][0].w, x0.w, dot, false);
      dot = __builtin_amdgcn_sdot4(wv[i][1].x, x1.x, dot, false);
      dot = __builtin_amdgcn_sdot4(wv[i][1].y, x1.y, dot, false);
      dot = __builtin_amdgcn_sdot4(wv[i][1].z, x1.z, dot, false);
      dot = __builtin_amdgcn_sdot4(wv[i][1].w, x1.w, dot, false);
      prod_s[b * R + r] = fmul(fmul((float)dot, Scale::get(sv[i])), xs_s[b]);
    }
  }
  lds_barrier();

  // 5. Ordered block sum from 0f, one lane per row (rows live in wave 0).
  if (tid >= kWave) return;
  float sum = 0.0f;
  if (tid < nrows) {
    int b = 0;
    for (; b + 8 <= B; b += 8) {
      float p[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) p[k] = prod_s[(b + k) * R + tid];
#pragma unroll
      for (int k = 0; k < 8; ++k) sum = fadd(sum, p[k]);
    }
    for (; b < B; ++b) sum = fadd(sum, prod_s[b * R + tid]);
  }

  // 6. Epilogue.
  float* out = a.out + (size_t)frame * a.out_rows;
  if (OUT == kOutPlain) {
    if (tid < nrows) out[row0 + tid] = a.bias ? fadd(rv, sum) : sum;
  } else if (OUT == kOutResidual) {
    if (tid < nrows) out[row0 + tid] = fadd(sum, rv);
  } else if (OUT == kOutSwiGLU) {
    // Rows of a group: R/2 gate rows, then the matching up rows
    // (src/FunAsrNet/TensorMath.Elementwise.cs:167-196: g / (1 + exp(-g)) * up).
    if (tid < nrows) sums_s[tid] = sum;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    int half = R >> 1;
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
    // Rows are lanes [0, nrows) of wave 0; the other lanes contribute 0.
    for (int m = 32; m >= 1; m >>= 1) {
      unsigned long long o = __shfl_xor(key, m, kWave);
      key = o > key ? o : key;
    }
    if (tid == 0) a.partial_keys[(size_t)frame * gridDim.x + blockIdx.x] = key;
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
  const int frame = blockIdx.y;
  const int hs = a.head_size, half = hs >> 1;
  int pos, capacity;
  const float *rope_cos, *rope_sin;
  _Float16 *kcache, *vcache;
  if (a.sessions) {
    const SessionRef& ss = a.sessions[frame];
    pos = *ss.position;
    capacity = ss.capacity;
    rope_cos = ss.rope_cos;
    rope_sin = ss.rope_sin;
    const size_t layer = (size_t)a.layer * a.kv_heads * capacity * hs;
    kcache = ss.kcache + layer;
    vcache = ss.vcache + layer;
  } else {
    pos = *a.position + frame;
    capacity = a.capacity;
    rope_cos = a.rope_cos;
    rope_sin = a.rope_sin;
    kcache = a.kcache;
    vcache = a.vcache;
  }
  const bool is_q = blockIdx.x < a.heads;
  const int head = is_q ? blockIdx.x : blockIdx.x - a.heads;
  const float* qkv = a.qkv + (size_t)frame * (a.q_width + 2 * a.kv_width);
  const float* src = is_q ? qkv + head * hs : qkv + a.q_width + head * hs;
  const float* w = is_q ? a.q_norm : a.k_norm;
  float v = src[c];
  double sq = wave_sum_double((double)v * (double)v);
  if (c % kWave == 0) red_s[c / kWave] = sq;
  __syncthreads();
  float inverse = rms_inverse(red_s[0] + red_s[1], hs, a.eps, [&](int k) { return src[k]; });
  y_s[c] = fmul(fmul(v, inverse), w[c]);
  __syncthreads();
  float r;
  const float* cosine = rope_cos + (size_t)pos * half;
  const float* sine = rope_sin + (size_t)pos * half;
  if (c < half) {
    float x0 = y_s[c], x1 = y_s[c + half];
    r = fadd(fmul(x0, cosine[c]), -fmul(x1, sine[c]));
  } else {
    float x0 = y_s[c - half], x1 = y_s[c];
    r = fadd(fmul(x0, sine[c - half]), fmul(x1, cosine[c - half]));
  }
  if (is_q) {
    a.q_out[(size_t)frame * a.q_width + head * hs + c] = r;
  } else {
    size_t row = ((size_t)head * capacity + pos) * hs + c;
    kcache[row] = to_half(r);
    vcache[row] = to_half(qkv[a.q_width + a.kv_width + head * hs + c]);
  }
}

// NaN-propagating maximum (Math.Max semantics for the softmax shift).
__device__ __forceinline__ float nan_max(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  return b > a ? b : a;
}

// Attention scores of one query head over positions [0, pos]: eight
// accumulators (channel c -> accumulator c % 8) of product-then-add, folded
// as ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)), divided by sqrtf(head_size)
// (TensorMath.AttentionAvx.cs:74-160, AudioKernels.cs:94-147). Grid (heads,
// position blocks of kThreads): one lane per position, its K row loaded
// whole (16 x 16 bytes in flight), q read from LDS. The products are one
// mixed-precision fma with a +0 addend: round(q * k) except that a -0
// product becomes +0, and no accumulator is ever -0 (they start at +0), so
// every sum is the reference's.
__global__ __launch_bounds__(kThreads) void attn_scores_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) float q_s[128];
  __shared__ float bm_s[kThreads / kWave];
  const int head = blockIdx.x, kh = head / (a.heads / a.kv_heads);
  const int hs = a.head_size, tid = threadIdx.x;
  const int n = *a.position + 1;
  if ((int)blockIdx.y * kThreads >= n) return;  // a block past the current position
  const int t = blockIdx.y * kThreads + tid;
  if (tid < hs) q_s[tid] = a.q[head * hs + tid];
  uint4 kk[16];
  const uint4* row = reinterpret_cast<const uint4*>(a.kcache + ((size_t)kh * a.capacity + min(t, n - 1)) * hs);
#pragma unroll
  for (int i = 0; i < 16; ++i) kk[i] = row[i];
  __syncthreads();
  // Lanes past the current position compute the last position's score
  // again: it joins the block maximum only, the score store is skipped.
  float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float4 q0 = *reinterpret_cast<const float4*>(q_s + 8 * i);
    const float4 q1 = *reinterpret_cast<const float4*>(q_s + 8 * i + 4);
    const float qv[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    const uint32_t w[4] = {kk[i].x, kk[i].y, kk[i].z, kk[i].w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const _Float16 k = __builtin_bit_cast(_Float16, (uint16_t)((j & 1) ? w[j >> 1] >> 16 : w[j >> 1] & 0xffffu));
      acc[j] = fadd(acc[j], mulh(qv[j], k));
    }
  }
  const float s = fadd(fadd(fadd(acc[0], acc[4]), fadd(acc[1], acc[5])), fadd(fadd(acc[2], acc[6]), fadd(acc[3], acc[7])));
  const float sd = fdiv(s, a.divisor);
  if (t < n) a.scores[(size_t)head * a.capacity + t] = sd;
  // The block's maximum (NaN-propagating, order-free) for the softmax shift.
  float m = sd;
  for (int o = 32; o >= 1; o >>= 1) m = nan_max(m, __shfl_xor(m, o, kWave));
  if ((tid & (kWave - 1)) == 0) bm_s[tid / kWave] = m;
  __syncthreads();
  if (tid == 0) {
    const int waves = (min(n - (int)blockIdx.y * kThreads, kThreads) + kWave - 1) / kWave;
    float b = bm_s[0];
    for (int w = 1; w < waves; ++w) b = nan_max(b, bm_s[w]);
    a.block_max[(size_t)head * gridDim.y + blockIdx.y] = b;
  }
}

// Softmax numerators (TensorMath.SoftmaxAvx.cs:11-58) in place: e[t] =
// exp(s[t] - max) (ExpAvx), the maximum over the score blocks' maxima
// (NaN-propagating). Grid (heads, position blocks of kThreads). Each value
// is also stored as a double by residue t % 8 (exp_t), the layout of the
// denominator's lane sums; the denominator and the normalisation run in
// attn_values_kernel.
__global__ __launch_bounds__(kThreads) void attn_exp_kernel(AttnArgs a) {
  const int head = blockIdx.x, tid = threadIdx.x;
  const int n = *a.position + 1, blocks = (n + kThreads - 1) / kThreads;
  const int t = blockIdx.y * kThreads + tid;
  if ((int)blockIdx.y >= blocks) return;
  const float* bm = a.block_max + (size_t)head * gridDim.y;
  float mx = bm[0];
  for (int b = 1; b < blocks; ++b) mx = nan_max(mx, bm[b]);
  double part = 0.0;
  bool exact = n < 8192;
  if (t < n) {
    float* sc = a.scores + (size_t)head * a.capacity + t;
    const float e = exp_ref(fadd(*sc, -mx));
    *sc = e;
    // By residue for the denominator's eight in-order lane sums.
    a.exp_t[((size_t)head * 8 + (t & 7)) * a.exp_stride + (t >> 3)] = (double)e;
    part = (double)e;
    exact = exact && (e == 0.0f || (e >= 0x1p-17f && e <= 1.0f));
  }
  // The block's sum for the denominator's exact shortcut: when every
  // numerator is 0 or in [2^-17, 1] and there are fewer than 8192, all
  // partial sums are exact doubles, so any order of addition is the
  // reference's (NaN marks a block that does not qualify).
  __shared__ double part_s[kThreads / kWave];
  __shared__ int exact_s[kThreads / kWave];
  part = wave_sum_double(part);
  const bool wexact = __all(exact);
  const int wave = tid / kWave;
  if ((tid & (kWave - 1)) == 0) {
    part_s[wave] = part;
    exact_s[wave] = wexact ? 1 : 0;
  }
  lds_barrier();
  if (tid == 0) {
    double sum = 0.0;
    int all = 1;
    for (int w = 0; w < kThreads / kWave; ++w) {
      sum += part_s[w];
      all &= exact_s[w];
    }
    a.block_sum[(size_t)head * gridDim.y + blockIdx.y] = all ? sum : __builtin_nan("");
  }
}

// One wave: (float)(1 / sum) of the softmax denominator in double
// (SoftmaxAvx.cs:11-58): lane j < 8 adds e[j], e[j+8], ... (t < full) in
// order from row j of et (the values as doubles by residue, row stride
// `stride` doubles, two a 16-byte read, 16 reads a batch), then the eight
// sums' pairwise tree, then the tail [full, n) of e (position order) in
// order. Valid in lane 0.
__device__ __forceinline__ float softmax_inverse(const double* et, int stride, const float* e, int n) {
  const int lane = threadIdx.x & (kWave - 1), full = n & ~7, m = full >> 3;  // values a lane adds
  double l = 0.0;
  if (lane < 8) {
    const double* row = et + (size_t)lane * stride;
    int i = 0;
    for (; i + 32 <= m; i += 32) {
      double2 v[16];
#pragma unroll
      for (int k = 0; k < 16; ++k) v[k] = *reinterpret_cast<const double2*>(row + i + 2 * k);
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        l = l + v[k].x;
        l = l + v[k].y;
      }
    }
    for (; i < m; ++i) l = l + row[i];
  }
  double L[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) L[j] = readlane_double(l, j);
  double sum = ((L[0] + L[4]) + (L[1] + L[5])) + ((L[2] + L[6]) + (L[3] + L[7]));
  for (int t = full; t < n; ++t) sum = sum + (double)e[t];
  return (float)(1.0 / sum);
}

// Value sums out[c] = sum over t of v[t][c] * p[t] in time order from 0f
// (TensorMath.AttentionAvx.cs:173-224) for the G query heads of one KV head
// (G = heads / kv_heads, 2 or 4) and a slice of kValC = 32 / G channels:
// 32 chains, run by lanes of wave 0 (one add per position); wave 4 copies V
// rows of the slice into a three-slot LDS ring two blocks ahead (direct
// global->LDS loads) and the other six waves form the products v * p of the
// next block into a two-slot product ring, so each chain step is one add
// (the product's rounding is the same wherever it is made). Before the first
// block, waves 0..G-1 form the heads' softmax denominators from the
// numerators by residue (staged in the product ring's space when they fit).
// Dynamic LDS: see values_lds.
constexpr int kValThreads = 512;
constexpr int kValChains = 32;                 // chains per workgroup: G heads x 32 / G channels
constexpr int kValBlk = 256;                   // positions per ring block
constexpr int kValRow = kValBlk + 12;          // product ring row (floats; also the residue rows' room)
constexpr int kValPSlot = kValChains * kValRow * 4;  // product ring slot (bytes)
constexpr int val_vslot(int group) { return kValBlk * (kValChains / group) * 2; }  // V ring slot (bytes)

template <int G>
__global__ __launch_bounds__(kValThreads) void attn_values_kernel(AttnArgs a) {
  constexpr int kValC = kValChains / G;        // channels per workgroup
  constexpr int kValVSlot = val_vslot(G);
  constexpr int kPieces = kValC / 8;           // 16-byte pieces of a position's V slice
  constexpr int kQuarters = kValC / 4;         // 4-channel producer tasks per position
  extern __shared__ __attribute__((aligned(16))) float dyn_s[];
  __shared__ float inv_s[G];
  constexpr int kWaves = kValThreads / kWave;
  const int slices = a.head_size / kValC;
  const int kh = blockIdx.x / slices, c0 = (blockIdx.x % slices) * kValC;
  const int hs = a.head_size, n = *a.position + 1, tid = threadIdx.x, wave = tid / kWave, lane = tid & (kWave - 1);
  const int group = a.heads / a.kv_heads;
  const int np = (n + 3) & ~3;
  float* p_s = dyn_s;                                               // [G][np]
  char* vring = reinterpret_cast<char*>(dyn_s + G * np);            // [3][kValBlk][kValC] fp16
  float* pring = reinterpret_cast<float*>(vring + 3 * kValVSlot);   // [2][kValChains][kValRow]
  const int blocks = (n + kValBlk - 1) / kValBlk;
  const _Float16* vbase = a.vcache + (size_t)kh * a.capacity * hs + c0;
  // V block j into ring slot j % 3: kPieces pieces of 16 bytes a position,
  // piece q of the block at byte 16 q; `first`/`step` spread the pieces over
  // the calling waves (positions past n repeat the last one, never used).
  auto fill = [&](int j, int first, int step) {
    char* dst = vring + (size_t)(j % 3) * kValVSlot;
    for (int q0 = first * 64; q0 < kPieces * kValBlk; q0 += step * 64) {
      const int q = q0 + lane, t = min(j * kValBlk + q / kPieces, n - 1);
      __builtin_amdgcn_global_load_lds(vbase + (size_t)t * hs + 8 * (q % kPieces), (lds_ptr)(dst + 16 * q0), 16, 0, 0);
    }
  };
  // The residue rows of the heads' numerators (m doubles a row, 16-byte
  // pieces; row r at `rs` doubles, two more than m rounded up to 2 so that
  // the eight lanes reading a column hit different banks), in the product
  // ring's space when they fit; else read from global memory.
  const int m = (n & ~7) >> 3, rs = ((m + 1) & ~1) + 2;
  const bool staged = (size_t)8 * G * rs * 8 <= (size_t)2 * kValPSlot;
  double* et_s = reinterpret_cast<double*>(pring);
  const double* et_g = a.exp_t + (size_t)kh * group * 8 * a.exp_stride;
  // Wave 0 runs the chains; wave 4, which shares its SIMD, only issues the
  // V loads, so that the chains have the SIMD's issue slots to themselves;
  // the other six waves form the products.
  constexpr int kProducers = kWaves - 2;
  const bool producer = wave != 0 && wave != kWaves / 2;
  const int prank = wave < kWaves / 2 ? wave - 1 : wave - 2;
  // Products of block j into product slot j & 1: task = (four positions,
  // 4-channel quarter), whose 4 G product rows of four positions each are
  // written as float4; rows [h kValC, (h + 1) kValC) head h. Positions past
  // n are formed from the clamped V rows and garbage probabilities and never
  // added.
  float inv[G];  // the heads' softmax inverses
  auto produce = [&](int j) {
    const char* vs = vring + (size_t)(j % 3) * kValVSlot;
    float* ps = pring + (size_t)(j & 1) * kValChains * kValRow;
    const int t0 = j * kValBlk, len = min(kValBlk, n - t0);
    for (int task = prank * kWave + lane; task < kQuarters * ((len + 3) >> 2); task += kProducers * kWave) {
      const int tq = 4 * (task / kQuarters), q = task % kQuarters, t = t0 + tq;
      uint2 raw[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) raw[u] = *reinterpret_cast<const uint2*>(vs + 2 * kValC * (tq + u) + 8 * q);
      // The probabilities p = e * inverse (the softmax's last step).
      float4 p[G];
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float4 e = *reinterpret_cast<const float4*>(p_s + h * np + t);
        p[h] = make_float4(fmul(e.x, inv[h]), fmul(e.y, inv[h]), fmul(e.z, inv[h]), fmul(e.w, inv[h]));
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = from_half(reinterpret_cast<const _Float16*>(&raw[u])[k]);
#pragma unroll
        for (int h = 0; h < G; ++h)
          *reinterpret_cast<float4*>(ps + (size_t)(h * kValC + 4 * q + k) * kValRow + tq) =
              make_float4(fmul(v[0], p[h].x), fmul(v[1], p[h].y), fmul(v[2], p[h].z), fmul(v[3], p[h].w));
      }
    }
  };
  // The numerators of the heads (written by attn_exp_kernel), their
  // residue rows and the first two V blocks, by all waves.
  {
    for (int h = 0; h < G; ++h) {
      const char* src = reinterpret_cast<const char*>(a.scores + (size_t)(kh * group + h) * a.capacity);
      char* dst = reinterpret_cast<char*>(p_s + h * np);
      const int bytes = np * 4;
      for (int c = wave * 1024; c < bytes; c += kWaves * 1024)
        if (c + 16 * lane < bytes) __builtin_amdgcn_global_load_lds(src + c + 16 * lane, (lds_ptr)(dst + c), 16, 0, 0);
    }
    if (staged) {
      const int rb = rs * 8;  // bytes a staged row
      for (int r = wave; r < 8 * G; r += kWaves) {
        const char* src = reinterpret_cast<const char*>(et_g + (size_t)r * a.exp_stride);
        char* dst = reinterpret_cast<char*>(et_s) + (size_t)r * rb;
        for (int c = 0; c < m * 8; c += 1024)
          if (c + 16 * lane < m * 8 + 8) __builtin_amdgcn_global_load_lds(src + c + 16 * lane, (lds_ptr)(dst + c), 16, 0, 0);
      }
    }
    fill(0, wave, kWaves);
    if (blocks > 1) fill(1, wave, kWaves);
    __builtin_amdgcn_s_waitcnt(0);
  }
  lds_barrier();
  // The heads' denominators, one wave each: the exact block sums of
  // attn_exp_kernel when every block qualifies (any order of exact
  // additions is the reference's), else the residue chains.
  if (wave < G) {
    const double* bs = a.block_sum + (size_t)(kh * group + wave) * ((a.capacity + kThreads - 1) / kThreads);
    double total = 0.0;
    for (int b = lane; b < blocks; b += kWave) total += bs[b];
    total = wave_sum_double(total);
    float inv;
    if (total == total) inv = (float)(1.0 / total);
    else inv = staged ? softmax_inverse(et_s + (size_t)wave * 8 * rs, rs, p_s + wave * np, n)
                      : softmax_inverse(et_g + (size_t)wave * 8 * a.exp_stride, a.exp_stride, p_s + wave * np, n);
    if (lane == 0) inv_s[wave] = inv;
  }
  lds_barrier();
#pragma unroll
  for (int h = 0; h < G; ++h) inv[h] = inv_s[h];
  if (producer) produce(0);
  lds_barrier();
  float acc = 0.0f;
  for (int j = 0; j < blocks; ++j) {
    if (producer) {
      if (j + 1 < blocks) produce(j + 1);
    } else if (wave == kWaves / 2) {
      if (j + 2 < blocks) fill(j + 2, 0, 1);
      __builtin_amdgcn_s_waitcnt(0);
    } else if (tid < kValChains) {
      const float* row = pring + (size_t)(j & 1) * kValChains * kValRow + (size_t)tid * kValRow;
      const int len = min(kValBlk, n - j * kValBlk);
      int tt = 0;
      if (len == kValBlk) {
        // Full block: products read three groups of 16 ahead of the adds
        // (the scheduling barrier keeps the loads that far ahead, so that
        // each add finds its product in registers: LDS latency is several
        // adds long).
        float4 q[4][4];
#pragma unroll
        for (int g = 0; g < 3; ++g)
#pragma unroll
          for (int k = 0; k < 4; ++k) q[g][k] = *reinterpret_cast<const float4*>(row + 16 * g + 4 * k);
#pragma unroll
        for (int i = 0; i < kValBlk / 16; ++i) {
          if (i + 3 < kValBlk / 16) {
#pragma unroll
            for (int k = 0; k < 4; ++k) q[(i + 3) & 3][k] = *reinterpret_cast<const float4*>(row + 16 * (i + 3) + 4 * k);
          }
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            acc = fadd(acc, q[i & 3][k].x);
            acc = fadd(acc, q[i & 3][k].y);
            acc = fadd(acc, q[i & 3][k].z);
            acc = fadd(acc, q[i & 3][k].w);
          }
        }
        tt = kValBlk;
      }
      for (; tt + 4 <= len; tt += 4) {
        const float4 q = *reinterpret_cast<const float4*>(row + tt);
        acc = fadd(acc, q.x);
        acc = fadd(acc, q.y);
        acc = fadd(acc, q.z);
        acc = fadd(acc, q.w);
      }
      for (; tt < len; ++tt) acc = fadd(acc, row[tt]);
    }
    lds_barrier();
  }
  if (tid < kValChains) {
    const int h2 = tid / kValC, ch = tid % kValC;
    a.out[(size_t)(kh * group + h2) * hs + c0 + ch] = acc;
  }
}

// Lock-step sessions: row f of x is the embedding of session f's token
// (QwenDecoder.Embed, QwenDecoder.cs:143-152), which joins its history.
template <class Scale>
__global__ __launch_bounds__(kThreads) void session_embed_kernel(const int8_t* q, const void* scales, int K, int vocab,
                                                                 const SessionRef* sessions, float* x) {
  const SessionRef& ss = sessions[blockIdx.x];
  int t = *ss.token;
  if (t < 0 || t >= vocab) t = 0;
  const typename Scale::type* s = reinterpret_cast<const typename Scale::type*>(scales);
  float* row = x + (size_t)blockIdx.x * K;
  for (int j = threadIdx.x; j < K; j += blockDim.x) {
    size_t at = (size_t)t * K + j;
    row[j] = fmul((float)q[at], Scale::get(s[at / 32]));
  }
  if (threadIdx.x == 0) {
    int n = *ss.history_count;
    ss.history[n] = t;
    *ss.history_count = n + 1;
  }
}

// Step-batcher bookkeeping around one lock-step step of the table's
// sessions: before it (out == nullptr) every history count is cleared; after
// it, each session's emitted token (its history's first entry) is gathered
// into out[i], so that one copy brings the batch's tokens back.
__global__ __launch_bounds__(64) void session_batch_io_kernel(const SessionRef* sessions, int count, int* out) {
  const int i = threadIdx.x;
  if (i >= count) return;
  if (out) out[i] = sessions[i].history[0];
  else *sessions[i].history_count = 0;
}

// One GGUF Q8_0 block per thread (TensorMath.Q8Model.cs:15-39 without the
// fp32 widening: the device keeps the fp16 scale bits): 17 aligned 16-bit
// reads (blocks start at even offsets), 8 words of codes and the scale out.
__global__ __launch_bounds__(kThreads) void unpack_q8_blocks_kernel(const uint16_t* raw, int64_t blocks, uint32_t* q,
                                                                    uint16_t* s) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= blocks) return;
  const uint16_t* src = raw + b * 17;
  s[b] = src[0];
#pragma unroll
  for (int i = 0; i < 8; ++i) q[b * 8 + i] = (uint32_t)src[1 + 2 * i] | ((uint32_t)src[2 + 2 * i] << 16);
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

template <typename Scale, int IN, int OUT, int CH>
static hipError_t launch_gemv_pairs_ch(const GemvArgs& a, int frames, int pairs_per_thread, hipStream_t s) {
  dim3 grid((a.rows + a.group_rows - 1) / a.group_rows, frames);
  switch (pairs_per_thread) {
    case 1: q8_gemv_kernel<Scale, IN, OUT, 1, CH><<<grid, kThreads, 0, s>>>(a); break;
    case 2: q8_gemv_kernel<Scale, IN, OUT, 2, CH><<<grid, kThreads, 0, s>>>(a); break;
    case 3: q8_gemv_kernel<Scale, IN, OUT, 3, CH><<<grid, kThreads, 0, s>>>(a); break;
    case 4: q8_gemv_kernel<Scale, IN, OUT, 4, CH><<<grid, kThreads, 0, s>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename Scale, int IN, int OUT>
static hipError_t launch_gemv_pairs(const GemvArgs& a, int frames, int pairs_per_thread, hipStream_t s) {
  return a.K <= kMaxK ? launch_gemv_pairs_ch<Scale, IN, OUT, kMaxK / (4 * kThreads)>(a, frames, pairs_per_thread, s)
                      : launch_gemv_pairs_ch<Scale, IN, OUT, kMaxKLarge / (4 * kThreads)>(a, frames, pairs_per_thread, s);
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

int gemv_max_k() { return kMaxKLarge; }

int gemv_pairs_per_thread(int group_rows, int K) {
  int pairs = group_rows * (K >> 5);
  return (pairs + kThreads - 1) / kThreads;
}

hipError_t launch_gemv(const GemvArgs& a, bool half_scales, int in, int out, int frames, hipStream_t s) {
  if (a.K % 32 != 0 || a.K > kMaxKLarge || a.group_rows < 1 || a.group_rows > 64 || a.rows < 1) return hipErrorInvalidValue;
  if (a.group_rows * (a.K / 32) > 4 * kThreads) return hipErrorInvalidValue;
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

hipError_t launch_session_embed(const int8_t* q, const void* scales, bool half_scales, int K, int vocab,
                                const SessionRef* sessions, int count, float* x, hipStream_t s) {
  if (count < 1) return hipErrorInvalidValue;
  if (half_scales)
    session_embed_kernel<ScaleHalf><<<count, kThreads, 0, s>>>(q, scales, K, vocab, sessions, x);
  else
    session_embed_kernel<ScaleFloat><<<count, kThreads, 0, s>>>(q, scales, K, vocab, sessions, x);
  return hipGetLastError();
}

hipError_t launch_unpack_q8_blocks(const uint8_t* raw, int64_t blocks, int8_t* q, uint16_t* s, hipStream_t st) {
  if (blocks < 0 || (reinterpret_cast<uintptr_t>(raw) & 1) || (reinterpret_cast<uintptr_t>(q) & 3))
    return hipErrorInvalidValue;
  if (blocks == 0) return hipSuccess;
  const int64_t grid = (blocks + kThreads - 1) / kThreads;
  unpack_q8_blocks_kernel<<<(unsigned)grid, kThreads, 0, st>>>(reinterpret_cast<const uint16_t*>(raw), blocks,
                                                               reinterpret_cast<uint32_t*>(q), s);
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
  qk_prepare_kernel<<<dim3(a.heads + a.kv_heads, a.frames > 1 ? a.frames : 1), 128, 0, s>>>(a);
  return hipGetLastError();
}

// Dynamic LDS of attn_values_kernel for `capacity` positions and G =
// `group` query heads a KV head: the heads' probabilities (rounded up to 4
// positions), the three-slot V ring and the two-slot product ring.
static size_t values_lds(int capacity, int group) {
  return (size_t)group * ((capacity + 3) & ~3) * 4 + 3 * val_vslot(group) + 2 * kValPSlot;
}

int attention_slices(int capacity, int head_size, int group) {
  if (group != 2 && group != 4) return 0;
  const int channels = kValChains / group;
  if (head_size % channels != 0 || values_lds(capacity, group) > 160 * 1024 - 1024) return 0;
  return head_size / channels;
}

size_t attention_lds_bytes(int capacity, int head_size, int group) {
  return attention_slices(capacity, head_size, group) ? values_lds(capacity, group) : 0;
}

hipError_t prepare_attention(int capacity, int head_size, int group) {
  if (!attention_lds_bytes(capacity, head_size, group)) return hipErrorInvalidValue;
  // The limits are per kernel, not per decoder: set the largest size any
  // capacity that attention_slices accepts can ask for, so decoders of
  // different capacities do not lower each other's limit.
  const void* kernel = group == 2 ? reinterpret_cast<const void*>(attn_values_kernel<2>)
                                  : reinterpret_cast<const void*>(attn_values_kernel<4>);
  return hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 - 1024);
}

hipError_t launch_attention(const AttnArgs& a, int /*score_groups*/, hipStream_t s) {
  const int group = a.kv_heads > 0 ? a.heads / a.kv_heads : 0;
  if (a.head_size != 128 || a.heads != group * a.kv_heads || !a.block_max || !a.exp_t ||
      a.exp_stride < attention_exp_stride(a.capacity))
    return hipErrorInvalidValue;
  const int slices = attention_slices(a.capacity, a.head_size, group);
  if (!slices) return hipErrorInvalidValue;
  const dim3 grid(a.heads, (a.capacity + kThreads - 1) / kThreads);
  attn_scores_kernel<<<grid, kThreads, 0, s>>>(a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  attn_exp_kernel<<<grid, kThreads, 0, s>>>(a);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  const size_t lds = attention_lds_bytes(a.capacity, a.head_size, group);
  if (group == 2) attn_values_kernel<2><<<a.kv_heads * slices, kValThreads, lds, s>>>(a);
  else attn_values_kernel<4><<<a.kv_heads * slices, kValThreads, lds, s>>>(a);
  return hipGetLastError();
}

hipError_t launch_advance(int* position, int frames, hipStream_t s) {
  advance_kernel<<<1, 64, 0, s>>>(position, frames);
  return hipGetLastError();
}

// RMSNorm of rows with the decoder kernels' norm arithmetic (the ABI's
// fah_rms_norm_device): width 128 as the persistent step's QK-norm (one full
// wave, lane c holding channels c and c + 64), other widths (a multiple of 4,
// at most 4096) as the norm prologues (256 threads holding values 4t + 1024c,
// then the block tree). y = (x * inverse) * scale, TensorMath.Elementwise.cs:80-92.
__global__ __launch_bounds__(256) void rms_norm_rows_kernel(const float* x, int width, const float* scale, float eps,
                                                            float* y) {
  __shared__ double red_s[4];
  const int tid = threadIdx.x;
  const float* row = x + (size_t)blockIdx.x * width;
  float* out = y + (size_t)blockIdx.x * width;
  if (width == 128) {
    if (tid >= kWave) return;
    const float2 r = head_norm_rope<false>(row[tid], row[tid + 64], scale, nullptr, eps);
    out[tid] = r.x;
    out[tid + 64] = r.y;
    return;
  }
  constexpr int kChunks = 4;
  float4 v[kChunks];
  double sq = 0.0;
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int e = c * 1024 + 4 * tid;
    v[c] = e < width ? *reinterpret_cast<const float4*>(row + e) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    sq += (double)v[c].x * (double)v[c].x + (double)v[c].y * (double)v[c].y;
    sq += (double)v[c].z * (double)v[c].z + (double)v[c].w * (double)v[c].w;
  }
  const float inverse = rms_inverse(block_sum_double(sq, red_s), width, eps, [&](int k) { return row[k]; });
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int e = c * 1024 + 4 * tid;
    if (e < width) {
      const float4 w = *reinterpret_cast<const float4*>(scale + e);
      *reinterpret_cast<float4*>(out + e) =
          make_float4(fmul(fmul(v[c].x, inverse), w.x), fmul(fmul(v[c].y, inverse), w.y),
                      fmul(fmul(v[c].z, inverse), w.z), fmul(fmul(v[c].w, inverse), w.w));
    }
  }
}

hipError_t launch_rms_norm_rows(const float* x, int rows, int width, const float* scale, float eps, float* y,
                                hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  if (width != 128 && (width % 4 != 0 || width > 4096)) return hipErrorInvalidValue;
  rms_norm_rows_kernel<<<(unsigned)rows, 256, 0, s>>>(x, width, scale, eps, y);
  return hipGetLastError();
}

hipError_t launch_session_batch_io(const SessionRef* sessions, int count, int* out, hipStream_t s) {
  if (count < 1 || count > 64) return hipErrorInvalidValue;
  session_batch_io_kernel<<<1, 64, 0, s>>>(sessions, count, out);
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
