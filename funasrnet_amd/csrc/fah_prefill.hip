// Prefill kernels: QwenDecoder.Decode with frames > 1
// (src/FunAsrNet/QwenDecoder.cs:161-271; grouped Q8 over frames,
// TensorMath.QuantizedGroupAvx.cs:156-199 / QuantizedVnni.cs:77-126, whose
// float order equals the single-frame one).
//
// q8_gemm_kernel: out[t][r] = sum over blocks b, in order, from 0f, of
// ((float)dot_b * w_scale[r][b]) * x_scale[t][b]. The exact int32 32-term
// block dots come from one v_mfma_i32_16x16x32_i8 per block and 16x16 tile
// with a zero accumulator; the fp32 steps then run on the result registers
// in block order, so the result is the one of the reference's per-row loop
// for every frame. Row and frame scales are staged in LDS as fp32.
//
// Lane layout of v_mfma_i32_16x16x32_i8 (checked on gfx950): the A (B)
// operand of lane l is the 8 bytes [8 (l / 16), 8 (l / 16) + 8) of row
// (column) l % 16; result register j of lane l is C[4 (l / 16) + j][l % 16].
#include <algorithm>
#include <cstdlib>

#include "fah_device.h"
#include "fah_internal.h"

namespace fah {
namespace {

constexpr int kGT = 256;  // threads per GEMM workgroup
using lds_ptr = __attribute__((address_space(3))) void*;
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));

struct ScaleF16 {
  using type = _Float16;
  static __device__ __forceinline__ float get(type v) { return (float)v; }
};
struct ScaleF32 {
  using type = float;
  static __device__ __forceinline__ float get(type v) { return v; }
};

// Storage row of logical gate (kind 0) or up (kind 1) row r when the rows are
// stored as tiles of count gate rows followed by the same count up rows; the
// first `extra` tiles hold base + 1 rows, the others base.
__device__ __forceinline__ int gate_up_row(int r, int kind, int base, int extra) {
  const int big = extra * (base + 1);
  int r0, count;
  if (r < big) {
    r0 = r / (base + 1) * (base + 1);
    count = base + 1;
  } else {
    r0 = big + (r - big) / base * base;
    count = base;
  }
  return 2 * r0 + kind * count + (r - r0);
}

// One wave owns a (16 TR) x (16 TF) tile of 16x16 MFMA tiles; a workgroup
// (4 waves, 2 x 2) owns (32 TR) x (32 TF). SwiGLU workgroups hold 16 TR gate
// rows (waves 0 and 2) and the matching 16 TR up rows (waves 1 and 3).
// Operands move through LDS in stages of four blocks (128 bytes of every
// tile row, 16 bytes a lane): the next stage's global loads are in flight in
// registers while the current stage is computed, then written to the other
// LDS buffer. The 16-byte chunk c of tile row t sits at slot c ^ (t & 7), so
// that the 16 rows of an MFMA operand read spread over the banks.
constexpr int kStages = 2;
constexpr int kStageBlocks = 4;

template <class Scale, int OUT, int TR, int TF>
__global__ __launch_bounds__(kGT) void q8_gemm_kernel(GemmArgs g) {
  extern __shared__ __attribute__((aligned(16))) float gemm_s[];
  constexpr bool kSwiGLU = OUT == kGemmSwiGLU;
  constexpr int RW = 16 * TR, FW = 16 * TF;  // wave tile
  constexpr int RT = 2 * RW, FT = 2 * FW;    // workgroup tile (SwiGLU: gate rows then up rows)
  constexpr int LR = kSwiGLU ? RW : RT;      // logical rows per workgroup
  constexpr int US = LR + 4;                 // up_s row stride (floats)
  constexpr int kRowBytes = 32 * kStageBlocks;
  // A stage: operand rows [RT + FT][128 B], then the stage's scales as fp32,
  // [4][RT] for the rows and [4][FT] for the frames.
  constexpr int kOperandBytes = (RT + FT) * kRowBytes;
  constexpr int kStageBytes = kOperandBytes + (RT + FT) * kStageBlocks * 4;
  const int B = g.K >> 5;
  char* stage_s = reinterpret_cast<char*>(gemm_s);                                 // [kStages][kStageBytes]
  float* up_s = reinterpret_cast<float*>(stage_s + kStages * kStageBytes);         // SwiGLU: [FT][US] up sums
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wr = wave & 1, wf = wave >> 1;
  const int row0 = blockIdx.x * LR, f0 = blockIdx.y * FT;
  // Tile row tr (0..RT-1) -> storage row, or -1 past the end.
  auto storage_row = [&](int tr) -> int {
    if (kSwiGLU) {
      const int r = row0 + tr % RW;
      if (r >= g.rows) return -1;
      return g.gu_map ? g.gu_map[2 * r + tr / RW] : gate_up_row(r, tr / RW, g.split_base, g.split_extra);
    }
    const int r = row0 + tr;
    return r < g.rows ? r : -1;
  };

  // Stage loads: piece j of a stage is tile rows 8j..8j+7 (rows [0, RT) are
  // weight rows, [RT, RT + FT) frames); lane l takes row 8j + l/8, chunk
  // (l%8) ^ (row & 7), and writes it to slot l%8. Threads [0, RT) also take
  // their row's four block scales, threads [RT, RT + FT) their frame's. Rows
  // past the matrix and frames past the input load row / frame 0 (scale 0):
  // never stored.
  constexpr int kLoads = (RT + FT) / 8;
  static_assert(kLoads % 4 == 0, "every wave moves the same number of pieces");
  static_assert(RT + FT <= kGT, "one scale load per thread");
  constexpr int kPerWave = kLoads / 4;
  const int8_t* src[kPerWave];
#pragma unroll
  for (int i = 0; i < kPerWave; ++i) {
    const int t = 8 * (wave + 4 * i) + (lane >> 3);
    const int chunk = (lane & 7) ^ (t & 7);
    if (t < RT) {
      const int sr = storage_row(t);
      src[i] = g.w + (size_t)max(sr, 0) * g.K + 16 * chunk;
    } else {
      const int f = f0 + t - RT;
      src[i] = g.xq + (size_t)(f < g.frames ? f : 0) * g.K + 16 * chunk;
    }
  }
  // Scales of a stage: thread t takes block t % 4 of row t / 4 and of frame
  // t / 4 (rows and frames past the tile or the matrix read row / frame 0,
  // and past the matrix store scale 0).
  using ST = typename Scale::type;
  static_assert(RT <= 64 && FT <= 64, "one row scale and one frame scale per thread");
  const int sblk = tid & 3, srow = tid >> 2;
  const int s_sr = srow < RT ? storage_row(srow) : -1;
  const int s_f = f0 + srow;
  const bool row_live = s_sr >= 0, frame_live = srow < FT && s_f < g.frames;
  const ST* wsrc = reinterpret_cast<const ST*>(g.ws) + (size_t)max(s_sr, 0) * B + sblk;
  const float* xsrc = g.xs + (size_t)(frame_live ? s_f : 0) * B + sblk;
  v4i pending[kPerWave];
  ST wraw;
  float xraw;
  auto fetch = [&](int st) {  // stage st: blocks [4 st, 4 st + 4)
#pragma unroll
    for (int i = 0; i < kPerWave; ++i) pending[i] = *reinterpret_cast<const v4i*>(src[i] + (size_t)st * kRowBytes);
    wraw = wsrc[kStageBlocks * st];
    xraw = xsrc[kStageBlocks * st];
  };
  auto put = [&](int st) {
    char* base = stage_s + (st % kStages) * kStageBytes;
#pragma unroll
    for (int i = 0; i < kPerWave; ++i) *reinterpret_cast<v4i*>(base + (wave + 4 * i) * 1024 + 16 * lane) = pending[i];
    float* sc = reinterpret_cast<float*>(base + kOperandBytes);  // [4][RT] rows, then [4][FT] frames
    if (srow < RT) sc[sblk * RT + srow] = row_live ? Scale::get(wraw) : 0.0f;
    if (srow < FT) sc[kStageBlocks * RT + sblk * FT + srow] = frame_live ? xraw : 0.0f;
  };
  const int stages = B / kStageBlocks;
  fetch(0);
  put(0);
  fetch(min(1, stages - 1));
  lds_barrier();

  // MFMA operand of lane l: 8 bytes of row (frame) l % 16 at byte 8 (l / 16)
  // of the block; result register j of lane l: row 4 (l / 16) + j, frame l % 16.
  const int l16 = lane & 15, kq = lane >> 4;
  int a_at[TR], b_at[TF];  // byte offsets of this lane's operand rows in a stage
#pragma unroll
  for (int tr = 0; tr < TR; ++tr) a_at[tr] = (wr * RW + 16 * tr + l16) * kRowBytes;
#pragma unroll
  for (int tf = 0; tf < TF; ++tf) b_at[tf] = (RT + wf * FW + 16 * tf + l16) * kRowBytes;
  // Chunk 2 blk + kq/2 of row t sits at slot (2 blk + kq/2) ^ (t & 7); every
  // operand row of this lane has t & 7 == l16 & 7.
  auto at = [&](int row_at, int blk) { return row_at + 16 * ((2 * blk + (kq >> 1)) ^ (l16 & 7)) + 8 * (kq & 1); };
  const v4i zero4 = {0, 0, 0, 0};
  float acc[TR][TF][4];
#pragma unroll
  for (int tr = 0; tr < TR; ++tr)
#pragma unroll
    for (int tf = 0; tf < TF; ++tf)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[tr][tf][j] = 0.0f;

  for (int st = 0; st < stages; ++st) {
    const char* sa = stage_s + (st % kStages) * kStageBytes;
    const float* ws_s = reinterpret_cast<const float*>(sa + kOperandBytes);  // [4][RT]
    const float* xs_s = ws_s + kStageBlocks * RT;                           // [4][FT]
    // Four-tile waves keep two blocks in flight (fewer registers, more waves
    // a SIMD); single-tile waves all four.
    constexpr int kBlkUnroll = TR * TF >= 4 ? 2 : kStageBlocks;
#pragma unroll kBlkUnroll
    for (int blk = 0; blk < kStageBlocks; ++blk) {
      long av[TR], bv[TF];
#pragma unroll
      for (int tr = 0; tr < TR; ++tr) av[tr] = *reinterpret_cast<const long*>(sa + at(a_at[tr], blk));
#pragma unroll
      for (int tf = 0; tf < TF; ++tf) bv[tf] = *reinterpret_cast<const long*>(sa + at(b_at[tf], blk));
      v4i d[TR][TF];
#pragma unroll
      for (int tr = 0; tr < TR; ++tr)
#pragma unroll
        for (int tf = 0; tf < TF; ++tf) d[tr][tf] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[tr], bv[tf], zero4, 0, 0, 0);
      // The reference's ((float)dot * w_scale) * x_scale, added in block order.
      float4 w4[TR];
      float xv[TF];
#pragma unroll
      for (int tr = 0; tr < TR; ++tr) w4[tr] = *reinterpret_cast<const float4*>(ws_s + blk * RT + wr * RW + 16 * tr + 4 * kq);
#pragma unroll
      for (int tf = 0; tf < TF; ++tf) xv[tf] = xs_s[blk * FT + wf * FW + 16 * tf + l16];
#pragma unroll
      for (int tr = 0; tr < TR; ++tr)
#pragma unroll
        for (int tf = 0; tf < TF; ++tf) {
          acc[tr][tf][0] = fadd(acc[tr][tf][0], fmul(fmul((float)d[tr][tf][0], w4[tr].x), xv[tf]));
          acc[tr][tf][1] = fadd(acc[tr][tf][1], fmul(fmul((float)d[tr][tf][1], w4[tr].y), xv[tf]));
          acc[tr][tf][2] = fadd(acc[tr][tf][2], fmul(fmul((float)d[tr][tf][2], w4[tr].z), xv[tf]));
          acc[tr][tf][3] = fadd(acc[tr][tf][3], fmul(fmul((float)d[tr][tf][3], w4[tr].w), xv[tf]));
        }
    }
    // Stage st + 1 into the other buffer (last read at stage st - 1, before
    // the previous barrier), then stage st + 2's loads into the registers
    // (past the last stage: the last one again, unused).
    put(st + 1);
    fetch(min(st + 2, stages - 1));
    lds_barrier();
  }

  if (!kSwiGLU) {
#pragma unroll
    for (int tf = 0; tf < TF; ++tf) {
      const int f = f0 + wf * FW + 16 * tf + l16;
      if (f >= g.frames) continue;
#pragma unroll
      for (int tr = 0; tr < TR; ++tr) {
        const int r = row0 + wr * RW + 16 * tr + 4 * kq;
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[j] = acc[tr][tf][j];
          if (r + j < g.rows) {
            if (OUT == kGemmResidual) v[j] = fadd(v[j], g.resid[(size_t)f * g.out_stride + r + j]);
            if (OUT == kGemmPlain && g.bias) v[j] = fadd(g.bias[r + j], v[j]);
          }
        }
        float* o = g.out + (size_t)f * g.out_stride + r;
        if (r + 3 < g.rows && ((g.out_stride | r) & 3) == 0) {
          *reinterpret_cast<float4*>(o) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (r + j < g.rows) o[j] = v[j];
        }
      }
    }
  } else {
    // SwiGLU (Elementwise.cs:167-196): gate waves meet their up rows in LDS.
    if (wr == 1) {
#pragma unroll
      for (int tf = 0; tf < TF; ++tf)
#pragma unroll
        for (int tr = 0; tr < TR; ++tr)
          *reinterpret_cast<float4*>(up_s + (wf * FW + 16 * tf + l16) * US + 16 * tr + 4 * kq) =
              make_float4(acc[tr][tf][0], acc[tr][tf][1], acc[tr][tf][2], acc[tr][tf][3]);
    }
    lds_barrier();
    if (wr == 0) {
#pragma unroll
      for (int tf = 0; tf < TF; ++tf) {
        const int f = f0 + wf * FW + 16 * tf + l16;
        float h[TR][4];
#pragma unroll
        for (int tr = 0; tr < TR; ++tr) {
          const float4 u = *reinterpret_cast<const float4*>(up_s + (wf * FW + 16 * tf + l16) * US + 16 * tr + 4 * kq);
          const float uj[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float gv = acc[tr][tf][j];
            const float silu = fdiv(gv, fadd(1.0f, exp_ref(-gv)));
            h[tr][j] = fmul(silu, uj[j]);
          }
        }
        if (TR == 2 && g.out_q) {
          // The 32 rows of the workgroup are one Q8_0 block of frame f, held
          // by lanes l16, l16 + 16, l16 + 32, l16 + 48 (eight values each):
          // TensorMath.Quantize of the block (amax over the bit patterns).
          uint32_t m = 0;
#pragma unroll
          for (int tr = 0; tr < TR; ++tr)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const uint32_t a = f2u(h[tr][j]) & 0x7fffffffu;
              m = a > m ? a : m;
            }
          uint32_t o = (uint32_t)__shfl_xor((int)m, 16);
          m = o > m ? o : m;
          o = (uint32_t)__shfl_xor((int)m, 32);
          m = o > m ? o : m;
          float inverse;
          const float d = block_scale(m, &inverse);
          if (f < g.frames) {
            int8_t* q = g.out_q + (size_t)f * g.rows + row0 + 4 * kq;
#pragma unroll
            for (int tr = 0; tr < TR; ++tr) {
              const uint32_t packed = (uint32_t)(uint8_t)quantize_value(h[tr][0], inverse) |
                                      ((uint32_t)(uint8_t)quantize_value(h[tr][1], inverse) << 8) |
                                      ((uint32_t)(uint8_t)quantize_value(h[tr][2], inverse) << 16) |
                                      ((uint32_t)(uint8_t)quantize_value(h[tr][3], inverse) << 24);
              *reinterpret_cast<uint32_t*>(q + 16 * tr) = packed;
            }
            if (kq == 0) g.out_s[(size_t)f * (g.rows / 32) + row0 / 32] = d;
          }
        } else if (f < g.frames) {
#pragma unroll
          for (int tr = 0; tr < TR; ++tr) {
            const int r = row0 + 16 * tr + 4 * kq;
#pragma unroll
            for (int j = 0; j < 4; ++j)
              if (r + j < g.rows) g.out[(size_t)f * g.out_stride + r + j] = h[tr][j];
          }
        }
      }
    }
  }
}

// RMSNorm (when norm_w is set) and activation quantisation of one row per
// workgroup: the GEMV prologue's arithmetic (TensorMath.Elementwise.cs:26-100,
// TensorMath.cs:378-412), four values per thread per 1024-value chunk.
__global__ __launch_bounds__(256) void norm_quantize_rows_kernel(const float* x, int K, const float* norm_w, float eps,
                                                                 int8_t* xq, float* xs) {
  __shared__ double red_s[4];
  constexpr int kChunks = 4;  // K <= 4096
  const int frame = blockIdx.x, tid = threadIdx.x;
  const float* row = x + (size_t)frame * K;
  float4 v[kChunks];
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int e = c * 1024 + 4 * tid;
    v[c] = e < K ? *reinterpret_cast<const float4*>(row + e) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  if (norm_w) {
    double sq = 0.0;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      sq += (double)v[c].x * (double)v[c].x + (double)v[c].y * (double)v[c].y;
      sq += (double)v[c].z * (double)v[c].z + (double)v[c].w * (double)v[c].w;
    }
    const float inverse = rms_inverse(block_sum_double(sq, red_s), K, eps, [&](int k) { return row[k]; });
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      const int e = c * 1024 + 4 * tid;
      if (e < K) {
        const float4 w = *reinterpret_cast<const float4*>(norm_w + e);
        v[c].x = fmul(fmul(v[c].x, inverse), w.x);
        v[c].y = fmul(fmul(v[c].y, inverse), w.y);
        v[c].z = fmul(fmul(v[c].z, inverse), w.z);
        v[c].w = fmul(fmul(v[c].w, inverse), w.w);
      }
    }
  }
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int e = c * 1024 + 4 * tid;
    if (e < K) {
      float d;
      const int packed = quantize4(v[c].x, v[c].y, v[c].z, v[c].w, &d);
      *reinterpret_cast<int*>(xq + (size_t)frame * K + e) = packed;
      if ((tid & 7) == 0) xs[(size_t)frame * (K >> 5) + (e >> 5)] = d;
    }
  }
}

// Causal attention of one query head for one frame (row t at position
// p + t sees positions [0, p + t]): scores one position per lane (eight
// channel-strided accumulators and their pairwise tree), exact softmax with
// a double denominator, time-ordered value sums one lane per channel --
// the decode arithmetic (AttentionAvx.cs:74-224, SoftmaxAvx.cs:11-58) applied
// per row, as the oracle restates the prefill path (QwenDecoder.cs:206-224).
__global__ __launch_bounds__(256) void attn_prefill_kernel(PrefillAttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) float attn_s[];  // probabilities [n]
  __shared__ __attribute__((aligned(16))) float q_s[128];
  __shared__ __attribute__((aligned(16))) _Float16 kcur_s[128];  // fused QK: this position's K and V rows
  __shared__ _Float16 vcur_s[128];
  __shared__ float y_s[2][128];
  __shared__ double red_s[4];
  __shared__ float tmax_s[4];
  __shared__ double lane_s[8];
  __shared__ float inv_s;
  __shared__ int exact_s[4];
  const int head = blockIdx.x, t = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hs = 128, group = a.heads / a.kv_heads, kh = head / group;
  const bool fused = a.qkv != nullptr;
  int pos, capacity;
  const _Float16 *kcache, *vcache;
  const float *rope_cos = nullptr, *rope_sin = nullptr;
  if (a.sessions) {
    const SessionRef& ss = a.sessions[t];
    pos = min(*ss.position, a.max_positions - 1);
    capacity = ss.capacity;
    const size_t layer = (size_t)a.layer * a.kv_heads * capacity * hs;
    kcache = ss.kcache + layer;
    vcache = ss.vcache + layer;
    rope_cos = ss.rope_cos;
    rope_sin = ss.rope_sin;
  } else {
    pos = a.position + t;
    capacity = a.capacity;
    kcache = a.kcache;
    vcache = a.vcache;
  }
  const int n = pos + 1;
  const int nv = fused ? pos : n;  // K/V rows read from the cache (fused: this position's are local)
  const _Float16* kc = kcache + (size_t)kh * capacity * hs;
  const _Float16* vc = vcache + (size_t)kh * capacity * hs;
  float* p_s = attn_s;
  // V rows [0, nv) into LDS (direct global->LDS loads, 1 KiB = 4 rows per
  // instruction), in flight while the scores are computed.
  char* v_s = reinterpret_cast<char*>(attn_s) + ((4 * a.stage + 15) & ~15);
  if (a.stage) {
    const char* src = reinterpret_cast<const char*>(vc);
    const int bytes = nv * hs * 2;
    for (int c = wave * 1024; c < bytes; c += 4 * 1024)
      if (c + 16 * lane < bytes) __builtin_amdgcn_global_load_lds(src + c + 16 * lane, (lds_ptr)(v_s + c), 16, 0, 0);
  }
  // The K row of this thread's first position, requested now so that its
  // latency passes during the q/k preparation.
  uint4 k0[16];
  if (tid < nv) {
    const uint4* row = reinterpret_cast<const uint4*>(kc + (size_t)tid * hs);
#pragma unroll
    for (int i = 0; i < 16; ++i) k0[i] = row[i];
  }
  if (fused) {
    // QK-norm and RoPE of this head's q (threads 0-127) and of its KV head's
    // k (128-255), v rounded to F16: qk_prepare_kernel's arithmetic
    // (QwenDecoder.cs:186-203, Rope.cs:14-55). The first query head of the
    // pair writes the K/V row; both keep it locally for this position. The
    // norm weight and the RoPE factors are loaded with the raw value.
    const int part = tid >> 7, c = tid & 127, half = hs >> 1;
    const float* raw = a.qkv + (size_t)t * (a.q_width + 2 * a.kv_width);
    const float v = raw[part == 0 ? head * hs + c : a.q_width + kh * hs + c];
    const float nw = (part == 0 ? a.q_norm : a.k_norm)[c];
    const float cs = rope_cos[(size_t)pos * half + (c & (half - 1))];
    const float sn = rope_sin[(size_t)pos * half + (c & (half - 1))];
    const double sq = wave_sum_double((double)v * (double)v);
    if (lane == 0) red_s[wave] = sq;
    lds_barrier();
    const float* src = raw + (part == 0 ? head * hs : a.q_width + kh * hs);
    const float inverse =
        rms_inverse(red_s[2 * part] + red_s[2 * part + 1], hs, a.eps, [&](int k) { return src[k]; });
    y_s[part][c] = fmul(fmul(v, inverse), nw);
    lds_barrier();
    float r;
    if (c < half) r = fadd(fmul(y_s[part][c], cs), -fmul(y_s[part][c + half], sn));
    else r = fadd(fmul(y_s[part][c - half], sn), fmul(y_s[part][c], cs));
    if (part == 0) {
      q_s[c] = r;
      const _Float16 v16 = to_half(raw[a.q_width + a.kv_width + kh * hs + c]);
      vcur_s[c] = v16;
      if (head % group == 0) const_cast<_Float16*>(vc)[(size_t)pos * hs + c] = v16;
    } else {
      const _Float16 k16 = to_half(r);
      kcur_s[c] = k16;
      if (head % group == 0) const_cast<_Float16*>(kc)[(size_t)pos * hs + c] = k16;
    }
  } else if (tid < hs) {
    q_s[tid] = a.q[((size_t)t * a.heads + head) * hs + tid];
  }
  lds_barrier();

  if (tid < nv) {
    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 16; ++i) score8(acc, k0[i], q_s + 8 * i);
    const float sc = fadd(fadd(fadd(acc[0], acc[4]), fadd(acc[1], acc[5])), fadd(fadd(acc[2], acc[6]), fadd(acc[3], acc[7])));
    p_s[tid] = fdiv(sc, a.divisor);
  }
  for (int s = tid < nv ? tid + 256 : tid; s < n; s += 256) {
    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    if (s < nv) {
      const uint4* row = reinterpret_cast<const uint4*>(kc + (size_t)s * hs);
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
    const float sc = fadd(fadd(fadd(acc[0], acc[4]), fadd(acc[1], acc[5])), fadd(fadd(acc[2], acc[6]), fadd(acc[3], acc[7])));
    p_s[s] = fdiv(sc, a.divisor);
  }
  lds_barrier();
  float m = -__builtin_inff();
  for (int s = tid; s < n; s += 256) m = nan_max_p(m, p_s[s]);
  m = wave_max_nan(m);
  if (lane == 0) tmax_s[wave] = m;
  lds_barrier();
  const float mx = nan_max_p(nan_max_p(tmax_s[0], tmax_s[1]), nan_max_p(tmax_s[2], tmax_s[3]));
  // The numerators; when each is 0 or in [2^-17, 1] and there are fewer
  // than 8192, every partial sum of them is an exact double, so their wave
  // trees give the reference's in-order sum bit for bit. Otherwise the
  // reference's order: eight residue chains, their pairwise tree, the tail.
  double dpart = 0.0;
  bool dexact = n < 8192;
  for (int s = tid; s < n; s += 256) {
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
      lane_s[tid] = acc;
    }
    lds_barrier();
    if (tid == 0) {
      double sum = ((lane_s[0] + lane_s[4]) + (lane_s[1] + lane_s[5])) + ((lane_s[2] + lane_s[6]) + (lane_s[3] + lane_s[7]));
      for (int s = full; s < n; ++s) sum = sum + (double)p_s[s];
      inv_s = (float)(1.0 / sum);
    }
    lds_barrier();
    inverse = inv_s;
  }
  for (int s = tid; s < n; s += 256) p_s[s] = fmul(p_s[s], inverse);
  if (a.stage) __builtin_amdgcn_s_waitcnt(0);  // this wave's V rows are in LDS
  lds_barrier();
  if (tid < hs && a.stage) {
    const _Float16* v = reinterpret_cast<const _Float16*>(v_s) + tid;
    float acc = 0.0f;
    int s = 0;
    for (; s + 16 <= nv; s += 16) {
      _Float16 x[16];
#pragma unroll
      for (int k = 0; k < 16; ++k) x[k] = v[(s + k) * hs];
#pragma unroll
      for (int k = 0; k < 16; ++k) acc = fadd(acc, mulh(p_s[s + k], x[k]));
    }
    for (; s < nv; ++s) acc = fadd(acc, mulh(p_s[s], v[s * hs]));
    if (fused) acc = fadd(acc, mulh(p_s[pos], vcur_s[tid]));
    if (a.out) a.out[((size_t)t * a.heads + head) * hs + tid] = acc;
    q_s[tid] = acc;
  } else if (tid < hs) {
    const _Float16* v = vc + tid;
    float acc = 0.0f;
    int s = 0;
    for (; s + 16 <= nv; s += 16) {
      _Float16 x[16];
#pragma unroll
      for (int k = 0; k < 16; ++k) x[k] = v[(size_t)(s + k) * hs];
#pragma unroll
      for (int k = 0; k < 16; ++k) acc = fadd(acc, mulh(p_s[s + k], x[k]));
    }
    for (; s < nv; ++s) acc = fadd(acc, mulh(p_s[s], v[(size_t)s * hs]));
    if (fused) acc = fadd(acc, mulh(p_s[pos], vcur_s[tid]));
    if (a.out) a.out[((size_t)t * a.heads + head) * hs + tid] = acc;
    q_s[tid] = acc;
  }
  if (a.xq) {
    // Q8_0 blocks of this head's output (32 channels each, 8 lanes x 4).
    lds_barrier();
    if (tid < hs / 4) {
      const float4 v4 = *reinterpret_cast<const float4*>(q_s + 4 * tid);
      float d;
      const int packed = quantize4(v4.x, v4.y, v4.z, v4.w, &d);
      const size_t row = (size_t)t * a.heads * hs + (size_t)head * hs;
      *reinterpret_cast<int*>(a.xq + row + 4 * tid) = packed;
      if ((tid & 7) == 0) a.xs[row / 32 + tid / 8] = d;
    }
  }
}

// Few-frame Q8_0 GEMM (lock-step sessions, short prefills): the same
// per-row block order as q8_gemm_kernel, for frames <= kFewFrames, with a
// few rows per workgroup so that even the 1024-row projections spread over
// the whole chip. Each lane takes (row, block) pairs, consecutive lanes
// consecutive blocks of a row (coalesced 32-byte weight loads, issued before
// the activations are staged); for every frame it forms the exact int32
// block dot (v_dot4_i32_i8 x 8) and the term (float)dot * w_scale * x_scale
// into LDS; then one lane per (row, frame) adds the terms in block order
// from 0f and applies the epilogue. LDS: activations [frames][K], their
// scales [frames][B], terms [slots][frames][B + 4].
constexpr int kFewThreads = 256;
constexpr int kFewPairs = 4;  // (row, block) pairs per lane
constexpr int kFewMaxK = 3072;
constexpr size_t kFewLds = 80 * 1024;  // two workgroups per CU

__host__ __device__ inline size_t few_lds_bytes(int slots, int K, int frames) {
  const int B = K / 32;
  return (size_t)frames * K + (size_t)frames * B * 4 + (size_t)slots * frames * (B + 4) * 4 +
         (size_t)frames * 8;
}

template <class Scale, int OUT>
__global__ __launch_bounds__(kFewThreads) void q8_gemm_few_kernel(GemmArgs g, int R) {
  extern __shared__ __attribute__((aligned(16))) char few_s[];
  constexpr bool kSwiGLU = OUT == kGemmSwiGLU;
  const int K = g.K, B = K >> 5, S = g.frames, TB = B + 4, tid = threadIdx.x;
  const int slots = kSwiGLU ? 2 * R : R;
  const int r0 = blockIdx.x * R;
  int8_t* x_s = reinterpret_cast<int8_t*>(few_s);                          // [S][K]
  float* xs_s = reinterpret_cast<float*>(few_s + (size_t)S * K);           // [S][B]
  float* t_s = xs_s + S * B;                                               // [slots][S][TB]
  unsigned long long* key_s = reinterpret_cast<unsigned long long*>(t_s + (size_t)slots * S * TB);  // [S]
  // Storage row of slot i (SwiGLU: slots [0,R) gate rows, [R,2R) up rows).
  auto storage_row = [&](int i) -> int {
    if (kSwiGLU) {
      const int p = r0 + (i < R ? i : i - R);
      if (p >= g.rows) return -1;
      return g.gu_map ? g.gu_map[2 * p + (i < R ? 0 : 1)] : gate_up_row(p, i < R ? 0 : 1, g.split_base, g.split_extra);
    }
    const int r = r0 + i;
    return r < g.rows ? r : -1;
  };
  const typename Scale::type* ws = reinterpret_cast<const typename Scale::type*>(g.ws);
  // Lane -> (row step, block): every lane keeps one block b for all its rows,
  // so one LDS read of a frame's activation block serves kFewPairs rows.
  const int RS = kFewThreads / B;  // rows per step
  const int lrow = tid / B, b = tid - lrow * B;
  const bool active = lrow < RS;
  // Activations and their scales go to LDS by direct global->LDS loads,
  // issued together with the weight loads; one wait covers both.
  {
    const int wave = tid >> 6, lane = tid & 63;
    const char* src = reinterpret_cast<const char*>(g.xq);
    const int xbytes = S * K;
    for (int c = wave * 1024; c < xbytes; c += 4 * 1024)
      if (c + 16 * lane < xbytes)
        __builtin_amdgcn_global_load_lds(src + c + 16 * lane, (lds_ptr)(few_s + c), 16, 0, 0);
    const char* ssrc = reinterpret_cast<const char*>(g.xs);
    char* sdst = reinterpret_cast<char*>(xs_s);
    const int sbytes = S * B * 4;
    for (int c = wave * 1024; c < sbytes; c += 4 * 1024)
      if (c + 16 * lane < sbytes)
        __builtin_amdgcn_global_load_lds(ssrc + c + 16 * lane, (lds_ptr)(sdst + c), 16, 0, 0);
    if (OUT == kGemmGreedy && tid < S) key_s[tid] = 0ull;
  }
  uint4 w0[kFewPairs], w1[kFewPairs];
  float wsc[kFewPairs];
#pragma unroll
  for (int k = 0; k < kFewPairs; ++k) {
    // Unconditional loads (row clamped into the matrix); rows past the tile
    // or the matrix are never summed.
    const int i = lrow + RS * k;
    const int sr = max(0, active && i < slots ? storage_row(i) : 0);
    const uint4* wp = reinterpret_cast<const uint4*>(g.w + (size_t)sr * K + 32 * b);
    w0[k] = wp[0];
    w1[k] = wp[1];
    wsc[k] = Scale::get(ws[(size_t)sr * B + b]);
  }
  __builtin_amdgcn_s_waitcnt(0);
  lds_barrier();
  if (active) {
    for (int f = 0; f < S; ++f) {
      const uint4* xp = reinterpret_cast<const uint4*>(x_s + (size_t)f * K + 32 * b);
      const uint4 x0 = xp[0], x1 = xp[1];
      const float xsv = xs_s[f * B + b];
#pragma unroll
      for (int k = 0; k < kFewPairs; ++k) {
        const int i = lrow + RS * k;
        if (i < slots) {
          int dot = 0;
          dot = __builtin_amdgcn_sdot4((int)w0[k].x, (int)x0.x, dot, false);
          dot = __builtin_amdgcn_sdot4((int)w0[k].y, (int)x0.y, dot, false);
          dot = __builtin_amdgcn_sdot4((int)w0[k].z, (int)x0.z, dot, false);
          dot = __builtin_amdgcn_sdot4((int)w0[k].w, (int)x0.w, dot, false);
          dot = __builtin_amdgcn_sdot4((int)w1[k].x, (int)x1.x, dot, false);
          dot = __builtin_amdgcn_sdot4((int)w1[k].y, (int)x1.y, dot, false);
          dot = __builtin_amdgcn_sdot4((int)w1[k].z, (int)x1.z, dot, false);
          dot = __builtin_amdgcn_sdot4((int)w1[k].w, (int)x1.w, dot, false);
          t_s[((size_t)i * S + f) * TB + b] = fmul(fmul((float)dot, wsc[k]), xsv);
        }
      }
    }
  }
  lds_barrier();
  // Ordered block sums: one lane per (row, frame).
  auto row_sum = [&](int i, int f) {
    const float* t = t_s + ((size_t)i * S + f) * TB;
    float sum = 0.0f;
    int b = 0;
    for (; b + 4 <= B; b += 4) {
      const float4 v = *reinterpret_cast<const float4*>(t + b);
      sum = fadd(sum, v.x);
      sum = fadd(sum, v.y);
      sum = fadd(sum, v.z);
      sum = fadd(sum, v.w);
    }
    for (; b < B; ++b) sum = fadd(sum, t[b]);
    return sum;
  };
  for (int t = tid; t < R * S; t += kFewThreads) {
    const int i = t / S, f = t - i * S, r = r0 + i;
    if (r >= g.rows) continue;
    float v = row_sum(i, f);
    if (kSwiGLU) {
      // SwiGLU (Elementwise.cs:167-196).
      const float u = row_sum(R + i, f);
      v = fmul(fdiv(v, fadd(1.0f, exp_ref(-v))), u);
    } else if (OUT == kGemmResidual) {
      v = fadd(v, g.resid[(size_t)f * g.out_stride + r]);
    } else if (g.bias) {
      v = fadd(g.bias[r], v);
    }
    g.out[(size_t)f * g.out_stride + r] = v;
    if (OUT == kGemmGreedy) atomicMax(&key_s[f], greedy_key(v, (uint32_t)r));
  }
  if (OUT == kGemmGreedy) {
    lds_barrier();
    if (tid < S) g.keys[(size_t)tid * gridDim.x + blockIdx.x] = key_s[tid];
  }
}

// The lm_head of 8 to 16 frames (lock-step sessions): each wave takes
// tiles of 16 rows and all frames, one v_mfma_i32_16x16x32_i8 per block
// with the frames' activations as the A operand and the tile's weights as B
// (lane l: 8 bytes of frame / row l % 16 at byte 8 (l / 16) of the block),
// so that result register j of lane l is the exact int32 block dot of
// frame 4 (l / 16) + j and row l % 16. Each lane adds its four terms
// ((float)dot * w_scale) * x_scale in block order from 0f in registers: the
// row sums of q8_gemm_few_kernel, bit for bit. The frames' activations are
// staged in LDS once per workgroup (rows padded by 16 bytes, so that the 16
// frames of an operand read spread over the banks), their block scales
// transposed to [block][frame]. The weights come straight from memory, each
// lane the 8-byte pieces of its row, 16 blocks a step, the next step's
// (the next tile's first, at a tile's end) requested before the current
// one is used. Per frame, the greedy key of the workgroup's rows.
constexpr int kM16MaxK = 3072;
constexpr int kM16Waves = 4;
constexpr int kM16MaxGroups = 1024;

__host__ __device__ inline size_t m16_lds_bytes(int K) {
  return (size_t)16 * (K + 16) + (size_t)(K / 32) * 16 * 4 + 16 * 8;
}

template <class Scale>
__global__ __launch_bounds__(64 * kM16Waves) void q8_head_mfma16_kernel(GemmArgs g, int tiles) {
  extern __shared__ __attribute__((aligned(16))) char m16_s[];
  const int K = g.K, B = K >> 5, S = g.frames, XR = K + 16;
  int8_t* x_s = reinterpret_cast<int8_t*>(m16_s);                                    // [16][XR]
  float* xs_s = reinterpret_cast<float*>(m16_s + (size_t)16 * XR);                   // [B][16]
  unsigned long long* key_s = reinterpret_cast<unsigned long long*>(xs_s + B * 16);  // [16]
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l16 = lane & 15, kq = lane >> 4;
  const typename Scale::type* ws = reinterpret_cast<const typename Scale::type*>(g.ws);
  const int stride = gridDim.x * kM16Waves;
  int t = blockIdx.x * kM16Waves + wave;
  // One step's weights: 16 blocks from block b0 of tile tt (row clamped into
  // the matrix; rows past the end are never written).
  auto load = [&](int tt, int b0, long* wv, float* wsv) {
    const int sr = min(16 * tt + l16, g.rows - 1);
    const int8_t* wrow = g.w + (size_t)sr * K + 8 * kq + 32 * b0;
    const typename Scale::type* wsr = ws + (size_t)sr * B + b0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      wv[i] = *reinterpret_cast<const long*>(wrow + 32 * i);
      wsv[i] = Scale::get(wsr[i]);
    }
  };
  long wa[16], wb[16];
  float sa[16], sb[16];
  if (t < tiles) load(t, 0, wa, sa);
  {
    const char* src = reinterpret_cast<const char*>(g.xq);
    for (int f = wave; f < S; f += kM16Waves)
      for (int c = 0; c < K; c += 1024)
        if (c + 16 * lane < K)
          __builtin_amdgcn_global_load_lds(src + (size_t)f * K + c + 16 * lane, (lds_ptr)(x_s + f * XR + c), 16, 0, 0);
    for (int i = tid; i < S * B; i += 64 * kM16Waves) {
      const int f = i / B, b = i - f * B;
      xs_s[b * 16 + f] = g.xs[i];
    }
    if (tid < 16) key_s[tid] = 0ull;
  }
  __builtin_amdgcn_s_waitcnt(0);
  lds_barrier();
  const v4i zero4 = {0, 0, 0, 0};
  float acc[4];
  auto step = [&](int b0, const long* wv, const float* wsv) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int b = b0 + i;
      const long av = *reinterpret_cast<const long*>(x_s + l16 * XR + 32 * b + 8 * kq);
      const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, wv[i], zero4, 0, 0, 0);
      const float4 xv = *reinterpret_cast<const float4*>(xs_s + b * 16 + 4 * kq);
      acc[0] = fadd(acc[0], fmul(fmul((float)d[0], wsv[i]), xv.x));
      acc[1] = fadd(acc[1], fmul(fmul((float)d[1], wsv[i]), xv.y));
      acc[2] = fadd(acc[2], fmul(fmul((float)d[2], wsv[i]), xv.z));
      acc[3] = fadd(acc[3], fmul(fmul((float)d[3], wsv[i]), xv.w));
    }
  };
  for (; t < tiles; t += stride) {
    acc[0] = acc[1] = acc[2] = acc[3] = 0.0f;
    // Steps in pairs (B is a multiple of 32): buffer a holds block b0,
    // buffer b block b0 + 16; each is refilled one step ahead.
    for (int b0 = 0; b0 < B; b0 += 32) {
      load(t, b0 + 16, wb, sb);
      step(b0, wa, sa);
      if (b0 + 32 < B) load(t, b0 + 32, wa, sa);
      else if (t + stride < tiles) load(t + stride, 0, wa, sa);
      step(b0 + 16, wb, sb);
    }
    const int r = 16 * t + l16;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int f = 4 * kq + j;
      if (f < S && r < g.rows) {
        g.out[(size_t)f * g.out_stride + r] = acc[j];
        atomicMax(&key_s[f], greedy_key(acc[j], (uint32_t)r));
      }
    }
  }
  lds_barrier();
  if (tid < S) g.keys[(size_t)tid * gridDim.x + blockIdx.x] = key_s[tid];
}

// Greedy token of each session's logits row from the per-workgroup keys of
// the few-frame lm_head (QwenDecoder.Greedy, QwenDecoder.cs:278-326: first
// maximum wins, NaN never wins, NaN at index 0 returns 0), into the
// session's token word; then the session's position advances.
__global__ __launch_bounds__(256) void greedy_keys_kernel(const unsigned long long* keys, int groups,
                                                          const float* logits, int vocab,
                                                          const SessionRef* sessions) {
  __shared__ unsigned long long best_s[4];
  const int f = blockIdx.x, tid = threadIdx.x;
  const unsigned long long* k = keys + (size_t)f * groups;
  unsigned long long best = 0ull;
  int i = tid;
  for (; i + 3 * 256 < groups; i += 4 * 256) {
    const unsigned long long a = k[i], b = k[i + 256], c = k[i + 512], d = k[i + 768];
    const unsigned long long ab = a > b ? a : b, cd = c > d ? c : d;
    const unsigned long long m = ab > cd ? ab : cd;
    best = m > best ? m : best;
  }
  for (; i < groups; i += 256) best = k[i] > best ? k[i] : best;
  best = wave_max_u64(best);
  if ((tid & 63) == 0) best_s[tid >> 6] = best;
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; ++w) best = best_s[w] > best ? best_s[w] : best;
    const float first = logits[(size_t)f * vocab];
    const SessionRef& ss = sessions[f];
    *ss.token = (first != first || best == 0ull) ? 0 : (int)greedy_index(best);
    *ss.position = *ss.position + 1;
  }
}

// Causal attention for a block of kRowBlock query rows and both query heads
// of one KV head: 16 (head, row) pairs share every K and V row the block
// reads. Per pair the arithmetic is the decode path's (AttentionAvx.cs:74-224,
// SoftmaxAvx.cs:11-58, per row as QwenDecoder.cs:206-224 does): eight
// channel-strided score accumulators and their pairwise tree, the exact
// softmax with a double denominator, time-ordered value sums; output rows
// quantised to Q8_0 per 32-block.
//
// The products go to the matrix cores: a K = 1 fp32 MFMA
// (v_mfma_f32_16x16x1f32, four 16 x 16 blocks, zero accumulator input) is an
// outer product whose every element is the IEEE product round(a * b) -- the
// reference's fmul, signed zeros included -- so the VALU only runs the adds,
// in the reference's order. Scores: for each channel, the outer product of
// 64 positions' k (one per lane) and the 16 pairs' q; lane l then holds pair
// l % 16 at positions t0 + 16 b + 4 (l / 16) + r (vgpr 4 b + r). Value sums:
// for each position, the outer product of the 16 pairs' probabilities and 64
// channels' v; lane l of value wave w holds channel 64 w + 16 b + l % 16 for
// pair 4 (l / 16) + r. Probabilities are [pair][position] in LDS; V rows
// pass through a two-slot LDS ring filled by waves 2-3 while waves 0-1 add.
constexpr int kRowBlock = 8;
constexpr int kRowPairs = 2 * kRowBlock;
constexpr int kQRow = 132;   // q_s row stride (floats): 16 pair rows on distinct bank groups
constexpr int kVRing = 32;   // V rows per ring slot (8 KB)

// Probability row stride (floats) for nmax positions: whole 64-position
// score passes, plus four so that the 16 pair rows start on distinct banks.
__host__ __device__ inline int rows_p_stride(int nmax) { return ((nmax + 63) & ~63) + 4; }

// Dynamic LDS of attn_rows_kernel: at 750 positions two workgroups fit a CU.
__host__ __device__ inline size_t rows_lds_bytes(int nmax) {
  return (size_t)kRowPairs * rows_p_stride(nmax) * 4 + (size_t)2 * kVRing * 256;
}

__device__ __forceinline__ float max16_nan(float m) {  // over each row of 16 lanes
  m = nan_max_p(m, u2f(dpp_u32<kDppQuadXor1>(f2u(m))));
  m = nan_max_p(m, u2f(dpp_u32<kDppQuadXor2>(f2u(m))));
  m = nan_max_p(m, u2f(dpp_u32<kDppHalfMirror>(f2u(m))));
  return nan_max_p(m, u2f(dpp_u32<kDppMirror>(f2u(m))));
}

typedef float f32x16 __attribute__((ext_vector_type(16)));

// Every element of the 4-block 16 x 16 outer product: round(a * b) exactly.
__device__ __forceinline__ f32x16 outer16(float a, float b) {
  const f32x16 zero = {};
  return __builtin_amdgcn_mfma_f32_16x16x1f32(a, b, zero, 0, 0, 0);
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void attn_rows_kernel(PrefillAttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) float rows_s[];
  __shared__ __attribute__((aligned(16))) float q_s[kRowPairs * kQRow];  // q rows, then output rows
  __shared__ double lane_s[kRowPairs * 8];
  __shared__ float inv_s[kRowPairs];
  // The last row blocks see the most positions: they are dispatched first.
  const int kh = blockIdx.x, r0 = (gridDim.y - 1 - blockIdx.y) * kRowBlock, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6, hs = 128;
  const int rows = min(kRowBlock, a.frames - r0);
  const int n0 = a.position + r0 + 1;  // positions the block's first row sees; row rr sees n0 + rr
  const int nmax = n0 + rows - 1;
  const int PS = rows_p_stride(nmax);
  float* p_s = rows_s;  // [pair][PS]
  char* ring = reinterpret_cast<char*>(rows_s + (size_t)kRowPairs * PS);
  const _Float16* kc = a.kcache + (size_t)kh * a.capacity * hs;
  const _Float16* vc = a.vcache + (size_t)kh * a.capacity * hs;
  for (int i = tid; i < kRowPairs * hs; i += 256) {
    const int pi = i >> 7, c = i & 127, hh = pi >> 3, rr = pi & 7;
    q_s[pi * kQRow + c] = rr < rows ? a.q[((size_t)(r0 + rr) * a.heads + 2 * kh + hh) * hs + c] : 0.0f;
  }
  __syncthreads();

  // 1. Scores, 64 positions per wave pass: lane l loads position t0 + l's K
  // row; per channel one outer product with the pairs' q (pair l % 16's q
  // from LDS), its 16 products added to the channel's accumulator (c % 8) of
  // each (pair, position) the lane holds.
  const int mp = lane & 15, mg = lane >> 4;
  for (int t0 = 64 * wave; t0 < nmax; t0 += 256) {
    const uint4* row = reinterpret_cast<const uint4*>(kc + (size_t)min(t0 + lane, nmax - 1) * hs);
    uint4 kk[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) kk[i] = row[i];
    const float* qrow = q_s + mp * kQRow;
    // Two passes over the row, each with four of the eight accumulators:
    // channels 8i + {0, 1, 4, 5}, then 8i + {2, 3, 6, 7}; the tree
    // ((a0 + a4) + (a1 + a5)) + ((a2 + a6) + (a3 + a7)) is formed half by half.
    f32x16 half[2];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      f32x16 acc[4];  // channels j = 2g, 2g + 1, 2g + 4, 2g + 5
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[u] = f32x16{};
      // Operands of step s = 4 i + u: piece i's channel 8i + {2g, 2g+1, 2g+4, 2g+5}[u].
      auto qload = [&](int i, float* qv) {
        const float2 qa = *reinterpret_cast<const float2*>(qrow + 8 * i + 2 * g);
        const float2 qb = *reinterpret_cast<const float2*>(qrow + 8 * i + 4 + 2 * g);
        qv[0] = qa.x;
        qv[1] = qa.y;
        qv[2] = qb.x;
        qv[3] = qb.y;
      };
      auto kval = [&](int i, int u) {
        const uint32_t w = (u < 2) ? (g ? kk[i].y : kk[i].x) : (g ? kk[i].w : kk[i].z);
        return (float)__builtin_bit_cast(_Float16, (uint16_t)((u & 1) ? w >> 16 : w & 0xffffu));
      };
      // Software pipeline: the next step's outer product is issued before
      // this step's adds, the next piece's q is read a piece ahead.
      float qc[4], qn[4];
      qload(0, qc);
      f32x16 dc = outer16(kval(0, 0), qc[0]);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (i + 1 < 16) qload(i + 1, qn);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          f32x16 dn;
          if (u < 3) dn = outer16(kval(i, u + 1), qc[u + 1]);
          else if (i + 1 < 16) dn = outer16(kval(i + 1, 0), qn[0]);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int v = 0; v < 16; ++v) acc[u][v] = fadd(acc[u][v], dc[v]);
          __builtin_amdgcn_sched_barrier(0);
          dc = dn;
        }
        if (i + 1 < 16) {
#pragma unroll
          for (int u = 0; u < 4; ++u) qc[u] = qn[u];
        }
      }
#pragma unroll
      for (int v = 0; v < 16; ++v) half[g][v] = fadd(fadd(acc[0][v], acc[2][v]), fadd(acc[1][v], acc[3][v]));
    }
    float* prow = p_s + (size_t)mp * PS + t0 + 4 * mg;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      float sc[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int v = 4 * b + r;
        sc[r] = fdiv(fadd(half[0][v], half[1][v]), a.divisor);
      }
      *reinterpret_cast<float4*>(prow + 16 * b) = make_float4(sc[0], sc[1], sc[2], sc[3]);
    }
  }
  __syncthreads();

  // 2. Softmax: 16 lanes per pair, four pairs per wave.
  const int pi = wave * 4 + (lane >> 4), sub = lane & 15;
  const int n = (pi & 7) < rows ? n0 + (pi & 7) : 0;
  float* pp = p_s + (size_t)pi * PS;
  {
    float m = -__builtin_inff();
    for (int t = sub; t < n; t += 16) m = nan_max_p(m, pp[t]);
    m = max16_nan(m);
    for (int t = sub; t < n; t += 16) pp[t] = exp_ref(fadd(pp[t], -m));
  }
  __syncthreads();
  const int full = n & ~7;
  if (sub < 8) {
    // Lane j of the pair: p[j] + p[j+8] + ... in order, in double.
    double l = 0.0;
    int t = sub;
    for (; t + 56 < full; t += 64) {
      float v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = pp[t + 8 * k];
#pragma unroll
      for (int k = 0; k < 8; ++k) l = l + (double)v[k];
    }
    for (; t < full; t += 8) l = l + (double)pp[t];
    lane_s[pi * 8 + sub] = l;
  }
  __syncthreads();
  if (sub == 0 && n > 0) {
    const double* L = lane_s + pi * 8;
    double sum = ((L[0] + L[4]) + (L[1] + L[5])) + ((L[2] + L[6]) + (L[3] + L[7]));
    for (int t = full; t < n; ++t) sum = sum + (double)pp[t];
    inv_s[pi] = (float)(1.0 / sum);
  }
  __syncthreads();
  {
    const float inverse = n > 0 ? inv_s[pi] : 0.0f;
    for (int t = sub; t < n; t += 16) pp[t] = fmul(pp[t], inverse);
  }

  // 3. Time-ordered value sums, all four waves: wave w owns channels
  // 32 w .. 32 w + 31 as two groups of 16. One outer product covers four
  // positions t .. t + 3 (one per 16 x 16 block: the 16 pairs' probabilities
  // at t + b times 16 channels' v at t + b), so lane l holds, for channel
  // 32 w + 16 h + l % 16 and pairs 4 (l / 16) + r, the products of four
  // consecutive positions and adds them in order. V rows pass through a
  // two-slot LDS ring (direct global->LDS loads of 16-byte pieces, the next
  // chunk's issued before this one is added; a slot is refilled only after
  // the barrier that follows its last use).
  const int chunks = (nmax + kVRing - 1) / kVRing;
  auto fill = [&](int j) {  // rows past the last are read again, unused
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int piece = tid + 256 * m, rr = piece >> 4;
      const int row = min(j * kVRing + rr, nmax - 1);
      const char* src = reinterpret_cast<const char*>(vc) + (size_t)row * 256 + 16 * (piece & 15);
      __builtin_amdgcn_global_load_lds(src, (lds_ptr)(ring + (size_t)(j & 1) * kVRing * 256 + 1024 * (4 * m + wave)), 16, 0, 0);
    }
  };
  fill(0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();  // the normalised probabilities and the first V chunk
  float acc[2][4] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
  const float* pa = p_s + (size_t)mp * PS + mg;  // A operand: pair mp at position t + l / 16
  for (int j = 0; j < chunks; ++j) {
    if (j + 1 < chunks) fill(j + 1);
    const _Float16* vr = reinterpret_cast<const _Float16*>(ring + (size_t)(j & 1) * kVRing * 256) + mg * hs + 32 * wave + mp;
    const int t0 = j * kVRing, len = min(kVRing, nmax - t0);
    for (int s = 0; s < len; s += 4) {
      const int t = t0 + s;
      const float av = pa[t];
      const f32x16 d0 = outer16(av, (float)vr[s * hs]);
      const f32x16 d1 = outer16(av, (float)vr[s * hs + 16]);
      if (t + 3 < n0) {  // every row of the block sees all four positions
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            acc[0][r] = fadd(acc[0][r], d0[4 * b + r]);
            acc[1][r] = fadd(acc[1][r], d1[4 * b + r]);
          }
      } else {
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int rr = (4 * mg + r) & 7;  // the pair's row: it sees positions < n0 + rr
            if (t + b < n0 + rr) {
              acc[0][r] = fadd(acc[0][r], d0[4 * b + r]);
              acc[1][r] = fadd(acc[1][r], d1[4 * b + r]);
            }
          }
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

  // 4. Output rows (float and/or Q8_0 blocks): pair 4 mg + r, channel
  // 32 w + 16 h + mp.
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int pq = 4 * mg + r, c = 32 * wave + 16 * h + mp, rr = pq & 7;
      q_s[pq * kQRow + c] = acc[h][r];
      if (a.out && rr < rows) a.out[((size_t)(r0 + rr) * a.heads + 2 * kh + (pq >> 3)) * hs + c] = acc[h][r];
    }
  if (a.xq) {
    __syncthreads();
#pragma unroll
    for (int g0 = 0; g0 < kRowPairs * hs / 4; g0 += 256) {
      const int g = g0 + tid, pq = g >> 5, c4 = (g & 31) * 4, rr = pq & 7;
      const float4 v4 = *reinterpret_cast<const float4*>(q_s + pq * kQRow + c4);
      float d;
      const int packed = quantize4(v4.x, v4.y, v4.z, v4.w, &d);
      if (rr < rows) {
        const size_t at = ((size_t)(r0 + rr) * a.heads + 2 * kh + (pq >> 3)) * hs + c4;
        *reinterpret_cast<int*>(a.xq + at) = packed;
        if ((g & 7) == 0) a.xs[at / 32] = d;
      }
    }
  }
}

template <class Scale, int OUT, int TR, int TF>
static hipError_t launch_gemm_tiles(const GemmArgs& g, hipStream_t s) {
  constexpr int RW = 16 * TR, FW = 16 * TF;
  constexpr int LR = OUT == kGemmSwiGLU ? RW : 2 * RW;
  const size_t lds = (size_t)kStages * (2 * RW + 2 * FW) * (32 + 4) * kStageBlocks +
                     (OUT == kGemmSwiGLU ? (size_t)2 * FW * (LR + 4) * 4 : 0);
  static const hipError_t raised = hipFuncSetAttribute(reinterpret_cast<const void*>(q8_gemm_kernel<Scale, OUT, TR, TF>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  if (raised != hipSuccess) return raised;
  dim3 grid((g.rows + LR - 1) / LR, (g.frames + 2 * FW - 1) / (2 * FW));
  q8_gemm_kernel<Scale, OUT, TR, TF><<<grid, kGT, lds, s>>>(g);
  return hipGetLastError();
}

// Largest wave tile that still gives the chip about two waves per SIMD.
template <class Scale, int OUT>
static hipError_t launch_gemm_out(const GemmArgs& g, hipStream_t s) {
  const long rows = (long)g.rows * (OUT == kGemmSwiGLU ? 2 : 1);
  auto waves = [&](int tr, int tf) { return ((rows + 16 * tr - 1) / (16 * tr)) * ((g.frames + 16 * tf - 1) / (16 * tf)); };
  constexpr long kWant = 2048;
  if (waves(2, 2) >= kWant) return launch_gemm_tiles<Scale, OUT, 2, 2>(g, s);
  // A quantised SwiGLU output needs 32-row tiles (one Q8_0 block a frame).
  if (waves(2, 1) >= kWant || (OUT == kGemmSwiGLU && g.out_q)) return launch_gemm_tiles<Scale, OUT, 2, 1>(g, s);
  return launch_gemm_tiles<Scale, OUT, 1, 1>(g, s);
}

template <class Scale>
hipError_t launch_gemm_scaled(const GemmArgs& g, int out, hipStream_t s) {
  switch (out) {
    case kGemmPlain: return launch_gemm_out<Scale, kGemmPlain>(g, s);
    case kGemmResidual: return launch_gemm_out<Scale, kGemmResidual>(g, s);
    case kGemmSwiGLU: return launch_gemm_out<Scale, kGemmSwiGLU>(g, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_gemm(const GemmArgs& g, bool half_scales, int out, hipStream_t s) {
  // Operands and scales move through LDS in stages of four blocks, so K only
  // bounds the int32 offsets; 3072 is the widest decoder matrix.
  if (g.K % 128 != 0 || g.K > 3072 || g.rows < 1 || g.frames < 1) return hipErrorInvalidValue;
  if (out == kGemmSwiGLU && !g.gu_map && (g.split_base < 1 || g.split_extra < 0)) return hipErrorInvalidValue;
  if (g.out_q && (out != kGemmSwiGLU || g.rows % 32 != 0 || !g.out_s)) return hipErrorInvalidValue;
  return half_scales ? launch_gemm_scaled<ScaleF16>(g, out, s) : launch_gemm_scaled<ScaleF32>(g, out, s);
}

// Rows per workgroup of the few-frame GEMM: about rows/256 (so that the grid
// covers the chip), at most kFewPairs pairs per lane and within kFewLds.
static int few_rows(int rows, int K, int frames, int out) {
  const int B = K / 32, per = out == kGemmSwiGLU ? 2 : 1;
  const int cap = kFewPairs * (kFewThreads / B) / per;  // rows a workgroup's lanes can hold
  int R = std::max(1, std::min(rows / 256, cap));
  while (R > 1 && few_lds_bytes(per * R, K, frames) > kFewLds) --R;
  if (R > cap || few_lds_bytes(per * R, K, frames) > kFewLds) return 0;
  return R;
}

// Workgroups of q8_head_mfma16_kernel for this shape, or 0 where it does not
// apply (FAH_FEW_MFMA=0 turns it off). At the q/k/v and gate/up shapes of
// the sessions it measured slower than q8_gemm_few_kernel (its 256-384
// single-tile waves each run a 32-block chain), so only the lm_head
// (thousands of tiles) takes it.
static int mfma16_groups(int rows, int K, int frames, int out) {
  static const bool on = [] {
    const char* v = std::getenv("FAH_FEW_MFMA");
    return !(v && v[0] == '0');
  }();
  if (!on || out != kGemmGreedy || frames < 8 || frames > 16 || K % 1024 != 0 || K > kM16MaxK || rows < 16) return 0;
  const int tiles = (rows + 15) / 16;
  return std::min((tiles + kM16Waves - 1) / kM16Waves, kM16MaxGroups);
}

int few_frame_groups(int rows, int K, int frames, int out) {
  if (const int m = mfma16_groups(rows, K, frames, out)) return m;
  if (frames < 1 || frames > kFewFrames || K % 128 != 0 || K > kFewMaxK || rows < 1) return 0;
  const int R = few_rows(rows, K, frames, out);
  return R ? (rows + R - 1) / R : 0;
}

template <class Scale, int OUT>
static hipError_t launch_few_kernel(const GemmArgs& g, int R, int groups, size_t lds, hipStream_t s) {
  // Dynamic LDS above the 64 KiB default needs the kernel's limit raised
  // (once per instantiation; not a stream operation, so capture-safe).
  static const hipError_t raised = hipFuncSetAttribute(
      reinterpret_cast<const void*>(q8_gemm_few_kernel<Scale, OUT>), hipFuncAttributeMaxDynamicSharedMemorySize,
      (int)kFewLds);
  if (raised != hipSuccess) return raised;
  q8_gemm_few_kernel<Scale, OUT><<<groups, kFewThreads, lds, s>>>(g, R);
  return hipGetLastError();
}

template <class Scale>
static hipError_t launch_few_scaled(const GemmArgs& g, int out, hipStream_t s) {
  if (const int m = mfma16_groups(g.rows, g.K, g.frames, out)) {
    q8_head_mfma16_kernel<Scale><<<m, 64 * kM16Waves, m16_lds_bytes(g.K), s>>>(g, (g.rows + 15) / 16);
    return hipGetLastError();
  }
  const int R = few_rows(g.rows, g.K, g.frames, out);
  const int groups = (g.rows + R - 1) / R;
  const size_t lds = few_lds_bytes(out == kGemmSwiGLU ? 2 * R : R, g.K, g.frames);
  switch (out) {
    case kGemmPlain: return launch_few_kernel<Scale, kGemmPlain>(g, R, groups, lds, s);
    case kGemmResidual: return launch_few_kernel<Scale, kGemmResidual>(g, R, groups, lds, s);
    case kGemmSwiGLU: return launch_few_kernel<Scale, kGemmSwiGLU>(g, R, groups, lds, s);
    case kGemmGreedy: return launch_few_kernel<Scale, kGemmGreedy>(g, R, groups, lds, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_gemm_few(const GemmArgs& g, bool half_scales, int out, hipStream_t s) {
  if (!few_frame_groups(g.rows, g.K, g.frames, out)) return hipErrorInvalidValue;
  if (out == kGemmSwiGLU && !g.gu_map && (g.split_base < 1 || g.split_extra < 0)) return hipErrorInvalidValue;
  if (out == kGemmGreedy && !g.keys) return hipErrorInvalidValue;
  return half_scales ? launch_few_scaled<ScaleF16>(g, out, s) : launch_few_scaled<ScaleF32>(g, out, s);
}

hipError_t launch_greedy_keys(const unsigned long long* keys, int groups, const float* logits, int vocab,
                              const SessionRef* sessions, int count, hipStream_t s) {
  if (count < 1 || groups < 1) return hipErrorInvalidValue;
  greedy_keys_kernel<<<count, 256, 0, s>>>(keys, groups, logits, vocab, sessions);
  return hipGetLastError();
}

hipError_t launch_norm_quantize_rows(const float* x, int frames, int K, const float* norm_w, float eps, int8_t* xq,
                                     float* xs, hipStream_t s) {
  if (K % 32 != 0 || K > 4096 || frames < 1) return hipErrorInvalidValue;
  norm_quantize_rows_kernel<<<frames, 256, 0, s>>>(x, K, norm_w, eps, xq, xs);
  return hipGetLastError();
}

hipError_t launch_attn_prefill(const PrefillAttnArgs& args, hipStream_t s) {
  PrefillAttnArgs a = args;
  if (a.head_size != 128 || a.frames < 1 || a.heads % a.kv_heads != 0) return hipErrorInvalidValue;
  if (!a.out && !a.xq) return hipErrorInvalidValue;
  if (a.qkv && (!a.sessions || !a.q_norm || !a.k_norm)) return hipErrorInvalidValue;
  if (!a.qkv && !a.q) return hipErrorInvalidValue;
  const int n = a.sessions ? a.max_positions : a.position + a.frames;
  if ((!a.sessions && n > a.capacity) || n < 1 || (size_t)n * 4 > 60 * 1024) return hipErrorInvalidValue;
  // V rows are staged in LDS when that keeps three workgroups per CU, or,
  // for grids of at most two workgroups per CU, up to kStageLds.
  constexpr size_t kStageLds = 150 * 1024;
  const size_t staged = (((size_t)4 * n + 15) & ~(size_t)15) + (size_t)n * 256;
  const bool small_grid = (size_t)a.heads * a.frames <= 512;
  a.stage = staged <= 48 * 1024 || (small_grid && staged <= kStageLds) ? n : 0;
  static const hipError_t raised = hipFuncSetAttribute(reinterpret_cast<const void*>(attn_prefill_kernel),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)kStageLds);
  if (raised != hipSuccess) return raised;
  // Many rows of one cache (a prefill): blocks of rows share K/V reads.
  if (!a.sessions && a.heads == 2 * a.kv_heads && a.frames >= 2 * kRowBlock && rows_lds_bytes(n) <= kStageLds) {
    static const hipError_t raised_rows = hipFuncSetAttribute(
        reinterpret_cast<const void*>(attn_rows_kernel), hipFuncAttributeMaxDynamicSharedMemorySize, (int)kStageLds);
    if (raised_rows != hipSuccess) return raised_rows;
    attn_rows_kernel<<<dim3(a.kv_heads, (a.frames + kRowBlock - 1) / kRowBlock), 256, rows_lds_bytes(n), s>>>(a);
    return hipGetLastError();
  }
  attn_prefill_kernel<<<dim3(a.heads, a.frames), 256, a.stage ? staged : (size_t)n * 4, s>>>(a);
  return hipGetLastError();
}

}  // namespace fah
