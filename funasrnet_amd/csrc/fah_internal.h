// Internal interface between the C ABI host code and the kernel launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fah {

enum InputMode { kInputQuantized = 0, kInputFloat = 1, kInputNorm = 2 };
enum OutputMode { kOutPlain = 0, kOutResidual = 1, kOutSwiGLU = 2, kOutGreedy = 3 };

struct GemvArgs {
  const int8_t* w;     // [rows][K] int8, storage order
  const void* ws;      // [rows][K/32] fp16 or fp32 scales, storage order
  int rows;            // storage rows
  int K;               // columns (multiple of 32)
  int group_rows;      // rows per workgroup (SwiGLU: gate half then up half)
  const float* x;      // fp32 input [frames][K] (kInputFloat / kInputNorm)
  const int8_t* xq;    // quantised input [frames][K] (kInputQuantized)
  const float* xs;     // [frames][K/32]
  const float* norm_w; // [K] (kInputNorm)
  float eps;
  float* out;          // [frames][out_rows]
  int out_rows;
  const float* resid;  // [frames][out_rows] (kOutResidual)
  const float* bias;   // [out_rows] or null (kOutPlain)
  unsigned long long* partial_keys;  // [frames][groups] (kOutGreedy)
};

struct QkArgs {
  const float* qkv;    // [q_width + 2*kv_width] raw projections
  const float* q_norm; // [head_size]
  const float* k_norm;
  const float* rope_cos;  // [capacity][head_size/2]
  const float* rope_sin;
  const int* position;    // device decode position
  float* q_out;           // [heads][head_size]
  _Float16* kcache;       // [kv_heads][capacity][head_size] (this layer)
  _Float16* vcache;
  int heads, kv_heads, head_size, q_width, kv_width, capacity;
  float eps;
};

struct AttnArgs {
  const float* q;          // [heads][head_size]
  const _Float16* kcache;  // [kv_heads][capacity][head_size]
  const _Float16* vcache;
  const int* position;
  float* scores;           // [heads][capacity]
  float* out;              // [heads][head_size]
  int heads, kv_heads, head_size, capacity;
  float divisor;           // sqrtf(head_size)
};

int gemv_max_k();
int gemv_pairs_per_thread(int group_rows, int K);
hipError_t launch_gemv(const GemvArgs& a, bool half_scales, int in, int out, int frames, hipStream_t s);
hipError_t launch_greedy_reduce(const unsigned long long* keys, int count, const float* logits, int* token,
                                hipStream_t s);
hipError_t launch_embed(const int8_t* q, const void* scales, bool half_scales, int K, int vocab, const int* token,
                        float* x, int* history, int* history_count, hipStream_t s);
hipError_t launch_qk_prepare(const QkArgs& a, hipStream_t s);
int attention_slices(int capacity, int head_size);
hipError_t prepare_attention(int capacity, int head_size);
hipError_t launch_attention(const AttnArgs& a, int score_groups, hipStream_t s);
hipError_t launch_advance(int* position, int frames, hipStream_t s);
hipError_t launch_quantize(const float* x, int64_t n, int8_t* q, float* scales, hipStream_t s);
hipError_t launch_block_dots(const int8_t* x, const int8_t* w, int rows, int K, int* dots, hipStream_t s);

}  // namespace fah
