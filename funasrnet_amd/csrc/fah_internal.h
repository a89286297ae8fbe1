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

// One decoder session of a lock-step batch: row f of a batched step reads and
// writes session f's cache, position and token.
struct SessionRef {
  _Float16* kcache;        // [layers][kv_heads][capacity][head_size]
  _Float16* vcache;
  const float* rope_cos;   // [capacity][head_size/2]
  const float* rope_sin;
  int* position;
  int* token;
  int* history;
  int* history_count;
  int capacity;
  int reserved;
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
  int frames;             // rows (0 or 1: decode); row t sits at position + t
  // Batched sessions (when set): row t is session t's next position; its
  // cache, RoPE tables and capacity replace the fields above for layer `layer`.
  const SessionRef* sessions;
  int layer;
};

struct AttnArgs {
  const float* q;          // [heads][head_size]
  const _Float16* kcache;  // [kv_heads][capacity][head_size]
  const _Float16* vcache;
  const int* position;
  float* scores;           // [heads][capacity]: scores, then exponentials in place
  float* block_max;        // [heads][capacity / 256 rounded up]: each score block's maximum
  double* exp_t;           // [heads][8][exp_stride]: numerators as doubles, position 8 i + j at [j][i]
  // [heads][capacity / 256 rounded up]: each numerator block's exact double
  // sum, NaN when a numerator of the block is outside {0} u [2^-17, 1] or
  // there are 8192 positions or more (the denominator then takes exp_t).
  double* block_sum;
  int exp_stride;          // capacity / 8 rounded up to a multiple of 2
  float* out;              // [heads][head_size]
  int heads, kv_heads, head_size, capacity;
  float divisor;           // sqrtf(head_size)
};

struct PersistentLayer {
  const int8_t* wqkv;
  const _Float16* sqkv;
  const int8_t* wo;
  const _Float16* so;
  const int8_t* wgu;   // tiles of rgu gate rows then rgu up rows
  const _Float16* sgu;
  const int8_t* wd;
  const _Float16* sd;
  const float* attn_norm;
  const float* q_norm;
  const float* k_norm;
  const float* ffn_norm;
};

// Persistent decode, row ownership by XCD. A vector of `rows` rows is cut
// into blocks of `block` rows; block b belongs to XCD b % 8 (role w runs on
// XCD w % 8). XCD x's rows / 8 rows (its blocks in order: list entry e is
// row block (x + 8 (e / block)) + e % block) are split evenly over its
// projection roles, the first ones taking one more. The ffn rows use 64-row
// blocks (pairs of Q8_0 blocks): role (x, j) stores its gate rows then its
// up rows at storage row 2 (x ffn / 8 + first entry).
struct XcdEntries {
  int r0, count;
};
__host__ __device__ inline int persistent_xcd_roles(int x, int kv_heads, int group, int blocks) {
  return blocks / 8 - (x < kv_heads ? group : 0);
}
__host__ __device__ inline XcdEntries persistent_xcd_entries(int x, int j, int rows, int kv_heads, int group,
                                                             int blocks) {
  const int ex = rows / 8, n = persistent_xcd_roles(x, kv_heads, group, blocks);
  const int base = ex / n, extra = ex % n;
  return {j * base + (j < extra ? j : extra), base + (j < extra ? 1 : 0)};
}
__host__ __device__ inline int persistent_xcd_row(int x, int e, int block) {
  return block * (x + 8 * (e / block)) + e % block;
}

// A quantised vector in exchange form (K values, K / 32 Q8_0 blocks): eight
// 64-bit words per block, word 8b + k holding the packed int8 values
// 32b + 4k .. +3 in its low half and, in its high half, a 16-bit tag above
// 16 side bits, which carry the low and high halves of block b's float
// scale in words 8b and 8b + 1. K / 4 words in all. Every 128-byte line has
// a single writer (the ffn owners publish two blocks, the attention
// workgroups four): such lines reach the other XCDs far sooner than lines
// that several workgroups write parts of.
__host__ __device__ constexpr int qblock_words(int K) { return K / 4; }

struct PersistentArgs {
  const PersistentLayer* layer_table;  // device array [layers]
  int layers;
  const int8_t* embed_q;
  const _Float16* embed_s;
  const int8_t* head_q;
  const _Float16* head_s;
  const float* output_norm;
  const float* rope_cos;
  const float* rope_sin;
  _Float16* kcache;  // [layers][kv_heads][capacity][head_size]
  _Float16* vcache;
  int width, heads, kv_heads, head_size, ffn, vocab, capacity;
  int q_width, kv_width;
  float eps, divisor;
  int rq, ro, rgu, rd;  // rows per workgroup: qkv, o, gate (and up), down
  int head_chunks;      // lm_head chunks of 32 rows
  unsigned long long *tx, *tqkv, *tatt, *ta, *th, *tkeys;  // tagged exchange words
  // Quantised exchanges (qblock_words layout): the attention output
  // for the o projection and the ffn activations for the down projection.
  unsigned long long *tattq, *thq;
  // Long caches: scores of the earlier positions, [heads][score_stride]
  // tagged words (score_stride = capacity rounded up to 128), written by
  // the projection workgroups of the kv head's XCD from position long_from
  // on, then overwritten with the probabilities by the attention
  // workgroups (see tready).
  unsigned long long* tscore;
  int score_stride;
  int long_from;
  const float* x_in;    // modes 0/1: the input row
  int mode;             // 0 layers, 1 layers + lm_head + greedy, 2 embed token + 1
  int* position;
  int* token;
  int* history;
  int* history_count;
  unsigned* epoch;
  unsigned* error;
  float* logits;
  unsigned long long* timeline;  // optional [2][kTimelineEvents] s_memrealtime stamps
  // 1: workgroup w runs on XCD w % 8 (checked at creation and by every
  // launch), so the q/k/v rows of kv head x are computed on XCD x and handed
  // to its attention workgroups through that XCD's L2.
  int local_l2;
  // Long caches: tready[2 h], [2 h + 1] carry head h's generation once its
  // probabilities are all written over its scores (the first word carries
  // p[pos]).
  unsigned long long* tready;
};

constexpr int kTimelineEvents = 480;

// Prefill (many frames): Q8_0 GEMM with the reference's per-row block order.
struct GemmArgs {
  const int8_t* w;      // storage rows [*][K] int8
  const void* ws;       // storage scales [*][K/32] (fp16 or fp32)
  int rows;             // logical output rows (SwiGLU: ffn)
  int K;
  const int8_t* xq;     // [frames][K]
  const float* xs;      // [frames][K/32]
  int frames;
  float* out;           // [frames][out_stride]
  int out_stride;
  const float* resid;   // [frames][out_stride] (residual epilogue; may equal out)
  const float* bias;    // [rows] or null (plain epilogue)
  int split_base, split_extra;  // SwiGLU storage: tiles of base(+1) gate rows then the same up rows
  const int* gu_map;            // or, when set, the SwiGLU storage row of row r: [2r] gate, [2r + 1] up
  // Greedy epilogue (few-frame kernel): the largest greedy key of each
  // workgroup's rows per frame, [frames][workgroups].
  unsigned long long* keys;
  // Optional Q8_0 output of the SwiGLU epilogue of q8_gemm_kernel (rows a
  // multiple of 32), in place of `out`: codes [frames][rows], scales
  // [frames][rows/32].
  int8_t* out_q;
  float* out_s;
};
enum GemmOut { kGemmPlain = 0, kGemmResidual = 1, kGemmSwiGLU = 2, kGemmGreedy = 3 };

struct PrefillAttnArgs {
  const float* q;          // [frames][heads*head_size], normalised and rotated
  const _Float16* kcache;  // [kv_heads][capacity][head_size] (this layer)
  const _Float16* vcache;
  float* out;              // [frames][heads*head_size], or null with xq set
  int frames, position;    // query row t sits at position + t
  int heads, kv_heads, head_size, capacity;
  float divisor;
  // Optional Q8_0 quantisation of the output rows ([frames][heads*head_size]
  // codes, [frames][heads*head_size/32] scales), block by block.
  int8_t* xq;
  float* xs;
  // Batched sessions (when set): row t attends over session t's cache for
  // layer `layer` at its position; max_positions bounds position + 1.
  const SessionRef* sessions;
  int layer, max_positions;
  // Set by launch_attn_prefill: V rows are staged in LDS when every row's
  // positions fit (bound on positions + 1; 0 = read V from global memory).
  int stage;
  // Sessions only: when set, the kernel forms this row's q, k and v from the
  // raw projections ([frames][q_width + 2*kv_width]) itself (QK-norm, RoPE
  // from the session's tables, F16 rounding) and writes the K/V row, instead
  // of a separate QK preparation (q is then unused).
  const float* qkv;
  const float* q_norm;
  const float* k_norm;
  float eps;
  int q_width, kv_width;
};

hipError_t launch_gemm(const GemmArgs& g, bool half_scales, int out, hipStream_t s);
// Few-frame Q8_0 GEMM (frames <= kFewFrames): rows per workgroup chosen for
// ~256+ workgroups; returns the workgroup count through *groups (0 = the
// shape does not fit its LDS, use launch_gemm).
constexpr int kFewFrames = 16;
int few_frame_groups(int rows, int K, int frames, int out);
hipError_t launch_gemm_few(const GemmArgs& g, bool half_scales, int out, hipStream_t s);
hipError_t launch_greedy_keys(const unsigned long long* keys, int groups, const float* logits, int vocab,
                              const SessionRef* sessions, int count, hipStream_t s);
hipError_t launch_norm_quantize_rows(const float* x, int frames, int K, const float* norm_w, float eps, int8_t* xq,
                                     float* xs, hipStream_t s);
hipError_t launch_attn_prefill(const PrefillAttnArgs& a, hipStream_t s);
hipError_t launch_session_embed(const int8_t* q, const void* scales, bool half_scales, int K, int vocab,
                                const SessionRef* sessions, int count, float* x, hipStream_t s);


// FP32 projections y[M][N] = x[M][K] W[N][K]^T (+ bias) (ReLU): fp32 MFMA
// GEMM, or a GEMV for up to 4 frames of at most 4096 columns.
hipError_t launch_f32_linear(const float* x, const float* w, const float* bias, float* out, int M, int N, int K,
                             bool relu, hipStream_t s);
// Non-causal multi-head attention over [frames][width] rows (head size
// width / heads <= 256, frames <= 4096).
bool f32_attention_supported(int frames, int width, int heads);
hipError_t launch_f32_attention(const float* q, const float* k, const float* v, float* out, int frames, int width,
                                int heads, hipStream_t s);

bool persistent_shape_supported(int width, int heads, int kv_heads, int head_size, int ffn, int blocks);
// long_cache: the step at a position from a.long_from on (the long-cache
// attention); the kernel ends with error 4 if the device position disagrees.
hipError_t launch_decode_step(const PersistentArgs& a, int blocks, hipStream_t s, bool long_cache);
// Whether 256 workgroups of the persistent kernel's size land on XCD
// w % 8 (one launch of a placement probe; false if it cannot tell).
bool persistent_xcd_round_robin(hipStream_t s);
// Positions the persistent kernel takes (position + 1 at most this), and
// the positions below which its attention workgroups hold every earlier
// K/V row (PersistentArgs::long_from at most this).
int persistent_max_positions();
int persistent_exact_positions();
int persistent_threads();
int persistent_blocks_per_cu(int width);

// Lock-step sessions step in one launch (fah_sessions.hip): the decoder
// layers of S sessions, one token each, with tagged-word exchanges between
// the phases; the output-normalised Q8_0 rows go to xq_out/xs_out for the
// lm_head.
struct SessionStepArgs {
  const PersistentLayer* layer_table;  // device array [layers]
  int layers;
  int width, heads, kv_heads, head_size, ffn;
  const float* output_norm;
  const SessionRef* sessions;  // [S]
  int S;
  int max_positions;  // bound on every session's position + 1
  const int* gu_map;  // gate/up storage rows (or null: tiles of gu_base rows)
  int gu_base, gu_extra;
  float eps, divisor;
  const float* x_in;  // [S][width] embeddings
  int8_t* xq_out;     // [S][width]
  float* xs_out;      // [S][width / 32]
  // Exchange words: residual rows, attention-norm rows (Q8_0), q/k/v,
  // attention output (Q8_0), o + residual, ffn-norm rows (Q8_0), gate/up
  // half-block maxima, ffn activations (Q8_0).
  unsigned long long *tx, *txq, *tqkv, *tattq, *ta, *taq, *tmax, *thq;
  unsigned* epoch;
  unsigned* error;
};
bool session_step_supported(int width, int heads, int kv_heads, int head_size, int ffn);
int session_step_positions();
int session_step_groups();
int session_step_blocks_per_cu(int width);
hipError_t launch_session_step(const SessionStepArgs& a, hipStream_t s);

int gemv_max_k();
int gemv_pairs_per_thread(int group_rows, int K);
hipError_t launch_gemv(const GemvArgs& a, bool half_scales, int in, int out, int frames, hipStream_t s);
hipError_t launch_greedy_reduce(const unsigned long long* keys, int count, const float* logits, int* token,
                                hipStream_t s);
// GGUF Q8_0 blocks (34 B: fp16 scale, 32 int8) -> int8 plane + fp16 scale bits.
hipError_t launch_unpack_q8_blocks(const uint8_t* raw, int64_t blocks, int8_t* q, uint16_t* s, hipStream_t st);
hipError_t launch_embed(const int8_t* q, const void* scales, bool half_scales, int K, int vocab, const int* token,
                        float* x, int* history, int* history_count, hipStream_t s);
hipError_t launch_qk_prepare(const QkArgs& a, hipStream_t s);
// Value-kernel workgroups per KV head for G = `group` query heads a KV head
// (2 or 4); 0 when the capacity exceeds its LDS budget.
int attention_slices(int capacity, int head_size, int group);
// Row stride (doubles) of AttnArgs::exp_t for a cache of `capacity` positions.
inline int attention_exp_stride(int capacity) { return ((capacity + 7) / 8 + 1) & ~1; }
hipError_t prepare_attention(int capacity, int head_size, int group);
hipError_t launch_attention(const AttnArgs& a, int score_groups, hipStream_t s);
hipError_t launch_advance(int* position, int frames, hipStream_t s);
hipError_t launch_quantize(const float* x, int64_t n, int8_t* q, float* scales, hipStream_t s);
hipError_t launch_session_batch_io(const SessionRef* sessions, int count, int* out, hipStream_t s);
hipError_t launch_rms_norm_rows(const float* x, int rows, int width, const float* scale, float eps, float* y,
                                hipStream_t s);
hipError_t launch_block_dots(const int8_t* x, const int8_t* w, int rows, int K, int* dots, hipStream_t s);

}  // namespace fah
