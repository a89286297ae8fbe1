/*
 * CPU oracle for the Qwen3 Q8_0 decoder path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a scalar C restatement of the reference's
 * x64 C# path (src/FunAsrNet, .NET 10, AVX2/AVX-VNNI branch), written as the
 * parity reference for the HIP library. Only tests/, the smoke() entry
 * point and bench.py's cpu_baseline leg may load it. The product path never
 * calls into it and has no CPU fallback.
 *
 * Every function cites the reference lines whose operation order it follows.
 * Build flags: -O2 -ffp-contract=off (no FMA contraction), no -ffast-math.
 *
 * Pinning status (what checks each function against something independent):
 *   oracle_quantize            pinned: reference KATs (halfway +-1ulp, denormal
 *                              scales, specials), closed form in numpy
 *   oracle_block_dot /
 *   oracle_q8_linear           pinned: reference deterministic KAT
 *                              (QuantizedAvxChecks.cs:17-50) brute force in numpy
 *   oracle_round_half          pinned: exhaustive vs numpy float16 RNE
 *   oracle_half_to_float       pinned: exhaustive 65536 patterns vs numpy
 *   oracle_rotate_half         pinned: scalar rotation restated in numpy
 *   oracle_greedy              pinned: numpy first-max scan incl. NaN/inf/-0
 *   oracle_rms_norm            pinned bit for bit: the four chains restated
 *                              with numpy's sequential sums, then the float
 *                              steps in numpy float32; and a double reference
 *                              at 1e-5 (tests/test_oracle_norm_order.py)
 *   oracle_sum_sq_gpu_tree     pinned: an independent numpy pairwise tree
 *   oracle_norm_order_*        counts built on the two sums above
 *   oracle_exp                 pinned: follows ExpAvx.cs (reference's own x64
 *                              exp on .NET 11); vs double exp <= 1 ulp. The
 *                              .NET 10 runtime Vector256.Exp is not in the
 *                              reference tree: bit values parity unpinned.
 *   oracle_softmax             pinned: double reference at 5e-7 (tolerance)
 *   oracle_silu_multiply       pinned: double reference at 2e-6 (tolerance)
 *   oracle_attention           pinned: float64 attention at 5e-5 (tolerance);
 *                              lane-sum grouping of Vector128.Sum assumed
 *                              (a0+a1)+(a2+a3): parity unpinned for that detail
 *   oracle_rope_table          glibc powf/cosf/sinf (CoreCLR forwards MathF to
 *                              the C runtime): parity unpinned, checked vs
 *                              double cos/sin at 2 ulp-scale tolerance
 *   oracle_decoder_*           composition of the above; pinned by the
 *                              properties in tests/test_oracle_decoder.py
 *   oracle_float_linear_f64    the independent double reference the
 *                              reference's device checks use for FP32
 *                              projections; pinned: integer-valued inputs
 *                              exactly equal to an int64 brute force, random
 *                              inputs vs numpy's float64 matmul, identity and
 *                              zero weights (tests/test_oracle_float.py)
 *   oracle_attention_f64       double reference of non-causal multi-head
 *                              attention (AttentionGpuChecks.cs Reference);
 *                              pinned: q = k = 0 gives the mean of v, one
 *                              frame gives v, one dominant key gives its v,
 *                              heads computed independently, permuting keys
 *                              and values together changes nothing
 */
#ifndef FAH_ORACLE_H
#define FAH_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* --- scalar helpers --------------------------------------------------- */
float oracle_half_to_float(uint16_t h);
uint16_t oracle_float_to_half(float f);
float oracle_round_half(float f);
void oracle_round_half_copy(const float* x, int64_t n, float* y);
float oracle_exp(float x);
int oracle_set_threads(int threads);

/* --- Q8_0 ------------------------------------------------------------- */
int oracle_unpack_q8(const uint8_t* raw, int64_t blocks, int8_t* q, float* scales);
int oracle_quantize(const float* x, int64_t n, int8_t* q, float* scales);
int32_t oracle_block_dot(const int8_t* w, const int8_t* x);
void oracle_q8_block_dots(const int8_t* xq, const int8_t* wq, int rows, int cols, int32_t* dots);
void oracle_q8_gemv_quantized(const int8_t* xq, const float* xs, int frames,
                              const int8_t* wq, const float* ws, int rows, int cols,
                              const float* bias, float* out);
int oracle_q8_linear(const float* input, int frames, const int8_t* wq, const float* ws,
                     int rows, int cols, const float* bias, float* out);
void oracle_embed_row(const int8_t* q, const float* scales, int cols, int token, float* out);

/* --- element-wise ----------------------------------------------------- */
int oracle_rms_norm(const float* x, int64_t n, int width, const float* scale, float eps, float* y);
void oracle_rope_table(int capacity, int head_size, float base, float* cos_out, float* sin_out);
void oracle_rotate_half(float* x, const float* cosine, const float* sine, int half);
void oracle_softmax(float* x, int n);
void oracle_silu_multiply(float* gate, const float* up, int64_t n);
void oracle_add(float* target, const float* other, int64_t n);
float oracle_dot(const float* a, const float* b, int n);
int32_t oracle_greedy(const float* logits, int64_t n);
void oracle_attention(const float* q, const float* kcache, const float* vcache,
                      int frames, int position, int heads, int kv_heads, int head_size,
                      float* out);

/* --- decoder (QwenDecoder.cs:9-385) ------------------------------------ */
typedef struct oracle_q8 {
    const int8_t* q;      /* [rows][cols] row-major */
    const float* scales;  /* [rows][cols/32] */
    int rows, cols;
} oracle_q8;

typedef struct oracle_layer {
    oracle_q8 wq, wk, wv, wo, gate, up, down;
    const float* attn_norm;  /* [width] */
    const float* q_norm;     /* [head_size] */
    const float* k_norm;     /* [head_size] */
    const float* ffn_norm;   /* [width] */
} oracle_layer;

typedef struct oracle_model {
    int width, heads, kv_heads, head_size, layers, ffn, vocab;
    float eps, rope_base;
    const oracle_layer* layer;  /* [layers] */
    oracle_q8 token_embd;       /* [vocab][width] */
    oracle_q8 output;           /* q == NULL -> tied to token_embd */
    const float* output_norm;   /* [width] */
} oracle_model;

/* FP32 projection in double: out[f][n] = sum_k x[f][k] w[n][k] (+ bias[n]),
 * each product and sum in double, then rounded once. */
void oracle_float_linear_f64(const float* x, int frames, int cols, const float* w, int rows, const float* bias,
                             double* out);
/* Non-causal multi-head attention in double over [frames][width] rows. */
void oracle_attention_f64(const float* q, const float* k, const float* v, int frames, int width, int heads,
                          double* out);

typedef struct oracle_decoder oracle_decoder;

oracle_decoder* oracle_decoder_create(const oracle_model* model, int capacity);
void oracle_decoder_destroy(oracle_decoder* d);
void oracle_decoder_reset(oracle_decoder* d);
int oracle_decoder_position(const oracle_decoder* d);
int oracle_decoder_set_position(oracle_decoder* d, int position);
int oracle_decoder_decode(oracle_decoder* d, const float* embeddings, int frames, float* logits);
int oracle_decoder_embed(const oracle_decoder* d, const int32_t* tokens, int count, float* out);
/* Cached K/V rows (fp32 holding F16-rounded values), [capacity][kv_heads*head_size]. */
/* Tests only: copy the input rows of the width-wide RMSNorms (attention,
 * ffn, output) and of the QK-norms (per head) of the next decodes, up to the
 * given row counts; oracle_decoder_captured reports how many were taken. */
void oracle_decoder_capture_norms(oracle_decoder* d, float* wide, int64_t wide_rows, float* heads, int64_t head_rows);
int64_t oracle_decoder_captured(const oracle_decoder* d, int heads);
float* oracle_decoder_keys(oracle_decoder* d, int layer);
float* oracle_decoder_values(oracle_decoder* d, int layer);
const char* oracle_last_error(void);

/* --- RMSNorm square-sum order (tests only) ----------------------------- */
double oracle_sum_sq_gpu_tree(const float* x, int width);
double oracle_sum_sq_reference(const float* x, int width);
int oracle_rms_mean_settled(double tree, int width, float* mean);
int oracle_norm_order_stats(const float* pool, int64_t pool_n, int width, int rowwise, int64_t rows, uint64_t seed,
                            int64_t* counts);
int64_t oracle_norm_order_find(const float* pool, int64_t pool_n, int width, int rowwise, uint64_t seed,
                               int64_t start, int64_t rows, int64_t want, float* out);

#ifdef __cplusplus
}
#endif
#endif
