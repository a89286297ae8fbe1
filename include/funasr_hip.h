/*
 * funasr_hip.h -- C ABI of the MI355X (gfx950) Qwen3 Q8_0 decoder library.
 *
 * This is the drop-in boundary behind FunAsrNet's FloatBackend seam. A C#
 * FunAsrNet.Hip assembly binds these symbols with [LibraryImport]; every
 * entry point names the reference interface it replaces (paths relative to
 * the FunAsrNet source tree).
 *
 * Conventions (from the reference's Try* contract,
 * src/FunAsrNet/IQuantizedComputeBackend.cs:4-14, IFloatComputeBackend.cs:18):
 *   FAH_OK (0)        the call completed; outputs are written.
 *   FAH_DECLINED (1)  unsupported shape or type: outputs are untouched and
 *                     the caller continues on its CPU path ("return false").
 *   < 0               error: argument mismatch (ArgumentException), device
 *                     failure (InvalidOperationException) or use after
 *                     destroy (ObjectDisposedException); fah_last_error()
 *                     returns the message for the calling thread.
 * Host pointers are only read or written during the call. Weights are copied
 * to the device once at upload and are immutable afterwards. A context owns
 * one HIP stream; calls on one context are serialised by the library. Calls
 * on different contexts may be made from different threads: their work is
 * enqueued under a per-device lock, and a persistent decode step or a
 * lock-step sessions step that runs the layers in one launch (both need
 * every CU of the device) first waits for the work already enqueued by the
 * other contexts and keeps the device to itself until it has finished, so
 * their kernels never run beside it.
 *
 * Lifetime: weights and decoders keep their context's state alive.
 * fah_context_destroy releases the handle (which must not be used again);
 * later calls on its weights and decoders return FAH_ERROR_DISPOSED, and
 * fah_weight_release / fah_decoder_destroy still free them, in any order.
 */
#ifndef FUNASR_HIP_H
#define FUNASR_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FAH_OK 0
#define FAH_DECLINED 1
#define FAH_ERROR_ARGUMENT (-1)
#define FAH_ERROR_DEVICE (-2)
#define FAH_ERROR_DISPOSED (-3)
#define FAH_ERROR_STATE (-4)

#define FAH_ABI_VERSION 1

typedef struct fah_context fah_context;
typedef struct fah_weight fah_weight;
typedef struct fah_decoder fah_decoder;
typedef struct fah_batcher fah_batcher;

/* Library ------------------------------------------------------------------ */

/* ABI version of the loaded library (FAH_ABI_VERSION). */
int fah_abi_version(void);

/* Message of the last failing call on this thread (never NULL). Replaces the
 * exception text the reference raises (VulkanQuantizedBackend.cs:49-52). */
const char* fah_last_error(void);

/* Number of visible HIP devices; 0 when none (the C# loader then keeps the
 * CPU path, as VulkanFloatBackend creation failure does). */
int fah_device_count(void);

/* Context: one device plus one stream. Replaces the backend object assigned
 * to FunAsr.FloatBackend (src/FunAsrNet/FunAsr.cs:67-71). */
int fah_context_create(int device, fah_context** out);
int fah_context_destroy(fah_context* context);
int fah_context_synchronize(fah_context* context);
/* Backend name (IFloatComputeBackend.Name, IFloatComputeBackend.cs:6-9). */
const char* fah_context_name(const fah_context* context);
/* Projections below this many multiply-adds (frames*rows*cols) are declined
 * so the caller's CPU path runs them, as VulkanFloatBackend.MinimumOperations
 * does (src/FunAsrNet.Vulkan/VulkanFloatBackend.cs:36; default 250000). */
int fah_context_set_minimum_operations(fah_context* context, int64_t operations);
/* The context's hipStream_t, for callers that order their own device work
 * (device-pointer entry points below) with the library's. */
void* fah_context_stream(fah_context* context);

/* Seam-call statistics. Replaces the counters of
 * VulkanFloatBackend.Statistics() (src/FunAsrNet.Vulkan/VulkanFloatBackend.cs:86-118:
 * calls per kind, uploaded/downloaded bytes, end-to-end seconds) and the
 * per-projection timing of TensorMath.LinearMeasured
 * (src/FunAsrNet/TensorMath.cs:37-40, invoked at TensorMath.cs:198 and
 * TensorMath.QuantizedGroupAvx.cs:100), with the device time of each call's
 * kernels added (HIP events on the context stream around them). */
enum {
  FAH_CALL_QUANTIZED_LINEAR = 0,   /* fah_quantized_linear */
  FAH_CALL_QUANTIZED_LINEAR_NOALLOC = 1,
  FAH_CALL_LINEAR_MANY = 2,        /* fah_linear_many, Q8_0 or FP32 group */
  FAH_CALL_LINEAR = 3,             /* fah_linear */
  FAH_CALL_RELU_PROJECTION = 4,    /* fah_relu_projection */
  FAH_CALL_ATTENTION = 5,          /* fah_attention */
  FAH_CALL_KINDS = 6
};
typedef struct fah_call_stats {
  int64_t calls;             /* calls that ran on the device */
  int64_t declined;          /* calls declined (FAH_DECLINED: the CPU path ran) */
  int64_t operations;        /* multiply-adds of the calls that ran */
  int64_t uploaded_bytes;    /* host -> device, inputs and biases */
  int64_t downloaded_bytes;  /* device -> host, outputs */
  double device_ms;          /* kernel time of the calls that ran */
  double total_ms;           /* wall time inside those calls, copies and waits included */
} fah_call_stats;
/* Copies the first min(kinds, FAH_CALL_KINDS) records (index = FAH_CALL_*). */
int fah_context_statistics(fah_context* context, fah_call_stats* out, int kinds);
int fah_context_reset_statistics(fah_context* context);
/* Called on the calling thread at the end of every seam call that ran on the
 * device (kind, frames, input columns, output rows of all its weights,
 * kernel milliseconds, wall milliseconds), before the call returns; it must
 * not call this library on the same context. NULL removes it. */
typedef void (*fah_call_observer)(void* user, int kind, int frames, int cols, int rows, double device_ms,
                                  double total_ms);
int fah_context_set_call_observer(fah_context* context, fah_call_observer observer, void* user);

/* Weights ------------------------------------------------------------------ */

/* Upload a Q8_0 matrix in the reference's post-load layout: `quantized` is
 * sbyte[rows*cols] row-major, `scales` float[rows*cols/32]
 * (Weight.Quantized / Weight.Scales, src/FunAsrNet/Gguf.cs:289-307,
 * Columns = cols = Shape[0], Rows = rows = Shape[1]). Scales are kept as
 * fp16 on the device when every scale converts exactly (always true for
 * GGUF Q8_0), otherwise as fp32. cols must be a multiple of 32. */
int fah_weight_q8_upload(fah_context* context, const int8_t* quantized, const float* scales,
                         int rows, int cols, fah_weight** out);
/* Upload a Q8_0 matrix straight from its GGUF blocks: `blocks` holds
 * rows*cols/32 blocks of 34 bytes (little-endian fp16 scale, then 32 int8),
 * row-major, as the tensor data of a GGUF file. Replaces reading the tensor
 * and unpacking it on the host (src/FunAsrNet/Gguf.cs:132-173,
 * src/FunAsrNet/TensorMath.Q8Model.cs:15-39) before the upload: the blocks
 * are split into the int8 plane and the fp16 scale plane on the device, so
 * no sbyte[]/float[] copy of the matrix exists on the host. */
int fah_weight_q8_upload_blocks(fah_context* context, const uint8_t* blocks, int rows, int cols, fah_weight** out);
/* Upload an FP32 matrix (Weight.Values, src/FunAsrNet/Gguf.cs:264-345:
 * float[rows*cols] row-major, Columns = cols, Rows = rows; F16 tensors come
 * widened exactly). Serves fah_linear, fah_relu_projection and FP32 groups
 * of fah_linear_many; the Q8_0 entry points decline it. */
int fah_weight_f32_upload(fah_context* context, const float* values, int rows, int cols, fah_weight** out);
int fah_weight_release(fah_weight* weight);
/* Device bytes held by the weight (int8 plane plus scale plane). */
int64_t fah_weight_device_bytes(const fah_weight* weight);

/* Projections (host buffers) ------------------------------------------------ */

/* IQuantizedComputeBackend.TryQuantizedLinear
 * (src/FunAsrNet/IQuantizedComputeBackend.cs:4-14; reference device version
 * src/FunAsrNet.Vulkan/VulkanQuantizedBackend.cs:40-133):
 * output[frames*rows] = bias + Q8 projection of the per-32-block quantised
 * input[frames*cols], with the reference's exact activation quantisation and
 * per-row block-ordered fp32 accumulation. bias may be NULL. */
int fah_quantized_linear(fah_context* context, const float* input, int frames, const fah_weight* weight,
                         const float* bias, float* output);

/* fah_quantized_linear without any device allocation. No counterpart in the
 * reference: for callers that cannot allocate device memory (tight serving
 * loops, code that must not call hipMalloc). Same arguments, results
 * (bit for bit), declines and errors as fah_quantized_linear; the staged
 * input, bias and output and the quantised activations live in a fixed
 * 8 MiB workspace per GPU (a static device array, held until the process
 * ends) instead of context buffers. A projection whose workspace
 * (frames*cols*5.125 + rows*4*(frames+1) bytes, each part rounded up to 256)
 * exceeds 8 MiB is rejected with FAH_ERROR_ARGUMENT. Nothing in the
 * workspace needs to start at zero. Calls that overlap on one GPU would race
 * on its workspace: the library serialises them (the call keeps the
 * device's work lock until its output is back). */
int fah_quantized_linear_noalloc(fah_context* context, const float* input, int frames, const fah_weight* weight,
                                 const float* bias, float* output);

/* IFloatComputeBackend.TryLinear (src/FunAsrNet/IFloatComputeBackend.cs:11-18;
 * reference device version src/FunAsrNet.Vulkan/VulkanFloatBackend.cs:127-171):
 * output[frames*rows] = input[frames*cols] W^T (+ bias) for an FP32 weight,
 * on fp32 MFMA (or a bandwidth-bound GEMV for up to 4 frames). Declines
 * (output untouched) Q8_0 weights and projections below the minimum
 * operations. Float order differs from the CPU kernels, as the reference's
 * own device path does (its check: 2e-4 x max(1, |expected|)). The encoder's
 * projections (src/FunAsrNet/FunEncoder.cs:100) and the original-weights
 * decoder's GEMVs (FloatVectorShader.cs) go through it. */
int fah_linear(fah_context* context, const float* input, int frames, const fah_weight* weight, const float* bias,
               float* output);

/* IReluProjectionBackend.TryReluProjection (src/FunAsrNet/IReluProjectionBackend.cs:4-16;
 * device version VulkanReluProjection.cs): output = ReLU(input W1^T + b1)
 * W2^T + b2 with the intermediate kept on the device; bit for bit the two
 * fah_linear calls with the ReLU (v < 0 ? 0 : v) between them. Biases may be
 * NULL. Declines unless both weights are FP32, first rows == second cols and
 * first rows % 4 == 0 (the reference's conditions), or below the minimum
 * operations. */
int fah_relu_projection(fah_context* context, const float* input, int frames, const fah_weight* first,
                        const float* first_bias, const fah_weight* second, const float* second_bias, float* output);

/* IAttentionComputeBackend.TryAttention (src/FunAsrNet/IAttentionComputeBackend.cs:4-16;
 * CPU version TensorMath.cs:619-666, device version VulkanAttention.cs):
 * non-causal multi-head attention over [frames][width] query, key and value
 * rows, `heads` heads of width / heads channels: per head and query row,
 * scores dot(q, k) / sqrtf(size), softmax, weighted values. Declines frames
 * outside 1..4096, width not a multiple of heads, head size above 256, and
 * (with a positive minimum) fewer than 160 frames or frames^2 * width below
 * the minimum operations -- the reference's conditions. */
int fah_attention(fah_context* context, const float* query, const float* key, const float* value, int frames,
                  int width, int heads, float* output);

/* IGroupedComputeBackend.TryLinearMany
 * (src/FunAsrNet/IGroupedComputeBackend.cs:4-13; CPU version
 * src/FunAsrNet/TensorMath.Interleaved.cs:22-46): one shared activation
 * quantisation, outputs[i][frames*rows_i]. All weights share cols. A group of
 * FP32 weights gives, per weight, the bits of fah_linear. */
int fah_linear_many(fah_context* context, const float* input, int frames, const fah_weight* const* weights,
                    int count, float* const* outputs);

/* Projections on device-resident buffers (pointers from hipMalloc on the
 * context's device; work is ordered on the context stream) ------------------ */

/* TensorMath.Quantize (src/FunAsrNet/TensorMath.cs:378-412): n % 32 == 0. */
int fah_quantize_device(fah_context* context, const float* x, int64_t n, int8_t* q, float* scales);

/* RMSNorm of `rows` rows, TensorMath.Norm with rms = true
 * (src/FunAsrNet/TensorMath.cs:537-573, TensorMath.Elementwise.cs:26-100, as
 * QwenDecoder.Norm calls it, QwenDecoder.cs:354-360): y = (x * inverse) *
 * scale with the reference's float mean of its ordered double square sum.
 * Width 128 runs the decode step's QK-norm arithmetic, other widths (a
 * multiple of 4, at most 4096) its layer-norm arithmetic. */
int fah_rms_norm_device(fah_context* context, const float* x, int rows, int width, const float* scale, float eps,
                        float* y);

/* Q8_0 x quantised-activation GEMV/GEMM: out[frames*rows] from q[frames*cols],
 * scales[frames*cols/32] (TensorMath.QuantizedRowsAvx.cs:17-60 order). */
int fah_q8_gemv_device(fah_context* context, const int8_t* q, const float* scales, int frames,
                       const fah_weight* weight, float* out);

/* fah_linear on device-resident buffers: out[frames*rows] = x[frames*cols]
 * W^T (+ bias[rows], may be NULL) for an FP32 weight, ordered on the context
 * stream (no copies, no wait). */
int fah_linear_device(fah_context* context, const float* x, int frames, const fah_weight* weight, const float* bias,
                      float* out);

/* fah_attention on device-resident [frames][width] buffers, ordered on the
 * context stream (no copies, no wait); same declines. */
int fah_attention_device(fah_context* context, const float* query, const float* key, const float* value, int frames,
                         int width, int heads, float* output);

/* Exact int32 block dots dots[rows*cols/32] of one quantised activation row
 * against every weight row (the integer part of the projection,
 * TensorMath.QuantizedRowsAvx.cs:80-87), for bit-exact verification. */
int fah_q8_block_dots_device(fah_context* context, const int8_t* q, const fah_weight* weight, int32_t* dots);

/* Decoder ------------------------------------------------------------------- */

typedef struct fah_decoder_config {
    int width;      /* qwen3.embedding_length, 1024 */
    int heads;      /* qwen3.attention.head_count, 16 */
    int kv_heads;   /* qwen3.attention.head_count_kv, 8 (heads == 2 or 4 * kv_heads) */
    int head_size;  /* qwen3.attention.key_length, 128 */
    int layers;     /* qwen3.block_count, 28 */
    int ffn;        /* ffn_gate rows, 3072 */
    int vocab;      /* token_embd rows, 151936 */
    float eps;      /* qwen3.attention.layer_norm_rms_epsilon, 1e-6 */
    float rope_base;/* qwen3.rope.freq_base, 1e6 */
    int capacity;   /* maximum positions (QwenDecoder ctor `capacity`, default 2048) */
} fah_decoder_config;

typedef struct fah_q8_host {
    const int8_t* quantized; /* [rows*cols] */
    const float* scales;     /* [rows*cols/32] */
    int rows, cols;
    /* Alternatively (quantized and scales NULL): the GGUF Q8_0 blocks,
     * rows*cols/32 x 34 bytes, as fah_weight_q8_upload_blocks takes them. */
    const uint8_t* blocks;
} fah_q8_host;

typedef struct fah_layer_host {
    fah_q8_host wq, wk, wv, wo, gate, up, down;
    const float* attn_norm; /* [width] */
    const float* q_norm;    /* [head_size] */
    const float* k_norm;    /* [head_size] */
    const float* ffn_norm;  /* [width] */
} fah_layer_host;

/* Device-resident QwenDecoder (src/FunAsrNet/QwenDecoder.cs:46-112): copies
 * every weight, builds the RoPE table with the C runtime's powf/cosf/sinf as
 * the reference does (QwenDecoder.cs:78-95), allocates the F16 KV cache for
 * `capacity` positions. `output` NULL means the lm_head is tied to
 * token_embd (QwenDecoder.cs:267). There is no reference counterpart for a
 * step-level seam: the C# side probes an optional IDecoderStepBackend at the
 * top of QwenDecoder.Decode, like IAttentionComputeBackend (TensorMath.cs:619).
 * Shapes: head_size 128, heads == 2 or 4 * kv_heads, width and
 * heads*head_size at most 4096, ffn at most 16384, all multiples of 32
 * (Qwen3-0.6B, 1.7B, 4B and 8B); others return FAH_ERROR_ARGUMENT.
 * Qwen3-0.6B's shape steps on the persistent kernel; other shapes on the
 * multi-kernel step, with multi-row inputs decoded row by row when ffn
 * exceeds 3072 (lock-step sessions and the step batcher need ffn <= 3072). */
int fah_decoder_create(fah_context* context, const fah_decoder_config* config, const fah_layer_host* layers,
                       const fah_q8_host* token_embd, const fah_q8_host* output, const float* output_norm,
                       fah_decoder** out);
int fah_decoder_destroy(fah_decoder* decoder);

/* QwenDecoder.Reset (QwenDecoder.cs:117) and RestorePrefix (:137): set the
 * decode position; cached K/V rows below it stay valid. */
int fah_decoder_set_position(fah_decoder* decoder, int position);
int fah_decoder_position(const fah_decoder* decoder, int* position);

/* QwenDecoder.Decode (QwenDecoder.cs:161-271): run `frames` embedding rows
 * (host, [frames*width]) through the decoder at the current position,
 * append their K/V, advance the position, and write the last row's logits
 * (host, [vocab]) when `logits` is not NULL. Throws (returns <0) when
 * position + frames exceeds capacity, as the reference does (:163-166). */
int fah_decoder_decode(fah_decoder* decoder, const float* embeddings, int frames, float* logits);

/* QwenDecoder.Embed (QwenDecoder.cs:143-152) for host tokens -> host rows. */
int fah_decoder_embed(fah_decoder* decoder, const int32_t* tokens, int count, float* out);

/* QwenDecoder.Greedy (QwenDecoder.cs:278-326) of the logits produced by the
 * last decode, computed on the device. */
int fah_decoder_greedy(fah_decoder* decoder, int32_t* token);

/* The FunAsr.Transcribe loop (src/FunAsrNet/FunAsr.cs:167-178) without the
 * tokenizer's end check: `steps` times Greedy -> Embed -> Decode(1), entirely
 * on the device (token feedback stays in device memory; one persistent
 * launch per step, or one captured HIP graph per step on the multi-kernel
 * path). The first token is the greedy choice of the logits of the
 * preceding decode. tokens[steps] receives the chosen tokens. */
int fah_decoder_generate(fah_decoder* decoder, int steps, int32_t* tokens);

/* A decoder session: shares `parent`'s device weights (they stay alive while
 * any session does) and has its own F16 KV cache of `capacity` positions,
 * RoPE table, position and token state. Replaces constructing one
 * QwenDecoder per FunAsr instance over the same model
 * (src/FunAsrNet/QwenDecoder.cs:46-112; sessions served by
 * src/FunAsrNet/BoundedInferencePool.cs:78), without a second weight copy.
 * Every fah_decoder_* call accepts a session. */
int fah_decoder_create_session(fah_decoder* parent, int capacity, fah_decoder** session);

/* The FunAsr.Transcribe loop (src/FunAsrNet/FunAsr.cs:167-178) of `count`
 * sessions in lock step: each step embeds every session's token, runs the
 * layers over all `count` rows at once (each weight read once per step) and
 * takes every row's greedy token. Each session's tokens equal those of
 * fah_decoder_generate on it alone. All sessions share one weight set
 * (fah_decoder_create_session) and each must hold logits from its last
 * decode. tokens[count][steps], row i for sessions[i]. Qwen3-0.6B-shaped
 * batches whose largest capacity is at most 320 run the layers in one
 * launch that needs every CU (the call holds the device meanwhile); if it
 * cannot complete, the call returns FAH_ERROR_DEVICE with every session back
 * at its starting position and without logits. */
int fah_decoder_generate_sessions(fah_decoder* const* sessions, int count, int steps, int32_t* tokens);

/* Cross-context step batching (the server side of FunAsr.Transcribe,
 * src/FunAsrNet/FunAsr.cs:167-178, run by the worker threads of
 * BoundedInferencePool, src/FunAsrNet/BoundedInferencePool.cs:22-230, over
 * the N contexts of SpeechRuntime, src/FunAsrNet.Server/SpeechRuntime.cs:16-23).
 * A batcher serves the sessions of one decoder's weights (the parent and its
 * fah_decoder_create_session sessions). Each worker thread calls
 * fah_batcher_step for its own session once per token; the steps requested
 * at the same time run as one lock-step batch (each weight read once per
 * step, up to 16 sessions), and each session's tokens equal those of
 * fah_decoder_generate on it alone. No reference counterpart: the reference
 * runs each context's decode separately.
 *
 * The first waiting thread collects: it runs the batch once every joined
 * session that is stepping has a step pending, 16 steps are pending, or
 * `window_us` has passed since it began to collect (sessions that never join
 * are batched with whatever arrives within the window). A joined session
 * with no step in the last batch counts as idle and is not waited for until
 * it requests a step again. Sessions must stay below `max_positions`
 * positions (at most 15360).
 *
 * Errors are per request: a session that cannot take its step (no logits,
 * its capacity or the batcher's bound reached, context destroyed) gets the
 * error at once and never enters a batch, and the other sessions' steps run
 * as usual. Only a device error of a batch reaches every request in it. */
int fah_batcher_create(fah_decoder* parent, int max_positions, int window_us, fah_batcher** out);
/* FAH_ERROR_STATE while a step is in progress. */
int fah_batcher_destroy(fah_batcher* batcher);
/* Register / unregister a session whose steps the collector waits for (a
 * worker joins when its session starts decoding and leaves when it stops). */
int fah_batcher_join(fah_batcher* batcher, fah_decoder* session);
int fah_batcher_leave(fah_batcher* batcher, fah_decoder* session);
/* One greedy step of `session` (Greedy -> Embed -> Decode(1), as
 * fah_decoder_generate(session, 1, token)), batched with the steps other
 * threads request at the same time; blocks until it has run (a waiting
 * thread yields in a loop for up to 3 ms, then sleeps; the collecting thread
 * yields for up to 0.5 ms between arrivals). The session must hold logits
 * from its last decode. */
int fah_batcher_step(fah_batcher* batcher, fah_decoder* session, int32_t* token);
/* Batches run and session steps served (successful steps) so far. */
int fah_batcher_stats(fah_batcher* batcher, int64_t* batches, int64_t* rows);

/* Overwrite cached K/V rows [0, positions) of one layer from fp16 bit
 * patterns laid out [positions][kv_heads*head_size] (long-context stress
 * inputs; no reference counterpart). */
int fah_decoder_kv_write(fah_decoder* decoder, int layer, const uint16_t* keys, const uint16_t* values,
                         int positions);
/* Read cached K/V rows [0, positions) of one layer as fp16 bits. */
int fah_decoder_kv_read(fah_decoder* decoder, int layer, uint16_t* keys, uint16_t* values, int positions);

/* Copy the newest value of an intermediate activation of the last decoded
 * row (the reference's Trace snapshots, QwenDecoder.cs:248-251, 269):
 * which = 0 layer output x [width], 1 raw q|k|v projections [q+2kv],
 * 2 attention output [heads*head_size], 3 post-attention residual a
 * [width], 4 SwiGLU output [ffn]; values are those of the last layer. */
int fah_decoder_trace(fah_decoder* decoder, int which, float* out, int count);

/* Phase timestamps (100 MHz device clock) of the last persistent step:
 * one row of 480 stamps per workgroup (256 rows): [1+16l .. 16+16l] the
 * phase boundaries of layer l
 * (input gathered, input quantised, output stored, attention sub-steps),
 * [1+16L] lm_head done, [2+16L] greedy token written. Only
 * recorded when FAH_TIMELINE=1 at creation (FAH_DECLINED otherwise); the
 * rocprof-style per-op timing of the reference's LinearMeasured callback
 * (src/FunAsrNet/TensorMath.cs:37-40) for a single-launch step. */
int fah_decoder_timeline(fah_decoder* decoder, uint64_t* ticks, int count);

/* Device time of the attention kernels (scores, softmax, value sums) of the
 * multi-kernel steps run since the last call, summed over layers and steps,
 * and the number of steps; reading resets both. Only recorded when
 * FAH_ATTENTION_TIMES=1 at creation (the steps then run one by one with
 * HIP events around each layer's attention, outside graphs; FAH_DECLINED
 * otherwise, and for steps of the persistent kernel). The per-operation
 * timing the reference reports through TensorMath.LinearMeasured
 * (src/FunAsrNet/TensorMath.cs:37-40), for the attention of long caches. */
int fah_decoder_attention_time(fah_decoder* decoder, double* milliseconds, int* steps);

/* Test hook for the persistent step's failure path: presets the device
 * error word, so that the next persistent launch of this decoder ends at its
 * entry check (every workgroup exits normally) and the call reports
 * FAH_ERROR_DEVICE. The failed call restores the device state from the
 * host's (position, epoch, empty history) and drops its logits, as after an
 * exchange that timed out. If the decoder's next device step is a lock-step
 * call that runs the layers in one launch (fah_decoder_generate_sessions or a
 * batcher batch), that launch fails the same way instead: every session of
 * the call returns to its starting position without logits. FAH_DECLINED
 * when the decoder does not run the persistent step. No reference
 * counterpart (the reference's failure path is a thrown exception,
 * Vk.cs:57-61). */
int fah_decoder_fail_next_step(fah_decoder* decoder);

/* 2 when decode steps run as one persistent launch with XCD-local roles
 * (workgroups take their role from the XCD they run on, and hand data to
 * workgroups of the same XCD through its L2), 1 for the persistent launch
 * with roles by workgroup index (after a launch found the XCD dealing it
 * relies on broken, or with FAH_LOCAL_L2=0 in the environment at creation),
 * 0 for the per-kernel graph path (FAH_PERSISTENT=0 at creation). A
 * persistent decoder runs the steps of positions below 5120 (below 483 with
 * every earlier K/V row held by the attention workgroups, from 483 with the
 * long-cache attention) on the persistent kernel and later steps on the
 * per-kernel graph path; FAH_PERSISTENT_POSITIONS and FAH_LONG_FROM at
 * creation move the two switches. */
int fah_decoder_persistent(const fah_decoder* decoder);

/* Device bytes of the weights streamed per decoded token (all projections
 * plus the lm_head, Q8_0 int8 and scale planes as stored). */
int64_t fah_decoder_weight_bytes(const fah_decoder* decoder);

#ifdef __cplusplus
}
#endif
#endif
