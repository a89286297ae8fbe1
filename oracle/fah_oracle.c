/*
 * CPU oracle for the Qwen3 Q8_0 decoder path -- TEST INFRASTRUCTURE ONLY.
 *
 * A scalar C restatement of the reference's x64 C# path. Tests compare the
 * HIP library against it; the product never links or calls it.
 * Each function names the reference lines (paths relative to the reference
 * checkout) whose arithmetic and operation order it follows. Compile with
 * -ffp-contract=off so that no multiply-add is fused: .NET's RyuJIT does not
 * contract a*b+c either.
 */
#include "fah_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static _Thread_local char g_error[256];

static int fail(const char* message) {
    snprintf(g_error, sizeof g_error, "%s", message);
    return -1;
}

const char* oracle_last_error(void) { return g_error; }

int oracle_set_threads(int threads) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
    return omp_get_max_threads();
#else
    (void)threads;
    return 1;
#endif
}

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline double u2d(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }

/* ---------------------------------------------------------------------
 * IEEE binary16 conversions (System.Half semantics).
 * ------------------------------------------------------------------- */

/* Exact widening, quieting NaN: the (float)Half conversion used by
 * UnpackQ8Model for non-normal scales (src/FunAsrNet/TensorMath.Q8Model.cs:34-36)
 * and by the normal fast path there (exact exponent rebias). */
float oracle_half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exponent = (h >> 10) & 0x1fu;
    uint32_t mantissa = h & 0x3ffu;
    if (exponent == 0) {
        float magnitude = (float)mantissa * (1.0f / 16777216.0f); /* exact: m * 2^-24 */
        return u2f(sign | f2u(magnitude));
    }
    if (exponent == 31) {
        return u2f(mantissa == 0 ? (sign | 0x7f800000u) : (sign | 0x7fc00000u | (mantissa << 13)));
    }
    return u2f(sign | ((exponent + 112u) << 23) | (mantissa << 13));
}

/* Round-to-nearest-even narrowing, the (Half)float conversion. */
uint16_t oracle_float_to_half(float f) {
    uint32_t x = f2u(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t a = x & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to infinity */
    if (a >= 0x38800000u) {                                   /* normal binary16 range */
        uint32_t r = a + 0xfffu + ((a >> 13) & 1u);
        return (uint16_t)(sign | ((r - 0x38000000u) >> 13));
    }
    uint32_t exponent = a >> 23;
    if (exponent < 102) return sign; /* below half of the smallest subnormal step */
    uint32_t mantissa = (a & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126u - exponent; /* 14..24 */
    uint32_t r = mantissa >> shift;
    uint32_t rem = mantissa & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (r & 1u))) r++;
    return (uint16_t)(sign | r);
}

/* src/FunAsrNet/TensorMath.Half.cs:18-53: normal-range integer rounding,
 * everything else through (float)(Half)x. */
float oracle_round_half(float f) {
    uint32_t bits = f2u(f);
    uint32_t a = bits & 0x7fffffffu;
    if (a >= 0x38800000u && a < 0x477fe000u) {
        return u2f((bits + 0xfffu + ((bits >> 13) & 1u)) & 0xffffe000u);
    }
    return oracle_half_to_float(oracle_float_to_half(f));
}

void oracle_round_half_copy(const float* x, int64_t n, float* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_round_half(x[i]);
}

/* ---------------------------------------------------------------------
 * exp: src/FunAsrNet/TensorMath.ExpAvx.cs:83-116 (clamp to +-104, double
 * range reduction x = n ln2 + r, degree-8 Taylor polynomial in FMA form,
 * scale by 2^n, narrow to float). NaN propagates through the clamp.
 * ------------------------------------------------------------------- */
float oracle_exp(float value) {
    if (value != value) return value;
    float clamped = value < -104.0f ? -104.0f : (value > 104.0f ? 104.0f : value);
    double x = (double)clamped;
    double n = rint(x * 1.4426950408889634074);
    double r = fma(n, -0.6931471805599453094, x);
    double square = r * r;
    double fourth = square * square;
    double p23 = fma(r, 1.0 / 6, 0.5);
    double p45 = fma(r, 1.0 / 120, 1.0 / 24);
    double p67 = fma(r, 1.0 / 5040, 1.0 / 720);
    double low = fma(square, p23, 1.0 + r);
    double high = fma(square, fma(square, 1.0 / 40320, p67), p45);
    double exponential = fma(fourth, high, low);
    int64_t biased = (int64_t)(int32_t)n + 1023;
    double scale = u2d((uint64_t)biased << 52);
    return (float)(exponential * scale);
}

/* ---------------------------------------------------------------------
 * Q8_0
 * ------------------------------------------------------------------- */

/* src/FunAsrNet/TensorMath.Q8Model.cs:15-39: 34-byte blocks, little-endian
 * fp16 scale then 32 signed bytes. */
int oracle_unpack_q8(const uint8_t* raw, int64_t blocks, int8_t* q, float* scales) {
    if (blocks < 0) return fail("Q8 model block dimensions differ");
    for (int64_t b = 0; b < blocks; ++b) {
        const uint8_t* block = raw + b * 34;
        uint16_t bits = (uint16_t)(block[0] | (block[1] << 8));
        scales[b] = oracle_half_to_float(bits);
        memcpy(q + b * 32, block + 2, 32);
    }
    return 0;
}

/* .NET 9+ float->int conversion saturates: NaN -> 0, out of range -> limits. */
static inline int32_t saturate_to_int(float v) {
    if (v != v) return 0;
    if (v >= 2147483648.0f) return INT32_MAX;
    if (v <= -2147483648.0f) return INT32_MIN;
    return (int32_t)v;
}

static inline int8_t quantize_one(float v, float inverse) {
    /* MathF.Round(x*inv, MidpointRounding.AwayFromZero) is C roundf. */
    int32_t i = saturate_to_int(roundf(v * inverse));
    if (i < -127) i = -127;
    if (i > 127) i = 127;
    return (int8_t)i;
}

/* Math.Max(float, float): a NaN argument wins. */
static inline float net_max(float a, float b) {
    if (a != a) return a;
    if (b != b) return b;
    return b > a ? b : a;
}

/* src/FunAsrNet/TensorMath.cs:397-411 (scalar formula) which
 * TensorMath.QuantizeAvx.cs:15-72 reproduces exactly: per 32-block
 * d = amax/127f, inv = d==0 ? 0 : 1f/d, q = clamp(round_away(x*inv), +-127).
 * The scale d stays fp32. */
int oracle_quantize(const float* x, int64_t n, int8_t* q, float* scales) {
    if (n % 32 != 0) return fail("Quantization needs matching complete blocks");
    for (int64_t b = 0; b < n / 32; ++b) {
        const float* in = x + b * 32;
        float max = 0.0f;
        for (int i = 0; i < 32; ++i) max = net_max(max, fabsf(in[i]));
        float d = max / 127.0f;
        float inverse = d == 0.0f ? 0.0f : 1.0f / d;
        scales[b] = d;
        for (int i = 0; i < 32; ++i) q[b * 32 + i] = quantize_one(in[i], inverse);
    }
    return 0;
}

/* Exact 32-term integer dot (TensorMath.QuantizedRowsAvx.cs:80-87,
 * TensorMath.Avx.cs:180-188): weights may be -128, activations in [-127,127]. */
int32_t oracle_block_dot(const int8_t* w, const int8_t* x) {
    int32_t dot = 0;
    for (int i = 0; i < 32; ++i) dot += (int32_t)w[i] * (int32_t)x[i];
    return dot;
}

void oracle_q8_block_dots(const int8_t* xq, const int8_t* wq, int rows, int cols, int32_t* dots) {
    int blocks = cols / 32;
#pragma omp parallel for schedule(static) if (rows >= 256)
    for (int r = 0; r < rows; ++r)
        for (int b = 0; b < blocks; ++b)
            dots[(int64_t)r * blocks + b] = oracle_block_dot(wq + (int64_t)r * cols + b * 32, xq + b * 32);
}

/* Per row, per frame: sum = 0f; sum += ((float)dot_b * ws_b) * xs_b over the
 * blocks in order, then bias + sum.
 * src/FunAsrNet/TensorMath.QuantizedRowsAvx.cs:27-58 (frames == 1),
 * TensorMath.QuantizedGroupAvx.cs:199-287, TensorMath.QuantizedVnni.cs:77-126
 * and TensorMath.Avx.cs:122-163 (frames > 1) all keep this order;
 * TensorMath.cs:458-489 is the scalar statement. */
void oracle_q8_gemv_quantized(const int8_t* xq, const float* xs, int frames,
                              const int8_t* wq, const float* ws, int rows, int cols,
                              const float* bias, float* out) {
    int blocks = cols / 32;
#pragma omp parallel for schedule(static) if ((int64_t)rows * frames >= 256)
    for (int r = 0; r < rows; ++r) {
        const int8_t* wrow = wq + (int64_t)r * cols;
        const float* wscale = ws + (int64_t)r * blocks;
        for (int t = 0; t < frames; ++t) {
            const int8_t* x = xq + (int64_t)t * cols;
            const float* xscale = xs + (int64_t)t * blocks;
            float sum = 0.0f;
            for (int b = 0; b < blocks; ++b) {
                float dot = (float)oracle_block_dot(wrow + b * 32, x + b * 32);
                float scaled = dot * wscale[b];
                scaled = scaled * xscale[b];
                sum = sum + scaled;
            }
            out[(int64_t)t * rows + r] = (bias ? bias[r] : 0.0f) + sum;
        }
    }
}

/* src/FunAsrNet/TensorMath.cs:79-200 (Linear, Q8 weights, no backend):
 * quantise the input once, then the ordered block sums. */
int oracle_q8_linear(const float* input, int frames, const int8_t* wq, const float* ws,
                     int rows, int cols, const float* bias, float* out) {
    if (cols % 32 != 0 || frames < 0 || rows < 0) return fail("Invalid row-major Q8 dimensions");
    int64_t n = (int64_t)frames * cols;
    int8_t* q = (int8_t*)malloc(n > 0 ? (size_t)n : 1);
    float* s = (float*)malloc(n > 0 ? (size_t)(n / 32) * sizeof(float) : sizeof(float));
    if (!q || !s) { free(q); free(s); return fail("out of memory"); }
    oracle_quantize(input, n, q, s);
    oracle_q8_gemv_quantized(q, s, frames, wq, ws, rows, cols, bias, out);
    free(q);
    free(s);
    return 0;
}

/* src/FunAsrNet/Gguf.cs:340-344: q[j] * scale[j/32], (float)sbyte * float. */
void oracle_embed_row(const int8_t* q, const float* scales, int cols, int token, float* out) {
    int64_t offset = (int64_t)token * cols;
    for (int j = 0; j < cols; ++j) out[j] = (float)q[offset + j] * scales[(offset + j) / 32];
}

/* ---------------------------------------------------------------------
 * Element-wise and reductions
 * ------------------------------------------------------------------- */

/* RMSNorm: src/FunAsrNet/TensorMath.Elementwise.cs:26-100 with rms=true,
 * bias=null (QwenDecoder.cs:354-360). Sum of squares in double with two
 * Vector128<double> accumulators holding lanes (4i, 4i+1) and (4i+2, 4i+3),
 * combined as (s0+s2)+(s1+s3); inverse = 1f / sqrtf((float)(sum/width) + eps);
 * y = ((x - 0f) * inverse) * scale. */
int oracle_rms_norm(const float* x, int64_t n, int width, const float* scale, float eps, float* y) {
    if (width <= 0 || n % width != 0) return fail("Invalid normalization dimensions");
    for (int64_t offset = 0; offset < n; offset += width) {
        const float* row = x + offset;
        double s0 = 0, s1 = 0, s2 = 0, s3 = 0;
        int k = 0;
        for (; k <= width - 4; k += 4) {
            double a = (double)row[k] - 0.0, b = (double)row[k + 1] - 0.0;
            double c = (double)row[k + 2] - 0.0, d = (double)row[k + 3] - 0.0;
            s0 = s0 + a * a;
            s1 = s1 + b * b;
            s2 = s2 + c * c;
            s3 = s3 + d * d;
        }
        double variance = (s0 + s2) + (s1 + s3);
        for (; k < width; ++k) {
            double z = (double)row[k] - 0.0;
            variance = variance + z * z;
        }
        float inverse = 1.0f / sqrtf((float)(variance / width) + eps);
        for (int j = 0; j < width; ++j) y[offset + j] = ((row[j] - 0.0f) * inverse) * scale[j];
    }
    return 0;
}

/* src/FunAsrNet/QwenDecoder.cs:78-95: f_i = MathF.Pow(base, -2f*i/headSize),
 * angle = t * f_i (float), cos/sin via the C runtime (MathF forwards there). */
void oracle_rope_table(int capacity, int head_size, float base, float* cos_out, float* sin_out) {
    int half = head_size / 2;
    float* frequencies = (float*)malloc(sizeof(float) * (size_t)half);
    for (int i = 0; i < half; ++i) frequencies[i] = powf(base, (-2.0f * (float)i) / (float)head_size);
    for (int t = 0; t < capacity; ++t) {
        for (int i = 0; i < half; ++i) {
            float angle = (float)t * frequencies[i];
            cos_out[(int64_t)t * half + i] = cosf(angle);
            sin_out[(int64_t)t * half + i] = sinf(angle);
        }
    }
    free(frequencies);
}

/* src/FunAsrNet/TensorMath.Rope.cs:14-55: x_i' = a*c - b*s,
 * x_{i+half}' = a*s + b*c, no fused multiply-add. */
void oracle_rotate_half(float* x, const float* cosine, const float* sine, int half) {
    for (int i = 0; i < half; ++i) {
        float a = x[i], b = x[i + half], c = cosine[i], s = sine[i];
        float ac = a * c, bs = b * s, as = a * s, bc = b * c;
        x[i] = ac - bs;
        x[i + half] = as + bc;
    }
}

/* src/FunAsrNet/TensorMath.SoftmaxAvx.cs:11-58 (x64, length >= 8) and the
 * scalar branch TensorMath.cs:587-604 (length < 8), which coincide when no
 * full 8-group exists. Max with Math.Max semantics; e = exp(x - max); the
 * denominator accumulates in double with 8 lane accumulators (one per
 * position mod 8), combined as ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)), then
 * the tail sequentially; inverse = (float)(1 / sum); x *= inverse. */
void oracle_softmax(float* x, int n) {
    float max = -INFINITY;
    int i = 0;
    if (n >= 8) {
        float lanes[8];
        for (int j = 0; j < 8; ++j) lanes[j] = -INFINITY;
        for (; i <= n - 8; i += 8)
            for (int j = 0; j < 8; ++j) lanes[j] = net_max(lanes[j], x[i + j]);
        for (int j = 0; j < 8; ++j) max = net_max(max, lanes[j]);
    }
    for (; i < n; ++i) max = net_max(max, x[i]);
    double l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    i = 0;
    if (n >= 8) {
        for (; i <= n - 8; i += 8)
            for (int j = 0; j < 8; ++j) {
                float e = oracle_exp(x[i + j] - max);
                x[i + j] = e;
                l[j] = l[j] + (double)e;
            }
    }
    double sum = ((l[0] + l[4]) + (l[1] + l[5])) + ((l[2] + l[6]) + (l[3] + l[7]));
    for (; i < n; ++i) {
        float e = oracle_exp(x[i] - max);
        x[i] = e;
        sum = sum + (double)e;
    }
    float inverse = (float)(1.0 / sum);
    for (i = 0; i < n; ++i) x[i] = x[i] * inverse;
}

/* The double reference the reference's FP32 device checks compare against
 * (tools/FunAsrNet.Benchmarks/FloatGpuChecks.cs compares with a CPU linear
 * at 2e-4 x max(1, |expected|); TensorMath.cs:79-200 computes
 * y = x W^T + b with Weight.Values rows of `cols` floats). */
void oracle_float_linear_f64(const float* x, int frames, int cols, const float* w, int rows, const float* bias,
                             double* out) {
#pragma omp parallel for schedule(static) if ((long)frames * rows * cols > 1000000)
    for (int index = 0; index < frames * rows; ++index) {
        int f = index / rows, n = index % rows;
        const float* xr = x + (int64_t)f * cols;
        const float* wr = w + (int64_t)n * cols;
        double sum = 0.0;
        for (int k = 0; k < cols; ++k) sum += (double)xr[k] * (double)wr[k];
        out[index] = sum + (bias ? (double)bias[n] : 0.0);
    }
}

/* tools/FunAsrNet.Benchmarks/AttentionGpuChecks.cs (Reference): per head and
 * query row, double dot products divided by sqrt(size), max-shifted exp,
 * probabilities and weighted values in double (the semantics of
 * TensorMath.cs:646-666 AttentionReference). */
void oracle_attention_f64(const float* q, const float* k, const float* v, int frames, int width, int heads,
                          double* out) {
    int size = width / heads;
    double divisor = sqrt((double)size);
#pragma omp parallel for schedule(dynamic)
    for (int index = 0; index < frames * heads; ++index) {
        int t = index / heads, h = index % heads, at = t * width + h * size;
        double* scores = (double*)malloc(sizeof(double) * (size_t)frames);
        double max = -INFINITY;
        for (int s = 0; s < frames; ++s) {
            double d = 0.0;
            for (int c = 0; c < size; ++c) d += (double)q[at + c] * (double)k[s * width + h * size + c];
            scores[s] = d / divisor;
            if (scores[s] > max) max = scores[s];
        }
        double sum = 0.0;
        for (int s = 0; s < frames; ++s) {
            scores[s] = exp(scores[s] - max);
            sum += scores[s];
        }
        for (int c = 0; c < size; ++c) {
            double acc = 0.0;
            for (int s = 0; s < frames; ++s) acc += scores[s] / sum * (double)v[s * width + h * size + c];
            out[at + c] = acc;
        }
        free(scores);
    }
}

/* src/FunAsrNet/TensorMath.Elementwise.cs:167-196: g / (1 + exp(-g)) * up. */
void oracle_silu_multiply(float* gate, const float* up, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        float g = gate[i];
        float denominator = 1.0f + oracle_exp(-g);
        float silu = g / denominator;
        gate[i] = silu * up[i];
    }
}

/* src/FunAsrNet/TensorMath.cs:508-525. */
void oracle_add(float* target, const float* other, int64_t n) {
    for (int64_t i = 0; i < n; ++i) target[i] = target[i] + other[i];
}

/* src/FunAsrNet/AudioKernels.cs:94-147 (Vector256 branch) and
 * TensorMath.AttentionAvx.cs:74-160: eight lane accumulators over
 * channel groups of 8 (product then add), lanes folded lower+upper, then
 * Vector128.Sum taken as (b0+b1)+(b2+b3), then the channel tail. */
float oracle_dot(const float* a, const float* b, int n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i <= n - 8; i += 8)
        for (int j = 0; j < 8; ++j) {
            float p = a[i + j] * b[i + j];
            acc[j] = acc[j] + p;
        }
    float b0 = acc[0] + acc[4], b1 = acc[1] + acc[5], b2 = acc[2] + acc[6], b3 = acc[3] + acc[7];
    float result = (b0 + b1) + (b2 + b3);
    for (; i < n; ++i) {
        float p = a[i] * b[i];
        result = result + p;
    }
    return result;
}

/* src/FunAsrNet/QwenDecoder.cs:278-326: first index of a strictly greater
 * value; NaN never wins; a NaN first element returns 0. */
int32_t oracle_greedy(const float* logits, int64_t n) {
    int64_t best = 0;
    for (int64_t i = 1; i < n; ++i)
        if (logits[i] > logits[best]) best = i;
    return (int32_t)best;
}

/* Causal GQA attention for `frames` query rows starting at `position`.
 * Decode (frames == 1): src/FunAsrNet/TensorMath.DecoderAttention.cs:17-52
 * with AttentionScores2x4Avx / AttentionValues2Avx
 * (TensorMath.AttentionAvx.cs:74-224). Prefill: QwenDecoder.cs:206-224 with
 * AudioKernels.Dot and AttentionValues (TensorMath.Attention.cs:140-213).
 * Both give, per query head and channel: scores = dot/sqrtf(size), softmax,
 * then out[c] = sum over t of v[t][c]*p[t] in time order from 0f. */
void oracle_attention(const float* q, const float* kcache, const float* vcache,
                      int frames, int position, int heads, int kv_heads, int head_size,
                      float* out) {
    int kv_width = kv_heads * head_size, q_width = heads * head_size, group = heads / kv_heads;
    float divisor = sqrtf((float)head_size);
#pragma omp parallel for schedule(dynamic) if (frames * heads >= 8)
    for (int index = 0; index < frames * heads; ++index) {
        int t = index / heads, head = index % heads, kh = head / group, end = position + t + 1;
        float* scores = (float*)malloc(sizeof(float) * (size_t)end);
        const float* query = q + (int64_t)t * q_width + (int64_t)head * head_size;
        for (int s = 0; s < end; ++s)
            scores[s] = oracle_dot(query, kcache + (int64_t)s * kv_width + (int64_t)kh * head_size, head_size) / divisor;
        oracle_softmax(scores, end);
        float* o = out + (int64_t)t * q_width + (int64_t)head * head_size;
        for (int c = 0; c < head_size; ++c) {
            float sum = 0.0f;
            for (int s = 0; s < end; ++s) {
                float p = vcache[(int64_t)s * kv_width + (int64_t)kh * head_size + c] * scores[s];
                sum = sum + p;
            }
            o[c] = sum;
        }
        free(scores);
    }
}

/* ---------------------------------------------------------------------
 * Decoder: src/FunAsrNet/QwenDecoder.cs:46-271
 * ------------------------------------------------------------------- */
struct oracle_decoder {
    oracle_model model;
    int capacity, position;
    float** keys;   /* [layers] -> [capacity][kv_width] */
    float** values;
    float* rope_cos; /* [capacity][head_size/2] */
    float* rope_sin;
    /* Optional capture of RMSNorm input rows (tests only): width-wide rows
     * (attention, ffn and output norms) and head rows (QK-norms). */
    float* cap_wide; int64_t cap_wide_max, cap_wide_n;
    float* cap_head; int64_t cap_head_max, cap_head_n;
};

void oracle_decoder_capture_norms(oracle_decoder* d, float* wide, int64_t wide_rows, float* heads, int64_t head_rows) {
    d->cap_wide = wide; d->cap_wide_max = wide ? wide_rows : 0; d->cap_wide_n = 0;
    d->cap_head = heads; d->cap_head_max = heads ? head_rows : 0; d->cap_head_n = 0;
}

int64_t oracle_decoder_captured(const oracle_decoder* d, int heads) { return heads ? d->cap_head_n : d->cap_wide_n; }

static void capture_rows(float* dst, int64_t max, int64_t* n, const float* rows, int64_t count, int width) {
    if (!dst) return;
    if (count > max - *n) count = max - *n;
    if (count <= 0) return;
    memcpy(dst + *n * width, rows, sizeof(float) * (size_t)(count * width));
    *n += count;
}

oracle_decoder* oracle_decoder_create(const oracle_model* model, int capacity) {
    if (!model || capacity < 1 || model->heads % model->kv_heads != 0) { fail("Invalid GQA head counts"); return NULL; }
    oracle_decoder* d = (oracle_decoder*)calloc(1, sizeof *d);
    d->model = *model;
    d->capacity = capacity;
    int kv_width = model->kv_heads * model->head_size;
    d->keys = (float**)calloc((size_t)model->layers, sizeof(float*));
    d->values = (float**)calloc((size_t)model->layers, sizeof(float*));
    for (int l = 0; l < model->layers; ++l) {
        d->keys[l] = (float*)calloc((size_t)capacity * kv_width, sizeof(float));
        d->values[l] = (float*)calloc((size_t)capacity * kv_width, sizeof(float));
    }
    int half = model->head_size / 2;
    d->rope_cos = (float*)malloc(sizeof(float) * (size_t)capacity * half);
    d->rope_sin = (float*)malloc(sizeof(float) * (size_t)capacity * half);
    oracle_rope_table(capacity, model->head_size, model->rope_base, d->rope_cos, d->rope_sin);
    return d;
}

void oracle_decoder_destroy(oracle_decoder* d) {
    if (!d) return;
    for (int l = 0; l < d->model.layers; ++l) { free(d->keys[l]); free(d->values[l]); }
    free(d->keys);
    free(d->values);
    free(d->rope_cos);
    free(d->rope_sin);
    free(d);
}

void oracle_decoder_reset(oracle_decoder* d) { d->position = 0; }
int oracle_decoder_position(const oracle_decoder* d) { return d->position; }
int oracle_decoder_set_position(oracle_decoder* d, int position) {
    if (position < 0 || position > d->capacity) return fail("position out of range");
    d->position = position;
    return 0;
}
float* oracle_decoder_keys(oracle_decoder* d, int layer) { return d->keys[layer]; }
float* oracle_decoder_values(oracle_decoder* d, int layer) { return d->values[layer]; }

/* QwenDecoder.cs:143-152 */
int oracle_decoder_embed(const oracle_decoder* d, const int32_t* tokens, int count, float* out) {
    const oracle_q8* e = &d->model.token_embd;
    for (int i = 0; i < count; ++i) {
        if (tokens[i] < 0 || tokens[i] >= e->rows) return fail("token out of range");
        oracle_embed_row(e->q, e->scales, e->cols, tokens[i], out + (int64_t)i * e->cols);
    }
    return 0;
}

static void linear(const oracle_q8* w, const float* x, int frames, float* out) {
    oracle_q8_linear(x, frames, w->q, w->scales, w->rows, w->cols, NULL, out);
}

/* QwenDecoder.cs:161-271. logits may be NULL (outputLogits = false). */
int oracle_decoder_decode(oracle_decoder* d, const float* embeddings, int frames, float* logits) {
    const oracle_model* m = &d->model;
    if (frames < 1 || d->position + frames > d->capacity)
        return fail("Decoder context exhausted or invalid embeddings");
    int width = m->width, hs = m->head_size, half = hs / 2;
    int q_width = m->heads * hs, kv_width = m->kv_heads * hs;
    size_t fw = (size_t)frames * width;
    float* x = (float*)malloc(sizeof(float) * fw);
    float* h = (float*)malloc(sizeof(float) * fw);
    float* a = (float*)malloc(sizeof(float) * fw);
    float* q = (float*)malloc(sizeof(float) * (size_t)frames * q_width);
    float* qn = (float*)malloc(sizeof(float) * (size_t)frames * q_width);
    float* k = (float*)malloc(sizeof(float) * (size_t)frames * kv_width);
    float* kn = (float*)malloc(sizeof(float) * (size_t)frames * kv_width);
    float* v = (float*)malloc(sizeof(float) * (size_t)frames * kv_width);
    float* attn = (float*)malloc(sizeof(float) * (size_t)frames * q_width);
    float* gate = (float*)malloc(sizeof(float) * (size_t)frames * m->ffn);
    float* up = (float*)malloc(sizeof(float) * (size_t)frames * m->ffn);
    int8_t* xq = (int8_t*)malloc((size_t)frames * (m->ffn > q_width ? m->ffn : q_width));
    float* xs = (float*)malloc(sizeof(float) * (size_t)frames * (m->ffn > q_width ? m->ffn : q_width) / 32);
    memcpy(x, embeddings, sizeof(float) * fw);
    for (int layer = 0; layer < m->layers; ++layer) {
        const oracle_layer* L = &m->layer[layer];
        capture_rows(d->cap_wide, d->cap_wide_max, &d->cap_wide_n, x, frames, width);
        oracle_rms_norm(x, (int64_t)fw, width, L->attn_norm, m->eps, h);
        /* LinearMany: one shared quantisation (TensorMath.QuantizedGroupAvx.cs:105-190) */
        oracle_quantize(h, (int64_t)fw, xq, xs);
        oracle_q8_gemv_quantized(xq, xs, frames, L->wq.q, L->wq.scales, L->wq.rows, width, NULL, q);
        oracle_q8_gemv_quantized(xq, xs, frames, L->wk.q, L->wk.scales, L->wk.rows, width, NULL, k);
        oracle_q8_gemv_quantized(xq, xs, frames, L->wv.q, L->wv.scales, L->wv.rows, width, NULL, v);
        capture_rows(d->cap_head, d->cap_head_max, &d->cap_head_n, q, (int64_t)frames * m->heads, hs);
        capture_rows(d->cap_head, d->cap_head_max, &d->cap_head_n, k, (int64_t)frames * m->kv_heads, hs);
        oracle_rms_norm(q, (int64_t)frames * q_width, hs, L->q_norm, m->eps, qn);
        oracle_rms_norm(k, (int64_t)frames * kv_width, hs, L->k_norm, m->eps, kn);
        for (int t = 0; t < frames; ++t) {
            const float* c = d->rope_cos + (int64_t)(d->position + t) * half;
            const float* s = d->rope_sin + (int64_t)(d->position + t) * half;
            for (int head = 0; head < m->heads; ++head) oracle_rotate_half(qn + ((int64_t)t * m->heads + head) * hs, c, s, half);
            for (int head = 0; head < m->kv_heads; ++head) oracle_rotate_half(kn + ((int64_t)t * m->kv_heads + head) * hs, c, s, half);
        }
        oracle_round_half_copy(kn, (int64_t)frames * kv_width, d->keys[layer] + (int64_t)d->position * kv_width);
        oracle_round_half_copy(v, (int64_t)frames * kv_width, d->values[layer] + (int64_t)d->position * kv_width);
        oracle_attention(qn, d->keys[layer], d->values[layer], frames, d->position, m->heads, m->kv_heads, hs, attn);
        linear(&L->wo, attn, frames, a);
        oracle_add(a, x, (int64_t)fw);
        capture_rows(d->cap_wide, d->cap_wide_max, &d->cap_wide_n, a, frames, width);
        oracle_rms_norm(a, (int64_t)fw, width, L->ffn_norm, m->eps, h);
        oracle_quantize(h, (int64_t)fw, xq, xs);
        oracle_q8_gemv_quantized(xq, xs, frames, L->gate.q, L->gate.scales, L->gate.rows, width, NULL, gate);
        oracle_q8_gemv_quantized(xq, xs, frames, L->up.q, L->up.scales, L->up.rows, width, NULL, up);
        oracle_silu_multiply(gate, up, (int64_t)frames * m->ffn);
        linear(&L->down, gate, frames, x);
        oracle_add(x, a, (int64_t)fw);
    }
    d->position += frames;
    if (logits) {
        float* last = x + (size_t)(frames - 1) * width;
        capture_rows(d->cap_wide, d->cap_wide_max, &d->cap_wide_n, last, 1, width);
        oracle_rms_norm(last, width, width, m->output_norm, m->eps, h);
        const oracle_q8* out = m->output.q ? &m->output : &m->token_embd;
        linear(out, h, 1, logits);
    }
    free(x); free(h); free(a); free(q); free(qn); free(k); free(kn); free(v);
    free(attn); free(gate); free(up); free(xq); free(xs);
    return 0;
}


/* ---- RMSNorm square-sum order (tests only) ---------------------------------
 *
 * The reference sums an RMSNorm row's squares in double in four chains
 * (TensorMath.Elementwise.cs:58-71, restated in oracle_rms_norm). The GPU
 * kernels sum them as pairwise trees and use the tree's float mean only when
 * its error bound cannot reach a float rounding boundary (rms_mean in
 * fah_device.h), otherwise the reference's chains. These functions restate
 * both and count how often the orders' float means differ. */

static double pair_tree(const double* v, int n) {
    if (n == 1) return v[0];
    return pair_tree(v, n / 2) + pair_tree(v + n / 2, n / 2);
}

/* The GPU kernels' square sum of one row. Width 128 (QK-norm): 64-lane wave
 * trees over channels 0-63 and 64-127, the low one first. Other widths (a
 * multiple of 4, at most 4096; the 1024-wide layer norms): 256 threads, thread
 * t holding values 4t + 1024c and summing ((0 + (a^2 + b^2)) + (c^2 + d^2)) per
 * chunk c in order; a pairwise tree over each 64-lane wave (DPP steps within
 * rows of 16 lanes, then (r0 + r16) + (r32 + r48)); the four wave sums added
 * in order from 0. */
double oracle_sum_sq_gpu_tree(const float* x, int width) {
    double lane[256];
    if (width == 128) {
        for (int c = 0; c < 128; ++c) lane[c] = (double)x[c] * (double)x[c];
        return pair_tree(lane, 64) + pair_tree(lane + 64, 64);
    }
    for (int t = 0; t < 256; ++t) {
        double sq = 0.0;
        for (int c = 0; c < 4; ++c) {
            const int e = c * 1024 + 4 * t;
            if (e >= width) continue;
            const double a = x[e], b = x[e + 1], cc = x[e + 2], dd = x[e + 3];
            sq = sq + (a * a + b * b);
            sq = sq + (cc * cc + dd * dd);
        }
        lane[t] = sq;
    }
    double total = 0.0;
    for (int w = 0; w < 4; ++w) total = total + pair_tree(lane + 64 * w, 64);
    return total;
}

/* The reference's square sum (oracle_rms_norm's chains). */
double oracle_sum_sq_reference(const float* x, int width) {
    double s0 = 0, s1 = 0, s2 = 0, s3 = 0;
    int k = 0;
    for (; k <= width - 4; k += 4) {
        double a = x[k], b = x[k + 1], c = x[k + 2], dd = x[k + 3];
        s0 = s0 + a * a;
        s1 = s1 + b * b;
        s2 = s2 + c * c;
        s3 = s3 + dd * dd;
    }
    double r = (s0 + s2) + (s1 + s3);
    for (; k < width; ++k) r = r + (double)x[k] * (double)x[k];
    return r;
}

/* rms_inverse's test (rms_mean_unsettled, fah_device.h): 1 and the mean
 * when the double mean m = tree / width lies more than 2 (width/4 + 40) + 2
 * ulps from a float rounding midpoint (its 29 bits below the float mantissa
 * against 2^28) and is at least 2^-126, else 0. */
int oracle_rms_mean_settled(double tree, int width, float* mean) {
    const double m = tree / (double)width;
    uint64_t bits;
    memcpy(&bits, &m, 8);
    const uint32_t low = (uint32_t)bits & 0x1fffffffu, high = (uint32_t)(bits >> 32);
    const uint32_t margin = 2u * (uint32_t)(width / 4 + 40) + 2u;
    *mean = (float)m;
    return !(low + margin - (1u << 28) <= 2u * margin || high < (897u << 20));
}

static uint64_t splitmix(uint64_t* s) {
    uint64_t z = (*s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

/* Row r of a sample. Mixed (pool_n a power of two): values of `pool` from a
 * random start with a random odd stride. Rowwise (pool holds whole rows,
 * pool_n a multiple of width): one of the pool's rows at random. Either way
 * each value gets a random sign and its three low mantissa bits replaced at
 * random (new rounding cases, same magnitudes and, rowwise, the same
 * per-channel structure). */
static void sample_row(const float* pool, int64_t pool_n, int width, int rowwise, uint64_t seed, int64_t r,
                       float* row) {
    uint64_t st = seed ^ ((uint64_t)r * 0x2545f4914f6cdd1dull);
    const uint64_t mask = (uint64_t)pool_n - 1;
    uint64_t base = splitmix(&st), stride = splitmix(&st) | 1u;
    if (rowwise) {
        base = (base % (uint64_t)(pool_n / width)) * (uint64_t)width;
        stride = 1;
    }
    uint64_t bits = 0;
    for (int k = 0; k < width; ++k) {
        if ((k & 7) == 0) bits = splitmix(&st);
        const uint64_t at = base + (uint64_t)k * stride;
        float v = pool[rowwise ? at : (at & mask)];
        uint32_t u;
        memcpy(&u, &v, 4);
        const uint32_t b = (uint32_t)(bits >> (8 * (k & 7)));
        if (u & 0x7f800000u) u = (u & ~7u) | (b & 7u);
        u ^= (b & 8u) << 28;
        memcpy(&v, &u, 4);
        row[k] = v;
    }
}

/* counts[0] rows, [1] rows whose GPU-tree float mean differs from the
 * reference's, [2] rows rms_mean does not settle from the tree (it then forms
 * the reference's sum), [3] rows it settles to a mean that differs from the
 * reference's (must stay 0). */
int oracle_norm_order_stats(const float* pool, int64_t pool_n, int width, int rowwise, int64_t rows, uint64_t seed,
                            int64_t* counts) {
    if (pool_n <= 0 || width < 4 || width > 4096 || width % 4) return fail("bad sample");
    if (rowwise ? pool_n % width != 0 : (pool_n & (pool_n - 1)) != 0) return fail("bad sample pool");
    int64_t differ = 0, unsettled = 0, wrong = 0;
#pragma omp parallel reduction(+ : differ, unsettled, wrong)
    {
        float* row = (float*)malloc(sizeof(float) * (size_t)width);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            sample_row(pool, pool_n, width, rowwise, seed, r, row);
            const double tree = oracle_sum_sq_gpu_tree(row, width);
            const float ref = (float)(oracle_sum_sq_reference(row, width) / (double)width);
            const float plain = (float)(tree / (double)width);
            float settled;
            differ += plain != ref;
            if (oracle_rms_mean_settled(tree, width, &settled)) wrong += settled != ref;
            else ++unsettled;
        }
        free(row);
    }
    counts[0] = rows;
    counts[1] = differ;
    counts[2] = unsettled;
    counts[3] = wrong;
    return 0;
}

/* Up to `want` sample rows (from row `start` on) whose GPU-tree float mean
 * differs from the reference's, into out [want][width]; returns how many. */
int64_t oracle_norm_order_find(const float* pool, int64_t pool_n, int width, int rowwise, uint64_t seed,
                               int64_t start, int64_t rows, int64_t want, float* out) {
    int64_t found = 0;
    float* row = (float*)malloc(sizeof(float) * (size_t)width);
    for (int64_t r = start; r < start + rows && found < want; ++r) {
        sample_row(pool, pool_n, width, rowwise, seed, r, row);
        const float plain = (float)(oracle_sum_sq_gpu_tree(row, width) / (double)width);
        const float ref = (float)(oracle_sum_sq_reference(row, width) / (double)width);
        if (plain != ref) memcpy(out + found++ * width, row, sizeof(float) * (size_t)width);
    }
    free(row);
    return found;
}
