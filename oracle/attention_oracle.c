/*
 * CPU oracle for the SDXL UNet SpatialTransformer attention path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker the parity tests, the
 * smoke check and bench.py's cpu_baseline leg compare the HIP kernels
 * against. Nothing in the product library links, loads or calls it, and the
 * product path has no CPU fallback.
 *
 * Each function restates the reference algorithm it cites (paths relative to
 * the reference tree Apache0ne/sdxl-end2end). Pinning of every function is
 * listed in tests/test_oracle.py; nothing here is "parity unpinned".
 *
 * Layout everywhere: BSHD contiguous, x[((b*S + s)*H + h)*D + d], the
 * [B, S, H*D] tensor the reference passes between its linears and attention.
 */
#include <math.h>
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* IEEE binary16 / bfloat16 conversions, written from the formats.      */
/* ------------------------------------------------------------------ */

/* binary16 -> binary32, exact. Follows the decode in src/unet.cpp:65-89. */
float oracle_half_to_float(uint16_t bits) {
    uint32_t sign = (uint32_t)(bits & 0x8000u) << 16;
    uint32_t exponent = (bits >> 10) & 0x1Fu;
    uint32_t mantissa = bits & 0x3FFu;
    uint32_t out;
    if (exponent == 0) {
        if (mantissa == 0) {
            out = sign;
        } else {
            int e = -14;
            while ((mantissa & 0x400u) == 0) { mantissa <<= 1; --e; }
            mantissa &= 0x3FFu;
            out = sign | ((uint32_t)(e + 127) << 23) | (mantissa << 13);
        }
    } else if (exponent == 0x1Fu) {
        out = sign | 0x7F800000u | (mantissa << 13);
    } else {
        out = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    }
    float f;
    memcpy(&f, &out, sizeof f);
    return f;
}

/* binary32 -> binary16, round to nearest, ties to even (the rounding of
 * Tensor::from_host_f32, src/cuda/tensor.cu:237-250). Overflow -> inf,
 * NaN stays NaN (quiet). */
uint16_t oracle_float_to_half(float value) {
    uint32_t x;
    memcpy(&x, &value, sizeof x);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t absx = x & 0x7FFFFFFFu;
    if (absx >= 0x7F800000u) {                      /* inf or NaN */
        return (uint16_t)(sign | 0x7C00u | (absx > 0x7F800000u ? 0x200u : 0u));
    }
    if (absx >= 0x477FF000u) {                      /* >= 65520 rounds to inf */
        return (uint16_t)(sign | 0x7C00u);
    }
    if (absx < 0x38800000u) {                       /* below 2^-14: subnormal half */
        if (absx < 0x33000000u) return (uint16_t)sign; /* < 2^-25: rounds to zero */
        uint32_t e = absx >> 23;
        uint32_t m = (absx & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e;                  /* 14 + (127-1-e) ... value = m * 2^(e-150) */
        /* half subnormal unit is 2^-24: result = m * 2^(e-150+24) = m >> (126-e) */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1u);
        if (rem > halfway || (rem == halfway && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (absx >> 23) - 112u;               /* rebias 127 -> 15 */
    uint32_t m = absx & 0x7FFFFFu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q; /* carry may roll into exponent: correct */
    return (uint16_t)(sign | q);
}

float oracle_bf16_to_float(uint16_t bits) {
    uint32_t u = (uint32_t)bits << 16;
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

uint16_t oracle_float_to_bf16(float value) {
    uint32_t x;
    memcpy(&x, &value, sizeof x);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
    uint32_t lsb = (x >> 16) & 1u;
    x += 0x7FFFu + lsb;
    return (uint16_t)(x >> 16);
}

/* ------------------------------------------------------------------ */
/* Seeded N(0,1) generator: SplitMix64 -> Box-Muller.                   */
/* Our own documented generator (the reference's benches use sinusoids, */
/* src/attention_bench.cu:19-30; its sampler uses MT19937, which this   */
/* path does not need).                                                 */
/* ------------------------------------------------------------------ */

static uint64_t splitmix64_next(uint64_t* state) {
    uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Uniform in (0, 1]: 53 random bits, offset so log() never sees zero. */
static double uniform_open(uint64_t* state) {
    return ((double)(splitmix64_next(state) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

/* Fills out[0..n) with N(0,1)*stddev as float32. Pairs (2i, 2i+1) come from
 * one Box-Muller draw: r = sqrt(-2 ln u1), theta = 2 pi u2. */
void oracle_fill_normal_f32(uint64_t seed, float stddev, float* out, size_t n) {
    uint64_t state = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        double u1 = uniform_open(&state);
        double u2 = uniform_open(&state);
        double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(r * cos(two_pi * u2) * stddev);
        if (i + 1 < n) out[i + 1] = (float)(r * sin(two_pi * u2) * stddev);
    }
}

void oracle_fill_normal_f16(uint64_t seed, float stddev, uint16_t* out, size_t n) {
    float* tmp = (float*)malloc(n * sizeof(float) + 8);
    oracle_fill_normal_f32(seed, stddev, tmp, n);
    for (size_t i = 0; i < n; ++i) out[i] = oracle_float_to_half(tmp[i]);
    free(tmp);
}

/* ------------------------------------------------------------------ */
/* Attention                                                            */
/* ------------------------------------------------------------------ */

/* Exact FP32 softmax attention for one (b, h) pair over query rows
 * [q_begin, q_end). Restates full_attention, src/unet.cpp:440-481:
 *   s_k = (sum_d q_d k_d) * scale          (ascending d, FP32)
 *   m   = max_k s_k
 *   p_k = exp(s_k - m); den = sum_k p_k    (ascending k)
 *   p_k *= 1/den                           (reciprocal, then multiply)
 *   o_d = sum_k p_k v_{k,d}                (ascending k)
 * Extended, for the masked/causal semantics of the GPU kernels
 * (src/cuda/ops_kernels.cu:491-556, src/cuda/flash_attention_sm80.cu:141-160,
 * :214-219): keys with key_mask[b*Sk+k]==0, or k > q when causal, are
 * excluded; a row with no visible key is all zeros. */
static void attention_rows(const float* q, const float* k, const float* v, float* o,
                           size_t b, size_t h, size_t q_begin, size_t q_end,
                           size_t Sq, size_t Sk, size_t H, size_t D, float scale,
                           const int32_t* key_mask, int causal,
                           float* score, float* prob) {
    const size_t width = H * D;
    const size_t base = h * D;
    for (size_t qi = q_begin; qi < q_end; ++qi) {
        const float* qrow = q + (b * Sq + qi) * width + base;
        float maxv = -INFINITY;
        int any = 0;
        for (size_t ki = 0; ki < Sk; ++ki) {
            int visible = (key_mask == NULL || key_mask[b * Sk + ki] != 0) && (!causal || ki <= qi);
            if (!visible) { score[ki] = -INFINITY; continue; }
            any = 1;
            const float* krow = k + (b * Sk + ki) * width + base;
            float s = 0.0f;
            for (size_t d = 0; d < D; ++d) s += qrow[d] * krow[d];
            s *= scale;
            score[ki] = s;
            if (s > maxv) maxv = s;
        }
        float* orow = o + (b * Sq + qi) * width + base;
        if (!any) { for (size_t d = 0; d < D; ++d) orow[d] = 0.0f; continue; }
        float denom = 0.0f;
        for (size_t ki = 0; ki < Sk; ++ki) {
            prob[ki] = score[ki] == -INFINITY ? 0.0f : expf(score[ki] - maxv);
            denom += prob[ki];
        }
        denom = 1.0f / denom;
        for (size_t ki = 0; ki < Sk; ++ki) prob[ki] *= denom;
        for (size_t d = 0; d < D; ++d) {
            float acc = 0.0f;
            for (size_t ki = 0; ki < Sk; ++ki) acc += prob[ki] * v[(b * Sk + ki) * width + base + d];
            orow[d] = acc;
        }
    }
}

typedef struct {
    const float *q, *k, *v;
    float* o;
    size_t B, Sq, Sk, H, D;
    float scale;
    const int32_t* key_mask;
    int causal;
    size_t task_begin, task_end; /* tasks are (b, h) pairs */
} attention_job;

static void* attention_worker(void* arg) {
    attention_job* job = (attention_job*)arg;
    float* score = (float*)malloc((job->Sk + 1) * sizeof(float));
    float* prob = (float*)malloc((job->Sk + 1) * sizeof(float));
    for (size_t t = job->task_begin; t < job->task_end; ++t) {
        size_t b = t / job->H, h = t % job->H;
        attention_rows(job->q, job->k, job->v, job->o, b, h, 0, job->Sq, job->Sq, job->Sk, job->H,
                       job->D, job->scale, job->key_mask, job->causal, score, prob);
    }
    free(score);
    free(prob);
    return NULL;
}

/* FP32 attention, src/unet.cpp:440-481. scale <= 0 selects 1/sqrt(D)
 * (src/unet.cpp:453). threads <= 1 runs the reference's single-threaded
 * loop order; threads > 1 splits (b, h) pairs over that many threads (each
 * row is computed exactly as in the single-threaded case). */
void oracle_attention_f32(const float* q, const float* k, const float* v, float* o,
                          size_t B, size_t Sq, size_t Sk, size_t H, size_t D, float scale,
                          const int32_t* key_mask, int causal, int threads) {
    if (scale <= 0.0f) scale = 1.0f / sqrtf((float)D);
    size_t tasks = B * H;
    if (threads < 1) threads = 1;
    if ((size_t)threads > tasks) threads = (int)tasks;
    if (threads <= 1) {
        attention_job job = {q, k, v, o, B, Sq, Sk, H, D, scale, key_mask, causal, 0, tasks};
        attention_worker(&job);
        return;
    }
    pthread_t* ids = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
    attention_job* jobs = (attention_job*)malloc(sizeof(attention_job) * (size_t)threads);
    for (int t = 0; t < threads; ++t) {
        attention_job j = {q, k, v, o, B, Sq, Sk, H, D, scale, key_mask, causal,
                           tasks * (size_t)t / (size_t)threads, tasks * (size_t)(t + 1) / (size_t)threads};
        jobs[t] = j;
        pthread_create(&ids[t], NULL, attention_worker, &jobs[t]);
    }
    for (int t = 0; t < threads; ++t) pthread_join(ids[t], NULL);
    free(ids);
    free(jobs);
}

/* Same as oracle_attention_f32, over fp16 storage (fp16 -> fp32 exactly,
 * as the reference's Tensor::to_host_f32 / TensorReader do). Output FP32. */
void oracle_attention_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v, float* o,
                          size_t B, size_t Sq, size_t Sk, size_t H, size_t D, float scale,
                          const int32_t* key_mask, int causal, int threads) {
    size_t nq = B * Sq * H * D, nk = B * Sk * H * D;
    float* qf = (float*)malloc(nq * sizeof(float) + 4);
    float* kf = (float*)malloc(nk * sizeof(float) + 4);
    float* vf = (float*)malloc(nk * sizeof(float) + 4);
    for (size_t i = 0; i < nq; ++i) qf[i] = oracle_half_to_float(q[i]);
    for (size_t i = 0; i < nk; ++i) { kf[i] = oracle_half_to_float(k[i]); vf[i] = oracle_half_to_float(v[i]); }
    oracle_attention_f32(qf, kf, vf, o, B, Sq, Sk, H, D, scale, key_mask, causal, threads);
    free(qf); free(kf); free(vf);
}

/* Row subset: only query rows [q_begin, q_end) of every (b, h); used for
 * bounded CPU timing samples and spot checks at full size. Rows outside the
 * range are left untouched in o. */
void oracle_attention_f16_rows(const uint16_t* q, const uint16_t* k, const uint16_t* v, float* o,
                               size_t B, size_t Sq, size_t Sk, size_t H, size_t D, float scale,
                               size_t q_begin, size_t q_end) {
    if (scale <= 0.0f) scale = 1.0f / sqrtf((float)D);
    size_t width = H * D;
    float* qf = (float*)malloc(D * sizeof(float));
    float* kf = (float*)malloc(B * Sk * width * sizeof(float) + 4);
    float* vf = (float*)malloc(B * Sk * width * sizeof(float) + 4);
    float* qall = (float*)calloc(B * Sq * width, sizeof(float));
    for (size_t i = 0; i < B * Sk * width; ++i) { kf[i] = oracle_half_to_float(k[i]); vf[i] = oracle_half_to_float(v[i]); }
    for (size_t b = 0; b < B; ++b)
        for (size_t s = q_begin; s < q_end; ++s)
            for (size_t c = 0; c < width; ++c) qall[(b * Sq + s) * width + c] = oracle_half_to_float(q[(b * Sq + s) * width + c]);
    float* score = (float*)malloc((Sk + 1) * sizeof(float));
    float* prob = (float*)malloc((Sk + 1) * sizeof(float));
    for (size_t b = 0; b < B; ++b)
        for (size_t h = 0; h < H; ++h)
            attention_rows(qall, kf, vf, o, b, h, q_begin, q_end, Sq, Sk, H, D, scale, NULL, 0, score, prob);
    free(qf); free(kf); free(vf); free(qall); free(score); free(prob);
}

/* Double-precision brute force of the same function, used only to pin the
 * FP32 restatement (independent arithmetic: exp in double, no reciprocal
 * trick). */
void oracle_attention_f64(const double* q, const double* k, const double* v, double* o,
                          size_t B, size_t Sq, size_t Sk, size_t H, size_t D, double scale,
                          const int32_t* key_mask, int causal) {
    size_t width = H * D;
    double* p = (double*)malloc((Sk + 1) * sizeof(double));
    for (size_t b = 0; b < B; ++b)
        for (size_t h = 0; h < H; ++h)
            for (size_t qi = 0; qi < Sq; ++qi) {
                double m = -INFINITY;
                for (size_t ki = 0; ki < Sk; ++ki) {
                    int vis = (key_mask == NULL || key_mask[b * Sk + ki] != 0) && (!causal || ki <= qi);
                    double s = -INFINITY;
                    if (vis) {
                        s = 0.0;
                        for (size_t d = 0; d < D; ++d) s += q[(b * Sq + qi) * width + h * D + d] * k[(b * Sk + ki) * width + h * D + d];
                        s *= scale;
                    }
                    p[ki] = s;
                    if (s > m) m = s;
                }
                double den = 0.0;
                for (size_t ki = 0; ki < Sk; ++ki) { p[ki] = (m == -INFINITY || p[ki] == -INFINITY) ? 0.0 : exp(p[ki] - m); den += p[ki]; }
                for (size_t d = 0; d < D; ++d) {
                    double acc = 0.0;
                    for (size_t ki = 0; ki < Sk; ++ki) acc += p[ki] * v[(b * Sk + ki) * width + h * D + d];
                    o[(b * Sq + qi) * width + h * D + d] = den > 0.0 ? acc / den : 0.0;
                }
            }
    free(p);
}

/* ------------------------------------------------------------------ */
/* Transformer-block pieces used around the attention.     */
/* ------------------------------------------------------------------ */

/* LayerNorm over the last dim, src/unet.cpp:237-263: mean (ascending sum,
 * divide), centred variance (ascending, divide), inv = 1/sqrt(var+eps),
 * y = (x-mean)*inv*w + b. */
void oracle_layer_norm(const float* x, const float* w, const float* bias, float* y,
                       size_t rows, size_t width, float eps) {
    for (size_t r = 0; r < rows; ++r) {
        const float* src = x + r * width;
        float mean = 0.0f;
        for (size_t i = 0; i < width; ++i) mean += src[i];
        mean /= (float)width;
        float var = 0.0f;
        for (size_t i = 0; i < width; ++i) { float d = src[i] - mean; var += d * d; }
        var /= (float)width;
        float inv = 1.0f / sqrtf(var + eps);
        float* dst = y + r * width;
        for (size_t i = 0; i < width; ++i) dst[i] = (src[i] - mean) * inv * w[i] + bias[i];
    }
}

/* y[r, o] = bias[o] + sum_i x[r, i] * W[o, i]; W stored [out, in] as the
 * reference stores linear weights, src/unet.cpp:202-222. */
void oracle_linear(const float* x, const float* W, const float* bias, float* y,
                   size_t rows, size_t in_features, size_t out_features) {
    for (size_t r = 0; r < rows; ++r)
        for (size_t o = 0; o < out_features; ++o) {
            float acc = bias ? bias[o] : 0.0f;
            const float* src = x + r * in_features;
            const float* wrow = W + o * in_features;
            for (size_t i = 0; i < in_features; ++i) acc += src[i] * wrow[i];
            y[r * out_features + o] = acc;
        }
}

/* FP8 E4M3 (finite-only "fn" variant) decode, src/unet.cpp:91-119 with
 * exponent_bits=4, mantissa_bits=3, bias=7, finite_only: 0x7F/0xFF are NaN,
 * subnormals m/8 * 2^-6. */
float oracle_e4m3_to_float(uint8_t bits) {
    int negative = (bits & 0x80u) != 0;
    unsigned e = (bits >> 3) & 0xFu;
    unsigned m = bits & 0x7u;
    float value;
    if (e == 0) {
        value = ldexpf((float)m / 8.0f, -6);
    } else if (e == 0xFu && m == 0x7u) {
        value = NAN;
    } else {
        value = ldexpf(1.0f + (float)m / 8.0f, (int)e - 7);
    }
    return negative ? -value : value;
}

/* Round-to-nearest-even float -> E4M3fn with saturation to +-448 (finite
 * format: no infinities). Chosen by searching the 126 finite positive codes,
 * so it depends only on the decode above. */
uint8_t oracle_float_to_e4m3(float value) {
    if (value != value) return 0x7Fu;
    uint8_t sign = value < 0.0f ? 0x80u : 0u;
    float a = fabsf(value);
    if (a >= 448.0f) return (uint8_t)(sign | 0x7Eu);
    uint8_t best = 0;
    float best_err = a;
    for (unsigned c = 1; c < 0x7Fu; ++c) {
        float cv = oracle_e4m3_to_float((uint8_t)c);
        float err = fabsf(cv - a);
        if (err < best_err || (err == best_err && (c & 1u) == 0u && (best & 1u) != 0u)) {
            best = (uint8_t)c;
            best_err = err;
        }
    }
    return (uint8_t)(sign | best);
}

/* Per-output-channel weight scale, src/cuda/weights.cu:119-142:
 * amax over the row (finite values), scale = amax>0 ? max(amax/448, 1e-12) : 1. */
void oracle_fp8_row_scales(const float* W, size_t out_features, size_t in_features, float* scales) {
    for (size_t o = 0; o < out_features; ++o) {
        float amax = 0.0f;
        for (size_t i = 0; i < in_features; ++i) {
            float a = fabsf(W[o * in_features + i]);
            if (isfinite(a) && a > amax) amax = a;
        }
        scales[o] = amax > 0.0f ? fmaxf(amax / 448.0f, 1.0e-12f) : 1.0f;
    }
}

/* Per-row E4M3 quantisation of W [rows, cols] (src/cuda/weights.cu:119-170):
 * scales from oracle_fp8_row_scales, codes = oracle_float_to_e4m3(W / scale). */
void oracle_quantize_e4m3_rows(const float* W, size_t rows, size_t cols, uint8_t* q, float* scales) {
    oracle_fp8_row_scales(W, rows, cols, scales);
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < cols; ++c) q[r * cols + c] = oracle_float_to_e4m3(W[r * cols + c] / scales[r]);
}

/* ------------------------------------------------------------------ */
/* The transformer block's two attention halves, in the reference's   */
/* block order (src/unet.cpp:495-512), FP32 throughout.                */
/* ------------------------------------------------------------------ */

/* Row-parallel helper: fn(ctx, r0, r1) over [0, n) split in `threads`
 * contiguous ranges. Every row is computed as in the single-threaded loop. */
typedef void (*oracle_rows_fn)(void* ctx, size_t r0, size_t r1);
typedef struct { oracle_rows_fn fn; void* ctx; size_t r0, r1; } rows_job;

static void* rows_worker(void* arg) {
    rows_job* j = (rows_job*)arg;
    j->fn(j->ctx, j->r0, j->r1);
    return NULL;
}

static void parallel_rows(oracle_rows_fn fn, void* ctx, size_t n, int threads) {
    if (threads < 1) threads = 1;
    if ((size_t)threads > n) threads = n > 0 ? (int)n : 1;
    if (threads == 1) { fn(ctx, 0, n); return; }
    pthread_t* ids = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
    rows_job* jobs = (rows_job*)malloc(sizeof(rows_job) * (size_t)threads);
    for (int t = 0; t < threads; ++t) {
        rows_job j = {fn, ctx, n * (size_t)t / (size_t)threads, n * (size_t)(t + 1) / (size_t)threads};
        jobs[t] = j;
        pthread_create(&ids[t], NULL, rows_worker, &jobs[t]);
    }
    for (int t = 0; t < threads; ++t) pthread_join(ids[t], NULL);
    free(ids);
    free(jobs);
}

typedef struct { const float *x, *W, *bias; float* y; size_t in, out; } linear_ctx;

static void linear_rows(void* c, size_t r0, size_t r1) {
    linear_ctx* l = (linear_ctx*)c;
    oracle_linear(l->x + r0 * l->in, l->W, l->bias, l->y + r0 * l->out, r1 - r0, l->in, l->out);
}

/* y[rows] = x[rows] W^T + bias, rows split over threads (same sums as oracle_linear). */
static void linear_mt(const float* x, const float* W, const float* bias, float* y, size_t rows, size_t in,
                      size_t out, int threads) {
    linear_ctx c = {x, W, bias, y, in, out};
    parallel_rows(linear_rows, &c, rows, threads);
}

typedef struct {
    const float *q, *k, *v;
    float* o;
    size_t Sq, Sk, H, D, q_begin, q_end;
    float scale;
} attn_rows_ctx;

static void attention_task_rows(void* c, size_t t0, size_t t1) {
    attn_rows_ctx* a = (attn_rows_ctx*)c;
    float* score = (float*)malloc((a->Sk + 1) * sizeof(float));
    float* prob = (float*)malloc((a->Sk + 1) * sizeof(float));
    for (size_t t = t0; t < t1; ++t)
        attention_rows(a->q, a->k, a->v, a->o, t / a->H, t % a->H, a->q_begin, a->q_end, a->Sq, a->Sk, a->H,
                       a->D, a->scale, NULL, 0, score, prob);
    free(score);
    free(prob);
}

/* Shared tail of both halves, for query rows [q_begin, q_end) of every batch:
 * attention of q against k/v (full_attention, src/unet.cpp:440-481), then
 * linear_3d with the output weight and bias, then add_in_place onto the
 * hidden state (src/unet.cpp:505-506, :511-512): y = x + out. */
static void attention_half_tail(const float* x, const float* q, const float* k, const float* v,
                                const float* wo, const float* bo, size_t B, size_t S, size_t Sk, size_t W,
                                size_t heads, size_t q_begin, size_t q_end, float* y, int threads) {
    const size_t D = W / heads, rows = q_end - q_begin;
    float* attn = (float*)calloc(B * S * W + 1, sizeof(float));
    attn_rows_ctx ac = {q, k, v, attn, S, Sk, heads, D, q_begin, q_end, 1.0f / sqrtf((float)D)};
    parallel_rows(attention_task_rows, &ac, B * heads, threads);
    float* proj = (float*)malloc(rows * W * sizeof(float) + 4);
    for (size_t b = 0; b < B; ++b) {
        const size_t r = b * S + q_begin;
        linear_mt(attn + r * W, wo, bo, proj, rows, W, W, threads);
        for (size_t i = 0; i < rows * W; ++i) y[r * W + i] = x[r * W + i] + proj[i];
    }
    free(proj);
    free(attn);
}

/* Self-attention half of UNet::transformer_block (src/unet.cpp:500-506):
 * norm1 = layer_norm(x); q, k, v = three separate bias-free linear_3d of
 * norm1 (weights [W, W], [out, in]); attn = full_attention(q, k, v, heads);
 * attn = linear_3d(attn, wo, bo); x += attn. Computes the block's output for
 * query rows [q_begin, q_end) of every batch into y ([B, S, W]; other rows
 * untouched). Keys and values are computed for every row. */
void oracle_attn_sublayer(const float* x, const float* gamma, const float* beta, const float* wq,
                          const float* wk, const float* wv, const float* wo, const float* bo, size_t B,
                          size_t S, size_t W, size_t heads, size_t q_begin, size_t q_end, float* y,
                          int threads) {
    const size_t n = B * S * W, rows = q_end - q_begin;
    float* norm = (float*)malloc(n * sizeof(float) + 4);
    float* q = (float*)calloc(n + 1, sizeof(float));
    float* k = (float*)malloc(n * sizeof(float) + 4);
    float* v = (float*)malloc(n * sizeof(float) + 4);
    oracle_layer_norm(x, gamma, beta, norm, B * S, W, 1.0e-5f);
    for (size_t b = 0; b < B; ++b)
        linear_mt(norm + (b * S + q_begin) * W, wq, NULL, q + (b * S + q_begin) * W, rows, W, W, threads);
    linear_mt(norm, wk, NULL, k, B * S, W, W, threads);
    linear_mt(norm, wv, NULL, v, B * S, W, W, threads);
    attention_half_tail(x, q, k, v, wo, bo, B, S, S, W, heads, q_begin, q_end, y, threads);
    free(norm); free(q); free(k); free(v);
}

/* Cross-attention half (src/unet.cpp:508-512): norm2 = layer_norm(x); q from
 * norm2; k, v = bias-free linear_3d of the context ctx [B, L, C] with
 * weights [W, C]; then as the self half. */
void oracle_cross_attn_sublayer(const float* x, const float* gamma, const float* beta, const float* wq,
                                const float* ctx, const float* wk, const float* wv, const float* wo,
                                const float* bo, size_t B, size_t S, size_t W, size_t L, size_t C,
                                size_t heads, size_t q_begin, size_t q_end, float* y, int threads) {
    const size_t n = B * S * W, rows = q_end - q_begin;
    float* norm = (float*)malloc(n * sizeof(float) + 4);
    float* q = (float*)calloc(n + 1, sizeof(float));
    float* k = (float*)malloc(B * L * W * sizeof(float) + 4);
    float* v = (float*)malloc(B * L * W * sizeof(float) + 4);
    oracle_layer_norm(x, gamma, beta, norm, B * S, W, 1.0e-5f);
    for (size_t b = 0; b < B; ++b)
        linear_mt(norm + (b * S + q_begin) * W, wq, NULL, q + (b * S + q_begin) * W, rows, W, W, threads);
    linear_mt(ctx, wk, NULL, k, B * L, C, W, threads);
    linear_mt(ctx, wv, NULL, v, B * L, C, W, threads);
    attention_half_tail(x, q, k, v, wo, bo, B, S, L, W, heads, q_begin, q_end, y, threads);
    free(norm); free(q); free(k); free(v);
}
