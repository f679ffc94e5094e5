/*
 * C restatement of the decode hot path, for full-size oracle runs and CPU
 * timing. TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
 *
 * It follows the same reference sources as oracle/ops.py and oracle/model.py
 * (paths relative to ios_kernels/kernels/, KL = the Llama-3.2-1B folder,
 * KG = the Gemma-4-E2B folder):
 *   matvec        KL/kernels.metal:106-137   (fp16 W, fp32 x; here fp64 sums)
 *   gate_up       KG/kernels.metal:205-234, gelu_tanh KG/kernels.metal:26-28
 *   rmsnorm       KL/kernels.metal:71-96     ((1 + w) weights for the Gemma shape)
 *   rope_kv       KL/kernels.metal:182-224, inv_freq KL/main.swift:92-94
 *   attention     KL/kernels.metal:235-305, GQA map :261, scale KL/main.swift:293
 *   argmax        KL/kernels.metal:310-345   (first maximum wins)
 *   embed         KL/kernels.metal:31-39, sqrt(D) scale KG/main.swift:397
 *   step order    KL/main.swift:321-347, tied head KG/main.swift:379-380,
 *                 untied lm_head KL/main.swift:306, llama3 inv_freq KL/main.swift:96-107
 * Values are rounded to fp32 between ops and K/V to fp16, as on the GPU.
 * Weights come from the same counter-based generator as mxd_fill_normal.
 */
#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- rng */

static inline uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline int32_t sum16x4(uint64_t h) {
    return (int32_t)(h & 0xFFFF) + (int32_t)((h >> 16) & 0xFFFF) + (int32_t)((h >> 32) & 0xFFFF) + (int32_t)(h >> 48);
}

static float rng_scale(float stddev) { return (float)((double)stddev / sqrt(8.0 * (65536.0 * 65536.0 - 1.0) / 12.0)); }

static inline float rng_value(uint64_t key, uint64_t i, float k) {
    const int32_t c = sum16x4(mix64(key + 2 * i)) + sum16x4(mix64(key + 2 * i + 1)) - 4 * 65535;
    return (float)c * k;
}

static inline float h2f(uint16_t h) { return _cvtsh_ss(h); }
static inline uint16_t f2h(float f) { return (uint16_t)_cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT); }

void oracle_fill_normal_f16(uint16_t* dst, uint64_t n, uint64_t seed, uint64_t tensor_id, float stddev) {
    const uint64_t key = mix64(mix64(seed) ^ tensor_id);
    const float k = rng_scale(stddev);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)n; ++i) dst[i] = f2h(rng_value(key, (uint64_t)i, k));
}

void oracle_fill_normal_f32(float* dst, uint64_t n, uint64_t seed, uint64_t tensor_id, float stddev) {
    const uint64_t key = mix64(mix64(seed) ^ tensor_id);
    const float k = rng_scale(stddev);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)n; ++i) dst[i] = rng_value(key, (uint64_t)i, k);
}

/* ---------------------------------------------------------------- ops */

static inline double hsum4(__m256d v) {
    __m128d lo = _mm256_castpd256_pd128(v), hi = _mm256_extractf128_pd(v, 1);
    lo = _mm_add_pd(lo, hi);
    return _mm_cvtsd_f64(_mm_add_sd(lo, _mm_unpackhi_pd(lo, lo)));
}

/* sum_k float(w[k]) * x[k] in fp64 (each product is exact in fp64). */
static double dot_f16_f32(const uint16_t* w, const float* x, int K) {
    __m256d a0 = _mm256_setzero_pd(), a1 = _mm256_setzero_pd();
    int k = 0;
    for (; k + 8 <= K; k += 8) {
        const __m256 wf = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(w + k)));
        const __m256 xf = _mm256_loadu_ps(x + k);
        a0 = _mm256_fmadd_pd(_mm256_cvtps_pd(_mm256_castps256_ps128(wf)), _mm256_cvtps_pd(_mm256_castps256_ps128(xf)), a0);
        a1 = _mm256_fmadd_pd(_mm256_cvtps_pd(_mm256_extractf128_ps(wf, 1)), _mm256_cvtps_pd(_mm256_extractf128_ps(xf, 1)), a1);
    }
    double s = hsum4(_mm256_add_pd(a0, a1));
    for (; k < K; ++k) s += (double)h2f(w[k]) * (double)x[k];
    return s;
}

/* y[r] = sum_k W[r][k] x[k]; W fp16 [M][K]; y fp64. */
void oracle_matvec_f16(const uint16_t* W, const float* x, double* y, int M, int K) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < M; ++r) y[r] = dot_f16_f32(W + (size_t)r * K, x, K);
}

/* y[r] = sum_b s[r][b] * sum_{k in b} q[r][k] x[k]; q int8 [M][K]; s fp16 [M][K/32]. */
void oracle_matvec_q8b32(const int8_t* q, const uint16_t* s, const float* x, double* y, int M, int K) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < M; ++r) {
        const int8_t* qr = q + (size_t)r * K;
        double acc = 0.0;
        for (int b = 0; b < K / 32; ++b) {
            double part = 0.0;
            for (int j = 0; j < 32; ++j) part += (double)qr[32 * b + j] * (double)x[32 * b + j];
            acc += part * (double)h2f(s[(size_t)r * (K / 32) + b]);
        }
        y[r] = acc;
    }
}

/* W fp32 [M][K]. */
void oracle_matvec_f32(const float* W, const float* x, double* y, int M, int K) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < M; ++r) {
        const float* w = W + (size_t)r * K;
        double acc = 0.0;
        for (int k = 0; k < K; ++k) acc += (double)w[k] * (double)x[k];
        y[r] = acc;
    }
}

static double gelu_tanh(double x) { return 0.5 * x * (1.0 + tanh(0.7978845608028654 * (x + 0.044715 * x * x * x))); }
static double silu(double x) { return x / (1.0 + exp(-x)); }

static void rmsnorm(const float* x, const float* w, float* y, int D, float eps, int plus_one) {
    double ss = 0.0;
    for (int i = 0; i < D; ++i) ss += (double)x[i] * (double)x[i];
    const double inv = 1.0 / sqrt(ss / D + (double)eps);
    for (int i = 0; i < D; ++i) y[i] = (float)((double)x[i] * inv * (plus_one ? 1.0 + (double)w[i] : (double)w[i]));
}

/* ---------------------------------------------------------------- model */

typedef struct {
    int n_layers, dim, n_heads, n_kv, head_dim, ffn_dim, vocab;
    float eps, theta;
    int act;          /* 0 gelu_tanh, 1 silu */
    int plus_one;     /* (1 + w) RMSNorm weights */
    int embed_scale;  /* x = E[tok] * sqrt(D) */
    int untied_head;  /* logits from a separate lm_head tensor (id 3), not the embedding */
    /* Llama-3 RoPE frequency scaling when rope_factor > 0 */
    float rope_factor, rope_low_freq_factor, rope_high_freq_factor;
    int rope_original_max_positions;
} oracle_cfg;

typedef struct {
    uint16_t *wqkv, *wo, *wgate, *wup, *wdown;
    float *attn_norm, *ffn_norm;
} oracle_layer;

typedef struct {
    oracle_cfg c;
    int max_ctx;
    uint16_t *embed, *lm_head;
    float* final_norm;
    oracle_layer* L;
    uint16_t *k, *v; /* both [layer][kvh][ctx][hd] */
    float *x, *xn, *qkv, *att, *h, *logits, *invf;
    double *tmp, *scores;
} oracle_model;

static uint64_t tid_of(int layer, int kind) { return 1000 + 16 * (uint64_t)layer + (uint64_t)kind; }

static uint16_t* gen16(size_t n, uint64_t seed, uint64_t id, float std) {
    uint16_t* p = (uint16_t*)malloc(n * 2);
    if (p) oracle_fill_normal_f16(p, n, seed, id, std);
    return p;
}

static float* gen32(size_t n, uint64_t seed, uint64_t id, float std) {
    float* p = (float*)malloc(n * 4);
    if (p) oracle_fill_normal_f32(p, n, seed, id, std);
    return p;
}

/* inv_freq[i] = theta^(-2i/hd) in double, with the Llama-3 band scaling when
 * rope_factor > 0: wavelengths 2 pi / f below original / high_freq_factor keep
 * f, above original / low_freq_factor take f / factor, and in between blend the
 * two linearly in original / wavelength; stored as float. */
static void compute_inv_freq(const oracle_cfg* c, float* invf) {
    const int HD = c->head_dim;
    for (int i = 0; i < HD / 2; ++i) {
        double f = 1.0 / pow((double)c->theta, (double)(2 * i) / (double)HD);
        if (c->rope_factor > 0.0f) {
            const double orig = (double)c->rope_original_max_positions, factor = (double)c->rope_factor;
            const double lo = (double)c->rope_low_freq_factor, hi = (double)c->rope_high_freq_factor;
            const double wave = 2.0 * 3.14159265358979323846 / f;
            if (wave > orig / lo) {
                f = f / factor;
            } else if (wave >= orig / hi) {
                const double t = (orig / wave - lo) / (hi - lo);
                f = (1.0 - t) * f / factor + t * f;
            }
        }
        invf[i] = (float)f;
    }
}

void oracle_model_destroy(oracle_model* m);

/* Synthetic weights: every tensor N(0, std^2) from the hash generator, the
 * embedding N(0, embed_std^2). */
oracle_model* oracle_model_create(const oracle_cfg* cfg, int max_ctx, uint64_t seed, float std, float embed_std) {
    oracle_model* m = (oracle_model*)calloc(1, sizeof(oracle_model));
    if (!m) return NULL;
    m->c = *cfg;
    m->max_ctx = max_ctx;
    const oracle_cfg* c = &m->c;
    const size_t D = c->dim, F = c->ffn_dim, HD = c->head_dim;
    const size_t qkv = (size_t)(c->n_heads + 2 * c->n_kv) * HD, qd = (size_t)c->n_heads * HD;
    m->embed = gen16((size_t)c->vocab * D, seed, 1, embed_std);
    m->final_norm = gen32(D, seed, 2, std);
    if (c->untied_head) {
        m->lm_head = gen16((size_t)c->vocab * D, seed, 3, std);
        if (!m->lm_head) goto fail;
    }
    m->L = (oracle_layer*)calloc(c->n_layers, sizeof(oracle_layer));
    if (!m->embed || !m->final_norm || !m->L) goto fail;
    for (int l = 0; l < c->n_layers; ++l) {
        oracle_layer* L = &m->L[l];
        L->attn_norm = gen32(D, seed, tid_of(l, 0), std);
        L->wqkv = gen16(qkv * D, seed, tid_of(l, 1), std);
        L->wo = gen16(D * qd, seed, tid_of(l, 2), std);
        L->ffn_norm = gen32(D, seed, tid_of(l, 3), std);
        L->wgate = gen16(F * D, seed, tid_of(l, 4), std);
        L->wup = gen16(F * D, seed, tid_of(l, 5), std);
        L->wdown = gen16(D * F, seed, tid_of(l, 6), std);
        if (!L->attn_norm || !L->wqkv || !L->wo || !L->ffn_norm || !L->wgate || !L->wup || !L->wdown) goto fail;
    }
    const size_t kv = (size_t)c->n_layers * c->n_kv * max_ctx * HD;
    m->k = (uint16_t*)calloc(kv, 2);
    m->v = (uint16_t*)calloc(kv, 2);
    size_t big = (size_t)c->vocab > F ? (size_t)c->vocab : F;
    if (qkv > big) big = qkv;
    m->x = (float*)malloc(D * 4);
    m->xn = (float*)malloc(D * 4);
    m->qkv = (float*)malloc(qkv * 4);
    m->att = (float*)malloc(qd * 4);
    m->h = (float*)malloc(F * 4);
    m->logits = (float*)malloc((size_t)c->vocab * 4);
    m->invf = (float*)malloc(HD / 2 * 4);
    m->tmp = (double*)malloc(2 * big * 8);
    m->scores = (double*)malloc((size_t)c->n_heads * max_ctx * 8);
    if (HD > 512 || !m->scores || !m->k || !m->v || !m->x || !m->xn || !m->qkv || !m->att || !m->h || !m->logits || !m->invf || !m->tmp) goto fail;
    compute_inv_freq(c, m->invf);
    return m;
fail:
    oracle_model_destroy(m);
    return NULL;
}

void oracle_model_destroy(oracle_model* m) {
    if (!m) return;
    if (m->L)
        for (int l = 0; l < m->c.n_layers; ++l) {
            oracle_layer* L = &m->L[l];
            free(L->wqkv); free(L->wo); free(L->wgate); free(L->wup); free(L->wdown);
            free(L->attn_norm); free(L->ffn_norm);
        }
    free(m->L); free(m->embed); free(m->lm_head); free(m->final_norm); free(m->k); free(m->v);
    free(m->x); free(m->xn); free(m->qkv); free(m->att); free(m->h); free(m->logits); free(m->invf); free(m->tmp); free(m->scores);
    free(m);
}

static void rope_head(float* v, int hd, int pos, const float* invf, double* out) {
    const int half = hd / 2;
    for (int i = 0; i < half; ++i) {
        const double ang = (double)((float)pos * invf[i]);
        const double c = cos(ang), s = sin(ang), a = v[i], b = v[i + half];
        out[i] = a * c - b * s;
        out[i + half] = b * c + a * s;
    }
}

/* One decode step at `pos`: reads tokens[pos]; with `sample`, writes the argmax
 * to tokens[pos + 1] (prefill steps other than the last leave the prompt alone).
 * Writes the fp32 logits to logits_out and the top-1 minus top-2 margin to
 * margin_out when they are not NULL. */
int oracle_model_step(oracle_model* m, int32_t* tokens, int pos, int sample, float* logits_out, float* margin_out) {
    const oracle_cfg* c = &m->c;
    const int D = c->dim, HD = c->head_dim, NH = c->n_heads, NKV = c->n_kv, F = c->ffn_dim, C = m->max_ctx;
    const int G = NH / NKV, qkvd = (NH + 2 * NKV) * HD, qd = NH * HD;
    if (pos < 0 || pos >= C) return -1;
    const int tok = tokens[pos];
    if (tok < 0 || tok >= c->vocab) return -2;
    const float es = c->embed_scale ? sqrtf((float)D) : 1.0f;
    for (int i = 0; i < D; ++i) m->x[i] = h2f(m->embed[(size_t)tok * D + i]) * es;
    const float scale = 1.0f / sqrtf((float)HD);
    double* t = m->tmp;
    double* t2 = m->tmp + (c->vocab > F ? c->vocab : F);
    for (int l = 0; l < c->n_layers; ++l) {
        const oracle_layer* L = &m->L[l];
        uint16_t* K = m->k + (size_t)l * NKV * C * HD;
        uint16_t* V = m->v + (size_t)l * NKV * C * HD;
        rmsnorm(m->x, L->attn_norm, m->xn, D, c->eps, c->plus_one);
        oracle_matvec_f16(L->wqkv, m->xn, t, qkvd, D);
        for (int i = 0; i < qkvd; ++i) m->qkv[i] = (float)t[i];
        double rot[512];
        for (int h = 0; h < NH + NKV; ++h) {
            rope_head(m->qkv + h * HD, HD, pos, m->invf, rot);
            if (h < NH) {
                for (int i = 0; i < HD; ++i) m->qkv[h * HD + i] = (float)rot[i];
            } else {
                const int kvh = h - NH;
                const float* vv = m->qkv + (NH + NKV + kvh) * HD;
                for (int i = 0; i < HD; ++i) {
                    K[((size_t)kvh * C + pos) * HD + i] = f2h((float)rot[i]);
                    V[((size_t)kvh * C + pos) * HD + i] = f2h(vv[i]);
                }
            }
        }
        const int n = pos + 1;
#pragma omp parallel for schedule(static)
        for (int h = 0; h < NH; ++h) {
            const int kvh = h / G;
            const float* q = m->qkv + h * HD;
            double* s = m->scores + (size_t)h * C;
            double mx = -INFINITY;
            for (int j = 0; j < n; ++j) {
                double d = 0.0;
                for (int i = 0; i < HD; ++i) d += (double)q[i] * (double)h2f(K[((size_t)kvh * C + j) * HD + i]);
                s[j] = d * (double)scale;
                if (s[j] > mx) mx = s[j];
            }
            double sum = 0.0;
            for (int j = 0; j < n; ++j) { s[j] = exp(s[j] - mx); sum += s[j]; }
            double o[512];
            for (int i = 0; i < HD; ++i) o[i] = 0.0;
            for (int j = 0; j < n; ++j) {
                const uint16_t* vr = V + ((size_t)kvh * C + j) * HD;
                for (int i = 0; i < HD; ++i) o[i] += s[j] * (double)h2f(vr[i]);
            }
            for (int i = 0; i < HD; ++i) m->att[h * HD + i] = (float)(o[i] / sum);
        }
        oracle_matvec_f16(L->wo, m->att, t, D, qd);
        for (int i = 0; i < D; ++i) m->x[i] = m->x[i] + (float)t[i];
        rmsnorm(m->x, L->ffn_norm, m->xn, D, c->eps, c->plus_one);
        oracle_matvec_f16(L->wgate, m->xn, t, F, D);
        oracle_matvec_f16(L->wup, m->xn, t2, F, D);
        for (int i = 0; i < F; ++i) m->h[i] = (float)((c->act == 1 ? silu(t[i]) : gelu_tanh(t[i])) * t2[i]);
        oracle_matvec_f16(L->wdown, m->h, t, D, F);
        for (int i = 0; i < D; ++i) m->x[i] = m->x[i] + (float)t[i];
    }
    rmsnorm(m->x, m->final_norm, m->xn, D, c->eps, c->plus_one);
    oracle_matvec_f16(c->untied_head ? m->lm_head : m->embed, m->xn, t, c->vocab, D);
    int best = 0;
    float b1 = -INFINITY, b2 = -INFINITY;
    for (int i = 0; i < c->vocab; ++i) {
        const float v = (float)t[i];
        m->logits[i] = v;
        if (v > b1) { b2 = b1; b1 = v; best = i; }
        else if (v > b2) b2 = v;
    }
    if (sample) tokens[pos + 1] = best;
    if (logits_out) memcpy(logits_out, m->logits, (size_t)c->vocab * 4);
    if (margin_out) *margin_out = b1 - b2;
    return 0;
}

int oracle_num_threads(void) { return omp_get_max_threads(); }
void oracle_set_num_threads(int n) { omp_set_num_threads(n); }

/* The model's inverse RoPE frequencies (head_dim / 2 floats). */
void oracle_model_inv_freq(const oracle_model* m, float* out) { memcpy(out, m->invf, (size_t)m->c.head_dim / 2 * 4); }
