/*
 * oracle.c -- CPU restatement of the YuE2 AR decode step.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h for the order spec, the parity pins
 * and who may use this file).  Built with gcc -O2 -ffp-contract=off so that
 * every multiply and add rounds exactly where written; fused multiply-adds
 * appear only as explicit fma()/fmaf() calls.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#if defined(__AVX2__) && defined(__FMA__)
#include <immintrin.h>
#define Y2O_SIMD 1
#endif

/* Protocol constants (src/protocol.rs:6-16). */
#define EOD 151643
#define ABC_END 151848
#define MUSIC_END 151852
#define CODEC_OFFSET 151853
#define CODEC_SIZE 32768
#define CONTEXT 24576

static int g_threads = 1;

void y2o_set_threads(int n) { g_threads = n > 0 ? n : 1; }
int y2o_get_threads(void) { return g_threads; }

/* ------------------------------------------------------------------------ */
/* Scalar helpers                                                           */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint64_t d2u(double f) { uint64_t u; memcpy(&u, &f, 8); return u; }
static inline double u2d(uint64_t u) { double f; memcpy(&f, &u, 8); return f; }

/* round_bf16: round to nearest even at bit 16, NaN -> quiet NaN
 * (src/tensor.rs:645-652). */
float y2o_round_bf16(float v) {
    uint32_t b = f2u(v);
    if ((b & 0x7fffffffu) > 0x7f800000u) return u2f((b & 0xffff0000u) | 0x00400000u);
    return u2f((b + 0x7fffu + ((b >> 16) & 1u)) & 0xffff0000u);
}
#define rb y2o_round_bf16

/* y2o_round_bf16 over bit patterns (no float passes through a call, so
 * signalling NaNs keep their payload): out[i] = bits of rb(bits in[i]). */
void y2o_round_bf16_bits(const uint32_t *in, uint32_t *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = f2u(rb(u2f(in[i])));
}

float y2o_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/*
 * exp for f32 arguments, replacing Accelerate vvexpf (src/tensor.rs:671-677,
 * 701-703) and Rust f32::exp (src/sampling.rs:177-195).
 * Method: Cody & Waite argument reduction x = n*ln2 + r, |r| <= ln2/2, with
 * ln2 split into a 43-bit head and a tail; e^r from its Taylor series to
 * degree 13 (truncation < 2^-56) in double precision; scale by 2^n exactly;
 * one final rounding to f32.  The double result is within ~2^-52 relative,
 * so the f32 result is the correctly rounded exp except when e^x lies within
 * ~2^-52 of an f32 rounding midpoint.
 */
static const double EXP_LOG2E = 0x1.71547652b82fep+0;
static const double EXP_LN2_HI = 0x1.62e42fefa3800p-1;
static const double EXP_LN2_LO = 0x1.ef35793c76730p-45;
static const double INV_FACT[14] = {
    0x1.0000000000000p+0,  0x1.0000000000000p+0,  0x1.0000000000000p-1,
    0x1.5555555555555p-3,  0x1.5555555555555p-5,  0x1.1111111111111p-7,
    0x1.6c16c16c16c17p-10, 0x1.a01a01a01a01ap-13, 0x1.a01a01a01a01ap-16,
    0x1.71de3a556c734p-19, 0x1.27e4fb7789f5cp-22, 0x1.ae64567f544e4p-26,
    0x1.1eed8eff8d898p-29, 0x1.6124613a86d09p-33};

float y2o_expf(float xf) {
    if (xf != xf) return xf + xf;
    if (xf > 89.0f) return INFINITY;
    if (xf < -104.0f) return 0.0f;
    double x = (double)xf;
    double n = rint(x * EXP_LOG2E);
    double r = fma(-n, EXP_LN2_HI, x);
    r = fma(-n, EXP_LN2_LO, r);
    double p = INV_FACT[13];
    for (int k = 12; k >= 0; --k) p = fma(p, r, INV_FACT[k]);
    int64_t ni = (int64_t)n;
    double scale = u2d((uint64_t)(ni + 1023) << 52);
    return (float)(p * scale);
}

/*
 * log1p in double precision, replacing Rust f64::ln_1p (src/sampling.rs:205).
 * Method: u = 1 + x with the correction c = (x - (u - 1)) / u; u = m * 2^k
 * with m in [sqrt(1/2), sqrt(2)); log m = 2 atanh(s), s = (m - 1)/(m + 1),
 * from the atanh series 2 s^(2j+1)/(2j+1) to j = 11 (truncation < 2^-60);
 * log u = k ln2 + log m.
 */
static const double ATANH_C[12] = {
    0x1.0000000000000p+1, 0x1.5555555555555p-1, 0x1.999999999999ap-2, 0x1.2492492492492p-2,
    0x1.c71c71c71c71cp-3, 0x1.745d1745d1746p-3, 0x1.3b13b13b13b14p-3, 0x1.1111111111111p-3,
    0x1.e1e1e1e1e1e1ep-4, 0x1.af286bca1af28p-4, 0x1.8618618618618p-4, 0x1.642c8590b2164p-4};
static const double SQRT_HALF = 0x1.6a09e667f3bcdp-1;

double y2o_log1p(double x) {
    if (x == 0.0) return x;
    if (x != x) return x + x;
    if (x <= -1.0) return x == -1.0 ? -INFINITY : NAN;
    if (x == INFINITY) return x;
    double u = 1.0 + x;
    double c = (x - (u - 1.0)) / u;
    uint64_t bits = d2u(u);
    int k = (int)((bits >> 52) & 0x7ff) - 1022;
    double f = u2d((bits & 0x000fffffffffffffull) | 0x3fe0000000000000ull); /* [0.5, 1) */
    double m;
    if (f < SQRT_HALF) {
        m = f + f;
        k -= 1;
    } else {
        m = f;
    }
    double f1 = m - 1.0;
    double s = f1 / (2.0 + f1);
    double z = s * s;
    double p = ATANH_C[11];
    for (int j = 10; j >= 1; --j) p = fma(p, z, ATANH_C[j]);
    double lm = fma(s * z, p, s + s);
    double kd = (double)k;
    return fma(kd, EXP_LN2_HI, lm + fma(kd, EXP_LN2_LO, c));
}

/* ------------------------------------------------------------------------ */
/* DOT: the documented substitute for cblas_sgemv / cblas_sgemm             */
/* ------------------------------------------------------------------------ */

static inline float butterfly64(float *acc) {
    /* xor butterfly with offsets 32..1; lane 0's value after each step is
     * acc[0] + acc[s], so halving the live range reproduces it exactly. */
    for (int s = 32; s >= 1; s >>= 1)
        for (int l = 0; l < s; ++l) acc[l] = acc[l] + acc[l + s];
    return acc[0];
}

float y2o_dot_bf16(const uint16_t *a, const float *b, int k) {
    float acc[64];
    for (int l = 0; l < 64; ++l) acc[l] = 0.0f;
    for (int base = 0; base < k; base += 512) {
        int lanes = (k - base) / 8;
        if (lanes > 64) lanes = 64;
        for (int l = 0; l < lanes; ++l) {
            const uint16_t *ap = a + base + 8 * l;
            const float *bp = b + base + 8 * l;
            float s = acc[l];
            for (int e = 0; e < 8; ++e) s = fmaf(y2o_bf16_to_f32(ap[e]), bp[e], s);
            acc[l] = s;
        }
    }
    return butterfly64(acc);
}

float y2o_dot_f32(const float *a, const float *b, int k) {
    float acc[64];
    for (int l = 0; l < 64; ++l) acc[l] = 0.0f;
    for (int base = 0; base < k; base += 512) {
        int lanes = (k - base) / 8;
        if (lanes > 64) lanes = 64;
        for (int l = 0; l < lanes; ++l) {
            const float *ap = a + base + 8 * l;
            const float *bp = b + base + 8 * l;
            float s = acc[l];
            for (int e = 0; e < 8; ++e) s = fmaf(ap[e], bp[e], s);
            acc[l] = s;
        }
    }
    return butterfly64(acc);
}

#ifdef Y2O_SIMD
/* The same DOT eight lanes at a time (speed only: every lane's chain is the
 * same fmaf sequence, so the result is y2o_dot_bf16's bit for bit).  xt is
 * x in lane-major order, xt[blk * 512 + e * 64 + l] = x[blk * 512 + 8 l + e]
 * (lane_major).  Lanes of a partial group of eight (k not a multiple of 64
 * in the last 512-block) run the scalar chain. */
static float dot_bf16_lanes(const uint16_t *a, const float *x, const float *xt, int k) {
    __m256 va[8];
    for (int v = 0; v < 8; ++v) va[v] = _mm256_setzero_ps();
    for (int base = 0; base < k; base += 512) {
        int lanes = (k - base) / 8;
        if (lanes > 64) lanes = 64;
        const int groups = lanes / 8;
        const float *xb = xt + base;
        for (int v = 0; v < groups; ++v) {
            /* lanes 8v .. 8v + 7: 64 consecutive weights, transposed so that
             * c[e] holds element e of each of the eight lanes */
            const __m128i *ap = (const __m128i *)(a + base + 64 * v);
            const __m128i r0 = _mm_loadu_si128(ap + 0), r1 = _mm_loadu_si128(ap + 1);
            const __m128i r2 = _mm_loadu_si128(ap + 2), r3 = _mm_loadu_si128(ap + 3);
            const __m128i r4 = _mm_loadu_si128(ap + 4), r5 = _mm_loadu_si128(ap + 5);
            const __m128i r6 = _mm_loadu_si128(ap + 6), r7 = _mm_loadu_si128(ap + 7);
            const __m128i t0 = _mm_unpacklo_epi16(r0, r1), t1 = _mm_unpackhi_epi16(r0, r1);
            const __m128i t2 = _mm_unpacklo_epi16(r2, r3), t3 = _mm_unpackhi_epi16(r2, r3);
            const __m128i t4 = _mm_unpacklo_epi16(r4, r5), t5 = _mm_unpackhi_epi16(r4, r5);
            const __m128i t6 = _mm_unpacklo_epi16(r6, r7), t7 = _mm_unpackhi_epi16(r6, r7);
            const __m128i u0 = _mm_unpacklo_epi32(t0, t2), u1 = _mm_unpackhi_epi32(t0, t2);
            const __m128i u2 = _mm_unpacklo_epi32(t1, t3), u3 = _mm_unpackhi_epi32(t1, t3);
            const __m128i u4 = _mm_unpacklo_epi32(t4, t6), u5 = _mm_unpackhi_epi32(t4, t6);
            const __m128i u6 = _mm_unpacklo_epi32(t5, t7), u7 = _mm_unpackhi_epi32(t5, t7);
            __m128i c[8];
            c[0] = _mm_unpacklo_epi64(u0, u4); c[1] = _mm_unpackhi_epi64(u0, u4);
            c[2] = _mm_unpacklo_epi64(u1, u5); c[3] = _mm_unpackhi_epi64(u1, u5);
            c[4] = _mm_unpacklo_epi64(u2, u6); c[5] = _mm_unpackhi_epi64(u2, u6);
            c[6] = _mm_unpacklo_epi64(u3, u7); c[7] = _mm_unpackhi_epi64(u3, u7);
            __m256 acc = va[v];
            for (int e = 0; e < 8; ++e) {
                const __m256 av = _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(c[e]), 16));
                acc = _mm256_fmadd_ps(av, _mm256_loadu_ps(xb + e * 64 + 8 * v), acc);
            }
            va[v] = acc;
        }
        if (lanes % 8) {
            float part[8];
            _mm256_storeu_ps(part, va[groups]);
            for (int j = 0; j < lanes % 8; ++j) {
                const int l = 8 * groups + j;
                const uint16_t *ap = a + base + 8 * l;
                const float *bp = x + base + 8 * l;
                float sacc = part[j];
                for (int e = 0; e < 8; ++e) sacc = fmaf(y2o_bf16_to_f32(ap[e]), bp[e], sacc);
                part[j] = sacc;
            }
            va[groups] = _mm256_loadu_ps(part);
        }
    }
    float acc[64];
    for (int v = 0; v < 8; ++v) _mm256_storeu_ps(acc + 8 * v, va[v]);
    return butterfly64(acc);
}

/* rows x vectors of length k in lane-major order (dot_bf16_lanes), each
 * padded to whole 512-blocks; NULL when out of memory. */
static float *lane_major(const float *x, int rows, int k) {
    const size_t xs = (size_t)((k + 511) / 512) * 512;
    float *xt = (float *)calloc(xs * (size_t)(rows > 0 ? rows : 1), sizeof(float));
    if (!xt) return NULL;
    for (int r = 0; r < rows; ++r)
        for (int base = 0; base < k; base += 512) {
            int lanes = (k - base) / 8;
            if (lanes > 64) lanes = 64;
            for (int l = 0; l < lanes; ++l)
                for (int e = 0; e < 8; ++e)
                    xt[(size_t)r * xs + base + e * 64 + l] = x[(size_t)r * k + base + 8 * l + e];
        }
    return xt;
}
#endif

/* DOT(W[i], x[r]) for i < out, r < rows into y[r * out + i] (rb: rounded to
 * BF16), optionally plus rb(bias[i]) before the rounding. */
static void dot_rows(const uint16_t *w, int out, int in, const float *x, int rows, const float *bias, int round,
                     float *y) {
#ifdef Y2O_SIMD
    float *xt = lane_major(x, rows, in);
    if (xt) {
        const size_t xs = (size_t)((in + 511) / 512) * 512;
#pragma omp parallel for schedule(static) num_threads(g_threads)
        for (int i = 0; i < out; ++i) {
            const uint16_t *wi = w + (size_t)i * in;
            const float bi = bias ? rb(bias[i]) : 0.0f;
            for (int r = 0; r < rows; ++r) {
                const float d = dot_bf16_lanes(wi, x + (size_t)r * in, xt + (size_t)r * xs, in);
                y[(size_t)r * out + i] = bias ? rb(d + bi) : round ? rb(d) : d;
            }
        }
        free(xt);
        return;
    }
#endif
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int i = 0; i < out; ++i) {
        const uint16_t *wi = w + (size_t)i * in;
        const float bi = bias ? rb(bias[i]) : 0.0f;
        for (int r = 0; r < rows; ++r) {
            const float d = y2o_dot_bf16(wi, x + (size_t)r * in, in);
            y[(size_t)r * out + i] = bias ? rb(d + bi) : round ? rb(d) : d;
        }
    }
}

/* Linear::apply_range + finish without bias (src/tensor.rs:946-1118): every
 * output is DOT(W[i], x[r]) rounded to BF16. */
void y2o_linear(const uint16_t *w, int out, int in, const float *x, int rows, float *y) {
    dot_rows(w, out, in, x, rows, NULL, 1, y);
}

/* Unrounded DOT of every row: the yue2_metal_vector contract (the caller's
 * Linear::finish rounds), src/metal.m:545-603. */
void y2o_gemv_raw(const uint16_t *w, int rows, int cols, const float *x, float *out) {
    dot_rows(w, rows, cols, x, 1, NULL, 0, out);
}

/* ------------------------------------------------------------------------ */
/* Norms and rotary                                                         */
/* ------------------------------------------------------------------------ */

/* Norm scale: sequential f32 sum of squares, /n, +eps, sqrt, reciprocal,
 * BF16 rounding (src/tensor.rs:1144-1147). */
float y2o_norm_scale(const float *x, int n, float eps) {
    float sum = -0.0f;
    for (int i = 0; i < n; ++i) sum = sum + x[i] * x[i];
    float s = 1.0f / sqrtf(sum / (float)n + eps);
    return rb(s);
}

/* Norm::apply (src/tensor.rs:1140-1157). */
void y2o_norm_apply(const float *x, int rows, int n, const float *gamma, float eps, float *out) {
    for (int r = 0; r < rows; ++r) {
        const float *xr = x + (size_t)r * n;
        float *yr = out + (size_t)r * n;
        float s = y2o_norm_scale(xr, n, eps);
        for (int i = 0; i < n; ++i) yr[i] = rb(rb(xr[i] * s) * gamma[i]);
    }
}

/* Norm::heads (src/tensor.rs:1158-1172). */
void y2o_norm_heads(float *x, int heads, int dim, const float *gamma, float eps) {
    for (int h = 0; h < heads; ++h) {
        float *v = x + (size_t)h * dim;
        float s = y2o_norm_scale(v, dim, eps);
        for (int i = 0; i < dim; ++i) v[i] = rb(rb(v[i] * s) * gamma[i]);
    }
}

/* Rotary::new (src/model.rs:137-149): libm powf/cosf/sinf, BF16-rounded. */
void y2o_rotary_table(int start, int rows, int head_dim, float theta, float *cos_out,
                      float *sin_out) {
    int half = head_dim / 2;
    for (int i = 0; i < half; ++i) {
        float freq = 1.0f / powf(theta, (float)(2 * i) / (float)head_dim);
        for (int r = 0; r < rows; ++r) {
            float angle = (float)(start + r) * freq;
            cos_out[r * half + i] = rb(cosf(angle));
            sin_out[r * half + i] = rb(sinf(angle));
        }
    }
}

/* Rotary::apply, rotate-half with a rounding after every product and sum
 * (src/model.rs:151-168). */
void y2o_rotary_apply(float *x, int rows, int cols, int half, const float *cos_t,
                      const float *sin_t) {
    for (int r = 0; r < rows; ++r)
        for (int i = 0; i < half; ++i) {
            float c = cos_t[r * half + i], s = sin_t[r * half + i];
            for (int h = 0; h < cols / (2 * half); ++h) {
                size_t a = (size_t)r * cols + (size_t)h * 2 * half + i, b = a + half;
                float left = x[a], right = x[b];
                x[a] = rb(rb(left * c) - rb(right * s));
                x[b] = rb(rb(right * c) + rb(left * s));
            }
        }
}

/* ------------------------------------------------------------------------ */
/* Attention (src/model.rs:313-397, softmax_row src/tensor.rs:706-724)      */
/* ------------------------------------------------------------------------ */

int y2o_superblock(int blocks) { return blocks < 256 ? 1 : 2; }

void y2o_attention_row(const float *q, const float *key, const float *value, int keys,
                       int heads, int kv, int dim, float *out) {
    int groups = heads / kv, width = kv * dim;
    int blocks = (keys + 63) / 64;
    int sb = y2o_superblock(blocks);
    int streams = 512 / dim;
    float scale = 1.0f / sqrtf((float)dim);
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int h = 0; h < heads; ++h) {
        int g = h / groups;
        const float *qh = q + (size_t)h * dim;
        float *e = (float *)malloc(sizeof(float) * (size_t)keys);
        float *blk = (float *)malloc(sizeof(float) * (size_t)blocks);
        /* scores, scale (vDSP_vsmul), max (vDSP_maxv) */
        float m = -INFINITY;
        for (int j = 0; j < keys; ++j) {
            float s = y2o_dot_f32(qh, key + (size_t)j * width + (size_t)g * dim, dim) * scale;
            e[j] = s;
            if (s > m) m = s;
        }
        /* subtract (vDSP_vsadd of -max) and exp (vvexpf) */
        for (int j = 0; j < keys; ++j) e[j] = y2o_expf(e[j] - m);
        /* vDSP_sve: 64-key blocks by butterfly; the blocks of a super-block
         * left to right, then the super-blocks left to right */
        float total = 0.0f, part = 0.0f;
        for (int b = 0; b < blocks; ++b) {
            float acc[64];
            for (int l = 0; l < 64; ++l) {
                int j = b * 64 + l;
                acc[l] = j < keys ? e[j] : 0.0f;
            }
            blk[b] = butterfly64(acc);
            part = b % sb == 0 ? blk[b] : part + blk[b];
            if (b % sb == sb - 1 || b == blocks - 1) total = b < sb ? part : total + part;
        }
        /* vDSP_vsdiv */
        for (int j = 0; j < keys; ++j) e[j] = e[j] / total;
        /* PV: per block, `streams` key streams, butterfly over streams */
        for (int d = 0; d < dim; ++d) {
            float o = 0.0f, po = 0.0f;
            for (int b = 0; b < blocks; ++b) {
                float acc[64];
                for (int t = 0; t < streams; ++t) {
                    float a = 0.0f;
                    for (int j = b * 64 + t; j < b * 64 + 64 && j < keys; j += streams)
                        a = fmaf(e[j], value[(size_t)j * width + (size_t)g * dim + d], a);
                    acc[t] = a;
                }
                for (int s = streams / 2; s >= 1; s >>= 1)
                    for (int t = 0; t < s; ++t) acc[t] = acc[t] + acc[t + s];
                /* the blocks of a super-block left to right, then the
                 * super-blocks left to right */
                po = b % sb == 0 ? acc[0] : po + acc[0];
                if (b % sb == sb - 1 || b == blocks - 1) o = b < sb ? po : o + po;
            }
            out[(size_t)h * dim + d] = rb(o);
        }
        free(e);
        free(blk);
    }
}

/* ------------------------------------------------------------------------ */
/* Cache and model step                                                     */
/* ------------------------------------------------------------------------ */

y2o_cache *y2o_cache_new(const y2o_config *c, int capacity) {
    y2o_cache *cache = (y2o_cache *)calloc(1, sizeof(y2o_cache));
    if (!cache) return NULL;
    cache->layers = c->layers;
    cache->width = c->kv_heads * c->head_dim;
    cache->capacity = capacity;
    cache->length = 0;
    size_t n = (size_t)c->layers * (size_t)capacity * (size_t)cache->width;
    cache->key = (float *)calloc(n ? n : 1, sizeof(float));
    cache->value = (float *)calloc(n ? n : 1, sizeof(float));
    if (!cache->key || !cache->value) {
        y2o_cache_free(cache);
        return NULL;
    }
    return cache;
}

void y2o_cache_free(y2o_cache *cache) {
    if (!cache) return;
    free(cache->key);
    free(cache->value);
    free(cache);
}

int y2o_cache_length(const y2o_cache *cache) { return cache->length; }

/* Model::hidden (src/model.rs:523-591), CPU branch (:571-590). */
static int hidden_impl(const y2o_model *m, y2o_cache *cache, const int32_t *ids, int n,
                       float *x_out, int final_norm) {
    const y2o_config *c = &m->c;
    if (n <= 0 || cache->length + n > cache->capacity || cache->length + n > c->max_pos ||
        cache->layers != c->layers)
        return Y2O_ERR_CONTEXT;
    int H = c->hidden, d = c->head_dim, qw = c->heads * d, kw = c->kv_heads * d;
    int I = c->intermediate;
    for (int r = 0; r < n; ++r)
        if (ids[r] < 0 || ids[r] >= c->vocab) return Y2O_ERR_TOKEN;
    float *x = (float *)malloc(sizeof(float) * (size_t)n * H);
    float *h = (float *)malloc(sizeof(float) * (size_t)n * H);
    float *q = (float *)malloc(sizeof(float) * (size_t)n * qw);
    float *k = (float *)malloc(sizeof(float) * (size_t)n * kw);
    float *v = (float *)malloc(sizeof(float) * (size_t)n * kw);
    float *att = (float *)malloc(sizeof(float) * (size_t)n * qw);
    float *g = (float *)malloc(sizeof(float) * (size_t)n * I);
    float *u = (float *)malloc(sizeof(float) * (size_t)n * I);
    float *cs = (float *)malloc(sizeof(float) * (size_t)n * (d / 2));
    float *sn = (float *)malloc(sizeof(float) * (size_t)n * (d / 2));
    int rc = Y2O_OK;
    if (!x || !h || !q || !k || !v || !att || !g || !u || !cs || !sn) {
        rc = Y2O_ERR_ALLOC;
        goto done;
    }
    /* embed (src/model.rs:452-464) */
    for (int r = 0; r < n; ++r)
        for (int i = 0; i < H; ++i)
            x[(size_t)r * H + i] = rb(y2o_bf16_to_f32(m->embed[(size_t)ids[r] * H + i]));
    y2o_rotary_table(cache->length, n, d, c->theta, cs, sn);
    for (int l = 0; l < c->layers; ++l) {
        const y2o_layer *L = &m->layers[l];
        y2o_norm_apply(x, n, H, L->input_norm, c->eps, h);
        y2o_linear(L->q, qw, H, h, n, q);
        y2o_linear(L->k, kw, H, h, n, k);
        y2o_linear(L->v, kw, H, h, n, v);
        y2o_norm_heads(q, n * c->heads, d, L->q_norm, c->eps);
        y2o_norm_heads(k, n * c->kv_heads, d, L->k_norm, c->eps);
        y2o_rotary_apply(q, n, qw, d / 2, cs, sn);
        y2o_rotary_apply(k, n, kw, d / 2, cs, sn);
        float *kc = cache->key + (size_t)l * cache->capacity * kw;
        float *vc = cache->value + (size_t)l * cache->capacity * kw;
        memcpy(kc + (size_t)cache->length * kw, k, sizeof(float) * (size_t)n * kw);
        memcpy(vc + (size_t)cache->length * kw, v, sizeof(float) * (size_t)n * kw);
        for (int r = 0; r < n; ++r)
            y2o_attention_row(q + (size_t)r * qw, kc, vc, cache->length + r + 1, c->heads,
                              c->kv_heads, d, att + (size_t)r * qw);
        y2o_linear(L->o, H, qw, att, n, h);
        for (size_t i = 0; i < (size_t)n * H; ++i) x[i] = rb(x[i] + h[i]);
        y2o_norm_apply(x, n, H, L->post_norm, c->eps, h);
        y2o_linear(L->gate, I, H, h, n, g);
        y2o_linear(L->up, I, H, h, n, u);
        /* silu_slice (src/tensor.rs:661-686) then rb(g*u) (src/model.rs:209-212) */
        for (size_t i = 0; i < (size_t)n * I; ++i) {
            float gv = g[i];
            gv = rb(gv / (1.0f + y2o_expf(-gv)));
            g[i] = rb(gv * u[i]);
        }
        y2o_linear(L->down, H, I, g, n, h);
        for (size_t i = 0; i < (size_t)n * H; ++i) x[i] = rb(x[i] + h[i]);
    }
    cache->length += n;
    if (final_norm) y2o_norm_apply(x, n, H, m->final_norm, c->eps, x_out);
    else memcpy(x_out, x, sizeof(float) * (size_t)n * H);
done:
    free(x); free(h); free(q); free(k); free(v); free(att); free(g); free(u); free(cs); free(sn);
    return rc;
}

int y2o_hidden(const y2o_model *m, y2o_cache *cache, const int32_t *ids, int n, float *x_out) {
    return hidden_impl(m, cache, ids, n, x_out, 1);
}

/* hidden_impl for one new token in each of R caches (CFG's two rows) in one
 * pass over the weights: every row's arithmetic is the single-cache
 * forward's (y2o_linear computes each row's DOTs on their own; norms,
 * rotary at each row's own position, attention over each row's own cache).
 * A test-speed device for the replays of batch-2 decode loops. */
static int hidden_rows(const y2o_model *m, y2o_cache *const *caches, const int32_t *ids, int R, float *x_out) {
    const y2o_config *c = &m->c;
    if (R <= 0 || R > 8) return Y2O_ERR_CONTEXT;
    for (int r = 0; r < R; ++r) {
        const y2o_cache *ca = caches[r];
        if (ca->length + 1 > ca->capacity || ca->length + 1 > c->max_pos || ca->layers != c->layers)
            return Y2O_ERR_CONTEXT;
        if (ids[r] < 0 || ids[r] >= c->vocab) return Y2O_ERR_TOKEN;
    }
    int H = c->hidden, d = c->head_dim, qw = c->heads * d, kw = c->kv_heads * d;
    int I = c->intermediate;
    float *x = (float *)malloc(sizeof(float) * (size_t)R * H);
    float *h = (float *)malloc(sizeof(float) * (size_t)R * H);
    float *q = (float *)malloc(sizeof(float) * (size_t)R * qw);
    float *k = (float *)malloc(sizeof(float) * (size_t)R * kw);
    float *v = (float *)malloc(sizeof(float) * (size_t)R * kw);
    float *att = (float *)malloc(sizeof(float) * (size_t)R * qw);
    float *g = (float *)malloc(sizeof(float) * (size_t)R * I);
    float *u = (float *)malloc(sizeof(float) * (size_t)R * I);
    float *cs = (float *)malloc(sizeof(float) * (size_t)R * (d / 2));
    float *sn = (float *)malloc(sizeof(float) * (size_t)R * (d / 2));
    int rc = Y2O_OK;
    if (!x || !h || !q || !k || !v || !att || !g || !u || !cs || !sn) {
        rc = Y2O_ERR_ALLOC;
        goto done;
    }
    for (int r = 0; r < R; ++r) {
        for (int i = 0; i < H; ++i) x[(size_t)r * H + i] = rb(y2o_bf16_to_f32(m->embed[(size_t)ids[r] * H + i]));
        y2o_rotary_table(caches[r]->length, 1, d, c->theta, cs + (size_t)r * (d / 2), sn + (size_t)r * (d / 2));
    }
    for (int l = 0; l < c->layers; ++l) {
        const y2o_layer *L = &m->layers[l];
        y2o_norm_apply(x, R, H, L->input_norm, c->eps, h);
        y2o_linear(L->q, qw, H, h, R, q);
        y2o_linear(L->k, kw, H, h, R, k);
        y2o_linear(L->v, kw, H, h, R, v);
        y2o_norm_heads(q, R * c->heads, d, L->q_norm, c->eps);
        y2o_norm_heads(k, R * c->kv_heads, d, L->k_norm, c->eps);
        for (int r = 0; r < R; ++r) {
            y2o_cache *ca = caches[r];
            float *qr = q + (size_t)r * qw, *kr = k + (size_t)r * kw;
            y2o_rotary_apply(qr, 1, qw, d / 2, cs + (size_t)r * (d / 2), sn + (size_t)r * (d / 2));
            y2o_rotary_apply(kr, 1, kw, d / 2, cs + (size_t)r * (d / 2), sn + (size_t)r * (d / 2));
            float *kc = ca->key + (size_t)l * ca->capacity * kw;
            float *vc = ca->value + (size_t)l * ca->capacity * kw;
            memcpy(kc + (size_t)ca->length * kw, kr, sizeof(float) * (size_t)kw);
            memcpy(vc + (size_t)ca->length * kw, v + (size_t)r * kw, sizeof(float) * (size_t)kw);
            y2o_attention_row(qr, kc, vc, ca->length + 1, c->heads, c->kv_heads, d, att + (size_t)r * qw);
        }
        y2o_linear(L->o, H, qw, att, R, h);
        for (size_t i = 0; i < (size_t)R * H; ++i) x[i] = rb(x[i] + h[i]);
        y2o_norm_apply(x, R, H, L->post_norm, c->eps, h);
        y2o_linear(L->gate, I, H, h, R, g);
        y2o_linear(L->up, I, H, h, R, u);
        for (size_t i = 0; i < (size_t)R * I; ++i) {
            float gv = g[i];
            gv = rb(gv / (1.0f + y2o_expf(-gv)));
            g[i] = rb(gv * u[i]);
        }
        y2o_linear(L->down, H, I, g, R, h);
        for (size_t i = 0; i < (size_t)R * H; ++i) x[i] = rb(x[i] + h[i]);
    }
    for (int r = 0; r < R; ++r) caches[r]->length += 1;
    y2o_norm_apply(x, R, H, m->final_norm, c->eps, x_out);
done:
    free(x); free(h); free(q); free(k); free(v); free(att); free(g); free(u); free(cs); free(sn);
    return rc;
}

/* The hidden state before final_norm: what yue2_metal_ar_stack returns
 * (src/metal.m:836-846; Rust applies the final norm, src/model.rs:567). */
int y2o_hidden_prenorm(const y2o_model *m, y2o_cache *cache, const int32_t *ids, int n, float *x_out) {
    return hidden_impl(m, cache, ids, n, x_out, 0);
}

int y2o_forward(const y2o_model *m, y2o_cache *cache, const int32_t *ids, int n,
                float *logits) {
    return y2o_forward_phase(m, cache, ids, n, Y2O_PHASE_NONE, logits);
}

/* project_phase (src/model.rs:478-507).  Y2O_PHASE_NONE is Model::forward's
 * full-vocabulary head (src/model.rs:465-468). */
int y2o_project_phase(const y2o_model *m, const float *x, int phase, float *logits) {
    int V = m->c.vocab, H = m->c.hidden;
    if (phase == Y2O_PHASE_NONE) {
        y2o_linear(m->lm_head, V, H, x, 1, logits);
        return Y2O_OK;
    }
    int start, end, stop;
    if (phase == Y2O_PHASE_ABC) {
        start = 0; end = EOD; stop = ABC_END;
    } else {
        start = CODEC_OFFSET; end = CODEC_OFFSET + CODEC_SIZE; stop = MUSIC_END;
    }
    if (end > V || stop >= V) return Y2O_ERR_VOCAB;
    for (int i = 0; i < V; ++i) logits[i] = -INFINITY;
    y2o_linear(m->lm_head + (size_t)start * H, end - start, H, x, 1, logits + start);
    y2o_linear(m->lm_head + (size_t)stop * H, 1, H, x, 1, logits + stop);
    return Y2O_OK;
}

/* y2o_forward_phase of one token in each of R caches (ids[r] into
 * caches[r]), logits[r * vocab ...]; the same results as R calls. */
int y2o_forward_rows(const y2o_model *m, y2o_cache *const *caches, const int32_t *ids, int R, int phase,
                     float *logits) {
    int H = m->c.hidden, V = m->c.vocab;
    if (R <= 0 || R > 8) return Y2O_ERR_CONTEXT;
    float *x = (float *)malloc(sizeof(float) * (size_t)R * H);
    if (!x) return Y2O_ERR_ALLOC;
    int rc = hidden_rows(m, caches, ids, R, x);
    for (int r = 0; r < R && rc == Y2O_OK; ++r) rc = y2o_project_phase(m, x + (size_t)r * H, phase, logits + (size_t)r * V);
    free(x);
    return rc;
}

int y2o_forward_phase(const y2o_model *m, y2o_cache *cache, const int32_t *ids, int n,
                      int phase, float *logits) {
    int H = m->c.hidden;
    float *x = (float *)malloc(sizeof(float) * (size_t)n * H);
    if (!x) return Y2O_ERR_ALLOC;
    int rc = y2o_hidden(m, cache, ids, n, x);
    if (rc == Y2O_OK) rc = y2o_project_phase(m, x + (size_t)(n - 1) * H, phase, logits);
    free(x);
    return rc;
}

static int prefill_phase(const y2o_model *m, y2o_cache *cache, const int32_t *ids, int n,
                         int phase, float *logits) {
    if (n <= 0) return Y2O_ERR_CONTEXT;
    int H = m->c.hidden;
    float *x = (float *)malloc(sizeof(float) * (size_t)256 * H);
    if (!x) return Y2O_ERR_ALLOC;
    int rc = Y2O_OK, rows = 0;
    for (int s = 0; s < n && rc == Y2O_OK; s += 256) {
        rows = n - s < 256 ? n - s : 256;
        rc = y2o_hidden(m, cache, ids + s, rows, x);
    }
    if (rc == Y2O_OK && logits) rc = y2o_project_phase(m, x + (size_t)(rows - 1) * H, phase, logits);
    free(x);
    return rc;
}

int y2o_prefill(const y2o_model *m, y2o_cache *cache, const int32_t *ids, int n,
                float *logits) {
    return prefill_phase(m, cache, ids, n, Y2O_PHASE_NONE, logits);
}

/* ------------------------------------------------------------------------ */
/* MT19937 (src/sampling.rs:10-63)                                          */
/* ------------------------------------------------------------------------ */

/* ------------------------------------------------------------------------ */
/* NAR velocity (src/model.rs:611-698)                                      */
/* ------------------------------------------------------------------------ */

/* Linear::apply + finish with a bias (src/tensor.rs:1101-1117):
 * y = rb(DOT(W[i], x[r]) + rb(b[i])). */
static void linear_bias(const uint16_t *w, const float *b, int out, int in, const float *x, int rows,
                        float *y) {
    dot_rows(w, out, in, x, rows, b, 1, y);
}

int y2o_velocity(const y2o_model *m, const y2o_nar *nar, const y2o_cache *cache, const float *state,
                 int frames, double raw_t, int nar_cond_end, float *out) {
    const y2o_config *c = &m->c;
    if (frames <= 0 || cache->layers != c->layers) return Y2O_ERR_CONTEXT;
    const int n = frames + 2, H = c->hidden, L = nar->latent, d = c->head_dim;
    const int qw = c->heads * d, kw = c->kv_heads * d, I = c->intermediate;
    const int visible = nar_cond_end > 0 ? (nar_cond_end < cache->length ? nar_cond_end : cache->length)
                                         : cache->length;
    const int keys = visible + n;
    float *pad = (float *)calloc((size_t)n * L, sizeof(float));
    float *x = (float *)malloc(sizeof(float) * (size_t)n * H);
    float *h = (float *)malloc(sizeof(float) * (size_t)n * H);
    float *q = (float *)malloc(sizeof(float) * (size_t)n * qw);
    float *k = (float *)malloc(sizeof(float) * (size_t)n * kw);
    float *v = (float *)malloc(sizeof(float) * (size_t)n * kw);
    float *att = (float *)malloc(sizeof(float) * (size_t)n * qw);
    float *g = (float *)malloc(sizeof(float) * (size_t)n * I);
    float *u = (float *)malloc(sizeof(float) * (size_t)n * I);
    float *kk = (float *)malloc(sizeof(float) * (size_t)keys * kw);
    float *vv = (float *)malloc(sizeof(float) * (size_t)keys * kw);
    float *cs = (float *)malloc(sizeof(float) * (size_t)n * (d / 2));
    float *sn = (float *)malloc(sizeof(float) * (size_t)n * (d / 2));
    float *t0 = (float *)malloc(sizeof(float) * (size_t)H);
    float *t1 = (float *)malloc(sizeof(float) * (size_t)H);
    int rc = Y2O_OK;
    if (!pad || !x || !h || !q || !k || !v || !att || !g || !u || !kk || !vv || !cs || !sn || !t0 || !t1) {
        rc = Y2O_ERR_ALLOC;
        goto done;
    }
    /* padded latents: zero first and last rows (:620-622), vae2llm (:623) */
    memcpy(pad + L, state, sizeof(float) * (size_t)frames * L);
    linear_bias(nar->vae2llm, nar->vae2llm_b, H, L, pad, n, x);
    /* timestep (:624-628) */
    {
        const float raw = rb((float)raw_t);
        const float sig = rb(1.0f / (1.0f + y2o_expf(-raw)));
        const float top = rb(nar->shift * sig);
        const float bottom = rb(1.0f + rb((nar->shift - 1.0f) * sig));
        const float t = rb(top / bottom);
        float sinus[256];
        for (int i = 0; i < 128; ++i) {
            const float f = y2o_expf(-logf(10000.0f) * (float)i / 128.0f);
            sinus[i] = rb(cosf(t * f));
            sinus[128 + i] = rb(sinf(t * f));
        }
        /* time_in, rb(silu), time_out (:635-639) */
        linear_bias(nar->time_in, nar->time_in_b, H, 256, sinus, 1, t0);
        for (int i = 0; i < H; ++i) t0[i] = rb(t0[i] / (1.0f + y2o_expf(-t0[i])));
        linear_bias(nar->time_out, nar->time_out_b, H, H, t0, 1, t1);
    }
    /* time and latent position rows (:640-649) */
    for (int r = 0; r < n; ++r) {
        const int pr = r < nar->max_frames - 1 ? r : nar->max_frames - 1;
        for (int i = 0; i < H; ++i) {
            const float pe = rb(y2o_bf16_to_f32(nar->latent_pos[(size_t)pr * H + i]));
            float *xv = x + (size_t)r * H + i;
            *xv = rb(rb(*xv + t1[i]) + pe);
        }
    }
    /* NAR layers (:680-695), RoPE from the cache length (src/model.rs:741) */
    y2o_rotary_table(cache->length, n, d, c->theta, cs, sn);
    for (int l = 0; l < c->layers; ++l) {
        const y2o_layer *P = &nar->layers[l];
        y2o_norm_apply(x, n, H, P->input_norm, c->eps, h);
        y2o_linear(P->q, qw, H, h, n, q);
        y2o_linear(P->k, kw, H, h, n, k);
        y2o_linear(P->v, kw, H, h, n, v);
        y2o_norm_heads(q, n * c->heads, d, P->q_norm, c->eps);
        y2o_norm_heads(k, n * c->kv_heads, d, P->k_norm, c->eps);
        y2o_rotary_apply(q, n, qw, d / 2, cs, sn);
        y2o_rotary_apply(k, n, kw, d / 2, cs, sn);
        const float *kc = cache->key + (size_t)l * cache->capacity * kw;
        const float *vc = cache->value + (size_t)l * cache->capacity * kw;
        memcpy(kk, kc, sizeof(float) * (size_t)visible * kw);
        memcpy(vv, vc, sizeof(float) * (size_t)visible * kw);
        memcpy(kk + (size_t)visible * kw, k, sizeof(float) * (size_t)n * kw);
        memcpy(vv + (size_t)visible * kw, v, sizeof(float) * (size_t)n * kw);
        /* attention(q, key, value, c, None, None): every row sees every key */
        for (int r = 0; r < n; ++r)
            y2o_attention_row(q + (size_t)r * qw, kk, vv, keys, c->heads, c->kv_heads, d, att + (size_t)r * qw);
        y2o_linear(P->o, H, qw, att, n, h);
        for (size_t i = 0; i < (size_t)n * H; ++i) x[i] = rb(x[i] + h[i]);
        y2o_norm_apply(x, n, H, P->post_norm, c->eps, h);
        y2o_linear(P->gate, I, H, h, n, g);
        y2o_linear(P->up, I, H, h, n, u);
        for (size_t i = 0; i < (size_t)n * I; ++i) {
            float gv = g[i];
            gv = rb(gv / (1.0f + y2o_expf(-gv)));
            g[i] = rb(gv * u[i]);
        }
        y2o_linear(P->down, H, I, g, n, h);
        for (size_t i = 0; i < (size_t)n * H; ++i) x[i] = rb(x[i] + h[i]);
    }
    /* llm2vae(final_norm(x)[1 .. n-1]) (:696-697) */
    y2o_norm_apply(x + H, frames, H, m->final_norm, c->eps, h);
    linear_bias(nar->llm2vae, nar->llm2vae_b, L, H, h, frames, out);
done:
    free(pad); free(x); free(h); free(q); free(k); free(v); free(att); free(g); free(u);
    free(kk); free(vv); free(cs); free(sn); free(t0); free(t1);
    return rc;
}

/* uniform_f32 (src/sampling.rs:56-58) */
static float mt_uniform_f32(y2o_mt *g) { return (float)(y2o_mt_next(g) & 0x00ffffffu) / 16777216.0f; }

void y2o_normal(uint64_t seed, int n, float *out) {
    y2o_mt g;
    y2o_mt_seed(&g, seed);
    for (int i = 0; i < n; ++i) out[i] = mt_uniform_f32(&g);
    for (int b = 0; b + 16 <= n; b += 16) {
        float *blk = out + b;
        for (int i = 0; i < 8; ++i) {
            const float radius = sqrtf(-2.0f * logf(1.0f - blk[i]));
            const float theta = (float)(2.0 * 3.14159265358979323846 * (double)blk[i + 8]);
            blk[i] = radius * cosf(theta);
            blk[i + 8] = radius * sinf(theta);
        }
    }
}

/* logit (src/model.rs:777-779) */
static double logit(double t) {
    double v = log(t / (1.0 - t));
    return v < -20.0 ? -20.0 : v > 20.0 ? 20.0 : v;
}


int y2o_synthesize(const y2o_model *m, const y2o_nar *nar, const int32_t *prefix, int prefix_len,
                   const int32_t *codec, int codec_len, uint64_t seed, int steps, float *out) {
    const int L = nar->latent;
    if (L != 64 || codec_len <= 0 || steps <= 0) return Y2O_ERR_CODEC;
    for (int i = 0; i < codec_len; ++i)
        if (codec[i] < 0 || codec[i] >= CODEC_SIZE) return Y2O_ERR_CODEC;
    const int capacity = CONTEXT < m->c.max_pos ? CONTEXT : m->c.max_pos;
    if (capacity < prefix_len + 3 || (capacity - prefix_len - 3) / 2 <= 0) return Y2O_ERR_CONTEXT;
    const int size = (capacity - prefix_len - 3) / 2;
    float *noise = (float *)malloc(sizeof(float) * (size_t)codec_len * L);
    float *first = (float *)malloc(sizeof(float) * (size_t)size * L);
    float *mid = (float *)malloc(sizeof(float) * (size_t)size * L);
    int32_t *ids = (int32_t *)malloc(sizeof(int32_t) * (size_t)(prefix_len + size + 1));
    float *logits = (float *)malloc(sizeof(float) * (size_t)m->c.vocab);
    int rc = Y2O_OK;
    if (!noise || !first || !mid || !ids || !logits) {
        rc = Y2O_ERR_ALLOC;
        goto done;
    }
    y2o_normal(seed, codec_len * L, noise);
    const float dt = 1.0f / (float)steps;
    for (int start = 0; start < codec_len; start += size) {
        const int end = start + size < codec_len ? start + size : codec_len, frames = end - start;
        int n = 0;
        for (int i = 0; i < prefix_len; ++i) ids[n++] = prefix[i];
        for (int i = start; i < end; ++i) ids[n++] = codec[i] + CODEC_OFFSET;
        ids[n++] = MUSIC_END;
        y2o_cache *cache = y2o_cache_new(&m->c, n);
        if (!cache) {
            rc = Y2O_ERR_ALLOC;
            goto done;
        }
        rc = y2o_prefill(m, cache, ids, n, logits);
        float *state = out + (size_t)start * L;
        for (size_t i = 0; i < (size_t)frames * L; ++i) state[i] = rb(noise[(size_t)start * L + i]);
        for (int step = 0; step < steps && rc == Y2O_OK; ++step) {
            const double t = 1.0 - (double)step / (double)steps;
            rc = y2o_velocity(m, nar, cache, state, frames, logit(t), 0, first);
            if (rc) break;
            for (size_t i = 0; i < (size_t)frames * L; ++i) mid[i] = rb(state[i] - rb(first[i] * (dt / 2.0f)));
            rc = y2o_velocity(m, nar, cache, mid, frames, logit(t - 0.5 / (double)steps), 0, first);
            if (rc) break;
            for (size_t i = 0; i < (size_t)frames * L; ++i) state[i] = rb(state[i] - rb(first[i] * dt));
        }
        y2o_cache_free(cache);
        if (rc) goto done;
        for (size_t i = 0; i < (size_t)frames * L; ++i)
            if (!isfinite(state[i])) {
                rc = Y2O_ERR_LOGITS;
                goto done;
            }
    }
done:
    free(noise); free(first); free(mid); free(ids); free(logits);
    return rc;
}

/* ------------------------------------------------------------------------ */
/* VAE decoder (src/vae.rs:49-611), FP32                                    */
/* ------------------------------------------------------------------------ */

int y2o_conv_length(int transpose, int n, int kernel, int stride, int padding, int dilation) {
    if (transpose) return (n - 1) * stride + dilation * (kernel - 1) + 1 - 2 * padding;
    return (n + 2 * padding - dilation * (kernel - 1) - 1) / stride + 1;
}

/* Each output is the f32 sum over the patch columns (input channel major,
 * tap minor, the im2col order of Conv::apply), then the bias. */
void y2o_conv(int transpose, int cin, int cout, int kernel, int stride, int padding, int dilation,
              const float *x, int frames, const float *w, const float *b, float *out) {
    const int length = y2o_conv_length(transpose, frames, kernel, stride, padding, dilation);
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int t = 0; t < length; ++t)
        for (int o = 0; o < cout; ++o) {
            float acc = 0.0f;
            for (int i = 0; i < cin; ++i)
                for (int j = 0; j < kernel; ++j) {
                    long src;
                    float wv;
                    if (transpose) {
                        const long pos = (long)t + padding - (long)j * dilation;
                        if (pos < 0 || pos % stride) continue;
                        src = pos / stride;
                        wv = w[((size_t)i * cout + o) * kernel + j];
                    } else {
                        src = (long)t * stride + (long)j * dilation - padding;
                        wv = w[((size_t)o * cin + i) * kernel + j];
                    }
                    if (src < 0 || src >= frames) continue;
                    acc += x[(size_t)src * cin + i] * wv;
                }
            out[(size_t)t * cout + o] = acc + (b ? b[o] : 0.0f);
        }
}

int y2o_vae_length(const y2o_vae_op *ops, int nops, int frames) {
    int n = frames;
    for (int k = 0; k < nops; ++k)
        if (ops[k].kind == Y2O_VAE_CONV || ops[k].kind == Y2O_VAE_CONVT)
            n = y2o_conv_length(ops[k].kind == Y2O_VAE_CONVT, n, ops[k].kernel, ops[k].stride, ops[k].padding,
                                ops[k].dilation);
    return n;
}

int y2o_vae_run(const y2o_vae_op *ops, int nops, const float *x0, int frames, int channels, float *out,
                int *out_frames, int *out_channels) {
    int n = frames, c = channels;
    float *x = (float *)malloc(sizeof(float) * (size_t)n * c);
    float *res = NULL;
    int res_n = 0, res_c = 0, rc = Y2O_OK;
    if (!x) return Y2O_ERR_ALLOC;
    memcpy(x, x0, sizeof(float) * (size_t)n * c);
    for (int k = 0; k < nops && rc == Y2O_OK; ++k) {
        const y2o_vae_op *op = &ops[k];
        if (op->kind == Y2O_VAE_CONV || op->kind == Y2O_VAE_CONVT) {
            const int tr = op->kind == Y2O_VAE_CONVT;
            if (c != op->cin) { rc = Y2O_ERR_CONTEXT; break; }
            /* weight norm (Conv::load, src/vae.rs:86-97): rows of v's first dimension */
            const int rows = tr ? op->cin : op->cout, cols = (tr ? op->cout : op->cin) * op->kernel;
            float *w = (float *)malloc(sizeof(float) * (size_t)rows * cols);
            const int len = y2o_conv_length(tr, n, op->kernel, op->stride, op->padding, op->dilation);
            float *y = (float *)malloc(sizeof(float) * (size_t)(len > 0 ? len : 1) * op->cout);
            if (!w || !y || len <= 0) { free(w); free(y); rc = len <= 0 ? Y2O_ERR_CONTEXT : Y2O_ERR_ALLOC; break; }
            for (int r = 0; r < rows; ++r) {
                float ss = 0.0f;
                for (int q = 0; q < cols; ++q) ss += op->v[(size_t)r * cols + q] * op->v[(size_t)r * cols + q];
                const float norm = sqrtf(ss), f = op->g[r] / norm;
                for (int q = 0; q < cols; ++q) w[(size_t)r * cols + q] = op->v[(size_t)r * cols + q] * f;
            }
            y2o_conv(tr, op->cin, op->cout, op->kernel, op->stride, op->padding, op->dilation, x, n, w, op->b, y);
            free(w);
            free(x);
            x = y;
            n = len;
            c = op->cout;
        } else if (op->kind == Y2O_VAE_SNAKE) {
            /* Activation::Snake (src/vae.rs:292-306): alpha, beta = exp(params) */
            for (int i = 0; i < c; ++i) {
                const float a = expf(op->alpha[i]), ib = 1.0f / (expf(op->beta[i]) + 1e-9f);
                for (int t = 0; t < n; ++t) {
                    float *v = x + (size_t)t * c + i;
                    const float s = sinf(*v * a);
                    *v += ib * (s * s);
                }
            }
        } else if (op->kind == Y2O_VAE_ELU) {
            for (size_t i = 0; i < (size_t)n * c; ++i)
                if (x[i] < 0.0f) x[i] = expf(x[i]) - 1.0f;
        } else if (op->kind == Y2O_VAE_TANH) {
            for (size_t i = 0; i < (size_t)n * c; ++i) x[i] = tanhf(x[i]);
        } else if (op->kind == Y2O_VAE_RES_BEGIN) {
            free(res);
            res = (float *)malloc(sizeof(float) * (size_t)n * c);
            if (!res) { rc = Y2O_ERR_ALLOC; break; }
            memcpy(res, x, sizeof(float) * (size_t)n * c);
            res_n = n;
            res_c = c;
        } else if (op->kind == Y2O_VAE_RES_END) {
            /* Op::Residual: h.add(&x, false) (src/vae.rs:390-394) */
            if (!res || res_n != n || res_c != c) { rc = Y2O_ERR_CONTEXT; break; }
            for (size_t i = 0; i < (size_t)n * c; ++i) x[i] = x[i] + res[i];
            free(res);
            res = NULL;
        }
    }
    if (rc == Y2O_OK) {
        memcpy(out, x, sizeof(float) * (size_t)n * c);
        *out_frames = n;
        *out_channels = c;
    }
    free(x);
    free(res);
    return rc;
}

void y2o_mt_seed(y2o_mt *g, uint64_t seed) {
    g->state[0] = (uint32_t)seed;
    for (int i = 1; i < 624; ++i)
        g->state[i] = 1812433253u * (g->state[i - 1] ^ (g->state[i - 1] >> 30)) + (uint32_t)i;
    g->next = 624;
}

uint32_t y2o_mt_next(y2o_mt *g) {
    if (g->next == 624) {
        for (int i = 0; i < 624; ++i) {
            uint32_t bits = (g->state[i] & 0x80000000u) | (g->state[(i + 1) % 624] & 0x7fffffffu);
            g->state[i] = g->state[(i + 397) % 624] ^ (bits >> 1) ^ ((bits & 1u) ? 0x9908b0dfu : 0u);
        }
        g->next = 0;
    }
    uint32_t y = g->state[g->next++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
}

void y2o_mt_discard(y2o_mt *g, uint64_t count) {
    while (count > 0) {
        if (g->next == 624) {
            y2o_mt_next(g);
            count -= 1;
        } else {
            uint64_t skip = (uint64_t)(624 - g->next);
            if (skip > count) skip = count;
            g->next += (int)skip;
            count -= skip;
        }
    }
}

double y2o_mt_uniform_f64(y2o_mt *g) {
    uint64_t hi = y2o_mt_next(g), lo = y2o_mt_next(g);
    return (double)(((hi << 32) | lo) & ((1ull << 53) - 1)) / 9007199254740992.0;
}

/* ------------------------------------------------------------------------ */
/* CFG mix and choose (src/sampling.rs:100-215, 261-266)                    */
/* ------------------------------------------------------------------------ */

void y2o_cfg_mix(const float *cond, const float *uncond, int n, float scale, float *out) {
    for (int i = 0; i < n; ++i) {
        float v = uncond[i];
        out[i] = rb(v + rb(scale * rb(cond[i] - v)));
    }
}

static inline float cast(float x, int legacy) { return legacy ? rb(x) : x; }

/* compiler-rt __powisf2 binary exponentiation, which Rust's f32::powi lowers
 * to for a run-time exponent. */
static float powi_f32(float a, int b) {
    int recip = b < 0;
    float r = 1.0f;
    for (;;) {
        if (b & 1) r *= a;
        b /= 2;
        if (b == 0) break;
        a *= a;
    }
    return recip ? 1.0f / r : r;
}

/* f32::total_cmp key: order-preserving map of the bit pattern. */
static inline int32_t total_key(float f) {
    int32_t b = (int32_t)f2u(f);
    return b ^ (int32_t)((uint32_t)(b >> 31) >> 1);
}

static const float *g_sort_scores;
/* descending by score (total order), ascending by id */
static int cmp_desc(const void *pa, const void *pb) {
    int32_t a = *(const int32_t *)pa, b = *(const int32_t *)pb;
    int32_t ka = total_key(g_sort_scores[a]), kb = total_key(g_sort_scores[b]);
    if (ka != kb) return ka > kb ? -1 : 1;
    return a < b ? -1 : (a > b);
}

typedef struct { int32_t id; float p; } idp;
static int cmp_id(const void *pa, const void *pb) {
    int32_t a = ((const idp *)pa)->id, b = ((const idp *)pb)->id;
    return a < b ? -1 : (a > b);
}

static int phase_end(int phase) {
    return phase == Y2O_PHASE_ABC ? ABC_END : phase == Y2O_PHASE_SEMANTIC ? MUSIC_END : -1;
}

int y2o_choose(const float *logits, int n, const y2o_sampling *s, const int32_t *history,
               int history_len, int step, int phase, int legacy, y2o_mt *rng, int32_t *out) {
    int end = phase_end(phase);
    if (phase != Y2O_PHASE_NONE && n <= end) return Y2O_ERR_VOCAB;
    float *scores = (float *)malloc(sizeof(float) * (size_t)n);
    int32_t *sorted = (int32_t *)malloc(sizeof(int32_t) * (size_t)n);
    idp *probs = NULL;
    int rc = Y2O_OK;
    if (!scores || !sorted) { rc = Y2O_ERR_ALLOC; goto done; }
    for (int i = 0; i < n; ++i) scores[i] = -INFINITY;
    if (phase == Y2O_PHASE_ABC) {
        memcpy(scores, logits, sizeof(float) * EOD);
    } else if (phase == Y2O_PHASE_SEMANTIC) {
        if (n < CODEC_OFFSET + CODEC_SIZE) { rc = Y2O_ERR_CODEC; goto done; }
        memcpy(scores + CODEC_OFFSET, logits + CODEC_OFFSET, sizeof(float) * CODEC_SIZE);
    } else {
        memcpy(scores, logits, sizeof(float) * (size_t)n);
    }
    if (phase != Y2O_PHASE_NONE && step >= s->min_tokens) scores[end] = logits[end];
    /* repetition penalty over the last penalty_window ids (:130-144); each
     * distinct id is updated once, so the map's order does not matter */
    {
        int from = history_len > s->penalty_window ? history_len - s->penalty_window : 0;
        for (int i = from; i < history_len; ++i) {
            int id = history[i], seen = 0, count = 0;
            for (int j = from; j < i; ++j) seen |= history[j] == id;
            if (seen) continue;
            for (int j = i; j < history_len; ++j) count += history[j] == id;
            float alpha = cast(powi_f32(s->repetition_penalty, count), legacy);
            scores[id] = cast(scores[id] < 0.0f ? scores[id] * alpha : scores[id] / alpha, legacy);
        }
    }
    for (int i = 0; i < n; ++i)
        if (scores[i] != scores[i] || scores[i] == INFINITY) { rc = Y2O_ERR_LOGITS; goto done; }
    if (s->temperature == 0.0f) {
        int best = -1;
        for (int i = 0; i < n; ++i)
            if (isfinite(scores[i]) && (best < 0 || total_key(scores[i]) > total_key(scores[best])))
                best = i;
        if (best < 0) { rc = Y2O_ERR_EMPTY; goto done; }
        *out = best;
        goto done;
    }
    if (s->temperature != 1.0f)
        for (int i = 0; i < n; ++i) scores[i] = cast(scores[i] / s->temperature, legacy);
    int count = 0;
    for (int i = 0; i < n; ++i)
        if (isfinite(scores[i])) sorted[count++] = i;
    if (count == 0) { rc = Y2O_ERR_EMPTY; goto done; }
    /* select_nth_unstable_by + retain(>= threshold) + sort (:168-174) */
    g_sort_scores = scores;
    qsort(sorted, (size_t)count, sizeof(int32_t), cmp_desc);
    int rank = s->top_k - 1 < count - 1 ? s->top_k - 1 : count - 1;
    float threshold = scores[sorted[rank]];
    int kept = 0;
    for (int i = 0; i < count; ++i)
        if (scores[sorted[i]] >= threshold) sorted[kept++] = sorted[i];
    count = kept;
    if (s->top_p < 1.0f) {
        float max = scores[sorted[0]];
        float sum = -0.0f;
        for (int i = 0; i < count; ++i) sum = sum + y2o_expf(scores[sorted[i]] - max);
        float cumulative = 0.0f;
        int protect = legacy ? 3 : 1, keep = 0;
        for (int i = 0; i < count; ++i) {
            int id = sorted[i];
            float p = cast(y2o_expf(scores[id] - max) / sum, legacy);
            cumulative += p;
            float prior = cast(cast(cumulative, legacy) - p, legacy);
            if (prior <= s->top_p || i < protect) sorted[keep++] = id;
        }
        count = keep;
    }
    {
        float max = scores[sorted[0]];
        float sum = -0.0f;
        for (int i = 0; i < count; ++i) sum = sum + y2o_expf(scores[sorted[i]] - max);
        probs = (idp *)malloc(sizeof(idp) * (size_t)count);
        if (!probs) { rc = Y2O_ERR_ALLOC; goto done; }
        for (int i = 0; i < count; ++i) {
            probs[i].id = sorted[i];
            probs[i].p = cast(y2o_expf(scores[sorted[i]] - max) / sum, legacy);
        }
        qsort(probs, (size_t)count, sizeof(idp), cmp_id);
        /* exponential race over the full-vocabulary stream (:198-214) */
        float best = -INFINITY;
        int32_t selected = 0;
        int64_t cursor = 0;
        for (int i = 0; i < count; ++i) {
            int64_t id = probs[i].id;
            y2o_mt_discard(rng, (uint64_t)(id - cursor) * 2);
            float noise = cast((float)(-y2o_log1p(-y2o_mt_uniform_f64(rng))), legacy);
            cursor = id + 1;
            float score = cast(probs[i].p / noise, legacy);
            if (score > best) {
                best = score;
                selected = (int32_t)id;
            }
        }
        y2o_mt_discard(rng, (uint64_t)((int64_t)n - cursor) * 2);
        *out = selected;
    }
done:
    free(scores);
    free(sorted);
    free(probs);
    return rc;
}

/* Sampling::validate (src/protocol.rs:178-194). */
static int validate(const y2o_sampling *s) {
    if (!isfinite(s->temperature) || !(s->temperature >= 0.0f && s->temperature <= 5.0f) ||
        !isfinite(s->top_p) || s->top_p <= 0.0f || s->top_p > 1.0f || s->top_k < 1 ||
        !isfinite(s->repetition_penalty) || s->repetition_penalty <= 0.0f ||
        s->penalty_window < 1 || s->penalty_window > 100 || s->min_tokens > s->max_tokens ||
        s->max_tokens < 1)
        return Y2O_ERR_SAMPLING;
    return Y2O_OK;
}

/* sampling::generate (src/sampling.rs:222-294). */
int y2o_generate(const y2o_model *m, const int32_t *prefix, int prefix_len,
                 const y2o_sampling *s, uint64_t seed, int phase, const int32_t *negative,
                 int negative_len, float scale, int legacy, int32_t *tokens, int *count,
                 int *truncated) {
    int rc = validate(s);
    if (rc) return rc;
    if (prefix_len + s->max_tokens > CONTEXT ||
        (negative && negative_len + s->max_tokens > CONTEXT))
        return Y2O_ERR_BUDGET;
    if (scale != 1.0f && !negative) return Y2O_ERR_GUIDANCE;
    int V = m->c.vocab;
    y2o_cache *cache = y2o_cache_new(&m->c, prefix_len + s->max_tokens);
    y2o_cache *neg = NULL;
    float *cond = (float *)malloc(sizeof(float) * (size_t)V);
    float *uncond = (float *)malloc(sizeof(float) * (size_t)V);
    float *mixed = (float *)malloc(sizeof(float) * (size_t)V);
    *count = 0;
    *truncated = 1;
    if (!cache || !cond || !uncond || !mixed) { rc = Y2O_ERR_ALLOC; goto done; }
    rc = prefill_phase(m, cache, prefix, prefix_len, phase, cond);
    if (rc) goto done;
    if (scale != 1.0f) {
        neg = y2o_cache_new(&m->c, negative_len + s->max_tokens);
        if (!neg) { rc = Y2O_ERR_ALLOC; goto done; }
        rc = prefill_phase(m, neg, negative, negative_len, phase, uncond);
        if (rc) goto done;
    }
    y2o_mt rng;
    y2o_mt_seed(&rng, seed);
    int end = phase_end(phase);
    for (int step = 0; step < s->max_tokens; ++step) {
        if (neg) y2o_cfg_mix(cond, uncond, V, scale, mixed);
        else memcpy(mixed, cond, sizeof(float) * (size_t)V);
        int32_t id;
        rc = y2o_choose(mixed, V, s, tokens, *count, step, phase, legacy, &rng, &id);
        if (rc) goto done;
        if (id == end) { *truncated = 0; break; }
        tokens[(*count)++] = id;
        if (step + 1 < s->max_tokens) {
            rc = y2o_forward_phase(m, cache, &id, 1, phase, cond);
            if (rc) goto done;
            if (neg) {
                rc = y2o_forward_phase(m, neg, &id, 1, phase, uncond);
                if (rc) goto done;
            }
        }
    }
done:
    y2o_cache_free(cache);
    y2o_cache_free(neg);
    free(cond); free(uncond); free(mixed);
    return rc;
}
