/*
 * vvo.c — CPU oracle for the Qwen2 self-attention path.
 *
 * TEST INFRASTRUCTURE ONLY (checker and CPU baseline; never linked into the
 * product).  Restates the ggml CPU arithmetic that vibevoice.cpp's attention
 * path runs; ggml is absent from the reference tree, so every function here
 * is pinned by the tests under tests/ (closed forms, invariants, fp64 brute
 * force, exhaustive conversion sweeps, known-answer Q8_0 blocks).
 *
 * Reference call sites restated:
 *   ggml_rope_ext NEOX, theta 1e6       src/qwen2.cpp:282-287, src/rope.hpp:14-15
 *   ggml_cpy into the resident views    src/qwen2.cpp:293-306
 *   ggml_cast F32->F16 of K/V           src/qwen2.cpp:328-331
 *   ggml_flash_attn_ext + prec F32      src/qwen2.cpp:332-335
 *   eager mul_mat/soft_max_ext/mul_mat  src/qwen2.cpp:337-343
 *   causal F16 mask (0 / -inf)          src/vibevoice_asr.cpp:616-627
 */
#define _GNU_SOURCE
#include "vvo.h"

#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdlib.h>
#include <string.h>

#if defined(__F16C__) && defined(__AVX2__) && defined(__FMA__)
#include <immintrin.h>
#define VVO_F16C 1
#endif

/* The ggml-order attention's F16 rows may be converted 8 at a time with the
 * F16C instructions (vcvtph2ps, and vcvtps2ph with round-to-nearest-even: the
 * same values as the scalar conversions below for every finite input).
 * vvo_set_simd(0) selects the scalar loops, so the tests can compare the two. */
static int g_simd = 1;
void vvo_set_simd(int on) { g_simd = on; }

/* ------------------------------------------------------------ conversions */

static inline uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float    bits_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* f32 -> f16, round to nearest even.  Method: F. Giesen's "float_to_half
 * RTNE" construction — normal results round by adding a bias that includes
 * the lowest kept mantissa bit; subnormal results let the FPU round by adding
 * a magic constant whose ulp equals the f16 subnormal step (2^-24). */
uint16_t vvo_f32_to_f16(float f) {
    uint32_t x    = f_bits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    x &= 0x7fffffffu;
    uint16_t o;
    if (x >= (uint32_t)(127 + 16) << 23) {               /* >= 65536, inf, nan */
        o = (x > 0x7f800000u) ? 0x7e00u : 0x7c00u;
    } else if (x < (uint32_t)113 << 23) {                /* < 2^-14: subnormal or 0 */
        /* 0.5 has ulp 2^-24 = the f16 subnormal step: adding it rounds x
         * (< 2^-14) to a multiple of 2^-24 with the FPU's RNE */
        const float magic = 0.5f;
        float y = bits_f(x) + magic;
        o = (uint16_t)(f_bits(y) - f_bits(magic));
    } else {
        uint32_t odd = (x >> 13) & 1u;
        x += ((uint32_t)(15 - 127) << 23) + 0xfffu + odd;  /* rebias + round */
        o = (uint16_t)(x >> 13);
    }
    return (uint16_t)(o | sign);
}

static float g_f16_table[65536];
static pthread_once_t g_f16_once = PTHREAD_ONCE_INIT;

static float f16_to_f32_slow(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-08f;       /* m * 2^-24, exact */
        return bits_f(f_bits(v) | sign);
    }
    if (e == 31) return bits_f(sign | 0x7f800000u | (m << 13));
    return bits_f(sign | ((e + 112u) << 23) | (m << 13));
}
static void f16_table_init(void) {
    for (uint32_t i = 0; i < 65536; ++i) g_f16_table[i] = f16_to_f32_slow((uint16_t)i);
}
float vvo_f16_to_f32(uint16_t h) {
    pthread_once(&g_f16_once, f16_table_init);
    return g_f16_table[h];
}
static inline float h2f(uint16_t h) { return g_f16_table[h]; }

/* f32 -> bf16, round to nearest even; NaN kept quiet (ggml_compute_fp32_to_bf16
 * behaviour). */
uint16_t vvo_f32_to_bf16(float f) {
    uint32_t x = f_bits(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    return (uint16_t)((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
}
float vvo_bf16_to_f32(uint16_t h) { return bits_f((uint32_t)h << 16); }

/* ------------------------------------------------------------------ Q8_0 */
/* GGUF Q8_0 block (ggml's block_q8_0): fp16 scale d, then 32 int8 codes.
 * Quantization as ggml's reference quantize_row_q8_0: d = amax/127,
 * id = d ? 1/d : 0, code = roundf(x*id) (ties away from zero). */

void vvo_quantize_q8_0(const float* x, void* y, int64_t n) {
    uint8_t* out = (uint8_t*)y;
    for (int64_t b = 0; b < n / VVO_QK8_0; ++b) {
        const float* xb = x + b * VVO_QK8_0;
        float amax = 0.0f;
        for (int j = 0; j < VVO_QK8_0; ++j) {
            float a = fabsf(xb[j]);
            if (a > amax) amax = a;
        }
        const float d  = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint16_t dh = vvo_f32_to_f16(d);
        uint8_t* blk = out + b * 34;
        memcpy(blk, &dh, 2);
        for (int j = 0; j < VVO_QK8_0; ++j) {
            int8_t c = (int8_t)roundf(xb[j] * id);
            memcpy(blk + 2 + j, &c, 1);
        }
    }
}

void vvo_dequantize_q8_0(const void* x, float* y, int64_t n) {
    pthread_once(&g_f16_once, f16_table_init);
    const uint8_t* in = (const uint8_t*)x;
    for (int64_t b = 0; b < n / VVO_QK8_0; ++b) {
        const uint8_t* blk = in + b * 34;
        uint16_t dh; memcpy(&dh, blk, 2);
        const float d = h2f(dh);
        for (int j = 0; j < VVO_QK8_0; ++j) y[b * VVO_QK8_0 + j] = (float)(int8_t)blk[2 + j] * d;
    }
}

int64_t vvo_row_bytes(int type, int64_t n) {
    switch (type) {
        case VVO_F32:  return 4 * n;
        case VVO_F16:
        case VVO_BF16: return 2 * n;
        case VVO_Q8_0: return (n / VVO_QK8_0) * 34;
        default:       return -1;
    }
}

void vvo_from_f32(const float* src, void* dst, int type, int64_t n) {
    switch (type) {
        case VVO_F32:  memcpy(dst, src, 4 * n); break;
        case VVO_F16:  for (int64_t i = 0; i < n; ++i) ((uint16_t*)dst)[i] = vvo_f32_to_f16(src[i]); break;
        case VVO_BF16: for (int64_t i = 0; i < n; ++i) ((uint16_t*)dst)[i] = vvo_f32_to_bf16(src[i]); break;
        case VVO_Q8_0: vvo_quantize_q8_0(src, dst, n); break;
        default: break;
    }
}

void vvo_to_f32(const void* src, int type, float* dst, int64_t n) {
    pthread_once(&g_f16_once, f16_table_init);
    switch (type) {
        case VVO_F32:  memcpy(dst, src, 4 * n); break;
        case VVO_F16:  for (int64_t i = 0; i < n; ++i) dst[i] = h2f(((const uint16_t*)src)[i]); break;
        case VVO_BF16: for (int64_t i = 0; i < n; ++i) dst[i] = vvo_bf16_to_f32(((const uint16_t*)src)[i]); break;
        case VVO_Q8_0: vvo_dequantize_q8_0(src, dst, n); break;
        default: break;
    }
}

/* ------------------------------------------------------------------ RoPE */
/* NeoX: pair (x[i], x[i + d/2]) rotated by theta_i = pos * base^(-2i/d)
 * (tests/dump_rope_reference.py:22-37).  Recurrence mode builds theta as
 * ggml's CPU rope cache does: theta_0 = (float)pos, theta_{i+1} = theta_i *
 * powf(base, -2/d) in fp32, then cosf/sinf.  Pow mode is the fp64 closed
 * form. */
void vvo_rope_neox(const float* x, float* y, const int32_t* pos, int64_t pos_stride_b,
                   int64_t d, int64_t n_heads, int64_t T, int64_t B,
                   float freq_base, int theta_mode) {
    const int64_t half = d / 2;
    float*  cs = (float*)malloc(sizeof(float) * 2 * half);
    double* cd = (double*)malloc(sizeof(double) * 2 * half);
    const float theta_scale = powf(freq_base, -2.0f / (float)d);
    for (int64_t b = 0; b < B; ++b) {
        for (int64_t t = 0; t < T; ++t) {
            const int32_t p = pos[b * pos_stride_b + t];
            if (theta_mode == VVO_THETA_RECURRENCE) {
                float theta = (float)p;
                for (int64_t i = 0; i < half; ++i) {
                    cs[2 * i] = cosf(theta);
                    cs[2 * i + 1] = sinf(theta);
                    theta *= theta_scale;
                }
            } else {
                for (int64_t i = 0; i < half; ++i) {
                    double th = (double)p * pow((double)freq_base, -2.0 * (double)i / (double)d);
                    cd[2 * i] = cos(th);
                    cd[2 * i + 1] = sin(th);
                }
            }
            for (int64_t h = 0; h < n_heads; ++h) {
                const int64_t off = ((b * T + t) * n_heads + h) * d;
                for (int64_t i = 0; i < half; ++i) {
                    const float x0 = x[off + i], x1 = x[off + i + half];
                    if (theta_mode == VVO_THETA_RECURRENCE) {
                        const float c = cs[2 * i], s = cs[2 * i + 1];
                        y[off + i]        = fmaf(x0, c, -(x1 * s));
                        y[off + i + half] = fmaf(x0, s, x1 * c);
                    } else {
                        const double c = cd[2 * i], s = cd[2 * i + 1];
                        y[off + i]        = (float)((double)x0 * c - (double)x1 * s);
                        y[off + i + half] = (float)((double)x0 * s + (double)x1 * c);
                    }
                }
            }
        }
    }
    free(cs);
    free(cd);
}

/* ------------------------------------------------------------- attention */

typedef struct {
    const vvo_attn_args* a;
    int64_t n_items;            /* rows * Hq */
    int64_t next;               /* shared work counter */
    int     err;
} attn_job;

/* Row j, kv head h of a cache of `type` as doubles. */
static void load_row_f64(const void* base, int type, int64_t row_bytes, int64_t head_bytes,
                         int64_t j, int h, int d, double* out) {
    const uint8_t* p = (const uint8_t*)base + j * row_bytes + (int64_t)h * head_bytes;
    switch (type) {
        case VVO_F32: for (int i = 0; i < d; ++i) out[i] = ((const float*)p)[i]; break;
        case VVO_F16: for (int i = 0; i < d; ++i) out[i] = h2f(((const uint16_t*)p)[i]); break;
        case VVO_BF16: for (int i = 0; i < d; ++i) out[i] = vvo_bf16_to_f32(((const uint16_t*)p)[i]); break;
        case VVO_Q8_0:
            for (int b = 0; b < d / VVO_QK8_0; ++b) {
                uint16_t dh; memcpy(&dh, p + b * 34, 2);
                const double sc = h2f(dh);
                for (int i = 0; i < VVO_QK8_0; ++i)
                    out[b * VVO_QK8_0 + i] = sc * (double)(int8_t)p[b * 34 + 2 + i];
            }
            break;
    }
}

/* Q rounded to K's vec-dot type, as ggml's flash_attn_ext converts Q with
 * the K type's from_float before the dot (F16 -> f16, BF16 -> bf16,
 * Q8_0 -> Q8_0 blocks, F32 unchanged). */
static void round_q(const float* q, int k_type, int d, float* qr, uint8_t* q8) {
    switch (k_type) {
        case VVO_F16:  for (int i = 0; i < d; ++i) qr[i] = h2f(vvo_f32_to_f16(q[i])); break;
        case VVO_BF16: for (int i = 0; i < d; ++i) qr[i] = vvo_bf16_to_f32(vvo_f32_to_bf16(q[i])); break;
        case VVO_Q8_0: vvo_quantize_q8_0(q, q8, d); vvo_dequantize_q8_0(q8, qr, d); break;
        default:       memcpy(qr, q, sizeof(float) * d); break;
    }
}

/* fp32 dot with 32 independent partial sums (the lane structure of ggml's
 * AVX2 F16/F32 dot: 4 accumulators x 8 lanes), reduced pairwise. */
static float dot32(const float* a, const float* b, int d) {
    float acc[32] = {0};
    for (int i = 0; i < d; i += 32)
        for (int j = 0; j < 32; ++j) acc[j] = fmaf(a[i + j], b[i + j], acc[j]);
    for (int w = 16; w >= 1; w >>= 1)
        for (int j = 0; j < w; ++j) acc[j] += acc[j + w];
    return acc[0];
}

static void attn_exact_one(const vvo_attn_args* a, int b, int t, int h,
                           double* s, double* krow, double* acc, float* qr, uint8_t* q8) {
    const int d = a->d, g = a->n_q_heads / a->n_kv_heads, kvh = h / g;
    const int64_t hk = vvo_row_bytes(a->k_type, d), hv = vvo_row_bytes(a->v_type, d);
    const int64_t rk = hk * a->n_kv_heads, rv = hv * a->n_kv_heads;
    const float* q = a->q + (((int64_t)b * a->T + t) * a->n_q_heads + h) * d;
    float* o = a->out + (((int64_t)b * a->T + t) * a->n_q_heads + h) * d;
    if (a->q_round) round_q(q, a->k_type, d, qr, q8);
    else memcpy(qr, q, sizeof(float) * d);
    const int L = a->L[b];
    double m = -INFINITY;
    for (int j = 0; j < L; ++j) {
        double mv = 0.0;
        if (a->mask_mode == VVO_MASK_CAUSAL) {
            if (j > a->past[b] + t) { s[j] = -INFINITY; continue; }
        } else if (a->mask_mode == VVO_MASK_EXPLICIT) {
            mv = h2f(a->mask[b * a->mask_b_stride + (int64_t)t * a->mask_row_stride + j]);
            if (mv == -INFINITY) { s[j] = -INFINITY; continue; }
        }
        load_row_f64(a->k[b], a->k_type, rk, hk, j, kvh, d, krow);
        double dot = 0.0;
        for (int i = 0; i < d; ++i) dot += (double)qr[i] * krow[i];
        s[j] = dot * (double)a->scale + mv;
        if (s[j] > m) m = s[j];
    }
    for (int i = 0; i < d; ++i) acc[i] = 0.0;
    if (m == -INFINITY) { for (int i = 0; i < d; ++i) o[i] = 0.0f; return; }
    double sum = 0.0;
    for (int j = 0; j < L; ++j) {
        if (s[j] == -INFINITY) continue;
        const double p = exp(s[j] - m);
        sum += p;
        load_row_f64(a->v[b], a->v_type, rv, hv, j, kvh, d, krow);
        for (int i = 0; i < d; ++i) acc[i] += p * krow[i];
    }
    for (int i = 0; i < d; ++i) o[i] = (float)(acc[i] / sum);
}

/* ggml CPU flash_attn_ext, one query row: keys in order, online softmax in
 * fp32 with expf; the running V sum is F16 when V is F16 (scaled and
 * accumulated with an f16 rounding per step), F32 otherwise (and always F32
 * in VVO_GGML_F32ACC mode); 1/S with S == 0 treated as 0. */
static void attn_ggml_one(const vvo_attn_args* a, int b, int t, int h,
                          float* vkq, uint16_t* vkq16, float* qr, uint8_t* q8, float* krow) {
    const int d = a->d, g = a->n_q_heads / a->n_kv_heads, kvh = h / g;
    const int64_t hk = vvo_row_bytes(a->k_type, d), hv = vvo_row_bytes(a->v_type, d);
    const int64_t rk = hk * a->n_kv_heads, rv = hv * a->n_kv_heads;
    const float* q = a->q + (((int64_t)b * a->T + t) * a->n_q_heads + h) * d;
    float* o = a->out + (((int64_t)b * a->T + t) * a->n_q_heads + h) * d;
    round_q(q, a->k_type, d, qr, q8);
    const int L = a->L[b];
    const int v16 = a->v_type == VVO_F16 && a->mode == VVO_GGML;
    for (int i = 0; i < d; ++i) { vkq[i] = 0.0f; vkq16[i] = 0; }
    float S = 0.0f, M = -INFINITY;
    for (int j = 0; j < L; ++j) {
        float mv = 0.0f;
        if (a->mask_mode == VVO_MASK_CAUSAL) {
            if (j > a->past[b] + t) continue;
        } else if (a->mask_mode == VVO_MASK_EXPLICIT) {
            mv = h2f(a->mask[b * a->mask_b_stride + (int64_t)t * a->mask_row_stride + j]);
            if (mv == -INFINITY) continue;
        }
        const uint8_t* kp = (const uint8_t*)a->k[b] + (int64_t)j * rk + (int64_t)kvh * hk;
        float s;
        if (a->k_type == VVO_Q8_0) {
            s = 0.0f;
            for (int blk = 0; blk < d / VVO_QK8_0; ++blk) {
                uint16_t dk, dq;
                memcpy(&dk, kp + blk * 34, 2);
                memcpy(&dq, q8 + blk * 34, 2);
                int sumi = 0;
                for (int i = 0; i < VVO_QK8_0; ++i)
                    sumi += (int)(int8_t)kp[blk * 34 + 2 + i] * (int)(int8_t)q8[blk * 34 + 2 + i];
                s += (float)sumi * (h2f(dk) * h2f(dq));
            }
        } else {
#ifdef VVO_F16C
            if (g_simd && a->k_type == VVO_F16 && d % 8 == 0) {
                for (int i = 0; i < d; i += 8)
                    _mm256_storeu_ps(krow + i, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(kp + 2 * i))));
            } else
#endif
            vvo_to_f32(kp, a->k_type, krow, d);
            s = dot32(qr, krow, d);
        }
        s = s * a->scale;
        s += mv;
        const float Mold = M;
        float ms = 1.0f, vs = 1.0f;
        const uint8_t* vp = (const uint8_t*)a->v[b] + (int64_t)j * rv + (int64_t)kvh * hv;
#ifdef VVO_F16C
        const int vec16 = v16 && g_simd && d % 8 == 0;
#else
        const int vec16 = 0;
#endif
        if (s > M) {
            M = s;
            ms = expf(Mold - M);
            if (vec16) {
#ifdef VVO_F16C
                const __m256 f = _mm256_set1_ps(ms);
                for (int i = 0; i < d; i += 8) {
                    const __m256 x = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(vkq16 + i)));
                    _mm_storeu_si128((__m128i*)(vkq16 + i), _mm256_cvtps_ph(_mm256_mul_ps(x, f), _MM_FROUND_TO_NEAREST_INT));
                }
#endif
            } else if (v16) {
                for (int i = 0; i < d; ++i) vkq16[i] = vvo_f32_to_f16(h2f(vkq16[i]) * ms);
            } else {
                for (int i = 0; i < d; ++i) vkq[i] *= ms;
            }
        } else {
            vs = expf(s - M);
        }
        if (vec16) {
#ifdef VVO_F16C
            const __m256 f = _mm256_set1_ps(vs);
            for (int i = 0; i < d; i += 8) {
                const __m256 v = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(vp + 2 * i)));
                const __m256 x = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(vkq16 + i)));
                _mm_storeu_si128((__m128i*)(vkq16 + i), _mm256_cvtps_ph(_mm256_fmadd_ps(v, f, x), _MM_FROUND_TO_NEAREST_INT));
            }
#endif
        } else if (v16) {
            const uint16_t* vv = (const uint16_t*)vp;
            for (int i = 0; i < d; ++i) vkq16[i] = vvo_f32_to_f16(fmaf(h2f(vv[i]), vs, h2f(vkq16[i])));
        } else {
            vvo_to_f32(vp, a->v_type, krow, d);
            for (int i = 0; i < d; ++i) vkq[i] = fmaf(krow[i], vs, vkq[i]);
        }
        S = S * ms + vs;
    }
    if (v16) for (int i = 0; i < d; ++i) vkq[i] = h2f(vkq16[i]);
    const float S_inv = S == 0.0f ? 0.0f : 1.0f / S;
    for (int i = 0; i < d; ++i) o[i] = vkq[i] * S_inv;
}

static void* attn_worker(void* arg) {
    attn_job* job = (attn_job*)arg;
    const vvo_attn_args* a = job->a;
    const int d = a->d;
    int Lmax = 1;
    for (int b = 0; b < a->B; ++b) if (a->L[b] > Lmax) Lmax = a->L[b];
    double* s    = (double*)malloc(sizeof(double) * Lmax);
    double* krow = (double*)malloc(sizeof(double) * d);
    double* acc  = (double*)malloc(sizeof(double) * d);
    float*  vkq  = (float*)malloc(sizeof(float) * d);
    float*  qr   = (float*)malloc(sizeof(float) * d);
    float*  kf   = (float*)malloc(sizeof(float) * d);
    uint16_t* vkq16 = (uint16_t*)malloc(sizeof(uint16_t) * d);
    uint8_t*  q8    = (uint8_t*)malloc((size_t)(d / VVO_QK8_0) * 34 + 34);
    if (!s || !krow || !acc || !vkq || !qr || !kf || !vkq16 || !q8) {
        job->err = 1;
    } else {
        const int64_t chunk = 4;
        for (;;) {
            int64_t it0 = __atomic_fetch_add(&job->next, chunk, __ATOMIC_RELAXED);
            if (it0 >= job->n_items) break;
            int64_t it1 = it0 + chunk < job->n_items ? it0 + chunk : job->n_items;
            for (int64_t it = it0; it < it1; ++it) {
                const int64_t ri = it / a->n_q_heads;
                const int h = (int)(it % a->n_q_heads);
                const int64_t row = a->rows ? a->rows[ri] : ri;
                const int b = (int)(row / a->T), t = (int)(row % a->T);
                if (a->mode == VVO_EXACT) attn_exact_one(a, b, t, h, s, krow, acc, qr, q8);
                else                      attn_ggml_one(a, b, t, h, vkq, vkq16, qr, q8, kf);
            }
        }
    }
    free(s); free(krow); free(acc); free(vkq); free(qr); free(kf); free(vkq16); free(q8);
    return NULL;
}

int vvo_n_cores(void) {
    cpu_set_t set;
    if (sched_getaffinity(0, sizeof(set), &set) == 0) return CPU_COUNT(&set);
    return 1;
}

int vvo_attn(const vvo_attn_args* a) {
    if (!a || a->d <= 0 || a->d % VVO_QK8_0 || a->n_kv_heads <= 0 || a->n_q_heads % a->n_kv_heads ||
        a->B <= 0 || a->B > VVO_MAX_B || a->T <= 0)
        return -2;
    pthread_once(&g_f16_once, f16_table_init);
    attn_job job;
    job.a = a;
    job.n_items = (int64_t)(a->rows ? a->n_rows : a->B * a->T) * a->n_q_heads;
    job.next = 0;
    job.err = 0;
    int nt = a->n_threads > 0 ? a->n_threads : vvo_n_cores();
    if (nt > 256) nt = 256;
    pthread_t th[256];
    int started = 0;
    for (int i = 1; i < nt; ++i)
        if (pthread_create(&th[started], NULL, attn_worker, &job) == 0) ++started;
    attn_worker(&job);
    for (int i = 0; i < started; ++i) pthread_join(th[i], NULL);
    return job.err ? -5 : 0;
}

/* ------------------------------------------------------------ linear */

typedef struct {
    const uint8_t* w; int w_type; int64_t w_row_bytes;
    const float* bias; const float* x; float* y;
    int64_t N, K, M; int mode;
    const float* xr;          /* GGML, F16: x rounded to f16 (as f32) [N][K] */
    const uint8_t* xq;        /* GGML, Q8_0: x as Q8_0 blocks [N][K/32 * 34] */
    int64_t next;
} linear_job;

static void* linear_worker(void* arg) {
    linear_job* j = (linear_job*)arg;
    const int64_t K = j->K, nb = K / VVO_QK8_0;
    double* wd = (double*)malloc(sizeof(double) * K);
    float* wf = (float*)malloc(sizeof(float) * K);
    if (!wd || !wf) { free(wd); free(wf); return NULL; }
    for (;;) {
        const int64_t m = __atomic_fetch_add(&j->next, 1, __ATOMIC_RELAXED);
        if (m >= j->M) break;
        const uint8_t* wr = j->w + m * j->w_row_bytes;
        vvo_to_f32(wr, j->w_type, wf, K);
        for (int64_t k = 0; k < K; ++k) wd[k] = wf[k];
        for (int64_t n = 0; n < j->N; ++n) {
            float out;
            if (j->mode == VVO_EXACT) {
                const float* xn = j->x + n * K;
                double acc = 0.0;
                for (int64_t k = 0; k < K; ++k) acc += wd[k] * (double)xn[k];
                if (j->bias) acc += (double)j->bias[m];
                out = (float)acc;
            } else if (j->w_type == VVO_Q8_0) {
                const uint8_t* xb = j->xq + n * nb * 34;
                float acc = 0.0f;
                for (int64_t b = 0; b < nb; ++b) {
                    uint16_t dw, dx;
                    memcpy(&dw, wr + b * 34, 2);
                    memcpy(&dx, xb + b * 34, 2);
                    int sumi = 0;
                    for (int i = 0; i < VVO_QK8_0; ++i)
                        sumi += (int)(int8_t)wr[b * 34 + 2 + i] * (int)(int8_t)xb[b * 34 + 2 + i];
                    acc += (float)sumi * (h2f(dw) * h2f(dx));
                }
                out = j->bias ? acc + j->bias[m] : acc;
            } else {
                const float* xn = j->xr + n * K;
                float acc = 0.0f;
                for (int64_t k = 0; k < K; ++k) acc = fmaf(wf[k], xn[k], acc);
                out = j->bias ? acc + j->bias[m] : acc;
            }
            j->y[n * j->M + m] = out;
        }
    }
    free(wd);
    free(wf);
    return NULL;
}

int vvo_linear(const void* w, int w_type, int64_t w_row_bytes, const float* bias, const float* x, float* y,
               int64_t N, int64_t K, int64_t M, int mode, int n_threads) {
    if (!w || !x || !y || N <= 0 || K <= 0 || M <= 0) return -2;
    if (w_type != VVO_F16 && w_type != VVO_Q8_0) return -2;
    if (w_type == VVO_Q8_0 && K % VVO_QK8_0) return -2;
    if (w_row_bytes < vvo_row_bytes(w_type, K)) return -2;
    pthread_once(&g_f16_once, f16_table_init);
    linear_job j = {(const uint8_t*)w, w_type, w_row_bytes, bias, x, y, N, K, M, mode, NULL, NULL, 0};
    float* xr = NULL;
    uint8_t* xq = NULL;
    if (mode != VVO_EXACT) {
        if (w_type == VVO_F16) {
            xr = (float*)malloc(sizeof(float) * N * K);
            if (!xr) return -5;
            for (int64_t i = 0; i < N * K; ++i) xr[i] = h2f(vvo_f32_to_f16(x[i]));
            j.xr = xr;
        } else {
            xq = (uint8_t*)malloc((size_t)(N * (K / VVO_QK8_0) * 34));
            if (!xq) return -5;
            for (int64_t n = 0; n < N; ++n) vvo_quantize_q8_0(x + n * K, xq + n * (K / VVO_QK8_0) * 34, K);
            j.xq = xq;
        }
    }
    int nt = n_threads > 0 ? n_threads : vvo_n_cores();
    if (nt > 256) nt = 256;
    pthread_t th[256];
    int started = 0;
    for (int i = 1; i < nt; ++i)
        if (pthread_create(&th[started], NULL, linear_worker, &j) == 0) ++started;
    linear_worker(&j);
    for (int i = 0; i < started; ++i) pthread_join(th[i], NULL);
    free(xr);
    free(xq);
    return 0;
}
