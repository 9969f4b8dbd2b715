/*
 * vvo.h — CPU oracle for the Qwen2 self-attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the arithmetic
 * that vibevoice.cpp delegates to ggml's CPU backend on its attention path
 * (src/qwen2.cpp:101-185, :278-347).  It is the checker for the HIP library
 * and the timed CPU baseline; nothing in the product links or calls it.
 *
 * ggml itself is absent from the reference tree (third_party/ggml is an
 * empty submodule, .gitmodules:1-3; pinned commit unknown), so the ggml
 * semantics below are restated from ggml's published algorithm and are
 * pinned by closed forms, invariants and fp64 brute force in tests/.
 *
 * Two attention modes:
 *   VVO_EXACT  — fp64 softmax(scale*QK^T + mask)V on the stored operands
 *                (Q optionally rounded to K's dot type first);
 *   VVO_GGML   — ggml CPU flash_attn_ext one-chunk order: per-key online
 *                softmax in fp32 with expf, F16 running V accumulator when V
 *                is F16, F32 otherwise.
 *   VVO_GGML_F32ACC — the same order with an F32 running V accumulator for
 *                every V type (identical to VVO_GGML unless V is F16): it
 *                separates the F16 accumulator's own rounding, which grows
 *                with the number of keys a row sees, from the rest of
 *                ggml's order.
 *
 * Parity unpinned: the bit-level ggml choices VVO_GGML encodes (the fp32
 * theta recurrence of VVO_THETA_RECURRENCE, Q rounded to K's dot type, the
 * F16 V accumulator, expf per key) cannot be checked against ggml itself,
 * which is absent; the tests bound VVO_GGML against VVO_EXACT, which closed
 * forms, invariants and fp64 brute force do pin.
 */
#ifndef VVO_H
#define VVO_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Type numbering = ggml_type (and vva_type). */
enum { VVO_F32 = 0, VVO_F16 = 1, VVO_Q8_0 = 8, VVO_BF16 = 30 };
enum { VVO_EXACT = 0, VVO_GGML = 1, VVO_GGML_F32ACC = 2 };
enum { VVO_MASK_NONE = 0, VVO_MASK_EXPLICIT = 1, VVO_MASK_CAUSAL = 2 };
enum { VVO_THETA_RECURRENCE = 0, VVO_THETA_POW = 1 };

#define VVO_MAX_B 16
#define VVO_QK8_0 32

/* scalar conversions (round-to-nearest-even, IEEE special values kept) */
uint16_t vvo_f32_to_f16(float x);
float    vvo_f16_to_f32(uint16_t h);
uint16_t vvo_f32_to_bf16(float x);
float    vvo_bf16_to_f32(uint16_t h);

/* bytes of one row of n elements of `type` */
int64_t  vvo_row_bytes(int type, int64_t n);
/* F32 -> type (n a multiple of 32 for Q8_0) and type -> F32 */
void     vvo_from_f32(const float* src, void* dst, int type, int64_t n);
void     vvo_to_f32(const void* src, int type, float* dst, int64_t n);
/* GGUF Q8_0 blocks */
void     vvo_quantize_q8_0(const float* x, void* y, int64_t n);
void     vvo_dequantize_q8_0(const void* x, float* y, int64_t n);

/* NeoX RoPE on contiguous x[B][T][H][d] -> y (may alias).
 * pos[b*pos_stride_b + t] is the absolute position of token t of batch b. */
void     vvo_rope_neox(const float* x, float* y, const int32_t* pos, int64_t pos_stride_b,
                       int64_t d, int64_t n_heads, int64_t T, int64_t B,
                       float freq_base, int theta_mode);

typedef struct {
    int32_t d, n_q_heads, n_kv_heads, T, B;
    const float* q;                  /* F32 [B][T][Hq][d], RoPE'd */
    int32_t k_type, v_type;
    const void* k[VVO_MAX_B];        /* cache of batch b: rows [L_b][Hkv] of d */
    const void* v[VVO_MAX_B];
    int32_t L[VVO_MAX_B];            /* visible keys of batch b */
    int32_t past[VVO_MAX_B];         /* causal: query t sees keys j <= past_b + t */
    const uint16_t* mask;            /* F16, row t of batch b at mask + b*mask_b_stride + t*mask_row_stride */
    int64_t mask_row_stride, mask_b_stride;  /* in elements */
    int32_t mask_mode;
    float   scale;
    float*  out;                     /* F32 [B][T][Hq][d] */
    int32_t mode;                    /* VVO_EXACT / VVO_GGML / VVO_GGML_F32ACC */
    int32_t q_round;                 /* 1: round Q to K's dot type first */
    int32_t n_threads;               /* <= 0: all cores */
    const int32_t* rows;             /* optional subset of flattened rows b*T+t (NULL: all) */
    int32_t n_rows;
} vvo_attn_args;

int      vvo_attn(const vvo_attn_args* a);
int      vvo_n_cores(void);
/* 1 (default): F16 rows of the ggml-order attention converted 8 at a time
 * with F16C (same values); 0: the scalar conversions */
void     vvo_set_simd(int on);

/* Linear layer y = x W^T (+ bias): ggml_mul_mat(W, x) followed by ggml_add
 * of the bias (linear(), src/qwen2.cpp:19-25), as used for the q/k/v
 * projections (src/qwen2.cpp:273-275) and the output projection
 * (src/qwen2.cpp:348).
 *   w: M rows of K elements of w_type (F16, or Q8_0 blocks along K), row
 *      stride w_row_bytes;  x: F32 [N][K];  bias: F32 [M] or NULL;
 *   y: F32 [N][M].
 * VVO_EXACT: fp64 sum of dequantized w times unrounded x.
 * VVO_GGML:  ggml's CPU vec-dot order: x converted to W's vec-dot type
 *            first (F16: rounded to f16, products summed in fp32 in k
 *            order; Q8_0: x quantized to Q8_0 blocks, integer block sums
 *            times d_w * d_x summed in fp32 in block order), then the bias
 *            added in fp32.
 * Returns 0, or -2 on bad arguments. */
int      vvo_linear(const void* w, int w_type, int64_t w_row_bytes, const float* bias, const float* x,
                    float* y, int64_t N, int64_t K, int64_t M, int mode, int n_threads);

#ifdef __cplusplus
}
#endif
#endif
