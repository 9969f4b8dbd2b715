/*
 * vva.h — C ABI of the MI355X (gfx950) Qwen2 self-attention path.
 *
 * Scope: NeoX RoPE, KV-cache append, causal grouped-query attention for
 * prefill and single-token decode — the attention section of
 * vibevoice.cpp's Qwen2 layer builders (src/qwen2.cpp:101-185 classic,
 * src/qwen2.cpp:278-347 resident).  Everything else in the layer
 * (projections, norms, FFN) stays in the caller.
 *
 * Conventions (mirroring include/vibevoice.h:23-33 and src/vibevoice_capi.cpp):
 *   - every entry point returns vva_status: 0 = OK, negative = error, with
 *     the same numbering as vv_status; nothing aborts, nothing throws;
 *   - all tensor arguments are device pointers described by vva_tensor, a
 *     ggml-shaped view (ne[] element counts fastest-first, nb[] byte strides),
 *     so a ggml custom op can forward ggml_tensor fields unchanged;
 *   - a vva_context owns (or borrows) exactly one HIP stream; every call on a
 *     context is enqueued on that stream in call order, so a KV append issued
 *     before an attention call is always visible to it.  A context is not
 *     re-entrant: callers serialize, as vv_capi does with its global mutex
 *     (src/vibevoice_capi.cpp:29).
 *   - no HIP/CUDA types appear here; the stream is passed as void*.
 */
#ifndef VVA_H
#define VVA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VVA_API __attribute__((visibility("default")))

/* Status codes: numbering follows vv_status (include/vibevoice.h:23-33). */
typedef enum {
    VVA_OK                  =  0,
    VVA_ERR_GENERIC         = -1,
    VVA_ERR_INVALID_ARG     = -2,
    VVA_ERR_OUT_OF_MEMORY   = -5,
    VVA_ERR_NOT_IMPLEMENTED = -6,
    VVA_ERR_DEVICE          = -9
} vva_status;

/* Element types: numbering is ggml's enum ggml_type, so t->type of a
 * ggml_tensor can be passed straight through. */
typedef enum {
    VVA_TYPE_F32  = 0,
    VVA_TYPE_F16  = 1,
    VVA_TYPE_Q8_0 = 8,   /* GGUF block: { fp16 d; int8 qs[32]; } = 34 bytes */
    VVA_TYPE_I32  = 26,
    VVA_TYPE_BF16 = 30
} vva_type;

/* RoPE mode: ggml's GGML_ROPE_TYPE_NEOX (src/rope.hpp:14). */
#define VVA_ROPE_TYPE_NEOX 2

/* Largest number of sequences one call may touch (CFG uses 2). */
#define VVA_MAX_BATCH 16

/* ggml-shaped strided view of a device tensor.
 * ne[0] is the fastest dimension; nb[i] is the byte stride of dimension i.
 * For VVA_TYPE_Q8_0, ne[0] counts elements (a multiple of 32) and nb[0] is
 * the block size (34).  Every ne[i] must be >= 1 and data non-NULL: a call
 * with an empty tensor (e.g. zero new tokens) returns VVA_ERR_INVALID_ARG
 * and enqueues nothing. */
typedef struct {
    void*    data;
    int32_t  type;
    int64_t  ne[4];
    size_t   nb[4];
} vva_tensor;

typedef struct vva_context vva_context;
typedef struct vva_kv      vva_kv;

/* ---------------------------------------------------------------- context */

/* Create a context on HIP device `device`.  `stream` is the hipStream_t all
 * work is enqueued on (borrowed, never destroyed here); NULL selects the
 * device's null stream.  Replaces vv::backend() / init
 * (src/backend.cpp:64-133). */
VVA_API vva_status  vva_create(int device, void* stream, vva_context** out);
/* Destroys the context and every cache created on it that is still alive
 * (their handles become invalid: vva_kv_free ignores them, other calls
 * return VVA_ERR_INVALID_ARG). */
VVA_API void        vva_destroy(vva_context* ctx);
/* Rebind the context to another stream (NULL = the null stream) after
 * waiting for the work already queued on the current one. */
VVA_API vva_status  vva_set_stream(vva_context* ctx, void* stream);
/* Block until all work enqueued on the context's stream is done. */
VVA_API vva_status  vva_synchronize(vva_context* ctx);
/* Last error message recorded on this context ("" if none).  With ctx NULL
 * returns the message of the last failed vva_create. */
VVA_API const char* vva_last_error(const vva_context* ctx);
/* Library version string. */
VVA_API const char* vva_version(void);

/* Log levels: numbering follows vv_log_level (include/vibevoice.h:36-41). */
typedef enum {
    VVA_LOG_ERROR = 0,
    VVA_LOG_WARN  = 1,
    VVA_LOG_INFO  = 2,
    VVA_LOG_DEBUG = 3
} vva_log_level;

typedef void (*vva_log_cb)(vva_log_level lvl, const char* msg, void* user_data);

/* Route the library's messages to cb (NULL: none are delivered; every
 * error message stays readable through vva_last_error either way).
 * Delivered: each failed call's message (ERROR), the device a context is
 * created on (INFO), and the plans calls settle on: decode key splits,
 * prefill key splits (DEBUG).  Messages above max_lvl are dropped before
 * formatting.  cb may be called from any thread that calls the library,
 * one call at a time (a process-wide lock).  Replaces vv_set_log_callback
 * (src/common.cpp:79-84), with the level filter made explicit. */
VVA_API void        vva_set_log_callback(vva_log_cb cb, void* user_data, vva_log_level max_lvl);

/* ------------------------------------------------------------- KV cache */

/* Resident KV cache: one K and one V tensor per (layer, sequence), each
 * ggml-shaped ne = [head_dim, n_kv_heads, max_seq, 1] (memory [s][h][d]),
 * exactly the layout of ResidentKV (src/qwen2.cpp:218-220) but in any of
 * F32 / F16 / BF16 / Q8_0 and for n_seq independent sequences (the CFG
 * positive and negative streams, src/vibevoice_tts.cpp:727-730). */
typedef struct {
    int32_t n_layers;
    int32_t n_kv_heads;
    int32_t head_dim;
    int32_t max_seq;
    int32_t n_seq;
    int32_t type;       /* vva_type of the cache rows */
} vva_kv_desc;

/* Allocate (hipMalloc, one slab) and zero a cache.
 * Replaces ResidentKV::init (src/qwen2.cpp:207-229). */
VVA_API vva_status vva_kv_create(vva_context* ctx, const vva_kv_desc* desc, vva_kv** out);
/* Replaces ResidentKV::free (src/qwen2.cpp:231-244).  A handle already
 * released, by vva_kv_free or by vva_destroy of its context, is ignored. */
VVA_API void       vva_kv_free(vva_kv* kv);
/* Number of valid rows of sequence `seq` — ResidentKV::past_len
 * (src/qwen2.hpp:83), owned and advanced by the caller
 * (src/qwen2.hpp:116-121, src/vibevoice_asr.cpp:641). */
VVA_API vva_status vva_kv_get_len(const vva_kv* kv, int seq, int32_t* len);
VVA_API vva_status vva_kv_set_len(vva_kv* kv, int seq, int32_t len);
/* ggml-shaped views of the resident K and V tensors of (layer, seq):
 * ne = [head_dim, n_kv_heads, max_seq, 1].  Equivalent of kvs.k[layer] /
 * kvs.v[layer] (src/qwen2.cpp:293-294).  Either output may be NULL. */
VVA_API vva_status vva_kv_view(const vva_kv* kv, int layer, int seq,
                               vva_tensor* k, vva_tensor* v);
/* Copy host F32 rows [len][n_kv_heads][head_dim] of K and V into rows
 * [start, start+len) of (layer, seq), converting to the cache type.  Used for
 * the pre-baked voice-prompt KV (src/vibevoice_tts.cpp:735-749, layout
 * scripts/convert_voice_to_gguf.py:115-128).  Synchronous. */
VVA_API vva_status vva_kv_upload(vva_context* ctx, vva_kv* kv, int layer, int seq,
                                 int32_t start, int32_t len,
                                 const float* k_host, const float* v_host);

/* ------------------------------------------------------------------ ops */

/* NeoX RoPE, ggml_rope_ext(ctx, x, pos, NULL, n_dims, GGML_ROPE_TYPE_NEOX,
 * 0, freq_base, 1, 0, 1, 0, 0) (src/qwen2.cpp:282-287):
 *   x, dst: ne = [head_dim, n_heads, T, B], F32 / F16 / BF16 (may alias);
 *   pos:    I32, ne = [T] or [T, B] (per-sequence positions).
 * Requires n_dims == head_dim, head_dim even. */
VVA_API vva_status vva_rope_ext(vva_context* ctx, const vva_tensor* x, const vva_tensor* pos,
                                int n_dims, int mode, float freq_base, const vva_tensor* dst);

/* Fused RoPE + KV append — the RoPE of Q and K plus the two ggml_cpy's into
 * the resident views at past_len (src/qwen2.cpp:282-306):
 *   q: ne = [d, Hq,  T, B]   k, v: ne = [d, Hkv, T, B]   (F32 / F16 / BF16)
 *   pos: I32 ne = [T] or [T, B]
 *   seq_ids: host array [B] mapping batch b to a cache sequence (NULL = b)
 *   q_out: ne = [d, Hq, T, B] in F32 / F16 / BF16 (may alias q when the
 *          types match); receives RoPE(q).
 * Writes RoPE(k) and v into rows [len(seq_b), len(seq_b)+T) of (layer,
 * seq_b), converted to the cache type (Q8_0: one block per 32 values, scale
 * amax/127, codes round(x*127/amax)).  Does NOT advance len (the caller does,
 * after attention, like kv.past_len at src/vibevoice_asr.cpp:641). */
VVA_API vva_status vva_rope_append(vva_context* ctx, vva_kv* kv, int layer,
                                   const vva_tensor* q, const vva_tensor* k, const vva_tensor* v,
                                   const vva_tensor* pos, const int32_t* seq_ids,
                                   float freq_base, const vva_tensor* q_out);

/* Attention over the resident window — the FA branch
 * ggml_flash_attn_ext(q_p, k_full, v_full, mask, scale, 0, 0) with
 * set_prec(F32) and cont_2d (src/qwen2.cpp:312-335):
 *   q:    ne = [d, Hq, T, B] (F32 / F16 / BF16), already RoPE'd;
 *   seq_ids: host [B] (NULL = b);  each sequence sees L_b = len(seq_b) + T
 *         keys (the T new rows were appended by vva_rope_append);
 *   mask: NULL for implicit causal masking (key j visible to query row i
 *         iff j <= len(seq_b) + i), or F16 ne = [>=L_b, T, 1, 1 or B] with
 *         0 / -inf entries as built at src/vibevoice_asr.cpp:616-627; F32
 *         masks (ggml_soft_max_ext's type, the eager branch
 *         src/qwen2.cpp:336-344) are read as F32;
 *   out:  F32 ne = [d, Hq, T, B], the FA output layout (src/qwen2.cpp:156-159).
 * Q is rounded to the dot type of K as ggml's CPU FA does (F16 -> f16,
 * BF16 -> bf16, Q8_0 -> Q8_0 blocks, F32 -> f32, or f16 under
 * vva_set_flash_attn(1)).  T == 1 runs the split-K decode kernels; larger T
 * runs the MFMA prefill kernel (F16 / BF16 caches directly, Q8_0 and F32
 * windows after an on-device conversion to F16), or the fp32 VALU kernel
 * (F32 caches with vva_set_flash_attn(0)). */
VVA_API vva_status vva_attn(vva_context* ctx, const vva_kv* kv, int layer,
                            const vva_tensor* q, const int32_t* seq_ids,
                            const vva_tensor* mask, float scale, const vva_tensor* out);

/* Single-token decode step: vva_rope_append with T = 1 followed by vva_attn
 * over the len(seq_b) + 1 keys with the implicit causal mask, i.e. the
 * attention section of src/qwen2.cpp:282-335 for one new token per
 * sequence (the decode loops, src/vibevoice_tts.cpp:862-880,
 * src/vibevoice_asr.cpp:760-800), with the same arguments and results:
 * q, k, v ne = [d, H, 1, B]; pos I32 ne = [1] or [1, B]; q_out receives
 * RoPE(q); out F32 ne = [d, Hq, 1, B].  Unless q_out aliases q: F16 / BF16
 * caches with windows up to 8192 keys run as one kernel (RoPE, append,
 * split attention and the merge of its splits); dense Q8_0 caches run the
 * streamed decode kernel in step mode (RoPE of q, the new row appended by
 * the split that holds it) and its merge kernel, with q_out rows 16-byte
 * aligned.  Other cases run the two calls.  Results equal the two calls'
 * (bit for bit on Q8_0 caches).  Does not advance len.  No counterpart of
 * its own in the reference: it fuses three of its ops per decode step. */
VVA_API vva_status vva_decode_step(vva_context* ctx, vva_kv* kv, int layer,
                                   const vva_tensor* q, const vva_tensor* k, const vva_tensor* v,
                                   const vva_tensor* pos, const int32_t* seq_ids, float freq_base,
                                   float scale, const vva_tensor* q_out, const vva_tensor* out);

/* vva_attn without any allocation, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the reference.  Same arguments,
 * kernels and results as vva_attn; the split partials of decode and of
 * key-split prefill go to a static per-device scratch array of 36 MiB
 * (resolved once per device by vva_create) instead of the context's
 * workspace, so the call makes no hipMalloc / hipFree.  A call whose
 * partials would exceed 36 MiB returns VVA_ERR_INVALID_ARG (the automatic
 * schedule stays below 32.5 MiB for head_dim <= 128 on MI355X; forced
 * split counts of vva_set_schedule may not).  Every call on one GPU shares
 * that GPU's scratch, whose contents persist from call to call: calls that
 * overlap in time on one GPU (other streams or contexts) race; calls
 * ordered on one stream do not. */
VVA_API vva_status vva_attn_noalloc(vva_context* ctx, const vva_kv* kv, int layer,
                                    const vva_tensor* q, const int32_t* seq_ids,
                                    const vva_tensor* mask, float scale, const vva_tensor* out);

/* ggml_flash_attn_ext on arbitrary strided device tensors (ggml.h semantics):
 *   q: ne = [d, T, Hq, B] (F32 / F16 / BF16)  — the permuted q_p of
 *      src/qwen2.cpp:320;
 *   k, v: ne = [d, L, Hkv, B] (F32 / F16 / BF16 / Q8_0), any strides;
 *   mask: NULL (no masking, as in ggml) or F16 / F32 ne = [>=L, T, 1, 1 or B];
 *   dst: F32 ne = [d, Hq, T, B] (contiguous rows of d).
 * max_bias and logit_softcap must be 0 (the reference passes 0, 0 at
 * src/qwen2.cpp:332-333); anything else returns VVA_ERR_NOT_IMPLEMENTED. */
VVA_API vva_status vva_flash_attn_ext(vva_context* ctx, const vva_tensor* q, const vva_tensor* k,
                                      const vva_tensor* v, const vva_tensor* mask, float scale,
                                      float max_bias, float logit_softcap, const vva_tensor* dst);

/* Fused Q/K/V projection + bias + RoPE + KV append: the three linear()
 * calls (ggml_mul_mat + ggml_add of the bias, src/qwen2.cpp:19-25, :273-275)
 * and everything vva_rope_append does (src/qwen2.cpp:282-306), in one GEMM
 * whose epilogue rotates and stores:
 *   x:  ne = [hidden, T, B] (F32 / F16 / BF16), the normed layer input xn;
 *   wq: ne = [hidden, Hq*d], wk, wv: ne = [hidden, Hkv*d], all F16 or all
 *       Q8_0 (GGUF blocks along hidden), rows contiguous (F16: 16-byte
 *       aligned rows, Q8_0: 4-byte aligned);
 *   bq, bk, bv: F32 ne = [Hq*d] / [Hkv*d], or NULL (no bias);
 *   pos, seq_ids, freq_base: as vva_rope_append;
 *   q_out: ne = [d, Hq, T, B] (F32 / F16 / BF16), receives RoPE(x wq^T + bq).
 * Writes RoPE(x wk^T + bk) and x wv^T + bv into cache rows [len(seq_b),
 * len(seq_b) + T) of (layer, seq_b) in the cache type; does not advance len.
 * Numerics of ggml's CPU mul_mat: x is rounded to f16 (F16 weights) or
 * quantized to Q8_0 blocks (Q8_0 weights) before the dot products.
 * Requires hidden % 64 == 0, Hq*d and Hkv*d multiples of 128, d = 64 or 128;
 * otherwise VVA_ERR_NOT_IMPLEMENTED. */
VVA_API vva_status vva_qkv_rope_append(vva_context* ctx, vva_kv* kv, int layer, const vva_tensor* x,
                                       const vva_tensor* wq, const vva_tensor* wk, const vva_tensor* wv,
                                       const vva_tensor* bq, const vva_tensor* bk, const vva_tensor* bv,
                                       const vva_tensor* pos, const int32_t* seq_ids, float freq_base,
                                       const vva_tensor* q_out);

/* Q/K/V projections with bias and nothing else, for a decode step: the three
 * linear() calls (ggml_mul_mat + ggml_add of the bias, src/qwen2.cpp:19-25,
 * :273-275) at most 8 token rows at a time, whose outputs a following
 * vva_decode_step rotates and appends itself (into a Q8_0 cache the append
 * needs whole 32-dim blocks, which the fused projection of
 * vva_qkv_rope_append cannot form in its epilogue):
 *   x, wq, wk, wv, bq, bk, bv: as vva_qkv_rope_append (Mq, Mk, Mv = the
 *       weights' output rows, multiples of 64);
 *   y: F32 ne = [Mq + Mk + Mv, T, B], contiguous: token row (b, t) holds
 *      [x wq^T + bq | x wk^T + bk | x wv^T + bv].
 * Same numerics as vva_qkv_rope_append.  T * B > 8 (a prefill chunk: use
 * vva_qkv_rope_append) returns VVA_ERR_NOT_IMPLEMENTED. */
VVA_API vva_status vva_qkv_proj(vva_context* ctx, const vva_tensor* x, const vva_tensor* wq, const vva_tensor* wk,
                                const vva_tensor* wv, const vva_tensor* bq, const vva_tensor* bk,
                                const vva_tensor* bv, const vva_tensor* y);

/* Output projection + residual: h = o w_o^T + x, the ggml_mul_mat(attn_o)
 * and ggml_add(x, o) of src/qwen2.cpp:348-349:
 *   o:   ne = [Hq*d, T, B] (F32 / F16 / BF16), e.g. vva_attn's output viewed
 *        as rows of Hq*d;
 *   w_o: ne = [Hq*d, hidden], F16 or Q8_0 (same layout rules as above);
 *   x:   F32 ne = [hidden, T, B], the layer input (residual);
 *   h:   F32 ne = [hidden, T, B], may alias x.
 * Requires Hq*d % 64 == 0 and hidden % 128 == 0. */
VVA_API vva_status vva_out_proj_residual(vva_context* ctx, const vva_tensor* o, const vva_tensor* w_o,
                                         const vva_tensor* x, const vva_tensor* h);

/* Capability probe — analogue of backend_supports_flash_attn()
 * (src/backend.cpp:157-196).  Returns 1 if vva_attn / vva_flash_attn_ext can
 * run this combination on the context's device, 0 otherwise. */
VVA_API int vva_supports(const vva_context* ctx, int head_dim, int n_q_heads, int n_kv_heads,
                         int q_type, int kv_type);

/* Attention branch, as Qwen2Hparams::use_flash_attn selects it in the
 * reference (src/qwen2.hpp:38, src/qwen2.cpp:327-344).  It matters for F32
 * caches only:
 *   1 (default): the flash-attention branch, which casts the F32 window to
 *      F16 before ggml_flash_attn_ext (src/qwen2.cpp:328-331): the library
 *      does the same cast on the device and runs the MFMA prefill;
 *   0: the eager branch (mul_mat with F32 precision, soft_max_ext, mul_mat):
 *      fp32 throughout.
 * F16 / BF16 / Q8_0 caches are read in their own type either way. */
VVA_API vva_status vva_set_flash_attn(vva_context* ctx, int use_flash_attn);

/* ------------------------------------------------------------ debugging */

/* Kernel path selection for tests: 0 = automatic (default), 1 = force the
 * VALU row kernel for every attention call, 2 = automatic except that
 * single-token calls on Q8_0 caches use the register-streamed decode kernel
 * instead of the LDS-streamed one.  Per context. */
VVA_API vva_status vva_set_attn_path(vva_context* ctx, int path);
/* Number of key splits used by the last attention call: per (sequence, kv
 * head) for a single-token call, per row tile for a prefill; 0 for the row
 * kernel.  Diagnostics for tests and benchmarks. */
VVA_API int        vva_last_decode_splits(const vva_context* ctx);
/* Scheduling overrides for tests and benchmarks, per context; 0 restores the
 * automatic choice:
 *   decode_wgs      workgroups a single-token call is planned for (default:
 *                   the device's CU count);
 *   decode_splits   key splits per (sequence, head group) of the LDS-streamed
 *                   Q8_0 decode, 1..1024;
 *   prefill_splits  key splits per row tile of the MFMA prefill, 1..32.
 * No counterpart in the reference (ggml chooses its own schedule). */
VVA_API vva_status vva_set_schedule(vva_context* ctx, int decode_wgs, int decode_splits, int prefill_splits);

#ifdef __cplusplus
}
#endif

#endif /* VVA_H */
