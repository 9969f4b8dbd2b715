// qwen2_attn.hpp — C++ host side of the Qwen2 self-attention path.
//
// This is the caller half of the drop-in: the code that takes the place of
// the attention section of vv::qwen2_layer_forward_resident
// (src/qwen2.cpp:250-347) and of vv::ResidentKV (src/qwen2.hpp:78-89,
// src/qwen2.cpp:205-246), written against the C ABI of include/vva.h
// instead of ggml ops.  Names, argument meanings and the division of labour
// between callee and caller follow the reference:
//   - ResidentKV owns the per-layer K/V storage and a past_len that the
//     caller advances after the whole layer stack ran (src/qwen2.hpp:116-121,
//     src/vibevoice_asr.cpp:641);
//   - qwen2_attention_resident takes the reshaped projections
//     q ne=[hd, n_h, T, B], k/v ne=[hd, n_kv_h, T, B] (src/qwen2.cpp:278-280),
//     the absolute positions and an optional F16 mask, and produces the
//     cont_2d'd attention output o ne=[hd, n_h, T, B] (src/qwen2.cpp:335).
// Differences: no aborts (GGML_ASSERT at src/qwen2.cpp:269-270 becomes
// VVA_ERR_INVALID_ARG), one past_len per sequence so the two CFG streams can
// share one cache and one call, and a null mask meaning the causal mask the
// callers build on the host (src/vibevoice_asr.cpp:616-627).
#pragma once

#include <stdint.h>

#include <vector>

#include "../../include/vva.h"

namespace vva {

// Attention fields of vv::Qwen2Hparams (src/qwen2.hpp:24-39).
// use_flash_attn picks the branch of src/qwen2.cpp:327-344 for F32 caches:
// the flash branch casts the window to F16 (and runs the MFMA prefill), the
// eager branch stays fp32; other cache types are read in their own type
// either way, and no branch materialises the score matrix.
struct Qwen2Hparams {
    int   hidden_size    = 0;
    int   n_heads        = 0;
    int   n_kv_heads     = 0;
    int   head_dim       = 0;
    float rope_theta     = 1.0e6f;
    bool  use_flash_attn = true;
};

// Resident K/V of a layer stack: one K and one V tensor per (layer,
// sequence), ne=[hd, n_kv, max_seq, 1] in the chosen cache type, in one
// device allocation owned by the library (src/qwen2.cpp:207-229).
// Destruction order: free (or destroy) every ResidentKV before
// vva_destroy of its context.  vva_destroy releases the caches still alive,
// and a later free() or destructor of such a ResidentKV is then a no-op
// (the library ignores released handles), but its views are dangling.
struct ResidentKV {
    vva_context*     ctx      = nullptr;     // borrowed
    vva_kv*          kv       = nullptr;
    int              n_layers = 0;
    int              max_seq  = 0;
    int              n_seq    = 0;
    int              type     = VVA_TYPE_F16;   // cache type (ggml type number)
    std::vector<int> past_len;               // valid rows per sequence

    ResidentKV() = default;
    ResidentKV(const ResidentKV&) = delete;
    ResidentKV& operator=(const ResidentKV&) = delete;
    ~ResidentKV();

    // ResidentKV::init (src/qwen2.cpp:207-229), plus the sequence count and
    // the cache type.  Zeroes the cache.  The reference stores F32 and casts
    // the whole window to F16 before every flash-attention call
    // (src/qwen2.cpp:328-331); an F16 cache rounds each row once, at append,
    // to the same F16 values, so F16 is the default: the attention sees the
    // reference's operands at half the memory and without the per-call cast.
    bool init(vva_context* c, int n_layers, int hd, int n_kv, int max_seq, int n_seq = 1,
              int type = VVA_TYPE_F16);
    // ResidentKV::free (src/qwen2.cpp:231-244).
    void free();
    // kvs.k[layer] / kvs.v[layer] (src/qwen2.cpp:293-294) of one sequence.
    vva_tensor k(int layer, int seq = 0) const;
    vva_tensor v(int layer, int seq = 0) const;
    // Pre-baked rows (host F32 [len][n_kv][hd]) into rows [0, len) of one
    // (layer, sequence): the voice-prompt ingest of src/vibevoice_tts.cpp:735-749.
    // Does not change past_len.
    int upload(int layer, int seq, int len, const float* k_rows, const float* v_rows);
    // Error text of the last failed library call on the context.
    const char* last_error() const;
};

// The attention section of qwen2_layer_forward_resident (src/qwen2.cpp:278-347):
// RoPE of q and k (NeoX, hp.rope_theta, src/qwen2.cpp:282-287), the k/v rows
// written into the resident window at each sequence's past_len
// (src/qwen2.cpp:293-306), then attention of q over the window
// [0, past_len + T) with scale 1/sqrt(hd) (src/qwen2.cpp:312-335).
//   q:       F32/F16/BF16 ne=[hd, n_heads, T, B], rotated in place (unless q_ws);
//   k, v:    F32/F16/BF16 ne=[hd, n_kv_heads, T, B];
//   pos:     I32 ne=[T] (shared) or [T, B] (per sequence): absolute positions;
//   mask:    nullptr = causal (key j visible to row t iff j <= past_len + t),
//            or F16 ne=[>= past_len + T, T, 1, 1 or B] with 0 / -inf entries;
//   o:       F32 ne=[hd, n_heads, T, B];
//   seq_ids: host [B], the cache sequence of batch b (nullptr: b).
//   q_ws:    nullptr, or a work tensor of q's shape that receives RoPE(q)
//            instead of q: then a decode step (T = 1, mask nullptr) runs as
//            one vva_decode_step (RoPE, append and attention fused; q left
//            as it was), with the two calls' results.
// All device tensors are read and written in stream order on the context's
// stream.  past_len is not advanced: the caller does that once the whole
// stack ran for these T tokens (ResidentKV::past_len += T).  Returns a
// vva_status.
int qwen2_attention_resident(ResidentKV& kvs, int layer_idx, const vva_tensor& q, const vva_tensor& k,
                             const vva_tensor& v, const vva_tensor& pos, const vva_tensor* mask,
                             const Qwen2Hparams& hp, const vva_tensor& o, const int32_t* seq_ids = nullptr,
                             const vva_tensor* q_ws = nullptr);

// Device views of the attention weights of a layer (the attn_q / attn_k /
// attn_v / attn_o fields of vv::Qwen2LayerWeights, src/qwen2.hpp:41-54):
// ggml layout ne=[in, out] (rows of `in` contiguous), all F16 or all Q8_0;
// biases F32 ne=[out], or data == nullptr for none.
struct Qwen2AttnWeights {
    vva_tensor q, k, v, o;
    vva_tensor q_bias, k_bias, v_bias;
};

// The attention half of qwen2_layer_forward_resident from the normed input
// to the residual sum (src/qwen2.cpp:273-350): q/k/v = linear(xn) with
// bias, RoPE of q and k and the k/v rows into the resident window at each
// sequence's past_len (one fused GEMM, vva_qkv_rope_append), attention over
// the window (vva_attn), then h = x + o w_o^T (vva_out_proj_residual).
//   xn:    F32/F16/BF16 ne=[hidden, T, B], rms_norm(x) (src/qwen2.cpp:274);
//   x:     F32 ne=[hidden, T, B], the layer input;
//   q_ws:  F32 ne=[hd, n_heads, T, B], contiguous: receives the rotated q;
//   o_ws:  F32 ne=[hd, n_heads, T, B], contiguous: the attention output;
//   h:     F32 ne=[hidden, T, B], x + attn_o(o) (src/qwen2.cpp:349-350),
//          may alias x;
//   y_ws:  nullptr, or F32 ne=[(n_heads + 2 n_kv_heads) hd, T, B],
//          contiguous: then a decode step (T * B <= 8, mask nullptr) on a
//          Q8_0 cache runs as the bare projections (vva_qkv_proj into y_ws)
//          and one vva_decode_step, which rotates q and k and quantizes the
//          new rows itself, instead of vva_qkv_rope_append (projection, then
//          RoPE and the Q8_0 append as a second launch) and vva_attn; same
//          results.
// pos, mask, seq_ids, hp and the past_len contract are as for
// qwen2_attention_resident.  Returns a vva_status.
int qwen2_attention_block_resident(ResidentKV& kvs, int layer_idx, const vva_tensor& xn, const vva_tensor& x,
                                   const Qwen2AttnWeights& w, const vva_tensor& pos, const vva_tensor* mask,
                                   const Qwen2Hparams& hp, const vva_tensor& q_ws, const vva_tensor& o_ws,
                                   const vva_tensor& h, const int32_t* seq_ids = nullptr,
                                   const vva_tensor* y_ws = nullptr);

}  // namespace vva
