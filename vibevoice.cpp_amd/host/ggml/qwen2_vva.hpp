// qwen2_vva.hpp — ggml side of the drop-in, for the reference's src/ tree.
//
// Not built in this repository: it includes the reference's qwen2.hpp /
// backend.hpp and ggml's headers, and ggml is not here.  A CPU test checks
// its syntax against stand-in declarations of ggml's API
// (tests/ggml_standin/).  A maintainer adds
// qwen2_vva.cpp to the reference's library target with the include
// directories <repo>/include and <repo>/vibevoice.cpp_amd/host and links
// <repo>/vibevoice.cpp_amd/lib/libvva_qwen2.a, libvva.so and amdhip64.
// Everything it does beyond moving ggml_tensor fields into vva_tensor and
// cutting the layer graph lives in the C++ host layer (qwen2_attn.hpp),
// which is compiled and GPU-tested here (tests/cpp/test_qwen2_resident.cpp).
//
// It replaces, in src/qwen2.cpp:
//   - the attention section of qwen2_layer_forward_resident (:282-335): the
//     RoPE, the ggml_cpy of the new rows into the resident tensors, the
//     window views, the per-call ggml_cast of the whole window to F16
//     (:328-331) and ggml_flash_attn_ext: qwen2_attention_vva, for callers
//     that keep ggml's projections;
//   - the whole resident layer (:250-359), computed rather than built:
//     qwen2_layer_forward_vva runs rms_norm in a ggml graph, the fused
//     projection + RoPE + append, the attention and the output projection +
//     residual through the library, and the FFN half in a second graph.
// The resident cache moves from ResidentKV's per-layer ggml tensors
// (src/qwen2.hpp:78-89) into the library (VvaAttn::kv), with one past_len
// per stream so the two CFG streams share a cache and a call.
#pragma once

#include "backend.hpp"            // vv::backend, vv::compute_graph, vv::allocate_ctx_tensors
#include "qwen2.hpp"              // vv::Qwen2Hparams, vv::Qwen2LayerWeights
#include "qwen2_attn.hpp"         // vva::ResidentKV, vva::qwen2_attention_*_resident
#include "vva.h"

#include <hip/hip_runtime_api.h>

namespace vv {

// The library context, the resident cache of a layer stack and the work
// tensors of qwen2_layer_forward_vva, on ggml's backend buffer.
struct VvaAttn {
    vva_context*          ctx    = nullptr;
    hipStream_t           stream = nullptr;   // the library's stream (null: the legacy default stream)
    vva::ResidentKV       kv;
    vva::Qwen2Hparams     hp;
    struct ggml_context*  wctx   = nullptr;   // work tensor metadata
    ggml_backend_buffer_t wbuf   = nullptr;
    struct ggml_tensor*   xn = nullptr;       // F32 [hidden, max_tokens]: rms_norm(x)
    struct ggml_tensor*   h  = nullptr;       // F32 [hidden, max_tokens]: x + attention
    struct ggml_tensor*   q  = nullptr;       // F32 [head_dim, n_heads, max_tokens]: rotated q
    struct ggml_tensor*   o  = nullptr;       // F32 [head_dim, n_heads, max_tokens]: attention output
    struct ggml_tensor*   qkv = nullptr;      // F32 [(n_heads + 2 n_kv_heads) head_dim, max_tokens]: a decode
                                              // step's bare q/k/v projections (Q8_0 caches)
    int                   max_tokens = 0;     // T * B of one call at most

    // hp: the layer stack's hyperparameters; cache_type VVA_TYPE_F16 /
    // BF16 / Q8_0 / F32.  Creates the context on `stream`.
    bool init(const Qwen2Hparams& hp, int n_layers, int max_seq, int n_seq, int cache_type, int max_tokens,
              hipStream_t stream = nullptr);
    void free();
    ~VvaAttn() { free(); }
};

// A ggml tensor as the library's view of it (same ne / nb / type numbers).
vva_tensor as_vva(const struct ggml_tensor* t);

// The attention section of qwen2_layer_forward_resident (src/qwen2.cpp:282-335)
// on tensors a ggml graph has already computed (device memory):
//   q ne=[hd, n_h, T, B], rotated in place, except for a decode step (T = 1,
//   no mask), which rotates it into a.q and runs as one vva_decode_step;
//   k, v ne=[hd, n_kv_h, T, B];
//   pos I32 ne=[T] or [T, B]; mask NULL (causal) or the F16 mask;
//   o F32 ne=[hd, n_h, T, B] (the cont_2d'd FA output).
// Returns when the result is in o.  past_len is not advanced.
bool qwen2_attention_vva(VvaAttn& a, int layer_idx, struct ggml_tensor* q, struct ggml_tensor* k,
                         struct ggml_tensor* v, struct ggml_tensor* pos, const int32_t* seq_ids,
                         struct ggml_tensor* mask, struct ggml_tensor* o);

// One resident layer, y = x + Attn(RMSNorm(x)) followed by the FFN half
// (src/qwen2.cpp:250-359), executed:
//   x, y F32 ne=[hidden, T, B] on the backend (y may be x); pos, seq_ids and
//   mask as above; T * B <= a.max_tokens.  past_len is not advanced (the
//   caller adds T after the last layer, src/vibevoice_asr.cpp:641).
bool qwen2_layer_forward_vva(VvaAttn& a, struct ggml_tensor* x, struct ggml_tensor* pos, const int32_t* seq_ids,
                             struct ggml_tensor* mask, int layer_idx, const Qwen2LayerWeights& w,
                             const Qwen2Hparams& hp, struct ggml_tensor* y);

}  // namespace vv
