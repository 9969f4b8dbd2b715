// Stand-in for the reference's src/qwen2.hpp (syntax check only, where the
// reference tree is absent): the members of Qwen2Hparams
// (src/qwen2.hpp:24-39) and Qwen2LayerWeights (src/qwen2.hpp:41-54) that the
// adapter reads.
#pragma once
#include "ggml.h"

namespace vv {
struct Qwen2Hparams {
    int hidden_size = 0, n_heads = 0, n_kv_heads = 0, head_dim = 0, intermediate_size = 0;
    float rope_theta = 1.0e6f, rms_norm_eps = 1.0e-6f;
    bool use_flash_attn = false;
};
struct Qwen2LayerWeights {
    struct ggml_tensor *attn_norm = nullptr, *attn_q = nullptr, *attn_q_bias = nullptr, *attn_k = nullptr,
                       *attn_k_bias = nullptr, *attn_v = nullptr, *attn_v_bias = nullptr, *attn_o = nullptr,
                       *ffn_norm = nullptr, *ffn_gate = nullptr, *ffn_up = nullptr, *ffn_down = nullptr;
};
}  // namespace vv
