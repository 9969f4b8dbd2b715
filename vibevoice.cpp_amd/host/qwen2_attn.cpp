// qwen2_attn.cpp — C++ host side of the Qwen2 self-attention path (see
// qwen2_attn.hpp).  Calls only the C ABI of include/vva.h.
#include "qwen2_attn.hpp"

#include <math.h>

namespace vva {

ResidentKV::~ResidentKV() { free(); }

bool ResidentKV::init(vva_context* c, int n_layers_in, int hd, int n_kv, int max_seq_in, int n_seq_in,
                      int type) {
    free();
    if (!c || n_seq_in < 1) return false;
    const vva_kv_desc d = {n_layers_in, n_kv, hd, max_seq_in, n_seq_in, type};
    if (vva_kv_create(c, &d, &kv) != VVA_OK) {
        kv = nullptr;
        return false;
    }
    ctx = c;
    n_layers = n_layers_in;
    max_seq = max_seq_in;
    n_seq = n_seq_in;
    past_len.assign(n_seq_in, 0);
    return true;
}

void ResidentKV::free() {
    if (kv) vva_kv_free(kv);
    kv = nullptr;
    ctx = nullptr;
    n_layers = 0;
    max_seq = 0;
    n_seq = 0;
    past_len.clear();
}

vva_tensor ResidentKV::k(int layer, int seq) const {
    vva_tensor t = {};
    if (kv) vva_kv_view(kv, layer, seq, &t, nullptr);
    return t;
}

vva_tensor ResidentKV::v(int layer, int seq) const {
    vva_tensor t = {};
    if (kv) vva_kv_view(kv, layer, seq, nullptr, &t);
    return t;
}

int ResidentKV::upload(int layer, int seq, int len, const float* k_rows, const float* v_rows) {
    if (!kv) return VVA_ERR_INVALID_ARG;
    return vva_kv_upload(ctx, kv, layer, seq, 0, len, k_rows, v_rows);
}

const char* ResidentKV::last_error() const { return vva_last_error(ctx); }

int qwen2_attention_resident(ResidentKV& kvs, int layer_idx, const vva_tensor& q, const vva_tensor& k,
                             const vva_tensor& v, const vva_tensor& pos, const vva_tensor* mask,
                             const Qwen2Hparams& hp, const vva_tensor& o, const int32_t* seq_ids) {
    // shape checks of src/qwen2.cpp:262-270, as status codes
    if (!kvs.kv || layer_idx < 0 || layer_idx >= kvs.n_layers) return VVA_ERR_INVALID_ARG;
    const int hd = hp.head_dim;
    const int64_t n_tokens = q.ne[2];
    const int64_t n_batch = q.ne[3] > 0 ? q.ne[3] : 1;
    if (q.ne[0] != hd || q.ne[1] != hp.n_heads || k.ne[1] != hp.n_kv_heads || v.ne[1] != hp.n_kv_heads)
        return VVA_ERR_INVALID_ARG;
    if (n_batch > VVA_MAX_BATCH) return VVA_ERR_INVALID_ARG;
    for (int64_t b = 0; b < n_batch; ++b) {
        const int s = seq_ids ? seq_ids[b] : (int)b;
        if (s < 0 || s >= kvs.n_seq) return VVA_ERR_INVALID_ARG;
        if (kvs.past_len[s] + n_tokens > kvs.max_seq) return VVA_ERR_INVALID_ARG;   // full_len <= max_seq
    }
    // the caller's past_len is the source of truth (src/qwen2.cpp:266)
    for (int s = 0; s < kvs.n_seq; ++s) {
        const int st = vva_kv_set_len(kvs.kv, s, kvs.past_len[s]);
        if (st != VVA_OK) return st;
    }
    // the branch of src/qwen2.cpp:327-344 (for F32 caches: F16 cast + flash
    // attention, or fp32 eager)
    int fa = vva_set_flash_attn(kvs.ctx, hp.use_flash_attn ? 1 : 0);
    if (fa != VVA_OK) return fa;
    // rope(q), rope(k), cpy(k -> window at past_len), cpy(v -> ...)  src/qwen2.cpp:282-306
    int st = vva_rope_append(kvs.ctx, kvs.kv, layer_idx, &q, &k, &v, &pos, seq_ids, hp.rope_theta, &q);
    if (st != VVA_OK) return st;
    // views of the window + flash_attn_ext(scale 1/sqrt(hd)), prec F32  src/qwen2.cpp:312-335
    const float scale = 1.0f / sqrtf((float)hd);
    return vva_attn(kvs.ctx, kvs.kv, layer_idx, &q, seq_ids, mask, scale, &o);
}

}  // namespace vva
