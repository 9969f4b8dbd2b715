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
    this->type = type;
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

namespace {

// The shape checks of src/qwen2.cpp:262-270 as status codes, then the
// caller's past_len made the library's (src/qwen2.cpp:266: past_len is the
// source of truth) and the attention branch of src/qwen2.cpp:327-344 chosen
// (for F32 caches: F16 cast + flash attention, or fp32 eager).
int prepare(ResidentKV& kvs, int layer_idx, int64_t n_tokens, int64_t n_batch, const Qwen2Hparams& hp,
            const int32_t* seq_ids) {
    if (!kvs.kv || layer_idx < 0 || layer_idx >= kvs.n_layers) return VVA_ERR_INVALID_ARG;
    if (n_batch > VVA_MAX_BATCH) return VVA_ERR_INVALID_ARG;
    for (int64_t b = 0; b < n_batch; ++b) {
        const int s = seq_ids ? seq_ids[b] : (int)b;
        if (s < 0 || s >= kvs.n_seq) return VVA_ERR_INVALID_ARG;
        if (kvs.past_len[s] + n_tokens > kvs.max_seq) return VVA_ERR_INVALID_ARG;   // full_len <= max_seq
    }
    for (int s = 0; s < kvs.n_seq; ++s) {
        const int st = vva_kv_set_len(kvs.kv, s, kvs.past_len[s]);
        if (st != VVA_OK) return st;
    }
    return vva_set_flash_attn(kvs.ctx, hp.use_flash_attn ? 1 : 0);
}

}  // namespace

int qwen2_attention_resident(ResidentKV& kvs, int layer_idx, const vva_tensor& q, const vva_tensor& k,
                             const vva_tensor& v, const vva_tensor& pos, const vva_tensor* mask,
                             const Qwen2Hparams& hp, const vva_tensor& o, const int32_t* seq_ids,
                             const vva_tensor* q_ws) {
    const int hd = hp.head_dim;
    if (q.ne[0] != hd || q.ne[1] != hp.n_heads || k.ne[1] != hp.n_kv_heads || v.ne[1] != hp.n_kv_heads)
        return VVA_ERR_INVALID_ARG;
    if (q_ws && (q_ws->ne[0] != q.ne[0] || q_ws->ne[1] != q.ne[1] || q_ws->ne[2] != q.ne[2] ||
                 q_ws->ne[3] != q.ne[3]))
        return VVA_ERR_INVALID_ARG;
    int fa = prepare(kvs, layer_idx, q.ne[2], q.ne[3] > 0 ? q.ne[3] : 1, hp, seq_ids);
    if (fa != VVA_OK) return fa;
    const float scale = 1.0f / sqrtf((float)hd);
    const vva_tensor& qr = q_ws ? *q_ws : q;                 // where RoPE(q) goes
    if (q_ws && q.ne[2] == 1 && !mask) {
        // one new token per sequence under the causal mask: RoPE, append and
        // attention as one fused step (src/qwen2.cpp:282-335 for T = 1)
        return vva_decode_step(kvs.ctx, kvs.kv, layer_idx, &q, &k, &v, &pos, seq_ids, hp.rope_theta, scale, &qr,
                               &o);
    }
    // rope(q), rope(k), cpy(k -> window at past_len), cpy(v -> ...)  src/qwen2.cpp:282-306
    int st = vva_rope_append(kvs.ctx, kvs.kv, layer_idx, &q, &k, &v, &pos, seq_ids, hp.rope_theta, &qr);
    if (st != VVA_OK) return st;
    // views of the window + flash_attn_ext(scale 1/sqrt(hd)), prec F32  src/qwen2.cpp:312-335
    return vva_attn(kvs.ctx, kvs.kv, layer_idx, &qr, seq_ids, mask, scale, &o);
}

int qwen2_attention_block_resident(ResidentKV& kvs, int layer_idx, const vva_tensor& xn, const vva_tensor& x,
                                   const Qwen2AttnWeights& w, const vva_tensor& pos, const vva_tensor* mask,
                                   const Qwen2Hparams& hp, const vva_tensor& q_ws, const vva_tensor& o_ws,
                                   const vva_tensor& h, const int32_t* seq_ids, const vva_tensor* y_ws) {
    const int hd = hp.head_dim;
    const int64_t n_tokens = xn.ne[1], n_batch = xn.ne[2] > 0 ? xn.ne[2] : 1;
    if (xn.ne[0] != hp.hidden_size || q_ws.ne[0] != hd || q_ws.ne[1] != hp.n_heads || q_ws.ne[2] != n_tokens ||
        o_ws.ne[0] != hd || o_ws.ne[1] != hp.n_heads || o_ws.ne[2] != n_tokens)
        return VVA_ERR_INVALID_ARG;
    // o_ws is read back as rows of n_heads * hd (the cont_2d of src/qwen2.cpp:335)
    if (o_ws.type != VVA_TYPE_F32 || o_ws.nb[0] != 4 || o_ws.nb[1] != (size_t)4 * hd) return VVA_ERR_INVALID_ARG;
    int st = prepare(kvs, layer_idx, n_tokens, n_batch, hp, seq_ids);
    if (st != VVA_OK) return st;
    // q, k, v = linear(xn) + bias; rope(q), rope(k); k, v -> window  src/qwen2.cpp:273-306
    const vva_tensor* bq = w.q_bias.data ? &w.q_bias : nullptr;
    const vva_tensor* bk = w.k_bias.data ? &w.k_bias : nullptr;
    const vva_tensor* bv = w.v_bias.data ? &w.v_bias : nullptr;
    const float scale = 1.0f / sqrtf((float)hd);
    if (y_ws && !mask && n_tokens * n_batch <= 8 && kvs.type == VVA_TYPE_Q8_0) {
        // a decode step into a Q8_0 cache: the bare projections, then RoPE,
        // the append and attention as one fused step (src/qwen2.cpp:273-335)
        const int64_t mq = (int64_t)hp.n_heads * hd, mkv = (int64_t)hp.n_kv_heads * hd;
        if (y_ws->ne[0] != mq + 2 * mkv) return VVA_ERR_INVALID_ARG;
        st = vva_qkv_proj(kvs.ctx, &xn, &w.q, &w.k, &w.v, bq, bk, bv, y_ws);
        if (st != VVA_OK) return st;
        auto part = [&](int64_t first, int64_t heads) {     // q, k or v of every token row
            vva_tensor t = *y_ws;
            t.data = (char*)y_ws->data + first * 4;
            t.ne[0] = hd; t.ne[1] = heads; t.ne[2] = n_tokens; t.ne[3] = n_batch;
            t.nb[0] = 4; t.nb[1] = (size_t)4 * hd; t.nb[2] = y_ws->nb[1]; t.nb[3] = y_ws->nb[2];
            return t;
        };
        const vva_tensor q = part(0, hp.n_heads), k = part(mq, hp.n_kv_heads), v = part(mq + mkv, hp.n_kv_heads);
        st = vva_decode_step(kvs.ctx, kvs.kv, layer_idx, &q, &k, &v, &pos, seq_ids, hp.rope_theta, scale, &q_ws,
                             &o_ws);
        if (st != VVA_OK) return st;
    } else {
        st = vva_qkv_rope_append(kvs.ctx, kvs.kv, layer_idx, &xn, &w.q, &w.k, &w.v, bq, bk, bv, &pos, seq_ids,
                                 hp.rope_theta, &q_ws);
        if (st != VVA_OK) return st;
        // flash_attn_ext over the window  src/qwen2.cpp:312-335
        st = vva_attn(kvs.ctx, kvs.kv, layer_idx, &q_ws, seq_ids, mask, scale, &o_ws);
        if (st != VVA_OK) return st;
    }
    // h = x + attn_o(o)  src/qwen2.cpp:349-350
    vva_tensor rows = o_ws;
    rows.ne[0] = (int64_t)hp.n_heads * hd; rows.ne[1] = n_tokens; rows.ne[2] = n_batch; rows.ne[3] = 1;
    rows.nb[1] = o_ws.nb[2]; rows.nb[2] = o_ws.nb[3]; rows.nb[3] = o_ws.nb[3] * n_batch;
    return vva_out_proj_residual(kvs.ctx, &rows, &w.o, &x, &h);
}

}  // namespace vva
