// qwen2_vva.cpp — ggml side of the drop-in (see qwen2_vva.hpp).  Not built
// in this repository: it needs the reference's headers and ggml's (its
// syntax is checked against stand-in declarations, tests/ggml_standin/).
#include "qwen2_vva.hpp"

#include "rms_norm.hpp"           // vv::rms_norm (src/rms_norm.hpp)

#include <math.h>

namespace vv {

namespace {

vva_tensor view_of(const struct ggml_tensor* t) { return as_vva(t); }

// the first n columns of a work tensor, reshaped to ne = [n0, n1, n2, n3]
// (contiguous)
struct ggml_tensor* work_view(struct ggml_context* g, struct ggml_tensor* w, int64_t n0, int64_t n1, int64_t n2,
                              int64_t n3) {
    const size_t es = ggml_element_size(w);
    return ggml_view_4d(g, w, n0, n1, n2, n3, n0 * es, n0 * n1 * es, n0 * n1 * n2 * es, 0);
}

// down(silu(gate(x)) * up(x)): the FFN of src/qwen2.cpp (its swiglu_ffn
// helper is file-local there)
struct ggml_tensor* swiglu(struct ggml_context* g, struct ggml_tensor* x, const Qwen2LayerWeights& w) {
    struct ggml_tensor* gt = ggml_mul_mat(g, w.ffn_gate, x);
    struct ggml_tensor* up = ggml_mul_mat(g, w.ffn_up, x);
    return ggml_mul_mat(g, w.ffn_down, ggml_swiglu_split(g, gt, up));
}

// A graph over metadata of its own (no data: vv::compute_graph allocates
// the intermediates), built by `build` and computed to completion.
template <typename F>
bool run_graph(F build) {
    struct ggml_init_params ip = {ggml_tensor_overhead() * 64 + ggml_graph_overhead(), nullptr, true};
    struct ggml_context* g = ggml_init(ip);
    if (!g) return false;
    struct ggml_cgraph* gf = ggml_new_graph(g);
    ggml_build_forward_expand(gf, build(g));
    const bool ok = compute_graph(gf);
    ggml_free(g);
    return ok;
}

bool sync(const VvaAttn& a) { return hipStreamSynchronize(a.stream) == hipSuccess; }

// the first n0 * n1 * n2 * n3 elements of an F32 work tensor as a contiguous
// library view of ne = [n0, n1, n2, n3]
vva_tensor work_rows(const struct ggml_tensor* w, int64_t n0, int64_t n1, int64_t n2, int64_t n3) {
    vva_tensor v = {};
    v.data = w->data;
    v.type = VVA_TYPE_F32;
    v.ne[0] = n0; v.ne[1] = n1; v.ne[2] = n2; v.ne[3] = n3;
    v.nb[0] = 4; v.nb[1] = 4 * n0; v.nb[2] = 4 * n0 * n1; v.nb[3] = 4 * n0 * n1 * n2;
    return v;
}

}  // namespace

vva_tensor as_vva(const struct ggml_tensor* t) {
    vva_tensor v = {};
    v.data = t->data;
    v.type = (int32_t)t->type;                  // the library uses ggml's type numbers
    for (int i = 0; i < 4; ++i) {
        v.ne[i] = t->ne[i];
        v.nb[i] = t->nb[i];
    }
    return v;
}

bool VvaAttn::init(const Qwen2Hparams& p, int n_layers, int max_seq, int n_seq, int cache_type, int max_tok,
                   hipStream_t s) {
    free();
    stream = s;
    if (vva_create(/*device=*/0, (void*)s, &ctx) != VVA_OK) return false;
    hp = {p.hidden_size, p.n_heads, p.n_kv_heads, p.head_dim, p.rope_theta, p.use_flash_attn};
    if (!kv.init(ctx, n_layers, p.head_dim, p.n_kv_heads, max_seq, n_seq, cache_type)) return false;
    struct ggml_init_params ip = {ggml_tensor_overhead() * 8, nullptr, true};
    wctx = ggml_init(ip);
    if (!wctx) return false;
    max_tokens = max_tok;
    xn = ggml_new_tensor_2d(wctx, GGML_TYPE_F32, p.hidden_size, max_tok);
    h  = ggml_new_tensor_2d(wctx, GGML_TYPE_F32, p.hidden_size, max_tok);
    q  = ggml_new_tensor_3d(wctx, GGML_TYPE_F32, p.head_dim, p.n_heads, max_tok);
    o  = ggml_new_tensor_3d(wctx, GGML_TYPE_F32, p.head_dim, p.n_heads, max_tok);
    qkv = ggml_new_tensor_2d(wctx, GGML_TYPE_F32, (p.n_heads + 2 * p.n_kv_heads) * p.head_dim, max_tok);
    wbuf = allocate_ctx_tensors(wctx);
    return wbuf != nullptr;
}

void VvaAttn::free() {
    kv.free();                                   // before the context (qwen2_attn.hpp)
    if (ctx) vva_destroy(ctx);
    ctx = nullptr;
    if (wbuf) ggml_backend_buffer_free(wbuf);
    wbuf = nullptr;
    if (wctx) ggml_free(wctx);
    wctx = nullptr;
    xn = h = q = o = qkv = nullptr;
    max_tokens = 0;
}

bool qwen2_attention_vva(VvaAttn& a, int layer_idx, struct ggml_tensor* q, struct ggml_tensor* k,
                         struct ggml_tensor* v, struct ggml_tensor* pos, const int32_t* seq_ids,
                         struct ggml_tensor* mask, struct ggml_tensor* o) {
    const vva_tensor tq = view_of(q), tk = view_of(k), tv = view_of(v), tp = view_of(pos), to = view_of(o);
    vva_tensor tm = {};
    if (mask) tm = view_of(mask);
    // a decode step (one token per stream, causal) rotates q into the work
    // tensor a.q and runs as one fused vva_decode_step
    const int64_t T = q->ne[2], B = q->ne[3] > 0 ? q->ne[3] : 1;
    vva_tensor tw = {};
    const bool step = T == 1 && !mask && B <= a.max_tokens;
    if (step) tw = work_rows(a.q, q->ne[0], q->ne[1], T, B);
    // the graph that produced q / k / v has completed (ggml_backend_graph_compute
    // returns after synchronizing); the library works on its own stream
    const int st = vva::qwen2_attention_resident(a.kv, layer_idx, tq, tk, tv, tp, mask ? &tm : nullptr, a.hp, to,
                                                 seq_ids, step ? &tw : nullptr);
    return st == VVA_OK && sync(a);
}

bool qwen2_layer_forward_vva(VvaAttn& a, struct ggml_tensor* x, struct ggml_tensor* pos, const int32_t* seq_ids,
                             struct ggml_tensor* mask, int layer_idx, const Qwen2LayerWeights& w,
                             const Qwen2Hparams& hp, struct ggml_tensor* y) {
    const int64_t hidden = x->ne[0], T = x->ne[1], B = x->ne[2] > 0 ? x->ne[2] : 1;
    if (T * B > a.max_tokens || hidden != hp.hidden_size) return false;
    // graph 1: xn = rms_norm(x) * attn_norm  (src/qwen2.cpp:273)
    struct ggml_tensor* xn = nullptr;
    const bool ok1 = run_graph([&](struct ggml_context* g) {
        xn = work_view(g, a.xn, hidden, T, B, 1);
        return ggml_cpy(g, rms_norm(g, x, w.attn_norm, hp.rms_norm_eps), xn);
    });
    if (!ok1) return false;
    // library: q/k/v + bias + RoPE + append, attention, h = x + attn_o(o)
    // (src/qwen2.cpp:274-350); the metadata of the views lives in a small
    // context of its own
    struct ggml_init_params ip = {ggml_tensor_overhead() * 8, nullptr, true};
    struct ggml_context* vc = ggml_init(ip);
    if (!vc) return false;
    struct ggml_tensor* xv = work_view(vc, a.xn, hidden, T, B, 1);
    struct ggml_tensor* hv = work_view(vc, a.h, hidden, T, B, 1);
    struct ggml_tensor* qv = work_view(vc, a.q, hp.head_dim, hp.n_heads, T, B);
    struct ggml_tensor* ov = work_view(vc, a.o, hp.head_dim, hp.n_heads, T, B);
    vva::Qwen2AttnWeights W;
    W.q = view_of(w.attn_q);
    W.k = view_of(w.attn_k);
    W.v = view_of(w.attn_v);
    W.o = view_of(w.attn_o);
    W.q_bias = w.attn_q_bias ? view_of(w.attn_q_bias) : vva_tensor{};
    W.k_bias = w.attn_k_bias ? view_of(w.attn_k_bias) : vva_tensor{};
    W.v_bias = w.attn_v_bias ? view_of(w.attn_v_bias) : vva_tensor{};
    vva_tensor tm = {};
    if (mask) tm = view_of(mask);
    // (a decode step into a Q8_0 cache projects into qkv, then one fused step)
    const vva_tensor ty = work_rows(a.qkv, (int64_t)(hp.n_heads + 2 * hp.n_kv_heads) * hp.head_dim, T, B, 1);
    const int st = vva::qwen2_attention_block_resident(a.kv, layer_idx, view_of(xv), view_of(x), W, view_of(pos),
                                                       mask ? &tm : nullptr, a.hp, view_of(qv), view_of(ov),
                                                       view_of(hv), seq_ids, &ty);
    ggml_free(vc);
    if (st != VVA_OK || !sync(a)) return false;
    // graph 2: y = h + ffn(rms_norm(h) * ffn_norm)  (src/qwen2.cpp:351-355)
    return run_graph([&](struct ggml_context* g) {
        struct ggml_tensor* h = work_view(g, a.h, hidden, T, B, 1);
        struct ggml_tensor* f = swiglu(g, rms_norm(g, h, w.ffn_norm, hp.rms_norm_eps), w);
        return ggml_cpy(g, ggml_add(g, h, f), y);
    });
}

}  // namespace vv
