// test_qwen2_resident.cpp — the resident-KV call sequences of the reference's
// tests/test_qwen2_resident.cpp, driven through the C++ host layer
// (vibevoice.cpp_amd/host/qwen2_attn.hpp) and the C ABI, on the GPU.
//
// Like the reference test, one program runs several paths over the same
// inputs and asserts that they agree, returning a distinct non-zero code for
// each failure:
//   chunks     one layer, 7B shapes (28 q / 4 kv heads, d 128), F16 cache, BF16
//              projections: one shot (path B), two chunks (C), four uneven
//              chunks (D).  Cache bytes identical across paths; outputs within
//              the reference's chunked-FA tolerance 1e-3
//              (tests/test_qwen2_resident.cpp:478-479); the one-shot output
//              against the oracle at 2e-3 max-abs / 1e-3 mean-abs; the cache
//              rows against RoPE + conversion on the host (V byte-exact, K
//              within one f16 ulp).
//   stack      three layers fed chunk by chunk, past_len advanced once per
//              chunk after the whole stack (src/vibevoice_asr.cpp:641), against
//              each layer run in one shot (path E's per-layer isolation).
//   cfg        the TTS CFG decode of the 0.5B LM (14 q / 2 kv heads, d 64, F16
//              cache): two sequences with voice prompts of different lengths
//              (src/vibevoice_tts.cpp:735-749), then decode steps with B = 2,
//              per-sequence positions pos ne=[1, 2], against the oracle.
//   q8         the ASR CFG decode on Q8_0 caches at the 7B shapes, ragged
//              lengths, against the oracle.
//   block      the attention half of the layer through
//              qwen2_attention_block_resident (fused Q/K/V projection + bias +
//              RoPE + append, attention, output projection + residual) at the
//              0.5B shapes, F16 and Q8_0 weights: a 96-token chunk over a
//              40-token past, then a B = 2 CFG decode step over ragged pasts;
//              q, the appended rows, o and h against the oracle (ggml-order
//              linear layers, RoPE recurrence, attention on the device's own
//              operands).
//   step       the cfg and q8 decodes with a q work buffer, so each layer's
//              step runs as one vva_decode_step, in lockstep with the two-call
//              path on a twin cache: rotated q and cache rows bit-identical,
//              outputs bit-identical on Q8_0 caches and within 2e-3 / 1e-3 on
//              F16, and against the oracle.
//   timing     a 28-layer 7B CFG decode step (B = 2, Q8_0 cache, 32k and 2k
//              keys) four ways: the two calls or the fused step, with a
//              stream synchronization after every layer (as the ggml adapter
//              does between its graphs) or once per step.  Prints the time per
//              step; asserts only that every call succeeds.
//   errors     past_len + T > max_seq, a bad layer and a bad sequence id come
//              back as VVA_ERR_INVALID_ARG (the reference's GGML_ASSERTs,
//              src/qwen2.cpp:269-270).
//   supports   the flash-attention probe shape of src/backend.cpp:157-196.
//
// The oracle (oracle/vvo.h) is the checker only.  Usage: test_qwen2_resident
// [--list | name ...]; no names runs everything.
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <chrono>
#include <functional>
#include <string>
#include <vector>

#include "../../oracle/vvo.h"
#include "../../vibevoice.cpp_amd/host/qwen2_attn.hpp"

namespace {

// ------------------------------------------------------------ inputs

// splitmix64 -> Box-Muller in double, cast to float
struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed) {}
    uint64_t next() {
        uint64_t z = (s += 0x9e3779b97f4a7c15ull);
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        return z ^ (z >> 31);
    }
    double uniform() { return ((next() >> 11) + 0.5) * (1.0 / 9007199254740992.0); }
    std::vector<float> normal(size_t n) {
        std::vector<float> x(n);
        for (size_t i = 0; i < n; i += 2) {
            const double r = sqrt(-2.0 * log(uniform())), t = 6.283185307179586 * uniform();
            x[i] = (float)(r * cos(t));
            if (i + 1 < n) x[i + 1] = (float)(r * sin(t));
        }
        return x;
    }
};

// values as stored in `type` and read back
std::vector<float> rounded(const std::vector<float>& x, int type) {
    if (type == VVO_F32) return x;
    std::vector<uint16_t> h(x.size());
    vvo_from_f32(x.data(), h.data(), type, (int64_t)x.size());
    std::vector<float> y(x.size());
    vvo_to_f32(h.data(), type, y.data(), (int64_t)x.size());
    return y;
}

// ------------------------------------------------------------ device buffers

struct Dev {
    void* p = nullptr;
    size_t n = 0;
    explicit Dev(size_t bytes) : n(bytes) {
        if (hipMalloc(&p, bytes) != hipSuccess) p = nullptr;
    }
    ~Dev() {
        if (p) (void)hipFree(p);
    }
    Dev(const Dev&) = delete;
    Dev& operator=(const Dev&) = delete;
};

size_t elt(int type) { return type == VVA_TYPE_F32 || type == VVA_TYPE_I32 ? 4 : 2; }

// contiguous ggml-shaped view
vva_tensor view4(void* data, int type, int64_t n0, int64_t n1, int64_t n2, int64_t n3) {
    vva_tensor t = {};
    t.data = data;
    t.type = type;
    t.ne[0] = n0; t.ne[1] = n1; t.ne[2] = n2; t.ne[3] = n3;
    t.nb[0] = elt(type);
    t.nb[1] = t.nb[0] * n0;
    t.nb[2] = t.nb[1] * n1;
    t.nb[3] = t.nb[2] * n2;
    return t;
}

// host F32 [B][T][H][d] -> device tensor of `type`
void upload_as(Dev& d, const std::vector<float>& x, int type) {
    if (type == VVA_TYPE_F32) {
        (void)hipMemcpy(d.p, x.data(), x.size() * 4, hipMemcpyHostToDevice);
        return;
    }
    std::vector<uint16_t> h(x.size());
    vvo_from_f32(x.data(), h.data(), type, (int64_t)x.size());
    (void)hipMemcpy(d.p, h.data(), h.size() * 2, hipMemcpyHostToDevice);
}

std::vector<float> download_f32(const void* p, size_t n, int type) {
    std::vector<float> y(n);
    if (type == VVA_TYPE_F32) {
        (void)hipMemcpy(y.data(), p, n * 4, hipMemcpyDeviceToHost);
    } else {
        std::vector<uint16_t> h(n);
        (void)hipMemcpy(h.data(), p, n * 2, hipMemcpyDeviceToHost);
        vvo_to_f32(h.data(), type, y.data(), (int64_t)n);
    }
    return y;
}

// raw rows [0, rows) of a resident K or V tensor
std::vector<uint8_t> cache_bytes(const vva_tensor& t, int rows) {
    std::vector<uint8_t> b((size_t)rows * t.nb[2]);
    (void)hipMemcpy(b.data(), t.data, b.size(), hipMemcpyDeviceToHost);
    return b;
}

// ------------------------------------------------------------ checks

struct Stats {
    double max_abs = 0.0, mean_abs = 0.0;
    bool finite = true;
};

Stats compare(const std::vector<float>& got, const std::vector<float>& ref, size_t off = 0, size_t n = 0) {
    if (n == 0) n = got.size() - off;
    Stats s;
    double sum = 0.0;
    for (size_t i = off; i < off + n; ++i) {
        if (!std::isfinite(got[i])) s.finite = false;
        const double d = fabs((double)got[i] - (double)ref[i]);
        s.max_abs = d > s.max_abs ? d : s.max_abs;
        sum += d;
    }
    s.mean_abs = sum / (double)n;
    return s;
}

bool within(const char* what, const Stats& s, double max_tol, double mean_tol) {
    const bool ok = s.finite && s.max_abs <= max_tol && s.mean_abs <= mean_tol;
    printf("  %-44s max %.3e (tol %.0e)  mean %.3e (tol %.0e)  %s\n", what, s.max_abs, max_tol, s.mean_abs,
           mean_tol, ok ? "ok" : "FAIL");
    return ok;
}

bool status_ok(const char* what, int st, const vva::ResidentKV& kvs) {
    if (st == VVA_OK) return true;
    printf("  %s: status %d (%s)\n", what, st, kvs.last_error());
    return false;
}

// The oracle on the device's own operands: the rotated q (read back from the
// device) and the cache rows [0, L_b) of each sequence.
std::vector<float> oracle_out(const std::vector<float>& q32, const vva::ResidentKV& kvs, int layer,
                              const std::vector<int>& seqs, const std::vector<int>& L, int T, int Hq,
                              int Hkv, int d, int kv_type) {
    const int B = (int)seqs.size();
    std::vector<std::vector<uint8_t>> kb(B), vb(B);
    vvo_attn_args a;
    memset(&a, 0, sizeof(a));
    a.d = d; a.n_q_heads = Hq; a.n_kv_heads = Hkv; a.T = T; a.B = B;
    a.q = q32.data();
    a.k_type = kv_type; a.v_type = kv_type;
    for (int b = 0; b < B; ++b) {
        kb[b] = cache_bytes(kvs.k(layer, seqs[b]), L[b]);
        vb[b] = cache_bytes(kvs.v(layer, seqs[b]), L[b]);
        a.k[b] = kb[b].data();
        a.v[b] = vb[b].data();
        a.L[b] = L[b];
        a.past[b] = L[b] - T;
    }
    a.mask_mode = VVO_MASK_CAUSAL;
    a.scale = 1.0f / sqrtf((float)d);
    std::vector<float> out((size_t)B * T * Hq * d);
    a.out = out.data();
    a.mode = VVO_EXACT;
    a.q_round = 1;
    if (vvo_attn(&a) != 0) out.assign(out.size(), NAN);
    return out;
}

// One layer's projections of N tokens (B = 1), as the three linear layers
// would hand them over (src/qwen2.cpp:273-280), already in `in_type`.
struct Proj {
    std::vector<float> q, k, v;   // f32 [N][H][d], values representable in in_type
};

Proj make_proj(uint64_t seed, int N, int Hq, int Hkv, int d, int in_type) {
    Rng r(seed);
    Proj p;
    p.q = rounded(r.normal((size_t)N * Hq * d), in_type);
    p.k = rounded(r.normal((size_t)N * Hkv * d), in_type);
    p.v = rounded(r.normal((size_t)N * Hkv * d), in_type);
    return p;
}

// Runs tokens [bounds[i], bounds[i+1]) of every layer's projections chunk by
// chunk through qwen2_attention_resident, layer-major inside a chunk, and
// advances past_len once per chunk.  Returns the outputs per layer
// (f32 [N][Hq][d]) and the rotated q per layer (read back, f32).
struct Replay {
    std::vector<std::vector<float>> out, qr;
    bool ok = true;
};

Replay replay(vva::ResidentKV& kvs, const std::vector<Proj>& layers, const std::vector<int>& bounds, int Hq,
              int Hkv, int d, int in_type) {
    Replay r;
    const int N = bounds.back();
    const vva::Qwen2Hparams hp = {Hq * d, Hq, Hkv, d, 1.0e6f, true};
    for (size_t l = 0; l < layers.size(); ++l) {
        r.out.emplace_back((size_t)N * Hq * d);
        r.qr.emplace_back((size_t)N * Hq * d);
    }
    for (size_t c = 0; c + 1 < bounds.size(); ++c) {
        const int a = bounds[c], T = bounds[c + 1] - bounds[c];
        std::vector<int32_t> pos(T);
        for (int t = 0; t < T; ++t) pos[t] = a + t;
        Dev dpos(4 * (size_t)T);
        (void)hipMemcpy(dpos.p, pos.data(), 4 * (size_t)T, hipMemcpyHostToDevice);
        for (size_t l = 0; l < layers.size(); ++l) {
            const Proj& p = layers[l];
            const size_t nq = (size_t)T * Hq * d, nk = (size_t)T * Hkv * d;
            Dev dq(nq * elt(in_type)), dk(nk * elt(in_type)), dv(nk * elt(in_type)), dout(nq * 4);
            upload_as(dq, std::vector<float>(p.q.begin() + (size_t)a * Hq * d, p.q.begin() + (size_t)a * Hq * d + nq),
                      in_type);
            upload_as(dk, std::vector<float>(p.k.begin() + (size_t)a * Hkv * d,
                                             p.k.begin() + (size_t)a * Hkv * d + nk), in_type);
            upload_as(dv, std::vector<float>(p.v.begin() + (size_t)a * Hkv * d,
                                             p.v.begin() + (size_t)a * Hkv * d + nk), in_type);
            const vva_tensor tq = view4(dq.p, in_type, d, Hq, T, 1), tk = view4(dk.p, in_type, d, Hkv, T, 1),
                             tv = view4(dv.p, in_type, d, Hkv, T, 1), tp = view4(dpos.p, VVA_TYPE_I32, T, 1, 1, 1),
                             to = view4(dout.p, VVA_TYPE_F32, d, Hq, T, 1);
            if (!status_ok("qwen2_attention_resident",
                           vva::qwen2_attention_resident(kvs, (int)l, tq, tk, tv, tp, nullptr, hp, to), kvs)) {
                r.ok = false;
                return r;
            }
            const std::vector<float> o = download_f32(dout.p, nq, VVA_TYPE_F32);
            const std::vector<float> q = download_f32(dq.p, nq, in_type);
            std::copy(o.begin(), o.end(), r.out[l].begin() + (size_t)a * Hq * d);
            std::copy(q.begin(), q.end(), r.qr[l].begin() + (size_t)a * Hq * d);
        }
        kvs.past_len[0] += T;          // after the stack, as the callers do
    }
    return r;
}

constexpr double kMaxTol = 2e-3, kMeanTol = 1e-3;   // fp16 / bf16 paths
constexpr double kChunkTol = 1e-3;                   // chunked FA, tests/test_qwen2_resident.cpp:478-479

// ------------------------------------------------------------ paths

int test_chunks(vva_context* ctx) {
    const int d = 128, Hq = 28, Hkv = 4, N = 700;
    const std::vector<Proj> layer = {make_proj(11, N, Hq, Hkv, d, VVA_TYPE_BF16)};
    const std::vector<std::vector<int>> plans = {{0, N}, {0, N / 2, N}, {0, N / 4, N / 2, 3 * N / 4, N}};
    std::vector<Replay> runs;
    std::vector<std::vector<uint8_t>> kc, vc;
    for (const auto& b : plans) {
        vva::ResidentKV kvs;
        if (!kvs.init(ctx, 1, d, Hkv, N, 1, VVA_TYPE_F16)) return 10;
        runs.push_back(replay(kvs, layer, b, Hq, Hkv, d, VVA_TYPE_BF16));
        if (!runs.back().ok) return 11;
        if (kvs.past_len[0] != N) return 12;
        kc.push_back(cache_bytes(kvs.k(0), N));
        vc.push_back(cache_bytes(kvs.v(0), N));
        if (runs.size() == 1) {
            const std::vector<float> ref = oracle_out(runs[0].qr[0], kvs, 0, {0}, {N}, N, Hq, Hkv, d, VVA_TYPE_F16);
            if (!within("one shot vs oracle", compare(runs[0].out[0], ref), kMaxTol, kMeanTol)) return 13;
        }
    }
    for (size_t i = 1; i < runs.size(); ++i) {
        if (kc[i] != kc[0] || vc[i] != vc[0]) {
            printf("  chunk plan %zu: cache bytes differ from the one shot\n", i);
            return 14;
        }
        const std::string what = "chunk plan " + std::to_string(plans[i].size() - 1) + " vs one shot";
        if (!within(what.c_str(), compare(runs[i].out[0], runs[0].out[0]), kChunkTol, kChunkTol)) return 15;
    }
    // cache rows against RoPE + conversion on the host
    std::vector<float> kr(layer[0].k.size());
    std::vector<int32_t> pos(N);
    for (int t = 0; t < N; ++t) pos[t] = t;
    vvo_rope_neox(layer[0].k.data(), kr.data(), pos.data(), 0, d, Hkv, N, 1, 1.0e6f, VVO_THETA_RECURRENCE);
    std::vector<uint16_t> kh(kr.size()), vh(kr.size());
    vvo_from_f32(kr.data(), kh.data(), VVO_F16, (int64_t)kr.size());
    vvo_from_f32(layer[0].v.data(), vh.data(), VVO_F16, (int64_t)kr.size());
    const uint16_t* kg = (const uint16_t*)kc[0].data();
    if (memcmp(vh.data(), vc[0].data(), vc[0].size()) != 0) {
        printf("  V rows differ from the converted projections\n");
        return 16;
    }
    int worst = 0;
    for (size_t i = 0; i < kh.size(); ++i) {
        const int diff = abs((int)kh[i] - (int)kg[i]);
        worst = diff > worst ? diff : worst;
    }
    printf("  K rows vs host RoPE: worst %d f16 ulp (tol 1)\n", worst);
    return worst <= 1 ? 0 : 17;
}

int test_stack(vva_context* ctx) {
    const int d = 64, Hq = 14, Hkv = 2, N = 520, depth = 3;
    std::vector<Proj> layers;
    for (int l = 0; l < depth; ++l) layers.push_back(make_proj(100 + l, N, Hq, Hkv, d, VVA_TYPE_F32));
    vva::ResidentKV chained;
    if (!chained.init(ctx, depth, d, Hkv, N, 1, VVA_TYPE_F16)) return 20;
    const Replay c = replay(chained, layers, {0, 200, N}, Hq, Hkv, d, VVA_TYPE_F32);
    if (!c.ok) return 21;
    for (int l = 0; l < depth; ++l) {
        vva::ResidentKV one;
        if (!one.init(ctx, 1, d, Hkv, N, 1, VVA_TYPE_F16)) return 22;
        const Replay s = replay(one, {layers[l]}, {0, N}, Hq, Hkv, d, VVA_TYPE_F32);
        if (!s.ok) return 23;
        if (cache_bytes(one.k(0), N) != cache_bytes(chained.k(l), N) ||
            cache_bytes(one.v(0), N) != cache_bytes(chained.v(l), N)) {
            printf("  layer %d: cache bytes differ between the stack and the one shot\n", l);
            return 24;
        }
        const std::string what = "layer " + std::to_string(l) + ": stack of 2 chunks vs one shot";
        if (!within(what.c_str(), compare(c.out[l], s.out[0]), kChunkTol, kChunkTol)) return 25;
    }
    return 0;
}

// Decode steps of B = 2 sequences after voice prompts of lengths `prompt`.
// fused: every step also runs through the q work buffer (one
// vva_decode_step per layer) on a twin cache holding the same rows, checked
// against the two-call path and the oracle.
int decode_steps(vva_context* ctx, int d, int Hq, int Hkv, int type, const int prompt[2], int steps,
                 uint64_t seed, int code, bool fused = false) {
    const int layers = 2;
    vva::ResidentKV kvs, kvf;
    if (!kvs.init(ctx, layers, d, Hkv, prompt[0] + prompt[1] + steps, 2, type)) return code;
    if (fused && !kvf.init(ctx, layers, d, Hkv, prompt[0] + prompt[1] + steps, 2, type)) return code;
    Rng r(seed);
    for (int l = 0; l < layers; ++l)
        for (int s = 0; s < 2; ++s) {
            const std::vector<float> k = r.normal((size_t)prompt[s] * Hkv * d), v = r.normal(k.size());
            if (!status_ok("upload", kvs.upload(l, s, prompt[s], k.data(), v.data()), kvs)) return code + 1;
            if (fused && !status_ok("upload", kvf.upload(l, s, prompt[s], k.data(), v.data()), kvf)) return code + 1;
        }
    kvs.past_len = {prompt[0], prompt[1]};
    kvf.past_len = kvs.past_len;
    const vva::Qwen2Hparams hp = {Hq * d, Hq, Hkv, d, 1.0e6f, true};
    const int32_t seq_ids[2] = {0, 1};
    const size_t nq = (size_t)2 * Hq * d;
    Dev dq(nq * 4), dk((size_t)2 * Hkv * d * 4), dv((size_t)2 * Hkv * d * 4), dout(nq * 4), dpos(8), dqf(nq * 4),
        dqw(nq * 4), doutf(nq * 4);
    double worst = 0.0, worst_pair = 0.0;
    for (int step = 0; step < steps; ++step) {
        const int32_t pos[2] = {kvs.past_len[0], kvs.past_len[1]};
        (void)hipMemcpy(dpos.p, pos, 8, hipMemcpyHostToDevice);
        for (int l = 0; l < layers; ++l) {
            const std::vector<float> q0 = r.normal(nq);
            upload_as(dq, q0, VVA_TYPE_F32);
            upload_as(dk, r.normal((size_t)2 * Hkv * d), VVA_TYPE_F32);
            upload_as(dv, r.normal((size_t)2 * Hkv * d), VVA_TYPE_F32);
            vva_tensor tp = view4(dpos.p, VVA_TYPE_I32, 1, 2, 1, 1);     // pos ne=[T=1, B=2]
            const vva_tensor tq = view4(dq.p, VVA_TYPE_F32, d, Hq, 1, 2), tk = view4(dk.p, VVA_TYPE_F32, d, Hkv, 1, 2),
                             tv = view4(dv.p, VVA_TYPE_F32, d, Hkv, 1, 2),
                             to = view4(dout.p, VVA_TYPE_F32, d, Hq, 1, 2);
            if (fused) {
                upload_as(dqf, q0, VVA_TYPE_F32);
                const vva_tensor tqf = view4(dqf.p, VVA_TYPE_F32, d, Hq, 1, 2),
                                 tqw = view4(dqw.p, VVA_TYPE_F32, d, Hq, 1, 2),
                                 tof = view4(doutf.p, VVA_TYPE_F32, d, Hq, 1, 2);
                if (!status_ok("fused decode step",
                               vva::qwen2_attention_resident(kvf, l, tqf, tk, tv, tp, nullptr, hp, tof, seq_ids, &tqw),
                               kvf))
                    return code + 4;
            }
            if (!status_ok("decode step", vva::qwen2_attention_resident(kvs, l, tq, tk, tv, tp, nullptr, hp, to, seq_ids),
                           kvs))
                return code + 2;
            const std::vector<float> got = download_f32(dout.p, nq, VVA_TYPE_F32);
            const std::vector<float> q = download_f32(dq.p, nq, VVA_TYPE_F32);
            if (fused) {
                const std::vector<float> gotf = download_f32(doutf.p, nq, VVA_TYPE_F32);
                const std::vector<float> qw = download_f32(dqw.p, nq, VVA_TYPE_F32);
                const std::vector<float> qf = download_f32(dqf.p, nq, VVA_TYPE_F32);
                if (qw != q || qf != q0) {
                    printf("  step %d layer %d: the work buffer's q differs from the in-place rotation, or q changed\n",
                           step, l);
                    return code + 5;
                }
                for (int s = 0; s < 2; ++s) {
                    const int rows = kvs.past_len[s] + 1;
                    if (cache_bytes(kvs.k(l, s), rows) != cache_bytes(kvf.k(l, s), rows) ||
                        cache_bytes(kvs.v(l, s), rows) != cache_bytes(kvf.v(l, s), rows)) {
                        printf("  step %d layer %d seq %d: cache rows differ between the paths\n", step, l, s);
                        return code + 6;
                    }
                }
                const Stats p = compare(gotf, got);
                worst_pair = p.max_abs > worst_pair ? p.max_abs : worst_pair;
                if (type == VVA_TYPE_Q8_0 ? gotf != got : !(p.finite && p.max_abs <= kMaxTol && p.mean_abs <= kMeanTol)) {
                    within("fused step vs the two calls", p, 0.0, 0.0);
                    return code + 7;
                }
                const std::vector<float> reff =
                    oracle_out(qw, kvf, l, {0, 1}, {kvf.past_len[0] + 1, kvf.past_len[1] + 1}, 1, Hq, Hkv, d, type);
                const Stats sf = compare(gotf, reff);
                if (!sf.finite || sf.max_abs > kMaxTol || sf.mean_abs > kMeanTol) {
                    within("fused step vs oracle", sf, kMaxTol, kMeanTol);
                    return code + 8;
                }
            }
            const std::vector<float> ref =
                oracle_out(q, kvs, l, {0, 1}, {kvs.past_len[0] + 1, kvs.past_len[1] + 1}, 1, Hq, Hkv, d, type);
            const Stats s = compare(got, ref);
            worst = s.max_abs > worst ? s.max_abs : worst;
            if (!s.finite || s.max_abs > kMaxTol || s.mean_abs > kMeanTol) {
                within("decode step vs oracle", s, kMaxTol, kMeanTol);
                printf("  step %d layer %d, lengths %d / %d\n", step, l, kvs.past_len[0] + 1, kvs.past_len[1] + 1);
                return code + 3;
            }
        }
        kvs.past_len[0] += 1;
        kvs.past_len[1] += 1;
        kvf.past_len = kvs.past_len;
    }
    printf("  %d steps x %d layers, lengths %d / %d -> %d / %d: worst max-abs %.3e (tol %.0e)\n", steps, layers,
           prompt[0], prompt[1], kvs.past_len[0], kvs.past_len[1], worst, kMaxTol);
    if (fused)
        printf("  fused step (q work buffer) vs the two calls: q and cache rows bit-identical, output worst %.3e%s\n",
               worst_pair, type == VVA_TYPE_Q8_0 ? " (bit-identical)" : "");
    return 0;
}

int test_cfg(vva_context* ctx) {
    const int prompt[2] = {1024, 957};
    return decode_steps(ctx, 64, 14, 2, VVA_TYPE_F16, prompt, 6, 31, 30);
}

int test_q8(vva_context* ctx) {
    const int prompt[2] = {3000, 2311};
    return decode_steps(ctx, 128, 28, 4, VVA_TYPE_Q8_0, prompt, 3, 41, 40);
}

int test_step(vva_context* ctx) {
    const int p05[2] = {1024, 957}, p7[2] = {3000, 2311};
    const int rc = decode_steps(ctx, 64, 14, 2, VVA_TYPE_F16, p05, 4, 131, 90, true);
    return rc ? rc : decode_steps(ctx, 128, 28, 4, VVA_TYPE_Q8_0, p7, 3, 141, 100, true);
}

// A 28-layer 7B CFG decode step (B = 2) on a Q8_0 cache, timed four ways.
// The cache holds zeros (the time does not depend on the values); pos and
// the lengths stay fixed, so every step appends at the same row.
int test_timing(vva_context* ctx) {
    const int d = 128, Hq = 28, Hkv = 4, layers = 28, B = 2, steps = 20;
    const vva::Qwen2Hparams hp = {Hq * d, Hq, Hkv, d, 1.0e6f, true};
    const int32_t seq_ids[2] = {0, 1};
    for (const int past : {32768, 2048}) {
        vva::ResidentKV kvs;
        if (!kvs.init(ctx, layers, d, Hkv, past + 1, B, VVA_TYPE_Q8_0)) return 110;
        kvs.past_len = {past, past};
        const size_t nq = (size_t)B * Hq * d, nk = (size_t)B * Hkv * d;
        Dev dq(nq * 4), dqw(nq * 4), dk(nk * 4), dv(nk * 4), dout(nq * 4), dpos(8);
        Rng r(7);
        upload_as(dq, r.normal(nq), VVA_TYPE_F32);
        upload_as(dk, r.normal(nk), VVA_TYPE_F32);
        upload_as(dv, r.normal(nk), VVA_TYPE_F32);
        const int32_t pos[2] = {past, past};
        (void)hipMemcpy(dpos.p, pos, 8, hipMemcpyHostToDevice);
        const vva_tensor tq = view4(dq.p, VVA_TYPE_F32, d, Hq, 1, B), tqw = view4(dqw.p, VVA_TYPE_F32, d, Hq, 1, B),
                         tk = view4(dk.p, VVA_TYPE_F32, d, Hkv, 1, B), tv = view4(dv.p, VVA_TYPE_F32, d, Hkv, 1, B),
                         to = view4(dout.p, VVA_TYPE_F32, d, Hq, 1, B), tp = view4(dpos.p, VVA_TYPE_I32, 1, B, 1, 1);
        double us[2][2];
        for (int fused = 0; fused < 2; ++fused)
            for (int per_layer = 0; per_layer < 2; ++per_layer) {
                auto step = [&]() {
                    for (int l = 0; l < layers; ++l) {
                        const int st = vva::qwen2_attention_resident(kvs, l, tq, tk, tv, tp, nullptr, hp, to, seq_ids,
                                                                     fused ? &tqw : nullptr);
                        if (st != VVA_OK) return st;
                        if (per_layer && hipStreamSynchronize(nullptr) != hipSuccess) return (int)VVA_ERR_DEVICE;
                    }
                    return hipStreamSynchronize(nullptr) == hipSuccess ? (int)VVA_OK : (int)VVA_ERR_DEVICE;
                };
                for (int w = 0; w < 3; ++w)
                    if (!status_ok("timing warm-up", step(), kvs)) return 111;
                const auto t0 = std::chrono::steady_clock::now();
                for (int i = 0; i < steps; ++i)
                    if (!status_ok("timing", step(), kvs)) return 112;
                const auto t1 = std::chrono::steady_clock::now();
                us[fused][per_layer] = std::chrono::duration<double, std::micro>(t1 - t0).count() / steps;
            }
        printf("  %d keys x 2 sequences, 28 layers, us per step:\n", past);
        printf("    two calls,  sync per layer %8.1f   sync per step %8.1f\n", us[0][1], us[0][0]);
        printf("    fused step, sync per layer %8.1f   sync per step %8.1f\n", us[1][1], us[1][0]);
    }
    return 0;
}

// ------------------------------------------------------------ the attention block

int64_t weight_row_bytes(int64_t K, int type) { return type == VVA_TYPE_F16 ? K * 2 : K / 32 * 34; }

// M rows of K weights, N(0,1) / sqrt(K), stored as `type` (ggml layout)
std::vector<uint8_t> make_weight(Rng& r, int64_t M, int64_t K, int type) {
    std::vector<float> w = r.normal((size_t)(M * K));
    const float s = 1.0f / sqrtf((float)K);
    for (float& x : w) x *= s;
    std::vector<uint8_t> raw((size_t)(M * weight_row_bytes(K, type)));
    if (type == VVA_TYPE_F16) vvo_from_f32(w.data(), raw.data(), type, M * K);
    else vvo_quantize_q8_0(w.data(), raw.data(), M * K);
    return raw;
}

vva_tensor weight_view(void* p, int type, int64_t K, int64_t M) {
    vva_tensor t = {};
    t.data = p;
    t.type = type;
    const int64_t rb = weight_row_bytes(K, type);
    t.ne[0] = K; t.ne[1] = M; t.ne[2] = 1; t.ne[3] = 1;
    t.nb[0] = type == VVA_TYPE_F16 ? 2 : 34;
    t.nb[1] = rb; t.nb[2] = rb * M; t.nb[3] = rb * M;
    return t;
}

// |got - ref| <= tol + (rounding of ref to `type`), and the mean excess <= mean_tol
bool within_rounded(const char* what, const std::vector<float>& got, const std::vector<float>& ref, int type,
                    double tol, double mean_tol) {
    const double ulp = type == VVA_TYPE_F16 ? 1.0 / 2048.0 : 0.0;
    double worst = 0.0, max_err = 0.0, sum = 0.0;
    bool finite = true;
    for (size_t i = 0; i < got.size(); ++i) {
        if (!std::isfinite(got[i])) finite = false;
        const double e = fabs((double)got[i] - (double)ref[i]), r = fabs((double)ref[i]) * ulp;
        max_err = e > max_err ? e : max_err;
        worst = e - r - tol > worst ? e - r - tol : worst;
        sum += e - r > 0.0 ? e - r : 0.0;
    }
    const double mean = sum / (double)got.size();
    const bool ok = finite && worst <= 0.0 && mean <= mean_tol;
    printf("  %-44s max %.3e (tol %.0e + rounding)  mean %.3e  %s\n", what, max_err, tol, mean, ok ? "ok" : "FAIL");
    return ok;
}

int block_case(vva_context* ctx, int wt) {
    const int hidden = 896, Hq = 14, Hkv = 2, d = 64, qd = Hq * d, kd = Hkv * d;
    Rng r(900 + (uint64_t)wt);
    const std::vector<uint8_t> wq = make_weight(r, qd, hidden, wt), wk = make_weight(r, kd, hidden, wt),
                               wv = make_weight(r, kd, hidden, wt), wo = make_weight(r, hidden, qd, wt);
    std::vector<float> bq = r.normal(qd), bk = r.normal(kd), bv = r.normal(kd);
    Dev dwq(wq.size()), dwk(wk.size()), dwv(wv.size()), dwo(wo.size()), dbq(4 * (size_t)qd), dbk(4 * (size_t)kd),
        dbv(4 * (size_t)kd);
    (void)hipMemcpy(dwq.p, wq.data(), wq.size(), hipMemcpyHostToDevice);
    (void)hipMemcpy(dwk.p, wk.data(), wk.size(), hipMemcpyHostToDevice);
    (void)hipMemcpy(dwv.p, wv.data(), wv.size(), hipMemcpyHostToDevice);
    (void)hipMemcpy(dwo.p, wo.data(), wo.size(), hipMemcpyHostToDevice);
    (void)hipMemcpy(dbq.p, bq.data(), 4 * (size_t)qd, hipMemcpyHostToDevice);
    (void)hipMemcpy(dbk.p, bk.data(), 4 * (size_t)kd, hipMemcpyHostToDevice);
    (void)hipMemcpy(dbv.p, bv.data(), 4 * (size_t)kd, hipMemcpyHostToDevice);
    vva::Qwen2AttnWeights W;
    W.q = weight_view(dwq.p, wt, hidden, qd);
    W.k = weight_view(dwk.p, wt, hidden, kd);
    W.v = weight_view(dwv.p, wt, hidden, kd);
    W.o = weight_view(dwo.p, wt, qd, hidden);
    W.q_bias = view4(dbq.p, VVA_TYPE_F32, qd, 1, 1, 1);
    W.k_bias = view4(dbk.p, VVA_TYPE_F32, kd, 1, 1, 1);
    W.v_bias = view4(dbv.p, VVA_TYPE_F32, kd, 1, 1, 1);
    const int64_t rbq = weight_row_bytes(hidden, wt), rbo = weight_row_bytes(qd, wt);

    vva::ResidentKV kvs;
    if (!kvs.init(ctx, 1, d, Hkv, 256, 2, VVA_TYPE_F16)) return 80;
    const int pasts[2] = {40, 23};
    for (int s = 0; s < 2; ++s) {
        const std::vector<float> k = r.normal((size_t)pasts[s] * kd), v = r.normal((size_t)pasts[s] * kd);
        if (!status_ok("upload", kvs.upload(0, s, pasts[s], k.data(), v.data()), kvs)) return 81;
        kvs.past_len[s] = pasts[s];
    }
    const vva::Qwen2Hparams hp = {hidden, Hq, Hkv, d, 1.0e6f, true};
    struct Step {
        int T;
        std::vector<int32_t> seqs;
    };
    const Step steps[2] = {{96, {0}}, {1, {0, 1}}};
    for (const Step& st : steps) {
        const int T = st.T, B = (int)st.seqs.size(), N = B * T;
        const std::vector<float> x = r.normal((size_t)N * hidden), xn = r.normal((size_t)N * hidden);
        std::vector<int32_t> pos((size_t)N);
        std::vector<int> L(B);
        for (int b = 0; b < B; ++b) {
            L[b] = kvs.past_len[st.seqs[b]] + T;
            for (int t = 0; t < T; ++t) pos[(size_t)b * T + t] = kvs.past_len[st.seqs[b]] + t;
        }
        Dev dx(4 * (size_t)N * hidden), dxn(4 * (size_t)N * hidden), dh(4 * (size_t)N * hidden),
            dq(4 * (size_t)N * qd), dout(4 * (size_t)N * qd), dpos(4 * (size_t)N);
        (void)hipMemcpy(dx.p, x.data(), 4 * x.size(), hipMemcpyHostToDevice);
        (void)hipMemcpy(dxn.p, xn.data(), 4 * xn.size(), hipMemcpyHostToDevice);
        (void)hipMemcpy(dpos.p, pos.data(), 4 * pos.size(), hipMemcpyHostToDevice);
        const vva_tensor tx = view4(dx.p, VVA_TYPE_F32, hidden, T, B, 1), txn = view4(dxn.p, VVA_TYPE_F32, hidden, T, B, 1),
                         th = view4(dh.p, VVA_TYPE_F32, hidden, T, B, 1), tq = view4(dq.p, VVA_TYPE_F32, d, Hq, T, B),
                         to = view4(dout.p, VVA_TYPE_F32, d, Hq, T, B), tp = view4(dpos.p, VVA_TYPE_I32, T, B, 1, 1);
        const int32_t* ids = B > 1 ? st.seqs.data() : nullptr;
        if (!status_ok("qwen2_attention_block_resident",
                       vva::qwen2_attention_block_resident(kvs, 0, txn, tx, W, tp, nullptr, hp, tq, to, th, ids), kvs))
            return 82;
        (void)hipDeviceSynchronize();
        printf("  %s weights, T = %d, B = %d\n", wt == VVA_TYPE_F16 ? "F16" : "Q8_0", T, B);
        // q = RoPE(linear(xn, Wq) + bq)
        std::vector<float> ql((size_t)N * qd), kl((size_t)N * kd), vl((size_t)N * kd);
        vvo_linear(wq.data(), wt, rbq, bq.data(), xn.data(), ql.data(), N, hidden, qd, VVO_GGML, 0);
        vvo_linear(wk.data(), wt, rbq, bk.data(), xn.data(), kl.data(), N, hidden, kd, VVO_GGML, 0);
        vvo_linear(wv.data(), wt, rbq, bv.data(), xn.data(), vl.data(), N, hidden, kd, VVO_GGML, 0);
        vvo_rope_neox(ql.data(), ql.data(), pos.data(), T, d, Hq, T, B, 1.0e6f, VVO_THETA_RECURRENCE);
        vvo_rope_neox(kl.data(), kl.data(), pos.data(), T, d, Hkv, T, B, 1.0e6f, VVO_THETA_RECURRENCE);
        const std::vector<float> qdev = download_f32(dq.p, (size_t)N * qd, VVA_TYPE_F32);
        if (!within("rotated q vs oracle", compare(qdev, ql), kMaxTol, kMeanTol)) return 83;
        // the appended rows [past, past + T) of each sequence, F16
        for (int b = 0; b < B; ++b) {
            const int s = st.seqs[b], p0 = L[b] - T;
            const std::vector<uint8_t> kb = cache_bytes(kvs.k(0, s), L[b]), vb = cache_bytes(kvs.v(0, s), L[b]);
            std::vector<float> kg((size_t)T * kd), vg((size_t)T * kd);
            vvo_to_f32(kb.data() + (size_t)p0 * kd * 2, VVA_TYPE_F16, kg.data(), (int64_t)T * kd);
            vvo_to_f32(vb.data() + (size_t)p0 * kd * 2, VVA_TYPE_F16, vg.data(), (int64_t)T * kd);
            const std::vector<float> kr(kl.begin() + (size_t)b * T * kd, kl.begin() + (size_t)(b + 1) * T * kd),
                vr(vl.begin() + (size_t)b * T * kd, vl.begin() + (size_t)(b + 1) * T * kd);
            if (!within_rounded("appended K rows vs oracle", kg, kr, VVA_TYPE_F16, kMaxTol, kMeanTol)) return 84;
            if (!within_rounded("appended V rows vs oracle", vg, vr, VVA_TYPE_F16, kMaxTol, kMeanTol)) return 85;
        }
        // o over the window, on the device's own q and cache rows
        const std::vector<float> odev = download_f32(dout.p, (size_t)N * qd, VVA_TYPE_F32);
        const std::vector<float> oref = oracle_out(qdev, kvs, 0, std::vector<int>(st.seqs.begin(), st.seqs.end()), L,
                                                   T, Hq, Hkv, d, VVA_TYPE_F16);
        if (!within("attention output vs oracle", compare(odev, oref), kMaxTol, kMeanTol)) return 86;
        // h = x + o Wo^T, on the device's own o
        std::vector<float> href((size_t)N * hidden);
        vvo_linear(wo.data(), wt, rbo, nullptr, odev.data(), href.data(), N, qd, hidden, VVO_GGML, 0);
        for (size_t i = 0; i < href.size(); ++i) href[i] += x[i];
        const std::vector<float> hdev = download_f32(dh.p, (size_t)N * hidden, VVA_TYPE_F32);
        if (!within("h = x + attn_o(o) vs oracle", compare(hdev, href), kMaxTol, kMeanTol)) return 87;
        for (int b = 0; b < B; ++b) kvs.past_len[st.seqs[b]] += T;
    }
    return 0;
}

// A decode step into a Q8_0 cache through the attention block: given a y
// work tensor the block runs vva_qkv_proj + vva_decode_step, without it
// vva_qkv_rope_append + vva_attn.  Twin caches with the same history take
// three consecutive steps (B = 2) each way; h, the rotated q, the attention
// output and every cache row must agree bit for bit.
int block_step_case(vva_context* ctx, int wt) {
    const int hidden = 896, Hq = 14, Hkv = 2, d = 64, qd = Hq * d, kd = Hkv * d, M = qd + 2 * kd, B = 2;
    Rng r(950 + (uint64_t)wt);
    const std::vector<uint8_t> wq = make_weight(r, qd, hidden, wt), wk = make_weight(r, kd, hidden, wt),
                               wv = make_weight(r, kd, hidden, wt), wo = make_weight(r, hidden, qd, wt);
    std::vector<float> bq = r.normal(qd), bk = r.normal(kd), bv = r.normal(kd);
    Dev dwq(wq.size()), dwk(wk.size()), dwv(wv.size()), dwo(wo.size()), dbq(4 * (size_t)qd), dbk(4 * (size_t)kd),
        dbv(4 * (size_t)kd);
    (void)hipMemcpy(dwq.p, wq.data(), wq.size(), hipMemcpyHostToDevice);
    (void)hipMemcpy(dwk.p, wk.data(), wk.size(), hipMemcpyHostToDevice);
    (void)hipMemcpy(dwv.p, wv.data(), wv.size(), hipMemcpyHostToDevice);
    (void)hipMemcpy(dwo.p, wo.data(), wo.size(), hipMemcpyHostToDevice);
    (void)hipMemcpy(dbq.p, bq.data(), 4 * (size_t)qd, hipMemcpyHostToDevice);
    (void)hipMemcpy(dbk.p, bk.data(), 4 * (size_t)kd, hipMemcpyHostToDevice);
    (void)hipMemcpy(dbv.p, bv.data(), 4 * (size_t)kd, hipMemcpyHostToDevice);
    vva::Qwen2AttnWeights W;
    W.q = weight_view(dwq.p, wt, hidden, qd);
    W.k = weight_view(dwk.p, wt, hidden, kd);
    W.v = weight_view(dwv.p, wt, hidden, kd);
    W.o = weight_view(dwo.p, wt, qd, hidden);
    W.q_bias = view4(dbq.p, VVA_TYPE_F32, qd, 1, 1, 1);
    W.k_bias = view4(dbk.p, VVA_TYPE_F32, kd, 1, 1, 1);
    W.v_bias = view4(dbv.p, VVA_TYPE_F32, kd, 1, 1, 1);
    vva::ResidentKV ka, kb;                                   // with / without y_ws
    if (!ka.init(ctx, 1, d, Hkv, 256, B, VVA_TYPE_Q8_0) || !kb.init(ctx, 1, d, Hkv, 256, B, VVA_TYPE_Q8_0)) return 90;
    const int pasts[2] = {70, 33};
    for (int s = 0; s < B; ++s) {
        const std::vector<float> k = r.normal((size_t)pasts[s] * kd), v = r.normal((size_t)pasts[s] * kd);
        if (!status_ok("upload", ka.upload(0, s, pasts[s], k.data(), v.data()), ka)) return 91;
        if (!status_ok("upload", kb.upload(0, s, pasts[s], k.data(), v.data()), kb)) return 91;
        ka.past_len[s] = kb.past_len[s] = pasts[s];
    }
    const vva::Qwen2Hparams hp = {hidden, Hq, Hkv, d, 1.0e6f, true};
    for (int step = 0; step < 3; ++step) {
        const std::vector<float> x = r.normal((size_t)B * hidden), xn = r.normal((size_t)B * hidden);
        const std::vector<int32_t> pos = {ka.past_len[0], ka.past_len[1]};
        Dev dx(4 * (size_t)B * hidden), dxn(4 * (size_t)B * hidden), dpos(4 * (size_t)B), dy(4 * (size_t)B * M);
        Dev dh[2] = {Dev(4 * (size_t)B * hidden), Dev(4 * (size_t)B * hidden)};
        Dev dq[2] = {Dev(4 * (size_t)B * qd), Dev(4 * (size_t)B * qd)};
        Dev dout[2] = {Dev(4 * (size_t)B * qd), Dev(4 * (size_t)B * qd)};
        (void)hipMemcpy(dx.p, x.data(), 4 * x.size(), hipMemcpyHostToDevice);
        (void)hipMemcpy(dxn.p, xn.data(), 4 * xn.size(), hipMemcpyHostToDevice);
        (void)hipMemcpy(dpos.p, pos.data(), 4 * pos.size(), hipMemcpyHostToDevice);
        const vva_tensor tx = view4(dx.p, VVA_TYPE_F32, hidden, 1, B, 1), txn = view4(dxn.p, VVA_TYPE_F32, hidden, 1, B, 1),
                         tp = view4(dpos.p, VVA_TYPE_I32, 1, B, 1, 1), ty = view4(dy.p, VVA_TYPE_F32, M, 1, B, 1);
        for (int way = 0; way < 2; ++way) {
            vva::ResidentKV& kv = way == 0 ? ka : kb;
            const vva_tensor th = view4(dh[way].p, VVA_TYPE_F32, hidden, 1, B, 1),
                             tq = view4(dq[way].p, VVA_TYPE_F32, d, Hq, 1, B),
                             to = view4(dout[way].p, VVA_TYPE_F32, d, Hq, 1, B);
            if (!status_ok("qwen2_attention_block_resident",
                           vva::qwen2_attention_block_resident(kv, 0, txn, tx, W, tp, nullptr, hp, tq, to, th, nullptr,
                                                               way == 0 ? &ty : nullptr),
                           kv))
                return 92;
        }
        (void)hipDeviceSynchronize();
        auto same = [](const Dev& a, const Dev& b, size_t n) {
            std::vector<uint8_t> ha(n), hb(n);
            (void)hipMemcpy(ha.data(), a.p, n, hipMemcpyDeviceToHost);
            (void)hipMemcpy(hb.data(), b.p, n, hipMemcpyDeviceToHost);
            return ha == hb;
        };
        if (!same(dq[0], dq[1], 4 * (size_t)B * qd)) return 93;
        if (!same(dout[0], dout[1], 4 * (size_t)B * qd)) return 94;
        if (!same(dh[0], dh[1], 4 * (size_t)B * hidden)) return 95;
        for (int s = 0; s < B; ++s) {
            const int L = ka.past_len[s] + 1;
            if (cache_bytes(ka.k(0, s), L) != cache_bytes(kb.k(0, s), L)) return 96;
            if (cache_bytes(ka.v(0, s), L) != cache_bytes(kb.v(0, s), L)) return 97;
        }
        for (int s = 0; s < B; ++s) ka.past_len[s] = ++kb.past_len[s];
    }
    printf("  %s weights, Q8_0 cache, 3 steps B = 2: vva_qkv_proj + vva_decode_step equal vva_qkv_rope_append + "
           "vva_attn bit for bit (q, o, h, cache rows)\n", wt == VVA_TYPE_F16 ? "F16" : "Q8_0");
    return 0;
}

int test_block(vva_context* ctx) {
    for (const int wt : {VVA_TYPE_F16, VVA_TYPE_Q8_0}) {
        int rc = block_case(ctx, wt);
        if (rc) return rc;
        if ((rc = block_step_case(ctx, wt))) return rc;
    }
    return 0;
}

int test_errors(vva_context* ctx) {
    const int d = 64, Hq = 14, Hkv = 2, T = 8;
    vva::ResidentKV kvs;
    if (!kvs.init(ctx, 2, d, Hkv, 16, 1, VVA_TYPE_F16)) return 50;
    const vva::Qwen2Hparams hp = {Hq * d, Hq, Hkv, d, 1.0e6f, true};
    Dev dq((size_t)T * Hq * d * 4), dk((size_t)T * Hkv * d * 4), dv((size_t)T * Hkv * d * 4), dout((size_t)T * Hq * d * 4),
        dpos(4 * T);
    const vva_tensor tq = view4(dq.p, VVA_TYPE_F32, d, Hq, T, 1), tk = view4(dk.p, VVA_TYPE_F32, d, Hkv, T, 1),
                     tv = view4(dv.p, VVA_TYPE_F32, d, Hkv, T, 1), tp = view4(dpos.p, VVA_TYPE_I32, T, 1, 1, 1),
                     to = view4(dout.p, VVA_TYPE_F32, d, Hq, T, 1);
    kvs.past_len[0] = 12;                                    // 12 + 8 > 16
    if (vva::qwen2_attention_resident(kvs, 0, tq, tk, tv, tp, nullptr, hp, to) != VVA_ERR_INVALID_ARG) return 51;
    kvs.past_len[0] = 0;
    if (vva::qwen2_attention_resident(kvs, 2, tq, tk, tv, tp, nullptr, hp, to) != VVA_ERR_INVALID_ARG) return 52;
    const int32_t bad_seq[1] = {1};
    if (vva::qwen2_attention_resident(kvs, 0, tq, tk, tv, tp, nullptr, hp, to, bad_seq) != VVA_ERR_INVALID_ARG)
        return 53;
    vva::Qwen2Hparams wrong = hp;
    wrong.n_kv_heads = 7;
    if (vva::qwen2_attention_resident(kvs, 0, tq, tk, tv, tp, nullptr, wrong, to) != VVA_ERR_INVALID_ARG) return 54;
    printf("  over-long window, bad layer, bad sequence, wrong head count: VVA_ERR_INVALID_ARG\n");
    return 0;
}

int test_supports(vva_context* ctx) {
    // probe shape of backend_supports_flash_attn: hd 128, 8 q / 2 kv heads
    if (vva_supports(ctx, 128, 8, 2, VVA_TYPE_F32, VVA_TYPE_F16) != 1) return 60;
    if (vva_supports(ctx, 128, 28, 4, VVA_TYPE_BF16, VVA_TYPE_Q8_0) != 1) return 61;
    if (vva_supports(ctx, 128, 8, 3, VVA_TYPE_F32, VVA_TYPE_F16) != 0) return 62;   // 8 % 3 != 0
    if (vva_supports(ctx, 128, 8, 2, VVA_TYPE_F32, 2) != 0) return 63;             // Q4_0 cache
    printf("  probe shape supported; uneven groups and Q4_0 caches refused\n");
    return 0;
}

// Destruction order: a ResidentKV that outlives its context.  vva_destroy
// releases the cache; the ResidentKV's later free() (and its destructor)
// must be no-ops, and calls with the released handle must fail cleanly.
int test_order(vva_context*) {
    vva_context* own = nullptr;
    if (vva_create(0, nullptr, &own) != VVA_OK) return 70;
    vva::ResidentKV kvs;
    if (!kvs.init(own, 2, 64, 2, 32, 1, VVA_TYPE_F16)) return 71;
    vva_kv* released = kvs.kv;
    vva_destroy(own);
    int32_t len = -1;
    if (vva_kv_get_len(released, 0, &len) != VVA_ERR_INVALID_ARG) return 72;
    kvs.free();                                              // handle already released: ignored
    kvs.free();
    printf("  context destroyed first: released handle refused, ResidentKV::free a no-op\n");
    return 0;
}

struct Case {
    const char* name;
    std::function<int(vva_context*)> fn;
};

}  // namespace

int main(int argc, char** argv) {
    const std::vector<Case> cases = {{"chunks", test_chunks},     {"stack", test_stack},   {"cfg", test_cfg},
                                     {"q8", test_q8},             {"step", test_step},     {"timing", test_timing},
                                     {"block", test_block},       {"errors", test_errors}, {"supports", test_supports},
                                     {"order", test_order}};
    std::vector<std::string> want;
    for (int i = 1; i < argc; ++i) {
        if (!strcmp(argv[i], "--list")) {
            for (const Case& c : cases) printf("%s\n", c.name);
            return 0;
        }
        want.push_back(argv[i]);
    }
    vva_context* ctx = nullptr;
    if (vva_create(0, nullptr, &ctx) != VVA_OK) {
        fprintf(stderr, "vva_create: %s\n", vva_last_error(nullptr));
        return 2;
    }
    int rc = 0, ran = 0;
    for (const Case& c : cases) {
        bool run = want.empty();
        for (const std::string& w : want) run = run || w == c.name;
        if (!run) continue;
        printf("[%s]\n", c.name);
        fflush(stdout);
        rc = c.fn(ctx);
        ++ran;
        printf("[%s] %s\n", c.name, rc == 0 ? "PASS" : "FAIL");
        fflush(stdout);
        if (rc != 0) break;
    }
    vva_destroy(ctx);
    if (ran == 0) {
        fprintf(stderr, "no such case\n");
        return 3;
    }
    return rc;
}
