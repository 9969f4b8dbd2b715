// vva.cpp — host side of the C ABI declared in include/vva.h.
//
// Owns the context (device + one stream), the resident KV cache slab, input
// validation and kernel dispatch.  Error conventions follow vibevoice.cpp's
// public API (include/vibevoice.h:23-33): every call returns a status, the
// message is kept per context, nothing aborts.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <set>
#include <string>
#include <vector>

#include "vva_internal.hpp"

using namespace vva;

struct vva_context {
    int device = 0;
    hipStream_t stream = nullptr;        // borrowed stream; nullptr = the HIP null stream
    std::string err;
    int n_cu = 256;
    int attn_path = 0;
    int use_flash_attn = 1;              // F32 caches: 1 = F16 cast + MFMA prefill, 0 = fp32 throughout
    int last_splits = 0;
    int logged_splits = -1;              // the decode split count last logged
    // scheduling overrides (vva_set_schedule); 0 = automatic
    int sched_decode_wgs = 0, sched_decode_splits = 0, sched_prefill_splits = 0;
    float* ws = nullptr;                 // split partials (decode and key-split prefill)
    size_t ws_bytes = 0;
    // Workspaces outgrown by a later call.  A kernel already enqueued, or a
    // HIP graph captured earlier, may still hold their address, so they stay
    // allocated until vva_destroy.
    std::vector<float*> ws_retired;
    float* scratch = nullptr;            // this device's `scratch` (vva_attn_noalloc)
    // merge tickets, zeroed once: vva_decode_step's [kMaxStepTickets], then the
    // prefill's in-launch merge [kMaxPrefillTickets], then the projection
    // GEMM's split along K [kMaxProjTickets]
    unsigned* tickets = nullptr;
    // the f16 window of a Q8_0 prefill flags an out-of-range value here
    // with the call's epoch; the call's gated fp32 fallback then runs
    unsigned long long* ovf = nullptr;
    unsigned long long ovf_epoch = 0;
    std::set<vva_kv*> caches;            // released by vva_destroy if still alive
    // the last prefill plan and the call shape it was made for: a layer stack
    // repeats one shape layer after layer
    // (a fixed array: the key is built on every prefill call, vva_attn_noalloc's included)
    std::array<int64_t, 10 + 2 * VVA_MAX_BATCH> plan_key{};
    int plan_key_n = 0;
    PrefillPlan plan{1, 0, 0, 1};
};

struct vva_kv {
    vva_context* ctx = nullptr;
    vva_kv_desc desc{};
    char* base = nullptr;
    size_t tensor_bytes = 0;             // one K or V tensor of one (layer, seq)
    int64_t row_bytes = 0;               // one token row: [Hkv][d]
    int64_t head_bytes = 0;              // one head row: [d]
    std::vector<int32_t> len;
};

// Split-partial scratch of vva_attn_noalloc, one copy per GPU, held until
// the process ends.  The decode planners stay far below it (3.6 MiB at the
// 7B CFG shape on 256 CUs) and the prefill planner is given its size as a
// cap (it picks fewer key splits when the partials would not fit), so only
// split counts forced by vva_set_schedule can exceed it.  In host code
// `scratch` only names the symbol: its device address comes from
// hipGetSymbolAddress (g_scratch below).
constexpr size_t kScratchBytes = (size_t)36 << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

namespace {

thread_local std::string g_create_err;

// The vva_set_log_callback sink: process-wide, one delivery at a time (a
// recursive lock: a callback that calls a failing entry point logs again on
// the same thread rather than deadlocking).
struct LogSink {
    std::recursive_mutex mu;
    vva_log_cb cb = nullptr;
    void* user = nullptr;
    int max_lvl = -1;                        // nothing delivered until a callback is set
};
LogSink& log_sink() {
    static LogSink s;
    return s;
}

// Formats into a stack buffer (no allocation: vva_attn_noalloc logs too).
void log_msg(vva_log_level lvl, const char* fmt, ...) {
    LogSink& s = log_sink();
    std::lock_guard<std::recursive_mutex> lk(s.mu);
    if (!s.cb || (int)lvl > s.max_lvl) return;
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    s.cb(lvl, buf, s.user);
}

// Device address of `scratch` per device, resolved once per device by
// vva_create with that device current.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch[kMaxDevices] = {};

// Every live cache handle of every context.  vva_kv_free of a handle that is
// not here (already freed, or released by vva_destroy of its context) does
// nothing, so a caller that destroys the context first cannot double-free.
std::mutex g_kv_mu;
std::set<const vva_kv*> g_kv_live;

bool kv_live(const vva_kv* kv) {
    std::lock_guard<std::mutex> lk(g_kv_mu);
    return g_kv_live.count(kv) != 0;
}

struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) (void)hipSetDevice(dev);
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

vva_status fail(vva_context* ctx, vva_status st, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    if (ctx) ctx->err = buf;
    else g_create_err = buf;
    log_msg(VVA_LOG_ERROR, "%s", buf);
    return st;
}

vva_status hip_fail(vva_context* ctx, hipError_t e, const char* what) {
    return fail(ctx, e == hipErrorOutOfMemory ? VVA_ERR_OUT_OF_MEMORY : VVA_ERR_DEVICE,
                "%s: %s", what, hipGetErrorString(e));
}

bool float_type(int t) { return t == VVA_TYPE_F32 || t == VVA_TYPE_F16 || t == VVA_TYPE_BF16; }
bool cache_type(int t) { return float_type(t) || t == VVA_TYPE_Q8_0; }

// head_dim constraints shared by every kernel: multiple of 32 (Q8_0 blocks),
// even halves for NeoX pairs, at most 256 (LDS angle table).
bool head_dim_ok(int d, int type) {
    if (d <= 0 || d > 256 || d % 32) return false;
    if (type == VVA_TYPE_Q8_0 && d % 64) return false;   // two whole blocks per rotation pair group
    return true;
}

char* kv_tensor(const vva_kv* kv, int layer, int seq, int which) {
    const size_t idx = ((size_t)layer * kv->desc.n_seq + seq) * 2 + which;
    return kv->base + idx * kv->tensor_bytes;
}

// Bytes [data, data + span) a tensor's elements occupy (ne >= 1 everywhere).
// For Q8_0, ne[0] counts elements and nb[0] is the 34-byte block.
size_t tensor_span(const vva_tensor* t) {
    const bool q8 = t->type == VVA_TYPE_Q8_0;
    int64_t last = ((q8 ? t->ne[0] / kQK8 : t->ne[0]) - 1) * (int64_t)t->nb[0];
    for (int i = 1; i < 4; ++i) last += (t->ne[i] - 1) * (int64_t)t->nb[i];
    const int64_t eb = q8 ? kQ8Bytes : type_elem_bytes(t->type);
    return (size_t)(last + (eb > 0 ? eb : 1));
}
bool overlaps(const vva_tensor* a, const vva_tensor* b) {
    const uintptr_t a0 = (uintptr_t)a->data, b0 = (uintptr_t)b->data;
    return a0 < b0 + tensor_span(b) && b0 < a0 + tensor_span(a);
}

vva_status check_tensor(vva_context* ctx, const vva_tensor* t, const char* name) {
    if (!t || !t->data) return fail(ctx, VVA_ERR_INVALID_ARG, "%s: null tensor", name);
    for (int i = 0; i < 4; ++i)
        if (t->ne[i] < 1) return fail(ctx, VVA_ERR_INVALID_ARG, "%s: ne[%d] = %lld", name, i, (long long)t->ne[i]);
    return VVA_OK;
}

// Grows the context's split workspace to at least `bytes`.  Growing
// allocates, which a stream under HIP graph capture must not do: such a call
// fails with VVA_ERR_INVALID_ARG (run one call of the largest shape before
// capturing).  The outgrown workspace is retired, not freed (see
// vva_context::ws_retired).  The size at least doubles at every growth (a
// power of two, 1 MiB at least), so the retired buffers together never
// exceed the live one: a chunked prefill whose window grows by one chunk per
// call retires O(log n) buffers, not one per chunk.
vva_status ensure_ws(vva_context* ctx, size_t bytes) {
    if (bytes <= ctx->ws_bytes) return VVA_OK;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(ctx->stream, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone)
        return fail(ctx, VVA_ERR_INVALID_ARG,
                    "split workspace must grow to %zu bytes during stream capture; run one call of this "
                    "shape before capturing", bytes);
    size_t sz = (size_t)1 << 20;
    while (sz < bytes) sz <<= 1;
    float* p = nullptr;
    hipError_t e = hipMalloc(&p, sz);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipMalloc(split workspace)");
    if (ctx->ws) ctx->ws_retired.push_back(ctx->ws);
    ctx->ws = p;
    ctx->ws_bytes = sz;
    return VVA_OK;
}

// Split workspace of one call: the context's, grown on demand, or (fixed)
// the device's static scratch, which never allocates and refuses sizes
// beyond kScratchBytes.
vva_status get_ws(vva_context* ctx, bool fixed, size_t bytes, float** ws) {
    if (fixed) {
        if (bytes > kScratchBytes)
            return fail(ctx, VVA_ERR_INVALID_ARG,
                        "attn_noalloc: this call needs %zu bytes of split workspace, more than the %zu-byte "
                        "static scratch", bytes, kScratchBytes);
        *ws = ctx->scratch;
        return VVA_OK;
    }
    vva_status st = ensure_ws(ctx, bytes);
    *ws = ctx->ws;
    return st;
}

// Shared by vva_attn, vva_attn_noalloc (fixed) and vva_flash_attn_ext once
// AttnArgs is filled.
vva_status run_attention(vva_context* ctx, AttnArgs& a, bool fixed = false) {
    hipError_t e;
    float* ws = nullptr;
    ctx->last_splits = 0;
    if (ctx->attn_path == 0 && a.T == 1 && decode_stream_supported(a)) {
        const int wgs = ctx->sched_decode_wgs > 0 ? ctx->sched_decode_wgs : ctx->n_cu;
        int n_splits = decode_stream_plan(a, wgs);
        if (ctx->sched_decode_splits > 0) n_splits = ctx->sched_decode_splits;
        if (n_splits > 1) {
            vva_status st = get_ws(ctx, fixed, (size_t)n_splits * a.B * a.Hq * (a.d + 2) * sizeof(float), &ws);
            if (st != VVA_OK) return st;
        }
        e = launch_decode_stream(a, ws, n_splits, ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "decode launch");
        if (n_splits != ctx->logged_splits)
            log_msg(VVA_LOG_DEBUG, "decode: streamed Q8_0 kernel, %d key splits per sequence (B=%d, L[0]=%d)",
                    n_splits, a.B, a.L[0]);
        ctx->last_splits = ctx->logged_splits = n_splits;
        return VVA_OK;
    }
    if (ctx->attn_path != 1 && a.T == 1 && decode_supported(a)) {
        const int nw = decode_waves(a);
        int Lmax = 1;
        for (int b = 0; b < a.B; ++b) Lmax = a.L[b] > Lmax ? a.L[b] : Lmax;
        // about one workgroup per CU over (split, sequence); each of the
        // nw / Hkv waves of a kv head takes at least 32 keys
        const int R = nw / a.Hkv;
        int target = (ctx->sched_decode_wgs > 0 ? ctx->sched_decode_wgs : ctx->n_cu) / a.B;
        if (target < 1) target = 1;
        constexpr int min_sub = 32;
        int sub_len = (Lmax + target * R - 1) / (target * R);
        if (sub_len < min_sub) sub_len = min_sub;
        const int split_len = sub_len * R;
        const int n_splits = (Lmax + split_len - 1) / split_len;
        if (n_splits > 1) {
            vva_status st = get_ws(ctx, fixed, (size_t)n_splits * a.B * a.Hq * (a.d + 2) * sizeof(float), &ws);
            if (st != VVA_OK) return st;
        }
        e = launch_decode(a, ws, n_splits, split_len, ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "decode launch");
        if (n_splits != ctx->logged_splits)
            log_msg(VVA_LOG_DEBUG, "decode: register-streamed kernel, %d key splits of %d keys (B=%d, L[0]=%d)",
                    n_splits, split_len, a.B, a.L[0]);
        ctx->last_splits = ctx->logged_splits = n_splits;
        return VVA_OK;
    }
    // Q8_0 windows, and F32 windows under flash-attention semantics (the
    // reference casts them to F16 before ggml_flash_attn_ext,
    // src/qwen2.cpp:328-331): converted to f16 on the device, then the MFMA
    // prefill (Q through a Q8_0 round trip for Q8_0 K, ggml's dot type).  On
    // the no-allocation path the converted window and the split partials
    // share the static scratch; a call whose window does not fit there is
    // refused rather than sent to a different kernel.
    const bool convert = a.k_type == a.v_type &&
                         (a.k_type == VVA_TYPE_Q8_0 || (a.k_type == VVA_TYPE_F32 && ctx->use_flash_attn));
    // prefill plan of call shape c, reused while the shape repeats
    // (the merge in the launch needs the context's tickets: not vva_attn_noalloc)
    auto plan_for = [&](const AttnArgs& c, size_t cap) {
        std::array<int64_t, 10 + 2 * VVA_MAX_BATCH> key{c.d, c.Hq, c.Hkv, c.T, c.B, c.mask_mode, ctx->n_cu,
                                                       ctx->sched_prefill_splits, (int64_t)cap, (int64_t)fixed};
        int n = 10;
        for (int b = 0; b < c.B; ++b) {
            key[n++] = c.L[b];
            key[n++] = c.past[b];
        }
        if (n != ctx->plan_key_n || !std::equal(key.begin(), key.begin() + n, ctx->plan_key.begin())) {
            ctx->plan = prefill_plan(c, ctx->n_cu, ctx->sched_prefill_splits, cap, !fixed);
            ctx->plan_key = key;
            ctx->plan_key_n = n;
            log_msg(VVA_LOG_DEBUG, "prefill plan: T=%d B=%d L[0]=%d: row tiles from %d split %d ways%s", c.T, c.B,
                    c.L[0], ctx->plan.R, ctx->plan.max_ks, ctx->plan.in_launch ? ", merged in the launch" : "");
        }
        return ctx->plan;
    };
    if (ctx->attn_path != 1 && a.T > 1 && convert && (a.d == 64 || a.d == 128)) {
        AttnArgs c = a;
        const size_t wb = window_f16_bytes(a);
        c.k_type = c.v_type = VVA_TYPE_F16;
        c.k_nb_tok = c.v_nb_tok = (int64_t)a.Hkv * a.d * 2;
        c.k_nb_head = c.v_nb_head = (int64_t)a.d * 2;
        c.q_round_q8 = a.k_type == VVA_TYPE_Q8_0;
        // pointers into the workspace only after it is sized: placeholders
        // with the final alignment for the support check
        for (int b = 0; b < a.B; ++b) c.k[b] = c.v[b] = (const char*)(uintptr_t)256;
        if (prefill_supported(c)) {
            if (fixed && wb >= kScratchBytes)
                return fail(ctx, VVA_ERR_NOT_IMPLEMENTED,
                            "attn_noalloc: the f16 window of this %s cache (%zu bytes) does not fit the %zu-byte "
                            "static scratch", a.k_type == VVA_TYPE_Q8_0 ? "Q8_0" : "F32", wb, kScratchBytes);
            const PrefillPlan plan = plan_for(c, fixed ? kScratchBytes - wb : ((size_t)1 << 34));
            const size_t need = wb + prefill_ws_bytes(c, plan);
            char* wbase = nullptr;
            if (fixed) {
                if (need > kScratchBytes)
                    return fail(ctx, VVA_ERR_NOT_IMPLEMENTED,
                                "attn_noalloc: the f16 window and split partials of this call (%zu bytes) do not "
                                "fit the %zu-byte static scratch", need, kScratchBytes);
                wbase = (char*)ctx->scratch;
            } else {
                vva_status st = ensure_ws(ctx, need);
                if (st != VVA_OK) return st;
                wbase = (char*)ctx->ws;
            }
            size_t off = 0;
            for (int b = 0; b < a.B; ++b) {
                c.k[b] = wbase + off;
                c.v[b] = wbase + off + (size_t)a.L[b] * a.Hkv * a.d * 2;
                off += (size_t)2 * a.L[b] * a.Hkv * a.d * 2;
            }
            // Q8_0: a value beyond the f16 range flags the call, and the fp32
            // row kernel, launched gated behind the prefill, recomputes it
            // from the Q8_0 cache (ggml dequantizes Q8_0 to fp32: finite);
            // F32 windows overflow in the reference's own F16 cast too
            const bool q8 = a.k_type == VVA_TYPE_Q8_0;
            const unsigned long long epoch = q8 ? ++ctx->ovf_epoch : 0;
            e = launch_window_to_f16(a, wbase, q8 ? ctx->ovf : nullptr, epoch, ctx->stream);
            if (e == hipSuccess)
                e = launch_prefill(c, (float*)(wbase + wb), ctx->tickets + kMaxStepTickets, plan, ctx->stream);
            if (e == hipSuccess && q8) {
                AttnArgs g = a;
                g.gate = ctx->ovf;
                g.gate_epoch = epoch;
                e = launch_attn_rows(g, ctx->stream);
            }
            if (e != hipSuccess) return hip_fail(ctx, e, "prefill launch");
            ctx->last_splits = plan.max_ks;
            return VVA_OK;
        }
    }
    if (ctx->attn_path != 1 && a.T > 1 && prefill_supported(a)) {
        const PrefillPlan plan = plan_for(a, fixed ? kScratchBytes : ((size_t)1 << 34));
        if (plan.max_ks > 1) {
            vva_status st = get_ws(ctx, fixed, prefill_ws_bytes(a, plan), &ws);
            if (st != VVA_OK) return st;
        }
        e = launch_prefill(a, ws, ctx->tickets + kMaxStepTickets, plan, ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "prefill launch");
        ctx->last_splits = plan.max_ks;
        return VVA_OK;
    }
    e = launch_attn_rows(a, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "attention launch");
    return VVA_OK;
}

vva_status fill_mask(vva_context* ctx, AttnArgs& a, const vva_tensor* mask, int T, int B, int Lmax) {
    if (!mask) return VVA_OK;
    vva_status st = check_tensor(ctx, mask, "mask");
    if (st != VVA_OK) return st;
    // F16 (ggml_flash_attn_ext's mask type, the reference's callers) or F32
    // (ggml_soft_max_ext's, the eager branch src/qwen2.cpp:336-344)
    if (mask->type != VVA_TYPE_F16 && mask->type != VVA_TYPE_F32)
        return fail(ctx, VVA_ERR_INVALID_ARG, "mask must be F16 or F32");
    const size_t es = mask->type == VVA_TYPE_F32 ? 4 : 2;
    if (mask->nb[0] != es) return fail(ctx, VVA_ERR_INVALID_ARG, "mask rows must be contiguous");
    if (mask->ne[0] < Lmax || mask->ne[1] < T)
        return fail(ctx, VVA_ERR_INVALID_ARG, "mask ne=[%lld,%lld] smaller than [L=%d,T=%d]",
                    (long long)mask->ne[0], (long long)mask->ne[1], Lmax, T);
    if (mask->ne[2] != 1) return fail(ctx, VVA_ERR_NOT_IMPLEMENTED, "per-head masks are not supported");
    if (mask->ne[3] != 1 && mask->ne[3] != B)
        return fail(ctx, VVA_ERR_INVALID_ARG, "mask ne[3] must be 1 or B");
    a.mask = (const char*)mask->data;
    a.mask_nb_row = (int64_t)mask->nb[1];
    a.mask_nb_b = mask->ne[3] == 1 ? 0 : (int64_t)mask->nb[3];
    a.mask_mode = kMaskExplicit;
    a.mask_f32 = mask->type == VVA_TYPE_F32;
    return VVA_OK;
}

}  // namespace

// ------------------------------------------------------------------ context

extern "C" vva_status vva_create(int device, void* stream, vva_context** out) {
    if (!out) return fail(nullptr, VVA_ERR_INVALID_ARG, "out is null");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) return fail(nullptr, VVA_ERR_DEVICE, "no HIP device available");
    if (device < 0 || device >= n) return fail(nullptr, VVA_ERR_INVALID_ARG, "device %d out of range", device);
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return fail(nullptr, VVA_ERR_DEVICE, "hipGetDeviceProperties failed");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(nullptr, VVA_ERR_NOT_IMPLEMENTED, "kernels are built for gfx950, device is %s", prop.gcnArchName);
    DeviceGuard g(device);
    float* scr = nullptr;
    if (device < kMaxDevices) {
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        if (!g_scratch[device]) {
            e = hipGetSymbolAddress((void**)&g_scratch[device], HIP_SYMBOL(scratch));
            if (e != hipSuccess) {
                g_scratch[device] = nullptr;
                return fail(nullptr, VVA_ERR_DEVICE, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
            }
        }
        scr = g_scratch[device];
    }
    auto* ctx = new vva_context();
    ctx->device = device;
    ctx->n_cu = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
    ctx->stream = (hipStream_t)stream;
    ctx->scratch = scr;
    ctx->err.reserve(512);               // error messages (< 512 bytes) then never allocate
    constexpr size_t ticket_bytes = sizeof(unsigned) * (kMaxStepTickets + kMaxPrefillTickets + kMaxProjTickets);
    e = hipMalloc(&ctx->tickets, ticket_bytes);
    if (e == hipSuccess) e = hipMemset(ctx->tickets, 0, ticket_bytes);
    if (e == hipSuccess) e = hipMalloc(&ctx->ovf, 256);
    if (e == hipSuccess) e = hipMemset(ctx->ovf, 0, 256);
    if (e != hipSuccess) {
        if (ctx->tickets) (void)hipFree(ctx->tickets);
        if (ctx->ovf) (void)hipFree(ctx->ovf);
        delete ctx;
        *out = nullptr;
        return fail(nullptr, VVA_ERR_DEVICE, "vva_create: ticket buffer: %s", hipGetErrorString(e));
    }
    log_msg(VVA_LOG_INFO, "context on device %d (%s, %s, %d CUs)", device, prop.name, prop.gcnArchName, ctx->n_cu);
    *out = ctx;
    return VVA_OK;
}

extern "C" void vva_destroy(vva_context* ctx) {
    if (!ctx) return;
    DeviceGuard g(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    {
        std::lock_guard<std::mutex> lk(g_kv_mu);
        for (vva_kv* kv : ctx->caches) g_kv_live.erase(kv);
    }
    for (vva_kv* kv : ctx->caches) {
        (void)hipFree(kv->base);
        delete kv;
    }
    ctx->caches.clear();
    if (ctx->ws) (void)hipFree(ctx->ws);
    for (float* p : ctx->ws_retired) (void)hipFree(p);
    if (ctx->tickets) (void)hipFree(ctx->tickets);
    if (ctx->ovf) (void)hipFree(ctx->ovf);
    delete ctx;
}

extern "C" vva_status vva_set_stream(vva_context* ctx, void* stream) {
    if (!ctx) return VVA_ERR_INVALID_ARG;
    DeviceGuard g(ctx->device);
    // finish work queued on the previous stream before switching
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamSynchronize");
    ctx->stream = (hipStream_t)stream;
    return VVA_OK;
}

extern "C" vva_status vva_synchronize(vva_context* ctx) {
    if (!ctx) return VVA_ERR_INVALID_ARG;
    DeviceGuard g(ctx->device);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? VVA_OK : hip_fail(ctx, e, "hipStreamSynchronize");
}

extern "C" const char* vva_last_error(const vva_context* ctx) {
    return ctx ? ctx->err.c_str() : g_create_err.c_str();
}

extern "C" const char* vva_version(void) { return "vva 0.1.0 (gfx950)"; }

extern "C" void vva_set_log_callback(vva_log_cb cb, void* user_data, vva_log_level max_lvl) {
    LogSink& s = log_sink();
    std::lock_guard<std::recursive_mutex> lk(s.mu);
    s.cb = cb;
    s.user = user_data;
    s.max_lvl = cb ? (int)max_lvl : -1;
}

extern "C" vva_status vva_set_attn_path(vva_context* ctx, int path) {
    if (!ctx || path < 0 || path > 2) return VVA_ERR_INVALID_ARG;
    ctx->attn_path = path;
    return VVA_OK;
}

extern "C" int vva_last_decode_splits(const vva_context* ctx) { return ctx ? ctx->last_splits : 0; }

extern "C" vva_status vva_set_flash_attn(vva_context* ctx, int use_flash_attn) {
    if (!ctx || (use_flash_attn != 0 && use_flash_attn != 1)) return VVA_ERR_INVALID_ARG;
    ctx->use_flash_attn = use_flash_attn;
    return VVA_OK;
}

extern "C" vva_status vva_set_schedule(vva_context* ctx, int decode_wgs, int decode_splits, int prefill_splits) {
    if (!ctx) return VVA_ERR_INVALID_ARG;
    if (decode_wgs < 0 || decode_splits < 0 || decode_splits > 1024 || prefill_splits < 0 || prefill_splits > 32)
        return fail(ctx, VVA_ERR_INVALID_ARG, "set_schedule: out of range (%d, %d, %d)", decode_wgs, decode_splits,
                    prefill_splits);
    ctx->sched_decode_wgs = decode_wgs;
    ctx->sched_decode_splits = decode_splits;
    ctx->sched_prefill_splits = prefill_splits;
    return VVA_OK;
}

// ----------------------------------------------------------------- KV cache

extern "C" vva_status vva_kv_create(vva_context* ctx, const vva_kv_desc* d, vva_kv** out) {
    if (!ctx) return VVA_ERR_INVALID_ARG;
    if (!d || !out) return fail(ctx, VVA_ERR_INVALID_ARG, "kv_create: null argument");
    *out = nullptr;
    if (d->n_layers < 1 || d->n_kv_heads < 1 || d->max_seq < 1 || d->n_seq < 1 || d->n_seq > 1024)
        return fail(ctx, VVA_ERR_INVALID_ARG, "kv_create: bad sizes");
    if (!cache_type(d->type)) return fail(ctx, VVA_ERR_INVALID_ARG, "kv_create: unsupported type %d", d->type);
    if (!head_dim_ok(d->head_dim, d->type))
        return fail(ctx, VVA_ERR_NOT_IMPLEMENTED, "kv_create: head_dim %d unsupported for type %d", d->head_dim, d->type);
    DeviceGuard g(ctx->device);
    auto* kv = new vva_kv();
    kv->ctx = ctx;
    kv->desc = *d;
    kv->head_bytes = type_row_bytes(d->type, d->head_dim);
    kv->row_bytes = kv->head_bytes * d->n_kv_heads;
    kv->tensor_bytes = ((size_t)kv->row_bytes * d->max_seq + 255) / 256 * 256;
    const size_t total = kv->tensor_bytes * 2 * (size_t)d->n_layers * d->n_seq;
    hipError_t e = hipMalloc(&kv->base, total);
    if (e != hipSuccess) { delete kv; return hip_fail(ctx, e, "kv_create: hipMalloc"); }
    e = hipMemsetAsync(kv->base, 0, total, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) { (void)hipFree(kv->base); delete kv; return hip_fail(ctx, e, "kv_create: memset"); }
    kv->len.assign(d->n_seq, 0);
    ctx->caches.insert(kv);
    {
        std::lock_guard<std::mutex> lk(g_kv_mu);
        g_kv_live.insert(kv);
    }
    *out = kv;
    return VVA_OK;
}

extern "C" void vva_kv_free(vva_kv* kv) {
    if (!kv) return;
    {
        // a handle already released (by vva_kv_free or vva_destroy) is ignored
        std::lock_guard<std::mutex> lk(g_kv_mu);
        if (!g_kv_live.erase(kv)) return;
    }
    vva_context* ctx = kv->ctx;
    DeviceGuard g(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipFree(kv->base);
    ctx->caches.erase(kv);
    delete kv;
}

extern "C" vva_status vva_kv_get_len(const vva_kv* kv, int seq, int32_t* len) {
    if (!kv || !kv_live(kv) || !len || seq < 0 || seq >= kv->desc.n_seq) return VVA_ERR_INVALID_ARG;
    *len = kv->len[seq];
    return VVA_OK;
}

extern "C" vva_status vva_kv_set_len(vva_kv* kv, int seq, int32_t len) {
    if (!kv || !kv_live(kv) || seq < 0 || seq >= kv->desc.n_seq || len < 0 || len > kv->desc.max_seq) return VVA_ERR_INVALID_ARG;
    kv->len[seq] = len;
    return VVA_OK;
}

extern "C" vva_status vva_kv_view(const vva_kv* kv, int layer, int seq, vva_tensor* k, vva_tensor* v) {
    if (!kv || !kv_live(kv) || layer < 0 || layer >= kv->desc.n_layers || seq < 0 || seq >= kv->desc.n_seq)
        return VVA_ERR_INVALID_ARG;
    for (int which = 0; which < 2; ++which) {
        vva_tensor* t = which == 0 ? k : v;
        if (!t) continue;
        t->data = kv_tensor(kv, layer, seq, which);
        t->type = kv->desc.type;
        t->ne[0] = kv->desc.head_dim;
        t->ne[1] = kv->desc.n_kv_heads;
        t->ne[2] = kv->desc.max_seq;
        t->ne[3] = 1;
        t->nb[0] = (size_t)type_elem_bytes(kv->desc.type);
        t->nb[1] = (size_t)kv->head_bytes;
        t->nb[2] = (size_t)kv->row_bytes;
        t->nb[3] = (size_t)kv->row_bytes * kv->desc.max_seq;
    }
    return VVA_OK;
}

extern "C" vva_status vva_kv_upload(vva_context* ctx, vva_kv* kv, int layer, int seq, int32_t start,
                                    int32_t len, const float* k_host, const float* v_host) {
    if (!ctx) return VVA_ERR_INVALID_ARG;
    if (!kv || !kv_live(kv) || kv->ctx != ctx || layer < 0 || layer >= kv->desc.n_layers || seq < 0 ||
        seq >= kv->desc.n_seq)
        return fail(ctx, VVA_ERR_INVALID_ARG, "kv_upload: bad cache / layer / seq");
    if (start < 0 || len < 0 || (int64_t)start + len > kv->desc.max_seq)
        return fail(ctx, VVA_ERR_INVALID_ARG, "kv_upload: rows [%d,%d) outside max_seq %d", start, start + len,
                    kv->desc.max_seq);
    if (len == 0) return VVA_OK;
    if (!k_host || !v_host) return fail(ctx, VVA_ERR_INVALID_ARG, "kv_upload: null host rows");
    DeviceGuard g(ctx->device);
    // Stage the F32 rows on the device and convert with the append kernel
    // (no rotation: positions are irrelevant for V, and K rows of a voice
    // prompt are stored post-RoPE, scripts/convert_voice_to_gguf.py:115-128).
    const int d = kv->desc.head_dim, H = kv->desc.n_kv_heads;
    const size_t n = (size_t)len * H * d;
    float* dev = nullptr;
    hipError_t e = hipMalloc(&dev, 2 * n * sizeof(float));
    if (e != hipSuccess) return hip_fail(ctx, e, "kv_upload: hipMalloc");
    e = hipMemcpyAsync(dev, k_host, n * sizeof(float), hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(dev + n, v_host, n * sizeof(float), hipMemcpyHostToDevice, ctx->stream);
    int32_t* zero_pos = nullptr;
    if (e == hipSuccess) e = hipMalloc(&zero_pos, sizeof(int32_t) * len);
    if (e == hipSuccess) e = hipMemsetAsync(zero_pos, 0, sizeof(int32_t) * len, ctx->stream);
    if (e == hipSuccess) {
        RopeAppendArgs a{};
        a.k = (const char*)dev;
        a.v = (const char*)(dev + n);
        a.k_type = a.v_type = VVA_TYPE_F32;
        a.k_nb_h = a.v_nb_h = (int64_t)d * 4;
        a.k_nb_t = a.v_nb_t = (int64_t)H * d * 4;
        a.k_nb_b = a.v_nb_b = 0;
        a.pos = zero_pos;              // position 0: the rotation is the identity
        a.pos_stride_b = 0;
        a.k_dst[0] = kv_tensor(kv, layer, seq, 0) + (int64_t)start * kv->row_bytes;
        a.v_dst[0] = kv_tensor(kv, layer, seq, 1) + (int64_t)start * kv->row_bytes;
        a.cache_row_bytes = kv->row_bytes;
        a.cache_head_bytes = kv->head_bytes;
        a.cache_type = kv->desc.type;
        a.d = d; a.Hq = 0; a.Hkv = H; a.T = len; a.B = 1;
        a.do_q = 0; a.do_kv = 1;
        a.theta_scale = 1.0f;
        e = launch_rope_append(a, ctx->stream);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    (void)hipFree(dev);
    if (zero_pos) (void)hipFree(zero_pos);
    return e == hipSuccess ? VVA_OK : hip_fail(ctx, e, "kv_upload");
}

// ---------------------------------------------------------------------- ops

namespace {

// Validates x/dst for RoPE: ne = [d, H, T, B], float types, contiguous rows.
vva_status check_rows(vva_context* ctx, const vva_tensor* t, const char* name, int64_t d, int64_t H,
                      int64_t T, int64_t B) {
    vva_status st = check_tensor(ctx, t, name);
    if (st != VVA_OK) return st;
    if (!float_type(t->type)) return fail(ctx, VVA_ERR_INVALID_ARG, "%s: type %d not F32/F16/BF16", name, t->type);
    if ((int64_t)t->nb[0] != type_elem_bytes(t->type))
        return fail(ctx, VVA_ERR_INVALID_ARG, "%s: rows must be contiguous (nb[0])", name);
    if (t->ne[0] != d || (H > 0 && t->ne[1] != H) || t->ne[2] != T || t->ne[3] != B)
        return fail(ctx, VVA_ERR_INVALID_ARG, "%s: ne=[%lld,%lld,%lld,%lld] expected [%lld,%lld,%lld,%lld]", name,
                    (long long)t->ne[0], (long long)t->ne[1], (long long)t->ne[2], (long long)t->ne[3],
                    (long long)d, (long long)H, (long long)T, (long long)B);
    return VVA_OK;
}

vva_status check_pos(vva_context* ctx, const vva_tensor* pos, int64_t T, int64_t B, int64_t* stride_b) {
    vva_status st = check_tensor(ctx, pos, "pos");
    if (st != VVA_OK) return st;
    if (pos->type != VVA_TYPE_I32 || pos->nb[0] != 4) return fail(ctx, VVA_ERR_INVALID_ARG, "pos must be contiguous I32");
    if (pos->ne[0] != T) return fail(ctx, VVA_ERR_INVALID_ARG, "pos ne[0]=%lld != T=%lld", (long long)pos->ne[0], (long long)T);
    if (pos->ne[1] != 1 && pos->ne[1] != B) return fail(ctx, VVA_ERR_INVALID_ARG, "pos ne[1] must be 1 or B");
    if (pos->nb[1] % 4) return fail(ctx, VVA_ERR_INVALID_ARG, "pos nb[1] misaligned");
    *stride_b = (pos->ne[1] == 1) ? 0 : (int64_t)(pos->nb[1] / 4);
    return VVA_OK;
}

}  // namespace

extern "C" vva_status vva_rope_ext(vva_context* ctx, const vva_tensor* x, const vva_tensor* pos, int n_dims,
                                   int mode, float freq_base, const vva_tensor* dst) {
    if (!ctx) return VVA_ERR_INVALID_ARG;
    if (mode != VVA_ROPE_TYPE_NEOX) return fail(ctx, VVA_ERR_NOT_IMPLEMENTED, "rope: only NEOX mode");
    vva_status st = check_tensor(ctx, x, "x");
    if (st != VVA_OK) return st;
    const int64_t d = x->ne[0], H = x->ne[1], T = x->ne[2], B = x->ne[3];
    if (n_dims != d) return fail(ctx, VVA_ERR_NOT_IMPLEMENTED, "rope: n_dims must equal ne[0]");
    if (!head_dim_ok((int)d, VVA_TYPE_F32)) return fail(ctx, VVA_ERR_NOT_IMPLEMENTED, "rope: head dim %lld", (long long)d);
    if (B > VVA_MAX_BATCH) return fail(ctx, VVA_ERR_INVALID_ARG, "rope: B > %d", VVA_MAX_BATCH);
    if ((st = check_rows(ctx, x, "x", d, H, T, B)) != VVA_OK) return st;
    if ((st = check_rows(ctx, dst, "dst", d, H, T, B)) != VVA_OK) return st;
    int64_t ps = 0;
    if ((st = check_pos(ctx, pos, T, B, &ps)) != VVA_OK) return st;
    DeviceGuard g(ctx->device);
    RopeAppendArgs a{};
    a.q = (const char*)x->data; a.q_type = x->type;
    a.q_nb_h = x->nb[1]; a.q_nb_t = x->nb[2]; a.q_nb_b = x->nb[3];
    a.q_out = (char*)dst->data; a.q_out_type = dst->type;
    a.qo_nb_h = dst->nb[1]; a.qo_nb_t = dst->nb[2]; a.qo_nb_b = dst->nb[3];
    a.pos = (const int32_t*)pos->data; a.pos_stride_b = ps;
    a.d = (int)d; a.Hq = (int)H; a.Hkv = 0; a.T = (int)T; a.B = (int)B;
    a.do_q = 1; a.do_kv = 0;
    a.theta_scale = powf(freq_base, -2.0f / (float)n_dims);
    hipError_t e = launch_rope_append(a, ctx->stream);
    return e == hipSuccess ? VVA_OK : hip_fail(ctx, e, "rope launch");
}

extern "C" vva_status vva_rope_append(vva_context* ctx, vva_kv* kv, int layer, const vva_tensor* q,
                                      const vva_tensor* k, const vva_tensor* v, const vva_tensor* pos,
                                      const int32_t* seq_ids, float freq_base, const vva_tensor* q_out) {
    if (!ctx) return VVA_ERR_INVALID_ARG;
    if (!kv || !kv_live(kv) || kv->ctx != ctx)
        return fail(ctx, VVA_ERR_INVALID_ARG, "rope_append: cache is null, released or of another context");
    if (layer < 0 || layer >= kv->desc.n_layers) return fail(ctx, VVA_ERR_INVALID_ARG, "rope_append: layer %d", layer);
    vva_status st = check_tensor(ctx, q, "q");
    if (st != VVA_OK) return st;
    const int64_t d = kv->desc.head_dim, Hkv = kv->desc.n_kv_heads;
    const int64_t Hq = q->ne[1], T = q->ne[2], B = q->ne[3];
    if (Hq % Hkv) return fail(ctx, VVA_ERR_INVALID_ARG, "rope_append: Hq %% Hkv != 0");
    if (B > VVA_MAX_BATCH) return fail(ctx, VVA_ERR_INVALID_ARG, "rope_append: B > %d", VVA_MAX_BATCH);
    if ((st = check_rows(ctx, q, "q", d, Hq, T, B)) != VVA_OK) return st;
    if ((st = check_rows(ctx, k, "k", d, Hkv, T, B)) != VVA_OK) return st;
    if ((st = check_rows(ctx, v, "v", d, Hkv, T, B)) != VVA_OK) return st;
    if ((st = check_rows(ctx, q_out, "q_out", d, Hq, T, B)) != VVA_OK) return st;
    int64_t ps = 0;
    if ((st = check_pos(ctx, pos, T, B, &ps)) != VVA_OK) return st;
    RopeAppendArgs a{};
    for (int b = 0; b < B; ++b) {
        const int seq = seq_ids ? seq_ids[b] : b;
        if (seq < 0 || seq >= kv->desc.n_seq) return fail(ctx, VVA_ERR_INVALID_ARG, "rope_append: seq %d", seq);
        for (int b2 = 0; b2 < b; ++b2)
            if ((seq_ids ? seq_ids[b2] : b2) == seq)
                return fail(ctx, VVA_ERR_INVALID_ARG, "rope_append: sequence %d appears twice", seq);
        const int64_t past = kv->len[seq];
        if (past + T > kv->desc.max_seq)
            return fail(ctx, VVA_ERR_INVALID_ARG, "rope_append: seq %d: %lld + %lld rows exceed max_seq %d", seq,
                        (long long)past, (long long)T, kv->desc.max_seq);
        a.k_dst[b] = kv_tensor(kv, layer, seq, 0) + past * kv->row_bytes;
        a.v_dst[b] = kv_tensor(kv, layer, seq, 1) + past * kv->row_bytes;
    }
    DeviceGuard g(ctx->device);
    a.q = (const char*)q->data; a.q_type = q->type;
    a.q_nb_h = q->nb[1]; a.q_nb_t = q->nb[2]; a.q_nb_b = q->nb[3];
    a.k = (const char*)k->data; a.k_type = k->type;
    a.k_nb_h = k->nb[1]; a.k_nb_t = k->nb[2]; a.k_nb_b = k->nb[3];
    a.v = (const char*)v->data; a.v_type = v->type;
    a.v_nb_h = v->nb[1]; a.v_nb_t = v->nb[2]; a.v_nb_b = v->nb[3];
    a.q_out = (char*)q_out->data; a.q_out_type = q_out->type;
    a.qo_nb_h = q_out->nb[1]; a.qo_nb_t = q_out->nb[2]; a.qo_nb_b = q_out->nb[3];
    a.pos = (const int32_t*)pos->data; a.pos_stride_b = ps;
    a.cache_row_bytes = kv->row_bytes;
    a.cache_head_bytes = kv->head_bytes;
    a.cache_type = kv->desc.type;
    a.d = (int)d; a.Hq = (int)Hq; a.Hkv = (int)Hkv; a.T = (int)T; a.B = (int)B;
    a.do_q = 1; a.do_kv = 1;
    a.theta_scale = powf(freq_base, -2.0f / (float)d);
    hipError_t e = launch_rope_append(a, ctx->stream);
    return e == hipSuccess ? VVA_OK : hip_fail(ctx, e, "rope_append launch");
}

namespace {

vva_status attn_impl(vva_context* ctx, const vva_kv* kv, int layer, const vva_tensor* q, const int32_t* seq_ids,
                     const vva_tensor* mask, float scale, const vva_tensor* out, bool fixed) {
    if (!ctx) return VVA_ERR_INVALID_ARG;
    if (fixed && !ctx->scratch)
        return fail(ctx, VVA_ERR_NOT_IMPLEMENTED, "attn_noalloc: no static scratch on device %d", ctx->device);
    if (!kv || !kv_live(kv) || kv->ctx != ctx)
        return fail(ctx, VVA_ERR_INVALID_ARG, "attn: cache is null, released or of another context");
    if (layer < 0 || layer >= kv->desc.n_layers) return fail(ctx, VVA_ERR_INVALID_ARG, "attn: layer %d", layer);
    vva_status st = check_tensor(ctx, q, "q");
    if (st != VVA_OK) return st;
    const int64_t d = kv->desc.head_dim, Hkv = kv->desc.n_kv_heads;
    const int64_t Hq = q->ne[1], T = q->ne[2], B = q->ne[3];
    if (Hq % Hkv) return fail(ctx, VVA_ERR_INVALID_ARG, "attn: Hq %% Hkv != 0");
    if (B > VVA_MAX_BATCH) return fail(ctx, VVA_ERR_INVALID_ARG, "attn: B > %d", VVA_MAX_BATCH);
    if ((st = check_rows(ctx, q, "q", d, Hq, T, B)) != VVA_OK) return st;
    if ((st = check_rows(ctx, out, "out", d, Hq, T, B)) != VVA_OK) return st;
    if (out->type != VVA_TYPE_F32) return fail(ctx, VVA_ERR_INVALID_ARG, "attn: out must be F32");
    AttnArgs a{};
    int Lmax = 0;
    for (int b = 0; b < B; ++b) {
        const int seq = seq_ids ? seq_ids[b] : b;
        if (seq < 0 || seq >= kv->desc.n_seq) return fail(ctx, VVA_ERR_INVALID_ARG, "attn: seq %d", seq);
        const int64_t past = kv->len[seq];
        if (past + T > kv->desc.max_seq)
            return fail(ctx, VVA_ERR_INVALID_ARG, "attn: seq %d window %lld exceeds max_seq", seq, (long long)(past + T));
        a.k[b] = kv_tensor(kv, layer, seq, 0);
        a.v[b] = kv_tensor(kv, layer, seq, 1);
        a.L[b] = (int)(past + T);
        a.past[b] = (int)past;
        Lmax = a.L[b] > Lmax ? a.L[b] : Lmax;
    }
    a.q = (const char*)q->data; a.q_type = q->type;
    a.q_nb_h = q->nb[1]; a.q_nb_t = q->nb[2]; a.q_nb_b = q->nb[3];
    a.k_nb_tok = a.v_nb_tok = kv->row_bytes;
    a.k_nb_head = a.v_nb_head = kv->head_bytes;
    a.k_type = a.v_type = kv->desc.type;
    a.mask_mode = kMaskCausal;
    if ((st = fill_mask(ctx, a, mask, (int)T, (int)B, Lmax)) != VVA_OK) return st;
    a.scale = scale;
    a.out = (float*)out->data;
    a.o_nb_h = out->nb[1]; a.o_nb_t = out->nb[2]; a.o_nb_b = out->nb[3];
    a.d = (int)d; a.Hq = (int)Hq; a.Hkv = (int)Hkv; a.T = (int)T; a.B = (int)B;
    DeviceGuard g(ctx->device);
    return run_attention(ctx, a, fixed);
}

}  // namespace

extern "C" vva_status vva_attn(vva_context* ctx, const vva_kv* kv, int layer, const vva_tensor* q,
                               const int32_t* seq_ids, const vva_tensor* mask, float scale, const vva_tensor* out) {
    return attn_impl(ctx, kv, layer, q, seq_ids, mask, scale, out, false);
}

extern "C" vva_status vva_attn_noalloc(vva_context* ctx, const vva_kv* kv, int layer, const vva_tensor* q,
                                       const int32_t* seq_ids, const vva_tensor* mask, float scale,
                                       const vva_tensor* out) {
    return attn_impl(ctx, kv, layer, q, seq_ids, mask, scale, out, true);
}

extern "C" vva_status vva_flash_attn_ext(vva_context* ctx, const vva_tensor* q, const vva_tensor* k,
                                         const vva_tensor* v, const vva_tensor* mask, float scale, float max_bias,
                                         float logit_softcap, const vva_tensor* dst) {
    if (!ctx) return VVA_ERR_INVALID_ARG;
    if (max_bias != 0.0f || logit_softcap != 0.0f)
        return fail(ctx, VVA_ERR_NOT_IMPLEMENTED, "flash_attn_ext: max_bias / logit_softcap must be 0");
    vva_status st;
    if ((st = check_tensor(ctx, q, "q")) != VVA_OK) return st;
    if ((st = check_tensor(ctx, k, "k")) != VVA_OK) return st;
    if ((st = check_tensor(ctx, v, "v")) != VVA_OK) return st;
    if ((st = check_tensor(ctx, dst, "dst")) != VVA_OK) return st;
    const int64_t d = q->ne[0], T = q->ne[1], Hq = q->ne[2], B = q->ne[3];
    const int64_t L = k->ne[1], Hkv = k->ne[2];
    if (!float_type(q->type) || (int64_t)q->nb[0] != type_elem_bytes(q->type))
        return fail(ctx, VVA_ERR_INVALID_ARG, "q: F32/F16/BF16 with contiguous rows");
    if (!cache_type(k->type) || !cache_type(v->type)) return fail(ctx, VVA_ERR_INVALID_ARG, "k/v: unsupported type");
    if (!head_dim_ok((int)d, k->type) || !head_dim_ok((int)d, v->type))
        return fail(ctx, VVA_ERR_NOT_IMPLEMENTED, "head dim %lld unsupported", (long long)d);
    if (k->ne[0] != d || v->ne[0] != d || v->ne[1] != L || v->ne[2] != Hkv)
        return fail(ctx, VVA_ERR_INVALID_ARG, "k/v shapes do not match q");
    if ((int64_t)k->nb[0] != type_elem_bytes(k->type) || (int64_t)v->nb[0] != type_elem_bytes(v->type))
        return fail(ctx, VVA_ERR_INVALID_ARG, "k/v rows must be contiguous");
    if (Hq % Hkv) return fail(ctx, VVA_ERR_INVALID_ARG, "Hq %% Hkv != 0");
    if ((k->ne[3] != 1 && k->ne[3] != B) || (v->ne[3] != 1 && v->ne[3] != B))
        return fail(ctx, VVA_ERR_INVALID_ARG, "k/v ne[3] must be 1 or B");
    if (B > VVA_MAX_BATCH) return fail(ctx, VVA_ERR_INVALID_ARG, "B > %d", VVA_MAX_BATCH);
    if (dst->type != VVA_TYPE_F32 || dst->nb[0] != 4 || dst->ne[0] != d || dst->ne[1] != Hq || dst->ne[2] != T ||
        dst->ne[3] != B)
        return fail(ctx, VVA_ERR_INVALID_ARG, "dst must be F32 ne=[d,Hq,T,B]");
    AttnArgs a{};
    for (int b = 0; b < B; ++b) {
        a.k[b] = (const char*)k->data + (k->ne[3] == 1 ? 0 : b * (int64_t)k->nb[3]);
        a.v[b] = (const char*)v->data + (v->ne[3] == 1 ? 0 : b * (int64_t)v->nb[3]);
        a.L[b] = (int)L;
        a.past[b] = (int)(L - T);
    }
    a.q = (const char*)q->data; a.q_type = q->type;
    a.q_nb_t = q->nb[1]; a.q_nb_h = q->nb[2]; a.q_nb_b = q->nb[3];
    a.k_nb_tok = k->nb[1]; a.k_nb_head = k->nb[2];
    a.v_nb_tok = v->nb[1]; a.v_nb_head = v->nb[2];
    a.k_type = k->type; a.v_type = v->type;
    a.mask_mode = kMaskNone;
    if ((st = fill_mask(ctx, a, mask, (int)T, (int)B, (int)L)) != VVA_OK) return st;
    a.scale = scale;
    a.out = (float*)dst->data;
    a.o_nb_h = dst->nb[1]; a.o_nb_t = dst->nb[2]; a.o_nb_b = dst->nb[3];
    a.d = (int)d; a.Hq = (int)Hq; a.Hkv = (int)Hkv; a.T = (int)T; a.B = (int)B;
    DeviceGuard g(ctx->device);
    return run_attention(ctx, a);
}

extern "C" int vva_supports(const vva_context* ctx, int head_dim, int n_q_heads, int n_kv_heads, int q_type,
                            int kv_type) {
    if (!ctx) return 0;
    if (n_kv_heads < 1 || n_q_heads < 1 || n_q_heads % n_kv_heads) return 0;
    if (!float_type(q_type) || !cache_type(kv_type)) return 0;
    return head_dim_ok(head_dim, kv_type) ? 1 : 0;
}

// ------------------------------------------------------------ projections

namespace {

// A weight matrix ne = [K, M] of F16 or Q8_0 rows.
vva_status check_weight(vva_context* ctx, const vva_tensor* w, const char* name, int64_t K, int64_t M, int type) {
    vva_status st = check_tensor(ctx, w, name);
    if (st != VVA_OK) return st;
    if (w->type != type) return fail(ctx, VVA_ERR_INVALID_ARG, "%s: type %d, expected %d", name, w->type, type);
    if (w->ne[0] != K || w->ne[1] != M || w->ne[2] != 1 || w->ne[3] != 1)
        return fail(ctx, VVA_ERR_INVALID_ARG, "%s: ne=[%lld,%lld,%lld,%lld], expected [%lld,%lld,1,1]", name,
                    (long long)w->ne[0], (long long)w->ne[1], (long long)w->ne[2], (long long)w->ne[3],
                    (long long)K, (long long)M);
    if ((int64_t)w->nb[0] != type_elem_bytes(type) || (int64_t)w->nb[1] < type_row_bytes(type, K))
        return fail(ctx, VVA_ERR_INVALID_ARG, "%s: rows must be contiguous", name);
    const size_t al = type == VVA_TYPE_F16 ? 16 : 4;
    if ((uintptr_t)w->data % al || w->nb[1] % al)
        return fail(ctx, VVA_ERR_INVALID_ARG, "%s: rows must be %zu-byte aligned", name, al);
    if ((uint64_t)w->nb[1] * 128 >= ((uint64_t)1 << 31))
        return fail(ctx, VVA_ERR_NOT_IMPLEMENTED, "%s: row stride too large", name);
    return VVA_OK;
}

vva_status check_bias(vva_context* ctx, const vva_tensor* b, const char* name, int64_t M) {
    if (!b) return VVA_OK;
    vva_status st = check_tensor(ctx, b, name);
    if (st != VVA_OK) return st;
    if (b->type != VVA_TYPE_F32 || b->ne[0] != M || b->nb[0] != 4 || b->ne[1] * b->ne[2] * b->ne[3] != 1)
        return fail(ctx, VVA_ERR_INVALID_ARG, "%s: must be F32 ne=[%lld]", name, (long long)M);
    return VVA_OK;
}

// x / o rows: ne = [K, T, B, 1] (or [K, T, 1, 1]), contiguous rows of a float type.
vva_status check_act(vva_context* ctx, const vva_tensor* x, const char* name, int64_t K, int64_t T, int64_t B) {
    vva_status st = check_tensor(ctx, x, name);
    if (st != VVA_OK) return st;
    if (!float_type(x->type) || (int64_t)x->nb[0] != type_elem_bytes(x->type))
        return fail(ctx, VVA_ERR_INVALID_ARG, "%s: F32/F16/BF16 with contiguous rows", name);
    if (x->ne[0] != K || x->ne[1] != T || x->ne[2] != B || x->ne[3] != 1)
        return fail(ctx, VVA_ERR_INVALID_ARG, "%s: ne=[%lld,%lld,%lld,%lld], expected [%lld,%lld,%lld,1]", name,
                    (long long)x->ne[0], (long long)x->ne[1], (long long)x->ne[2], (long long)x->ne[3],
                    (long long)K, (long long)T, (long long)B);
    return VVA_OK;
}

// Rows that start on 16-byte boundaries (the few-row projection reads them
// 16 bytes at a time).
bool rows16(const vva_tensor* x) {
    return (uintptr_t)x->data % 16 == 0 && x->nb[1] % 16 == 0 && x->nb[2] % 16 == 0;
}

}  // namespace

// The prep + GEMM launches of a projection with their workspace: the
// converted token rows (and RoPE table), then, for Q8_0 weights over a long
// call, the weights dequantized to f16 (the GEMM then runs on those), then,
// when the GEMM is split along K, the pieces' partials; the split tickets
// follow the decode step's and the prefill's in the context's ticket buffer.
static vva_status run_proj_gemm(vva_context* ctx, ProjPrepArgs& p, ProjArgs& a, int N, int K, int P) {
    const bool dq = proj_dequant_q8(a);
    ProjArgs g = a;                                    // the GEMM's view of the weights
    if (dq) g.w_type = VVA_TYPE_F16;
    g.ksplit = proj_ksplit(g, ctx->n_cu, &g.tail0);
    g.tickets = ctx->tickets + kMaxStepTickets + kMaxPrefillTickets;
    const size_t base = (proj_ws_bytes(N, K, P) + 255) / 256 * 256;
    const size_t wbytes = dq ? ((size_t)a.M * K * 2 + 255) / 256 * 256 : 0;
    vva_status st = ensure_ws(ctx, base + wbytes + proj_part_bytes(g));
    if (st != VVA_OK) return st;
    if (dq) {
        uint16_t* wd = (uint16_t*)((char*)ctx->ws + base);
        const hipError_t e = launch_proj_dequant_q8(a, wd, ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "projection weight dequantization");
        for (int i = 0; i < 3; ++i) {
            g.w[i] = (const char*)(wd + (int64_t)(i == 0 ? 0 : a.m_end[i - 1]) * K);
            g.w_nb[i] = (int64_t)K * 2;
        }
    }
    g.part = g.ksplit > 1 ? (char*)ctx->ws + base + wbytes : nullptr;
    const hipError_t e = launch_proj(p, g, ctx->ws, ctx->stream);
    return e == hipSuccess ? VVA_OK : hip_fail(ctx, e, "projection launch");
}

extern "C" vva_status vva_qkv_rope_append(vva_context* ctx, vva_kv* kv, int layer, const vva_tensor* x,
                                          const vva_tensor* wq, const vva_tensor* wk, const vva_tensor* wv,
                                          const vva_tensor* bq, const vva_tensor* bk, const vva_tensor* bv,
                                          const vva_tensor* pos, const int32_t* seq_ids, float freq_base,
                                          const vva_tensor* q_out) {
    if (!ctx) return VVA_ERR_INVALID_ARG;
    if (!kv || !kv_live(kv) || kv->ctx != ctx)
        return fail(ctx, VVA_ERR_INVALID_ARG, "qkv_rope_append: cache is null, released or of another context");
    if (layer < 0 || layer >= kv->desc.n_layers) return fail(ctx, VVA_ERR_INVALID_ARG, "qkv_rope_append: layer %d", layer);
    vva_status st;
    if ((st = check_tensor(ctx, x, "x")) != VVA_OK) return st;
    if ((st = check_tensor(ctx, q_out, "q_out")) != VVA_OK) return st;
    if ((st = check_tensor(ctx, wq, "wq")) != VVA_OK) return st;
    const int64_t d = kv->desc.head_dim, Hkv = kv->desc.n_kv_heads;
    const int64_t K = x->ne[0], T = x->ne[1], B = x->ne[2];
    const int64_t Hq = q_out->ne[1];
    if (Hq < 1 || Hq % Hkv) return fail(ctx, VVA_ERR_INVALID_ARG, "qkv_rope_append: Hq %% Hkv != 0");
    if (B > VVA_MAX_BATCH) return fail(ctx, VVA_ERR_INVALID_ARG, "qkv_rope_append: B > %d", VVA_MAX_BATCH);
    const int wt = wq->type;
    if (wt != VVA_TYPE_F16 && wt != VVA_TYPE_Q8_0)
        return fail(ctx, VVA_ERR_NOT_IMPLEMENTED, "qkv_rope_append: weights must be F16 or Q8_0");
    if (K % 64 || (Hq * d) % 128 || (Hkv * d) % 128 || (d != 64 && d != 128))
        return fail(ctx, VVA_ERR_NOT_IMPLEMENTED,
                    "qkv_rope_append: needs hidden %% 64 == 0, Hq*d and Hkv*d multiples of 128, head_dim 64 or 128");
    if ((st = check_act(ctx, x, "x", K, T, B)) != VVA_OK) return st;
    if ((st = check_weight(ctx, wq, "wq", K, Hq * d, wt)) != VVA_OK) return st;
    if ((st = check_weight(ctx, wk, "wk", K, Hkv * d, wt)) != VVA_OK) return st;
    if ((st = check_weight(ctx, wv, "wv", K, Hkv * d, wt)) != VVA_OK) return st;
    if ((st = check_bias(ctx, bq, "bq", Hq * d)) != VVA_OK) return st;
    if ((st = check_bias(ctx, bk, "bk", Hkv * d)) != VVA_OK) return st;
    if ((st = check_bias(ctx, bv, "bv", Hkv * d)) != VVA_OK) return st;
    if ((st = check_rows(ctx, q_out, "q_out", d, Hq, T, B)) != VVA_OK) return st;
    int64_t ps = 0;
    if ((st = check_pos(ctx, pos, T, B, &ps)) != VVA_OK) return st;
    const int64_t N = T * B;
    if (N * K * 2 >= ((int64_t)1 << 31) || 128 * K * 2 >= ((int64_t)1 << 31))
        return fail(ctx, VVA_ERR_NOT_IMPLEMENTED, "qkv_rope_append: %lld x %lld inputs exceed 2 GiB", (long long)N,
                    (long long)K);
    ProjArgs a{};
    for (int b = 0; b < B; ++b) {
        const int seq = seq_ids ? seq_ids[b] : b;
        if (seq < 0 || seq >= kv->desc.n_seq) return fail(ctx, VVA_ERR_INVALID_ARG, "qkv_rope_append: seq %d", seq);
        for (int b2 = 0; b2 < b; ++b2)
            if ((seq_ids ? seq_ids[b2] : b2) == seq)
                return fail(ctx, VVA_ERR_INVALID_ARG, "qkv_rope_append: sequence %d appears twice", seq);
        const int64_t past = kv->len[seq];
        if (past + T > kv->desc.max_seq)
            return fail(ctx, VVA_ERR_INVALID_ARG, "qkv_rope_append: seq %d: %lld + %lld rows exceed max_seq %d", seq,
                        (long long)past, (long long)T, kv->desc.max_seq);
        a.k_dst[b] = kv_tensor(kv, layer, seq, 0) + past * kv->row_bytes;
        a.v_dst[b] = kv_tensor(kv, layer, seq, 1) + past * kv->row_bytes;
    }
    const vva_tensor* ws_[3] = {wq, wk, wv};
    const vva_tensor* bs_[3] = {bq, bk, bv};
    const int64_t rows[3] = {Hq * d, Hkv * d, Hkv * d};
    int64_t m_end = 0;
    for (int i = 0; i < 3; ++i) {
        a.w[i] = (const char*)ws_[i]->data;
        a.w_nb[i] = (int64_t)ws_[i]->nb[1];
        m_end += rows[i];
        a.m_end[i] = (int)m_end;
        a.bias[i] = bs_[i] ? (const float*)bs_[i]->data : nullptr;
    }
    a.w_type = wt;
    a.N = (int)N; a.K = (int)K; a.M = (int)m_end;
    a.mode = kProjQKV;
    a.q_out = (char*)q_out->data; a.q_out_type = q_out->type;
    a.qo_nb_h = q_out->nb[1]; a.qo_nb_t = q_out->nb[2]; a.qo_nb_b = q_out->nb[3];
    a.cache_row_bytes = kv->row_bytes;
    a.cache_head_bytes = kv->head_bytes;
    a.cache_type = kv->desc.type;
    a.d = (int)d; a.Hq = (int)Hq; a.Hkv = (int)Hkv; a.T = (int)T;
    {
        // the GEMM epilogue stores 8 elements at a time where q_out and the
        // cache rows are of a float type and 16-byte aligned (Q8_0 caches
        // quantize per rotation pair)
        auto al16 = [](int64_t v) { return v % 16 == 0; };
        bool vec = float_type(a.q_out_type) && float_type(a.cache_type) && d % 8 == 0 &&
                   (int64_t)q_out->nb[0] == type_elem_bytes(a.q_out_type) && al16((int64_t)(uintptr_t)a.q_out) &&
                   al16(a.qo_nb_h) && al16(a.qo_nb_t) && al16(a.qo_nb_b) && al16(a.cache_row_bytes) &&
                   al16(a.cache_head_bytes);
        for (int b = 0; b < (int)B; ++b)
            vec = vec && al16((int64_t)(uintptr_t)a.k_dst[b]) && al16((int64_t)(uintptr_t)a.v_dst[b]);
        a.vec_store = vec;
    }
    ProjPrepArgs p{};
    p.x = (const char*)x->data; p.x_type = x->type;
    p.x_nb_t = (int64_t)x->nb[1]; p.x_nb_b = (int64_t)x->nb[2];
    p.K = (int)K; p.T = (int)T; p.N = (int)N;
    p.q8 = wt == VVA_TYPE_Q8_0;
    p.pos = (const int32_t*)pos->data; p.pos_stride_b = ps;
    p.P = (int)(d / 2);
    p.theta_scale = powf(freq_base, -2.0f / (float)d);
    DeviceGuard g(ctx->device);
    if (proj_gemv_supported((int)N, (int)K, a.M) && rows16(x)) {
        // a decode step: the weight-streaming GEMV.  F32 / F16 / BF16 caches:
        // it rotates q and k and stores q_out and the cache rows itself (each
        // wave computes two whole rotation pairs), one launch.  Q8_0 caches
        // (a block's scale needs 32 dims of a head): it writes the F32
        // projections and the RoPE + append kernel quantizes and stores them.
        a.x = p.x; a.x_type = p.x_type; a.x_nb_t = p.x_nb_t; a.x_nb_b = p.x_nb_b;
        a.pos = p.pos; a.pos_stride_b = p.pos_stride_b; a.theta_scale = p.theta_scale;
        if (proj_gemv_rope_ok(a)) {
            a.mode = kProjQKVRope;
            hipError_t e = launch_proj_gemv(a, nullptr, ctx->n_cu, ctx->stream);
            return e == hipSuccess ? VVA_OK : hip_fail(ctx, e, "qkv_rope_append launch");
        }
        if ((st = ensure_ws(ctx, (size_t)N * a.M * sizeof(float))) != VVA_OK) return st;
        float* y = ctx->ws;
        hipError_t e = launch_proj_gemv(a, y, ctx->n_cu, ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "qkv_rope_append launch");
        auto proj_view = [&](int64_t first_row, int64_t heads) {
            vva_tensor t{};
            t.data = y + first_row;
            t.type = VVA_TYPE_F32;
            t.ne[0] = d; t.ne[1] = heads; t.ne[2] = T; t.ne[3] = B;
            t.nb[0] = 4; t.nb[1] = 4 * d; t.nb[2] = 4 * (size_t)a.M; t.nb[3] = 4 * (size_t)a.M * T;
            return t;
        };
        const vva_tensor tq = proj_view(0, Hq), tk = proj_view(Hq * d, Hkv), tv = proj_view((Hq + Hkv) * d, Hkv);
        return vva_rope_append(ctx, kv, layer, &tq, &tk, &tv, pos, seq_ids, freq_base, q_out);
    }
    if ((st = run_proj_gemm(ctx, p, a, (int)N, (int)K, p.P)) != VVA_OK) return st;
    return VVA_OK;
}

extern "C" vva_status vva_qkv_proj(vva_context* ctx, const vva_tensor* x, const vva_tensor* wq, const vva_tensor* wk,
                                   const vva_tensor* wv, const vva_tensor* bq, const vva_tensor* bk,
                                   const vva_tensor* bv, const vva_tensor* y) {
    if (!ctx) return VVA_ERR_INVALID_ARG;
    vva_status st;
    if ((st = check_tensor(ctx, x, "x")) != VVA_OK) return st;
    if ((st = check_tensor(ctx, y, "y")) != VVA_OK) return st;
    if ((st = check_tensor(ctx, wq, "wq")) != VVA_OK) return st;
    if ((st = check_tensor(ctx, wk, "wk")) != VVA_OK) return st;
    if ((st = check_tensor(ctx, wv, "wv")) != VVA_OK) return st;
    const int64_t K = x->ne[0], T = x->ne[1], B = x->ne[2];
    const int64_t Mq = wq->ne[1], Mk = wk->ne[1], Mv = wv->ne[1], M = Mq + Mk + Mv;
    const int wt = wq->type;
    if (wt != VVA_TYPE_F16 && wt != VVA_TYPE_Q8_0)
        return fail(ctx, VVA_ERR_NOT_IMPLEMENTED, "qkv_proj: weights must be F16 or Q8_0");
    if (B < 1 || B > VVA_MAX_BATCH) return fail(ctx, VVA_ERR_INVALID_ARG, "qkv_proj: B must be 1..%d", VVA_MAX_BATCH);
    if (K % 64 || Mq % 64 || Mk % 64 || Mv % 64 || Mq < 64 || Mk < 64 || Mv < 64)
        return fail(ctx, VVA_ERR_NOT_IMPLEMENTED, "qkv_proj: needs hidden and the weights' output rows multiples of 64");
    if ((st = check_act(ctx, x, "x", K, T, B)) != VVA_OK) return st;
    if ((st = check_weight(ctx, wq, "wq", K, Mq, wt)) != VVA_OK) return st;
    if ((st = check_weight(ctx, wk, "wk", K, Mk, wt)) != VVA_OK) return st;
    if ((st = check_weight(ctx, wv, "wv", K, Mv, wt)) != VVA_OK) return st;
    if ((st = check_bias(ctx, bq, "bq", Mq)) != VVA_OK) return st;
    if ((st = check_bias(ctx, bk, "bk", Mk)) != VVA_OK) return st;
    if ((st = check_bias(ctx, bv, "bv", Mv)) != VVA_OK) return st;
    if (y->type != VVA_TYPE_F32 || y->ne[0] != M || y->ne[1] != T || y->ne[2] != B || y->ne[3] != 1 ||
        y->nb[0] != 4 || (int64_t)y->nb[1] != 4 * M || (int64_t)y->nb[2] != 4 * M * T)
        return fail(ctx, VVA_ERR_INVALID_ARG, "qkv_proj: y must be F32 ne=[%lld,%lld,%lld,1], contiguous", (long long)M,
                    (long long)T, (long long)B);
    const int64_t N = T * B;
    if (!proj_gemv_supported((int)N, (int)K, (int)M) || !rows16(x))
        return fail(ctx, VVA_ERR_NOT_IMPLEMENTED,
                    "qkv_proj: decode-sized calls only (at most 8 token rows of 16-byte aligned x; hidden <= 4096); "
                    "prefill chunks take vva_qkv_rope_append");
    ProjArgs a{};
    const vva_tensor* ws_[3] = {wq, wk, wv};
    const vva_tensor* bs_[3] = {bq, bk, bv};
    const int64_t rows[3] = {Mq, Mk, Mv};
    int64_t m_end = 0;
    for (int i = 0; i < 3; ++i) {
        a.w[i] = (const char*)ws_[i]->data;
        a.w_nb[i] = (int64_t)ws_[i]->nb[1];
        m_end += rows[i];
        a.m_end[i] = (int)m_end;
        a.bias[i] = bs_[i] ? (const float*)bs_[i]->data : nullptr;
    }
    a.w_type = wt;
    a.N = (int)N; a.K = (int)K; a.M = (int)M; a.T = (int)T;
    a.mode = kProjQKV;
    a.x = (const char*)x->data; a.x_type = x->type;
    a.x_nb_t = (int64_t)x->nb[1]; a.x_nb_b = (int64_t)x->nb[2];
    DeviceGuard g(ctx->device);
    const hipError_t e = launch_proj_gemv(a, (float*)y->data, ctx->n_cu, ctx->stream);
    return e == hipSuccess ? VVA_OK : hip_fail(ctx, e, "qkv_proj launch");
}

extern "C" vva_status vva_out_proj_residual(vva_context* ctx, const vva_tensor* o, const vva_tensor* w_o,
                                            const vva_tensor* x, const vva_tensor* h) {
    if (!ctx) return VVA_ERR_INVALID_ARG;
    vva_status st;
    if ((st = check_tensor(ctx, o, "o")) != VVA_OK) return st;
    if ((st = check_tensor(ctx, w_o, "w_o")) != VVA_OK) return st;
    if ((st = check_tensor(ctx, x, "x")) != VVA_OK) return st;
    if ((st = check_tensor(ctx, h, "h")) != VVA_OK) return st;
    const int64_t K = o->ne[0], T = o->ne[1], B = o->ne[2], M = w_o->ne[1];
    const int wt = w_o->type;
    if (wt != VVA_TYPE_F16 && wt != VVA_TYPE_Q8_0)
        return fail(ctx, VVA_ERR_NOT_IMPLEMENTED, "out_proj_residual: weights must be F16 or Q8_0");
    if (K % 64 || M % 128)
        return fail(ctx, VVA_ERR_NOT_IMPLEMENTED, "out_proj_residual: needs in %% 64 == 0 and out %% 128 == 0");
    if ((st = check_act(ctx, o, "o", K, T, B)) != VVA_OK) return st;
    if ((st = check_weight(ctx, w_o, "w_o", K, M, wt)) != VVA_OK) return st;
    if ((st = check_act(ctx, x, "x", M, T, B)) != VVA_OK) return st;
    if ((st = check_act(ctx, h, "h", M, T, B)) != VVA_OK) return st;
    if (x->type != VVA_TYPE_F32 || h->type != VVA_TYPE_F32)
        return fail(ctx, VVA_ERR_INVALID_ARG, "out_proj_residual: x and h must be F32");
    if ((uintptr_t)x->data % 16 || x->nb[1] % 16 || x->nb[2] % 16 || (uintptr_t)h->data % 16 || h->nb[1] % 16 ||
        h->nb[2] % 16)
        return fail(ctx, VVA_ERR_INVALID_ARG, "out_proj_residual: x and h rows must be 16-byte aligned");
    // h may alias x (the residual added in place), never o or the weights:
    // the few-row kernel reads every row of o in each workgroup while others
    // already write h
    if (overlaps(h, o) || overlaps(h, w_o))
        return fail(ctx, VVA_ERR_INVALID_ARG, "out_proj_residual: h overlaps o or w_o (only h == x may alias)");
    const int64_t N = T * B;
    if (N * K * 2 >= ((int64_t)1 << 31) || 128 * K * 2 >= ((int64_t)1 << 31))
        return fail(ctx, VVA_ERR_NOT_IMPLEMENTED, "out_proj_residual: %lld x %lld inputs exceed 2 GiB", (long long)N,
                    (long long)K);
    ProjArgs a{};
    a.w[0] = a.w[1] = a.w[2] = (const char*)w_o->data;
    a.w_nb[0] = a.w_nb[1] = a.w_nb[2] = (int64_t)w_o->nb[1];
    a.m_end[0] = a.m_end[1] = a.m_end[2] = (int)M;
    a.w_type = wt;
    a.N = (int)N; a.K = (int)K; a.M = (int)M;
    a.mode = kProjResidual;
    a.T = (int)T;
    a.res = (const char*)x->data; a.res_nb_t = (int64_t)x->nb[1]; a.res_nb_b = (int64_t)x->nb[2];
    a.h = (char*)h->data; a.h_nb_t = (int64_t)h->nb[1]; a.h_nb_b = (int64_t)h->nb[2];
    ProjPrepArgs p{};
    p.x = (const char*)o->data; p.x_type = o->type;
    p.x_nb_t = (int64_t)o->nb[1]; p.x_nb_b = (int64_t)o->nb[2];
    p.K = (int)K; p.T = (int)T; p.N = (int)N;
    p.q8 = wt == VVA_TYPE_Q8_0;
    p.P = 0;
    DeviceGuard g(ctx->device);
    hipError_t e;
    if (proj_gemv_supported((int)N, (int)K, (int)M) && rows16(o)) {
        a.x = p.x; a.x_type = p.x_type; a.x_nb_t = p.x_nb_t; a.x_nb_b = p.x_nb_b;
        e = launch_proj_gemv(a, nullptr, ctx->n_cu, ctx->stream);
        return e == hipSuccess ? VVA_OK : hip_fail(ctx, e, "out_proj_residual launch");
    }
    return run_proj_gemm(ctx, p, a, (int)N, (int)K, 0);
}

// --------------------------------------------------------- decode step

extern "C" vva_status vva_decode_step(vva_context* ctx, vva_kv* kv, int layer, const vva_tensor* q,
                                      const vva_tensor* k, const vva_tensor* v, const vva_tensor* pos,
                                      const int32_t* seq_ids, float freq_base, float scale, const vva_tensor* q_out,
                                      const vva_tensor* out) {
    if (!ctx) return VVA_ERR_INVALID_ARG;
    if (!kv || !kv_live(kv) || kv->ctx != ctx)
        return fail(ctx, VVA_ERR_INVALID_ARG, "decode_step: cache is null, released or of another context");
    if (layer < 0 || layer >= kv->desc.n_layers) return fail(ctx, VVA_ERR_INVALID_ARG, "decode_step: layer %d", layer);
    vva_status st = check_tensor(ctx, q, "q");
    if (st != VVA_OK) return st;
    const int64_t d = kv->desc.head_dim, Hkv = kv->desc.n_kv_heads;
    const int64_t Hq = q->ne[1], T = q->ne[2], B = q->ne[3];
    if (T != 1) return fail(ctx, VVA_ERR_INVALID_ARG, "decode_step: one new token per sequence (T = %lld)", (long long)T);
    if (Hq % Hkv) return fail(ctx, VVA_ERR_INVALID_ARG, "decode_step: Hq %% Hkv != 0");
    if (B > VVA_MAX_BATCH) return fail(ctx, VVA_ERR_INVALID_ARG, "decode_step: B > %d", VVA_MAX_BATCH);
    if ((st = check_rows(ctx, q, "q", d, Hq, 1, B)) != VVA_OK) return st;
    if ((st = check_rows(ctx, k, "k", d, Hkv, 1, B)) != VVA_OK) return st;
    if ((st = check_rows(ctx, v, "v", d, Hkv, 1, B)) != VVA_OK) return st;
    if ((st = check_rows(ctx, q_out, "q_out", d, Hq, 1, B)) != VVA_OK) return st;
    if ((st = check_rows(ctx, out, "out", d, Hq, 1, B)) != VVA_OK) return st;
    if (out->type != VVA_TYPE_F32) return fail(ctx, VVA_ERR_INVALID_ARG, "decode_step: out must be F32");
    int64_t ps = 0;
    if ((st = check_pos(ctx, pos, 1, B, &ps)) != VVA_OK) return st;
    StepArgs a{};
    for (int b = 0; b < B; ++b) {
        const int seq = seq_ids ? seq_ids[b] : b;
        if (seq < 0 || seq >= kv->desc.n_seq) return fail(ctx, VVA_ERR_INVALID_ARG, "decode_step: seq %d", seq);
        for (int b2 = 0; b2 < b; ++b2)
            if ((seq_ids ? seq_ids[b2] : b2) == seq)
                return fail(ctx, VVA_ERR_INVALID_ARG, "decode_step: sequence %d appears twice", seq);
        if (kv->len[seq] + 1 > kv->desc.max_seq)
            return fail(ctx, VVA_ERR_INVALID_ARG, "decode_step: seq %d is full (max_seq %d)", seq, kv->desc.max_seq);
        a.kc[b] = kv_tensor(kv, layer, seq, 0);
        a.vc[b] = kv_tensor(kv, layer, seq, 1);
        a.past[b] = kv->len[seq];
    }
    a.q = (const char*)q->data; a.q_type = q->type; a.q_nb_h = q->nb[1]; a.q_nb_b = q->nb[3];
    a.k = (const char*)k->data; a.k_type = k->type; a.k_nb_h = k->nb[1]; a.k_nb_b = k->nb[3];
    a.v = (const char*)v->data; a.v_type = v->type; a.v_nb_h = v->nb[1]; a.v_nb_b = v->nb[3];
    a.pos = (const int32_t*)pos->data; a.pos_stride_b = ps;
    a.q_out = (char*)q_out->data; a.q_out_type = q_out->type; a.qo_nb_h = q_out->nb[1]; a.qo_nb_b = q_out->nb[3];
    a.cache_row_bytes = kv->row_bytes; a.cache_head_bytes = kv->head_bytes; a.cache_type = kv->desc.type;
    a.theta_scale = powf(freq_base, -2.0f / (float)d);
    a.scale = scale;
    a.out = (float*)out->data; a.o_nb_h = out->nb[1]; a.o_nb_b = out->nb[3];
    a.tickets = ctx->tickets;
    a.d = (int)d; a.Hq = (int)Hq; a.Hkv = (int)Hkv; a.B = (int)B; a.G = (int)(Hq / Hkv);
    DeviceGuard g(ctx->device);
    // q_out aliasing q: every split reads q while split 0 writes q_out
    const bool alias = q_out->data == q->data;
    if (!alias && kv->desc.type == VVA_TYPE_Q8_0 && ctx->attn_path == 0) {
        // dense Q8_0 caches: the streamed decode kernel in step mode (RoPE of q,
        // the new row appended by the split that holds it), then its merge
        AttnArgs c{};
        for (int b = 0; b < B; ++b) {
            c.k[b] = a.kc[b];
            c.v[b] = a.vc[b];
            c.past[b] = a.past[b];
            c.L[b] = a.past[b] + 1;
        }
        c.q = a.q; c.q_type = a.q_type;
        c.q_nb_h = q->nb[1]; c.q_nb_t = q->nb[2]; c.q_nb_b = q->nb[3];
        c.k_nb_tok = c.v_nb_tok = kv->row_bytes;
        c.k_nb_head = c.v_nb_head = kv->head_bytes;
        c.k_type = c.v_type = VVA_TYPE_Q8_0;
        c.mask_mode = kMaskCausal;
        c.scale = scale;
        c.out = a.out; c.o_nb_h = out->nb[1]; c.o_nb_t = out->nb[2]; c.o_nb_b = out->nb[3];
        c.d = (int)d; c.Hq = (int)Hq; c.Hkv = (int)Hkv; c.T = 1; c.B = (int)B;
        // q_out rows are written 16 bytes at a time
        const bool qo_aligned = (uintptr_t)q_out->data % 16 == 0 && q_out->nb[1] % 16 == 0 && q_out->nb[3] % 16 == 0 &&
                                (int64_t)q_out->nb[0] == type_elem_bytes(q_out->type);
        if (qo_aligned && decode_stream_step_supported(c) && float_type(k->type) && float_type(v->type)) {
            StreamStep sp{};
            sp.k = a.k; sp.v = a.v; sp.k_type = a.k_type; sp.v_type = a.v_type;
            sp.k_nb_h = a.k_nb_h; sp.k_nb_b = a.k_nb_b; sp.v_nb_h = a.v_nb_h; sp.v_nb_b = a.v_nb_b;
            sp.pos = a.pos; sp.pos_stride_b = a.pos_stride_b;
            sp.theta_scale = a.theta_scale;
            sp.q_out = a.q_out; sp.q_out_type = a.q_out_type; sp.qo_nb_h = a.qo_nb_h; sp.qo_nb_b = a.qo_nb_b;
            const int wgs = ctx->sched_decode_wgs > 0 ? ctx->sched_decode_wgs : ctx->n_cu;
            int n_splits = decode_stream_plan(c, wgs);
            if (ctx->sched_decode_splits > 0) n_splits = ctx->sched_decode_splits;
            float* ws = nullptr;
            if (n_splits > 1) {
                if ((st = ensure_ws(ctx, (size_t)n_splits * B * Hq * (d + 2) * sizeof(float))) != VVA_OK) return st;
                ws = ctx->ws;
            }
            hipError_t e = launch_decode_stream_step(c, sp, ws, n_splits, ctx->stream);
            if (e != hipSuccess) return hip_fail(ctx, e, "decode_step launch");
            ctx->last_splits = n_splits;
            return VVA_OK;
        }
    }
    if (alias || !decode_step_supported(a)) {
        // the unfused path: RoPE + append, then attention (other cache types, longer windows)
        if ((st = vva_rope_append(ctx, kv, layer, q, k, v, pos, seq_ids, freq_base, q_out)) != VVA_OK) return st;
        return vva_attn(ctx, kv, layer, q_out, seq_ids, nullptr, scale, out);
    }
    const int n_splits = decode_step_splits(a);
    if (n_splits > 1) {
        if ((st = ensure_ws(ctx, (size_t)n_splits * B * Hq * (d + 2) * sizeof(float))) != VVA_OK) return st;
    }
    a.ws = ctx->ws;
    hipError_t e = launch_decode_step(a, n_splits, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "decode_step launch");
    ctx->last_splits = n_splits;
    return VVA_OK;
}
