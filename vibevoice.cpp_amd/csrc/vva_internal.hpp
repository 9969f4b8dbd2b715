// vva_internal.hpp — shared definitions for the gfx950 attention kernels and
// the host-side C ABI implementation.  Not installed; include/vva.h is the
// public interface.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/vva.h"

namespace vva {

constexpr int kMaxBatch = VVA_MAX_BATCH;
constexpr int kQK8 = 32;          // values per Q8_0 block
constexpr int kQ8Bytes = 34;      // fp16 scale + 32 int8 codes

__host__ __device__ inline int64_t type_row_bytes(int type, int64_t n) {
    switch (type) {
        case VVA_TYPE_F32:  return 4 * n;
        case VVA_TYPE_F16:
        case VVA_TYPE_BF16: return 2 * n;
        case VVA_TYPE_Q8_0: return (n / kQK8) * kQ8Bytes;
        default:            return -1;
    }
}
__host__ __device__ inline int64_t type_elem_bytes(int type) {
    switch (type) {
        case VVA_TYPE_F32: case VVA_TYPE_I32: return 4;
        case VVA_TYPE_F16: case VVA_TYPE_BF16: return 2;
        case VVA_TYPE_Q8_0: return kQ8Bytes;
        default: return -1;
    }
}

// ------------------------------------------------------------ kernel args

// Fused RoPE + KV append.  Element (i, h, t, b) of a source lives at
// base + b*nb_b + t*nb_t + h*nb_h + i*elem_bytes.
struct RopeAppendArgs {
    const char* q; const char* k; const char* v;
    int q_type, k_type, v_type;
    int64_t q_nb_h, q_nb_t, q_nb_b;
    int64_t k_nb_h, k_nb_t, k_nb_b;
    int64_t v_nb_h, v_nb_t, v_nb_b;
    char* q_out; int q_out_type;
    int64_t qo_nb_h, qo_nb_t, qo_nb_b;
    const int32_t* pos; int64_t pos_stride_b;     // in elements; 0 = shared
    char* k_dst[kMaxBatch];                        // row 0 of this call's slots
    char* v_dst[kMaxBatch];
    int64_t cache_row_bytes, cache_head_bytes;
    int cache_type;
    int d, Hq, Hkv, T, B;
    int do_q, do_kv;                               // which parts to run
    float theta_scale;                             // powf(base, -2/d), computed on host
};

// Attention over per-batch K/V windows.  K row j, head h of batch b lives at
// k[b] + j*k_nb_tok + h*k_nb_head.  Query (b, t, h) at
// q + b*q_nb_b + t*q_nb_t + h*q_nb_h; output (b, t, h) row likewise in out.
struct AttnArgs {
    const char* q; int q_type;
    int64_t q_nb_t, q_nb_h, q_nb_b;
    const char* k[kMaxBatch];
    const char* v[kMaxBatch];
    int64_t k_nb_tok, k_nb_head, v_nb_tok, v_nb_head;
    int k_type, v_type;
    int L[kMaxBatch];
    int past[kMaxBatch];
    const char* mask;                 // F16 or F32 rows (bytes strides)
    int64_t mask_nb_row, mask_nb_b;
    int mask_mode;                    // 0 none, 1 explicit, 2 causal
    int mask_f32;                     // explicit mask rows are F32 (else F16)
    float scale;
    float* out;
    int64_t o_nb_t, o_nb_h, o_nb_b;   // in bytes
    int d, Hq, Hkv, T, B;
    int q_round_q8;                   // prefill: Q through a Q8_0 round trip first (window of Q8_0 K)
    // attn_rows kernels: when gate is set, run only if *gate == gate_epoch
    // (the device-side fallback of a Q8_0 window that overflowed f16)
    const unsigned long long* gate;
    unsigned long long gate_epoch;
};

enum { kMaskNone = 0, kMaskExplicit = 1, kMaskCausal = 2 };

// K / V rows [0, L_b) of each sequence converted to f16 for the MFMA
// prefill: Q8_0 blocks dequantized, F32 rounded (the reference's ggml_cast
// to F16 before flash attention, src/qwen2.cpp:328-331).  dst holds, per
// sequence, K then V as [L_b][Hkv][d] f16; window_f16_bytes sizes it.
size_t window_f16_bytes(const AttnArgs& a);
// ovf (may be null): set to epoch when a Q8_0 value exceeds the f16 range
// (its f16 is infinite), for the gated fallback through launch_attn_rows.
hipError_t launch_window_to_f16(const AttnArgs& a, void* dst, unsigned long long* ovf, unsigned long long epoch,
                                hipStream_t s);

// Single-token decode step in one launch (decode_step.hip): RoPE + append +
// split attention + in-kernel merge.  F16 / BF16 caches, len + 1 <=
// kMaxStepSplits * 128 keys, B * Hkv <= kMaxStepTickets.
constexpr int kMaxStepSplits = 64;
constexpr int kMaxStepTickets = 256;
struct StepArgs {
    const char* q; int q_type; int64_t q_nb_h, q_nb_b;    // ne = [d, Hq, 1, B]
    const char* k; int k_type; int64_t k_nb_h, k_nb_b;    // ne = [d, Hkv, 1, B]
    const char* v; int v_type; int64_t v_nb_h, v_nb_b;
    const int32_t* pos; int64_t pos_stride_b;
    char* q_out; int q_out_type; int64_t qo_nb_h, qo_nb_b;
    char* kc[kMaxBatch]; char* vc[kMaxBatch];              // row 0 of each sequence's K / V of the layer
    int64_t cache_row_bytes, cache_head_bytes; int cache_type;
    int past[kMaxBatch];                                   // the new row's index = len(seq_b)
    float theta_scale, scale;
    float* out; int64_t o_nb_h, o_nb_b;
    float* ws;                                             // split partials
    unsigned* tickets;                                     // [B * Hkv], zero between calls
    int d, Hq, Hkv, B;
    int G;                                                 // Hq / Hkv
};
bool decode_step_supported(const StepArgs& a);
int decode_step_splits(const StepArgs& a);
hipError_t launch_decode_step(const StepArgs& a, int n_splits, hipStream_t s);

// Linear layers around the attention (proj.hip).  Token row n = b * T + t.
// kProjQKVRope: the few-row GEMV of kProjQKV with the RoPE and the append in
// its epilogue (F32 / F16 / BF16 caches)
enum { kProjQKV = 0, kProjResidual = 1, kProjQKVRope = 2 };
struct ProjPrepArgs {
    const char* x; int x_type; int64_t x_nb_t, x_nb_b;   // rows of K elements (F32 / F16 / BF16)
    int K, T, N;
    int q8;                                              // Q8_0 round trip (Q8_0 weights)
    uint16_t* xh;                                        // out: f16 [N][K]
    const int32_t* pos; int64_t pos_stride_b;            // RoPE table (P > 0)
    int P; float theta_scale;
    float2* rope;                                        // out: [N][P] (cos, sin)
};
struct ProjArgs {
    const char* w[3];            // weight matrices stacked along the output rows
    int64_t w_nb[3];             // row stride in bytes
    int m_end[3];                // first row past matrix i (cumulative)
    const float* bias[3];        // F32 per output row, or null
    int w_type;                  // F16 or Q8_0
    const uint16_t* xh;          // the prep kernel's rows
    int N, K, M;
    int mode;
    // kProjQKV: rows [0, Hq d) are q, then k, then v
    const float2* rope;
    char* q_out; int q_out_type; int64_t qo_nb_h, qo_nb_t, qo_nb_b;
    char* k_dst[kMaxBatch]; char* v_dst[kMaxBatch];      // row 0 of this call's cache slots
    int64_t cache_row_bytes, cache_head_bytes; int cache_type;
    int d, Hq, Hkv, T;
    // kProjResidual: h = y + res (F32 rows; may alias)
    const char* res; int64_t res_nb_t, res_nb_b;
    char* h; int64_t h_nb_t, h_nb_b;
    // few-row path: the token rows themselves (converted in each workgroup),
    // and, for kProjQKV, the projections y = x w^T + bias as F32 [N][M]
    const char* x; int x_type; int64_t x_nb_t, x_nb_b;
    float* y;
    // GEMM split along K (ksplit > 1): every piece stores its accumulators in
    // `part`, the last piece of a tile (ticket) sums them and runs the epilogue
    int ksplit;
    int tail0;                                             // > 0: only the tiles from this place of the order on are split
    char* part;
    unsigned* tickets;                                     // [split tiles], zero between calls
    // kProjQKV: q_out and cache rows take 8-element vector stores (F32 / F16 /
    // BF16 destinations, 16-byte aligned rows); else one element per lane
    int vec_store;
    // kProjQKVRope: the positions of the token rows and powf(base, -2 / d)
    const int32_t* pos; int64_t pos_stride_b;
    float theta_scale;
};
constexpr int kMaxProjTickets = 1024;
// K split of the GEMM of a call (1: none; *tail0 > 0: only the last round's
// tiles) and the bytes of its partials
int proj_ksplit(const ProjArgs& a, int n_cu, int* tail0);
size_t proj_part_bytes(const ProjArgs& a);

// --------------------------------------------------------- host launchers

hipError_t launch_rope_append(const RopeAppendArgs& a, hipStream_t s);
hipError_t launch_attn_rows(const AttnArgs& a, hipStream_t s);
// Split-K decode (T == 1): workgroups write partials into `ws`
// (B * Hq * n_splits * (d + 2) floats), a second launch combines them.
hipError_t launch_decode(const AttnArgs& a, float* ws, int n_splits, int split_len, hipStream_t s);
bool decode_supported(const AttnArgs& a);
int decode_waves(const AttnArgs& a);            // waves per workgroup (one key sub-range each)
int decode_max_splits();
// Second pass of a split decode: combines the (m, l, acc) partials of `ws`
// (layout of launch_decode) into the output rows.
hipError_t launch_decode_merge(const AttnArgs& a, const float* ws, int n_splits, hipStream_t s);
// LDS-streamed split-K decode over dense Q8_0 caches (T == 1): the cache
// tiles of each split are DMA'd into a 4-stage LDS ring.  Partials use the
// layout of launch_decode and are combined by launch_decode_merge.
bool decode_stream_supported(const AttnArgs& a);
// vva_decode_step on dense Q8_0 caches: AttnArgs::q is the raw q (not yet
// RoPE'd) and L_b = len(seq_b) + 1; the streamed decode kernel applies the
// RoPE to q itself (writing q_out), and the split that holds key len(seq_b)
// appends the new row: RoPE(k) and v quantized to Q8_0 blocks, to the cache
// and into its own tile.
struct StreamStep {
    const char* k; const char* v;
    int k_type, v_type;
    int64_t k_nb_h, k_nb_b, v_nb_h, v_nb_b;
    const int32_t* pos; int64_t pos_stride_b;
    float theta_scale;
    char* q_out; int q_out_type; int64_t qo_nb_h, qo_nb_b;
};
bool decode_stream_step_supported(const AttnArgs& a);
hipError_t launch_decode_stream_step(const AttnArgs& a, const StreamStep& st, float* ws, int n_splits, hipStream_t s);
// Key splits for one call (workgroups per sequence and head group); split s
// takes the sequence's tiles s, s + n_splits, s + 2 n_splits, ...
int decode_stream_plan(const AttnArgs& a, int n_cu);
hipError_t launch_decode_stream(const AttnArgs& a, float* ws, int n_splits, hipStream_t s);
// MFMA flash prefill (F16 / BF16 caches).  Row tiles (256 query rows of
// one kv group) rt >= R have their key range split over n workgroups (all
// row tiles over `forced` when forced > 0); split rows leave partials in ws
// (prefill_ws_bytes) that the last split of the row tile merges inside the
// launch (in_launch, at most kMaxInLaunchSplits splits) or a second kernel
// merges.
struct PrefillPlan {
    int n;             // splits of a heavy row tile (1: none)
    int R;             // first heavy row tile
    int forced;        // > 0: this many splits for every row tile
    int max_ks;        // largest split count of the call (1: no partials)
    int in_launch;     // 1: the last split of a row tile merges (tickets), no merge kernel
};
// Row-tile tickets of the in-launch merge: B * Hkv * row tiles of them,
// zero between calls (the last split of a row tile resets its ticket).
constexpr int kMaxPrefillTickets = 16384;
constexpr int kMaxInLaunchSplits = 4;
// whether plan p may merge in the launch (split count, ticket count)
bool prefill_in_launch_ok(const AttnArgs& a, const PrefillPlan& p);
hipError_t launch_prefill(const AttnArgs& a, float* ws, unsigned* tickets, const PrefillPlan& p, hipStream_t s);
bool prefill_supported(const AttnArgs& a);
// allow_in_launch: the caller passes the tickets (otherwise the merge kernel)
PrefillPlan prefill_plan(const AttnArgs& a, int n_cu, int forced, size_t ws_cap, bool allow_in_launch);
size_t prefill_ws_bytes(const AttnArgs& a, const PrefillPlan& p);
// Prep + GEMM of a linear layer; ws holds proj_ws_bytes(N, K, P) bytes.
size_t proj_ws_bytes(int N, int K, int P);
// Q8_0 weights over a long call (>= 1024 token rows): the rows are
// dequantized to f16 d * q (M x K) for the F16 GEMM
bool proj_dequant_q8(const ProjArgs& a);
hipError_t launch_proj_dequant_q8(const ProjArgs& a, uint16_t* dst, hipStream_t s);
hipError_t launch_proj(ProjPrepArgs& p, ProjArgs& a, void* ws, hipStream_t s);
// Few token rows (decode steps): one weight-streaming GEMV launch that
// converts the rows itself.  kProjQKV writes y = x w^T + bias (F32 [N][M],
// at `ws`) for the caller's RoPE + append; kProjResidual writes h.
bool proj_gemv_supported(int N, int K, int M);
hipError_t launch_proj_gemv(ProjArgs& a, float* y_ws, int n_cu, hipStream_t s);
// Whether launch_proj_gemv can run a kProjQKV call as kProjQKVRope (one
// launch: projections, bias, RoPE and the append of F32 / F16 / BF16 rows).
bool proj_gemv_rope_ok(const ProjArgs& a);

}  // namespace vva

// ------------------------------------------------------- device helpers
#if defined(__HIPCC__)
namespace vva {

// Loads one dword of every 64-byte line of the first BYTES bytes of the
// kernel-argument segment (BYTES = the explicit arguments' size, so every
// load is inside the segment), then waits once.  The scalar data cache starts
// cold at each launch, and the compiler reads argument fields where they are
// first needed, several dependent round trips apart; after this they hit.
// One asm block (loads, then the wait), so the scratch register it writes is
// the block's own until every load has returned.
template <int BYTES>
__device__ __forceinline__ void prefetch_kernargs() {
    const char* p = (const char*)__builtin_amdgcn_kernarg_segment_ptr();
    uint32_t x;
    asm volatile(".set .Lvva_ka_off, 0\n\t"
                 ".rept %2\n\t"
                 "s_load_dword %0, %1, .Lvva_ka_off\n\t"
                 ".set .Lvva_ka_off, .Lvva_ka_off + 64\n\t"
                 ".endr\n\t"
                 "s_waitcnt lgkmcnt(0)"
                 : "=&s"(x)
                 : "s"(p), "n"((BYTES + 63) / 64)
                 : "memory");
}

// Angle of rotation pair i at position p: p * ts * ts * ... with i products,
// each rounded to fp32 (ggml's rope-cache recurrence).  Every lane runs the
// same n - 1 steps and keeps its i-th product, so a wave does not run its
// lanes' different trip counts one after another; the products, and so the
// result, are those of the plain loop.
__device__ __forceinline__ float rope_theta(float p, float ts, int i, int n) {
    float th = p;
    for (int k = 0; k < n - 1; ++k) th = k < i ? th * ts : th;
    return th;
}
// The same for a pair count NP known at compile time: straight-line code
template <int NP>
__device__ __forceinline__ float rope_theta_n(float p, float ts, int i) {
    float th = p;
#pragma unroll
    for (int k = 0; k < NP - 1; ++k) th = k < i ? th * ts : th;
    return th;
}

// 64-bit agent-scope stores and loads of float pairs: coherent across the
// XCDs' L2 caches without an L2 write-back or invalidate (split partials
// handed from one workgroup to another within a launch)
__device__ __forceinline__ void store_coherent2(float* p, float x, float y) {
    const uint64_t v = (uint64_t)__float_as_uint(x) | ((uint64_t)__float_as_uint(y) << 32);
    __hip_atomic_store((uint64_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 load_coherent2(const float* p) {
    const uint64_t v = __hip_atomic_load((uint64_t*)const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_float2(__uint_as_float((uint32_t)v), __uint_as_float((uint32_t)(v >> 32)));
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    _Float16 v; __builtin_memcpy(&v, &h, 2); return (float)v;
}
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
    _Float16 v = (_Float16)f; uint16_t h; __builtin_memcpy(&h, &v, 2); return h;
}
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float((uint32_t)h << 16);
}
// round to nearest even; NaN kept quiet
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t x = __float_as_uint(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    return (uint16_t)((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
}
// value -> value as rounded to `type` and back (Q8_0 not handled here)
__device__ __forceinline__ float round_to_type(float f, int type) {
    if (type == VVA_TYPE_F16) return f16_to_f32(f32_to_f16(f));
    if (type == VVA_TYPE_BF16) return bf16_to_f32(f32_to_bf16(f));
    return f;
}
// element j of an explicit mask row (F32 or F16; -inf = masked)
__device__ __forceinline__ float mask_at(const char* mrow, int64_t j, int f32) {
    return f32 ? ((const float*)mrow)[j] : f16_to_f32(((const uint16_t*)mrow)[j]);
}
__device__ __forceinline__ float load_elem(const char* p, int type) {
    if (type == VVA_TYPE_F32) return *(const float*)p;
    uint16_t h = *(const uint16_t*)p;
    return type == VVA_TYPE_F16 ? f16_to_f32(h) : bf16_to_f32(h);
}
__device__ __forceinline__ void store_elem(char* p, int type, float f) {
    if (type == VVA_TYPE_F32) { *(float*)p = f; return; }
    *(uint16_t*)p = type == VVA_TYPE_F16 ? f32_to_f16(f) : f32_to_bf16(f);
}

// Q8_0 store of a NeoX rotation pair: elements i (block i/32) and i + P
// (block (i+P)/32) of one head row.  Called by the 32 lanes of an aligned
// group holding i = 32k .. 32k + 31, which cover both blocks completely, so
// each block's amax is a 32-lane butterfly.  GGUF rule: d = amax / 127 (fp16),
// codes round(x / d) with the fp32 d.
__device__ __forceinline__ void store_q8_pair(char* row, int i, int P, float y0, float y1) {
    float a0 = fabsf(y0), a1 = fabsf(y1);
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) {
        a0 = fmaxf(a0, __shfl_xor(a0, m, 32));
        a1 = fmaxf(a1, __shfl_xor(a1, m, 32));
    }
    const float d0 = a0 / 127.0f, d1 = a1 / 127.0f;
    const float id0 = d0 != 0.0f ? 1.0f / d0 : 0.0f;
    const float id1 = d1 != 0.0f ? 1.0f / d1 : 0.0f;
    const int j0 = i, j1 = i + P;
    char* b0 = row + (j0 / kQK8) * kQ8Bytes;
    char* b1 = row + (j1 / kQK8) * kQ8Bytes;
    if ((j0 & (kQK8 - 1)) == 0) {
        *(uint16_t*)b0 = f32_to_f16(d0);
        *(uint16_t*)b1 = f32_to_f16(d1);
    }
    b0[2 + (j0 & (kQK8 - 1))] = (char)(int8_t)roundf(y0 * id0);
    b1[2 + (j1 & (kQK8 - 1))] = (char)(int8_t)roundf(y1 * id1);
}

}  // namespace vva
#endif
