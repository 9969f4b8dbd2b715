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
    const char* mask;                 // F16 rows (bytes strides)
    int64_t mask_nb_row, mask_nb_b;
    int mask_mode;                    // 0 none, 1 explicit, 2 causal
    float scale;
    float* out;
    int64_t o_nb_t, o_nb_h, o_nb_b;   // in bytes
    int d, Hq, Hkv, T, B;
};

enum { kMaskNone = 0, kMaskExplicit = 1, kMaskCausal = 2 };

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
// Key splits for one call (workgroups per sequence and head group); split s
// takes the sequence's tiles s, s + n_splits, s + 2 n_splits, ...
int decode_stream_plan(const AttnArgs& a, int n_cu);
hipError_t launch_decode_stream(const AttnArgs& a, float* ws, int n_splits, hipStream_t s);
// MFMA flash prefill (F16 / BF16 caches).  n_ks > 1 splits each row
// tile's keys over n_ks workgroups, with partials in ws
// (prefill_ws_bytes) merged by a second kernel.
hipError_t launch_prefill(const AttnArgs& a, float* ws, int n_ks, hipStream_t s);
bool prefill_supported(const AttnArgs& a);
int prefill_plan(const AttnArgs& a, int n_cu);
size_t prefill_ws_bytes(const AttnArgs& a, int n_ks);

}  // namespace vva

// ------------------------------------------------------- device helpers
#if defined(__HIPCC__)
namespace vva {

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
__device__ __forceinline__ float load_elem(const char* p, int type) {
    if (type == VVA_TYPE_F32) return *(const float*)p;
    uint16_t h = *(const uint16_t*)p;
    return type == VVA_TYPE_F16 ? f16_to_f32(h) : bf16_to_f32(h);
}
__device__ __forceinline__ void store_elem(char* p, int type, float f) {
    if (type == VVA_TYPE_F32) { *(float*)p = f; return; }
    *(uint16_t*)p = type == VVA_TYPE_F16 ? f32_to_f16(f) : f32_to_bf16(f);
}

}  // namespace vva
#endif
