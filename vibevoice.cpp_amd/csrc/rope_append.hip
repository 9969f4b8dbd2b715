// rope_append.hip — fused NeoX RoPE of Q and K plus the KV-cache append.
//
// Replaces, in one launch, the four ggml ops the reference builds per layer
// (src/qwen2.cpp:282-306): ggml_rope_ext on q, ggml_rope_ext on k (NeoX,
// src/rope.hpp:14-15), and the two ggml_cpy's of k and v into the resident
// cache views at row past_len.  The cache may be F32 / F16 / BF16 / Q8_0; the
// rotated Q is written in the attention's input type.
//
// Launch: one workgroup per (token t, batch b), 256 threads.  Threads
// 0..d/2-1 first build the angle table of the token in LDS with the fp32
// recurrence ggml's CPU rope cache uses (theta_0 = pos, theta_{i+1} =
// theta_i * base^(-2/d)); then every thread takes rotation pairs
// (x[i], x[i+d/2]) of the Hq q heads, the Hkv k heads and the Hkv v heads
// ("slots").  With d/2 a multiple of 32, each aligned group of 32 threads
// holds exactly two Q8_0 blocks of one head (elements i and i + d/2), so the
// block amax is a 32-lane butterfly and the codes are written without LDS.
//
// Memory: HBM-bound elementwise pass; per token it reads Hq+2*Hkv source rows
// and writes Hq rows of Q plus one K and one V cache row.
#include "vva_internal.hpp"

namespace vva {

namespace {

__global__ void __launch_bounds__(256) rope_append_kernel(RopeAppendArgs a, int items_per_block) {
    prefetch_kernargs<sizeof(RopeAppendArgs)>();
    const int t = blockIdx.x, b = blockIdx.y;
    const int P = a.d >> 1;
    __shared__ float cs[128], sn[128];
    const float p = (float)a.pos[b * a.pos_stride_b + t];
    for (int i = threadIdx.x; i < P; i += blockDim.x) {
        const float th = rope_theta(p, a.theta_scale, i, P);
        cs[i] = cosf(th);
        sn[i] = sinf(th);
    }
    __syncthreads();

    const int nq = a.do_q ? a.Hq : 0;
    const int nslots = nq + (a.do_kv ? 2 * a.Hkv : 0);
    // blockIdx.z takes a multiple-of-256 slice of the token's items, so few-token
    // calls (decode) still spread over many workgroups
    const int w_begin = blockIdx.z * items_per_block;
    const int total = min(nslots * P, w_begin + items_per_block);
    for (int w = w_begin + threadIdx.x; w < total; w += blockDim.x) {
        const int slot = w / P;
        const int i = w - slot * P;
        const float c = cs[i], s = sn[i];
        if (slot < nq) {
            const int64_t es = type_elem_bytes(a.q_type);
            const char* src = a.q + b * a.q_nb_b + t * a.q_nb_t + slot * a.q_nb_h;
            const float x0 = load_elem(src + i * es, a.q_type);
            const float x1 = load_elem(src + (i + P) * es, a.q_type);
            const float y0 = fmaf(x0, c, -(x1 * s));
            const float y1 = fmaf(x0, s, x1 * c);
            const int64_t eo = type_elem_bytes(a.q_out_type);
            char* dst = a.q_out + b * a.qo_nb_b + t * a.qo_nb_t + slot * a.qo_nb_h;
            store_elem(dst + i * eo, a.q_out_type, y0);
            store_elem(dst + (i + P) * eo, a.q_out_type, y1);
        } else {
            const int hs = slot - nq;
            const bool is_k = hs < a.Hkv;
            const int h = is_k ? hs : hs - a.Hkv;
            const int typ = is_k ? a.k_type : a.v_type;
            const int64_t es = type_elem_bytes(typ);
            const char* src = is_k ? a.k + b * a.k_nb_b + t * a.k_nb_t + h * a.k_nb_h
                                   : a.v + b * a.v_nb_b + t * a.v_nb_t + h * a.v_nb_h;
            const float x0 = load_elem(src + i * es, typ);
            const float x1 = load_elem(src + (i + P) * es, typ);
            float y0 = x0, y1 = x1;
            if (is_k) {
                y0 = fmaf(x0, c, -(x1 * s));
                y1 = fmaf(x0, s, x1 * c);
            }
            char* row = (is_k ? a.k_dst[b] : a.v_dst[b]) + t * a.cache_row_bytes + h * a.cache_head_bytes;
            if (a.cache_type == VVA_TYPE_Q8_0) {
                store_q8_pair(row, i, P, y0, y1);
            } else {
                const int64_t ec = type_elem_bytes(a.cache_type);
                store_elem(row + i * ec, a.cache_type, y0);
                store_elem(row + (i + P) * ec, a.cache_type, y1);
            }
        }
    }
}

// 8 consecutive elements (16-byte aligned) as fp32, and back.
__device__ __forceinline__ void load8(const char* p, int type, float (&x)[8]) {
    if (type == VVA_TYPE_F32) {
        const float4 u = ((const float4*)p)[0], v = ((const float4*)p)[1];
        x[0] = u.x; x[1] = u.y; x[2] = u.z; x[3] = u.w;
        x[4] = v.x; x[5] = v.y; x[6] = v.z; x[7] = v.w;
        return;
    }
    const uint4 u = *(const uint4*)p;
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint16_t lo = (uint16_t)(w[e] & 0xffffu), hi = (uint16_t)(w[e] >> 16);
        x[2 * e] = type == VVA_TYPE_F16 ? f16_to_f32(lo) : bf16_to_f32(lo);
        x[2 * e + 1] = type == VVA_TYPE_F16 ? f16_to_f32(hi) : bf16_to_f32(hi);
    }
}
__device__ __forceinline__ void store8(char* p, int type, const float (&y)[8]) {
    if (type == VVA_TYPE_F32) {
        ((float4*)p)[0] = make_float4(y[0], y[1], y[2], y[3]);
        ((float4*)p)[1] = make_float4(y[4], y[5], y[6], y[7]);
        return;
    }
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint16_t lo = type == VVA_TYPE_F16 ? f32_to_f16(y[2 * e]) : f32_to_bf16(y[2 * e]);
        const uint16_t hi = type == VVA_TYPE_F16 ? f32_to_f16(y[2 * e + 1]) : f32_to_bf16(y[2 * e + 1]);
        w[e] = (uint32_t)lo | ((uint32_t)hi << 16);
    }
    *(uint4*)p = make_uint4(w[0], w[1], w[2], w[3]);
}

constexpr int kRopeTokens = 8;         // tokens per workgroup of the vector path

// The same pass for 16-byte aligned rows and F32 / F16 / BF16 caches: a
// workgroup takes kRopeTokens tokens, a lane 8 rotation pairs (16-byte
// loads and stores of elements i .. i + 7 and i + P .. i + P + 7), with the
// angles from the same fp32 recurrence, so the results are the scalar
// kernel's bit for bit.
template <int P>
__global__ void __launch_bounds__(256) rope_append_vec_kernel(RopeAppendArgs a) {
    prefetch_kernargs<sizeof(RopeAppendArgs)>();
    constexpr int C = P / 8;                          // 8-pair chunks per row
    const int t0 = blockIdx.x * kRopeTokens, b = blockIdx.y;
    const int nt = min(kRopeTokens, a.T - t0);
    __shared__ float cs[kRopeTokens][P], sn[kRopeTokens][P];
    for (int k = threadIdx.x; k < nt * P; k += blockDim.x) {
        const int tl = k / P, i = k - tl * P;
        const float th = rope_theta((float)a.pos[b * a.pos_stride_b + t0 + tl], a.theta_scale, i, P);
        cs[tl][i] = cosf(th);
        sn[tl][i] = sinf(th);
    }
    __syncthreads();

    const int nq = a.do_q ? a.Hq : 0;
    const int per_tok = (nq + (a.do_kv ? 2 * a.Hkv : 0)) * C;
    for (int w = threadIdx.x; w < nt * per_tok; w += blockDim.x) {
        const int tl = w / per_tok, r = w - tl * per_tok;
        const int slot = r / C, i0 = (r - slot * C) * 8;
        const int t = t0 + tl;
        float c[8], sv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            c[e] = cs[tl][i0 + e];
            sv[e] = sn[tl][i0 + e];
        }
        float x0[8], x1[8], y0[8], y1[8];
        if (slot < nq) {
            const int64_t es = type_elem_bytes(a.q_type), eo = type_elem_bytes(a.q_out_type);
            const char* src = a.q + b * a.q_nb_b + t * a.q_nb_t + slot * a.q_nb_h;
            load8(src + i0 * es, a.q_type, x0);
            load8(src + (i0 + P) * es, a.q_type, x1);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                y0[e] = fmaf(x0[e], c[e], -(x1[e] * sv[e]));
                y1[e] = fmaf(x0[e], sv[e], x1[e] * c[e]);
            }
            char* dst = a.q_out + b * a.qo_nb_b + t * a.qo_nb_t + slot * a.qo_nb_h;
            store8(dst + i0 * eo, a.q_out_type, y0);
            store8(dst + (i0 + P) * eo, a.q_out_type, y1);
        } else {
            const int hs = slot - nq;
            const bool is_k = hs < a.Hkv;
            const int h = is_k ? hs : hs - a.Hkv;
            const int typ = is_k ? a.k_type : a.v_type;
            const int64_t es = type_elem_bytes(typ), ec = type_elem_bytes(a.cache_type);
            const char* src = is_k ? a.k + b * a.k_nb_b + t * a.k_nb_t + h * a.k_nb_h
                                   : a.v + b * a.v_nb_b + t * a.v_nb_t + h * a.v_nb_h;
            load8(src + i0 * es, typ, x0);
            load8(src + (i0 + P) * es, typ, x1);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                y0[e] = is_k ? fmaf(x0[e], c[e], -(x1[e] * sv[e])) : x0[e];
                y1[e] = is_k ? fmaf(x0[e], sv[e], x1[e] * c[e]) : x1[e];
            }
            char* row = (is_k ? a.k_dst[b] : a.v_dst[b]) + t * a.cache_row_bytes + h * a.cache_head_bytes;
            store8(row + i0 * ec, a.cache_type, y0);
            store8(row + (i0 + P) * ec, a.cache_type, y1);
        }
    }
}

bool rope_vec_ok(const RopeAppendArgs& a) {
    if (a.d != 64 && a.d != 128) return false;
    if (a.do_kv && a.cache_type == VVA_TYPE_Q8_0) return false;
    auto al = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    auto al64 = [](int64_t x) { return (x & 15) == 0; };
    if (a.do_q && (!al(a.q) || !al(a.q_out) || !al64(a.q_nb_h) || !al64(a.q_nb_t) || !al64(a.q_nb_b) ||
                   !al64(a.qo_nb_h) || !al64(a.qo_nb_t) || !al64(a.qo_nb_b)))
        return false;
    if (a.do_kv) {
        if (!al(a.k) || !al(a.v) || !al64(a.k_nb_h) || !al64(a.k_nb_t) || !al64(a.k_nb_b) || !al64(a.v_nb_h) ||
            !al64(a.v_nb_t) || !al64(a.v_nb_b) || !al64(a.cache_row_bytes) || !al64(a.cache_head_bytes))
            return false;
        for (int b = 0; b < a.B; ++b)
            if (!al(a.k_dst[b]) || !al(a.v_dst[b])) return false;
    }
    return true;
}

}  // namespace

hipError_t launch_rope_append(const RopeAppendArgs& a, hipStream_t s) {
    if (a.T <= 0 || a.B <= 0) return hipSuccess;
    const int items = ((a.do_q ? a.Hq : 0) + (a.do_kv ? 2 * a.Hkv : 0)) * (a.d / 2);
    if (items <= 0) return hipSuccess;
    // the vector path for many tokens; a few-token call (decode) is launch-
    // bound and spreads wider over the scalar kernel's item slices
    if ((int64_t)a.T * a.B >= 64 && rope_vec_ok(a)) {
        const dim3 grid((a.T + kRopeTokens - 1) / kRopeTokens, a.B);
        if (a.d == 64)
            hipLaunchKernelGGL(rope_append_vec_kernel<32>, grid, dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL(rope_append_vec_kernel<64>, grid, dim3(256), 0, s, a);
        return hipGetLastError();
    }
    int split = 1;
    if ((int64_t)a.T * a.B < 512) split = (items + 255) / 256;       // one item per thread
    const int per_block = ((items + split - 1) / split + 255) / 256 * 256;
    split = (items + per_block - 1) / per_block;
    dim3 grid(a.T, a.B, split);
    hipLaunchKernelGGL(rope_append_kernel, grid, dim3(256), 0, s, a, per_block);
    return hipGetLastError();
}

}  // namespace vva
