// attn_rows.hip — VALU attention, one wavefront per query row.
//
// Covers every combination the MFMA prefill and split-K decode kernels do
// not: F32 caches (the eager mul_mat -> soft_max_ext -> mul_mat branch,
// src/qwen2.cpp:337-343, computed in fp32 throughout), Q8_0 caches with more
// than one new token, and explicit masks of any shape.  Semantics follow
// ggml's flash_attn_ext (src/qwen2.cpp:332-334): Q rounded to K's dot type
// (F16 -> f16, BF16 -> bf16, Q8_0 -> Q8_0 blocks with integer dots), scores
// scaled then masked, fp32 online softmax, fp32 V accumulation, rows with no
// visible key produce 0.
//
// Mapping: lane l owns dims l, l+64, ... (DPL = d/64 rounded up per lane);
// each key's dot is a 64-lane butterfly sum.  Keys are taken four at a time
// so four butterflies are in flight.  Latency-oriented: it serves the small
// shapes (0.5B prefill of 256 tokens, chunk tails) rather than the roofline
// configurations.
#include "vva_internal.hpp"

namespace vva {

namespace {

#include "wave_ops.hpp"

constexpr int kRowsPerBlock = 4;   // one row per wave

template <int DPL>
__global__ void __launch_bounds__(256) attn_rows_kernel(AttnArgs a) {
    prefetch_kernargs<sizeof(AttnArgs)>();
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= a.B * a.T * a.Hq) return;        // whole wave leaves together
    const int h = row % a.Hq;
    const int bt = row / a.Hq;
    const int t = bt % a.T;
    const int b = bt / a.T;
    const int kvh = h / (a.Hq / a.Hkv);
    const int d = a.d;

    // ---- query, rounded to K's dot type
    const int64_t qes = type_elem_bytes(a.q_type);
    const char* qrow = a.q + b * a.q_nb_b + t * a.q_nb_t + h * a.q_nb_h;
    float q[DPL];
    float qs[DPL];          // Q8_0: per-lane block scale of q
#pragma unroll
    for (int r = 0; r < DPL; ++r) {
        const int i = lane + 64 * r;
        q[r] = i < d ? load_elem(qrow + i * qes, a.q_type) : 0.0f;
        qs[r] = 0.0f;
    }
    const bool k_q8 = a.k_type == VVA_TYPE_Q8_0;
    if (k_q8) {
#pragma unroll
        for (int r = 0; r < DPL; ++r) {
            // lanes 0-31 / 32-63 hold blocks 2r / 2r+1 of the row
            float am = fabsf(q[r]);
#pragma unroll
            for (int m = 16; m >= 1; m >>= 1) am = fmaxf(am, __shfl_xor(am, m, 32));
            const float dq = am / 127.0f;
            const float id = dq != 0.0f ? 1.0f / dq : 0.0f;
            q[r] = roundf(q[r] * id);              // integer code, exact in f32
            qs[r] = f16_to_f32(f32_to_f16(dq));
        }
    } else {
#pragma unroll
        for (int r = 0; r < DPL; ++r) q[r] = round_to_type(q[r], a.k_type);
    }

    // ---- visible window
    const int L = a.L[b];
    int jend = L;
    if (a.mask_mode == kMaskCausal) jend = min(L, a.past[b] + t + 1);
    const char* kbase = a.k[b] + kvh * a.k_nb_head;
    const char* vbase = a.v[b] + kvh * a.v_nb_head;
    const char* mrow = a.mask ? a.mask + b * a.mask_nb_b + t * a.mask_nb_row : nullptr;
    const int64_t kes = type_elem_bytes(a.k_type), ves = type_elem_bytes(a.v_type);

    float M = -INFINITY, S = 0.0f;
    float acc[DPL];
#pragma unroll
    for (int r = 0; r < DPL; ++r) acc[r] = 0.0f;

    for (int j0 = 0; j0 < jend; j0 += 4) {
        float part[4];
        float mv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int j = j0 + u;
            part[u] = 0.0f;
            mv[u] = -INFINITY;
            if (j < jend) {
                mv[u] = (a.mask_mode == kMaskExplicit)
                            ? mask_at(mrow, j, a.mask_f32) : 0.0f;
                const char* kr = kbase + (int64_t)j * a.k_nb_tok;
#pragma unroll
                for (int r = 0; r < DPL; ++r) {
                    const int i = lane + 64 * r;
                    if (i < d) {
                        if (k_q8) {
                            const char* blk = kr + (i / kQK8) * kQ8Bytes;
                            const float dk = f16_to_f32(*(const uint16_t*)blk);
                            const float ck = (float)(int8_t)blk[2 + (i & (kQK8 - 1))];
                            part[u] = fmaf(q[r] * ck, dk * qs[r], part[u]);
                        } else {
                            part[u] = fmaf(q[r], load_elem(kr + i * kes, a.k_type), part[u]);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
#pragma unroll
            for (int u = 0; u < 4; ++u) part[u] += __shfl_xor(part[u], m, 64);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (mv[u] == -INFINITY) continue;         // masked / past the window
            const int j = j0 + u;
            const float s = part[u] * a.scale + mv[u];
            float ms = 1.0f, vs = 1.0f;
            if (s > M) { ms = __expf(M - s); M = s; }   // exp(-inf) = 0 on the first key
            else       { vs = __expf(s - M); }
            const char* vr = vbase + (int64_t)j * a.v_nb_tok;
#pragma unroll
            for (int r = 0; r < DPL; ++r) {
                const int i = lane + 64 * r;
                float vv = 0.0f;
                if (i < d) {
                    if (a.v_type == VVA_TYPE_Q8_0) {
                        const char* blk = vr + (i / kQK8) * kQ8Bytes;
                        vv = (float)(int8_t)blk[2 + (i & (kQK8 - 1))] * f16_to_f32(*(const uint16_t*)blk);
                    } else {
                        vv = load_elem(vr + i * ves, a.v_type);
                    }
                }
                acc[r] = fmaf(vv, vs, acc[r] * ms);
            }
            S = S * ms + vs;
        }
    }
    const float inv = S == 0.0f ? 0.0f : 1.0f / S;
    float* orow = (float*)((char*)a.out + b * a.o_nb_b + t * a.o_nb_t + h * a.o_nb_h);
#pragma unroll
    for (int r = 0; r < DPL; ++r) {
        const int i = lane + 64 * r;
        if (i < d) orow[i] = acc[r] * inv;
    }
}

// Max over all 64 lanes (every lane gets it).
__device__ __forceinline__ float wave_max(float x) {
    x = fmaxf(x, dpp<kDppXor1>(x));
    x = fmaxf(x, dpp<kDppXor2>(x));
    x = fmaxf(x, dpp<kDppHalfMirror>(x));
    x = fmaxf(x, dpp<kDppMirror>(x));
    x = max_swap16(x);
    return max_swap32(x);
}

// F32 K and V (the eager branch, src/qwen2.cpp:337-343, in fp32): one wave
// per query row, keys 64 at a time.  Lane l computes the whole dot product
// of key j0 + l (16-byte loads of its K row against Q broadcast from LDS),
// so no cross-lane sum per key; the 64 scores then take one online-softmax
// step (max and sum over the wave), and P.V runs with lane l owning dims
// l, l + 64, ... over the 64 keys (V rows read whole by the wave, p
// broadcast from LDS).  Same semantics as attn_rows_kernel: scores scaled
// then masked, keys at -inf skipped, a row with no visible key gives 0.
// D > 0: head_dim known at compile time, so that the K row's loads go out
// together and the V rows come in batches of kVBatch keys (the products and
// their order are those of the D = 0 form, which loads as it goes).
constexpr int kVBatch = 16;
template <int DPL, int D>
__global__ void __launch_bounds__(256) attn_rows_f32_kernel(AttnArgs a) {
    prefetch_kernargs<sizeof(AttnArgs)>();
    __shared__ __attribute__((aligned(16))) float qsh[kRowsPerBlock][256];
    __shared__ __attribute__((aligned(16))) float psh[kRowsPerBlock][64];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int row = blockIdx.x * kRowsPerBlock + wv;
    if (row >= a.B * a.T * a.Hq) return;        // whole wave leaves together
    const int h = row % a.Hq;
    const int bt = row / a.Hq;
    const int t = bt % a.T;
    const int b = bt / a.T;
    const int kvh = h / (a.Hq / a.Hkv);
    const int d = D > 0 ? D : a.d;

    const int64_t qes = type_elem_bytes(a.q_type);
    const char* qrow = a.q + b * a.q_nb_b + t * a.q_nb_t + h * a.q_nb_h;
#pragma unroll
    for (int r = 0; r < DPL; ++r) {
        const int i = lane + 64 * r;
        if (i < d) qsh[wv][i] = load_elem(qrow + i * qes, a.q_type);
    }
    wave_lds_sync();

    const int L = a.L[b];
    int jend = L;
    if (a.mask_mode == kMaskCausal) jend = min(L, a.past[b] + t + 1);
    const char* kbase = a.k[b] + kvh * a.k_nb_head;
    const char* vbase = a.v[b] + kvh * a.v_nb_head;
    const char* mrow = a.mask ? a.mask + b * a.mask_nb_b + t * a.mask_nb_row : nullptr;

    float M = -INFINITY, S = 0.0f;
    float acc[DPL];
#pragma unroll
    for (int r = 0; r < DPL; ++r) acc[r] = 0.0f;

    for (int j0 = 0; j0 < jend; j0 += 64) {
        const int j = j0 + lane;
        const bool live = j < jend;
        const float4* kr = (const float4*)(kbase + (int64_t)(live ? j : j0) * a.k_nb_tok);
        float dot0 = 0.0f, dot1 = 0.0f;
        // D = 64: the 64 keys' V values of the lane's dim load beside K (rows
        // past the last visible key repeat it: their p is 0)
        constexpr int VA = D == 64 ? 64 : 1;
        float va[VA];
        if constexpr (D > 0) {
            float4 kv[D / 4];
#pragma unroll
            for (int i4 = 0; i4 < D / 4; ++i4) kv[i4] = kr[i4];
            if constexpr (D == 64) {
                const int last = min(64, jend - j0) - 1;
                const char* vr0 = vbase + (int64_t)j0 * a.v_nb_tok;
#pragma unroll
                for (int u = 0; u < 64; ++u) va[u] = *((const float*)(vr0 + (int64_t)min(u, last) * a.v_nb_tok) + lane);
            }
#pragma unroll
            for (int i4 = 0; i4 < D / 4; i4 += 2) {
                const float4 q0 = *(const float4*)&qsh[wv][4 * i4];
                dot0 = fmaf(q0.x, kv[i4].x, dot0); dot0 = fmaf(q0.y, kv[i4].y, dot0);
                dot0 = fmaf(q0.z, kv[i4].z, dot0); dot0 = fmaf(q0.w, kv[i4].w, dot0);
                if (i4 + 1 < D / 4) {
                    const float4 q1 = *(const float4*)&qsh[wv][4 * i4 + 4];
                    dot1 = fmaf(q1.x, kv[i4 + 1].x, dot1); dot1 = fmaf(q1.y, kv[i4 + 1].y, dot1);
                    dot1 = fmaf(q1.z, kv[i4 + 1].z, dot1); dot1 = fmaf(q1.w, kv[i4 + 1].w, dot1);
                }
            }
        } else {
            for (int i4 = 0; i4 < d / 4; i4 += 2) {
                const float4 k0 = kr[i4], q0 = *(const float4*)&qsh[wv][4 * i4];
                dot0 = fmaf(q0.x, k0.x, dot0); dot0 = fmaf(q0.y, k0.y, dot0);
                dot0 = fmaf(q0.z, k0.z, dot0); dot0 = fmaf(q0.w, k0.w, dot0);
                if (i4 + 1 < d / 4) {
                    const float4 k1 = kr[i4 + 1], q1 = *(const float4*)&qsh[wv][4 * i4 + 4];
                    dot1 = fmaf(q1.x, k1.x, dot1); dot1 = fmaf(q1.y, k1.y, dot1);
                    dot1 = fmaf(q1.z, k1.z, dot1); dot1 = fmaf(q1.w, k1.w, dot1);
                }
            }
        }
        float sc = -INFINITY;
        if (live) {
            const float mv = (a.mask_mode == kMaskExplicit) ? mask_at(mrow, j, a.mask_f32) : 0.0f;
            sc = mv == -INFINITY ? -INFINITY : (dot0 + dot1) * a.scale + mv;
        }
        const float mx = wave_max(sc);
        if (mx == -INFINITY) continue;              // nothing visible in these 64 keys (uniform)
        const float Mn = fmaxf(M, mx);
        const float alpha = __expf(M - Mn);         // 0 while M = -inf
        const float p = sc == -INFINITY ? 0.0f : __expf(sc - Mn);
        S = fmaf(S, alpha, wave_sum(p));
#pragma unroll
        for (int r = 0; r < DPL; ++r) acc[r] *= alpha;
        M = Mn;
        psh[wv][lane] = p;
        wave_lds_sync();
        const int nk = min(64, jend - j0);
        const char* vr = vbase + (int64_t)j0 * a.v_nb_tok;
        int u = 0;
        if constexpr (D == 64) {
            // every key of the step (p = 0 past nk: acc is unchanged)
#pragma unroll
            for (int e = 0; e < 64; e += 4) {
                const float4 pu = *(const float4*)&psh[wv][e];
                acc[0] = fmaf(pu.x, va[e], acc[0]);
                acc[0] = fmaf(pu.y, va[e + 1], acc[0]);
                acc[0] = fmaf(pu.z, va[e + 2], acc[0]);
                acc[0] = fmaf(pu.w, va[e + 3], acc[0]);
            }
            u = nk;
        } else if constexpr (D > 0) {
            // kVBatch keys' V values of the lane's dims loaded together, then
            // summed in key order
            for (; u + kVBatch <= nk; u += kVBatch) {
                float vv[kVBatch][DPL];
#pragma unroll
                for (int e = 0; e < kVBatch; ++e)
#pragma unroll
                    for (int r = 0; r < DPL; ++r)
                        vv[e][r] = lane + 64 * r < D ? *((const float*)(vr + (int64_t)(u + e) * a.v_nb_tok) + lane + 64 * r) : 0.0f;
#pragma unroll
                for (int e = 0; e < kVBatch; e += 4) {
                    const float4 pu = *(const float4*)&psh[wv][u + e];
#pragma unroll
                    for (int r = 0; r < DPL; ++r) {
                        acc[r] = fmaf(pu.x, vv[e][r], acc[r]);
                        acc[r] = fmaf(pu.y, vv[e + 1][r], acc[r]);
                        acc[r] = fmaf(pu.z, vv[e + 2][r], acc[r]);
                        acc[r] = fmaf(pu.w, vv[e + 3][r], acc[r]);
                    }
                }
            }
        }
        for (; u + 4 <= nk; u += 4) {
            const float4 pu = *(const float4*)&psh[wv][u];
#pragma unroll
            for (int r = 0; r < DPL; ++r) {
                const int i = lane + 64 * r;
                if (i < d) {
                    const float* vc = (const float*)(vr + (int64_t)u * a.v_nb_tok) + i;
                    const float v0 = vc[0];
                    const float v1 = *(const float*)((const char*)vc + a.v_nb_tok);
                    const float v2 = *(const float*)((const char*)vc + 2 * a.v_nb_tok);
                    const float v3 = *(const float*)((const char*)vc + 3 * a.v_nb_tok);
                    acc[r] = fmaf(pu.x, v0, acc[r]);
                    acc[r] = fmaf(pu.y, v1, acc[r]);
                    acc[r] = fmaf(pu.z, v2, acc[r]);
                    acc[r] = fmaf(pu.w, v3, acc[r]);
                }
            }
        }
        for (; u < nk; ++u) {
            const float pu = psh[wv][u];
#pragma unroll
            for (int r = 0; r < DPL; ++r) {
                const int i = lane + 64 * r;
                if (i < d) acc[r] = fmaf(pu, *((const float*)(vr + (int64_t)u * a.v_nb_tok) + i), acc[r]);
            }
        }
        wave_lds_sync();                            // psh is rewritten by the next step
    }
    const float inv = S == 0.0f ? 0.0f : 1.0f / S;
    float* orow = (float*)((char*)a.out + b * a.o_nb_b + t * a.o_nb_t + h * a.o_nb_h);
#pragma unroll
    for (int r = 0; r < DPL; ++r) {
        const int i = lane + 64 * r;
        if (i < d) orow[i] = acc[r] * inv;
    }
}

// F32 K and V, the query heads of one kv head together (GQA): one workgroup
// per (sequence, token, kv head), four waves.  Wave w takes the 64-key steps
// w, w + 4, ... of the row's visible keys: lane l loads key j0 + l's K row
// once and scores it against all G query heads (Q from LDS), each head takes
// its online-softmax step (max and sum over the wave), and P.V runs with lane
// l owning dims l, l + 64, ... (the 64 keys' V values loaded together, p
// broadcast from LDS).  The waves' (max, sum, accumulator) per head are then
// combined through LDS.  K and V are read once per token and kv head instead
// of once per query head.  Same semantics as attn_rows_f32_kernel.
constexpr int kGqaWaves = 4;
constexpr int kGqaMaxG = 8;
template <int D>
__global__ void __launch_bounds__(64 * kGqaWaves) attn_gqa_f32_kernel(AttnArgs a) {
    prefetch_kernargs<sizeof(AttnArgs)>();
    constexpr int DPL = (D + 63) / 64;
    constexpr int VB = D == 64 ? 64 : 16;                    // V keys loaded together
    __shared__ __attribute__((aligned(16))) float qsh[kGqaMaxG][D];
    __shared__ __attribute__((aligned(16))) float psh[kGqaWaves][kGqaMaxG][64];
    __shared__ float msh[kGqaWaves][kGqaMaxG], lsh[kGqaWaves][kGqaMaxG];
    __shared__ __attribute__((aligned(16))) float ash[kGqaWaves][kGqaMaxG][D];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int G = a.Hq / a.Hkv;
    const int kvh = blockIdx.x % a.Hkv;
    const int bt = blockIdx.x / a.Hkv;
    const int t = bt % a.T, b = bt / a.T;

    // the G query rows of this token and kv head
    const int64_t qes = type_elem_bytes(a.q_type);
    for (int i = threadIdx.x; i < kGqaMaxG * D; i += 64 * kGqaWaves) {
        const int h = i / D, e = i - h * D;
        qsh[h][e] = h < G ? load_elem(a.q + b * a.q_nb_b + t * a.q_nb_t + (int64_t)(kvh * G + h) * a.q_nb_h + e * qes,
                                      a.q_type)
                          : 0.0f;
    }
    __syncthreads();

    const int L = a.L[b];
    int jend = L;
    if (a.mask_mode == kMaskCausal) jend = min(L, a.past[b] + t + 1);
    const char* kbase = a.k[b] + kvh * a.k_nb_head;
    const char* vbase = a.v[b] + kvh * a.v_nb_head;
    const char* mrow = a.mask ? a.mask + b * a.mask_nb_b + t * a.mask_nb_row : nullptr;

    float M[kGqaMaxG], S[kGqaMaxG], acc[kGqaMaxG][DPL];
#pragma unroll
    for (int h = 0; h < kGqaMaxG; ++h) {
        M[h] = -INFINITY;
        S[h] = 0.0f;
#pragma unroll
        for (int r = 0; r < DPL; ++r) acc[h][r] = 0.0f;
    }
    for (int j0 = 64 * wv; j0 < jend; j0 += 64 * kGqaWaves) {
        const int j = j0 + lane;
        const bool live = j < jend;
        const int nk = min(64, jend - j0);
        const float4* kr = (const float4*)(kbase + (int64_t)(live ? j : j0) * a.k_nb_tok);
        float4 kv[D / 4];
#pragma unroll
        for (int i4 = 0; i4 < D / 4; ++i4) kv[i4] = kr[i4];
        // V of the step's first VB keys (rows past the last visible key repeat it: p = 0)
        const char* vr = vbase + (int64_t)j0 * a.v_nb_tok;
        float vv[VB][DPL];
#pragma unroll
        for (int u = 0; u < VB; ++u)
#pragma unroll
            for (int r = 0; r < DPL; ++r)
                vv[u][r] = lane + 64 * r < D ? *((const float*)(vr + (int64_t)min(u, nk - 1) * a.v_nb_tok) + lane + 64 * r) : 0.0f;
        const float mv = live && a.mask_mode == kMaskExplicit ? mask_at(mrow, j, a.mask_f32) : 0.0f;
        // every head slot in straight-line code (slots past G score -inf),
        // so that the heads' dot products and wave reductions interleave
        float sc[kGqaMaxG], p[kGqaMaxG], alpha[kGqaMaxG], mx[kGqaMaxG], ps[kGqaMaxG];
#pragma unroll
        for (int h = 0; h < kGqaMaxG; ++h) {
            float dot0 = 0.0f, dot1 = 0.0f;
#pragma unroll
            for (int i4 = 0; i4 < D / 4; i4 += 2) {
                const float4 q0 = *(const float4*)&qsh[h][4 * i4];
                dot0 = fmaf(q0.x, kv[i4].x, dot0); dot0 = fmaf(q0.y, kv[i4].y, dot0);
                dot0 = fmaf(q0.z, kv[i4].z, dot0); dot0 = fmaf(q0.w, kv[i4].w, dot0);
                if (i4 + 1 < D / 4) {
                    const float4 q1 = *(const float4*)&qsh[h][4 * i4 + 4];
                    dot1 = fmaf(q1.x, kv[i4 + 1].x, dot1); dot1 = fmaf(q1.y, kv[i4 + 1].y, dot1);
                    dot1 = fmaf(q1.z, kv[i4 + 1].z, dot1); dot1 = fmaf(q1.w, kv[i4 + 1].w, dot1);
                }
            }
            sc[h] = !live || mv == -INFINITY || h >= G ? -INFINITY : (dot0 + dot1) * a.scale + mv;
        }
#pragma unroll
        for (int h = 0; h < kGqaMaxG; ++h) mx[h] = wave_max(sc[h]);
#pragma unroll
        for (int h = 0; h < kGqaMaxG; ++h) {
            const float Mn = fmaxf(M[h], mx[h]);
            alpha[h] = Mn == -INFINITY ? 1.0f : __expf(M[h] - Mn);     // 0 while M = -inf
            p[h] = sc[h] == -INFINITY ? 0.0f : __expf(sc[h] - Mn);
            M[h] = Mn;
        }
#pragma unroll
        for (int h = 0; h < kGqaMaxG; ++h) ps[h] = wave_sum(p[h]);
#pragma unroll
        for (int h = 0; h < kGqaMaxG; ++h) {
            S[h] = fmaf(S[h], alpha[h], ps[h]);
            psh[wv][h][lane] = p[h];
#pragma unroll
            for (int r = 0; r < DPL; ++r) acc[h][r] *= alpha[h];
        }
        wave_lds_sync();
        for (int u0 = 0; u0 < nk; u0 += VB) {
            if (u0 > 0) {                                        // D > 64: the next VB keys
#pragma unroll
                for (int u = 0; u < VB; ++u)
#pragma unroll
                    for (int r = 0; r < DPL; ++r)
                        vv[u][r] = lane + 64 * r < D
                                       ? *((const float*)(vr + (int64_t)min(u0 + u, nk - 1) * a.v_nb_tok) + lane + 64 * r)
                                       : 0.0f;
            }
#pragma unroll
            for (int h = 0; h < kGqaMaxG; ++h) {
#pragma unroll
                for (int u = 0; u < VB; u += 4) {
                    const float4 pu = *(const float4*)&psh[wv][h][u0 + u];
#pragma unroll
                    for (int r = 0; r < DPL; ++r) {
                        acc[h][r] = fmaf(pu.x, vv[u][r], acc[h][r]);
                        acc[h][r] = fmaf(pu.y, vv[u + 1][r], acc[h][r]);
                        acc[h][r] = fmaf(pu.z, vv[u + 2][r], acc[h][r]);
                        acc[h][r] = fmaf(pu.w, vv[u + 3][r], acc[h][r]);
                    }
                }
            }
        }
        wave_lds_sync();                                         // psh is rewritten by the next step
    }
    // combine the waves per head: log-sum-exp of (M, S, acc)
#pragma unroll
    for (int h = 0; h < kGqaMaxG; ++h) {
        if (h >= G) break;
        if (lane == 0) {
            msh[wv][h] = M[h];
            lsh[wv][h] = S[h];
        }
#pragma unroll
        for (int r = 0; r < DPL; ++r)
            if (lane + 64 * r < D) ash[wv][h][lane + 64 * r] = acc[h][r];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < G * D; i += 64 * kGqaWaves) {
        const int h = i / D, e = i - h * D;
        float Mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < kGqaWaves; ++w) Mx = fmaxf(Mx, msh[w][h]);
        float num = 0.0f, den = 0.0f;
        if (Mx != -INFINITY) {
#pragma unroll
            for (int w = 0; w < kGqaWaves; ++w) {
                const float f = __expf(msh[w][h] - Mx);          // 0 for a wave that saw nothing
                num = fmaf(ash[w][h][e], f, num);
                den = fmaf(lsh[w][h], f, den);
            }
        }
        float* orow = (float*)((char*)a.out + b * a.o_nb_b + t * a.o_nb_t + (int64_t)(kvh * G + h) * a.o_nb_h);
        orow[e] = den == 0.0f ? 0.0f : num / den;
    }
}

// F32 K and V with 16-byte aligned rows take attn_rows_f32_kernel.
bool rows_f32_ok(const AttnArgs& a) {
    if (a.k_type != VVA_TYPE_F32 || a.v_type != VVA_TYPE_F32) return false;
    if (a.d % 8 != 0 || a.d > 256) return false;
    if (a.k_nb_tok % 16 || a.k_nb_head % 16) return false;
    for (int b = 0; b < a.B; ++b)
        if ((uintptr_t)a.k[b] % 16) return false;
    return true;
}

}  // namespace

hipError_t launch_attn_rows(const AttnArgs& a, hipStream_t s) {
    const int64_t rows = (int64_t)a.B * a.T * a.Hq;
    if (rows == 0) return hipSuccess;
    dim3 grid((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock));
    const int dpl = (a.d + 63) / 64;
    if (rows_f32_ok(a) && (a.d == 64 || a.d == 128) && a.Hq / a.Hkv <= kGqaMaxG) {
        const dim3 g((unsigned)((int64_t)a.B * a.T * a.Hkv));
        if (a.d == 64) hipLaunchKernelGGL((attn_gqa_f32_kernel<64>), g, dim3(64 * kGqaWaves), 0, s, a);
        else           hipLaunchKernelGGL((attn_gqa_f32_kernel<128>), g, dim3(64 * kGqaWaves), 0, s, a);
        return hipGetLastError();
    }
    if (rows_f32_ok(a)) {
        if (a.d == 64) {
            hipLaunchKernelGGL((attn_rows_f32_kernel<1, 64>), grid, dim3(256), 0, s, a);
            return hipGetLastError();
        }
        if (a.d == 128) {
            hipLaunchKernelGGL((attn_rows_f32_kernel<2, 128>), grid, dim3(256), 0, s, a);
            return hipGetLastError();
        }
        switch (dpl) {
            case 1: hipLaunchKernelGGL((attn_rows_f32_kernel<1, 0>), grid, dim3(256), 0, s, a); break;
            case 2: hipLaunchKernelGGL((attn_rows_f32_kernel<2, 0>), grid, dim3(256), 0, s, a); break;
            case 3: hipLaunchKernelGGL((attn_rows_f32_kernel<3, 0>), grid, dim3(256), 0, s, a); break;
            case 4: hipLaunchKernelGGL((attn_rows_f32_kernel<4, 0>), grid, dim3(256), 0, s, a); break;
            default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    switch (dpl) {
        case 1: hipLaunchKernelGGL(attn_rows_kernel<1>, grid, dim3(256), 0, s, a); break;
        case 2: hipLaunchKernelGGL(attn_rows_kernel<2>, grid, dim3(256), 0, s, a); break;
        case 3: hipLaunchKernelGGL(attn_rows_kernel<3>, grid, dim3(256), 0, s, a); break;
        case 4: hipLaunchKernelGGL(attn_rows_kernel<4>, grid, dim3(256), 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace vva
