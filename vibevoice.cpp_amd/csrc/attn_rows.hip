// attn_rows.hip — attention for the shapes the MFMA prefill and split-K
// decode kernels do not take: VALU kernels (one wavefront per query row, or
// per token and kv head), and the fp32 MFMA kernel of the eager branch for
// several tokens over F32 caches (attn_gqa_f32_mfma_kernel).
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
constexpr unsigned kGatedGrid = 512; // workgroups of a gated attn_rows_kernel launch

// One query row (b, t, head) on one wave.
template <int DPL>
__device__ __forceinline__ void attn_row(const AttnArgs& a, int row) {
    const int lane = threadIdx.x & 63;
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

// Rows on waves, grid-stride (a gated launch takes a small grid: when its
// gate is closed every workgroup leaves after one load).
template <int DPL>
__global__ void __launch_bounds__(256) attn_rows_kernel(AttnArgs a) {
    prefetch_kernargs<sizeof(AttnArgs)>();
    if (a.gate && *a.gate != a.gate_epoch) return;     // a gated fallback that is not needed
    const int rows = a.B * a.T * a.Hq;
    for (int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6); row < rows; row += gridDim.x * kRowsPerBlock)
        attn_row<DPL>(a, row);                         // (row is uniform per wave)
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
    if (a.gate && *a.gate != a.gate_epoch) return;     // a gated fallback that is not needed
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
    if (a.gate && *a.gate != a.gate_epoch) return;     // a gated fallback that is not needed
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

// F32 K and V on fp32 MFMA (v_mfma_f32_16x16x4f32): the eager branch's two
// mul_mats (src/qwen2.cpp:337-343) as matrix products.  A workgroup takes 16
// consecutive query rows i = t G + h of one (sequence, kv head), so the kv
// head's K and V rows are read once for its whole query-head group, and
// kMfWaves waves; wave w takes the 16-key blocks w, w + W, ... of the keys
// visible to any of the rows, the next block's K and V loads in flight while
// it computes one.  Per block, with lane l = 16 g + c (c = l % 16, g = l / 16)
// owning query row c:
//   S^T = K Q^T (keys x rows): the contraction over d in D / 4 steps, lane
//     group g supplying d = g D/4 + s at step s (K row key0 + c and Q row c
//     read as contiguous chunks); lane l receives S^T[key 4 g + j][row c];
//   the online softmax of row c over the block: scale, mask, max and sum over
//     the lane's 4 keys and across the 4 lane groups (permlane swaps);
//   O^T += V^T P^T (d x rows) in D / 16 tiles of 16 d: at step s lane group g
//     supplies key 4 g + s (its own p[s] as the B operand, V[key][D/16 c + ct]
//     of tile ct as the A operand), so lane l accumulates O[row c][d] for the
//     D / 4 consecutive d = g D/4 .. g D/4 + D/4 - 1.
// Products and sums in fp32 (MFMA accumulation order instead of ggml's
// sequential one); the waves' (max, sum, O) per row are combined through
// LDS by log-sum-exp.  Same semantics as attn_gqa_f32_kernel.
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int kMfWaves = 8;
template <int D>
__global__ void __launch_bounds__(64 * kMfWaves) attn_gqa_f32_mfma_kernel(AttnArgs a) {
    prefetch_kernargs<sizeof(AttnArgs)>();
    if (a.gate && *a.gate != a.gate_epoch) return;     // a gated fallback that is not needed
    constexpr int DQ = D / 4;                                // d per lane group (S^T steps)
    constexpr int CT = D / 16;                               // O^T tiles
    __shared__ float msh[kMfWaves][16], lsh[kMfWaves][16];
    __shared__ __attribute__((aligned(16))) float osh[kMfWaves][16][D + 4];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int c = lane & 15, g = lane >> 4;
    const int G = a.Hq / a.Hkv;
    const int rows = a.T * G;
    const int ntile = (rows + 15) / 16;
    const int tile = blockIdx.x % ntile;
    const int kvh = (blockIdx.x / ntile) % a.Hkv;
    const int b = blockIdx.x / (ntile * a.Hkv);
    const int i = tile * 16 + c;                             // this lane's query row
    const bool rlive = i < rows;
    const int ii = rlive ? i : rows - 1;
    const int t = ii / G, h = ii - t * G;
    const int L = a.L[b];
    const int t_last = min(tile * 16 + 15, rows - 1) / G;
    const bool causal = a.mask_mode == kMaskCausal;
    const int jend = causal ? min(L, a.past[b] + t_last + 1) : L;   // keys any row of the tile may see
    const int jrow = !rlive ? 0 : causal ? min(L, a.past[b] + t + 1) : L;
    const char* mrow = a.mask_mode == kMaskExplicit ? a.mask + b * a.mask_nb_b + t * a.mask_nb_row : nullptr;

    // Q[row c][g DQ .. g DQ + DQ): one code path per type, so the DQ loads
    // go out together (a per-element type switch would wait on each)
    float q[DQ];
    {
        const char* qr = a.q + b * a.q_nb_b + t * a.q_nb_t + (int64_t)(kvh * G + h) * a.q_nb_h;
        if (a.q_type == VVA_TYPE_F32) {
#pragma unroll
            for (int s = 0; s < DQ; ++s) q[s] = *(const float*)(qr + (int64_t)(g * DQ + s) * 4);
        } else {
            uint16_t q16[DQ];
#pragma unroll
            for (int s = 0; s < DQ; ++s) q16[s] = *(const uint16_t*)(qr + (int64_t)(g * DQ + s) * 2);
            if (a.q_type == VVA_TYPE_BF16) {
#pragma unroll
                for (int s = 0; s < DQ; ++s) q[s] = bf16_to_f32(q16[s]);
            } else {
#pragma unroll
                for (int s = 0; s < DQ; ++s) q[s] = f16_to_f32(q16[s]);
            }
        }
    }
    const char* kbase = a.k[b] + kvh * a.k_nb_head;
    const char* vbase = a.v[b] + kvh * a.v_nb_head;
    float m = -INFINITY, l = 0.0f;
    f32x4 o[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) o[ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // K row key0 + c as DQ / 4 vectors; V rows key0 + 4 g + s, d = CT c ..
    // CT c + CT - 1 as CT / 4 vectors each (rows past the window repeat the
    // last one: their scores are masked)
    float4 kr4[DQ / 4], vv4[4][CT / 4];
    auto load_block = [&](int key0, float4 (&kq)[DQ / 4], float4 (&vq)[4][CT / 4]) {
        const float4* kp = (const float4*)(kbase + (int64_t)min(key0 + c, L - 1) * a.k_nb_tok) + g * (DQ / 4);
#pragma unroll
        for (int s4 = 0; s4 < DQ / 4; ++s4) kq[s4] = kp[s4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const float4* vp = (const float4*)(vbase + (int64_t)min(key0 + 4 * g + s, L - 1) * a.v_nb_tok) + c * (CT / 4);
#pragma unroll
            for (int c4 = 0; c4 < CT / 4; ++c4) vq[s][c4] = vp[c4];
        }
    };
    load_block(16 * wv, kr4, vv4);
    for (int kb = wv; kb * 16 < jend; kb += kMfWaves) {
        const int key0 = kb * 16;
        float4 krn[DQ / 4], vvn[4][CT / 4];
        load_block(key0 + 16 * kMfWaves, krn, vvn);          // the next block's rows, in flight meanwhile
        float kr[DQ], vv[4][CT];
#pragma unroll
        for (int s4 = 0; s4 < DQ / 4; ++s4) {
            kr[4 * s4] = kr4[s4].x; kr[4 * s4 + 1] = kr4[s4].y; kr[4 * s4 + 2] = kr4[s4].z; kr[4 * s4 + 3] = kr4[s4].w;
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int c4 = 0; c4 < CT / 4; ++c4) {
                vv[s][4 * c4] = vv4[s][c4].x; vv[s][4 * c4 + 1] = vv4[s][c4].y;
                vv[s][4 * c4 + 2] = vv4[s][c4].z; vv[s][4 * c4 + 3] = vv4[s][c4].w;
            }
        f32x4 st = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < DQ; ++s) st = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[s], q[s], st, 0, 0, 0);
        // scores of row c for keys key0 + 4 g + j
        float sc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int key = key0 + 4 * g + j;
            const float mv = mrow && key < L ? mask_at(mrow, key, a.mask_f32) : 0.0f;
            sc[j] = key >= jrow || mv == -INFINITY ? -INFINITY : st[j] * a.scale + mv;
        }
        float mx = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
        mx = max_swap32(max_swap16(mx));
        const float mn = fmaxf(m, mx);
        const float alpha = mn == -INFINITY ? 1.0f : __expf(m - mn);   // 0 while m = -inf
        float p[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) p[j] = sc[j] == -INFINITY ? 0.0f : __expf(sc[j] - mn);
        const float ps = add_swap32(add_swap16((p[0] + p[1]) + (p[2] + p[3])));
        l = fmaf(l, alpha, ps);
        m = mn;
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) o[ct] *= alpha;
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) o[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[s][ct], p[s], o[ct], 0, 0, 0);
#pragma unroll
        for (int s4 = 0; s4 < DQ / 4; ++s4) kr4[s4] = krn[s4];
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int c4 = 0; c4 < CT / 4; ++c4) vv4[s][c4] = vvn[s][c4];
    }
    // combine the waves per row: log-sum-exp of (m, l, O)
    if (g == 0) {
        msh[wv][c] = m;
        lsh[wv][c] = l;
    }
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int j = 0; j < 4; ++j) osh[wv][c][g * DQ + CT * j + ct] = o[ct][j];
    __syncthreads();
    // thread -> (row r, EPT consecutive d): the waves' weights once per thread
    constexpr int EPT = 16 * D / (64 * kMfWaves);
    const int r = threadIdx.x / (D / EPT), e0 = (threadIdx.x - r * (D / EPT)) * EPT;
    const int ir = tile * 16 + r;
    if (ir >= rows) return;
    float Mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kMfWaves; ++w) Mx = fmaxf(Mx, msh[w][r]);
    float num[EPT], den = 0.0f;
#pragma unroll
    for (int e = 0; e < EPT; ++e) num[e] = 0.0f;
    if (Mx != -INFINITY) {
#pragma unroll
        for (int w = 0; w < kMfWaves; ++w) {
            const float f = __expf(msh[w][r] - Mx);          // 0 for a wave that saw nothing
            den = fmaf(lsh[w][r], f, den);
#pragma unroll
            for (int e = 0; e < EPT; ++e) num[e] = fmaf(osh[w][r][e0 + e], f, num[e]);
        }
    }
    const int tr = ir / G, hr = ir - tr * G;
    float* orow = (float*)((char*)a.out + b * a.o_nb_b + tr * a.o_nb_t + (int64_t)(kvh * G + hr) * a.o_nb_h) + e0;
#pragma unroll
    for (int e = 0; e < EPT; ++e) orow[e] = den == 0.0f ? 0.0f : num[e] / den;
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

// V rows 16-byte aligned (the MFMA kernel reads them as float4)
bool v_rows_aligned(const AttnArgs& a) {
    if (a.v_nb_tok % 16 || a.v_nb_head % 16) return false;
    for (int b = 0; b < a.B; ++b)
        if ((uintptr_t)a.v[b] % 16) return false;
    return true;
}

}  // namespace

hipError_t launch_attn_rows(const AttnArgs& a, hipStream_t s) {
    const int64_t rows = (int64_t)a.B * a.T * a.Hq;
    if (rows == 0) return hipSuccess;
    dim3 grid((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock));
    const int dpl = (a.d + 63) / 64;
    if (rows_f32_ok(a) && (a.d == 64 || a.d == 128) && a.T >= 4 && v_rows_aligned(a)) {
        // several tokens: the fp32 MFMA kernel, 16 query rows of a kv head per workgroup
        const int G = a.Hq / a.Hkv;
        const dim3 g((unsigned)((int64_t)a.B * a.Hkv * ((a.T * G + 15) / 16)));
        if (a.d == 64) hipLaunchKernelGGL((attn_gqa_f32_mfma_kernel<64>), g, dim3(64 * kMfWaves), 0, s, a);
        else           hipLaunchKernelGGL((attn_gqa_f32_mfma_kernel<128>), g, dim3(64 * kMfWaves), 0, s, a);
        return hipGetLastError();
    }
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
    if (a.gate && grid.x > kGatedGrid) grid.x = kGatedGrid;
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
