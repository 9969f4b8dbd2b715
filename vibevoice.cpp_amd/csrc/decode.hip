// decode.hip — split-K single-token attention (T == 1) over an F16, BF16 or
// Q8_0 KV cache, the per-step attention of the TTS / ASR decode loops
// (src/vibevoice_tts.cpp:862-880, src/vibevoice_asr.cpp:760-800), i.e.
// ggml_flash_attn_ext with one query row per head (src/qwen2.cpp:332-334).
//
// Bandwidth-bound, no MFMA.  Grid = (n_splits, B).  A workgroup takes one
// contiguous key range of one sequence for ALL kv heads, so together its
// waves read whole cache rows ([Hkv][d] per token) and no cache line is
// fetched by two CUs.  Wave w handles kv head w % Hkv and the (w / Hkv)-th
// part of the range, with all g = Hq/Hkv query heads of that kv head held in
// registers (GQA: every K/V byte is read once per group, not once per head).
//
// Per wave iteration TPI = 64 / (d/32) tokens are processed:
//   K phase  lane l = (token l/(d/32), 32-dim chunk l%(d/32)); the chunk is
//            loaded with 128-bit loads (F16/BF16: 64 B; Q8_0: its 34-byte
//            block via 2x dwordx4 + dword and a byte align); dots use
//            v_dot2_f32_f16 / v_dot2_f32_bf16 against Q rounded to f16/bf16,
//            or v_dot4_i32_i8 against Q quantized to Q8_0 per 32-dim block
//            (ggml's Q8_0 x Q8_0 vec dot: integer block sums scaled by
//            d_k * d_q); a (d/32)-lane butterfly completes each score.
//   softmax  chunk max per head by butterfly, exp2 in registers, running
//            (m, l) per head; p goes to LDS (one float per token and head).
//   V phase  lane l owns d/64 consecutive dims; each token's V row is one
//            coalesced 256 B (F16, d=128) / 136 B (Q8_0) wave read,
//            dequantized in registers, fp32 accumulate with p from LDS.
// Waves of one kv head merge through LDS (log-sum-exp), then the workgroup
// writes (m, l, acc[d]) per (head, split); decode_merge_kernel combines the
// splits.  With a single split the output is written directly.
#include "vva_internal.hpp"

namespace vva {

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4), aligned(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kMaxWaves = 8;

__device__ __forceinline__ float dot2_f16(uint32_t a, uint32_t b, float c) {
    h2 x, y;
    __builtin_memcpy(&x, &a, 4);
    __builtin_memcpy(&y, &b, 4);
    return __builtin_amdgcn_fdot2(x, y, c, false);
}
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    bf2 x, y;
    __builtin_memcpy(&x, &a, 4);
    __builtin_memcpy(&y, &b, 4);
    return __builtin_amdgcn_fdot2_f32_bf16(x, y, c, false);
}

template <int KT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    uint16_t x = KT == VVA_TYPE_BF16 ? f32_to_bf16(a) : f32_to_f16(a);
    uint16_t y = KT == VVA_TYPE_BF16 ? f32_to_bf16(b) : f32_to_f16(b);
    return (uint32_t)x | ((uint32_t)y << 16);
}

template <int KT>
__device__ __forceinline__ float unpack_lo(uint32_t v) {
    return KT == VVA_TYPE_BF16 ? bf16_to_f32((uint16_t)v) : f16_to_f32((uint16_t)v);
}
template <int KT>
__device__ __forceinline__ float unpack_hi(uint32_t v) {
    return KT == VVA_TYPE_BF16 ? bf16_to_f32((uint16_t)(v >> 16)) : f16_to_f32((uint16_t)(v >> 16));
}

// D: head dim (64 / 128); G: query heads per kv head; KT: cache type.
template <int D, int G, int KT>
__global__ void __launch_bounds__(256)
decode_kernel(AttnArgs a, float* __restrict__ ws, int n_splits, int split_len) {
    constexpr int LPT = D / 32;          // lanes per token in the K phase
    constexpr int TPI = 64 / LPT;        // tokens per iteration
    constexpr int DV = D / 64;           // dims per lane in the V phase
    constexpr bool Q8 = KT == VVA_TYPE_Q8_0;
    constexpr int QW = Q8 ? 8 : 16;      // 32-bit words of Q per head per lane

    __shared__ float pbuf[kMaxWaves][TPI][G];
    __shared__ float mbuf[kMaxWaves][G];
    __shared__ float lbuf[kMaxWaves][G];
    __shared__ float abuf[kMaxWaves][G][D];

    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int nw = blockDim.x >> 6;
    const int Hkv = a.Hkv;
    const int R = nw / Hkv;
    const int kvh = w % Hkv, r = w / Hkv;
    const int split = blockIdx.x, b = blockIdx.y;
    const int L = a.L[b];
    const int sub_len = split_len / R;
    const int j_begin = split * split_len + r * sub_len;
    const int j_end = min(L, j_begin + sub_len);
    const int tl = lane / LPT, c = lane % LPT;
    const int h0 = kvh * G;

    // ---- Q for this lane's 32-dim chunk, all G heads, in K's dot type
    uint32_t qw[G][QW];
    float qd[G];
    {
        const int64_t es = type_elem_bytes(a.q_type);
#pragma unroll
        for (int hh = 0; hh < G; ++hh) {
            const char* qrow = a.q + b * a.q_nb_b + (h0 + hh) * a.q_nb_h + (int64_t)(c * 32) * es;
            float x[32];
#pragma unroll
            for (int i = 0; i < 32; ++i) x[i] = load_elem(qrow + i * es, a.q_type);
            if constexpr (Q8) {
                float am = 0.0f;
#pragma unroll
                for (int i = 0; i < 32; ++i) am = fmaxf(am, fabsf(x[i]));
                const float dq = am / 127.0f;
                const float id = dq != 0.0f ? 1.0f / dq : 0.0f;
                qd[hh] = f16_to_f32(f32_to_f16(dq));
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    uint32_t v = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        v |= ((uint32_t)(uint8_t)(int8_t)roundf(x[4 * k + e] * id)) << (8 * e);
                    qw[hh][k] = v;
                }
            } else {
                qd[hh] = 1.0f;
#pragma unroll
                for (int k = 0; k < 16; ++k) qw[hh][k] = pack2<KT>(x[2 * k], x[2 * k + 1]);
            }
        }
    }

    const char* kb = a.k[b] + kvh * a.k_nb_head;
    const char* vb = a.v[b] + kvh * a.v_nb_head;
    const char* mrow = a.mask ? a.mask + b * a.mask_nb_b : nullptr;   // query row 0

    float m[G], l[G], acc[G][DV];
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
        m[hh] = -INFINITY;
        l[hh] = 0.0f;
#pragma unroll
        for (int e = 0; e < DV; ++e) acc[hh][e] = 0.0f;
    }

    for (int j0 = j_begin; j0 < j_end; j0 += TPI) {
        const int j = j0 + tl;
        const bool valid = j < j_end;
        // ---------------- K phase: scores (log2 domain)
        float s[G];
#pragma unroll
        for (int hh = 0; hh < G; ++hh) s[hh] = 0.0f;
        if (valid) {
            const char* kr = kb + (int64_t)j * a.k_nb_tok;
            if constexpr (Q8) {
                const char* blk = kr + c * kQ8Bytes;
                const bool odd = (c & 1) != 0;
                const char* base = blk - (odd ? 2 : 0);
                const u32x4 v0 = *(const u32x4*)base;
                const u32x4 v1 = *(const u32x4*)(base + 16);
                const uint32_t v8 = *(const uint32_t*)(base + 32);
                const uint32_t dw[9] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w, v8};
                const float dk = f16_to_f32((uint16_t)(odd ? (dw[0] >> 16) : (dw[0] & 0xffffu)));
                uint32_t kc[8];
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    kc[k] = odd ? dw[k + 1] : __builtin_amdgcn_alignbyte(dw[k + 1], dw[k], 2);
#pragma unroll
                for (int hh = 0; hh < G; ++hh) {
                    int si = 0;
#pragma unroll
                    for (int k = 0; k < 8; ++k) si = __builtin_amdgcn_sdot4((int)qw[hh][k], (int)kc[k], si, false);
                    s[hh] = (float)si * (dk * qd[hh]);
                }
            } else {
                const u32x4* kp = (const u32x4*)(kr + c * 64);
                uint32_t kw[16];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const u32x4 v = kp[k];
                    kw[4 * k] = v.x; kw[4 * k + 1] = v.y; kw[4 * k + 2] = v.z; kw[4 * k + 3] = v.w;
                }
#pragma unroll
                for (int hh = 0; hh < G; ++hh) {
                    float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
                    for (int k = 0; k < 16; k += 2) {
                        if constexpr (KT == VVA_TYPE_BF16) {
                            d0 = dot2_bf16(qw[hh][k], kw[k], d0);
                            d1 = dot2_bf16(qw[hh][k + 1], kw[k + 1], d1);
                        } else {
                            d0 = dot2_f16(qw[hh][k], kw[k], d0);
                            d1 = dot2_f16(qw[hh][k + 1], kw[k + 1], d1);
                        }
                    }
                    s[hh] = d0 + d1;
                }
            }
        }
        // complete the dot across the LPT lanes of the token
#pragma unroll
        for (int msk = 1; msk < LPT; msk <<= 1) {
#pragma unroll
            for (int hh = 0; hh < G; ++hh) s[hh] += __shfl_xor(s[hh], msk, 64);
        }
        float mv = 0.0f;
        if (valid && a.mask_mode == kMaskExplicit)
            mv = f16_to_f32(*(const uint16_t*)(mrow + 2 * (int64_t)j));
        const bool live = valid && mv != -INFINITY;
        // ---------------- online softmax
        float p[G];
#pragma unroll
        for (int hh = 0; hh < G; ++hh) {
            const float sv = live ? (s[hh] * a.scale + mv) * kLog2e : -INFINITY;
            float cm = sv;
#pragma unroll
            for (int msk = LPT; msk < 64; msk <<= 1) cm = fmaxf(cm, __shfl_xor(cm, msk, 64));
            const float mn = fmaxf(m[hh], cm);
            const float alpha = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m[hh] - mn);
            p[hh] = live ? __builtin_amdgcn_exp2f(sv - mn) : 0.0f;
            m[hh] = mn;
            l[hh] = l[hh] * alpha + (c == 0 ? p[hh] : 0.0f);
#pragma unroll
            for (int e = 0; e < DV; ++e) acc[hh][e] *= alpha;
        }
        if (c == 0) {
#pragma unroll
            for (int hh = 0; hh < G; ++hh) pbuf[w][tl][hh] = p[hh];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // ---------------- V phase
        const int nt = min(TPI, j_end - j0);
        for (int u = 0; u < nt; ++u) {
            const char* vr = vb + (int64_t)(j0 + u) * a.v_nb_tok;
            float vv[DV];
            if constexpr (Q8) {
                const int dim0 = lane * DV;
                const char* blk = vr + (dim0 / kQK8) * kQ8Bytes;
                const float dv = f16_to_f32(*(const uint16_t*)blk);
                if constexpr (DV == 2) {
                    const uint16_t cc = *(const uint16_t*)(blk + 2 + (dim0 & (kQK8 - 1)));
                    vv[0] = (float)(int8_t)(cc & 0xff) * dv;
                    vv[1] = (float)(int8_t)(cc >> 8) * dv;
                } else {
                    vv[0] = (float)(int8_t)blk[2 + (dim0 & (kQK8 - 1))] * dv;
                }
            } else {
                if constexpr (DV == 2) {
                    const uint32_t x = *(const uint32_t*)(vr + 4 * lane);
                    vv[0] = unpack_lo<KT>(x);
                    vv[1] = unpack_hi<KT>(x);
                } else {
                    const uint16_t x = *(const uint16_t*)(vr + 2 * lane);
                    vv[0] = unpack_lo<KT>(x);
                }
            }
#pragma unroll
            for (int hh = 0; hh < G; ++hh) {
                const float pp = pbuf[w][u][hh];
#pragma unroll
                for (int e = 0; e < DV; ++e) acc[hh][e] = fmaf(pp, vv[e], acc[hh][e]);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    // total l per head over the lanes (only chunk-0 lanes contributed)
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
#pragma unroll
        for (int msk = 1; msk < 64; msk <<= 1) l[hh] += __shfl_xor(l[hh], msk, 64);
    }

    // ---- merge the R parts of each kv head (log-sum-exp) through LDS
    if (R > 1) {
        if (r > 0) {
#pragma unroll
            for (int hh = 0; hh < G; ++hh) {
                if (lane == 0) { mbuf[w][hh] = m[hh]; lbuf[w][hh] = l[hh]; }
#pragma unroll
                for (int e = 0; e < DV; ++e) abuf[w][hh][lane * DV + e] = acc[hh][e];
            }
        }
        __syncthreads();
        if (r == 0) {
            for (int rr = 1; rr < R; ++rr) {
                const int ow = rr * Hkv + kvh;
#pragma unroll
                for (int hh = 0; hh < G; ++hh) {
                    const float mo = mbuf[ow][hh];
                    const float mn = fmaxf(m[hh], mo);
                    const float fa = mn == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m[hh] - mn);
                    const float fb = mn == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mo - mn);
                    l[hh] = l[hh] * fa + lbuf[ow][hh] * fb;
#pragma unroll
                    for (int e = 0; e < DV; ++e)
                        acc[hh][e] = acc[hh][e] * fa + abuf[ow][hh][lane * DV + e] * fb;
                    m[hh] = mn;
                }
            }
        }
    }
    if (r != 0) return;

    if (n_splits == 1) {
#pragma unroll
        for (int hh = 0; hh < G; ++hh) {
            const float inv = l[hh] == 0.0f ? 0.0f : 1.0f / l[hh];
            float* orow = (float*)((char*)a.out + b * a.o_nb_b + (h0 + hh) * a.o_nb_h);
#pragma unroll
            for (int e = 0; e < DV; ++e) orow[lane * DV + e] = acc[hh][e] * inv;
        }
        return;
    }
    // partials: acc [B][Hq][n_splits][D], then (m, l) [B][Hq][n_splits][2]
    const int Hq = a.Hq;
    float* wacc = ws;
    float* wml = ws + (size_t)a.B * Hq * n_splits * D;
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
        const size_t idx = ((size_t)b * Hq + (h0 + hh)) * n_splits + split;
#pragma unroll
        for (int e = 0; e < DV; ++e) wacc[idx * D + lane * DV + e] = acc[hh][e];
        if (lane == 0) { wml[idx * 2] = m[hh]; wml[idx * 2 + 1] = l[hh]; }
    }
}

// One workgroup per (query head, batch); thread i owns output dim i.
template <int D>
__global__ void __launch_bounds__(D) decode_merge_kernel(AttnArgs a, const float* __restrict__ ws, int n_splits) {
    const int h = blockIdx.x, b = blockIdx.y, i = threadIdx.x;
    const float* wacc = ws;
    const float* wml = ws + (size_t)a.B * a.Hq * n_splits * D;
    const size_t base = ((size_t)b * a.Hq + h) * n_splits;
    float M = -INFINITY;
    for (int s = 0; s < n_splits; ++s) M = fmaxf(M, wml[(base + s) * 2]);
    float num = 0.0f, den = 0.0f;
    if (M != -INFINITY) {
        for (int s = 0; s < n_splits; ++s) {
            const float ms = wml[(base + s) * 2];
            const float f = __builtin_amdgcn_exp2f(ms - M);   // 0 for empty splits
            den = fmaf(wml[(base + s) * 2 + 1], f, den);
            num = fmaf(wacc[(base + s) * D + i], f, num);
        }
    }
    float* orow = (float*)((char*)a.out + b * a.o_nb_b + h * a.o_nb_h);
    orow[i] = den == 0.0f ? 0.0f : num / den;
}

template <int D, int KT>
hipError_t launch_dg(const AttnArgs& a, float* ws, int n_splits, int split_len, int nw, hipStream_t s) {
    dim3 grid(n_splits, a.B), block(64 * nw);
    const int g = a.Hq / a.Hkv;
    switch (g) {
#define VVA_DG(G) case G: hipLaunchKernelGGL((decode_kernel<D, G, KT>), grid, block, 0, s, a, ws, n_splits, split_len); break;
        VVA_DG(1) VVA_DG(2) VVA_DG(3) VVA_DG(4) VVA_DG(5) VVA_DG(6) VVA_DG(7) VVA_DG(8)
#undef VVA_DG
        default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || n_splits == 1) return e;
    hipLaunchKernelGGL(decode_merge_kernel<D>, dim3(a.Hq, a.B), dim3(D), 0, s, a, ws, n_splits);
    return hipGetLastError();
}

}  // namespace

int decode_waves(const AttnArgs& a) { return a.Hkv <= 4 ? 4 : 8; }
int decode_tokens_per_iter(const AttnArgs& a) { return 64 / (a.d / 32); }

bool decode_supported(const AttnArgs& a) {
    if (a.T != 1) return false;
    if (a.d != 64 && a.d != 128) return false;
    if (a.k_type != a.v_type) return false;
    if (a.k_type != VVA_TYPE_F16 && a.k_type != VVA_TYPE_BF16 && a.k_type != VVA_TYPE_Q8_0) return false;
    if (a.Hq % a.Hkv != 0 || a.Hq / a.Hkv > 8) return false;
    if (a.Hkv != 1 && a.Hkv != 2 && a.Hkv != 4 && a.Hkv != 8) return false;
    if (a.mask_mode == kMaskExplicit && (a.mask_nb_b % 2 != 0)) return false;
    // vector-load alignment of cache rows
    const int64_t need = a.k_type == VVA_TYPE_Q8_0 ? 4 : 16;
    if (a.k_nb_tok % need || a.k_nb_head % need || a.v_nb_tok % 4 || a.v_nb_head % 4) return false;
    for (int b = 0; b < a.B; ++b)
        if (((uintptr_t)a.k[b] % need) || ((uintptr_t)a.v[b] % 4)) return false;
    return true;
}

hipError_t launch_decode(const AttnArgs& a, float* ws, int n_splits, int split_len, hipStream_t s) {
    const int nw = decode_waves(a);
    if (a.d == 64) {
        switch (a.k_type) {
            case VVA_TYPE_F16:  return launch_dg<64, VVA_TYPE_F16>(a, ws, n_splits, split_len, nw, s);
            case VVA_TYPE_BF16: return launch_dg<64, VVA_TYPE_BF16>(a, ws, n_splits, split_len, nw, s);
            case VVA_TYPE_Q8_0: return launch_dg<64, VVA_TYPE_Q8_0>(a, ws, n_splits, split_len, nw, s);
        }
    } else {
        switch (a.k_type) {
            case VVA_TYPE_F16:  return launch_dg<128, VVA_TYPE_F16>(a, ws, n_splits, split_len, nw, s);
            case VVA_TYPE_BF16: return launch_dg<128, VVA_TYPE_BF16>(a, ws, n_splits, split_len, nw, s);
            case VVA_TYPE_Q8_0: return launch_dg<128, VVA_TYPE_Q8_0>(a, ws, n_splits, split_len, nw, s);
        }
    }
    return hipErrorInvalidValue;
}

}  // namespace vva
