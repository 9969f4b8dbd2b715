// decode.hip — split-K single-token attention (T == 1) over an F16, BF16 or
// Q8_0 KV cache: the per-step attention of the TTS / ASR decode loops
// (src/vibevoice_tts.cpp:862-880, src/vibevoice_asr.cpp:760-800), i.e.
// ggml_flash_attn_ext with one query row per head (src/qwen2.cpp:332-334).
//
// Bandwidth-bound, no MFMA.
//
// Grid: one workgroup of 8 waves per (key split, sequence).  Wave w takes kv
// head w % Hkv and the (w / Hkv)-th part of the split, with the g = Hq / Hkv
// query heads of that kv head (GQA: each K/V byte is read once per group).
// The waves of a workgroup together read whole cache rows ([Hkv][d] per
// token), so no cache line is fetched by two CUs.
//
// Lane l of a wave owns key l / (d/32) and 32-dim chunk l % (d/32) of each
// group of 64 / (d/32) keys ("a step").  Per step the lane loads its K and V
// chunks with wide loads one step ahead of use (two register sets used in
// turn).  F16 / BF16: 4 x 16 B per chunk.  Q8_0: the 32 codes of the 34-byte
// block from the 4-byte aligned address at or below them (2 x 16 B + 4 B,
// aligned by v_alignbyte with a per-lane shift) plus the fp16 scale.
//   K      dots against Q rounded to K's dot type: v_dot2_f32_f16 /
//          v_dot2_f32_bf16, or v_dot4_i32_i8 against Q quantized to Q8_0 per
//          32-dim block (ggml's Q8_0 x Q8_0 dot: integer block sums times
//          d_k * d_q); DPP completes each score across the key's lanes.
//   soft-  two steps (32 keys at d = 128) per update; the running max is raised
//   max    lazily (only when a score exceeds it by 2^8), so the common path
//          needs no cross-lane max and no rescale.
//   V      raw V chunks go to the wave's slice of LDS, p * (V block scale) goes
//          to LDS as f16 pairs of consecutive keys; lane l then owns d/64 dims
//          and accumulates over key pairs with v_dot2_f32_f16 (codes and f16
//          values are exact in f16; fp32 accumulation).
// The waves of one kv head merge through LDS (log-sum-exp).  With one split
// the output is written directly; otherwise the workgroup writes (m, l,
// acc[d]) per head and decode_merge_kernel combines the splits (a second
// launch: kernel boundaries give the cross-XCD visibility that a device-scope
// fence would buy with an L2 write-back per workgroup).
#include "vva_internal.hpp"

namespace vva {

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4), aligned(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 8.0f;      // running-max slack in log2 units: p <= 256
constexpr int kWaves = 8;
constexpr int kMaxSplits = 256;

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
__device__ __forceinline__ float half_to_f32_rt(uint32_t v, int type) {
    return type == VVA_TYPE_BF16 ? bf16_to_f32((uint16_t)v) : f16_to_f32((uint16_t)v);
}

__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Cross-lane steps without LDS: DPP within rows of 16 lanes, permlane swaps
// across rows (v_permlane16_swap pairs rows 0-1 / 2-3, v_permlane32_swap the
// two halves of the wave).
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __uint_as_float(__builtin_amdgcn_mov_dpp(__float_as_uint(x), CTRL, 0xf, 0xf, true));
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;
__device__ __forceinline__ float max_swap16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_swap32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// Sum over the LPT lanes of one key (aligned groups of 2 or 4), for N values
// at once so consecutive DPP steps do not wait on each other.
template <int LPT, int N>
__device__ __forceinline__ void key_sum(float (&x)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] += dpp<kDppXor1>(x[i]);
    if constexpr (LPT == 4) {
#pragma unroll
        for (int i = 0; i < N; ++i) x[i] += dpp<kDppXor2>(x[i]);
    }
}
// Max over all keys of the wave, for values equal within each LPT group.
template <int LPT, int N>
__device__ __forceinline__ void keys_max(float (&x)[N]) {
    if constexpr (LPT == 2) {
#pragma unroll
        for (int i = 0; i < N; ++i) x[i] = fmaxf(x[i], dpp<kDppXor2>(x[i]));
    }
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] = fmaxf(x[i], dpp<kDppHalfMirror>(x[i]));
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] = fmaxf(x[i], dpp<kDppMirror>(x[i]));
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] = max_swap16(x[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] = max_swap32(x[i]);
}

// int8 code -> f16 (exact)
__device__ __forceinline__ _Float16 code_f16(uint32_t byte) {
    return (_Float16)(int16_t)(int8_t)(uint8_t)byte;
}

// Per-lane 32-dim chunk of a cache row.
template <int KT> struct Chunk;
template <> struct Chunk<VVA_TYPE_Q8_0> {
    static constexpr int W = 9;
    // Codes of block c start at byte c*34 + 2 of the row: 2 mod 4 for even
    // c, 0 mod 4 for odd c.  Load 9 dwords from the aligned address at or
    // below them (odd lanes, which need only 8, re-read an in-block dword as
    // the 9th so no load leaves the block) plus the fp16 scale.
    static __device__ __forceinline__ void load(const char* row, int c, uint32_t (&w)[W], float& scale) {
        const char* blk = row + c * kQ8Bytes;
        const bool odd = (c & 1) != 0;
        const char* base = blk + (odd ? 2 : 0);
        const u32x4 a = *(const u32x4*)base;
        const u32x4 b = *(const u32x4*)(base + 16);
        w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
        w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
        w[8] = *(const uint32_t*)(base + (odd ? 28 : 32));
        scale = f16_to_f32(*(const uint16_t*)blk);
    }
    // byte offset of code 0 within the loaded words
    static __device__ __forceinline__ int shift(int c) { return (c & 1) ? 0 : 2; }
};
template <> struct Chunk<VVA_TYPE_F16> {
    static constexpr int W = 16;
    static __device__ __forceinline__ void load(const char* row, int c, uint32_t (&w)[W], float& scale) {
        const u32x4* p = (const u32x4*)(row + c * 64);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const u32x4 v = p[k];
            w[4 * k] = v.x; w[4 * k + 1] = v.y; w[4 * k + 2] = v.z; w[4 * k + 3] = v.w;
        }
        scale = 1.0f;
    }
    static __device__ __forceinline__ int shift(int) { return 0; }
};
template <> struct Chunk<VVA_TYPE_BF16> : Chunk<VVA_TYPE_F16> {};

// D: head dim (64 / 128); G: query heads per kv head; KT: cache type.
template <int D, int G, int KT>
__global__ void __launch_bounds__(kWaves * 64)
decode_kernel(AttnArgs a, float* __restrict__ ws, int n_splits, int split_len) {
    constexpr int NW = kWaves;
    constexpr int LPT = D / 32;                 // lanes per key in the K phase
    constexpr int TPS = 64 / LPT;               // keys per step
    constexpr int SPI = D == 128 ? 2 : 1;       // steps per softmax update
    constexpr int TPI = TPS * SPI;              // keys per iteration
    constexpr int DV = D / 64;                  // dims per lane in the V phase
    constexpr int NB = D / 32;                  // 32-dim blocks per row
    constexpr bool Q8 = KT == VVA_TYPE_Q8_0;
    constexpr int QW = Q8 ? 8 : 16;             // Q words per head per lane
    constexpr int CW = Chunk<KT>::W;
    constexpr int SLOT = CW * 4;                // LDS bytes per staged V chunk
    constexpr int GP = G == 7 ? 8 : G;          // p row padded for 16-byte reads

    constexpr int STAGE_BYTES = NW * TPI * LPT * SLOT;
    constexpr int MERGE_BYTES = NW * G * D * 4;
    constexpr int QAREA_BYTES = 8 * G * NB * (QW + 1) * 4;           // Hkv <= 8
    constexpr int A1 = STAGE_BYTES > MERGE_BYTES ? STAGE_BYTES : MERGE_BYTES;
    // one area serves, in turn: Q conversion, V staging, the cross-wave merge
    __shared__ __attribute__((aligned(16))) char smem[A1 > QAREA_BYTES ? A1 : QAREA_BYTES];
    // p * (V block scale) as f16 pairs of consecutive keys: [wave][chunk][pair][head]
    __shared__ __attribute__((aligned(16))) uint32_t pbuf[NW][LPT][TPI / 2][GP];
    __shared__ float mbuf[NW][G];
    __shared__ float lbuf[NW][G];

    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int Hkv = a.Hkv;
    const int R = NW / Hkv;                                 // waves per kv head
    const int kvh = w % Hkv, r = w / Hkv;
    const int split = blockIdx.x, b = blockIdx.y;
    const int L = a.L[b];
    const int sub_len = split_len / R;
    const int j_begin = min(L, split * split_len + r * sub_len);
    const int j_end = min(L, j_begin + sub_len);
    const int tl = lane / LPT, c = lane % LPT;
    const int h0 = kvh * G;

    // ---- Q in K's dot type: one thread per (query head, 32-dim block)
    // converts it with vector loads (Q8_0: codes + fp16 scale; F16 / BF16:
    // packed pairs) into LDS; each lane then reads its chunk of its g heads
    uint32_t qw[G][QW];
    float qd[G];
    {
        constexpr int QSLOT = QW + 1;
        uint32_t* qlds = (uint32_t*)smem;
        if (threadIdx.x < a.Hq * NB) {
            const int hq = threadIdx.x / NB, blk = threadIdx.x % NB;
            const char* src = a.q + b * a.q_nb_b + hq * a.q_nb_h + (int64_t)(blk * 32) * type_elem_bytes(a.q_type);
            float x[32];
            if (a.q_type == VVA_TYPE_F32) {
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const float4 v = ((const float4*)src)[k];
                    x[4 * k] = v.x; x[4 * k + 1] = v.y; x[4 * k + 2] = v.z; x[4 * k + 3] = v.w;
                }
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint4 v = ((const uint4*)src)[k];
                    const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        x[8 * k + 2 * e] = half_to_f32_rt(wv[e] & 0xffffu, a.q_type);
                        x[8 * k + 2 * e + 1] = half_to_f32_rt(wv[e] >> 16, a.q_type);
                    }
                }
            }
            uint32_t* dst = qlds + threadIdx.x * QSLOT;
            if constexpr (Q8) {
                float am = 0.0f;
#pragma unroll
                for (int i = 0; i < 32; ++i) am = fmaxf(am, fabsf(x[i]));
                const float dq = am / 127.0f;
                const float id = dq != 0.0f ? 1.0f / dq : 0.0f;
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    uint32_t v = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        v |= ((uint32_t)(uint8_t)(int8_t)roundf(x[4 * k + e] * id)) << (8 * e);
                    dst[k] = v;
                }
                dst[8] = __float_as_uint(f16_to_f32(f32_to_f16(dq)));
            } else {
#pragma unroll
                for (int k = 0; k < 16; ++k) dst[k] = pack2<KT>(x[2 * k], x[2 * k + 1]);
                dst[16] = __float_as_uint(1.0f);
            }
        }
        __syncthreads();
        const float sl2 = a.scale * kLog2e;      // scores come out in the exp2 domain
#pragma unroll
        for (int hh = 0; hh < G; ++hh) {
            const uint32_t* srcw = qlds + ((h0 + hh) * NB + c) * QSLOT;
#pragma unroll
            for (int k = 0; k < QW; ++k) qw[hh][k] = srcw[k];
            qd[hh] = __uint_as_float(srcw[QW]) * sl2;
        }
        __syncthreads();                         // the area becomes V staging
    }

    const char* kb = a.k[b] + kvh * a.k_nb_head;
    const char* vb = a.v[b] + kvh * a.v_nb_head;
    const char* mrow = a.mask ? a.mask + b * a.mask_nb_b : nullptr;   // query row 0
    char* my_stage = smem + w * (TPI * LPT * SLOT);
    const int ksh = Chunk<KT>::shift(c);

    float m[G], l[G], acc[G][DV];
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
        m[hh] = -INFINITY;
        l[hh] = 0.0f;
#pragma unroll
        for (int e = 0; e < DV; ++e) acc[hh][e] = 0.0f;
    }

    // one step ahead: K and V chunks in one of two register sets
    uint32_t kbuf[2][CW], vbuf[2][CW];
    float kscale[2], vscale[2];
    auto issue = [&](int j0, int set) {
        const int j = min(j0 + tl, L - 1);                // clamped: masked later
        Chunk<KT>::load(kb + (int64_t)j * a.k_nb_tok, c, kbuf[set], kscale[set]);
        Chunk<KT>::load(vb + (int64_t)j * a.v_nb_tok, c, vbuf[set], vscale[set]);
    };
    if (j_begin < j_end) issue(j_begin, 0);

    for (int i0 = j_begin; i0 < j_end; i0 += TPI) {
        float sc[SPI][G];
        float dvs[SPI];
        bool live[SPI];
        float mv[SPI];
#pragma unroll
        for (int st = 0; st < SPI; ++st) {
            const int j0 = i0 + st * TPS;
            const int cur = SPI == 2 ? st : 0;
            // the second step of an iteration is always loaded (rows clamped to
            // the window) so staged values stay finite where p = 0; the next
            // iteration's first step only if it exists
            const bool more = (st + 1 < SPI) || (i0 + TPI < j_end);
            if constexpr (SPI == 2) {
                if (more) issue(j0 + TPS, st ^ 1);
            } else {
#pragma unroll
                for (int k = 0; k < CW; ++k) { kbuf[1][k] = kbuf[0][k]; vbuf[1][k] = vbuf[0][k]; }
                kscale[1] = kscale[0];
                vscale[1] = vscale[0];
                if (more) issue(j0 + TPS, 0);
            }
            const int rs = SPI == 2 ? cur : 1;
            const uint32_t* kc = kbuf[rs];
            const uint32_t* vc = vbuf[rs];
            {
                uint32_t* dst = (uint32_t*)(my_stage + ((st * TPS + tl) * LPT + c) * SLOT);
#pragma unroll
                for (int k = 0; k < CW; ++k) dst[k] = vc[k];
            }
            dvs[st] = vscale[rs];
            const int j = j0 + tl;
            mv[st] = 0.0f;
            if (a.mask_mode == kMaskExplicit && j < j_end)
                mv[st] = f16_to_f32(*(const uint16_t*)(mrow + 2 * (int64_t)j)) * kLog2e;
            live[st] = j < j_end && mv[st] != -INFINITY;
            if constexpr (Q8) {
                uint32_t kq[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) kq[k] = __builtin_amdgcn_alignbyte(kc[k + 1], kc[k], ksh);
                const float dk = kscale[rs];
#pragma unroll
                for (int hh = 0; hh < G; ++hh) {
                    int si = 0;
#pragma unroll
                    for (int k = 0; k < 8; ++k) si = __builtin_amdgcn_sdot4((int)qw[hh][k], (int)kq[k], si, false);
                    sc[st][hh] = (float)si * (dk * qd[hh]);
                }
            } else {
#pragma unroll
                for (int hh = 0; hh < G; ++hh) {
                    float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
                    for (int k = 0; k < 16; k += 2) {
                        if constexpr (KT == VVA_TYPE_BF16) {
                            d0 = dot2_bf16(qw[hh][k], kc[k], d0);
                            d1 = dot2_bf16(qw[hh][k + 1], kc[k + 1], d1);
                        } else {
                            d0 = dot2_f16(qw[hh][k], kc[k], d0);
                            d1 = dot2_f16(qw[hh][k + 1], kc[k + 1], d1);
                        }
                    }
                    sc[st][hh] = (d0 + d1) * qd[hh];
                }
            }
        }
        {
            float* flat = &sc[0][0];
            float (&all)[SPI * G] = *reinterpret_cast<float (*)[SPI * G]>(flat);
            key_sum<LPT, SPI * G>(all);
        }
        if (a.mask_mode == kMaskExplicit) {
#pragma unroll
            for (int st = 0; st < SPI; ++st)
#pragma unroll
                for (int hh = 0; hh < G; ++hh) sc[st][hh] += mv[st];
        }
#pragma unroll
        for (int st = 0; st < SPI; ++st)
#pragma unroll
            for (int hh = 0; hh < G; ++hh) sc[st][hh] = live[st] ? sc[st][hh] : -INFINITY;
        // ---------------- online softmax, running max raised lazily
        bool raise = false;
#pragma unroll
        for (int hh = 0; hh < G; ++hh) {
            float x = sc[0][hh];
#pragma unroll
            for (int st = 1; st < SPI; ++st) x = fmaxf(x, sc[st][hh]);
            raise |= x > m[hh] + kLazy;
        }
        if (__any(raise)) {
            float cm[G];
#pragma unroll
            for (int hh = 0; hh < G; ++hh) {
                cm[hh] = sc[0][hh];
#pragma unroll
                for (int st = 1; st < SPI; ++st) cm[hh] = fmaxf(cm[hh], sc[st][hh]);
            }
            keys_max<LPT, G>(cm);
#pragma unroll
            for (int hh = 0; hh < G; ++hh) {
                if (cm[hh] > m[hh] + kLazy) {
                    const float alpha = __builtin_amdgcn_exp2f(m[hh] - cm[hh]);   // 0 when m = -inf
                    l[hh] *= alpha;
#pragma unroll
                    for (int e = 0; e < DV; ++e) acc[hh][e] *= alpha;
                    m[hh] = cm[hh];
                }
            }
        }
#pragma unroll
        for (int hh = 0; hh < G; ++hh) {
            const float base = m[hh] == -INFINITY ? 0.0f : m[hh];
            float ls = 0.0f;
#pragma unroll
            for (int st = 0; st < SPI; ++st) {
                const float pv = __builtin_amdgcn_exp2f(sc[st][hh] - base);  // 0 when masked
                sc[st][hh] = pv;
                ls += pv;
            }
            l[hh] += ls;              // every lane of a key adds it: divided by LPT at the end
        }
#pragma unroll
        for (int st = 0; st < SPI; ++st) {
            const int u = st * TPS + tl;
            uint16_t* dst = (uint16_t*)&pbuf[w][c][u >> 1][0] + (u & 1);
#pragma unroll
            for (int hh = 0; hh < G; ++hh) dst[2 * hh] = f32_to_f16(sc[st][hh] * dvs[st]);
        }
        wave_lds_sync();
        // ---------------- V phase: lane owns dims [lane*DV, lane*DV + DV)
        const int dim0 = lane * DV;
        const int cc = dim0 / 32, e0 = dim0 % 32;
        const int voff = Chunk<KT>::shift(cc) + (Q8 ? e0 : 2 * e0);
#pragma unroll
        for (int u = 0; u < TPI; u += 2) {
            const char* s0 = my_stage + (u * LPT + cc) * SLOT + voff;
            const char* s1 = s0 + LPT * SLOT;
            uint32_t x[DV];                   // f16 pairs (key u, key u+1) per owned dim
            typedef _Float16 hv2 __attribute__((ext_vector_type(2)));
            if constexpr (Q8) {
                if constexpr (DV == 2) {
                    const uint32_t w0 = *(const uint16_t*)s0;
                    const uint32_t w1 = *(const uint16_t*)s1;
                    hv2 a0 = {code_f16(w0 & 0xff), code_f16(w1 & 0xff)};
                    hv2 a1 = {code_f16(w0 >> 8), code_f16(w1 >> 8)};
                    __builtin_memcpy(&x[0], &a0, 4);
                    __builtin_memcpy(&x[1], &a1, 4);
                } else {
                    hv2 a0 = {code_f16((uint8_t)s0[0]), code_f16((uint8_t)s1[0])};
                    __builtin_memcpy(&x[0], &a0, 4);
                }
            } else {
                if constexpr (DV == 2) {
                    uint32_t w0 = *(const uint32_t*)s0;
                    uint32_t w1 = *(const uint32_t*)s1;
                    if constexpr (KT == VVA_TYPE_BF16) {
                        w0 = pack2<VVA_TYPE_F16>(bf16_to_f32(w0 & 0xffffu), bf16_to_f32(w0 >> 16));
                        w1 = pack2<VVA_TYPE_F16>(bf16_to_f32(w1 & 0xffffu), bf16_to_f32(w1 >> 16));
                    }
                    x[0] = (w0 & 0xffffu) | (w1 << 16);
                    x[1] = (w0 >> 16) | (w1 & 0xffff0000u);
                } else {
                    uint32_t w0 = *(const uint16_t*)s0;
                    uint32_t w1 = *(const uint16_t*)s1;
                    if constexpr (KT == VVA_TYPE_BF16) {
                        w0 = f32_to_f16(bf16_to_f32(w0));
                        w1 = f32_to_f16(bf16_to_f32(w1));
                    }
                    x[0] = w0 | (w1 << 16);
                }
            }
            uint32_t pw[GP];
            const uint32_t* prow = &pbuf[w][cc][u >> 1][0];
            if constexpr (GP % 4 == 0) {
#pragma unroll
                for (int k = 0; k < GP; k += 4) {
                    const uint4 q4 = *(const uint4*)(prow + k);
                    pw[k] = q4.x; pw[k + 1] = q4.y; pw[k + 2] = q4.z; pw[k + 3] = q4.w;
                }
            } else {
#pragma unroll
                for (int k = 0; k < GP; ++k) pw[k] = prow[k];
            }
#pragma unroll
            for (int hh = 0; hh < G; ++hh)
#pragma unroll
                for (int e = 0; e < DV; ++e) acc[hh][e] = dot2_f16(pw[hh], x[e], acc[hh][e]);
        }
        wave_lds_sync();
    }

    // l over the lanes (each key counted by its LPT lanes)
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
#pragma unroll
        for (int msk = 1; msk < 64; msk <<= 1) l[hh] += __shfl_xor(l[hh], msk, 64);
        l[hh] *= 1.0f / LPT;
    }

    // ---- merge the R waves of each kv head (log-sum-exp) through LDS
    float (*abuf)[G][D] = (float (*)[G][D])smem;
    if (R > 1) {
        __syncthreads();                    // every wave is done with its V staging
        if (r > 0) {
#pragma unroll
            for (int hh = 0; hh < G; ++hh) {
                if (lane == 0) { mbuf[w][hh] = m[hh]; lbuf[w][hh] = l[hh]; }
#pragma unroll
                for (int e = 0; e < DV; ++e) abuf[w][hh][lane * DV + e] = acc[hh][e];
            }
        }
        __syncthreads();
        if (r > 0) return;
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
                for (int e = 0; e < DV; ++e) acc[hh][e] = acc[hh][e] * fa + abuf[ow][hh][lane * DV + e] * fb;
                m[hh] = mn;
            }
        }
    }
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
    float* wacc = ws;
    float* wml = ws + (size_t)a.B * a.Hq * n_splits * D;
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
        const size_t idx = ((size_t)b * a.Hq + (h0 + hh)) * n_splits + split;
#pragma unroll
        for (int e = 0; e < DV; ++e) wacc[idx * D + lane * DV + e] = acc[hh][e];
        if (lane == 0) { wml[idx * 2] = m[hh]; wml[idx * 2 + 1] = l[hh]; }
    }
}

// One workgroup of 1024 threads per (query head, batch): the split maxima go
// through LDS once, then 1024 / D groups of D threads each keep up to
// kMergeDepth partial rows in flight (clamped unconditional loads, so they
// issue together) and their sums meet in LDS.
constexpr int kMergeThreads = 1024;
constexpr int kMergeDepth = 16;

template <int D>
__global__ void __launch_bounds__(kMergeThreads) decode_merge_kernel(AttnArgs a, const float* __restrict__ ws,
                                                                     int n_splits) {
    constexpr int NG = kMergeThreads / D;
    __shared__ float wmax[kMergeThreads / 64];
    __shared__ float num_s[NG][D];
    __shared__ float den_s[NG];
    const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
    const int grp = tid / D, i = tid % D;
    const float* wacc = ws;
    const float* wml = ws + (size_t)a.B * a.Hq * n_splits * D;
    const size_t base = ((size_t)b * a.Hq + h) * n_splits;
    float M = -INFINITY;
    for (int s = tid; s < n_splits; s += kMergeThreads) M = fmaxf(M, wml[(base + s) * 2]);
#pragma unroll
    for (int msk = 32; msk >= 1; msk >>= 1) M = fmaxf(M, __shfl_xor(M, msk, 64));
    if ((tid & 63) == 0) wmax[tid >> 6] = M;
    __syncthreads();
    M = wmax[0];
#pragma unroll
    for (int k = 1; k < kMergeThreads / 64; ++k) M = fmaxf(M, wmax[k]);
    float num = 0.0f, den = 0.0f;
    if (M != -INFINITY) {
        for (int s0 = grp; s0 < n_splits; s0 += NG * kMergeDepth) {
            float av[kMergeDepth], mv[kMergeDepth], lv[kMergeDepth];
#pragma unroll
            for (int k = 0; k < kMergeDepth; ++k) {
                const size_t id = base + min(s0 + k * NG, n_splits - 1);
                av[k] = wacc[id * D + i];
                mv[k] = wml[id * 2];
                lv[k] = wml[id * 2 + 1];
            }
#pragma unroll
            for (int k = 0; k < kMergeDepth; ++k) {
                const float f = s0 + k * NG < n_splits ? __builtin_amdgcn_exp2f(mv[k] - M) : 0.0f;
                num = fmaf(av[k], f, num);
                den = fmaf(lv[k], f, den);
            }
        }
    }
    num_s[grp][i] = num;
    if (i == 0) den_s[grp] = den;
    __syncthreads();
    if (grp == 0) {
        float n = 0.0f, d = 0.0f;
#pragma unroll
        for (int k = 0; k < NG; ++k) { n += num_s[k][i]; d += den_s[k]; }
        float* orow = (float*)((char*)a.out + b * a.o_nb_b + h * a.o_nb_h);
        orow[i] = d == 0.0f ? 0.0f : n / d;
    }
}

template <int D, int KT>
hipError_t launch_dg(const AttnArgs& a, float* ws, int n_splits, int split_len, hipStream_t s) {
    dim3 grid(n_splits, a.B), block(kWaves * 64);
    switch (a.Hq / a.Hkv) {
#define VVA_DG(G) case G: hipLaunchKernelGGL((decode_kernel<D, G, KT>), grid, block, 0, s, a, ws, n_splits, split_len); break;
        VVA_DG(1) VVA_DG(2) VVA_DG(3) VVA_DG(4) VVA_DG(5) VVA_DG(6) VVA_DG(7) VVA_DG(8)
#undef VVA_DG
        default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || n_splits == 1) return e;
    hipLaunchKernelGGL(decode_merge_kernel<D>, dim3(a.Hq, a.B), dim3(kMergeThreads), 0, s, a, ws, n_splits);
    return hipGetLastError();
}

}  // namespace

int decode_waves(const AttnArgs&) { return kWaves; }
int decode_max_splits() { return kMaxSplits; }

bool decode_supported(const AttnArgs& a) {
    if (a.T != 1) return false;
    if (a.d != 64 && a.d != 128) return false;
    if (a.k_type != a.v_type) return false;
    if (a.k_type != VVA_TYPE_F16 && a.k_type != VVA_TYPE_BF16 && a.k_type != VVA_TYPE_Q8_0) return false;
    if (a.Hq % a.Hkv != 0 || a.Hq / a.Hkv > 8) return false;
    if (kWaves % a.Hkv != 0) return false;
    if (a.mask_mode == kMaskExplicit && (a.mask_nb_b % 2 != 0)) return false;
    // vector-load alignment of cache rows and Q rows
    const int64_t need = a.k_type == VVA_TYPE_Q8_0 ? 4 : 16;
    if (a.k_nb_tok % need || a.k_nb_head % need || a.v_nb_tok % need || a.v_nb_head % need) return false;
    for (int b = 0; b < a.B; ++b)
        if (((uintptr_t)a.k[b] % need) || ((uintptr_t)a.v[b] % need)) return false;
    if (((uintptr_t)a.q % 16) || a.q_nb_h % 16 || a.q_nb_b % 16) return false;
    return true;
}

hipError_t launch_decode(const AttnArgs& a, float* ws, int n_splits, int split_len, hipStream_t s) {
    if (a.d == 64) {
        switch (a.k_type) {
            case VVA_TYPE_F16:  return launch_dg<64, VVA_TYPE_F16>(a, ws, n_splits, split_len, s);
            case VVA_TYPE_BF16: return launch_dg<64, VVA_TYPE_BF16>(a, ws, n_splits, split_len, s);
            case VVA_TYPE_Q8_0: return launch_dg<64, VVA_TYPE_Q8_0>(a, ws, n_splits, split_len, s);
        }
    } else {
        switch (a.k_type) {
            case VVA_TYPE_F16:  return launch_dg<128, VVA_TYPE_F16>(a, ws, n_splits, split_len, s);
            case VVA_TYPE_BF16: return launch_dg<128, VVA_TYPE_BF16>(a, ws, n_splits, split_len, s);
            case VVA_TYPE_Q8_0: return launch_dg<128, VVA_TYPE_Q8_0>(a, ws, n_splits, split_len, s);
        }
    }
    return hipErrorInvalidValue;
}

}  // namespace vva
