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
// The waves of a workgroup together read whole cache rows, so no cache line
// is fetched by two CUs.  A wave walks its keys 32 at a time ("an
// iteration") in two layouts of its 64 lanes:
//
//   K phase  lane = (key, chunk of KD dims): KD = 32 for Q8_0 (one block),
//            16 for F16 / BF16.  Dots against Q rounded to K's dot type:
//            v_dot4_i32_i8 against Q quantized to Q8_0 per block (ggml's
//            Q8_0 x Q8_0 dot: integer block sums times d_k * d_q), or
//            v_dot2_f32_f16 / v_dot2_f32_bf16; DPP completes each score over
//            the key's lanes.  Online softmax in the exp2 domain with a lazy
//            running max (raised only when a score exceeds it by 2^8).  Each
//            lane writes p (times its V block scale for Q8_0) as f16 to LDS.
//   V phase  lane = (pair of dims, every key pair at d = 128; half of them
//            at d = 64).  The lane reads its 2 dims of each key straight from
//            HBM (2 bytes of Q8_0 codes or 4 bytes of F16 / BF16), turns pairs
//            of consecutive keys into f16 pairs (SDWA byte converts; int8
//            codes are exact in f16), and accumulates every head with
//            v_dot2_f32_f16 against the f16 p pairs from LDS (fp32 sums).
//
// Loads run one iteration ahead: each step's K chunk and each key's V
// bytes are re-issued for the next iteration as soon as they are consumed,
// and the first iteration's loads are issued before Q is converted.  All
// cache loads are raw buffer loads whose range ends at the wave's last key.
// At d = 64 the two halves of the key pairs are added with
// v_permlane32_swap; the waves of one kv head merge through LDS
// (log-sum-exp).  With one split the output
// is written directly; otherwise the workgroup writes (m, l, acc[d]) per head
// and decode_merge_kernel combines the splits in one pass (a second launch:
// kernel boundaries give the cross-XCD visibility that a device-scope fence
// would buy with an L2 write-back per workgroup).
#include "vva_internal.hpp"

namespace vva {

namespace {

#include "wave_ops.hpp"

constexpr float kLazy = 8.0f;      // running-max slack in log2 units: p <= 256
constexpr int kWaves = 8;
constexpr int kMaxSplits = 256;

template <int KT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    uint16_t x = KT == VVA_TYPE_BF16 ? f32_to_bf16(a) : f32_to_f16(a);
    uint16_t y = KT == VVA_TYPE_BF16 ? f32_to_bf16(b) : f32_to_f16(b);
    return (uint32_t)x | ((uint32_t)y << 16);
}
__device__ __forceinline__ float half_to_f32_rt(uint32_t v, int type) {
    return type == VVA_TYPE_BF16 ? bf16_to_f32((uint16_t)v) : f16_to_f32((uint16_t)v);
}

template <int D, int G, int KT>
struct Cfg {
    static constexpr bool Q8 = KT == VVA_TYPE_Q8_0;
    static constexpr int KD = Q8 ? 32 : 16;         // dims per lane, K phase
    static constexpr int LPT = D / KD;              // lanes per key, K phase
    static constexpr int TPS = 64 / LPT;            // keys per K step
    static constexpr int TPI = 32;                  // keys per iteration
    static constexpr int SPI = TPI / TPS;           // K steps per iteration
    static constexpr int CW = 8 + (Q8 ? 1 : 0);     // K words per lane per step
    static constexpr int QW = 8;                    // Q words per head per lane
    static constexpr int VD = 2;                    // dims per lane, V phase
    static constexpr int DG = D / VD;               // V dim groups
    static constexpr int KG = 64 / DG;              // V key groups (1 at d = 128, 2 at d = 64)
    static constexpr int PPI = TPI / 2 / KG;        // key pairs per lane per iteration
    static constexpr int NPB = Q8 ? D / 32 : 1;     // p rows per key pair (one per V block)
    static constexpr int GP = (G + 3) / 4 * 4;      // p row padded for 16-byte reads
};

// D: head dim (64 / 128); G: query heads per kv head; KT: cache type.
template <int D, int G, int KT>
__global__ void __launch_bounds__(kWaves * 64)
decode_kernel(AttnArgs a, float* __restrict__ ws, int n_splits, int split_len) {
    prefetch_kernargs<sizeof(AttnArgs)>();
    using C = Cfg<D, G, KT>;
    constexpr bool Q8 = C::Q8;
    constexpr int NW = kWaves, LPT = C::LPT, TPS = C::TPS, TPI = C::TPI, SPI = C::SPI;
    constexpr int CW = C::CW, QW = C::QW, VD = C::VD, DG = C::DG, KG = C::KG, PPI = C::PPI;
    constexpr int NPB = C::NPB, GP = C::GP;
    constexpr int QSLOT = QW + 1;
    static_assert(KG == 1 || KG == 2, "V key groups are combined with v_permlane32_swap");

    constexpr int QAREA_BYTES = 64 * LPT * QSLOT * 4;                // Hq <= 64
    constexpr int MERGE_BYTES = NW * G * D * 4;
    __shared__ __attribute__((aligned(16))) char smem[QAREA_BYTES > MERGE_BYTES ? QAREA_BYTES : MERGE_BYTES];
    // p (times the V block scale) as f16 pairs of consecutive keys:
    // [wave][V block][key pair][head]
    __shared__ __attribute__((aligned(16))) uint32_t pbuf[NW][NPB][TPI / 2][GP];
    __shared__ float mbuf[NW][G];
    __shared__ float lbuf[NW][G];

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform
    const int Hkv = a.Hkv;
    const int R = NW / Hkv;                                 // waves per kv head
    const int kvh = w % Hkv, r = w / Hkv;
    const int split = blockIdx.x, b = blockIdx.y;
    const int L = a.L[b];
    const int sub_len = split_len / R;
    const int j_begin = min(L, split * split_len + r * sub_len);
    const int j_end = min(L, j_begin + sub_len);
    const int tl = lane / LPT, c = lane % LPT;              // K-phase key, chunk
    const int dg = lane % DG, kg = lane / DG;               // V-phase dim group, key group
    const int h0 = kvh * G;

    // K and V of this kv head as raw buffers: SGPR descriptor + 32-bit
    // offsets (row offsets are wave-uniform scalars, lane offsets fixed per
    // lane).  The range ends with the wave's last key, so loads for keys at
    // or past j_end return 0 without touching memory: the next iteration's
    // loads are issued unconditionally (a branch around them would keep two
    // register sets alive), and the last one's cost no traffic.
    constexpr int HEAD_BYTES = Q8 ? D / 32 * kQ8Bytes : 2 * D;
    const uint32_t nbk = (uint32_t)a.k_nb_tok, nbv = (uint32_t)a.v_nb_tok;
    const BufRsrc krs = make_rsrc(a.k[b] + kvh * a.k_nb_head, j_end > 0 ? (uint32_t)(j_end - 1) * nbk + HEAD_BYTES : 0);
    const BufRsrc vrs = make_rsrc(a.v[b] + kvh * a.v_nb_head, j_end > 0 ? (uint32_t)(j_end - 1) * nbv + HEAD_BYTES : 0);

    // K-phase lane offsets.  Q8_0: the 32 codes of block c from the 4-byte
    // aligned address at or below them (2 x 16 B + 4 B; odd blocks, which need
    // only 8 dwords, re-read an in-block dword as the 9th), plus the K and V
    // block scales.  F16 / BF16: 2 x 16 B.
    const uint32_t ko = tl * nbk + (Q8 ? c * kQ8Bytes + ((c & 1) ? 2 : 0) : c * 32);
    const uint32_t ko9 = ko + ((c & 1) ? 28 : 32);
    const uint32_t kso = tl * nbk + c * kQ8Bytes;
    const uint32_t vso = tl * nbv + c * kQ8Bytes;
    // V-phase lane offset of dims [2dg, 2dg+2): Q8_0 codes 2 (dg mod 16) and
    // 2 (dg mod 16) + 1 of block dg / 16 (2 bytes); F16 / BF16 4 bytes.
    const uint32_t vo = 2 * kg * nbv + (Q8 ? (dg * VD) / 32 * kQ8Bytes + 2 + (dg * VD) % 32 : dg * VD * 2);

    // register sets for one iteration: K chunk per step, V dwords per key pair
    uint32_t kbuf[SPI][CW];
    float ksc[SPI], vsc[SPI];
    // V: Q8_0 codes as loaded (2 bytes), F16 / BF16 pairs (4 bytes)
    typedef std::conditional_t<Q8, uint16_t, uint32_t> vword;
    vword vbuf[PPI][2];
    auto issue_k = [&](int i0, int st) {
        const uint32_t sk = (uint32_t)(i0 + st * TPS) * nbk;
        const uint32_t sv = (uint32_t)(i0 + st * TPS) * nbv;
        const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(krs, ko, sk, 0);
        const u32x4 y = __builtin_amdgcn_raw_buffer_load_b128(krs, ko + 16, sk, 0);
        kbuf[st][0] = x.x; kbuf[st][1] = x.y; kbuf[st][2] = x.z; kbuf[st][3] = x.w;
        kbuf[st][4] = y.x; kbuf[st][5] = y.y; kbuf[st][6] = y.z; kbuf[st][7] = y.w;
        if constexpr (Q8) {
            kbuf[st][8] = __builtin_amdgcn_raw_buffer_load_b32(krs, ko9, sk, 0);
            ksc[st] = f16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(krs, kso, sk, 0));
            vsc[st] = f16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(vrs, vso, sv, 0));
        }
    };
    auto issue_v = [&](int i0, int k) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const uint32_t sv = (uint32_t)(i0 + 2 * KG * k + t) * nbv;
            if constexpr (Q8)
                vbuf[k][t] = __builtin_amdgcn_raw_buffer_load_b16(vrs, vo, sv, 0);
            else
                vbuf[k][t] = __builtin_amdgcn_raw_buffer_load_b32(vrs, vo, sv, 0);
        }
    };
    // Q, then the first iteration's K and V, go out before Q is converted:
    // one thread per (query head, KD-dim chunk) loads its chunk (threads past
    // the last chunk re-load chunk 0 so every load is unconditional)
    constexpr int KD = C::KD;
    const int qslot = threadIdx.x < a.Hq * LPT ? (int)threadIdx.x : 0;
    uint4 qraw[KD / 4];
    {
        const int hq = qslot / LPT, ch = qslot % LPT;
        const char* src = a.q + b * a.q_nb_b + hq * a.q_nb_h + (int64_t)(ch * KD) * type_elem_bytes(a.q_type);
        if (a.q_type == VVA_TYPE_F32) {
#pragma unroll
            for (int k = 0; k < KD / 4; ++k) qraw[k] = ((const uint4*)src)[k];
        } else {
#pragma unroll
            for (int k = 0; k < KD / 8; ++k) qraw[k] = ((const uint4*)src)[k];
        }
    }
#pragma unroll
    for (int st = 0; st < SPI; ++st) issue_k(j_begin, st);
#pragma unroll
    for (int k = 0; k < PPI; ++k) issue_v(j_begin, k);

    // ---- Q in K's dot type (Q8_0: codes + fp16 scale; F16 / BF16: packed
    // pairs), through LDS; each lane then reads its chunk of its g heads
    uint32_t qw[G][QW];
    float qd[G];
    {
        uint32_t* qlds = (uint32_t*)smem;
        if (threadIdx.x < a.Hq * LPT) {
            float x[KD];
            if (a.q_type == VVA_TYPE_F32) {
#pragma unroll
                for (int k = 0; k < KD / 4; ++k) {
                    const uint4 v = qraw[k];
                    x[4 * k] = __uint_as_float(v.x); x[4 * k + 1] = __uint_as_float(v.y);
                    x[4 * k + 2] = __uint_as_float(v.z); x[4 * k + 3] = __uint_as_float(v.w);
                }
            } else {
#pragma unroll
                for (int k = 0; k < KD / 8; ++k) {
                    const uint4 v = qraw[k];
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
                for (int k = 0; k < 8; ++k) dst[k] = pack2<KT>(x[2 * k], x[2 * k + 1]);
                dst[8] = __float_as_uint(1.0f);
            }
        }
        __syncthreads();
        const float sl2 = a.scale * kLog2e;      // scores come out in the exp2 domain
#pragma unroll
        for (int hh = 0; hh < G; ++hh) {
            const uint32_t* srcw = qlds + ((h0 + hh) * LPT + c) * QSLOT;
#pragma unroll
            for (int k = 0; k < QW; ++k) qw[hh][k] = srcw[k];
            qd[hh] = __uint_as_float(srcw[QW]) * sl2;
        }
        __syncthreads();                         // the area is reused by the merge
    }

    const char* mrow = a.mask ? a.mask + b * a.mask_nb_b : nullptr;   // query row 0
    const int pblk = Q8 ? (dg * VD) / 32 : 0;                          // V-phase p row

    float m[G], l[G], acc[G][VD];
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
        m[hh] = -INFINITY;
        l[hh] = 0.0f;
#pragma unroll
        for (int e = 0; e < VD; ++e) acc[hh][e] = 0.0f;
    }

    for (int i0 = j_begin; i0 < j_end; i0 += TPI) {
        // ---------------- K phase
        float sc[SPI][G];
        float dvs[SPI];
        bool live[SPI];
        float mv[SPI];
#pragma unroll
        for (int st = 0; st < SPI; ++st) {
            const int j = i0 + st * TPS + tl;
            mv[st] = 0.0f;
            if (a.mask_mode == kMaskExplicit && j < j_end)
                mv[st] = mask_at(mrow, j, a.mask_f32) * kLog2e;
            live[st] = j < j_end && mv[st] != -INFINITY;
            const uint32_t* kc = kbuf[st];
            if constexpr (Q8) {
                const int ksh = (c & 1) ? 0 : 2;
                uint32_t kq[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) kq[k] = __builtin_amdgcn_alignbyte(kc[k + 1], kc[k], ksh);
                const float dk = ksc[st];
                dvs[st] = vsc[st];
#pragma unroll
                for (int hh = 0; hh < G; ++hh) {
                    int si = sdot4_first(qw[hh][0], kq[0]);
#pragma unroll
                    for (int k = 1; k < 8; ++k) si = __builtin_amdgcn_sdot4((int)qw[hh][k], (int)kq[k], si, false);
                    sc[st][hh] = (float)si * (dk * qd[hh]);
                }
            } else {
                dvs[st] = 1.0f;
#pragma unroll
                for (int hh = 0; hh < G; ++hh) {
                    float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
                    for (int k = 0; k < 8; k += 2) {
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
            issue_k(i0 + TPI, st);
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
        // keys past the wave's range or masked to -inf: only the last
        // iteration and explicit masks have any
        if (i0 + TPI > j_end || a.mask_mode == kMaskExplicit) {
#pragma unroll
            for (int st = 0; st < SPI; ++st)
#pragma unroll
                for (int hh = 0; hh < G; ++hh) sc[st][hh] = live[st] ? sc[st][hh] : -INFINITY;
        }
        // online softmax, running max raised lazily
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
                    for (int e = 0; e < VD; ++e) acc[hh][e] *= alpha;
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
            uint16_t* dst = (uint16_t*)&pbuf[w][Q8 ? c : 0][u >> 1][0] + (u & 1);
            if constexpr (Q8) {
#pragma unroll
                for (int hh = 0; hh < G; ++hh) dst[2 * hh] = f32_to_f16(sc[st][hh] * dvs[st]);
            } else {
                // the LPT lanes of a key hold the same p: lane c writes heads c, c + LPT, ...
#pragma unroll
                for (int hh = 0; hh < G; ++hh)
                    if (hh % LPT == c) dst[2 * hh] = f32_to_f16(sc[st][hh]);
            }
        }
        wave_lds_sync();
        // ---------------- V phase: lane owns dims [2 dg, 2 dg + 2) of its key pairs
#pragma unroll
        for (int k = 0; k < PPI; ++k) {
            const int pi = kg + KG * k;
            uint32_t x[VD];           // f16 pairs (key 2 pi, key 2 pi + 1), one per dim
            const vword wa = vbuf[k][0], wb = vbuf[k][1];
            if constexpr (Q8) {
                x[0] = i8_pair_b0(wa, wb);
                x[1] = i8_pair_b1(wa, wb);
            } else if constexpr (KT == VVA_TYPE_F16) {
                x[0] = __builtin_amdgcn_perm(wb, wa, 0x05040100u);
                x[1] = __builtin_amdgcn_perm(wb, wa, 0x07060302u);
            } else {
                h2 lo = {(_Float16)__uint_as_float(wa << 16), (_Float16)__uint_as_float(wb << 16)};
                h2 hi = {(_Float16)__uint_as_float(wa & 0xffff0000u), (_Float16)__uint_as_float(wb & 0xffff0000u)};
                __builtin_memcpy(&x[0], &lo, 4);
                __builtin_memcpy(&x[1], &hi, 4);
            }
            // convert before the next iteration's load of the same key is
            // issued, so it can land in the register just freed
            __builtin_amdgcn_sched_barrier(0);
            issue_v(i0 + TPI, k);
            uint32_t pw[GP];
            const uint32_t* prow = &pbuf[w][pblk][pi][0];
#pragma unroll
            for (int q = 0; q < GP; q += 4) {
                const uint4 q4 = *(const uint4*)(prow + q);
                pw[q] = q4.x; pw[q + 1] = q4.y; pw[q + 2] = q4.z; pw[q + 3] = q4.w;
            }
#pragma unroll
            for (int hh = 0; hh < G; ++hh)
#pragma unroll
                for (int e = 0; e < VD; ++e) acc[hh][e] = dot2_f16(pw[hh], x[e], acc[hh][e]);
            // keep each pair's LDS reads next to their use: hoisting them all
            // would cost a register set per pair
            __builtin_amdgcn_sched_barrier(0);
        }
        wave_lds_sync();
    }

    // l over the lanes (each key counted by its LPT lanes); acc over the key
    // groups (lanes dg, dg + DG, ...)
#pragma unroll
    for (int hh = 0; hh < G; ++hh) l[hh] = wave_sum(l[hh]) * (1.0f / LPT);
    if constexpr (KG == 2) {
#pragma unroll
        for (int hh = 0; hh < G; ++hh)
#pragma unroll
            for (int e = 0; e < VD; ++e) acc[hh][e] = add_swap32(acc[hh][e]);
    }

    // ---- merge the R waves of each kv head (log-sum-exp) through LDS; the
    // key groups hold identical sums, the first writes
    float (*abuf)[G][D] = (float (*)[G][D])smem;
    if (R > 1) {
        if (r > 0) {
#pragma unroll
            for (int hh = 0; hh < G; ++hh) {
                if (lane == 0) { mbuf[w][hh] = m[hh]; lbuf[w][hh] = l[hh]; }
                if (kg == 0) *(float2*)&abuf[w][hh][dg * VD] = make_float2(acc[hh][0], acc[hh][1]);
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
                const float2 o = *(const float2*)&abuf[ow][hh][dg * VD];
                acc[hh][0] = acc[hh][0] * fa + o.x * fb;
                acc[hh][1] = acc[hh][1] * fa + o.y * fb;
                m[hh] = mn;
            }
        }
    }
    // the KG copies of each head's row split the stores: group kg writes heads kg, kg + KG, ...
    if (n_splits == 1) {
#pragma unroll
        for (int hh = 0; hh < G; ++hh) {
            if (hh % KG != kg) continue;
            const float inv = l[hh] == 0.0f ? 0.0f : 1.0f / l[hh];
            float* orow = (float*)((char*)a.out + b * a.o_nb_b + (h0 + hh) * a.o_nb_h);
            *(float2*)(orow + dg * VD) = make_float2(acc[hh][0] * inv, acc[hh][1] * inv);
        }
        return;
    }
    // partials: acc [B][Hq][n_splits][D], then (m, l) [B][Hq][n_splits][2]
    float* wacc = ws;
    float* wml = ws + (size_t)a.B * a.Hq * n_splits * D;
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
        if (hh % KG != kg) continue;
        const size_t idx = ((size_t)b * a.Hq + (h0 + hh)) * n_splits + split;
        *(float2*)(wacc + idx * D + dg * VD) = make_float2(acc[hh][0], acc[hh][1]);
        if (dg == 0) *(float2*)(wml + idx * 2) = make_float2(m[hh], l[hh]);
    }
}

// One workgroup of 256 threads per (32-dim quarter, query head, sequence):
// NG = 32 groups of 8 threads (one float4 of the quarter each) take every
// NG-th split, with up to kMergeDepth partial rows in flight at once.  The
// row max M over all splits is found first (in-wave DPP / permlane steps,
// then the 4 waves through LDS); each thread then weighs its rows by
// exp2(m - M), and the 32 groups' sums meet by cross-lane adds within each
// wave and one LDS step across the waves.  For n_splits <= NG * kMergeDepth
// (128) every load goes out in one round trip; the quarter split puts D/32
// workgroups on each row so the round trips of one row run on several CUs.
constexpr int kMergeThreads = 256;
constexpr int kMergeDepth = 4;
constexpr int kMergeDims = 32;
constexpr int kDppRowRor8 = 0x128;

template <int D>
__global__ void __launch_bounds__(kMergeThreads) decode_merge_kernel(AttnArgs a, const float* __restrict__ ws,
                                                                     int n_splits) {
    prefetch_kernargs<sizeof(AttnArgs)>();
    constexpr int TPR = kMergeDims / 4;         // threads per partial row quarter
    constexpr int NG = kMergeThreads / TPR;     // row groups
    constexpr int NW = kMergeThreads / 64;
    __shared__ float smax[NW];
    __shared__ float4 snum[NW][TPR];
    __shared__ float sden[NW];
    const int h = blockIdx.x, b = blockIdx.y, q4 = blockIdx.z;
    const int grp = threadIdx.x / TPR, i4 = threadIdx.x % TPR;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const size_t base = ((size_t)b * a.Hq + h) * n_splits;
    const float4* wacc = (const float4*)ws + base * (D / 4) + q4 * TPR;
    const float* wml = ws + (size_t)a.B * a.Hq * n_splits * D + base * 2;
    float M = -INFINITY, den = 0.0f;
    float4 num = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    // first round (all rows when n_splits <= 128): loads, then the global max
    float4 av[kMergeDepth];
    float mv[kMergeDepth], lv[kMergeDepth];
#pragma unroll
    for (int k = 0; k < kMergeDepth; ++k) {
        const int s = min(grp + k * NG, n_splits - 1);     // clamped: unconditional loads
        av[k] = wacc[(size_t)s * (D / 4) + i4];
        const float2 ml = *(const float2*)(wml + 2 * s);
        mv[k] = grp + k * NG < n_splits ? ml.x : -INFINITY;
        lv[k] = ml.y;
    }
    float mt = -INFINITY;
#pragma unroll
    for (int k = 0; k < kMergeDepth; ++k) mt = fmaxf(mt, mv[k]);
    for (int s0 = grp + NG * kMergeDepth; s0 < n_splits; s0 += NG) {   // more than 128 splits
        const float2 ml = *(const float2*)(wml + 2 * s0);
        mt = fmaxf(mt, ml.x);
    }
    mt = fmaxf(mt, dpp<kDppRowRor8>(mt));
    mt = max_swap32(max_swap16(mt));
    if (lane == 0) smax[wv] = mt;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, smax[w]);
    if (M != -INFINITY) {
        auto add = [&](float m, float l, const float4& v) {
            const float f = __builtin_amdgcn_exp2f(m - M);     // 0 for -inf
            num.x = fmaf(v.x, f, num.x);
            num.y = fmaf(v.y, f, num.y);
            num.z = fmaf(v.z, f, num.z);
            num.w = fmaf(v.w, f, num.w);
            den = fmaf(l, f, den);
        };
#pragma unroll
        for (int k = 0; k < kMergeDepth; ++k) add(mv[k], lv[k], av[k]);
        for (int s0 = grp + NG * kMergeDepth; s0 < n_splits; s0 += NG) {
            const float2 ml = *(const float2*)(wml + 2 * s0);
            add(ml.x, ml.y, wacc[(size_t)s0 * (D / 4) + i4]);
        }
    }
    // sum over the 8 groups of the wave (lanes i4, i4 + 8, ..., i4 + 56)
    auto gsum = [](float x) { return add_swap32(add_swap16(x + dpp<kDppRowRor8>(x))); };
    num.x = gsum(num.x);
    num.y = gsum(num.y);
    num.z = gsum(num.z);
    num.w = gsum(num.w);
    den = gsum(den);
    if (lane < TPR) {
        snum[wv][lane] = num;
        if (lane == 0) sden[wv] = den;
    }
    __syncthreads();
    if (threadIdx.x >= TPR) return;
    float4 n = snum[0][i4];
    float d = sden[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) {
        const float4 v = snum[w][i4];
        n.x += v.x; n.y += v.y; n.z += v.z; n.w += v.w;
        d += sden[w];
    }
    const float inv = d == 0.0f ? 0.0f : 1.0f / d;
    float* orow = (float*)((char*)a.out + b * a.o_nb_b + h * a.o_nb_h) + q4 * kMergeDims;
    *(float4*)(orow + 4 * i4) = make_float4(n.x * inv, n.y * inv, n.z * inv, n.w * inv);
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
    hipLaunchKernelGGL(decode_merge_kernel<D>, dim3(a.Hq, a.B, D / kMergeDims), dim3(kMergeThreads), 0, s, a, ws, n_splits);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_decode_merge(const AttnArgs& a, const float* ws, int n_splits, hipStream_t s) {
    if (a.d == 64)
        hipLaunchKernelGGL(decode_merge_kernel<64>, dim3(a.Hq, a.B, 64 / kMergeDims), dim3(kMergeThreads), 0, s, a, ws, n_splits);
    else if (a.d == 128)
        hipLaunchKernelGGL(decode_merge_kernel<128>, dim3(a.Hq, a.B, 128 / kMergeDims), dim3(kMergeThreads), 0, s, a, ws, n_splits);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

int decode_waves(const AttnArgs&) { return kWaves; }
int decode_max_splits() { return kMaxSplits; }

bool decode_supported(const AttnArgs& a) {
    if (a.T != 1) return false;
    if (a.d != 64 && a.d != 128) return false;
    if (a.k_type != a.v_type) return false;
    if (a.k_type != VVA_TYPE_F16 && a.k_type != VVA_TYPE_BF16 && a.k_type != VVA_TYPE_Q8_0) return false;
    if (a.Hq % a.Hkv != 0 || a.Hq / a.Hkv > 8) return false;
    if (kWaves % a.Hkv != 0) return false;
    if (a.mask_mode == kMaskExplicit && (a.mask_nb_b % (a.mask_f32 ? 4 : 2) != 0)) return false;
    // vector-load alignment of cache rows, Q rows and output rows
    const int64_t need = a.k_type == VVA_TYPE_Q8_0 ? 4 : 16;
    if (a.k_nb_tok % need || a.k_nb_head % need || a.v_nb_tok % need || a.v_nb_head % need) return false;
    for (int b = 0; b < a.B; ++b)
        if (((uintptr_t)a.k[b] % need) || ((uintptr_t)a.v[b] % need)) return false;
    // 32-bit buffer offsets: rows up to one iteration past the last key
    for (int b = 0; b < a.B; ++b)
        if ((int64_t)(a.L[b] + 64) * a.k_nb_tok >= ((int64_t)1 << 31) ||
            (int64_t)(a.L[b] + 64) * a.v_nb_tok >= ((int64_t)1 << 31)) return false;
    if (((uintptr_t)a.q % 16) || a.q_nb_h % 16 || a.q_nb_b % 16) return false;
    if (((uintptr_t)a.out % 16) || a.o_nb_h % 16 || a.o_nb_b % 16) return false;
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
