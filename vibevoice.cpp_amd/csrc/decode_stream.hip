// decode_stream.hip — split-K single-token attention (T == 1) over a dense
// Q8_0 KV cache: the per-step attention of the ASR / TTS decode loops
// (src/vibevoice_asr.cpp:760-800, src/vibevoice_tts.cpp:862-880), i.e.
// ggml_flash_attn_ext with one query row per head (src/qwen2.cpp:332-334)
// on Q8_0 K/V.
//
// Streaming.  Every workgroup (8 waves, one per CU) takes a contiguous key
// range of one sequence and streams it through a 4-stage LDS ring filled by
// buffer_load_dwordx4 ... lds, so three tiles (102 KB per CU) are on their
// way from HBM while one is computed.  A tile is 512 (key, kv head, 32-dim
// block) rows of the cache = 17,408 B of K plus the same of V, read as the
// cache lays them out ([token][kv head][34-byte GGUF block]): one contiguous
// byte range per operand, 1 KB per wave instruction.  The buffer ranges of
// a split end at its last key, so chunks past it come back as zeros without
// a memory access.
//
// Arithmetic on the matrix cores.  With g = 7 query heads per kv head, the
// VALU form of this loop (v_dot4 scores, v_dot2 P.V) needs ~800 VALU lane
// operations per (key, kv head) and runs VALU-bound at about a third of
// HBM speed; on MFMA the VALU keeps only the conversions and the softmax.
// Per tile, wave w takes kv head w % Hkv and 16 (d = 128) or 32 (d = 64) of
// the tile's keys, in groups of 16 keys; lane = (g = lane / 16, n = lane % 16).
// MFMA row/column m of a group stands for its key sigma(m) = 4 (m % 4) +
// m / 4, so lane group g works on keys g, g + 4, g + 8, g + 12: with the
// cache's 544-byte token rows the four groups' LDS reads then fall in
// different banks.
//   scores  S^T[key][row] per 32-dim block b with v_mfma_i32_16x16x32_i8:
//           A = the K codes of block b (lane: key sigma(n), codes 8g..8g+7),
//           B = Q quantized to Q8_0 (lane: row n, same codes), so each
//           block's dot is ggml's exact integer Q8_0 x Q8_0 block sum; the
//           lane receives keys sigma(4g + i) of row n and scales them by
//           d_k * d_q in fp32.
//   softmax fp32, exp2 domain, one row per lane (max over the row's 16 keys:
//           in-lane, then two permlane swaps).  The running max is raised
//           only when a score exceeds it by 2^8.
//   P.V     O^T[dim][row] += V^T P'^T with v_mfma_f32_16x16x16_f16 per 16
//           dims: A = V codes (exact in f16; lane: dims 2n, 2n+1 of block b,
//           keys sigma(4g + i)), B = P' = p * d_v(key, b) as f16 — the score
//           accumulator layout is already B's layout, so P never leaves the
//           registers.  MFMA j = 2b + s holds dims 32b + 2m + s in its row m.
// The waves of one kv head merge through LDS (log-sum-exp); the workgroup
// writes (m, l, acc[d]) per query head, or the output when there is one
// split, and decode_merge_kernel (decode.hip) combines the splits.
#include "vva_internal.hpp"

#include <type_traits>

namespace vva {

namespace {

#include "wave_ops.hpp"

typedef __attribute__((address_space(3))) char lds_char;
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kW = 8;                        // waves per workgroup
constexpr int kStages = 4;                   // LDS ring depth (power of 2)
constexpr int kTileOpBytes = 17408;          // one operand of a tile: 512 Q8_0 blocks
constexpr int kOpChunks = 18;                // 1 KB chunks per operand: 17 KB + alignment slack
constexpr int kOpBytes = kOpChunks * 1024;
constexpr int kStage = 2 * kOpBytes;         // K, then V
constexpr int kJunk = kStages * kStage;      // 1 KB target of the padding loads
constexpr int kLdsBytes = kJunk + 1024;
constexpr int kLoads = (2 * kOpChunks + kW - 1) / kW;   // DMA loads per wave per tile
constexpr int kQLoads = 3;                   // DMA loads per wave for the raw Q rows
constexpr int kQRawBytes = kQLoads * kW * 1024;   // raw Q area: up to 24 KB
constexpr int kDead = 0x40000000;            // buffer offset past every range
constexpr float kLazy = 8.0f;                // running-max slack in log2 units: p <= 256
static_assert(kLdsBytes <= 160 * 1024, "LDS budget");

// buffer_load_dwordx4 ... lds: each lane's 16 bytes land at LDS address
// m0 + 16 * lane.  Inline asm, so the compiler neither fences LDS reads on it
// nor waits for it; completion is awaited explicitly (wait_vm_barrier).  The
// whole offset is in the VGPR (soffset 0), so the range check sees all of it.
// STREAM marks the load non-temporal: the cache is read once, so its lines
// should not displace what the next call reads again (Q, the partials).
template <bool STREAM = false>
__device__ __forceinline__ void dma16(i32x4 rsrc, uint32_t lds_addr, int voffset) {
    if constexpr (STREAM)
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 4\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds"
                     :
                     : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voffset), "s"(rsrc)
                     : "memory", "m0");
    else
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 4\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                     :
                     : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voffset), "s"(rsrc)
                     : "memory", "m0");
}

// wait until at most N of this wave's loads are outstanding (and its LDS
// operations are done), then meet the workgroup at a barrier
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(N) : "memory");
}

// f16 half HI of dword `h` times f32 `x` (v_fma_mix_f32 reads the half in
// place: no conversion or extraction instruction).  The result feeds VALU
// instructions only.
template <int HI>
__device__ __forceinline__ float mix_mul(uint32_t h, float x) {
    float r;
    if constexpr (HI)
        asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(x));
    else
        asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[0,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(x));
    return r;
}

__device__ __forceinline__ h2 as_h2(uint16_t lo, uint16_t hi) {
    const uint32_t u = (uint32_t)lo | ((uint32_t)hi << 16);
    h2 v;
    __builtin_memcpy(&v, &u, 4);
    return v;
}
__device__ __forceinline__ h4 as_h4(uint32_t lo, uint32_t hi) {
    const uint64_t u = (uint64_t)lo | ((uint64_t)hi << 32);
    h4 v;
    __builtin_memcpy(&v, &u, 8);
    return v;
}
__device__ __forceinline__ h4 cat_h4(h2 lo, h2 hi) { return h4{lo[0], lo[1], hi[0], hi[1]}; }

// D: head dim (64 / 128); HKV: kv heads (1, 2, 4, 8), which fixes the token
// row pitch, so every LDS offset inside a tile is a constant.
template <int D, int HKV>
__global__ void __launch_bounds__(kW * 64)
decode_stream_kernel(AttnArgs a, float* __restrict__ ws, int n_splits, int split_len) {
    constexpr int NB = D / 32;                // Q8_0 blocks per head row
    constexpr int HB = NB * kQ8Bytes;         // bytes per head row
    constexpr int NSUB = 128 / D;             // groups of 16 keys per wave per tile
    constexpr int KPW = 16 * NSUB;            // keys per wave per tile
    constexpr int NJ = 2 * NB;                // P.V MFMAs (16 dims each) per key group
    static_assert(KPW * kW * HB == kTileOpBytes, "tile size");
    static_assert(kW % HKV == 0, "whole waves per kv head");

    __shared__ __attribute__((aligned(16))) char lds[kLdsBytes];

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, n = lane & 15;
    constexpr int R = kW / HKV;               // waves per kv head
    constexpr int RB = HKV * HB;              // bytes per token row (all kv heads)
    const int G = a.Hq / HKV;                 // query heads per kv head (<= 16)
    const int h = w % HKV, r = w / HKV;
    const int TT = KPW * R;                   // keys per tile
    const int split = blockIdx.x, b = blockIdx.y;
    const int L = a.L[b];
    const int j0 = min(L, split * split_len);
    const int j1 = min(L, j0 + split_len);
    const int n_tiles = (j1 - j0 + TT - 1) / TT;

    // One raw buffer per operand: from the 16-byte boundary at or below the
    // split's first row to its last row.  delta = the row start's offset
    // from that boundary (a multiple of 4), also its offset in the LDS tile.
    const char* kfirst = a.k[b] + (int64_t)j0 * RB;
    const char* vfirst = a.v[b] + (int64_t)j0 * RB;
    const int dk = (int)((uintptr_t)kfirst & 15), dv = (int)((uintptr_t)vfirst & 15);
    const uint32_t span = (uint32_t)(j1 - j0) * (uint32_t)RB;
    const i32x4 krs = make_rsrc_sgpr(kfirst - dk, dk + span);
    const i32x4 vrs = make_rsrc_sgpr(vfirst - dv, dv + span);
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_char*)lds;

    // Tile t of an operand is bytes [t * 17408, t * 17408 + 18 KB) of its
    // buffer, chunk c (1 KB) loaded by wave c % kW as its (c / kW)-th load.
    // Every wave issues kLoads loads per tile: the 36 chunks of K and V, then
    // padding loads (from past the range: zeros, no memory access) into the
    // junk kilobyte.  A tile past the last one loads nothing but zeros; the
    // 18th chunk of an operand is needed only when delta > 0.  The plan of
    // each of the wave's loads (operand, LDS offset, whether it ever fetches)
    // is fixed for the kernel, so a tile's issue has no branches.
    i32x4 lrs[kLoads];
    uint32_t llds[kLoads], lstage[kLoads];
    int loff[kLoads];
    bool lvalid[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const int c = i * kW + w;
        const bool isk = c < kOpChunks, isv = !isk && c < 2 * kOpChunks;
        const int cc = isk ? c : c - kOpChunks;
        lrs[i] = isv ? vrs : krs;
        llds[i] = isk ? (uint32_t)(c * 1024) : isv ? (uint32_t)(kOpBytes + cc * 1024) : (uint32_t)kJunk;
        lstage[i] = isk || isv ? 0xffffffffu : 0u;
        loff[i] = cc * 1024;
        lvalid[i] = (isk && (cc < kOpChunks - 1 || dk > 0)) || (isv && (cc < kOpChunks - 1 || dv > 0));
    }
    auto issue = [&](int t) {
        const bool live = t < n_tiles;
        const uint32_t st = (uint32_t)(t & (kStages - 1)) * kStage;
        const int tb = t * kTileOpBytes + lane * 16;
#pragma unroll
        for (int i = 0; i < kLoads; ++i)
            dma16<true>(lrs[i], lds0 + (st & lstage[i]) + llds[i], live && lvalid[i] ? tb + loff[i] : kDead);
    };

    // ---- Q: its rows (contiguous, at most 24 KB) are DMA'd first into the
    // ring's last stage, which the loop does not load before its first
    // barrier, then tile 0 goes out.  Once the wave's own Q loads have landed
    // (they were issued first) and the workgroup has met, Q is quantized to
    // Q8_0 blocks (codes + fp16-rounded scale) next to the raw rows, and
    // tiles 1 and 2 go out.  Four adjacent lanes share a block (8 values each; the block max
    // over the quad by DPP); with more than 128 blocks a thread takes a
    // second quarter.
    const int eb = (int)type_elem_bytes(a.q_type);
    {
        const i32x4 qrs = make_rsrc_sgpr(a.q + b * a.q_nb_b, (uint32_t)(a.Hq * D * eb));
#pragma unroll
        for (int i = 0; i < kQLoads; ++i) {
            const int c = i * kW + w;
            dma16(qrs, lds0 + (kStages - 1) * kStage + c * 1024, c * 1024 + lane * 16);
        }
    }
    // only tile 0 goes out with Q: the fewer requests ahead of Q's, the
    // sooner the quantization starts
    issue(0);
    wait_vm_barrier<kLoads>();

    const char* qraw = lds + (kStages - 1) * kStage;
    uint32_t* qlds = (uint32_t*)(lds + (kStages - 1) * kStage + kQRawBytes);
    constexpr int QI = 2;                             // quarters per thread (Hq * NB <= 256)
    const int nqi = a.Hq * NB * 4;
#pragma unroll
    for (int it = 0; it < QI; ++it) {
        if (it * kW * 64 >= nqi) break;               // uniform
        const int t = (int)threadIdx.x + it * kW * 64;
        const int tt = t < nqi ? t : 0;
        const char* src = qraw + (int64_t)((tt >> 2) * 32 + (tt & 3) * 8) * eb;   // block tt/4, quarter tt%4
        float x[8];
        if (a.q_type == VVA_TYPE_F32) {
            const uint4 u0 = ((const uint4*)src)[0], u1 = ((const uint4*)src)[1];
            x[0] = __uint_as_float(u0.x); x[1] = __uint_as_float(u0.y);
            x[2] = __uint_as_float(u0.z); x[3] = __uint_as_float(u0.w);
            x[4] = __uint_as_float(u1.x); x[5] = __uint_as_float(u1.y);
            x[6] = __uint_as_float(u1.z); x[7] = __uint_as_float(u1.w);
        } else {
            const bool bf = a.q_type == VVA_TYPE_BF16;
            const uint4 u0 = ((const uint4*)src)[0];
            const uint32_t wv[4] = {u0.x, u0.y, u0.z, u0.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint16_t lo = (uint16_t)(wv[e] & 0xffffu), hi = (uint16_t)(wv[e] >> 16);
                x[2 * e] = bf ? bf16_to_f32(lo) : f16_to_f32(lo);
                x[2 * e + 1] = bf ? bf16_to_f32(hi) : f16_to_f32(hi);
            }
        }
        float am = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) am = fmaxf(am, fabsf(x[i]));
        am = fmaxf(am, dpp<kDppXor1>(am));
        am = fmaxf(am, dpp<kDppXor2>(am));
        const float dq = am / 127.0f;
        const float id = dq != 0.0f ? 1.0f / dq : 0.0f;
        uint32_t c[2] = {0, 0};
#pragma unroll
        for (int i = 0; i < 8; ++i) c[i >> 2] |= ((uint32_t)(uint8_t)(int8_t)roundf(x[i] * id)) << (8 * (i & 3));
        if (t < nqi) {
            uint32_t* dst = qlds + (t >> 2) * 9;
            dst[2 * (t & 3)] = c[0];
            dst[2 * (t & 3) + 1] = c[1];
            if ((t & 3) == 0) dst[8] = __float_as_uint(f16_to_f32(f32_to_f16(dq)));
        }
    }
#pragma unroll
    for (int t = 1; t < kStages - 1; ++t) issue(t);
    // LDS only: the tile loads stay in flight
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory");

    // B operand of the score MFMAs: row n's Q codes 8g..8g+7 of each block,
    // and its block scales times scale * log2(e) (rows past g are zero)
    long qb[NB];
    float qd[NB];
    {
        const float sl2 = a.scale * kLog2e;          // scores come out in the exp2 domain
#pragma unroll
        for (int bb = 0; bb < NB; ++bb) {
            qb[bb] = 0;
            qd[bb] = 0.0f;
            if (n < G) {
                const uint32_t* src = qlds + ((h * G + n) * NB + bb) * 9;
                qb[bb] = (long)((uint64_t)src[2 * g] | ((uint64_t)src[2 * g + 1] << 32));
                qd[bb] = __uint_as_float(src[8]) * sl2;
            }
        }
    }

    float m = -INFINITY, l = 0.0f;            // row n's running max (log2 domain) and sum
    float mb = 0.0f;                          // m, or 0 while m = -inf: the exp2 base
    f32x4 acc[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const char* mrow = a.mask_mode == kMaskExplicit ? a.mask + b * a.mask_nb_b : nullptr;   // query row 0
    const int ka_off = (4 * (n & 3) + (n >> 2)) * RB;       // A-operand key sigma(n) of a group
    const int kc_off = g * RB;                              // C-layout keys 4i + g: i * 4 RB further
    const int vc_off = g * RB + 2 + 2 * n;                  // their V codes of dims 2n, 2n + 1

    // One group of 16 keys starting at tile key kb.  CHECK: the group may
    // hold keys past the split or the caller passed a mask.
    auto group = [&](const char* kt, const char* vt, int kb, int jt, auto check) {
        constexpr bool CHECK = decltype(check)::value;
        // ---- scores: per block, A = key (kb + sigma(n))'s codes 8g..8g+7
        i32x4 cs[NB];
        {
            const char* ka = kt + kb * RB + ka_off;
#pragma unroll
            for (int bb = 0; bb < NB; ++bb) {
                const int off = bb * kQ8Bytes + 2 + 8 * g;       // 2 mod 4 for even blocks
                const uint32_t* p = (const uint32_t*)(ka + (off & ~3));
                const uint32_t w0 = p[0], w1 = p[1];
                uint32_t lo = w0, hi = w1;
                if ((bb & 1) == 0) {
                    const uint32_t w2 = p[2];
                    lo = __builtin_amdgcn_alignbyte(w1, w0, 2);
                    hi = __builtin_amdgcn_alignbyte(w2, w1, 2);
                }
                const long av = (long)((uint64_t)lo | ((uint64_t)hi << 32));
                cs[bb] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, qb[bb], i32x4{0, 0, 0, 0}, 0, 0, 0);
            }
        }
        // the lane's keys kb + sigma(4g + i) = kb + 4i + g: the dwords that
        // hold their K and V block scales, and their V codes of dims 2n, 2n + 1
        uint32_t kd[4][NB], vd[4][NB], vc[4][NB];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const char* kr = kt + (kb + 4 * i) * RB + kc_off;
            const char* vr = vt + (kb + 4 * i) * RB + kc_off;
            const char* vcr = vt + (kb + 4 * i) * RB + vc_off;
#pragma unroll
            for (int bb = 0; bb < NB; ++bb) {
                const int dw = (bb * kQ8Bytes - (bb & 1) * 2) / 4;
                kd[i][bb] = ((const uint32_t*)kr)[dw];
                vd[i][bb] = ((const uint32_t*)vr)[dw];
                vc[i][bb] = *(const uint16_t*)(vcr + bb * kQ8Bytes);
                asm("" : "+v"(vc[i][bb]));     // widened here, next to its load: no masking later
            }
        }
        float s[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float x = 0.0f;
#pragma unroll
            for (int bb = 0; bb < NB; ++bb) {
                const float e = (bb & 1) ? mix_mul<1>(kd[i][bb], qd[bb]) : mix_mul<0>(kd[i][bb], qd[bb]);
                x = fmaf((float)cs[bb][i], e, x);
            }
            s[i] = x;
        }
        if constexpr (CHECK) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int j = jt + kb + 4 * i + g;
                bool live = j < j1;
                if (mrow) {
                    const float mv = live ? f16_to_f32(*(const uint16_t*)(mrow + 2 * (int64_t)j)) * kLog2e : 0.0f;
                    live = live && mv != -INFINITY;
                    s[i] += mv;
                }
                s[i] = live ? s[i] : -INFINITY;
            }
        }

        // ---- online softmax of row n, running max raised lazily
        const float smax = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
        if (__any(smax > m + kLazy)) {
            const float cm = max_swap32(max_swap16(smax));
            if (cm > m + kLazy) {
                const float alpha = __builtin_amdgcn_exp2f(m - cm);     // 0 when m = -inf
                l *= alpha;
#pragma unroll
                for (int j = 0; j < NJ; ++j) acc[j] *= alpha;
                m = cm;
                mb = cm;
            }
        }
        float p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f(s[i] - mb);   // 0 when masked
        l += (p[0] + p[1]) + (p[2] + p[3]);
        const h2 p01 = h2{(_Float16)p[0], (_Float16)p[1]};
        const h2 p23 = h2{(_Float16)p[2], (_Float16)p[3]};

        // ---- O^T += V^T P'^T per 16 dims
#pragma unroll
        for (int bb = 0; bb < NB; ++bb) {
            const uint32_t sel = (bb & 1) ? 0x07060302u : 0x05040100u;      // high or low halves
            h2 dv01, dv23;
            const uint32_t u01 = __builtin_amdgcn_perm(vd[1][bb], vd[0][bb], sel);
            const uint32_t u23 = __builtin_amdgcn_perm(vd[3][bb], vd[2][bb], sel);
            __builtin_memcpy(&dv01, &u01, 4);
            __builtin_memcpy(&dv23, &u23, 4);
            const h4 pb = cat_h4(p01 * dv01, p23 * dv23);
            uint32_t c0, c1, c2, c3;
            i8_quad_mfma(vc[0][bb], vc[1][bb], vc[2][bb], vc[3][bb], c0, c1, c2, c3);
            const h4 a0 = as_h4(c0, c1), a1 = as_h4(c2, c3);
            acc[2 * bb] = __builtin_amdgcn_mfma_f32_16x16x16f16(a0, pb, acc[2 * bb], 0, 0, 0);
            acc[2 * bb + 1] = __builtin_amdgcn_mfma_f32_16x16x16f16(a1, pb, acc[2 * bb + 1], 0, 0, 0);
        }
    };

    // tile t has landed in every wave's share; every wave is done with t - 1
    auto tile = [&](int t, auto check) {
        wait_vm_barrier<(kStages - 2) * kLoads>();
        issue(t + kStages - 1);
        const char* kt = lds + (t & (kStages - 1)) * kStage + dk + h * HB;
        const char* vt = lds + (t & (kStages - 1)) * kStage + kOpBytes + dv + h * HB;
        const int jt = j0 + t * TT;
#pragma unroll
        for (int u = 0; u < NSUB; ++u) group(kt, vt, r * KPW + 16 * u, jt, check);
    };
    // tiles whose keys all lie inside the split run without checks; only the
    // last can hold keys past its end (all tiles are checked under a mask)
    const int n_plain = mrow != nullptr ? 0 : (j1 - j0) / TT;
    int t = 0;
    for (; t < n_plain; ++t) tile(t, std::false_type{});
    for (; t < n_tiles; ++t) tile(t, std::true_type{});
    // the padding tiles' loads land before the ring is reused
    asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
    __syncthreads();

    // row n's sum over the four lane groups
    l = add_swap32(add_swap16(l));

    // lane (g, n) holds O[row n][32 b + 8 g + 2 i + s] = acc[2 b + s][i]
    auto dims = [&](int bb, int half) -> float4 {
        const f32x4 e = acc[2 * bb], o = acc[2 * bb + 1];
        return half == 0 ? make_float4(e[0], o[0], e[1], o[1]) : make_float4(e[2], o[2], e[3], o[3]);
    };

    // ---- merge the R waves of each kv head (log-sum-exp) through LDS
    float (*abuf)[16][D] = (float (*)[16][D])lds;
    float (*mbuf)[16] = (float (*)[16])(lds + kW * 16 * D * 4);
    float (*lbuf)[16] = (float (*)[16])(lds + kW * 16 * D * 4 + kW * 16 * 4);
    if (R > 1) {
        if (r > 0) {
            if (g == 0) { mbuf[w][n] = m; lbuf[w][n] = l; }
#pragma unroll
            for (int bb = 0; bb < NB; ++bb) {
                *(float4*)&abuf[w][n][32 * bb + 8 * g] = dims(bb, 0);
                *(float4*)&abuf[w][n][32 * bb + 8 * g + 4] = dims(bb, 1);
            }
        }
        __syncthreads();
        if (r == 0) {
            for (int rr = 1; rr < R; ++rr) {
                const int ow = rr * HKV + h;
                const float mo = mbuf[ow][n];
                const float mn = fmaxf(m, mo);
                const float fa = mn == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - mn);
                const float fb = mn == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mo - mn);
                l = l * fa + lbuf[ow][n] * fb;
#pragma unroll
                for (int bb = 0; bb < NB; ++bb) {
                    const float4 x = *(const float4*)&abuf[ow][n][32 * bb + 8 * g];
                    const float4 y = *(const float4*)&abuf[ow][n][32 * bb + 8 * g + 4];
                    f32x4& e = acc[2 * bb];
                    f32x4& o = acc[2 * bb + 1];
                    e[0] = e[0] * fa + x.x * fb; o[0] = o[0] * fa + x.y * fb;
                    e[1] = e[1] * fa + x.z * fb; o[1] = o[1] * fa + x.w * fb;
                    e[2] = e[2] * fa + y.x * fb; o[2] = o[2] * fa + y.y * fb;
                    e[3] = e[3] * fa + y.z * fb; o[3] = o[3] * fa + y.w * fb;
                }
                m = mn;
            }
        }
    }
    const int hq = h * G + n;
    if (r == 0 && n < G) {
        if (n_splits == 1) {
            const float inv = l == 0.0f ? 0.0f : 1.0f / l;
            float* orow = (float*)((char*)a.out + b * a.o_nb_b + hq * a.o_nb_h);
#pragma unroll
            for (int bb = 0; bb < NB; ++bb) {
                const float4 x = dims(bb, 0), y = dims(bb, 1);
                *(float4*)(orow + 32 * bb + 8 * g) = make_float4(x.x * inv, x.y * inv, x.z * inv, x.w * inv);
                *(float4*)(orow + 32 * bb + 8 * g + 4) = make_float4(y.x * inv, y.y * inv, y.z * inv, y.w * inv);
            }
        } else {
            // partials: acc [B][Hq][n_splits][D], then (m, l) [B][Hq][n_splits][2]
            const size_t idx = ((size_t)b * a.Hq + hq) * n_splits + split;
            float* wacc = ws + idx * D;
#pragma unroll
            for (int bb = 0; bb < NB; ++bb) {
                *(float4*)(wacc + 32 * bb + 8 * g) = dims(bb, 0);
                *(float4*)(wacc + 32 * bb + 8 * g + 4) = dims(bb, 1);
            }
            if (g == 0) *(float2*)(ws + (size_t)a.B * a.Hq * n_splits * D + idx * 2) = make_float2(m, l);
        }
    }
}

template <int D>
hipError_t launch_ds(const AttnArgs& a, float* ws, int n_splits, int split_len, hipStream_t s) {
    const dim3 grid(n_splits, a.B), block(kW * 64);
    switch (a.Hkv) {
#define VVA_DS(H) case H: hipLaunchKernelGGL((decode_stream_kernel<D, H>), grid, block, 0, s, a, ws, n_splits, split_len); break;
        VVA_DS(1) VVA_DS(2) VVA_DS(4) VVA_DS(8)
#undef VVA_DS
        default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || n_splits == 1) return e;
    return launch_decode_merge(a, ws, n_splits, s);
}

}  // namespace

bool decode_stream_supported(const AttnArgs& a) {
    if (a.T != 1) return false;
    if (a.d != 64 && a.d != 128) return false;
    if (a.k_type != VVA_TYPE_Q8_0 || a.v_type != VVA_TYPE_Q8_0) return false;
    if (a.Hkv < 1 || a.Hq % a.Hkv != 0 || a.Hq / a.Hkv > 8) return false;
    if (kW % a.Hkv != 0) return false;
    // dense rows: [token][kv head][blocks], as the resident cache stores them
    const int64_t hb = (int64_t)(a.d / 32) * kQ8Bytes;
    if (a.k_nb_head != hb || a.v_nb_head != hb) return false;
    if (a.k_nb_tok != hb * a.Hkv || a.v_nb_tok != hb * a.Hkv) return false;
    for (int b = 0; b < a.B; ++b) {
        if (((uintptr_t)a.k[b] % 4) || ((uintptr_t)a.v[b] % 4)) return false;
        // every buffer range and live offset stays below the padding offset
        if ((int64_t)(a.L[b] + 1) * a.k_nb_tok + 2 * kOpBytes >= kDead) return false;
    }
    if (a.mask_mode == kMaskExplicit && (a.mask_nb_b % 2 != 0)) return false;
    if (((uintptr_t)a.q % 16) || a.q_nb_h % 16 || a.q_nb_b % 16) return false;
    // Q rows contiguous and small enough for the raw-Q area, codes after them
    const int64_t qrow = (int64_t)a.d * type_elem_bytes(a.q_type);
    if (a.q_nb_h != qrow || a.Hq * qrow > kQRawBytes) return false;
    if (kQRawBytes + (int64_t)a.Hq * (a.d / 32) * 36 > kStage) return false;
    if (((uintptr_t)a.out % 16) || a.o_nb_h % 16 || a.o_nb_b % 16) return false;
    return true;
}

int decode_stream_plan(const AttnArgs& a, int n_cu, int* split_len) {
    int Lmax = 1;
    for (int b = 0; b < a.B; ++b) Lmax = a.L[b] > Lmax ? a.L[b] : Lmax;
    // one workgroup per CU over (split, sequence); at least two tiles' worth
    // of keys per split
    int target = n_cu / a.B;
    if (target < 1) target = 1;
    int sl = (Lmax + target - 1) / target;
    const int min_len = 2 * kTileOpBytes / (int)((a.d / 32) * kQ8Bytes * a.Hkv);
    if (sl < min_len) sl = min_len;
    *split_len = sl;
    return (Lmax + sl - 1) / sl;
}

hipError_t launch_decode_stream(const AttnArgs& a, float* ws, int n_splits, int split_len, hipStream_t s) {
    if (a.d == 64) return launch_ds<64>(a, ws, n_splits, split_len, s);
    if (a.d == 128) return launch_ds<128>(a, ws, n_splits, split_len, s);
    return hipErrorInvalidValue;
}

}  // namespace vva
