// prefill.hip — causal GQA flash-attention prefill on CDNA4 MFMA.
//
// The prefill call of ggml_flash_attn_ext over the resident window
// (src/qwen2.cpp:332-335) for F16 / BF16 caches: voice-prompt, text and
// speech-latent prefills (src/vibevoice_tts.cpp:1199-1204) and the chunked
// ASR prefill (src/vibevoice_asr.cpp:542-652).
//
// Work decomposition.  Query rows are the (token, head) pairs of one KV
// group flattened as r = t * g + (h - kvh * g), so the g = Hq / Hkv heads of
// a group share every K/V tile a workgroup stages in LDS (GQA sharing) and no
// padding is wasted for g = 7 or 6.  Grid = (row tiles of 256, Hkv, B); a
// workgroup is 4 waves x 64 rows and walks the key tiles (64 keys) its rows
// can see; row tiles are issued heaviest-first for the causal imbalance.
//
// Per wave and key tile, with v_mfma_f32_32x32x16_{f16,bf16}:
//   S^T[key][row] = K . Q^T  A = K rows from LDS (16 B per lane), B = Q^T
//                            held in registers for the whole kernel, so each
//                            lane owns one query row (column) of S^T and the
//                            softmax row reductions are in-register plus one
//                            cross-half exchange;
//   online softmax           fp32, exp2 domain, causal / length / explicit
//                            masks applied only on tiles that need them;
//   O^T[d][row] += V^T . P^T A = V^T from LDS (stored transposed),
//                            B = P^T converted in place from the S^T
//                            accumulators: the key order of an MFMA step is
//                            chosen to be the one the accumulator layout
//                            already has, so no shuffle is needed.
// P and V enter the second product as f16 (BF16 V is converted on its way to
// LDS): an 8-bit-mantissa P would cost up to ~4e-3 on short rows, f16 P stays
// below 4e-4.  Q is rounded to K's type, as ggml's CPU flash attention does.
// K/V tiles are double-buffered in LDS: the next tile's global loads are in
// flight while the current tile is computed.
#include "vva_internal.hpp"

namespace vva {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kBN = 64;        // keys per tile
constexpr int kRowsWave = 64;  // query rows per wave
constexpr int kWaves = 4;
constexpr int kRowsWG = kRowsWave * kWaves;

template <int KT> struct Frag;
template <> struct Frag<VVA_TYPE_F16> {
    typedef h8 type;
    static __device__ __forceinline__ f32x16 mma(const h8& a, const h8& b, const f32x16& c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint16_t cvt(float x) { return f32_to_f16(x); }
};
template <> struct Frag<VVA_TYPE_BF16> {
    typedef b8 type;
    static __device__ __forceinline__ f32x16 mma(const b8& a, const b8& b, const f32x16& c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint16_t cvt(float x) { return f32_to_bf16(x); }
};

template <typename V>
__device__ __forceinline__ V as_vec(const u32x4& u) {
    V v;
    __builtin_memcpy(&v, &u, 16);
    return v;
}

__device__ __forceinline__ uint32_t bf16x2_to_f16x2(uint32_t x) {
    const float lo = __uint_as_float(x << 16), hi = __uint_as_float(x & 0xffff0000u);
    return (uint32_t)f32_to_f16(lo) | ((uint32_t)f32_to_f16(hi) << 16);
}

template <int D, int KT>
__global__ void __launch_bounds__(256) prefill_kernel(AttnArgs a) {
    using F = Frag<KT>;
    using QF = typename F::type;
    constexpr int DS = D / 16;                 // 16-dim MFMA steps of Q.K
    constexpr int DT = D / 32;                 // 32-dim output tiles
    constexpr int KROW = D * 2 + 16;           // LDS bytes per K row (padded)
    constexpr int VROW = kBN * 2 + 8;          // LDS bytes per V^T row (padded)
    constexpr int KBUF = kBN * KROW;
    constexpr int VBUF = D * VROW;
    constexpr int STAGE = KBUF + VBUF;
    constexpr int KCH = D / 8;                 // 16-byte chunks per K row
    constexpr int KLD = kBN * KCH / 256;       // K chunks loaded per thread
    constexpr int VITEMS = (kBN / 4) * (D / 8);  // (4 keys x 8 dims) items per V tile

    __shared__ __attribute__((aligned(16))) char lds[2 * STAGE];

    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6, half = lane >> 5, l32 = lane & 31;
    const int b = blockIdx.z, kvh = blockIdx.y;
    const int g = a.Hq / a.Hkv;
    const int nrows = a.T * g;
    const int n_rt = (nrows + kRowsWG - 1) / kRowsWG;
    const int R0 = (n_rt - 1 - (int)blockIdx.x) * kRowsWG;    // heaviest tiles first
    const int wr0 = R0 + w * kRowsWave;
    const int L = a.L[b], past = a.past[b];
    const bool causal = a.mask_mode == kMaskCausal;
    const bool explicit_mask = a.mask_mode == kMaskExplicit;

    // key range of the workgroup and of this wave
    const int t_hi_wg = min(a.T - 1, (min(R0 + kRowsWG, nrows) - 1) / g);
    const int kend = causal ? min(L, past + t_hi_wg + 1) : L;
    const int n_tiles = (kend + kBN - 1) / kBN;
    const bool wave_live = wr0 < nrows;
    const int t_lo_w = min(a.T - 1, wr0 / g);
    const int t_hi_w = min(a.T - 1, (min(wr0 + kRowsWave, nrows) - 1) / g);
    const int kend_w = !wave_live ? 0 : (causal ? min(L, past + t_hi_w + 1) : L);

    // ---- this lane's query rows (one per 32-row column block) and Q^T fragments
    int tcol[2];
    QF qf[2][DS];
    {
        const int64_t es = type_elem_bytes(a.q_type);
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            const int row = wr0 + cb * 32 + l32;
            const bool ok = row < nrows;
            const int t = ok ? row / g : 0;
            const int h = kvh * g + (ok ? row % g : 0);
            tcol[cb] = ok ? t : a.T - 1;
            const char* qrow = a.q + b * a.q_nb_b + t * a.q_nb_t + h * a.q_nb_h;
#pragma unroll
            for (int ds = 0; ds < DS; ++ds) {
                const int d0 = ds * 16 + half * 8;
                u32x4 u = {0u, 0u, 0u, 0u};
                if (ok) {
                    if (a.q_type == KT) {
                        u = *(const u32x4*)(qrow + d0 * 2);
                    } else {
                        uint16_t hv[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e) hv[e] = F::cvt(load_elem(qrow + (d0 + e) * es, a.q_type));
                        __builtin_memcpy(&u, hv, 16);
                    }
                }
                qf[cb][ds] = as_vec<QF>(u);
            }
        }
    }

    float m[2] = {-INFINITY, -INFINITY};
    float lsum[2] = {0.0f, 0.0f};
    f32x16 o[DT][2];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[dt][cb][r] = 0.0f;

    const float sl2 = a.scale * kLog2e;
    const char* kg = a.k[b] + kvh * a.k_nb_head;
    const char* vg = a.v[b] + kvh * a.v_nb_head;

    // ---- tile staging: global -> registers -> LDS
    u32x4 kst[KLD];
    u32x4 vst[4];
    const int v_item = tid;                           // (key group, dim chunk)
    const bool v_active = v_item < VITEMS;
    const int v_kg = v_item / (D / 8), v_dc = v_item % (D / 8);

    auto load_tile = [&](int j) {
        const int k0 = j * kBN;
#pragma unroll
        for (int i = 0; i < KLD; ++i) {
            const int c = tid + i * 256;
            const int key = min(k0 + c / KCH, L - 1);
            kst[i] = *(const u32x4*)(kg + (int64_t)key * a.k_nb_tok + (c % KCH) * 16);
        }
        if (v_active) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = min(k0 + v_kg * 4 + i, L - 1);
                vst[i] = *(const u32x4*)(vg + (int64_t)key * a.v_nb_tok + v_dc * 16);
            }
        }
    };
    auto store_tile = [&](int stage) {
        char* kb = lds + stage * STAGE;
        char* vb = kb + KBUF;
#pragma unroll
        for (int i = 0; i < KLD; ++i) {
            const int c = tid + i * 256;
            *(u32x4*)(kb + (c / KCH) * KROW + (c % KCH) * 16) = kst[i];
        }
        if (v_active) {
            uint32_t x[4][4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                u32x4 u = vst[i];
                if constexpr (KT == VVA_TYPE_BF16) {
                    u.x = bf16x2_to_f16x2(u.x); u.y = bf16x2_to_f16x2(u.y);
                    u.z = bf16x2_to_f16x2(u.z); u.w = bf16x2_to_f16x2(u.w);
                }
                x[i][0] = u.x; x[i][1] = u.y; x[i][2] = u.z; x[i][3] = u.w;
            }
            // dims v_dc*8 + e, keys v_kg*4 + 0..3 -> one 8-byte row segment each
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const uint32_t lo01 = (x[0][p] & 0xffffu) | (x[1][p] << 16);
                const uint32_t lo23 = (x[2][p] & 0xffffu) | (x[3][p] << 16);
                const uint32_t hi01 = (x[0][p] >> 16) | (x[1][p] & 0xffff0000u);
                const uint32_t hi23 = (x[2][p] >> 16) | (x[3][p] & 0xffff0000u);
                const int d = v_dc * 8 + 2 * p;
                *(u32x2*)(vb + d * VROW + v_kg * 8) = u32x2{lo01, lo23};
                *(u32x2*)(vb + (d + 1) * VROW + v_kg * 8) = u32x2{hi01, hi23};
            }
        }
    };

    if (n_tiles > 0) {
        load_tile(0);
        store_tile(0);
    }
    __syncthreads();

    for (int j = 0; j < n_tiles; ++j) {
        const int stage = j & 1;
        if (j + 1 < n_tiles) load_tile(j + 1);
        const int k0 = j * kBN;
        if (k0 < kend_w) {
            const char* kb = lds + stage * STAGE;
            const char* vb = kb + KBUF;
            const bool need_mask = explicit_mask || k0 + kBN > L || (causal && k0 + kBN - 1 > past + t_lo_w);
            // the 64-key tile is processed as two 32-key halves to bound the
            // number of live accumulators
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                if (causal && k0 + kt * 32 > past + t_hi_w) break;     // wave-uniform
                // ---------------- S^T = K Q^T (32 keys x 64 rows)
                f32x16 s[2];
#pragma unroll
                for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) s[cb][r] = 0.0f;
#pragma unroll
                for (int ds = 0; ds < DS; ++ds) {
                    const QF kf = as_vec<QF>(*(const u32x4*)(kb + (kt * 32 + l32) * KROW + ds * 32 + half * 16));
#pragma unroll
                    for (int cb = 0; cb < 2; ++cb) s[cb] = F::mma(kf, qf[cb][ds], s[cb]);
                }
                // ---------------- online softmax (exp2 domain)
                h8 pf[2][2];
#pragma unroll
                for (int cb = 0; cb < 2; ++cb) {
                    float x[16];
#pragma unroll
                    for (int r = 0; r < 16; ++r) x[r] = s[cb][r] * sl2;
                    if (need_mask) {
                        const int lim = causal ? min(L - 1, past + tcol[cb]) : L - 1;
                        const char* mrow =
                            explicit_mask ? a.mask + b * a.mask_nb_b + tcol[cb] * a.mask_nb_row : nullptr;
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int key = k0 + kt * 32 + 8 * (r / 4) + 4 * half + (r % 4);
                            if (key > lim) x[r] = -INFINITY;
                            else if (explicit_mask)
                                x[r] = fmaf(f16_to_f32(*(const uint16_t*)(mrow + 2 * key)), kLog2e, x[r]);
                        }
                    }
                    float mx = x[0];
#pragma unroll
                    for (int i = 1; i < 16; ++i) mx = fmaxf(mx, x[i]);
                    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
                    const float mn = fmaxf(m[cb], mx);
                    const float base = mn == -INFINITY ? 0.0f : mn;
                    const float alpha = __builtin_amdgcn_exp2f(m[cb] - base);   // m = -inf -> 0
                    m[cb] = mn;
                    float ps = 0.0f;
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) {
                        h8 p;
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            const _Float16 ph = (_Float16)__builtin_amdgcn_exp2f(x[ks * 8 + e] - base);
                            p[e] = ph;
                            ps += (float)ph;
                        }
                        pf[cb][ks] = p;
                    }
                    lsum[cb] = lsum[cb] * alpha + ps;
                    if (!__all(alpha == 1.0f)) {
#pragma unroll
                        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                            for (int r = 0; r < 16; ++r) o[dt][cb][r] *= alpha;
                    }
                }
                // ---------------- O^T += V^T P^T (the two 16-key steps of this half)
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
                    const char* vrow = vb + (dt * 32 + l32) * VROW;
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) {
                        const int kk = (kt * 2 + ks) * 16;
                        const u32x2 lo = *(const u32x2*)(vrow + (kk + 4 * half) * 2);
                        const u32x2 hi = *(const u32x2*)(vrow + (kk + 8 + 4 * half) * 2);
                        const h8 vf = as_vec<h8>(u32x4{lo.x, lo.y, hi.x, hi.y});
#pragma unroll
                        for (int cb = 0; cb < 2; ++cb)
                            o[dt][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[cb][ks], o[dt][cb], 0, 0, 0);
                    }
                }
            }
        }
        if (j + 1 < n_tiles) store_tile(stage ^ 1);
        __syncthreads();
    }

    // ---- normalize and write (each lane owns one row per column block)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
        const int row = wr0 + cb * 32 + l32;
        const float lt = lsum[cb] + __shfl_xor(lsum[cb], 32, 64);
        if (row >= nrows) continue;
        const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
        const int t = row / g, h = kvh * g + row % g;
        float* orow = (float*)((char*)a.out + b * a.o_nb_b + t * a.o_nb_t + h * a.o_nb_h);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const int d = dt * 32 + 8 * q4 + 4 * half;
                float4 v = make_float4(o[dt][cb][4 * q4] * inv, o[dt][cb][4 * q4 + 1] * inv,
                                       o[dt][cb][4 * q4 + 2] * inv, o[dt][cb][4 * q4 + 3] * inv);
                *(float4*)(orow + d) = v;
            }
    }
}

template <int D, int KT>
hipError_t launch_pf(const AttnArgs& a, hipStream_t s) {
    const int g = a.Hq / a.Hkv;
    const int nrows = a.T * g;
    dim3 grid((nrows + kRowsWG - 1) / kRowsWG, a.Hkv, a.B);
    hipLaunchKernelGGL((prefill_kernel<D, KT>), grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace

bool prefill_supported(const AttnArgs& a) {
    if (a.T < 2) return false;
    if (a.d != 64 && a.d != 128) return false;
    if (a.k_type != a.v_type) return false;
    if (a.k_type != VVA_TYPE_F16 && a.k_type != VVA_TYPE_BF16) return false;
    if (a.Hq % a.Hkv != 0) return false;
    // 16-byte vector access to K/V rows and Q rows of the matching type,
    // 16-byte aligned float4 output rows
    if (a.k_nb_tok % 16 || a.k_nb_head % 16 || a.v_nb_tok % 16 || a.v_nb_head % 16) return false;
    for (int b = 0; b < a.B; ++b) {
        if ((uintptr_t)a.k[b] % 16 || (uintptr_t)a.v[b] % 16) return false;
        if (a.L[b] < 1) return false;
    }
    if (a.q_type == a.k_type && (((uintptr_t)a.q % 16) || a.q_nb_t % 16 || a.q_nb_h % 16 || a.q_nb_b % 16))
        return false;
    if (((uintptr_t)a.out % 16) || a.o_nb_t % 16 || a.o_nb_h % 16 || a.o_nb_b % 16) return false;
    if (a.mask_mode == kMaskExplicit && (a.mask_nb_row % 2 || a.mask_nb_b % 2)) return false;
    return true;
}

hipError_t launch_prefill(const AttnArgs& a, hipStream_t s) {
    if (a.d == 64) {
        return a.k_type == VVA_TYPE_F16 ? launch_pf<64, VVA_TYPE_F16>(a, s) : launch_pf<64, VVA_TYPE_BF16>(a, s);
    }
    return a.k_type == VVA_TYPE_F16 ? launch_pf<128, VVA_TYPE_F16>(a, s) : launch_pf<128, VVA_TYPE_BF16>(a, s);
}

}  // namespace vva
