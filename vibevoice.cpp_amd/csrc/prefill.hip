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
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 15.0f;     // running-max slack in log2 units: p <= 2^15 (f16-safe)
constexpr int kBN = 64;        // keys per tile
constexpr int kRowsWave = 64;  // query rows per wave
constexpr int kWaves = 4;
constexpr int kRowsWG = kRowsWave * kWaves;

// max of x over lanes l and l ^ 32 (v_permlane32_swap exchanges the halves)
__device__ __forceinline__ float max_swap32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

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

// EXPL: explicit F16 mask (otherwise implicit causal / length masking only).
template <int D, int KT, bool EXPL>
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
    const bool causal = !EXPL && a.mask_mode == kMaskCausal;
    constexpr bool explicit_mask = EXPL;

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

    // Per 64-key tile: both 32-key halves of S^T are issued on the MFMA pipe
    // first, then each half's softmax VALU runs while the MFMAs of the other
    // half or of the previous P.V product are in flight.
    //
    // The reference max m of a row is fixed by the first tile with a visible
    // key and never moves inside the tile loop, so O stays in MFMA
    // accumulators with no VALU rescale: p = 2^(x - m) is allowed up to 2^15
    // (f16).  If a row's score exceeds m + 15 (rare: logits rarely grow by
    // 2^15 after the first tile), the workgroup restarts its key loop from
    // tile 0 with the raised m (each restart raises it by more than 15, so
    // restarts are few).
    for (;;) {
    if (n_tiles > 0) {
        load_tile(0);
        store_tile(0);
    }
    __syncthreads();
    bool restart = false;
    for (int j = 0; j < n_tiles; ++j) {
        const int stage = j & 1;
        if (j + 1 < n_tiles) load_tile(j + 1);
        const int k0 = j * kBN;
        bool raise = false;
        if (k0 < kend_w) {
            const char* kb = lds + stage * STAGE;
            const char* vb = kb + KBUF;
            // the second half is skipped when no row of the wave sees it
            const bool two = !(causal && k0 + 32 > past + t_hi_w);             // wave-uniform
            // ---------------- S^T = K Q^T (32 keys x 64 rows per half)
            f32x16 s[2][2];
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
                for (int ds = 0; ds < DS; ++ds) {
                    const QF kf = as_vec<QF>(*(const u32x4*)(kb + (kt * 32 + l32) * KROW + ds * 32 + half * 16));
#pragma unroll
                    for (int cb = 0; cb < 2; ++cb)
                        s[kt][cb] = ds == 0 ? F::mma(kf, qf[cb][0], f32x16{}) : F::mma(kf, qf[cb][ds], s[kt][cb]);
                }
                if (!two) break;
            }
            // ---------------- masks: raw scores, or scores already in the
            // exp2 domain (scaled, mask added) when the mask is explicit
            float mul = sl2;
            const bool need_mask = EXPL || k0 + kBN > L || (causal && k0 + kBN - 1 > past + t_lo_w);
            if (need_mask) {
#pragma unroll
                for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                    for (int cb = 0; cb < 2; ++cb) {
                        const int lim = causal ? min(L - 1, past + tcol[cb]) : L - 1;
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int key = k0 + kt * 32 + 8 * (r / 4) + 4 * half + (r % 4);
                            float x = s[kt][cb][r];
                            if constexpr (EXPL) {
                                const char* mrow = a.mask + b * a.mask_nb_b + tcol[cb] * a.mask_nb_row;
                                x = fmaf(x, sl2, f16_to_f32(*(const uint16_t*)(mrow + 2 * min(key, L - 1))) * kLog2e);
                            }
                            s[kt][cb][r] = (key > lim || (kt == 1 && !two)) ? -INFINITY : x;
                        }
                    }
                if constexpr (EXPL) mul = 1.0f;
            } else if (!two) {
#pragma unroll
                for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) s[1][cb][r] = -INFINITY;
            }
            // ---------------- row max of the tile against the reference
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) {
                float mx = fmaxf(s[0][cb][0], s[1][cb][0]);
#pragma unroll
                for (int r = 1; r < 16; ++r) mx = fmaxf(fmaxf(mx, s[0][cb][r]), s[1][cb][r]);
                mx = max_swap32(mx) * mul;
                if (m[cb] == -INFINITY) m[cb] = mx;        // O and the row sum are still 0
                if (mx > m[cb] + kLazy) {
                    raise = true;
                    m[cb] = mx;                            // the restart uses the raised max
                }
            }
            // a raising wave skips the rest of the tile: the restart discards it
            if (!__any(raise)) {
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                if (kt == 1 && !two) break;
                // ---------------- p = 2^(x * mul - m) as f16, row sums from the f16 values
                h8 pf[2][2];
#pragma unroll
                for (int cb = 0; cb < 2; ++cb) {
                    const float nb = m[cb] == -INFINITY ? 0.0f : -m[cb];
                    float ps = lsum[cb];
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) {
                        h8 p;
#pragma unroll
                        for (int e = 0; e < 8; e += 2) {
                            const float p0 = __builtin_amdgcn_exp2f(fmaf(s[kt][cb][ks * 8 + e], mul, nb));
                            const float p1 = __builtin_amdgcn_exp2f(fmaf(s[kt][cb][ks * 8 + e + 1], mul, nb));
                            h2 pp = {(_Float16)p0, (_Float16)p1};
                            p[e] = pp.x;
                            p[e + 1] = pp.y;
                            ps = __builtin_amdgcn_fdot2(pp, h2{(_Float16)1.0f, (_Float16)1.0f}, ps, false);
                        }
                        pf[cb][ks] = p;
                    }
                    lsum[cb] = ps;
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
        }
        if (j + 1 < n_tiles) store_tile(stage ^ 1);
        if (__syncthreads_or(raise)) {                      // workgroup-uniform
            restart = true;
            break;
        }
    }
    if (!restart) break;
    lsum[0] = lsum[1] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) o[dt][cb] = f32x16{};
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
    if (a.mask_mode == kMaskExplicit)
        hipLaunchKernelGGL((prefill_kernel<D, KT, true>), grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((prefill_kernel<D, KT, false>), grid, dim3(256), 0, s, a);
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
