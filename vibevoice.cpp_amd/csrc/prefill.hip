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
// Staging.  K and V tiles go from HBM straight into LDS with buffer loads
// that write LDS (no registers, no VALU), into a ring of four stages: the
// loads of tile j + 3 are issued, spread over the work of tile j, while
// tile j is computed.  Both tiles are kept row-major ([key][dim]); K rows
// are padded to 16 mod 256 bytes and V rows to 64 mod 256 bytes, which
// keeps both operand reads free of bank conflicts.  The V^T operand of the
// second product is read with ds_read_b64_tr_b16, whose 16-lane transpose
// hands each lane 4 consecutive keys of one dim.  Keys past L read as 0
// through the buffer range check.
//
// Per wave and key tile, with v_mfma_f32_32x32x16_{f16,bf16}:
//   S^T[key][row] = K . Q^T  A = K rows from LDS (16 B per lane), B = Q^T
//                            held in registers for the whole kernel, so each
//                            lane owns one query row (column) of S^T and the
//                            softmax row reductions are in-register plus one
//                            cross-half exchange;
//   softmax                  fp32, exp2 domain;
//   O^T[d][row] += V^T . P^T B = P^T converted in place from the S^T
//                            accumulators: the key order of an MFMA step is
//                            chosen to be the one the accumulator layout
//                            already has, so no shuffle is needed.
// Tiles every row of the workgroup sees whole run a branch-free loop that is
// pipelined across tiles: the scores of half 0 of tile j + 1 are computed
// while P.V of tile j still runs, so that each group of 16 MFMAs has a
// quarter of a softmax to overlap.  The diagonal and length-boundary tiles
// at the end of a workgroup's range run a second loop with masks.
// The reference max m of a row is taken from half 0 of the first tile (key 0
// is visible to every row) and never moves inside the tile loop, so O stays
// in MFMA accumulators with no rescale and no max is tracked per tile.  A
// later score beyond m + 16 turns its f16 p into inf; the row sum shows it,
// and the workgroup restarts its key loop with m raised to that tile's row
// max (rare: logits rarely grow by 2^16 after the first tile).  With an
// explicit mask the row max is tracked per tile instead (masked loop only).
// P and V enter the second product as f16 (BF16 V is converted after the
// transposing read): an 8-bit-mantissa P would cost up to ~4e-3 on short
// rows, f16 P stays below 4e-4.  Q is rounded to K's type, as ggml's CPU
// flash attention does.
#include "vva_internal.hpp"

namespace vva {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) char lds_char;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 15.0f;     // headroom of p over 2^0 in log2 units: p <= 2^15 (f16-safe)
constexpr int kBN = 64;            // keys per tile
constexpr int kRowsWave = 64;      // query rows per wave
constexpr int kWaves = 4;
constexpr int kRowsWG = kRowsWave * kWaves;
constexpr int kStages = 4;         // LDS ring: tile j + 3 loads while tile j is computed
constexpr int kMaxRestarts = 16;   // bound on key-loop restarts per workgroup
constexpr int kMaxKeySplits = 32;  // key splits per row tile

// buffer_load_dwordx4 ... lds: each lane's 16 bytes land at LDS address
// m0 + 16 * lane.  Issued as inline asm so the compiler does not fence LDS
// reads on them; completion is waited for explicitly (wait_vmcnt) before the
// workgroup barrier that publishes a stage.
__device__ __forceinline__ void dma16(i32x4 rsrc, uint32_t lds_addr, int voffset, int soffset) {
    // lds_addr and soffset are wave-uniform; readfirstlane keeps them in SGPRs
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 4\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voffset), "s"(rsrc),
                   "s"(__builtin_amdgcn_readfirstlane(soffset))
                 : "memory", "m0");
}

__device__ __forceinline__ i32x4 make_rsrc(const char* base, uint32_t bytes) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), (short)0, (int)bytes, 0x00020000);
    i32x4 v;
    __builtin_memcpy(&v, &r, 16);
    // wave-uniform: keep it in SGPRs for the inline-asm loads
    return i32x4{__builtin_amdgcn_readfirstlane(v.x), __builtin_amdgcn_readfirstlane(v.y),
                 __builtin_amdgcn_readfirstlane(v.z), __builtin_amdgcn_readfirstlane(v.w)};
}

// wait until at most N of this wave's loads are outstanding (and its LDS
// operations are done), then meet the workgroup at a barrier
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(N) : "memory");
}

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

__device__ __forceinline__ float bits16_to_f32(uint32_t v, int type) {
    return type == VVA_TYPE_BF16 ? bf16_to_f32((uint16_t)v) : f16_to_f32((uint16_t)v);
}

template <typename V>
__device__ __forceinline__ V as_vec(const u32x4& u) {
    V v;
    __builtin_memcpy(&v, &u, 16);
    return v;
}

// V^T fragment of the second product: dims dt*32 + l%32, keys k0 + (0..3)
// and k1 + (0..3), from the row-major V tile.  In each 16-lane group, lane i
// points at row k + i/4, dims d0 + 4 (i%4) .. +3; the transposing read then
// gives lane i the 4 keys of dim d0 + i.
template <int KT>
__device__ __forceinline__ h8 v_frag(const lds_char* vrow0, const lds_char* vrow1) {
    const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)vrow0);
    const s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)vrow1);
    h8 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint16_t x = (uint16_t)lo[e], y = (uint16_t)hi[e];
        if constexpr (KT == VVA_TYPE_BF16) {
            // the 16-bit patterns are bf16: widen to f32 and round to f16
            v[e] = (_Float16)bf16_to_f32(x);
            v[e + 4] = (_Float16)bf16_to_f32(y);
        } else {
            _Float16 fx, fy;
            __builtin_memcpy(&fx, &x, 2);
            __builtin_memcpy(&fy, &y, 2);
            v[e] = fx;
            v[e + 4] = fy;
        }
    }
    return v;
}

__device__ __forceinline__ const lds_char* lds_at(uint32_t addr) { return (const lds_char*)(uintptr_t)addr; }

// EXPL: explicit F16 mask (otherwise implicit causal / length masking only).
template <int D, int KT, bool EXPL>
__global__ void __launch_bounds__(256) prefill_kernel(AttnArgs a, float* __restrict__ ws, int n_ks) {
    using F = Frag<KT>;
    using QF = typename F::type;
    constexpr int DS = D / 16;                     // 16-dim MFMA steps of Q.K
    constexpr int DT = D / 32;                     // 32-dim output tiles
    // Row pitches in LDS.  K is read 16 B per lane, 16 rows per bank pass:
    // a pitch of 16 mod 256 bytes puts them on distinct banks.  V is read by
    // the transposing 8-byte load, 4 rows x 64 B per 32 lanes: a pitch of
    // 64 mod 256 bytes puts the 4 rows on distinct banks.
    constexpr int KP = D * 2 + 16;
    constexpr int VP = D * 2 + 64;
    constexpr int NCK = (kBN * KP + 1023) / 1024;  // 1 KB chunks of a K tile
    constexpr int NCV = (kBN * VP + 1023) / 1024;  // (V)
    constexpr int NIK = (NCK + kWaves - 1) / kWaves;   // loads per wave per tile (K)
    constexpr int NIV = (NCV + kWaves - 1) / kWaves;   // (V)
    constexpr int KREG = NCK * 1024;               // LDS bytes per stage (K, then V)
    constexpr int STAGE = KREG + NCV * 1024;
    constexpr int NLD = NIK + NIV;                 // loads per wave per tile
    constexpr int JUNK = kStages * STAGE;          // 1 KB that loads past a tile's chunks write

    __shared__ __attribute__((aligned(16))) char lds[kStages * STAGE + 1024];

    const int tid = threadIdx.x;
    const int lane = tid & 63, half = lane >> 5, l32 = lane & 31;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int b = blockIdx.z, kvh = blockIdx.y;
    const int g = a.Hq / a.Hkv;
    const int nrows = a.T * g;
    const int n_rt = (nrows + kRowsWG - 1) / kRowsWG;
    const int ks = (int)blockIdx.x % n_ks;                       // key split of the row tile
    const int R0 = (n_rt - 1 - (int)blockIdx.x / n_ks) * kRowsWG;   // heaviest tiles first
    const int wr0 = R0 + w * kRowsWave;
    const int L = a.L[b], past = a.past[b];
    const bool causal = !EXPL && a.mask_mode == kMaskCausal;

    // key range of the workgroup and of this wave
    const int t_hi_wg = min(a.T - 1, (min(R0 + kRowsWG, nrows) - 1) / g);
    const int kend = causal ? min(L, past + t_hi_wg + 1) : L;
    // the workgroup's share of the row tile's key tiles: [j_lo, j_lo + n_tiles);
    // tile j below is local, its first key kb0 + j * kBN
    const int n_tiles_rt = (kend + kBN - 1) / kBN;
    const int j_lo = (int)((int64_t)ks * n_tiles_rt / n_ks);
    const int n_tiles = (int)((int64_t)(ks + 1) * n_tiles_rt / n_ks) - j_lo;
    const int kb0 = j_lo * kBN;
    const bool wave_live = wr0 < nrows;
    const int t_lo_w = min(a.T - 1, wr0 / g);
    const int t_hi_w = min(a.T - 1, (min(wr0 + kRowsWave, nrows) - 1) / g);
    const int kend_w = !wave_live ? 0 : (causal ? min(L, past + t_hi_w + 1) : L);

    // ---- tile loads: per lane and 1 KB chunk q = i * 4 + w of an operand,
    // the byte x = 1024 q + 16 lane of the padded tile is row x / pitch,
    // column x % pitch; pad bytes load from an offset past the buffer (0
    // bytes read, zeros written), and a wave's loads past the last chunk
    // write zeros to the junk kilobyte (every wave issues the same number
    // of loads per tile, with no branch)
    const uint32_t nbk = (uint32_t)a.k_nb_tok, nbv = (uint32_t)a.v_nb_tok;
    const int kl = max(L - kb0, 1);                           // rows from the split's first key
    const i32x4 krs = make_rsrc(a.k[b] + kvh * a.k_nb_head + (int64_t)kb0 * nbk, (uint32_t)(kl - 1) * nbk + 2 * D);
    const i32x4 vrs = make_rsrc(a.v[b] + kvh * a.v_nb_head + (int64_t)kb0 * nbv, (uint32_t)(kl - 1) * nbv + 2 * D);
    int koff[NIK], voff[NIV];
#pragma unroll
    for (int i = 0; i < NIK; ++i) {
        const int x = (i * kWaves + w) * 1024 + lane * 16;
        const int r = x / KP, c = x % KP;
        koff[i] = r < kBN && c < 2 * D ? (int)(r * nbk) + c : 0x40000000;
    }
#pragma unroll
    for (int i = 0; i < NIV; ++i) {
        const int x = (i * kWaves + w) * 1024 + lane * 16;
        const int r = x / VP, c = x % VP;
        voff[i] = r < kBN && c < 2 * D ? (int)(r * nbv) + c : 0x40000000;
    }
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_char*)lds;
    // loads lo .. hi - 1 of this wave's NLD for tile j (K chunks, then V).
    // A dead load (a tile past the last one, or any load once a restart is
    // decided) reads from past the buffer (zeros, no memory traffic) into
    // the junk kilobyte, so the count of loads per tile stays the same and
    // no stage is touched.
    auto issue_range = [&](int j, int lo, int hi, bool live) {
        const uint32_t st = lds0 + (j % kStages) * STAGE;
        const int sk = live ? (int)((uint32_t)(j * kBN) * nbk) : 0x40000000;
        const int sv = live ? (int)((uint32_t)(j * kBN) * nbv) : 0x40000000;
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            if (i < lo || i >= hi) continue;
            if (i < NIK) {
                const int c = i * kWaves + w;
                dma16(krs, live && c < NCK ? st + c * 1024 : lds0 + JUNK, koff[i], sk);
            } else {
                const int c = (i - NIK) * kWaves + w;
                dma16(vrs, live && c < NCV ? st + KREG + c * 1024 : lds0 + JUNK, voff[i - NIK], sv);
            }
        }
    };
    auto issue = [&](int j) { issue_range(j, 0, NLD, j < n_tiles); };
    // workgroup OR of `flag` at the barrier that ends tile j: each wave
    // publishes its own word in a slot that alternates with j (a slot is
    // rewritten two tiles later, after every wave has read it)
    __shared__ int any_flag[2][kWaves];

    // ---- this lane's query rows (one per 32-row column block) and Q^T
    // fragments, rounded to K's type; one loop nest per Q type so the loads
    // of a nest issue back to back
    int tcol[2];
    const char* qrow[2];
    bool qok[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
        const int row = wr0 + cb * 32 + l32;
        qok[cb] = row < nrows;
        const int t = qok[cb] ? row / g : 0;
        const int h = kvh * g + (qok[cb] ? row % g : 0);
        tcol[cb] = qok[cb] ? t : a.T - 1;
        qrow[cb] = a.q + b * a.q_nb_b + t * a.q_nb_t + h * a.q_nb_h;
    }
    QF qf[2][DS];
    u32x4 qraw[2][DS];
    if (a.q_type == VVA_TYPE_F32) {
        float4 x[2][DS][2];
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int ds = 0; ds < DS; ++ds) {
                const int d0 = ds * 16 + half * 8;
                x[cb][ds][0] = *(const float4*)(qrow[cb] + d0 * 4);
                x[cb][ds][1] = *(const float4*)(qrow[cb] + d0 * 4 + 16);
            }
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int ds = 0; ds < DS; ++ds) {
                const float4 x0 = x[cb][ds][0], x1 = x[cb][ds][1];
                qraw[cb][ds] = u32x4{F::cvt(x0.x) | ((uint32_t)F::cvt(x0.y) << 16), F::cvt(x0.z) | ((uint32_t)F::cvt(x0.w) << 16),
                                     F::cvt(x1.x) | ((uint32_t)F::cvt(x1.y) << 16), F::cvt(x1.z) | ((uint32_t)F::cvt(x1.w) << 16)};
            }
    } else {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int ds = 0; ds < DS; ++ds) qraw[cb][ds] = *(const u32x4*)(qrow[cb] + (ds * 16 + half * 8) * 2);
        if (a.q_type != KT) {           // the other 16-bit type
            const int qt = a.q_type;
#pragma unroll
            for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                for (int ds = 0; ds < DS; ++ds) {
                    const u32x4 r = qraw[cb][ds];
                    const uint32_t rw[4] = {r.x, r.y, r.z, r.w};
                    uint32_t cw[4];
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        cw[k] = F::cvt(bits16_to_f32(rw[k] & 0xffffu, qt)) |
                                ((uint32_t)F::cvt(bits16_to_f32(rw[k] >> 16, qt)) << 16);
                    qraw[cb][ds] = u32x4{cw[0], cw[1], cw[2], cw[3]};
                }
        }
    }
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) qf[cb][ds] = as_vec<QF>(qok[cb] ? qraw[cb][ds] : u32x4{0u, 0u, 0u, 0u});

    float m[2] = {-INFINITY, -INFINITY};
    float lsum[2] = {0.0f, 0.0f};
    f32x16 o[DT][2];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) o[dt][cb] = f32x16{};

    const float sl2 = a.scale * kLog2e;
    // per-lane LDS offsets of the operand reads within a stage
    const int k_rd = l32 * KP + half * 16;                                   // K: key l32, dims 8 half ..
    const int v_rd = ((lane & 15) >> 2) * VP + (16 * ((lane >> 4) & 1) + 4 * (lane & 3)) * 2 +
                     4 * half * VP;                                          // V^T, see v_frag

    // S^T of one 32-key half of the tile; ka = stage K base + k_rd, so
    // every read is at an immediate offset
    auto s_half = [&](const lds_char* ka, int kt, f32x16 (&s)[2]) {
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
            const u32x4 kraw = *(const __attribute__((address_space(3))) u32x4*)(ka + kt * 32 * KP + ds * 32);
            const QF kf = as_vec<QF>(kraw);
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) s[cb] = ds == 0 ? F::mma(kf, qf[cb][0], f32x16{}) : F::mma(kf, qf[cb][ds], s[cb]);
        }
    };
    // p = 2^(x * mul - m) as f16 in the order of the second product's k
    // steps, row sums from the f16 values
    auto probs = [&](const f32x16 (&s)[2], float mul, h8 (&pf)[2][2]) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            const float nb = m[cb] == -INFINITY ? 0.0f : -m[cb];
            float ps = lsum[cb];
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                h8 pv;
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    const float p0 = __builtin_amdgcn_exp2f(fmaf(s[cb][ks * 8 + e], mul, nb));
                    const float p1 = __builtin_amdgcn_exp2f(fmaf(s[cb][ks * 8 + e + 1], mul, nb));
                    h2 pp = {(_Float16)p0, (_Float16)p1};
                    pv[e] = pp.x;
                    pv[e + 1] = pp.y;
                    ps = __builtin_amdgcn_fdot2(pp, h2{(_Float16)1.0f, (_Float16)1.0f}, ps, false);
                }
                pf[cb][ks] = pv;
            }
            lsum[cb] = ps;
        }
    };
    // O^T += V^T P^T for the two 16-key steps of half kt; va = stage V base
    // + v_rd
    auto pv_half = [&](const lds_char* va, int kt, const h8 (&pf)[2][2]) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const int kk = (kt * 2 + ks) * 16;
                const lds_char* base = va + dt * 64;
                const h8 vf = v_frag<KT>(base + kk * VP, base + (kk + 8) * VP);
#pragma unroll
                for (int cb = 0; cb < 2; ++cb)
                    o[dt][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[cb][ks], o[dt][cb], 0, 0, 0);
            }
    };
    // max over the 32 keys of half s of each row, in the exp2 domain
    auto half_max = [&](const f32x16 (&s)[2], float mul, float (&mx)[2]) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            float x = fmaxf(fmaxf(s[cb][0], s[cb][1]), s[cb][2]);
#pragma unroll
            for (int r = 3; r < 15; r += 2) x = fmaxf(fmaxf(x, s[cb][r]), s[cb][r + 1]);
            mx[cb] = max_swap32(fmaxf(x, s[cb][15])) * mul;
        }
    };
    // implicit masks on half kt of the tile at key k0: keys past L, and past
    // the row's own position when causal
    auto mask_half = [&](f32x16 (&s)[2], int k0, int kt) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            const int lim = causal ? min(L - 1, past + tcol[cb]) : L - 1;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = k0 + kt * 32 + 8 * (r / 4) + 4 * half + (r % 4);
                s[cb][r] = key > lim ? -INFINITY : s[cb][r];
            }
        }
    };

    // stage bases of tile j, through an empty asm so that each read keeps
    // one base register and a constant offset
    auto bases = [&](int j, const lds_char*& ka, const lds_char*& va) {
        uint32_t kaddr = lds0 + (j % kStages) * STAGE + k_rd;
        uint32_t vaddr = lds0 + (j % kStages) * STAGE + KREG + v_rd;
        asm volatile("" : "+v"(kaddr), "+v"(vaddr));
        ka = lds_at(kaddr);
        va = lds_at(vaddr);
    };
    // operand fragments of half kt, read ahead of their MFMAs into
    // registers of their own
    auto load_k = [&](const lds_char* ka, int kt, QF (&kf)[DS]) {
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
            const u32x4 kraw = *(const __attribute__((address_space(3))) u32x4*)(ka + kt * 32 * KP + ds * 32);
            kf[ds] = as_vec<QF>(kraw);
        }
    };
    auto mma_k = [&](const QF (&kf)[DS], f32x16 (&s)[2]) {
#pragma unroll
        for (int ds = 0; ds < DS; ++ds)
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) s[cb] = ds == 0 ? F::mma(kf[0], qf[cb][0], f32x16{}) : F::mma(kf[ds], qf[cb][ds], s[cb]);
    };
    auto load_v = [&](const lds_char* va, int kt, h8 (&vf)[DT][2]) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const int kk = (kt * 2 + ks) * 16;
                vf[dt][ks] = v_frag<KT>(va + dt * 64 + kk * VP, va + dt * 64 + (kk + 8) * VP);
            }
    };
    auto mma_v = [&](const h8 (&vf)[DT][2], const h8 (&pf)[2][2]) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                for (int cb = 0; cb < 2; ++cb)
                    o[dt][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[dt][ks], pf[cb][ks], o[dt][cb], 0, 0, 0);
    };
    // softmax of k step ks (16 keys) of a half for both column blocks, with
    // the fixed exponent offsets of the loop
    float nbf[2];
    auto probs_ks = [&](const f32x16 (&s)[2], int ks, h8 (&pf)[2][2]) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            float ps = lsum[cb];
            h8 pv;
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const float p0 = __builtin_amdgcn_exp2f(fmaf(s[cb][ks * 8 + e], sl2, nbf[cb]));
                const float p1 = __builtin_amdgcn_exp2f(fmaf(s[cb][ks * 8 + e + 1], sl2, nbf[cb]));
                h2 pp = {(_Float16)p0, (_Float16)p1};
                pv[e] = pp.x;
                pv[e + 1] = pp.y;
                ps = __builtin_amdgcn_fdot2(pp, h2{(_Float16)1.0f, (_Float16)1.0f}, ps, false);
            }
            pf[cb][ks] = pv;
            lsum[cb] = ps;
        }
    };
    // a tile with masks: the implicit ones, or the explicit mask (scores
    // then carried in the exp2 domain, the row max tracked per tile: the
    // first visible tile sets m, a later one beyond m + 15 raises it)
    auto slow_tile = [&](const lds_char* ka, const lds_char* va, int k0, int restarts) -> bool {
        f32x16 s[2][2];
        s_half(ka, 0, s[0]);
        s_half(ka, 1, s[1]);
        float mul = sl2;
        bool raise = false;
        if constexpr (EXPL) {
            mul = 1.0f;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int cb = 0; cb < 2; ++cb) {
                    const char* mrow = a.mask + b * a.mask_nb_b + tcol[cb] * a.mask_nb_row;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int key = k0 + kt * 32 + 8 * (r / 4) + 4 * half + (r % 4);
                        const float x = fmaf(s[kt][cb][r], sl2,
                                             f16_to_f32(*(const uint16_t*)(mrow + 2 * min(key, L - 1))) * kLog2e);
                        s[kt][cb][r] = key > L - 1 ? -INFINITY : x;
                    }
                }
            float mx0[2], mx1[2];
            half_max(s[0], 1.0f, mx0);
            half_max(s[1], 1.0f, mx1);
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) {
                const float mx = fmaxf(mx0[cb], mx1[cb]);
                if (m[cb] == -INFINITY) m[cb] = mx;            // O and the row sum are still 0
                if (mx > m[cb] + kLazy && restarts < kMaxRestarts) {
                    raise = true;
                    m[cb] = mx;
                }
            }
            if (__any(raise)) return true;
        } else {
            mask_half(s[0], k0, 0);
            mask_half(s[1], k0, 1);
        }
        h8 pf0[2][2], pf1[2][2];
        probs(s[0], mul, pf0);
        pv_half(va, 0, pf0);
        probs(s[1], mul, pf1);
        pv_half(va, 1, pf1);
        return false;
    };
    // a p of the last tile overflowed f16 (its score passed m + 16), seen as
    // an inf or nan row sum
    auto overflow = [&](int restarts) -> bool {
        return !EXPL && restarts < kMaxRestarts && (!(lsum[0] <= 3.0e38f) || !(lsum[1] <= 3.0e38f));
    };
    // all tiles before j_fast are seen whole by every row of the workgroup
    const int t_lo_wg = min(a.T - 1, R0 / g);
    const int j_fast = EXPL ? 0 : max(0, min(n_tiles, (causal ? min(L, past + t_lo_wg + 1) : L) / kBN - j_lo));

    for (int restarts = 0;; ++restarts) {
        issue(0);
        issue(1);
        issue(2);
        wait_vm_barrier<2 * NLD>();                             // tile 0 is in LDS
        if (!EXPL && restarts == 0 && n_tiles > 0) {
            // m from half 0 of the first tile: visible to every row when it
            // lies in the fully visible range (the single-split case: key 0);
            // a row that cannot see it keeps m = -inf (exponent offset 0)
            // and a restart raises m should a later p overflow f16
            const lds_char *ka, *va;
            bases(0, ka, va);
            f32x16 s0[2];
            s_half(ka, 0, s0);
            mask_half(s0, kb0, 0);
            half_max(s0, sl2, m);
        }
        int j = 0;
        bool restart = false;
        // (the loops leave through their conditions only: an exit from the
        // middle makes the compiler copy O through VGPRs on every tile)
        int jb = 0;                                             // the tile that asked for the restart
        int bar = 0;                                            // barriers passed (flag slot parity)
        nbf[0] = m[0] == -INFINITY ? 0.0f : -m[0];
        nbf[1] = m[1] == -INFINITY ? 0.0f : -m[1];
        // ---- tiles every row of the workgroup sees whole: no masks, no
        // branches, pipelined across tiles.  Iteration j, in four scheduling
        // regions (sched_barrier) of 16 MFMAs, each beside a quarter of a
        // softmax that reads scores finished at least one region earlier:
        //   1  S of half 1 of tile j         | softmax, 2nd k step of half 0
        //      barrier: tile j + 1 in LDS, every wave done with tile j - 1
        //   2  S of half 0 of tile j + 1     | softmax, 1st k step of half 1
        //   3  P.V of half 0 of tile j       | softmax, 2nd k step of half 1
        //   4  P.V of half 1 of tile j       | softmax, 1st k step of half 0
        //                                      of tile j + 1
        // The loads of tile j + 3 go, after the barrier, into the stage tile
        // j - 1 used; a tile past the last, or any tile once a restart is
        // decided (the restart re-reads the stage of the tile that asked for
        // it), loads nothing.  A tile's overflow verdict is complete after
        // region 3 and published at the next barrier.
        f32x16 sc[2];                                           // S of half 0 of the current tile
        h8 pc[2][2];                                            // its p, first k step filled
        QF kf1[DS];                                             // K of half 1 of the current tile
        bool verdict = false;                                   // overflow up to the previous tile
        auto barrier_flags = [&](bool flag, bool two_ahead) -> bool {
            if (lane == 0) any_flag[bar & 1][w] = flag;
            if (two_ahead) wait_vm_barrier<2 * NLD>(); else wait_vm_barrier<NLD>();
            int any = 0;
#pragma unroll
            for (int i = 0; i < kWaves; ++i) any |= any_flag[bar & 1][i];
            ++bar;
            return any != 0;                                    // workgroup-uniform
        };
        if (j_fast > 0) {
            const lds_char *ka, *va;
            bases(0, ka, va);
            QF kf0[DS];
            load_k(ka, 0, kf0);
            mma_k(kf0, sc);
            probs_ks(sc, 0, pc);
            load_k(ka, 1, kf1);
        }
        // region 1 of tile j (shared by the loop and its last tile)
        auto region1 = [&](const lds_char* va, f32x16 (&s1)[2], h8 (&vf0)[DT][2]) {
            load_v(va, 0, vf0);
            mma_k(kf1, s1);
            probs_ks(sc, 1, pc);
            __builtin_amdgcn_sched_barrier(0);
        };
        for (; j + 1 < j_fast && !restart; ++j) {
            // O stays in AGPRs across the back-edge (without the hint the
            // compiler moves part of it through VGPRs on every tile)
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int cb = 0; cb < 2; ++cb) asm volatile("" : "+a"(o[dt][cb]));
            const lds_char *ka, *va, *kn, *vn;
            bases(j, ka, va);
            bases(j + 1, kn, vn);
            f32x16 s1[2], sn[2];
            h8 p1[2][2], pn[2][2], vf0[DT][2], vf1[DT][2];
            QF kf0[DS];
            region1(va, s1, vf0);
            if (barrier_flags(verdict, false)) {
                restart = true;
                jb = j - 1;
            }
            const bool live = !restart && j + 3 < n_tiles;
            // region 2
            load_k(kn, 0, kf0);
            issue_range(j + 3, 0, NLD / 2, live);
            mma_k(kf0, sn);
            probs_ks(s1, 0, p1);
            __builtin_amdgcn_sched_barrier(0);
            // region 3
            load_v(va, 1, vf1);
            issue_range(j + 3, NLD / 2, NLD, live);
            mma_v(vf0, pc);
            probs_ks(s1, 1, p1);
            __builtin_amdgcn_sched_barrier(0);
            verdict = __any(overflow(restarts));
            // region 4
            load_k(kn, 1, kf1);
            mma_v(vf1, p1);
            probs_ks(sn, 0, pn);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) {
                sc[cb] = sn[cb];
                pc[cb][0] = pn[cb][0];
            }
        }
        if (j_fast > 0 && !restart) {
            // the last of these tiles, j = j_fast - 1: no next tile to start;
            // the barrier at its end makes its stage free for the masked loop
            const lds_char *ka, *va;
            bases(j, ka, va);
            f32x16 s1[2];
            h8 p1[2][2], vf0[DT][2], vf1[DT][2];
            region1(va, s1, vf0);
            if (barrier_flags(verdict, false)) {
                restart = true;
                jb = j - 1;
            }
            issue_range(j + 3, 0, NLD, !restart && j + 3 < n_tiles);
            load_v(va, 1, vf1);
            probs_ks(s1, 0, p1);
            mma_v(vf0, pc);
            probs_ks(s1, 1, p1);
            mma_v(vf1, p1);
            if (barrier_flags(__any(overflow(restarts)), true) && !restart) {
                restart = true;
                jb = j;
            }
            ++j;
        }
        for (; j < n_tiles && !restart; ++j) {
            issue(j + 3);
            const lds_char *ka, *va;
            bases(j, ka, va);
            bool flag = false;
            if (kb0 + j * kBN < kend_w) flag = slow_tile(ka, va, kb0 + j * kBN, restarts) || overflow(restarts);
            // end of tile j: publish the restart flags, wait for tile j + 1
            // (the loads of tiles j + 2 and j + 3 may still fly)
            if (barrier_flags(__any(flag), true)) {
                restart = true;
                jb = j;
            }
        }
        if (!restart) {
            wait_vm_barrier<0>();                               // loads past the last tile
            break;
        }
        j = jb;
        wait_vm_barrier<0>();                                   // no load may land in a stage after the restart
        if (!EXPL && kb0 + j * kBN < kend_w) {
            // raise m for the rows whose scores on tile j passed m + 15 (tile j
            // is still in its stage: tile j + 4 was never issued)
            const lds_char *ka, *va;
            bases(j, ka, va);
            f32x16 s[2][2];
            s_half(ka, 0, s[0]);
            s_half(ka, 1, s[1]);
            mask_half(s[0], kb0 + j * kBN, 0);
            mask_half(s[1], kb0 + j * kBN, 1);
            float mx0[2], mx1[2];
            half_max(s[0], sl2, mx0);
            half_max(s[1], sl2, mx1);
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) {
                const float mx = fmaxf(mx0[cb], mx1[cb]);
                if (mx > m[cb] + kLazy) m[cb] = mx;
            }
        }
        __syncthreads();                                        // every wave is done with the stages
        lsum[0] = lsum[1] = 0.0f;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) o[dt][cb] = f32x16{};
    }

    // ---- normalize and write (each lane owns one row per column block);
    // with several key splits, write the split's partial instead: O
    // unnormalized, and (exponent base, row sum) of the row
    const int64_t nr_all = (int64_t)a.B * a.T * a.Hq;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
        const int row = wr0 + cb * 32 + l32;
        const float lt = lsum[cb] + __shfl_xor(lsum[cb], 32, 64);
        if (row >= nrows) continue;
        const int t = row / g, h = kvh * g + row % g;
        float* orow;
        float inv = 1.0f;
        if (n_ks == 1) {
            inv = lt > 0.0f ? 1.0f / lt : 0.0f;
            orow = (float*)((char*)a.out + b * a.o_nb_b + t * a.o_nb_t + h * a.o_nb_h);
        } else {
            const int64_t rg = ((int64_t)b * a.T + t) * a.Hq + h;
            orow = ws + ((int64_t)ks * nr_all + rg) * D;
            if (half == 0) {
                // p = 2^(s - base): base = m, or 0 while m = -inf; an empty row is -inf
                const float base = m[cb] != -INFINITY ? m[cb] : (lt > 0.0f ? 0.0f : -INFINITY);
                *(float2*)(ws + nr_all * D * n_ks + ((int64_t)ks * nr_all + rg) * 2) = make_float2(base, lt);
            }
        }
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

// Combines the key splits of every query row: one thread per (row, 4 dims),
// log-sum-exp over the n_ks partials (exp2 domain), normalized into out.
template <int D>
__global__ void __launch_bounds__(256) prefill_merge_kernel(AttnArgs a, const float* __restrict__ ws, int n_ks) {
    const int64_t nr_all = (int64_t)a.B * a.T * a.Hq;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t rg = idx / (D / 4);
    const int d4 = (int)(idx % (D / 4));
    if (rg >= nr_all) return;
    const float* ml = ws + nr_all * D * n_ks;
    float M = -INFINITY;
    for (int k = 0; k < n_ks; ++k) M = fmaxf(M, ml[((int64_t)k * nr_all + rg) * 2]);
    float den = 0.0f;
    float4 num = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (M != -INFINITY) {
        for (int k = 0; k < n_ks; ++k) {
            const float2 e = *(const float2*)(ml + ((int64_t)k * nr_all + rg) * 2);
            const float f = __builtin_amdgcn_exp2f(e.x - M);          // 0 for an empty split
            const float4 v = *(const float4*)(ws + ((int64_t)k * nr_all + rg) * D + 4 * d4);
            num.x = fmaf(v.x, f, num.x);
            num.y = fmaf(v.y, f, num.y);
            num.z = fmaf(v.z, f, num.z);
            num.w = fmaf(v.w, f, num.w);
            den = fmaf(e.y, f, den);
        }
    }
    const float inv = den > 0.0f ? 1.0f / den : 0.0f;
    const int h = (int)(rg % a.Hq), t = (int)((rg / a.Hq) % a.T), b = (int)(rg / ((int64_t)a.Hq * a.T));
    float* orow = (float*)((char*)a.out + b * a.o_nb_b + t * a.o_nb_t + h * a.o_nb_h);
    *(float4*)(orow + 4 * d4) = make_float4(num.x * inv, num.y * inv, num.z * inv, num.w * inv);
}

template <int D, int KT>
hipError_t launch_pf(const AttnArgs& a, float* ws, int n_ks, hipStream_t s) {
    const int g = a.Hq / a.Hkv;
    const int nrows = a.T * g;
    dim3 grid((nrows + kRowsWG - 1) / kRowsWG * n_ks, a.Hkv, a.B);
    if (a.mask_mode == kMaskExplicit)
        hipLaunchKernelGGL((prefill_kernel<D, KT, true>), grid, dim3(256), 0, s, a, ws, n_ks);
    else
        hipLaunchKernelGGL((prefill_kernel<D, KT, false>), grid, dim3(256), 0, s, a, ws, n_ks);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || n_ks == 1) return e;
    const int64_t threads = (int64_t)a.B * a.T * a.Hq * (D / 4);
    hipLaunchKernelGGL(prefill_merge_kernel<D>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, a, ws, n_ks);
    return hipGetLastError();
}

}  // namespace

bool prefill_supported(const AttnArgs& a) {
    if (a.T < 2) return false;
    if (a.d != 64 && a.d != 128) return false;
    if (a.k_type != a.v_type) return false;
    if (a.k_type != VVA_TYPE_F16 && a.k_type != VVA_TYPE_BF16) return false;
    if (a.Hq % a.Hkv != 0) return false;
    // 16-byte buffer loads of K/V rows, 32-bit buffer offsets (rows up to L),
    // 16-byte Q and output rows
    if (a.k_nb_tok % 16 || a.k_nb_head % 16 || a.v_nb_tok % 16 || a.v_nb_head % 16) return false;
    for (int b = 0; b < a.B; ++b) {
        if ((uintptr_t)a.k[b] % 16 || (uintptr_t)a.v[b] % 16) return false;
        if (a.L[b] < 1) return false;
        if ((int64_t)(a.L[b] + kBN) * a.k_nb_tok >= ((int64_t)1 << 30) ||
            (int64_t)(a.L[b] + kBN) * a.v_nb_tok >= ((int64_t)1 << 30)) return false;
    }
    if (((uintptr_t)a.q % 16) || a.q_nb_t % 16 || a.q_nb_h % 16 || a.q_nb_b % 16) return false;
    if (((uintptr_t)a.out % 16) || a.o_nb_t % 16 || a.o_nb_h % 16 || a.o_nb_b % 16) return false;
    if (a.mask_mode == kMaskExplicit && (a.mask_nb_row % 2 || a.mask_nb_b % 2)) return false;
    return true;
}

int prefill_plan(const AttnArgs& a, int n_cu) {
    // Key splits per row tile: only when the row tiles alone leave CUs idle
    // (a short chunk over a long past); as many as keep every workgroup in
    // one round on the CUs (a partial second round costs more than the
    // idle CUs it fills), each split at least 4 key tiles of the longest row
    // tile.
    const int g = a.Hq / a.Hkv;
    const int64_t base = (int64_t)((a.T * g + kRowsWG - 1) / kRowsWG) * a.Hkv * a.B;
    if (base >= n_cu) return 1;
    int Lmax = 1;
    for (int b = 0; b < a.B; ++b) Lmax = a.L[b] > Lmax ? a.L[b] : Lmax;
    const int max_ks = ((Lmax + kBN - 1) / kBN) / 4;
    int n_ks = (int)(n_cu / base);
    if (n_ks > max_ks) n_ks = max_ks;
    if (n_ks > kMaxKeySplits) n_ks = kMaxKeySplits;
    return n_ks < 1 ? 1 : n_ks;
}

size_t prefill_ws_bytes(const AttnArgs& a, int n_ks) {
    return n_ks <= 1 ? 0 : (size_t)n_ks * a.B * a.T * a.Hq * (a.d + 2) * sizeof(float);
}

hipError_t launch_prefill(const AttnArgs& a, float* ws, int n_ks, hipStream_t s) {
    if (a.d == 64) {
        return a.k_type == VVA_TYPE_F16 ? launch_pf<64, VVA_TYPE_F16>(a, ws, n_ks, s)
                                        : launch_pf<64, VVA_TYPE_BF16>(a, ws, n_ks, s);
    }
    return a.k_type == VVA_TYPE_F16 ? launch_pf<128, VVA_TYPE_F16>(a, ws, n_ks, s)
                                    : launch_pf<128, VVA_TYPE_BF16>(a, ws, n_ks, s);
}

}  // namespace vva
