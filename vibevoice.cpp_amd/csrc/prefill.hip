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
// padding is wasted for g = 7 or 6.  A workgroup is 8 waves (two per SIMD) x
// 32 rows = a 256-row tile and walks the key tiles (64 keys) its rows can
// see.  Workgroups go out heaviest row tile first, with the kv heads
// innermost so that the heads of one row tile run side by side (their K/V
// tiles stay in the XCD's L2).  When the row tiles alone would leave CUs
// idle (short chunks over a long past), a row tile's key tiles are split
// over several workgroups (PrefillPlan) whose partials prefill_merge_kernel
// combines by log-sum-exp.
//
// Staging.  K and V tiles go from HBM straight into LDS with buffer loads
// that write LDS (no registers, no VALU), into a ring of four stages: the
// loads of tile j + 3 go out at the start of tile j.  Both tiles are kept
// row-major ([key][dim]); K rows are padded to 16 mod 256 bytes and V rows
// to 64 mod 256 bytes, which keeps both operand reads free of bank
// conflicts.  The V^T operand of the second product is read with
// ds_read_b64_tr_b16, whose 16-lane transpose hands each lane 4 consecutive
// keys of one dim.  Keys past L read as 0 through the buffer range check.
//
// Per wave and key tile, with v_mfma_f32_32x32x16_{f16,bf16}:
//   S^T[key][row] = K . Q^T  A = K rows from LDS (16 B per lane), B = Q^T
//                            held in registers for the whole kernel, so each
//                            lane owns one query row (column) of S^T and the
//                            softmax row reductions are in-register plus one
//                            cross-half exchange;
//   softmax                  fp32, exp2 domain, on the raw scores (the scale
//                            folded into the exp's fma); the running max m of
//                            a row is raised lazily, only when a tile's row
//                            max passes it by more than 2^8, so p <= 256 fits
//                            f16 and O and the row sum are rescaled rarely;
//   O^T[d][row] += V^T . P^T B = P^T converted in place from the S^T
//                            accumulators: the key order of an MFMA step is
//                            chosen to be the one the accumulator layout
//                            already has, so no shuffle is needed.
// Tiles whose last key some row of the wave must not see (the diagonal, the
// length boundary, or an explicit mask) set those scores to -inf first.
// P and V enter the second product as f16 (BF16 V is converted after the
// transposing read): an 8-bit-mantissa P would cost up to ~4e-3 on short
// rows, f16 P stays below 4e-4.  Q is rounded to K's type, as ggml's CPU
// flash attention does.  Q8_0 and F32 windows are converted to f16 first by
// window_to_f16_kernel (the reference casts F32 windows the same way before
// flash attention, src/qwen2.cpp:328-331; for Q8_0 K, Q takes the Q8_0
// round trip ggml's vec-dot type implies).
#include "vva_internal.hpp"

#include <algorithm>
#include <type_traits>
#include <functional>
#include <vector>

namespace vva {

namespace {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

#include "mfma_ops.hpp"

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 8.0f;      // running-max slack in log2 units: p <= 2^8 (f16-safe, rare rescales)
constexpr int kBN = 64;            // keys per tile
constexpr int kRowsWave = 32;      // query rows per wave: one 32-wide MFMA column block
constexpr int kWaves = 8;          // two per SIMD
constexpr int kRowsWG = kRowsWave * kWaves;
constexpr int kStages = 4;         // LDS ring: tile j + 3 loads while tile j is computed
constexpr int kMaxKeySplits = 32;  // key splits per row tile

// Key tiles of row tile rt (rows rt * kRowsWG ..) of sequence b: the keys
// its last row sees (causal), or all of them.
__host__ __device__ inline int rt_key_tiles(const AttnArgs& a, int b, int rt, bool causal) {
    const int g = a.Hq / a.Hkv, nrows = a.T * g;
    const int t_hi = min(a.T - 1, (min((rt + 1) * kRowsWG, nrows) - 1) / g);
    const int kend = causal ? min(a.L[b], a.past[b] + t_hi + 1) : a.L[b];
    return (kend + kBN - 1) / kBN;
}
// Workgroups row tile rt is split over.
__host__ __device__ inline int rt_splits(const PrefillPlan& p, int rt) {
    return p.forced > 0 ? p.forced : (rt >= p.R ? p.n : 1);
}
// Pieces (workgroups per kv head and sequence) of a plan over n_rt row tiles.
__host__ __device__ inline int plan_pieces(const PrefillPlan& p, int n_rt) {
    return p.forced > 0 ? n_rt * p.forced : (n_rt - p.R) * p.n + p.R;
}

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

// Raw buffer descriptor as four wave-uniform dwords (kept in SGPRs for the
// inline-asm loads): base address (48 bits, stride 0), range in bytes, and
// the gfx9 raw-buffer configuration word; loads past the range return 0.
__device__ __forceinline__ i32x4 make_rsrc(const char* base, uint32_t bytes) {
    const uint64_t p = (uint64_t)(uintptr_t)base;
    return i32x4{__builtin_amdgcn_readfirstlane((int)(uint32_t)p),
                 __builtin_amdgcn_readfirstlane((int)((uint32_t)(p >> 32) & 0xffffu)),
                 __builtin_amdgcn_readfirstlane((int)bytes), 0x00020000};
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

__device__ __forceinline__ float bits16_to_f32(uint32_t v, int type) {
    return type == VVA_TYPE_BF16 ? bf16_to_f32((uint16_t)v) : f16_to_f32((uint16_t)v);
}

__device__ __forceinline__ const lds_char* lds_at(uint32_t addr) { return (const lds_char*)(uintptr_t)addr; }

// EXPL: explicit F16 mask (otherwise implicit causal / length masking only).
template <int D, int KT, bool EXPL>
__global__ void __launch_bounds__(kWaves * 64) prefill_kernel(AttnArgs a, float* __restrict__ ws, unsigned* tickets,
                                                               PrefillPlan plan) {
    prefetch_kernargs<sizeof(AttnArgs)>();
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
    const int b = blockIdx.z;
    const int g = a.Hq / a.Hkv;
    const int nrows = a.T * g;
    const int n_rt = (nrows + kRowsWG - 1) / kRowsWG;
    const bool causal = !EXPL && a.mask_mode == kMaskCausal;
    // Workgroups go out heaviest row tile first, the kv heads innermost (so
    // every head's heaviest tiles start in the first round), then the row
    // tile's key splits: piece x of the sequence is found by walking the row
    // tiles from the last (heaviest) down.
    const int kvh = (int)blockIdx.x % a.Hkv;
    const int x = (int)blockIdx.x / a.Hkv;
    const int nh = plan.forced > 0 ? plan.forced : plan.n;                // splits of a heavy row tile
    const int R = plan.forced > 0 ? 0 : plan.R;
    const int heavy = (n_rt - R) * nh;                                   // pieces of the heavy row tiles
    const int rt = x < heavy ? n_rt - 1 - x / nh : R - 1 - (x - heavy);
    const int ks = x < heavy ? x % nh : 0;                               // key split of the row tile
    const int n_ks = x < heavy ? nh : 1;
    const int R0 = rt * kRowsWG;
    const int wr0 = R0 + w * kRowsWave;
    const int L = a.L[b], past = a.past[b];

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
    // keys [0, kend_w) are seen by some row of the wave; keys up to lim_w by
    // every row (a tile whose last key is at most lim_w needs no mask)
    const int kend_w = !wave_live ? 0 : (causal ? min(L, past + t_hi_w + 1) : L);
    const int lim_w = causal ? min(L - 1, past + t_lo_w) : L - 1;

    // ---- tile loads: per lane and 1 KB chunk q = i * kWaves + w of an
    // operand, the byte x = 1024 q + 16 lane of the padded tile is row x /
    // pitch, column x % pitch; pad bytes load from an offset past the buffer
    // (0 bytes read, zeros written), and a wave's loads past the last chunk
    // write zeros to the junk kilobyte (every wave issues the same number of
    // loads per tile, with no branch)
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
    // the loads of tile j (K chunks, then V); a tile past the last one reads
    // from past the buffer (zeros, no memory traffic) into the junk
    // kilobyte, so the count of loads per tile stays the same
    auto issue = [&](int j) {
        const bool live = j < n_tiles;
        const uint32_t st = lds0 + (j % kStages) * STAGE;
        const int sk = live ? (int)((uint32_t)(j * kBN) * nbk) : 0x40000000;
        const int sv = live ? (int)((uint32_t)(j * kBN) * nbv) : 0x40000000;
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            if (i < NIK) {
                const int c = i * kWaves + w;
                dma16(krs, live && c < NCK ? st + c * 1024 : lds0 + JUNK, koff[i], sk);
            } else {
                const int c = (i - NIK) * kWaves + w;
                dma16(vrs, live && c < NCV ? st + KREG + c * 1024 : lds0 + JUNK, voff[i - NIK], sv);
            }
        }
    };
    // tile 0 goes out before Q is loaded: the wait for Q then covers it
    // (the loads complete in order), and tiles 1 and 2 follow once Q is in
    // registers
    issue(0);

    // ---- this lane's query row (column l32 of the wave's 32-row block) and
    // its Q^T fragments, rounded to K's type
    const int row = wr0 + l32;
    const bool qok = row < nrows;
    const int tcol = qok ? row / g : a.T - 1;
    const char* qrow = a.q + b * a.q_nb_b + (int64_t)(qok ? row / g : 0) * a.q_nb_t +
                       (int64_t)(kvh * g + (qok ? row % g : 0)) * a.q_nb_h;
    QF qf[DS];
    {
        // the lane's 8 dims ds * 16 + 8 half .. of each 16-dim step, as fp32
        float x[DS][8];
        if (a.q_type == VVA_TYPE_F32) {
#pragma unroll
            for (int ds = 0; ds < DS; ++ds) {
                const float4 x0 = *(const float4*)(qrow + (ds * 16 + half * 8) * 4);
                const float4 x1 = *(const float4*)(qrow + (ds * 16 + half * 8) * 4 + 16);
                x[ds][0] = x0.x; x[ds][1] = x0.y; x[ds][2] = x0.z; x[ds][3] = x0.w;
                x[ds][4] = x1.x; x[ds][5] = x1.y; x[ds][6] = x1.z; x[ds][7] = x1.w;
            }
        } else {
            const int qt = a.q_type;
#pragma unroll
            for (int ds = 0; ds < DS; ++ds) {
                const u32x4 r = *(const u32x4*)(qrow + (ds * 16 + half * 8) * 2);
                const uint32_t rw[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    x[ds][2 * k] = bits16_to_f32(rw[k] & 0xffffu, qt);
                    x[ds][2 * k + 1] = bits16_to_f32(rw[k] >> 16, qt);
                }
            }
        }
        if (a.q_round_q8) {
            // Q8_0 round trip per 32-dim block (steps 2 bb, 2 bb + 1; the
            // other 16 values of the block sit in lane l ^ 32): ggml's dot
            // type for Q8_0 K, as fp16 d times the integer code
#pragma unroll
            for (int bb = 0; bb < DS / 2; ++bb) {
                float am = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) am = fmaxf(am, fmaxf(fabsf(x[2 * bb][e]), fabsf(x[2 * bb + 1][e])));
                am = max_swap32(am);
                const float dq = am / 127.0f;
                const float id = dq != 0.0f ? 1.0f / dq : 0.0f;
                const float dh = bits16_to_f32(f32_to_f16(dq), VVA_TYPE_F16);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    x[2 * bb][e] = dh * roundf(x[2 * bb][e] * id);
                    x[2 * bb + 1][e] = dh * roundf(x[2 * bb + 1][e] * id);
                }
            }
        }
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
            uint32_t cw[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) cw[k] = F::cvt(x[ds][2 * k]) | ((uint32_t)F::cvt(x[ds][2 * k + 1]) << 16);
            qf[ds] = as_vec<QF>(qok ? u32x4{cw[0], cw[1], cw[2], cw[3]} : u32x4{0u, 0u, 0u, 0u});
        }
    }
    issue(1);
    issue(2);

    // Running max m (log2 domain) of the lane's row, raised lazily: only when
    // a tile's row max passes it by more than kLazy, so p <= 2^kLazy in f16
    // and O / the row sum are rescaled rarely.
    float m = -INFINITY, lsum = 0.0f;
    f32x16 o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt] = f32x16{};
    const float sl2 = a.scale * kLog2e;
    // per-lane LDS offsets of the operand reads within a stage
    const int k_rd = l32 * KP + half * 16;                                   // K: key l32, dims 8 half ..
    const int v_rd = v_frag_offset(lane, VP);                                // V^T, see v_frag
    const char* mrow = EXPL ? a.mask + b * a.mask_nb_b + tcol * a.mask_nb_row : nullptr;

    // S^T of the tile's two 32-key halves: key 8 (r / 4) + 4 half + r % 4
    // of half kt in register r, for the lane's row
    // (the two halves' MFMA chains interleaved, every K fragment of the tile
    // read up front)
    auto scores = [&](const lds_char* ka, f32x16 (&s)[2]) {
        u32x4 kraw[2][DS];
#pragma unroll
        for (int ds = 0; ds < DS; ++ds)
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
                kraw[kt][ds] = *(const __attribute__((address_space(3))) u32x4*)(ka + kt * 32 * KP + ds * 32);
#pragma unroll
        for (int ds = 0; ds < DS; ++ds)
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
                s[kt] = F::mma(as_vec<QF>(kraw[kt][ds]), qf[ds], ds == 0 ? f32x16{} : s[kt]);
    };
    // Masked keys to -inf and explicit mask values added in score units
    // (mask / scale, so that 2^(s * scale * log2 e) carries e^mask).  MASKED:
    // the tile may hold keys past the row's last visible one (causal or
    // length) or the caller passed a mask.
    const float inv_scale = 1.0f / a.scale;
    auto apply_mask = [&](f32x16 (&s)[2], int k0) {
        const int lim = causal ? min(L - 1, past + tcol) : L - 1;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = k0 + kt * 32 + 8 * (r / 4) + 4 * half + (r % 4);
                float x = s[kt][r];
                if constexpr (EXPL)
                    x = fmaf(mask_at(mrow, min(key, L - 1), a.mask_f32), inv_scale, x);
                s[kt][r] = key > lim ? -INFINITY : x;
            }
    };
    // The row max of a tile's raw scores, in the exp2 domain (with the row's
    // other 32 keys in lane l ^ 32).
    auto rowmax = [&](const f32x16 (&s)[2]) {
        float mr = fmaxf(fmaxf(s[0][0], s[0][1]), s[0][2]);
#pragma unroll
        for (int r = 3; r < 15; r += 2) mr = fmaxf(fmaxf(mr, s[0][r]), s[0][r + 1]);
        mr = fmaxf(mr, s[0][15]);
#pragma unroll
        for (int r = 0; r < 16; r += 2) mr = fmaxf(fmaxf(mr, s[1][r]), s[1][r + 1]);
        return max_swap32(mr) * sl2;
    };
    // Raise the running max lazily to a tile's row max mx: O and the row sum
    // are rescaled only when mx passes m by more than kLazy.
    auto rescale = [&](float mx) {
        if (__any(mx > m + kLazy)) {
            if (mx > m + kLazy) {
                const float alpha = __builtin_amdgcn_exp2f(m - mx);   // 0 while m = -inf
                lsum *= alpha;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) o[dt] *= alpha;
                m = mx;
            }
        }
    };
    // Software pipeline over the key tiles.  Step j first raises the running
    // max to tile j's row max (found by the previous step), then runs one
    // straight-line block of 2 DS + 4 DT matrix-core slots: the score MFMAs of
    // tile j + 1, then the P.V MFMAs of tile j.  Between them go the VALU
    // work of tile j's softmax (one fma and one exp2 per score, the f16
    // packing and the row sum) and the LDS operand reads, each placed a few
    // slots before its MFMA, so that the VALU issues while the matrix cores
    // run.  Tile j + 1's mask (on the tiles that need one) and row max follow
    // the block.  Scheduling fences between the slots keep this order.  The wave's live tiles are its first n_live (the tiles
    // are in key order and the wave sees keys below kend_w only).
    const int n_live = wave_live ? max(0, min(n_tiles, (kend_w - kb0 + kBN - 1) / kBN)) : 0;
    auto k_addr = [&](int j) {
        uint32_t x = lds0 + (j % kStages) * STAGE + k_rd;
        asm volatile("" : "+v"(x));                              // one base register, constant offsets
        return lds_at(x);
    };
    auto needs_mask = [&](int j) { return EXPL || kb0 + j * kBN + kBN - 1 > lim_w; };
    constexpr int NQ = 2 * DS;                                   // score MFMAs per tile
    constexpr int NP = 4 * DT;                                   // P.V MFMAs per tile
    constexpr int KAHEAD = 2;                                    // K fragment reads ahead of their MFMA
    constexpr int VAHEAD = 2;                                    // V^T fragment reads ahead of their MFMA
    auto block = [&](const f32x16 (&cur)[2], f32x16 (&nxt)[2], const lds_char* ka, const lds_char* va) {
        const float nb = m == -INFINITY ? 0.0f : -m;            // no visible key yet: every s is -inf
        u32x4 kf[NQ];
        h8 vf[NP];
        float pe[32];
        h8 pf[4];
        float ps = lsum;
        auto read_k = [&](int i) {
            kf[i] = *(const __attribute__((address_space(3))) u32x4*)(ka + (i & 1) * 32 * KP + (i >> 1) * 32);
        };
        auto read_v = [&](int p) {
            const int kk = (p / DT) * 16, dt = p % DT;
            vf[p] = v_frag<KT>(va + dt * 64 + kk * VP, va + dt * 64 + (kk + 8) * VP);
        };
        // The softmax of score v (p = 2^(s * scale * log2 e - m), then f16
        // pairs packed into chunk v / 8 = one 16-key MFMA step's P^T, and
        // the row sum) is itself pipelined over the slots, so that no VALU
        // instruction waits on the one before it: the fma of v in slot
        // fslot(v), its exp2 one slot later, the f16 pack of pair (2i, 2i + 1)
        // three slots after the fma of 2i + 1, its row-sum term one slot
        // after that.  The fmas are spread over the first NS - 8 slots, which
        // completes chunk c before its first P.V MFMA (slot NQ + c DT).
        constexpr int NS = NQ + NP;
        auto fslot = [](int v) { return v * (NS - 8) / 32; };
        auto pair_slot = [&](int i) { return fslot(2 * i + 1) + 3; };
        static_assert(((31 * (NQ + NP - 8)) / 32) + 3 < NQ + 3 * DT, "chunk 3 packed before its P.V");
        auto valu_slot = [&](int sl) {
#pragma unroll
            for (int v = 0; v < 32; ++v) {
                if (fslot(v) == sl) pe[v] = fmaf(cur[v >> 4][v & 15], sl2, nb);
                if (fslot(v) + 1 == sl) pe[v] = __builtin_amdgcn_exp2f(pe[v]);
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                if (pair_slot(i) == sl) {
                    const h2 pp = {(_Float16)pe[2 * i], (_Float16)pe[2 * i + 1]};
                    pf[i >> 2][2 * (i & 3)] = pp.x;
                    pf[i >> 2][2 * (i & 3) + 1] = pp.y;
                }
                if (pair_slot(i) + 1 == sl) {
                    const h2 pp = {pf[i >> 2][2 * (i & 3)], pf[i >> 2][2 * (i & 3) + 1]};
                    ps = __builtin_amdgcn_fdot2(pp, h2{(_Float16)1.0f, (_Float16)1.0f}, ps, false);
                }
            }
        };
#pragma unroll
        for (int i = 0; i < KAHEAD; ++i) read_k(i);
#pragma unroll
        for (int sl = 0; sl < NS; ++sl) {
            if (sl < NQ) {
                const int ds = sl >> 1, kt = sl & 1;
                nxt[kt] = F::mma(as_vec<QF>(kf[sl]), qf[ds], ds == 0 ? f32x16{} : nxt[kt]);
                if (sl + KAHEAD < NQ) read_k(sl + KAHEAD);
            } else if (sl < NS) {
                const int p = sl - NQ;
                o[p % DT] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[p], pf[p / DT], o[p % DT], 0, 0, 0);
            }
            if (sl - NQ + VAHEAD >= 0 && sl - NQ + VAHEAD < NP) read_v(sl - NQ + VAHEAD);
            valu_slot(sl);
            __builtin_amdgcn_sched_barrier(0);
        }
        lsum = ps;
    };
    // K of tile 0 has landed (its V and tiles 1, 2 may still fly)
    wait_vm_barrier<NIV + 2 * NLD>();
    f32x16 sa[2], sb[2];
    float mx = 0.0f;
    if (n_live > 0) {
        scores(k_addr(0), sa);
        if (needs_mask(0)) apply_mask(sa, kb0);
        mx = rowmax(sa);
    }
    auto step = [&](int j, const f32x16 (&cur)[2], f32x16 (&nxt)[2]) {
        // K of tile j + 1 and V of tile j have landed (loads complete in
        // order; V of j + 1 and tile j + 2 may still fly), and every wave is
        // done with tile j - 1, whose stage tile j + 3 now takes
        wait_vm_barrier<NIV + NLD>();
        issue(j + 3);
        if (j < n_live) {                                        // wave-uniform
            rescale(mx);
            uint32_t vaddr = lds0 + (j % kStages) * STAGE + KREG + v_rd;
            asm volatile("" : "+v"(vaddr));
            // tile j + 1's scores are computed whether or not the wave sees
            // it: past the wave's last live tile no step reads them
            block(cur, nxt, k_addr(j + 1), lds_at(vaddr));
            if (needs_mask(j + 1)) apply_mask(nxt, kb0 + (j + 1) * kBN);
            mx = rowmax(nxt);
        }
    };
    int j = 0;
    for (; j + 1 < n_tiles; j += 2) {
        step(j, sa, sb);
        step(j + 1, sb, sa);
    }
    if (j < n_tiles) step(j, sa, sb);
    wait_vm_barrier<0>();                                       // the padding tiles' loads

    // ---- normalize and write (each lane owns its row; lanes l and l ^ 32
    // summed different keys); with several key splits, write the split's
    // partial instead: O unnormalized, and (exponent base, row sum)
    const int64_t nr_all = (int64_t)a.B * a.T * a.Hq;
    const float lt = lsum + __shfl_xor(lsum, 32, 64);
    const int t = row / g, h = kvh * g + row % g;
    float* const orow = (float*)((char*)a.out + b * a.o_nb_b + (int64_t)t * a.o_nb_t + (int64_t)h * a.o_nb_h);
    if (n_ks == 1) {
        if (!qok) return;
        const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const int d = dt * 32 + 8 * q4 + 4 * half;
                *(float4*)(orow + d) = make_float4(o[dt][4 * q4] * inv, o[dt][4 * q4 + 1] * inv,
                                                   o[dt][4 * q4 + 2] * inv, o[dt][4 * q4 + 3] * inv);
            }
        return;
    }
    // p = 2^(x - base): base = m, or 0 while m = -inf; an empty row is -inf
    const float base = m != -INFINITY ? m : (lt > 0.0f ? 0.0f : -INFINITY);
    const int64_t rg = ((int64_t)b * a.T + t) * a.Hq + h;
    float* const wml = ws + nr_all * D * plan.max_ks;            // (base, row sum) of [split][row]
    if (!plan.in_launch) {
        // prefill_merge_kernel combines the partials
        if (!qok) return;
        float* prow = ws + ((int64_t)ks * nr_all + rg) * D;
        if (half == 0) *(float2*)(wml + ((int64_t)ks * nr_all + rg) * 2) = make_float2(base, lt);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const int d = dt * 32 + 8 * q4 + 4 * half;
                *(float4*)(prow + d) = make_float4(o[dt][4 * q4], o[dt][4 * q4 + 1], o[dt][4 * q4 + 2], o[dt][4 * q4 + 3]);
            }
        return;
    }
    // In-launch merge (n_ks <= kMaxInLaunchSplits).  Each split's partial is
    // one block of the workspace, [wave][16-dim group][lane] float4s then
    // [wave][lane] (base, row sum), so that every store and load instruction
    // moves whole contiguous lines; they go out with agent-scope (sc1)
    // buffer stores, coherent across the XCDs without an L2 write-back.  The
    // workgroup then takes its row tile's ticket; the last of the n_ks splits
    // combines every partial with its own registers, in split order and with
    // the arithmetic of prefill_merge_kernel (the same result bit for bit),
    // and resets the ticket for the next call.
    constexpr int kSc1 = 16;                                     // cache policy: agent scope
    constexpr int WAVE_O = DT * 16 * 64 * 4;                     // bytes of a wave's O block
    constexpr int PIECE = kWaves * (WAVE_O + 64 * 8);            // bytes of one split's partial
    const int64_t tile_piece = (((int64_t)b * a.Hkv + kvh) * n_rt + rt) * plan.max_ks;
    auto piece_rsrc = [&](int k) {
        return __builtin_amdgcn_make_buffer_rsrc((char*)ws + (tile_piece + k) * PIECE, 0, PIECE, 0x00020000);
    };
    const int o_off = w * WAVE_O + lane * 16;                   // + 1024 per 16-dim group
    const int ml_off = kWaves * WAVE_O + w * 512 + lane * 8;
    {
        const __amdgpu_buffer_rsrc_t rs = piece_rsrc(ks);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const u32x4 v = {__float_as_uint(o[dt][4 * q4]), __float_as_uint(o[dt][4 * q4 + 1]),
                                 __float_as_uint(o[dt][4 * q4 + 2]), __float_as_uint(o[dt][4 * q4 + 3])};
                __builtin_amdgcn_raw_buffer_store_b128(v, rs, o_off + (dt * 4 + q4) * 1024, 0, kSc1);
            }
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(base), __float_as_uint(lt)}, rs, ml_off, 0, kSc1);
    }
    // every partial store of the workgroup has completed before its ticket;
    // the ring's LDS is idle (every wave passed the last tile barrier)
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    int* const last = (int*)lds;
    if (tid == 0) {
        unsigned* tk = tickets + ((int64_t)b * a.Hkv + kvh) * n_rt + rt;
        const unsigned old = __hip_atomic_fetch_add(tk, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *last = old == (unsigned)(n_ks - 1);
        if (*last) __hip_atomic_store(tk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!*last || !qok) return;
    // every other split's (base, row sum) and the first other split's O go
    // out in one batch (one memory round trip at two splits)
    const int k0 = ks == 0 ? 1 : 0;
    float2 mlk[kMaxInLaunchSplits];
#pragma unroll
    for (int k = 0; k < kMaxInLaunchSplits; ++k) {
        if (k >= n_ks) continue;
        if (k == ks) {
            mlk[k] = make_float2(base, lt);
        } else {
            const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(piece_rsrc(k), ml_off, 0, kSc1);
            mlk[k] = make_float2(__uint_as_float(v.x), __uint_as_float(v.y));
        }
    }
    u32x4 ov[DT * 4];
    {
        const __amdgpu_buffer_rsrc_t rs = piece_rsrc(k0);
#pragma unroll
        for (int i = 0; i < DT * 4; ++i) ov[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, o_off + i * 1024, 0, kSc1);
        // keep the loads here, in the batch (not sunk into the branch below)
#pragma unroll
        for (int i = 0; i < DT * 4; ++i) asm volatile("" : "+v"(ov[i]));
    }
    float M = -INFINITY;
#pragma unroll
    for (int k = 0; k < kMaxInLaunchSplits; ++k)
        if (k < n_ks) M = fmaxf(M, mlk[k].x);
    float num[DT][16];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) num[dt][r] = 0.0f;
    float den = 0.0f;
    if (M != -INFINITY) {
#pragma unroll
        for (int k = 0; k < kMaxInLaunchSplits; ++k) {
            if (k >= n_ks) continue;
            const float f = __builtin_amdgcn_exp2f(mlk[k].x - M);       // 0 for an empty split
            if (k == ks) {
#pragma unroll
                for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                    for (int r = 0; r < 16; ++r) num[dt][r] = fmaf(o[dt][r], f, num[dt][r]);
            } else {
                if (k != k0) {
                    const __amdgpu_buffer_rsrc_t rs = piece_rsrc(k);
#pragma unroll
                    for (int i = 0; i < DT * 4; ++i)
                        ov[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, o_off + i * 1024, 0, kSc1);
                }
#pragma unroll
                for (int i = 0; i < DT * 4; ++i)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        num[i / 4][4 * (i % 4) + e] = fmaf(__uint_as_float(ov[i][e]), f, num[i / 4][4 * (i % 4) + e]);
            }
            den = fmaf(mlk[k].y, f, den);
        }
    }
    const float inv = den > 0.0f ? 1.0f / den : 0.0f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            const int d = dt * 32 + 8 * q4 + 4 * half;
            *(float4*)(orow + d) = make_float4(num[dt][4 * q4] * inv, num[dt][4 * q4 + 1] * inv,
                                               num[dt][4 * q4 + 2] * inv, num[dt][4 * q4 + 3] * inv);
        }
}


// Combines the key splits of every split query row: one thread per (row,
// 4 dims), log-sum-exp over the row tile's partials (exp2 domain),
// normalized into out.  Rows of unsplit row tiles were written directly.
template <int D>
__global__ void __launch_bounds__(256) prefill_merge_kernel(AttnArgs a, const float* __restrict__ ws, PrefillPlan plan) {
    prefetch_kernargs<sizeof(AttnArgs)>();
    const int64_t nr_all = (int64_t)a.B * a.T * a.Hq;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t rg = idx / (D / 4);
    const int d4 = (int)(idx % (D / 4));
    if (rg >= nr_all) return;
    const int h = (int)(rg % a.Hq), t = (int)((rg / a.Hq) % a.T), b = (int)(rg / ((int64_t)a.Hq * a.T));
    const int g = a.Hq / a.Hkv, kvh = h / g;
    const int rt = (t * g + (h - kvh * g)) / kRowsWG;
    const int n_ks = rt_splits(plan, rt);
    if (n_ks == 1) return;
    const float* ml = ws + nr_all * D * plan.max_ks;
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
    float* orow = (float*)((char*)a.out + b * a.o_nb_b + t * a.o_nb_t + h * a.o_nb_h);
    *(float4*)(orow + 4 * d4) = make_float4(num.x * inv, num.y * inv, num.z * inv, num.w * inv);
}

template <int D, int KT>
hipError_t launch_pf(const AttnArgs& a, float* ws, unsigned* tickets, const PrefillPlan& p, hipStream_t s) {
    const int n_rt = (a.T * (a.Hq / a.Hkv) + kRowsWG - 1) / kRowsWG;
    dim3 grid(plan_pieces(p, n_rt) * a.Hkv, 1, a.B);
    if (a.mask_mode == kMaskExplicit)
        hipLaunchKernelGGL((prefill_kernel<D, KT, true>), grid, dim3(kWaves * 64), 0, s, a, ws, tickets, p);
    else
        hipLaunchKernelGGL((prefill_kernel<D, KT, false>), grid, dim3(kWaves * 64), 0, s, a, ws, tickets, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || p.max_ks == 1 || p.in_launch) return e;
    const int64_t threads = (int64_t)a.B * a.T * a.Hq * (D / 4);
    hipLaunchKernelGGL(prefill_merge_kernel<D>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, a, ws, p);
    return hipGetLastError();
}

// Strided windows (and F32 ones): quarter q of 32-element block k of a K or
// V head row of one sequence (8 consecutive elements) per thread and pass; consecutive threads take
// consecutive quarters, so a wave's store writes 1 KB contiguously.  Each
// thread takes kWinPasses quarters a grid apart, every load issued before
// the first conversion: grid (quarters of the longest window /
// (256 * kWinPasses), 2 B: K and V of each sequence).  Q8_0: d * q in fp32
// (exact: an 11-bit scale times a 7-bit code) rounded once to f16; F32:
// rounded to f16.
constexpr int kWinPasses = 1;       // 4 measured no faster on Q8_0 windows (13.8 against 13.1 us average)

__global__ void __launch_bounds__(256) window_to_f16_kernel(AttnArgs a, uint16_t* __restrict__ dst,
                                                            unsigned long long* ovf, unsigned long long epoch) {
    prefetch_kernargs<sizeof(AttnArgs)>();
    const int b = blockIdx.y >> 1, which = blockIdx.y & 1;
    const int nblk = a.d / 32;
    const int L = a.L[b];
    const int64_t n4 = (int64_t)L * a.Hkv * nblk * 4;                 // quarters of the window
    const int64_t stride = (int64_t)gridDim.x * 256;
    const int64_t i0 = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i0 >= n4) return;
    const int type = which ? a.v_type : a.k_type;
    const int64_t nb_tok = which ? a.v_nb_tok : a.k_nb_tok, nb_head = which ? a.v_nb_head : a.k_nb_head;
    const char* base = which ? a.v[b] : a.k[b];
    size_t off = 0;                                                   // this sequence's K, then V
    for (int b2 = 0; b2 < b; ++b2) off += (size_t)2 * a.L[b2] * a.Hkv * a.d;
    uint16_t* const obase = dst + off + (size_t)which * L * a.Hkv * a.d;
    // the source bytes of quarter i4 (row, head, block, quarter)
    auto src_of = [&](int64_t i4, int& q) {
        q = (int)(i4 & 3);
        const int64_t i = i4 >> 2;
        const int bk = (int)(i % nblk), h = (int)((i / nblk) % a.Hkv);
        const int64_t row = i / ((int64_t)nblk * a.Hkv);
        return base + row * nb_tok + h * nb_head + (type == VVA_TYPE_Q8_0 ? bk * kQ8Bytes : bk * 32 * 4);
    };
    uint32_t w[kWinPasses][4];
    if (type == VVA_TYPE_Q8_0) {
        // the block's scale and codes 8 q .. 8 q + 7 (2-byte aligned): dwords
        // from the 4-byte boundary at or below them (a dword holding a byte
        // of the block lies in the block's page)
        uint32_t sw[kWinPasses], c0[kWinPasses], c1[kWinPasses], c2[kWinPasses];
        bool odd[kWinPasses], sodd[kWinPasses];
#pragma unroll
        for (int u = 0; u < kWinPasses; ++u) {
            const int64_t i4 = min(i0 + u * stride, n4 - 1);        // (clamped: stored only when in range)
            int q;
            const uintptr_t sa = (uintptr_t)src_of(i4, q), ca = sa + 2 + 8 * q;
            sodd[u] = (sa & 2) != 0;
            odd[u] = (ca & 2) != 0;
            sw[u] = *(const uint32_t*)(sa & ~(uintptr_t)3);
            const uint32_t* cw = (const uint32_t*)(ca & ~(uintptr_t)3);
            c0[u] = cw[0];
            c1[u] = cw[1];
            c2[u] = odd[u] ? cw[2] : 0u;
        }
        bool inf = false;
#pragma unroll
        for (int u = 0; u < kWinPasses; ++u) {
            const float d = f16_to_f32((uint16_t)(sodd[u] ? (sw[u] >> 16) : (sw[u] & 0xffffu)));
            const uint32_t x0 = odd[u] ? __builtin_amdgcn_alignbyte(c1[u], c0[u], 2) : c0[u];
            const uint32_t x1 = odd[u] ? __builtin_amdgcn_alignbyte(c2[u], c1[u], 2) : c1[u];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t c = e < 2 ? x0 : x1, sh = 16 * (e & 1);
                w[u][e] = (uint32_t)f32_to_f16(d * (float)(int8_t)(c >> sh)) |
                          ((uint32_t)f32_to_f16(d * (float)(int8_t)(c >> (sh + 8))) << 16);
                // a value beyond the f16 range (ggml dequantizes Q8_0 to
                // fp32: it stays finite there) flags the call for the fp32
                // fallback
                inf |= (w[u][e] & 0x7c00u) == 0x7c00u || (w[u][e] & 0x7c000000u) == 0x7c000000u;
            }
        }
        if (inf && ovf) *ovf = epoch;
    } else {
        // 16-byte loads where the view's rows allow them, else 4-byte ones
        const bool al16 = (((uintptr_t)base | (uintptr_t)nb_tok | (uintptr_t)nb_head) & 15) == 0;
        float4 f[kWinPasses][2];
#pragma unroll
        for (int u = 0; u < kWinPasses; ++u) {
            const int64_t i4 = min(i0 + u * stride, n4 - 1);
            int q;
            const char* src = src_of(i4, q) + q * 32;
            if (al16) {
                f[u][0] = ((const float4*)src)[0];
                f[u][1] = ((const float4*)src)[1];
            } else {
                const float* x = (const float*)src;
                f[u][0] = make_float4(x[0], x[1], x[2], x[3]);
                f[u][1] = make_float4(x[4], x[5], x[6], x[7]);
            }
        }
#pragma unroll
        for (int u = 0; u < kWinPasses; ++u) {
            w[u][0] = (uint32_t)f32_to_f16(f[u][0].x) | ((uint32_t)f32_to_f16(f[u][0].y) << 16);
            w[u][1] = (uint32_t)f32_to_f16(f[u][0].z) | ((uint32_t)f32_to_f16(f[u][0].w) << 16);
            w[u][2] = (uint32_t)f32_to_f16(f[u][1].x) | ((uint32_t)f32_to_f16(f[u][1].y) << 16);
            w[u][3] = (uint32_t)f32_to_f16(f[u][1].z) | ((uint32_t)f32_to_f16(f[u][1].w) << 16);
        }
    }
#pragma unroll
    for (int u = 0; u < kWinPasses; ++u) {
        const int64_t i4 = i0 + u * stride;
        if (i4 < n4) *(uint4*)(obase + i4 * 8) = make_uint4(w[u][0], w[u][1], w[u][2], w[u][3]);
    }
}

// Q8_0 windows whose rows are contiguous ([row][kv head][block], no gaps):
// the window is one run of blocks.  A workgroup takes kWinBlocks of them:
// their bytes come in as consecutive dwords (one coalesced 4-byte load per
// thread and pass) into LDS, then each thread converts quarters t and
// t + 256 (8 values each, one 16-byte store, so a wave writes 1 KB
// contiguously).  Grid (blocks of the longest window / kWinBlocks, 2 B).
constexpr int kWinBlocks = 128;
constexpr int kWinDwords = kWinBlocks * kQ8Bytes / 4;                 // 1088

__global__ void __launch_bounds__(256) window_q8_flat_kernel(AttnArgs a, uint16_t* __restrict__ dst,
                                                             unsigned long long* ovf, unsigned long long epoch) {
    prefetch_kernargs<sizeof(AttnArgs)>();
    __shared__ uint32_t buf[kWinDwords + 4];
    const int b = blockIdx.y >> 1, which = blockIdx.y & 1;
    const int L = a.L[b];
    const int64_t nblk = (int64_t)L * a.Hkv * (a.d / 32);             // blocks of the window
    const int64_t blk0 = (int64_t)blockIdx.x * kWinBlocks;
    if (blk0 >= nblk) return;
    const char* base = which ? a.v[b] : a.k[b];
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(base + blk0 * kQ8Bytes), (short)0,
        (int)((min(nblk - blk0, (int64_t)kWinBlocks) * kQ8Bytes + 3) & ~3), 0x00020000);   // (whole dwords)
    for (int i = threadIdx.x; i < kWinDwords; i += 256) buf[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, 4 * i, 0, 0);
    if (threadIdx.x < 4) buf[kWinDwords + threadIdx.x] = 0u;
    __syncthreads();
    size_t off = 0;                                                   // this sequence's K, then V
    for (int b2 = 0; b2 < b; ++b2) off += (size_t)2 * a.L[b2] * a.Hkv * a.d;
    uint4* const o = (uint4*)(dst + off + (size_t)which * L * a.Hkv * a.d + blk0 * 32);
    const char* rb = (const char*)buf;
    const int nq = (int)min((nblk - blk0) * 4, (int64_t)kWinBlocks * 4);
    bool inf = false;
    for (int t = threadIdx.x; t < nq; t += 256) {
        const int k = t >> 2, q = t & 3;
        const int sb = k * kQ8Bytes;                                  // even
        const float d = f16_to_f32(*(const uint16_t*)(rb + sb));
        // codes 8 q .. 8 q + 7: bytes sb + 2 + 8 q .., from the dword at or below
        const int cb = sb + 2 + 8 * q;
        const uint32_t* w = (const uint32_t*)(rb + (cb & ~3));
        const uint32_t w0 = w[0], w1 = w[1], w2 = w[2];
        const bool mis = cb & 2;
        const uint32_t c0 = mis ? __builtin_amdgcn_alignbyte(w1, w0, 2) : w0;
        const uint32_t c1 = mis ? __builtin_amdgcn_alignbyte(w2, w1, 2) : w1;
        uint32_t r[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t c = e < 2 ? c0 : c1, sh = 16 * (e & 1);
            r[e] = (uint32_t)f32_to_f16(d * (float)(int8_t)(c >> sh)) |
                   ((uint32_t)f32_to_f16(d * (float)(int8_t)(c >> (sh + 8))) << 16);
            inf |= (r[e] & 0x7c00u) == 0x7c00u || (r[e] & 0x7c000000u) == 0x7c000000u;
        }
        o[t] = make_uint4(r[0], r[1], r[2], r[3]);
    }
    // a value beyond the f16 range flags the call for the fp32 fallback
    if (inf && ovf) *ovf = epoch;
}

}  // namespace

size_t window_f16_bytes(const AttnArgs& a) {
    size_t n = 0;
    for (int b = 0; b < a.B; ++b) n += (size_t)2 * a.L[b] * a.Hkv * a.d * 2;
    return (n + 255) / 256 * 256;
}

hipError_t launch_window_to_f16(const AttnArgs& a, void* dst, unsigned long long* ovf, unsigned long long epoch,
                                hipStream_t s) {
    int Lmax = 1;
    for (int b = 0; b < a.B; ++b) Lmax = max(Lmax, a.L[b]);
    // contiguous 4-byte aligned Q8_0 rows: the flat run of blocks
    bool flat = a.k_type == VVA_TYPE_Q8_0 && a.v_type == VVA_TYPE_Q8_0;
    const int64_t hb = (int64_t)(a.d / 32) * kQ8Bytes;
    flat = flat && a.k_nb_head == hb && a.v_nb_head == hb && a.k_nb_tok == a.Hkv * hb && a.v_nb_tok == a.Hkv * hb;
    for (int b = 0; b < a.B; ++b) flat = flat && (uintptr_t)a.k[b] % 4 == 0 && (uintptr_t)a.v[b] % 4 == 0;
    if (flat) {
        const int64_t nb = (int64_t)Lmax * a.Hkv * (a.d / 32);
        hipLaunchKernelGGL(window_q8_flat_kernel, dim3((unsigned)((nb + kWinBlocks - 1) / kWinBlocks), 2 * a.B),
                           dim3(256), 0, s, a, (uint16_t*)dst, ovf, epoch);
        return hipGetLastError();
    }
    const int64_t n = (int64_t)Lmax * a.Hkv * (a.d / 32) * 4;
    const int64_t per = 256 * kWinPasses;
    hipLaunchKernelGGL(window_to_f16_kernel, dim3((unsigned)((n + per - 1) / per), 2 * a.B), dim3(256), 0, s, a,
                       (uint16_t*)dst, ovf, epoch);
    return hipGetLastError();
}

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
    if (a.mask_mode == kMaskExplicit && (a.mask_nb_row % (a.mask_f32 ? 4 : 2) || a.mask_nb_b % (a.mask_f32 ? 4 : 2))) return false;
    return true;
}

// Split plan.  The candidates split the key tiles of the row tiles rt >= R
// n ways (R = 0: every row tile; or the smallest R that keeps the whole
// grid in one round on the CUs).  Each is scored by replaying the
// hardware's dispatch: workgroups go out in launch order (heaviest row tile
// first, kv heads innermost), each to the CU that frees first, costing its
// key tiles plus a fixed prologue (Q rows loaded, the first tiles staged);
// a split plan adds its merge: in the launch (up to kMaxInLaunchSplits
// splits), the last split's epilogue (partial stores completed, ticket, the
// other partials loaded: ~4.7 us at two splits, ~1.5 us more per further
// split, measured at the 1.5B and 7B shapes); otherwise the merge kernel's
// launch and its exposed traffic.  Causal
// row tiles differ in length, so a plan with more, smaller pieces over
// several rounds can finish sooner than one round of equal-count splits.
// Calls with many more row tiles than CUs balance unsplit.
PrefillPlan prefill_plan(const AttnArgs& a, int n_cu, int forced, size_t ws_cap, bool allow_in_launch) {
    const int n_rt = (a.T * (a.Hq / a.Hkv) + kRowsWG - 1) / kRowsWG;
    const bool causal = a.mask_mode == kMaskCausal;
    auto with_merge = [&](PrefillPlan p) {
        p.in_launch = allow_in_launch && prefill_in_launch_ok(a, p);
        return p;
    };
    if (forced > 0) return with_merge(PrefillPlan{forced, 0, forced, forced, 0});
    const PrefillPlan none{1, 0, 0, 1, 0};
    const int per = a.Hkv * a.B;                 // workgroups per piece index
    const int budget = n_cu / per;               // pieces per (kv head, sequence) in one round
    if (n_rt >= 4 * budget) return none;
    // time in key-tile units (one tile of 64 keys x 256 rows for one workgroup)
    const double unit_us = 64.0 * kRowsWG * a.d * 4.0 / 4.0e6;
    const double bytes_per_unit = 5.0e6 * unit_us;   // 5 TB/s
    const double merge_launch = 5.0 / unit_us;
    const double prologue = 3.0;                 // ~6 us per workgroup, measured at the 7B shape
    // cost of piece x of sequence b under plan p (key tiles + prologue)
    auto piece_cost = [&](const PrefillPlan& p, int b, int x) {
        const int nh = p.forced > 0 ? p.forced : p.n, R = p.forced > 0 ? 0 : p.R;
        const int heavy = (n_rt - R) * nh;
        const int rt = x < heavy ? n_rt - 1 - x / nh : R - 1 - (x - heavy);
        const int ks = x < heavy ? x % nh : 0, n_ks = x < heavy ? nh : 1;
        const int n_all = rt_key_tiles(a, b, rt, causal);
        return (double)((int64_t)(ks + 1) * n_all / n_ks - (int64_t)ks * n_all / n_ks) + prologue;
    };
    // finish time of plan p: the kv heads of one piece index cost the same,
    // so the CUs are taken in groups of Hkv; pieces go out in the kernel's
    // order (sequence-major, heaviest row tile first) to the group that frees
    // first.  One round (every piece has a group): the largest piece.
    // (fixed storage: the planner allocates nothing, for vva_attn_noalloc too;
    // beyond kPlanMaxGroups groups the replay models that many)
    constexpr int kPlanMaxGroups = 1024;
    const int groups = min(max(1, n_cu / a.Hkv), kPlanMaxGroups);
    double cu[kPlanMaxGroups];
    auto makespan = [&](const PrefillPlan& p) {
        const int pieces = plan_pieces(p, n_rt);
        double m = 0.0;
        if ((int64_t)pieces * a.B <= groups) {
            for (int b = 0; b < a.B; ++b)
                for (int x = 0; x < pieces; ++x) m = max(m, piece_cost(p, b, x));
            return m;
        }
        std::fill(cu, cu + groups, 0.0);
        for (int b = 0; b < a.B; ++b)
            for (int x = 0; x < pieces; ++x) {
                std::pop_heap(cu, cu + groups, std::greater<double>());
                cu[groups - 1] += piece_cost(p, b, x);
                std::push_heap(cu, cu + groups, std::greater<double>());
            }
        for (int i = 0; i < groups; ++i) m = max(m, cu[i]);
        return m;
    };
    PrefillPlan best = none;
    double best_t = makespan(none);
    for (int n = 2; n <= kMaxKeySplits; ++n) {
        // the smallest R with (n_rt - R) n + R <= budget (one round), and for
        // a few split counts R = 0 (every row tile split, several rounds)
        const int R_fit = max(0, (n_rt * n - budget + n - 2) / (n - 1));
        for (int R : {R_fit, 0}) {
            if (R >= n_rt || (R == 0 && R_fit > 0 && n > 8)) continue;
            const PrefillPlan p = with_merge(PrefillPlan{n, R, 0, n, 0});
            if (prefill_ws_bytes(a, p) > ws_cap) continue;
            const double split_rows = (double)(n_rt - R) * kRowsWG * per;
            // merge kernel: the partials are written while other workgroups
            // compute; its reads of the n partials and its output write are not
            // hidden
            const double merge = p.in_launch ? (4.7 + 1.5 * (n - 2)) / unit_us
                                             : merge_launch + split_rows * (n + 1) * (a.d + 2) * 4.0 / bytes_per_unit;
            const double t = makespan(p) + merge;
            if (t < best_t * 0.95) {             // a split must pay for itself
                best_t = t;
                best = p;
            }
            if (R_fit == 0) break;
        }
    }
    return best;
}

size_t prefill_ws_bytes(const AttnArgs& a, const PrefillPlan& p) {
    if (p.max_ks <= 1) return 0;
    if (!p.in_launch) return (size_t)p.max_ks * a.B * a.T * a.Hq * (a.d + 2) * sizeof(float);
    // the in-launch layout: one block of kRowsWG rows x (d + 4) floats per piece
    const int n_rt = (a.T * (a.Hq / a.Hkv) + kRowsWG - 1) / kRowsWG;
    return (size_t)p.max_ks * a.B * a.Hkv * n_rt * kRowsWG * (a.d + 4) * sizeof(float);
}

bool prefill_in_launch_ok(const AttnArgs& a, const PrefillPlan& p) {
    const int n_rt = (a.T * (a.Hq / a.Hkv) + kRowsWG - 1) / kRowsWG;
    return p.max_ks > 1 && p.max_ks <= kMaxInLaunchSplits && (int64_t)a.B * a.Hkv * n_rt <= kMaxPrefillTickets;
}

hipError_t launch_prefill(const AttnArgs& a, float* ws, unsigned* tickets, const PrefillPlan& p, hipStream_t s) {
    if (p.in_launch && (!tickets || !prefill_in_launch_ok(a, p))) return hipErrorInvalidValue;
    if (a.d == 64) {
        return a.k_type == VVA_TYPE_F16 ? launch_pf<64, VVA_TYPE_F16>(a, ws, tickets, p, s)
                                        : launch_pf<64, VVA_TYPE_BF16>(a, ws, tickets, p, s);
    }
    return a.k_type == VVA_TYPE_F16 ? launch_pf<128, VVA_TYPE_F16>(a, ws, tickets, p, s)
                                    : launch_pf<128, VVA_TYPE_BF16>(a, ws, tickets, p, s);
}

}  // namespace vva
