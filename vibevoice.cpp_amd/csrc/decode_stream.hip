// decode_stream.hip — split-K single-token attention (T == 1) over a dense
// Q8_0 KV cache: the per-step attention of the ASR / TTS decode loops
// (src/vibevoice_asr.cpp:760-800, src/vibevoice_tts.cpp:862-880), i.e.
// ggml_flash_attn_ext with one query row per head (src/qwen2.cpp:332-334)
// on Q8_0 K/V.
//
// Streaming.  Every workgroup (4 compute waves, one per SIMD, and 3 producer
// waves; one workgroup per CU) takes every n_splits-th whole tile of one
// sequence (split s: tiles s, s + n_splits, ...) plus an equal piece of the
// keys past the last whole round, and streams them through a 4-stage LDS
// ring filled by buffer_load_dwordx4 ... lds (non-temporal: the cache is read
// once), so two tiles (70 KB per CU) are on their way from HBM while one is
// computed.  A tile is 512 (key, kv head, 32-dim block) rows of the cache =
// 17,408 B of K plus the same of V (256 rows at d = 64), read as the cache lays them out
// ([token][kv head][34-byte GGUF block]): one contiguous byte range per
// operand, 1 KB per wave instruction.  The buffer ranges end at the
// sequence's last key, so chunks past it come back as zeros without a
// memory access.
//
// Arithmetic on the matrix cores.  With g <= 8 query heads per kv head, a
// 16 x 16 MFMA tile with one kv head's query rows would leave half its
// columns idle; instead each wave packs two slots into the 16 columns:
// rows 0-7 are the query heads of kv head 2p and rows 8-15 those of kv head
// 2p + 1 (or, with one kv head, the same heads over a second group of 16
// keys), over the same 16 keys.  Lane = (g = lane / 16, n = lane % 16).
// MFMA row m of a group stands for its key sigma(m) = 4 (m % 4) + m / 4, so
// lane group g works on keys g, g + 4, g + 8, g + 12: with the cache's
// 544-byte token rows the four groups' LDS reads then fall in different
// banks.
//   scores  S^T[key][row] per 32-dim Q8_0 block with two
//           v_mfma_i32_16x16x32_i8, block-diagonal over k: in the MFMA for
//           dims 16j .. 16j + 15, k 0-15 carry slot 0's K codes and slot
//           0's Q codes (zero in slot 1's columns), k 16-31 slot 1's.  Each
//           block's dot is ggml's exact integer Q8_0 x Q8_0 block sum; the
//           lane receives keys sigma(4g + i) of its row n and scales them by
//           d_k * d_q in fp32.
//   softmax fp32, exp2 domain, one row per lane (max over the row's 16 keys:
//           in-lane, then two permlane swaps).  The running max is raised
//           only when a score exceeds it by 2^8.
//   P.V     O^T[dim][row] += V^T P'^T with v_mfma_f32_16x16x16_f16 per 16
//           dims and slot: A = that slot's V codes (exact in f16; lane: dims
//           2n, 2n+1 of block b, keys sigma(4g + i)), B = P' = p * d_v(key,
//           b) as f16 — the score accumulator layout is already B's layout,
//           so P never leaves the registers.  Each slot's MFMA is right for
//           its own 8 columns; a lane keeps the accumulator of its slot.
// A tile's P.V runs one tile late, beside the next tile's scores (its V
// codes wait in registers), so the two dependency chains overlap.
// The workgroup's records merge through LDS (log-sum-exp) into one row per
// query head; the workgroup writes (m, l, acc[d]) per query head, or the
// output when there is one split, and decode_merge_kernel (decode.hip)
// combines the splits.
//
// Step mode (STEP; vva_decode_step on Q8_0 caches, the ASR decode loop of
// src/vibevoice_asr.cpp:760-800 with src/qwen2.cpp:282-306 fused in): q
// arrives raw and is RoPE'd while it is quantized (split 0 writes q_out),
// and the split that holds key len(seq_b) computes the new row itself
// (RoPE(k), v, both quantized to Q8_0 blocks exactly as rope_append.hip
// does), writes it to the cache and copies it into its own tile once that
// tile has landed; its DMA copy of the row, older or newer, is overwritten.
#include "vva_internal.hpp"

#include <type_traits>

namespace vva {

namespace {

#include "wave_ops.hpp"

typedef __attribute__((address_space(3))) char lds_char;
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kW = 4;                        // compute waves per workgroup (one per SIMD)
constexpr int kP = 3;                        // producer waves: they only issue the tile loads and wait
constexpr int kStages = 4;                   // LDS ring depth (power of 2)
constexpr int kTileOpBytes = 17408;          // one operand of a tile: 512 Q8_0 blocks (d = 128; 256 at d = 64)
constexpr int kOpChunks = 18;                // 1 KB chunks per operand: 17 KB + alignment slack
constexpr int kOpBytes = kOpChunks * 1024;
constexpr int kStage = 2 * kOpBytes;         // K, then V
constexpr int kLdsBytes = kStages * kStage;
constexpr int kOpLoads = kOpChunks / kP;     // DMA loads per producer, operand and tile
constexpr int kLoads = 2 * kOpLoads;         // DMA loads per producer per tile
constexpr int kQLoads = 8;                   // DMA loads per producer for the raw Q rows
constexpr int kQRawBytes = kQLoads * kP * 1024;   // raw Q area: up to 24 KB
static_assert(kOpChunks % kP == 0, "chunks split evenly over the producers");
static_assert(kQLoads + 2 * kLoads <= 63, "Q and two tiles of a producer's loads fit its 6-bit vmcnt");
constexpr int kDead = 0x40000000;            // buffer offset past every range
constexpr float kLazy = 8.0f;                // running-max slack in log2 units: p <= 256
constexpr int kStepLds = 2048;               // step mode: angle table + the new K / V rows
static_assert(kLdsBytes + kStepLds <= 160 * 1024, "LDS budget");

// buffer_load_dwordx4 ... lds: each lane's 16 bytes land at LDS address
// m0 + 16 * lane.  Inline asm, so the compiler neither fences LDS reads on it
// nor waits for it; completion is awaited explicitly (wait_vm_barrier, whose
// memory clobber is what orders LDS reads after the data lands).  No memory
// clobber here: a load writes a stage nobody reads until a later barrier, so
// the compiler may move the current tile's LDS reads across it.  The whole
// offset is in the VGPR (soffset 0), so the range check sees all of it.
// STREAM marks the load non-temporal: the cache is read once, so its lines
// should not displace what the next call reads again (Q, the partials).
template <bool STREAM = false>
__device__ __forceinline__ void dma16(i32x4 rsrc, uint32_t lds_addr, int voffset) {
    if constexpr (STREAM)
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 4\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds"
                     :
                     : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voffset), "s"(rsrc)
                     : "m0");
    else
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 4\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                     :
                     : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voffset), "s"(rsrc)
                     : "m0");
}

// wait until at most N of this wave's loads are outstanding (and its LDS
// operations are done), then meet the workgroup at a barrier
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(N) : "memory");
}

// meet the workgroup at a barrier once this wave's LDS operations are done
// (its memory loads, if any, stay in flight)
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory");
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
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u16x2 as_u16x2(uint32_t w) {
    u16x2 v;
    __builtin_memcpy(&v, &w, 4);
    return v;
}

// D: head dim (64 / 128); HKV: kv heads of the workgroup's tile (1, 2, 4,
// 8), which fixes the row pitch in LDS, so every LDS offset inside a tile is
// a constant; NHG: head groups of the cache row (the cache holds HKV * NHG kv
// heads per token).  With NHG > 1 workgroup (split, b * NHG + group) gathers
// its group's slice of every cache row (RB bytes, a multiple of 16, at
// group * RB in a row of NHG * RB bytes): the split partials then cover HKV
// kv heads over NHG times the keys, NHG times fewer of them.
template <int D, int HKV, int NHG, bool STEP>
__global__ void __launch_bounds__((kW + kP) * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
decode_stream_kernel(AttnArgs a, float* __restrict__ ws, int n_splits, StreamStep st) {
    prefetch_kernargs<sizeof(AttnArgs) + 16 + (STEP ? sizeof(StreamStep) : 0)>();
    constexpr int NB = D / 32;                // Q8_0 blocks per head row
    constexpr int HB = NB * kQ8Bytes;         // bytes per head row
    constexpr int RB = HKV * HB;              // bytes per token row in LDS (the group's kv heads)
    constexpr int RBM = NHG * RB;             // bytes per token row in the cache
    static_assert(NHG == 1 || RB % 16 == 0, "16-byte pieces of a row slice");
    // d = 64 tiles hold half the bytes, so that every wave takes one slot
    // pair per tile at both head dims (two pairs at d = 64 would need more
    // than the 256 VGPRs of a wave)
    constexpr int TB = D == 64 ? kTileOpBytes / 2 : kTileOpBytes;   // bytes per operand and tile
    constexpr int OPL = D == 64 ? kOpLoads / 2 : kOpLoads;          // DMA loads per producer, operand and tile
    constexpr int LD = 2 * OPL;                                     // DMA loads per producer per tile
    static_assert(OPL * kP * 1024 >= TB + 16, "a tile's chunks cover it at any 16-byte delta");
    constexpr int TT = TB / RB;               // keys per tile
    constexpr int NPAIR = TT * HKV / 32;      // slot pairs (2 slots of 16 keys x 1 kv head) per tile
    constexpr int NSUB = NPAIR / kW;          // slot pairs per wave per tile
    constexpr int HP = HKV >= 2 ? HKV / 2 : 1;    // kv head pairs
    constexpr int NJ = 2 * NB;                // P.V MFMAs (16 dims each) per slot
    static_assert(TT * RB == TB && NSUB * kW == NPAIR && NSUB >= 1, "tile size");
    static_assert(kW % HP == 0, "a wave keeps its head pair across its slot pairs");

    // step mode: the RoPE angle table and the new K and V rows after the ring
    __shared__ __attribute__((aligned(16))) char lds[kLdsBytes + (STEP ? kStepLds : 0)];

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, n = lane & 15;
    const int G = a.Hq / (HKV * NHG);         // query heads per kv head (<= 8)
    const int HQL = HKV * G;                  // the workgroup's query heads
    // The wave's two slots: kv heads 2 hp and 2 hp + 1 over the same 16 keys,
    // or (HKV = 1) the one kv head over two consecutive groups of 16 keys.
    // Column n of the MFMAs is query row n & 7 of slot n >> 3.
    const int hp = w % HP;
    auto slot_head = [&](int s) { return HKV >= 2 ? 2 * hp + s : 0; };
    constexpr int SK = HKV >= 2 ? 0 : 16;     // key offset of slot 1 from slot 0
    // first key of slot 0 of the wave's slot pair u in a tile
    auto pair_key = [&](int u) {
        const int p = w + kW * u;
        return HKV >= 2 ? 16 * (p / HP) : 32 * p;
    };
    const int sr = n >> 3, rr = n & 7;        // the lane's slot and query row in it
    const bool rvalid = rr < G;
    const int hq_row = slot_head(sr) * G + rr;
    const int split = blockIdx.x, b = blockIdx.y / NHG, hgrp = blockIdx.y % NHG;
    const int hq0 = hgrp * HQL;               // first query head of the group
    const int L = a.L[b];
    // Keys are dealt so that every split streams the same bytes (within one
    // key).  The first RF = n_rounds * n_splits * TT keys are whole tiles
    // dealt round-robin: the split's tile 1 + f is tile split + f * n_splits
    // of the sequence, so at any moment the workgroups of a sequence stream
    // neighbouring tiles of the cache (measured 4 % faster than a contiguous
    // key range per split).  The remaining keys (fewer than n_splits tiles'
    // worth) are cut into n_splits nearly equal pieces: the split's piece
    // (possibly empty) is its tile 0, computed while its first whole tiles are
    // still on their way, so no split streams an extra tile at the end.
    const int span_keys = TT * n_splits;
    const int n_rounds = L / span_keys;
    const int RF = n_rounds * span_keys;
    const int p_begin = RF + (int)(((int64_t)(L - RF) * split) / n_splits);
    const int p_end = RF + (int)(((int64_t)(L - RF) * (split + 1)) / n_splits);
    const int n_tiles = 1 + n_rounds;
    // first key of tile t
    auto tile_key = [&](int t) { return t == 0 ? p_begin : (split + (t - 1) * n_splits) * TT; };
    // step mode: the split holding key L - 1 (the new row) is the last one:
    // the key ends its piece, or (no remainder) its last whole tile
    const bool owns_new = STEP && split == n_splits - 1 && L > 0;
    const int new_t = owns_new ? (p_end > p_begin ? 0 : n_tiles - 1) : -1;
    float* const rope_cs = (float*)(lds + kLdsBytes);                  // [D / 2]
    float* const rope_sn = rope_cs + D / 2;
    char* const new_rows = (char*)(rope_sn + D / 2);                   // K slice, then V slice (RB each)

    // Two raw buffers per operand, both from the 16-byte boundary at or
    // below the sequence's row 0: the whole tiles' ends at row RF - 1, the
    // piece's at row p_end - 1, so a piece's 17 KB load fetches its own rows
    // only.  delta = row 0's offset from that boundary (a multiple of 4),
    // also a tile's offset in its LDS stage (a tile at key j starts j * RBM
    // bytes into the buffer).  (NHG > 1: the cache rows are 16-byte aligned,
    // delta = 0)
    const char* kfirst = a.k[b];
    const char* vfirst = a.v[b];
    const int dk = (int)((uintptr_t)kfirst & 15), dv = (int)((uintptr_t)vfirst & 15);
    const uint32_t span = (uint32_t)RF * (uint32_t)RBM, pspan = (uint32_t)p_end * (uint32_t)RBM;
    const i32x4 krs = make_rsrc_sgpr(kfirst - dk, dk + span);
    const i32x4 vrs = make_rsrc_sgpr(vfirst - dv, dv + span);
    const i32x4 kprs = make_rsrc_sgpr(kfirst - dk, dk + pspan);
    const i32x4 vprs = make_rsrc_sgpr(vfirst - dv, dv + pspan);
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_char*)lds;

    // ---- Loads.  Only the kP producer waves (w >= kW) issue memory loads:
    // a load instruction stalls its wave while the CU's queue of outstanding
    // loads is full, and a compute wave stalled there leaves the matrix and
    // vector units idle and the queue unrefilled while it computes.  The
    // producers meet the compute waves at every barrier: A (raw Q landed),
    // B (Q quantized), one per tile t (tile t landed, every compute wave done
    // with tile t - 1, so the stage of tile t - 2 takes tile t + 2), then the
    // two barriers of the epilogue.
    // A tile of an operand is TB bytes of its buffer from the tile's first
    // key on (17,408 B, or 8,704 B at d = 64), loaded as 1 KB chunks, chunk c
    // by producer c % kP; the chunk holding the 16-byte delta's overhang is
    // loaded only when delta > 0.  A tile past the last one loads nothing
    // but zeros (offsets past the range: no memory access).
    const int eb = (int)type_elem_bytes(a.q_type);
    if (w >= kW) {
        const int pw = w - kW;
        // Byte offset, in the split's buffer, of this lane's 16 bytes of chunk
        // c of tile 0: the tile is contiguous in the cache (NHG = 1), or the
        // group's RB-byte slice of each of its rows (NHG > 1).  Tile t is
        // t * TT rows on.
        int loff[OPL];
#pragma unroll
        for (int i = 0; i < OPL; ++i) {
            const int bt = (pw + kP * i) * 1024 + lane * 16;
            loff[i] = NHG == 1 ? bt : (bt / RB) * RBM + hgrp * RB + bt % RB;
        }
        auto issue = [&](int t) {
            const bool live = t < n_tiles;
            const uint32_t st = lds0 + (uint32_t)(t & (kStages - 1)) * kStage;
            const int tb = tile_key(t) * RBM;
            const bool pc = t == 0;                  // wave-uniform
            const i32x4 ks = pc ? kprs : krs, vs = pc ? vprs : vrs;
#pragma unroll
            for (int op = 0; op < 2; ++op)
#pragma unroll
                for (int i = 0; i < OPL; ++i) {
                    const int c = pw + kP * i;
                    const bool need = live && c * 1024 < TB + (op ? dv : dk);
                    dma16<true>(op ? vs : ks, st + op * kOpBytes + c * 1024, need ? tb + loff[i] : kDead);
                }
        };
        // Q's rows (contiguous, at most 24 KB) go to the ring's last stage,
        // which takes no tile before barrier T_1 (its quantized codes are in
        // registers from barrier B on)
        {
            const i32x4 qrs = make_rsrc_sgpr(a.q + b * a.q_nb_b + (int64_t)hq0 * D * eb, (uint32_t)(HQL * D * eb));
#pragma unroll
            for (int i = 0; i < kQLoads; ++i) {
                const int c = i * kP + pw;
                dma16(qrs, lds0 + (kStages - 1) * kStage + c * 1024, c * 1024 + lane * 16);
            }
        }
        // Q, tile 0 (the piece) and the first whole tile go out together;
        // from then on tile t + 2 goes out once tile t has landed, so two
        // tiles (70 KB per CU) are on their way while one is computed.  More
        // at once (three tiles, or a second whole tile at the start) measured
        // slower: Q lands later behind them and every tile waits for Q.
        issue(0);
        issue(1);
        wait_vm_barrier<2 * LD>();                   // A: Q landed
        wait_vm_barrier<2 * LD>();                   // B
        for (int t = 0; t < n_tiles; ++t) {
            wait_vm_barrier<LD>();                   // T_t: tile t landed
            if (STEP && t == new_t) lds_barrier();   // N: the new row is in tile t's stage
            issue(t + 2);
        }
        // the padding tiles' loads land before the ring is reused
        asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
        __syncthreads();                             // epilogue: records written
        __syncthreads();                             // epilogue: records read
        return;
    }

    // ---- step mode, while q flies: the raw new k / v pair of this lane
    // (the split holding key L - 1; waves 0, 1: k of the group's kv heads,
    // waves 2, 3: v) and the angle table of the new token's position (the
    // fp32 theta recurrence of rope_append.hip)
    float nx0 = 0.0f, nx1 = 0.0f;
    if constexpr (STEP) {
        constexpr int P = D / 2;
        const int kind = w >> 1, hh = w & 1;
        if (owns_new && hh < HKV) {                  // wave-uniform
            const int head = hgrp * HKV + hh;
            const int typ = kind ? st.v_type : st.k_type;
            const int64_t es = type_elem_bytes(typ);
            const char* src = (kind ? st.v + b * st.v_nb_b + head * st.v_nb_h : st.k + b * st.k_nb_b + head * st.k_nb_h);
            const int ii = lane < P ? lane : 0;
            nx0 = load_elem(src + ii * es, typ);
            nx1 = load_elem(src + (ii + P) * es, typ);
        }
        if (threadIdx.x < D / 2) {
            const int i = threadIdx.x;
            const float th = rope_theta((float)st.pos[b * st.pos_stride_b], st.theta_scale, i, D / 2);
            rope_cs[i] = cosf(th);
            rope_sn[i] = sinf(th);
        }
    }

    // ---- Q is quantized to Q8_0 blocks (codes + fp16-rounded scale) next
    // to the raw rows.  Four adjacent lanes share a block (8 values each; the
    // block max over the quad by DPP); a thread takes every (kW * 64)-th
    // quarter block.
    lds_barrier();                                   // A

    const char* qraw = lds + (kStages - 1) * kStage;
    uint32_t* qlds = (uint32_t*)(lds + (kStages - 1) * kStage + kQRawBytes);
    constexpr int QI = 1024 / (kW * 64);              // quarters per thread (Hq * NB <= 256)
    const int nqi = HQL * NB * 4;
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
        if constexpr (STEP) {
            // RoPE (pairs i, i + D / 2 of the head row; the partners of this
            // quarter block's 8 dims sit D / 2 further or nearer in qraw),
            // rounded to q_out's type as the unfused path stores it; split 0
            // writes q_out
            constexpr int P = D / 2;
            const int hr = (tt >> 2) / NB, dim0 = ((tt >> 2) % NB) * 32 + (tt & 3) * 8;
            const bool lo = dim0 < P;
            const char* prow = qraw + (int64_t)((tt >> 2) * 32 + (tt & 3) * 8 + (lo ? P : -P)) * eb;
            float xp[8];
            if (a.q_type == VVA_TYPE_F32) {
                const uint4 u0 = ((const uint4*)prow)[0], u1 = ((const uint4*)prow)[1];
                xp[0] = __uint_as_float(u0.x); xp[1] = __uint_as_float(u0.y);
                xp[2] = __uint_as_float(u0.z); xp[3] = __uint_as_float(u0.w);
                xp[4] = __uint_as_float(u1.x); xp[5] = __uint_as_float(u1.y);
                xp[6] = __uint_as_float(u1.z); xp[7] = __uint_as_float(u1.w);
            } else {
                const bool bf = a.q_type == VVA_TYPE_BF16;
                const uint4 u0 = ((const uint4*)prow)[0];
                const uint32_t wv[4] = {u0.x, u0.y, u0.z, u0.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint16_t l16 = (uint16_t)(wv[e] & 0xffffu), h16 = (uint16_t)(wv[e] >> 16);
                    xp[2 * e] = bf ? bf16_to_f32(l16) : f16_to_f32(l16);
                    xp[2 * e + 1] = bf ? bf16_to_f32(h16) : f16_to_f32(h16);
                }
            }
            const float4 c0 = *(const float4*)(rope_cs + (dim0 & (P - 1))), c1 = *(const float4*)(rope_cs + (dim0 & (P - 1)) + 4);
            const float4 s0 = *(const float4*)(rope_sn + (dim0 & (P - 1))), s1 = *(const float4*)(rope_sn + (dim0 & (P - 1)) + 4);
            const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
            const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
            float y[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) y[e] = lo ? fmaf(x[e], cv[e], -(xp[e] * sv[e])) : fmaf(xp[e], sv[e], x[e] * cv[e]);
            // rounded to q_out's type, as the unfused path reads it back; split
            // 0 writes q_out
            const int qot = st.q_out_type;
            const bool wq = split == 0 && t < nqi;
            char* qo = st.q_out + b * st.qo_nb_b + (int64_t)(hq0 + hr) * st.qo_nb_h;
            if (qot == VVA_TYPE_F32) {
#pragma unroll
                for (int e = 0; e < 8; ++e) x[e] = y[e];
                if (wq) {
                    ((float4*)(qo + dim0 * 4))[0] = make_float4(y[0], y[1], y[2], y[3]);
                    ((float4*)(qo + dim0 * 4))[1] = make_float4(y[4], y[5], y[6], y[7]);
                }
            } else {
                const bool bf = qot == VVA_TYPE_BF16;
                uint32_t hw[4];
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    const uint16_t h0 = bf ? f32_to_bf16(y[e]) : f32_to_f16(y[e]);
                    const uint16_t h1 = bf ? f32_to_bf16(y[e + 1]) : f32_to_f16(y[e + 1]);
                    x[e] = bf ? bf16_to_f32(h0) : f16_to_f32(h0);
                    x[e + 1] = bf ? bf16_to_f32(h1) : f16_to_f32(h1);
                    hw[e / 2] = (uint32_t)h0 | ((uint32_t)h1 << 16);
                }
                if (wq) *(uint4*)(qo + dim0 * 2) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
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
    lds_barrier();                                   // B

    // ---- step mode, the split holding key L - 1 (after Q is quantized: its
    // raw k/v rows land late, ~3 us into the launch, and the row is needed
    // only from tile new_t on): the new K row (waves 0,
    // 1: RoPE'd) and V row (waves 2, 3) of the group's kv heads, one
    // rotation pair (i, i + D / 2) per lane, quantized per 32-dim block
    // (block max over a half-wave) like rope_append.hip's Q8_0 append; to the
    // cache row and to new_rows
    if constexpr (STEP) {
        const int kind = w >> 1, hh = w & 1, i = lane;
        if (owns_new && hh < HKV) {                  // wave-uniform
            constexpr int P = D / 2;
            const int head = hgrp * HKV + hh;
            const int ii = i < P ? i : 0;
            const float x0 = nx0, x1 = nx1;
            float y0 = x0, y1 = x1;
            if (kind == 0) {
                const float c = rope_cs[ii], sn = rope_sn[ii];
                y0 = fmaf(x0, c, -(x1 * sn));
                y1 = fmaf(x0, sn, x1 * c);
            }
            // block max over the half-wave: DPP within rows, then the row pair
            float a0 = fabsf(y0), a1 = fabsf(y1);
            a0 = fmaxf(a0, dpp<kDppXor1>(a0)); a1 = fmaxf(a1, dpp<kDppXor1>(a1));
            a0 = fmaxf(a0, dpp<kDppXor2>(a0)); a1 = fmaxf(a1, dpp<kDppXor2>(a1));
            a0 = fmaxf(a0, dpp<kDppHalfMirror>(a0)); a1 = fmaxf(a1, dpp<kDppHalfMirror>(a1));
            a0 = fmaxf(a0, dpp<kDppMirror>(a0)); a1 = fmaxf(a1, dpp<kDppMirror>(a1));
            a0 = max_swap16(a0); a1 = max_swap16(a1);
            const float d0 = a0 / 127.0f, d1 = a1 / 127.0f;
            const float id0 = d0 != 0.0f ? 1.0f / d0 : 0.0f;
            const float id1 = d1 != 0.0f ? 1.0f / d1 : 0.0f;
            if (i < P) {
                char* crow = (char*)(kind ? a.v[b] : a.k[b]) + (int64_t)(L - 1) * RBM + (int64_t)head * HB;
                char* lrow = new_rows + kind * RB + hh * HB;
                const int j0 = i, j1 = i + P;
                const char c0 = (char)(int8_t)roundf(y0 * id0), c1 = (char)(int8_t)roundf(y1 * id1);
                if ((j0 & 31) == 0) {
                    const uint16_t h0 = f32_to_f16(d0), h1 = f32_to_f16(d1);
                    *(uint16_t*)(crow + (j0 / 32) * kQ8Bytes) = h0;
                    *(uint16_t*)(crow + (j1 / 32) * kQ8Bytes) = h1;
                    *(uint16_t*)(lrow + (j0 / 32) * kQ8Bytes) = h0;
                    *(uint16_t*)(lrow + (j1 / 32) * kQ8Bytes) = h1;
                }
                crow[(j0 / 32) * kQ8Bytes + 2 + (j0 & 31)] = c0;
                crow[(j1 / 32) * kQ8Bytes + 2 + (j1 & 31)] = c1;
                lrow[(j0 / 32) * kQ8Bytes + 2 + (j0 & 31)] = c0;
                lrow[(j1 / 32) * kQ8Bytes + 2 + (j1 & 31)] = c1;
            }
        }
    }

    // B operands of the score MFMAs, block-diagonal over k: per block and
    // 16-dim half j, lane (g, n) holds codes 16 j + 8 (g & 1) .. + 7 of row
    // n's Q block when its k range (slot g >> 1) is row n's slot, else 0.
    // qd: row n's block scales times scale * log2(e).
    long qb[NB][2];
    float qd[NB];
    {
        const float sl2 = a.scale * kLog2e;          // scores come out in the exp2 domain
        const bool mine = (g >> 1) == sr && rvalid;
        const uint32_t* src = qlds + hq_row * NB * 9;
#pragma unroll
        for (int bb = 0; bb < NB; ++bb) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int wd = bb * 9 + 4 * j + 2 * (g & 1);
                qb[bb][j] = mine ? (long)((uint64_t)src[wd] | ((uint64_t)src[wd + 1] << 32)) : 0;
            }
            qd[bb] = rvalid ? __uint_as_float(src[bb * 9 + 8]) * sl2 : 0.0f;
        }
    }

    float m = -INFINITY, l = 0.0f;            // row n's running max (log2 domain) and sum
    float mb = 0.0f;                          // m, or 0 while m = -inf: the exp2 base
    f32x4 acc[2][NJ];                         // per slot's V: only the lane's own slot is kept
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[s][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // V-range exponent of row n.  P' = p * d_v is an f16 MFMA operand and p
    // <= 2^8, so a V block scale d_v >= 2^8 could overflow it.  Once a tile
    // of the row holds such a block, the row's exp2 base is raised by e
    // beyond its running max (mb = m + e, so p <= 2^(8 - e)) and P' =
    // f16(p * d_v) is formed in fp32, with e = x - 6 for the largest d_v in
    // [2^x, 2^(x+1)) seen so far (P' < 2^15).  The row's record carries m + e
    // as its max, so records on different bases merge exactly.  Caches whose
    // d_v stay below 2^8 (|V| <= 32512) never take this path, so their
    // results are those of the plain f16 P'.
    int vexp = 0;
    bool vscaled = false;                     // wave-uniform: some row of the wave has e > 0
    const char* mrow = a.mask_mode == kMaskExplicit ? a.mask + b * a.mask_nb_b : nullptr;   // query row 0
    // LDS offsets from a slot pair's first key.  Score A operand: key
    // sigma(n) = 4 (n % 4) + n / 4 of slot g >> 1, codes 8 (g & 1) .. of each
    // 16-dim half; the 4-byte word at or below them.
    const int ka_off = (4 * (n & 3) + (n >> 2) + SK * (g >> 1)) * RB + slot_head(g >> 1) * HB + 8 * (g & 1);
    // C layout: keys 4i + g of the lane's own slot (i * 4 RB further)
    const int kc_off = (g + SK * sr) * RB + slot_head(sr) * HB;
    // P.V A operands: V codes of dims 2n, 2n + 1 of keys 4i + g of each slot
    int vc_off[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) vc_off[s] = (g + SK * s) * RB + slot_head(s) * HB + 2 + 2 * n;

    // A slot pair's P.V operands, carried from its scores to the P.V step one
    // tile later: the V codes (in registers, so the stage can be refilled)
    // and P' = p * d_v per block.
    struct PendingPV {
        uint32_t vc[2][4][NB];
        h4 pb[NB];
    };
    // O^T += V^T P'^T per 16 dims, once with each slot's V
    auto pv = [&](const PendingPV& q) {
#pragma unroll
        for (int bb = 0; bb < NB; ++bb)
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                uint32_t c0, c1, c2, c3;
                i8_quad_mfma(q.vc[s][0][bb], q.vc[s][1][bb], q.vc[s][2][bb], q.vc[s][3][bb], c0, c1, c2, c3);
                acc[s][2 * bb] = __builtin_amdgcn_mfma_f32_16x16x16f16(as_h4(c0, c1), q.pb[bb], acc[s][2 * bb], 0, 0, 0);
                acc[s][2 * bb + 1] = __builtin_amdgcn_mfma_f32_16x16x16f16(as_h4(c2, c3), q.pb[bb], acc[s][2 * bb + 1], 0, 0, 0);
            }
    };
    // The LDS operands of one slot pair (2 x 16 keys) starting at tile key
    // kb: the score A operands per block and 16-dim half, the dwords that
    // hold the K and V block scales of the lane's keys 4i + g of its slot,
    // and both slots' V codes of dims 2n, 2n + 1.  Read right after the
    // barrier, before the next tile's loads are issued (an asm volatile the
    // compiler does not move LDS reads across).
    struct PairOps {
        uint32_t aw[NB][2][3];                // A words (the third only for even blocks)
        uint32_t kd[4][NB], vd[4][NB], vc[2][4][NB];
    };
    auto read_pair = [&](const char* kt, const char* vt, int kb, PairOps& o) {
        const char* ka = kt + kb * RB + ka_off;
#pragma unroll
        for (int bb = 0; bb < NB; ++bb)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int off = bb * kQ8Bytes + 2 + 16 * j;      // 2 mod 4 for even blocks
                const uint32_t* p = (const uint32_t*)(ka + (off & ~3));
                o.aw[bb][j][0] = p[0];
                o.aw[bb][j][1] = p[1];
                o.aw[bb][j][2] = (bb & 1) == 0 ? p[2] : 0u;
            }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const char* kr = kt + (kb + 4 * i) * RB + kc_off;
            const char* vr = vt + (kb + 4 * i) * RB + kc_off;
#pragma unroll
            for (int bb = 0; bb < NB; ++bb) {
                const int dw = (bb * kQ8Bytes - (bb & 1) * 2) / 4;
                o.kd[i][bb] = ((const uint32_t*)kr)[dw];
                o.vd[i][bb] = ((const uint32_t*)vr)[dw];
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    o.vc[s][i][bb] = *(const uint16_t*)(vt + (kb + 4 * i) * RB + vc_off[s] + bb * kQ8Bytes);
                    asm("" : "+v"(o.vc[s][i][bb]));     // widened here, next to its load: no masking later
                }
            }
        }
    };
    // Scores of one slot pair (keys kb .. of the tile at key jt) from its
    // operands, with the P.V of the previous tile's pair (prev; zeros before
    // the first tile) in the same instruction stream: the two are
    // independent.  The pair's V codes go to cur.  CHECK: the group may hold
    // keys past the split or the caller passed a mask.
    auto group_scores = [&](const PairOps& o, int kb, int jt, int jend, auto check, const PendingPV& prev,
                            PendingPV& cur, float (&sc)[4]) {
        constexpr bool CHECK = decltype(check)::value;
        pv(prev);
        // ---- scores: per block, two block-diagonal halves into one sum
        i32x4 cs[NB];
#pragma unroll
        for (int bb = 0; bb < NB; ++bb) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                uint32_t lo = o.aw[bb][j][0], hi = o.aw[bb][j][1];
                if ((bb & 1) == 0) {
                    lo = __builtin_amdgcn_alignbyte(o.aw[bb][j][1], o.aw[bb][j][0], 2);
                    hi = __builtin_amdgcn_alignbyte(o.aw[bb][j][2], o.aw[bb][j][1], 2);
                }
                const long av = (long)((uint64_t)lo | ((uint64_t)hi << 32));
                cs[bb] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, qb[bb][j], j == 0 ? i32x4{0, 0, 0, 0} : cs[bb], 0, 0, 0);
            }
        }
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int bb = 0; bb < NB; ++bb) cur.vc[s][i][bb] = o.vc[s][i][bb];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float x = 0.0f;
#pragma unroll
            for (int bb = 0; bb < NB; ++bb) {
                const float e = (bb & 1) ? mix_mul<1>(o.kd[i][bb], qd[bb]) : mix_mul<0>(o.kd[i][bb], qd[bb]);
                x = fmaf((float)cs[bb][i], e, x);
            }
            sc[i] = x;
        }
        if constexpr (CHECK) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int j = jt + kb + SK * sr + 4 * i + g;
                bool live = j < jend;
                if (mrow) {
                    const float mv = live ? mask_at(mrow, j, a.mask_f32) * kLog2e : 0.0f;
                    live = live && mv != -INFINITY;
                    sc[i] += mv;
                }
                sc[i] = live ? sc[i] : -INFINITY;
            }
        }
    };
    // Running max of row n, raised lazily to the row's max over smax (the
    // lane's scores of every slot pair of the tile).  Called once per tile,
    // after every pending P.V has gone into acc and before any of the tile's
    // P' is formed, so acc and l are the only quantities on the old base.
    auto rescale = [&](float smax) {
        if (__any(smax > m + kLazy)) {
            const float cm = max_swap32(max_swap16(smax));
            if (cm > m + kLazy) {
                const float alpha = __builtin_amdgcn_exp2f(m - cm);     // 0 when m = -inf
                l *= alpha;
#pragma unroll
                for (int s = 0; s < 2; ++s)
#pragma unroll
                    for (int j = 0; j < NJ; ++j) acc[s][j] *= alpha;
                m = cm;
                mb = cm + (float)vexp;
            }
        }
    };
    // The V block scales of keys 0, 1 (h = 0) or 2, 3 (h = 1) of a slot pair,
    // block bb, as an f16 pair.
    auto pair_dv = [&](const PairOps& o, int bb, int h) {
        const uint32_t sel = (bb & 1) ? 0x07060302u : 0x05040100u;          // high or low halves
        return __builtin_amdgcn_perm(o.vd[2 * h + 1][bb], o.vd[2 * h][bb], sel);
    };
    // Raises row n's V-range exponent when a block of the tile has d_v >=
    // 2^8 (e = 0) or 2^(7 + e) (d_v >= 0, so f16 bits compare as integers).  Called after
    // the softmax rescale, when every pending P.V is in acc, before the
    // tile's P' is formed.  The test reads the scale dwords as they are:
    // even blocks hold d_v in the low half, odd blocks in the high half.
    auto vrange = [&](const PairOps (&ops)[NSUB]) {
        u16x2 me = {0, 0}, mo = {0, 0};
#pragma unroll
        for (int u = 0; u < NSUB; ++u)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int bb = 0; bb < NB; ++bb) {
                    if (bb & 1) mo = __builtin_elementwise_max(mo, as_u16x2(ops[u].vd[i][bb]));
                    else me = __builtin_elementwise_max(me, as_u16x2(ops[u].vd[i][bb]));
                }
        uint32_t m16 = __builtin_elementwise_max((uint32_t)me[0], (uint32_t)mo[1]);
        const uint32_t lim = __builtin_elementwise_max(0x5c00u, 0x5800u + ((uint32_t)vexp << 10));
        if (__any(m16 >= lim)) {
            // row n's max over the four lane groups
            auto r16 = __builtin_amdgcn_permlane16_swap(m16, m16, false, false);
            m16 = __builtin_elementwise_max(r16[0], r16[1]);
            auto r32 = __builtin_amdgcn_permlane32_swap(m16, m16, false, false);
            m16 = __builtin_elementwise_max(r32[0], r32[1]);
            const int need = m16 >= lim ? (int)(m16 >> 10) - 15 - 6 : vexp;
            const float f = __builtin_amdgcn_ldexpf(1.0f, vexp - need);
            l *= f;
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
                for (int j = 0; j < NJ; ++j) acc[s2][j] *= f;
            mb += (float)(need - vexp);
            vexp = need;
            vscaled = true;
        }
    };
    // p = 2^(s - mb) of one slot pair, its row sums, and its P' = p * d_v
    // (formed in fp32 once the wave's V range needs it).
    auto group_probs = [&](const PairOps& o, const float (&sc)[4], PendingPV& cur) {
        float p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f(sc[i] - mb);   // 0 when masked
        l += (p[0] + p[1]) + (p[2] + p[3]);
        if (!vscaled) {
            const h2 p01 = h2{(_Float16)p[0], (_Float16)p[1]};
            const h2 p23 = h2{(_Float16)p[2], (_Float16)p[3]};
#pragma unroll
            for (int bb = 0; bb < NB; ++bb) {
                h2 dv01, dv23;
                const uint32_t u01 = pair_dv(o, bb, 0), u23 = pair_dv(o, bb, 1);
                __builtin_memcpy(&dv01, &u01, 4);
                __builtin_memcpy(&dv23, &u23, 4);
                cur.pb[bb] = cat_h4(p01 * dv01, p23 * dv23);
            }
        } else {
#pragma unroll
            for (int bb = 0; bb < NB; ++bb) {
                h4 r;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t w = pair_dv(o, bb, i >> 1);
                    r[i] = (_Float16)(p[i] * f16_to_f32((uint16_t)((i & 1) ? (w >> 16) : (w & 0xffffu))));
                }
                cur.pb[bb] = r;
            }
        }
    };

    // tile t has landed in every wave's share; every wave is done with t - 1
    // (whose V codes wait in registers for their P.V).  The pending P.V
    // operands alternate between two sets, tile by tile, so they stay put.
    PendingPV pa[NSUB], pz[NSUB];
#pragma unroll
    for (int u = 0; u < NSUB; ++u) {
#pragma unroll
        for (int bb = 0; bb < NB; ++bb) {
            pz[u].pb[bb] = h4{};
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
                for (int i = 0; i < 4; ++i) pz[u].vc[s][i][bb] = 0;
        }
    }
    auto tile = [&](int t, auto check, const PendingPV (&prev)[NSUB], PendingPV (&cur)[NSUB]) {
        lds_barrier();                               // T_t
        const char* kt = lds + (t & (kStages - 1)) * kStage + dk;
        const char* vt = lds + (t & (kStages - 1)) * kStage + kOpBytes + dv;
        const int jt = tile_key(t);
        const int jend = t == 0 ? p_end : L;         // the piece ends early
        if constexpr (STEP) {
            if (t == new_t) {                        // wave-uniform: the new row into the tile
                const int r = L - 1 - jt;
                for (int x = threadIdx.x; x < 2 * RB / 4; x += kW * 64) {
                    const int op = x / (RB / 4), wd = x % (RB / 4);
                    ((uint32_t*)((op ? vt : kt) + r * RB))[wd] = ((const uint32_t*)(new_rows + op * RB))[wd];
                }
                lds_barrier();                       // N
            }
        }
        PairOps ops[NSUB];
#pragma unroll
        for (int u = 0; u < NSUB; ++u) read_pair(kt, vt, pair_key(u), ops[u]);
        // every pending P.V into acc and every score of the tile first, then
        // one rescale decision, then the tile's P' on the final base: with
        // NSUB > 1 (d = 64) a raise decided per slot pair would leave P'
        // formed on the old base unscaled
        float sc[NSUB][4];
#pragma unroll
        for (int u = 0; u < NSUB; ++u) group_scores(ops[u], pair_key(u), jt, jend, check, prev[u], cur[u], sc[u]);
        float smax = -INFINITY;
#pragma unroll
        for (int u = 0; u < NSUB; ++u) smax = fmaxf(smax, fmaxf(fmaxf(sc[u][0], sc[u][1]), fmaxf(sc[u][2], sc[u][3])));
        rescale(smax);
        vrange(ops);
#pragma unroll
        for (int u = 0; u < NSUB; ++u) group_probs(ops[u], sc[u], cur[u]);
    };
    // The piece (tile 0) is checked against its end; the whole tiles run
    // without checks (all tiles are checked under a mask).  Tiles go in pairs
    // (pa -> pz, pz -> pa) after the piece (pz -> pa); an even count ends
    // with one more tile into pz, whose P.V is the last.
    tile(0, std::true_type{}, pz, pa);
    int t = 1;
    if (mrow != nullptr) {
        for (; t + 1 < n_tiles; t += 2) {
            tile(t, std::true_type{}, pa, pz);
            tile(t + 1, std::true_type{}, pz, pa);
        }
    } else {
        for (; t + 1 < n_tiles; t += 2) {
            tile(t, std::false_type{}, pa, pz);
            tile(t + 1, std::false_type{}, pz, pa);
        }
    }
    if (t < n_tiles) {
        tile(t, std::true_type{}, pa, pz);
#pragma unroll
        for (int u = 0; u < NSUB; ++u) pv(pz[u]);
    } else {
#pragma unroll
        for (int u = 0; u < NSUB; ++u) pv(pa[u]);
    }
    __syncthreads();                                 // the producers' last loads have landed

    // row n's sum over the four lane groups
    l = add_swap32(add_swap16(l));

    // ---- every (wave, row) result to LDS: (m, l, O[D]) of query row rr of
    // slot sr.  Lane (g, n) holds O[32 b + 8 g + 2 i + s] = acc[sr][2 b + s][i].
    constexpr int PS = D + 4;                 // floats per (wave, row) record
    float* part = (float*)lds;
    {
        float* prow = part + (w * 16 + n) * PS;
#pragma unroll
        for (int bb = 0; bb < NB; ++bb) {
            const f32x4 e = sr ? acc[1][2 * bb] : acc[0][2 * bb];
            const f32x4 o = sr ? acc[1][2 * bb + 1] : acc[0][2 * bb + 1];
            *(float4*)(prow + 32 * bb + 8 * g) = make_float4(e[0], o[0], e[1], o[1]);
            *(float4*)(prow + 32 * bb + 8 * g + 4) = make_float4(e[2], o[2], e[3], o[3]);
        }
        if (g == 0) { prow[D] = m + (float)vexp; prow[D + 1] = l; }   // the record's base (-inf stays -inf)
    }
    __syncthreads();

    // ---- per (query head, 8 dims): log-sum-exp over the records of its
    // rows: the waves of its head pair (HKV >= 2: row 8 (h & 1) + r) or all
    // waves and both slots (HKV = 1: rows r and 8 + r).  Every record is
    // read first (one LDS round trip), then weighed by exp2(m - M): a record
    // with nothing visible has m = -inf, weight 0, and zero l and O.
    constexpr int NREC = HKV >= 2 ? kW / HP : 2 * kW;
    constexpr int D8 = D / 8;
    const int ntask = HQL * D8;
    for (int task = threadIdx.x; task < ntask; task += kW * 64) {
        const int hql = task / D8, d8 = task % D8;
        const int hq = hq0 + hql;                    // global query head
        const int h = hql / G, r = hql % G;
        float mm[NREC], ll[NREC];
        float4 v0[NREC], v1[NREC];
#pragma unroll
        for (int k = 0; k < NREC; ++k) {
            const int ww = HKV >= 2 ? h / 2 + HP * k : k >> 1;
            const int nn = HKV >= 2 ? 8 * (h & 1) + r : 8 * (k & 1) + r;
            const float* rec = part + (ww * 16 + nn) * PS;
            mm[k] = rec[D];
            ll[k] = rec[D + 1];
            v0[k] = *(const float4*)(rec + 8 * d8);
            v1[k] = *(const float4*)(rec + 8 * d8 + 4);
        }
        float M = mm[0];
#pragma unroll
        for (int k = 1; k < NREC; ++k) M = fmaxf(M, mm[k]);
        const float Mb = M == -INFINITY ? 0.0f : M;  // all records empty: every weight 0
        float den = 0.0f;
        float4 n0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), n1 = n0;
#pragma unroll
        for (int k = 0; k < NREC; ++k) {
            const float f = __builtin_amdgcn_exp2f(mm[k] - Mb);
            den = fmaf(ll[k], f, den);
            n0.x = fmaf(v0[k].x, f, n0.x); n0.y = fmaf(v0[k].y, f, n0.y);
            n0.z = fmaf(v0[k].z, f, n0.z); n0.w = fmaf(v0[k].w, f, n0.w);
            n1.x = fmaf(v1[k].x, f, n1.x); n1.y = fmaf(v1[k].y, f, n1.y);
            n1.z = fmaf(v1[k].z, f, n1.z); n1.w = fmaf(v1[k].w, f, n1.w);
        }
        if (n_splits == 1) {
            const float inv = den == 0.0f ? 0.0f : 1.0f / den;
            float* orow = (float*)((char*)a.out + b * a.o_nb_b + hq * a.o_nb_h) + 8 * d8;
            *(float4*)orow = make_float4(n0.x * inv, n0.y * inv, n0.z * inv, n0.w * inv);
            *(float4*)(orow + 4) = make_float4(n1.x * inv, n1.y * inv, n1.z * inv, n1.w * inv);
        } else {
            // partials: acc [B][Hq][n_splits][D], then (m, l) [B][Hq][n_splits][2]
            const size_t idx = ((size_t)b * a.Hq + hq) * n_splits + split;
            *(float4*)(ws + idx * D + 8 * d8) = n0;
            *(float4*)(ws + idx * D + 8 * d8 + 4) = n1;
            if (d8 == 0) *(float2*)(ws + (size_t)a.B * a.Hq * n_splits * D + idx * 2) = make_float2(M, den);
        }
    }
}

// Head groups of the cache rows: d = 128 caches with 4 or 8 kv heads are
// split into pairs (272-byte row slices) when every row is 16-byte aligned.
int stream_groups(const AttnArgs& a) {
    if (a.d != 128 || a.Hkv < 4) return 1;
    for (int b = 0; b < a.B; ++b)
        if (((uintptr_t)a.k[b] % 16) || ((uintptr_t)a.v[b] % 16)) return 1;
    return a.Hkv / 2;
}

template <int D, bool STEP>
hipError_t launch_ds(const AttnArgs& a, const StreamStep& st, float* ws, int n_splits, hipStream_t s) {
    const int ng = stream_groups(a);
    const dim3 grid(n_splits, a.B * ng), block((kW + kP) * 64);
    auto finish = [&]() -> hipError_t {
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess || n_splits == 1) return e;
        return launch_decode_merge(a, ws, n_splits, s);
    };
#define VVA_DS(H, NG) hipLaunchKernelGGL((decode_stream_kernel<D, H, NG, STEP>), grid, block, 0, s, a, ws, n_splits, st)
    if constexpr (D == 128) {
        if (ng == 2) { VVA_DS(2, 2); return finish(); }
        if (ng == 4) { VVA_DS(2, 4); return finish(); }
    }
    if (a.Hkv == 1) VVA_DS(1, 1);
    else if (a.Hkv == 2) VVA_DS(2, 1);
    else if (!STEP && a.Hkv == 4) VVA_DS(4, 1);
    else if (!STEP && a.Hkv == 8) VVA_DS(8, 1);
    else return hipErrorInvalidValue;
#undef VVA_DS
    return finish();
}

}  // namespace

bool decode_stream_supported(const AttnArgs& a) {
    if (a.T != 1) return false;
    if (a.d != 64 && a.d != 128) return false;
    if (a.k_type != VVA_TYPE_Q8_0 || a.v_type != VVA_TYPE_Q8_0) return false;
    if (a.Hkv < 1 || a.Hq % a.Hkv != 0 || a.Hq / a.Hkv > 8) return false;
    if (a.Hkv != 1 && a.Hkv != 2 && a.Hkv != 4 && a.Hkv != 8) return false;
    // dense rows: [token][kv head][blocks], as the resident cache stores them
    const int64_t hb = (int64_t)(a.d / 32) * kQ8Bytes;
    if (a.k_nb_head != hb || a.v_nb_head != hb) return false;
    if (a.k_nb_tok != hb * a.Hkv || a.v_nb_tok != hb * a.Hkv) return false;
    for (int b = 0; b < a.B; ++b) {
        if (((uintptr_t)a.k[b] % 4) || ((uintptr_t)a.v[b] % 4)) return false;
        // every buffer range and live offset stays below the padding offset
        if ((int64_t)(a.L[b] + 1) * a.k_nb_tok + 2 * kOpBytes >= kDead) return false;
    }
    if (a.mask_mode == kMaskExplicit && (a.mask_nb_b % (a.mask_f32 ? 4 : 2) != 0)) return false;
    if (((uintptr_t)a.q % 16) || a.q_nb_h % 16 || a.q_nb_b % 16) return false;
    // Q rows contiguous and small enough for the raw-Q area, codes after them
    const int64_t qrow = (int64_t)a.d * type_elem_bytes(a.q_type);
    if (a.q_nb_h != qrow || a.Hq * qrow > kQRawBytes) return false;
    if (kQRawBytes + (int64_t)a.Hq * (a.d / 32) * 36 > kStage) return false;
    if (((uintptr_t)a.out % 16) || a.o_nb_h % 16 || a.o_nb_b % 16) return false;
    return true;
}

int decode_stream_plan(const AttnArgs& a, int n_cu) {
    int Lmax = 1;
    for (int b = 0; b < a.B; ++b) Lmax = a.L[b] > Lmax ? a.L[b] : Lmax;
    // one workgroup per CU over (split, sequence, head group); at least two
    // tiles' worth of keys per split
    const int ng = stream_groups(a);
    int target = n_cu / (a.B * ng);
    if (target < 1) target = 1;
    int sl = (Lmax + target - 1) / target;
    const int min_len = 2 * kTileOpBytes / (int)((a.d / 32) * kQ8Bytes * (a.Hkv / ng));
    if (sl < min_len) sl = min_len;
    return (Lmax + sl - 1) / sl;
}

hipError_t launch_decode_stream(const AttnArgs& a, float* ws, int n_splits, hipStream_t s) {
    const StreamStep none{};
    if (a.d == 64) return launch_ds<64, false>(a, none, ws, n_splits, s);
    if (a.d == 128) return launch_ds<128, false>(a, none, ws, n_splits, s);
    return hipErrorInvalidValue;
}

// Step mode: the kv heads of a workgroup (a head pair, or one or two heads
// without head groups) are one wave's rotation pairs each, for K and for V.
bool decode_stream_step_supported(const AttnArgs& a) {
    if (!decode_stream_supported(a)) return false;
    return a.Hkv / stream_groups(a) <= 2;
}

hipError_t launch_decode_stream_step(const AttnArgs& a, const StreamStep& st, float* ws, int n_splits, hipStream_t s) {
    if (a.d == 64) return launch_ds<64, true>(a, st, ws, n_splits, s);
    if (a.d == 128) return launch_ds<128, true>(a, st, ws, n_splits, s);
    return hipErrorInvalidValue;
}

}  // namespace vva
