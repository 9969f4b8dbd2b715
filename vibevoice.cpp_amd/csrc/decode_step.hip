// decode_step.hip — one launch per layer for a single-token decode step on
// F16 / BF16 caches of moderate length: the RoPE of q and k, the K/V append
// at len(seq_b), the attention over the len + 1 keys and the merge of its key
// splits (src/qwen2.cpp:282-335 with one new token per sequence; the TTS CFG
// loop, src/vibevoice_tts.cpp:862-880, runs two such steps per frame).  At
// these sizes (a 1 MB window per layer, L2 / MALL resident) a call is a
// chain of latencies, and the kernel is laid out to keep the chain short.
//
// Grid (n_splits, Hkv, B); 4 waves.  Workgroup (s, h, b) takes keys
// [128 s, 128 s + 128) of sequence b's window, 32 per wave, and the G <= 8
// query heads of kv head h:
//   0. every kernel argument is read in one batch (each scalar-cache miss is
//      a round trip, and that cache starts cold at every launch), then every
//      global load is issued before any is used: q and the new k / v rows as
//      raw 32-bit words, the wave's K rows as MFMA operands, its V rows;
//   1. the angle table of the token's position (the fp32 theta recurrence of
//      rope_append.hip) while the loads fly; RoPE(q), rounded to the cache
//      type (ggml's flash attention casts Q to K's type); split 0 writes
//      q_out;
//   2. the split holding key len(seq_b) rotates k and writes the new K and V
//      rows to the cache and into its own operands;
//   3. per wave, with v_mfma_f32_32x32x16: S^T = K Q^T (K rows from memory
//      as the A operand, the G heads as the columns of B), softmax over the
//      wave's 32 keys per head (fp32, exp2 domain), O^T = V^T P^T (P^T
//      converted in place from S^T as f16, V^T read from the wave's LDS V
//      tile with the transposing load);
//   4. the waves' (max, sum, O) are combined in LDS; with one split that is
//      the output, otherwise the workgroup writes (max, sum, acc) with
//      agent-scope stores (coherent across XCDs without an L2 write-back),
//      takes a ticket, and the last workgroup of (b, h) merges the splits
//      with one batch of agent-scope loads and resets the ticket for the
//      next call.
#include "vva_internal.hpp"

namespace vva {

namespace {

#include "wave_ops.hpp"
#include "mfma_ops.hpp"

constexpr int kStepWaves = 4;
constexpr int kKPW = 32 * kStepWaves;    // keys per workgroup
constexpr int kMaxG = 8;                 // query heads per kv head

// Barrier for LDS hand-offs only: unlike __syncthreads it does not wait for
// the wave's outstanding global loads and stores.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory");
}

// Element i of a row held as raw 32-bit words (F32, or F16 / BF16 pairs).
__device__ __forceinline__ float raw_elem(const uint32_t* row, int i, int type) {
    if (type == VVA_TYPE_F32) return __uint_as_float(row[i]);
    const uint32_t w = row[i >> 1];
    const uint16_t x = (uint16_t)(i & 1 ? w >> 16 : w);
    return type == VVA_TYPE_F16 ? f16_to_f32(x) : bf16_to_f32(x);
}

template <int D, int KT>
__global__ void __launch_bounds__(64 * kStepWaves) decode_step_kernel(StepArgs a) {
    using F = Frag<KT>;
    using QF = typename F::type;
    constexpr int P = D / 2, DS = D / 16, DT = D / 32;
    constexpr int VP = D * 2 + 64;             // V tile row pitch in bytes: conflict-free transposing reads
    constexpr int CPR = D / 8;                 // 16-byte chunks per K / V head row
    constexpr int NVC = 32 * CPR / 64;         // V chunks per lane (the wave's 32 rows)
    constexpr int NQW = kMaxG * D / 256;       // q words per thread at most (F32 q)
    __shared__ float cs[P], sn[P];
    __shared__ uint32_t qraw[kMaxG * D], kraw[D], vraw[D];                 // raw input words
    __shared__ __attribute__((aligned(16))) uint16_t qh[kMaxG][D];         // RoPE(q), cache type
    __shared__ __attribute__((aligned(16))) uint16_t knew[D];              // the new K row
    __shared__ __attribute__((aligned(16))) char vt[kStepWaves][32 * VP];  // V rows per wave
    __shared__ float wm[kStepWaves][kMaxG], wl[kStepWaves][kMaxG];
    __shared__ __attribute__((aligned(16))) float wo[kStepWaves][kMaxG][D];
    __shared__ int ticket;

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l32 = lane & 31, half = lane >> 5;
    const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int n_splits = gridDim.x;

    // ---- 0. kernel arguments (one scalar round trip for all of them)
    prefetch_kernargs<sizeof(StepArgs)>();
    const int past = a.past[b], G = a.G, Hq = a.Hq;
    const int q_type = a.q_type, k_type = a.k_type, v_type = a.v_type, qo_type = a.q_out_type;
    const int64_t rb = a.cache_row_bytes, q_nb_h = a.q_nb_h, qo_nb_h = a.qo_nb_h, o_nb_h = a.o_nb_h;
    const char* const kch = a.kc[b] + h * a.cache_head_bytes;      // row 0 of head h
    const char* const vch = a.vc[b] + h * a.cache_head_bytes;
    const char* const qb = a.q + b * a.q_nb_b + (int64_t)h * G * q_nb_h;
    const char* const kn = a.k + b * a.k_nb_b + h * a.k_nb_h;
    const char* const vn = a.v + b * a.v_nb_b + h * a.v_nb_h;
    const int32_t* const posp = a.pos + b * a.pos_stride_b;
    const bool has_qo = a.q_out != nullptr;
    char* const qob = a.q_out + b * a.qo_nb_b + (int64_t)h * G * qo_nb_h;     // used only when has_qo
    char* const ob = (char*)a.out + b * a.o_nb_b + (int64_t)h * G * o_nb_h;
    float* const ws = a.ws;
    unsigned* const tk = a.tickets + b * a.Hkv + h;
    const float theta_scale = a.theta_scale, scale = a.scale;
    const size_t ml_off = (size_t)a.B * Hq * n_splits * D;       // (max, sum) pairs after the accumulators
    const int pos_i = *posp;

    const int L = past + 1;
    const int j0 = split * kKPW, j1 = min(L, j0 + kKPW);
    const int kb = j0 + 32 * w;                                   // the wave's first key
    const bool owns_new = j0 <= past && past < j1;
    // q: G head rows of raw words
    const int qwpr_sh = __builtin_ctz(D) - (q_type == VVA_TYPE_F32 ? 0 : 1);   // log2(words per row)
    const int nqw = G << qwpr_sh;
    uint32_t qw[NQW];
#pragma unroll
    for (int u = 0; u < NQW; ++u) {
        const int idx = tid + 256 * u;
        const int r = idx >> qwpr_sh, c = idx - (r << qwpr_sh);
        const bool ok = idx < nqw;
        qw[u] = ((const uint32_t*)(qb + (ok ? r : 0) * q_nb_h))[ok ? c : 0];
    }
    // the new k row (waves 0, 1) and v row (waves 2, 3): a wave-uniform choice
    const bool is_k = __builtin_amdgcn_readfirstlane(w) < 2;
    const int nwi = is_k ? tid : tid - 128;
    const bool nw_ok = nwi < (D >> ((is_k ? k_type : v_type) == VVA_TYPE_F32 ? 0 : 1));
    uint32_t nw = 0;
    if (owns_new) {
        if (is_k) nw = ((const uint32_t*)kn)[nw_ok ? nwi : 0];
        else      nw = ((const uint32_t*)vn)[nw_ok ? nwi : 0];
    }
    // K as the A operand: lane (l32, half) holds key kb + l32, dims
    // 16 ds + 8 half .. + 7 (keys past the window read row 0 and are masked)
    const int kkey = kb + l32;
    u32x4 kf[DS];
    {
        const char* kr = kch + (int64_t)(kkey < j1 ? kkey : 0) * rb + half * 16;
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) kf[ds] = *(const u32x4*)(kr + ds * 32);
    }
    // the wave's 32 V rows: chunk c = lane + 64 u is row c / CPR, bytes 16 (c % CPR) ..
    u32x4 vq[NVC];
#pragma unroll
    for (int u = 0; u < NVC; ++u) {
        const int c = lane + 64 * u, row = c / CPR, key = kb + row;
        vq[u] = *(const u32x4*)(vch + (int64_t)(key < j1 ? key : 0) * rb + (c % CPR) * 16);
    }

    // ---- 1. angle table; the raw q / k / v words to LDS
    if (tid < P) {
        const float th = rope_theta((float)pos_i, theta_scale, tid, P);
        cs[tid] = cosf(th);
        sn[tid] = sinf(th);
    }
#pragma unroll
    for (int u = 0; u < NQW; ++u)
        if (tid + 256 * u < nqw) qraw[tid + 256 * u] = qw[u];
    if (owns_new && nw_ok) (is_k ? kraw : vraw)[nwi] = nw;
    lds_barrier();
    // RoPE(q), rounded to the cache type for the scores
    for (int t = tid; t < G * P; t += 256) {
        const int r = t / P, i = t - r * P;
        const uint32_t* qrow = qraw + (r << qwpr_sh);
        const float x0 = raw_elem(qrow, i, q_type), x1 = raw_elem(qrow, i + P, q_type);
        const float y0 = fmaf(x0, cs[i], -(x1 * sn[i])), y1 = fmaf(x0, sn[i], x1 * cs[i]);
        qh[r][i] = F::cvt(y0);
        qh[r][i + P] = F::cvt(y1);
        if (split == 0 && has_qo) {
            const int64_t eo = type_elem_bytes(qo_type);
            char* dst = qob + r * qo_nb_h;
            store_elem(dst + i * eo, qo_type, y0);
            store_elem(dst + (i + P) * eo, qo_type, y1);
        }
    }
    // ---- 2. the new K / V row (the split holding key L - 1): to the cache,
    // to knew (substituted into the K operand) and to the V tile
    if (owns_new && tid < P) {
        const int i = tid;
        const float x0 = raw_elem(kraw, i, k_type), x1 = raw_elem(kraw, i + P, k_type);
        const float y0 = fmaf(x0, cs[i], -(x1 * sn[i])), y1 = fmaf(x0, sn[i], x1 * cs[i]);
        const uint16_t k0h = F::cvt(y0), k1h = F::cvt(y1);
        const uint16_t v0h = F::cvt(raw_elem(vraw, i, v_type)), v1h = F::cvt(raw_elem(vraw, i + P, v_type));
        knew[i] = k0h;
        knew[i + P] = k1h;
        const int rn = past - j0;
        uint16_t* vtr = (uint16_t*)(vt[rn >> 5] + (rn & 31) * VP);
        vtr[i] = v0h;
        vtr[i + P] = v1h;
        uint16_t* krow = (uint16_t*)(kch + (int64_t)past * rb);
        uint16_t* vrow = (uint16_t*)(vch + (int64_t)past * rb);
        krow[i] = k0h;
        krow[i + P] = k1h;
        vrow[i] = v0h;
        vrow[i + P] = v1h;
    }
    // the wave's V rows into its tile: zeros past the window (their p is 0,
    // and 0 * inf would not be), the new row from step 2
#pragma unroll
    for (int u = 0; u < NVC; ++u) {
        const int c = lane + 64 * u, row = c / CPR, key = kb + row;
        if (!(owns_new && key == past))
            *(u32x4*)(vt[w] + row * VP + (c % CPR) * 16) = key < j1 ? vq[u] : u32x4{0u, 0u, 0u, 0u};
    }
    lds_barrier();

    // ---- 3. S^T = K Q^T over the wave's 32 keys (column l32 = head)
    if (kkey == past) {
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) kf[ds] = *(const u32x4*)&knew[ds * 16 + half * 8];
    }
    f32x16 s = {};
    {
        const bool hv = l32 < G;
        const uint16_t* qrow = qh[hv ? l32 : 0];
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
            const u32x4 u = *(const u32x4*)(qrow + ds * 16 + half * 8);
            s = F::mma(as_vec<QF>(kf[ds]), as_vec<QF>(hv ? u : u32x4{0u, 0u, 0u, 0u}), s);
        }
    }
    // softmax over the wave's keys: register r holds key kb + 8 (r / 4) + 4 half + r % 4
    const float sl2 = scale * kLog2e;
    float mr = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int key = kb + 8 * (r >> 2) + 4 * half + (r & 3);
        s[r] = key < j1 ? s[r] : -INFINITY;
        mr = fmaxf(mr, s[r]);
    }
    const float mx = max_swap32(mr) * sl2;                     // the wave's max for head l32 (log2 units)
    const float nb = mx == -INFINITY ? 0.0f : -mx;
    h8 pf[2];
    float psum = 0.0f;
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const float p0 = __builtin_amdgcn_exp2f(fmaf(s[k2 * 8 + e], sl2, nb));
            const float p1 = __builtin_amdgcn_exp2f(fmaf(s[k2 * 8 + e + 1], sl2, nb));
            const h2 pp = {(_Float16)p0, (_Float16)p1};
            pf[k2][e] = pp.x;
            pf[k2][e + 1] = pp.y;
            psum = __builtin_amdgcn_fdot2(pp, h2{(_Float16)1.0f, (_Float16)1.0f}, psum, false);
        }
    const float lw = add_swap32(psum);
    // O^T = V^T P^T: o[dt] register r holds dim 32 dt + 8 (r / 4) + 4 half + r % 4
    f32x16 o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt] = f32x16{};
    {
        const lds_char* va = (const lds_char*)vt[w] + v_frag_offset(lane, VP);
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const h8 vf = v_frag<KT>(va + dt * 64 + k2 * 16 * VP, va + dt * 64 + (k2 * 16 + 8) * VP);
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[k2], o[dt], 0, 0, 0);
            }
    }

    // ---- 4. the waves' (max, sum, O) combined in LDS
    if (l32 < G) {
        if (half == 0) {
            wm[w][l32] = mx;
            wl[w][l32] = lw;
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4)
                *(float4*)&wo[w][l32][dt * 32 + 8 * q4 + 4 * half] =
                    make_float4(o[dt][4 * q4], o[dt][4 * q4 + 1], o[dt][4 * q4 + 2], o[dt][4 * q4 + 3]);
    }
    lds_barrier();
    // thread t: head t / P, dims 2 (t % P) and 2 (t % P) + 1
    for (int t = tid; t < G * P; t += 256) {
        const int r = t / P, dp = t - r * P;
        float M = -INFINITY;
#pragma unroll
        for (int v = 0; v < kStepWaves; ++v) M = fmaxf(M, wm[v][r]);
        const float Mb = M == -INFINITY ? 0.0f : M;
        float l = 0.0f, o0 = 0.0f, o1 = 0.0f;
#pragma unroll
        for (int v = 0; v < kStepWaves; ++v) {
            const float f = __builtin_amdgcn_exp2f(wm[v][r] - Mb);      // 0 for a wave with no key
            const float2 ov = *(const float2*)&wo[v][r][2 * dp];
            l = fmaf(wl[v][r], f, l);
            o0 = fmaf(ov.x, f, o0);
            o1 = fmaf(ov.y, f, o1);
        }
        if (n_splits == 1) {
            float* orow = (float*)(ob + r * o_nb_h);
            const float inv = l > 0.0f ? 1.0f / l : 0.0f;
            *(float2*)(orow + 2 * dp) = make_float2(o0 * inv, o1 * inv);
        } else {
            const size_t rowi = ((size_t)b * Hq + h * G + r) * n_splits + split;
            store_coherent2(ws + rowi * D + 2 * dp, o0, o1);
            if (dp == 0) store_coherent2(ws + ml_off + rowi * 2, M, l);
        }
    }
    if (n_splits == 1) return;
    // every partial store of this workgroup has completed before its ticket
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) ticket = (int)__hip_atomic_fetch_add(tk, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    lds_barrier();
    if (ticket != n_splits - 1) return;
    // ---- the last workgroup of (b, h): log-sum-exp over the splits, every
    // split's (max, sum) and accumulator pair loaded in one batch (16 splits
    // per batch)
    for (int t = tid; t < G * P; t += 256) {
        const int r = t / P, dp = t - r * P;
        const size_t row0 = ((size_t)b * Hq + h * G + r) * n_splits;
        float Mx = -INFINITY, n0 = 0.0f, n1 = 0.0f, den = 0.0f;   // running log-sum-exp over the batches
        for (int s0 = 0; s0 < n_splits; s0 += 16) {
            float2 ml[16], ac[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const bool in = s0 + e < n_splits;
                const size_t ri = row0 + (in ? s0 + e : 0);
                ml[e] = load_coherent2(ws + ml_off + ri * 2);
                ac[e] = load_coherent2(ws + ri * D + 2 * dp);
                if (!in) ml[e] = make_float2(-INFINITY, 0.0f);
            }
            float bm = Mx;
#pragma unroll
            for (int e = 0; e < 16; ++e) bm = fmaxf(bm, ml[e].x);
            const float base = bm == -INFINITY ? 0.0f : bm;
            const float rescale = __builtin_amdgcn_exp2f(Mx - base);     // 0 while Mx = -inf
            n0 *= rescale;
            n1 *= rescale;
            den *= rescale;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float f = __builtin_amdgcn_exp2f(ml[e].x - base);
                n0 = fmaf(ac[e].x, f, n0);
                n1 = fmaf(ac[e].y, f, n1);
                den = fmaf(ml[e].y, f, den);
            }
            Mx = bm;
        }
        float* orow = (float*)(ob + r * o_nb_h);
        const float inv = den > 0.0f ? 1.0f / den : 0.0f;
        *(float2*)(orow + 2 * dp) = make_float2(n0 * inv, n1 * inv);
    }
    if (tid == 0) __hip_atomic_store(tk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

bool decode_step_supported(const StepArgs& a) {
    if (a.cache_type != VVA_TYPE_F16 && a.cache_type != VVA_TYPE_BF16) return false;
    if (a.d != 64 && a.d != 128) return false;
    if (a.Hq % a.Hkv || a.Hq / a.Hkv > kMaxG) return false;
    if (a.B * a.Hkv > kMaxStepTickets) return false;
    // q, k and v are read as 32-bit words
    for (const int64_t x : {(int64_t)(uintptr_t)a.q, a.q_nb_h, a.q_nb_b, (int64_t)(uintptr_t)a.k, a.k_nb_h, a.k_nb_b,
                            (int64_t)(uintptr_t)a.v, a.v_nb_h, a.v_nb_b})
        if (x % 4) return false;
    for (int b = 0; b < a.B; ++b) {
        if (a.past[b] + 1 > kKPW * kMaxStepSplits) return false;
        if ((uintptr_t)a.kc[b] % 16 || (uintptr_t)a.vc[b] % 16) return false;
    }
    // the output is written as float pairs
    if ((uintptr_t)a.out % 8 || a.o_nb_h % 8 || a.o_nb_b % 8) return false;
    return a.cache_row_bytes % 16 == 0 && a.cache_head_bytes % 16 == 0;
}

int decode_step_splits(const StepArgs& a) {
    int Lmax = 1;
    for (int b = 0; b < a.B; ++b) Lmax = max(Lmax, a.past[b] + 1);
    return (Lmax + kKPW - 1) / kKPW;
}

hipError_t launch_decode_step(const StepArgs& a, int n_splits, hipStream_t s) {
    const dim3 grid(n_splits, a.Hkv, a.B), block(64 * kStepWaves);
    const bool bf = a.cache_type == VVA_TYPE_BF16;
    if (a.d == 64) {
        if (bf) hipLaunchKernelGGL((decode_step_kernel<64, VVA_TYPE_BF16>), grid, block, 0, s, a);
        else    hipLaunchKernelGGL((decode_step_kernel<64, VVA_TYPE_F16>), grid, block, 0, s, a);
    } else {
        if (bf) hipLaunchKernelGGL((decode_step_kernel<128, VVA_TYPE_BF16>), grid, block, 0, s, a);
        else    hipLaunchKernelGGL((decode_step_kernel<128, VVA_TYPE_F16>), grid, block, 0, s, a);
    }
    return hipGetLastError();
}

}  // namespace vva
