// decode_step.hip — one launch per layer for a single-token decode step on
// F16 / BF16 caches of moderate length: the RoPE of q and k, the K/V append
// at len(seq_b), the attention over the len + 1 keys and the merge of its key
// splits (src/qwen2.cpp:282-335 with one new token per sequence; the TTS CFG
// loop, src/vibevoice_tts.cpp:862-880, runs two such steps per frame).  At
// these sizes (a 1 MB window per layer, L2 / MALL resident) the three
// dependent launches of the unfused path cost more than the work.
//
// Grid (n_splits, B * Hkv); 256 threads.  Workgroup (s, b, h) takes keys
// [s * KPW, (s + 1) * KPW) of sequence b's window and the G query heads of kv
// head h:
//   1. the angle table of the token's position (fp32 theta recurrence, as
//      rope_append.hip) and RoPE(q) of the G heads, rounded to the cache
//      type (the F16 cast ggml's flash attention applies to Q for F16 K);
//      split 0 writes q_out when asked for;
//   2. the split holding key len(seq_b) rotates k, writes the new K and V
//      rows into the cache and keeps them in LDS for its own use;
//   3. scores with one key per lane (v_dot2 against the f16 / bf16 Q pairs
//      in LDS), softmax per head over the workgroup's keys (fp32), then P.V
//      with lanes over dims (coalesced V rows);
//   4. with one split the workgroup writes the output; otherwise it writes
//      (max, sum, acc[d]) per head with agent-scope stores (coherent across
//      XCDs without an L2 write-back), takes a ticket, and the last
//      workgroup of (b, h) merges the partials (agent-scope loads) and
//      resets the ticket for the next call.
#include "vva_internal.hpp"

namespace vva {

namespace {

#include "wave_ops.hpp"

constexpr int kKPW = 128;                // keys per workgroup
constexpr int kMaxG = 8;                 // query heads per kv head

__device__ __forceinline__ void store_coherent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int D, int KT>
__global__ void __launch_bounds__(256) decode_step_kernel(StepArgs a) {
    constexpr int P = D / 2;
    constexpr int KW = D / 2;               // 32-bit words (two 16-bit values) per K / V head row
    __shared__ float cs[P], sn[P];
    __shared__ __attribute__((aligned(16))) uint32_t qp[kMaxG][KW];   // RoPE(q) as 16-bit pairs
    __shared__ __attribute__((aligned(16))) uint32_t knew[KW], vnew[KW];
    __shared__ float ps[kKPW][kMaxG];                                  // p of the workgroup's keys
    __shared__ float wmax[4][kMaxG], wsum[4][kMaxG];
    __shared__ float red[256 / (D / 2) > 0 ? 256 / (D / 2) : 1][kMaxG][D];  // per key group, P.V partials
    __shared__ int ticket;

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int split = blockIdx.x, bh = blockIdx.y;
    const int b = bh / a.Hkv, h = bh % a.Hkv;
    const int G = a.Hq / a.Hkv;
    const int past = a.past[b], L = past + 1;
    const int n_splits = gridDim.x;
    const int j0 = split * kKPW, j1 = min(L, j0 + kKPW);

    // ---- 1. angle table and RoPE(q)
    const float pos = (float)a.pos[b * a.pos_stride_b];
    for (int i = tid; i < P; i += 256) {
        float th = pos;
        for (int k = 0; k < i; ++k) th *= a.theta_scale;
        cs[i] = cosf(th);
        sn[i] = sinf(th);
    }
    __syncthreads();
    for (int idx = tid; idx < G * P; idx += 256) {
        const int r = idx / P, i = idx - r * P;
        const int hq = h * G + r;
        const char* src = a.q + b * a.q_nb_b + hq * a.q_nb_h;
        const int64_t es = type_elem_bytes(a.q_type);
        const float x0 = load_elem(src + i * es, a.q_type), x1 = load_elem(src + (i + P) * es, a.q_type);
        const float y0 = fmaf(x0, cs[i], -(x1 * sn[i])), y1 = fmaf(x0, sn[i], x1 * cs[i]);
        uint16_t* qh = (uint16_t*)&qp[r][0];
        qh[i] = KT == VVA_TYPE_BF16 ? f32_to_bf16(y0) : f32_to_f16(y0);
        qh[i + P] = KT == VVA_TYPE_BF16 ? f32_to_bf16(y1) : f32_to_f16(y1);
        if (split == 0 && a.q_out) {
            const int64_t eo = type_elem_bytes(a.q_out_type);
            char* dst = a.q_out + b * a.qo_nb_b + hq * a.qo_nb_h;
            store_elem(dst + i * eo, a.q_out_type, y0);
            store_elem(dst + (i + P) * eo, a.q_out_type, y1);
        }
    }
    // ---- 2. the new K / V row (the split holding key L - 1)
    const bool owns_new = j0 <= past && past < j1;
    if (owns_new) {
        for (int i = tid; i < P; i += 256) {
            const char* ks = a.k + b * a.k_nb_b + h * a.k_nb_h;
            const char* vs = a.v + b * a.v_nb_b + h * a.v_nb_h;
            const int64_t ek = type_elem_bytes(a.k_type), ev = type_elem_bytes(a.v_type);
            const float x0 = load_elem(ks + i * ek, a.k_type), x1 = load_elem(ks + (i + P) * ek, a.k_type);
            const float y0 = fmaf(x0, cs[i], -(x1 * sn[i])), y1 = fmaf(x0, sn[i], x1 * cs[i]);
            const float v0 = load_elem(vs + i * ev, a.v_type), v1 = load_elem(vs + (i + P) * ev, a.v_type);
            const uint16_t k0h = KT == VVA_TYPE_BF16 ? f32_to_bf16(y0) : f32_to_f16(y0);
            const uint16_t k1h = KT == VVA_TYPE_BF16 ? f32_to_bf16(y1) : f32_to_f16(y1);
            const uint16_t v0h = KT == VVA_TYPE_BF16 ? f32_to_bf16(v0) : f32_to_f16(v0);
            const uint16_t v1h = KT == VVA_TYPE_BF16 ? f32_to_bf16(v1) : f32_to_f16(v1);
            ((uint16_t*)knew)[i] = k0h;
            ((uint16_t*)knew)[i + P] = k1h;
            ((uint16_t*)vnew)[i] = v0h;
            ((uint16_t*)vnew)[i + P] = v1h;
            uint16_t* krow = (uint16_t*)(a.kc[b] + (int64_t)past * a.cache_row_bytes + h * a.cache_head_bytes);
            uint16_t* vrow = (uint16_t*)(a.vc[b] + (int64_t)past * a.cache_row_bytes + h * a.cache_head_bytes);
            krow[i] = k0h;
            krow[i + P] = k1h;
            vrow[i] = v0h;
            vrow[i + P] = v1h;
        }
    }
    __syncthreads();

    // ---- 3a. scores: thread = key (waves 0 and 1; 128 keys)
    const float sl2 = a.scale * kLog2e;
    float sc[kMaxG];
    const int j = j0 + tid;
    const bool live = tid < kKPW && j < j1;
    if (tid < kKPW) {
        uint32_t kw[KW];
        if (live && j == past) {
#pragma unroll
            for (int i = 0; i < KW; ++i) kw[i] = knew[i];
        } else if (live) {
            const uint4* kr = (const uint4*)(a.kc[b] + (int64_t)j * a.cache_row_bytes + h * a.cache_head_bytes);
#pragma unroll
            for (int i = 0; i < KW / 4; ++i) {
                const uint4 u = kr[i];
                kw[4 * i] = u.x; kw[4 * i + 1] = u.y; kw[4 * i + 2] = u.z; kw[4 * i + 3] = u.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < KW; ++i) kw[i] = 0u;
        }
#pragma unroll
        for (int r = 0; r < kMaxG; ++r) {
            if (r >= G) { sc[r] = -INFINITY; continue; }
            float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
            for (int i = 0; i < KW; i += 2) {
                if constexpr (KT == VVA_TYPE_BF16) {
                    s0 = dot2_bf16(qp[r][i], kw[i], s0);
                    s1 = dot2_bf16(qp[r][i + 1], kw[i + 1], s1);
                } else {
                    s0 = dot2_f16(qp[r][i], kw[i], s0);
                    s1 = dot2_f16(qp[r][i + 1], kw[i + 1], s1);
                }
            }
            sc[r] = live ? (s0 + s1) * sl2 : -INFINITY;      // log2 domain
        }
        // ---- 3b. max and sum per head over the workgroup's keys
#pragma unroll
        for (int r = 0; r < kMaxG; ++r) {
            float m = sc[r];
            m = fmaxf(m, dpp<kDppXor1>(m));
            m = fmaxf(m, dpp<kDppXor2>(m));
            m = fmaxf(m, dpp<kDppHalfMirror>(m));
            m = fmaxf(m, dpp<kDppMirror>(m));
            m = max_swap32(max_swap16(m));
            if (lane == 0) wmax[w][r] = m;
        }
    }
    __syncthreads();
    float M[kMaxG];
#pragma unroll
    for (int r = 0; r < kMaxG; ++r) M[r] = fmaxf(wmax[0][r], wmax[1][r]);
    if (tid < kKPW) {
#pragma unroll
        for (int r = 0; r < kMaxG; ++r) {
            const float mb = M[r] == -INFINITY ? 0.0f : M[r];
            const float p = __builtin_amdgcn_exp2f(sc[r] - mb);        // 0 for a dead key
            ps[tid][r] = p;
            const float sum = wave_sum(p);
            if (lane == 0) wsum[w][r] = sum;
        }
    }
    __syncthreads();

    // ---- 3c. P.V: thread = (key group kg, dim pair dp); key group kg takes
    // keys kg, kg + NG, ... of the workgroup
    constexpr int DP = D / 2;                 // dim pairs
    constexpr int NG = 256 / DP;              // key groups
    const int dp = tid % DP, kg = tid / DP;
    float acc[kMaxG][2];
#pragma unroll
    for (int r = 0; r < kMaxG; ++r) acc[r][0] = acc[r][1] = 0.0f;
    for (int jj = kg; jj < j1 - j0; jj += NG) {
        const int jk = j0 + jj;
        const uint32_t vw = jk == past ? vnew[dp]
                                       : *(const uint32_t*)(a.vc[b] + (int64_t)jk * a.cache_row_bytes +
                                                            h * a.cache_head_bytes + dp * 4);
        const float v0 = KT == VVA_TYPE_BF16 ? bf16_to_f32((uint16_t)vw) : f16_to_f32((uint16_t)vw);
        const float v1 = KT == VVA_TYPE_BF16 ? bf16_to_f32((uint16_t)(vw >> 16)) : f16_to_f32((uint16_t)(vw >> 16));
#pragma unroll
        for (int r = 0; r < kMaxG; ++r) {
            const float p = ps[jj][r];
            acc[r][0] = fmaf(p, v0, acc[r][0]);
            acc[r][1] = fmaf(p, v1, acc[r][1]);
        }
    }
#pragma unroll
    for (int r = 0; r < kMaxG; ++r) {
        red[kg][r][2 * dp] = acc[r][0];
        red[kg][r][2 * dp + 1] = acc[r][1];
    }
    __syncthreads();

    // ---- 4. the workgroup's (max, sum, acc) per head; one thread per (head, dim)
    float* part_acc = a.ws;                                                   // [B Hq][n_splits][D]
    float* part_ml = a.ws + (size_t)a.B * a.Hq * n_splits * D;               // [B Hq][n_splits][2]
    for (int idx = tid; idx < G * D; idx += 256) {
        const int r = idx / D, d = idx - r * D;
        float o = 0.0f;
#pragma unroll
        for (int k = 0; k < NG; ++k) o += red[k][r][d];
        const float l = wsum[0][r] + wsum[1][r];
        const int hq = h * G + r;
        if (n_splits == 1) {
            float* orow = (float*)((char*)a.out + b * a.o_nb_b + hq * a.o_nb_h);
            orow[d] = l > 0.0f ? o / l : 0.0f;
        } else {
            const size_t rowi = ((size_t)b * a.Hq + hq) * n_splits + split;
            store_coherent(part_acc + rowi * D + d, o);
            if (d == 0) {
                store_coherent(part_ml + rowi * 2, M[r]);
                store_coherent(part_ml + rowi * 2 + 1, l);
            }
        }
    }
    if (n_splits == 1) return;
    // every partial store of this workgroup has completed before its ticket
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0)
        ticket = (int)__hip_atomic_fetch_add(a.tickets + bh, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (ticket != n_splits - 1) return;
    // ---- the last workgroup of (b, h): log-sum-exp over the splits
    for (int idx = tid; idx < G * D; idx += 256) {
        const int r = idx / D, d = idx - r * D;
        const int hq = h * G + r;
        const size_t row0 = ((size_t)b * a.Hq + hq) * n_splits;
        float Mx = -INFINITY;
        for (int s = 0; s < n_splits; ++s) Mx = fmaxf(Mx, load_coherent(part_ml + (row0 + s) * 2));
        const float Mb = Mx == -INFINITY ? 0.0f : Mx;
        float num = 0.0f, den = 0.0f;
        for (int s = 0; s < n_splits; ++s) {
            const float f = __builtin_amdgcn_exp2f(load_coherent(part_ml + (row0 + s) * 2) - Mb);
            num = fmaf(load_coherent(part_acc + (row0 + s) * D + d), f, num);
            den = fmaf(load_coherent(part_ml + (row0 + s) * 2 + 1), f, den);
        }
        float* orow = (float*)((char*)a.out + b * a.o_nb_b + hq * a.o_nb_h);
        orow[d] = den > 0.0f ? num / den : 0.0f;
    }
    if (tid == 0) __hip_atomic_store(a.tickets + bh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

bool decode_step_supported(const StepArgs& a) {
    if (a.cache_type != VVA_TYPE_F16 && a.cache_type != VVA_TYPE_BF16) return false;
    if (a.d != 64 && a.d != 128) return false;
    if (a.Hq % a.Hkv || a.Hq / a.Hkv > kMaxG) return false;
    if (a.B * a.Hkv > kMaxStepTickets) return false;
    for (int b = 0; b < a.B; ++b) {
        if (a.past[b] + 1 > kKPW * kMaxStepSplits) return false;
        if ((uintptr_t)a.kc[b] % 16 || (uintptr_t)a.vc[b] % 16) return false;
    }
    return a.cache_row_bytes % 16 == 0 && a.cache_head_bytes % 16 == 0;
}

int decode_step_splits(const StepArgs& a) {
    int Lmax = 1;
    for (int b = 0; b < a.B; ++b) Lmax = max(Lmax, a.past[b] + 1);
    return (Lmax + kKPW - 1) / kKPW;
}

hipError_t launch_decode_step(const StepArgs& a, int n_splits, hipStream_t s) {
    const dim3 grid(n_splits, a.B * a.Hkv), block(256);
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
