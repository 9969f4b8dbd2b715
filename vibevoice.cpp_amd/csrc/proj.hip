// proj.hip — the linear layers on either side of the attention, on CDNA4
// MFMA, with their neighbouring elementwise ops fused into the epilogue:
//   * q/k/v projections (linear(): ggml_mul_mat + bias, src/qwen2.cpp:19-25,
//     :273-275), NeoX RoPE of q and k (:282-287) and the append of k and v to
//     the resident cache (:293-306) — one GEMM over the stacked weights whose
//     epilogue writes RoPE(q) and the cache rows;
//   * the output projection plus the residual add (src/qwen2.cpp:348-349).
//
// Numerics follow ggml's CPU mul_mat: x is first converted to the weight's
// vec-dot type by proj_prep_kernel (F16 weights: x rounded to f16; Q8_0
// weights: x quantized to Q8_0 blocks, kept as f16 d_x * q values), then
// every product of f16 operands is exact in the fp32 MFMA accumulators.
// Q8_0 weight blocks are dequantized to f16 d_w * q values while the tile is
// staged in LDS.  (The two f16 roundings of d * q are the only departure from
// ggml's integer block sums; each is below 2^-12 relative.)
//
// GEMM.  D[m][n] = sum_k W[m][k] X[n][k]: m = output feature, n = token row
// (b * T + t), k = input feature.  A workgroup computes a 128 x 128 tile
// over k in steps of 64 with 4 waves, each a 64 x 64 quadrant of 2 x 2
// v_mfma_f32_32x32x16_f16 blocks.  Both operands are k-contiguous rows, so
// every MFMA fragment is one 16-byte LDS read; rows are padded to 144 bytes
// (16 mod 256: conflict-free fragment reads).  Tiles are staged through
// registers into two LDS stages (the loads of tile j + 1 fly while tile j is
// computed); the compiler tracks every load.  Workgroups are ordered so that
// each XCD (workgroups are dealt to the 8 XCDs round-robin) walks a
// contiguous run of tiles: the 36 weight tiles of one token tile share its
// X tile in that XCD's L2.
//
// Few token rows (a decode step: B * T <= 8).  The GEMM's 128-row token tile
// would be almost empty and its 36 workgroups too few to stream the weights,
// so proj_gemv_kernel reads each weight row once, one wave of 4 rows per
// workgroup (1152 workgroups for the 7B q/k/v stack, evenly spread over the
// CUs), all of a lane's weight loads in flight before any is used: F16
// weights with v_dot2 on the f16-rounded x, Q8_0 weights with integer
// v_dot4 block sums times d_w * d_x (ggml's Q8_0 x Q8_0 block dot, x
// quantized by the lane that uses the block).  The token rows are read from
// the layer input directly (L2-resident).  The q/k/v variant writes the F32
// projections, which the RoPE + append kernel then rotates and stores.
//
// Epilogue.  The accumulators go through LDS as a [token][feature] tile, so
// the epilogue threads see whole head rows: bias, then the NeoX rotation of
// pair (i, i + d/2) with the token's (cos, sin) row written by the prep
// kernel (the fp32 theta recurrence of rope_append.hip), then stores in the
// q_out / cache types (Q8_0 rows quantized per 32-dim block).
#include "vva_internal.hpp"

namespace vva {

namespace {

#include "wave_ops.hpp"

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kTM = 128;                    // output features per tile
constexpr int kTN = 128;                    // token rows per tile
constexpr int kTK = 64;                     // inputs per k step
constexpr int kPitch = kTK * 2 + 16;        // LDS bytes per operand row
constexpr int kOpBytes = 128 * kPitch;      // one operand tile: 18,432
constexpr int kStage = 2 * kOpBytes;        // A (weights) then B (x)
constexpr int kCPitch = kTM + 4;            // floats per token row of the epilogue tile
static_assert(2 * kStage >= kTN * kCPitch * 4 + 16, "the epilogue tile (and the split ticket flag) reuse the two stages");

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// ---- q/k/v epilogue with vector stores.  The tile's C (TN tokens x TM
// features, cpitch floats per token row): each thread keeps one 8-feature
// chunk of the tile and walks its tokens; it adds the bias, rotates q and k
// (NeoX pairs i, i + P, the RoPE table's (cos, sin) of the token), and
// stores the 8 results as one 16-byte (f16 / bf16) or two (f32) stores.
// One element per lane and store instruction would issue one lane per cycle.
// The arithmetic per element is the pair epilogue's.
template <int TM, int TN, int NTH>
__device__ __forceinline__ void qkv_epilogue_vec(const ProjArgs& a, const float* C, int cpitch, int m0, int n0, int tid) {
    constexpr int CPT = TM / 8;                        // chunks per token row of the tile
    static_assert(NTH % CPT == 0, "a thread keeps its chunk");
    constexpr int TPP = NTH / CPT;                     // tokens per pass
    constexpr int EB = 4;                              // passes whose RoPE loads go out together
    const int d = a.d, P = d >> 1;
    const int c = tid % CPT, f = c * 8;
    const int hl = f / d, i0 = f - hl * d;             // head within the tile, its first dim
    const int f0 = m0 + hl * d;
    if (f0 >= a.M) return;                             // past the last matrix
    const int mat = f0 < a.m_end[0] ? 0 : (f0 < a.m_end[1] ? 1 : 2);
    const int mrow = f0 - (mat == 0 ? 0 : mat == 1 ? a.m_end[0] : a.m_end[1]);
    const int head = mrow / d;
    const bool lo = i0 < P;                            // first halves of the rotation pairs
    const int ip = lo ? i0 + P : i0 - P;               // the partners' first dim
    const int j0 = lo ? i0 : ip;                       // pair index of the first dim
    const float* bias = mat == 0 ? a.bias[0] : mat == 1 ? a.bias[1] : a.bias[2];
    float bs[8], bp[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        bs[e] = bias ? bias[mrow + i0 + e] : 0.0f;
        bp[e] = bias ? bias[mrow + ip + e] : 0.0f;
    }
    const int dt = mat == 0 ? a.q_out_type : a.cache_type;
    const int64_t es = type_elem_bytes(dt);
    const bool one_seq = a.N == a.T;
    for (int nb = tid / CPT; nb < TN; nb += TPP * EB) {
        float4 csr[EB][4];                             // (cos, sin) of pairs j0 .. j0 + 7
#pragma unroll
        for (int e = 0; e < EB; ++e) {
            const float4* rp = (const float4*)(a.rope + (int64_t)min(n0 + nb + TPP * e, a.N - 1) * P + j0);
#pragma unroll
            for (int q = 0; q < 4; ++q) csr[e][q] = rp[q];
        }
#pragma unroll
        for (int e = 0; e < EB; ++e) {
            const int nl = nb + TPP * e, n = n0 + nl;
            if (nl >= TN || n >= a.N) break;
            const float* cr = C + nl * cpitch + hl * d;
            // the chunk and its partners' chunk as 16-byte reads (the row
            // pitch, d and i0 keep them 16-byte aligned): 8 scalar reads at a
            // 32-byte lane stride would meet on the same banks
            float yv[8], qv[8];
            *(float4*)&yv[0] = *(const float4*)(cr + i0);
            *(float4*)&yv[4] = *(const float4*)(cr + i0 + 4);
            *(float4*)&qv[0] = *(const float4*)(cr + ip);
            *(float4*)&qv[4] = *(const float4*)(cr + ip + 4);
            float out[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const float y = yv[k] + bs[k], yq = qv[k] + bp[k];
                const float cs = (k & 1) ? csr[e][k >> 1].z : csr[e][k >> 1].x;
                const float sn = (k & 1) ? csr[e][k >> 1].w : csr[e][k >> 1].y;
                // pair (y0, y1) = (dim j, dim j + P): lo threads hold y0
                out[k] = mat == 2 ? y : (lo ? fmaf(y, cs, -(yq * sn)) : fmaf(yq, sn, y * cs));
            }
            const int b = one_seq ? 0 : n / a.T, t = n - b * a.T;
            char* dst;
            if (mat == 0) {
                dst = a.q_out + b * a.qo_nb_b + t * a.qo_nb_t + head * a.qo_nb_h + i0 * es;
            } else {
                char* const kd = one_seq ? a.k_dst[0] : a.k_dst[b];
                char* const vd = one_seq ? a.v_dst[0] : a.v_dst[b];
                dst = (mat == 1 ? kd : vd) + t * a.cache_row_bytes + head * a.cache_head_bytes + i0 * es;
            }
            if (dt == VVA_TYPE_F32) {
                *(float4*)dst = make_float4(out[0], out[1], out[2], out[3]);
                *(float4*)(dst + 16) = make_float4(out[4], out[5], out[6], out[7]);
            } else {
                const bool bf = dt == VVA_TYPE_BF16;
                uint32_t w4[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t x0 = bf ? f32_to_bf16(out[2 * k]) : f32_to_f16(out[2 * k]);
                    const uint32_t x1 = bf ? f32_to_bf16(out[2 * k + 1]) : f32_to_f16(out[2 * k + 1]);
                    w4[k] = x0 | (x1 << 16);
                }
                *(u32x4*)dst = u32x4{w4[0], w4[1], w4[2], w4[3]};
            }
        }
    }
}

// ---- split along K.  Each piece of a tile stores its accumulators (NW
// compute waves x 2 x 2 blocks of v_mfma_f32_32x32x16) as one block of the
// partial area, in the accumulators' own order [wave][block][4-register
// group][lane] so that every store instruction writes 1 KB of whole lines,
// with agent-scope (sc1) buffer stores: coherent across the XCDs' L2 caches
// without an L2 write-back.  After the stores have completed, thread 0 takes
// the tile's ticket; the last piece sums the pieces' blocks in split order
// (deterministic whatever the arrival order) into the epilogue's LDS tile C
// and resets the ticket for the next call.
constexpr int kSc1 = 16;                               // buffer cache policy: agent scope
// Epilogue passes whose loads go out together, before the batch's stores:
// vmcnt counts stores too, so a load waited for after a store waits for
// that store as well (a batch of 8 keeps the unrolled code small)
constexpr int kEpiQkv = 8, kEpiRes = 8;
template <int NW>
__device__ __forceinline__ void splitk_store(const f32x16 (&acc)[2][2], char* piece, int w, int lane) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(piece, (short)0, NW * 4096 * 4, 0x00020000);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const u32x4 v = {__float_as_uint(acc[i][j][4 * g]), __float_as_uint(acc[i][j][4 * g + 1]),
                                 __float_as_uint(acc[i][j][4 * g + 2]), __float_as_uint(acc[i][j][4 * g + 3])};
                __builtin_amdgcn_raw_buffer_store_b128(v, rs, (w * 16 + (i * 2 + j) * 4 + g) * 1024 + lane * 16, 0, kSc1);
            }
}
// Thread 0 takes the ticket (after every piece store of the workgroup has
// completed and a barrier); returns, to every thread, whether this piece is
// the tile's last.  `flag` is an int of LDS that nothing else uses meanwhile.
__device__ __forceinline__ bool splitk_ticket(unsigned* tk, int ksplit, int* flag) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned old = __hip_atomic_fetch_add(tk, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag = old == (unsigned)(ksplit - 1);
        if (*flag) __hip_atomic_store(tk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    return *flag != 0;
}
// C[token][feature] (cpitch floats per token row) = sum over the pieces of
// the tile, in split order; every thread of the workgroup (NT) takes part,
// FB float4s at a time with all their loads in flight.  WM: compute waves
// along the features (the wave's quadrant is wm = w % WM, wn = w / WM).
template <int NW, int NT, int WM, int FB>
__device__ __forceinline__ void splitk_sum(const char* piece0, int ksplit, float* C, int cpitch) {
    constexpr int PIECE = NW * 4096 * 4;
    constexpr int NF = NW * 1024 / NT;                 // float4s per thread
    static_assert(NF % FB == 0, "whole batches");
#pragma unroll
    for (int f0 = 0; f0 < NF; f0 += FB) {
        u32x4 v[FB][4];
#pragma unroll
        for (int e = 0; e < FB; ++e) {
            const int f = (int)threadIdx.x + NT * (f0 + e);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if (k >= ksplit) break;                // uniform
                const __amdgpu_buffer_rsrc_t rs =
                    __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(piece0) + (int64_t)k * PIECE, (short)0, PIECE, 0x00020000);
                v[e][k] = __builtin_amdgcn_raw_buffer_load_b128(rs, f * 16, 0, kSc1);
            }
        }
#pragma unroll
        for (int e = 0; e < FB; ++e) {
            const int f = (int)threadIdx.x + NT * (f0 + e);
            float4 s = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if (k >= ksplit) break;
                s.x += __uint_as_float(v[e][k].x);
                s.y += __uint_as_float(v[e][k].y);
                s.z += __uint_as_float(v[e][k].z);
                s.w += __uint_as_float(v[e][k].w);
            }
            const int w = f >> 10, gi = (f >> 6) & 15, lane = f & 63;
            const int i = gi >> 3, j = (gi >> 2) & 1, g = gi & 3;
            const int wm = w % WM, wn = w / WM, l32 = lane & 31, half = lane >> 5;
            *(float4*)(C + (wn * 64 + 32 * j + l32) * cpitch + wm * 64 + 32 * i + 4 * half + 8 * g) = s;
        }
    }
}

// ------------------------------------------------------------ prep

// One workgroup per token row n = b * T + t: the row in the weights'
// vec-dot type, as f16 (F16 weights: x rounded; Q8_0 weights: the Q8_0
// round trip, d * q with the fp16 d), and, for the q/k/v projections, the
// row's RoPE (cos, sin) pairs with the fp32 theta recurrence.
__global__ void __launch_bounds__(256) proj_prep_kernel(ProjPrepArgs a) {
    prefetch_kernargs<sizeof(ProjPrepArgs)>();
    const int n = blockIdx.x;
    const int b = n / a.T, t = n - b * a.T;
    const char* src = a.x + b * a.x_nb_b + t * a.x_nb_t;
    const int64_t es = type_elem_bytes(a.x_type);
    uint16_t* dst = a.xh + (int64_t)n * a.K;
    // 8 consecutive elements per thread; four threads make one 32-block.  A
    // 16-byte aligned row is read with vector loads, two passes' loads out
    // together (K <= 4096); otherwise element by element.
    const bool f32 = a.x_type == VVA_TYPE_F32, bf = a.x_type == VVA_TYPE_BF16;
    const bool vec = ((uintptr_t)src & 15) == 0;
    u32x4 raw[2][2];
    if (vec) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int k0 = min((int)threadIdx.x * 8 + 2048 * u, a.K - 8);
            raw[u][0] = *(const u32x4*)(src + k0 * es);
            raw[u][1] = *(const u32x4*)(src + k0 * es + (f32 ? 16 : 0));
        }
    }
    for (int k0 = threadIdx.x * 8, u = 0; k0 < a.K; k0 += 256 * 8, ++u) {
        float x[8];
        if (vec && u < 2) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t wd = raw[u][0][e / 2];
                const uint16_t v16 = (uint16_t)(e & 1 ? wd >> 16 : wd & 0xffffu);
                x[e] = f32 ? __uint_as_float(raw[u][e / 4][e % 4]) : (bf ? bf16_to_f32(v16) : f16_to_f32(v16));
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = load_elem(src + (k0 + e) * es, a.x_type);
        }
        uint16_t h[8];
        if (a.q8) {
            float am = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) am = fmaxf(am, fabsf(x[e]));
            am = fmaxf(am, __shfl_xor(am, 1, 4));
            am = fmaxf(am, __shfl_xor(am, 2, 4));
            const float d = am / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            const float dh = f16_to_f32(f32_to_f16(d));
#pragma unroll
            for (int e = 0; e < 8; ++e) h[e] = f32_to_f16(dh * roundf(x[e] * id));
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) h[e] = f32_to_f16(x[e]);
        }
        uint4 v;
        v.x = (uint32_t)h[0] | ((uint32_t)h[1] << 16);
        v.y = (uint32_t)h[2] | ((uint32_t)h[3] << 16);
        v.z = (uint32_t)h[4] | ((uint32_t)h[5] << 16);
        v.w = (uint32_t)h[6] | ((uint32_t)h[7] << 16);
        *(uint4*)(dst + k0) = v;
    }
    if (a.rope) {
        const float p = (float)a.pos[b * a.pos_stride_b + t];
        for (int i = threadIdx.x; i < a.P; i += 256) {
            const float th = rope_theta(p, a.theta_scale, i, a.P);
            a.rope[(int64_t)n * a.P + i] = make_float2(cosf(th), sinf(th));
        }
    }
}

// ------------------------------------------------------------ GEMM

// WQ8: Q8_0 weights (else F16).  MODE: kProjQKV or kProjResidual.
template <bool WQ8, int MODE>
__global__ void __launch_bounds__(256) proj_gemm_kernel(ProjArgs a) {
    prefetch_kernargs<sizeof(ProjArgs)>();
    __shared__ __attribute__((aligned(16))) char lds[2 * kStage];

    const int tid = threadIdx.x, lane = tid & 63, half = lane >> 5, l32 = lane & 31;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = w & 1, wn = w >> 1;             // the wave's 64 x 64 quadrant

    // Workgroup i runs on XCD i % 8; XCD x takes the contiguous run of tiles
    // [x * q + min(x, r), ...) of its c_x = q + (x < r) workgroups.
    const int n_mt = a.M / kTM, n_nt = (a.N + kTN - 1) / kTN;
    const int ksplit = a.ksplit, tail0 = a.tail0;
    int mt, nt, ks = 0, tile = 0;                             // tile: its ticket and partials
    if (ksplit > 1 && tail0 == 0) {
        // every tile split along K: the order walks (k piece, weight tile,
        // token tile), token tiles innermost, so that the workgroups an XCD
        // runs together share one weight slice in its L2
        const int q = gridDim.x / 8, r = gridDim.x % 8, x = blockIdx.x % 8;
        const int wo = x * q + min(x, r) + (int)blockIdx.x / 8;
        ks = wo / (n_nt * n_mt);
        mt = (wo / n_nt) % n_mt;
        nt = wo % n_nt;
        tile = mt * n_nt + nt;
    } else if (ksplit > 1 && (int)blockIdx.x >= tail0) {
        // the last round's tiles, split along K (after the unsplit ones)
        const int qq = (int)blockIdx.x - tail0, wo = tail0 + qq / ksplit;
        ks = qq % ksplit;
        tile = qq / ksplit;
        mt = wo % n_mt;
        nt = wo / n_mt;
    } else {
        const int hp = ksplit > 1 ? tail0 : (int)gridDim.x;
        const int q = hp / 8, r = hp % 8, x = blockIdx.x % 8;
        const int wo = x * q + min(x, r) + (int)blockIdx.x / 8;   // the XCD's contiguous run of the order
        mt = wo % n_mt;
        nt = wo / n_mt;
    }
    const bool split = ksplit > 1 && (tail0 == 0 || (int)blockIdx.x >= tail0);
    const int m0 = mt * kTM, n0 = nt * kTN;
    const int mat = m0 < a.m_end[0] ? 0 : (m0 < a.m_end[1] ? 1 : 2);
    const int mrow0 = m0 - (mat ? a.m_end[mat - 1] : 0);     // first row in its matrix
    const char* wbase = a.w[mat] + (int64_t)mrow0 * a.w_nb[mat];
    const int64_t wnb = a.w_nb[mat];

    // x rows past N read as zeros through the buffer range
    const __amdgpu_buffer_rsrc_t xrs = rsrc(a.xh + (int64_t)n0 * a.K, (uint32_t)(min(a.N - n0, kTN) * a.K * 2));
    const __amdgpu_buffer_rsrc_t wrs = rsrc(wbase, (uint32_t)(kTM * wnb));
    const int nk_all = a.K / kTK;
    const int nsp = split ? ksplit : 1;
    const int k_lo = ks * nk_all / nsp;
    const int nk = (ks + 1) * nk_all / nsp - k_lo;

    // per thread and k step: 4 x 16 bytes of B (and of an F16 A): chunk c =
    // tid + 256 i is row c / 8, 16-byte column c % 8
    u32x4 breg[4], areg[4];
    uint32_t qreg[9];
    auto load = [&](int kt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = tid + 256 * i, row = c >> 3, col = c & 7;
            breg[i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, (row * a.K + (k_lo + kt) * kTK) * 2 + col * 16, 0, 0);
        }
        if constexpr (!WQ8) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int c = tid + 256 * i, row = c >> 3, col = c & 7;
                areg[i] = __builtin_amdgcn_raw_buffer_load_b128(wrs, (uint32_t)(row * wnb) + (k_lo + kt) * kTK * 2 + col * 16, 0, 0);
            }
        } else {
            // block kt * 2 + (tid & 1) of row tid / 2: 34 bytes from the
            // 4-byte boundary at or below it (9 dwords; the block of an odd
            // index starts 2 bytes in, an even one's 9th dword is the next
            // block's scale, always inside the row)
            const uint32_t off = (uint32_t)((tid >> 1) * wnb) + (uint32_t)((k_lo + kt) * 2 + (tid & 1)) * kQ8Bytes;
#pragma unroll
            for (int i = 0; i < 9; ++i) qreg[i] = __builtin_amdgcn_raw_buffer_load_b32(wrs, (off & ~3u) + 4 * i, 0, 0);
        }
    };
    auto store = [&](int st) {
        char* sa = lds + st * kStage;
        char* sb = sa + kOpBytes;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = tid + 256 * i, row = c >> 3, col = c & 7;
            *(u32x4*)(sb + row * kPitch + col * 16) = breg[i];
        }
        if constexpr (!WQ8) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int c = tid + 256 * i, row = c >> 3, col = c & 7;
                *(u32x4*)(sa + row * kPitch + col * 16) = areg[i];
            }
        } else {
            const bool odd = tid & 1;                  // the block starts 2 bytes into dword 0
            const uint32_t dbits = odd ? (qreg[0] >> 16) : (qreg[0] & 0xffffu);
            _Float16 dh;
            const uint16_t d16 = (uint16_t)dbits;
            __builtin_memcpy(&dh, &d16, 2);
            const h2 dd = {dh, dh};
            uint32_t codes[8];                         // the 32 codes, 4 per dword
#pragma unroll
            for (int i = 0; i < 8; ++i) codes[i] = odd ? qreg[i + 1] : __builtin_amdgcn_alignbyte(qreg[i + 1], qreg[i], 2);
            uint32_t outw[16];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t c = codes[i];
                const h2 lo = {(_Float16)(int8_t)(c & 0xff), (_Float16)(int8_t)((c >> 8) & 0xff)};
                const h2 hi = {(_Float16)(int8_t)((c >> 16) & 0xff), (_Float16)(int8_t)(c >> 24)};
                const h2 plo = lo * dd, phi = hi * dd;   // exact product rounded once to f16
                __builtin_memcpy(&outw[2 * i], &plo, 4);
                __builtin_memcpy(&outw[2 * i + 1], &phi, 4);
            }
            char* dst = sa + (tid >> 1) * kPitch + (tid & 1) * 64;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                *(u32x4*)(dst + 16 * i) = u32x4{outw[4 * i], outw[4 * i + 1], outw[4 * i + 2], outw[4 * i + 3]};
        }
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

    load(0);
    store(0);
    if (nk > 1) load(1);
    __syncthreads();
    // fragment offsets within a stage: row l32 of each 32-row block, the
    // lane's 8-element k group
    const int a_rd = (wm * 64 + l32) * kPitch + half * 16;
    const int b_rd = kOpBytes + (wn * 64 + l32) * kPitch + half * 16;
    for (int kt = 0; kt < nk; ++kt) {
        const char* st = lds + (kt & 1) * kStage;
#pragma unroll
        for (int ks = 0; ks < kTK / 16; ++ks) {
            h8 af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const u32x4 ua = *(const u32x4*)(st + a_rd + i * 32 * kPitch + ks * 32);
                const u32x4 ub = *(const u32x4*)(st + b_rd + i * 32 * kPitch + ks * 32);
                __builtin_memcpy(&af[i], &ua, 16);
                __builtin_memcpy(&bf[i], &ub, 16);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) {
            store((kt + 1) & 1);      // that stage held tile kt - 1: every wave is past it
            if (kt + 2 < nk) load(kt + 2);
        }
        __syncthreads();
    }

    // ---- accumulators to LDS as C[token][feature]: lane (half, l32) of
    // block (i, j) holds features 8 (r / 4) + 4 half + r % 4 of token l32
    // (split along K: the tile's last piece sums every piece's partial there)
    float* C = (float*)lds;
    if (split) {
        constexpr int PIECE = 4 * 4096 * 4;
        splitk_store<4>(acc, a.part + ((int64_t)tile * ksplit + ks) * PIECE, w, lane);
        if (!splitk_ticket(a.tickets + tile, ksplit, (int*)(lds + 2 * kStage - 16))) return;
        splitk_sum<4, 256, 2, 8>(a.part + (int64_t)tile * ksplit * PIECE, ksplit, C, kCPitch);
    } else {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                float* crow = C + (wn * 64 + 32 * j + l32) * kCPitch + wm * 64 + 32 * i + 4 * half;
#pragma unroll
                for (int g = 0; g < 4; ++g)
                    *(float4*)(crow + 8 * g) = make_float4(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                                                           acc[i][j][4 * g + 3]);
            }
    }
    __syncthreads();

    if constexpr (MODE == kProjQKV) {
        if (a.vec_store) {
            qkv_epilogue_vec<kTM, kTN, 256>(a, C, kCPitch, m0, n0, tid);
            return;
        }
        // 64 rotation pairs per token (one head of d = 128, two of d = 64):
        // thread (token tid / 64 + 4 pass, pair tid % 64)
        const int d = a.d, P = d >> 1;
        const int pi = tid & 63, hl = pi / P, i = pi - hl * P;
        const int head = (mrow0 + hl * d) / d;
        const float* bias = a.bias[mat];
        const float b0 = bias ? bias[mrow0 + hl * d + i] : 0.0f;
        const float b1 = bias ? bias[mrow0 + hl * d + i + P] : 0.0f;
        // the batch's RoPE pairs loaded first (one memory round trip per batch)
        for (int nb = tid >> 6; nb < kTN; nb += 4 * kEpiQkv) {
            float2 csb[kEpiQkv];
#pragma unroll
            for (int e = 0; e < kEpiQkv; ++e)
                csb[e] = a.rope[(int64_t)min(n0 + nb + 4 * e, a.N - 1) * P + i];      // used for q and k only
#pragma unroll
            for (int e = 0; e < kEpiQkv; ++e) {
            const int nl = nb + 4 * e;
            const int n = n0 + nl;
            if (nl >= kTN || n >= a.N) break;              // wave-uniform
            float y0 = C[nl * kCPitch + hl * d + i] + b0;
            float y1 = C[nl * kCPitch + hl * d + i + P] + b1;
            if (mat < 2) {
                const float2 cs = csb[e];
                const float r0 = fmaf(y0, cs.x, -(y1 * cs.y));
                const float r1 = fmaf(y0, cs.y, y1 * cs.x);
                y0 = r0;
                y1 = r1;
            }
            const int b = a.N == a.T ? 0 : n / a.T, t = n - b * a.T;
            if (mat == 0) {
                const int64_t eo = type_elem_bytes(a.q_out_type);
                char* dst = a.q_out + b * a.qo_nb_b + t * a.qo_nb_t + head * a.qo_nb_h;
                store_elem(dst + i * eo, a.q_out_type, y0);
                store_elem(dst + (i + P) * eo, a.q_out_type, y1);
            } else {
                // (one sequence: constant indices, no indexed kernel-argument load per pass)
                char* const kd = a.N == a.T ? a.k_dst[0] : a.k_dst[b];
                char* const vd = a.N == a.T ? a.v_dst[0] : a.v_dst[b];
                char* row = (mat == 1 ? kd : vd) + t * a.cache_row_bytes + head * a.cache_head_bytes;
                if (a.cache_type == VVA_TYPE_Q8_0) {
                    store_q8_pair(row, i, P, y0, y1);
                } else {
                    const int64_t ec = type_elem_bytes(a.cache_type);
                    store_elem(row + i * ec, a.cache_type, y0);
                    store_elem(row + (i + P) * ec, a.cache_type, y1);
                }
            }
            }
        }
    } else {
        // h = y + x, 4 features per thread: thread (token tid / 32 + 8 pass,
        // features 4 (tid % 32) ..)
        const int c4 = (tid & 31) * 4;
        // the batch's residual rows loaded first (one memory round trip per batch)
        for (int nb = tid >> 5; nb < kTN; nb += 8 * kEpiRes) {
            float4 xrb[kEpiRes];
#pragma unroll
            for (int e = 0; e < kEpiRes; ++e) {
                const int n = min(n0 + nb + 8 * e, a.N - 1);
                const int b = a.N == a.T ? 0 : n / a.T, t = n - b * a.T;
                xrb[e] = *(const float4*)(a.res + b * a.res_nb_b + t * a.res_nb_t + (int64_t)(m0 + c4) * 4);
            }
#pragma unroll
            for (int e = 0; e < kEpiRes; ++e) {
                const int nl = nb + 8 * e;
                const int n = n0 + nl;
                if (nl >= kTN || n >= a.N) break;
                const int b = a.N == a.T ? 0 : n / a.T, t = n - b * a.T;
                const float4 xr = xrb[e];
                const float* cr = C + nl * kCPitch + c4;
                *(float4*)(a.h + b * a.h_nb_b + t * a.h_nb_t + (int64_t)(m0 + c4) * 4) =
                    make_float4(cr[0] + xr.x, cr[1] + xr.y, cr[2] + xr.z, cr[3] + xr.w);
            }
        }
    }
}

// ------------------------------------------------------------ wide GEMM (F16 weights)

// 256 output features x 128 token rows per workgroup, k in steps of 64.
// Eight producer waves DMA the tiles straight into a 3-stage LDS ring
// (buffer_load_dwordx4 ... lds).  From L2 one wave's LDS loads stream at
// ~20 GB/s whatever their number in flight, so eight issuing waves are what
// a CU needs to feed its matrix cores (~110 GB/s at this tile shape); the
// compute waves issue none, so they never wait behind a full load queue.
// Eight compute waves, two per SIMD, each own a 64 x 64 quadrant of 2 x 2
// v_mfma_f32_32x32x16_f16 blocks.  Rows are 128 bytes (64 f16 of k) in LDS;
// a DMA instruction fills 8 rows, and its lane l writes LDS 16-byte slot
// l % 8 of row l / 8 with the row's 16-byte k chunk (l % 8) ^ sw(row),
// sw(row) = (row / 2) % 8: a fragment read (16 lanes x 16 bytes per LDS
// cycle, rows r .. r + 15 at one k chunk) then touches every bank once.
constexpr int kWM = 256, kWN = 128, kWK = 64;
constexpr int kWStages = 3;
constexpr int kWA = kWM * kWK * 2;             // 32 KB of weights per stage
constexpr int kWB = kWN * kWK * 2;             // 16 KB of token rows per stage
constexpr int kWStage = kWA + kWB;
constexpr int kWCompute = 8, kWProd = 8;
constexpr int kWLoadsA = kWA / 1024 / kWProd;  // DMA loads per producer and stage
constexpr int kWLoadsB = kWB / 1024 / kWProd;
constexpr int kWLoads = kWLoadsA + kWLoadsB;
constexpr int kWCPitch = kWM + 4;              // floats per token row of the epilogue tile
static_assert(2 * kWLoads <= 63, "two stages of a producer's loads fit its 6-bit vmcnt");
static_assert(kWN * kWCPitch * 4 + 16 <= kWStages * kWStage, "the epilogue tile (and the split ticket flag) reuse the ring");

__device__ __forceinline__ void wdma16(i32x4 rsrc, uint32_t lds_addr, int voffset) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 4\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voffset), "s"(rsrc)
                 : "m0");
}
template <int N>
__device__ __forceinline__ void wwait_barrier() {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(N) : "memory");
}
__device__ __forceinline__ void wlds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory");
}

template <int MODE>
__global__ void __launch_bounds__((kWCompute + kWProd) * 64) proj_gemm_wide_kernel(ProjArgs a) {
    prefetch_kernargs<sizeof(ProjArgs)>();
    __shared__ __attribute__((aligned(16))) char lds[kWStages * kWStage];
    const int tid = threadIdx.x, lane = tid & 63, half = lane >> 5, l32 = lane & 31;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);

    // Workgroup i runs on XCD i % 8; XCD x takes the contiguous run of tiles
    // [x * q + min(x, r), ...) of an order that walks groups of 4 token
    // tiles, the 4 token tiles of every weight tile in turn: the tiles an
    // XCD runs at one time share few weight and token rows in its L2.
    const int n_mt = (a.M + kWM - 1) / kWM, n_nt = (a.N + kWN - 1) / kWN;
    const int ksplit = a.ksplit, tail0 = a.tail0;
    int mt, nt, ks = 0, tile = 0;                             // tile: its ticket and partials
    auto order = [&](int wo) {
        const int grp = wo / (n_mt * 4), gn = min(4, n_nt - grp * 4), j = wo - grp * n_mt * 4;
        mt = j / gn;
        nt = grp * 4 + j % gn;
    };
    if (ksplit > 1 && tail0 == 0) {
        // every tile split along K: the order walks (k piece, weight tile,
        // token tile), token tiles innermost, so that the workgroups an XCD
        // runs together share one weight slice in its L2
        const int q = gridDim.x / 8, r = gridDim.x % 8, x = blockIdx.x % 8;
        const int wo = x * q + min(x, r) + (int)blockIdx.x / 8;
        nt = wo % n_nt;
        mt = (wo / n_nt) % n_mt;
        ks = wo / (n_nt * n_mt);
        tile = mt * n_nt + nt;
    } else if (ksplit > 1 && (int)blockIdx.x >= tail0) {
        // the last round's tiles, split along K (after the unsplit ones)
        const int qq = (int)blockIdx.x - tail0;
        order(tail0 + qq / ksplit);
        ks = qq % ksplit;
        tile = qq / ksplit;
    } else {
        const int hp = ksplit > 1 ? tail0 : (int)gridDim.x;
        const int q = hp / 8, r = hp % 8, x = blockIdx.x % 8;
        order(x * q + min(x, r) + (int)blockIdx.x / 8);      // the XCD's contiguous run of the order
    }
    const bool split = ksplit > 1 && (tail0 == 0 || (int)blockIdx.x >= tail0);
    const int m0 = mt * kWM, n0 = nt * kWN;
    const int nk_all = a.K / kWK;
    const int nsp = split ? ksplit : 1;
    const int k_lo = ks * nk_all / nsp;
    const int nk = (ks + 1) * nk_all / nsp - k_lo;
    constexpr int PIECE = kWCompute * 4096 * 4;
    int* const split_flag = (int*)(lds + kWStages * kWStage - 16);
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;

    if (w >= kWCompute) {
        // ---- producers: chunks p, p + 2, ... of each operand's stage
        const int pw = w - kWCompute;
        const int sub = lane >> 3, slot = lane & 7;
        int aoff[kWLoadsA], boff[kWLoadsB];
        i32x4 ars[kWLoadsA];
#pragma unroll
        for (int i = 0; i < kWLoadsA; ++i) {
            const int row = (pw + kWProd * i) * 8 + sub;            // tile row of this lane
            const int g = m0 + (pw + kWProd * i) * 8;               // its 8-row group (one matrix)
            const int mat = g < a.m_end[0] ? 0 : (g < a.m_end[1] ? 1 : (g < a.m_end[2] ? 2 : 3));
            const int mbeg = mat == 0 ? 0 : a.m_end[mat - 1];
            const int mrows = mat < 3 ? a.m_end[mat] - mbeg : 0;
            ars[i] = make_rsrc_sgpr(mat < 3 ? a.w[mat] : a.w[0], (uint32_t)(mrows * a.w_nb[mat < 3 ? mat : 0]));
            const int mr = m0 + row - mbeg;
            aoff[i] = mr * (int)a.w_nb[mat < 3 ? mat : 0] + (((slot ^ ((row >> 1) & 7))) << 4);
        }
        const int nrows = min(a.N - n0, kWN);
        const i32x4 brs = make_rsrc_sgpr((const char*)(a.xh + (int64_t)n0 * a.K), (uint32_t)(nrows * a.K * 2));
#pragma unroll
        for (int i = 0; i < kWLoadsB; ++i) {
            const int row = (pw + kWProd * i) * 8 + sub;
            boff[i] = row * a.K * 2 + (((slot ^ ((row >> 1) & 7))) << 4);
        }
        // a stage past the last loads zeros (offsets past every range)
        auto issue = [&](int kt) {
            const uint32_t st = lds0 + (uint32_t)(kt % kWStages) * kWStage;
            const bool live = kt < nk;
            const int ko = (k_lo + kt) * kWK * 2;
#pragma unroll
            for (int i = 0; i < kWLoadsA; ++i)
                wdma16(ars[i], st + (pw + kWProd * i) * 1024, live ? aoff[i] + ko : 0x40000000);
#pragma unroll
            for (int i = 0; i < kWLoadsB; ++i)
                wdma16(brs, st + kWA + (pw + kWProd * i) * 1024, live ? boff[i] + ko : 0x40000000);
        };
        issue(0);
        issue(1);
        for (int kt = 0; kt < nk; ++kt) {
            wwait_barrier<kWLoads>();                      // T_kt: stage kt landed
            issue(kt + 2);                                 // into the stage of kt - 1
        }
        asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
        __syncthreads();                                   // every wave is done with the ring
        if (split) {
            if (!splitk_ticket(a.tickets + tile, ksplit, split_flag)) return;
            splitk_sum<kWCompute, (kWCompute + kWProd) * 64, 4, 4>(a.part + (int64_t)tile * ksplit * PIECE, ksplit,
                                                                 (float*)lds, kWCPitch);
        }
        __syncthreads();                                   // the epilogue tile is written
        return;
    }

    // ---- compute waves: quadrant (wm, wn) of 64 features x 64 tokens
    const int wm = w & 3, wn = w >> 2;
    const int sw = (l32 >> 1) & 7;
    const int a_rd = (wm * 64 + l32) * 128;
    const int b_rd = kWA + (wn * 64 + l32) * 128;
    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};
    for (int kt = 0; kt < nk; ++kt) {
        wlds_barrier();                                    // T_kt
        const char* st = lds + (kt % kWStages) * kWStage;
#pragma unroll
        for (int ks = 0; ks < kWK / 16; ++ks) {
            const int ch = ((2 * ks + half) ^ sw) << 4;
            h8 af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const u32x4 ua = *(const u32x4*)(st + a_rd + i * 32 * 128 + ch);
                const u32x4 ub = *(const u32x4*)(st + b_rd + i * 32 * 128 + ch);
                __builtin_memcpy(&af[i], &ua, 16);
                __builtin_memcpy(&bf[i], &ub, 16);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    }
    __syncthreads();                                       // every wave is done with the ring

    // ---- accumulators to LDS as C[token][feature]: lane (half, l32) of
    // block (i, j) holds features 8 (r / 4) + 4 half + r % 4 of token l32
    // (split along K: the tile's last piece sums every piece's partial there,
    // with the producer waves)
    float* C = (float*)lds;
    if (split) {
        splitk_store<kWCompute>(acc, a.part + ((int64_t)tile * ksplit + ks) * PIECE, w, lane);
        if (!splitk_ticket(a.tickets + tile, ksplit, split_flag)) return;
        splitk_sum<kWCompute, (kWCompute + kWProd) * 64, 4, 4>(a.part + (int64_t)tile * ksplit * PIECE, ksplit, C,
                                                             kWCPitch);
    } else {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                float* crow = C + (wn * 64 + 32 * j + l32) * kWCPitch + wm * 64 + 32 * i + 4 * half;
#pragma unroll
                for (int g = 0; g < 4; ++g)
                    *(float4*)(crow + 8 * g) = make_float4(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                                                           acc[i][j][4 * g + 3]);
            }
    }
    __syncthreads();

    if constexpr (MODE == kProjQKV) {
        if (a.vec_store) {
            if (tid < kWCompute * 64) qkv_epilogue_vec<kWM, kWN, kWCompute * 64>(a, C, kWCPitch, m0, n0, tid);
            return;
        }
        // 128 rotation pairs per token (two heads of d = 128, four of d = 64):
        // thread (token tid / 128 + 4 pass, pair tid % 128)
        const int d = a.d, P = d >> 1;
        const int pi = tid & 127, hl = pi / P, i = pi - hl * P;
        const int f0 = m0 + hl * d;                        // first feature of the head
        if (f0 >= a.M) return;                             // past the last matrix (uniform per half-wave)
        const int mat = f0 < a.m_end[0] ? 0 : (f0 < a.m_end[1] ? 1 : 2);
        const int mrow = f0 - (mat ? a.m_end[mat - 1] : 0);
        const int head = mrow / d;
        const float* bias = a.bias[mat];
        const float b0 = bias ? bias[mrow + i] : 0.0f;
        const float b1 = bias ? bias[mrow + i + P] : 0.0f;
        // the batch's RoPE pairs loaded first (one memory round trip per batch)
        constexpr int PS = kWCompute * 64 / 128;          // token stride between passes
        for (int nb = tid >> 7; nb < kWN; nb += PS * kEpiQkv) {
            float2 csb[kEpiQkv];
#pragma unroll
            for (int e = 0; e < kEpiQkv; ++e)
                csb[e] = a.rope[(int64_t)min(n0 + nb + PS * e, a.N - 1) * P + i];     // used for q and k only
#pragma unroll
            for (int e = 0; e < kEpiQkv; ++e) {
            const int nl = nb + PS * e;
            const int n = n0 + nl;
            if (nl >= kWN || n >= a.N) break;              // uniform per wave
            float y0 = C[nl * kWCPitch + hl * d + i] + b0;
            float y1 = C[nl * kWCPitch + hl * d + i + P] + b1;
            if (mat < 2) {
                const float2 cs = csb[e];
                const float r0 = fmaf(y0, cs.x, -(y1 * cs.y));
                const float r1 = fmaf(y0, cs.y, y1 * cs.x);
                y0 = r0;
                y1 = r1;
            }
            const int b = a.N == a.T ? 0 : n / a.T, t = n - b * a.T;
            if (mat == 0) {
                const int64_t eo = type_elem_bytes(a.q_out_type);
                char* dst = a.q_out + b * a.qo_nb_b + t * a.qo_nb_t + head * a.qo_nb_h;
                store_elem(dst + i * eo, a.q_out_type, y0);
                store_elem(dst + (i + P) * eo, a.q_out_type, y1);
            } else {
                // (one sequence: constant indices, no indexed kernel-argument load per pass)
                char* const kd = a.N == a.T ? a.k_dst[0] : a.k_dst[b];
                char* const vd = a.N == a.T ? a.v_dst[0] : a.v_dst[b];
                char* row = (mat == 1 ? kd : vd) + t * a.cache_row_bytes + head * a.cache_head_bytes;
                if (a.cache_type == VVA_TYPE_Q8_0) {
                    store_q8_pair(row, i, P, y0, y1);
                } else {
                    const int64_t ec = type_elem_bytes(a.cache_type);
                    store_elem(row + i * ec, a.cache_type, y0);
                    store_elem(row + (i + P) * ec, a.cache_type, y1);
                }
            }
            }
        }
    } else {
        // h = y + x, 4 features per thread: thread (token tid / 64 + 8 pass,
        // features 4 (tid % 64) ..)
        const int c4 = (tid & 63) * 4;
        if (m0 + c4 >= a.M) return;
        // the batch's residual rows loaded first (one memory round trip per batch)
        for (int nb = tid >> 6; nb < kWN; nb += kWCompute * kEpiRes) {
            float4 xrb[kEpiRes];
#pragma unroll
            for (int e = 0; e < kEpiRes; ++e) {
                const int n = min(n0 + nb + kWCompute * e, a.N - 1);
                const int b = a.N == a.T ? 0 : n / a.T, t = n - b * a.T;
                xrb[e] = *(const float4*)(a.res + b * a.res_nb_b + t * a.res_nb_t + (int64_t)(m0 + c4) * 4);
            }
#pragma unroll
            for (int e = 0; e < kEpiRes; ++e) {
                const int nl = nb + kWCompute * e;
                const int n = n0 + nl;
                if (nl >= kWN || n >= a.N) break;
                const int b = a.N == a.T ? 0 : n / a.T, t = n - b * a.T;
                const float4 xr = xrb[e];
                const float* cr = C + nl * kWCPitch + c4;
                *(float4*)(a.h + b * a.h_nb_b + t * a.h_nb_t + (int64_t)(m0 + c4) * 4) =
                    make_float4(cr[0] + xr.x, cr[1] + xr.y, cr[2] + xr.z, cr[3] + xr.w);
            }
        }
    }
}

// ------------------------------------------------------------ big GEMM (F16 weights, long calls)

// 256 output features x 256 token rows per workgroup, k in steps of 64, eight
// waves (two per SIMD), each a 128 x 64 block of 4 x 2
// v_mfma_f32_32x32x16_f16 blocks whose 128 accumulators live in AGPRs: per
// k16 step a wave reads 6 fragments (6 KB of LDS) for 8 MFMAs, 3/4 of the LDS
// reads per MFMA of the wide kernel's 64 x 64 quadrants, whose fragment
// reads and DMA writes kept LDS saturated.  The waves DMA the tiles into a
// 2-stage LDS ring themselves (buffer_load_dwordx4 ... lds, 8 loads per wave
// and stage): eight issuing waves, since one wave's LDS loads stream at
// ~20 GB/s.  Rows are 128 bytes (64 f16 of k) in LDS, laid out as the
// wide kernel's: a DMA instruction fills 8 rows, lane l writing 16-byte slot
// l % 8 of row l / 8 with the row's k chunk (l % 8) ^ ((row / 2) % 8), so a
// fragment read (16 lanes, rows r .. r + 15 at one k chunk) touches every
// bank once.  Step kt: the MFMAs of each k16 quarter run while the next
// quarter's fragments are read; after the third quarter, the barrier that
// publishes stage kt + 1 (every wave has read all of stage kt by then, so
// stage kt takes the loads of kt + 2), the first fragments of kt + 1, and
// the fourth quarter's MFMAs.  (A 5-stage ring of 32-wide k steps, four
// stages in flight, measured slower: the loads' latency is not what the
// loop waits for.)  The epilogue runs in two halves of 128 tokens
// (the [token][feature] tile of 256 tokens would not fit LDS).
constexpr int kBM = 256, kBN = 256, kBK = 64;
constexpr int kBStages = 2;
constexpr int kBA = kBM * kBK * 2;             // 32 KB of weights per stage
constexpr int kBB = kBN * kBK * 2;             // 32 KB of token rows per stage
constexpr int kBStage = kBA + kBB;
constexpr int kBWaves = 8;
constexpr int kBLoadsA = kBA / 1024 / kBWaves;  // DMA loads per wave, operand and stage
constexpr int kBLoadsB = kBB / 1024 / kBWaves;
constexpr int kBLoads = kBLoadsA + kBLoadsB;
constexpr int kBHalf = kBN / 2;                 // tokens per epilogue half
constexpr int kBCPitch = kBM + 4;               // floats per token row of the epilogue tile
constexpr int kBRing = kBStages * kBStage;
constexpr int kBCBytes = kBHalf * kBCPitch * 4;
constexpr int kBLds = kBRing > kBCBytes ? kBRing : kBCBytes;
constexpr int kBPiece = kBWaves * 8 * 4096;     // bytes of one K piece's accumulators (256 x 256 f32)
constexpr int kBMaxSplit = 8;
constexpr int kBigMinRows = 1024;             // token rows from which the big GEMM runs (shorter: the wide one measured faster)
static_assert(kBStages == 2 && kBStages * kBLoads <= 63, "two stages of a wave's loads fit its 6-bit vmcnt");
static_assert(kBLds <= 160 * 1024, "LDS");

// q/k/v epilogue, one element pair per thread (Q8_0 caches, unaligned rows):
// NTH threads over the tile's TM / 2 rotation pairs of each token
template <int TN, int NTH>
__device__ __forceinline__ void qkv_epilogue_pair(const ProjArgs& a, const float* C, int cpitch, int m0, int n0, int tid) {
    constexpr int PAIRS = kBM / 2;                     // pairs per token of the tile
    constexpr int PS = NTH / PAIRS;                    // tokens per pass
    const int d = a.d, P = d >> 1;
    const int pi = tid % PAIRS, hl = pi / P, i = pi - hl * P;
    const int f0 = m0 + hl * d;                        // first feature of the head
    if (f0 >= a.M) return;                             // past the last matrix
    const int mat = f0 < a.m_end[0] ? 0 : (f0 < a.m_end[1] ? 1 : 2);
    const int mrow = f0 - (mat ? a.m_end[mat - 1] : 0);
    const int head = mrow / d;
    const float* bias = a.bias[mat];
    const float b0 = bias ? bias[mrow + i] : 0.0f;
    const float b1 = bias ? bias[mrow + i + P] : 0.0f;
    for (int nb = tid / PAIRS; nb < TN; nb += PS * kEpiQkv) {
        float2 csb[kEpiQkv];
#pragma unroll
        for (int e = 0; e < kEpiQkv; ++e)
            csb[e] = a.rope[(int64_t)min(n0 + nb + PS * e, a.N - 1) * P + i];      // used for q and k only
#pragma unroll
        for (int e = 0; e < kEpiQkv; ++e) {
            const int nl = nb + PS * e, n = n0 + nl;
            if (nl >= TN || n >= a.N) break;
            float y0 = C[nl * cpitch + hl * d + i] + b0;
            float y1 = C[nl * cpitch + hl * d + i + P] + b1;
            if (mat < 2) {
                const float2 cs = csb[e];
                const float r0 = fmaf(y0, cs.x, -(y1 * cs.y));
                const float r1 = fmaf(y0, cs.y, y1 * cs.x);
                y0 = r0;
                y1 = r1;
            }
            const int b = a.N == a.T ? 0 : n / a.T, t = n - b * a.T;
            if (mat == 0) {
                const int64_t eo = type_elem_bytes(a.q_out_type);
                char* dst = a.q_out + b * a.qo_nb_b + t * a.qo_nb_t + head * a.qo_nb_h;
                store_elem(dst + i * eo, a.q_out_type, y0);
                store_elem(dst + (i + P) * eo, a.q_out_type, y1);
            } else {
                char* const kd = a.N == a.T ? a.k_dst[0] : a.k_dst[b];
                char* const vd = a.N == a.T ? a.v_dst[0] : a.v_dst[b];
                char* row = (mat == 1 ? kd : vd) + t * a.cache_row_bytes + head * a.cache_head_bytes;
                if (a.cache_type == VVA_TYPE_Q8_0) {
                    store_q8_pair(row, i, P, y0, y1);
                } else {
                    const int64_t ec = type_elem_bytes(a.cache_type);
                    store_elem(row + i * ec, a.cache_type, y0);
                    store_elem(row + (i + P) * ec, a.cache_type, y1);
                }
            }
        }
    }
}

// h = y + x over a tile's TN tokens: 4 features per thread, NTH / 64 tokens per pass
template <int TN, int NTH>
__device__ __forceinline__ void residual_epilogue(const ProjArgs& a, const float* C, int cpitch, int m0, int n0, int tid) {
    constexpr int PS = NTH / (kBM / 4);
    const int c4 = (tid % (kBM / 4)) * 4;
    if (m0 + c4 >= a.M) return;
    for (int nb = tid / (kBM / 4); nb < TN; nb += PS * kEpiRes) {
        float4 xrb[kEpiRes];
#pragma unroll
        for (int e = 0; e < kEpiRes; ++e) {
            const int n = min(n0 + nb + PS * e, a.N - 1);
            const int b = a.N == a.T ? 0 : n / a.T, t = n - b * a.T;
            xrb[e] = *(const float4*)(a.res + b * a.res_nb_b + t * a.res_nb_t + (int64_t)(m0 + c4) * 4);
        }
#pragma unroll
        for (int e = 0; e < kEpiRes; ++e) {
            const int nl = nb + PS * e, n = n0 + nl;
            if (nl >= TN || n >= a.N) break;
            const int b = a.N == a.T ? 0 : n / a.T, t = n - b * a.T;
            const float4 xr = xrb[e];
            const float* cr = C + nl * cpitch + c4;
            *(float4*)(a.h + b * a.h_nb_b + t * a.h_nb_t + (int64_t)(m0 + c4) * 4) =
                make_float4(cr[0] + xr.x, cr[1] + xr.y, cr[2] + xr.z, cr[3] + xr.w);
        }
    }
}

// Tile order of the big GEMM: XCD x (workgroup i runs on XCD i % 8) takes a
// contiguous run of an order that walks groups of 4 token tiles, the 4 token
// tiles of every weight tile in turn.  Returns (weight tile, token tile) of
// place wo.
__device__ __forceinline__ int2 big_order(int wo, int n_mt, int n_nt) {
    const int grp = wo / (n_mt * 4), gn = min(4, n_nt - grp * 4), j = wo - grp * n_mt * 4;
    return make_int2(j / gn, grp * 4 + j % gn);
}

// A K piece's accumulators as [wave][block][4-register group][lane] (1 KB of
// whole lines per store instruction); a later launch sums them
__device__ __forceinline__ void big_split_store(const f32x16 (&acc)[4][2], char* piece, int w, int lane) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(piece, (short)0, kBPiece, 0x00020000);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const u32x4 v = {__float_as_uint(acc[i][j][4 * g]), __float_as_uint(acc[i][j][4 * g + 1]),
                                 __float_as_uint(acc[i][j][4 * g + 2]), __float_as_uint(acc[i][j][4 * g + 3])};
                __builtin_amdgcn_raw_buffer_store_b128(v, rs, (w * 32 + (i * 2 + j) * 4 + g) * 1024 + lane * 16, 0, 0);
            }
}

template <int MODE>
__global__ void __launch_bounds__(kBWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
proj_gemm_big_kernel(ProjArgs a) {
    prefetch_kernargs<sizeof(ProjArgs)>();
    __shared__ __attribute__((aligned(16))) char lds[kBLds];
    const int tid = threadIdx.x, lane = tid & 63, half = lane >> 5, l32 = lane & 31;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);

    // Tile order as in the wide kernel: XCD x (workgroup i runs on XCD i % 8)
    // takes a contiguous run of an order that walks groups of 4 token tiles,
    // the 4 token tiles of every weight tile in turn.
    const int n_mt = (a.M + kBM - 1) / kBM, n_nt = (a.N + kBN - 1) / kBN;
    const int ksplit = a.ksplit, tail0 = a.tail0;
    int ks = 0, tile = 0;
    int2 mn;
    if (ksplit > 1 && (int)blockIdx.x >= tail0) {
        // the last round's tiles, split along K (after the unsplit ones)
        const int qq = (int)blockIdx.x - tail0;
        mn = big_order(tail0 + qq / ksplit, n_mt, n_nt);
        ks = qq % ksplit;
        tile = qq / ksplit;
    } else {
        const int hp = ksplit > 1 ? tail0 : (int)gridDim.x;
        const int q = hp / 8, r = hp % 8, x = blockIdx.x % 8;
        mn = big_order(x * q + min(x, r) + (int)blockIdx.x / 8, n_mt, n_nt);
    }
    const int mt = mn.x, nt = mn.y;
    const bool split = ksplit > 1 && (int)blockIdx.x >= tail0;
    const int m0 = mt * kBM, n0 = nt * kBN;
    const int nk_all = a.K / kBK;
    const int nsp = split ? ksplit : 1;
    const int k_lo = ks * nk_all / nsp;
    const int nk = (ks + 1) * nk_all / nsp - k_lo;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;

    // ---- the wave's DMA loads: instructions w, w + 8, ... of each operand
    // (8 rows each); lane l takes row l / 8, LDS slot l % 8
    const int sub = lane >> 3, slot = lane & 7;
    // the k chunk that slot holds in row r of the tile
    auto chunk = [&](int r) { return (slot ^ ((r >> 1) & 7)) << 4; };
    int aoff[kBLoadsA], boff[kBLoadsB];
    i32x4 ars[kBLoadsA];
#pragma unroll
    for (int i = 0; i < kBLoadsA; ++i) {
        const int ins = w + kBWaves * i;
        const int g = m0 + ins * 8;                              // its 8-row group (one matrix)
        const int mat = g < a.m_end[0] ? 0 : (g < a.m_end[1] ? 1 : (g < a.m_end[2] ? 2 : 3));
        const int mbeg = mat == 0 ? 0 : a.m_end[mat - 1];
        const int mrows = mat < 3 ? a.m_end[mat] - mbeg : 0;
        ars[i] = make_rsrc_sgpr(mat < 3 ? a.w[mat] : a.w[0], (uint32_t)(mrows * a.w_nb[mat < 3 ? mat : 0]));
        aoff[i] = (g + sub - mbeg) * (int)a.w_nb[mat < 3 ? mat : 0] + chunk(ins * 8 + sub);
    }
    const int nrows = max(0, min(a.N - n0, kBN));
    const i32x4 brs = make_rsrc_sgpr((const char*)(a.xh + (int64_t)n0 * a.K), (uint32_t)(nrows * a.K * 2));
#pragma unroll
    for (int i = 0; i < kBLoadsB; ++i) {
        const int r = (w + kBWaves * i) * 8 + sub;
        boff[i] = r * a.K * 2 + chunk(r);
    }
    // a stage past the last loads zeros (offsets past every range)
    auto issue = [&](int kt, int stage) {
        const uint32_t st = lds0 + (uint32_t)stage * kBStage;
        const bool live = kt < nk;
        const int ko = (k_lo + kt) * kBK * 2;
#pragma unroll
        for (int i = 0; i < kBLoadsA; ++i)
            wdma16(ars[i], st + (w + kBWaves * i) * 1024, live ? aoff[i] + ko : 0x40000000);
#pragma unroll
        for (int i = 0; i < kBLoadsB; ++i)
            wdma16(brs, st + kBA + (w + kBWaves * i) * 1024, live ? boff[i] + ko : 0x40000000);
    };

    // ---- block (wm, wn): 128 features x 64 tokens
    const int wm = w & 1, wn = w >> 1;
    const int sw = (l32 >> 1) & 7;
    const int a_rd = (wm * 128 + l32) * 128;
    const int b_rd = kBA + (wn * 64 + l32) * 128;
    auto frags = [&](const char* st, int k16, h8 (&af)[4], h8 (&bf)[2]) {
        const int ch = ((2 * k16 + half) ^ sw) << 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4 ua = *(const u32x4*)(st + a_rd + i * 32 * 128 + ch);
            __builtin_memcpy(&af[i], &ua, 16);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const u32x4 ub = *(const u32x4*)(st + b_rd + j * 32 * 128 + ch);
            __builtin_memcpy(&bf[j], &ub, 16);
        }
    };
    f32x16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};
    auto mma = [&](const h8 (&af)[4], const h8 (&bf)[2]) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    };
    issue(0, 0);
    issue(1, 1);
    wwait_barrier<kBLoads>();                              // stage 0 landed
    // (scheduling fences keep this order: the compiler would otherwise read
    // each fragment just before its first MFMA and expose the LDS latency)
    h8 a0[4], b0[2], a1[4], b1[2];
    frags(lds, 0, a0, b0);
    for (int kt = 0; kt < nk; ++kt) {
        const char* st = lds + (kt & 1) * kBStage;
        frags(st, 1, a1, b1);
        __builtin_amdgcn_sched_barrier(0);
        mma(a0, b0);
        __builtin_amdgcn_sched_barrier(0);
        frags(st, 2, a0, b0);
        __builtin_amdgcn_sched_barrier(0);
        mma(a1, b1);
        __builtin_amdgcn_sched_barrier(0);
        frags(st, 3, a1, b1);
        __builtin_amdgcn_sched_barrier(0);
        mma(a0, b0);
        __builtin_amdgcn_sched_barrier(0);
        wwait_barrier<0>();                                // stage kt + 1 landed; stage kt read by all
        issue(kt + 2, kt & 1);                             // into stage kt's place
        frags(lds + ((kt + 1) & 1) * kBStage, 0, a0, b0);
        __builtin_amdgcn_sched_barrier(0);
        mma(a1, b1);
        __builtin_amdgcn_sched_barrier(0);
    }
    asm volatile("s_waitcnt vmcnt(0)" : : : "memory");     // the padding stages' zeros have landed
    __syncthreads();

    if (split) {                                           // proj_big_merge_kernel finishes the tile
        big_split_store(acc, a.part + ((int64_t)tile * ksplit + ks) * kBPiece, w, lane);
        return;
    }
    float* C = (float*)lds;
#pragma unroll 1
    for (int hh = 0; hh < 2; ++hh) {
        // ---- accumulators to LDS as C[token][feature] for tokens 128 hh ..:
        // lane (half, l32) of block (i, j) holds features 8 (r / 4) + 4 half +
        // r % 4 of token l32
        if ((wn >> 1) == hh) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    float* crow = C + ((wn & 1) * 64 + 32 * j + l32) * kBCPitch + wm * 128 + 32 * i + 4 * half;
#pragma unroll
                    for (int g = 0; g < 4; ++g)
                        *(float4*)(crow + 8 * g) = make_float4(acc[i][j][4 * g], acc[i][j][4 * g + 1],
                                                               acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
                }
        }
        __syncthreads();
        const int nh = n0 + kBHalf * hh;
        if constexpr (MODE == kProjQKV) {
            if (a.vec_store) qkv_epilogue_vec<kBM, kBHalf, kBWaves * 64>(a, C, kBCPitch, m0, nh, tid);
            else             qkv_epilogue_pair<kBHalf, kBWaves * 64>(a, C, kBCPitch, m0, nh, tid);
        } else {
            residual_epilogue<kBHalf, kBWaves * 64>(a, C, kBCPitch, m0, nh, tid);
        }
        __syncthreads();
    }
}

// The split tail of the big GEMM: one workgroup per (split tile, 32-token
// slab) sums the tile's K pieces for its slab, in split order, into a
// [token][feature] LDS tile and runs the epilogue on it.  A piece's slab s
// is the blocks j = s % 2 of waves wn = s / 2 (both wm), 32 KB.
constexpr int kBSlab = 32;
template <int MODE>
__global__ void __launch_bounds__(256) proj_big_merge_kernel(ProjArgs a) {
    prefetch_kernargs<sizeof(ProjArgs)>();
    __shared__ __attribute__((aligned(16))) float C[kBSlab * kBCPitch];
    const int n_mt = (a.M + kBM - 1) / kBM, n_nt = (a.N + kBN - 1) / kBN;
    constexpr int NS = kBN / kBSlab;
    const int tile = blockIdx.x / NS, slab = blockIdx.x % NS;
    const int2 mn = big_order(a.tail0 + tile, n_mt, n_nt);
    const int m0 = mn.x * kBM, n0 = mn.y * kBN + slab * kBSlab;
    if (n0 >= a.N) return;                                 // a slab past the tokens (uniform)
    const int tid = threadIdx.x;
    const int wn = slab >> 1, j = slab & 1;
    const char* piece0 = a.part + (int64_t)tile * a.ksplit * kBPiece;
    // float4 f of the slab: wm = f / 1024, i = (f / 256) % 4, g = (f / 64) % 4, lane = f % 64;
    // pieces summed in split order, four at a time with their loads in flight
    constexpr int NF = 2 * 4 * 4 * 64 / 256;               // float4s per thread
    constexpr int KB = 4;
    int off[NF];
    float4 s[NF];
#pragma unroll
    for (int e = 0; e < NF; ++e) {
        const int f = tid + 256 * e;
        const int wm = f >> 10, i = (f >> 8) & 3, g = (f >> 6) & 3, lane = f & 63;
        off[e] = ((2 * wn + wm) * 32 + (i * 2 + j) * 4 + g) * 1024 + lane * 16;
        s[e] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll 1
    for (int k0 = 0; k0 < a.ksplit; k0 += KB) {
        u32x4 v[NF][KB];
#pragma unroll
        for (int k = 0; k < KB; ++k) {
            if (k0 + k >= a.ksplit) break;                 // uniform
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<char*>(piece0) + (int64_t)(k0 + k) * kBPiece, (short)0, kBPiece, 0x00020000);
#pragma unroll
            for (int e = 0; e < NF; ++e) v[e][k] = __builtin_amdgcn_raw_buffer_load_b128(rs, off[e], 0, 0);
        }
#pragma unroll
        for (int k = 0; k < KB; ++k) {
            if (k0 + k >= a.ksplit) break;
#pragma unroll
            for (int e = 0; e < NF; ++e) {
                s[e].x += __uint_as_float(v[e][k].x);
                s[e].y += __uint_as_float(v[e][k].y);
                s[e].z += __uint_as_float(v[e][k].z);
                s[e].w += __uint_as_float(v[e][k].w);
            }
        }
    }
#pragma unroll
    for (int e = 0; e < NF; ++e) {
        const int f = tid + 256 * e;
        const int wm = f >> 10, i = (f >> 8) & 3, g = (f >> 6) & 3, lane = f & 63;
        const int l32 = lane & 31, half = lane >> 5;
        *(float4*)(C + l32 * kBCPitch + wm * 128 + 32 * i + 4 * half + 8 * g) = s[e];
    }
    __syncthreads();
    if constexpr (MODE == kProjQKV) {
        if (a.vec_store) qkv_epilogue_vec<kBM, kBSlab, 256>(a, C, kBCPitch, m0, n0, tid);
        else             qkv_epilogue_pair<kBSlab, 256>(a, C, kBCPitch, m0, n0, tid);
    } else {
        residual_epilogue<kBSlab, 256>(a, C, kBCPitch, m0, n0, tid);
    }
}

// ------------------------------------------------------------ GEMV

constexpr int kGvRows = 4;                       // output rows per workgroup (one wave)
constexpr int kGvMaxN = 8;                       // token rows
constexpr int kGvMaxK = 4096;                    // inputs
constexpr int kGvF16It = kGvMaxK / 8 / 64;       // 8-element chunks per lane and row
constexpr int kGvQ8It = kGvMaxK / 32 / 64;       // Q8_0 blocks per lane and row

// Elements k0 .. k0 + 7 of token row n = b * T + t of the layer input.
__device__ __forceinline__ void load_x8(const ProjArgs& a, int n, int k0, float (&x)[8]) {
    const int b = n / a.T, t = n - b * a.T;
    const char* src = a.x + b * a.x_nb_b + t * a.x_nb_t;
    if (a.x_type == VVA_TYPE_F32) {
        const float4 u0 = *(const float4*)(src + k0 * 4), u1 = *(const float4*)(src + k0 * 4 + 16);
        x[0] = u0.x; x[1] = u0.y; x[2] = u0.z; x[3] = u0.w;
        x[4] = u1.x; x[5] = u1.y; x[6] = u1.z; x[7] = u1.w;
    } else {
        const uint4 u = *(const uint4*)(src + k0 * 2);
        const uint32_t wv[4] = {u.x, u.y, u.z, u.w};
        const bool bf = a.x_type == VVA_TYPE_BF16;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint16_t lo = (uint16_t)(wv[e] & 0xffffu), hi = (uint16_t)(wv[e] >> 16);
            x[2 * e] = bf ? bf16_to_f32(lo) : f16_to_f32(lo);
            x[2 * e + 1] = bf ? bf16_to_f32(hi) : f16_to_f32(hi);
        }
    }
}
__device__ __forceinline__ uint32_t pack_f16(float lo, float hi) {
    return (uint32_t)f32_to_f16(lo) | ((uint32_t)f32_to_f16(hi) << 16);
}

// One wave: rows m0 .. m0 + 3 over every token row.  Lane l takes the
// 8-element chunks (F16) or Q8_0 blocks l, l + 64, ... of the rows: all its
// weight loads go out first, then it converts (F16: rounds to f16) or
// quantizes (Q8_0: ggml's quantize_row_q8_0, d = amax / 127 kept as fp16,
// codes round(x / d)) the matching elements of each token row once and uses
// them for all four rows.  The sums over lanes end in DPP reductions.
template <bool WQ8, int MODE>
__global__ void __launch_bounds__(64) proj_gemv_kernel(ProjArgs a) {
    prefetch_kernargs<sizeof(ProjArgs)>();
    const int lane = threadIdx.x;
    const int N = a.N, K = a.K;
    const int m0 = blockIdx.x * kGvRows;           // matrix boundaries are multiples of 128
    const int mat = m0 < a.m_end[0] ? 0 : (m0 < a.m_end[1] ? 1 : 2);
    const int mrow0 = m0 - (mat ? a.m_end[mat - 1] : 0);
    const char* wb = a.w[mat] + (int64_t)mrow0 * a.w_nb[mat];
    const int64_t wnb = a.w_nb[mat];
    float acc[kGvRows][kGvMaxN];
#pragma unroll
    for (int r = 0; r < kGvRows; ++r)
#pragma unroll
        for (int n = 0; n < kGvMaxN; ++n) acc[r][n] = 0.0f;

    if constexpr (!WQ8) {
        const int nch = K / 8;
        u32x4 wv[kGvF16It][kGvRows];
#pragma unroll
        for (int it = 0; it < kGvF16It; ++it) {
            const int c = lane + 64 * it;
            const int cc = c < nch ? c : 0;
#pragma unroll
            for (int r = 0; r < kGvRows; ++r) wv[it][r] = *(const u32x4*)(wb + r * wnb + (int64_t)cc * 16);
        }
#pragma unroll
        for (int it = 0; it < kGvF16It; ++it) {
            if (64 * it >= nch) break;                               // uniform
            const int c = lane + 64 * it;
            const bool live = c < nch;
#pragma unroll
            for (int n = 0; n < kGvMaxN; ++n) {
                if (n >= N) break;                                   // uniform
                float x[8];
                load_x8(a, n, (live ? c : 0) * 8, x);
                const uint32_t x0 = live ? pack_f16(x[0], x[1]) : 0u, x1 = live ? pack_f16(x[2], x[3]) : 0u;
                const uint32_t x2 = live ? pack_f16(x[4], x[5]) : 0u, x3 = live ? pack_f16(x[6], x[7]) : 0u;
#pragma unroll
                for (int r = 0; r < kGvRows; ++r) {
                    float s = acc[r][n];
                    s = dot2_f16(wv[it][r].x, x0, s);
                    s = dot2_f16(wv[it][r].y, x1, s);
                    s = dot2_f16(wv[it][r].z, x2, s);
                    s = dot2_f16(wv[it][r].w, x3, s);
                    acc[r][n] = s;
                }
            }
        }
    } else {
        // Q8_0 weight block j: 34 bytes from the 4-byte boundary at or below
        // it (rows are 4-byte aligned: K is a multiple of 64, so a row holds
        // an even number of blocks)
        const int nbk = K / 32;
        uint32_t qw[kGvQ8It][kGvRows][9];
#pragma unroll
        for (int it = 0; it < kGvQ8It; ++it) {
            const int j = lane + 64 * it;
            const int jj = j < nbk ? j : 0;
#pragma unroll
            for (int r = 0; r < kGvRows; ++r) {
                const uint32_t* p = (const uint32_t*)(wb + r * wnb + (((int64_t)jj * kQ8Bytes) & ~(int64_t)3));
#pragma unroll
                for (int i = 0; i < 9; ++i) qw[it][r][i] = p[i];
            }
        }
#pragma unroll
        for (int it = 0; it < kGvQ8It; ++it) {
            if (64 * it >= nbk) break;                               // uniform
            const int j = lane + 64 * it;
            const bool live = j < nbk;
            const int jj = live ? j : 0;
            const bool odd = jj & 1;                                 // the block starts 2 bytes into dword 0
            float dw[kGvRows];
            uint32_t codes[kGvRows][8];
#pragma unroll
            for (int r = 0; r < kGvRows; ++r) {
                const uint32_t* q = qw[it][r];
                dw[r] = live ? f16_to_f32((uint16_t)(odd ? q[0] >> 16 : q[0] & 0xffffu)) : 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i) codes[r][i] = odd ? q[i + 1] : __builtin_amdgcn_alignbyte(q[i + 1], q[i], 2);
            }
#pragma unroll
            for (int n = 0; n < kGvMaxN; ++n) {
                if (n >= N) break;                                   // uniform
                float x[32];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float xs[8];
                    load_x8(a, n, jj * 32 + 8 * q, xs);
#pragma unroll
                    for (int e = 0; e < 8; ++e) x[8 * q + e] = xs[e];
                }
                float am = 0.0f;
#pragma unroll
                for (int e = 0; e < 32; ++e) am = fmaxf(am, fabsf(x[e]));
                const float d = am / 127.0f;
                const float id = d != 0.0f ? 1.0f / d : 0.0f;
                const float dx = f16_to_f32(f32_to_f16(d));
                uint32_t xc[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    uint32_t c = 0u;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        c |= ((uint32_t)(uint8_t)(int8_t)roundf(x[4 * i + e] * id)) << (8 * e);
                    xc[i] = c;
                }
#pragma unroll
                for (int r = 0; r < kGvRows; ++r) {
                    int s = 0;
#pragma unroll
                    for (int i = 0; i < 8; ++i) s = __builtin_amdgcn_sdot4((int)codes[r][i], (int)xc[i], s, false);
                    acc[r][n] = fmaf((float)s, dw[r] * dx, acc[r][n]);
                }
            }
        }
    }

    // sums over the lanes; lane r * N + n keeps (row r, token n)
    float outv = 0.0f;
#pragma unroll
    for (int r = 0; r < kGvRows; ++r)
#pragma unroll
        for (int n = 0; n < kGvMaxN; ++n) {
            if (n >= N) break;                                       // uniform
            const float s = wave_sum(acc[r][n]);
            if (lane == r * N + n) outv = s;
        }
    if (lane < kGvRows * N) {
        const int r = lane / N, n = lane - r * N;
        const int m = m0 + r;
        if constexpr (MODE == kProjQKV) {
            const float* bias = a.bias[mat];
            a.y[(int64_t)n * a.M + m] = outv + (bias ? bias[mrow0 + r] : 0.0f);
        } else {
            const int b = n / a.T, t = n - b * a.T;
            const float xr = *(const float*)(a.res + b * a.res_nb_b + t * a.res_nb_t + (int64_t)m * 4);
            *(float*)(a.h + b * a.h_nb_b + t * a.h_nb_t + (int64_t)m * 4) = outv + xr;
        }
    }
}

// Raw bytes of elements k0 .. k0 + 7 (F16 / BF16: r[0]) or k0 .. k0 + 31
// (Q8_0 blocks: F32 r[0..7], 16-bit r[0..3]) of token row n, as loads the
// caller converts later (so that they stay in flight meanwhile).
template <int E>
__device__ __forceinline__ void load_x_raw(const ProjArgs& a, int n, int k0, u32x4 (&r)[E / 4]) {
    const int b = n / a.T, t = n - b * a.T;
    const char* src = a.x + b * a.x_nb_b + t * a.x_nb_t;
    if (a.x_type == VVA_TYPE_F32) {
#pragma unroll
        for (int i = 0; i < E / 4; ++i) r[i] = *(const u32x4*)(src + k0 * 4 + 16 * i);
    } else {
#pragma unroll
        for (int i = 0; i < E / 8; ++i) r[i] = *(const u32x4*)(src + k0 * 2 + 16 * i);
    }
}
template <int E>
__device__ __forceinline__ void x_from_raw(const ProjArgs& a, const u32x4 (&r)[E / 4], float (&x)[E]) {
    if (a.x_type == VVA_TYPE_F32) {
#pragma unroll
        for (int i = 0; i < E / 4; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) x[4 * i + e] = __uint_as_float(r[i][e]);
    } else {
        const bool bf = a.x_type == VVA_TYPE_BF16;
#pragma unroll
        for (int i = 0; i < E / 8; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint16_t lo = (uint16_t)(r[i][e] & 0xffffu), hi = (uint16_t)(r[i][e] >> 16);
                x[8 * i + 2 * e] = bf ? bf16_to_f32(lo) : f16_to_f32(lo);
                x[8 * i + 2 * e + 1] = bf ? bf16_to_f32(hi) : f16_to_f32(hi);
            }
    }
}

// The weight rows of a wave, as offsets from its slot's first row mrow0 (a
// multiple of 4 within its matrix).  kProjQKVRope: the slot's 4 rows are two
// NeoX rotation pairs of one head, dims 2w, 2w + 1, 2w + d/2 and 2w + d/2 + 1
// for the slot's index w in the head, so the wave holds both members of each
// pair; otherwise the slot's rows in order.
template <int MODE>
__device__ __forceinline__ void gemv_rofs(const ProjArgs& a, int mrow0, int (&ro)[kGvRows]) {
    if constexpr (MODE == kProjQKVRope) {
        const int P = a.d >> 1;
        const int hr = mrow0 & (a.d - 1);                   // d is 64 or 128
        const int w2 = 2 * (hr >> 2);
        ro[0] = w2 - hr;
        ro[1] = w2 + 1 - hr;
        ro[2] = w2 + P - hr;
        ro[3] = w2 + P + 1 - hr;
    } else {
#pragma unroll
        for (int r = 0; r < kGvRows; ++r) ro[r] = r;
    }
}
__device__ __forceinline__ int pick4(const int (&v)[kGvRows], int r) {
    return r == 0 ? v[0] : r == 1 ? v[1] : r == 2 ? v[2] : v[3];
}

// Output lane l = r N + n of a slot: row r, token row n; token row n =
// (sequence b, position t); MAXN = 2 (the decode step's one or two token
// rows) takes shifts and compares instead of integer divisions.
template <int MAXN>
__device__ __forceinline__ void lane_rn(int l, int N, int& r, int& n) {
    if constexpr (MAXN == 2) {
        r = N == 2 ? l >> 1 : l;
        n = N == 2 ? l & 1 : 0;
    } else {
        r = l / N;
        n = l - r * N;
    }
}
template <int MAXN>
__device__ __forceinline__ void tok_bt(const ProjArgs& a, int n, int& b, int& t) {
    if constexpr (MAXN == 2) {
        b = n >= a.T ? 1 : 0;
        t = n - b * a.T;
    } else {
        b = n / a.T;
        t = n - b * a.T;
    }
}

// What the output of lane (row r of the slot, token n = lane - r N) adds:
// its row's bias (kProjQKV, kProjQKVRope) or the residual (kProjResidual).
// Loaded before the weights, branch-free (lanes past the outputs and a
// missing bias read a valid address and add 0), so that it is not a second
// round trip at the end.
template <int MODE, int MAXN = kGvMaxN>
__device__ __forceinline__ float gemv_addend(const ProjArgs& a, int lane, int N, int m0, int mat, int mrow0,
                                             const char* any, const int (&ro)[kGvRows]) {
    const bool out = lane < kGvRows * N;
    const int l = out ? lane : 0;
    int r, n;
    lane_rn<MAXN>(l, N, r, n);
    if constexpr (MODE != kProjResidual) {
        const float* bias = mat == 0 ? a.bias[0] : mat == 1 ? a.bias[1] : a.bias[2];
        const float v = *(bias ? bias + mrow0 + pick4(ro, r) : (const float*)any);
        return out && bias ? v : 0.0f;
    } else {
        int b, t;
        tok_bt<MAXN>(a, n, b, t);
        const float v = *(const float*)(a.res + b * a.res_nb_b + t * a.res_nb_t + (int64_t)(m0 + r) * 4);
        return out ? v : 0.0f;
    }
}
template <int MODE, int MAXN = kGvMaxN>
__device__ __forceinline__ void gemv_store(const ProjArgs& a, int lane, int N, int m0, float v) {
    if (lane < kGvRows * N) {
        int r, n;
        lane_rn<MAXN>(lane, N, r, n);
        const int m = m0 + r;
        if constexpr (MODE == kProjQKV) {
            a.y[(int64_t)n * a.M + m] = v;
        } else {
            int b, t;
            tok_bt<MAXN>(a, n, b, t);
            *(float*)(a.h + b * a.h_nb_b + t * a.h_nb_t + (int64_t)m * 4) = v;
        }
    }
}
// kProjQKVRope, lane (r, n) of a slot: its output is dim 2w + (r & 1) (+ d/2
// for r >= 2) of the slot's head for token n.  Where it goes (q_out or the
// cache row), the token's position and the dim's angle index, found before
// the weight loads' wait so that none of it is a round trip at the end.
struct RopeLane {
    char* dst;
    int pos;                                                // 0 for v rows and without POS
    int i, r, n;                                            // angle index, slot row, token row
};
// arr[b] for b < NB, by selects of argument fields (no indexed load)
template <int NB>
__device__ __forceinline__ char* pick_ptr(char* const (&arr)[kMaxBatch], int b) {
    static_assert(NB <= kMaxBatch, "batch index range");
    char* p = arr[0];
#pragma unroll
    for (int i = 1; i < NB; ++i) p = b == i ? arr[i] : p;
    return p;
}
template <bool POS, int MAXN = kGvMaxN>
__device__ __forceinline__ RopeLane gemv_rope_lane(const ProjArgs& a, int lane, int N, int mat, int mrow0,
                                                   const int (&ro)[kGvRows]) {
    const bool out = lane < kGvRows * N;
    const int l = out ? lane : 0;
    int r, n, b, t;
    lane_rn<MAXN>(l, N, r, n);
    tok_bt<MAXN>(a, n, b, t);
    // d is 64 or 128; destinations are F32, F16 or BF16
    const int dim = (mrow0 & (a.d - 1)) + pick4(ro, r), head = mrow0 >> (a.d == 128 ? 7 : 6);
    const int qes = a.q_out_type == VVA_TYPE_F32 ? 4 : 2, ces = a.cache_type == VVA_TYPE_F32 ? 4 : 2;
    RopeLane o;
    o.pos = 0;
    if constexpr (POS) o.pos = mat < 2 ? a.pos[b * a.pos_stride_b + t] : 0;
    o.i = dim & ((a.d >> 1) - 1);
    o.r = r;
    o.n = n;
    if (mat == 0)
        o.dst = a.q_out + b * a.qo_nb_b + t * a.qo_nb_t + head * a.qo_nb_h + dim * qes;
    else
        o.dst = pick_ptr<MAXN>(mat == 1 ? a.k_dst : a.v_dst, b) + t * a.cache_row_bytes +
                head * a.cache_head_bytes + dim * ces;
    return o;
}
// kProjQKVRope epilogue: lane (r, n) holds projection + bias v and takes its
// partner's value (row r ^ 2, same token) across the wave.  q and k rows are
// rotated by the angle with cosine c and sine sn (the fp32 angle recurrence
// and operation order of rope_append.hip), so the stored values equal the
// GEMV + rope_append pair's; q goes to q_out, k and v to the cache rows
// (F32 / F16 / BF16).
__device__ __forceinline__ void gemv_rope_finish(const ProjArgs& a, int lane, int N, int mat, const RopeLane& rl,
                                                 float c, float sn, float v) {
    const bool out = lane < kGvRows * N;
    const float vp = __shfl(v, (rl.r ^ 2) * N + rl.n);
    if (!out) return;
    float y = v;
    if (mat < 2) {
        const bool hi = rl.r >= 2;
        const float x0 = hi ? vp : v, x1 = hi ? v : vp;
        y = hi ? fmaf(x0, sn, x1 * c) : fmaf(x0, c, -(x1 * sn));
    }
    store_elem(rl.dst, mat == 0 ? a.q_out_type : a.cache_type, y);
}
__device__ __forceinline__ void gemv_rope_store(const ProjArgs& a, int lane, int N, int mat, const RopeLane& rl,
                                                float v) {
    float c = 1.0f, sn = 0.0f;
    if (mat < 2) {
        const float th = rope_theta((float)rl.pos, a.theta_scale, rl.i, a.d >> 1);
        c = cosf(th);
        sn = sinf(th);
    }
    gemv_rope_finish(a, lane, N, mat, rl, c, sn, v);
}

// F16 weights, one or two token rows (the decode step), 8 weight rows per
// workgroup (2 waves of 4), NIT = ceil(K / 512) chunks of 8 per lane and row.
// Straight-line loads, so that every wait is exact: the token rows' chunks go
// out first, then all of the workgroup's weight loads; the token rows are
// rounded to f16 into LDS while the weights are in flight, and the dot loop
// takes chunk it as soon as it has landed (loads complete in order), so the
// arithmetic overlaps the rest of the stream.  Products and summation order
// are those of proj_gemv_kernel.
constexpr int kGvhWaves = 2;
constexpr int kGvhRows = kGvRows * kGvhWaves;
constexpr int kGvhN = 2;                                    // token rows
__device__ __forceinline__ void lds_barrier_only() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory");
}
template <int MODE, int NIT>
__global__ void __launch_bounds__(64 * kGvhWaves) proj_gemv_f16_kernel(ProjArgs a) {
    prefetch_kernargs<sizeof(ProjArgs)>();
    constexpr int NT = 64 * kGvhWaves;
    constexpr int XT = kGvhN * NIT * 64 / NT;                 // token-row chunks per thread
    __shared__ __attribute__((aligned(16))) uint32_t xh[kGvhN][NIT * 64][4];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int N = a.N, K = a.K, nch = K / 8, tasks = N * nch;
    // the wave's weight rows (selects, not an indexed kernel-argument load,
    // which would wait for the loads below)
    const int m0 = blockIdx.x * kGvhRows + wv * kGvRows;     // matrix boundaries are multiples of 128
    const int mat = m0 < a.m_end[0] ? 0 : (m0 < a.m_end[1] ? 1 : 2);
    const int mrow0 = m0 - (mat == 0 ? 0 : mat == 1 ? a.m_end[0] : a.m_end[1]);
    const int64_t wnb = mat == 0 ? a.w_nb[0] : mat == 1 ? a.w_nb[1] : a.w_nb[2];
    const char* wb = (mat == 0 ? a.w[0] : mat == 1 ? a.w[1] : a.w[2]) + (int64_t)mrow0 * wnb;
    int ro[kGvRows];
    gemv_rofs<MODE>(a, mrow0, ro);
    const float addend = gemv_addend<MODE>(a, lane, N, m0, mat, mrow0, wb, ro);
    RopeLane rl{};
    if constexpr (MODE == kProjQKVRope) rl = gemv_rope_lane<true>(a, lane, N, mat, mrow0, ro);
    // token-row chunk t = (n, c): 16 bytes, and for F32 rows the next 16
    // (16-bit rows load the same 16 bytes twice: no branch, no read past the row)
    const bool f32 = a.x_type == VVA_TYPE_F32;
    const int es = f32 ? 4 : 2;
    u32x4 xr[XT][2];
#pragma unroll
    for (int i = 0; i < XT; ++i) {
        // (n, c) and (b, t) without integer divisions (n < 2), which would
        // hold back the weight loads below
        const int t0 = tid + NT * i, t = t0 < tasks ? t0 : 0;
        const int n = t >= nch ? 1 : 0, c = t - n * nch;
        const int b = n >= a.T ? 1 : 0, tt = n - b * a.T;
        const char* src = a.x + b * a.x_nb_b + tt * a.x_nb_t + (int64_t)c * 8 * es;
        xr[i][0] = *(const u32x4*)src;
        xr[i][1] = *(const u32x4*)(src + (f32 ? 16 : 0));
    }
    u32x4 wq[NIT][kGvRows];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int c = lane + 64 * it;
        const int cc = c < nch ? c : 0;
#pragma unroll
        for (int r = 0; r < kGvRows; ++r) wq[it][r] = *(const u32x4*)(wb + ro[r] * wnb + (int64_t)cc * 16);
    }
    const bool bf = a.x_type == VVA_TYPE_BF16;
#pragma unroll
    for (int i = 0; i < XT; ++i) {
        const int t = tid + NT * i;
        // 16-bit rows: elements 2e, 2e + 1 sit in dword e of the first 16 bytes
        float y[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t h = xr[i][0][e / 2];
            const uint16_t v16 = (uint16_t)(e & 1 ? h >> 16 : h & 0xffffu);
            const float v = bf ? bf16_to_f32(v16) : f16_to_f32(v16);
            y[e] = f32 ? __uint_as_float(xr[i][e / 4][e % 4]) : v;
        }
        if (t < tasks) {
            const int n = t >= nch ? 1 : 0, c = t - n * nch;
            *(u32x4*)xh[n][c] = u32x4{pack_f16(y[0], y[1]), pack_f16(y[2], y[3]), pack_f16(y[4], y[5]), pack_f16(y[6], y[7])};
        }
    }
    lds_barrier_only();

    float acc[kGvRows][kGvhN];
#pragma unroll
    for (int r = 0; r < kGvRows; ++r)
#pragma unroll
        for (int n = 0; n < kGvhN; ++n) acc[r][n] = 0.0f;
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int c = lane + 64 * it;
        const bool live = c < nch;
#pragma unroll
        for (int n = 0; n < kGvhN; ++n) {
            // row n >= N: its LDS chunks were never written; its sums are not stored
            const u32x4 xv = *(const u32x4*)xh[n][c];
            const uint32_t x0 = live ? xv.x : 0u, x1 = live ? xv.y : 0u, x2 = live ? xv.z : 0u, x3 = live ? xv.w : 0u;
#pragma unroll
            for (int r = 0; r < kGvRows; ++r) {
                float s = acc[r][n];
                s = dot2_f16(wq[it][r].x, x0, s);
                s = dot2_f16(wq[it][r].y, x1, s);
                s = dot2_f16(wq[it][r].z, x2, s);
                s = dot2_f16(wq[it][r].w, x3, s);
                acc[r][n] = s;
            }
        }
    }

    // sums over the lanes; lane r * N + n keeps (row r, token n)
    float outv = 0.0f;
#pragma unroll
    for (int r = 0; r < kGvRows; ++r)
#pragma unroll
        for (int n = 0; n < kGvhN; ++n) {
            const float sum = wave_sum(acc[r][n]);
            if (n < N && lane == r * N + n) outv = sum;
        }
    if constexpr (MODE == kProjQKVRope) gemv_rope_store(a, lane, N, mat, rl, outv + addend);
    else gemv_store<MODE>(a, lane, N, m0, outv + addend);
}
template <int MODE>
hipError_t launch_gemv_f16(const ProjArgs& a, hipStream_t s) {
    const dim3 g(a.M / kGvhRows), bl(64 * kGvhWaves);
    switch ((a.K + 511) / 512) {
    case 1: hipLaunchKernelGGL((proj_gemv_f16_kernel<MODE, 1>), g, bl, 0, s, a); break;
    case 2: hipLaunchKernelGGL((proj_gemv_f16_kernel<MODE, 2>), g, bl, 0, s, a); break;
    case 3: hipLaunchKernelGGL((proj_gemv_f16_kernel<MODE, 3>), g, bl, 0, s, a); break;
    case 4: hipLaunchKernelGGL((proj_gemv_f16_kernel<MODE, 4>), g, bl, 0, s, a); break;
    case 5: hipLaunchKernelGGL((proj_gemv_f16_kernel<MODE, 5>), g, bl, 0, s, a); break;
    case 6: hipLaunchKernelGGL((proj_gemv_f16_kernel<MODE, 6>), g, bl, 0, s, a); break;
    case 7: hipLaunchKernelGGL((proj_gemv_f16_kernel<MODE, 7>), g, bl, 0, s, a); break;
    default: hipLaunchKernelGGL((proj_gemv_f16_kernel<MODE, 8>), g, bl, 0, s, a); break;
    }
    return hipGetLastError();
}

// Q8_0 weights, 16 rows per workgroup (4 waves of 4): every weight load of
// the workgroup goes out first, then its 256 threads quantize the token rows
// once into LDS (ggml's quantize_row_q8_0, as proj_gemv_kernel does per
// lane: the same codes and fp16-rounded scales), and each wave takes its 4
// rows' integer block dots against them.
constexpr int kGv8Waves = 4;
constexpr int kGv8Rows = kGvRows * kGv8Waves;
template <int MODE>
__global__ void __launch_bounds__(64 * kGv8Waves) proj_gemv_q8_kernel(ProjArgs a) {
    prefetch_kernargs<sizeof(ProjArgs)>();
    __shared__ __attribute__((aligned(16))) uint32_t xq[kGvMaxN][kGvMaxK / 32][8];   // codes of row n, block j
    __shared__ float xd[kGvMaxN][kGvMaxK / 32];         // their fp16-rounded scales
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int N = a.N, K = a.K, nbk = K / 32;
    const int m0 = blockIdx.x * kGv8Rows + wv * kGvRows; // matrix boundaries are multiples of 16
    // (selects, not an indexed kernel-argument load, which would wait for
    // the token-row loads below)
    const int mat = m0 < a.m_end[0] ? 0 : (m0 < a.m_end[1] ? 1 : 2);
    const int mrow0 = m0 - (mat == 0 ? 0 : mat == 1 ? a.m_end[0] : a.m_end[1]);
    const int64_t wnb = mat == 0 ? a.w_nb[0] : mat == 1 ? a.w_nb[1] : a.w_nb[2];
    const char* wb = (mat == 0 ? a.w[0] : mat == 1 ? a.w[1] : a.w[2]) + (int64_t)mrow0 * wnb;
    int ro[kGvRows];
    gemv_rofs<MODE>(a, mrow0, ro);
    const float addend = gemv_addend<MODE>(a, lane, N, m0, mat, mrow0, wb, ro);
    RopeLane rl{};
    if constexpr (MODE == kProjQKVRope) rl = gemv_rope_lane<true>(a, lane, N, mat, mrow0, ro);
    // this thread's first token-row block goes out ahead of the weights
    const int tasks = N * nbk;
    u32x4 xr0[8];
    {
        // row n = task / nbk and its (b, t) by comparisons (n < kGvMaxN):
        // integer divisions would hold back the weight loads below
        const int task = threadIdx.x < tasks ? (int)threadIdx.x : 0;
        int n = 0, b = 0;
#pragma unroll
        for (int k = 1; k < kGvMaxN; ++k) n += task >= k * nbk ? 1 : 0;
#pragma unroll
        for (int k = 1; k < kGvMaxN; ++k) b += n >= k * a.T ? 1 : 0;
        const int t = n - b * a.T, j = task - n * nbk;
        const char* src = a.x + b * a.x_nb_b + t * a.x_nb_t;
        const bool f32 = a.x_type == VVA_TYPE_F32;
        // 16-bit rows: the 64 bytes of the block, then the same 64 again
#pragma unroll
        for (int i = 0; i < 8; ++i)
            xr0[i] = *(const u32x4*)(src + (int64_t)j * 32 * (f32 ? 4 : 2) + 16 * (f32 ? i : i % 4));
    }
    // weight block j of each row: 34 bytes from the 4-byte boundary at or
    // below it (rows are 4-byte aligned: K is a multiple of 64)
    uint32_t qw[kGvQ8It][kGvRows][9];
#pragma unroll
    for (int it = 0; it < kGvQ8It; ++it) {
        const int j = lane + 64 * it;
        const int jj = j < nbk ? j : 0;
#pragma unroll
        for (int r = 0; r < kGvRows; ++r) {
            const uint32_t* p = (const uint32_t*)(wb + ro[r] * wnb + (((int64_t)jj * kQ8Bytes) & ~(int64_t)3));
#pragma unroll
            for (int i = 0; i < 9; ++i) qw[it][r][i] = p[i];
        }
    }
    for (int task = threadIdx.x; task < tasks; task += 64 * kGv8Waves) {
        const int n = task / nbk, j = task - n * nbk;
        u32x4 raw[8];
        if (task == (int)threadIdx.x) {
#pragma unroll
            for (int i = 0; i < 8; ++i) raw[i] = xr0[i];
        } else {
            load_x_raw<32>(a, n, j * 32, raw);
        }
        float x[32];
        x_from_raw<32>(a, raw, x);
        float am = 0.0f;
#pragma unroll
        for (int e = 0; e < 32; ++e) am = fmaxf(am, fabsf(x[e]));
        const float d = am / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            uint32_t c = 0u;
#pragma unroll
            for (int e = 0; e < 4; ++e) c |= ((uint32_t)(uint8_t)(int8_t)roundf(x[4 * i + e] * id)) << (8 * e);
            xq[n][j][i] = c;
        }
        xd[n][j] = f16_to_f32(f32_to_f16(d));
    }
    __syncthreads();

    float acc[kGvRows][kGvMaxN];
#pragma unroll
    for (int r = 0; r < kGvRows; ++r)
#pragma unroll
        for (int n = 0; n < kGvMaxN; ++n) acc[r][n] = 0.0f;
#pragma unroll
    for (int it = 0; it < kGvQ8It; ++it) {
        if (64 * it >= nbk) break;                                   // uniform
        const int j = lane + 64 * it;
        const bool live = j < nbk;
        const int jj = live ? j : 0;
        const bool odd = jj & 1;                                     // the block starts 2 bytes into dword 0
        float dw[kGvRows];
        uint32_t codes[kGvRows][8];
#pragma unroll
        for (int r = 0; r < kGvRows; ++r) {
            const uint32_t* q = qw[it][r];
            dw[r] = live ? f16_to_f32((uint16_t)(odd ? q[0] >> 16 : q[0] & 0xffffu)) : 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) codes[r][i] = odd ? q[i + 1] : __builtin_amdgcn_alignbyte(q[i + 1], q[i], 2);
        }
#pragma unroll
        for (int n = 0; n < kGvMaxN; ++n) {
            if (n >= N) break;                                       // uniform
            const u32x4 c0 = *(const u32x4*)&xq[n][jj][0], c1 = *(const u32x4*)&xq[n][jj][4];
            const uint32_t xc[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
            const float dx = xd[n][jj];
#pragma unroll
            for (int r = 0; r < kGvRows; ++r) {
                int s = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i) s = __builtin_amdgcn_sdot4((int)codes[r][i], (int)xc[i], s, false);
                acc[r][n] = fmaf((float)s, dw[r] * dx, acc[r][n]);
            }
        }
    }

    // sums over the lanes; lane r * N + n keeps (row r, token n)
    float outv = 0.0f;
#pragma unroll
    for (int r = 0; r < kGvRows; ++r)
#pragma unroll
        for (int n = 0; n < kGvMaxN; ++n) {
            if (n >= N) break;                                       // uniform
            const float sum = wave_sum(acc[r][n]);
            if (lane == r * N + n) outv = sum;
        }
    if constexpr (MODE == kProjQKVRope) gemv_rope_store(a, lane, N, mat, rl, outv + addend);
    else gemv_store<MODE>(a, lane, N, m0, outv + addend);
}

}  // namespace

bool proj_gemv_supported(int N, int K, int M) {
    return N >= 1 && N <= kGvMaxN && K <= kGvMaxK && K % 64 == 0 && M % kGvRows == 0;
}

// Sums over the wave of 4 values per lane at once, value k ending in every
// lane of 16 k .. 16 k + 15: lane halves exchanged by permlane32 swaps
// (values k and k + 2 meet), rows of 16 by a permlane16 swap, then a row
// rotation by 8 and 3 DPP steps within each row of 16; 10 exchanges and
// adds instead of 4 full butterflies.
__device__ __forceinline__ float sum4_rows(float w0, float w1) {
    // w0: lanes 0..31 carry value 0, lanes 32..63 value 2; w1: values 1, 3
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(w0), __float_as_uint(w1), false, false);
    float z = __uint_as_float(p[0]) + __uint_as_float(p[1]);   // row k of 16 carries value k
    z += dpp<0x128>(z);                                     // row_ror:8: lanes l and l ^ 8
    z += dpp<kDppXor1>(z);
    z += dpp<kDppXor2>(z);
    z += dpp<kDppHalfMirror>(z);
    return z;
}
__device__ __forceinline__ float wave_sum4(const float (&v)[4]) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[0]), __float_as_uint(v[2]), false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[1]), __float_as_uint(v[3]), false, false);
    return sum4_rows(__uint_as_float(a[0]) + __uint_as_float(a[1]), __uint_as_float(b[0]) + __uint_as_float(b[1]));
}
// The same where lanes 0..31 hold only values 0, 1 and lanes 32..63 only
// values 2, 3, as h[0], h[1] (the halves' partial sums need no exchange)
__device__ __forceinline__ float wave_sum4_halves(const float (&h)[2]) { return sum4_rows(h[0], h[1]); }

// Few-row GEMV with the weights streamed into LDS (the decode step's
// projections, one or two token rows).  A workgroup holds 2 (F16 weights)
// or 4 (Q8_0) staging waves, launched first, and up to kGlMaxSlots "slot"
// waves; slot wave w owns the 2 weight rows of slot blockIdx.x * SW + w: two
// consecutive rows, or under kProjQKVRope one NeoX rotation pair (dims i
// and i + d/2 of a head), so the wave holds both members of its pair.  Two
// rows per slot deal a 7B layer's rows to 256 workgroups evenly (q/k/v: 9
// slots each, o: 7).  The staging waves first issue the loads of the token
// rows (and positions), and only then, after barrier 0, do the slot waves
// issue every 1 KB chunk of their rows as buffer_load_dwordx4 ... nt lds into
// their own LDS area, chunk-major, so the token rows are not queued behind
// the weights and each CU has all of its rows' bytes in flight.  The staging
// waves convert the token rows once for the workgroup, rounded to f16 (F16
// weights) or quantized to Q8_0 blocks as ggml's quantize_row_q8_0 does
// (Q8_0 weights), and tabulate the RoPE cosines and sines of the tokens'
// positions, while the slot waves are still issuing; barrier 1.  A slot
// wave then takes each part of its rows as soon as the chunks under it have
// landed (loads complete in order: a vmcnt wait per part), so its dot
// products overlap the rest of the stream.  F16: part it is chunk it, lane l takes 8-element
// chunk l + 64 it of both rows, with the products of proj_gemv_f16_kernel.
// Q8_0: part it is blocks 32 it .. 32 it + 31, lanes 0..31 take row 0's
// blocks and lanes 32..63 row 1's, one whole block each (ggml's integer
// block dot, then one scaled fma).
constexpr int kGlRows = 2;                    // weight rows per slot (one wave)
constexpr int kGlMaxSlots = 12;
constexpr int kGlMaxXWaves = 4;
__host__ __device__ constexpr int gl_xwaves(bool q8) { return q8 ? 4 : 2; }   // Q8_0 quantizes: more hands
constexpr int kGlMaxTok = 2;                  // token rows
constexpr int kGlMaxK = 4096;
constexpr int kGlLdsMax = 160 * 1024;         // the whole of a CU's LDS (one workgroup per CU)
constexpr int kGlDead = 0x40000000;           // DMA offset past every range: zeros, no memory access

__device__ __forceinline__ void gldma16(i32x4 rsrc, uint32_t lds_addr, int voffset) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 4\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voffset), "s"(rsrc)
                 : "m0");
}
// s_waitcnt vmcnt(n) for a wave-uniform n in [0, 31]
__device__ __forceinline__ void wait_vmcnt_le(int n) {
    switch (n) {
#define VVA_W(I) case I: asm volatile("s_waitcnt vmcnt(" #I ")" : : : "memory"); break;
        VVA_W(0) VVA_W(1) VVA_W(2) VVA_W(3) VVA_W(4) VVA_W(5) VVA_W(6) VVA_W(7)
        VVA_W(8) VVA_W(9) VVA_W(10) VVA_W(11) VVA_W(12) VVA_W(13) VVA_W(14) VVA_W(15)
        VVA_W(16) VVA_W(17) VVA_W(18) VVA_W(19) VVA_W(20) VVA_W(21) VVA_W(22) VVA_W(23)
        VVA_W(24) VVA_W(25) VVA_W(26) VVA_W(27) VVA_W(28) VVA_W(29) VVA_W(30) VVA_W(31)
#undef VVA_W
        default: asm volatile("s_waitcnt vmcnt(0)" : : : "memory"); break;
    }
}

// LDS layout: [token rows: xbytes][RoPE table: kGlMaxTok x 64 (cos, sin)]
// [dummy 1 KB for dead loads][slot w: 2 rows x rp]
__host__ __device__ inline int gl_xbytes(bool q8, int K) {
    return q8 ? kGlMaxTok * (K + K / 32 * 4) : kGlMaxTok * K * 2;
}
__host__ __device__ inline int gl_row_pitch(bool q8, int K) {
    const int rb = q8 ? K / 32 * kQ8Bytes : K * 2;
    return (rb + 1023) / 1024 * 1024;
}
__host__ __device__ inline int gl_slots_at(bool q8, int K) { return gl_xbytes(q8, K) + 2048; }

// Output lane l = r N + n (N <= 2) of a slot: row r, token row n = (sequence
// b, position t), by compares (T is 1 with two sequences, or 2 with one).
struct GlLane {
    int r, n, b, t;
    bool out;
};
__device__ __forceinline__ GlLane gl_lane(const ProjArgs& a, int lane, int N) {
    GlLane o;
    o.out = lane < kGlRows * N;
    const int l = o.out ? lane : 0;
    o.r = N == 2 ? l >> 1 : l;
    o.n = N == 2 ? l & 1 : 0;
    o.b = o.n >= a.T ? 1 : 0;
    o.t = o.n - o.b * a.T;
    return o;
}
// The slot's rows as offsets from its first row mrow0: under kProjQKVRope
// dims i and i + d/2 of the head for the slot's index i in it, else the two
// rows in order.
template <int MODE>
__device__ __forceinline__ void gl_rofs(const ProjArgs& a, int mrow0, int (&ro)[kGlRows]) {
    if constexpr (MODE == kProjQKVRope) {
        const int hr = mrow0 & (a.d - 1);                   // d is 64 or 128; hr = 2 i
        ro[0] = (hr >> 1) - hr;
        ro[1] = (hr >> 1) + (a.d >> 1) - hr;
    } else {
        ro[0] = 0;
        ro[1] = 1;
    }
}
// What the output of lane L adds: its row's bias (kProjQKV, kProjQKVRope)
// or the residual (kProjResidual).  Loaded before the weights, branch-free
// (lanes past the outputs and a missing bias read a valid address and add 0).
template <int MODE>
__device__ __forceinline__ float gl_addend(const ProjArgs& a, const GlLane& L, int m0, int mat, int mrow0,
                                           const char* any, const int (&ro)[kGlRows]) {
    const int rr = L.r == 0 ? ro[0] : ro[1];
    if constexpr (MODE != kProjResidual) {
        const float* bias = mat == 0 ? a.bias[0] : mat == 1 ? a.bias[1] : a.bias[2];
        const float v = *(bias ? bias + mrow0 + rr : (const float*)any);
        return L.out && bias ? v : 0.0f;
    } else {
        const float v = *(const float*)(a.res + L.b * a.res_nb_b + L.t * a.res_nb_t + (int64_t)(m0 + L.r) * 4);
        return L.out ? v : 0.0f;
    }
}

// Staging of token-row tasks t = tid, tid + NT, ... (row n = t >= per, part
// c): E elements of row type XT, as loaded (F32: E / 4 vectors; 16-bit: the
// first E / 8), rounded to f16 (F16 weights) or quantized to a Q8_0 block
// (Q8_0 weights: ggml's quantize_row_q8_0, d = amax / 127 rounded to fp16,
// codes roundf(x / d) with the fp32 d) into LDS.
template <bool Q8, int XT, int E, int XI, int NT>
__device__ __forceinline__ void gl_stage(char* glds, const u32x4 (&raw)[XI][E / 4], int tid, int tasks, int per,
                                         int K) {
#pragma unroll
    for (int i = 0; i < XI; ++i) {
        const int t = tid + NT * i;
        if (t >= tasks) break;
        const int n = t >= per ? 1 : 0, c = t - n * per;
        float x[E];
        if constexpr (XT == VVA_TYPE_F32) {
#pragma unroll
            for (int e = 0; e < E; ++e) x[e] = __uint_as_float(raw[i][e / 4][e % 4]);
        } else {
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const uint32_t h = raw[i][e / 8][(e % 8) / 2];
                const uint16_t v16 = (uint16_t)(e & 1 ? h >> 16 : h & 0xffffu);
                x[e] = XT == VVA_TYPE_BF16 ? bf16_to_f32(v16) : f16_to_f32(v16);
            }
        }
        if constexpr (!Q8) {
            uint16_t* xh = (uint16_t*)glds;                 // [kGlMaxTok][K] f16
            *(u32x4*)(xh + (int64_t)n * K + c * 8) =
                u32x4{pack_f16(x[0], x[1]), pack_f16(x[2], x[3]), pack_f16(x[4], x[5]), pack_f16(x[6], x[7])};
        } else {
            uint32_t* xq = (uint32_t*)glds;                 // [kGlMaxTok][K / 32][8] codes
            float* xd = (float*)(glds + kGlMaxTok * K);     // [kGlMaxTok][K / 32] fp16-rounded scales
            float am = 0.0f;
#pragma unroll
            for (int e = 0; e < 32; ++e) am = fmaxf(am, fabsf(x[e]));
            const float d = am / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            uint32_t cw[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                cw[q] = 0u;
#pragma unroll
                for (int e = 0; e < 4; ++e) cw[q] |= ((uint32_t)(uint8_t)(int8_t)roundf(x[4 * q + e] * id)) << (8 * e);
            }
            *(u32x4*)(xq + ((int64_t)n * per + c) * 8) = u32x4{cw[0], cw[1], cw[2], cw[3]};
            *(u32x4*)(xq + ((int64_t)n * per + c) * 8 + 4) = u32x4{cw[4], cw[5], cw[6], cw[7]};
            xd[(int64_t)n * per + c] = f16_to_f32(f32_to_f16(d));
        }
    }
}

template <bool Q8, int MODE, int IPR>
__global__ void __launch_bounds__(64 * (kGlMaxSlots + kGlMaxXWaves)) proj_gemv_lds_kernel(ProjArgs a, int sw) {
    prefetch_kernargs<sizeof(ProjArgs) + 4>();
    __shared__ __attribute__((aligned(16))) char glds[kGlLdsMax];
    const int lane = threadIdx.x & 63;
    // waves 0 .. XW - 1 stage the token rows (launched first, their loads go
    // out first); wave XW + w is slot wave w
    constexpr int XW = gl_xwaves(Q8);
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int w = wv - XW;
    const int N = a.N, K = a.K;
    const int xbytes = gl_xbytes(Q8, K);
    float2* tab = (float2*)(glds + xbytes);                 // [kGlMaxTok][64]
    if (wv < XW) {
        // ---- staging waves: the token rows (and positions), once per workgroup
        constexpr int NT = XW * 64;
        constexpr int E = Q8 ? 32 : 8;                      // elements per task
        constexpr int XI = kGlMaxTok * (kGlMaxK / E) / NT;  // tasks per thread at most
        const int tid = threadIdx.x;
        const int per = K / E, tasks = N * per;
        // every load unconditional and back to back (no branch, no division:
        // n < 2): task t = (row n, part c) reads its E elements, F32 rows in
        // E / 4 vectors, 16-bit rows in E / 8 vectors read twice (no read past
        // the row); tasks past the end re-read task 0
        const bool f32 = a.x_type == VVA_TYPE_F32;
        const int eb = E * (f32 ? 4 : 2);
        const char* row0 = a.x;                             // token rows 0 and 1
        const char* row1 = a.x + (a.T == 1 ? a.x_nb_b : a.x_nb_t);
        u32x4 raw[XI][E / 4];
#pragma unroll
        for (int i = 0; i < XI; ++i) {
            const int t0 = tid + NT * i, t = t0 < tasks ? t0 : 0;
            const bool second = t >= per;
            const char* src = (second ? row1 : row0) + (uint32_t)((t - (second ? per : 0)) * eb);
#pragma unroll
            for (int q = 0; q < E / 4; ++q) raw[i][q] = *(const u32x4*)(src + 16 * (f32 ? q : q % (E / 8)));
        }
        const int P = a.d >> 1;
        int pv = 0;
        if constexpr (MODE == kProjQKVRope) {
            const int n = tid < N * P && tid >= P ? 1 : 0, b = n >= a.T ? 1 : 0, t = n - b * a.T;
            pv = a.pos[b * a.pos_stride_b + t];
        }
        asm volatile("s_barrier" : : : "memory");          // 0: the token-row loads are out
        // one code path per row type (a select between the types' decodes
        // would run both)
        if (f32) gl_stage<Q8, VVA_TYPE_F32, E, XI, NT>(glds, raw, tid, tasks, per, K);
        else if (a.x_type == VVA_TYPE_BF16) gl_stage<Q8, VVA_TYPE_BF16, E, XI, NT>(glds, raw, tid, tasks, per, K);
        else gl_stage<Q8, VVA_TYPE_F16, E, XI, NT>(glds, raw, tid, tasks, per, K);
        // the RoPE table (cos, sin of the tokens' angles), while the slot
        // waves are still issuing their loads
        if constexpr (MODE == kProjQKVRope) {
            if (tid < N * P) {
                const int n = tid >= P ? 1 : 0, i = tid - n * P;
                const float th = P == 64 ? rope_theta_n<64>((float)pv, a.theta_scale, i)
                                         : rope_theta_n<32>((float)pv, a.theta_scale, i);
                tab[n * 64 + i] = make_float2(cosf(th), sinf(th));
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory");   // 1: token rows and table staged
        return;
    }
    // ---- slot waves
    const int rb = Q8 ? K / 32 * kQ8Bytes : K * 2;          // weight row bytes
    const int rp = IPR * 1024;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)glds;
    const uint32_t dummy = lds0 + (uint32_t)xbytes + 1024;
    const int S = a.M / kGlRows;
    const int slot = blockIdx.x * sw + w;
    const bool has = slot < S;                              // wave-uniform
    const int m0 = (has ? slot : 0) * kGlRows;
    const int mat = m0 < a.m_end[0] ? 0 : (m0 < a.m_end[1] ? 1 : 2);
    const int mstart = mat == 0 ? 0 : mat == 1 ? a.m_end[0] : a.m_end[1];
    const int mrow0 = m0 - mstart;
    const int64_t wnb = mat == 0 ? a.w_nb[0] : mat == 1 ? a.w_nb[1] : a.w_nb[2];
    const char* wmat = mat == 0 ? a.w[0] : mat == 1 ? a.w[1] : a.w[2];
    int ro[kGlRows];
    gl_rofs<MODE>(a, mrow0, ro);
    const GlLane L = gl_lane(a, lane, N);
    const float addend = gl_addend<MODE>(a, L, m0, mat, mrow0, wmat, ro);
    const int sofs = gl_slots_at(Q8, K) + w * kGlRows * rp;
    asm volatile("s_barrier" : : : "memory");              // 0: the token-row loads are out
    {
        const i32x4 rs = make_rsrc_sgpr(wmat, (uint32_t)((a.m_end[mat] - mstart) * wnb));
#pragma unroll
        for (int c = 0; c < IPR; ++c)
#pragma unroll
            for (int r = 0; r < kGlRows; ++r) {
                const int b = c * 1024 + lane * 16;
                const bool live = has && c * 1024 < rb;     // wave-uniform
                const int off = b < rb ? (int)((mrow0 + ro[r]) * wnb) + b : kGlDead;
                gldma16(rs, live ? lds0 + (uint32_t)(sofs + r * rp + c * 1024) : dummy, live ? off : kGlDead);
            }
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory");   // 1: token rows staged
    if (!has) {
        asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
        return;
    }
    const char* srow = glds + sofs;
    float tot;
    if constexpr (!Q8) {
        // v[r * 2 + n]: this lane's partial sum of (row r, token n)
        float v[kGlRows * kGlMaxTok];
#pragma unroll
        for (int i = 0; i < kGlRows * kGlMaxTok; ++i) v[i] = 0.0f;
        const uint16_t* xh = (const uint16_t*)glds;
        const int nch = K / 8;
#pragma unroll
        for (int it = 0; it < IPR; ++it) {
            wait_vmcnt_le(kGlRows * (IPR - 1 - it));      // chunk it of both rows landed
            const int c = lane + 64 * it;
            if (c < nch) {
                u32x4 xv[kGlMaxTok];
#pragma unroll
                for (int n = 0; n < kGlMaxTok; ++n) xv[n] = *(const u32x4*)(xh + (int64_t)(n < N ? n : 0) * K + c * 8);
#pragma unroll
                for (int r = 0; r < kGlRows; ++r) {
                    const u32x4 wq = *(const u32x4*)(srow + r * rp + c * 16);
#pragma unroll
                    for (int n = 0; n < kGlMaxTok; ++n) {
                        float s2 = v[r * 2 + n];
                        s2 = dot2_f16(wq.x, xv[n].x, s2);
                        s2 = dot2_f16(wq.y, xv[n].y, s2);
                        s2 = dot2_f16(wq.z, xv[n].z, s2);
                        s2 = dot2_f16(wq.w, xv[n].w, s2);
                        v[r * 2 + n] = s2;
                    }
                }
            }
        }
        tot = wave_sum4(v);
    } else {
        // lanes 0..31: row 0, lanes 32..63: row 1; lane l takes whole block
        // 32 it + (l & 31) of its row
        const uint32_t* xq = (const uint32_t*)glds;
        const float* xd = (const float*)(glds + kGlMaxTok * K);
        const int nbk = K / 32;
        const char* row = srow + (lane >> 5) * rp;
        float acc[kGlMaxTok];
#pragma unroll
        for (int n = 0; n < kGlMaxTok; ++n) acc[n] = 0.0f;
        for (int it = 0; 32 * it < nbk; ++it) {
            // the part's last byte read: 9 dwords from below block jl's codes
            const int jl = min(32 * it + 31, nbk - 1);
            const int last = ((jl * kQ8Bytes + 2) & ~3) + 35;
            const int cl = min(last >> 10, IPR - 1);
            wait_vmcnt_le(kGlRows * (IPR - 1 - cl));
            const int j = 32 * it + (lane & 31);
            const bool live = j < nbk;
            const int jj = live ? j : 0;
            const int ca = (jj * kQ8Bytes + 2) & ~3;         // codes from this dword boundary
            const int sh = (jj * kQ8Bytes + 2) & 3;          // at this byte offset (0 or 2)
            const uint32_t sc = *(const uint32_t*)(row + ((jj * kQ8Bytes) & ~3));
            const float dw = f16_to_f32((uint16_t)((jj & 1) ? sc >> 16 : sc & 0xffffu));
            const uint32_t* q = (const uint32_t*)(row + ca);
            uint32_t qv[9], codes[8];
#pragma unroll
            for (int e = 0; e < 9; ++e) qv[e] = q[e];
#pragma unroll
            for (int e = 0; e < 8; ++e) codes[e] = __builtin_amdgcn_alignbyte(qv[e + 1], qv[e], sh);
#pragma unroll
            for (int n = 0; n < kGlMaxTok; ++n) {
                if (n >= N) break;                           // uniform
                const u32x4 c0 = *(const u32x4*)(xq + ((int64_t)n * nbk + jj) * 8);
                const u32x4 c1 = *(const u32x4*)(xq + ((int64_t)n * nbk + jj) * 8 + 4);
                const uint32_t xc[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
                const float dx = xd[(int64_t)n * nbk + jj];
                int sm = 0;
#pragma unroll
                for (int e = 0; e < 8; ++e) sm = __builtin_amdgcn_sdot4((int)codes[e], (int)xc[e], sm, false);
                const float f = fmaf((float)sm, dw * dx, acc[n]);
                acc[n] = live ? f : acc[n];
            }
        }
        tot = wave_sum4_halves(acc);
    }
    // (row r, token n) sums end in lanes 16 (2 r + n) .. + 15; lane r N + n takes its own
    const float outv = __shfl(tot, 16 * (L.r * 2 + L.n)) + addend;
    if constexpr (MODE == kProjQKVRope) {
        // the rotation partner (row r ^ 1, same token) across the wave
        const float vp = __shfl(outv, (L.r ^ 1) * N + L.n);
        const int dim = (mrow0 & (a.d - 1)) + (L.r == 0 ? ro[0] : ro[1]);
        const int head = mrow0 >> (a.d == 128 ? 7 : 6);
        float c = 1.0f, sn = 0.0f;
        if (mat < 2) {
            const float2 cs = tab[L.n * 64 + (dim & ((a.d >> 1) - 1))];
            c = cs.x;
            sn = cs.y;
        }
        if (!L.out) return;
        float y = outv;
        if (mat < 2) {
            const bool hi = L.r == 1;
            const float x0 = hi ? vp : outv, x1 = hi ? outv : vp;
            y = hi ? fmaf(x0, sn, x1 * c) : fmaf(x0, c, -(x1 * sn));
        }
        // destinations are F32, F16 or BF16
        char* dst;
        if (mat == 0) {
            dst = a.q_out + L.b * a.qo_nb_b + L.t * a.qo_nb_t + head * a.qo_nb_h +
                  dim * (a.q_out_type == VVA_TYPE_F32 ? 4 : 2);
        } else {
            char* base = mat == 1 ? (L.b ? a.k_dst[1] : a.k_dst[0]) : (L.b ? a.v_dst[1] : a.v_dst[0]);
            dst = base + L.t * a.cache_row_bytes + head * a.cache_head_bytes +
                  dim * (a.cache_type == VVA_TYPE_F32 ? 4 : 2);
        }
        store_elem(dst, mat == 0 ? a.q_out_type : a.cache_type, y);
    } else {
        if (!L.out) return;
        const int m = m0 + L.r;
        if constexpr (MODE == kProjQKV) {
            a.y[(int64_t)L.n * a.M + m] = outv;
        } else {
            *(float*)(a.h + L.b * a.h_nb_b + L.t * a.h_nb_t + (int64_t)m * 4) = outv;
        }
    }
}

// Slots per workgroup of proj_gemv_lds_kernel (0: the call does not fit it)
int gemv_lds_slots(const ProjArgs& a, int n_cu) {
    const bool q8 = a.w_type == VVA_TYPE_Q8_0;
    if (a.N > kGlMaxTok || a.K > kGlMaxK || a.K % 64 || a.M % kGlRows) return 0;
    if (a.mode == kProjQKVRope && a.d > 128) return 0;        // the RoPE table holds 64 angles
    // Q8_0: the last block's reads (9 dwords from below its codes) stay in the row pitch
    if (q8 && a.K / 32 * kQ8Bytes + 4 > gl_row_pitch(true, a.K)) return 0;
    if (a.m_end[0] % kGlRows || a.m_end[1] % kGlRows) return 0;
    for (int i = 0; i < 3; ++i) {                    // every row offset below the dead offset
        const int64_t rows = a.m_end[i] - (i == 0 ? 0 : a.m_end[i - 1]);
        if (rows > 0 && rows * a.w_nb[i] >= kGlDead) return 0;
    }
    const int rp = gl_row_pitch(q8, a.K);
    const int fit = (kGlLdsMax - gl_slots_at(q8, a.K)) / (kGlRows * rp);
    const int S = a.M / kGlRows;
    int sw = (S + n_cu - 1) / n_cu;
    if (sw > fit) sw = fit;
    if (sw > kGlMaxSlots) sw = kGlMaxSlots;
    return sw >= 1 ? sw : 0;
}

template <bool Q8, int MODE>
hipError_t launch_gemv_lds(const ProjArgs& a, int sw, hipStream_t s) {
    const int rp = gl_row_pitch(Q8, a.K);
    const dim3 g((a.M / kGlRows + sw - 1) / sw), bl(64 * (sw + gl_xwaves(Q8)));
    const int ipr = rp / 1024;
#define VVA_GL(I) case I: hipLaunchKernelGGL((proj_gemv_lds_kernel<Q8, MODE, I>), g, bl, 0, s, a, sw); break;
    switch (ipr) {
        VVA_GL(1) VVA_GL(2) VVA_GL(3) VVA_GL(4) VVA_GL(5) VVA_GL(6) VVA_GL(7) VVA_GL(8)
        default: return hipErrorInvalidValue;
    }
#undef VVA_GL
    return hipGetLastError();
}

namespace {
bool gemv_q8_ok(const ProjArgs& a) {
    return a.w_type == VVA_TYPE_Q8_0 && a.M % kGv8Rows == 0 && a.m_end[0] % kGv8Rows == 0 &&
           a.m_end[1] % kGv8Rows == 0;
}
bool gemv_f16_ok(const ProjArgs& a) {
    return a.w_type == VVA_TYPE_F16 && a.N <= kGvhN && a.M % kGvhRows == 0 && a.m_end[0] % kGvhRows == 0 &&
           a.m_end[1] % kGvhRows == 0;
}
}  // namespace

bool proj_gemv_rope_ok(const ProjArgs& a) {
    const bool float_cache = a.cache_type == VVA_TYPE_F32 || a.cache_type == VVA_TYPE_F16 ||
                             a.cache_type == VVA_TYPE_BF16;
    const bool float_q = a.q_out_type == VVA_TYPE_F32 || a.q_out_type == VVA_TYPE_F16 ||
                         a.q_out_type == VVA_TYPE_BF16;
    return a.mode == kProjQKV && float_cache && float_q && (a.d == 64 || a.d == 128) &&
           a.m_end[0] % a.d == 0 && a.m_end[1] % a.d == 0 &&
           (gemv_lds_slots(a, 1) > 0 || gemv_q8_ok(a) || gemv_f16_ok(a));
}

hipError_t launch_proj_gemv(ProjArgs& a, float* y_ws, int n_cu, hipStream_t s) {
    const bool q8 = a.w_type == VVA_TYPE_Q8_0;
    a.y = y_ws;
    if (const int sw = gemv_lds_slots(a, n_cu)) {
        if (q8) {
            if (a.mode == kProjQKVRope) return launch_gemv_lds<true, kProjQKVRope>(a, sw, s);
            if (a.mode == kProjQKV) return launch_gemv_lds<true, kProjQKV>(a, sw, s);
            return launch_gemv_lds<true, kProjResidual>(a, sw, s);
        }
        if (a.mode == kProjQKVRope) return launch_gemv_lds<false, kProjQKVRope>(a, sw, s);
        if (a.mode == kProjQKV) return launch_gemv_lds<false, kProjQKV>(a, sw, s);
        return launch_gemv_lds<false, kProjResidual>(a, sw, s);
    }
    if (gemv_q8_ok(a)) {
        const dim3 g8(a.M / kGv8Rows), b8(64 * kGv8Waves);
        if (a.mode == kProjQKVRope)  hipLaunchKernelGGL((proj_gemv_q8_kernel<kProjQKVRope>), g8, b8, 0, s, a);
        else if (a.mode == kProjQKV) hipLaunchKernelGGL((proj_gemv_q8_kernel<kProjQKV>), g8, b8, 0, s, a);
        else                         hipLaunchKernelGGL((proj_gemv_q8_kernel<kProjResidual>), g8, b8, 0, s, a);
        return hipGetLastError();
    }
    if (gemv_f16_ok(a))
        return a.mode == kProjQKVRope ? launch_gemv_f16<kProjQKVRope>(a, s)
               : a.mode == kProjQKV   ? launch_gemv_f16<kProjQKV>(a, s)
                                      : launch_gemv_f16<kProjResidual>(a, s);
    if (a.mode == kProjQKVRope) return hipErrorInvalidValue;
    const dim3 grid(a.M / kGvRows), block(64);
    if (a.mode == kProjQKV) {
        if (q8) hipLaunchKernelGGL((proj_gemv_kernel<true, kProjQKV>), grid, block, 0, s, a);
        else    hipLaunchKernelGGL((proj_gemv_kernel<false, kProjQKV>), grid, block, 0, s, a);
    } else {
        if (q8) hipLaunchKernelGGL((proj_gemv_kernel<true, kProjResidual>), grid, block, 0, s, a);
        else    hipLaunchKernelGGL((proj_gemv_kernel<false, kProjResidual>), grid, block, 0, s, a);
    }
    return hipGetLastError();
}

// The GEMM's tiles against the workgroups resident at once (one wide F16
// workgroup per CU, two of the 128 x 128 kernel): a call whose tiles fill
// at most half of them (short chunks, e.g. 512 tokens) is split along K, at
// least 4 k steps per piece, up to 4 pieces, one round.
namespace {
// F16 weights over at least kBigMinRows token rows take the big kernel (256 x 256
// tiles); shorter calls the wide one (256 x 128), whose split pieces are half
// the size
bool proj_big(const ProjArgs& a) { return a.w_type != VVA_TYPE_Q8_0 && a.N >= kBigMinRows; }
}  // namespace

int proj_ksplit(const ProjArgs& a, int n_cu, int* tail0) {
    const bool q8 = a.w_type == VVA_TYPE_Q8_0;
    if (proj_big(a)) {
        // the last round's tiles, when they fill at most a quarter of the CUs,
        // split along K (at most kBMaxSplit pieces of at least 8 k steps)
        const int tiles = ((a.M + kBM - 1) / kBM) * ((a.N + kBN - 1) / kBN);
        const int nk = a.K / kBK, r = tiles % n_cu;
        *tail0 = 0;
        if (r == 0 || 4 * r > n_cu || r > kMaxProjTickets || nk < 16) return 1;
        *tail0 = tiles - r;
        return max(1, min(min(kBMaxSplit, n_cu / r), nk / 8));
    }
    const int tiles = q8 ? (a.M / kTM) * ((a.N + kTN - 1) / kTN) : ((a.M + kWM - 1) / kWM) * ((a.N + kWN - 1) / kWN);
    const int slots = q8 ? 2 * n_cu : n_cu;
    const int nk = a.K / (q8 ? kTK : kWK);
    *tail0 = 0;
    if (tiles < 1 || nk < 8) return 1;
    if (2 * tiles <= slots) {                          // every tile: one round
        if (tiles > kMaxProjTickets) return 1;
        return max(1, min(min(4, slots / tiles), nk / 4));
    }
    // the last round's tiles when they fill at most a quarter of the slots
    const int r = tiles % slots;
    if (r == 0 || 4 * r > slots || r > kMaxProjTickets) return 1;
    *tail0 = tiles - r;
    return max(1, min(min(4, slots / r), nk / 4));
}
size_t proj_part_bytes(const ProjArgs& a) {
    if (a.ksplit <= 1) return 0;
    if (proj_big(a)) {
        const size_t tiles = (size_t)((a.M + kBM - 1) / kBM) * ((a.N + kBN - 1) / kBN);
        return (tiles - a.tail0) * a.ksplit * kBPiece;
    }
    const bool q8 = a.w_type == VVA_TYPE_Q8_0;
    const size_t tiles = q8 ? (size_t)(a.M / kTM) * ((a.N + kTN - 1) / kTN)
                            : (size_t)((a.M + kWM - 1) / kWM) * ((a.N + kWN - 1) / kWN);
    const size_t split = a.tail0 > 0 ? tiles - a.tail0 : tiles;
    return split * a.ksplit * (q8 ? 4 : kWCompute) * 4096 * sizeof(float);
}

// Q8_0 weight rows dequantized to f16 rows of d * q: the products the Q8_0
// GEMM forms while staging its tiles (code and fp16 scale multiplied in
// f16, the exact product rounded once), so that long calls run the F16 GEMM
// on them.  One workgroup per row: the row's blocks are read as consecutive
// dwords into LDS (coalesced; the buffer range ends at the matrix's last
// row, so a dword past it reads as zero), then thread t converts the 8
// codes t % 4 of block t / 4 and stores their 16 bytes, so that every store
// instruction writes 1 KB of the row contiguously.
constexpr int kDqMaxK = 8192;
constexpr int kDqThreads = 256;
__global__ void __launch_bounds__(kDqThreads) proj_dequant_q8_kernel(ProjArgs a, uint16_t* dst) {
    __shared__ uint32_t rowbuf[kDqMaxK / 32 * kQ8Bytes / 4 + 4];
    const int row = blockIdx.x, nb = a.K / 32;
    const int mat = row < a.m_end[0] ? 0 : (row < a.m_end[1] ? 1 : 2);
    const int mbeg = mat == 0 ? 0 : a.m_end[mat - 1];
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(a.w[mat]), (short)0, (int)((a.m_end[mat] - mbeg) * a.w_nb[mat]), 0x00020000);
    const uint32_t base = (uint32_t)((row - mbeg) * a.w_nb[mat]);
    const int nd = (nb * kQ8Bytes + 3) / 4;
    for (int i = threadIdx.x; i < nd; i += kDqThreads) rowbuf[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, base + 4 * i, 0, 0);
    __syncthreads();
    const char* rb = (const char*)rowbuf;
    u32x4* orow = (u32x4*)(dst + (int64_t)row * a.K);
    for (int t = threadIdx.x; t < 4 * nb; t += kDqThreads) {
        const int blk = t >> 2, qd = t & 3;
        const int off = blk * kQ8Bytes;                    // even
        const uint16_t d16 = *(const uint16_t*)(rb + off);
        _Float16 dh;
        __builtin_memcpy(&dh, &d16, 2);
        const h2 dd = {dh, dh};
        // codes 8 qd .. 8 qd + 7: bytes off + 2 + 8 qd .., from the dword at or below
        const int cb = off + 2 + 8 * qd;
        const uint32_t* w = (const uint32_t*)(rb + (cb & ~3));
        const uint32_t w0 = w[0], w1 = w[1], w2 = w[2];
        const bool mis = cb & 2;
        const uint32_t c0 = mis ? __builtin_amdgcn_alignbyte(w1, w0, 2) : w0;
        const uint32_t c1 = mis ? __builtin_amdgcn_alignbyte(w2, w1, 2) : w1;
        uint32_t outw[4];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t c = i ? c1 : c0;
            const h2 lo = {(_Float16)(int8_t)(c & 0xff), (_Float16)(int8_t)((c >> 8) & 0xff)};
            const h2 hi = {(_Float16)(int8_t)((c >> 16) & 0xff), (_Float16)(int8_t)(c >> 24)};
            const h2 plo = lo * dd, phi = hi * dd;
            __builtin_memcpy(&outw[2 * i], &plo, 4);
            __builtin_memcpy(&outw[2 * i + 1], &phi, 4);
        }
        orow[t] = u32x4{outw[0], outw[1], outw[2], outw[3]};
    }
}

bool proj_dequant_q8(const ProjArgs& a) { return a.w_type == VVA_TYPE_Q8_0 && a.N >= kBigMinRows && a.K <= kDqMaxK; }

hipError_t launch_proj_dequant_q8(const ProjArgs& a, uint16_t* dst, hipStream_t s) {
    hipLaunchKernelGGL(proj_dequant_q8_kernel, dim3((unsigned)a.M), dim3(kDqThreads), 0, s, a, dst);
    return hipGetLastError();
}

size_t proj_ws_bytes(int N, int K, int P) {
    const size_t xh = ((size_t)N * K * 2 + 255) / 256 * 256;
    return xh + (size_t)N * P * sizeof(float2);
}

hipError_t launch_proj(ProjPrepArgs& p, ProjArgs& a, void* ws, hipStream_t s) {
    p.xh = (uint16_t*)ws;
    p.rope = p.P > 0 ? (float2*)((char*)ws + ((size_t)p.N * p.K * 2 + 255) / 256 * 256) : nullptr;
    a.xh = p.xh;
    a.rope = p.rope;
    hipLaunchKernelGGL(proj_prep_kernel, dim3(p.N), dim3(256), 0, s, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const bool q8 = a.w_type == VVA_TYPE_Q8_0;
    if (a.ksplit < 1 || !a.part || !a.tickets) {
        a.ksplit = 1;
        a.tail0 = 0;
    }
    // every tile's pieces, or the unsplit tiles then the split tail's pieces
    auto grid = [&](int tiles) { return a.tail0 > 0 ? a.tail0 + (tiles - a.tail0) * a.ksplit : tiles * a.ksplit; };
    if (proj_big(a)) {
        const int tiles = ((a.M + kBM - 1) / kBM) * ((a.N + kBN - 1) / kBN);
        const dim3 g(grid(tiles)), b(kBWaves * 64);
        if (a.mode == kProjQKV) hipLaunchKernelGGL((proj_gemm_big_kernel<kProjQKV>), g, b, 0, s, a);
        else                    hipLaunchKernelGGL((proj_gemm_big_kernel<kProjResidual>), g, b, 0, s, a);
        if ((e = hipGetLastError()) != hipSuccess || a.ksplit <= 1) return e;
        const dim3 gm((tiles - a.tail0) * (kBN / kBSlab));
        if (a.mode == kProjQKV) hipLaunchKernelGGL((proj_big_merge_kernel<kProjQKV>), gm, dim3(256), 0, s, a);
        else                    hipLaunchKernelGGL((proj_big_merge_kernel<kProjResidual>), gm, dim3(256), 0, s, a);
        return hipGetLastError();
    }
    if (!q8) {
        const int wtiles = grid(((a.M + kWM - 1) / kWM) * ((a.N + kWN - 1) / kWN));
        const dim3 block((kWCompute + kWProd) * 64);
        if (a.mode == kProjQKV) hipLaunchKernelGGL((proj_gemm_wide_kernel<kProjQKV>), dim3(wtiles), block, 0, s, a);
        else                    hipLaunchKernelGGL((proj_gemm_wide_kernel<kProjResidual>), dim3(wtiles), block, 0, s, a);
        return hipGetLastError();
    }
    // Q8_0 weights below the big-kernel threshold (F16 ones took the wide
    // kernel above; the 128 x 128 kernel on F16 weights measured no faster)
    const int tiles = grid((a.M / kTM) * ((a.N + kTN - 1) / kTN));
    if (a.mode == kProjQKV) hipLaunchKernelGGL((proj_gemm_kernel<true, kProjQKV>), dim3(tiles), dim3(256), 0, s, a);
    else                    hipLaunchKernelGGL((proj_gemm_kernel<true, kProjResidual>), dim3(tiles), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace vva
