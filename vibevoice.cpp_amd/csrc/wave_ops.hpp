// wave_ops.hpp — wave-level building blocks shared by the decode kernels:
// cross-lane reductions without LDS (DPP within rows of 16 lanes, permlane
// swaps across rows), packed dot products, int8 -> f16 pair conversion and
// raw buffer descriptors.  gfx950 only.  Included inside an anonymous
// namespace of each kernel file.
#pragma once

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t BufRsrc;
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;

// Raw buffer descriptor (stride 0, range `bytes`; word 3 = 0x00020000, the
// gfx9 raw-buffer configuration): loads at offsets past the range return 0
// without a memory access.
__device__ __forceinline__ BufRsrc make_rsrc(const char* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), (short)0, (int)bytes, 0x00020000);
}
// The same descriptor as four wave-uniform dwords, for inline-asm loads:
// base address (48 bits, stride 0), range in bytes, raw-buffer word 3.
__device__ __forceinline__ i32x4 make_rsrc_sgpr(const char* base, uint32_t bytes) {
    const uint64_t p = (uint64_t)(uintptr_t)base;
    return i32x4{__builtin_amdgcn_readfirstlane((int)(uint32_t)p),
                 __builtin_amdgcn_readfirstlane((int)((uint32_t)(p >> 32) & 0xffffu)),
                 __builtin_amdgcn_readfirstlane((int)bytes), 0x00020000};
}

__device__ __forceinline__ float dot2_f16(uint32_t a, uint32_t b, float c) {
    h2 x, y;
    __builtin_memcpy(&x, &a, 4);
    __builtin_memcpy(&y, &b, 4);
    return __builtin_amdgcn_fdot2(x, y, c, false);
}
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    bf2 x, y;
    __builtin_memcpy(&x, &a, 4);
    __builtin_memcpy(&y, &b, 4);
    return __builtin_amdgcn_fdot2_f32_bf16(x, y, c, false);
}

// Orders this wave's LDS writes before its later LDS reads by other lanes.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Cross-lane steps: DPP within rows of 16 lanes, permlane swaps across rows
// (v_permlane16_swap pairs rows 0-1 / 2-3, v_permlane32_swap the two halves
// of the wave).
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __uint_as_float(__builtin_amdgcn_mov_dpp(__float_as_uint(x), CTRL, 0xf, 0xf, true));
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;
__device__ __forceinline__ float max_swap16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_swap32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float add_swap16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_swap32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// Sum over the LPT lanes of one key (aligned groups of 2, 4 or 8), for N
// values at once so consecutive DPP steps do not wait on each other.
template <int LPT, int N>
__device__ __forceinline__ void key_sum(float (&x)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] += dpp<kDppXor1>(x[i]);
    if constexpr (LPT >= 4) {
#pragma unroll
        for (int i = 0; i < N; ++i) x[i] += dpp<kDppXor2>(x[i]);
    }
    if constexpr (LPT == 8) {
#pragma unroll
        for (int i = 0; i < N; ++i) x[i] += dpp<kDppHalfMirror>(x[i]);
    }
}
// Max over all keys of the wave, for values equal within each LPT group.
template <int LPT, int N>
__device__ __forceinline__ void keys_max(float (&x)[N]) {
    if constexpr (LPT == 2) {
#pragma unroll
        for (int i = 0; i < N; ++i) x[i] = fmaxf(x[i], dpp<kDppXor2>(x[i]));
    }
    if constexpr (LPT <= 4) {
#pragma unroll
        for (int i = 0; i < N; ++i) x[i] = fmaxf(x[i], dpp<kDppHalfMirror>(x[i]));
    }
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] = fmaxf(x[i], dpp<kDppMirror>(x[i]));
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] = max_swap16(x[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] = max_swap32(x[i]);
}
// Sum over all 64 lanes (every lane gets the total).
__device__ __forceinline__ float wave_sum(float x) {
    x += dpp<kDppXor1>(x);
    x += dpp<kDppXor2>(x);
    x += dpp<kDppHalfMirror>(x);
    x += dpp<kDppMirror>(x);
    x = add_swap16(x);
    return add_swap32(x);
}

// First dot of a chain: the VOP3P form with an inline 0 accumulator (the
// accumulate-in-place form would need the zero moved in first).
__device__ __forceinline__ int sdot4_first(uint32_t a, uint32_t b) {
    int r;
    asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// (int8 byte N of a, int8 byte N of b) -> f16 pair (exact): two SDWA
// converts, the second writing the high half in place.
#define VVA_I8_PAIR(N)                                                                          \
    __device__ __forceinline__ uint32_t i8_pair_b##N(uint16_t a, uint16_t b) {                  \
        uint32_t r;                                                                             \
        asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_" #N "\n\t" \
            "v_cvt_f16_i16_sdwa %0, sext(%2) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_" #N \
            : "=&v"(r) : "v"(a), "v"(b));                                                       \
        return r;                                                                               \
    }
VVA_I8_PAIR(0)
VVA_I8_PAIR(1)
VVA_I8_PAIR(2)
VVA_I8_PAIR(3)
#undef VVA_I8_PAIR

// The two f16 MFMA A operands of one Q8_0 block from the code words of four
// keys (c0..c3, each holding dims 2n and 2n + 1 in bytes 0 and 1): r0:r1 =
// dim 2n of keys 0-3, r2:r3 = dim 2n + 1 (exact).  The compiler's hazard
// checks do not look inside inline asm, and an MFMA that reads a VGPR written
// by a VALU instruction needs two wait states in between; the trailing
// s_nop 1 provides them for the last register written, whatever the compiler
// schedules next (the others are further back).
__device__ __forceinline__ void i8_quad_mfma(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                             uint32_t& r0, uint32_t& r1, uint32_t& r2, uint32_t& r3) {
    asm("v_cvt_f16_i16_sdwa %0, sext(%4) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_cvt_f16_i16_sdwa %0, sext(%5) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_0\n\t"
        "v_cvt_f16_i16_sdwa %1, sext(%6) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_cvt_f16_i16_sdwa %1, sext(%7) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_0\n\t"
        "v_cvt_f16_i16_sdwa %2, sext(%4) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_1\n\t"
        "v_cvt_f16_i16_sdwa %2, sext(%5) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_1\n\t"
        "v_cvt_f16_i16_sdwa %3, sext(%6) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_1\n\t"
        "v_cvt_f16_i16_sdwa %3, sext(%7) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_1\n\t"
        "s_nop 1"
        : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3)
        : "v"(c0), "v"(c1), "v"(c2), "v"(c3));
}

