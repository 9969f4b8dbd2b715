// mfma_ops.hpp — operands of v_mfma_f32_32x32x16_{f16,bf16} shared by the
// prefill and the fused decode step: the 16-bit operand types, the product
// per cache type, and the V^T fragment read with the transposing LDS load.
// gfx950 only.  Included inside an anonymous namespace of each kernel file.
//
// Layouts (lane l, l32 = l % 32, half = l / 32):
//   A (32 x 16): row l32, k = 8 half .. 8 half + 7
//   B (16 x 32): column l32, k = 8 half .. 8 half + 7
//   C (32 x 32): column l32, register r holds row 8 (r / 4) + 4 half + r % 4
#pragma once

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) char lds_char;

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

// Byte offset of lane `lane`'s V^T reads in a row-major V tile of row pitch
// VP, for v_frag(tile + off + 64 dt + k * VP, tile + off + 64 dt + (k + 8) * VP)
// over the 16 keys k .. k + 15 of one MFMA step.
__device__ __forceinline__ int v_frag_offset(int lane, int VP) {
    return ((lane & 15) >> 2) * VP + (16 * ((lane >> 4) & 1) + 4 * (lane & 3)) * 2 + 4 * (lane >> 5) * VP;
}
