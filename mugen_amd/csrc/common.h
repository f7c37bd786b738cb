// common.h -- shared device helpers for the gfx950 attention kernels.
//
// Storage elements are 16-bit (IEEE fp16 or bf16) held as uint16_t; all
// arithmetic is fp32.  Matrix products use the gfx950 MFMA
// v_mfma_f32_16x16x32_{f16,bf16}: wave64, A 16x32, B 32x16, D 16x16 fp32.
// Operand layout (lane l, g = l/16, n = l%16):
//   A: lane holds A[n][8g .. 8g+7]        (8 consecutive k of row n)
//   B: lane holds B[8g .. 8g+7][n]        (8 consecutive k of column n)
//   D: lane holds D[4g + i][n], i = 0..3
// Only the pairing "A slot (g,j) <-> B slot (g,j) is the same k" is relied
// on, so every kernel is free to assign k-slots to any index permutation as
// long as both operands agree.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mugen_attn.h"

namespace mugen_attn {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

enum { DT_F32 = MUGEN_ATTN_F32, DT_F16 = MUGEN_ATTN_F16, DT_BF16 = MUGEN_ATTN_BF16 };

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

// ---------------------------------------------------------------- scalars

template <int DT>
__device__ __forceinline__ float to_f32(uint16_t h) {
    if constexpr (DT == DT_BF16) {
        return __uint_as_float(uint32_t(h) << 16);
    } else {
        _Float16 f = __builtin_bit_cast(_Float16, h);
        return float(f);
    }
}

// low / high 16-bit element of a packed dword
template <int DT>
__device__ __forceinline__ float lo_f32(uint32_t w) {
    if constexpr (DT == DT_BF16) return __uint_as_float(w << 16);
    else return float(__builtin_bit_cast(_Float16, uint16_t(w & 0xffffu)));
}
template <int DT>
__device__ __forceinline__ float hi_f32(uint32_t w) {
    if constexpr (DT == DT_BF16) return __uint_as_float(w & 0xffff0000u);
    else return float(__builtin_bit_cast(_Float16, uint16_t(w >> 16)));
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return uint16_t(u >> 16);
}

template <int DT>
__device__ __forceinline__ uint16_t from_f32(float f) {
    if constexpr (DT == DT_BF16) return f32_to_bf16_rne(f);
    else return __builtin_bit_cast(uint16_t, _Float16(f));
}

template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    return uint32_t(from_f32<DT>(a)) | (uint32_t(from_f32<DT>(b)) << 16);
}

// store one fp32 value as OUT_DT
template <int OUT_DT>
__device__ __forceinline__ void store_out(void* base, int64_t idx, float v) {
    if constexpr (OUT_DT == DT_F32) static_cast<float*>(base)[idx] = v;
    else static_cast<uint16_t*>(base)[idx] = from_f32<OUT_DT>(v);
}

// Number of 16-bit terms the softmax weights P are split into for the P.V
// MFMA: fp16 (11-bit significand) is used as is; bf16 (8-bit) is split
// into hi + lo so the weights keep ~16 significant bits.
template <int DT>
__host__ __device__ constexpr int p_terms() { return DT == DT_BF16 ? 2 : 1; }

// Pack 8 fp32 weights into NP A-operand fragments (hi, then lo residual).
template <int DT, int NP>
__device__ __forceinline__ void split_p(const float* x, u32x4_t* frag) {
    uint32_t hi[4], lo[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint16_t h0 = from_f32<DT>(x[2 * j]), h1 = from_f32<DT>(x[2 * j + 1]);
        hi[j] = uint32_t(h0) | (uint32_t(h1) << 16);
        if constexpr (NP > 1) lo[j] = pack2<DT>(x[2 * j] - to_f32<DT>(h0), x[2 * j + 1] - to_f32<DT>(h1));
    }
    frag[0] = u32x4_t{hi[0], hi[1], hi[2], hi[3]};
    if constexpr (NP > 1) frag[1] = u32x4_t{lo[0], lo[1], lo[2], lo[3]};
}

// ---------------------------------------------------------------- MFMA

template <int DT>
__device__ __forceinline__ f32x4_t mfma16x16x32(u32x4_t a, u32x4_t b, f32x4_t c) {
    if constexpr (DT == DT_BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                      __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// ---------------------------------------------------------------- wave ops

__device__ __forceinline__ float wave_xor(float v, int mask) {
    return __shfl_xor(v, mask, 64);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ u32x4_t load16(const void* p) {
    return *reinterpret_cast<const u32x4_t*>(p);
}
__device__ __forceinline__ u32x2_t load8(const void* p) {
    return *reinterpret_cast<const u32x2_t*>(p);
}

}  // namespace mugen_attn
