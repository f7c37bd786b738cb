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

#include <type_traits>

#include "mugen_attn.h"

namespace mugen_attn {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2v_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));

enum { DT_F32 = MUGEN_ATTN_F32, DT_F16 = MUGEN_ATTN_F16, DT_BF16 = MUGEN_ATTN_BF16 };

// Phase timestamps for development profiling, compiled only with
// -DMUGEN_ATTN_TRACE (a single-translation-unit build that defines the
// buffer): lane 0 of every wave stores the 100 MHz real-time counter of
// numbered points (k < 16) of its kernel, indexed by workgroup and wave.
#ifdef MUGEN_ATTN_TRACE
extern __device__ uint64_t mugen_attn_trace[];
#define MUGEN_TRACE(k)                                                                          \
    do {                                                                                        \
        if ((threadIdx.x & 63) == 0)                                                            \
            mugen_attn_trace[(((size_t)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * \
                                 (blockDim.x >> 6) * 16 + (threadIdx.x >> 6) * 16               \
                             + (k)] = __builtin_amdgcn_s_memrealtime();                         \
    } while (0)
#define MUGEN_TRACE_CLK(k)                                                                      \
    do {                                                                                        \
        if ((threadIdx.x & 63) == 0)                                                            \
            mugen_attn_trace[(((size_t)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * \
                                 (blockDim.x >> 6) * 16 + (threadIdx.x >> 6) * 16               \
                             + (k)] = __builtin_readcyclecounter();                             \
    } while (0)
#else
#define MUGEN_TRACE_CLK(k) \
    do {                   \
    } while (0)
#define MUGEN_TRACE(k) \
    do {               \
    } while (0)
#endif

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

// two fp32 -> packed 16-bit pair (RNE); gfx950 converts bf16 in hardware
// (v_cvt_pk_bf16_f32) and fp16 with v_cvt_pk_f16_f32
template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    if constexpr (DT == DT_BF16) {
        typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
    } else {
        typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, f16x2_t));
    }
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

// Pack 8 fp32 weights into NP A/B-operand fragments (hi, then the lo
// residual), both rounded to nearest even by the hardware pack.
template <int DT, int NP>
__device__ __forceinline__ void split_p(const float* x, u32x4_t* frag) {
    uint32_t hi[4], lo[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        hi[j] = pack2<DT>(x[2 * j], x[2 * j + 1]);
        if constexpr (NP > 1)
            lo[j] = pack2<DT>(x[2 * j] - lo_f32<DT>(hi[j]), x[2 * j + 1] - hi_f32<DT>(hi[j]));
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

// Reductions with the lane 16 / 32 apart, in every lane, on the VALU
// (gfx950 v_permlane16_swap / v_permlane32_swap; no LDS round trip like
// ds_bpermute).  With both operands = v the swap returns, per lane, v and
// its partner in some order, so their sum / max is the pair's.
__device__ __forceinline__ float sum_x32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_x32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_x16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_x16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// LDS transpose read (gfx950 ds_read_b64_tr_b16).  Within each 16-lane
// group, lane i receives element (i % 4) of the 8-byte chunks addressed by
// lanes 4r + i/4, r = 0..3: with lane (4r + c) pointing at row r, columns
// [4c, 4c+4) of a row-major 16-bit tile, lane i gets column i of rows 0..3.
// LDS byte address -> LDS pointer: constant offsets added to the pointer
// go into the instructions' offset field (one address register per base)
typedef __attribute__((address_space(3))) char lds_char_t;
__device__ __forceinline__ const lds_char_t* lds_ptr(uint32_t byte_addr) {
    return reinterpret_cast<const lds_char_t*>(static_cast<uintptr_t>(byte_addr));
}
__device__ __forceinline__ u32x2_t lds_read_tr16(const lds_char_t* p) {
    typedef short s16x4_t __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) const s16x4_t* lds_s16x4_cptr;
    const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        const_cast<__attribute__((address_space(3))) s16x4_t*>(reinterpret_cast<lds_s16x4_cptr>(p)));
    return __builtin_bit_cast(u32x2_t, v);
}

__device__ __forceinline__ u32x4_t lds_read_b128(const lds_char_t* p) {
    return *reinterpret_cast<const __attribute__((address_space(3))) u32x4_t*>(p);
}

__device__ __forceinline__ u32x2_t lds_read_tr16(const uint16_t* p) {
    typedef short s16x4_t __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) s16x4_t* lds_s16x4_ptr;
    const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(const_cast<uint16_t*>(p)));
    return __builtin_bit_cast(u32x2_t, v);
}

// the value of lane (this lane ^ M), M = 1, 2, 4 or 8, by DPP (no LDS
// round trip as with ds_bpermute): quad permutations for 1 and 2, a
// half-row mirror (i -> 7 - i) then a quad reversal (i -> 3 - i) for 4, a
// row rotation by 8 for 8
template <int M>
__device__ __forceinline__ float dpp_xor(float v) {
    const int b = __float_as_int(v);
    if constexpr (M == 1) return __int_as_float(__builtin_amdgcn_mov_dpp(b, 0xB1, 0xF, 0xF, false));
    if constexpr (M == 2) return __int_as_float(__builtin_amdgcn_mov_dpp(b, 0x4E, 0xF, 0xF, false));
    if constexpr (M == 4)
        return __int_as_float(
            __builtin_amdgcn_mov_dpp(__builtin_amdgcn_mov_dpp(b, 0x141, 0xF, 0xF, false), 0x1B, 0xF, 0xF, false));
    if constexpr (M == 8) return __int_as_float(__builtin_amdgcn_mov_dpp(b, 0x128, 0xF, 0xF, false));
}

// max / sum over the wave's 64 lanes, in every lane: lane swaps for 32 and
// 16 apart, DPP below (the pairs of the xor butterfly 32, 16, .., 1, so the
// sum's order is that butterfly's)
__device__ __forceinline__ float wave_max(float v) {
    v = max_x16(max_x32(v));
    v = fmaxf(v, dpp_xor<8>(v));
    v = fmaxf(v, dpp_xor<4>(v));
    v = fmaxf(v, dpp_xor<2>(v));
    return fmaxf(v, dpp_xor<1>(v));
}
__device__ __forceinline__ int wave_min_i32(int v) {
    const auto r32 = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
    v = min((int)r32[0], (int)r32[1]);
    const auto r16 = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
    v = min((int)r16[0], (int)r16[1]);
    v = min(v, __float_as_int(dpp_xor<8>(__int_as_float(v))));
    v = min(v, __float_as_int(dpp_xor<4>(__int_as_float(v))));
    v = min(v, __float_as_int(dpp_xor<2>(__int_as_float(v))));
    return min(v, __float_as_int(dpp_xor<1>(__int_as_float(v))));
}
__device__ __forceinline__ float wave_sum(float v) {
    v = sum_x16(sum_x32(v));
    v += dpp_xor<8>(v);
    v += dpp_xor<4>(v);
    v += dpp_xor<2>(v);
    return v + dpp_xor<1>(v);
}

// Split-K log-sum-exp weights for one output row: given the (m, l) pairs of
// nact splits (m in log2 units, stride 2 floats apart by `ml_stride`),
// writes f_s = 2^(m_s - M) to LDS and returns 1 / sum_s f_s l_s (0 when
// no split saw a token).  All threads of the block must call it.
constexpr int kMaxSplits = 4096;
constexpr int kMaxMlaSplits = 512;  // MLA combine keeps per-row split weights in LDS
// Split weights of a log-sum-exp merge: f_lds[s] = 2^(m_s - M), returns
// 1 / sum_s f_s * l_s.  (m0, l0) is the (m, l) pair of split threadIdx.x,
// loaded by the caller (so that its latency can overlap other loads); the
// splits beyond blockDim.x are read here.
__device__ __forceinline__ float lse_weights(const float* ml, int64_t ml_stride, int nact, float m0, float l0,
                                             float* f_lds, float* red_lds) {
    const int tid = threadIdx.x, nw = blockDim.x >> 6, w = tid >> 6;
    float mloc = m0;
    for (int s = tid + blockDim.x; s < nact; s += blockDim.x) mloc = fmaxf(mloc, ml[s * ml_stride]);
    mloc = wave_max(mloc);
    if ((tid & 63) == 0) red_lds[w] = mloc;
    __syncthreads();
    float M = red_lds[0];
    for (int i = 1; i < nw; i++) M = fmaxf(M, red_lds[i]);
    __syncthreads();
    float lloc = 0.f;
    if (tid < nact) {
        const float f = (m0 == kNegInf) ? 0.f : fast_exp2(m0 - M);
        f_lds[tid] = f;
        lloc = f * l0;
    }
    for (int s = tid + blockDim.x; s < nact; s += blockDim.x) {
        const float m = ml[s * ml_stride];
        const float f = (m == kNegInf) ? 0.f : fast_exp2(m - M);
        f_lds[s] = f;
        lloc += f * ml[s * ml_stride + 1];
    }
    lloc = wave_sum(lloc);
    if ((tid & 63) == 0) red_lds[w] = lloc;
    __syncthreads();
    float L = 0.f;
    for (int i = 0; i < nw; i++) L += red_lds[i];
    return L > 0.f ? 1.f / L : 0.f;
}

// ---------------------------------------------------------------- LDS DMA
//
// gfx950 global_load_lds_dwordx4: each lane's 16 bytes at `src` land in LDS
// at M0 + 16*lane (one contiguous KiB per wave instruction).  Issued from
// inline asm so the compiler's wait-count pass, which cannot tell an
// in-flight DMA from the LDS reads of another buffer, does not serialise
// the ring buffer with vmcnt(0); callers order it with vm_wait<N>() and
// lds_barrier().  `lds_byte_addr` must be wave-uniform.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// `sbase` (wave-uniform, SGPR pair) + per-lane 32-bit byte offset `voff`
__device__ __forceinline__ void dma16s(uint32_t lds_byte_addr, const void* sbase, uint32_t voff) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_byte_addr);
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %2"
        :
        : "s"(m0), "v"(voff), "s"(sbase)
        : "memory", "m0");
}

// wait until at most N vector-memory operations of this wave are in flight
template <int N>
__device__ __forceinline__ void vm_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// workgroup barrier that also orders the compiler's memory accesses,
// without the full fence (and its vmcnt(0)) of __syncthreads()
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory");
}

// Write-through vector stores (sc0 sc1) for large split partials: each line goes
// through L2 to the memory-side cache when it is written, instead of staying
// dirty until the end-of-kernel L2 writeback, which otherwise sits between
// the split kernel and the merge kernel that reads the partials.
__device__ __forceinline__ void store_wt(u32x4_t* p, u32x4_t v) {
    asm volatile("global_store_dwordx4 %0, %1, off sc0 sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store_wt(float* p, float v) {
    asm volatile("global_store_dword %0, %1, off sc0 sc1" ::"v"(p), "v"(v) : "memory");
}

__device__ __forceinline__ u32x4_t load16(const void* p) {
    return *reinterpret_cast<const u32x4_t*>(p);
}
__device__ __forceinline__ u32x2_t load8(const void* p) {
    return *reinterpret_cast<const u32x2_t*>(p);
}

// ---------------------------------------------------------------- RoPE

// position of row r: positions[r], or (positions null) the r % rows_per_seq
// -th new token of sequence r / rows_per_seq, appended at seq_base[seq]
__device__ __forceinline__ int row_position(const int32_t* positions, const int32_t* seq_base, int rows_per_seq,
                                            int r) {
    return positions ? positions[r] : seq_base[r / rows_per_seq] + r % rows_per_seq;
}

// One NeoX pair (x0 = dim i, x1 = dim i + 32) rotated by pos * freq as the
// reference's float code does (transformer.cpp:3903-3917): angle rounded
// to float, full-precision cosf / sinf, each output a product difference
// with separately rounded products (contraction off, like the scalar host
// loop), then rounded to f16 (the reference stores the result as f16).
__device__ __forceinline__ void rope_pair_f16(float x0, float x1, int pos, float freq, uint16_t& y0, uint16_t& y1) {
#pragma clang fp contract(off)
    const float angle = (float)pos * freq;
    const float cv = cosf(angle), sv = sinf(angle);
    y0 = from_f32<DT_F16>(x0 * cv - x1 * sv);
    y1 = from_f32<DT_F16>(x1 * cv + x0 * sv);
}

}  // namespace mugen_attn
