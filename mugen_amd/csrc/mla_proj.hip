// mla_proj.hip -- the MLA absorption and up-projection around the latent
// core: q_abs = q_nope . k_b (transformer.cpp:2563-2573) and out = o . v_b^T
// (transformer.cpp:2610-2620), with the weights dequantised on the fly from
// the reference's GGUF block encodings (dequant_weight_row,
// transformer.cpp:2488-2534: F16, Q8_0, Q4_0).
//
// At decode sizes (rows = batch * q_len of a few to a few tens) both are
// skinny per-head GEMMs bound by the weight stream (16.8 MB per matrix per
// layer in F16 at DeepSeek-V3 shape, 8.9 MB Q8_0, 4.7 MB Q4_0), so they run
// as fp32 VALU dot products that read every weight element once per 16
// rows, the reference's fp32 arithmetic:
//  * absorb: workgroup = (head, 256 columns of kv_rank); thread = one
//    column d; q_nope of up to 16 rows staged in LDS; the k-loop over the
//    128 nope dims streams weight row h*128 + i (coalesced along d);
//  * project: workgroup = (head, 16 output rows j); wave = 4 rows j; lane =
//    8 consecutive kv_rank dims, so one weight row is one coalesced 1 KiB
//    (F16) read; o of up to 16 rows in LDS; per-row wave reductions.
#include "common.h"
#include "kernels.h"

namespace mugen_attn {

namespace {

constexpr int kRCH = 16;  // rows per pass (register accumulators / LDS rows)

template <int WT>
__host__ __device__ constexpr int wrow_bytes(int K) {
    return WT == W_F16 ? 2 * K : (WT == W_Q8_0 ? K / 32 * 34 : K / 32 * 18);
}

__device__ __forceinline__ float half_at(const uint8_t* p) {  // 2-byte aligned f16
    return to_f32<DT_F16>(*reinterpret_cast<const uint16_t*>(p));
}

// element d of a dequantised weight row (dequant_weight_row)
template <int WT>
__device__ __forceinline__ float wval(const uint8_t* row, int d) {
    if constexpr (WT == W_F16) {
        return half_at(row + 2 * d);
    } else if constexpr (WT == W_Q8_0) {
        const uint8_t* blk = row + (d >> 5) * 34;
        return half_at(blk) * (float)(int8_t)blk[2 + (d & 31)];
    } else {
        const uint8_t* blk = row + (d >> 5) * 18;
        const uint8_t byte = blk[2 + (d & 15)];
        const int nib = (d & 16) ? (byte >> 4) : (byte & 15);
        return (float)(nib - 8) * half_at(blk);
    }
}

// elements d0 .. d0+7 of a dequantised row (d0 a multiple of 8)
template <int WT>
__device__ __forceinline__ void wval8(const uint8_t* row, int d0, float* w) {
    if constexpr (WT == W_F16) {
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(row + 2 * d0);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            w[2 * e] = lo_f32<DT_F16>(v[e]);
            w[2 * e + 1] = hi_f32<DT_F16>(v[e]);
        }
    } else if constexpr (WT == W_Q8_0) {
        const uint8_t* blk = row + (d0 >> 5) * 34;
        const float s = half_at(blk);
        const uint16_t* q2 = reinterpret_cast<const uint16_t*>(blk + 2 + (d0 & 31));  // even offset
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint16_t v = q2[e];
            w[2 * e] = s * (float)(int8_t)(v & 0xff);
            w[2 * e + 1] = s * (float)(int8_t)(v >> 8);
        }
    } else {
        const uint8_t* blk = row + (d0 >> 5) * 18;
        const float s = half_at(blk);
        const int p = d0 & 31;  // 0, 8: low nibbles of bytes p..p+7; 16, 24: high nibbles of p-16..
        const uint16_t* b2 = reinterpret_cast<const uint16_t*>(blk + 2 + (p & 15));
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint16_t v = b2[e];
            const int lo = v & 0xff, hi = v >> 8;
            const int n0 = (p & 16) ? (lo >> 4) : (lo & 15);
            const int n1 = (p & 16) ? (hi >> 4) : (hi & 15);
            w[2 * e] = (float)(n0 - 8) * s;
            w[2 * e + 1] = (float)(n1 - 8) * s;
        }
    }
}

}  // namespace

template <int WT, int OUT_DT>
__global__ __launch_bounds__(256) void mla_absorb_kernel(MlaProjParams p) {
    constexpr int NOPE = 128, ROPE = 64, KR = 512;
    __shared__ float qs[kRCH][NOPE];
    const int h = blockIdx.x, tid = threadIdx.x;
    const int d = blockIdx.y * 256 + tid;
    constexpr int RB = wrow_bytes<WT>(KR);
    const uint8_t* wh = static_cast<const uint8_t*>(p.w) + (size_t)h * NOPE * RB;
    const uint16_t* q = static_cast<const uint16_t*>(p.in);
    for (int r0 = 0; r0 < p.rows; r0 += kRCH) {
        const int nr = min(kRCH, p.rows - r0);
        __syncthreads();
        for (int k = tid; k < kRCH * NOPE; k += 256) {
            const int r = k / NOPE, i = k % NOPE;
            qs[r][i] = r < nr ? to_f32<DT_F16>(q[((int64_t)(r0 + r) * p.H + h) * (NOPE + ROPE) + i]) : 0.f;
        }
        __syncthreads();
        float acc[kRCH];
#pragma unroll
        for (int r = 0; r < kRCH; r++) acc[r] = 0.f;
        for (int i0 = 0; i0 < NOPE; i0 += 8) {
            float w[8];
#pragma unroll
            for (int e = 0; e < 8; e++) w[e] = wval<WT>(wh + (size_t)(i0 + e) * RB, d);
#pragma unroll
            for (int e = 0; e < 8; e++) {
#pragma unroll
                for (int r = 0; r < kRCH; r++) {
                    const float qi = qs[r][i0 + e];
                    acc[r] = qi != 0.f ? fmaf(qi, w[e], acc[r]) : acc[r];  // zero terms skipped, as the reference
                }
            }
        }
#pragma unroll
        for (int r = 0; r < kRCH; r++)
            if (r < nr) store_out<OUT_DT>(p.out, ((int64_t)(r0 + r) * p.H + h) * (KR + ROPE) + d, acc[r]);
        if (blockIdx.y == 0 && tid < ROPE) {  // q_rope appended unchanged
            for (int r = 0; r < nr; r++)
                store_out<OUT_DT>(p.out, ((int64_t)(r0 + r) * p.H + h) * (KR + ROPE) + KR + tid,
                                  to_f32<DT_F16>(q[((int64_t)(r0 + r) * p.H + h) * (NOPE + ROPE) + NOPE + tid]));
        }
    }
}

template <int WT, int OUT_DT>
__global__ __launch_bounds__(256) void mla_project_kernel(MlaProjParams p) {
    constexpr int KR = 512, VH = 128;
    __shared__ __attribute__((aligned(16))) float os[kRCH][KR];
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int j0 = blockIdx.y * 16 + 4 * w;
    constexpr int RB = wrow_bytes<WT>(KR);
    const uint8_t* wh = static_cast<const uint8_t*>(p.w) + (size_t)h * VH * RB;
    const float* o = static_cast<const float*>(p.in);
    for (int r0 = 0; r0 < p.rows; r0 += kRCH) {
        const int nr = min(kRCH, p.rows - r0);
        __syncthreads();
        for (int k = tid; k < kRCH * KR / 4; k += 256) {
            const int r = k / (KR / 4), c4 = k % (KR / 4);
            *reinterpret_cast<f32x4_t*>(&os[r][4 * c4]) =
                r < nr ? *reinterpret_cast<const f32x4_t*>(o + ((int64_t)(r0 + r) * p.H + h) * KR + 4 * c4)
                       : f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
        __syncthreads();
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
            const int j = j0 + jj;
            float wv[8];
            wval8<WT>(wh + (size_t)j * RB, 8 * lane, wv);
            for (int r = 0; r < nr; r++) {
                const f32x4_t a = *reinterpret_cast<const f32x4_t*>(&os[r][8 * lane]);
                const f32x4_t b = *reinterpret_cast<const f32x4_t*>(&os[r][8 * lane + 4]);
                float part = a[0] * wv[0];
                part = fmaf(a[1], wv[1], part);
                part = fmaf(a[2], wv[2], part);
                part = fmaf(a[3], wv[3], part);
                part = fmaf(b[0], wv[4], part);
                part = fmaf(b[1], wv[5], part);
                part = fmaf(b[2], wv[6], part);
                part = fmaf(b[3], wv[7], part);
                part = wave_sum(part);
                if (lane == 0) store_out<OUT_DT>(p.out, ((int64_t)(r0 + r) * p.H + h) * VH + j, part);
            }
        }
    }
}

template <int WT>
static hipError_t launch_absorb_w(const MlaProjParams& p, int out_dt, hipStream_t st) {
    const dim3 grid(p.H, 512 / 256);
    if (out_dt == DT_BF16) hipLaunchKernelGGL((mla_absorb_kernel<WT, DT_BF16>), grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((mla_absorb_kernel<WT, DT_F32>), grid, dim3(256), 0, st, p);
    return hipGetLastError();
}

hipError_t launch_mla_absorb(const MlaProjParams& p, int w_type, int out_dt, hipStream_t st, KernelTimer* t) {
    timer_begin(t, "mla_absorb", st);
    hipError_t e = w_type == W_F16 ? launch_absorb_w<W_F16>(p, out_dt, st)
                 : w_type == W_Q8_0 ? launch_absorb_w<W_Q8_0>(p, out_dt, st)
                                    : launch_absorb_w<W_Q4_0>(p, out_dt, st);
    timer_end(t, "mla_absorb", st);
    return e;
}

template <int WT>
static hipError_t launch_project_w(const MlaProjParams& p, int out_dt, hipStream_t st) {
    const dim3 grid(p.H, 128 / 16);
    if (out_dt == DT_F16) hipLaunchKernelGGL((mla_project_kernel<WT, DT_F16>), grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((mla_project_kernel<WT, DT_F32>), grid, dim3(256), 0, st, p);
    return hipGetLastError();
}

hipError_t launch_mla_project(const MlaProjParams& p, int w_type, int out_dt, hipStream_t st, KernelTimer* t) {
    timer_begin(t, "mla_project", st);
    hipError_t e = w_type == W_F16 ? launch_project_w<W_F16>(p, out_dt, st)
                 : w_type == W_Q8_0 ? launch_project_w<W_Q8_0>(p, out_dt, st)
                                    : launch_project_w<W_Q4_0>(p, out_dt, st);
    timer_end(t, "mla_project", st);
    return e;
}

}  // namespace mugen_attn
