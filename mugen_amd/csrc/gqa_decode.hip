// gqa_decode.hip -- split-K GQA decode over a token-major fp16/bf16 K/V cache.
//
// Semantics: cpu_attention (src/core/model/transformer.cpp:2441-2485) and the
// Metal flash_attention_decode (src/metal/kernel_sources.h:2900-2999): one
// query token per head, kv head = h / (H/Hk), softmax(q.K^T * scale) V with
// fp32 accumulation.
//
// Design (HBM-bound: ~7 flop per K/V byte at the 7B shape):
//  * one workgroup = (context split, kv head, sequence); all G = H/Hk query
//    heads of the group are served from ONE read of the group's K/V rows
//    (the Metal kernel re-reads them once per query head);
//  * 4 waves per workgroup; wave w takes 16-token blocks w, w+4, ... of
//    the split so the workgroup streams one contiguous token range;
//  * S^T[16 tok x 16 heads] = K . Q^T on MFMA 16x16x32 (K rows are the A
//    operand straight from global memory, Q^T stays in registers; heads
//    beyond G are zero columns);
//  * online softmax in registers (exp2 domain), probabilities to LDS;
//  * P.V on VALU: V is read fully coalesced (LPT lanes x 8 B per token row)
//    and each lane accumulates all G heads for its 4 dims;
//  * the 4 waves merge (m, l, o) through LDS; with one split the result is
//    normalised and stored, otherwise (m, l, o) partials go to the
//    workspace and gqa_decode_combine merges them with fp32 log-sum-exp.
#include "common.h"
#include "kernels.h"

namespace mugen_attn {

template <int D, int GMAX, int DT, int OUT_DT>
__global__ __launch_bounds__(256) void gqa_decode_kernel(GqaDecodeParams p) {
    constexpr int KK = D / 32;     // MFMA k-steps per row
    constexpr int LPT = D / 4;     // lanes per token row in the V layout
    constexpr int TPI = 64 / LPT;  // token rows per V load instruction
    constexpr int VI = 16 / TPI;   // V load instructions per 16-token block

    __shared__ float p_lds[4][16][16];  // [wave][token][head]
    __shared__ float a_lds[4][16];      // per-head rescale of the step
    __shared__ float m_lds[4][16];
    __shared__ float l_lds[4][16];
    __shared__ float o_lds[4][GMAX][D];

    const int s = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int T = p.seq_lens[b];
    const int t_begin = s * p.chunk;
    const int t_end = min(t_begin + p.chunk, T);
    if (p.num_splits > 1 && t_begin >= T) return;  // empty split: combine skips it
    const int G = p.G;
    const int h0 = kvh * G;

    const uint16_t* kbase = p.k + (int64_t)b * p.seq_stride + (int64_t)kvh * D;
    const uint16_t* vbase = p.v + (int64_t)b * p.seq_stride + (int64_t)kvh * D;

    // Q^T as the B operand: lane holds q[head n][32kk + 8g .. +8]
    u32x4_t qf[KK];
    if (n < G) {
        const uint16_t* qp = p.q + ((int64_t)b * p.H + h0 + n) * D;
#pragma unroll
        for (int kk = 0; kk < KK; kk++) qf[kk] = load16(qp + 32 * kk + 8 * g);
    } else {
#pragma unroll
        for (int kk = 0; kk < KK; kk++) qf[kk] = u32x4_t{0, 0, 0, 0};
    }

    float m_run = kNegInf;  // running max (log2 domain) of head n
    float l_part = 0.f;     // this lane's share of the running sum
    float o[GMAX][4];
#pragma unroll
    for (int h = 0; h < GMAX; h++) o[h][0] = o[h][1] = o[h][2] = o[h][3] = 0.f;

    const int vp = lane / LPT;         // token sub-row of this lane in V loads
    const int vd = (lane % LPT) * 4;   // first of the 4 dims this lane owns

    for (int t0 = t_begin + 16 * w; t0 < t_end; t0 += 64) {
        // loads first (K as MFMA A operand, V coalesced); clamp rows past
        // the split end onto the last valid row: finite, and masked below
        const int tk = min(t0 + n, t_end - 1);
        const uint16_t* kp = kbase + (int64_t)tk * p.row_stride + 8 * g;
        u32x4_t kf[KK];
#pragma unroll
        for (int kk = 0; kk < KK; kk++) kf[kk] = load16(kp + 32 * kk);
        u32x2_t vf[VI];
#pragma unroll
        for (int i = 0; i < VI; i++) {
            const int tv = min(t0 + i * TPI + vp, t_end - 1);
            vf[i] = load8(vbase + (int64_t)tv * p.row_stride + vd);
        }

        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < KK; kk++) acc = mfma16x16x32<DT>(kf[kk], qf[kk], acc);

        // acc[i] = score of token t0 + 4g + i for head n
        float x[4];
        float mt = kNegInf;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            x[i] = (t0 + 4 * g + i < t_end) ? acc[i] * p.scale_log2 : kNegInf;
            mt = fmaxf(mt, x[i]);
        }
        mt = fmaxf(mt, wave_xor(mt, 16));
        mt = fmaxf(mt, wave_xor(mt, 32));
        const float m_new = fmaxf(m_run, mt);  // finite: token t0 is valid
        const float alpha = fast_exp2(m_run - m_new);
        float ps = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            x[i] = fast_exp2(x[i] - m_new);
            ps += x[i];
        }
        l_part = l_part * alpha + ps;
        m_run = m_new;

#pragma unroll
        for (int i = 0; i < 4; i++) p_lds[w][4 * g + i][n] = x[i];
        if (g == 0) a_lds[w][n] = alpha;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

#pragma unroll
        for (int h = 0; h < GMAX; h++) {
            if (h < G) {
                const float a = a_lds[w][h];
                o[h][0] *= a; o[h][1] *= a; o[h][2] *= a; o[h][3] *= a;
            }
        }
#pragma unroll
        for (int i = 0; i < VI; i++) {
            const int tl = i * TPI + vp;
            const float v0 = lo_f32<DT>(vf[i][0]), v1 = hi_f32<DT>(vf[i][0]);
            const float v2 = lo_f32<DT>(vf[i][1]), v3 = hi_f32<DT>(vf[i][1]);
#pragma unroll
            for (int h = 0; h < GMAX; h++) {
                if (h < G) {
                    const float pw = p_lds[w][tl][h];
                    o[h][0] += pw * v0; o[h][1] += pw * v1;
                    o[h][2] += pw * v2; o[h][3] += pw * v3;
                }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    // wave-level reductions: l over the 4 token groups, o over token sub-rows
    l_part += wave_xor(l_part, 16);
    l_part += wave_xor(l_part, 32);
#pragma unroll
    for (int h = 0; h < GMAX; h++) {
#pragma unroll
        for (int c = 0; c < 4; c++) {
            float v = o[h][c];
            if (LPT <= 16) v += wave_xor(v, 16);
            v += wave_xor(v, 32);
            o[h][c] = v;
        }
    }
    if (g == 0) {
        m_lds[w][n] = m_run;
        l_lds[w][n] = l_part;
    }
    if (vp == 0) {
#pragma unroll
        for (int h = 0; h < GMAX; h++) {
            if (h < G) {
                o_lds[w][h][vd + 0] = o[h][0];
                o_lds[w][h][vd + 1] = o[h][1];
                o_lds[w][h][vd + 2] = o[h][2];
                o_lds[w][h][vd + 3] = o[h][3];
            }
        }
    }
    __syncthreads();

    // merge the 4 waves' (m, l, o) for each (head, dim)
    for (int idx = threadIdx.x; idx < G * D; idx += 256) {
        const int h = idx / D, d = idx - h * D;
        float M = kNegInf;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) M = fmaxf(M, m_lds[ww][h]);
        float L = 0.f, O = 0.f;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) {
            const float mw = m_lds[ww][h];
            const float f = (mw == kNegInf) ? 0.f : fast_exp2(mw - M);
            L += f * l_lds[ww][h];
            O += f * o_lds[ww][h][d];
        }
        const int64_t bh = (int64_t)b * p.H + h0 + h;
        if (p.num_splits == 1) {
            store_out<OUT_DT>(p.out, bh * D + d, L > 0.f ? O / L : 0.f);
        } else {
            const int64_t slot = bh * p.num_splits + s;
            p.ws_o[slot * D + d] = O;
            if (d == 0) {
                p.ws_ml[slot * 2 + 0] = M;
                p.ws_ml[slot * 2 + 1] = L;
            }
        }
    }
}

// Log-sum-exp merge of the split partials of one (sequence, head): the
// split weights are computed in parallel, then each thread sums its dim
// over the splits with independent (unrolled) loads.
template <int D, int OUT_DT>
__global__ __launch_bounds__(D) void gqa_decode_combine_kernel(GqaDecodeParams p) {
    __shared__ float f_lds[kMaxSplits];
    __shared__ float red_lds[4];
    const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
    const int T = p.seq_lens[b];
    const int nact = min(p.num_splits, (T + p.chunk - 1) / p.chunk);
    const int64_t bh = (int64_t)b * p.H + h;
    const float inv = lse_weights(p.ws_ml + bh * p.num_splits * 2, 2, nact, f_lds, red_lds);
    const float* os = p.ws_o + bh * p.num_splits * D + d;
    float O0 = 0.f, O1 = 0.f, O2 = 0.f, O3 = 0.f;
    int s = 0;
    for (; s + 4 <= nact; s += 4) {
        O0 += f_lds[s] * os[(int64_t)s * D];
        O1 += f_lds[s + 1] * os[(int64_t)(s + 1) * D];
        O2 += f_lds[s + 2] * os[(int64_t)(s + 2) * D];
        O3 += f_lds[s + 3] * os[(int64_t)(s + 3) * D];
    }
    for (; s < nact; s++) O0 += f_lds[s] * os[(int64_t)s * D];
    store_out<OUT_DT>(p.out, bh * D + d, ((O0 + O1) + (O2 + O3)) * inv);
}

// ------------------------------------------------------------------ launch

template <int D, int GMAX, int DT, int OUT_DT>
static hipError_t launch_gqa_t(const GqaDecodeParams& p, int B, int Hk, hipStream_t st,
                               KernelTimer* timer) {
    dim3 grid(p.num_splits, Hk, B);
    timer_begin(timer, "gqa_decode", st);
    hipLaunchKernelGGL((gqa_decode_kernel<D, GMAX, DT, OUT_DT>), grid, dim3(256), 0, st, p);
    timer_end(timer, "gqa_decode", st);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || p.num_splits == 1) return e;
    timer_begin(timer, "gqa_decode_combine", st);
    hipLaunchKernelGGL((gqa_decode_combine_kernel<D, OUT_DT>), dim3(p.H, B), dim3(D), 0, st, p);
    timer_end(timer, "gqa_decode_combine", st);
    return hipGetLastError();
}

template <int D, int GMAX, int DT>
static hipError_t launch_gqa_o(const GqaDecodeParams& p, int B, int Hk, int out_dt, hipStream_t st,
                               KernelTimer* t) {
    switch (out_dt) {
        case DT_F32: return launch_gqa_t<D, GMAX, DT, DT_F32>(p, B, Hk, st, t);
        case DT_F16: return launch_gqa_t<D, GMAX, DT, DT_F16>(p, B, Hk, st, t);
        default: return launch_gqa_t<D, GMAX, DT, DT_BF16>(p, B, Hk, st, t);
    }
}

template <int D, int GMAX>
static hipError_t launch_gqa_d(const GqaDecodeParams& p, int B, int Hk, int kv_dt, int out_dt,
                               hipStream_t st, KernelTimer* t) {
    if (kv_dt == DT_F16) return launch_gqa_o<D, GMAX, DT_F16>(p, B, Hk, out_dt, st, t);
    return launch_gqa_o<D, GMAX, DT_BF16>(p, B, Hk, out_dt, st, t);
}

template <int D>
static hipError_t launch_gqa_g(const GqaDecodeParams& p, int B, int Hk, int kv_dt, int out_dt,
                               hipStream_t st, KernelTimer* t) {
    // GMAX sizes the per-lane accumulator array; G <= GMAX is masked
    if (p.G <= 1) return launch_gqa_d<D, 1>(p, B, Hk, kv_dt, out_dt, st, t);
    if (p.G <= 2) return launch_gqa_d<D, 2>(p, B, Hk, kv_dt, out_dt, st, t);
    if (p.G <= 4) return launch_gqa_d<D, 4>(p, B, Hk, kv_dt, out_dt, st, t);
    if (p.G <= 8) return launch_gqa_d<D, 8>(p, B, Hk, kv_dt, out_dt, st, t);
    return launch_gqa_d<D, 16>(p, B, Hk, kv_dt, out_dt, st, t);
}

hipError_t launch_gqa_decode(const GqaDecodeParams& p, int B, int Hk, int D, int kv_dt, int out_dt,
                             hipStream_t st, KernelTimer* t) {
    if (D == 128) return launch_gqa_g<128>(p, B, Hk, kv_dt, out_dt, st, t);
    return launch_gqa_g<64>(p, B, Hk, kv_dt, out_dt, st, t);
}

}  // namespace mugen_attn
