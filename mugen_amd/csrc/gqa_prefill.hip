// gqa_prefill.hip -- causal GQA flash-attention prefill on MFMA.
//
// Semantics: flash_prefill_attention (src/metal/kernel_sources.h:2769-2896):
// Q_batch [N][H][D], K/V cache [kv_len][Hk*D], O_batch [N][H][D]; token i
// attends to keys [0, start_position + i] (kernel_sources.h:2796), kv head
// = h / (H/Hk), scale 1/sqrt(D), fp32 softmax accumulation.
//
// Design (MFMA-bound):
//  * workgroup = (16-token query block, kv head); its 4 waves take the G
//    query heads of that kv head (wave w: heads w, w+4, ...), so every K/V
//    tile staged in LDS feeds all G heads of the group (GQA reuse);
//  * query blocks are launched longest-first (causal rows near the end see
//    the most keys) to shorten the tail;
//  * per 64-key tile: S^T = K . Q^T on MFMA 16x16x32 with the token
//    permutation that leaves each lane 8 consecutive keys of its query row,
//    online softmax in registers, then O += P . V with P taken straight from
//    registers as the A operand and V gathered from LDS as the B operand;
//  * tiles entirely above the causal diagonal are never visited;
//  * with bf16 inputs P is split into hi + lo bf16 terms (two MFMAs on the
//    same V operand): a single bf16 P carries 2^-9 relative error per
//    weight, which short causal rows do not average away.
#include "common.h"
#include "kernels.h"

namespace mugen_attn {

template <int D, int MB, int DT, int OUT_DT>
__global__ __launch_bounds__(256) void gqa_prefill_kernel(GqaPrefillParams p) {
    constexpr int KK = D / 32;     // k-steps of S over head_dim
    constexpr int DB = D / 16;     // 16-wide output column blocks
    constexpr int KT = 64;         // keys per tile
    constexpr int LROW = D + 8;    // padded LDS row (halves)
    constexpr int CPR = D / 8;     // 16-byte chunks per row
    constexpr int CPT = KT * CPR / 256;  // chunks per thread per matrix
    constexpr int NP = p_terms<DT>();    // 16-bit terms P is split into
    __shared__ __attribute__((aligned(16))) uint16_t ks[KT * LROW];
    __shared__ __attribute__((aligned(16))) uint16_t vs[KT * LROW];

    const int qb = gridDim.x - 1 - blockIdx.x;  // longest rows first
    const int kvh = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int t0 = qb * 16;
    const int G = p.G;

    // Q^T fragments: lane holds q[token t0+n][head][32kk + 8g .. +8]
    u32x4_t qf[MB][KK];
    bool head_ok[MB];
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
        const int hg = w + 4 * mb;
        head_ok[mb] = hg < G;
        const int tok = min(t0 + n, p.N - 1);
        const uint16_t* qp = p.q + ((int64_t)tok * p.H + kvh * G + (head_ok[mb] ? hg : 0)) * D + 8 * g;
#pragma unroll
        for (int kk = 0; kk < KK; kk++) qf[mb][kk] = load16(qp + 32 * kk);
    }

    // keys visible to the last token of the block
    int kend = p.kv_len;
    if (p.causal) kend = min(kend, p.start_pos + min(t0 + 16, p.N));
    // this lane's S-row (token t0 + n) limit
    const int row_lim = p.causal ? min(p.start_pos + t0 + n + 1, p.kv_len) : p.kv_len;

    f32x4_t o[MB][DB];
    float m_run[MB], l_part[MB];
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
        m_run[mb] = kNegInf;
        l_part[mb] = 0.f;
#pragma unroll
        for (int d = 0; d < DB; d++) o[mb][d] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }

    const uint16_t* kbase = p.k + (int64_t)kvh * D;
    const uint16_t* vbase = p.v + (int64_t)kvh * D;
    const int arow0 = 8 * (n >> 2) + (n & 3);

    for (int kt = 0; kt < kend; kt += KT) {
        u32x4_t kr[CPT], vr[CPT];
#pragma unroll
        for (int i = 0; i < CPT; i++) {
            const int c = tid + 256 * i;
            const int key = min(kt + c / CPR, kend - 1);
            kr[i] = load16(kbase + (int64_t)key * p.row_stride + (c % CPR) * 8);
            vr[i] = load16(vbase + (int64_t)key * p.row_stride + (c % CPR) * 8);
        }
        __syncthreads();  // previous tile consumed
#pragma unroll
        for (int i = 0; i < CPT; i++) {
            const int c = tid + 256 * i;
            *reinterpret_cast<u32x4_t*>(&ks[(c / CPR) * LROW + (c % CPR) * 8]) = kr[i];
            *reinterpret_cast<u32x4_t*>(&vs[(c / CPR) * LROW + (c % CPR) * 8]) = vr[i];
        }
        __syncthreads();

#pragma unroll
        for (int mb = 0; mb < MB; mb++) {
            if (!head_ok[mb]) continue;
            // S^T for 2 groups of 32 keys, each 2 permuted 16-key blocks
            f32x4_t sacc[2][2];
#pragma unroll
            for (int grp = 0; grp < 2; grp++) {
#pragma unroll
                for (int nb = 0; nb < 2; nb++) {
                    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
                    const uint16_t* arow = &ks[(32 * grp + arow0 + 4 * nb) * LROW + 8 * g];
#pragma unroll
                    for (int kk = 0; kk < KK; kk++)
                        acc = mfma16x16x32<DT>(*reinterpret_cast<const u32x4_t*>(arow + 32 * kk),
                                               qf[mb][kk], acc);
                    sacc[grp][nb] = acc;
                }
            }
            // lane: row t0+n, keys kt + 32grp + 8g + 4nb + i
            float x[2][8];
            float mt = kNegInf;
#pragma unroll
            for (int grp = 0; grp < 2; grp++) {
#pragma unroll
                for (int nb = 0; nb < 2; nb++) {
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int key = kt + 32 * grp + 8 * g + 4 * nb + i;
                        const float v = key < row_lim ? sacc[grp][nb][i] * p.scale_log2 : kNegInf;
                        x[grp][4 * nb + i] = v;
                        mt = fmaxf(mt, v);
                    }
                }
            }
            mt = fmaxf(mt, wave_xor(mt, 16));
            mt = fmaxf(mt, wave_xor(mt, 32));
            const float m_new = fmaxf(m_run[mb], mt);
            const float m_use = (m_new == kNegInf) ? 0.f : m_new;
            const float alpha = fast_exp2(m_run[mb] - m_use);
            float ps = 0.f;
            u32x4_t pfr[2][NP];
#pragma unroll
            for (int grp = 0; grp < 2; grp++) {
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    x[grp][j] = fast_exp2(x[grp][j] - m_use);
                    ps += x[grp][j];
                }
                split_p<DT, NP>(x[grp], pfr[grp]);
            }
            l_part[mb] = l_part[mb] * alpha + ps;
            m_run[mb] = m_new;
            float arow_[4];
#pragma unroll
            for (int i = 0; i < 4; i++) arow_[i] = __shfl(alpha, 4 * g + i, 64);
#pragma unroll
            for (int d = 0; d < DB; d++) {
#pragma unroll
                for (int i = 0; i < 4; i++) o[mb][d][i] *= arow_[i];
            }
            // O += P . V ; B operand V[kt + 32grp + 8g + j][16d + n]
#pragma unroll
            for (int grp = 0; grp < 2; grp++) {
                const uint16_t* bcol = &vs[(32 * grp + 8 * g) * LROW + n];
#pragma unroll
                for (int d = 0; d < DB; d++) {
                    uint32_t bw[4];
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const uint32_t e0 = bcol[(2 * j) * LROW + 16 * d];
                        const uint32_t e1 = bcol[(2 * j + 1) * LROW + 16 * d];
                        bw[j] = e0 | (e1 << 16);
                    }
                    const u32x4_t bf = u32x4_t{bw[0], bw[1], bw[2], bw[3]};
#pragma unroll
                    for (int pp = 0; pp < NP; pp++) o[mb][d] = mfma16x16x32<DT>(pfr[grp][pp], bf, o[mb][d]);
                }
            }
        }
    }

    // epilogue: normalise and store rows t0 + 4g + i
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
        if (!head_ok[mb]) continue;
        float l = l_part[mb];
        l += wave_xor(l, 16);
        l += wave_xor(l, 32);
        const int h = kvh * G + w + 4 * mb;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float lr = __shfl(l, 4 * g + i, 64);
            const float inv = lr > 0.f ? 1.f / lr : 0.f;
            const int tok = t0 + 4 * g + i;
            if (tok < p.N) {
                const int64_t base = ((int64_t)tok * p.H + h) * D + n;
#pragma unroll
                for (int d = 0; d < DB; d++) store_out<OUT_DT>(p.out, base + 16 * d, o[mb][d][i] * inv);
            }
        }
    }
}

// ------------------------------------------------------------------ launch

template <int D, int MB, int DT, int OUT_DT>
static hipError_t launch_pf_t(const GqaPrefillParams& p, int Hk, hipStream_t st, KernelTimer* t) {
    dim3 grid((p.N + 15) / 16, Hk);
    timer_begin(t, "gqa_prefill", st);
    hipLaunchKernelGGL((gqa_prefill_kernel<D, MB, DT, OUT_DT>), grid, dim3(256), 0, st, p);
    timer_end(t, "gqa_prefill", st);
    return hipGetLastError();
}

template <int D, int MB, int DT>
static hipError_t launch_pf_o(const GqaPrefillParams& p, int Hk, int out_dt, hipStream_t st, KernelTimer* t) {
    if (out_dt == DT_F32) return launch_pf_t<D, MB, DT, DT_F32>(p, Hk, st, t);
    if (out_dt == DT_F16) return launch_pf_t<D, MB, DT, DT_F16>(p, Hk, st, t);
    return launch_pf_t<D, MB, DT, DT_BF16>(p, Hk, st, t);
}

template <int D, int MB>
static hipError_t launch_pf_d(const GqaPrefillParams& p, int Hk, int dt, int out_dt, hipStream_t st,
                              KernelTimer* t) {
    if (dt == DT_F16) return launch_pf_o<D, MB, DT_F16>(p, Hk, out_dt, st, t);
    return launch_pf_o<D, MB, DT_BF16>(p, Hk, out_dt, st, t);
}

template <int D>
static hipError_t launch_pf_g(const GqaPrefillParams& p, int Hk, int dt, int out_dt, hipStream_t st,
                              KernelTimer* t) {
    if (p.G <= 4) return launch_pf_d<D, 1>(p, Hk, dt, out_dt, st, t);
    return launch_pf_d<D, 2>(p, Hk, dt, out_dt, st, t);
}

hipError_t launch_gqa_prefill(const GqaPrefillParams& p, int Hk, int D, int dt, int out_dt,
                              hipStream_t st, KernelTimer* t) {
    if (D == 128) return launch_pf_g<128>(p, Hk, dt, out_dt, st, t);
    return launch_pf_g<64>(p, Hk, dt, out_dt, st, t);
}

}  // namespace mugen_attn
