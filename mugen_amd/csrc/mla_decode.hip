// mla_decode.hip -- MLA absorbed attention over the 576-dim latent cache.
//
// Semantics: the latent core of cpu_mla_attention
// (src/core/model/transformer.cpp:2576-2608): for each query row (head h of
// verify token i) score_t = (q[0:512].c_t[0:512] + q[512:576].c_t[512:576])
// * scale, softmax over the row's visible tokens, o = sum_t p_t c_t[0:512].
// Query i of q_len sees seq_len - q_len + i + 1 tokens (the per-token calls
// seq_len = start_position + t + 1 at transformer.cpp:1325-1337).
//
// Design: all heads share one latent row, so attention is a pair of dense
// contractions, S = Q[rows x 576] . L^T and O = P . L[:, 0:512], run on
// MFMA 16x16x32 (bf16 or fp16 in, fp32 accumulate):
//  * workgroup = (block of 64*MB query rows, context split, sequence);
//    4 waves, each owning 16*MB rows; Q of those rows stays in registers as
//    the B operand of S^T = L . Q^T; O[rows x 512] is accumulated in
//    registers (MB x 32 MFMA tiles per wave);
//  * latent tiles of 32 tokens are staged into LDS (padded rows, 16-byte
//    reads conflict-free), the next tile is prefetched into registers while
//    the current one is consumed;
//  * S^T uses a token permutation (A-row m of token block nb is token
//    8*(m/4) + 4*nb + m%4) so that each lane ends up holding 8 CONSECUTIVE
//    tokens of its query row: exactly the k-slots of its P operand for the
//    P.L product, so P never leaves registers;
//  * online softmax in the exp2 domain; the split-K partials (m, l, o) are
//    merged by mla_decode_combine with fp32 log-sum-exp.
//  * q in fp32 is split into hi + lo 16-bit halves (two MFMAs), which keeps
//    the scores fp32-accurate like the reference's float q_absorbed;
//  * with a bf16 cache P is split the same way (hi + lo bf16, two MFMAs on
//    one latent B operand), keeping the weights at ~2^-17 relative error.
#include "common.h"
#include "kernels.h"

namespace mugen_attn {

constexpr int kKR = 512;               // kv_lora_rank
constexpr int kRD = 64;                // rope dims
constexpr int kCD = kKR + kRD;         // 576 latent dims per token
constexpr int kTT = 32;                // tokens per LDS tile
constexpr int kLROW = kCD + 8;         // LDS row stride (halves): 1168 B
constexpr int kChunks = kTT * kCD / 8; // 16-byte chunks per tile (2304)
constexpr int kCPT = kChunks / 256;    // chunks per thread (9)

template <int MB, int QDT, int DT, int OUT_DT>
__global__ __launch_bounds__(256) void mla_decode_kernel(MlaParams p) {
    constexpr int KS = kCD / 32;  // 18 k-steps over the 576 dims
    constexpr int NQ = (QDT == DT_F32) ? 2 : 1;
    constexpr int NP = p_terms<DT>();
    __shared__ __attribute__((aligned(16))) uint16_t lds[kTT * kLROW];

    const int rb = blockIdx.x, s = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int T = p.seq_lens[b];
    const int t_begin = s * p.chunk;
    const int t_end = min(t_begin + p.chunk, T);
    if (p.num_splits > 1 && t_begin >= T) return;

    const int row0 = rb * (64 * MB) + w * (16 * MB);
    const uint16_t* lat = p.lat + (int64_t)b * p.seq_stride;

    // ---- Q^T fragments (B operand): lane holds Q[row0+16mb+n][32ks+8g .. +8]
    u32x4_t qf[MB][NQ][KS];
    int teff[MB];  // visible tokens of this lane's S-row
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
        const int row = row0 + 16 * mb + n;
        const bool ok = row < p.R;
        teff[mb] = ok ? (T - p.q_len + row / p.H + 1) : 0;
        const int64_t qoff = ((int64_t)b * p.R + (ok ? row : 0)) * kCD + 8 * g;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            if constexpr (QDT == DT_F32) {
                const float* qp = static_cast<const float*>(p.q) + qoff + 32 * ks;
                float x[8];
#pragma unroll
                for (int j = 0; j < 8; j++) x[j] = ok ? qp[j] : 0.f;
                uint32_t hi[4], lo[4];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint16_t h0 = from_f32<DT>(x[2 * j]), h1 = from_f32<DT>(x[2 * j + 1]);
                    hi[j] = uint32_t(h0) | (uint32_t(h1) << 16);
                    lo[j] = pack2<DT>(x[2 * j] - to_f32<DT>(h0), x[2 * j + 1] - to_f32<DT>(h1));
                }
                qf[mb][0][ks] = u32x4_t{hi[0], hi[1], hi[2], hi[3]};
                qf[mb][NQ - 1][ks] = u32x4_t{lo[0], lo[1], lo[2], lo[3]};
            } else {
                const uint16_t* qp = static_cast<const uint16_t*>(p.q) + qoff + 32 * ks;
                qf[mb][0][ks] = ok ? load16(qp) : u32x4_t{0, 0, 0, 0};
            }
        }
    }

    f32x4_t o[MB][32];
    float m_run[MB], l_part[MB];
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
        m_run[mb] = kNegInf;
        l_part[mb] = 0.f;
#pragma unroll
        for (int d = 0; d < 32; d++) o[mb][d] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }

    // ---- tile staging: chunk c = tid + 256*i -> token c/72, dims (c%72)*8
    u32x4_t pf[kCPT];
    auto fetch = [&](int tt) {
#pragma unroll
        for (int i = 0; i < kCPT; i++) {
            const int c = tid + 256 * i;
            const int tok = min(tt + c / 72, t_end - 1);
            pf[i] = load16(lat + (int64_t)tok * kCD + (c % 72) * 8);
        }
    };
    if (t_begin < t_end) fetch(t_begin);

    // A-operand row of token block nb for this lane: token 8*(n/4) + 4*nb + n%4
    const int arow0 = 8 * (n >> 2) + (n & 3);

    for (int tt = t_begin; tt < t_end; tt += kTT) {
        __syncthreads();  // previous tile fully consumed
#pragma unroll
        for (int i = 0; i < kCPT; i++) {
            const int c = tid + 256 * i;
            *reinterpret_cast<u32x4_t*>(&lds[(c / 72) * kLROW + (c % 72) * 8]) = pf[i];
        }
        __syncthreads();
        if (tt + kTT < t_end) fetch(tt + kTT);

        // ---- S^T = L . Q^T  (two 16-token blocks)
        f32x4_t sacc[MB][2];
#pragma unroll
        for (int mb = 0; mb < MB; mb++) sacc[mb][0] = sacc[mb][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
#pragma unroll
            for (int nb = 0; nb < 2; nb++) {
                const u32x4_t a = *reinterpret_cast<const u32x4_t*>(
                    &lds[(arow0 + 4 * nb) * kLROW + 32 * ks + 8 * g]);
#pragma unroll
                for (int mb = 0; mb < MB; mb++) {
#pragma unroll
                    for (int qq = 0; qq < NQ; qq++)
                        sacc[mb][nb] = mfma16x16x32<DT>(a, qf[mb][qq][ks], sacc[mb][nb]);
                }
            }
        }

        // ---- online softmax; lane holds tokens tt + 8g + (4nb + i) of row n
        u32x4_t pfrag[MB][NP];
        float alpha_row[MB][4];
#pragma unroll
        for (int mb = 0; mb < MB; mb++) {
            float x[8];
            float mt = kNegInf;
#pragma unroll
            for (int nb = 0; nb < 2; nb++) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int tok = tt + 8 * g + 4 * nb + i;
                    const bool vis = tok < t_end && tok < teff[mb];
                    x[4 * nb + i] = vis ? sacc[mb][nb][i] * p.scale_log2 : kNegInf;
                    mt = fmaxf(mt, x[4 * nb + i]);
                }
            }
            mt = fmaxf(mt, wave_xor(mt, 16));
            mt = fmaxf(mt, wave_xor(mt, 32));
            const float m_new = fmaxf(m_run[mb], mt);
            const float m_use = (m_new == kNegInf) ? 0.f : m_new;
            const float alpha = fast_exp2(m_run[mb] - m_use);
            float ps = 0.f;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                x[j] = fast_exp2(x[j] - m_use);
                ps += x[j];
            }
            l_part[mb] = l_part[mb] * alpha + ps;
            m_run[mb] = m_new;
            split_p<DT, NP>(x, pfrag[mb]);
            // O rows are 4g+i: fetch their alpha from lane (4g+i)
#pragma unroll
            for (int i = 0; i < 4; i++) alpha_row[mb][i] = __shfl(alpha, 4 * g + i, 64);
        }
#pragma unroll
        for (int mb = 0; mb < MB; mb++) {
#pragma unroll
            for (int d = 0; d < 32; d++) {
#pragma unroll
                for (int i = 0; i < 4; i++) o[mb][d][i] *= alpha_row[mb][i];
            }
        }

        // ---- O += P . L[:, 0:512]; B operand: L[tt + 8g + j][16d + n], j < 8
        const uint16_t* bcol = &lds[(8 * g) * kLROW + n];
#pragma unroll
        for (int d = 0; d < 32; d++) {
            uint32_t bw[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t e0 = bcol[(2 * j) * kLROW + 16 * d];
                const uint32_t e1 = bcol[(2 * j + 1) * kLROW + 16 * d];
                bw[j] = e0 | (e1 << 16);
            }
            const u32x4_t bf = u32x4_t{bw[0], bw[1], bw[2], bw[3]};
#pragma unroll
            for (int mb = 0; mb < MB; mb++) {
#pragma unroll
                for (int pp = 0; pp < NP; pp++) o[mb][d] = mfma16x16x32<DT>(pfrag[mb][pp], bf, o[mb][d]);
            }
        }
    }

    // ---- epilogue
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
        float l = l_part[mb];
        l += wave_xor(l, 16);
        l += wave_xor(l, 32);
        const int srow = row0 + 16 * mb + n;  // S-layout row of this lane
        float l_row[4], inv_row[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            l_row[i] = __shfl(l, 4 * g + i, 64);
            inv_row[i] = l_row[i] > 0.f ? 1.f / l_row[i] : 0.f;
        }
        if (p.num_splits == 1) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int row = row0 + 16 * mb + 4 * g + i;
                if (row < p.R) {
                    const int64_t base = ((int64_t)b * p.R + row) * kKR + n;
#pragma unroll
                    for (int d = 0; d < 32; d++)
                        store_out<OUT_DT>(p.out, base + 16 * d, o[mb][d][i] * inv_row[i]);
                }
            }
        } else {
            const int64_t sbase = ((int64_t)b * p.num_splits + s) * p.R;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int row = row0 + 16 * mb + 4 * g + i;
                if (row < p.R) {
                    float* dst = p.ws_o + (sbase + row) * kKR + n;
#pragma unroll
                    for (int d = 0; d < 32; d++) dst[16 * d] = o[mb][d][i];
                }
            }
            if (g == 0 && srow < p.R) {
                p.ws_ml[(sbase + srow) * 2 + 0] = m_run[mb];
                p.ws_ml[(sbase + srow) * 2 + 1] = l;
            }
        }
    }
}

// Log-sum-exp merge of split partials: one workgroup per (row, sequence),
// 128 threads x 4 dims.
template <int OUT_DT>
__global__ __launch_bounds__(128) void mla_decode_combine_kernel(MlaParams p) {
    const int row = blockIdx.x, b = blockIdx.y, d = threadIdx.x * 4;
    const int T = p.seq_lens[b];
    const int nact = min(p.num_splits, (T + p.chunk - 1) / p.chunk);
    float M = kNegInf;
    for (int s = 0; s < nact; s++)
        M = fmaxf(M, p.ws_ml[(((int64_t)b * p.num_splits + s) * p.R + row) * 2]);
    float L = 0.f;
    f32x4_t O = {0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < nact; s++) {
        const int64_t slot = ((int64_t)b * p.num_splits + s) * p.R + row;
        const float m = p.ws_ml[slot * 2];
        const float f = (m == kNegInf) ? 0.f : fast_exp2(m - M);
        L += f * p.ws_ml[slot * 2 + 1];
        const f32x4_t v = *reinterpret_cast<const f32x4_t*>(p.ws_o + slot * kKR + d);
        O += f * v;
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    const int64_t base = ((int64_t)b * p.R + row) * kKR + d;
#pragma unroll
    for (int c = 0; c < 4; c++) store_out<OUT_DT>(p.out, base + c, O[c] * inv);
}

// ------------------------------------------------------------------ launch

int mla_rows_per_block(int variant) { return 64 * variant; }

template <int MB, int QDT, int DT, int OUT_DT>
static hipError_t launch_mla_t(const MlaParams& p, int B, hipStream_t st, KernelTimer* t) {
    const int nrb = (p.R + 64 * MB - 1) / (64 * MB);
    timer_begin(t, "mla_decode", st);
    hipLaunchKernelGGL((mla_decode_kernel<MB, QDT, DT, OUT_DT>), dim3(nrb, p.num_splits, B),
                       dim3(256), 0, st, p);
    timer_end(t, "mla_decode", st);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || p.num_splits == 1) return e;
    timer_begin(t, "mla_decode_combine", st);
    hipLaunchKernelGGL((mla_decode_combine_kernel<OUT_DT>), dim3(p.R, B), dim3(128), 0, st, p);
    timer_end(t, "mla_decode_combine", st);
    return hipGetLastError();
}

template <int MB, int QDT, int DT>
static hipError_t launch_mla_o(const MlaParams& p, int B, int out_dt, hipStream_t st, KernelTimer* t) {
    if (out_dt == DT_F32) return launch_mla_t<MB, QDT, DT, DT_F32>(p, B, st, t);
    if (out_dt == DT_F16) return launch_mla_t<MB, QDT, DT, DT_F16>(p, B, st, t);
    return launch_mla_t<MB, QDT, DT, DT_BF16>(p, B, st, t);
}

template <int MB>
static hipError_t launch_mla_mb(const MlaParams& p, int B, int q_dt, int lat_dt, int out_dt,
                                hipStream_t st, KernelTimer* t) {
    if (lat_dt == DT_F16) {
        if (q_dt == DT_F32) return launch_mla_o<MB, DT_F32, DT_F16>(p, B, out_dt, st, t);
        return launch_mla_o<MB, DT_F16, DT_F16>(p, B, out_dt, st, t);
    }
    if (q_dt == DT_F32) return launch_mla_o<MB, DT_F32, DT_BF16>(p, B, out_dt, st, t);
    return launch_mla_o<MB, DT_BF16, DT_BF16>(p, B, out_dt, st, t);
}

hipError_t launch_mla_decode(const MlaParams& p, int B, int variant, int q_dt, int lat_dt, int out_dt,
                             hipStream_t st, KernelTimer* t) {
    (void)variant;
    return launch_mla_mb<1>(p, B, q_dt, lat_dt, out_dt, st, t);
}

}  // namespace mugen_attn
