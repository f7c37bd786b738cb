// gqa_decode.hip -- split-K GQA decode over a token-major fp16/bf16 K/V cache.
//
// Semantics: cpu_attention (src/core/model/transformer.cpp:2441-2485) and the
// Metal flash_attention_decode (src/metal/kernel_sources.h:2900-2999): one
// query token per head, kv head = h / (H/Hk), softmax(q.K^T * scale) V with
// fp32 accumulation.
//
// Design (HBM-bound: ~7 flop per K/V byte at the 7B shape):
//  * one workgroup = (context split, kv head, sequence); all G = H/Hk
//    (<= 16) query heads of the group are served from ONE read of the
//    group's K/V rows (the Metal kernel re-reads them once per query head);
//  * 4 waves; wave w takes 32-token blocks w, w+4, ... of the split and
//    loads the next block's K and V into registers while computing the
//    current one;
//  * S^T[32 tok x 16 heads] = K . Q^T on MFMA 16x16x32: K rows are the A
//    operand straight from global memory, read in the token permutation
//    that leaves each lane 8 consecutive tokens of its head (A row m of
//    block nb is token 8*(m/4) + 4*nb + m%4); Q^T stays in registers and
//    heads >= G are zero columns whose weights are forced to 0;
//  * O^T[D x 16 heads] += V^T . P^T on MFMA as well: P is the B operand
//    straight from registers (fp16, or bf16 hi + lo for 16 significant
//    bits), V^T the A operand, staged through a per-wave LDS buffer
//    (XOR-swizzled rows) and read with ds_read_b64_tr_b16; each lane owns
//    one head, so softmax factors never cross lanes;
//  * online softmax in the exp2 domain with a lazy max (a head is re-based
//    only when a weight would exceed 2^8);
//  * the grid is a compact list of the active (sequence, split, kv head)
//    items -- max(1, ceil(T_b / chunk)) splits per sequence -- that the host
//    planner sizes to one dispatch round (two workgroups per CU);
//  * the 4 waves merge (m, l, o) through LDS; with one split the result is
//    normalised and stored, otherwise (m, l, o) partials go to the
//    workspace and gqa_decode_combine merges them with fp32 log-sum-exp.
#include "common.h"
#include "kernels.h"

namespace mugen_attn {

namespace {

// 16-byte chunk c of staged V row r is stored at chunk c ^ vswz<D>(r): the
// transpose reads of lane groups g, g+1 (rows 8g + r', r' < 4, chunks 2d,
// 2d + 1) then hit distinct banks (rows of 128 B for D = 64, 256 B for 128)
template <int D>
__device__ constexpr int vswz(int r) {
    if constexpr (D == 64)
        return (((r >> 1) & 1) * 2) ^ (((r >> 3) & 1) * 4) ^ ((r >> 4) & 1);
    else
        return ((r & 1) * 2) ^ (((r >> 1) & 1) * 4) ^ (((r >> 3) & 1) * 8) ^ ((r >> 4) & 1);
}

// Eight values of a 20-byte 4-bit group (dequantize_group,
// kv_cache.cpp:58-73): `sm` = the group's f16 scale (low half) and min
// (high half), `nib` = the 4 bytes holding values 2i (low nibble) and 2i+1
// (high nibble); each value f16(min + nibble * scale).  nibble * scale is
// exact in fp32 (4 x 11 significant bits), so one fma rounds exactly like
// the reference's product-then-sum; the nibbles are masked into bytes and
// converted with the byte-select conversions.
__device__ __forceinline__ u32x4_t dequant_q4x8(uint32_t sm, uint32_t nib) {
    const float sf = lo_f32<DT_F16>(sm), mf = hi_f32<DT_F16>(sm);
    const uint32_t lo = nib & 0x0f0f0f0fu, hi = (nib >> 4) & 0x0f0f0f0fu;
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; e++)
        w[e] = pack2<DT_F16>(fmaf((float)((lo >> (8 * e)) & 0xffu), sf, mf),
                             fmaf((float)((hi >> (8 * e)) & 0xffu), sf, mf));
    return u32x4_t{w[0], w[1], w[2], w[3]};
}

// splits of sequence j in the compact work list: ceil(T / chunk) (at least
// one), or for the 4-bit store those of the Q4 tokens plus those of the f16
// ring tokens (at least one)
template <bool Q4>
__device__ __forceinline__ int splits_of(const GqaDecodeParams& p, int j) {
    const int Tj = clamp_len(p.seq_lens[j], p.max_T);
    if constexpr (Q4) {
        const int nqj = min(p.n_q4[j], max(Tj, 0));
        const int n = (nqj + p.chunk - 1) / p.chunk + (max(Tj - nqj, 0) + p.chunk - 1) / p.chunk;
        return n > 0 ? n : 1;
    } else {
        return Tj > 0 ? (Tj + p.chunk - 1) / p.chunk : 1;
    }
}

}  // namespace

// two waves per SIMD (the planner sizes the grid for two workgroups per CU)
// PAD: head_dim p.hd < D (dims past it masked); otherwise p.hd == D
// (head_dim 256: one wave per SIMD, so that its operands fit in registers).
// PF: prompt mode (see GqaDecodeParams::pf_start).
template <int D, int DT, int OUT_DT, bool Q4 = false, bool PAD = false, bool PF = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D > 128 ? 1 : 2))) void gqa_decode_kernel(
    GqaDecodeParams p) {
    constexpr int KK = D / 32;           // MFMA k-steps of S
    constexpr int DB = D / 16;           // 16-dim blocks of O^T
    constexpr int RB = 2 * D;            // bytes per staged V row
    constexpr int VL = 32 * RB / 1024;   // 16-byte V loads per lane per 32-token block
    constexpr int RPL = 1024 / RB;       // V rows per load instruction
    constexpr int NP = p_terms<DT>();
    constexpr float kHeadroom = 8.f;
    // per-wave V staging (32 rows), reused after the loop for the wave merge
    constexpr int STAGE = 4 * 32 * RB;
    constexpr int OROW = D + 4;  // merge rows padded: lanes n of one write land on distinct banks
    constexpr int MERGE = 4 * 16 * OROW * 4 + 2 * 4 * 16 * 4 + 4 * 16 * 4 + 2 * 16 * 4;
    __shared__ __attribute__((aligned(16))) char lds[STAGE > MERGE ? STAGE : MERGE];

    // compact work list: item r of sequence b is split r / Hk of kv head r % Hk
    int b = -1, s = 0, kvh = 0;
    // 4-bit store: a kv head's 80-byte group run shares cache lines with its
    // neighbours', so the kv heads of one (sequence, split) -- consecutive
    // items -- go to one XCD (workgroups are dealt to the 8 XCDs round-robin
    // by blockIdx): item = xcd * per_xcd + slot
    const int item = (Q4 && p.per_xcd > 0) ? (int)(blockIdx.x % 8) * p.per_xcd + (int)(blockIdx.x / 8) : (int)blockIdx.x;
    if constexpr (PF) {  // prompt mode: one split per (token, kv head)
        if (item < p.B * p.Hk) {
            b = item / p.Hk;
            kvh = item - b * p.Hk;
        }
    } else
    for (int j = 0, r = item; j < p.B; j++) {  // uniform scalar loop over the batch
        const int nsj = splits_of<Q4>(p, j);
        if (r < nsj * p.Hk) {
            b = j;
            s = r / p.Hk;
            kvh = r - s * p.Hk;
            break;
        }
        r -= nsj * p.Hk;
    }
    if (b < 0) return;  // grid padding (sized from an upper bound)
    // a split past the workspace's stride (a device length above the host
    // copy the plan was made from): nothing to write it to
    if (p.num_splits > 1 && s >= p.num_splits) return;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int T = PF ? (p.pf_causal ? min(p.pf_start + b + 1, p.max_T) : p.max_T) : clamp_len(p.seq_lens[b], p.max_T);
    // 4-bit store: the Q4 tokens [0, n_q4) and the f16 ring tokens
    // [n_q4, T) are split separately, so a split -- and every 32-token block
    // of it -- holds one kind only (Q4 splits first)
    const int nq = Q4 ? min(p.n_q4[b], max(T, 0)) : 0;
    const int nsq = Q4 ? (nq + p.chunk - 1) / p.chunk : 0;
    const bool q4_split = Q4 && s < nsq;
    const int t_begin = q4_split || !Q4 ? s * p.chunk : nq + (s - nsq) * p.chunk;
    const int t_end = min(t_begin + p.chunk, q4_split ? nq : T);
    if (p.num_splits > 1 && t_begin >= t_end) return;  // empty split (T <= 0): the combine skips it
    MUGEN_TRACE(0);
    const int G = p.G;
    const int h0 = kvh * G;

    // head_dim hd below the kernel's D: q's dims >= hd are zero, and the K / V
    // loads of those dims re-read dims (x mod hd) of the same head and token
    // (finite cache values: they meet q's zeros in S, and O's columns >= hd
    // are never stored), so every lane's loads stay uniform and in bounds
    const int hd = PAD ? p.hd : D;
    auto dim_alias = [&](int x) {
        if constexpr (PAD) return x < hd ? x : x % hd;
        else return x;
    };
    const uint16_t* kbase = p.k + (int64_t)b * p.seq_stride + (int64_t)kvh * hd;
    const uint16_t* vbase = p.v + (int64_t)b * p.seq_stride + (int64_t)kvh * hd;
    // 4-bit store: tokens below nq are 20-byte groups (group kvh*D/32 + c of
    // a token row holds dims 32c .. 32c+31 of this kv head), the rest f16
    // ring rows (token t at slot t % ring, a power of two).  The Q4 rows are
    // read through buffer resources (one per sequence, 32-bit offsets) a
    // whole group run per load, arrive raw and are expanded one block later
    // (unpack_block), so the loads stay in flight:
    //  * K: in a Q4 split the S contraction runs over a permuted dim order --
    //    in MFMA k-step kk lane (g, n) supplies dims 8*KK*g + 8kk .. +7, so
    //    a lane's dims are one contiguous run of 8*KK inside one group, and q
    //    is loaded in the same order (S = K.Q^T is unchanged).  Per token a
    //    lane reads the group's (scale|min) dword and its 4*KK nibble bytes:
    //    two loads instead of 2*KK;
    //  * V: a lane reads whole groups (dword + 16 bytes) and writes their 32
    //    dequantised values to the staging rows itself.
    const int64_t q4sb = Q4 ? (int64_t)b * p.q4_seq_stride : 0;
    const __amdgpu_buffer_rsrc_t rq4k =
        __builtin_amdgcn_make_buffer_rsrc((void*)(Q4 ? p.q4k + q4sb : nullptr), 0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rq4v =
        __builtin_amdgcn_make_buffer_rsrc((void*)(Q4 ? p.q4v + q4sb : nullptr), 0, 0x7fffffff, 0x00020000);
    const uint32_t q4head = (uint32_t)kvh * (D / 32) * 20;
    // byte offset of group gq (of this kv head) of token t
    auto q4_off = [&](int t, int gq) -> int {
        return (int)((uint32_t)t * (uint32_t)p.q4_row_bytes + q4head + (uint32_t)(gq * 20));
    };
    constexpr int NGV = D / 64;  // V groups per lane per 32-token block
    auto load_f16 = [&](const uint16_t* base, int t, int d0) -> u32x4_t {
        if constexpr (Q4) return load16(base + ((uint32_t)(t & (p.ring - 1)) * (uint32_t)p.row_stride + (uint32_t)d0));
        else return load16(base + (int64_t)t * p.row_stride + d0);
    };
    // Q^T as the B operand: lane holds q[head n][32kk + 8g .. +8] (Q4
    // splits: q[head n][8*KK*g + 8kk .. +8], the permuted order above)
    u32x4_t qf[KK];
    if (n < G) {
        const uint16_t* qp = p.q + ((int64_t)b * p.H + h0 + n) * hd;
#pragma unroll
        for (int kk = 0; kk < KK; kk++) {
            const int dq = q4_split ? 8 * KK * g + 8 * kk : 32 * kk + 8 * g;  // (4-bit store: hd == D)
            qf[kk] = (!PAD || dq < hd) ? load16(qp + dq) : u32x4_t{0, 0, 0, 0};
        }
    } else {
#pragma unroll
        for (int kk = 0; kk < KK; kk++) qf[kk] = u32x4_t{0, 0, 0, 0};
    }

    // block loads: K rows in the permuted order (A operand), V rows coalesced
    const int kr0 = 8 * (n >> 2) + (n & 3);  // + 4nb
    int kd[KK];  // the lane's K dims per k-step, and its V dim
#pragma unroll
    for (int kk = 0; kk < KK; kk++) kd[kk] = dim_alias(32 * kk + 8 * g);
    const int vd = dim_alias(8 * (lane % (RB / 16)));
    // QB: this split's tokens are Q4 groups (a compile-time kind, so the
    // main loop has no data-dependent branches around its loads and the
    // prefetch's wait counts stay exact)
    auto load_block = [&](int t0, u32x4_t (&kq)[2][KK], u32x4_t (&vq)[VL], auto qb_tag) {
        constexpr bool QB = decltype(qb_tag)::value;
        if constexpr (QB) {
            // K: kq[nb][0] = the lane's 4*KK nibble bytes, kq[nb][1][0] = (scale|min)
            // (head_dim 256: the lane's 64 dims are two groups, the second in
            // kq[nb][2] / kq[nb][3][0])
            const int d0 = 8 * KK * g;
#pragma unroll
            for (int nb = 0; nb < 2; nb++) {
                const int tk = min(t0 + kr0 + 4 * nb, t_end - 1);
                if constexpr (KK == 8) {
#pragma unroll
                    for (int h2 = 0; h2 < 2; h2++) {
                        const int off = q4_off(tk, 2 * g + h2);
                        kq[nb][2 * h2] = __builtin_amdgcn_raw_buffer_load_b128(rq4k, off + 4, 0, 0);
                        kq[nb][2 * h2 + 1][0] = __builtin_amdgcn_raw_buffer_load_b32(rq4k, off, 0, 0);
                    }
                    continue;
                }
                const int off = q4_off(tk, d0 >> 5);
                const int noff = off + 4 + ((d0 & 31) >> 1);
                if constexpr (KK == 4) {
                    kq[nb][0] = __builtin_amdgcn_raw_buffer_load_b128(rq4k, noff, 0, 0);
                } else {
                    const auto h = __builtin_amdgcn_raw_buffer_load_b64(rq4k, noff, 0, 0);
                    kq[nb][0][0] = h[0];
                    kq[nb][0][1] = h[1];
                }
                kq[nb][1][0] = __builtin_amdgcn_raw_buffer_load_b32(rq4k, off, 0, 0);
            }
            // V: group G = lane + 64i of the block (row G / (D/32), group G % (D/32)):
            // vq[2i] = its 16 nibble bytes, vq[2i+1][0] = its (scale|min)
#pragma unroll
            for (int i = 0; i < NGV; i++) {
                const int G = lane + 64 * i;
                const int tv = min(t0 + G / (D / 32), t_end - 1);
                const int off = q4_off(tv, G % (D / 32));
                vq[2 * i] = __builtin_amdgcn_raw_buffer_load_b128(rq4v, off + 4, 0, 0);
                vq[2 * i + 1][0] = __builtin_amdgcn_raw_buffer_load_b32(rq4v, off, 0, 0);
            }
        } else {
#pragma unroll
            for (int nb = 0; nb < 2; nb++) {
                const int tk = min(t0 + kr0 + 4 * nb, t_end - 1);
#pragma unroll
                for (int kk = 0; kk < KK; kk++) kq[nb][kk] = load_f16(kbase, tk, PAD ? kd[kk] : 32 * kk + 8 * g);
            }
#pragma unroll
            for (int j = 0; j < VL; j++) {
                const int tv = min(t0 + j * RPL + lane / (RB / 16), t_end - 1);
                vq[j] = load_f16(vbase, tv, PAD ? vd : 8 * (lane % (RB / 16)));
            }
        }
    };
    // V staging: load j of lane l is row j*RPL + l/(RB/16), chunk l%(RB/16)
    char* stage = &lds[w * 32 * RB];
    uint32_t st_off[VL];
#pragma unroll
    for (int j = 0; j < VL; j++) {
        const int r = j * RPL + lane / (RB / 16), c = lane % (RB / 16);
        // Q4 splits: chunk j % 4 of the lane's group j / 4 (see load_block)
        const int G = lane + 64 * (j >> 2);
        const int rq = G / (D / 32), cq = 4 * (G % (D / 32)) + (j & 3);
        st_off[j] = q4_split ? rq * RB + ((cq ^ vswz<D>(rq)) * 16) : r * RB + ((c ^ vswz<D>(r)) * 16);
    }
    // transpose reads: lane (g, n) reads row 8g + n/4 (+4), logical bytes
    // 32d + 8(n%4) = chunk 2d + (n%4)/2, half n%2
    const int tr = 8 * g + (n >> 2);
    uint32_t t_off[DB];
#pragma unroll
    for (int d = 0; d < DB; d++)
        t_off[d] = tr * RB + (((2 * d + ((n & 3) >> 1)) ^ vswz<D>(tr)) * 16) + 8 * (n & 1);

    f32x4_t o[DB];  // lane (g, n): O[head n][16d + 4g + i]
#pragma unroll
    for (int d = 0; d < DB; d++) o[d] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float m_run = kNegInf;  // running max (log2 domain) of head n
    float l_part = 0.f;     // this lane's share of head n's sum

    // 4-bit store: the block's Q4 loads arrive raw and are expanded here,
    // one block after they were issued, so the loads stay in flight
    auto unpack_block = [&](u32x4_t (&kq)[2][KK], u32x4_t (&vq)[VL], auto qb_tag) {
        if constexpr (decltype(qb_tag)::value) {
#pragma unroll
            for (int nb = 0; nb < 2; nb++) {
                if constexpr (KK == 8) {
                    const u32x4_t nib0 = kq[nb][0], nib1 = kq[nb][2];
                    const uint32_t sm0 = kq[nb][1][0], sm1 = kq[nb][3][0];
#pragma unroll
                    for (int kk = 0; kk < KK; kk++)
                        kq[nb][kk] = dequant_q4x8(kk < 4 ? sm0 : sm1, kk < 4 ? nib0[kk] : nib1[kk - 4]);
                    continue;
                }
                const u32x4_t nib = kq[nb][0];
                const uint32_t sm = kq[nb][1][0];
#pragma unroll
                for (int kk = 0; kk < KK; kk++) kq[nb][kk] = dequant_q4x8(sm, nib[kk]);
            }
#pragma unroll
            for (int i = NGV - 1; i >= 0; i--) {
                const u32x4_t nib = vq[2 * i];
                const uint32_t sm = vq[2 * i + 1][0];
#pragma unroll
                for (int c = 0; c < 4; c++) vq[4 * i + c] = dequant_q4x8(sm, nib[c]);
            }
        }
    };
    auto main_loop = [&](auto qb_tag) {
    u32x4_t kf[2][KK], kn[2][KK], vf[VL], vn[VL];
    int t0 = t_begin + 32 * w;
    if (t0 < t_end) load_block(t0, kf, vf, qb_tag);
    for (; t0 < t_end; t0 += 128) {
        const bool more = t0 + 128 < t_end;
        if (more) load_block(t0 + 128, kn, vn, qb_tag);  // streams in during this block
        unpack_block(kf, vf, qb_tag);

        // stage V (this wave's buffer: its previous reads are consumed)
#pragma unroll
        for (int j = 0; j < VL; j++) *reinterpret_cast<u32x4_t*>(stage + st_off[j]) = vf[j];

        f32x4_t sacc[2];
#pragma unroll
        for (int nb = 0; nb < 2; nb++) {
            f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < KK; kk++) acc = mfma16x16x32<DT>(kf[nb][kk], qf[kk], acc);
            sacc[nb] = acc;
        }
        // lane (g, n): head n, tokens t0 + 8g + 4nb + i
        float x[8];
        float smax = kNegInf;
#pragma unroll
        for (int nb = 0; nb < 2; nb++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float v = (t0 + 8 * g + 4 * nb + i < t_end) ? sacc[nb][i] * p.scale_log2 : kNegInf;
                x[4 * nb + i] = v;
                smax = fmaxf(smax, v);
            }
        if (__any(smax > m_run + kHeadroom)) {  // re-base head n (wave-uniform branch)
            const float m_new = fmaxf(m_run, max_x32(max_x16(smax)));
            if (m_new > m_run) {
                const float alpha = fast_exp2(m_run - m_new);  // 0 while m_run = -inf
                l_part *= alpha;
#pragma unroll
                for (int d = 0; d < DB; d++) o[d] *= alpha;
                m_run = m_new;
            }
        }
        const float nm = (m_run == kNegInf || n >= G) ? 0.f : -m_run;
        float ps = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            x[e] = n < G ? fast_exp2(x[e] + nm) : 0.f;
            ps += x[e];
        }
        l_part += ps;
        u32x4_t pfr[NP];
        split_p<DT, NP>(x, pfr);

        // O^T += V^T . P^T (staged rows visible to the wave's own reads)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int d = 0; d < DB; d++) {
            const u32x2_t lo = lds_read_tr16(reinterpret_cast<const uint16_t*>(stage + t_off[d]));
            const u32x2_t hi = lds_read_tr16(reinterpret_cast<const uint16_t*>(stage + t_off[d] + 4 * RB));
            const u32x4_t vt = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
            for (int pp = 0; pp < NP; pp++) o[d] = mfma16x16x32<DT>(vt, pfr[pp], o[d]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (more) {
#pragma unroll
            for (int nb = 0; nb < 2; nb++)
#pragma unroll
                for (int kk = 0; kk < KK; kk++) kf[nb][kk] = kn[nb][kk];
#pragma unroll
            for (int j = 0; j < VL; j++) vf[j] = vn[j];
        }
    }
    };
    if (q4_split) {
        if constexpr (Q4) main_loop(std::true_type{});
    } else {
        main_loop(std::false_type{});
    }

    MUGEN_TRACE(1);
    // ---- merge the 4 waves' (m, l, O) per head through LDS
    l_part = sum_x32(sum_x16(l_part));
    __syncthreads();  // staging buffers are free
    float* o_lds = reinterpret_cast<float*>(&lds[0]);   // [4][16][OROW]
    float* m_lds = o_lds + 4 * 16 * OROW;               // [4][16]
    float* l_lds = m_lds + 4 * 16;                      // [4][16]
#pragma unroll
    for (int d = 0; d < DB; d++)
        *reinterpret_cast<f32x4_t*>(&o_lds[(w * 16 + n) * OROW + 16 * d + 4 * g]) = o[d];
    if (g == 0) {
        m_lds[w * 16 + n] = m_run;
        l_lds[w * 16 + n] = l_part;
    }
    // per head: the 4 waves' factors 2^(m_w - M) (divided by the sum when
    // this is the only split), once, then every output element is a 4-term sum
    float* f_lds = l_lds + 4 * 16;    // [4][16]
    float* ml_out = f_lds + 4 * 16;   // [16][2]: the head's (M, L)
    __syncthreads();
    if (threadIdx.x < 16) {
        const int h = threadIdx.x;
        float M = kNegInf;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) M = fmaxf(M, m_lds[ww * 16 + h]);
        float f[4], L = 0.f;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) {
            const float mw = m_lds[ww * 16 + h];
            f[ww] = (mw == kNegInf) ? 0.f : fast_exp2(mw - M);
            L += f[ww] * l_lds[ww * 16 + h];
        }
        const float c = p.num_splits == 1 ? (L > 0.f ? 1.f / L : 0.f) : 1.f;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) f_lds[ww * 16 + h] = f[ww] * c;
        ml_out[2 * h] = M;
        ml_out[2 * h + 1] = L;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < G * D; idx += 256) {
        const int h = idx / D, d = idx - h * D;
        float O = 0.f;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) O += f_lds[ww * 16 + h] * o_lds[(ww * 16 + h) * OROW + d];
        const int64_t bh = (int64_t)b * p.H + h0 + h;
        if (p.num_splits == 1) {
            if (!PAD || d < hd) store_out<OUT_DT>(p.out, bh * hd + d, O);
        } else {
            const int64_t slot = bh * p.num_splits + s;
            p.ws_o[slot * D + d] = O;
            if (d == 0) {
                p.ws_ml[slot * 2 + 0] = ml_out[2 * h];
                p.ws_ml[slot * 2 + 1] = ml_out[2 * h + 1];
            }
        }
    }
    MUGEN_TRACE(2);
}

// Log-sum-exp merge of the split partials of one (sequence, head); thread d
// owns output dim d.
//  * up to 64 splits (every decode plan at 7B-class shapes): each wave
//    reads all (m, l) pairs (lane s holds split s) and forms the weights with
//    wave reductions, while the first kPre splits' partials are already in
//    flight -- one memory round trip, no block barrier;
//  * more splits: the weights are formed block-wide in LDS (lse_weights),
//    then the partials are summed 8 splits at a time.
template <int D, int OUT_DT, bool PAD>
__global__ __launch_bounds__(64) void gqa_decode_combine_kernel(GqaDecodeParams p) {
    constexpr int kPre = 32;
    __shared__ float f_lds[kMaxSplits];
    __shared__ float red_lds[4];
    const int h = blockIdx.x, b = blockIdx.y, d = blockIdx.z * 64 + threadIdx.x;
    MUGEN_TRACE(8);
    const int T = clamp_len(p.seq_lens[b], p.max_T);
    const int nact = p.n_q4 ? min(p.num_splits, T > 0 ? splits_of<true>(p, b) : 0)
                            : min(p.num_splits, (T + p.chunk - 1) / p.chunk);
    const int64_t bh = (int64_t)b * p.H + h;
    const float* ml = p.ws_ml + bh * p.num_splits * 2;
    const float* os = p.ws_o + bh * p.num_splits * D + d;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float inv;
    if (nact <= 64) {
        const int lane = d & 63;
        float* fw = &f_lds[0];  // this wave's weights
        const float ms = lane < nact ? ml[2 * lane] : kNegInf;
        const float ls = lane < nact ? ml[2 * lane + 1] : 0.f;
        float v[kPre];  // clamped, unconditional loads: exact wait counts
#pragma unroll
        for (int j = 0; j < kPre; j++) v[j] = os[(int64_t)max(0, min(j, nact - 1)) * D];
        const float M = wave_max(ms);
        const float f = (ms == kNegInf) ? 0.f : fast_exp2(ms - M);
        const float L = wave_sum(f * ls);
        inv = L > 0.f ? 1.f / L : 0.f;
        fw[lane] = f;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int j = 0; j < kPre; j++)
            if (j < nact) acc[j & 7] += fw[j] * v[j];
        for (int s = kPre; s < nact; s += 8) {
            float u[8];
#pragma unroll
            for (int j = 0; j < 8; j++) u[j] = os[(int64_t)min(s + j, nact - 1) * D];
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (s + j < nact) acc[j] += fw[s + j] * u[j];
        }
    } else {
        // this thread's split (m, l), then the first 8 splits' partials,
        // all in flight before the weights are formed
        const int ts = threadIdx.x;  // this thread's split for the weights (lse_weights' convention)
        const float m0 = ts < nact ? ml[2 * ts] : kNegInf, l0 = ts < nact ? ml[2 * ts + 1] : 0.f;
        float v0[8];
#pragma unroll
        for (int j = 0; j < 8; j++) v0[j] = os[(int64_t)j * D];
        inv = lse_weights(ml, 2, nact, m0, l0, f_lds, red_lds);
#pragma unroll
        for (int j = 0; j < 8; j++) acc[j] = f_lds[j] * v0[j];
        int s = 8;
        for (; s + 8 <= nact; s += 8) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = os[(int64_t)(s + j) * D];
#pragma unroll
            for (int j = 0; j < 8; j++) acc[j] += f_lds[s + j] * v[j];
        }
        for (; s < nact; s++) acc[0] += f_lds[s] * os[(int64_t)s * D];
    }
    const float O = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
    const int hd = PAD ? p.hd : D;
    if (!PAD || d < hd) store_out<OUT_DT>(p.out, bh * hd + d, O * inv);
    MUGEN_TRACE(9);
}

// ------------------------------------------------------------------ launch

template <int D, int DT, int OUT_DT, bool Q4 = false>
static hipError_t launch_gqa_t(const GqaDecodeParams& p, int nwg, hipStream_t st, KernelTimer* timer) {
    const int grid = (Q4 && p.per_xcd > 0) ? 8 * p.per_xcd : nwg;
    hipError_t e = (!Q4 && p.hd != D)
                       ? launch_k(timer, "gqa_decode", gqa_decode_kernel<D, DT, OUT_DT, false, true>, dim3(grid),
                                  dim3(256), st, p)
                       : launch_k(timer, "gqa_decode", gqa_decode_kernel<D, DT, OUT_DT, Q4>, dim3(grid), dim3(256), st, p);
    if (e != hipSuccess || p.num_splits == 1) return e;
    if (!Q4 && p.hd != D)
        return launch_k(timer, "gqa_decode_combine", gqa_decode_combine_kernel<D, OUT_DT, true>, dim3(p.H, p.B, D / 64),
                        dim3(64), st, p);
    return launch_k(timer, "gqa_decode_combine", gqa_decode_combine_kernel<D, OUT_DT, false>, dim3(p.H, p.B, D / 64), dim3(64),
                    st, p);
}

template <int D, int DT>
static hipError_t launch_gqa_o(const GqaDecodeParams& p, int nwg, int out_dt, hipStream_t st, KernelTimer* t) {
    switch (out_dt) {
        case DT_F32: return launch_gqa_t<D, DT, DT_F32>(p, nwg, st, t);
        case DT_F16: return launch_gqa_t<D, DT, DT_F16>(p, nwg, st, t);
        default: return launch_gqa_t<D, DT, DT_BF16>(p, nwg, st, t);
    }
}

template <int D>
static hipError_t launch_gqa_g(const GqaDecodeParams& p, int nwg, int kv_dt, int out_dt, hipStream_t st,
                               KernelTimer* t) {
    if (kv_dt == DT_F16) return launch_gqa_o<D, DT_F16>(p, nwg, out_dt, st, t);
    return launch_gqa_o<D, DT_BF16>(p, nwg, out_dt, st, t);
}

hipError_t launch_gqa_decode(const GqaDecodeParams& p, int nwg, int D, int kv_dt, int out_dt, hipStream_t st,
                             KernelTimer* t) {
    if (D == 256) return launch_gqa_g<256>(p, nwg, kv_dt, out_dt, st, t);
    if (D == 128) return launch_gqa_g<128>(p, nwg, kv_dt, out_dt, st, t);
    return launch_gqa_g<64>(p, nwg, kv_dt, out_dt, st, t);
}

// prompt mode at head_dim 129..256 (one split per item: no combine)
template <int DT, int OUT_DT>
static hipError_t launch_pf_wide_t(const GqaDecodeParams& p, hipStream_t st, KernelTimer* t) {
    const dim3 grid(p.B * p.Hk);
    if (p.hd != 256)
        return launch_k(t, "gqa_prefill", gqa_decode_kernel<256, DT, OUT_DT, false, true, true>, grid, dim3(256), st, p);
    return launch_k(t, "gqa_prefill", gqa_decode_kernel<256, DT, OUT_DT, false, false, true>, grid, dim3(256), st, p);
}

template <int DT>
static hipError_t launch_pf_wide_o(const GqaDecodeParams& p, int out_dt, hipStream_t st, KernelTimer* t) {
    switch (out_dt) {
        case DT_F32: return launch_pf_wide_t<DT, DT_F32>(p, st, t);
        case DT_F16: return launch_pf_wide_t<DT, DT_F16>(p, st, t);
        default: return launch_pf_wide_t<DT, DT_BF16>(p, st, t);
    }
}

hipError_t launch_gqa_prefill_wide(const GqaDecodeParams& p, int kv_dt, int out_dt, hipStream_t st, KernelTimer* t) {
    if (kv_dt == DT_F16) return launch_pf_wide_o<DT_F16>(p, out_dt, st, t);
    return launch_pf_wide_o<DT_BF16>(p, out_dt, st, t);
}

// 4-bit store: f16 values (the reference's format), fp16 MFMA
template <int D>
static hipError_t launch_gqa_q4_d(const GqaDecodeParams& p, int nwg, int out_dt, hipStream_t st, KernelTimer* t) {
    switch (out_dt) {
        case DT_F32: return launch_gqa_t<D, DT_F16, DT_F32, true>(p, nwg, st, t);
        case DT_F16: return launch_gqa_t<D, DT_F16, DT_F16, true>(p, nwg, st, t);
        default: return launch_gqa_t<D, DT_F16, DT_BF16, true>(p, nwg, st, t);
    }
}

hipError_t launch_gqa_decode_q4(const GqaDecodeParams& p, int nwg, int D, int out_dt, hipStream_t st, KernelTimer* t) {
    if (D == 256) return launch_gqa_q4_d<256>(p, nwg, out_dt, st, t);
    if (D == 128) return launch_gqa_q4_d<128>(p, nwg, out_dt, st, t);
    return launch_gqa_q4_d<64>(p, nwg, out_dt, st, t);
}

}  // namespace mugen_attn
