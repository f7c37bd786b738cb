// gqa_prefill.hip -- causal GQA flash-attention prefill on MFMA.
//
// Semantics: flash_prefill_attention (src/metal/kernel_sources.h:2769-2896):
// Q_batch [N][H][D], K/V cache [kv_len][Hk*D], O_batch [N][H][D]; token i
// attends to keys [0, start_position + i] (kernel_sources.h:2796), kv head
// = h / (H/Hk), scale 1/sqrt(D), fp32 softmax accumulation.
//
// Design.  At prefill sizes of a small model (N = 512, 32 heads) the whole
// problem is ~1 GFLOP: the kernel is bound by the length of each
// workgroup's serial tile chain, not by MFMA throughput, so the layout aims
// at a short chain with every load in flight early:
//  * workgroup = (16-token query block, kv head), 8 waves: wave w takes
//    query heads w%4 (+4) of the group and key half w/4 of every 64-key
//    tile, so a tile costs each wave half the MFMA work and the two halves'
//    (max, sum, O) are merged through LDS at the end;
//  * K/V tiles reach LDS by global_load_lds DMA into a 4-deep ring, three
//    tiles ahead of the compute; rows are XOR-swizzled in 16-byte chunks so
//    the K operand reads (ds_read_b128) and the V operand transpose reads
//    (ds_read_b64_tr_b16) are both free of bank conflicts;
//  * S^T = K . Q^T with the token permutation that leaves each lane 8
//    consecutive keys of its query row, so P feeds O += P . V as the A
//    operand straight from registers;
//  * query blocks are launched longest-first; tiles above the causal
//    diagonal are never loaded;
//  * with bf16 inputs a single bf16 P would carry 2^-9 relative error per
//    weight, which short causal rows do not average away.  So P.V runs in
//    fp16 (P with 11 significant bits): the V tiles are converted from bf16
//    to fp16 in LDS by the waves that moved them (exact inside the f16
//    range, the range of the reference's f16 cache).  The per-block kernel
//    at head_dim 64 (two tiles per barrier) instead splits P into hi + lo
//    bf16 terms, two MFMAs on the same V operand.
#include "common.h"
#include "kernels.h"

namespace mugen_attn {

namespace {

constexpr int kKT = 64;    // keys per tile
constexpr int kNBuf = 4;   // ring depth: three tiles in flight
constexpr int kWaves = 8;

// 16-byte chunk c of tile row r is stored at chunk c ^ pf_swz<D>(r).  LDS
// has 64 banks x 4 B; a ds_read_b128 runs in four 16-lane phases (each
// 32-lane half split by the parity of its lane-quad index: lanes 0-3,
// 12-15, 20-23, 24-27 share one), a transpose read in two phases of 32
// consecutive lanes (measured with bank-conflict counters).  The K reads
// touch rows 32kh + 8(n/4) + n%4 (+4) at one logical chunk per lane group g;
// the transpose reads touch rows 8g + n/4 (+4) at chunks 2d, 2d + 1.  D = 64
// rows are 128 B, D = 128 rows 256 B.  Both swizzles (an exhaustive search
// against that phase model) make both read kinds conflict-free and ignore
// row bits 2, 4 and 5 (the +4 and key-half row offsets).
template <int D>
__host__ __device__ constexpr int pf_swz(int r) {
    if constexpr (D == 64)
        return (((r >> 1) & 1) * 2) ^ (((r >> 3) & 1) * 4);
    else
        return ((r & 1) * 2) ^ (((r >> 1) & 1) * 4) ^ (((r >> 3) & 1) * 8);
}

// Logical 16-byte chunk c of a D-wide tile row holds dims 8c .. 8c+7; with
// head_dim hd < D the chunks at and past hd/8 are loaded from chunk c mod
// hd/8 of the same head and token instead (finite cache values, in bounds:
// they meet q's zero dims in S, and O's columns past hd are not stored).
__device__ __forceinline__ int dim_chunk(int c, int hd) {
    const int ch = hd >> 3;
    return c < ch ? c : c % ch;
}

}  // namespace

// PAD: head_dim hd < D (dims past it masked); otherwise hd == D.
// DTI: the input type, or kDtBf16V16 (bf16 q / K, V already fp16).
template <int D, int MB, int DTI, int OUT_DT, int TPB, bool PAD>
__global__ __launch_bounds__(512) void gqa_prefill_kernel(GqaPrefillParams p) {
    constexpr int DT = DTI == kDtBf16V16 ? DT_BF16 : DTI;  // q and K
    const int hd = PAD ? p.hd : D;
    constexpr int KK = D / 32;                 // k-steps of S over head_dim
    constexpr int DB = D / 16;                 // 16-wide output column blocks
    constexpr int RB = D * 2;                  // bytes per tile row
    constexpr int CR = D / 8;                  // 16-byte chunks per row
    constexpr int MAT = kKT * RB;              // bytes of one K or V tile
    constexpr int DPW = 2 * MAT / 1024 / kWaves;  // 1-KiB DMA ops per wave per tile (K and V)
    // bf16 inputs, one tile per barrier: each wave converts the V chunks it
    // moved into the ring to fp16 in place (bf16 -> fp16 is exact inside
    // the f16 range, which the reference's f16 cache has too), so P.V runs
    // as ONE fp16 MFMA with an fp16 P (11 significant bits) instead of two
    // bf16 MFMAs on a hi + lo split of P
    // bf16 V converted to fp16 before the call (kDtBf16V16) needs neither
    constexpr bool VCVT = DTI == DT_BF16 && TPB == 1;
    constexpr int PDT = (VCVT || DTI == kDtBf16V16) ? DT_F16 : DT;  // operand type of P.V
    constexpr int NP = p_terms<PDT>();
    static_assert(DPW >= 2 && DPW % 2 == 0, "tile split");
    constexpr int NB = TPB == 1 ? kNBuf : 2 * TPB;  // ring slots
    __shared__ __attribute__((aligned(16))) char ring[NB][2 * MAT];

    const int qb = gridDim.x - 1 - blockIdx.x;  // longest rows first
    const int kvh = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int hs = w & 3, kh = w >> 2;
    const int n = lane & 15, g = lane >> 4;
    const int t0 = qb * 16;
    const int G = p.G;
    MUGEN_TRACE(0);

    // keys visible to the last token of the block; this lane's row limit
    int kend = p.kv_len;
    if (p.causal) kend = min(kend, p.start_pos + min(t0 + 16, p.N));
    const int ntiles = (kend + kKT - 1) / kKT;
    const int row_lim = p.causal ? min(p.start_pos + t0 + n + 1, p.kv_len) : p.kv_len;
    // the first row's limit: tiles wholly below it need no mask
    const int mask_from = p.causal ? min(p.start_pos + t0 + 1, p.kv_len) : p.kv_len;

    // ---- DMA of tile rows: wave w moves K chunks [64(w + 8k), +64) and the
    // same V chunks; slot s = row s / CR, physical chunk s % CR, whose data
    // is logical chunk (s % CR) ^ pf_swz(row)
    const uint32_t ring_base = lds_addr(&ring[0][0]);
    const int rs_bytes = p.row_stride * 2;
    int dma_row[DPW / 2];
    uint32_t dma_col[DPW / 2];
#pragma unroll
    for (int k = 0; k < DPW / 2; k++) {
        const int slot = 64 * (w + kWaves * k) + lane;
        const int r = slot / CR, pc = slot % CR;
        dma_row[k] = r;
        dma_col[k] = (uint32_t)(dim_chunk(pc ^ pf_swz<D>(r), hd) * 16);
    }
    const uint16_t* kb = p.k + (int64_t)kvh * hd;
    const uint16_t* vb = p.v + (int64_t)kvh * hd;
    auto issue = [&](int it) {
        const int kt = it * kKT;
        const uint32_t lds0 = ring_base + (it % NB) * (2 * MAT) + w * 1024;
#pragma unroll
        for (int k = 0; k < DPW / 2; k++) {
            const uint32_t off = (uint32_t)min(kt + dma_row[k], kend - 1) * rs_bytes + dma_col[k];
            dma16s(lds0 + k * kWaves * 1024, kb, off);
            dma16s(lds0 + MAT + k * kWaves * 1024, vb, off);
        }
    };
    // fp16 conversion of this wave's V chunks of a tile: the chunks its own
    // DMA wrote, so the wave waits for its own loads only.  The chunks are
    // read before a tile's compute and written back after it, so the LDS
    // latency hides behind the MFMAs
    auto cv_addr = [&](int it, int k) {
        return reinterpret_cast<u32x4_t*>(&ring[it % NB][MAT] + (64 * (w + kWaves * k) + lane) * 16);
    };
    auto cv_write = [&](int it, const u32x4_t (&x)[DPW / 2]) {
#pragma unroll
        for (int k = 0; k < DPW / 2; k++) {
            u32x4_t y;
#pragma unroll
            for (int e = 0; e < 4; e++) y[e] = pack2<DT_F16>(lo_f32<DT_BF16>(x[k][e]), hi_f32<DT_BF16>(x[k][e]));
            *cv_addr(it, k) = y;
        }
    };
    auto cv_read = [&](int it, u32x4_t (&x)[DPW / 2]) {
#pragma unroll
        for (int k = 0; k < DPW / 2; k++) x[k] = *cv_addr(it, k);
    };
    // TPB = 1: three tiles in flight, one barrier per tile.  TPB > 1: TPB
    // tiles per barrier (the later tiles' operands are read during the
    // first tile's MFMAs), TPB tiles in flight in a ring of 2 TPB slots
    for (int it = 0; it < min(ntiles, TPB == 1 ? kNBuf - 1 : TPB); it++) issue(it);

    // Q^T fragments: lane holds q[token t0+n][head][32kk + 8g .. +8]
    u32x4_t qf[MB][KK];
    bool head_ok[MB];
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
        const int hg = hs + 4 * mb;
        head_ok[mb] = hg < G;
        const int tok = min(t0 + n, p.N - 1);
        const uint16_t* qp = p.q + ((int64_t)tok * p.H + kvh * G + (head_ok[mb] ? hg : 0)) * hd + 8 * g;
#pragma unroll
        for (int kk = 0; kk < KK; kk++) qf[mb][kk] = 32 * kk + 8 * g < hd ? load16(qp + 32 * kk) : u32x4_t{0, 0, 0, 0};
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): no compiler waits inside the loop
    MUGEN_TRACE(1);

    // K operand (A): row 32kh + 8(n/4) + n%4 (+4nb), logical chunk g + 4kk
    const int ar = 32 * kh + 8 * (n >> 2) + (n & 3);
    uint32_t a_off[KK];
#pragma unroll
    for (int kk = 0; kk < KK; kk++) a_off[kk] = ar * RB + (((g + 4 * kk) ^ pf_swz<D>(ar)) * 16);
    // V operand (B, transpose reads): row 32kh + 8g + n/4 (+4), logical
    // bytes 32d + 8(n%4) = chunk 2d + (n%4)/2, half (n%2)
    const int tr = 32 * kh + 8 * g + (n >> 2);
    uint32_t t_off[DB];
#pragma unroll
    for (int d = 0; d < DB; d++) t_off[d] = MAT + tr * RB + (((2 * d + ((n & 3) >> 1)) ^ pf_swz<D>(tr)) * 16) + 8 * (n & 1);

    // O^T accumulators: o[mb][d] lane (g, n) holds O[query t0+n][16d + 4g + i]
    // (O^T = V^T . P^T, so each lane owns one query row and the softmax's
    // per-row factors need no cross-lane moves)
    f32x4_t o[MB][DB];
    float m_run[MB], l_part[MB];  // running max (log2 units) of row t0+n, partial sum
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
        m_run[mb] = kNegInf;
        l_part[mb] = 0.f;
#pragma unroll
        for (int d = 0; d < DB; d++) o[mb][d] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    // lazy max: weights may grow to 2^kHeadroom before the row is re-based
    // (the block's first tile); later tiles re-base when a lane's 8 weights
    // sum past kClampW = 2^15 (each weight then stays within the 16-bit P
    // range, fp16 max 65504)
    constexpr float kHeadroom = 8.f;
    constexpr float kClampW = 32768.f;

    // operands of one tile: K fragments (A, shared by the MB heads) and the
    // V transpose fragments
    auto load_ops = [&](int it, u32x4_t (&af)[2][KK], u32x4_t (&vf)[DB]) {
        const char* tile = &ring[it % NB][0];
#pragma unroll
        for (int nb = 0; nb < 2; nb++)
#pragma unroll
            for (int kk = 0; kk < KK; kk++)
                af[nb][kk] = *reinterpret_cast<const u32x4_t*>(tile + a_off[kk] + nb * 4 * RB);
#pragma unroll
        for (int d = 0; d < DB; d++) {
            const u32x2_t lo = lds_read_tr16(reinterpret_cast<const uint16_t*>(tile + t_off[d]));
            const u32x2_t hi = lds_read_tr16(reinterpret_cast<const uint16_t*>(tile + t_off[d] + 4 * RB));
            vf[d] = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
        }
    };
    auto compute = [&](int it, const u32x4_t (&af)[2][KK], const u32x4_t (&vf)[DB]) {
        const int kt = it * kKT;
        const bool need_mask = kt + kKT > mask_from;
        // S of one head, raw scores (lane: query row t0+n, keys
        // kt + 32kh + 8g + 4nb + i)
        auto s_mfma = [&](int mb, f32x4_t (&sacc)[2]) {
#pragma unroll
            for (int nb = 0; nb < 2; nb++) {
                f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kk = 0; kk < KK; kk++) acc = mfma16x16x32<DT>(af[nb][kk], qf[mb][kk], acc);
                sacc[nb] = acc;
            }
        };
        // with the fp16 P.V of bf16 inputs the S MFMAs of every head go first, so a
        // head's softmax overlaps the next head's S and the previous head's
        // P.V in the MFMA pipe (measured 7% faster at 7B N = 8192; with the
        // bf16 hi + lo P it measured slower, so that order stays per head)
        constexpr bool SFIRST = PDT == DT_F16 && DT == DT_BF16;
        f32x4_t s_all[MB][2];
        if constexpr (SFIRST) {
#pragma unroll
            for (int mb = 0; mb < MB; mb++)
                if (head_ok[mb]) s_mfma(mb, s_all[mb]);
        }
        // The block's first tile sets each row's reference max (re-base
        // test on the tile's max).  Later tiles test the sums instead: the
        // weights 2^(s - m_run) are formed first, and only when a lane's sum
        // of its 8 weights passes 2^kClamp -- every weight is >= 0, so any
        // weight past 2^kClamp (also an infinite one) shows -- is the row
        // re-based and its weights formed again (rare).  That takes one
        // compare per head and tile instead of a max over the 8 scores.
        const bool first = it == 0;
#pragma unroll
        for (int mb = 0; mb < MB; mb++) {
            if (!head_ok[mb]) continue;
            f32x4_t sacc[2];
            if constexpr (SFIRST) {
                sacc[0] = s_all[mb][0];
                sacc[1] = s_all[mb][1];
            } else {
                s_mfma(mb, sacc);
            }
            float s[8];
#pragma unroll
            for (int nb = 0; nb < 2; nb++)
#pragma unroll
                for (int i = 0; i < 4; i++) s[4 * nb + i] = sacc[nb][i];
            if (need_mask) {
                const int key0 = kt + 32 * kh + 8 * g;
#pragma unroll
                for (int j = 0; j < 8; j++)
                    if (key0 + j >= row_lim) s[j] = kNegInf;
            }
            if (first) {
                float smax = s[0];
#pragma unroll
                for (int j = 1; j < 8; j++) smax = fmaxf(smax, s[j]);
                // re-base the row only when a weight would exceed 2^kHeadroom
                if (__any(smax * p.scale_log2 > m_run[mb] + kHeadroom)) {
                    float mt = smax * p.scale_log2;
                    mt = max_x32(max_x16(mt));
                    const float m_new = fmaxf(m_run[mb], mt);
                    if (m_new > m_run[mb]) {
                        const float alpha = fast_exp2(m_run[mb] - m_new);  // 0 when m_run = -inf
                        l_part[mb] *= alpha;
#pragma unroll
                        for (int d = 0; d < DB; d++) o[mb][d] *= alpha;
                        m_run[mb] = m_new;
                    }
                }
            }
            // every row with a visible key in the block's first tile has a
            // finite m_run here; a row without one sees no later key either
            // (its keys are [0, start_pos + token], or all of them)
            float nm = m_run[mb] == kNegInf ? 0.f : -m_run[mb];
            float x[8];
            float ps = 0.f;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                x[j] = fast_exp2(fmaf(s[j], p.scale_log2, nm));
                ps += x[j];
            }
            if (!first && __any(!(ps <= kClampW))) {  // rare: re-base on the tile's row max
                float mt = kNegInf;
#pragma unroll
                for (int j = 0; j < 8; j++) mt = fmaxf(mt, fmaf(s[j], p.scale_log2, nm));
                mt = max_x32(max_x16(mt));
                const float shift = fmaxf(mt, 0.f);  // rows under their reference keep it
                const float alpha = fast_exp2(-shift);
                l_part[mb] *= alpha;
#pragma unroll
                for (int d = 0; d < DB; d++) o[mb][d] *= alpha;
                m_run[mb] = (m_run[mb] == kNegInf ? 0.f : m_run[mb]) + shift;
                nm -= shift;
                ps = 0.f;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    x[j] = fast_exp2(fmaf(s[j], p.scale_log2, nm));
                    ps += x[j];
                }
            }
            l_part[mb] += ps;
            u32x4_t pfr[NP];
            split_p<PDT, NP>(x, pfr);
#pragma unroll
            for (int d = 0; d < DB; d++)
#pragma unroll
                for (int pp = 0; pp < NP; pp++) o[mb][d] = mfma16x16x32<PDT>(vf[d], pfr[pp], o[mb][d]);
        }
    };

    if constexpr (TPB == 1) {
        for (int it = 0; it < ntiles; it++) {
            // tiles issued after `it`: min(ntiles - 1, it + kNBuf - 2) - it
            const int after = min(ntiles - 1, it + kNBuf - 2) - it;
            if (after >= 2) vm_wait<2 * DPW>();
            else if (after == 1) vm_wait<DPW>();
            else vm_wait<0>();
            if constexpr (VCVT) {
                if (it == 0) {  // the first tile: converted before its barrier
                    u32x4_t cv[DPW / 2];
                    cv_read(0, cv);
                    cv_write(0, cv);
                }
            }
            lds_barrier();  // tile `it` landed (and is converted) for all waves; tile it-1's buffer is free
            if (it + kNBuf - 1 < ntiles) issue(it + kNBuf - 1);
            u32x4_t af[2][KK], vf[DB];
            load_ops(it, af, vf);
            // tile it+1 is converted around this tile's compute, before
            // B_{it+1}: this wave's DMA of it is done once at most the tiles
            // issued after it are outstanding
            u32x4_t cv[DPW / 2];
            const int after1 = min(ntiles - 1, it + kNBuf - 1) - (it + 1);
            if constexpr (VCVT) {
                if (after1 >= 0) {
                    if (after1 >= 2) vm_wait<2 * DPW>();
                    else if (after1 == 1) vm_wait<DPW>();
                    else vm_wait<0>();
                    cv_read(it + 1, cv);
                }
            }
            compute(it, af, vf);
            if constexpr (VCVT)
                if (after1 >= 0) cv_write(it + 1, cv);
        }
    } else {
        for (int it = 0; it < ntiles; it += TPB) {
            vm_wait<0>();   // tiles it .. it+TPB-1 (everything issued) landed
            if (it == 0) MUGEN_TRACE(4);
            lds_barrier();  // ... for all waves; the slots of the previous TPB tiles are free
            if (it == 0) MUGEN_TRACE(5);
#pragma unroll
            for (int k = 0; k < TPB; k++)
                if (it + TPB + k < ntiles) issue(it + TPB + k);
            u32x4_t af[TPB][2][KK], vf[TPB][DB];
#pragma unroll
            for (int k = 0; k < TPB; k++)
                if (it + k < ntiles) load_ops(it + k, af[k], vf[k]);
#pragma unroll
            for (int k = 0; k < TPB; k++)
                if (it + k < ntiles) compute(it + k, af[k], vf[k]);
        }
    }

    MUGEN_TRACE(2);
    // ---- merge the two key halves: waves 4..7 hand (m, l, O) to waves 0..3
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
        float l = l_part[mb];
        l = sum_x32(sum_x16(l));
        l_part[mb] = l;
    }
    __syncthreads();  // every wave is done with the ring
    float* xf = reinterpret_cast<float*>(&ring[0][0]);
    // per (head slot, mb): DB*64 f32x4 of O^T, then 16 m and 16 l
    constexpr int XS = DB * 64 * 4 + 32;
    if (kh == 1) {
#pragma unroll
        for (int mb = 0; mb < MB; mb++) {
            if (!head_ok[mb]) continue;
            float* xb = xf + (hs * MB + mb) * XS;
#pragma unroll
            for (int d = 0; d < DB; d++) reinterpret_cast<f32x4_t*>(xb)[d * 64 + lane] = o[mb][d];
            if (g == 0) {
                xb[DB * 256 + n] = m_run[mb];
                xb[DB * 256 + 16 + n] = l_part[mb];
            }
        }
    }
    __syncthreads();
    if (kh == 1) return;
    const int tok = t0 + n;
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
        if (!head_ok[mb]) continue;
        const float* xb = xf + (hs * MB + mb) * XS;
        const float m0 = m_run[mb], l0 = l_part[mb];
        const float m1 = xb[DB * 256 + n], l1 = xb[DB * 256 + 16 + n];
        const float M = fmaxf(m0, m1);
        const float a0 = m0 == kNegInf ? 0.f : fast_exp2(m0 - M);
        const float a1 = m1 == kNegInf ? 0.f : fast_exp2(m1 - M);
        const float lt = a0 * l0 + a1 * l1;
        const float inv = lt > 0.f ? 1.f / lt : 0.f;
        const float c0 = a0 * inv, c1 = a1 * inv;
        if (tok < p.N) {
            const int h = kvh * G + hs + 4 * mb;
            const int64_t base = ((int64_t)tok * p.H + h) * hd + 4 * g;
#pragma unroll
            for (int d = 0; d < DB; d++) {
                if (16 * d + 4 * g >= hd) break;  // padded dims (head_dim < D)
                const f32x4_t o1 = reinterpret_cast<const f32x4_t*>(xb)[d * 64 + lane];
                const f32x4_t r = o[mb][d] * c0 + o1 * c1;
                if constexpr (OUT_DT == DT_F32) {
                    *reinterpret_cast<f32x4_t*>(static_cast<float*>(p.out) + base + 16 * d) = r;
                } else {
                    *reinterpret_cast<u32x2_t*>(static_cast<uint16_t*>(p.out) + base + 16 * d) =
                        u32x2_t{pack2<OUT_DT>(r[0], r[1]), pack2<OUT_DT>(r[2], r[3])};
                }
            }
        }
    }
    MUGEN_TRACE(3);
}

// ------------------------------------------------------------------ warp-specialised kernel
//
// For long prompts the kernel above is bound neither by MFMA issue nor by
// LDS bandwidth but by its serial per-tile chain: the two waves of a SIMD
// run their MFMA and softmax phases in lock step (one barrier per tile).
// This kernel gives the two phases to different waves, as the MLA decode
// kernel does:
//  * workgroup = (16-token query block, kv head, slice of NS = 4 or 8 heads
//    of the group); blocks are numbered longest-first across all kv heads
//    and slices;
//  * waves 0..NS-1 ("S waves"): head NS*slice + w: S^T = K . Q^T for a 32-key
//    tile (the same operand layouts as above with one key half), causal
//    mask, lazy-max softmax, and P (hi + lo for bf16) written to LDS in the
//    B-operand layout of the PV product, with the row's re-base factor when
//    its max moved;
//  * the last NPV = 4 or 8 waves ("PV waves"): NS/NPV heads each, every
//    output column:
//    O^T += V^T . P^T for the previous tile, after applying that
//    tile's re-base factors, and the K / V tile DMA into a 4-slot ring;
//  * one barrier per tile: at barrier j tile j has landed, the S waves have
//    written P(j-1), and the PV waves have finished tile j-2, whose slot
//    then receives tile j+2.
template <int D, int NS, int SMB, int NPV, int DTI, int OUT_DT, bool PAD, int TPS, bool SPLIT>
__global__ __launch_bounds__(64 * (NS / SMB + NPV)) void gqa_prefill_ws_kernel(GqaPrefillParams p, int nqb,
                                                                               int nslice, int Hk) {
    constexpr int DT = DTI == kDtBf16V16 ? DT_BF16 : DTI;  // q and K
    const int hd = PAD ? p.hd : D;
    constexpr int TK = 32;                      // keys per tile (one MFMA k-step of P.V)
    constexpr int KS = TK * TPS;                // keys per step: TPS tiles between two barriers
    constexpr int KK = D / 32;                  // k-steps of S over head_dim
    constexpr int DB = D / 16;                  // 16-wide output column blocks
    constexpr int RB = D * 2;                   // bytes per tile row
    constexpr int CR = D / 8;                   // 16-byte chunks per row
    constexpr int MAT = TK * RB;                // bytes of one K or V tile
    constexpr int VOFF = TPS * MAT;             // a slot: the step's K rows, then its V rows
    constexpr int SLOT = 2 * VOFF;
    constexpr int NSLOT = TPS == 1 ? 4 : 3;     // NSLOT - 2 steps in flight
    constexpr int DPW = SLOT / 1024 / NPV;      // 1-KiB DMA ops per PV wave per step (K and V)
    // bf16 inputs: P.V in fp16 as in the per-block kernel (the PV waves
    // convert the V chunks they moved; P goes to LDS as one fp16 term)
    constexpr bool VCVT = DTI == DT_BF16;
    constexpr int PDT = (VCVT || DTI == kDtBf16V16) ? DT_F16 : DT;
    constexpr int NP = p_terms<PDT>();
    constexpr int PB = TPS * NS * NP * 64 * 16; // one P buffer: TPS tiles x NS heads x NP terms x 64 lanes x 16 B
    static_assert(DPW >= 2 && DPW % 2 == 0 && NS % NPV == 0, "tile split");
    static_assert(TPS == 1 || !VCVT, "in-LDS V conversion: one tile per step");
    __shared__ __attribute__((aligned(1024))) char ring[NSLOT * SLOT + 2 * PB];
    __shared__ float alpha_x[2][NS][16];        // per P buffer: re-base factor of (head, query)
    __shared__ int resc_x[2][NS];               // per P buffer: head's factors apply
    __shared__ float linv_x[NS][16];
    constexpr float kHeadroom = 8.f;
    constexpr float kClampW = 32768.f;  // later tiles: re-base when a lane's 8 weights sum past 2^15

    // longest-first over (query block, kv head, slice)
    const int lin = blockIdx.x;
    // (query block, kv head, slice, key split), longest-first by query block
    const int ks_id = SPLIT ? lin % p.ksplit : 0;
    const int lq = SPLIT ? lin / p.ksplit : lin;
    const int per_qb = Hk * nslice;
    const int qb = nqb - 1 - lq / per_qb;
    const int kvh = (lq / nslice) % Hk;
    const int slice = lq % nslice;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    constexpr int NSW = NS / SMB;               // S waves, SMB heads each
    const bool s_wave = w < NSW;
    const int wr = s_wave ? w : w - NSW;        // S wave index; PV wave index
    const int n = lane & 15, g = lane >> 4;
    MUGEN_TRACE(6);
    const int t0 = qb * 16;
    const int G = p.G;
    const int nh = min(NS, G - NS * slice);     // heads of this slice
    int kend = p.kv_len;
    if (p.causal) kend = min(kend, p.start_pos + min(t0 + 16, p.N));
    // this workgroup's keys [k_beg, kend) (the block's whole range unless split)
    const int k_beg = SPLIT ? ks_id * p.kchunk : 0;
    if (SPLIT) kend = min(kend, k_beg + p.kchunk);
    const int ntiles = SPLIT ? (kend > k_beg ? (kend - k_beg + KS - 1) / KS : 0) : (kend + KS - 1) / KS;  // steps
    const uint32_t ring_base = lds_addr(&ring[0]);
    char* pbuf = &ring[NSLOT * SLOT];

    if (s_wave) {
        // ================================================== S waves
        // heads wr*SMB .. +SMB-1 of the slice share each K fragment read
        bool hok[SMB];
        u32x4_t qf[SMB][KK];
#pragma unroll
        for (int mb = 0; mb < SMB; mb++) {
            const int hs = wr * SMB + mb;
            hok[mb] = hs < nh;
            const int tok = min(t0 + n, p.N - 1);
            const uint16_t* qp =
                p.q + ((int64_t)tok * p.H + kvh * G + NS * slice + (hok[mb] ? hs : 0)) * hd + 8 * g;
#pragma unroll
            for (int kk = 0; kk < KK; kk++)
                qf[mb][kk] = 32 * kk + 8 * g < hd ? load16(qp + 32 * kk) : u32x4_t{0, 0, 0, 0};
        }
        const int row_lim = p.causal ? min(p.start_pos + t0 + n + 1, p.kv_len) : p.kv_len;
        const int mask_from = p.causal ? min(p.start_pos + t0 + 1, p.kv_len) : p.kv_len;
        // K operand (A): tile row 8(n/4) + n%4 (+4nb), logical chunk g + 4kk
        const int ar = 8 * (n >> 2) + (n & 3);
        uint32_t a_off[KK];
#pragma unroll
        for (int kk = 0; kk < KK; kk++) a_off[kk] = ar * RB + (((g + 4 * kk) ^ pf_swz<D>(ar)) * 16);
        float m_run[SMB], l_part[SMB];
#pragma unroll
        for (int mb = 0; mb < SMB; mb++) {
            m_run[mb] = kNegInf;
            l_part[mb] = 0.f;
        }
        for (int j = 0; j <= ntiles; j++) {
            if (j == 8) MUGEN_TRACE(0);
            lds_barrier();  // B_j: tile j landed
            if (j == 8) MUGEN_TRACE(1);
            if (j == 16) MUGEN_TRACE(5);
            if (j == 0) MUGEN_TRACE(7);
            if (j == 24) MUGEN_TRACE(11);
            if (j == 28) MUGEN_TRACE(12);
            if (j == ntiles) break;
            if (!hok[0]) continue;
            const uint32_t slot_addr = ring_base + (uint32_t)((j % NSLOT) * SLOT);
            const int kt = k_beg + j * KS;
            // block nb of tile u: keys kt + 32u + 8g + 4(nb % 2) + i; one
            // address register per k-step, the tile and half-block offsets
            // in the instruction
            constexpr int NB = 2 * TPS;
            u32x4_t af[NB][KK];
#pragma unroll
            for (int kk = 0; kk < KK; kk++) {
                const lds_char_t* ka = lds_ptr(slot_addr + a_off[kk]);
#pragma unroll
                for (int nb = 0; nb < NB; nb++) af[nb][kk] = lds_read_b128(ka + (nb >> 1) * MAT + (nb & 1) * 4 * RB);
            }
            constexpr int NV = 4 * NB;          // scores per lane per head
            float sv[SMB][NV];
#pragma unroll
            for (int mb = 0; mb < SMB; mb++)
#pragma unroll
                for (int nb = 0; nb < NB; nb++) {
                    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int kk = 0; kk < KK; kk++) acc = mfma16x16x32<DT>(af[nb][kk], qf[mb][kk], acc);
#pragma unroll
                    for (int i = 0; i < 4; i++) sv[mb][4 * nb + i] = acc[i];
                }
            if (j == 8) MUGEN_TRACE(2);
#pragma unroll
            for (int mb = 0; mb < SMB; mb++) {
                if (!hok[mb]) continue;
                const int hs = wr * SMB + mb;
                float* s = sv[mb];
                // lane: query t0+n, keys kt + 32u + 8g + 4nb + i
                if (kt + KS > mask_from) {
#pragma unroll
                    for (int jj = 0; jj < NV; jj++)
                        if (kt + 32 * (jj >> 3) + 8 * g + (jj & 7) >= row_lim) s[jj] = kNegInf;
                }
                // the block's first tile sets each row's reference max (test
                // on the tile's max); later tiles form the weights first and
                // re-base only when a lane's weights of one tile sum past kClampW
                // (every weight >= 0: any weight past it, also an infinite
                // one, shows), one compare instead of a max over the scores
                float alpha = 1.f;
                bool rebase = false;
                if (j == 0) {
                    float smax = s[0];
#pragma unroll
                    for (int jj = 1; jj < NV; jj++) smax = fmaxf(smax, s[jj]);
                    rebase = __any(smax * p.scale_log2 > m_run[mb] + kHeadroom);
                    if (rebase) {
                        const float mt = max_x32(max_x16(smax * p.scale_log2));
                        const float m_new = fmaxf(m_run[mb], mt);
                        if (m_new > m_run[mb]) {
                            alpha = fast_exp2(m_run[mb] - m_new);  // 0 when m_run = -inf
                            l_part[mb] *= alpha;
                            m_run[mb] = m_new;
                        }
                    }
                }
                // a row without a visible key in the first tile sees no later key
                float nm = m_run[mb] == kNegInf ? 0.f : -m_run[mb];
                float x[NV];
                float ps[TPS];
#pragma unroll
                for (int u = 0; u < TPS; u++) {
                    ps[u] = 0.f;
#pragma unroll
                    for (int jj = 8 * u; jj < 8 * u + 8; jj++) {
                        x[jj] = fast_exp2(fmaf(s[jj], p.scale_log2, nm));
                        ps[u] += x[jj];
                    }
                }
                bool over = false;
#pragma unroll
                for (int u = 0; u < TPS; u++) over |= !(ps[u] <= kClampW);
                if (j > 0 && __any(over)) {  // rare: re-base on the step's row max
                    rebase = true;
                    float mt = kNegInf;
#pragma unroll
                    for (int jj = 0; jj < NV; jj++) mt = fmaxf(mt, fmaf(s[jj], p.scale_log2, nm));
                    mt = max_x32(max_x16(mt));
                    const float shift = fmaxf(mt, 0.f);  // rows under their reference keep it
                    alpha = fast_exp2(-shift);
                    l_part[mb] *= alpha;
                    m_run[mb] = (m_run[mb] == kNegInf ? 0.f : m_run[mb]) + shift;
                    nm -= shift;
#pragma unroll
                    for (int u = 0; u < TPS; u++) {
                        ps[u] = 0.f;
#pragma unroll
                        for (int jj = 8 * u; jj < 8 * u + 8; jj++) {
                            x[jj] = fast_exp2(fmaf(s[jj], p.scale_log2, nm));
                            ps[u] += x[jj];
                        }
                    }
                }
                char* pb = pbuf + (j & 1) * PB;
#pragma unroll
                for (int u = 0; u < TPS; u++) {
                    l_part[mb] += ps[u];
                    u32x4_t pfr[NP];
                    split_p<PDT, NP>(x + 8 * u, pfr);
#pragma unroll
                    for (int pp = 0; pp < NP; pp++)
                        *reinterpret_cast<u32x4_t*>(pb + (((u * NS + hs) * NP + pp) * 64 + lane) * 16) = pfr[pp];
                }
                if (g == 0) alpha_x[j & 1][hs][n] = alpha;
                if (lane == 0) resc_x[j & 1][hs] = rebase ? 1 : 0;
            }
            if (j == 8) MUGEN_TRACE(3);
        }
#pragma unroll
        for (int mb = 0; mb < SMB; mb++) {
            const float l = sum_x32(sum_x16(l_part[mb]));
            if (g == 0) linv_x[wr * SMB + mb][n] = l > 0.f ? 1.f / l : 0.f;
            if (SPLIT && g == 0 && hok[mb] && t0 + n < p.N) {
                // split partial: the row's reference max (log2 units) and sum
                const int64_t row = (int64_t)(t0 + n) * p.H + kvh * G + NS * slice + wr * SMB + mb;
                *reinterpret_cast<f32x2v_t*>(p.ws_ml + (row * p.ksplit + ks_id) * 2) = f32x2v_t{m_run[mb], l};
            }
        }
        MUGEN_TRACE(9);
        __syncthreads();  // E: 1/l published
    } else {
        // ================================================== PV waves
        const uint16_t* kb = p.k + (int64_t)kvh * hd;
        const uint16_t* vb = p.v + (int64_t)kvh * hd;
        const int rs_bytes = p.row_stride * 2;
        // DMA op k of this wave moves K / V chunks [64(wr + NPV k), +64) of the
        // step: chunk slot s = row s / CR, physical chunk s % CR, holding
        // logical chunk (s % CR) ^ pf_swz(row); rows past kend are clamped.
        // Op k's rows are op 0's + k RSTEP, a multiple of 16: same swizzle
        constexpr int RSTEP = 64 * NPV / CR;
        static_assert(RSTEP % 16 == 0, "swizzle period");
        const int dma_row = (64 * wr + lane) / CR;
        const uint32_t dma_col = (uint32_t)(dim_chunk((lane % CR) ^ pf_swz<D>(dma_row), hd) * 16);
        auto issue = [&](int it) {
            const int kt = k_beg + it * KS + dma_row;
            const uint32_t lds0 = ring_base + (it % NSLOT) * SLOT + wr * 1024;
            if (k_beg + (it + 1) * KS <= kend) {
                // every row in range: one offset, op k's rows through the
                // scalar base (no per-op vector arithmetic)
                const uint32_t off = (uint32_t)kt * rs_bytes + dma_col;
#pragma unroll
                for (int k = 0; k < DPW / 2; k++) {
                    const int64_t sk = (int64_t)k * RSTEP * rs_bytes;
                    dma16s(lds0 + k * NPV * 1024, reinterpret_cast<const char*>(kb) + sk, off);
                    dma16s(lds0 + VOFF + k * NPV * 1024, reinterpret_cast<const char*>(vb) + sk, off);
                }
            } else {
#pragma unroll
                for (int k = 0; k < DPW / 2; k++) {
                    const uint32_t off = (uint32_t)min(kt + k * RSTEP, kend - 1) * rs_bytes + dma_col;
                    dma16s(lds0 + k * NPV * 1024, kb, off);
                    dma16s(lds0 + VOFF + k * NPV * 1024, vb, off);
                }
            }
        };
        for (int it = 0; it < min(ntiles, NSLOT - 2); it++) issue(it);
        // fp16 conversion (VCVT) of this wave's V chunks of a tile: read
        // after the barrier that shows the tile landed, written back after
        // this interval's P.V, visible to the other PV waves from the next
        // barrier on (the interval in which they read that tile)
        auto cv_addr = [&](int it, int k) {
            return reinterpret_cast<u32x4_t*>(&ring[(it % NSLOT) * SLOT + VOFF] + (64 * (wr + NPV * k) + lane) * 16);
        };
        u32x4_t cv[DPW / 2];
        auto cv_write = [&](int it) {
#pragma unroll
            for (int k = 0; k < DPW / 2; k++) {
                u32x4_t y;
#pragma unroll
                for (int e = 0; e < 4; e++) y[e] = pack2<DT_F16>(lo_f32<DT_BF16>(cv[k][e]), hi_f32<DT_BF16>(cv[k][e]));
                *cv_addr(it, k) = y;
            }
        };
        // V operand (A, transpose reads): tile row 8g + n/4 (+4), logical
        // bytes 32d + 8(n%4) = chunk 2d + (n%4)/2, half n%2
        const int tr = 8 * g + (n >> 2);
        uint32_t t_off[DB];
#pragma unroll
        for (int d = 0; d < DB; d++)
            t_off[d] = VOFF + tr * RB + (((2 * d + ((n & 3) >> 1)) ^ pf_swz<D>(tr)) * 16) + 8 * (n & 1);
        // this wave's heads: HPW consecutive heads of the slice, every column
        constexpr int HPW = NS / NPV;
        const int hb = wr * HPW;
        f32x4_t o[HPW][DB];
#pragma unroll
        for (int hh = 0; hh < HPW; hh++)
#pragma unroll
            for (int d = 0; d < DB; d++) o[hh][d] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        for (int j = 0; j <= ntiles; j++) {
            if (j == 8) MUGEN_TRACE(0);
            // tile j landed before B_j: the tiles issued after it are
            // j+1 .. min(j + NSLOT - 3, ntiles - 1), DPW operations each
            switch (min(NSLOT - 3, max(ntiles - 1 - j, 0))) {  // one s_waitcnt
#define PF_VMW(C) case C: vm_wait<C * DPW>(); break;
                PF_VMW(0) PF_VMW(1) PF_VMW(2) PF_VMW(3) PF_VMW(4) PF_VMW(5)
#undef PF_VMW
            }
            static_assert(NSLOT - 3 <= 5, "wait cases");
            if (j == 8) MUGEN_TRACE(4);
            lds_barrier();  // B_j
            if (j == 8) MUGEN_TRACE(1);
            if (j == 16) MUGEN_TRACE(5);
            if (j == 0) MUGEN_TRACE(7);
            if (j + NSLOT - 2 < ntiles) issue(j + NSLOT - 2);  // into the slot of tile j-2
            if constexpr (VCVT) {
                if (j < ntiles) {
#pragma unroll
                    for (int k = 0; k < DPW / 2; k++) cv[k] = *cv_addr(j, k);
                }
                if (j == 0) {
                    if (ntiles > 0) cv_write(0);
                    continue;
                }
            }
            if (j == 0) continue;
            const int jp = j - 1;
            const uint32_t slot_addr = ring_base + (uint32_t)((jp % NSLOT) * SLOT);
            const char* pb = pbuf + (jp & 1) * PB;
            // the step's re-base flags first: the branch on them then waits
            // for these reads only, and the MFMAs for their own operands
            int any_rs = 0;
#pragma unroll
            for (int hh = 0; hh < HPW; hh++) any_rs |= resc_x[jp & 1][hb + hh];
            // this wave's heads' P, then the V^T fragments, in flight together
            u32x4_t pf[TPS][HPW][NP];
#pragma unroll
            for (int u = 0; u < TPS; u++)
#pragma unroll
                for (int hh = 0; hh < HPW; hh++)
#pragma unroll
                    for (int pp = 0; pp < NP; pp++)
                        pf[u][hh][pp] = *reinterpret_cast<const u32x4_t*>(
                            pb + (((u * NS + hb + hh) * NP + pp) * 64 + lane) * 16);
            // one address register per column block: tile u and the upper
            // half rows are constant offsets of the instruction
            const lds_char_t* va[DB];
#pragma unroll
            for (int d = 0; d < DB; d++) va[d] = lds_ptr(slot_addr + t_off[d]);
            auto read_v = [&](int u, u32x4_t* vf) {
#pragma unroll
                for (int d = 0; d < DB; d++) {
                    const u32x2_t lo = lds_read_tr16(va[d] + u * MAT);
                    const u32x2_t hi = lds_read_tr16(va[d] + u * MAT + 4 * RB);
                    vf[d] = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
                }
            };
            // every tile's V^T reads in flight before the first MFMA (left
            // to itself the scheduler keeps two: -1.4% at 7B N = 8192; the
            // same for the S waves' K reads measured 3.9% slower).  Both
            // tiles' fragments up front, in their own registers (165 VGPRs,
            // within the 168 of three waves per SIMD), instead of the second
            // tile's reads after the first tile's MFMAs: 7B N = 8192 539.5 ->
            // 522.5 us, N = 2048 46.4 -> 44.9
            u32x4_t vf[TPS][DB];
#pragma unroll
            for (int u = 0; u < TPS; u++) read_v(u, vf[u]);
            __builtin_amdgcn_sched_barrier(0);
            // re-base (rare after the first tiles): the factors are read only
            // when one of this wave's heads moved its max (factor 1 otherwise)
            if (__builtin_amdgcn_readfirstlane(any_rs)) {
#pragma unroll
                for (int hh = 0; hh < HPW; hh++) {
                    const float a = hb + hh < nh ? alpha_x[jp & 1][hb + hh][n] : 1.f;
#pragma unroll
                    for (int d = 0; d < DB; d++) o[hh][d] *= a;
                }
            }
            // (heads past nh accumulate stale P; their sums are never stored)
#pragma unroll
            for (int u = 0; u < TPS; u++) {
#pragma unroll
                for (int pp = 0; pp < NP; pp++)
#pragma unroll
                    for (int d = 0; d < DB; d++)
#pragma unroll
                        for (int hh = 0; hh < HPW; hh++)
                            o[hh][d] = mfma16x16x32<PDT>(vf[u][d], pf[u][hh][pp], o[hh][d]);
            }
            if constexpr (VCVT)
                if (j < ntiles) cv_write(j);
            if (j == 8) MUGEN_TRACE(3);
        }
        MUGEN_TRACE(9);
        __syncthreads();  // E: the S waves' 1/l
        // lane (g, n): O[query t0+n][16d + 4g + i]
        const int tok = t0 + n;
        if (tok < p.N) {
#pragma unroll
            for (int hh = 0; hh < HPW; hh++) {
                if (hb + hh >= nh) continue;
                const float inv = linv_x[hb + hh][n];
                if (SPLIT) {
                    // split partial: O / l in fp16 (a convex combination of
                    // V rows, inside V's +-65504); l and the max from the S waves
                    const int64_t row = (int64_t)tok * p.H + kvh * G + NS * slice + hb + hh;
                    uint16_t* dst = p.ws_o + (row * p.ksplit + ks_id) * hd + 4 * g;
#pragma unroll
                    for (int d = 0; d < DB; d++) {
                        if (16 * d + 4 * g >= hd) break;  // padded dims (head_dim < D)
                        const f32x4_t r = o[hh][d] * inv;
                        *reinterpret_cast<u32x2_t*>(dst + 16 * d) =
                            u32x2_t{pack2<DT_F16>(r[0], r[1]), pack2<DT_F16>(r[2], r[3])};
                    }
                    continue;
                }
                const int64_t base = ((int64_t)tok * p.H + kvh * G + NS * slice + hb + hh) * hd + 4 * g;
#pragma unroll
                for (int d = 0; d < DB; d++) {
                    if (16 * d + 4 * g >= hd) break;  // padded dims (head_dim < D)
                    const f32x4_t r = o[hh][d] * inv;
                    if constexpr (OUT_DT == DT_F32) {
                        *reinterpret_cast<f32x4_t*>(static_cast<float*>(p.out) + base + 16 * d) = r;
                    } else {
                        *reinterpret_cast<u32x2_t*>(static_cast<uint16_t*>(p.out) + base + 16 * d) =
                            u32x2_t{pack2<OUT_DT>(r[0], r[1]), pack2<OUT_DT>(r[2], r[3])};
                    }
                }
            }
        }
    }
    MUGEN_TRACE(10);
}

// ------------------------------------------------------------------ short-prompt kernel
//
// When every key a query block can see fits in LDS (kv range <= 512 keys at
// head_dim 64: 64 KiB each of K and V per workgroup), the serial chain of
// 64-key tiles goes away.  Workgroup = (16-token query block, kv head), 8
// waves = 4 contiguous key ranges x 2 head pairs of the group (G <= 4):
//  * all K rows, then all V rows, of the block's range move into LDS by DMA
//    at once (the two waves of a key range move half each);
//  * after the K rows land, each wave computes S^T = K . Q^T for its range
//    and its 2 heads (the operand layouts of the kernels above) and an exact
//    softmax over the range (all its scores are in registers: one max, no
//    re-base) while the V rows are still in flight;
//  * bf16 V rows are converted to fp16 in LDS by the wave whose DMA moved
//    them (exact inside the f16 range), so O^T += V^T . P^T is one fp16
//    MFMA with P (11 significant bits) straight from registers; each row's
//    weight sum comes from one more MFMA against an all-ones V block (the
//    sum of exactly the fp16 weights P.V used, with no per-lane adds or
//    cross-lane reduction);
//  * merge: each wave stages (max, sum) and its O^T in the K rows' space
//    (free once every wave has passed the V barrier); after one barrier
//    every wave sums and stores an eighth of the block's output.
// The longest block's chain is one range of <= 128 keys instead of eight
// dependent 64-key tiles.
constexpr int kShortMaxKeys = 512;  // kv range the short kernel serves (head_dim 64)

template <int DT, int OUT_DT>
__global__ __launch_bounds__(512) void gqa_prefill_short_kernel(GqaPrefillParams p) {
    constexpr int D = 64, KK = D / 32, DB = D / 16, RB = D * 2, CR = D / 8;
    constexpr int MBW = 2;                      // heads (16-row blocks) per wave
    constexpr int NU = kShortMaxKeys / 4 / 32;  // 32-key units per range, at most
    constexpr int MAT = NU * 32 * RB;           // 16 KiB: K (or V) rows of one range
    __shared__ __attribute__((aligned(1024))) char lds[2 * 4 * MAT];  // [K, V][range]
    __shared__ float2 mlx[8][MBW][16];          // per wave, head, row: (max, sum) of its range
    __shared__ __attribute__((aligned(16))) char qlds[4 * 16 * RB];  // q rows [head slot][token]

    // XCD-aware mapping: workgroups are dealt to the 8 XCDs round-robin by
    // blockIdx, and units (kv head-major: unit = kvh * nqb + i) go to the XCDs
    // in contiguous ranges, so the blocks of one kv head share one XCD's L2
    // for its K / V rows (Hk = 8: one kv head per XCD) instead of every XCD
    // fetching every head; within a range the longest rows go first
    const int nqb = (p.N + 15) / 16;
    const int units = nqb * (p.H / p.G);  // x kv heads
    const int upx = (units + 7) / 8;
    const int slot = blockIdx.x / 8, unit = (blockIdx.x % 8) * upx + slot;
    if (slot >= upx || unit >= units) return;
    const int kvh = unit / nqb;
    const int qb = nqb - 1 - (unit - kvh * nqb);  // longest rows first
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kr = w & 3, rh = w >> 2;          // key range, head pair
    const int n = lane & 15, g = lane >> 4;
    const int t0 = qb * 16;
    const int G = p.G;

    int kend = p.kv_len;  // keys the block's last token sees
    if (p.causal) kend = min(kend, p.start_pos + min(t0 + 16, p.N));
    // range kr = keys [kr R, kr R + R), R a multiple of 32 (<= 128)
    const int R = ((kend + 127) / 128) * 32;
    const int kb0 = kr * R;
    const int nu = max(0, min(R, kend - kb0) + 31) / 32;  // units holding keys (wave-uniform)
    const int row_lim = p.causal ? min(p.start_pos + t0 + n + 1, p.kv_len) : p.kv_len;
    const int mask_from = p.causal ? min(p.start_pos + t0 + 1, kend) : kend;  // first row's limit

    // ---- q rows by DMA too (so that no compiler-tracked load is waited for
    // behind the V rows): wave w moves LDS rows [8w, 8w+8) = head slot w/2,
    // tokens t0 + 8(w%2) + r; tokens past N and head slots past G read a
    // valid row (never stored)
    {
        const int r = lane >> 3, pc = lane & 7;
        const int hs = w >> 1, tok = min(t0 + 8 * (w & 1) + r, p.N - 1);
        const uint16_t* qbase = p.q + (int64_t)t0 * p.H * D;  // offsets stay within the block's 16 tokens
        const uint32_t off = (uint32_t)(((tok - t0) * p.H + kvh * G + (hs < G ? hs : 0)) * D * 2 + pc * 16);
        dma16s(lds_addr(qlds) + w * 1024, qbase, off);
    }
    // ---- K rows, then V rows, of range kr by DMA: op k moves rows [8k, 8k+8)
    // (64 lanes x 16 B); the range's 4 nu ops per matrix are split between
    // its two waves (op parity = rh), 2 nu each.  Chunk pc of row r holds
    // source chunk pc ^ pf_swz(r); rows past kend read row kend - 1 (masked)
    char* kreg = &lds[kr * MAT];
    char* vreg = &lds[(4 + kr) * MAT];
    {
        const int rs_bytes = p.row_stride * 2;
        const int r = lane / CR, pc = lane % CR;
        uint32_t off[NU * 2];
#pragma unroll
        for (int k2 = 0; k2 < NU * 2; k2++) {
            const int k = 2 * k2 + rh;
            const int key = min(kb0 + 8 * k + r, kend - 1);
            off[k2] = (uint32_t)key * rs_bytes + (uint32_t)((pc ^ pf_swz<D>(8 * k + r)) * 16);
        }
        const uint16_t* ksrc = p.k + (int64_t)kvh * D;
        const uint16_t* vsrc = p.v + (int64_t)kvh * D;
#pragma unroll
        for (int k2 = 0; k2 < NU * 2; k2++)
            if (k2 < 2 * nu) dma16s(lds_addr(kreg) + (2 * k2 + rh) * 1024, ksrc, off[k2]);
#pragma unroll
        for (int k2 = 0; k2 < NU * 2; k2++)
            if (k2 < 2 * nu) dma16s(lds_addr(vreg) + (2 * k2 + rh) * 1024, vsrc, off[k2]);
    }
    // K operand (A): unit row 8(n/4) + n%4 (+4nb), logical chunk g + 4kk
    const int ar = 8 * (n >> 2) + (n & 3);
    uint32_t a_off[KK];
#pragma unroll
    for (int kk = 0; kk < KK; kk++) a_off[kk] = ar * RB + (((g + 4 * kk) ^ pf_swz<D>(ar)) * 16);
    // V operand (A of O^T, transpose reads): unit row 8g + n/4 (+4), logical
    // bytes 32d + 8(n%4) = chunk 2d + (n%4)/2, half n%2
    const int tr = 8 * g + (n >> 2);
    uint32_t t_off[DB];
#pragma unroll
    for (int d = 0; d < DB; d++) t_off[d] = tr * RB + (((2 * d + ((n & 3) >> 1)) ^ pf_swz<D>(tr)) * 16) + 8 * (n & 1);

    // this wave's q and K rows landed: at most its 2 nu V ops are in flight
    switch (nu) {
        case 4: vm_wait<8>(); break;
        case 3: vm_wait<6>(); break;
        case 2: vm_wait<4>(); break;
        case 1: vm_wait<2>(); break;
        default: vm_wait<0>(); break;
    }
    lds_barrier();  // B1: the range's K rows from both of its waves, every wave's q rows
    // Q^T fragments (B operand) of the wave's heads: lane holds
    // q[t0+n][head][32kk+8g .. +8]
    u32x4_t qf[MBW][KK];
#pragma unroll
    for (int mb = 0; mb < MBW; mb++)
#pragma unroll
        for (int kk = 0; kk < KK; kk++)
            qf[mb][kk] = *reinterpret_cast<const u32x4_t*>(qlds + ((MBW * rh + mb) * 16 + n) * RB + (4 * kk + g) * 16);

    // ---- S^T, then the exact softmax of the range.  Lane (n, g) holds row
    // t0+n, keys kb0 + 32u + 8g + j (j < 8) in s[u][mb][j]
    float s[NU][MBW][8];
#pragma unroll
    for (int u = 0; u < NU; u++) {
        if (u >= nu) continue;
        u32x4_t af[2][KK];
#pragma unroll
        for (int nb = 0; nb < 2; nb++)
#pragma unroll
            for (int kk = 0; kk < KK; kk++)
                af[nb][kk] = *reinterpret_cast<const u32x4_t*>(kreg + u * 32 * RB + nb * 4 * RB + a_off[kk]);
#pragma unroll
        for (int mb = 0; mb < MBW; mb++) {
#pragma unroll
            for (int nb = 0; nb < 2; nb++) {
                f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kk = 0; kk < KK; kk++) acc = mfma16x16x32<DT>(af[nb][kk], qf[mb][kk], acc);
#pragma unroll
                for (int i = 0; i < 4; i++) s[u][mb][4 * nb + i] = acc[i];  // raw score (scale > 0)
            }
            const int key0 = kb0 + 32 * u + 8 * g;
            if (kb0 + 32 * u + 32 > mask_from) {  // wave-uniform: units below the diagonal carry no mask
#pragma unroll
                for (int j = 0; j < 8; j++)
                    if (key0 + j >= row_lim || key0 + j >= kend) s[u][mb][j] = kNegInf;
            }
        }
    }
    float m[MBW], l[MBW];
    u32x4_t pf[NU][MBW];  // fp16 weights, the B operand of O^T = V^T . P^T
#pragma unroll
    for (int mb = 0; mb < MBW; mb++) {
        float mx = kNegInf;
#pragma unroll
        for (int u = 0; u < NU; u++)
            if (u < nu)
#pragma unroll
                for (int j = 0; j < 8; j++) mx = fmaxf(mx, s[u][mb][j]);
        mx = max_x32(max_x16(mx));
        m[mb] = mx * p.scale_log2;  // the range's max in log2 units
        const float nm = mx == kNegInf ? 0.f : -m[mb];
#pragma unroll
        for (int u = 0; u < NU; u++) {
            if (u >= nu) continue;
            float x[8];
#pragma unroll
            for (int j = 0; j < 8; j++) x[j] = fast_exp2(fmaf(s[u][mb][j], p.scale_log2, nm));
            split_p<DT_F16, 1>(x, &pf[u][mb]);
        }
    }

    // ---- V rows: bf16 -> fp16 by the wave whose DMA moved them
    vm_wait<0>();
    if constexpr (DT == DT_BF16) {
        // all reads first, so their LDS latencies overlap
        u32x4_t x[NU * 2];
#pragma unroll
        for (int k2 = 0; k2 < NU * 2; k2++)
            if (k2 < 2 * nu) x[k2] = *reinterpret_cast<const u32x4_t*>(vreg + (2 * k2 + rh) * 1024 + lane * 16);
#pragma unroll
        for (int k2 = 0; k2 < NU * 2; k2++) {
            if (k2 < 2 * nu) {
                u32x4_t y;
#pragma unroll
                for (int e = 0; e < 4; e++) y[e] = pack2<DT_F16>(lo_f32<DT_BF16>(x[k2][e]), hi_f32<DT_BF16>(x[k2][e]));
                *reinterpret_cast<u32x4_t*>(vreg + (2 * k2 + rh) * 1024 + lane * 16) = y;
            }
        }
    }
    lds_barrier();  // B2: the range's V rows (fp16) from both waves; every wave is done with K

    f32x4_t o[MBW][DB];
    f32x4_t osum[MBW];  // O^T rows of an all-ones V block: every row holds the row's weight sum
    const u32x4_t ones = u32x4_t{0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u};  // fp16 1.0 pairs
#pragma unroll
    for (int mb = 0; mb < MBW; mb++) {
        osum[mb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int d = 0; d < DB; d++) o[mb][d] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < NU; u++) {
        if (u >= nu) continue;
        u32x4_t vf[DB];
#pragma unroll
        for (int d = 0; d < DB; d++) {
            const char* tp = vreg + u * 32 * RB + t_off[d];
            const u32x2_t lo = lds_read_tr16(reinterpret_cast<const uint16_t*>(tp));
            const u32x2_t hi = lds_read_tr16(reinterpret_cast<const uint16_t*>(tp + 4 * RB));
            vf[d] = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
        }
#pragma unroll
        for (int mb = 0; mb < MBW; mb++) {
#pragma unroll
            for (int d = 0; d < DB; d++) o[mb][d] = mfma16x16x32<DT_F16>(vf[d], pf[u][mb], o[mb][d]);
            osum[mb] = mfma16x16x32<DT_F16>(ones, pf[u][mb], osum[mb]);
        }
    }

    // ---- merge the 4 key ranges of each head pair: (max, sum) and the
    // unscaled O^T go to LDS (O^T into the K rows' space), one barrier
    f32x4_t* stage = reinterpret_cast<f32x4_t*>(&lds[0]);  // [wave][mb][d][lane]: 64 KiB, the K rows
#pragma unroll
    for (int mb = 0; mb < MBW; mb++) {
        l[mb] = osum[mb][0];  // the sum over the range's keys of the fp16 weights P.V used
        if (g == 0) mlx[w][mb][n] = make_float2(m[mb], l[mb]);
#pragma unroll
        for (int d = 0; d < DB; d++) stage[((w * MBW + mb) * DB + d) * 64 + lane] = o[mb][d];
    }
    __syncthreads();
    // wave (kr, rh) sums and stores fragments 2kr, 2kr+1 of its head pair's
    // MBW * DB = 8 (head, column block) fragments; both are of head mb = kr / 2
    const int mb = kr >> 1;
    const int tok = t0 + n;
    if (MBW * rh + mb >= G || tok >= p.N) return;
    float a[4], M = kNegInf, L = 0.f;
#pragma unroll
    for (int r = 0; r < 4; r++) M = fmaxf(M, mlx[4 * rh + r][mb][n].x);
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const float2 v = mlx[4 * rh + r][mb][n];
        a[r] = v.x == kNegInf ? 0.f : fast_exp2(v.x - M);
        L += a[r] * v.y;
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    const int h = kvh * G + MBW * rh + mb;
#pragma unroll
    for (int f2 = 0; f2 < 2; f2++) {
        const int f = 2 * kr + f2, d = f % DB;
        f32x4_t r = stage[((4 * rh) * MBW * DB + f) * 64 + lane] * (a[0] * inv);
#pragma unroll
        for (int q = 1; q < 4; q++) r += stage[((4 * rh + q) * MBW * DB + f) * 64 + lane] * (a[q] * inv);
        const int64_t base = ((int64_t)tok * p.H + h) * D + 16 * d + 4 * g;
        if constexpr (OUT_DT == DT_F32) {
            *reinterpret_cast<f32x4_t*>(static_cast<float*>(p.out) + base) = r;
        } else {
            *reinterpret_cast<u32x2_t*>(static_cast<uint16_t*>(p.out) + base) =
                u32x2_t{pack2<OUT_DT>(r[0], r[1]), pack2<OUT_DT>(r[2], r[3])};
        }
    }
}

// bf16 -> fp16 copy of the V rows [0, kv_len) (RNE; exact inside the f16
// range), 8 values per thread: the optional per-call pre-pass that lets the
// prefill kernels read V as fp16 (kDtBf16V16)
__global__ __launch_bounds__(256) void v_to_f16_kernel(const uint16_t* __restrict__ v, uint16_t* __restrict__ dst,
                                                       int64_t n8) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n8) return;
    const u32x4_t x = load16(v + 8 * i);
    u32x4_t y;
#pragma unroll
    for (int e = 0; e < 4; e++) y[e] = pack2<DT_F16>(lo_f32<DT_BF16>(x[e]), hi_f32<DT_BF16>(x[e]));
    *reinterpret_cast<u32x4_t*>(dst + 8 * i) = y;
}

hipError_t launch_v_to_f16(const uint16_t* v, uint16_t* dst, int64_t n, hipStream_t st, KernelTimer* t) {
    const int64_t n8 = n / 8;
    return launch_k(t, "gqa_prefill_v16", v_to_f16_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), st, v, dst,
                    n8);
}

// ------------------------------------------------------------------ launch

template <int D, bool PAD, int MB, int DT, int OUT_DT>
static hipError_t launch_pf_t(const GqaPrefillParams& p, int Hk, hipStream_t st, KernelTimer* t) {
    dim3 grid((p.N + 15) / 16, Hk);
    // head_dim 64: two tiles per barrier (Llama-3.2-1B N = 512: 8.7 -> 8.0-8.2
    // us; four per barrier, in an 8-slot ring, measured the same); head_dim
    // 128 keeps one (the second tile's operands would not fit in registers)
    constexpr int TPB = D == 64 ? 2 : 1;
    return launch_k(t, "gqa_prefill", gqa_prefill_kernel<D, MB, DT, OUT_DT, TPB, PAD>, grid, dim3(64 * kWaves), st, p);
}

template <int D, bool PAD, int MB, int DT>
static hipError_t launch_pf_o(const GqaPrefillParams& p, int Hk, int out_dt, hipStream_t st, KernelTimer* t) {
    if (out_dt == DT_F32) return launch_pf_t<D, PAD, MB, DT, DT_F32>(p, Hk, st, t);
    if (out_dt == DT_F16) return launch_pf_t<D, PAD, MB, DT, DT_F16>(p, Hk, st, t);
    return launch_pf_t<D, PAD, MB, DT, DT_BF16>(p, Hk, st, t);
}

template <int D, bool PAD, int MB>
static hipError_t launch_pf_d(const GqaPrefillParams& p, int Hk, int dt, int out_dt, hipStream_t st,
                              KernelTimer* t) {
    if (dt == DT_F16) return launch_pf_o<D, PAD, MB, DT_F16>(p, Hk, out_dt, st, t);
    if (dt == kDtBf16V16) return launch_pf_o<D, PAD, MB, kDtBf16V16>(p, Hk, out_dt, st, t);
    return launch_pf_o<D, PAD, MB, DT_BF16>(p, Hk, out_dt, st, t);
}

template <int D, bool PAD>
static hipError_t launch_pf_g(const GqaPrefillParams& p, int Hk, int dt, int out_dt, hipStream_t st,
                              KernelTimer* t) {
    if (p.G <= 4) return launch_pf_d<D, PAD, 1>(p, Hk, dt, out_dt, st, t);
    return launch_pf_d<D, PAD, 2>(p, Hk, dt, out_dt, st, t);
}

// tiles per barrier interval of the warp-specialised kernel's 8-head
// blocks: 2 where V arrives as fp16 (Qwen2.5-7B shape N = 2048 52.3 -> 48.5
// us, N = 8192 619 -> 576). 4-head blocks keep 1: their smaller LDS ring
// lets two (head_dim 128) or three (64) blocks share a CU, which two tiles
// per step would halve (H32 Hk8 d128 N = 8192 673 against 805 us, d64
// 400 against 429)
template <int DT>
constexpr int kWsTps = DT == DT_BF16 ? 1 : 2;

// Merge of the key splits' partials: thread = (row, 4 output dims), rows
// (token, head); with o_s = O_s / l_s stored, out = sum_s w_s o_s / sum_s w_s,
// w_s = 2^(m_s - M) l_s, M the largest reference max (a split that saw no
// key of the row: m = -inf, l = 0, weight 0)
template <int OUT_DT, int MAXS>
__global__ __launch_bounds__(256) void gqa_prefill_combine_kernel(GqaPrefillParams p) {
    const int dq = p.hd >> 2;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t row = i / dq;
    if (row >= (int64_t)p.N * p.H) return;
    const int c = (int)(i - row * dq);
    const int ks = p.ksplit;  // <= MAXS
    const f32x2v_t* ml = reinterpret_cast<const f32x2v_t*>(p.ws_ml) + row * ks;
    const uint16_t* o = p.ws_o + row * ks * p.hd + 4 * c;
    // every split's (max, sum) and partial requested at once, unconditionally
    // (indices past ks re-read the last split and get weight 0): one memory
    // round trip instead of one per split
    f32x2v_t mls[MAXS];
    u32x2_t h[MAXS];
#pragma unroll
    for (int s = 0; s < MAXS; s++) {
        const int sc = min(s, ks - 1);
        mls[s] = ml[sc];
        h[s] = *reinterpret_cast<const u32x2_t*>(o + sc * p.hd);
    }
    float M = kNegInf;
#pragma unroll
    for (int s = 0; s < MAXS; s++) M = fmaxf(M, mls[s][0]);
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    float L = 0.f;
#pragma unroll
    for (int s = 0; s < MAXS; s++) {
        const bool live = s < ks && mls[s][0] != kNegInf;
        const float w = live ? fast_exp2(mls[s][0] - M) * mls[s][1] : 0.f;
        L += w;
        acc += w * f32x4_t{lo_f32<DT_F16>(h[s][0]), hi_f32<DT_F16>(h[s][0]), lo_f32<DT_F16>(h[s][1]),
                           hi_f32<DT_F16>(h[s][1])};
    }
    const f32x4_t r = acc * (L > 0.f ? 1.f / L : 0.f);
    const int64_t base = row * p.hd + 4 * c;
    if constexpr (OUT_DT == DT_F32) {
        *reinterpret_cast<f32x4_t*>(static_cast<float*>(p.out) + base) = r;
    } else {
        *reinterpret_cast<u32x2_t*>(static_cast<uint16_t*>(p.out) + base) =
            u32x2_t{pack2<OUT_DT>(r[0], r[1]), pack2<OUT_DT>(r[2], r[3])};
    }
}

template <int OUT_DT>
static hipError_t launch_pf_combine(const GqaPrefillParams& p, hipStream_t st, KernelTimer* t) {
    const int64_t threads = (int64_t)p.N * p.H * (p.hd / 4);
    const dim3 grid((unsigned)((threads + 255) / 256));
    static_assert(kPrefillMaxSplits == 32, "merge instantiations");
    if (p.ksplit <= 4)
        return launch_k(t, "gqa_prefill_combine", gqa_prefill_combine_kernel<OUT_DT, 4>, grid, dim3(256), st, p);
    if (p.ksplit <= 8)
        return launch_k(t, "gqa_prefill_combine", gqa_prefill_combine_kernel<OUT_DT, 8>, grid, dim3(256), st, p);
    if (p.ksplit <= 16)
        return launch_k(t, "gqa_prefill_combine", gqa_prefill_combine_kernel<OUT_DT, 16>, grid, dim3(256), st, p);
    return launch_k(t, "gqa_prefill_combine", gqa_prefill_combine_kernel<OUT_DT, 32>, grid, dim3(256), st, p);
}

int gqa_prefill_ws_slices(int G) { return G <= 4 ? 1 : (G + 7) / 8; }
int gqa_prefill_ws_step_keys(int G, int dt) { return (G <= 4 || dt == DT_BF16) ? 32 : 64; }
// one 8-head block per CU (128 KiB of LDS at head_dim 128); 4-head blocks:
// two at head_dim 128, three at 64
int gqa_prefill_ws_blocks_per_cu(int G, int D) { return G > 4 ? 1 : (D > 64 ? 2 : 3); }

// SPLIT: the kernel stores fp16 partials whatever the output type (one
// instantiation, OUT_DT = f32), and the combine writes the output
template <int D, bool PAD, int DT, int OUT_DT, bool SPLIT>
static hipError_t launch_pf_ws_k(const GqaPrefillParams& p, int Hk, hipStream_t st, KernelTimer* t) {
    const int nqb = (p.N + 15) / 16;
    const int ks = SPLIT ? p.ksplit : 1;
    if (p.G <= 4)
        return launch_k(t, "gqa_prefill", gqa_prefill_ws_kernel<D, 4, 1, 4, DT, OUT_DT, PAD, 1, SPLIT>,
                        dim3(nqb * Hk * ((p.G + 3) / 4) * ks), dim3(64 * 8), st, p, nqb, (p.G + 3) / 4, Hk);
    const int nslice = (p.G + 7) / 8;
    // 8-head blocks keep 4 PV waves (2 heads each): 8 PV waves (one head
    // each, 16-wave blocks) measured no faster
    constexpr int NPV = 4;
    // one head per S wave (two S waves per SIMD overlap each other's MFMA
    // and softmax phases); two heads per S wave, which halves the K reads
    // per row, measured slower (859 against 804 us at 7B N = 8192; with two
    // tiles per step 547 against 541 us)
    constexpr int SMB = 1;
    return launch_k(t, "gqa_prefill", gqa_prefill_ws_kernel<D, 8, SMB, NPV, DT, OUT_DT, PAD, kWsTps<DT>, SPLIT>,
                    dim3(nqb * Hk * nslice * ks), dim3(64 * (8 / SMB + NPV)), st, p, nqb, nslice, Hk);
}

template <int D, bool PAD, int DT, int OUT_DT>
static hipError_t launch_pf_ws_t(const GqaPrefillParams& p, int Hk, hipStream_t st, KernelTimer* t) {
    if (p.ksplit <= 1) return launch_pf_ws_k<D, PAD, DT, OUT_DT, false>(p, Hk, st, t);
    if (p.ksplit > kPrefillMaxSplits) return hipErrorInvalidValue;  // the merge's unrolled bound
    const hipError_t e = launch_pf_ws_k<D, PAD, DT, DT_F32, true>(p, Hk, st, t);
    return e != hipSuccess ? e : launch_pf_combine<OUT_DT>(p, st, t);
}

template <int D, bool PAD, int DT>
static hipError_t launch_pf_ws_o(const GqaPrefillParams& p, int Hk, int out_dt, hipStream_t st, KernelTimer* t) {
    if (out_dt == DT_F32) return launch_pf_ws_t<D, PAD, DT, DT_F32>(p, Hk, st, t);
    if (out_dt == DT_F16) return launch_pf_ws_t<D, PAD, DT, DT_F16>(p, Hk, st, t);
    return launch_pf_ws_t<D, PAD, DT, DT_BF16>(p, Hk, st, t);
}

template <int D, bool PAD>
static hipError_t launch_pf_ws(const GqaPrefillParams& p, int Hk, int dt, int out_dt, hipStream_t st,
                               KernelTimer* t) {
    if (dt == DT_F16) return launch_pf_ws_o<D, PAD, DT_F16>(p, Hk, out_dt, st, t);
    if (dt == kDtBf16V16) return launch_pf_ws_o<D, PAD, kDtBf16V16>(p, Hk, out_dt, st, t);
    return launch_pf_ws_o<D, PAD, DT_BF16>(p, Hk, out_dt, st, t);
}

template <int DT>
static hipError_t launch_pf_short(const GqaPrefillParams& p, int Hk, int out_dt, hipStream_t st, KernelTimer* t) {
    // a 1-D deal of (kv head, query block) units over the XCDs (see the kernel)
    const int units = (p.N + 15) / 16 * Hk;
    const dim3 grid(8 * ((units + 7) / 8));
    if (out_dt == DT_F32) return launch_k(t, "gqa_prefill", gqa_prefill_short_kernel<DT, DT_F32>, grid, dim3(512), st, p);
    if (out_dt == DT_F16) return launch_k(t, "gqa_prefill", gqa_prefill_short_kernel<DT, DT_F16>, grid, dim3(512), st, p);
    return launch_k(t, "gqa_prefill", gqa_prefill_short_kernel<DT, DT_BF16>, grid, dim3(512), st, p);
}

bool gqa_prefill_short_fits(const GqaPrefillParams& p, int D) {
    const int kend = p.causal ? p.start_pos + p.N : p.kv_len;
    return D == 64 && p.hd == 64 && p.G <= 4 && kend <= kShortMaxKeys;
}

hipError_t launch_gqa_prefill(const GqaPrefillParams& p, int Hk, int D, int dt, int out_dt, int kernel,
                              hipStream_t st, KernelTimer* t) {
    const bool pad = p.hd != D;
    if (kernel == 3) {
        if (!gqa_prefill_short_fits(p, D) || dt == kDtBf16V16) return hipErrorInvalidValue;
        return dt == DT_F16 ? launch_pf_short<DT_F16>(p, Hk, out_dt, st, t) : launch_pf_short<DT_BF16>(p, Hk, out_dt, st, t);
    }
    if (kernel == 2) {
        if (D == 128) return pad ? launch_pf_ws<128, true>(p, Hk, dt, out_dt, st, t)
                                 : launch_pf_ws<128, false>(p, Hk, dt, out_dt, st, t);
        return pad ? launch_pf_ws<64, true>(p, Hk, dt, out_dt, st, t) : launch_pf_ws<64, false>(p, Hk, dt, out_dt, st, t);
    }
    if (D == 128) return pad ? launch_pf_g<128, true>(p, Hk, dt, out_dt, st, t)
                             : launch_pf_g<128, false>(p, Hk, dt, out_dt, st, t);
    return pad ? launch_pf_g<64, true>(p, Hk, dt, out_dt, st, t) : launch_pf_g<64, false>(p, Hk, dt, out_dt, st, t);
}

}  // namespace mugen_attn
