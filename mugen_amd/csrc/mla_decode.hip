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
//  * workgroup = (64 query rows, context split, sequence).  Two kernels:
//    "rows" (mla_decode_kernel: 4 waves of 16 rows, each doing S, softmax
//    and P.L for its rows; small 16-bit-q problems) and the warp-specialised
//    mla_decode_ws_kernel (S waves and P.L waves, everything else);
//  * latent tiles of 32 tokens stream into an LDS ring by direct
//    global->LDS DMA (global_load_lds_dwordx4), two tiles in flight; rows
//    are XOR-swizzled in 16-byte chunks so both MFMA operand reads are
//    bank-conflict free;
//  * S^T uses a token permutation (A-row m of token block nb is token
//    8*(m/4) + 4*nb + m%4) so each lane ends up holding 8 CONSECUTIVE tokens
//    of its query row: exactly its k-slots as the A operand of P.L, so P
//    never leaves registers;
//  * the P.L B operand (8 tokens of one latent dim per lane) comes from the
//    row-major tile through two ds_read_b64_tr_b16 transpose reads;
//  * softmax in the exp2 domain against a reference max set at each row's
//    first visible tile: later weights may exceed 1, so O is normally never
//    rescaled.  Only a score more than the weights' headroom above the
//    reference (rare) moves the row's reference up to that tile's max and
//    scales the row's sum and O by 2^(old - new) ("lazy re-base");
//  * every workgroup writes its split's (m, l) in fp32 and the normalised
//    o/l (a convex combination of latent rows) in fp16, in accumulator-
//    fragment order; mla_decode_combine merges the splits of a row with
//    fp32 log-sum-exp weights and fp32 accumulation;
//  * q in fp32 is split into hi + lo 16-bit halves (two MFMAs), keeping the
//    scores fp32-accurate like the reference's float q_absorbed.
#include "common.h"
#include "kernels.h"

namespace mugen_attn {

constexpr int kKR = 512;                // kv_lora_rank
constexpr int kRD = 64;                 // rope dims
constexpr int kCD = kKR + kRD;          // 576 latent dims per token
constexpr int kTT = 32;                 // tokens per LDS tile
constexpr int kRowBytes = kCD * 2;      // 1152 B per latent row (72 x 16-byte chunks)
constexpr int kTileBytes = kTT * kRowBytes;       // 36 KiB
constexpr int kDmaPerTile = kTileBytes / 1024;    // 36 one-KiB DMA instructions per 32-token tile
constexpr int kNBuf = 3;                // ring depth: two tiles in flight

// LDS swizzle: 16-byte chunk c of tile row r is stored at chunk c ^ swz(r).
// gfx950 LDS has 64 banks x 4 B.  Measured on the MI355X (bank-conflict
// counters of single-pattern probes): a ds_read_b128 runs in four phases of
// 16 lanes -- each 32-lane half split by the parity of its lane-quad index
// (lanes 0-3, 12-15, 20-23, 24-27 share a phase) -- and a ds_read_b64 /
// ds_read_b64_tr_b16 in two phases of 32 consecutive lanes.  1152-byte rows
// put every even row on bank 0 and every odd row on bank 32, so unswizzled
// the S operand reads (rows 8*(n/4) + n%4 + 4nb) cost 4x and the transpose
// reads (rows 8g + n/4 + 4hh) 4x their minimum.  XOR of row bits 1 and 3
// (an exhaustive search over XOR swizzles against that phase model) makes
// both conflict-free; it ignores row bits 2, 4 and 5, so the nb / hh row
// offsets and the token slices keep the same swizzle.
__host__ __device__ constexpr int swz(int r) {
    return (((r >> 1) & 1) * 2) ^ (((r >> 3) & 1) * 4);
}

// Reference-max headroom (log2 units): weights up to 2^TH are kept against
// a row's reference; a larger score re-bases the row.  bf16 P keeps fp32's
// exponent range (O stays far from fp32 overflow); fp16 P tops out at 65504.
template <int DT>
__device__ constexpr float headroom_log2() { return DT == DT_BF16 ? 64.f : 15.f; }

// O partial blob (normalised o/l, fp16), in MFMA accumulator-fragment
// order.  For sequence b, split s and 16-row block q, the 16-byte unit
//   (((b*S + s)*nq + q)*16 + dp)*64 + lane
// holds the 4-element fragments of column blocks 2dp and 2dp+1 (8 bytes
// each): rows 16q + 4*(lane/16) + i (i = 0..3) at column 16d + lane%16.  A
// wave stores, and the combine loads, 1 KiB contiguous per instruction.
__device__ __forceinline__ int64_t blob_pair(const MlaParams& p, int b, int s, int q, int dp, int lane) {
    return ((((int64_t)b * p.num_splits + s) * p.nq + q) * 16 + dp) * 64 + lane;
}

// First 64-row block of a sequence of T tokens that sees a key of split s.
// Query row r of a q_len-token step sees T - q_len + r / H + 1 keys, so
// block rb (rows 64 rb .. 64 rb + 63) sees split s iff (64 rb + 63) / H >=
// s chunk - T + q_len; the last block, whose last row sees all T keys, sees
// every split.  Decode steps (q_len 1): every block sees every split.
__device__ __forceinline__ int mla_rb_first(const MlaParams& p, int T, int s) {
    const int x = s * p.chunk - T + p.q_len;
    return x <= 0 ? 0 : min((p.H * x) >> 6, p.nrb - 1);
}

// XCD-aware work mapping, shared by both kernels.  Workgroups are dealt to
// the 8 XCDs round-robin by blockIdx.  The work units are the (sequence,
// split, 64-row block) triples that see at least one key: sequence j
// contributes ceil(seq_lens[j] / chunk) splits, and of split s the blocks
// from mla_rb_first on (all of them for decode steps; a causal prompt's
// early blocks see only its first splits).  Units are numbered group-major
// over the (sequence, split) groups, a group's blocks consecutive.  Each
// XCD takes a contiguous range of ceil(units / 8), so the row blocks of a
// group share one XCD's L2 for the latent tiles (a group straddles two XCDs
// at most at a range boundary), consecutive splits of a sequence share it
// for the query rows, and every XCD gets an even share, also with fewer
// groups than XCDs (a long prompt: many row blocks, few splits).  The grid
// is sized from the host's unit count (exact with the length hint, an upper
// bound without); surplus workgroups exit at once.
__device__ __forceinline__ bool mla_map(const MlaParams& p, int& b, int& s, int& rb) {
    const int xcd = blockIdx.x % 8, slot = blockIdx.x / 8;
    if (p.q_len == 1) {  // decode: every block of every split
        int nact = 0;
        for (int j = 0; j < p.B; j++) nact += (clamp_len(p.seq_lens[j], p.max_T) + p.chunk - 1) / p.chunk;  // uniform scalar loop
        const int units = nact * p.nrb;
        const int upx = (units + 7) / 8;
        const int unit = xcd * upx + slot;
        if (slot >= upx || unit >= units) return false;
        const int grp = unit / p.nrb;
        rb = unit - grp * p.nrb;
        for (int j = 0, acc = 0; j < p.B; j++) {
            const int nsj = (clamp_len(p.seq_lens[j], p.max_T) + p.chunk - 1) / p.chunk;
            if (grp < acc + nsj) {
                b = j;
                s = grp - acc;
                return s < p.num_splits;  // (a split past the partials' stride: nothing to write it to)
            }
            acc += nsj;
        }
        return false;
    }
    // causal multi-token step: the splits every block sees (s chunk <=
    // T - q_len) whole, then the last few from mla_rb_first on
    auto split_range = [&](int Tj, int& nsj, int& s0) {
        nsj = (Tj + p.chunk - 1) / p.chunk;
        s0 = min(nsj, Tj >= p.q_len ? (Tj - p.q_len) / p.chunk + 1 : 0);
    };
    int units = 0;  // uniform scalar loops
    for (int j = 0; j < p.B; j++) {
        const int Tj = clamp_len(p.seq_lens[j], p.max_T);
        int nsj, s0;
        split_range(Tj, nsj, s0);
        units += s0 * p.nrb;
        for (int sj = s0; sj < nsj; sj++) units += p.nrb - mla_rb_first(p, Tj, sj);
    }
    const int upx = (units + 7) / 8;
    const int unit = xcd * upx + slot;
    if (slot >= upx || unit >= units) return false;
    for (int j = 0, acc = 0; j < p.B; j++) {
        const int Tj = clamp_len(p.seq_lens[j], p.max_T);
        int nsj, s0;
        split_range(Tj, nsj, s0);
        if (unit < acc + s0 * p.nrb) {
            const int u = unit - acc;
            b = j;
            s = u / p.nrb;
            rb = u - s * p.nrb;
            return s < p.num_splits;
        }
        acc += s0 * p.nrb;
        for (int sj = s0; sj < nsj; sj++) {
            const int first = mla_rb_first(p, Tj, sj);
            if (unit < acc + p.nrb - first) {
                b = j;
                s = sj;
                rb = first + (unit - acc);
                return s < p.num_splits;
            }
            acc += p.nrb - first;
        }
    }
    return false;
}

// Kernel "rows" (16-bit q, at most 64 query rows: small-head decode):
// workgroup = (64 query rows, context split, sequence), 4 waves of 16
// rows, one wave per SIMD.  Each wave keeps the q of its rows in registers
// (B operand of S^T = L . Q^T) and its 16 x 512 O accumulator.
template <int QDT, int DT>
__global__ __launch_bounds__(256) void mla_decode_kernel(MlaParams p) {
    constexpr int KS = kCD / 32;  // 18 k-steps over the 576 dims
    constexpr int NQ = (QDT == DT_F32) ? 2 : 1;
    constexpr float TH = headroom_log2<DT>();
    constexpr int NW = 4;                      // waves, one per SIMD
    constexpr int DPW = kDmaPerTile / NW;      // 1-KiB DMA ops per wave per tile
    constexpr int DSTRIDE = NW * 1024;         // LDS bytes between a wave's DMA ops
    __shared__ __attribute__((aligned(1024))) char ring[kNBuf * kTileBytes];

    int b, s, rb;
    if (!mla_map(p, b, s, rb)) return;  // grid padding past the last active unit
    MUGEN_TRACE(0);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int n = lane & 15, g = lane >> 4;
    const int T = clamp_len(p.seq_lens[b], p.max_T);
    const int t_begin = s * p.chunk;
    const int t_end = min(t_begin + p.chunk, T);
    // tiles past the last visible token of the workgroup's last row (a
    // causal prompt's early rows) are not walked; a split that no row of
    // the workgroup sees stores an empty partial (m = -inf, l = 0, o = 0)
    const int t_stop = min(t_end, max(t_begin, T - p.q_len + min(rb * 64 + 63, p.R - 1) / p.H + 1));
    const int ntiles = (t_stop - t_begin + kTT - 1) / kTT;
    const int row0 = rb * 64 + w * 16;
    const uint16_t* lat = p.lat + (int64_t)b * p.seq_stride;

    // ---- tile staging by LDS DMA: wave w fills LDS chunks [64K, 64K+64) of
    // the tile for K = w + 4k; LDS chunk (r, pc) holds source chunk
    // (r, pc ^ swz(r)).  Offsets are clamped to the split's last valid byte,
    // so tokens past t_end read valid cache rows (masked later)
    const uint32_t ring_base = lds_addr(&ring[0]);
    uint32_t dma_off[DPW];
#pragma unroll
    for (int k = 0; k < DPW; k++) {
        const int sl = 64 * (w + NW * k) + lane;
        const int r = sl / (kRowBytes / 16), pc = sl - r * (kRowBytes / 16);
        dma_off[k] = (uint32_t)(r * kRowBytes + ((pc ^ swz(r)) * 16));
    }
    auto issue = [&](int tt, int buf) {
        const uint16_t* tbase = lat + (int64_t)tt * kCD;  // wave-uniform
        const uint32_t lds0 = ring_base + buf * kTileBytes + w * 1024;
        if (tt + kTT <= t_end) {  // whole tile valid: precomputed offsets
#pragma unroll
            for (int k = 0; k < DPW; k++) dma16s(lds0 + k * DSTRIDE, tbase, dma_off[k]);
        } else {  // last tile of the split: clamp to its last valid chunk
            const uint32_t lim = (uint32_t)(t_end - tt) * kRowBytes - 16;
#pragma unroll
            for (int k = 0; k < DPW; k++) dma16s(lds0 + k * DSTRIDE, tbase, min(dma_off[k], lim));
        }
    };

    // ---- Q^T fragments (B operand): lane holds Q[row0+n][32ks+8g .. +8].
    // The first tiles' DMA goes out before the q loads: both latencies overlap
    if (ntiles > 0) issue(t_begin, 0);
    if (ntiles > 1) issue(t_begin + kTT, 1);
    u32x4_t qf[NQ][KS];
    const int row = row0 + n;
    const bool row_ok = row < p.R;
    // rows past R (padding of the last row block) have q = 0 and are
    // treated as visible everywhere; their output is never stored
    const int teff = row_ok ? (T - p.q_len + row / p.H + 1) : T;  // visible tokens of this lane's S-row
    {
        const int64_t qoff = ((int64_t)b * p.R + (row_ok ? row : 0)) * kCD + 8 * g;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            if constexpr (QDT == DT_F32) {
                // two 16-byte loads (q is 16-byte aligned, qoff a multiple of 8)
                const float* qp = static_cast<const float*>(p.q) + qoff + 32 * ks;
                const f32x4_t q0 = *reinterpret_cast<const f32x4_t*>(qp);
                const f32x4_t q1 = *reinterpret_cast<const f32x4_t*>(qp + 4);
                float x[8];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    x[j] = row_ok ? q0[j] : 0.f;
                    x[4 + j] = row_ok ? q1[j] : 0.f;
                }
                // hi = RNE 16-bit pack of the pair, lo = RNE pack of the residual
                u32x4_t fr[2];
                split_p<DT, 2>(x, fr);
                qf[0][ks] = fr[0];
                qf[NQ - 1][ks] = fr[1];
            } else {
                const uint16_t* qp = static_cast<const uint16_t*>(p.q) + qoff + 32 * ks;
                qf[0][ks] = row_ok ? load16(qp) : u32x4_t{0, 0, 0, 0};
            }
        }
    }
    // smallest visible length over the wave's rows: tiles below it need no mask
    const int teff_min = wave_min_i32(teff);

    // Q loads complete here, through a wait the compiler's wait-count pass
    // understands: it then inserts no vmcnt(0) inside the tile loop (where
    // it would also drain the ring's in-flight DMA it cannot see)
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    MUGEN_TRACE(1);

    // S operand (A): row ar = 8*(n/4) + n%4 (+4nb), logical chunk 4ks + g.
    // swz(ar) does not depend on nb; (4ks + g) ^ h = 8*(ks/2) + ((4*(ks%2) + g) ^ h)
    const int ar0 = 8 * (n >> 2) + (n & 3);
    const int hA = swz(ar0);
    const uint32_t a_off0 = ar0 * kRowBytes + ((g ^ hA) * 16);
    const uint32_t a_off1 = ar0 * kRowBytes + (((4 + g) ^ hA) * 16);
    // P.L operand (transpose reads): lane (i, g) of read hh reads row
    // 8g + 4hh + i/4, logical bytes 32d + 8*(i%4) = chunk 2d + (i%4)/2
    const int tr0 = 8 * g + (n >> 2);
    const int hT = swz(tr0);  // independent of hh
    uint32_t t_off[4];
#pragma unroll
    for (int j = 0; j < 4; j++)
        t_off[j] = tr0 * kRowBytes + (((2 * j + ((n & 3) >> 1)) ^ hT) * 16) + 8 * (n & 1);

    f32x4_t o[32];
    float m_ref = kNegInf, l_part = 0.f;  // reference max (log2 units) and partial sum
#pragma unroll
    for (int d = 0; d < 32; d++) o[d] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    const char* ring_bytes = &ring[0];
    int buf = 0;  // (tiles 0 and 1 were issued with the query loads)
    for (int it = 0; it < ntiles; it++) {
        if (it + 1 < ntiles) vm_wait<DPW>();
        else vm_wait<0>();
        lds_barrier();  // tile `it` landed for every wave; the buffer of tile it-1 is free
        // the next tile's DMA goes into the buffer freed by the barrier; its
        // DPW instructions are spread over the S k-steps below, so the
        // per-CU address unit works through them while the MFMAs run
        // instead of holding up the wave's first MFMA behind all of them
        const bool pf = it + kNBuf - 1 < ntiles;
        const int pf_tt = t_begin + kTT * (it + kNBuf - 1);
        const uint16_t* pf_src = lat + (int64_t)pf_tt * kCD;  // wave-uniform
        const uint32_t pf_lds = ring_base + (buf == 0 ? kNBuf - 1 : buf - 1) * kTileBytes + w * 1024;
        const uint32_t pf_lim = pf_tt + kTT <= t_end ? 0xFFFFFFFFu : (uint32_t)(t_end - pf_tt) * kRowBytes - 16;
        auto issue_k = [&](int k) {
            if (pf) dma16s(pf_lds + k * DSTRIDE, pf_src, min(dma_off[k], pf_lim));
        };
        const char* tile = ring_bytes + buf * kTileBytes;
        buf = buf == kNBuf - 1 ? 0 : buf + 1;
        const int tt = t_begin + kTT * it;

        // ---- S^T = L . Q^T  (two 16-token blocks), VGPR accumulators.
        // Software-pipelined: operands of k-step ks+SPD are requested while
        // step ks runs, so each LDS read has ~2 steps of MFMA work to land.
        constexpr int SPD = 3;
        auto a_ptr = [&](int ks, int nb) {
            return reinterpret_cast<const u32x4_t*>(tile + ((ks & 1) ? a_off1 : a_off0) + 128 * (ks >> 1) +
                                                    4 * kRowBytes * nb);
        };
        u32x4_t abuf[SPD][2];
#pragma unroll
        for (int j = 0; j < SPD; j++) {
            abuf[j][0] = *a_ptr(j, 0);
            abuf[j][1] = *a_ptr(j, 1);
        }
        f32x4_t sacc[2];
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
#pragma unroll
            for (int nb = 0; nb < 2; nb++) {
                const u32x4_t a = abuf[ks % SPD][nb];
#pragma unroll
                for (int qq = 0; qq < NQ; qq++)
                    sacc[nb] = mfma16x16x32<DT>(a, qf[qq][ks], (ks == 0 && qq == 0) ? f32x4_t{0.f, 0.f, 0.f, 0.f} : sacc[nb]);
            }
            if (ks + SPD < KS) {
                abuf[ks % SPD][0] = *a_ptr(ks + SPD, 0);
                abuf[ks % SPD][1] = *a_ptr(ks + SPD, 1);
            }
#pragma unroll
            for (int k = 0; k < DPW; k++)
                if ((k * KS) / DPW == ks) issue_k(k);
            // keep each step's reads SPD steps ahead of their MFMAs
            __builtin_amdgcn_sched_barrier(0);
        }
        // first P.L operands requested now, to land during the softmax
        constexpr int VPD = 6;
        auto tr_load = [&](int d) {
            const char* tp = tile + t_off[d & 3] + 128 * (d >> 2);
            const u32x2_t lo = lds_read_tr16(reinterpret_cast<const uint16_t*>(tp));
            const u32x2_t hi = lds_read_tr16(reinterpret_cast<const uint16_t*>(tp + 4 * kRowBytes));
            return u32x4_t{lo[0], lo[1], hi[0], hi[1]};
        };
        u32x4_t bbuf[VPD];
#pragma unroll
        for (int j = 0; j < VPD; j++) bbuf[j] = tr_load(j);

        // ---- softmax weights; lane holds tokens tt + 8g + (4nb + i) of row n.
        // A row's reference max is the max of its first visible tile (a
        // cross-lane reduction, taken only while some row of the wave has
        // none yet); afterwards each weight is exp2(s*scale*log2e - m_ref),
        // one fma + one exp2, and only edge tiles (split end, causal rows)
        // pay for masking.
        if (__any(m_ref == kNegInf)) {
            float mt = kNegInf;
#pragma unroll
            for (int nb = 0; nb < 2; nb++) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int tok = tt + 8 * g + 4 * nb + i;
                    const bool vis = tok < t_end && tok < teff;
                    mt = fmaxf(mt, vis ? sacc[nb][i] * p.scale_log2 : kNegInf);
                }
            }
            mt = max_x32(max_x16(mt));
            if (m_ref == kNegInf) m_ref = mt;  // O of this row is still 0
        }
        const float mneg = (m_ref == kNegInf) ? 0.f : -m_ref;
        float x[8];  // scores relative to the reference (log2 units), then weights
        auto rel = [&](auto masked_tag) {
            constexpr bool MASKED = decltype(masked_tag)::value;
#pragma unroll
            for (int nb = 0; nb < 2; nb++) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    float v = fmaf(sacc[nb][i], p.scale_log2, mneg);
                    if constexpr (MASKED) {
                        const int tok = tt + 8 * g + 4 * nb + i;
                        v = (tok < t_end && tok < teff) ? v : kNegInf;
                    }
                    x[4 * nb + i] = v;
                }
            }
        };
        // wave-uniform: interior tiles (the common case) carry no mask
        if (tt + kTT <= t_end && tt + kTT <= teff_min) rel(std::false_type{});
        else rel(std::true_type{});
        // Lazy re-base (rare): a score more than TH above its row's
        // reference would overflow the 16-bit weights, so the row's
        // reference moves up to the tile's max and its sum and O so far
        // scale by alpha = 2^(old - new)
        bool over = false;
#pragma unroll
        for (int e = 0; e < 8; e++) over |= x[e] > TH;
        if (__any(over)) {  // wave-uniform
            float mt = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])), fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
            mt = max_x32(max_x16(mt));
            const float shift = fmaxf(mt, 0.f);
            const float alpha = fast_exp2(-shift);
            m_ref += shift;
            l_part *= alpha;
#pragma unroll
            for (int e = 0; e < 8; e++) x[e] -= shift;
            f32x4_t a4;  // the factors of O rows 4g+i
#pragma unroll
            for (int i = 0; i < 4; i++) a4[i] = __shfl(alpha, 4 * g + i, 64);
#pragma unroll
            for (int d = 0; d < 32; d++) o[d] *= a4;
        }
#pragma unroll
        for (int e = 0; e < 8; e++) x[e] = fast_exp2(x[e]);
        l_part += ((x[0] + x[1]) + (x[2] + x[3])) + ((x[4] + x[5]) + (x[6] + x[7]));
        const u32x4_t pfrag =
            u32x4_t{pack2<DT>(x[0], x[1]), pack2<DT>(x[2], x[3]), pack2<DT>(x[4], x[5]), pack2<DT>(x[6], x[7])};

        // ---- O += P . L[:, 0:512]; B operand L[tt + 8g + j][16d + n], j < 8.
        // The schedule is pinned to [MFMA][2 transpose reads of d+VPD] so
        // VPD steps of reads stay in flight behind the MFMAs.
#pragma unroll
        for (int d = 0; d < 32; d++) {
            const u32x4_t bf = bbuf[d % VPD];
            if (d + VPD < 32) bbuf[d % VPD] = tr_load(d + VPD);
            o[d] = mfma16x16x32<DT>(pfrag, bf, o[d]);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (d + VPD < 32) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
    }

    // ---- epilogue: (m, l, o/l) partial of this split.  The normalised O is
    // a convex combination of latent rows (within their f16 range) and goes
    // out as fp16 in accumulator-fragment order (4 rows x 1 column per lane,
    // 512 B contiguous per store instruction); m and l stay fp32.
    MUGEN_TRACE(3);
    const float lrow = sum_x32(sum_x16(l_part));  // S-layout row n: the split's full sum
    const float c0 = lrow > 0.f ? 1.f / lrow : 0.f;
    float k0[4];  // the factors of O rows 4g+i
#pragma unroll
    for (int i = 0; i < 4; i++) k0[i] = __shfl(c0, 4 * g + i, 64);
    if (row0 < p.R) {
        u32x4_t* dst = reinterpret_cast<u32x4_t*>(p.ws_o) + blob_pair(p, b, s, row0 >> 4, 0, lane);
#pragma unroll
        for (int d = 0; d < 32; d += 2) {
            uint32_t h[4];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const f32x4_t v = o[d + e] * f32x4_t{k0[0], k0[1], k0[2], k0[3]};
                h[2 * e] = pack2<DT_F16>(v[0], v[1]);
                h[2 * e + 1] = pack2<DT_F16>(v[2], v[3]);
            }
            dst[(d >> 1) * 64] = u32x4_t{h[0], h[1], h[2], h[3]};
        }
    }
    if (g == 0 && row_ok) {
        const int64_t slot_ml = ((int64_t)b * p.num_splits + s) * p.R + row;
        p.ws_ml[slot_ml * 2 + 0] = m_ref;
        p.ws_ml[slot_ml * 2 + 1] = lrow;
    }
    MUGEN_TRACE(5);
}

// Warp-specialised kernel: 8 waves, two per SIMD, 64 query rows per
// workgroup, 32-token tiles.  Waves 0-3 ("S waves") each hold the q of 16
// rows in registers, compute S^T = L . Q^T for the tile and its softmax
// weights, and write P to LDS in the A-operand layout of P . V.  Waves 4-7
// ("PV waves") each own a 128-column quarter of O for all 64 rows and
// accumulate O += P . L[:, cols] from that P; they also move the tiles by
// LDS DMA.  The S waves work on tile j while the PV waves consume tile
// j - 1, so each SIMD runs one wave of each kind: the MFMA pipe is fed from
// two instruction streams (one wave cannot issue MFMAs faster than about one
// per 18 clocks; two reach about one per 10) and one wave's softmax, LDS
// waits and barrier overlap the other's MFMAs.  Neither role holds both q
// (72 registers for 16 rows) and O (128 for a 64 x 128 quarter), so a wave
// fits the 256 registers of two waves per SIMD.
//
// LDS: a 4-slot ring of 32-token tiles (two tiles in flight, one read by the
// S waves, one by the PV waves) and a double-buffered P.  One barrier per
// tile: at barrier j the S waves have written P(j-1) and the PV waves have
// finished tile j-2, whose slot then receives tile j+2.
template <int QDT, int DT>
__global__ __launch_bounds__(512) void mla_decode_ws_kernel(MlaParams p) {
    constexpr int KS = kCD / 32;          // 18 k-steps over the 576 dims
    // fp32 q: each S wave holds q as hi + lo 16-bit parts (RNE split) and
    // issues two MFMAs per k-step, so S carries ~2^-16 relative q error
    // instead of 2^-8 / 2^-11
    constexpr int NQ = (QDT == DT_F32) ? 2 : 1;
    constexpr float TH = headroom_log2<DT>();
    constexpr int NSLOT = 4;
    constexpr int DPW = kDmaPerTile / 4;  // 9 one-KiB DMA ops per PV wave per tile
    constexpr int PBUF = 4 * 64 * 16;     // one P buffer: 4 row blocks x 64 lanes x 16 B
    __shared__ __attribute__((aligned(1024))) char ring[NSLOT * kTileBytes + 2 * PBUF];
    __shared__ float2 ml_x[64];           // per row: (reference max, sum) from the S waves
    __shared__ __attribute__((aligned(16))) float rs_alpha[2][64];  // per tile parity and row: O's re-base factor
    __shared__ __attribute__((aligned(16))) int rs_flag[2][4];  // per tile parity and S wave: any row re-based

    int b, s, rb;
    if (!mla_map(p, b, s, rb)) return;
    MUGEN_TRACE(0);

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool s_wave = w < 4;
    const int wr = w & 3;  // S wave: row block; PV wave: column quarter
    const int n = lane & 15, g = lane >> 4;
    const int T = clamp_len(p.seq_lens[b], p.max_T);
    const int t_begin = s * p.chunk;
    const int t_end = min(t_begin + p.chunk, T);
    const int row0 = rb * 64;  // first query row of the workgroup
    // tiles past the last visible token of the workgroup's last row (a
    // causal prompt's early rows) are not walked; a split that no row of
    // the workgroup sees stores an empty partial (m = -inf, l = 0, o = 0)
    const int t_stop = min(t_end, max(t_begin, T - p.q_len + min(row0 + 63, p.R - 1) / p.H + 1));
    const int ntiles = (t_stop - t_begin + kTT - 1) / kTT;
    const uint16_t* lat = p.lat + (int64_t)b * p.seq_stride;
    const uint32_t ring_base = lds_addr(&ring[0]);
    char* pbuf = &ring[NSLOT * kTileBytes];

    // ---- PV waves: DMA of tile tt into slot sl (wave wr moves LDS chunks
    // [64K, 64K+64) for K = wr + 4k; chunk (r, pc) holds source chunk
    // (r, pc ^ swz(r)); the split's last tile is clamped to valid rows)
    uint32_t dma_off[DPW];  // this lane's byte offset in a tile per DMA op (tile-invariant)
#pragma unroll
    for (int k = 0; k < DPW; k++) {
        const int sl = 64 * (wr + 4 * k) + lane;
        const int r = sl / (kRowBytes / 16), pc = sl - r * (kRowBytes / 16);
        dma_off[k] = (uint32_t)(r * kRowBytes + ((pc ^ swz(r)) * 16));
    }
    auto issue = [&](int tile_idx) {
        const int tt = t_begin + kTT * tile_idx;
        const uint16_t* src = lat + (int64_t)tt * kCD;
        const uint32_t lds0 = ring_base + (tile_idx % NSLOT) * kTileBytes + wr * 1024;
        if (tt + kTT <= t_end) {  // wave-uniform: interior tiles need no clamp
#pragma unroll
            for (int k = 0; k < DPW; k++) dma16s(lds0 + k * 4096, src, dma_off[k]);
        } else {
            const uint32_t lim = (uint32_t)(t_end - tt) * kRowBytes - 16;
#pragma unroll
            for (int k = 0; k < DPW; k++) dma16s(lds0 + k * 4096, src, min(dma_off[k], lim));
        }
    };

    if (s_wave) {
        // ================================================== S waves
        const int rowq = row0 + 16 * wr + n;  // S-layout row of this lane
        const bool ok = rowq < p.R;
        const int teff = ok ? (T - p.q_len + rowq / p.H + 1) : T;  // visible tokens of the row
        u32x4_t qf[NQ][KS];
        if constexpr (QDT == DT_F32) {
            const float* qp = static_cast<const float*>(p.q) + ((int64_t)b * p.R + (ok ? rowq : 0)) * kCD + 8 * g;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const f32x4_t q0 = *reinterpret_cast<const f32x4_t*>(qp + 32 * ks);
                const f32x4_t q1 = *reinterpret_cast<const f32x4_t*>(qp + 32 * ks + 4);
                float x[8];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    x[e] = ok ? q0[e] : 0.f;
                    x[4 + e] = ok ? q1[e] : 0.f;
                }
                u32x4_t fr[2];
                split_p<DT, 2>(x, fr);
                qf[0][ks] = fr[0];
                qf[1][ks] = fr[1];
            }
        } else {
            const uint16_t* qp = static_cast<const uint16_t*>(p.q) + ((int64_t)b * p.R + (ok ? rowq : 0)) * kCD + 8 * g;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) qf[0][ks] = ok ? load16(qp + 32 * ks) : u32x4_t{0, 0, 0, 0};
        }
        const int teff_min = __builtin_amdgcn_readfirstlane(wave_min_i32(teff));  // wave-uniform: the mask test branches on it
        // q is waited for chunk by chunk in the first tile's k-loop
        MUGEN_TRACE(1);
        const int ar0 = 8 * (n >> 2) + (n & 3);
        const int hA = swz(ar0);
        const uint32_t a_off0 = ar0 * kRowBytes + ((g ^ hA) * 16);
        const uint32_t a_off1 = ar0 * kRowBytes + (((4 + g) ^ hA) * 16);
        float m_ref = kNegInf, l_part = 0.f;

        for (int j = 0; j <= ntiles; j++) {
            if (j == 4) MUGEN_TRACE(6);
            lds_barrier();  // B_j: tile j landed (the PV waves waited for it)
            if (j == 4) MUGEN_TRACE(7);
            if (j == 1) MUGEN_TRACE(14);
            if (j == 2) MUGEN_TRACE(15);
            if (j == ntiles) break;
            const char* tile = &ring[(j % NSLOT) * kTileBytes];
            const int tt = t_begin + kTT * j;
            constexpr int SPD = 4;
            auto a_ptr = [&](int ks, int nb) {
                return reinterpret_cast<const u32x4_t*>(tile + ((ks & 1) ? a_off1 : a_off0) + 128 * (ks >> 1) +
                                                        4 * kRowBytes * nb);
            };
            u32x4_t abuf[SPD][2];
#pragma unroll
            for (int q = 0; q < SPD; q++) {
                abuf[q][0] = *a_ptr(q, 0);
                abuf[q][1] = *a_ptr(q, 1);
            }
            f32x4_t sacc[2];
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                // first tile: wait for q chunk ks only (the 18 q loads are the
                // S wave's only vector-memory operations before this loop)
                if (QDT != DT_F32 && j == 0) {  // (fp32 q was waited for by its split)
                    switch (KS - 1 - ks) {  // ks is a constant after unrolling: one s_waitcnt
#define MLA_VMW(N) case N: vm_wait<N>(); break;
                        MLA_VMW(0) MLA_VMW(1) MLA_VMW(2) MLA_VMW(3) MLA_VMW(4) MLA_VMW(5) MLA_VMW(6) MLA_VMW(7)
                        MLA_VMW(8) MLA_VMW(9) MLA_VMW(10) MLA_VMW(11) MLA_VMW(12) MLA_VMW(13) MLA_VMW(14)
                        MLA_VMW(15) MLA_VMW(16) MLA_VMW(17)
#undef MLA_VMW
                    }
                }
#pragma unroll
                for (int nb = 0; nb < 2; nb++)
#pragma unroll
                    for (int qq = 0; qq < NQ; qq++) {
                        sacc[nb] = mfma16x16x32<DT>(abuf[ks % SPD][nb], qf[qq][ks],
                                                    (ks == 0 && qq == 0) ? f32x4_t{0.f, 0.f, 0.f, 0.f} : sacc[nb]);
                    }
                if (ks + SPD < KS) {
                    abuf[ks % SPD][0] = *a_ptr(ks + SPD, 0);
                    abuf[ks % SPD][1] = *a_ptr(ks + SPD, 1);
                }
                // keep each step's reads SPD steps ahead of their MFMAs (the
                // scheduler would otherwise sink them next to their use)
                __builtin_amdgcn_sched_barrier(0);
            }
            if (j == 4) MUGEN_TRACE(11);
            // softmax weights against the row's reference max (the max of its
            // first visible tile); lane holds tokens tt + 8g + 4nb + i of row n
            if (__any(m_ref == kNegInf)) {
                float mt = kNegInf;
#pragma unroll
                for (int nb = 0; nb < 2; nb++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int tok = tt + 8 * g + 4 * nb + i;
                        mt = fmaxf(mt, (tok < t_end && tok < teff) ? sacc[nb][i] * p.scale_log2 : kNegInf);
                    }
                mt = max_x32(max_x16(mt));
                if (m_ref == kNegInf) m_ref = mt;
            }
            const float mneg = (m_ref == kNegInf) ? 0.f : -m_ref;
            float x[8];  // scores relative to the reference (log2 units), then weights
            auto rel = [&](auto masked_tag) {
                constexpr bool MASKED = decltype(masked_tag)::value;
#pragma unroll
                for (int nb = 0; nb < 2; nb++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        float v = fmaf(sacc[nb][i], p.scale_log2, mneg);
                        if constexpr (MASKED) {
                            const int tok = tt + 8 * g + 4 * nb + i;
                            v = (tok < t_end && tok < teff) ? v : kNegInf;
                        }
                        x[4 * nb + i] = v;
                    }
            };
            // wave-uniform branch: interior tiles (the common case) carry no mask
            if (tt + kTT <= t_end && tt + kTT <= teff_min) rel(std::false_type{});
            else rel(std::true_type{});
            // Lazy re-base: a score more than TH above its row's reference
            // would overflow the 16-bit weights, so the row's reference moves
            // up to the tile's max: its weights and sum so far scale by
            // alpha = 2^(old - new), and the PV waves scale the row's O by
            // the same alpha before they add this tile (rare: only scores
            // that climb far above the first tile's take this branch)
            bool over = false;
#pragma unroll
            for (int e = 0; e < 8; e++) over |= x[e] > TH;
            const bool rebase = __any(over);  // wave-uniform
            if (rebase) {
                float mt = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])), fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
                mt = max_x32(max_x16(mt));            // the row's tile max, relative to its reference
                const float shift = fmaxf(mt, 0.f);  // rows under their reference keep it
                const float alpha = fast_exp2(-shift);
                m_ref += shift;
                l_part *= alpha;
#pragma unroll
                for (int e = 0; e < 8; e++) x[e] -= shift;
                if (g == 0) rs_alpha[j & 1][16 * wr + n] = alpha;
            }
            if (lane == 0) rs_flag[j & 1][wr] = rebase ? 1 : 0;
#pragma unroll
            for (int e = 0; e < 8; e++) x[e] = fast_exp2(x[e]);
            l_part += ((x[0] + x[1]) + (x[2] + x[3])) + ((x[4] + x[5]) + (x[6] + x[7]));
            *reinterpret_cast<u32x4_t*>(pbuf + (j & 1) * PBUF + (wr * 64 + lane) * 16) =
                u32x4_t{pack2<DT>(x[0], x[1]), pack2<DT>(x[2], x[3]), pack2<DT>(x[4], x[5]), pack2<DT>(x[6], x[7])};
            if (j == 4) MUGEN_TRACE(12);
        }
        MUGEN_TRACE(3);
        // epilogue 1: the row's (reference max, sum) for the PV waves
        const float lrow = sum_x32(sum_x16(l_part));
        if (g == 0) ml_x[16 * wr + n] = make_float2(m_ref, lrow);
        __syncthreads();  // E1
        if (g == 0 && ok) {
            const int64_t slot_ml = ((int64_t)b * p.num_splits + s) * p.R + rowq;
            store_wt(&p.ws_ml[slot_ml * 2 + 0], m_ref);
            store_wt(&p.ws_ml[slot_ml * 2 + 1], lrow);
        }
        MUGEN_TRACE(5);
    } else {
        // ================================================== PV waves
        if (ntiles > 0) issue(0);
        if (ntiles > 1) issue(1);
        // V operand (transpose reads): lane (i, g) of read hh reads row
        // 8g + 4hh + i/4, logical bytes 32cb + 8*(i%4) (column block cb)
        const int tr0 = 8 * g + (n >> 2);
        const int hT = swz(tr0);
        uint32_t t_off[4];
#pragma unroll
        for (int q = 0; q < 4; q++)
            t_off[q] = tr0 * kRowBytes + (((2 * q + ((n & 3) >> 1)) ^ hT) * 16) + 8 * (n & 1);
        f32x4_t o[4][8];  // [row block][column block 8wr + d]
#pragma unroll
        for (int mb = 0; mb < 4; mb++)
#pragma unroll
            for (int d = 0; d < 8; d++) o[mb][d] = f32x4_t{0.f, 0.f, 0.f, 0.f};

        for (int j = 0; j <= ntiles; j++) {
            // tile j must have landed for the S waves: this wave's DMAs
            // complete in order and tile j+1 may still fly
            if (j == 4) MUGEN_TRACE(6);
            if (j + 1 < ntiles) vm_wait<DPW>();
            else vm_wait<0>();
            if (j == 4) MUGEN_TRACE(13);
            lds_barrier();  // B_j
            if (j == 0) MUGEN_TRACE(1);
            if (j == 4) MUGEN_TRACE(7);
            if (j + 2 < ntiles) issue(j + 2);  // into the slot of tile j-2, finished before B_j
            if (j == 0) continue;
            // O += P(j-1) . L(j-1)[:, 128wr .. +128]
            const char* tile = &ring[((j - 1) % NSLOT) * kTileBytes];
            const char* pb = pbuf + ((j - 1) & 1) * PBUF;
            // the S waves re-based some rows for tile j-1 (rare): their O
            // scales by the rows' factors before this tile is added
            const i32x4_t fl = *reinterpret_cast<const i32x4_t*>(&rs_flag[(j - 1) & 1][0]);
            u32x4_t pa[4];
#pragma unroll
            for (int mb = 0; mb < 4; mb++) pa[mb] = *reinterpret_cast<const u32x4_t*>(pb + (mb * 64 + lane) * 16);
            if (__builtin_amdgcn_readfirstlane(fl[0] | fl[1] | fl[2] | fl[3])) {
#pragma unroll
                for (int mb = 0; mb < 4; mb++) {
                    // row block mb belongs to S wave mb; only a wave that
                    // re-based wrote this tile's factors
                    if (!__builtin_amdgcn_readfirstlane(fl[mb])) continue;
                    const f32x4_t a = *reinterpret_cast<const f32x4_t*>(&rs_alpha[(j - 1) & 1][16 * mb + 4 * g]);
#pragma unroll
                    for (int d = 0; d < 8; d++) o[mb][d] *= a;
                }
            }
            auto tr_load = [&](int d) {
                const int cb = 8 * wr + d;
                const char* tp = tile + t_off[cb & 3] + 128 * (cb >> 2);
                const u32x2_t lo = lds_read_tr16(reinterpret_cast<const uint16_t*>(tp));
                const u32x2_t hi = lds_read_tr16(reinterpret_cast<const uint16_t*>(tp + 4 * kRowBytes));
                return u32x4_t{lo[0], lo[1], hi[0], hi[1]};
            };
            constexpr int VPD = 2;  // transpose reads ahead of their MFMAs (2 measured ahead of 1, 3, 4 and 8)
            u32x4_t vb[VPD];
#pragma unroll
            for (int q = 0; q < VPD; q++) vb[q] = tr_load(q);
#pragma unroll
            for (int d = 0; d < 8; d++) {
                const u32x4_t bf = vb[d % VPD];
                if (d + VPD < 8) vb[d % VPD] = tr_load(d + VPD);
#pragma unroll
                for (int mb = 0; mb < 4; mb++) o[mb][d] = mfma16x16x32<DT>(pa[mb], bf, o[mb][d]);
            }
            if (j == 4) MUGEN_TRACE(12);
        }
        MUGEN_TRACE(3);
        __syncthreads();  // E1: the S waves published (max, sum) per row
        // epilogue: o/l in fp16, accumulator-fragment order (16-byte pairs
        // of column blocks)
#pragma unroll
        for (int mb = 0; mb < 4; mb++) {
            const int rblk = row0 + 16 * mb;
            float k0[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float l = ml_x[16 * mb + 4 * g + i].y;
                k0[i] = l > 0.f ? 1.f / l : 0.f;
            }
            if (rblk < p.R) {
                u32x4_t* dst = reinterpret_cast<u32x4_t*>(p.ws_o) + blob_pair(p, b, s, rblk >> 4, 4 * wr, lane);
#pragma unroll
                for (int d = 0; d < 8; d += 2) {
                    uint32_t h[4];
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        const f32x4_t v = o[mb][d + e] * f32x4_t{k0[0], k0[1], k0[2], k0[3]};
                        h[2 * e] = pack2<DT_F16>(v[0], v[1]);
                        h[2 * e + 1] = pack2<DT_F16>(v[2], v[3]);
                    }
                    store_wt(&dst[(d >> 1) * 64], u32x4_t{h[0], h[1], h[2], h[3]});
                }
            }
        }
        MUGEN_TRACE(5);
    }
}

// Log-sum-exp merge of the split partials.  Workgroup = (16-row block,
// group of 2 NW column blocks, sequence), NW waves.  The per-row split
// weights w_s = 2^(m_s - M) l_s are formed once in LDS (4 NW splits x 16
// rows in parallel); then lane l of wave w reads, per split, the fp16
// fragments (4 rows x 1 column) of column blocks 2w, 2w+1 of the group --
// the order the main kernel wrote, 512 B contiguous per wave -- and
// accumulates in fp32.
template <int OUT_DT, int NW>
__global__ __launch_bounds__(64 * NW) void mla_decode_combine_kernel(MlaParams p) {
    constexpr int SP = 64 * NW / 16;  // split phases of the weights
    __shared__ __attribute__((aligned(16))) float wts[kMaxMlaSplits][16];
    __shared__ float red[SP][16];
    __shared__ float linv[16];
    const int qb = blockIdx.x, dg = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, dsub = tid >> 6;
    const int g = lane >> 4, n = lane & 15;
    const int T = clamp_len(p.seq_lens[b], p.max_T);
    int nact = min(p.num_splits, (T + p.chunk - 1) / p.chunk);
    if (p.q_len > 1) {
        // the rows' 64-row block has units for the splits its last row sees
        // only (mla_map): the first ceil(visible / chunk)
        const int vis = T - p.q_len + min(qb / 4 * 64 + 63, p.R - 1) / p.H + 1;
        nact = min(nact, (max(vis, 0) + p.chunk - 1) / p.chunk);
    }
    const int64_t ml_st = (int64_t)p.R * 2;  // floats between splits of one row
    const float* ml0 = p.ws_ml + (int64_t)b * p.num_splits * p.R * 2;

    MUGEN_TRACE(8);
    const int d0 = dg * 2 * NW + dsub * 2;
    const u32x4_t* src = reinterpret_cast<const u32x4_t*>(p.ws_o) + blob_pair(p, b, 0, qb, d0 >> 1, lane);
    const int64_t frag_st = (int64_t)p.nq * 16 * 64;  // 16-byte units between splits
    // the first PF splits' fp16 fragments are requested before the split
    // weights are known, so their latency overlaps the (m, l) reads
    constexpr int PF = 16;
    u32x4_t fa[PF];
    auto prefetch = [&]() {  // unconditional (clamped) loads keep the wait counts exact
#pragma unroll
        for (int j = 0; j < PF; j++) fa[j] = src[max(0, min(j, nact - 1)) * frag_st];
    };
    // split weights: thread (row r = tid%16, split phase sl = tid/16).  The
    // (m, l) of splits sl and sl + 16 are loaded once, ahead of the
    // fragments; further splits are read from the workspace in the loops.
    const int r = tid & 15, sl = tid >> 4, row = qb * 16 + r;
    const bool rok = row < p.R;
    constexpr int MLC = 32 / SP;
    f32x2v_t mlc[MLC];
#pragma unroll
    for (int k = 0; k < MLC; k++) {
        const int s = sl + SP * k;
        mlc[k] = (rok && s < nact) ? *reinterpret_cast<const f32x2v_t*>(ml0 + s * ml_st + row * 2)
                                   : f32x2v_t{kNegInf, 0.f};
    }
    prefetch();
    float mx = kNegInf;
#pragma unroll
    for (int k = 0; k < MLC; k++) mx = fmaxf(mx, mlc[k][0]);
    for (int s = sl + SP * MLC; s < nact; s += SP) mx = fmaxf(mx, rok ? ml0[s * ml_st + row * 2] : kNegInf);
    red[sl][r] = mx;
    __syncthreads();
    float M = kNegInf;
#pragma unroll
    for (int j = 0; j < SP; j++) M = fmaxf(M, red[j][r]);
    __syncthreads();
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < MLC; k++) {
        const int s = sl + SP * k;
        if (s < nact) {
            const float wgt = (mlc[k][0] == kNegInf) ? 0.f : fast_exp2(mlc[k][0] - M) * mlc[k][1];
            wts[s][r] = wgt;
            sum += wgt;
        }
    }
    for (int s = sl + SP * MLC; s < nact; s += SP) {
        const float m = rok ? ml0[s * ml_st + row * 2] : kNegInf;
        const float wgt = (m == kNegInf) ? 0.f : fast_exp2(m - M) * ml0[s * ml_st + row * 2 + 1];
        wts[s][r] = wgt;
        sum += wgt;
    }
    red[sl][r] = sum;
    __syncthreads();
    if (tid < 16) {
        float L = 0.f;
#pragma unroll
        for (int j = 0; j < SP; j++) L += red[j][tid];
        linv[tid] = L > 0.f ? 1.f / L : 0.f;
    }
    __syncthreads();
    MUGEN_TRACE(9);

    auto h4 = [](uint32_t a, uint32_t b) {
        return f32x4_t{lo_f32<DT_F16>(a), hi_f32<DT_F16>(a), lo_f32<DT_F16>(b), hi_f32<DT_F16>(b)};
    };
    f32x4_t A0 = {0.f, 0.f, 0.f, 0.f}, A1 = A0;
#pragma unroll
    for (int j = 0; j < PF; j++) {
        if (j < nact) {
            const f32x4_t w = *reinterpret_cast<const f32x4_t*>(&wts[j][4 * g]);
            A0 += w * h4(fa[j][0], fa[j][1]);
            A1 += w * h4(fa[j][2], fa[j][3]);
        }
    }
    // sequences with more than PF splits: 8 splits (16 loads) in flight per step
    constexpr int U = 8;
    int s = PF;
    for (; s + U <= nact; s += U) {
        u32x4_t ga[U];
#pragma unroll
        for (int j = 0; j < U; j++) ga[j] = src[(s + j) * frag_st];
#pragma unroll
        for (int j = 0; j < U; j++) {
            const f32x4_t w = *reinterpret_cast<const f32x4_t*>(&wts[s + j][4 * g]);
            A0 += w * h4(ga[j][0], ga[j][1]);
            A1 += w * h4(ga[j][2], ga[j][3]);
        }
    }
    for (; s < nact; s++) {
        const f32x4_t w0 = *reinterpret_cast<const f32x4_t*>(&wts[s][4 * g]);
        const u32x4_t v = src[s * frag_st];
        A0 += w0 * h4(v[0], v[1]);
        A1 += w0 * h4(v[2], v[3]);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int orow = qb * 16 + 4 * g + i;
        if (orow < p.R) {
            const float inv = linv[4 * g + i];
            const int64_t base = ((int64_t)b * p.R + orow) * kKR + 16 * d0 + n;
            store_out<OUT_DT>(p.out, base, A0[i] * inv);
            store_out<OUT_DT>(p.out, base + 16, A1[i] * inv);
        }
    }
    MUGEN_TRACE(10);
}

// ------------------------------------------------------------------ launch

// kernel 1: mla_decode_kernel ("rows", 16-bit q with at most 64 rows);
// kernel 2: mla_decode_ws_kernel (warp-specialised, every other case).
// Both take 64 query rows per workgroup and 32-token tiles.
int mla_rows_per_block(int) { return 64; }
int mla_tile_tokens(int) { return kTT; }

template <int QDT, int DT, int OUT_DT>
static hipError_t launch_mla_t(const MlaParams& p, int kernel, hipStream_t st, KernelTimer* t) {
    const int grid = 8 * ((p.units + 7) / 8);  // see mla_map
    hipError_t e = kernel == 1
                       ? launch_k(t, "mla_decode", mla_decode_kernel<QDT, DT>, dim3(grid), dim3(256), st, p)
                       : launch_k(t, "mla_decode", mla_decode_ws_kernel<QDT, DT>, dim3(grid), dim3(512), st, p);
    if (e != hipSuccess) return e;
    // tiny merges (V2-Lite decode: one 16-row block of one sequence) spread
    // over more, smaller workgroups: 2 waves of 2 column blocks each (10.8 ->
    // 10.3-10.6 us per V2-Lite step); larger grids keep 4 waves (a 512-token
    // prompt measured 9% slower with 2)
    if (p.nq * p.B <= 4)
        return launch_k(t, "mla_decode_combine", mla_decode_combine_kernel<OUT_DT, 2>, dim3(p.nq, 8, p.B), dim3(128),
                        st, p);
    return launch_k(t, "mla_decode_combine", mla_decode_combine_kernel<OUT_DT, 4>, dim3(p.nq, 4, p.B), dim3(256),
                    st, p);
}

template <int QDT, int DT>
static hipError_t launch_mla_o(const MlaParams& p, int kernel, int out_dt, hipStream_t st, KernelTimer* t) {
    if (out_dt == DT_F32) return launch_mla_t<QDT, DT, DT_F32>(p, kernel, st, t);
    if (out_dt == DT_F16) return launch_mla_t<QDT, DT, DT_F16>(p, kernel, st, t);
    return launch_mla_t<QDT, DT, DT_BF16>(p, kernel, st, t);
}

template <int DT>
static hipError_t launch_mla_q(const MlaParams& p, int kernel, int q_dt, int out_dt, hipStream_t st,
                               KernelTimer* t) {
    if (q_dt == DT_F32) return launch_mla_o<DT_F32, DT>(p, kernel, out_dt, st, t);
    return launch_mla_o<DT, DT>(p, kernel, out_dt, st, t);
}

hipError_t launch_mla_decode(const MlaParams& p, int kernel, int q_dt, int lat_dt, int out_dt,
                             hipStream_t st, KernelTimer* t) {
    if (lat_dt == DT_F16) return launch_mla_q<DT_F16>(p, kernel, q_dt, out_dt, st, t);
    return launch_mla_q<DT_BF16>(p, kernel, q_dt, out_dt, st, t);
}

}  // namespace mugen_attn
