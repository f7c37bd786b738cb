// mla_proj.hip -- the MLA absorption and up-projection around the latent
// core: q_abs = q_nope . k_b (transformer.cpp:2563-2573) and out = o . v_b^T
// (transformer.cpp:2610-2620), with the weights dequantised on the fly from
// the reference's GGUF block encodings (dequant_weight_row,
// transformer.cpp:2488-2534: F16, Q8_0, Q4_0).
//
// At decode sizes (rows = batch * q_len, a few to a few tens) both are
// skinny per-head GEMMs bound by the weight stream (16.8 MB per matrix per
// layer in F16 at DeepSeek-V3 shape, 8.9 MB Q8_0, 4.7 MB Q4_0).  Streaming
// it at HBM rate needs most of the matrix in flight at once, so every lane
// issues all of its weight loads before any arithmetic, keeps its slice of
// the weights in registers, and loops over the rows against them (each
// weight byte is read once for any number of rows).  Arithmetic is fp32 on
// the VALU, as the reference's:
//  * absorb: workgroup = (head, 256-column half of kv_rank), 8 waves; wave w
//    holds nope rows 16w..16w+15, lane 4 consecutive columns; per 8-row
//    chunk of q each lane sums its 16 rows, and the 8 waves' partials are
//    added in LDS in a fixed order;
//  * project: workgroup = (head, 32 output rows j), 4 waves of 8 rows j;
//    lane = 8 consecutive kv_rank dims, so a wave's load of one weight row is
//    one coalesced row; per 4 rows of o a lane forms 32 (row, j) partials
//    over its 8 dims and a halving butterfly over the 64 lanes (32 + 1
//    shuffles for the 32 sums) leaves each lane pair with one total.
#include "common.h"
#include "kernels.h"
#include "mla_latent.h"

namespace mugen_attn {

// rows (batch * q_len) from which absorb / project run on MFMA
constexpr int kProjMfmaRows = 64;

namespace {

template <int WT>
__host__ __device__ constexpr int wrow_bytes(int K) {
    return WT == W_F16 ? 2 * K : (WT == W_Q8_0 ? K / 32 * 34 : K / 32 * 18);
}

__device__ __forceinline__ float half_bits(uint32_t b) {
    return to_f32<DT_F16>(uint16_t(b & 0xffffu));
}

// Raw bits of N consecutive weights d0 .. d0+N-1 of one row (N = 4 or 8,
// d0 a multiple of N), loaded with as few instructions as the encoding's
// alignment allows; dequant() turns them into floats (dequant_weight_row).
template <int WT, int N>
struct WRaw {
    uint32_t v[N / 2];  // F16: N halfs; Q8_0: N int8; Q4_0: N bytes whose low/high nibble is used
    uint32_t s;         // block scale bits (unused for F16)
};

template <int WT, int N>
__device__ __forceinline__ WRaw<WT, N> wload(const uint8_t* row, int d0) {
    WRaw<WT, N> r{};
    if constexpr (WT == W_F16) {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(row + 2 * d0);  // 2N-byte aligned
#pragma unroll
        for (int e = 0; e < N / 2; e++) r.v[e] = p[e];
    } else {
        constexpr int BB = WT == W_Q8_0 ? 34 : 18;
        const uint8_t* blk = row + (d0 >> 5) * BB;
        const int off = WT == W_Q8_0 ? (d0 & 31) : (d0 & 15);  // byte offset of the first quant
        const uint16_t* p = reinterpret_cast<const uint16_t*>(blk + 2 + off);  // even: 2-byte loads
        r.s = *reinterpret_cast<const uint16_t*>(blk);
#pragma unroll
        for (int e = 0; e < N / 2; e++) r.v[e] = p[e];
    }
    return r;
}

template <int WT, int N>
__device__ __forceinline__ void dequant(const WRaw<WT, N>& r, int d0, float* w) {
    if constexpr (WT == W_F16) {
#pragma unroll
        for (int e = 0; e < N / 2; e++) {
            w[2 * e] = lo_f32<DT_F16>(r.v[e]);
            w[2 * e + 1] = hi_f32<DT_F16>(r.v[e]);
        }
    } else if constexpr (WT == W_Q8_0) {
        const float sc = half_bits(r.s);
#pragma unroll
        for (int e = 0; e < N / 2; e++) {
            w[2 * e] = sc * (float)(int8_t)(r.v[e] & 0xff);
            w[2 * e + 1] = sc * (float)(int8_t)((r.v[e] >> 8) & 0xff);
        }
    } else {
        const float sc = half_bits(r.s);
        const int sh = (d0 & 16) ? 4 : 0;  // elements 16..31 of a block: high nibbles
#pragma unroll
        for (int e = 0; e < N / 2; e++) {
            w[2 * e] = (float)((int)((r.v[e] >> sh) & 15) - 8) * sc;
            w[2 * e + 1] = (float)((int)((r.v[e] >> (8 + sh)) & 15) - 8) * sc;
        }
    }
}

// one butterfly step over lane bit M: the lane keeps half of its M/2 live
// values (the upper half if its bit M is set) plus its partner's copy of it.
// M = 32 / 16: one v_permlane32_swap / v_permlane16_swap per pair moves both
// halves at once (swapping x[t + N] of the lower lanes with x[t] of the
// upper ones leaves each lane its kept value and its partner's given one,
// whose sum is the step's result); smaller M: DPP.
template <int M>
__device__ __forceinline__ void halve(float* x, int lane) {
    constexpr int N = M / 2;
    if constexpr (M >= 16) {
#pragma unroll
        for (int t = 0; t < N; t++) {
            const auto r = M == 32 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(x[t]), __float_as_uint(x[t + N]),
                                                                     false, false)
                                   : __builtin_amdgcn_permlane16_swap(__float_as_uint(x[t]), __float_as_uint(x[t + N]),
                                                                     false, false);
            x[t] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
        }
    } else {
        const bool up = (lane & M) != 0;
#pragma unroll
        for (int t = 0; t < N; t++) {
            const float keep = up ? x[t + N] : x[t];
            const float give = up ? x[t] : x[t + N];
            x[t] = keep + dpp_xor<M>(give);
        }
    }
}

}  // namespace

// one absorb workgroup (512 threads): head h, 256-column half `half`
template <int WT, int OUT_DT>
__device__ __forceinline__ void absorb_block(const MlaProjParams& p, int h, int half) {
    constexpr int NOPE = 128, ROPE = 64, KR = 512, RC = 8, IPW = 16;  // rows per chunk, nope rows per wave
    __shared__ __attribute__((aligned(16))) float qs[RC][NOPE];
    __shared__ __attribute__((aligned(16))) f32x4_t red[8][RC][64];  // [wave][row][lane] partials
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    MUGEN_TRACE(6);
    const int d0 = half * 256 + 4 * lane;
    constexpr int RB = wrow_bytes<WT>(KR);
    const uint8_t* wrow = static_cast<const uint8_t*>(p.w) + ((size_t)h * NOPE + w * IPW) * RB;
    // a chunk's q (nope and rope parts), loaded ahead of use: the first
    // chunk's loads go out before the weights', so that staging them (and
    // the barrier after it) waits for q only -- loads return in order
    const uint16_t* q = static_cast<const uint16_t*>(p.in);
    constexpr int QPT = RC * NOPE / 512;  // nope values per thread per chunk
    uint16_t qn[QPT], qr0 = 0, qr1 = 0;
    auto q_load = [&](int r0, int nr) {
#pragma unroll
        for (int u = 0; u < QPT; u++) {
            const int k = tid + 512 * u, r = k / NOPE, i = k % NOPE;
            qn[u] = r < nr ? q[((int64_t)(r0 + r) * p.H + h) * (NOPE + ROPE) + i] : uint16_t(0x3c00);  // 1.0
        }
        if (half == 0 && tid < RC * ROPE / 2) {
            const int r = tid / (ROPE / 2), c = tid % (ROPE / 2);
            if (r < nr) {
                const uint16_t* qr = q + ((int64_t)(r0 + r) * p.H + h) * (NOPE + ROPE) + NOPE;
                qr0 = qr[c];
                qr1 = qr[c + ROPE / 2];
            }
        }
    };
    q_load(0, min(RC, p.rows));
    WRaw<WT, 4> raw[IPW];
#pragma unroll
    for (int k = 0; k < IPW; k++) raw[k] = wload<WT, 4>(wrow + (size_t)k * RB, d0);
    for (int r0 = 0; r0 < p.rows; r0 += RC) {
        const int nr = min(RC, p.rows - r0);
        if (r0 > 0) q_load(r0, nr);
        bool zero = false;  // a zero q term in a real row of the chunk
#pragma unroll
        for (int u = 0; u < QPT; u++) {
            const int k = tid + 512 * u, r = k / NOPE, i = k % NOPE;
            const float v = to_f32<DT_F16>(qn[u]);
            zero |= v == 0.f;
            qs[r][i] = r < nr ? v : 0.f;
        }
        if (half == 0 && tid < RC * ROPE / 2) {
            // q_rope appended: as is, or with the reference's q RoPE stage
            // (NeoX pairs c, c + 32, f16 results; transformer.cpp:3882-3921)
            const int r = tid / (ROPE / 2), c = tid % (ROPE / 2);
            if (r < nr) {
                uint16_t y0 = qr0, y1 = qr1;
                if (p.positions || p.seq_base)
                    rope_pair_f16(to_f32<DT_F16>(y0), to_f32<DT_F16>(y1),
                                  row_position(p.positions, p.seq_base, p.rows_per_seq, r0 + r), p.freqs.f[c], y0, y1);
                const int64_t o = ((int64_t)(r0 + r) * p.H + h) * (KR + ROPE) + KR + c;
                store_out<OUT_DT>(p.out, o, to_f32<DT_F16>(y0));
                store_out<OUT_DT>(p.out, o + ROPE / 2, to_f32<DT_F16>(y1));
            }
        }
        // The reference skips q == 0 terms; that differs from adding 0 * w
        // only for a non-finite weight, so chunks without a zero q take the
        // plain fma path.
        const bool skip_zero = __syncthreads_or(zero);
        f32x4_t acc[RC];
        auto accumulate = [&](auto skip_tag) {
            constexpr bool SKIP = decltype(skip_tag)::value;
#pragma unroll
            for (int r = 0; r < RC; r++) acc[r] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k4 = 0; k4 < IPW; k4 += 4) {
                float wv[4][4];
#pragma unroll
                for (int k = 0; k < 4; k++) dequant<WT, 4>(raw[k4 + k], d0, wv[k]);
#pragma unroll
                for (int r = 0; r < RC; r++) {
                    const f32x4_t qv = *reinterpret_cast<const f32x4_t*>(&qs[r][w * IPW + k4]);
#pragma unroll
                    for (int k = 0; k < 4; k++) {
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            const float t = fmaf(qv[k], wv[k][e], acc[r][e]);
                            acc[r][e] = (SKIP && qv[k] == 0.f) ? acc[r][e] : t;
                        }
                    }
                }
            }
        };
        MUGEN_TRACE(7);
        if (skip_zero) accumulate(std::true_type{});
        else accumulate(std::false_type{});
        MUGEN_TRACE(8);
#pragma unroll
        for (int r = 0; r < RC; r++) red[w][r][lane] = acc[r];
        __syncthreads();
        {   // thread (row r, lane l) adds the 8 waves' partials in wave order
            const int r = tid >> 6, l = tid & 63;
            f32x4_t t = red[0][r][l];
#pragma unroll
            for (int ww = 1; ww < 8; ww++) t += red[ww][r][l];
            if (r < nr) {
                const int64_t o = ((int64_t)(r0 + r) * p.H + h) * (KR + ROPE) + half * 256 + 4 * l;
                if constexpr (OUT_DT == DT_F32) {
                    *reinterpret_cast<f32x4_t*>(static_cast<float*>(p.out) + o) = t;  // 16-byte aligned
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++) store_out<OUT_DT>(p.out, o + e, t[e]);
                }
            }
        }
        __syncthreads();  // qs / red are rewritten by the next chunk
    }
    MUGEN_TRACE(9);
}

template <int WT, int OUT_DT>
__global__ __launch_bounds__(512) void mla_absorb_kernel(MlaProjParams p) {
    absorb_block<WT, OUT_DT>(p, blockIdx.x, blockIdx.y);
}

// One launch for the two independent stages before the latent core at decode
// sizes: workgroups [0, 2H) absorb (head, column half), the rest write the
// new tokens' latent rows, one wave per token.  Saves the writer's own launch
// (the layer step's kernels run back to back).
template <int WT, int OUT_DT, int LDT>
__global__ __launch_bounds__(512) void mla_prepare_kernel(MlaProjParams pa, LatentWriteParams pl) {
    const int nab = 2 * pa.H;
    if ((int)blockIdx.x < nab) {
        absorb_block<WT, OUT_DT>(pa, blockIdx.x % pa.H, blockIdx.x / pa.H);
        return;
    }
    const int r = ((int)blockIdx.x - nab) * 8 + (int)(threadIdx.x >> 6);
    if (r < pl.rows) latent_write_row<LDT>(pl, r, threadIdx.x & 63);
}

template <int WT, int OUT_DT>
__global__ __launch_bounds__(256) void mla_project_kernel(MlaProjParams p) {
    constexpr int KR = 512, VH = 128, RC = 16, JW = 8;  // o rows staged per pass, output rows per wave
    __shared__ __attribute__((aligned(16))) float os[RC][KR];
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    MUGEN_TRACE(10);
    const int j0 = blockIdx.y * 32 + JW * w;
    const int d0 = 8 * lane;
    constexpr int RB = wrow_bytes<WT>(KR);
    const uint8_t* wrow = static_cast<const uint8_t*>(p.w) + ((size_t)h * VH + j0) * RB;
    WRaw<WT, 8> raw[JW];
#pragma unroll
    for (int j = 0; j < JW; j++) raw[j] = wload<WT, 8>(wrow + (size_t)j * RB, d0);
    // the first pass's o rows requested with the weights (two round trips
    // in flight together instead of one after the other)
    const float* o = static_cast<const float*>(p.in);
    constexpr int OPT = RC * KR / 4 / 256;  // 16-byte o loads per thread per pass
    auto o_load = [&](int r0, int nr, f32x4_t* dst) {
#pragma unroll
        for (int i = 0; i < OPT; i++) {
            const int k = tid + 256 * i, r = k / (KR / 4), c4 = k % (KR / 4);
            dst[i] = r < nr ? *reinterpret_cast<const f32x4_t*>(o + ((int64_t)(r0 + r) * p.H + h) * KR + 4 * c4)
                            : f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
    };
    f32x4_t ov[OPT];
    o_load(0, min(RC, p.rows), ov);
    float wv[JW][8];
#pragma unroll
    for (int j = 0; j < JW; j++) dequant<WT, 8>(raw[j], d0, wv[j]);
    MUGEN_TRACE(11);
    // after the butterfly, lane pair (2v, 2v+1) holds sum v = 8 * row + j
    const int v = lane >> 1;
    for (int r0 = 0; r0 < p.rows; r0 += RC) {
        const int nr = min(RC, p.rows - r0);
        if (r0 > 0) o_load(r0, nr, ov);
        __syncthreads();
#pragma unroll
        for (int i = 0; i < OPT; i++) {
            const int k = tid + 256 * i, r = k / (KR / 4), c4 = k % (KR / 4);
            *reinterpret_cast<f32x4_t*>(&os[r][4 * c4]) = ov[i];
        }
        __syncthreads();
        MUGEN_TRACE(12);
        for (int rs = 0; rs < nr; rs += 4) {
            float x[32];  // x[8 * r + j]: rows rs..rs+3 x this wave's 8 output rows, over this lane's 8 dims
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const f32x4_t a = *reinterpret_cast<const f32x4_t*>(&os[rs + r][d0]);
                const f32x4_t b = *reinterpret_cast<const f32x4_t*>(&os[rs + r][d0 + 4]);
#pragma unroll
                for (int j = 0; j < JW; j++) {
                    float t = a[0] * wv[j][0];
                    t = fmaf(a[1], wv[j][1], t);
                    t = fmaf(a[2], wv[j][2], t);
                    t = fmaf(a[3], wv[j][3], t);
                    t = fmaf(b[0], wv[j][4], t);
                    t = fmaf(b[1], wv[j][5], t);
                    t = fmaf(b[2], wv[j][6], t);
                    t = fmaf(b[3], wv[j][7], t);
                    x[8 * r + j] = t;
                }
            }
            // halving butterfly: at lane bit m (32 .. 2) a lane keeps the half
            // of its values selected by that bit and adds its partner's copy
            halve<32>(x, lane);
            halve<16>(x, lane);
            halve<8>(x, lane);
            halve<4>(x, lane);
            halve<2>(x, lane);
            const float tot = x[0] + dpp_xor<1>(x[0]);
            const int r = v >> 3, j = v & 7;
            if ((lane & 1) == 0 && rs + r < nr)
                store_out<OUT_DT>(p.out, ((int64_t)(r0 + rs + r) * p.H + h) * VH + j0 + j, tot);
        }
    }
    MUGEN_TRACE(13);
}

// ---------------------------------------------------------------- MFMA forms
//
// At prompt sizes (rows = q_len * batch of 64 and more) the products are
// real GEMMs (per head: rows x 128 x 512) and the weight stream is no longer
// the bound; they run on bf16 MFMA with fp32-level accuracy:
//  * each fp32 (or f16) operand value x is split into bf16 hi = rne(x) and
//    lo = rne(x - hi) (16 significant bits; an f16 value splits exactly),
//    and every product is formed as hi.hi + hi.lo + lo.hi with fp32
//    accumulation -- the dropped lo.lo term and the rounding of lo leave a
//    relative error of ~2^-16 per product;
//  * the reference skips zero q terms (transformer.cpp:2567); that differs
//    from adding 0 * w only for a non-finite weight, which a GGUF attn_k_b /
//    attn_v_b does not hold.
// Row counts below kProjMfmaRows keep the weight-streaming VALU kernels
// above.

// absorb: workgroup = (head, 128-column quarter of kv_rank, row group);
// the quarter's weights (128 nope rows x 128 columns) are dequantised once
// into LDS as bf16 hi / lo planes, rows XOR-swizzled in 16-byte chunks so
// the transpose reads (ds_read_b64_tr_b16) that form the A operand
// W^T[column][nope] are conflict-free.  Q^T_abs = W^T . q^T: wave w owns
// columns 32w .. 32w+31 of the quarter and 64 rows at a time; q (f16) is
// the B operand straight from global memory (8 consecutive nope dims per
// lane).  Lane (g, n) ends with 4 consecutive columns of row n: one 16-byte
// store.
// one absorb workgroup (256 threads): head h, column quarter cq, row groups
// z, z + nz, ..
template <int WT, int OUT_DT>
__device__ __forceinline__ void absorb_mfma_block(const MlaProjParams& p, int h, int cq, int z, int nz) {
    constexpr int NOPE = 128, ROPE = 64, KR = 512, CQ = 128, RB = CQ * 2;  // LDS row bytes per plane
    constexpr int WRB = wrow_bytes<WT>(KR);
    __shared__ __attribute__((aligned(16))) char wl[2][NOPE * RB];  // [hi|lo][nope row][128 columns]
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    auto swz = [](int r) { return ((r & 1) * 2) ^ (((r >> 1) & 1) * 4) ^ (((r >> 3) & 1) * 8) ^ ((r >> 4) & 1); };
    MUGEN_TRACE(0);
    const uint16_t* q = static_cast<const uint16_t*>(p.in);
    // q of row block rb, k-step kk: lane (g, n) holds q[row n][32kk + 8g .. +7]
    u32x4_t qraw[4][NOPE / 32];
    auto load_q = [&](int r0) {
#pragma unroll
        for (int rb = 0; rb < 4; rb++) {
            const int r = min(r0 + 16 * rb + n, p.rows - 1);
#pragma unroll
            for (int kk = 0; kk < NOPE / 32; kk++)
                qraw[rb][kk] = load16(q + ((int64_t)r * p.H + h) * (NOPE + ROPE) + 32 * kk + 8 * g);
        }
    };
    load_q(z * 64);  // in flight during the dequantisation
    {   // dequantise the quarter: 128 rows x 16 chunks of 8 columns, all
        // of a thread's loads issued before any conversion
        const uint8_t* wh = static_cast<const uint8_t*>(p.w) + (size_t)h * NOPE * WRB;
        constexpr int JOBS = NOPE * 16 / 256;
        WRaw<WT, 8> raw[JOBS];
#pragma unroll
        for (int i = 0; i < JOBS; i++) {
            const int job = tid + 256 * i, k = job >> 4, c8 = job & 15;
            raw[i] = wload<WT, 8>(wh + (size_t)k * WRB, cq * CQ + 8 * c8);
        }
#pragma unroll
        for (int i = 0; i < JOBS; i++) {
            const int job = tid + 256 * i, k = job >> 4, c8 = job & 15;
            float x[8];
            dequant<WT, 8>(raw[i], cq * CQ + 8 * c8, x);
            u32x4_t fr[2];
            split_p<DT_BF16, 2>(x, fr);
            const int off = k * RB + ((c8 ^ swz(k)) * 16);
            *reinterpret_cast<u32x4_t*>(&wl[0][off]) = fr[0];
            *reinterpret_cast<u32x4_t*>(&wl[1][off]) = fr[1];
        }
    }
    // transpose-read offsets: lane (g, n) reads rows 8g + n/4 (+4) of a
    // k-step, column chunk 2cb + (n%4)/2 of its wave's 32 columns
    const int tr = 8 * g + (n >> 2);
    uint32_t t_off[2];
#pragma unroll
    for (int cb = 0; cb < 2; cb++)
        t_off[cb] = tr * RB + (((4 * w + 2 * cb + ((n & 3) >> 1)) ^ swz(tr)) * 16) + 8 * (n & 1);
    MUGEN_TRACE(1);
    __syncthreads();
    MUGEN_TRACE(2);
    for (int r0 = z * 64; r0 < p.rows; r0 += nz * 64) {
        if (r0 != z * 64) load_q(r0);
        {   // q_rope appended: as is, or rotated by the reference's q RoPE
            // stage (NeoX pairs c, c + 32, f16 results); the 4 quarter
            // workgroups of a row group take 16 of its rows each
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int job = tid + 256 * i;
                const int r = r0 + 16 * cq + (job >> 5), c = job & 31;
                if (r < p.rows) {
                    const uint16_t* qr = q + ((int64_t)r * p.H + h) * (NOPE + ROPE) + NOPE;
                    uint16_t y0 = qr[c], y1 = qr[c + ROPE / 2];
                    if (p.positions || p.seq_base)
                        rope_pair_f16(to_f32<DT_F16>(y0), to_f32<DT_F16>(y1),
                                      row_position(p.positions, p.seq_base, p.rows_per_seq, r), p.freqs.f[c], y0, y1);
                    const int64_t o = ((int64_t)r * p.H + h) * (KR + ROPE) + KR + c;
                    store_out<OUT_DT>(p.out, o, to_f32<DT_F16>(y0));
                    store_out<OUT_DT>(p.out, o + ROPE / 2, to_f32<DT_F16>(y1));
                }
            }
        }
        MUGEN_TRACE(3);
        f32x4_t acc[2][4];
#pragma unroll
        for (int cb = 0; cb < 2; cb++)
#pragma unroll
            for (int rb = 0; rb < 4; rb++) acc[cb][rb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < NOPE / 32; kk++) {
            u32x4_t qf[4][2];  // row block rb: q[row n][32kk + 8g .. +7] as bf16 hi / lo
#pragma unroll
            for (int rb = 0; rb < 4; rb++) {
                const u32x4_t v = qraw[rb][kk];
                float x[8];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    x[2 * e] = lo_f32<DT_F16>(v[e]);
                    x[2 * e + 1] = hi_f32<DT_F16>(v[e]);
                }
                split_p<DT_BF16, 2>(x, qf[rb]);
            }
#pragma unroll
            for (int cb = 0; cb < 2; cb++) {
                u32x4_t wf[2];
#pragma unroll
                for (int pl = 0; pl < 2; pl++) {
                    const char* base = &wl[pl][32 * kk * RB + t_off[cb]];
                    const u32x2_t lo = lds_read_tr16(reinterpret_cast<const uint16_t*>(base));
                    const u32x2_t hi = lds_read_tr16(reinterpret_cast<const uint16_t*>(base + 4 * RB));
                    wf[pl] = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
                }
#pragma unroll
                for (int rb = 0; rb < 4; rb++) {
                    acc[cb][rb] = mfma16x16x32<DT_BF16>(wf[0], qf[rb][0], acc[cb][rb]);
                    acc[cb][rb] = mfma16x16x32<DT_BF16>(wf[0], qf[rb][1], acc[cb][rb]);
                    acc[cb][rb] = mfma16x16x32<DT_BF16>(wf[1], qf[rb][0], acc[cb][rb]);
                }
            }
        }
        MUGEN_TRACE(4);
        // lane (g, n): columns 32w + 16cb + 4g .. +3 of row r0 + 16rb + n
#pragma unroll
        for (int rb = 0; rb < 4; rb++) {
            const int r = r0 + 16 * rb + n;
            if (r >= p.rows) continue;
#pragma unroll
            for (int cb = 0; cb < 2; cb++) {
                const int64_t o = ((int64_t)r * p.H + h) * (KR + ROPE) + cq * CQ + 32 * w + 16 * cb + 4 * g;
                if constexpr (OUT_DT == DT_F32) {
                    *reinterpret_cast<f32x4_t*>(static_cast<float*>(p.out) + o) = acc[cb][rb];
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++) store_out<OUT_DT>(p.out, o + e, acc[cb][rb][e]);
                }
            }
        }
    }
    MUGEN_TRACE(5);
}

template <int WT, int OUT_DT>
__global__ __launch_bounds__(256) void mla_absorb_mfma_kernel(MlaProjParams p) {
    absorb_mfma_block<WT, OUT_DT>(p, blockIdx.x, blockIdx.y, blockIdx.z, gridDim.z);
}

// One launch for the latent write and the absorption at prompt sizes: the
// first H * 4 * nz workgroups absorb (the order of mla_absorb_mfma_kernel's
// grid: head fastest, then column quarter, then row group), the rest write
// the new tokens' latent rows, one wave per token, beside them on the CUs
// (no LDS of their own)
template <int WT, int OUT_DT, int LDT>
__global__ __launch_bounds__(256) void mla_prepare_mfma_kernel(MlaProjParams pa, LatentWriteParams pl, int nz) {
    const int nab = pa.H * 4 * nz;
    const int bx = (int)blockIdx.x;
    if (bx < nab) {
        absorb_mfma_block<WT, OUT_DT>(pa, bx % pa.H, (bx / pa.H) % 4, bx / (pa.H * 4), nz);
        return;
    }
    const int r = (bx - nab) * 4 + (int)(threadIdx.x >> 6);
    if (r < pl.rows) latent_write_row<LDT>(pl, r, threadIdx.x & 63);
}

// project: workgroup = (head, half of the 128 output rows j, row group);
// out^T = W_v . o^T.  The half's weights (64 rows j x 512 kv_rank) are
// dequantised once into LDS as bf16 hi / lo planes (16-byte chunk c of row
// j at chunk c ^ (j % 16): the 16 rows a phase of ds_read_b128 touches
// land on distinct banks) and read as the A operand, 8 consecutive kv_rank
// dims of a row j per lane.  o (fp32) is the B operand straight from
// global memory, split into bf16 hi / lo, loaded kPf k-steps ahead.  Wave
// w owns 16 rows of o and the half's 4 j blocks; lane (g, n) ends with
// j .. j+3 of row n: one 8-byte (f16) or 16-byte (fp32) store.
template <int WT, int OUT_DT>
__global__ __launch_bounds__(256) void mla_project_mfma_kernel(MlaProjParams p) {
    constexpr int KR = 512, VH = 128, JH = 64, JB = JH / 16, RB = KR * 2, kPf = 4, KS = KR / 32;
    constexpr int WRB = wrow_bytes<WT>(KR);
    __shared__ __attribute__((aligned(16))) char wl[2][JH * RB];  // [hi|lo][j][512]
    const int h = blockIdx.x, jh = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const float* o = static_cast<const float*>(p.in);
    f32x4_t ob[kPf][2];  // o[row n][32kk + 8g .. +7] of the next kPf k-steps
    auto load_o = [&](int r0, int kk, f32x4_t (&dst)[2]) {
        const int r = min(r0 + 16 * w + n, p.rows - 1);
        const float* src = o + ((int64_t)r * p.H + h) * KR + 32 * kk + 8 * g;
        dst[0] = *reinterpret_cast<const f32x4_t*>(src);
        dst[1] = *reinterpret_cast<const f32x4_t*>(src + 4);
    };
#pragma unroll
    for (int i = 0; i < kPf; i++) load_o(blockIdx.z * 64, i, ob[i]);
    {   // dequantise the half: 64 rows x 64 chunks of 8 dims, 16 per
        // thread, every load issued before any conversion
        const uint8_t* wh = static_cast<const uint8_t*>(p.w) + ((size_t)h * VH + jh * JH) * WRB;
        constexpr int JOBS = 16;
#pragma unroll 1
        for (int j0 = 0; j0 < JH * 64; j0 += 256 * JOBS) {
            WRaw<WT, 8> raw[JOBS];
#pragma unroll
            for (int i = 0; i < JOBS; i++) {
                const int job = j0 + tid + 256 * i, j = job >> 6, c = job & 63;
                raw[i] = wload<WT, 8>(wh + (size_t)j * WRB, 8 * c);
            }
#pragma unroll
            for (int i = 0; i < JOBS; i++) {
                const int job = j0 + tid + 256 * i, j = job >> 6, c = job & 63;
                float x[8];
                dequant<WT, 8>(raw[i], 8 * c, x);
                u32x4_t fr[2];
                split_p<DT_BF16, 2>(x, fr);
                const int off = j * RB + ((c ^ (j & 15)) * 16);
                *reinterpret_cast<u32x4_t*>(&wl[0][off]) = fr[0];
                *reinterpret_cast<u32x4_t*>(&wl[1][off]) = fr[1];
            }
        }
    }
    __syncthreads();
    for (int r0 = blockIdx.z * 64; r0 < p.rows; r0 += gridDim.z * 64) {
        if (r0 != blockIdx.z * 64) {
#pragma unroll
            for (int i = 0; i < kPf; i++) load_o(r0, i, ob[i]);
        }
        f32x4_t acc[JB];
#pragma unroll
        for (int jb = 0; jb < JB; jb++) acc[jb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
        for (int k0 = 0; k0 < KS; k0 += kPf) {
#pragma unroll
            for (int i = 0; i < kPf; i++) {
                const int kk = k0 + i;
                const f32x4_t a = ob[i][0], b = ob[i][1];
                if (kk + kPf < KS) load_o(r0, kk + kPf, ob[i]);
                const float x[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
                u32x4_t of[2];
                split_p<DT_BF16, 2>(x, of);
#pragma unroll
                for (int jb = 0; jb < JB; jb++) {
                    const int j = 16 * jb + n;
                    const int off = j * RB + (((4 * kk + g) ^ n) * 16);
                    const u32x4_t whi = *reinterpret_cast<const u32x4_t*>(&wl[0][off]);
                    const u32x4_t wlo = *reinterpret_cast<const u32x4_t*>(&wl[1][off]);
                    acc[jb] = mfma16x16x32<DT_BF16>(whi, of[0], acc[jb]);
                    acc[jb] = mfma16x16x32<DT_BF16>(whi, of[1], acc[jb]);
                    acc[jb] = mfma16x16x32<DT_BF16>(wlo, of[0], acc[jb]);
                }
            }
        }
        const int r = r0 + 16 * w + n;
        if (r < p.rows) {
#pragma unroll
            for (int jb = 0; jb < JB; jb++) {
                const int64_t oo = ((int64_t)r * p.H + h) * VH + jh * JH + 16 * jb + 4 * g;
                if constexpr (OUT_DT == DT_F32) {
                    *reinterpret_cast<f32x4_t*>(static_cast<float*>(p.out) + oo) = acc[jb];
                } else {
                    const uint32_t lo = pack2<OUT_DT>(acc[jb][0], acc[jb][1]);
                    const uint32_t hi = pack2<OUT_DT>(acc[jb][2], acc[jb][3]);
                    *reinterpret_cast<u32x2_t*>(static_cast<uint16_t*>(p.out) + oo) = u32x2_t{lo, hi};
                }
            }
        }
    }
}

// absorb MFMA form: row groups of 64, enough workgroups for ~two per CU,
// each group of a workgroup reusing its dequantised quarter
static int absorb_mfma_groups(const MlaProjParams& p) {
    const int groups = (p.rows + 63) / 64;
    const int per = std::max(1, 512 / (p.H * 4));
    return std::min(groups, per);
}

template <int WT>
static hipError_t launch_absorb_w(const MlaProjParams& p, int out_dt, hipStream_t st, KernelTimer* t) {
    if (p.rows >= kProjMfmaRows) {
        const dim3 grid(p.H, 4, absorb_mfma_groups(p));
        if (out_dt == DT_BF16)
            return launch_k(t, "mla_absorb", mla_absorb_mfma_kernel<WT, DT_BF16>, grid, dim3(256), st, p);
        return launch_k(t, "mla_absorb", mla_absorb_mfma_kernel<WT, DT_F32>, grid, dim3(256), st, p);
    }
    const dim3 grid(p.H, 512 / 256);
    if (out_dt == DT_BF16) return launch_k(t, "mla_absorb", mla_absorb_kernel<WT, DT_BF16>, grid, dim3(512), st, p);
    return launch_k(t, "mla_absorb", mla_absorb_kernel<WT, DT_F32>, grid, dim3(512), st, p);
}

hipError_t launch_mla_absorb(const MlaProjParams& p, int w_type, int out_dt, hipStream_t st, KernelTimer* t) {
    return w_type == W_F16 ? launch_absorb_w<W_F16>(p, out_dt, st, t)
         : w_type == W_Q8_0 ? launch_absorb_w<W_Q8_0>(p, out_dt, st, t)
                            : launch_absorb_w<W_Q4_0>(p, out_dt, st, t);
}

template <int WT, int OUT_DT>
static hipError_t launch_prepare_o(const MlaProjParams& pa, const LatentWriteParams& pl, int lat_dt, hipStream_t st,
                                   KernelTimer* t) {
    const dim3 grid(2 * pa.H + (pl.rows + 7) / 8);
    if (lat_dt == DT_BF16)
        return launch_k(t, "mla_prepare", mla_prepare_kernel<WT, OUT_DT, DT_BF16>, grid, dim3(512), st, pa, pl);
    return launch_k(t, "mla_prepare", mla_prepare_kernel<WT, OUT_DT, DT_F16>, grid, dim3(512), st, pa, pl);
}

template <int WT>
static hipError_t launch_prepare_w(const MlaProjParams& pa, const LatentWriteParams& pl, int out_dt, int lat_dt,
                                   hipStream_t st, KernelTimer* t) {
    if (out_dt == DT_BF16) return launch_prepare_o<WT, DT_BF16>(pa, pl, lat_dt, st, t);
    return launch_prepare_o<WT, DT_F32>(pa, pl, lat_dt, st, t);
}

template <int WT, int OUT_DT>
static hipError_t launch_prepare_mfma_o(const MlaProjParams& pa, const LatentWriteParams& pl, int lat_dt,
                                        hipStream_t st, KernelTimer* t) {
    const int nz = absorb_mfma_groups(pa);
    const dim3 grid(pa.H * 4 * nz + (pl.rows + 3) / 4);
    if (lat_dt == DT_BF16)
        return launch_k(t, "mla_prepare", mla_prepare_mfma_kernel<WT, OUT_DT, DT_BF16>, grid, dim3(256), st, pa, pl, nz);
    return launch_k(t, "mla_prepare", mla_prepare_mfma_kernel<WT, OUT_DT, DT_F16>, grid, dim3(256), st, pa, pl, nz);
}

template <int WT>
static hipError_t launch_prepare_mfma_w(const MlaProjParams& pa, const LatentWriteParams& pl, int out_dt, int lat_dt,
                                        hipStream_t st, KernelTimer* t) {
    if (out_dt == DT_BF16) return launch_prepare_mfma_o<WT, DT_BF16>(pa, pl, lat_dt, st, t);
    return launch_prepare_mfma_o<WT, DT_F32>(pa, pl, lat_dt, st, t);
}

hipError_t launch_mla_prepare(const MlaProjParams& pa, const LatentWriteParams& pl, int w_type, int out_dt,
                              int lat_dt, hipStream_t st, KernelTimer* t) {
    if (pa.rows == 0 || pl.rows == 0) {
        // one stage empty: the other alone
        if (pl.rows > 0)
            if (hipError_t e = launch_mla_latent_write(pl, lat_dt, st, t); e != hipSuccess) return e;
        return pa.rows > 0 ? launch_mla_absorb(pa, w_type, out_dt, st, t) : hipSuccess;
    }
    if (pa.rows >= kProjMfmaRows)  // prompt sizes: the absorb MFMA form with the latent rows
        return w_type == W_F16 ? launch_prepare_mfma_w<W_F16>(pa, pl, out_dt, lat_dt, st, t)
             : w_type == W_Q8_0 ? launch_prepare_mfma_w<W_Q8_0>(pa, pl, out_dt, lat_dt, st, t)
                                : launch_prepare_mfma_w<W_Q4_0>(pa, pl, out_dt, lat_dt, st, t);
    return w_type == W_F16 ? launch_prepare_w<W_F16>(pa, pl, out_dt, lat_dt, st, t)
         : w_type == W_Q8_0 ? launch_prepare_w<W_Q8_0>(pa, pl, out_dt, lat_dt, st, t)
                            : launch_prepare_w<W_Q4_0>(pa, pl, out_dt, lat_dt, st, t);
}

template <int WT>
static hipError_t launch_project_w(const MlaProjParams& p, int out_dt, hipStream_t st, KernelTimer* t) {
    if (p.rows >= kProjMfmaRows) {
        const int groups = (p.rows + 63) / 64;
        const int per = std::max(1, 256 / (p.H * 2));
        const dim3 grid(p.H, 2, std::min(groups, per));
        if (out_dt == DT_F16)
            return launch_k(t, "mla_project", mla_project_mfma_kernel<WT, DT_F16>, grid, dim3(256), st, p);
        return launch_k(t, "mla_project", mla_project_mfma_kernel<WT, DT_F32>, grid, dim3(256), st, p);
    }
    const dim3 grid(p.H, 128 / 32);
    if (out_dt == DT_F16) return launch_k(t, "mla_project", mla_project_kernel<WT, DT_F16>, grid, dim3(256), st, p);
    return launch_k(t, "mla_project", mla_project_kernel<WT, DT_F32>, grid, dim3(256), st, p);
}

hipError_t launch_mla_project(const MlaProjParams& p, int w_type, int out_dt, hipStream_t st, KernelTimer* t) {
    return w_type == W_F16 ? launch_project_w<W_F16>(p, out_dt, st, t)
         : w_type == W_Q8_0 ? launch_project_w<W_Q8_0>(p, out_dt, st, t)
                            : launch_project_w<W_Q4_0>(p, out_dt, st, t);
}

}  // namespace mugen_attn
