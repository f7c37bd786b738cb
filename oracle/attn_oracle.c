/*
 * attn_oracle.c -- CPU restatement of Mugen's attention paths.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the parity tests,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg compare the HIP
 * kernels against.  Nothing in the product library (mugen_amd/) links,
 * loads or calls it.
 *
 * Restated from (reference paths relative to the Mugen source tree):
 *   oracle_gqa_attention  <- TransformerModel::Impl::cpu_attention,
 *                            src/core/model/transformer.cpp:2441-2485
 *                            (GQA map kv_h = h / (H/Hk) :2452, scale
 *                            1/sqrt(head_dim) :2444, fp32 dot :2458-2465,
 *                            max-subtract softmax with std::exp :2467-2473,
 *                            p-weighted V sum d-outer/s-inner :2476-2483)
 *   oracle_gqa_prefill    <- flash_prefill_attention semantics,
 *                            src/metal/kernel_sources.h:2769-2896, causal rule
 *                            causal_len = start + token + 1 (:2796), and the
 *                            per-token CPU rule transformer.cpp:1334-1335
 *   oracle_mla_attention  <- latent core of cpu_mla_attention,
 *                            src/core/model/transformer.cpp:2576-2608 (score
 *                            = q_abs . c[0:512] + q_rope . c[512:576] summed
 *                            into one fp32 accumulator, times scale :2550;
 *                            softmax :2591-2598; o = sum_t p_t c_t[0:512]
 *                            accumulated s-outer/d-inner :2602-2608);
 *                            multi-query (verify) rows follow the per-token
 *                            call seq_len = start_position + t + 1
 *                            (transformer.cpp:1325-1337).
 *   oracle_dequant_row    <- dequant_weight_row, transformer.cpp:2488-2534
 *   oracle_mla_absorb     <- q_absorbed = q_nope x k_b, transformer.cpp:2563-2573
 *   oracle_mla_project    <- out_h = out_comp x v_b^T, transformer.cpp:2610-2620
 *   (absorb + oracle_mla_attention + project = cpu_mla_attention,
 *    transformer.cpp:2539-2623)
 *   oracle_yarn_rope_freq <- yarn_rope_freq, transformer.cpp:41-70
 *   oracle_rope_neox_f16  <- q / k_rope NeoX RoPE, transformer.cpp:3903-3917,
 *                            :3968-3980
 *   oracle_mla_kv_prepare <- c_kv RMSNorm + k_rope RoPE, transformer.cpp:3935-3981
 *   oracle_mla_latent_write <- prepare + scatter into the latent cache,
 *                            transformer.cpp:3930-3987
 *   oracle_q4_*           <- quantize_group / dequantize_group / *_token,
 *                            src/core/memory/kv_cache.cpp:21-97
 *   oracle_kvq4_read      <- KVCache::append + read_k / read_v,
 *                            src/core/memory/kv_cache.cpp:163-278
 *   oracle_scatter_kv     <- scatter_kv, src/metal/kernel_sources.h:3018-3028
 *
 * The summation orders above are kept (sequential fp32 sums, expf, divide
 * by the sum) so that the float variant reproduces the reference's rounding
 * behaviour; the double variants are the same algorithm in fp64 and serve
 * as the tolerance anchor.  Inputs arrive as float arrays that already hold
 * the storage-dtype values (fp16/bf16 rounded); the reference widens each
 * f16 element with static_cast<float>, which is exact, so this is the same
 * arithmetic.
 *
 * Departure (documented): seq_len == 0 is undefined in the reference
 * (max_element of an empty range); here the output row is all zeros, which
 * is what the reference's Metal flash kernels produce (inv_sum = 0 when
 * running_sum == 0, kernel_sources.h:2982).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* dtype rounding helpers (IEEE binary16 and bfloat16, round-to-even)  */
/* ------------------------------------------------------------------ */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t oracle_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40); /* NaN */
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

float oracle_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0) {
        if (man == 0) return u2f(sign);
        /* subnormal: value = man * 2^-24 */
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (exp == 31) return u2f(sign | 0x7f800000u | (man << 13));
    return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t oracle_f32_to_f16(float f) {
    uint32_t u = f2u(f);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);          /* NaN */
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);         /* overflow -> inf */
    if (a < 0x38800000u) {                                            /* subnormal / zero */
        /* value in units of 2^-24, round to nearest even */
        float v = u2f(a) * 16777216.0f;
        float r = rintf(v); /* default rounding mode: nearest-even */
        return (uint16_t)(sign | (uint32_t)r);
    }
    uint32_t exp = (a >> 23) - 112u;
    uint32_t man = a & 0x7fffffu;
    uint32_t half = (exp << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half += 1u;
    return (uint16_t)(sign | half);
}

/* Round a float array in place to the values representable in `dtype`
 * (0 = f32: no-op, 1 = f16, 2 = bf16) and optionally emit the raw bits. */
void oracle_round_to_dtype(float* x, uint16_t* bits_out, int64_t n, int dtype) {
    for (int64_t i = 0; i < n; i++) {
        uint16_t b;
        if (dtype == 1) { b = oracle_f32_to_f16(x[i]); x[i] = oracle_f16_to_f32(b); }
        else if (dtype == 2) { b = oracle_f32_to_bf16(x[i]); x[i] = oracle_bf16_to_f32(b); }
        else continue;
        if (bits_out) bits_out[i] = b;
    }
}

/* ------------------------------------------------------------------ */
/* seeded normal generator: mt19937_64 + Box-Muller                    */
/* ------------------------------------------------------------------ */

typedef struct { uint64_t mt[312]; int idx; } mt64_t;

static void mt64_seed(mt64_t* s, uint64_t seed) {
    s->mt[0] = seed;
    for (int i = 1; i < 312; i++)
        s->mt[i] = 6364136223846793005ULL * (s->mt[i - 1] ^ (s->mt[i - 1] >> 62)) + (uint64_t)i;
    s->idx = 312;
}

static uint64_t mt64_next(mt64_t* s) {
    static const uint64_t UM = 0xFFFFFFFF80000000ULL, LM = 0x7FFFFFFFULL;
    if (s->idx >= 312) {
        for (int i = 0; i < 312; i++) {
            uint64_t x = (s->mt[i] & UM) | (s->mt[(i + 1) % 312] & LM);
            uint64_t xa = x >> 1;
            if (x & 1ULL) xa ^= 0xB5026F5AA96619E9ULL;
            s->mt[i] = s->mt[(i + 156) % 312] ^ xa;
        }
        s->idx = 0;
    }
    uint64_t x = s->mt[s->idx++];
    x ^= (x >> 29) & 0x5555555555555555ULL;
    x ^= (x << 17) & 0x71D67FFFEDA60000ULL;
    x ^= (x << 37) & 0xFFF7EEE000000000ULL;
    x ^= x >> 43;
    return x;
}

/* First output of mt19937_64 seeded with 5489 must be 14514284786278117030
 * (the C++ standard's required value); exposed for the self-test. */
uint64_t oracle_mt64_first(uint64_t seed, int64_t skip) {
    mt64_t s; mt64_seed(&s, seed);
    for (int64_t i = 0; i < skip; i++) mt64_next(&s);
    return mt64_next(&s);
}

/* n normal draws N(mean, std^2); pairs from Box-Muller, u in (0, 1]. */
void oracle_randn(uint64_t seed, int64_t n, float mean, float stdv, float* out) {
    mt64_t s; mt64_seed(&s, seed);
    const double two_pi = 6.283185307179586476925286766559;
    for (int64_t i = 0; i < n; i += 2) {
        double u1 = ((double)(mt64_next(&s) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        double u2 = (double)(mt64_next(&s) >> 11) * (1.0 / 9007199254740992.0);
        double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(mean + stdv * r * cos(two_pi * u2));
        if (i + 1 < n) out[i + 1] = (float)(mean + stdv * r * sin(two_pi * u2));
    }
}

/* n integers uniform in [lo, hi] (inclusive), for ragged context lengths. */
void oracle_randint(uint64_t seed, int64_t n, int32_t lo, int32_t hi, int32_t* out) {
    mt64_t s; mt64_seed(&s, seed);
    uint64_t span = (uint64_t)((int64_t)hi - lo + 1);
    for (int64_t i = 0; i < n; i++) out[i] = lo + (int32_t)(mt64_next(&s) % span);
}

/* ------------------------------------------------------------------ */
/* GQA decode: one query token per sequence (cpu_attention)            */
/* ------------------------------------------------------------------ */
/*
 * q        [B][H][D]
 * k, v     sequence b starts at b*seq_stride; token t, kv head j at
 *          t*(Hk*D) + j*D  (the reference's token-major [T][Hk*D] layout,
 *          kv_stride = Hk*D, transformer.cpp:2446)
 * out      [B][H][D]
 * scale    <= 0 selects 1/sqrt(D)
 */
#define GQA_PRE(REAL)                                                                \
    int G = H / Hk;                                                                        \
    int64_t kv_stride = (int64_t)Hk * D;                                                   \
    /* the reference computes the scale in float (transformer.cpp:2444) */ \
    REAL sc = (REAL)(scale > 0 ? scale : 1.0f / sqrtf((float)D));
#define GQA_BODY(REAL, EXP)                                                                \
    for (int64_t bh = 0; bh < (int64_t)B * H; bh++) {                                      \
        int b = (int)(bh / H), h = (int)(bh % H);                                          \
        int T = seq_lens[b];                                                               \
        const float* qh = q + ((int64_t)b * H + h) * D;                                    \
        const float* kb = k + b * seq_stride + (int64_t)(h / G) * D;                       \
        const float* vb = v + b * seq_stride + (int64_t)(h / G) * D;                       \
        OUT_T* oh = out + ((int64_t)b * H + h) * D;                                        \
        if (T <= 0) { for (int d = 0; d < D; d++) oh[d] = 0; continue; }                   \
        REAL* s = (REAL*)malloc(sizeof(REAL) * (size_t)T);                                 \
        for (int t = 0; t < T; t++) {                                                      \
            REAL dot = 0;                                                                  \
            for (int d = 0; d < D; d++) dot += (REAL)qh[d] * (REAL)kb[t * kv_stride + d]; \
            s[t] = dot * sc;                                                               \
        }                                                                                  \
        REAL mx = s[0];                                                                    \
        for (int t = 1; t < T; t++) if (s[t] > mx) mx = s[t];                              \
        REAL sum = 0;                                                                      \
        for (int t = 0; t < T; t++) { s[t] = EXP(s[t] - mx); sum += s[t]; }                \
        for (int t = 0; t < T; t++) s[t] /= sum;                                           \
        for (int d = 0; d < D; d++) {                                                      \
            REAL val = 0;                                                                  \
            for (int t = 0; t < T; t++) val += s[t] * (REAL)vb[t * kv_stride + d];         \
            oh[d] = (OUT_T)val;                                                            \
        }                                                                                  \
        free(s);                                                                           \
    }

#define OUT_T float
void oracle_gqa_attention_f32(const float* q, const float* k, const float* v,
                              const int32_t* seq_lens, float* out, int B, int H, int Hk,
                              int D, int64_t seq_stride, float scale, int nthreads) {
    GQA_PRE(float)
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 1) if (nthreads != 1)
#endif
    GQA_BODY(float, expf)
}
#undef OUT_T
#define OUT_T double
void oracle_gqa_attention_f64(const float* q, const float* k, const float* v,
                              const int32_t* seq_lens, double* out, int B, int H, int Hk,
                              int D, int64_t seq_stride, float scale) {
    GQA_PRE(double)
    GQA_BODY(double, exp)
}
#undef OUT_T

/* ------------------------------------------------------------------ */
/* GQA causal prefill (flash_prefill_attention semantics)              */
/* ------------------------------------------------------------------ */
/*
 * q     [N][H][D]  (token-major Q_batch)
 * k, v  [kv_len][Hk*D]
 * out   [N][H][D]
 * token i attends to keys [0, start + i]  (causal_len = start + i + 1,
 * clipped to kv_len)
 */
#define PREFILL_PRE(REAL)                                                            \
    int G = H / Hk;                                                                        \
    int64_t kv_stride = (int64_t)Hk * D;                                                   \
    /* the reference computes the scale in float (transformer.cpp:2444) */ \
    REAL sc = (REAL)(scale > 0 ? scale : 1.0f / sqrtf((float)D));
#define PREFILL_BODY(REAL, EXP)                                                            \
    for (int64_t ih = 0; ih < (int64_t)N * H; ih++) {                                      \
        int i = (int)(ih / H), h = (int)(ih % H);                                          \
        int T = start + i + 1;                                                             \
        if (T > kv_len) T = kv_len;                                                        \
        const float* qh = q + ((int64_t)i * H + h) * D;                                    \
        const float* kb = k + (int64_t)(h / G) * D;                                        \
        const float* vb = v + (int64_t)(h / G) * D;                                        \
        OUT_T* oh = out + ((int64_t)i * H + h) * D;                                        \
        if (T <= 0) { for (int d = 0; d < D; d++) oh[d] = 0; continue; }                   \
        REAL* s = (REAL*)malloc(sizeof(REAL) * (size_t)T);                                 \
        for (int t = 0; t < T; t++) {                                                      \
            REAL dot = 0;                                                                  \
            for (int d = 0; d < D; d++) dot += (REAL)qh[d] * (REAL)kb[t * kv_stride + d]; \
            s[t] = dot * sc;                                                               \
        }                                                                                  \
        REAL mx = s[0];                                                                    \
        for (int t = 1; t < T; t++) if (s[t] > mx) mx = s[t];                              \
        REAL sum = 0;                                                                      \
        for (int t = 0; t < T; t++) { s[t] = EXP(s[t] - mx); sum += s[t]; }                \
        for (int t = 0; t < T; t++) s[t] /= sum;                                           \
        for (int d = 0; d < D; d++) {                                                      \
            REAL val = 0;                                                                  \
            for (int t = 0; t < T; t++) val += s[t] * (REAL)vb[t * kv_stride + d];         \
            oh[d] = (OUT_T)val;                                                            \
        }                                                                                  \
        free(s);                                                                           \
    }

#define OUT_T float
void oracle_gqa_prefill_f32(const float* q, const float* k, const float* v, float* out,
                            int N, int H, int Hk, int D, int kv_len, int start, float scale,
                            int nthreads) {
    PREFILL_PRE(float)
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 1) if (nthreads != 1)
#endif
    PREFILL_BODY(float, expf)
}
#undef OUT_T
#define OUT_T double
void oracle_gqa_prefill_f64(const float* q, const float* k, const float* v, double* out,
                            int N, int H, int Hk, int D, int kv_len, int start, float scale) {
    PREFILL_PRE(double)
    PREFILL_BODY(double, exp)
}
#undef OUT_T

/* ------------------------------------------------------------------ */
/* MLA absorbed attention over the latent cache (cpu_mla_attention)    */
/* ------------------------------------------------------------------ */
/*
 * q       [B][q_len][H][kv_rank + rope]   absorbed query (q_nope.W_UK ++ q_rope)
 * latent  sequence b at b*seq_stride; token t at t*(kv_rank + rope)
 * out     [B][q_len][H][kv_rank]          o = sum_t p_t * c_t[0:kv_rank]
 * query i of q_len sees T_i = seq_len[b] - q_len + i + 1 tokens
 */
#define MLA_PRE(REAL)                                                                      \
    int C = kv_rank + rope;                                                                \
    REAL sc = (REAL)scale;
#define MLA_BODY(REAL, EXP)                                                                \
    for (int64_t bqh = 0; bqh < (int64_t)B * q_len * H; bqh++) {                           \
        int b = (int)(bqh / ((int64_t)q_len * H));                                         \
        int qi = (int)((bqh / H) % q_len);                                                 \
        int T = seq_lens[b] - q_len + qi + 1;                                              \
        const float* qa = q + bqh * C;                                                     \
        const float* cb = latent + b * seq_stride;                                         \
        OUT_T* oh = out + bqh * kv_rank;                                                   \
        if (T <= 0) { for (int d = 0; d < kv_rank; d++) oh[d] = 0; continue; }             \
        REAL* s = (REAL*)malloc(sizeof(REAL) * (size_t)T);                                 \
        for (int t = 0; t < T; t++) {                                                      \
            const float* cs = cb + (int64_t)t * C;                                         \
            REAL acc = 0;                                                                  \
            for (int d = 0; d < kv_rank; d++) acc += (REAL)qa[d] * (REAL)cs[d];            \
            for (int d = 0; d < rope; d++) acc += (REAL)qa[kv_rank + d] * (REAL)cs[kv_rank + d]; \
            s[t] = acc * sc;                                                               \
        }                                                                                  \
        REAL mx = s[0];                                                                    \
        for (int t = 1; t < T; t++) if (s[t] > mx) mx = s[t];                              \
        REAL sum = 0;                                                                      \
        for (int t = 0; t < T; t++) { s[t] = EXP(s[t] - mx); sum += s[t]; }                \
        for (int t = 0; t < T; t++) s[t] /= sum;                                           \
        REAL* o = (REAL*)calloc((size_t)kv_rank, sizeof(REAL));                            \
        for (int t = 0; t < T; t++) {                                                      \
            const float* cs = cb + (int64_t)t * C;                                         \
            REAL w = s[t];                                                                 \
            for (int d = 0; d < kv_rank; d++) o[d] += w * (REAL)cs[d];                     \
        }                                                                                  \
        for (int d = 0; d < kv_rank; d++) oh[d] = (OUT_T)o[d];                             \
        free(o);                                                                           \
        free(s);                                                                           \
    }

#define OUT_T float
void oracle_mla_attention_f32(const float* q, const float* latent, const int32_t* seq_lens,
                              float* out, int B, int q_len, int H, int kv_rank, int rope,
                              int64_t seq_stride, float scale, int nthreads) {
    MLA_PRE(float)
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 1) if (nthreads != 1)
#endif
    MLA_BODY(float, expf)
}
#undef OUT_T
#define OUT_T double
void oracle_mla_attention_f64(const float* q, const float* latent, const int32_t* seq_lens,
                              double* out, int B, int q_len, int H, int kv_rank, int rope,
                              int64_t seq_stride, float scale) {
    MLA_PRE(double)
    MLA_BODY(double, exp)
}
#undef OUT_T

/* ------------------------------------------------------------------ */
/* MLA absorption / up-projection (the rest of cpu_mla_attention)       */
/* ------------------------------------------------------------------ */
/*
 * oracle_dequant_row <- dequant_weight_row, transformer.cpp:2488-2534.
 * Weight types use the GGML ids of src/model/ggml_types.h:12-20:
 *   F16  (1): K little-endian halfs per row;
 *   Q8_0 (8): K/32 blocks of 34 bytes = f16 scale s + 32 int8 q; w = s * q;
 *   Q4_0 (2): K/32 blocks of 18 bytes = f16 scale s + 16 bytes; element j
 *             of a block is (low nibble of byte j) - 8 for j < 16 and
 *             (high nibble of byte j-16) - 8 for j >= 16, times s.
 * Any other type zero-fills the row (transformer.cpp:2530-2533).
 */
static size_t wrow_bytes(int type, int K) {
    if (type == 1) return (size_t)K * 2;
    if (type == 8) return (size_t)(K / 32) * 34;
    if (type == 2) return (size_t)(K / 32) * 18;
    return 0;
}
void oracle_dequant_row(const uint8_t* buf, int type, int64_t row, int K, float* out) {
    const uint8_t* rp = buf + (size_t)row * wrow_bytes(type, K);
    if (type == 1) {
        for (int i = 0; i < K; i++) {
            uint16_t h;
            memcpy(&h, rp + 2 * i, 2);
            out[i] = oracle_f16_to_f32(h);
        }
    } else if (type == 8) {
        for (int b = 0; b < K / 32; b++) {
            const uint8_t* blk = rp + (size_t)b * 34;
            uint16_t sh;
            memcpy(&sh, blk, 2);
            float sc = oracle_f16_to_f32(sh);
            for (int j = 0; j < 32; j++) out[b * 32 + j] = sc * (float)(int8_t)blk[2 + j];
        }
    } else if (type == 2) {
        for (int b = 0; b < K / 32; b++) {
            const uint8_t* blk = rp + (size_t)b * 18;
            uint16_t sh;
            memcpy(&sh, blk, 2);
            float sc = oracle_f16_to_f32(sh);
            for (int j = 0; j < 16; j++) {
                out[b * 32 + j] = (float)((blk[2 + j] & 0x0F) - 8) * sc;
                out[b * 32 + j + 16] = (float)((blk[2 + j] >> 4) - 8) * sc;
            }
        }
    } else {
        memset(out, 0, sizeof(float) * (size_t)K);
    }
}

/*
 * oracle_mla_absorb <- transformer.cpp:2563-2573: per query row r and head
 * h, q_abs[d] = sum_i q_nope[i] * W_kb[h*nope + i][d] over i in order
 * (terms with q_nope[i] == 0 skipped, as there), d < kv_rank; the q_rope
 * part is appended unchanged.  q [rows][H][nope + rope] (f16 values),
 * q_abs [rows][H][kv_rank + rope] fp32.
 */
void oracle_mla_absorb(const float* q, const uint8_t* w_kb, int w_type, float* q_abs, int rows, int H,
                       int nope, int rope, int kv_rank) {
    float* wrow = (float*)malloc(sizeof(float) * (size_t)kv_rank);
    for (int64_t rh = 0; rh < (int64_t)rows * H; rh++) {
        int h = (int)(rh % H);
        const float* qn = q + rh * (nope + rope);
        float* qa = q_abs + rh * (kv_rank + rope);
        for (int d = 0; d < kv_rank; d++) qa[d] = 0.f;
        for (int i = 0; i < nope; i++) {
            float qi = qn[i];
            if (qi == 0.0f) continue;
            oracle_dequant_row(w_kb, w_type, (int64_t)h * nope + i, kv_rank, wrow);
            for (int d = 0; d < kv_rank; d++) qa[d] += qi * wrow[d];
        }
        for (int j = 0; j < rope; j++) qa[kv_rank + j] = qn[nope + j];
    }
    free(wrow);
}

/*
 * oracle_mla_project <- transformer.cpp:2610-2620: out[r][h][j] =
 * sum_d o[r][h][d] * W_vb[h*v_head + j][d] (d in order), rounded to f16 as
 * the reference's static_cast<f16> does; out_f16 holds the rounded values
 * as floats.  o [rows][H][kv_rank] fp32.
 */
void oracle_mla_project(const float* o, const uint8_t* w_vb, int w_type, float* out_f16, int rows, int H,
                        int kv_rank, int v_head) {
    float* wrow = (float*)malloc(sizeof(float) * (size_t)kv_rank);
    for (int64_t rh = 0; rh < (int64_t)rows * H; rh++) {
        int h = (int)(rh % H);
        const float* oc = o + rh * kv_rank;
        for (int j = 0; j < v_head; j++) {
            oracle_dequant_row(w_vb, w_type, (int64_t)h * v_head + j, kv_rank, wrow);
            float val = 0.0f;
            for (int d = 0; d < kv_rank; d++) val += oc[d] * wrow[d];
            out_f16[rh * v_head + j] = oracle_f16_to_f32(oracle_f32_to_f16(val));
        }
    }
    free(wrow);
}

/* ------------------------------------------------------------------ */
/* MLA latent-cache writer and q RoPE                                  */
/* ------------------------------------------------------------------ */
/*
 * oracle_yarn_rope_freq <- yarn_rope_freq, transformer.cpp:41-70: base
 * frequency theta^(-2i/rope_dim) (powf), and for factor > 1 the YaRN
 * correction with beta_fast 32 / beta_slow 1: dims below
 * low = floor(d ln(ctx / (32 * 2 pi)) / (2 ln theta)) keep it, dims above
 * high = ceil(d ln(ctx / (2 pi)) / (2 ln theta)) (clamped to d/2 - 1) take
 * freq / factor, a linear ramp in between.  float arithmetic throughout,
 * as there (std::pow / std::log / std::floor on floats).
 */
float oracle_yarn_rope_freq(int dim_idx, int rope_dim, float factor, int original_ctx, float theta) {
    const float pi_f = 3.14159265358979323846f;
    float freq = 1.0f / powf(theta, 2.0f * (float)dim_idx / (float)rope_dim);
    if (factor <= 1.0f) return freq;
    float log_base = logf(theta);
    float ctx_f = (float)original_ctx;
    float dim_f = (float)rope_dim;
    float low = floorf(dim_f * logf(ctx_f / (32.0f * 2.0f * pi_f)) / (2.0f * log_base));
    float high = ceilf(dim_f * logf(ctx_f / (1.0f * 2.0f * pi_f)) / (2.0f * log_base));
    if (low < 0.0f) low = 0.0f;
    if (high > (float)(rope_dim / 2 - 1)) high = (float)(rope_dim / 2 - 1);
    float idx = (float)dim_idx;
    if (idx < low) return freq;
    if (idx > high) return freq / factor;
    float span = high - low;
    if (span < 0.001f) span = 0.001f;
    float ramp = (idx - low) / span;
    if (ramp < 0.0f) ramp = 0.0f;
    if (ramp > 1.0f) ramp = 1.0f;
    return freq * (1.0f - ramp) + (freq / factor) * ramp;
}

/*
 * oracle_rope_neox_f16 <- the NeoX RoPE of transformer.cpp:3903-3917 (q)
 * and :3968-3980 (k_rope): pairs (i, i + rope_dim/2), angle = pos * freq_i
 * in float, x0' = x0 cos - x1 sin, x1' = x1 cos + x0 sin, each rounded to
 * f16.  x holds rope_dim f16 bit patterns, rotated in place.
 */
void oracle_rope_neox_f16(uint16_t* x, int rope_dim, int pos, const float* freqs) {
    int half = rope_dim / 2;
    for (int i = 0; i < half; i++) {
        float angle = (float)pos * freqs[i];
        float cv = cosf(angle), sv = sinf(angle);
        float x0 = oracle_f16_to_f32(x[i]);
        float x1 = oracle_f16_to_f32(x[i + half]);
        x[i] = oracle_f32_to_f16(x0 * cv - x1 * sv);
        x[i + half] = oracle_f32_to_f16(x1 * cv + x0 * sv);
    }
}

/*
 * oracle_mla_kv_prepare <- transformer.cpp:3935-3981, one token: RMSNorm of
 * c_kv = kva[0:kv_rank] (sequential float sum of squares, scale
 * 1/sqrt(ss/kv_rank + eps), kva[i] = f16((kva[i] * scale) * w[i])), then
 * the NeoX RoPE of k_rope = kva[kv_rank : kv_rank + rope_dim].  kva and
 * norm_w are f16 bit patterns; kva is updated in place.
 */
void oracle_mla_kv_prepare(uint16_t* kva, const uint16_t* norm_w, int kv_rank, int rope_dim, float eps, int pos,
                           const float* freqs) {
    float ss = 0.0f;
    for (int i = 0; i < kv_rank; i++) {
        float v = oracle_f16_to_f32(kva[i]);
        ss += v * v;
    }
    ss = 1.0f / sqrtf(ss / (float)kv_rank + eps);
    for (int i = 0; i < kv_rank; i++) {
        float v = oracle_f16_to_f32(kva[i]) * ss;
        kva[i] = oracle_f32_to_f16(v * oracle_f16_to_f32(norm_w[i]));
    }
    oracle_rope_neox_f16(kva + kv_rank, rope_dim, pos, freqs);
}

/*
 * oracle_mla_latent_write <- transformer.cpp:3930-3987 (prepare, then the
 * scatter of :3982-3987 to cache offset pos * (kv_rank + rope_dim)) for
 * `rows` tokens: token r belongs to sequence r / rows_per_seq and goes to
 * row positions[r] of that sequence's cache (seq_stride elements apart).
 * Rows whose position is outside [0, max_seq_len) are not written.
 */
void oracle_mla_latent_write(const uint16_t* kv_a, const uint16_t* norm_w, const int32_t* positions,
                             uint16_t* cache, int rows, int rows_per_seq, int64_t seq_stride, int max_seq_len,
                             int kv_rank, int rope_dim, float eps, const float* freqs) {
    int C = kv_rank + rope_dim;
    uint16_t* tmp = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)C);
    for (int r = 0; r < rows; r++) {
        int pos = positions[r];
        if (pos < 0 || pos >= max_seq_len) continue;
        memcpy(tmp, kv_a + (size_t)r * C, sizeof(uint16_t) * (size_t)C);
        oracle_mla_kv_prepare(tmp, norm_w, kv_rank, rope_dim, eps, pos, freqs);
        memcpy(cache + (int64_t)(r / rows_per_seq) * seq_stride + (int64_t)pos * C, tmp, sizeof(uint16_t) * (size_t)C);
    }
    free(tmp);
}

/* ------------------------------------------------------------------ */
/* 4-bit group KV store (kv_cache.cpp)                                 */
/* ------------------------------------------------------------------ */
/*
 * oracle_q4_quantize_group <- quantize_group, kv_cache.cpp:21-56: a group
 * of up to 32 f16 values (missing ones are 0 and take part in min / max)
 * becomes 20 bytes: f16 scale = f16(range / 15) (0 when max == min), f16
 * min, then 16 bytes whose low / high nibble holds value 2i / 2i+1 as
 * min(15, roundf((v - min) / scale)) (all nibbles 0 when scale is 0).
 */
void oracle_q4_quantize_group(const uint16_t* src, uint8_t* dst, int count) {
    float vals[32];
    uint16_t bits[32];
    for (int i = 0; i < 32; i++) {
        bits[i] = i < count ? src[i] : 0;
        vals[i] = oracle_f16_to_f32(bits[i]);
    }
    int lo = 0, hi = 0;
    for (int i = 1; i < 32; i++) {
        if (vals[i] < vals[lo]) lo = i;
        if (vals[i] > vals[hi]) hi = i;
    }
    float range = vals[hi] - vals[lo];
    uint16_t scale = range == 0.0f ? 0 : oracle_f32_to_f16(range / 15.0f);
    uint16_t minv = bits[lo];
    memcpy(dst, &scale, 2);
    memcpy(dst + 2, &minv, 2);
    float sf = oracle_f16_to_f32(scale), mf = oracle_f16_to_f32(minv);
    for (int i = 0; i < 16; i++) {
        uint8_t n0 = 0, n1 = 0;
        if (sf > 0.0f) {
            float a = roundf((vals[2 * i] - mf) / sf), b = roundf((vals[2 * i + 1] - mf) / sf);
            n0 = (uint8_t)(a < 15.0f ? a : 15.0f);
            n1 = (uint8_t)(b < 15.0f ? b : 15.0f);
        }
        dst[4 + i] = (uint8_t)((n1 << 4) | n0);
    }
}

/*
 * oracle_q4_dequantize_group <- dequantize_group, kv_cache.cpp:58-73:
 * value 2i / 2i+1 = f16(min + nibble * scale), product and sum rounded
 * separately.
 */
void oracle_q4_dequantize_group(const uint8_t* src, uint16_t* dst) {
    uint16_t scale, minv;
    memcpy(&scale, src, 2);
    memcpy(&minv, src + 2, 2);
    float sf = oracle_f16_to_f32(scale), mf = oracle_f16_to_f32(minv);
    for (int i = 0; i < 16; i++) {
        uint8_t packed = src[4 + i];
        dst[2 * i] = oracle_f32_to_f16(mf + (float)(packed & 0x0F) * sf);
        dst[2 * i + 1] = oracle_f32_to_f16(mf + (float)((packed >> 4) & 0x0F) * sf);
    }
}

/* quantize_token / dequantize_token (kv_cache.cpp:75-97): groups of 32
 * consecutive values of the token's [n_kv_heads * head_dim] row, the last
 * one possibly short. */
void oracle_q4_quantize_token(const uint16_t* src, uint8_t* dst, int vpt) {
    for (int g = 0; g * 32 < vpt; g++) {
        int cnt = vpt - g * 32 < 32 ? vpt - g * 32 : 32;
        oracle_q4_quantize_group(src + g * 32, dst + g * 20, cnt);
    }
}
void oracle_q4_dequantize_token(const uint8_t* src, uint16_t* dst, int vpt) {
    uint16_t tmp[32];
    for (int g = 0; g * 32 < vpt; g++) {
        int cnt = vpt - g * 32 < 32 ? vpt - g * 32 : 32;
        oracle_q4_dequantize_group(src + g * 20, tmp);
        memcpy(dst + g * 32, tmp, sizeof(uint16_t) * (size_t)cnt);
    }
}

/*
 * oracle_kvq4_read <- KVCache::read_k / read_v (kv_cache.cpp:218-278) of a
 * layer whose first n_q4 tokens were quantised on append (append,
 * kv_cache.cpp:163-216: every token older than the newest
 * fp16_preserve_last is quantised from its own f16 values): tokens < n_q4
 * come back as dequant(quant(x)), the rest unchanged.  x [T][vpt] f16 bits.
 */
void oracle_kvq4_read(const uint16_t* x, uint16_t* out, int T, int vpt, int n_q4) {
    uint8_t* q = (uint8_t*)malloc((size_t)((vpt + 31) / 32) * 20);
    for (int t = 0; t < T; t++) {
        if (t < n_q4) {
            oracle_q4_quantize_token(x + (size_t)t * vpt, q, vpt);
            oracle_q4_dequantize_token(q, out + (size_t)t * vpt, vpt);
        } else {
            memcpy(out + (size_t)t * vpt, x + (size_t)t * vpt, sizeof(uint16_t) * (size_t)vpt);
        }
    }
    free(q);
}

/* ------------------------------------------------------------------ */
/* scatter_kv: dst[offset + i] = src[i] for i < count (16-bit elements) */
/* ------------------------------------------------------------------ */
void oracle_scatter_kv(const uint16_t* src, uint16_t* dst, int64_t offset, int64_t count) {
    for (int64_t i = 0; i < count; i++) dst[offset + i] = src[i];
}

int oracle_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
