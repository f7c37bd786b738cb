/*
 * oracle_sanitize_check.c -- every exported function of oracle/attn_oracle.c
 * run once on small shapes, built together with the oracle under
 * AddressSanitizer + UndefinedBehaviorSanitizer (tests/test_sanitizers.py).
 * Buffers are heap-allocated at their exact sizes so an access one element
 * past any of them is reported.  Shapes include the edges the parity tests
 * use: a zero-length sequence, ragged lengths, one query head per KV head
 * and many, a start offset, a partial 4-bit group, every weight encoding.
 * Prints "PASS" when every call returned (a sanitizer report aborts first).
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

uint16_t oracle_f32_to_bf16(float f);
float oracle_bf16_to_f32(uint16_t h);
float oracle_f16_to_f32(uint16_t h);
uint16_t oracle_f32_to_f16(float f);
void oracle_round_to_dtype(float* x, uint16_t* bits_out, int64_t n, int dtype);
uint64_t oracle_mt64_first(uint64_t seed, int64_t skip);
void oracle_randn(uint64_t seed, int64_t n, float mean, float stdv, float* out);
void oracle_randint(uint64_t seed, int64_t n, int32_t lo, int32_t hi, int32_t* out);
void oracle_gqa_attention_f32(const float* q, const float* k, const float* v, const int32_t* seq_lens, float* out,
                              int B, int H, int Hk, int D, int64_t seq_stride, float scale, int nthreads);
void oracle_gqa_attention_f64(const float* q, const float* k, const float* v, const int32_t* seq_lens, double* out,
                              int B, int H, int Hk, int D, int64_t seq_stride, float scale);
void oracle_gqa_prefill_f32(const float* q, const float* k, const float* v, float* out, int N, int H, int Hk, int D,
                            int kv_len, int start, float scale, int nthreads);
void oracle_gqa_prefill_f64(const float* q, const float* k, const float* v, double* out, int N, int H, int Hk, int D,
                            int kv_len, int start, float scale);
void oracle_mla_attention_f32(const float* q, const float* latent, const int32_t* seq_lens, float* out, int B,
                              int q_len, int H, int kv_rank, int rope, int64_t seq_stride, float scale, int nthreads);
void oracle_mla_attention_f64(const float* q, const float* latent, const int32_t* seq_lens, double* out, int B,
                              int q_len, int H, int kv_rank, int rope, int64_t seq_stride, float scale);
void oracle_dequant_row(const uint8_t* buf, int type, int64_t row, int K, float* out);
void oracle_mla_absorb(const float* q, const uint8_t* w_kb, int w_type, float* q_abs, int rows, int H, int nope,
                       int rope, int kv_rank);
void oracle_mla_project(const float* o, const uint8_t* w_vb, int w_type, float* out_f16, int rows, int H,
                        int kv_rank, int v_head);
float oracle_yarn_rope_freq(int dim_idx, int rope_dim, float factor, int original_ctx, float theta);
void oracle_rope_neox_f16(uint16_t* x, int rope_dim, int pos, const float* freqs);
void oracle_mla_kv_prepare(uint16_t* kva, const uint16_t* norm_w, int kv_rank, int rope_dim, float eps, int pos,
                           const float* freqs);
void oracle_mla_latent_write(const uint16_t* kv_a, const uint16_t* norm_w, const int32_t* positions,
                             uint16_t* cache, int rows, int rows_per_seq, int64_t seq_stride, int max_seq_len,
                             int kv_rank, int rope_dim, float eps, const float* freqs);
void oracle_q4_quantize_group(const uint16_t* src, uint8_t* dst, int count);
void oracle_q4_dequantize_group(const uint8_t* src, uint16_t* dst);
void oracle_q4_quantize_token(const uint16_t* src, uint8_t* dst, int vpt);
void oracle_q4_dequantize_token(const uint8_t* src, uint16_t* dst, int vpt);
void oracle_kvq4_read(const uint16_t* x, uint16_t* out, int T, int vpt, int n_q4);
void oracle_scatter_kv(const uint16_t* src, uint16_t* dst, int64_t offset, int64_t count);
int oracle_num_threads(void);

#define F32 0
#define F16 1
#define BF16 2
#define W_F16 1
#define W_Q4_0 2
#define W_Q8_0 8

static float* randf(uint64_t seed, int64_t n) {
    float* p = (float*)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    oracle_randn(seed, n, 0.f, 1.f, p);
    return p;
}

static uint16_t* rand_f16_bits(uint64_t seed, int64_t n) {
    float* f = randf(seed, n);
    uint16_t* b = (uint16_t*)malloc((size_t)n * 2);
    oracle_round_to_dtype(f, b, n, F16);
    free(f);
    return b;
}

/* GGUF-encoded weight rows: F16 2 B/value, Q8_0 34 B per 32, Q4_0 18 B per 32 */
static size_t row_bytes(int type, int K) {
    return type == W_F16 ? (size_t)K * 2 : type == W_Q8_0 ? (size_t)K / 32 * 34 : (size_t)K / 32 * 18;
}

static uint8_t* weights(uint64_t seed, int type, int rows, int K) {
    const size_t n = row_bytes(type, K) * rows;
    uint8_t* w = (uint8_t*)malloc(n);
    if (type == W_F16) {
        uint16_t* b = rand_f16_bits(seed, (int64_t)rows * K);
        memcpy(w, b, n);
        free(b);
        return w;
    }
    int32_t* r = (int32_t*)malloc(n * sizeof(int32_t));
    oracle_randint(seed, (int64_t)n, 0, 255, r);
    for (size_t i = 0; i < n; i++) w[i] = (uint8_t)r[i];
    const size_t blk = type == W_Q8_0 ? 34 : 18;
    for (size_t b = 0; b < n / blk; b++) { /* a modest f16 block scale */
        const uint16_t d = oracle_f32_to_f16(0.01f);
        memcpy(w + b * blk, &d, 2);
    }
    free(r);
    return w;
}

static void gqa(void) {
    const int B = 3, H = 12, Hk = 3, D = 64, maxT = 37;
    const int32_t lens[3] = {37, 0, 5};
    const int64_t stride = (int64_t)maxT * Hk * D;
    float *q = randf(1, (int64_t)B * H * D), *k = randf(2, B * stride), *v = randf(3, B * stride);
    float* o = (float*)malloc(sizeof(float) * B * H * D);
    double* o64 = (double*)malloc(sizeof(double) * B * H * D);
    oracle_gqa_attention_f32(q, k, v, lens, o, B, H, Hk, D, stride, 0.f, 2);
    oracle_gqa_attention_f64(q, k, v, lens, o64, B, H, Hk, D, stride, 0.125f);
    free(q), free(k), free(v), free(o), free(o64);
}

static void prefill(void) {
    const int N = 19, H = 8, Hk = 1, D = 128, start = 6, kv = N + start;
    float *q = randf(4, (int64_t)N * H * D), *k = randf(5, (int64_t)kv * Hk * D), *v = randf(6, (int64_t)kv * Hk * D);
    float* o = (float*)malloc(sizeof(float) * N * H * D);
    double* o64 = (double*)malloc(sizeof(double) * N * H * D);
    oracle_gqa_prefill_f32(q, k, v, o, N, H, Hk, D, kv, start, 0.f, 3);
    oracle_gqa_prefill_f64(q, k, v, o64, N, H, Hk, D, kv, start, 0.f);
    free(q), free(k), free(v), free(o), free(o64);
}

static void mla(void) {
    const int B = 2, q_len = 3, H = 4, R = 512, P = 64, maxT = 21;
    const int32_t lens[2] = {21, 3};
    const int64_t stride = (int64_t)maxT * (R + P);
    float *q = randf(7, (int64_t)B * q_len * H * (R + P)), *lat = randf(8, B * stride);
    float* o = (float*)malloc(sizeof(float) * B * q_len * H * R);
    double* o64 = (double*)malloc(sizeof(double) * B * q_len * H * R);
    oracle_mla_attention_f32(q, lat, lens, o, B, q_len, H, R, P, stride, 0.0721f, 2);
    oracle_mla_attention_f64(q, lat, lens, o64, B, q_len, H, R, P, stride, 0.0721f);
    free(q), free(lat), free(o), free(o64);
}

static void projections(void) {
    const int rows = 2, H = 3, nope = 128, rope = 64, R = 512, vh = 128;
    const int types[3] = {W_F16, W_Q8_0, W_Q4_0};
    for (int t = 0; t < 3; t++) {
        uint8_t* wk = weights(10 + t, types[t], H * nope, R);
        uint8_t* wv = weights(20 + t, types[t], H * vh, R);
        float* q = randf(30, (int64_t)rows * H * (nope + rope));
        float* qa = (float*)malloc(sizeof(float) * rows * H * (R + rope));
        oracle_mla_absorb(q, wk, types[t], qa, rows, H, nope, rope, R);
        float* o = randf(31, (int64_t)rows * H * R);
        float* out = (float*)malloc(sizeof(float) * rows * H * vh);
        oracle_mla_project(o, wv, types[t], out, rows, H, R, vh);
        float* row = (float*)malloc(sizeof(float) * R);
        oracle_dequant_row(wk, types[t], H * nope - 1, R, row); /* the last row */
        free(wk), free(wv), free(q), free(qa), free(o), free(out), free(row);
    }
}

static void latent(void) {
    const int R = 512, P = 64, maxT = 9, n_seq = 2, rps = 3;
    float* freqs = (float*)malloc(sizeof(float) * P / 2);
    for (int i = 0; i < P / 2; i++) freqs[i] = oracle_yarn_rope_freq(i, P, 40.f, 4096, 10000.f);
    (void)oracle_yarn_rope_freq(0, P, 0.f, 0, 10000.f);
    uint16_t* norm = rand_f16_bits(40, R);
    uint16_t* kva = rand_f16_bits(41, (int64_t)n_seq * rps * (R + P));
    uint16_t* cache = (uint16_t*)calloc((size_t)n_seq * maxT * (R + P), 2);
    const int32_t pos[6] = {0, 1, 2, 6, 7, 8}; /* sequence 1's rows end at the cache's last slot */
    oracle_mla_latent_write(kva, norm, pos, cache, n_seq * rps, rps, (int64_t)maxT * (R + P), maxT, R, P, 1e-6f,
                            freqs);
    uint16_t* one = rand_f16_bits(42, R + P);
    oracle_mla_kv_prepare(one, norm, R, P, 1e-6f, 5, freqs);
    oracle_rope_neox_f16(one + R, P, 3, freqs);
    free(freqs), free(norm), free(kva), free(cache), free(one);
}

static void q4(void) {
    const int vpt = 96, T = 11, n_q4 = 7;
    uint16_t* x = rand_f16_bits(50, (int64_t)T * vpt);
    uint16_t* out = (uint16_t*)malloc((size_t)T * vpt * 2);
    oracle_kvq4_read(x, out, T, vpt, n_q4);
    uint8_t* g = (uint8_t*)malloc(20);
    uint16_t* d = (uint16_t*)malloc(64);
    oracle_q4_quantize_group(x, g, 7); /* a partial group */
    oracle_q4_dequantize_group(g, d);
    uint8_t* tok = (uint8_t*)malloc((size_t)vpt / 32 * 20);
    oracle_q4_quantize_token(x, tok, vpt);
    oracle_q4_dequantize_token(tok, out, vpt);
    uint16_t* dst = (uint16_t*)calloc(64, 2);
    oracle_scatter_kv(x, dst, 60, 4); /* the destination's last four elements */
    free(x), free(out), free(g), free(d), free(tok), free(dst);
}

static void conversions(void) {
    float f[6] = {0.f, -0.f, 65504.f, 1e-8f, 3.3e38f, -2.5f};
    uint16_t b[6];
    oracle_round_to_dtype(f, b, 6, BF16);
    oracle_round_to_dtype(f, b, 6, F16);
    for (int i = 0; i < 6; i++) (void)oracle_bf16_to_f32(oracle_f32_to_bf16(f[i])), (void)oracle_f16_to_f32(b[i]);
    (void)oracle_mt64_first(42, 1000);
    int32_t r[16];
    oracle_randint(3, 16, -5, 5, r);
    (void)oracle_num_threads();
}

int main(void) {
    conversions();
    gqa();
    prefill();
    mla();
    projections();
    latent();
    q4();
    printf("PASS\n");
    return 0;
}
