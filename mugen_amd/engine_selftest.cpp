// engine_selftest.cpp -- checks the C++ attention provider
// (include/mugen_attn_engine.hpp) on the GPU: a multi-layer decode loop run
// eagerly and the same loop replayed from one captured StepGraph must give
// bit-identical outputs at every step (same kernels, same inputs), while the
// device-side lengths advance by one per step inside the graph (q_len per
// step for an MLA verify step).  A prompt chunk through prefill_layer is
// checked against a direct causal prefill over the same context, and the
// 4-bit store provider's replayed steps against eager ones.
//
// Built by mugen_amd/build.py next to libmugen_attn.so; run by
// tests/test_engine_gpu.py.  Prints PASS / FAIL lines; exit status 0 only
// if every check passed.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "mugen_attn_engine.hpp"

namespace {

using mugen_attn::Status;

// deterministic inputs: splitmix64 -> uniform in [-a, a) -> f16 bits
struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed) {}
    uint64_t next() {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    float uni(float a) { return a * (2.0f * (float)((next() >> 40) * (1.0 / 16777216.0)) - 1.0f); }
};

std::vector<uint16_t> f16_rand(Rng& r, size_t n, float a) {
    std::vector<uint16_t> v(n);
    for (auto& x : v) {
        _Float16 h = (_Float16)r.uni(a);
        std::memcpy(&x, &h, 2);
    }
    return v;
}

// bf16 values (round to nearest even) of uniform draws in [-a, a]
std::vector<uint16_t> bf16_rand(Rng& r, size_t n, float a) {
    std::vector<uint16_t> v(n);
    for (auto& x : v) {
        const float f = r.uni(a);
        uint32_t u;
        std::memcpy(&u, &f, 4);
        u += 0x7fffu + ((u >> 16) & 1u);
        x = (uint16_t)(u >> 16);
    }
    return v;
}

int failures = 0;

bool ok(const Status& st, const char* what) {
    if (st) return true;
    std::printf("FAIL %s: %s\n", what, st.error().c_str());
    failures++;
    return false;
}

bool hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    std::printf("FAIL %s: %s\n", what, hipGetErrorString(e));
    failures++;
    return false;
}

struct Dev {
    void* p = nullptr;
    size_t n = 0;
    explicit Dev(size_t bytes) : n(bytes) { hip(hipMalloc(&p, bytes), "hipMalloc"); }
    ~Dev() { (void)hipFree(p); }
    void put(const void* h, hipStream_t st) { hip(hipMemcpyAsync(p, h, n, hipMemcpyHostToDevice, st), "upload"); }
    std::vector<uint8_t> get(hipStream_t st) const {
        std::vector<uint8_t> h(n);
        hip(hipMemcpyAsync(h.data(), p, n, hipMemcpyDeviceToHost, st), "download");
        hip(hipStreamSynchronize(st), "sync");
        return h;
    }
};

bool finite_bf16(const std::vector<uint8_t>& b) {
    for (size_t i = 0; i + 1 < b.size(); i += 2) {
        uint16_t x;
        std::memcpy(&x, &b[i], 2);
        if ((x & 0x7f80u) == 0x7f80u) return false;
    }
    return true;
}

bool finite_f16(const std::vector<uint8_t>& b) {
    for (size_t i = 0; i + 1 < b.size(); i += 2) {
        uint16_t x;
        std::memcpy(&x, &b[i], 2);
        if ((x & 0x7c00u) == 0x7c00u) return false;
    }
    return true;
}

void check_lengths(const int32_t* dev_after, const std::vector<int32_t>& want, hipStream_t st, const char* what) {
    std::vector<int32_t> got(want.size());
    hip(hipMemcpyAsync(got.data(), dev_after, sizeof(int32_t) * got.size(), hipMemcpyDeviceToHost, st), "lengths");
    hip(hipStreamSynchronize(st), "sync");
    if (got != want) {
        std::printf("FAIL %s: device lengths", what);
        for (size_t i = 0; i < got.size(); i++) std::printf(" %d/%d", got[i], want[i]);
        std::printf("\n");
        failures++;
    }
}

// ---------------------------------------------------------------- GQA

void gqa_test(hipStream_t st) {
    mugen_attn::GqaShape s;
    s.n_layers = 3;
    s.batch = 3;
    s.n_heads = 28;
    s.n_kv_heads = 4;
    s.head_dim = 128;
    s.max_seq_len = 1024;
    const std::vector<int32_t> lens0 = {700, 1, 300};
    const int steps = 5;
    std::printf("gqa provider: layers %d batch %d H %d Hk %d d %d steps %d\n", s.n_layers, s.batch, s.n_heads,
                s.n_kv_heads, s.head_dim, steps);
    std::fflush(stdout);
    std::unique_ptr<mugen_attn::GqaAttention> eager, graphed;
    if (!ok(mugen_attn::GqaAttention::create(s, &eager), "create eager")) return;
    if (!ok(mugen_attn::GqaAttention::create(s, &graphed), "create graphed")) return;
    const size_t row = (size_t)s.n_kv_heads * s.head_dim;
    const size_t cache = (size_t)s.batch * s.max_seq_len * row * 2;
    Rng r(1);
    for (int L = 0; L < s.n_layers; L++) {  // the context already held
        auto k = f16_rand(r, cache / 2, 1.0f);
        auto v = f16_rand(r, cache / 2, 1.0f);
        for (auto* a : {eager.get(), graphed.get()}) {
            hip(hipMemcpyAsync(a->k_cache(L), k.data(), cache, hipMemcpyHostToDevice, st), "K init");
            hip(hipMemcpyAsync(a->v_cache(L), v.data(), cache, hipMemcpyHostToDevice, st), "V init");
        }
        hip(hipStreamSynchronize(st), "sync");
    }
    ok(eager->set_lengths(lens0, st), "eager lengths");
    ok(graphed->set_lengths(lens0, st), "graphed lengths");
    // fixed per-layer input / output buffers (the graph captures their addresses)
    std::vector<std::unique_ptr<Dev>> q, kn, vn, oe, og;
    const size_t qb = (size_t)s.batch * s.n_heads * s.head_dim * 2, kb = (size_t)s.batch * row * 2;
    for (int L = 0; L < s.n_layers; L++) {
        q.emplace_back(new Dev(qb));
        kn.emplace_back(new Dev(kb));
        vn.emplace_back(new Dev(kb));
        oe.emplace_back(new Dev(qb));
        og.emplace_back(new Dev(qb));
    }
    mugen_attn::StepGraph graph;
    auto body = [&](hipStream_t str) -> Status {
        for (int L = 0; L < s.n_layers; L++)
            if (auto rr = graphed->decode_layer(L, q[L]->p, kn[L]->p, vn[L]->p, og[L]->p, str); !rr) return rr;
        return graphed->advance(str);
    };
    if (!ok(graph.capture(st, body), "capture")) return;
    for (int step = 0; step < steps; step++) {
        Rng ri(100 + step);
        for (int L = 0; L < s.n_layers; L++) {  // the step's new inputs, uploaded outside the graph
            auto hq = f16_rand(ri, qb / 2, 1.0f), hk = f16_rand(ri, kb / 2, 1.0f), hv = f16_rand(ri, kb / 2, 1.0f);
            q[L]->put(hq.data(), st);
            kn[L]->put(hk.data(), st);
            vn[L]->put(hv.data(), st);
            hip(hipStreamSynchronize(st), "sync");
        }
        for (int L = 0; L < s.n_layers; L++)
            ok(eager->decode_layer(L, q[L]->p, kn[L]->p, vn[L]->p, oe[L]->p, st), "eager decode");
        ok(eager->advance(st), "eager advance");
        hip(hipStreamSynchronize(st), "sync");
        ok(graph.replay(st), "replay");
        hip(hipStreamSynchronize(st), "sync");
        for (int L = 0; L < s.n_layers; L++) {
            const auto a = oe[L]->get(st), b = og[L]->get(st);
            if (a != b || !finite_f16(a)) {
                std::printf("FAIL gqa step %d layer %d: graph replay differs from the eager call\n", step, L);
                failures++;
            }
        }
        std::vector<int32_t> want(lens0);  // the next step's post-append lengths
        for (auto& x : want) x += step + 2;
        check_lengths(eager->lengths_after(), want, st, "gqa eager");
        check_lengths(graphed->lengths_after(), want, st, "gqa graphed");
    }
    std::printf("gqa provider done\n");
}

// ---------------------------------------------------------------- MLA

void mla_test(hipStream_t st, int q_len) {
    mugen_attn::MlaShape s;
    s.n_layers = 2;
    s.batch = 2;
    s.n_heads = 16;
    s.max_seq_len = 512;
    s.q_len = q_len;
    s.rope = mugen_attn_rope_params{10000.f, 40.f, 4096};
    const std::vector<int32_t> lens0 = {300, 5};
    const int steps = 4;
    std::printf("mla provider: layers %d batch %d H %d q_len %d steps %d\n", s.n_layers, s.batch, s.n_heads, q_len,
                steps);
    std::fflush(stdout);
    std::unique_ptr<mugen_attn::MlaAttention> eager, graphed;
    if (!ok(mugen_attn::MlaAttention::create(s, &eager), "create eager")) return;
    if (!ok(mugen_attn::MlaAttention::create(s, &graphed), "create graphed")) return;
    Rng r(2);
    const size_t lat = (size_t)s.batch * s.max_seq_len * 576 * 2;
    std::vector<std::unique_ptr<Dev>> norm, wkb, wvb;
    std::vector<mugen_attn::MlaLayerWeights> w(s.n_layers);
    for (int L = 0; L < s.n_layers; L++) {
        auto c = f16_rand(r, lat / 2, 0.5f);
        for (auto* a : {eager.get(), graphed.get()})
            hip(hipMemcpyAsync(a->latent(L), c.data(), lat, hipMemcpyHostToDevice, st), "latent init");
        auto hn = f16_rand(r, 512, 0.2f);
        for (auto& x : hn) {  // weights near 1
            _Float16 h;
            std::memcpy(&h, &x, 2);
            h = (_Float16)(1.0f + (float)h);
            std::memcpy(&x, &h, 2);
        }
        auto hk = f16_rand(r, (size_t)s.n_heads * 128 * 512, 0.08f), hv = f16_rand(r, (size_t)s.n_heads * 128 * 512, 0.08f);
        norm.emplace_back(new Dev(512 * 2));
        wkb.emplace_back(new Dev(hk.size() * 2));
        wvb.emplace_back(new Dev(hv.size() * 2));
        norm[L]->put(hn.data(), st);
        wkb[L]->put(hk.data(), st);
        wvb[L]->put(hv.data(), st);
        hip(hipStreamSynchronize(st), "sync");
        w[L].kv_a_norm = norm[L]->p;
        w[L].w_kb = wkb[L]->p;
        w[L].w_vb = wvb[L]->p;
        w[L].w_type = MUGEN_ATTN_W_F16;
    }
    ok(eager->set_lengths(lens0, st), "eager lengths");
    ok(graphed->set_lengths(lens0, st), "graphed lengths");
    std::vector<std::unique_ptr<Dev>> q, kva, oe, og;
    const size_t rows = (size_t)s.batch * q_len;
    const size_t qb = rows * s.n_heads * 192 * 2, kb = rows * 576 * 2, ob = rows * s.n_heads * 128 * 2;
    for (int L = 0; L < s.n_layers; L++) {
        q.emplace_back(new Dev(qb));
        kva.emplace_back(new Dev(kb));
        oe.emplace_back(new Dev(ob));
        og.emplace_back(new Dev(ob));
    }
    mugen_attn::StepGraph graph;
    auto body = [&](hipStream_t str) -> Status {
        for (int L = 0; L < s.n_layers; L++)
            if (auto rr = graphed->decode_layer(L, w[L], q[L]->p, kva[L]->p, og[L]->p, str); !rr) return rr;
        return graphed->advance(str, q_len);
    };
    if (!ok(graph.capture(st, body), "capture")) return;
    for (int step = 0; step < steps; step++) {
        Rng ri(200 + step);
        for (int L = 0; L < s.n_layers; L++) {
            auto hq = f16_rand(ri, qb / 2, 1.0f), hk = f16_rand(ri, kb / 2, 1.0f);
            q[L]->put(hq.data(), st);
            kva[L]->put(hk.data(), st);
            hip(hipStreamSynchronize(st), "sync");
        }
        for (int L = 0; L < s.n_layers; L++)
            ok(eager->decode_layer(L, w[L], q[L]->p, kva[L]->p, oe[L]->p, st), "eager decode");
        ok(eager->advance(st, q_len), "eager advance");
        hip(hipStreamSynchronize(st), "sync");
        ok(graph.replay(st), "replay");
        hip(hipStreamSynchronize(st), "sync");
        for (int L = 0; L < s.n_layers; L++) {
            const auto a = oe[L]->get(st), b = og[L]->get(st);
            if (a != b || !finite_f16(a)) {
                std::printf("FAIL mla step %d layer %d: graph replay differs from the eager call\n", step, L);
                failures++;
            }
            // the latent rows written this step agree as well
            std::vector<uint8_t> le(lat), lg(lat);
            hip(hipMemcpyAsync(le.data(), eager->latent(L), lat, hipMemcpyDeviceToHost, st), "latent");
            hip(hipMemcpyAsync(lg.data(), graphed->latent(L), lat, hipMemcpyDeviceToHost, st), "latent");
            hip(hipStreamSynchronize(st), "sync");
            if (le != lg) {
                std::printf("FAIL mla step %d layer %d: latent caches differ\n", step, L);
                failures++;
            }
        }
        std::vector<int32_t> want(lens0);  // the next step's post-append lengths
        for (auto& x : want) x += q_len * (step + 2);
        check_lengths(eager->lengths_after(), want, st, "mla eager");
        check_lengths(graphed->lengths_after(), want, st, "mla graphed");
    }
    std::printf("mla provider done\n");
}

// ---------------------------------------------------------------- GQA, 4-bit store

float max_abs_diff_f16(const std::vector<uint8_t>& a, const std::vector<uint8_t>& b) {
    float m = 0.f;
    for (size_t i = 0; i + 1 < a.size(); i += 2) {
        _Float16 x, y;
        std::memcpy(&x, &a[i], 2);
        std::memcpy(&y, &b[i], 2);
        m = std::max(m, std::fabs((float)x - (float)y));
    }
    return m;
}

// A context appended in chunks, then decode steps eager and replayed from
// one captured graph (bit-identical, lengths and quantised counts advancing
// on the device); a store that quantises nothing (preserve >= length) must
// agree with the f16 provider fed the same tokens.
void gqa_q4_test(hipStream_t st) {
    mugen_attn::GqaQ4Shape s;
    s.n_layers = 2;
    s.batch = 2;
    s.n_heads = 28;
    s.n_kv_heads = 4;
    s.head_dim = 128;
    s.max_seq_len = 512;
    s.fp16_preserve_last = 16;
    s.max_new = 32;
    const std::vector<int32_t> lens0 = {0, 5};
    const int chunks = 3, steps = 4;
    std::printf("gqa q4 provider: layers %d batch %d preserve %d chunks %d steps %d\n", s.n_layers, s.batch,
                s.fp16_preserve_last, chunks, steps);
    std::fflush(stdout);
    mugen_attn::GqaQ4Shape s_wide = s;  // nothing quantised: compared with the f16 provider
    s_wide.fp16_preserve_last = 256;
    mugen_attn::GqaShape sf;
    sf.n_layers = s.n_layers;
    sf.batch = s.batch;
    sf.n_heads = s.n_heads;
    sf.n_kv_heads = s.n_kv_heads;
    sf.head_dim = s.head_dim;
    sf.max_seq_len = s.max_seq_len;
    std::unique_ptr<mugen_attn::GqaAttentionQ4> eager, graphed, wide;
    std::unique_ptr<mugen_attn::GqaAttention> f16;
    if (!ok(mugen_attn::GqaAttentionQ4::create(s, &eager), "create eager")) return;
    if (!ok(mugen_attn::GqaAttentionQ4::create(s, &graphed), "create graphed")) return;
    if (!ok(mugen_attn::GqaAttentionQ4::create(s_wide, &wide), "create wide")) return;
    if (!ok(mugen_attn::GqaAttention::create(sf, &f16), "create f16")) return;
    for (auto* a : {eager.get(), graphed.get(), wide.get()}) ok(a->set_lengths(lens0, st), "q4 lengths");
    ok(f16->set_lengths(lens0, st), "f16 lengths");
    const size_t row = (size_t)s.n_kv_heads * s.head_dim;
    Rng r(4);
    {   // the context: chunks of max_new tokens per sequence, every layer
        Dev kc((size_t)s.batch * s.max_new * row * 2), vc((size_t)s.batch * s.max_new * row * 2);
        Dev k1((size_t)s.max_new * row * 2), v1((size_t)s.max_new * row * 2);
        for (int c = 0; c < chunks; c++) {
            for (int L = 0; L < s.n_layers; L++) {
                auto hk = f16_rand(r, kc.n / 2, 1.0f), hv = f16_rand(r, vc.n / 2, 1.0f);
                kc.put(hk.data(), st);
                vc.put(hv.data(), st);
                for (auto* a : {eager.get(), graphed.get(), wide.get()})
                    ok(a->append_layer(L, kc.p, vc.p, s.max_new, st), "q4 append");
                // the f16 provider takes the same rows (sequence-major [batch][n_new][row])
                mugen_attn_kv_append_args ap{};
                ap.k_new = kc.p;
                ap.v_new = vc.p;
                ap.k_cache = f16->k_cache(L);
                ap.v_cache = f16->v_cache(L);
                ap.seq_lens = f16->lengths_after() - s.batch;
                ap.seq_stride = (int64_t)s.max_seq_len * row;
                ap.n_seq = s.batch;
                ap.n_new = s.max_new;
                ap.row = (int)row;
                ap.max_seq_len = s.max_seq_len;
                ok(mugen_attn::kv_append(ap, st), "f16 append");
                hip(hipStreamSynchronize(st), "sync");
            }
            for (auto* a : {eager.get(), graphed.get(), wide.get()}) ok(a->advance(st, s.max_new), "q4 advance");
            ok(f16->advance(st, s.max_new), "f16 advance");
        }
    }
    std::vector<std::unique_ptr<Dev>> q, kn, vn, oe, og, ow, of;
    const size_t qb = (size_t)s.batch * s.n_heads * s.head_dim * 2, kb = (size_t)s.batch * row * 2;
    for (int L = 0; L < s.n_layers; L++) {
        q.emplace_back(new Dev(qb));
        kn.emplace_back(new Dev(kb));
        vn.emplace_back(new Dev(kb));
        oe.emplace_back(new Dev(qb));
        og.emplace_back(new Dev(qb));
        ow.emplace_back(new Dev(qb));
        of.emplace_back(new Dev(qb));
    }
    mugen_attn::StepGraph graph;
    auto body = [&](hipStream_t str) -> Status {
        for (int L = 0; L < s.n_layers; L++)
            if (auto rr = graphed->decode_layer(L, q[L]->p, kn[L]->p, vn[L]->p, og[L]->p, str); !rr) return rr;
        return graphed->advance(str);
    };
    if (!ok(graph.capture(st, body), "q4 capture")) return;
    for (int step = 0; step < steps; step++) {
        Rng ri(300 + step);
        for (int L = 0; L < s.n_layers; L++) {
            auto hq = f16_rand(ri, qb / 2, 1.0f), hk = f16_rand(ri, kb / 2, 1.0f), hv = f16_rand(ri, kb / 2, 1.0f);
            q[L]->put(hq.data(), st);
            kn[L]->put(hk.data(), st);
            vn[L]->put(hv.data(), st);
            hip(hipStreamSynchronize(st), "sync");
        }
        for (int L = 0; L < s.n_layers; L++) {
            ok(eager->decode_layer(L, q[L]->p, kn[L]->p, vn[L]->p, oe[L]->p, st), "q4 eager decode");
            ok(wide->decode_layer(L, q[L]->p, kn[L]->p, vn[L]->p, ow[L]->p, st), "q4 wide decode");
            ok(f16->decode_layer(L, q[L]->p, kn[L]->p, vn[L]->p, of[L]->p, st), "f16 decode");
        }
        ok(eager->advance(st), "q4 eager advance");
        ok(wide->advance(st), "q4 wide advance");
        ok(f16->advance(st), "f16 advance");
        hip(hipStreamSynchronize(st), "sync");
        ok(graph.replay(st), "q4 replay");
        hip(hipStreamSynchronize(st), "sync");
        for (int L = 0; L < s.n_layers; L++) {
            const auto a = oe[L]->get(st), b = og[L]->get(st), w = ow[L]->get(st), f = of[L]->get(st);
            if (a != b || !finite_f16(a)) {
                std::printf("FAIL gqa q4 step %d layer %d: graph replay differs from the eager call\n", step, L);
                failures++;
            }
            const float d = max_abs_diff_f16(w, f);
            if (!(d <= 2e-3f)) {
                std::printf("FAIL gqa q4 step %d layer %d: unquantised store vs f16 provider max-abs %g\n", step, L,
                            d);
                failures++;
            }
        }
        std::vector<int32_t> want(lens0), wq4;
        for (auto& x : want) x += chunks * s.max_new + step + 2;
        check_lengths(eager->lengths_after(), want, st, "gqa q4 eager");
        check_lengths(graphed->lengths_after(), want, st, "gqa q4 graphed");
        for (int32_t x : want) wq4.push_back(std::max(0, x - 1 - s.fp16_preserve_last));
        check_lengths(graphed->quantised(), wq4, st, "gqa q4 quantised counts");
    }
    std::printf("gqa q4 provider done\n");
}

// ---------------------------------------------------------------- GQA prefill

// A prompt chunk appended to a held context through prefill_layer: the cache
// rows [start, start + N) must hold the chunk's K / V, and the output must be
// the causal prefill over context + chunk computed directly from a buffer
// assembled on the host; afterwards a decode step continues from start + N.
// With BF16 caches and a chunk of 1024+ tokens the provider hands the
// library its prefill workspace (the one-launch fp16 copy of V), while the
// direct call passes none (the kernels convert V on chip): both must agree
// bit for bit.  A short chunk after a long context (`direct_ws`): the
// provider's workspace holds the split key ranges' partials, and the direct
// call passes a workspace of the size the library asks for, so both split
// the same way and agree bit for bit.
void gqa_prefill_test(hipStream_t st, int dtype, int start, int n, int max_seq, bool direct_ws = false,
                      int n_heads = 32, int n_kv_heads = 8) {
    mugen_attn::GqaShape s;
    s.n_layers = 1;
    s.batch = 1;
    s.n_heads = n_heads;
    s.n_kv_heads = n_kv_heads;
    s.head_dim = 128;
    s.max_seq_len = max_seq;
    s.kv_dtype = dtype;
    s.out_dtype = dtype;
    auto rand16 = [&](Rng& rr, size_t cnt, float a) {
        return dtype == MUGEN_ATTN_BF16 ? bf16_rand(rr, cnt, a) : f16_rand(rr, cnt, a);
    };
    std::printf("gqa prefill provider: %s H %d Hk %d d %d start %d chunk %d\n",
                dtype == MUGEN_ATTN_BF16 ? "bf16" : "f16", s.n_heads, s.n_kv_heads, s.head_dim, start, n);
    std::fflush(stdout);
    std::unique_ptr<mugen_attn::GqaAttention> a;
    if (!ok(mugen_attn::GqaAttention::create(s, &a), "create")) return;
    const size_t row = (size_t)s.n_kv_heads * s.head_dim, cache = (size_t)s.max_seq_len * row * 2;
    Rng r(3);
    auto k = rand16(r, cache / 2, 1.0f), v = rand16(r, cache / 2, 1.0f);
    hip(hipMemcpyAsync(a->k_cache(0), k.data(), cache, hipMemcpyHostToDevice, st), "K init");
    hip(hipMemcpyAsync(a->v_cache(0), v.data(), cache, hipMemcpyHostToDevice, st), "V init");
    ok(a->set_lengths({start}, st), "lengths");
    const size_t qb = (size_t)n * s.n_heads * s.head_dim * 2, kb = (size_t)n * row * 2;
    auto hq = rand16(r, qb / 2, 1.0f), hk = rand16(r, kb / 2, 1.0f), hv = rand16(r, kb / 2, 1.0f);
    Dev q(qb), kn(kb), vn(kb), out(qb), ref(qb), kc((size_t)(start + n) * row * 2), vc((size_t)(start + n) * row * 2);
    q.put(hq.data(), st);
    kn.put(hk.data(), st);
    vn.put(hv.data(), st);
    // the context + chunk, assembled on the host
    std::vector<uint16_t> kall(k.begin(), k.begin() + (size_t)start * row), vall(v.begin(), v.begin() + (size_t)start * row);
    kall.insert(kall.end(), hk.begin(), hk.end());
    vall.insert(vall.end(), hv.begin(), hv.end());
    kc.put(kall.data(), st);
    vc.put(vall.data(), st);
    hip(hipStreamSynchronize(st), "sync");
    ok(a->prefill_layer(0, q.p, kn.p, vn.p, out.p, n, st), "prefill_layer");
    mugen_attn_gqa_prefill_args pf{};
    pf.q = q.p;
    pf.k = kc.p;
    pf.v = vc.p;
    pf.out = ref.p;
    pf.n_tokens = n;
    pf.n_heads = s.n_heads;
    pf.n_kv_heads = s.n_kv_heads;
    pf.head_dim = s.head_dim;
    pf.kv_len = start + n;
    pf.start_pos = start;
    pf.causal = 1;
    pf.dtype = dtype;
    pf.out_dtype = dtype;
    std::unique_ptr<Dev> ws;
    if (direct_ws) {
        const size_t need = mugen_attn_gqa_prefill_workspace_size(&pf);
        if (need == 0) {
            std::printf("FAIL gqa prefill: no split planned for a %d-token chunk after %d\n", n, start);
            failures++;
        } else {
            ws = std::make_unique<Dev>(need);
            pf.workspace = ws->p;
            pf.workspace_bytes = need;
        }
    }
    ok(mugen_attn::gqa_prefill(pf, st), "direct prefill");
    const auto o = out.get(st), o_ref = ref.get(st);
    if (o != o_ref || !(dtype == MUGEN_ATTN_BF16 ? finite_bf16(o) : finite_f16(o))) {
        std::printf("FAIL gqa prefill: provider output differs from the direct prefill\n");
        failures++;
    }
    std::vector<uint16_t> kgot(cache / 2), vgot(cache / 2);
    hip(hipMemcpyAsync(kgot.data(), a->k_cache(0), cache, hipMemcpyDeviceToHost, st), "K read");
    hip(hipMemcpyAsync(vgot.data(), a->v_cache(0), cache, hipMemcpyDeviceToHost, st), "V read");
    hip(hipStreamSynchronize(st), "sync");
    if (!std::equal(kall.begin(), kall.end(), kgot.begin()) || !std::equal(vall.begin(), vall.end(), vgot.begin()) ||
        !std::equal(k.begin() + kall.size(), k.end(), kgot.begin() + kall.size())) {
        std::printf("FAIL gqa prefill: cache rows not where the chunk belongs\n");
        failures++;
    }
    ok(a->advance(st, n), "advance");
    check_lengths(a->lengths_after(), {start + n + 1}, st, "gqa prefill");
    std::printf("gqa prefill provider done\n");
}


// ---------------------------------------------------------------- prompts in a batch

// A prompt for sequence 1 of a batch of 2 through GqaAttention and through
// GqaAttentionQ4 (whose prefill attends over its f16 caches, as the
// reference's prefill does whichever path decodes): both equal a direct
// prefill over the assembled context, sequence 0 is untouched, and the
// lengths advance for sequence 1 only.
void prefill_batch_test(hipStream_t st) {
    mugen_attn::GqaShape s;
    s.n_layers = 1;
    s.batch = 2;
    s.n_heads = 28;
    s.n_kv_heads = 4;
    s.head_dim = 128;
    s.max_seq_len = 512;
    mugen_attn::GqaQ4Shape s4;
    s4.n_layers = 1;
    s4.batch = 2;
    s4.n_heads = 28;
    s4.n_kv_heads = 4;
    s4.head_dim = 128;
    s4.max_seq_len = 512;
    s4.fp16_preserve_last = 16;
    s4.max_new = 64;
    const int n = 48, chunks = 3;
    std::printf("prompt in a batch: H %d Hk %d d %d, %d chunks of %d for sequence 1\n", s.n_heads, s.n_kv_heads,
                s.head_dim, chunks, n);
    std::fflush(stdout);
    std::unique_ptr<mugen_attn::GqaAttention> a;
    std::unique_ptr<mugen_attn::GqaAttentionQ4> a4;
    if (!ok(mugen_attn::GqaAttention::create(s, &a), "create")) return;
    if (!ok(mugen_attn::GqaAttentionQ4::create(s4, &a4), "create q4")) return;
    const size_t row = (size_t)s.n_kv_heads * s.head_dim;
    const size_t seq_bytes = (size_t)s.max_seq_len * row * 2;
    Rng r(7);
    auto k0 = f16_rand(r, seq_bytes / 2, 1.0f), v0 = f16_rand(r, seq_bytes / 2, 1.0f);  // sequence 0's cache
    hip(hipMemcpyAsync(a->k_cache(0), k0.data(), seq_bytes, hipMemcpyHostToDevice, st), "K0");
    hip(hipMemcpyAsync(a->v_cache(0), v0.data(), seq_bytes, hipMemcpyHostToDevice, st), "V0");
    ok(a->set_lengths({100, 0}, st), "lengths");
    ok(a4->set_lengths({0, 0}, st), "q4 lengths");
    const size_t qb = (size_t)n * s.n_heads * s.head_dim * 2, kb = (size_t)n * row * 2;
    Dev q(qb), kn(kb), vn(kb), out(qb), out4(qb), ref(qb), kc((size_t)chunks * n * row * 2),
        vc((size_t)chunks * n * row * 2);
    std::vector<uint16_t> kall, vall;
    for (int c = 0; c < chunks; c++) {
        auto hq = f16_rand(r, qb / 2, 1.0f), hk = f16_rand(r, kb / 2, 1.0f), hv = f16_rand(r, kb / 2, 1.0f);
        q.put(hq.data(), st);
        kn.put(hk.data(), st);
        vn.put(hv.data(), st);
        kall.insert(kall.end(), hk.begin(), hk.end());
        vall.insert(vall.end(), hv.begin(), hv.end());
        hip(hipStreamSynchronize(st), "sync");
        ok(a->prefill_layer(0, 1, q.p, kn.p, vn.p, out.p, n, st), "prefill_layer seq 1");
        ok(a4->prefill_layer(0, 1, q.p, kn.p, vn.p, out4.p, n, st), "q4 prefill_layer seq 1");
        // direct prefill over the context so far
        hip(hipMemcpyAsync(kc.p, kall.data(), kall.size() * 2, hipMemcpyHostToDevice, st), "kc");
        hip(hipMemcpyAsync(vc.p, vall.data(), vall.size() * 2, hipMemcpyHostToDevice, st), "vc");
        mugen_attn_gqa_prefill_args pf{};
        pf.q = q.p;
        pf.k = kc.p;
        pf.v = vc.p;
        pf.out = ref.p;
        pf.n_tokens = n;
        pf.n_heads = s.n_heads;
        pf.n_kv_heads = s.n_kv_heads;
        pf.head_dim = s.head_dim;
        pf.kv_len = (c + 1) * n;
        pf.start_pos = c * n;
        pf.causal = 1;
        pf.dtype = MUGEN_ATTN_F16;
        pf.out_dtype = MUGEN_ATTN_F16;
        ok(mugen_attn::gqa_prefill(pf, st), "direct prefill");
        const auto o = out.get(st), o4 = out4.get(st), o_ref = ref.get(st);
        if (o != o_ref || o4 != o_ref || !finite_f16(o)) {
            std::printf("FAIL prompt chunk %d: provider outputs differ from the direct prefill\n", c);
            failures++;
        }
        ok(a->advance_sequence(1, n, st), "advance_sequence");
        ok(a4->advance_sequence(1, n, st), "q4 advance_sequence");
    }
    std::vector<uint16_t> kgot(seq_bytes / 2);
    hip(hipMemcpyAsync(kgot.data(), a->k_cache(0), seq_bytes, hipMemcpyDeviceToHost, st), "K0 read");
    hip(hipStreamSynchronize(st), "sync");
    if (kgot != k0) {
        std::printf("FAIL prompt in a batch: sequence 0's cache changed\n");
        failures++;
    }
    check_lengths(a->lengths_after(), {101, chunks * n + 1}, st, "prompt in a batch");
    check_lengths(a4->lengths_after(), {1, chunks * n + 1}, st, "q4 prompt in a batch");
    // the store quantised what left its f16 window (preserve 16)
    check_lengths(a4->quantised(), {0, chunks * n - s4.fp16_preserve_last}, st, "q4 quantised count");
    std::printf("prompt in a batch done\n");
}

// MLA prompt: one prefill_layer call over n tokens equals the reference's
// token-by-token path (n decode steps of q_len 1): the same latent rows,
// outputs within the parity tolerance.
void mla_prefill_test(hipStream_t st) {
    mugen_attn::MlaShape s;
    s.n_layers = 1;
    s.batch = 1;
    s.n_heads = 16;
    s.max_seq_len = 256;
    s.q_len = 1;
    s.max_prefill = 64;
    s.rope = mugen_attn_rope_params{10000.f, 40.f, 4096};
    const int start = 20, n = 40;
    std::printf("mla prompt: H %d start %d n %d\n", s.n_heads, start, n);
    std::fflush(stdout);
    std::unique_ptr<mugen_attn::MlaAttention> pre, step;
    if (!ok(mugen_attn::MlaAttention::create(s, &pre), "create prefill")) return;
    if (!ok(mugen_attn::MlaAttention::create(s, &step), "create stepwise")) return;
    Rng r(9);
    const size_t lat = (size_t)s.max_seq_len * 576 * 2;
    auto c = f16_rand(r, lat / 2, 0.5f);
    for (auto* a : {pre.get(), step.get()})
        hip(hipMemcpyAsync(a->latent(0), c.data(), lat, hipMemcpyHostToDevice, st), "latent init");
    auto hn = f16_rand(r, 512, 0.2f);
    for (auto& x : hn) {
        _Float16 h;
        std::memcpy(&h, &x, 2);
        h = (_Float16)(1.0f + (float)h);
        std::memcpy(&x, &h, 2);
    }
    auto hk = f16_rand(r, (size_t)s.n_heads * 128 * 512, 0.08f), hv = f16_rand(r, (size_t)s.n_heads * 128 * 512, 0.08f);
    Dev norm(512 * 2), wkb(hk.size() * 2), wvb(hv.size() * 2);
    norm.put(hn.data(), st);
    wkb.put(hk.data(), st);
    wvb.put(hv.data(), st);
    mugen_attn::MlaLayerWeights w;
    w.kv_a_norm = norm.p;
    w.w_kb = wkb.p;
    w.w_vb = wvb.p;
    w.w_type = MUGEN_ATTN_W_F16;
    ok(pre->set_lengths({start}, st), "lengths");
    ok(step->set_lengths({start}, st), "lengths");
    const size_t qrow = (size_t)s.n_heads * 192 * 2, orow = (size_t)s.n_heads * 128 * 2;
    auto hq = f16_rand(r, n * qrow / 2, 1.0f), hkv = f16_rand(r, (size_t)n * 576, 1.0f);
    Dev q(n * qrow), kva((size_t)n * 576 * 2), out(n * orow), q1(qrow), kva1(576 * 2), out1(orow);
    q.put(hq.data(), st);
    kva.put(hkv.data(), st);
    ok(pre->prefill_layer(0, 0, w, q.p, kva.p, out.p, n, st), "prefill_layer");
    ok(pre->advance_sequence(0, n, st), "advance_sequence");
    const auto o_pre = out.get(st);
    float worst = 0.f;
    for (int t = 0; t < n; t++) {
        hip(hipMemcpyAsync(q1.p, hq.data() + t * qrow / 2, qrow, hipMemcpyHostToDevice, st), "q_t");
        hip(hipMemcpyAsync(kva1.p, hkv.data() + (size_t)t * 576, 576 * 2, hipMemcpyHostToDevice, st), "kv_a_t");
        ok(step->decode_layer(0, w, q1.p, kva1.p, out1.p, st), "decode_layer");
        ok(step->advance(st, 1), "advance");
        const auto o1 = out1.get(st);
        std::vector<uint8_t> ot(o_pre.begin() + t * orow, o_pre.begin() + (t + 1) * orow);
        worst = std::max(worst, max_abs_diff_f16(ot, o1));
    }
    if (!(worst <= 2e-3f) || !finite_f16(o_pre)) {
        std::printf("FAIL mla prompt: prefill vs token-by-token max-abs %g\n", worst);
        failures++;
    }
    std::vector<uint8_t> lp(lat), ls(lat);
    hip(hipMemcpyAsync(lp.data(), pre->latent(0), lat, hipMemcpyDeviceToHost, st), "latent");
    hip(hipMemcpyAsync(ls.data(), step->latent(0), lat, hipMemcpyDeviceToHost, st), "latent");
    hip(hipStreamSynchronize(st), "sync");
    if (lp != ls) {
        std::printf("FAIL mla prompt: latent caches differ\n");
        failures++;
    }
    check_lengths(pre->lengths_after(), {start + n + 1}, st, "mla prompt");
    std::printf("mla prompt done (max-abs %g)\n", worst);
}

// Lengths outside the caches are refused (the reference's KVCache::append
// refuses a token once the cache is full), and a new provider starts empty.
void bounds_test(hipStream_t st) {
    std::printf("length bounds\n");
    std::fflush(stdout);
    mugen_attn::GqaShape s;
    s.n_layers = 1;
    s.batch = 1;
    s.n_heads = 8;
    s.n_kv_heads = 2;
    s.head_dim = 64;
    s.max_seq_len = 64;
    std::unique_ptr<mugen_attn::GqaAttention> a;
    if (!ok(mugen_attn::GqaAttention::create(s, &a), "create")) return;
    check_lengths(a->lengths_after(), {1}, st, "fresh provider");
    if (a->set_lengths({64}, st) || a->set_lengths({-1}, st)) {
        std::printf("FAIL bounds: set_lengths accepted a length without room for the step\n");
        failures++;
    }
    ok(a->set_lengths({63}, st), "set_lengths max - 1");
    Dev q(8 * 64 * 2), kn(2 * 64 * 2), vn(2 * 64 * 2), out(8 * 64 * 2);
    ok(a->decode_layer(0, q.p, kn.p, vn.p, out.p, st), "last token");
    ok(a->advance(st), "advance to full");
    if (a->decode_layer(0, q.p, kn.p, vn.p, out.p, st) || a->advance(st)) {
        std::printf("FAIL bounds: a full cache accepted another token\n");
        failures++;
    }
    mugen_attn::MlaShape m;
    m.n_layers = 1;
    m.batch = 2;
    m.n_heads = 16;
    m.max_seq_len = 64;
    m.q_len = 5;
    std::unique_ptr<mugen_attn::MlaAttention> ma;
    if (!ok(mugen_attn::MlaAttention::create(m, &ma), "create mla")) return;
    check_lengths(ma->lengths_after(), {5, 5}, st, "fresh mla provider");
    if (ma->set_lengths({60, 0}, st)) {
        std::printf("FAIL bounds: MLA set_lengths accepted a length without room for q_len tokens\n");
        failures++;
    }
    ok(ma->set_lengths({59, 0}, st), "mla set_lengths max - q_len");
    // prompt chunks shorter than max_prefill get more splits from the
    // planner; the workspace sized at create() serves every chunk length
    mugen_attn::MlaShape p;
    p.n_layers = 1;
    p.batch = 1;
    p.n_heads = 16;
    p.max_seq_len = 8192;
    p.max_prefill = 300;
    std::unique_ptr<mugen_attn::MlaAttention> pa;
    if (!ok(mugen_attn::MlaAttention::create(p, &pa), "create mla prompt provider")) return;
    Dev norm(512 * 2), wk((size_t)16 * 128 * 512 * 2), wv(wk.n), pq((size_t)300 * 16 * 192 * 2), pkv(300 * 576 * 2),
        pout((size_t)300 * 16 * 128 * 2);
    for (Dev* d : {&norm, &wk, &wv, &pq, &pkv}) hip(hipMemsetAsync(d->p, 0, d->n, st), "zero");
    const mugen_attn::MlaLayerWeights w{norm.p, wk.p, wv.p, MUGEN_ATTN_W_F16};
    for (int n : {1, 64, 256, 300})
        if (!ok(pa->prefill_layer(0, 0, w, pq.p, pkv.p, pout.p, n, st), "mla prompt chunk shorter than max_prefill"))
            std::printf("  (chunk of %d tokens)\n", n);
    hip(hipStreamSynchronize(st), "sync");
    std::printf("length bounds done\n");
}

}  // namespace

int main() {
    hipStream_t st;
    if (!hip(hipStreamCreate(&st), "hipStreamCreate")) return 1;
    gqa_test(st);
    mla_test(st, 1);
    mla_test(st, 3);
    gqa_prefill_test(st, MUGEN_ATTN_F16, 200, 77, 1024);
    gqa_prefill_test(st, MUGEN_ATTN_BF16, 100, 1100, 1536);
    gqa_prefill_test(st, MUGEN_ATTN_F16, 7000, 200, 8192, true);  // 4-head blocks, split
    gqa_prefill_test(st, MUGEN_ATTN_BF16, 3000, 64, 4096, true);
    gqa_prefill_test(st, MUGEN_ATTN_BF16, 7000, 256, 8192, true, 28, 4);  // 8-head blocks: split + fp16 V copy
    gqa_q4_test(st);
    prefill_batch_test(st);
    mla_prefill_test(st);
    bounds_test(st);
    (void)hipStreamSynchronize(st);
    (void)hipStreamDestroy(st);
    std::printf(failures ? "FAIL (%d)\n" : "PASS\n", failures);
    return failures ? 1 : 0;
}
