// factory_check.cpp -- end-to-end check of create_attention_provider
// (include/mugen_attn_engine.hpp), the replacement of the reference's
// use_gpu_attention_ choice at model load (src/core/model/transformer.cpp:3430,
// override :2637).  For each model configuration named on the command line
// the factory creates the provider it selects; the program then feeds every
// sequence a prompt through prefill_layer (in chunks where the provider
// limits them), captures one decode step of every layer into a StepGraph and
// replays it twice with fresh inputs.  Every input and output is written as
// raw little-endian arrays under <out_dir>/<config>/ with a manifest
// ("name dtype dim0 dim1 ...") so that tests/test_factory_gpu.py can compare
// them with the CPU oracle.
//
//   factory_check <out_dir> <config>...     configs: llama1b qwen7b v2lite hk2_d64 wide_d256
//
// Exit status 0 when every provider was created and every call succeeded.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <sys/stat.h>
#include <vector>

#include "mugen_attn_engine.hpp"

namespace {

using mugen_attn::Status;

struct Rng {  // splitmix64 -> uniform in [-a, a)
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

std::vector<uint16_t> f16_rand(Rng& r, size_t n, float a, float offset = 0.f) {
    std::vector<uint16_t> v(n);
    for (auto& x : v) {
        _Float16 h = (_Float16)(offset + r.uni(a));
        std::memcpy(&x, &h, 2);
    }
    return v;
}

bool failed = false;

bool ok(const Status& st, const std::string& what) {
    if (st) return true;
    std::printf("FAIL %s: %s\n", what.c_str(), st.error().c_str());
    std::fflush(stdout);
    failed = true;
    return false;
}

bool hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    std::printf("FAIL %s: %s\n", what, hipGetErrorString(e));
    failed = true;
    return false;
}

struct Dev {
    void* p = nullptr;
    size_t n = 0;
    explicit Dev(size_t bytes) : n(bytes) { hip(hipMalloc(&p, bytes), "hipMalloc"); }
    ~Dev() { (void)hipFree(p); }
    void put(const void* h, hipStream_t st) {
        hip(hipMemcpyAsync(p, h, n, hipMemcpyHostToDevice, st), "upload");
        hip(hipStreamSynchronize(st), "sync");
    }
    std::vector<uint8_t> get(hipStream_t st) const {
        std::vector<uint8_t> h(n);
        hip(hipMemcpyAsync(h.data(), p, n, hipMemcpyDeviceToHost, st), "download");
        hip(hipStreamSynchronize(st), "sync");
        return h;
    }
};

// <dir>/<name>.bin plus a manifest line
struct Dump {
    std::string dir;
    FILE* manifest = nullptr;
    explicit Dump(const std::string& d) : dir(d) {
        mkdir(dir.c_str(), 0755);
        manifest = std::fopen((dir + "/manifest.txt").c_str(), "w");
    }
    ~Dump() {
        if (manifest) std::fclose(manifest);
    }
    void put(const std::string& name, const char* dtype, const void* data, size_t bytes, std::vector<int> dims) {
        FILE* f = std::fopen((dir + "/" + name + ".bin").c_str(), "wb");
        if (!f || std::fwrite(data, 1, bytes, f) != bytes) {
            std::printf("FAIL writing %s\n", name.c_str());
            failed = true;
        }
        if (f) std::fclose(f);
        std::fprintf(manifest, "%s %s", name.c_str(), dtype);
        for (int d : dims) std::fprintf(manifest, " %d", d);
        std::fprintf(manifest, "\n");
    }
    template <class T>
    void vec(const std::string& name, const char* dtype, const std::vector<T>& v, std::vector<int> dims) {
        put(name, dtype, v.data(), v.size() * sizeof(T), std::move(dims));
    }
};

constexpr int kLayers = 2, kBatch = 2, kSteps = 2;

// GQA (f16 caches) and 4-bit store providers: prompts through prefill_layer
// in chunks of at most `chunk` tokens, then kSteps captured decode steps
template <class P>
void run_gqa(P* prov, const mugen_attn::ModelAttentionConfig& c, const std::vector<int>& prompt, int chunk,
             Dump& d, hipStream_t st) {
    const int H = (int)c.n_heads, Hk = (int)c.n_kv_heads, D = (int)c.head_dim, row = Hk * D;
    Rng r(17 + H + 3 * Hk + D);
    // prompts in the engine's order: each chunk through every layer, then
    // advance_sequence; chunks of at most `chunk` tokens
    for (int b = 0; b < kBatch; b++) {
        const int P0 = prompt[b];
        std::vector<std::vector<uint16_t>> q(kLayers), k(kLayers), v(kLayers), out(kLayers);
        for (int L = 0; L < kLayers; L++) {
            q[L] = f16_rand(r, (size_t)P0 * H * D, 1.f);
            k[L] = f16_rand(r, (size_t)P0 * row, 1.f);
            v[L] = f16_rand(r, (size_t)P0 * row, 1.f);
            out[L].resize((size_t)P0 * H * D);
        }
        for (int t0 = 0; t0 < P0; t0 += chunk) {
            const int n = std::min(chunk, P0 - t0);
            for (int L = 0; L < kLayers; L++) {
                Dev dq((size_t)n * H * D * 2), dk((size_t)n * row * 2), dv((size_t)n * row * 2), dout(dq.n);
                dq.put(q[L].data() + (size_t)t0 * H * D, st);
                dk.put(k[L].data() + (size_t)t0 * row, st);
                dv.put(v[L].data() + (size_t)t0 * row, st);
                if (!ok(prov->prefill_layer(L, b, dq.p, dk.p, dv.p, dout.p, n, st), "prefill_layer")) return;
                auto h = dout.get(st);
                std::memcpy(out[L].data() + (size_t)t0 * H * D, h.data(), h.size());
            }
            if (!ok(prov->advance_sequence(b, n, st), "advance_sequence")) return;
        }
        for (int L = 0; L < kLayers; L++) {
            const std::string tag = "s" + std::to_string(b) + "_L" + std::to_string(L);
            d.vec("prompt_q_" + tag, "f16", q[L], {P0, H, D});
            d.vec("prompt_k_" + tag, "f16", k[L], {P0, row});
            d.vec("prompt_v_" + tag, "f16", v[L], {P0, row});
            d.vec("prompt_out_" + tag, "f16", out[L], {P0, H, D});
        }
    }
    std::vector<std::unique_ptr<Dev>> q, k, v, o;
    for (int L = 0; L < kLayers; L++) {
        q.emplace_back(new Dev((size_t)kBatch * H * D * 2));
        k.emplace_back(new Dev((size_t)kBatch * row * 2));
        v.emplace_back(new Dev((size_t)kBatch * row * 2));
        o.emplace_back(new Dev((size_t)kBatch * H * D * 2));
    }
    mugen_attn::StepGraph g;
    auto body = [&](hipStream_t s) -> Status {
        for (int L = 0; L < kLayers; L++)
            if (auto rr = prov->decode_layer(L, q[L]->p, k[L]->p, v[L]->p, o[L]->p, s); !rr) return rr;
        return prov->advance(s, 1);
    };
    if (!ok(g.capture(st, body), "capture")) return;
    for (int step = 0; step < kSteps; step++) {
        for (int L = 0; L < kLayers; L++) {
            auto hq = f16_rand(r, (size_t)kBatch * H * D, 1.f);
            auto hk = f16_rand(r, (size_t)kBatch * row, 1.f), hv = f16_rand(r, (size_t)kBatch * row, 1.f);
            q[L]->put(hq.data(), st);
            k[L]->put(hk.data(), st);
            v[L]->put(hv.data(), st);
            const std::string tag = "t" + std::to_string(step) + "_L" + std::to_string(L);
            d.vec("step_q_" + tag, "f16", hq, {kBatch, H, D});
            d.vec("step_k_" + tag, "f16", hk, {kBatch, row});
            d.vec("step_v_" + tag, "f16", hv, {kBatch, row});
        }
        if (!ok(g.replay(st), "replay")) return;
        hip(hipStreamSynchronize(st), "sync");
        for (int L = 0; L < kLayers; L++) {
            auto h = o[L]->get(st);
            d.put("step_out_t" + std::to_string(step) + "_L" + std::to_string(L), "f16", h.data(), h.size(),
                  {kBatch, H, D});
        }
    }
}

void run_mla(mugen_attn::MlaAttention* prov, const mugen_attn::ProviderLimits& lim, int H,
             const std::vector<int>& prompt, Dump& d, hipStream_t st) {
    Rng r(91 + H);
    std::vector<std::unique_ptr<Dev>> norm, wkb, wvb;
    std::vector<mugen_attn::MlaLayerWeights> w(kLayers);
    for (int L = 0; L < kLayers; L++) {
        auto hn = f16_rand(r, 512, 0.2f, 1.0f);  // RMSNorm weights near 1
        auto hk = f16_rand(r, (size_t)H * 128 * 512, 0.08f), hv = f16_rand(r, (size_t)H * 128 * 512, 0.08f);
        norm.emplace_back(new Dev(512 * 2));
        wkb.emplace_back(new Dev(hk.size() * 2));
        wvb.emplace_back(new Dev(hv.size() * 2));
        norm[L]->put(hn.data(), st);
        wkb[L]->put(hk.data(), st);
        wvb[L]->put(hv.data(), st);
        w[L] = {norm[L]->p, wkb[L]->p, wvb[L]->p, MUGEN_ATTN_W_F16};
        const std::string tag = "_L" + std::to_string(L);
        d.vec("norm_w" + tag, "f16", hn, {512});
        d.vec("w_kb" + tag, "f16", hk, {H * 128, 512});
        d.vec("w_vb" + tag, "f16", hv, {H * 128, 512});
    }
    // prompts: every layer's chunk before the sequence advances (the
    // engine's order), chunks of at most max_prefill tokens
    for (int b = 0; b < kBatch; b++) {
        for (int t0 = 0; t0 < prompt[b]; t0 += lim.max_prefill) {
            const int n = std::min(lim.max_prefill, prompt[b] - t0);
            for (int L = 0; L < kLayers; L++) {
                auto hq = f16_rand(r, (size_t)n * H * 192, 1.f), ha = f16_rand(r, (size_t)n * 576, 1.f);
                Dev dq(hq.size() * 2), da(ha.size() * 2), dout((size_t)n * H * 128 * 2);
                dq.put(hq.data(), st);
                da.put(ha.data(), st);
                if (!ok(prov->prefill_layer(L, b, w[L], dq.p, da.p, dout.p, n, st), "mla prefill_layer")) return;
                const std::string tag = "s" + std::to_string(b) + "_c" + std::to_string(t0) + "_L" + std::to_string(L);
                d.vec("prompt_kva_" + tag, "f16", ha, {n, 576});
            }
            if (!ok(prov->advance_sequence(b, n, st), "mla advance_sequence")) return;
        }
    }
    std::vector<std::unique_ptr<Dev>> q, a, o;
    for (int L = 0; L < kLayers; L++) {
        q.emplace_back(new Dev((size_t)kBatch * H * 192 * 2));
        a.emplace_back(new Dev((size_t)kBatch * 576 * 2));
        o.emplace_back(new Dev((size_t)kBatch * H * 128 * 2));
    }
    mugen_attn::StepGraph g;
    auto body = [&](hipStream_t s) -> Status {
        for (int L = 0; L < kLayers; L++)
            if (auto rr = prov->decode_layer(L, w[L], q[L]->p, a[L]->p, o[L]->p, s); !rr) return rr;
        return prov->advance(s, 1);
    };
    if (!ok(g.capture(st, body), "mla capture")) return;
    for (int step = 0; step < kSteps; step++) {
        for (int L = 0; L < kLayers; L++) {
            auto hq = f16_rand(r, (size_t)kBatch * H * 192, 1.f), ha = f16_rand(r, (size_t)kBatch * 576, 1.f);
            q[L]->put(hq.data(), st);
            a[L]->put(ha.data(), st);
            const std::string tag = "t" + std::to_string(step) + "_L" + std::to_string(L);
            d.vec("step_q_" + tag, "f16", hq, {kBatch, H, 192});
            d.vec("step_kva_" + tag, "f16", ha, {kBatch, 576});
        }
        if (!ok(g.replay(st), "mla replay")) return;
        hip(hipStreamSynchronize(st), "sync");
        for (int L = 0; L < kLayers; L++) {
            auto h = o[L]->get(st);
            d.put("step_out_t" + std::to_string(step) + "_L" + std::to_string(L), "f16", h.data(), h.size(),
                  {kBatch, H, 128});
        }
    }
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 3) {
        std::printf("usage: factory_check <out_dir> <config>...\n");
        return 2;
    }
    const std::string out_dir = argv[1];
    mkdir(out_dir.c_str(), 0755);
    hipStream_t st;
    if (!hip(hipStreamCreate(&st), "stream")) return 1;
    for (int i = 2; i < argc; i++) {
        const std::string name = argv[i];
        mugen_attn::ModelAttentionConfig c;
        mugen_attn::ProviderLimits lim;
        lim.n_layers = kLayers;
        lim.batch = kBatch;
        lim.max_seq_len = 640;
        lim.max_new = 64;
        lim.max_prefill = 64;
        std::vector<int> prompt = {300, 41};
        if (name == "llama1b") {  // Llama-3.2-1B: 32 / 8, d 64 -> GqaAttention
            c.n_heads = 32, c.n_kv_heads = 8, c.head_dim = 64;
        } else if (name == "qwen7b") {  // Qwen2.5-7B: 28 / 4, d 128 -> GqaAttention
            c.n_heads = 28, c.n_kv_heads = 4, c.head_dim = 128;
        } else if (name == "v2lite") {  // DeepSeek-V2-Lite: MLA, 16 heads -> MlaAttention
            c.n_heads = 16, c.n_kv_heads = 16, c.head_dim = 192, c.is_moe = true;
            c.kv_lora_rank = 512, c.qk_rope_head_dim = 64, c.qk_nope_head_dim = 128, c.v_head_dim = 128;
            lim.rope = mugen_attn_rope_params{10000.f, 40.f, 4096};
            prompt = {150, 20};
        } else if (name == "wide_d256") {  // head_dim 256 (Gemma-style), 8 KV heads -> GqaAttention
            c.n_heads = 16, c.n_kv_heads = 8, c.head_dim = 256;
        } else if (name == "hk2_d64") {  // 2 KV heads, d 64 -> GqaAttentionQ4 (cpu_attention path)
            c.n_heads = 16, c.n_kv_heads = 2, c.head_dim = 64;
        } else {
            std::printf("FAIL unknown config %s\n", name.c_str());
            return 2;
        }
        mugen_attn::AttentionProvider p;
        if (!ok(mugen_attn::create_attention_provider(c, lim, &p), "create " + name)) continue;
        std::printf("%s: %s\n", name.c_str(), mugen_attn::path_name(p.path));
        std::fflush(stdout);
        Dump d(out_dir + "/" + name);
        std::fprintf(d.manifest, "#path %s\n", mugen_attn::path_name(p.path));
        std::fprintf(d.manifest, "#shape %u %u %u %d %d %d %d\n", c.n_heads, c.n_kv_heads, c.head_dim, kLayers,
                     kBatch, kSteps, lim.max_seq_len);
        std::fprintf(d.manifest, "#prompt %d %d\n", prompt[0], prompt[1]);
        std::fprintf(d.manifest, "#rope %g %g %d %d\n", lim.rope.theta, lim.rope.factor, lim.rope.original_ctx,
                     lim.max_prefill);
        if (p.gqa)
            run_gqa(p.gqa.get(), c, prompt, 1 << 30, d, st);
        else if (p.gqa_q4)
            run_gqa(p.gqa_q4.get(), c, prompt, lim.max_new, d, st);
        else
            run_mla(p.mla.get(), lim, (int)c.n_heads, prompt, d, st);
        std::printf("%s done\n", name.c_str());
        std::fflush(stdout);
    }
    hip(hipStreamDestroy(st), "stream");
    std::printf(failed ? "FAIL\n" : "PASS\n");
    return failed ? 1 : 0;
}
