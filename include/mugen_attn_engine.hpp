// mugen_attn_engine.hpp -- attention provider for Mugen's TransformerModel
// decode loop, over the mugen_attn C ABI.
//
// The reference runs a decode step's attention in three ways
// (src/core/model/transformer.cpp):
//   * dense models, GPU attention: a cached "mega-chain" of Metal dispatches
//     per step (:3734-3833) -- scatter_kv of K and V (:3749-3754) and
//     flash_attention_decode (:3755-3758) per layer, with pos / kv_offset /
//     seq_len patched into the cached constants before each step;
//   * dense models, CPU attention: KVCache::append + cpu_attention (:3704-3731);
//   * MLA models: per layer, host q RoPE (:3882-3921), host c_kv RMSNorm +
//     k_rope RoPE (:3930-3981), scatter_kv (:3982-3987) and
//     cpu_mla_attention (:3988-3995).
// GqaAttention and MlaAttention own what those paths keep per model -- the
// per-layer caches, the sequence lengths (on the device) and the split-K
// workspace -- and issue one layer's attention with decode_layer().  Every
// per-step value is read from device memory, so the calls of a whole step,
// advance() included, can be captured once into a HIP graph (StepGraph)
// and replayed for every later step without patching: the MI355X form of
// the mega-chain.  The engine captures its own projections / FFN launches
// on the same stream between the decode_layer() calls.
//
// Memory is allocated once, at create(); decode_layer(), advance() and
// StepGraph::replay() allocate nothing.  Errors come back as Status
// (std::expected<void, std::string> with a C++23 library).
#pragma once

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "mugen_attn.hpp"

namespace mugen_attn {

namespace detail {

inline Status hip_ok(hipError_t e, const char* what) {
    if (e == hipSuccess) return Status{};
    return fail(std::string(what) + ": " + hipGetErrorString(e));
}

// device buffer owned for the provider's lifetime
struct DeviceBuffer {
    void* ptr = nullptr;
    size_t bytes = 0;
    DeviceBuffer() = default;
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&& o) noexcept : ptr(o.ptr), bytes(o.bytes) {
        o.ptr = nullptr;
        o.bytes = 0;
    }
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
        if (this != &o) {
            if (ptr) (void)hipFree(ptr);
            ptr = o.ptr;
            bytes = o.bytes;
            o.ptr = nullptr;
            o.bytes = 0;
        }
        return *this;
    }
    ~DeviceBuffer() {
        if (ptr) (void)hipFree(ptr);
    }
    Status alloc(size_t n, const char* what) {
        bytes = n;
        if (n == 0) return Status{};
        if (auto r = hip_ok(hipMalloc(&ptr, n), what); !r) return r;
        return hip_ok(hipMemset(ptr, 0, n), what);
    }
};

}  // namespace detail

// A captured HIP graph of one decode step's launches on a stream.
class StepGraph {
public:
    StepGraph() = default;
    StepGraph(const StepGraph&) = delete;
    StepGraph& operator=(const StepGraph&) = delete;
    ~StepGraph() { reset(); }

    // Capture body(stream) -- every launch it issues on `stream` -- into the
    // graph.  The body must not synchronise or allocate.
    template <class Body>
    Status capture(hipStream_t stream, Body&& body) {
        reset();
        if (auto r = detail::hip_ok(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal),
                                    "hipStreamBeginCapture");
            !r)
            return r;
        Status inner = body(stream);
        hipGraph_t g = nullptr;
        Status ended = detail::hip_ok(hipStreamEndCapture(stream, &g), "hipStreamEndCapture");
        if (!inner) {
            if (g) (void)hipGraphDestroy(g);
            return inner;
        }
        if (!ended) return ended;
        graph_ = g;
        return detail::hip_ok(hipGraphInstantiate(&exec_, graph_, nullptr, nullptr, 0), "hipGraphInstantiate");
    }
    Status replay(hipStream_t stream) const {
        if (!exec_) return fail("StepGraph: nothing captured");
        return detail::hip_ok(hipGraphLaunch(exec_, stream), "hipGraphLaunch");
    }
    bool captured() const { return exec_ != nullptr; }
    void reset() {
        if (exec_) (void)hipGraphExecDestroy(exec_);
        if (graph_) (void)hipGraphDestroy(graph_);
        exec_ = nullptr;
        graph_ = nullptr;
    }

private:
    hipGraph_t graph_ = nullptr;
    hipGraphExec_t exec_ = nullptr;
};

// ---------------------------------------------------------------- GQA

struct GqaShape {
    int n_layers = 0;
    int batch = 1;          // sequences decoded together
    int n_heads = 0;
    int n_kv_heads = 0;
    int head_dim = 0;
    int max_seq_len = 0;
    int kv_dtype = MUGEN_ATTN_F16;
    int out_dtype = MUGEN_ATTN_F16;
    float scale = 0.f;      // 0: 1/sqrt(head_dim), as transformer.cpp:2444
};

// Per-layer token-major K / V caches [batch][max_seq_len][Hk*d] (the
// reference's buf_kv_gpu_k/v, transformer.cpp:3382-3394) and the decode
// attention of one layer: append the step's K / V rows at the current
// length, then attend over length + n_new.
class GqaAttention {
public:
    static Status create(const GqaShape& s, std::unique_ptr<GqaAttention>* out) {
        if (s.n_layers <= 0 || s.batch <= 0 || s.max_seq_len <= 0)
            return fail("GqaAttention: n_layers, batch and max_seq_len must be > 0");
        std::unique_ptr<GqaAttention> a(new GqaAttention(s));
        const size_t row = (size_t)s.n_kv_heads * s.head_dim;
        const size_t cache = (size_t)s.batch * s.max_seq_len * row * 2;
        a->k_.resize(s.n_layers);
        a->v_.resize(s.n_layers);
        for (int L = 0; L < s.n_layers; L++) {
            if (auto r = a->k_[L].alloc(cache, "GqaAttention K cache"); !r) return r;
            if (auto r = a->v_[L].alloc(cache, "GqaAttention V cache"); !r) return r;
        }
        // lens_: [0, batch) tokens held before the step's append, [batch, 2 batch) after it
        if (auto r = a->lens_.alloc(sizeof(int32_t) * 2 * s.batch, "GqaAttention lengths"); !r) return r;
        mugen_attn_gqa_decode_args d = a->decode_args(0, nullptr, nullptr);
        d.q = d.out = a->k_[0].ptr;  // placeholders: only the shape matters for the size
        // (a shape the library rejects sizes to 0 here and fails at decode_layer)
        if (auto r = a->ws_.alloc(gqa_decode_workspace_size(d), "GqaAttention workspace"); !r) return r;
        *out = std::move(a);
        return Status{};
    }

    // Set every sequence's length, the tokens held before the next step
    // (outside any captured step; waits for the copy).
    Status set_lengths(const std::vector<int32_t>& lens, hipStream_t st) {
        if ((int)lens.size() != s_.batch) return fail("GqaAttention::set_lengths: one length per sequence");
        std::vector<int32_t> both(lens);  // [before | after]: a step appends one token and attends to it
        for (int32_t x : lens) both.push_back(x + 1);
        // from pageable host memory: wait for the copy before `both` goes away
        if (auto r = detail::hip_ok(hipMemcpyAsync(lens_.ptr, both.data(), sizeof(int32_t) * both.size(),
                                                   hipMemcpyHostToDevice, st),
                                    "GqaAttention::set_lengths");
            !r)
            return r;
        host_lens_ = lens;
        return detail::hip_ok(hipStreamSynchronize(st), "GqaAttention::set_lengths");
    }

    // One layer of a decode step: q [batch][H][d], k_new / v_new
    // [batch][n_new][Hk*d] (n_new = 1 for decode), out [batch][H][d].
    Status decode_layer(int L, const void* q, const void* k_new, const void* v_new, void* out, hipStream_t st,
                        int n_new = 1) {
        if (L < 0 || L >= s_.n_layers) return fail("GqaAttention::decode_layer: bad layer");
        if (n_new != 1) return fail("GqaAttention::decode_layer: one new token per sequence");
        mugen_attn_kv_append_args ap{};
        ap.k_new = k_new;
        ap.v_new = v_new;
        ap.k_cache = k_[L].ptr;
        ap.v_cache = v_[L].ptr;
        ap.seq_lens = before();
        ap.seq_stride = (int64_t)s_.max_seq_len * s_.n_kv_heads * s_.head_dim;
        ap.n_seq = s_.batch;
        ap.n_new = n_new;
        ap.row = s_.n_kv_heads * s_.head_dim;
        ap.max_seq_len = s_.max_seq_len;
        if (auto r = kv_append(ap, st); !r) return r;
        const mugen_attn_gqa_decode_args d = decode_args(L, q, out);
        return gqa_decode(d, ws_.ptr, ws_.bytes, st);
    }

    // Prompt of n_tokens for sequence 0 (batch 1), one layer: append its K / V
    // rows at the current length, then causal flash attention over the cache
    // (make_prefill_attention_dp, transformer.cpp:828-850, :1915).  Uses the
    // host copy of the length, so it is not for captured steps; call
    // advance(st, n_tokens) after the last layer.
    //   q [n_tokens][H][d], k_new / v_new [n_tokens][Hk*d], out [n_tokens][H][d]
    Status prefill_layer(int L, const void* q, const void* k_new, const void* v_new, void* out, int n_tokens,
                         hipStream_t st) {
        if (L < 0 || L >= s_.n_layers) return fail("GqaAttention::prefill_layer: bad layer");
        if (s_.batch != 1) return fail("GqaAttention::prefill_layer: one sequence (batch 1)");
        const int start = host_lens_.empty() ? 0 : host_lens_[0];
        if (start + n_tokens > s_.max_seq_len) return fail("GqaAttention::prefill_layer: prompt past max_seq_len");
        mugen_attn_kv_append_args ap{};
        ap.k_new = k_new;
        ap.v_new = v_new;
        ap.k_cache = k_[L].ptr;
        ap.v_cache = v_[L].ptr;
        ap.seq_lens = before();
        ap.seq_stride = (int64_t)s_.max_seq_len * s_.n_kv_heads * s_.head_dim;
        ap.n_seq = 1;
        ap.n_new = n_tokens;
        ap.row = s_.n_kv_heads * s_.head_dim;
        ap.max_seq_len = s_.max_seq_len;
        if (auto r = kv_append(ap, st); !r) return r;
        mugen_attn_gqa_prefill_args pf{};
        pf.q = q;
        pf.k = k_[L].ptr;
        pf.v = v_[L].ptr;
        pf.out = out;
        pf.n_tokens = n_tokens;
        pf.n_heads = s_.n_heads;
        pf.n_kv_heads = s_.n_kv_heads;
        pf.head_dim = s_.head_dim;
        pf.kv_len = start + n_tokens;
        pf.start_pos = start;
        pf.causal = 1;
        pf.scale = s_.scale;
        pf.dtype = s_.kv_dtype;
        pf.out_dtype = s_.out_dtype;
        return gqa_prefill(pf, st);
    }

    // End of a step: every length += n (device side, capturable; the host
    // copy used by prefill_layer follows).
    Status advance(hipStream_t st, int n = 1) {
        for (auto& x : host_lens_) x = std::min(x + n, s_.max_seq_len);
        return seq_advance(static_cast<int32_t*>(lens_.ptr), n, 2 * s_.batch, s_.max_seq_len, st);
    }

    void* k_cache(int L) const { return k_[L].ptr; }
    void* v_cache(int L) const { return v_[L].ptr; }
    const int32_t* lengths_after() const { return static_cast<const int32_t*>(lens_.ptr) + s_.batch; }
    const GqaShape& shape() const { return s_; }

private:
    explicit GqaAttention(const GqaShape& s) : s_(s) {}
    const int32_t* before() const { return static_cast<const int32_t*>(lens_.ptr); }
    mugen_attn_gqa_decode_args decode_args(int L, const void* q, void* out) const {
        mugen_attn_gqa_decode_args d{};
        d.q = q;
        d.k_cache = L < (int)k_.size() ? k_[L].ptr : nullptr;
        d.v_cache = L < (int)v_.size() ? v_[L].ptr : nullptr;
        d.seq_lens = lengths_after();
        d.out = out;
        d.batch = s_.batch;
        d.n_heads = s_.n_heads;
        d.n_kv_heads = s_.n_kv_heads;
        d.head_dim = s_.head_dim;
        d.max_seq_len = s_.max_seq_len;
        d.seq_stride = (int64_t)s_.max_seq_len * s_.n_kv_heads * s_.head_dim;
        d.scale = s_.scale;
        d.kv_dtype = s_.kv_dtype;
        d.out_dtype = s_.out_dtype;
        d.seq_lens_host = nullptr;  // the grid is planned for max_seq_len: one plan serves every step
        return d;
    }

    GqaShape s_;
    std::vector<detail::DeviceBuffer> k_, v_;
    detail::DeviceBuffer lens_, ws_;
    std::vector<int32_t> host_lens_;
};

// ---------------------------------------------------------------- GQA, 4-bit store

struct GqaQ4Shape {
    int n_layers = 0;
    int batch = 1;
    int n_heads = 0;
    int n_kv_heads = 0;
    int head_dim = 0;
    int max_seq_len = 0;
    int fp16_preserve_last = 256;  // KVCacheConfig (the engine's value)
    int max_new = 64;              // most tokens one append_layer call adds per sequence
    int out_dtype = MUGEN_ATTN_F16;
    float scale = 0.f;             // 0: 1/sqrt(head_dim)
};

// The same step interface over the reference's 4-bit group KV store
// (KVCache with quantize_4bit, transformer.cpp:3374-3377; kv_cache.cpp:
// 163-278): per layer and sequence, tokens older than the newest
// fp16_preserve_last as 20-byte groups of 32 values, the newest in an f16
// ring.  decode_layer appends the step's rows (quantising the tokens that
// leave the ring) and attends straight from the store; the lengths and the
// quantised counts live on the device, so a captured step replays as is.
class GqaAttentionQ4 {
public:
    static Status create(const GqaQ4Shape& s, std::unique_ptr<GqaAttentionQ4>* out) {
        if (s.n_layers <= 0 || s.batch <= 0 || s.max_seq_len <= 0 || s.fp16_preserve_last < 0 || s.max_new <= 0)
            return fail("GqaAttentionQ4: n_layers, batch, max_seq_len, max_new must be > 0");
        const int vpt = s.n_kv_heads * s.head_dim;
        if (vpt <= 0 || vpt % 32) return fail("GqaAttentionQ4: n_kv_heads * head_dim must be a multiple of 32");
        std::unique_ptr<GqaAttentionQ4> a(new GqaAttentionQ4(s));
        a->ring_ = 1;
        while (a->ring_ < s.fp16_preserve_last + s.max_new) a->ring_ <<= 1;  // a power of two
        a->row_bytes_ = vpt / 32 * 20;
        const size_t q4 = (size_t)s.batch * s.max_seq_len * a->row_bytes_;
        const size_t ring = (size_t)s.batch * a->ring_ * vpt * 2;
        a->q4k_.resize(s.n_layers);
        a->q4v_.resize(s.n_layers);
        a->rk_.resize(s.n_layers);
        a->rv_.resize(s.n_layers);
        for (int L = 0; L < s.n_layers; L++) {
            if (auto r = a->q4k_[L].alloc(q4, "GqaAttentionQ4 K groups"); !r) return r;
            if (auto r = a->q4v_[L].alloc(q4, "GqaAttentionQ4 V groups"); !r) return r;
            if (auto r = a->rk_[L].alloc(ring, "GqaAttentionQ4 K ring"); !r) return r;
            if (auto r = a->rv_[L].alloc(ring, "GqaAttentionQ4 V ring"); !r) return r;
        }
        // lens_: [before | after] as GqaAttention; q4_: [n_q4 | n_q4 after the step's append]
        if (auto r = a->lens_.alloc(sizeof(int32_t) * 2 * s.batch, "GqaAttentionQ4 lengths"); !r) return r;
        if (auto r = a->q4n_.alloc(sizeof(int32_t) * 2 * s.batch, "GqaAttentionQ4 quantised counts"); !r) return r;
        mugen_attn_gqa_decode_q4_args d = a->decode_args(0, nullptr, nullptr);
        d.q = d.out = a->rk_[0].ptr;  // placeholders: only the shape matters for the size
        if (auto r = a->ws_.alloc(gqa_decode_q4_workspace_size(d), "GqaAttentionQ4 workspace"); !r) return r;
        *out = std::move(a);
        return Status{};
    }

    // Set every sequence's length for an EMPTY store (a new conversation:
    // 0), or for one whose rows the caller filled to that length through
    // append_layer.  Outside any captured step; waits for the copy.
    Status set_lengths(const std::vector<int32_t>& lens, hipStream_t st) {
        if ((int)lens.size() != s_.batch) return fail("GqaAttentionQ4::set_lengths: one length per sequence");
        std::vector<int32_t> both(lens), q4(lens.size());
        for (int32_t x : lens) both.push_back(x + 1);
        for (size_t i = 0; i < lens.size(); i++) q4[i] = std::max(0, lens[i] - s_.fp16_preserve_last);
        q4.insert(q4.end(), q4.begin(), q4.end());
        if (auto r = detail::hip_ok(hipMemcpyAsync(lens_.ptr, both.data(), sizeof(int32_t) * both.size(),
                                                   hipMemcpyHostToDevice, st),
                                    "GqaAttentionQ4::set_lengths");
            !r)
            return r;
        if (auto r = detail::hip_ok(hipMemcpyAsync(q4n_.ptr, q4.data(), sizeof(int32_t) * q4.size(),
                                                   hipMemcpyHostToDevice, st),
                                    "GqaAttentionQ4::set_lengths");
            !r)
            return r;
        return detail::hip_ok(hipStreamSynchronize(st), "GqaAttentionQ4::set_lengths");
    }

    // KVCache::append of n_new (<= max_new) tokens per sequence to one layer,
    // without attention (a prompt's rows, fed in chunks); after every layer
    // of the chunk: advance(st, n_new).  k_new / v_new [batch][n_new][Hk*d].
    Status append_layer(int L, const void* k_new, const void* v_new, int n_new, hipStream_t st) {
        if (L < 0 || L >= s_.n_layers) return fail("GqaAttentionQ4::append_layer: bad layer");
        if (n_new <= 0 || n_new > s_.max_new) return fail("GqaAttentionQ4::append_layer: 0 < n_new <= max_new");
        mugen_attn_kv_q4_append_args ap{};
        ap.store = store(L);
        ap.k_new = k_new;
        ap.v_new = v_new;
        ap.seq_lens = before();
        ap.n_q4 = static_cast<const int32_t*>(q4n_.ptr);
        ap.n_q4_out = static_cast<int32_t*>(q4n_.ptr) + s_.batch;
        ap.n_seq = s_.batch;
        ap.n_new = n_new;
        ap.n_kv_heads = s_.n_kv_heads;
        ap.head_dim = s_.head_dim;
        ap.max_seq_len = s_.max_seq_len;
        return kv_q4_append(ap, st);
    }

    // One layer of a decode step: append the token's K / V, then cpu_attention
    // over the store including it.  q [batch][H][d], k_new / v_new
    // [batch][Hk*d], out [batch][H][d].
    Status decode_layer(int L, const void* q, const void* k_new, const void* v_new, void* out, hipStream_t st) {
        if (auto r = append_layer(L, k_new, v_new, 1, st); !r) return r;
        const mugen_attn_gqa_decode_q4_args d = decode_args(L, q, out);
        return gqa_decode_q4(d, ws_.ptr, ws_.bytes, st);
    }

    // End of a step (or of an appended chunk): lengths += n and the
    // quantised counts take the appends' result (device side, capturable).
    Status advance(hipStream_t st, int n = 1) {
        int32_t* lens = static_cast<int32_t*>(lens_.ptr);
        int32_t* q4 = static_cast<int32_t*>(q4n_.ptr);
        if (auto r = seq_advance(lens, n, s_.batch, s_.max_seq_len, st, q4, q4 + s_.batch); !r) return r;
        return seq_advance(lens + s_.batch, n, s_.batch, s_.max_seq_len, st);
    }

    mugen_attn_kv_q4_store store(int L) const {
        mugen_attn_kv_q4_store k{};
        k.q4_k = q4k_[L].ptr;
        k.q4_v = q4v_[L].ptr;
        k.ring_k = rk_[L].ptr;
        k.ring_v = rv_[L].ptr;
        k.q4_seq_stride = (int64_t)s_.max_seq_len * row_bytes_;
        k.ring_seq_stride = (int64_t)ring_ * s_.n_kv_heads * s_.head_dim;
        k.ring = ring_;
        k.fp16_preserve_last = s_.fp16_preserve_last;
        return k;
    }
    const int32_t* lengths_after() const { return static_cast<const int32_t*>(lens_.ptr) + s_.batch; }
    const int32_t* quantised() const { return static_cast<const int32_t*>(q4n_.ptr); }
    const GqaQ4Shape& shape() const { return s_; }

private:
    explicit GqaAttentionQ4(const GqaQ4Shape& s) : s_(s) {}
    const int32_t* before() const { return static_cast<const int32_t*>(lens_.ptr); }
    mugen_attn_gqa_decode_q4_args decode_args(int L, const void* q, void* out) const {
        mugen_attn_gqa_decode_q4_args d{};
        d.q = q;
        d.store = store(L);
        d.seq_lens = lengths_after();
        d.n_q4 = static_cast<const int32_t*>(q4n_.ptr) + s_.batch;  // the state after this step's append
        d.out = out;
        d.batch = s_.batch;
        d.n_heads = s_.n_heads;
        d.n_kv_heads = s_.n_kv_heads;
        d.head_dim = s_.head_dim;
        d.max_seq_len = s_.max_seq_len;
        d.scale = s_.scale;
        d.out_dtype = s_.out_dtype;
        d.seq_lens_host = nullptr;  // planned for max_seq_len: one plan serves every step
        return d;
    }

    GqaQ4Shape s_;
    int ring_ = 0, row_bytes_ = 0;
    std::vector<detail::DeviceBuffer> q4k_, q4v_, rk_, rv_;
    detail::DeviceBuffer lens_, q4n_, ws_;
};

// ---------------------------------------------------------------- MLA

struct MlaShape {
    int n_layers = 0;
    int batch = 1;
    int n_heads = 0;          // 128 (V3), 16 (V2-Lite)
    int max_seq_len = 0;
    int q_len = 1;            // tokens per sequence per step: 1 decode, > 1 speculative verify
    float scale = 0.f;        // 1/sqrt(qk_nope + qk_rope), transformer.cpp:2550
    float rms_norm_eps = 1e-6f;
    mugen_attn_rope_params rope{10000.f, 0.f, 0};
    int latent_dtype = MUGEN_ATTN_F16;
};

// Per-model MLA weights of one layer the attention needs (device, in their
// GGUF encodings): attn_kv_a_norm (f16 [512]), attn_k_b and attn_v_b.
struct MlaLayerWeights {
    const void* kv_a_norm = nullptr;
    const void* w_kb = nullptr;
    const void* w_vb = nullptr;
    int w_type = MUGEN_ATTN_W_F16;
};

// Per-layer latent caches [batch][max_seq_len][576] (buf_kv_compressed[L],
// transformer.cpp:3397-3407) and steps E-I of the MLA decode layer.
class MlaAttention {
public:
    static Status create(const MlaShape& s, std::unique_ptr<MlaAttention>* out) {
        if (s.n_layers <= 0 || s.batch <= 0 || s.max_seq_len <= 0 || s.n_heads <= 0)
            return fail("MlaAttention: n_layers, batch, n_heads and max_seq_len must be > 0");
        std::unique_ptr<MlaAttention> a(new MlaAttention(s));
        a->lat_.resize(s.n_layers);
        for (int L = 0; L < s.n_layers; L++)
            if (auto r = a->lat_[L].alloc((size_t)s.batch * s.max_seq_len * 576 * 2, "MlaAttention latent"); !r)
                return r;
        if (auto r = a->lens_.alloc(sizeof(int32_t) * 2 * s.batch, "MlaAttention lengths"); !r) return r;
        if (s.q_len <= 0) return fail("MlaAttention: q_len must be > 0");
        const size_t rows = (size_t)s.batch * s.q_len * s.n_heads;
        if (auto r = a->qabs_.alloc(rows * 576 * 4, "MlaAttention q_abs"); !r) return r;
        if (auto r = a->o_.alloc(rows * 512 * 4, "MlaAttention o"); !r) return r;
        mugen_attn_mla_decode_args m = a->core_args(0);
        m.q = m.out = a->qabs_.ptr;
        m.latent = a->lat_[0].ptr;
        const size_t ws = mla_decode_workspace_size(m);
        if (auto r = a->ws_.alloc(ws, "MlaAttention workspace"); !r) return r;
        *out = std::move(a);
        return Status{};
    }

    Status set_lengths(const std::vector<int32_t>& lens, hipStream_t st) {
        if ((int)lens.size() != s_.batch) return fail("MlaAttention::set_lengths: one length per sequence");
        std::vector<int32_t> both(lens);  // [before | after]: a step appends q_len tokens and attends to them
        for (int32_t x : lens) both.push_back(x + s_.q_len);
        // from pageable host memory: wait for the copy before `both` goes away
        if (auto r = detail::hip_ok(hipMemcpyAsync(lens_.ptr, both.data(), sizeof(int32_t) * both.size(),
                                                   hipMemcpyHostToDevice, st),
                                    "MlaAttention::set_lengths");
            !r)
            return r;
        return detail::hip_ok(hipStreamSynchronize(st), "MlaAttention::set_lengths");
    }

    // One layer of a step: q_len new tokens per sequence (1 for decode; the
    // draft tokens of a speculative verify otherwise, causal among them --
    // the reference's per-token calls, transformer.cpp:1325-1337):
    //   q    [batch][q_len][H][192] f16 (buf_mla_q, before its RoPE)
    //   kv_a [batch][q_len][576]    f16 (buf_mla_kv_a, before RMSNorm / RoPE)
    //   out  [batch][q_len][H][128] f16 (the attention output fed to wo)
    Status decode_layer(int L, const MlaLayerWeights& w, const void* q, const void* kv_a, void* out,
                        hipStream_t st) {
        if (L < 0 || L >= s_.n_layers) return fail("MlaAttention::decode_layer: bad layer");
        mugen_attn_mla_latent_write_args lw{};
        lw.kv_a = kv_a;
        lw.norm_w = w.kv_a_norm;
        lw.seq_base = before();  // token j of sequence b goes to before[b] + j
        lw.latent = lat_[L].ptr;
        lw.rows = s_.batch * s_.q_len;
        lw.rows_per_seq = s_.q_len;
        lw.max_seq_len = s_.max_seq_len;
        lw.kv_rank = 512;
        lw.rope_dim = 64;
        lw.latent_dtype = s_.latent_dtype;
        lw.seq_stride = (int64_t)s_.max_seq_len * 576;
        lw.eps = s_.rms_norm_eps;
        lw.rope = s_.rope;
        if (auto r = mla_latent_write(lw, st); !r) return r;
        mugen_attn_mla_absorb_args ab{};
        ab.q = q;
        ab.w_kb = w.w_kb;
        ab.q_abs = qabs_.ptr;
        ab.rows = s_.batch * s_.q_len;
        ab.n_heads = s_.n_heads;
        ab.nope_dim = 128;
        ab.rope_dim = 64;
        ab.kv_rank = 512;
        ab.w_type = w.w_type;
        ab.out_dtype = MUGEN_ATTN_F32;
        ab.seq_base = before();
        ab.rows_per_seq = s_.q_len;
        ab.rope = s_.rope;
        if (auto r = mla_absorb(ab, st); !r) return r;
        const mugen_attn_mla_decode_args m = core_args(L);
        if (auto r = mla_decode(m, ws_.ptr, ws_.bytes, st); !r) return r;
        mugen_attn_mla_project_args pr{};
        pr.o = o_.ptr;
        pr.w_vb = w.w_vb;
        pr.out = out;
        pr.rows = s_.batch * s_.q_len;
        pr.n_heads = s_.n_heads;
        pr.kv_rank = 512;
        pr.v_head_dim = 128;
        pr.w_type = w.w_type;
        pr.out_dtype = MUGEN_ATTN_F16;
        return mla_project(pr, st);
    }

    // End of a step: every length += n, the tokens kept (q_len for decode;
    // the accepted ones after a verify -- the others are overwritten by the
    // next step's writes).  Device side, capturable.
    Status advance(hipStream_t st, int n = 1) {
        return seq_advance(static_cast<int32_t*>(lens_.ptr), n, 2 * s_.batch, s_.max_seq_len, st);
    }

    void* latent(int L) const { return lat_[L].ptr; }
    const int32_t* lengths_after() const { return static_cast<const int32_t*>(lens_.ptr) + s_.batch; }
    const MlaShape& shape() const { return s_; }

private:
    explicit MlaAttention(const MlaShape& s) : s_(s) {}
    const int32_t* before() const { return static_cast<const int32_t*>(lens_.ptr); }
    mugen_attn_mla_decode_args core_args(int L) const {
        mugen_attn_mla_decode_args m{};
        m.q = qabs_.ptr;
        m.latent = L < (int)lat_.size() ? lat_[L].ptr : nullptr;
        m.seq_lens = lengths_after();
        m.out = o_.ptr;
        m.batch = s_.batch;
        m.q_len = s_.q_len;
        m.n_heads = s_.n_heads;
        m.kv_rank = 512;
        m.rope_dim = 64;
        m.max_seq_len = s_.max_seq_len;
        m.seq_stride = (int64_t)s_.max_seq_len * 576;
        m.scale = s_.scale > 0.f ? s_.scale : 0.07216878364870322f;  // 1/sqrt(192)
        m.q_dtype = MUGEN_ATTN_F32;
        m.latent_dtype = s_.latent_dtype;
        m.out_dtype = MUGEN_ATTN_F32;
        m.seq_lens_host = nullptr;
        return m;
    }

    MlaShape s_;
    std::vector<detail::DeviceBuffer> lat_;
    detail::DeviceBuffer lens_, qabs_, o_, ws_;
};

}  // namespace mugen_attn
