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
//
// Lengths.  Every provider keeps each sequence's length twice: on the device
// (what the kernels read, so that captured steps replay unchanged) and a host
// mirror (for validation and prefill grids).  set_lengths() and every eager
// call refuse lengths that would run past max_seq_len, as the reference's
// KVCache::append refuses a token once the cache is full
// (kv_cache.cpp:163-170).  A captured step does its host bookkeeping once,
// at capture: an engine that replays a StepGraph counts its own replays
// (steps_left() at capture time bounds them) and calls sync_lengths() before
// the next eager call.  Independently of the host checks, the kernels clamp
// device lengths to max_seq_len and drop rows past it, so a replay beyond the
// cache never reads or writes outside the caches or the workspace.
#pragma once

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "mugen_attn.hpp"
#include "mugen_attn_path.hpp"

namespace mugen_attn {

namespace detail {

inline Status hip_ok(hipError_t e, const char* what) {
    if (e == hipSuccess) return Status{};
    return fail(std::string(what) + ": " + hipGetErrorString(e));
}

// The prefill workspace that serves every prompt chunk of up to max_tokens
// tokens in a cache of max_seq_len rows: the largest
// mugen_attn_gqa_prefill_workspace_size over the chunk lengths (the fp16 V
// copy of BF16 prompts, and the key splits' partials of chunks that continue
// a long context; neither falls as the key range grows, so each length is
// sized at the end of the cache).  `placeholder`: any 16-byte aligned device pointer
// (only the shape matters for the size).
inline size_t prefill_workspace_bytes(int n_heads, int n_kv_heads, int head_dim, int dtype, int max_seq_len,
                                      int max_tokens, const void* placeholder) {
    mugen_attn_gqa_prefill_args a{};
    a.q = a.k = a.v = placeholder;
    a.out = const_cast<void*>(placeholder);
    a.n_heads = n_heads;
    a.n_kv_heads = n_kv_heads;
    a.head_dim = head_dim;
    a.causal = 1;
    a.dtype = dtype;
    a.out_dtype = dtype;
    a.kv_len = max_seq_len;
    size_t best = 0;
    // within one count of 16-token query blocks the size grows with the length
    for (int n = 16;; n += 16) {
        a.n_tokens = std::min(n, max_tokens);
        a.start_pos = max_seq_len - a.n_tokens;
        best = std::max(best, mugen_attn_gqa_prefill_workspace_size(&a));
        if (n >= max_tokens) break;
    }
    return best;
}

// every length in [0, max_seq_len - n_new]: room for the step's n_new tokens
inline Status check_lengths(const std::vector<int32_t>& lens, int batch, int max_seq_len, int n_new,
                            const char* who) {
    if ((int)lens.size() != batch) return fail(std::string(who) + ": one length per sequence");
    for (int32_t x : lens)
        if (x < 0 || x > max_seq_len - n_new)
            return fail(std::string(who) + ": length " + std::to_string(x) + " outside [0, max_seq_len - " +
                        std::to_string(n_new) + "] = [0, " + std::to_string(max_seq_len - n_new) + "]");
    return Status{};
}

// device int32 [n] -> host
inline Status read_ints(const void* dev, std::vector<int32_t>& host, size_t n, hipStream_t st, const char* who) {
    host.resize(n);
    if (auto r = hip_ok(hipMemcpyAsync(host.data(), dev, n * sizeof(int32_t), hipMemcpyDeviceToHost, st), who); !r)
        return r;
    return hip_ok(hipStreamSynchronize(st), who);
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
        // the prefill workspace: the fp16 copy of one sequence's V for long
        // BF16 prompts, and the key splits' partials of prompt chunks that
        // continue a long context
        const size_t pf = detail::prefill_workspace_bytes(s.n_heads, s.n_kv_heads, s.head_dim, s.kv_dtype,
                                                          s.max_seq_len, s.max_seq_len, a->k_[0].ptr);
        if (pf)
            if (auto r = a->pf_ws_.alloc(pf, "GqaAttention prefill workspace"); !r) return r;
        // empty sequences: [0 | 1], so a step before any set_lengths is well defined
        if (auto r = a->set_lengths(std::vector<int32_t>(s.batch, 0), nullptr); !r) return r;
        *out = std::move(a);
        return Status{};
    }

    // Set every sequence's length, the tokens held before the next step, each
    // in [0, max_seq_len - 1] (outside any captured step; waits for the copy).
    Status set_lengths(const std::vector<int32_t>& lens, hipStream_t st) {
        if (auto r = detail::check_lengths(lens, s_.batch, s_.max_seq_len, 1, "GqaAttention::set_lengths"); !r)
            return r;
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

    // Host mirror <- device lengths (after StepGraph replays); waits.
    Status sync_lengths(hipStream_t st) {
        return detail::read_ints(lens_.ptr, host_lens_, s_.batch, st, "GqaAttention::sync_lengths");
    }
    // Decode steps that still fit every sequence's cache (host mirror).
    int steps_left() const {
        int m = s_.max_seq_len;
        for (int32_t x : host_lens_) m = std::min(m, s_.max_seq_len - x);
        return m;
    }

    // One layer of a decode step: q [batch][H][d], k_new / v_new
    // [batch][Hk*d], out [batch][H][d].
    Status decode_layer(int L, const void* q, const void* k_new, const void* v_new, void* out, hipStream_t st,
                        int n_new = 1) {
        if (L < 0 || L >= s_.n_layers) return fail("GqaAttention::decode_layer: bad layer");
        if (n_new != 1) return fail("GqaAttention::decode_layer: one new token per sequence");
        if (steps_left() < 1) return fail("GqaAttention::decode_layer: KV cache full (max_seq_len reached)");
        mugen_attn_kv_append_args ap = append_args(L, k_new, v_new, 0, s_.batch, n_new);
        if (auto r = kv_append(ap, st); !r) return r;
        const mugen_attn_gqa_decode_args d = decode_args(L, q, out);
        return gqa_decode(d, ws_.ptr, ws_.bytes, st);
    }

    // Prompt of n_tokens for sequence `seq`, one layer: append its K / V
    // rows at the sequence's current length, then causal flash attention
    // over its cache (make_prefill_attention_dp, transformer.cpp:828-850,
    // :1915).  Sequences are prefilled one at a time, as the reference does
    // (a prompt joins a running batch).  Uses the host copy of the length,
    // so it is not for captured steps; after the last layer call
    // advance_sequence(seq, n_tokens, st).
    //   q [n_tokens][H][d], k_new / v_new [n_tokens][Hk*d], out [n_tokens][H][d]
    Status prefill_layer(int L, int seq, const void* q, const void* k_new, const void* v_new, void* out,
                         int n_tokens, hipStream_t st) {
        if (L < 0 || L >= s_.n_layers) return fail("GqaAttention::prefill_layer: bad layer");
        if (seq < 0 || seq >= s_.batch) return fail("GqaAttention::prefill_layer: bad sequence");
        if (n_tokens <= 0) return fail("GqaAttention::prefill_layer: n_tokens must be > 0");
        const int start = host_lens_[seq];
        if (start + n_tokens > s_.max_seq_len) return fail("GqaAttention::prefill_layer: prompt past max_seq_len");
        mugen_attn_kv_append_args ap = append_args(L, k_new, v_new, seq, 1, n_tokens);
        if (auto r = kv_append(ap, st); !r) return r;
        mugen_attn_gqa_prefill_args pf{};
        pf.q = q;
        pf.k = seq_ptr(k_[L].ptr, seq);
        pf.v = seq_ptr(v_[L].ptr, seq);
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
        pf.workspace = pf_ws_.ptr;
        pf.workspace_bytes = pf_ws_.bytes;
        return gqa_prefill(pf, st);
    }
    // batch-1 form: sequence 0
    Status prefill_layer(int L, const void* q, const void* k_new, const void* v_new, void* out, int n_tokens,
                         hipStream_t st) {
        return prefill_layer(L, 0, q, k_new, v_new, out, n_tokens, st);
    }

    // End of a step: every length += n (device side, capturable; the host
    // mirror follows).
    Status advance(hipStream_t st, int n = 1) {
        for (int32_t x : host_lens_)
            if (x + n > s_.max_seq_len) return fail("GqaAttention::advance: past max_seq_len");
        for (auto& x : host_lens_) x += n;
        return seq_advance(static_cast<int32_t*>(lens_.ptr), n, 2 * s_.batch, s_.max_seq_len, st);
    }
    // One sequence's length += n (after its prompt's prefill_layer calls).
    Status advance_sequence(int seq, int n, hipStream_t st) {
        if (seq < 0 || seq >= s_.batch) return fail("GqaAttention::advance_sequence: bad sequence");
        if (host_lens_[seq] + n > s_.max_seq_len) return fail("GqaAttention::advance_sequence: past max_seq_len");
        host_lens_[seq] += n;
        int32_t* lens = static_cast<int32_t*>(lens_.ptr);
        if (auto r = seq_advance(lens + seq, n, 1, s_.max_seq_len, st); !r) return r;
        return seq_advance(lens + s_.batch + seq, n, 1, s_.max_seq_len, st);
    }

    void* k_cache(int L) const { return k_[L].ptr; }
    void* v_cache(int L) const { return v_[L].ptr; }
    const int32_t* lengths_after() const { return static_cast<const int32_t*>(lens_.ptr) + s_.batch; }
    const std::vector<int32_t>& host_lengths() const { return host_lens_; }
    const GqaShape& shape() const { return s_; }

private:
    explicit GqaAttention(const GqaShape& s) : s_(s) {}
    const int32_t* before() const { return static_cast<const int32_t*>(lens_.ptr); }
    int64_t seq_stride() const { return (int64_t)s_.max_seq_len * s_.n_kv_heads * s_.head_dim; }
    void* seq_ptr(void* cache, int seq) const { return static_cast<uint16_t*>(cache) + seq * seq_stride(); }
    mugen_attn_kv_append_args append_args(int L, const void* k_new, const void* v_new, int seq, int n_seq,
                                          int n_new) const {
        mugen_attn_kv_append_args ap{};
        ap.k_new = k_new;
        ap.v_new = v_new;
        ap.k_cache = seq_ptr(k_[L].ptr, seq);
        ap.v_cache = seq_ptr(v_[L].ptr, seq);
        ap.seq_lens = before() + seq;
        ap.seq_stride = seq_stride();
        ap.n_seq = n_seq;
        ap.n_new = n_new;
        ap.row = s_.n_kv_heads * s_.head_dim;
        ap.max_seq_len = s_.max_seq_len;
        return ap;
    }
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
        d.seq_stride = seq_stride();
        d.scale = s_.scale;
        d.kv_dtype = s_.kv_dtype;
        d.out_dtype = s_.out_dtype;
        d.seq_lens_host = nullptr;  // the grid is planned for max_seq_len: one plan serves every step
        return d;
    }

    GqaShape s_;
    std::vector<detail::DeviceBuffer> k_, v_;
    detail::DeviceBuffer lens_, ws_, pf_ws_;
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
    int max_new = 64;              // most tokens one append_layer / prefill_layer call adds per sequence
    int out_dtype = MUGEN_ATTN_F16;
    float scale = 0.f;             // 0: 1/sqrt(head_dim)
    // Keep f16 per-layer caches beside the store, as the reference keeps
    // buf_kv_gpu_k/v for every dense model (transformer.cpp:3382-3394): its
    // prompt prefill attends over those f16 rows (:1915) whichever path
    // decodes.  Needed by prefill_layer.
    bool f16_cache = true;
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
        if (s.f16_cache) {
            const size_t cache = (size_t)s.batch * s.max_seq_len * vpt * 2;
            a->k16_.resize(s.n_layers);
            a->v16_.resize(s.n_layers);
            for (int L = 0; L < s.n_layers; L++) {
                if (auto r = a->k16_[L].alloc(cache, "GqaAttentionQ4 f16 K cache"); !r) return r;
                if (auto r = a->v16_[L].alloc(cache, "GqaAttentionQ4 f16 V cache"); !r) return r;
            }
        }
        // lens_: [before | after] as GqaAttention; q4_: [n_q4 | n_q4 after the step's append]
        if (auto r = a->lens_.alloc(sizeof(int32_t) * 2 * s.batch, "GqaAttentionQ4 lengths"); !r) return r;
        if (auto r = a->q4n_.alloc(sizeof(int32_t) * 2 * s.batch, "GqaAttentionQ4 quantised counts"); !r) return r;
        mugen_attn_gqa_decode_q4_args d = a->decode_args(0, nullptr, nullptr);
        d.q = d.out = a->rk_[0].ptr;  // placeholders: only the shape matters for the size
        if (auto r = a->ws_.alloc(gqa_decode_q4_workspace_size(d), "GqaAttentionQ4 workspace"); !r) return r;
        if (s.f16_cache) {  // prompt chunks of up to max_new tokens over the f16 cache
            const size_t pf = detail::prefill_workspace_bytes(s.n_heads, s.n_kv_heads, s.head_dim, MUGEN_ATTN_F16,
                                                              s.max_seq_len, s.max_new, a->k16_[0].ptr);
            if (pf)
                if (auto r = a->pf_ws_.alloc(pf, "GqaAttentionQ4 prefill workspace"); !r) return r;
        }
        if (auto r = a->set_lengths(std::vector<int32_t>(s.batch, 0), nullptr); !r) return r;
        *out = std::move(a);
        return Status{};
    }

    // Set every sequence's length for an EMPTY store (a new conversation:
    // 0), or for one whose rows the caller filled to that length through
    // append_layer.  Each in [0, max_seq_len - 1].  Outside any captured
    // step; waits for the copy.
    Status set_lengths(const std::vector<int32_t>& lens, hipStream_t st) {
        if (auto r = detail::check_lengths(lens, s_.batch, s_.max_seq_len, 1, "GqaAttentionQ4::set_lengths"); !r)
            return r;
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
        host_lens_ = lens;
        return detail::hip_ok(hipStreamSynchronize(st), "GqaAttentionQ4::set_lengths");
    }

    Status sync_lengths(hipStream_t st) {
        return detail::read_ints(lens_.ptr, host_lens_, s_.batch, st, "GqaAttentionQ4::sync_lengths");
    }
    int steps_left() const {
        int m = s_.max_seq_len;
        for (int32_t x : host_lens_) m = std::min(m, s_.max_seq_len - x);
        return m;
    }

    // KVCache::append of n_new (<= max_new) tokens per sequence to one layer,
    // without attention (a prompt's rows, fed in chunks); after every layer
    // of the chunk: advance(st, n_new).  k_new / v_new [batch][n_new][Hk*d].
    Status append_layer(int L, const void* k_new, const void* v_new, int n_new, hipStream_t st) {
        if (L < 0 || L >= s_.n_layers) return fail("GqaAttentionQ4::append_layer: bad layer");
        if (n_new <= 0 || n_new > s_.max_new) return fail("GqaAttentionQ4::append_layer: 0 < n_new <= max_new");
        if (steps_left() < n_new) return fail("GqaAttentionQ4::append_layer: KV cache full (max_seq_len reached)");
        if (auto r = kv_q4_append(append_args(L, k_new, v_new, 0, s_.batch, n_new), st); !r) return r;
        if (!s_.f16_cache) return Status{};
        return kv_append(f16_append_args(L, k_new, v_new, 0, s_.batch, n_new), st);
    }

    // One layer of a decode step: append the token's K / V, then cpu_attention
    // over the store including it.  q [batch][H][d], k_new / v_new
    // [batch][Hk*d], out [batch][H][d].
    Status decode_layer(int L, const void* q, const void* k_new, const void* v_new, void* out, hipStream_t st) {
        if (auto r = append_layer(L, k_new, v_new, 1, st); !r) return r;
        const mugen_attn_gqa_decode_q4_args d = decode_args(L, q, out);
        return gqa_decode_q4(d, ws_.ptr, ws_.bytes, st);
    }

    // A prompt chunk of n_tokens (<= max_new) for sequence `seq`, one
    // layer: the rows go into the 4-bit store (KVCache::append per token,
    // transformer.cpp:1891-1897) and the f16 cache, and the chunk attends
    // causally over the f16 cache (the reference's prefill attention,
    // :1915).  After every layer of the chunk: advance_sequence(seq,
    // n_tokens, st).  Host lengths: not for captured steps.
    //   q [n_tokens][H][d], k_new / v_new [n_tokens][Hk*d], out [n_tokens][H][d]
    Status prefill_layer(int L, int seq, const void* q, const void* k_new, const void* v_new, void* out,
                         int n_tokens, hipStream_t st) {
        if (!s_.f16_cache) return fail("GqaAttentionQ4::prefill_layer: created without f16_cache");
        if (L < 0 || L >= s_.n_layers) return fail("GqaAttentionQ4::prefill_layer: bad layer");
        if (seq < 0 || seq >= s_.batch) return fail("GqaAttentionQ4::prefill_layer: bad sequence");
        if (n_tokens <= 0 || n_tokens > s_.max_new)
            return fail("GqaAttentionQ4::prefill_layer: 0 < n_tokens <= max_new (feed longer prompts in chunks)");
        const int start = host_lens_[seq];
        if (start + n_tokens > s_.max_seq_len) return fail("GqaAttentionQ4::prefill_layer: prompt past max_seq_len");
        if (auto r = kv_q4_append(append_args(L, k_new, v_new, seq, 1, n_tokens), st); !r) return r;
        if (auto r = kv_append(f16_append_args(L, k_new, v_new, seq, 1, n_tokens), st); !r) return r;
        mugen_attn_gqa_prefill_args pf{};
        pf.q = q;
        pf.k = f16_seq(k16_[L].ptr, seq);
        pf.v = f16_seq(v16_[L].ptr, seq);
        pf.out = out;
        pf.n_tokens = n_tokens;
        pf.n_heads = s_.n_heads;
        pf.n_kv_heads = s_.n_kv_heads;
        pf.head_dim = s_.head_dim;
        pf.kv_len = start + n_tokens;
        pf.start_pos = start;
        pf.causal = 1;
        pf.scale = s_.scale;
        pf.dtype = MUGEN_ATTN_F16;
        pf.out_dtype = s_.out_dtype;
        pf.workspace = pf_ws_.ptr;
        pf.workspace_bytes = pf_ws_.bytes;
        return gqa_prefill(pf, st);
    }

    // End of a step (or of an appended chunk): lengths += n and the
    // quantised counts take the appends' result (device side, capturable).
    Status advance(hipStream_t st, int n = 1) {
        for (int32_t x : host_lens_)
            if (x + n > s_.max_seq_len) return fail("GqaAttentionQ4::advance: past max_seq_len");
        for (auto& x : host_lens_) x += n;
        int32_t* lens = static_cast<int32_t*>(lens_.ptr);
        int32_t* q4 = static_cast<int32_t*>(q4n_.ptr);
        if (auto r = seq_advance(lens, n, s_.batch, s_.max_seq_len, st, q4, q4 + s_.batch); !r) return r;
        return seq_advance(lens + s_.batch, n, s_.batch, s_.max_seq_len, st);
    }
    // One sequence's length += n and its quantised count committed (after
    // its prompt chunk's prefill_layer calls).
    Status advance_sequence(int seq, int n, hipStream_t st) {
        if (seq < 0 || seq >= s_.batch) return fail("GqaAttentionQ4::advance_sequence: bad sequence");
        if (host_lens_[seq] + n > s_.max_seq_len) return fail("GqaAttentionQ4::advance_sequence: past max_seq_len");
        host_lens_[seq] += n;
        int32_t* lens = static_cast<int32_t*>(lens_.ptr);
        int32_t* q4 = static_cast<int32_t*>(q4n_.ptr);
        if (auto r = seq_advance(lens + seq, n, 1, s_.max_seq_len, st, q4 + seq, q4 + s_.batch + seq); !r) return r;
        return seq_advance(lens + s_.batch + seq, n, 1, s_.max_seq_len, st);
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
    void* k_cache_f16(int L) const { return s_.f16_cache ? k16_[L].ptr : nullptr; }
    void* v_cache_f16(int L) const { return s_.f16_cache ? v16_[L].ptr : nullptr; }
    const int32_t* lengths_after() const { return static_cast<const int32_t*>(lens_.ptr) + s_.batch; }
    const int32_t* quantised() const { return static_cast<const int32_t*>(q4n_.ptr); }
    const std::vector<int32_t>& host_lengths() const { return host_lens_; }
    const GqaQ4Shape& shape() const { return s_; }

private:
    explicit GqaAttentionQ4(const GqaQ4Shape& s) : s_(s) {}
    const int32_t* before() const { return static_cast<const int32_t*>(lens_.ptr); }
    int64_t f16_stride() const { return (int64_t)s_.max_seq_len * s_.n_kv_heads * s_.head_dim; }
    void* f16_seq(void* cache, int seq) const { return static_cast<uint16_t*>(cache) + seq * f16_stride(); }
    // the store of sequences [seq, seq + n_seq)
    mugen_attn_kv_q4_append_args append_args(int L, const void* k_new, const void* v_new, int seq, int n_seq,
                                             int n_new) const {
        mugen_attn_kv_q4_append_args ap{};
        ap.store = store(L);
        ap.store.q4_k = static_cast<uint8_t*>(ap.store.q4_k) + seq * ap.store.q4_seq_stride;
        ap.store.q4_v = static_cast<uint8_t*>(ap.store.q4_v) + seq * ap.store.q4_seq_stride;
        ap.store.ring_k = static_cast<uint16_t*>(ap.store.ring_k) + seq * ap.store.ring_seq_stride;
        ap.store.ring_v = static_cast<uint16_t*>(ap.store.ring_v) + seq * ap.store.ring_seq_stride;
        ap.k_new = k_new;
        ap.v_new = v_new;
        ap.seq_lens = before() + seq;
        ap.n_q4 = static_cast<const int32_t*>(q4n_.ptr) + seq;
        ap.n_q4_out = static_cast<int32_t*>(q4n_.ptr) + s_.batch + seq;
        ap.n_seq = n_seq;
        ap.n_new = n_new;
        ap.n_kv_heads = s_.n_kv_heads;
        ap.head_dim = s_.head_dim;
        ap.max_seq_len = s_.max_seq_len;
        return ap;
    }
    mugen_attn_kv_append_args f16_append_args(int L, const void* k_new, const void* v_new, int seq, int n_seq,
                                              int n_new) const {
        mugen_attn_kv_append_args ap{};
        ap.k_new = k_new;
        ap.v_new = v_new;
        ap.k_cache = f16_seq(k16_[L].ptr, seq);
        ap.v_cache = f16_seq(v16_[L].ptr, seq);
        ap.seq_lens = before() + seq;
        ap.seq_stride = f16_stride();
        ap.n_seq = n_seq;
        ap.n_new = n_new;
        ap.row = s_.n_kv_heads * s_.head_dim;
        ap.max_seq_len = s_.max_seq_len;
        return ap;
    }
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
    std::vector<detail::DeviceBuffer> q4k_, q4v_, rk_, rv_, k16_, v16_;
    detail::DeviceBuffer lens_, q4n_, ws_, pf_ws_;
    std::vector<int32_t> host_lens_;
};

// ---------------------------------------------------------------- MLA

struct MlaShape {
    int n_layers = 0;
    int batch = 1;
    int n_heads = 0;          // 128 (V3), 16 (V2-Lite)
    int max_seq_len = 0;
    int q_len = 1;            // tokens per sequence per step: 1 decode, > 1 speculative verify
    int max_prefill = 0;      // most prompt tokens per prefill_layer call (0: no prompt prefill)
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
        if (s.q_len <= 0 || s.q_len > s.max_seq_len || s.max_prefill < 0)
            return fail("MlaAttention: q_len in [1, max_seq_len], max_prefill >= 0");
        std::unique_ptr<MlaAttention> a(new MlaAttention(s));
        a->lat_.resize(s.n_layers);
        for (int L = 0; L < s.n_layers; L++)
            if (auto r = a->lat_[L].alloc((size_t)s.batch * s.max_seq_len * 576 * 2, "MlaAttention latent"); !r)
                return r;
        // lens_: [before | after] per sequence, then one prefill length
        if (auto r = a->lens_.alloc(sizeof(int32_t) * (2 * s.batch + 1), "MlaAttention lengths"); !r) return r;
        const size_t rows = (size_t)std::max(s.batch * s.q_len, s.max_prefill) * s.n_heads;
        if (auto r = a->qabs_.alloc(rows * 576 * 4, "MlaAttention q_abs"); !r) return r;
        if (auto r = a->o_.alloc(rows * 512 * 4, "MlaAttention o"); !r) return r;
        mugen_attn_mla_decode_args m = a->core_args(0, s.batch, s.q_len, nullptr);
        m.q = m.out = a->qabs_.ptr;
        m.latent = a->lat_[0].ptr;
        m.seq_lens = a->lengths_after();
        size_t ws = mla_decode_workspace_size(m);
        // prompt chunks: the split planner gives shorter chunks more splits,
        // so a shorter chunk can need more workspace than max_prefill tokens
        // do -- size for every chunk length (a host-side loop over the planner)
        for (int n = 1; n <= s.max_prefill; n++) {
            mugen_attn_mla_decode_args pm = a->core_args(0, 1, n, a->lengths_after());
            pm.q = pm.out = a->qabs_.ptr;
            pm.latent = a->lat_[0].ptr;
            ws = std::max(ws, mla_decode_workspace_size(pm));
        }
        if (auto r = a->ws_.alloc(ws, "MlaAttention workspace"); !r) return r;
        if (auto r = a->set_lengths(std::vector<int32_t>(s.batch, 0), nullptr); !r) return r;
        *out = std::move(a);
        return Status{};
    }

    // Every sequence's length before the next step, each in
    // [0, max_seq_len - q_len].  Outside captured steps; waits for the copy.
    Status set_lengths(const std::vector<int32_t>& lens, hipStream_t st) {
        if (auto r = detail::check_lengths(lens, s_.batch, s_.max_seq_len, s_.q_len, "MlaAttention::set_lengths"); !r)
            return r;
        std::vector<int32_t> both(lens);  // [before | after]: a step appends q_len tokens and attends to them
        for (int32_t x : lens) both.push_back(x + s_.q_len);
        // from pageable host memory: wait for the copy before `both` goes away
        if (auto r = detail::hip_ok(hipMemcpyAsync(lens_.ptr, both.data(), sizeof(int32_t) * both.size(),
                                                   hipMemcpyHostToDevice, st),
                                    "MlaAttention::set_lengths");
            !r)
            return r;
        host_lens_ = lens;
        return detail::hip_ok(hipStreamSynchronize(st), "MlaAttention::set_lengths");
    }

    Status sync_lengths(hipStream_t st) {
        return detail::read_ints(lens_.ptr, host_lens_, s_.batch, st, "MlaAttention::sync_lengths");
    }
    // Steps of q_len tokens that still fit every sequence's cache (host mirror).
    int steps_left() const {
        int m = s_.max_seq_len;
        for (int32_t x : host_lens_) m = std::min(m, (s_.max_seq_len - x) / s_.q_len);
        return m;
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
        if (steps_left() < 1) return fail("MlaAttention::decode_layer: latent cache full (max_seq_len reached)");
        return layer(L, w, q, kv_a, out, 0, s_.batch, s_.q_len, lengths_after(), st);
    }

    // A prompt of n_tokens (<= max_prefill) for sequence `seq`, one layer:
    // the rows are written to the latent cache at the sequence's length and
    // every prompt token attends causally over the cache up to itself --
    // what the reference's prefill computes with one cpu_mla_attention call
    // per token at seq_len = start + t + 1 (transformer.cpp:1325-1337), here
    // as one verify-shaped call.  After the last layer:
    // advance_sequence(seq, n_tokens, st).  Host lengths: not for captured steps.
    //   q [n_tokens][H][192] f16, kv_a [n_tokens][576] f16, out [n_tokens][H][128] f16
    Status prefill_layer(int L, int seq, const MlaLayerWeights& w, const void* q, const void* kv_a, void* out,
                         int n_tokens, hipStream_t st) {
        if (L < 0 || L >= s_.n_layers) return fail("MlaAttention::prefill_layer: bad layer");
        if (seq < 0 || seq >= s_.batch) return fail("MlaAttention::prefill_layer: bad sequence");
        if (n_tokens <= 0 || n_tokens > s_.max_prefill)
            return fail("MlaAttention::prefill_layer: 0 < n_tokens <= max_prefill");
        if (host_lens_[seq] + n_tokens > s_.max_seq_len)
            return fail("MlaAttention::prefill_layer: prompt past max_seq_len");
        // the core's length, before + n_tokens, made on the device (stream
        // ordered, no host copy): the 32-bit value copied as two 16-bit
        // elements, then advanced
        int32_t* plen = static_cast<int32_t*>(lens_.ptr) + 2 * s_.batch;
        if (auto r = scatter_kv(before() + seq, plen, 0, 2, st); !r) return r;
        if (auto r = seq_advance(plen, n_tokens, 1, s_.max_seq_len, st); !r) return r;
        return layer(L, w, q, kv_a, out, seq, 1, n_tokens, plen, st);
    }

    // End of a step: every length += n, the tokens kept (q_len for decode;
    // the accepted ones after a verify -- the others are overwritten by the
    // next step's writes).  Device side, capturable.
    Status advance(hipStream_t st, int n = 1) {
        for (int32_t x : host_lens_)
            if (x + n > s_.max_seq_len) return fail("MlaAttention::advance: past max_seq_len");
        for (auto& x : host_lens_) x += n;
        return seq_advance(static_cast<int32_t*>(lens_.ptr), n, 2 * s_.batch, s_.max_seq_len, st);
    }
    Status advance_sequence(int seq, int n, hipStream_t st) {
        if (seq < 0 || seq >= s_.batch) return fail("MlaAttention::advance_sequence: bad sequence");
        if (host_lens_[seq] + n > s_.max_seq_len) return fail("MlaAttention::advance_sequence: past max_seq_len");
        host_lens_[seq] += n;
        int32_t* lens = static_cast<int32_t*>(lens_.ptr);
        if (auto r = seq_advance(lens + seq, n, 1, s_.max_seq_len, st); !r) return r;
        return seq_advance(lens + s_.batch + seq, n, 1, s_.max_seq_len, st);
    }

    void* latent(int L) const { return lat_[L].ptr; }
    const int32_t* lengths_after() const { return static_cast<const int32_t*>(lens_.ptr) + s_.batch; }
    const std::vector<int32_t>& host_lengths() const { return host_lens_; }
    const MlaShape& shape() const { return s_; }

private:
    explicit MlaAttention(const MlaShape& s) : s_(s) {}
    const int32_t* before() const { return static_cast<const int32_t*>(lens_.ptr); }
    int64_t seq_stride() const { return (int64_t)s_.max_seq_len * 576; }

    // latent write + absorb (q RoPE fused) -> core -> projection for
    // sequences [seq, seq + n_seq), rows_per_seq tokens each, the core
    // attending over `core_lens` (device, the lengths including the new rows)
    Status layer(int L, const MlaLayerWeights& w, const void* q, const void* kv_a, void* out, int seq, int n_seq,
                 int rows_per_seq, const int32_t* core_lens, hipStream_t st) {
        void* lat = static_cast<uint16_t*>(lat_[L].ptr) + seq * seq_stride();
        mugen_attn_mla_latent_write_args lw{};
        lw.kv_a = kv_a;
        lw.norm_w = w.kv_a_norm;
        lw.seq_base = before() + seq;  // token j of sequence b goes to before[b] + j
        lw.latent = lat;
        lw.rows = n_seq * rows_per_seq;
        lw.rows_per_seq = rows_per_seq;
        lw.max_seq_len = s_.max_seq_len;
        lw.kv_rank = 512;
        lw.rope_dim = 64;
        lw.latent_dtype = s_.latent_dtype;
        lw.seq_stride = seq_stride();
        lw.eps = s_.rms_norm_eps;
        lw.rope = s_.rope;
        mugen_attn_mla_absorb_args ab{};
        ab.q = q;
        ab.w_kb = w.w_kb;
        ab.q_abs = qabs_.ptr;
        ab.rows = n_seq * rows_per_seq;
        ab.n_heads = s_.n_heads;
        ab.nope_dim = 128;
        ab.rope_dim = 64;
        ab.kv_rank = 512;
        ab.w_type = w.w_type;
        ab.out_dtype = MUGEN_ATTN_F32;
        ab.seq_base = before() + seq;
        ab.rows_per_seq = rows_per_seq;
        ab.rope = s_.rope;
        // the latent write and the absorption in one launch (decode sizes)
        if (auto r = mla_prepare(lw, ab, st); !r) return r;
        mugen_attn_mla_decode_args m = core_args(L, n_seq, rows_per_seq, core_lens);
        m.latent = lat;
        if (auto r = mla_decode(m, ws_.ptr, ws_.bytes, st); !r) return r;
        mugen_attn_mla_project_args pr{};
        pr.o = o_.ptr;
        pr.w_vb = w.w_vb;
        pr.out = out;
        pr.rows = n_seq * rows_per_seq;
        pr.n_heads = s_.n_heads;
        pr.kv_rank = 512;
        pr.v_head_dim = 128;
        pr.w_type = w.w_type;
        pr.out_dtype = MUGEN_ATTN_F16;
        return mla_project(pr, st);
    }

    mugen_attn_mla_decode_args core_args(int L, int n_seq, int q_len, const int32_t* lens) const {
        mugen_attn_mla_decode_args m{};
        m.q = qabs_.ptr;
        m.latent = L < (int)lat_.size() ? lat_[L].ptr : nullptr;
        m.seq_lens = lens;
        m.out = o_.ptr;
        m.batch = n_seq;
        m.q_len = q_len;
        m.n_heads = s_.n_heads;
        m.kv_rank = 512;
        m.rope_dim = 64;
        m.max_seq_len = s_.max_seq_len;
        m.seq_stride = seq_stride();
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
    std::vector<int32_t> host_lens_;
};

// ---------------------------------------------------------------- path selection

// Sizes a provider needs beyond the model's attention config.
struct ProviderLimits {
    int n_layers = 0;
    int batch = 1;
    int max_seq_len = 0;             // the reference: context_length, or 8192 (transformer.cpp:3373)
    int q_len = 1;                   // MLA: tokens per step (> 1 for speculative verify)
    int max_prefill = 0;             // MLA: prompt tokens per prefill_layer call
    int fp16_preserve_last = 256;    // 4-bit store: the reference's KVCacheConfig value
    int max_new = 64;                // 4-bit store: tokens per append / prefill chunk
    int out_dtype = MUGEN_ATTN_F16;  // GQA output (the reference's buf_attn_out is f16)
    float rms_norm_eps = 1e-6f;      // MLA latent writer
    mugen_attn_rope_params rope{10000.f, 0.f, 0};  // MLA: rope_theta, rope_scaling_factor, rope_original_ctx
};

// The provider chosen for a model: exactly one pointer is set.
struct AttentionProvider {
    AttentionPath path = AttentionPath::Gqa;
    std::unique_ptr<GqaAttention> gqa;
    std::unique_ptr<GqaAttentionQ4> gqa_q4;
    std::unique_ptr<MlaAttention> mla;
};

// What replaces `use_gpu_attention_` at model load (transformer.cpp:3430,
// override :2637): select_attention_path() picks the provider that gives
// the reference's results, and this creates it.  Shapes the kernels do not
// serve fail with the reason, and the engine keeps its CPU attention.
inline Status create_attention_provider(const ModelAttentionConfig& c, const ProviderLimits& lim,
                                        AttentionProvider* out,
                                        GpuAttentionOverride ovr = GpuAttentionOverride::Auto) {
    const PathChoice choice = select_attention_path(c, ovr);
    if (!choice.supported) return fail(std::string("attention provider: ") + choice.reason);
    AttentionProvider p;
    p.path = choice.path;
    if (choice.path == AttentionPath::Mla) {
        MlaShape s;
        s.n_layers = lim.n_layers;
        s.batch = lim.batch;
        s.n_heads = (int)c.n_heads;
        s.max_seq_len = lim.max_seq_len;
        s.q_len = lim.q_len;
        s.max_prefill = lim.max_prefill;
        s.rms_norm_eps = lim.rms_norm_eps;
        s.rope = lim.rope;
        if (auto r = MlaAttention::create(s, &p.mla); !r) return r;
    } else if (choice.path == AttentionPath::Gqa) {
        GqaShape s;
        s.n_layers = lim.n_layers;
        s.batch = lim.batch;
        s.n_heads = (int)c.n_heads;
        s.n_kv_heads = (int)c.n_kv_heads;
        s.head_dim = (int)c.head_dim;
        s.max_seq_len = lim.max_seq_len;
        s.out_dtype = lim.out_dtype;
        if (auto r = GqaAttention::create(s, &p.gqa); !r) return r;
    } else {
        GqaQ4Shape s;
        s.n_layers = lim.n_layers;
        s.batch = lim.batch;
        s.n_heads = (int)c.n_heads;
        s.n_kv_heads = (int)c.n_kv_heads;
        s.head_dim = (int)c.head_dim;
        s.max_seq_len = lim.max_seq_len;
        s.fp16_preserve_last = lim.fp16_preserve_last;
        s.max_new = lim.max_new;
        s.out_dtype = lim.out_dtype;
        if (auto r = GqaAttentionQ4::create(s, &p.gqa_q4); !r) return r;
    }
    *out = std::move(p);
    return Status{};
}

}  // namespace mugen_attn
