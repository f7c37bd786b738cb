// mugen_attn_path.hpp -- which attention provider serves a model: the
// MI355X replacement of the reference's CPU / GPU attention switch.
//
// The reference picks the attention path per model once, at load
// (src/core/model/transformer.cpp):
//   * use_gpu_attention_ = !is_mla() && n_kv_heads >= 4          (:3426-3430)
//     -- GPU flash_attention_decode over the f16 per-layer caches
//     buf_kv_gpu_k/v (:3382-3394); dense models run it inside the cached
//     mega-chain (lazy_cpu_kv, :3701, :3734-3833), MoE layers dispatch it
//     per layer (:4190-4197) while the host KVCache is still appended;
//   * otherwise (n_kv_heads < 4, or the override off) cpu_attention
//     (:2441-2485) over the host KVCache created with quantize_4bit = true,
//     fp16_preserve_last = 256 (:3369-3377), read back through
//     KVCache::read_k / read_v (Q4 groups for all but the newest 256 tokens,
//     kv_cache.cpp:218-278);
//   * MLA models (kv_lora_rank > 0) always take cpu_mla_attention (:2539)
//     over buf_kv_compressed (:3397-3407);
//   * TransformerModel::set_use_gpu_attention(bool) (:2637) overrides the
//     GQA choice at run time.
// Results differ between the two GQA paths (the 4-bit store rounds tokens
// older than 256 positions), so the same rule picks between the two GQA
// providers here: GqaAttention (f16 caches, mugen_attn_gqa_decode) where the
// reference attends on the GPU, GqaAttentionQ4 (the 4-bit group store,
// mugen_attn_gqa_decode_q4) where it runs cpu_attention over its KVCache.
// MoE models take the same provider as dense ones: their attention is the
// same call; only the reference's scheduling around it differs.
//
// Plain C++17, no HIP: the selection is host logic and is tested on the CPU.
#pragma once

#include <cstdint>
#include <string>

namespace mugen_attn {

// The fields of the reference's ModelConfig (transformer.h:45-80) that the
// attention path depends on.
struct ModelAttentionConfig {
    uint32_t n_heads = 0;
    uint32_t n_kv_heads = 0;
    uint32_t head_dim = 0;
    bool is_moe = false;
    uint32_t kv_lora_rank = 0;      // > 0: MLA (ModelConfig::is_mla)
    uint32_t qk_rope_head_dim = 0;  // MLA: 64
    uint32_t qk_nope_head_dim = 0;  // MLA: 128
    uint32_t v_head_dim = 0;        // MLA: 128
    bool is_mla() const { return kv_lora_rank > 0; }
};

enum class AttentionPath {
    Gqa,    // GqaAttention: f16 caches, the reference's GPU attention
    GqaQ4,  // GqaAttentionQ4: 4-bit group store, the reference's cpu_attention path
    Mla,    // MlaAttention: cpu_mla_attention over the latent cache
};

// Override of the automatic GQA choice (set_use_gpu_attention).
enum class GpuAttentionOverride { Auto, On, Off };

// The reference's default, transformer.cpp:3430.
inline bool default_use_gpu_attention(const ModelAttentionConfig& c) { return !c.is_mla() && c.n_kv_heads >= 4; }

struct PathChoice {
    AttentionPath path = AttentionPath::Gqa;
    bool supported = false;  // the library's kernels serve this shape
    std::string reason;      // why not, when !supported
};

// The provider that gives the reference's results for this model.  An MLA
// model ignores the override, as the reference does (its MLA branch never
// reads use_gpu_attention_).  `supported` is false for shapes the kernels do
// not cover (head_dim not a multiple of 8 or above 256 -- only 64 / 128 /
// 256 for the 4-bit store --, more than 16 query heads per KV head, MLA dims other
// than 512 / 64 / 128 / 128); the engine keeps the
// reference's CPU attention for those.
inline PathChoice select_attention_path(const ModelAttentionConfig& c,
                                        GpuAttentionOverride ovr = GpuAttentionOverride::Auto) {
    PathChoice r;
    if (c.is_mla()) {
        r.path = AttentionPath::Mla;
        if (c.kv_lora_rank != 512 || c.qk_rope_head_dim != 64 || c.qk_nope_head_dim != 128 || c.v_head_dim != 128) {
            r.reason = "MLA dims kv_lora_rank/rope/nope/v " + std::to_string(c.kv_lora_rank) + "/" +
                       std::to_string(c.qk_rope_head_dim) + "/" + std::to_string(c.qk_nope_head_dim) + "/" +
                       std::to_string(c.v_head_dim) + " (supported: 512/64/128/128)";
            return r;
        }
        if (c.n_heads == 0) {
            r.reason = "n_heads must be > 0";
            return r;
        }
        r.supported = true;
        return r;
    }
    const bool gpu = ovr == GpuAttentionOverride::Auto ? default_use_gpu_attention(c) : ovr == GpuAttentionOverride::On;
    r.path = gpu ? AttentionPath::Gqa : AttentionPath::GqaQ4;
    if (c.n_kv_heads == 0 || c.n_heads == 0 || c.n_heads % c.n_kv_heads) {
        r.reason = "n_heads must be a positive multiple of n_kv_heads";
        return r;
    }
    // f16 caches: head_dim a multiple of 8 up to 256; the 4-bit store: 64, 128, 256
    const bool hd_ok = gpu ? (c.head_dim >= 8 && c.head_dim <= 256 && c.head_dim % 8 == 0)
                           : (c.head_dim == 64 || c.head_dim == 128 || c.head_dim == 256);
    if (!hd_ok) {
        r.reason = "head_dim " + std::to_string(c.head_dim) +
                   (gpu ? " (supported: multiples of 8 up to 256)" : " (4-bit store: 64, 128, 256)");
        return r;
    }
    if (c.n_heads / c.n_kv_heads > 16) {
        r.reason = "more than 16 query heads per KV head";
        return r;
    }
    r.supported = true;
    return r;
}

inline const char* path_name(AttentionPath p) {
    switch (p) {
        case AttentionPath::Gqa: return "GqaAttention";
        case AttentionPath::GqaQ4: return "GqaAttentionQ4";
        default: return "MlaAttention";
    }
}

}  // namespace mugen_attn
