// Host-only check of include/mugen_attn_path.hpp: the attention provider the
// factory picks for the reference's model configurations, against the
// reference's rule use_gpu_attention_ = !is_mla() && n_kv_heads >= 4
// (src/core/model/transformer.cpp:3430) and its override (:2637).
// Prints one line per case: "<name> <path> <supported>".
#include <cstdio>

#include "mugen_attn_path.hpp"

using namespace mugen_attn;

static void show(const char* name, const ModelAttentionConfig& c, GpuAttentionOverride o = GpuAttentionOverride::Auto) {
    const PathChoice p = select_attention_path(c, o);
    std::printf("%s %s %d\n", name, path_name(p.path), p.supported ? 1 : 0);
}

int main() {
    ModelAttentionConfig llama1b;  // Llama-3.2-1B: 32 heads, 8 KV heads, d 64
    llama1b.n_heads = 32;
    llama1b.n_kv_heads = 8;
    llama1b.head_dim = 64;
    ModelAttentionConfig qwen7b;  // Qwen2.5-7B: 28 / 4, d 128
    qwen7b.n_heads = 28;
    qwen7b.n_kv_heads = 4;
    qwen7b.head_dim = 128;
    ModelAttentionConfig v2lite;  // DeepSeek-V2-Lite: MLA, 16 heads, MoE
    v2lite.n_heads = 16;
    v2lite.n_kv_heads = 16;
    v2lite.head_dim = 192;
    v2lite.is_moe = true;
    v2lite.kv_lora_rank = 512;
    v2lite.qk_rope_head_dim = 64;
    v2lite.qk_nope_head_dim = 128;
    v2lite.v_head_dim = 128;
    ModelAttentionConfig v3 = v2lite;  // DeepSeek-V3: MLA, 128 heads
    v3.n_heads = v3.n_kv_heads = 128;
    ModelAttentionConfig tiny;  // the reference's unit-test model: 4 heads, 2 KV heads, d 16
    tiny.n_heads = 4;
    tiny.n_kv_heads = 2;
    tiny.head_dim = 16;
    ModelAttentionConfig small_kv;  // a GQA model with 2 KV heads at a served head_dim
    small_kv.n_heads = 16;
    small_kv.n_kv_heads = 2;
    small_kv.head_dim = 64;
    ModelAttentionConfig wide;  // head_dim 256 (Gemma-style), 8 KV heads
    wide.n_heads = 16;
    wide.n_kv_heads = 8;
    wide.head_dim = 256;
    ModelAttentionConfig wide_kv2 = wide;  // head_dim 256 with 2 KV heads: the 4-bit store
    wide_kv2.n_kv_heads = 2;
    ModelAttentionConfig odd = wide;  // head_dim 160: padded to 256 on f16 caches
    odd.head_dim = 160;
    ModelAttentionConfig huge = wide;  // head_dim 512: beyond the kernels
    huge.head_dim = 512;
    ModelAttentionConfig moe = qwen7b;  // a GQA MoE model: same attention as dense
    moe.is_moe = true;
    show("llama1b", llama1b);
    show("qwen7b", qwen7b);
    show("v2lite", v2lite);
    show("v3", v3);
    show("tiny", tiny);
    show("small_kv", small_kv);
    show("moe", moe);
    show("wide", wide);
    show("wide_kv2", wide_kv2);
    show("odd", odd);
    show("odd_kv_off", odd, GpuAttentionOverride::Off);
    show("huge", huge);
    show("qwen7b_off", qwen7b, GpuAttentionOverride::Off);
    show("small_kv_on", small_kv, GpuAttentionOverride::On);
    show("tiny_on", tiny, GpuAttentionOverride::On);
    show("v2lite_on", v2lite, GpuAttentionOverride::On);
    show("v2lite_off", v2lite, GpuAttentionOverride::Off);
    return 0;
}
