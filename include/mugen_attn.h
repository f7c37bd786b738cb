/*
 * mugen_attn.h -- C ABI of the MI355X (gfx950) attention library for Mugen.
 *
 * Drop-in boundary for Mugen's attention operators.  In the reference the
 * operators are private members of TransformerModel::Impl, reached through
 * two seams that this ABI replaces:
 *
 *   CPU:  void cpu_attention(const f16* q, uint32_t layer, uint32_t seq_len,
 *                            f16* out)           src/core/model/transformer.cpp:2441
 *         void cpu_mla_attention(const f16* q, const LayerWeights&,
 *                                uint32_t layer, uint32_t seq_len, f16* out)
 *                                                 src/core/model/transformer.cpp:2539
 *   GPU:  MetalCompute::DispatchParams built by
 *         make_flash_attention_decode_dp           src/core/model/transformer.cpp:852-870
 *         make_prefill_attention_dp                src/core/model/transformer.cpp:828-850
 *         make_scatter_kv_dp                       src/core/model/transformer.cpp:872-886
 *         and run by dispatch_sync / dispatch_chain_sync
 *                                                  src/core/compute/metal_compute.h:84-89
 *
 * Conventions (all entry points):
 *   - plain C: pointers, sizes, enums; no C++ or framework types cross it;
 *   - every pointer to tensor data is a DEVICE pointer owned by the caller,
 *     16-byte aligned (q, caches and outputs);
 *     the library never allocates device memory inside a compute call;
 *     scratch ("workspace") is caller-provided, sized by *_workspace_size;
 *   - `stream` is a hipStream_t passed as void* (NULL = default stream);
 *     calls are stream-ordered and never synchronise the host;
 *   - return 0 on success, a negative MUGEN_ATTN_E_* code otherwise;
 *     mugen_attn_last_error() gives a message (thread-local).  The
 *     reference's convention is std::expected<..., std::string>
 *     (metal_compute.h:84-89); the C++ adapter mugen_attn.hpp maps codes +
 *     message back to that shape;
 *   - calls on distinct streams with distinct workspaces are thread-safe.
 */
#ifndef MUGEN_ATTN_H
#define MUGEN_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MUGEN_ATTN_ABI_VERSION 3

/* status codes */
#define MUGEN_ATTN_OK 0
#define MUGEN_ATTN_E_INVALID (-1)     /* null pointer, bad shape or stride      */
#define MUGEN_ATTN_E_UNSUPPORTED (-2) /* shape/dtype combination not compiled   */
#define MUGEN_ATTN_E_WORKSPACE (-3)   /* workspace missing or too small         */
#define MUGEN_ATTN_E_HIP (-4)         /* HIP runtime error (launch / device)    */

/* element types (storage); arithmetic is always fp32-accumulate */
typedef enum {
    MUGEN_ATTN_F32 = 0,
    MUGEN_ATTN_F16 = 1, /* IEEE binary16, the reference's f16 (_Float16) */
    MUGEN_ATTN_BF16 = 2
} mugen_attn_dtype;

/*
 * GQA decode: one new query token per sequence against its K/V cache.
 * Replaces cpu_attention (transformer.cpp:2441-2485) and the
 * flash_attention_decode dispatch (kernel_sources.h:2900-2999,
 * transformer.cpp:852-870).
 *
 *   q        [batch][n_heads][head_dim]                       (kv_dtype)
 *   k_cache  sequence b starts at k_cache + b*seq_stride elements; token t of
 *   v_cache  kv head j sits at + t*n_kv_heads*head_dim + j*head_dim, i.e. the
 *            reference's per-layer token-major [max_seq][Hk*d] buffer
 *            (buf_kv_gpu_k/v, transformer.cpp:3382-3394)
 *   seq_lens device int32 [batch]: tokens 0..seq_lens[b]-1 are attended
 *            (the reference's seq_len argument); 0 gives a zero output row
 *   out      [batch][n_heads][head_dim]                       (out_dtype)
 *
 *   kv head of query head h = h / (n_heads / n_kv_heads)   (transformer.cpp:2452)
 *   scale <= 0 selects 1/sqrt(head_dim)                     (transformer.cpp:2444)
 *   max_seq_len (> 0): tokens each sequence's cache holds; sizes the split-K
 *            grid and workspace.  Device lengths are clamped to
 *            [0, max_seq_len], so a bad length never reads past the cache or
 *            writes past the workspace
 *   num_splits: 0 = automatic; otherwise the context-split count (>= 1)
 *
 * Supported: head_dim a multiple of 8 up to 256 (64, 128 and 256
 * natively, others on the next of those with the extra dims masked; the
 * 4-bit store entry point takes 64, 128 and 256 only); n_heads / n_kv_heads in [1, 16];
 * kv_dtype in {F16, BF16} (q has the same dtype); out_dtype F16/BF16/F32.
 */
typedef struct mugen_attn_gqa_decode_args {
    const void* q;
    const void* k_cache;
    const void* v_cache;
    const int32_t* seq_lens;
    void* out;
    int32_t batch;
    int32_t n_heads;
    int32_t n_kv_heads;
    int32_t head_dim;
    int32_t max_seq_len;
    int32_t num_splits;
    int64_t seq_stride; /* elements between consecutive sequences' caches */
    float scale;
    int32_t kv_dtype;   /* mugen_attn_dtype */
    int32_t out_dtype;  /* mugen_attn_dtype */
    /* optional HOST copy of seq_lens (NULL allowed): lets the planner size
     * the context splits for ragged batches.  It must equal the device
     * lengths; a copy that is too short gives wrong results but never writes
     * outside the workspace.  The workspace size depends on it; a size asked
     * for without it (and num_splits 0) covers every host copy. */
    const int32_t* seq_lens_host;
} mugen_attn_gqa_decode_args;

size_t mugen_attn_gqa_decode_workspace_size(const mugen_attn_gqa_decode_args* args);
int mugen_attn_gqa_decode(const mugen_attn_gqa_decode_args* args, void* workspace,
                          size_t workspace_bytes, void* stream);

/*
 * 4-bit group KV store: the reference's KVCache format (kv_cache.cpp:11-98)
 * on the GPU.  Per sequence (and layer), the quantised tokens [0, n_q4)
 * are kept as groups of 32 consecutive values of the token's
 * [n_kv_heads*head_dim] row, 20 bytes each: f16 scale, f16 min, 16 bytes of
 * nibbles (value 2i low, 2i+1 high), value = f16(min + nibble * scale).
 * The newest tokens stay f16 in a ring of `ring` rows (a power of two;
 * token t at slot t % ring), as the reference keeps its newest
 * fp16_preserve_last tokens.
 *   q4_k, q4_v      [n_seq][max_seq_len][n_kv_heads*head_dim/32][20 B],
 *                   q4_seq_stride bytes apart (a multiple of 4)
 *   ring_k, ring_v  [n_seq][ring][n_kv_heads*head_dim] F16,
 *                   ring_seq_stride elements apart (a multiple of 8)
 */
typedef struct mugen_attn_kv_q4_store {
    void* q4_k;
    void* q4_v;
    void* ring_k;
    void* ring_v;
    int64_t q4_seq_stride;
    int64_t ring_seq_stride;
    int32_t ring;
    int32_t fp16_preserve_last; /* the reference's KVCacheConfig field (256 in the engine) */
} mugen_attn_kv_q4_store;

/*
 * Append n_new tokens to each of n_seq sequences (KVCache::append,
 * kv_cache.cpp:163-216, applied n_new times): the new rows go to the ring,
 * and the tokens that leave the newest fp16_preserve_last are quantised
 * (quantize_group, kv_cache.cpp:21-56, bit for bit).
 *   k_new, v_new  [n_seq][n_new][n_kv_heads*head_dim] F16
 *   seq_lens      device [n_seq]: tokens held before the append
 *   n_q4          device [n_seq]: of which quantised (the store's state;
 *                 seq_lens - n_q4 <= fp16_preserve_last, as appends keep it)
 *   n_q4_out      device [n_seq]: quantised tokens after the append; must
 *                 not alias n_q4 (every layer's call reads the same n_q4)
 * Requires ring >= fp16_preserve_last + n_new; tokens at positions
 * >= max_seq_len are dropped (the reference's append refuses them).
 */
typedef struct mugen_attn_kv_q4_append_args {
    mugen_attn_kv_q4_store store;
    const void* k_new;
    const void* v_new;
    const int32_t* seq_lens;
    const int32_t* n_q4;
    int32_t* n_q4_out;
    int32_t n_seq;
    int32_t n_new;
    int32_t n_kv_heads;
    int32_t head_dim;
    int32_t max_seq_len;
} mugen_attn_kv_q4_append_args;
int mugen_attn_kv_q4_append(const mugen_attn_kv_q4_append_args* args, void* stream);

/*
 * GQA decode straight from the 4-bit store: cpu_attention
 * (transformer.cpp:2441-2485) over the K/V that KVCache::read_k / read_v
 * return (kv_cache.cpp:218-278) -- dequantised groups for t < n_q4[b], the
 * f16 ring rows for the rest -- without materialising them: 320 bytes per
 * token and kv head set instead of 1024 at n_kv_heads*head_dim = 512.
 * Same rules as mugen_attn_gqa_decode (q F16; out F16/BF16/F32; split-K
 * workspace from mugen_attn_gqa_decode_q4_workspace_size).
 */
typedef struct mugen_attn_gqa_decode_q4_args {
    const void* q;
    mugen_attn_kv_q4_store store;
    const int32_t* seq_lens;
    const int32_t* n_q4;
    void* out;
    int32_t batch;
    int32_t n_heads;
    int32_t n_kv_heads;
    int32_t head_dim;
    int32_t max_seq_len;
    int32_t num_splits;
    float scale;
    int32_t out_dtype;
    const int32_t* seq_lens_host; /* as in mugen_attn_gqa_decode_args */
} mugen_attn_gqa_decode_q4_args;
size_t mugen_attn_gqa_decode_q4_workspace_size(const mugen_attn_gqa_decode_q4_args* args);
int mugen_attn_gqa_decode_q4(const mugen_attn_gqa_decode_q4_args* args, void* workspace, size_t workspace_bytes,
                             void* stream);

/*
 * GQA causal prefill (flash attention) over one sequence.
 * Replaces flash_prefill_attention (kernel_sources.h:2769-2896) and
 * make_prefill_attention_dp (transformer.cpp:828-850); same buffers and
 * constants: Q_batch, K_cache, V_cache, O_batch, n_heads, n_kv_heads,
 * head_dim, kv_len, start_position, N.
 *
 *   q      [n_tokens][n_heads][head_dim]
 *   k, v   [kv_len][n_kv_heads*head_dim]  (the cache, new tokens included)
 *   out    [n_tokens][n_heads][head_dim]
 *   token i attends to keys [0, start_pos + i]   (kernel_sources.h:2796)
 *   causal = 0 lets every token see all kv_len keys.
 *
 * Supported: head_dim a multiple of 8 up to 256 (as gqa_decode; above 128
 * every query token attends in its own workgroup, the reference's per-token
 * CPU rule, and only kernel 0 is accepted);
 * n_heads / n_kv_heads in [1, 16] (more
 * than 8 runs on the warp-specialised kernel; forcing the per-block kernel
 * there is refused); dtype F16 or BF16 for q/k/v; out_dtype F16/BF16/F32.
 * With BF16 inputs the kernels may compute P.V in fp16 (V converted on
 * chip, exact inside the f16 range), so BF16 V values must lie
 * within +-65504 -- the range of the reference's f16 cache; V magnitudes
 * below 6.1e-5 keep an absolute precision of 2^-25.  The optional
 * workspace (below) holds an fp16 copy of BF16 V for long prompts, and the
 * partials of split key ranges for short chunks over a long context.
 */
typedef struct mugen_attn_gqa_prefill_args {
    const void* q;
    const void* k;
    const void* v;
    void* out;
    int32_t n_tokens;
    int32_t n_heads;
    int32_t n_kv_heads;
    int32_t head_dim;
    int32_t kv_len;
    int32_t start_pos;
    int32_t causal;
    float scale;
    int32_t dtype;
    int32_t out_dtype;
    /* 0 = automatic; MUGEN_ATTN_PREFILL_KERNEL_BLOCK / _WS / _SHORT force
     * one kernel (same results within rounding; for kernel comparisons) */
    int32_t kernel;
    /* optional workspace (NULL / 0: none).  For BF16 prompts of at least
     * 1024 tokens (and split calls, below, of more than 4 heads per kv head
     * over ranges of 1024+ keys), given at least kv_len *
     * n_kv_heads * head_dim * 2 + 256 bytes
     * (mugen_attn_gqa_prefill_workspace_size), the call first copies
     * V[0, kv_len) to fp16 there (one extra launch), so the attention
     * kernels need no per-workgroup conversion; same results.  When the
     * query blocks would occupy fewer than half the CUs (a short chunk
     * after a long context), a workspace of the full
     * mugen_attn_gqa_prefill_workspace_size also holds the partials of
     * split key ranges, merged by a second launch (same results to
     * rounding).  Smaller workspaces use what fits; a call never fails for
     * want of one.  It must not overlap q, k, v or out. */
    void* workspace;
    size_t workspace_bytes;
} mugen_attn_gqa_prefill_args;

#define MUGEN_ATTN_PREFILL_KERNEL_BLOCK 1 /* one (16-token block, kv head) per workgroup */
#define MUGEN_ATTN_PREFILL_KERNEL_WS 2    /* warp-specialised S / PV waves */
#define MUGEN_ATTN_PREFILL_KERNEL_SHORT 3 /* every visible key held on chip: head_dim 64, n_heads / n_kv_heads
                                           * <= 4, at most 512 keys (start_pos + n_tokens causal, kv_len
                                           * otherwise); forcing it outside that range is refused */

int mugen_attn_gqa_prefill(const mugen_attn_gqa_prefill_args* args, void* stream);
/* Bytes of the optional prefill workspace worth passing: the fp16 V copy
 * (kv_len * n_kv_heads * head_dim * 2 + 256 for BF16 prompts of at least
 * 1024 tokens and for some split calls, where the separate conversion pays
 * for its launch) plus the split partials (n_tokens * n_heads * splits *
 * (2 * head_dim + 8) + 512 when the key range is split), else 0 (also for
 * invalid args).  The size never falls as kv_len grows at a fixed n_tokens.
 * No counterpart in the reference (it runs each chunk on one pass over its
 * keys). */
size_t mugen_attn_gqa_prefill_workspace_size(const mugen_attn_gqa_prefill_args* args);

/*
 * MLA absorbed attention over the compressed latent cache: decode (q_len 1)
 * and speculative verify (q_len > 1, causal among the new tokens).
 * Replaces the latent core of cpu_mla_attention (transformer.cpp:2576-2608),
 * batched over sequences and over the verify tokens that the reference
 * processes one call at a time (transformer.cpp:1325-1337).
 *
 *   q       [batch][q_len][n_heads][kv_rank + rope_dim]: absorbed query,
 *           q_nope.W_UK (kv_rank) followed by q_rope (rope_dim)
 *   latent  sequence b at latent + b*seq_stride elements; token rows of
 *           kv_rank + rope_dim (c_kv then k_rope), the reference's
 *           buf_kv_compressed layout (transformer.cpp:3397-3407)
 *   seq_lens device int32 [batch]: cache length INCLUDING the q_len new
 *           tokens; query i sees seq_len - q_len + i + 1 tokens; clamped to
 *           [0, max_seq_len] (max_seq_len > 0: the cache's rows per sequence)
 *   out     [batch][q_len][n_heads][kv_rank]  o = sum_t p_t c_t[0:kv_rank]
 *   scale   must be > 0 (the reference uses 1/sqrt(qk_nope + qk_rope),
 *           transformer.cpp:2550; 1/sqrt(192) for DeepSeek V2/V3)
 *
 * Supported: kv_rank 512, rope_dim 64; latent dtype F16 or BF16 (bf16
 * latent values must lie within +-65504, the f16 range: the split partials
 * are f16, and values beyond it come out as inf); q dtype F32 (split into
 * two 16-bit halves, fp32-accurate) or equal to the latent dtype;
 * out_dtype F32, F16 or BF16.
 */
typedef struct mugen_attn_mla_decode_args {
    const void* q;
    const void* latent;
    const int32_t* seq_lens;
    void* out;
    int32_t batch;
    int32_t q_len;
    int32_t n_heads;
    int32_t kv_rank;
    int32_t rope_dim;
    int32_t max_seq_len;
    int32_t num_splits;
    int64_t seq_stride;
    float scale;
    int32_t q_dtype;
    int32_t latent_dtype;
    int32_t out_dtype;
    /* optional HOST copy of seq_lens (NULL allowed).  When given it sizes the
     * grid to exactly the active context splits, so every entry must be >=
     * the device value (normally equal; a larger value only costs idle
     * workgroups; a smaller one gives wrong results but never writes outside
     * the workspace).  NULL sizes the grid for batch * max_seq_len.  The
     * workspace size depends on it; a size asked for without it (and
     * num_splits 0) covers every host copy. */
    const int32_t* seq_lens_host;
    /* 0 = automatic; MUGEN_ATTN_MLA_KERNEL_ROWS / _WS force
     * one kernel (same results within rounding; for kernel comparisons) */
    int32_t kernel;
} mugen_attn_mla_decode_args;

#define MUGEN_ATTN_MLA_KERNEL_ROWS 1 /* 4 waves of 16 rows (16-bit q, <= 64 rows by default) */
#define MUGEN_ATTN_MLA_KERNEL_WS 2   /* warp-specialised S / P.L waves */

size_t mugen_attn_mla_decode_workspace_size(const mugen_attn_mla_decode_args* args);
int mugen_attn_mla_decode(const mugen_attn_mla_decode_args* args, void* workspace,
                          size_t workspace_bytes, void* stream);

/*
 * mugen_attn_mla_decode without a workspace argument and without any
 * allocation: the split partials go to a fixed device scratch that the
 * library holds per GPU (MUGEN_ATTN_MLA_SCRATCH_BYTES, until the process
 * ends).  No counterpart in the reference: this entry point is for callers
 * that cannot allocate -- code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc.  Same arguments, semantics and results
 * as mugen_attn_mla_decode; a call whose workspace size
 * (mugen_attn_mla_decode_workspace_size) exceeds the scratch fails with
 * MUGEN_ATTN_E_WORKSPACE.  Every call on one GPU shares that GPU's scratch:
 * calls that overlap on one GPU (two streams, two threads) race; serialise
 * them on one stream.  Nothing in the scratch needs clearing between calls.
 */
#define MUGEN_ATTN_MLA_SCRATCH_BYTES (32u << 20) /* 32 MiB: DeepSeek-V3 decode B8 needs 23 MiB */
int mugen_attn_mla_decode_noalloc(const mugen_attn_mla_decode_args* args, void* stream);

/*
 * MLA absorption and up-projection: the rest of cpu_mla_attention
 * (transformer.cpp:2539-2623) around the latent core above, so that
 *   mugen_attn_mla_absorb -> mugen_attn_mla_decode (q F32) -> mugen_attn_mla_project
 * computes the reference operator from its own inputs (f16 q_data, the
 * layer's attn_k_b / attn_v_b weights, the latent cache) to its f16 output.
 *
 * Weights keep the reference's GGUF block encodings, dequantised on the fly
 * exactly as dequant_weight_row (transformer.cpp:2488-2534) does; the ids
 * are GGML's (src/model/ggml_types.h:12-20):
 *   F16  : kv_rank halfs per row;
 *   Q8_0 : kv_rank/32 blocks of 34 bytes, f16 scale + 32 int8 (w = s*q);
 *   Q4_0 : kv_rank/32 blocks of 18 bytes, f16 scale + 16 bytes; element j
 *          of a block is low nibble of byte j (j < 16) or high nibble of
 *          byte j-16, minus 8, times s.
 * Weight rows start at row * row_bytes (no padding), byte-addressed.
 */
typedef enum {
    MUGEN_ATTN_W_F16 = 1,
    MUGEN_ATTN_W_Q4_0 = 2,
    MUGEN_ATTN_W_Q8_0 = 8
} mugen_attn_wtype;

/*
 * RoPE of the MLA path: NeoX pairs (i, i + rope_dim/2) with the YaRN
 * frequencies of yarn_rope_freq (transformer.cpp:41-70; beta_fast 32,
 * beta_slow 1), computed by the library on the host exactly as there.
 * factor <= 1 means plain RoPE, 1 / theta^(2i/rope_dim).
 */
typedef struct mugen_attn_rope_params {
    float theta;          /* rope_theta */
    float factor;         /* rope_scaling_factor */
    int32_t original_ctx; /* rope_original_ctx */
} mugen_attn_rope_params;

/*
 * q_absorbed = q_nope x k_b, then q_rope appended (transformer.cpp:2556-2573):
 *   q      [rows][n_heads][nope_dim + rope_dim]  F16 (the reference's q_data)
 *   w_kb   attn_k_b: n_heads*nope_dim rows of kv_rank values (w_type)
 *   q_abs  [rows][n_heads][kv_rank + rope_dim]   F32 (fp32 sums, as the
 *          reference's float q_absorbed) or BF16
 *   q_abs[r][h][d] = sum_i q[r][h][i] * k_b[h*nope_dim + i][d], d < kv_rank
 * rows = batch * q_len.  Supported: nope_dim 128, rope_dim 64, kv_rank 512.
 * With positions (device int32 [rows]) non-null, the appended q_rope is
 * first rotated by the reference's q RoPE stage (transformer.cpp:3882-3921,
 * f16 results) at positions[r]; q itself is not modified.  With positions
 * null and seq_base non-null, row r's position is
 * seq_base[r / rows_per_seq] + r % rows_per_seq (the tokens a sequence
 * appends in one step: a captured graph replays it unchanged).
 */
typedef struct mugen_attn_mla_absorb_args {
    const void* q;
    const void* w_kb;
    void* q_abs;
    int32_t rows;
    int32_t n_heads;
    int32_t nope_dim;
    int32_t rope_dim;
    int32_t kv_rank;
    int32_t w_type;    /* mugen_attn_wtype */
    int32_t out_dtype; /* F32 or BF16 */
    const int32_t* positions;    /* optional: RoPE q_rope at these positions */
    mugen_attn_rope_params rope; /* used when positions or seq_base is non-null */
    const int32_t* seq_base;     /* optional, with positions null: see above */
    int32_t rows_per_seq;        /* rows per sequence for seq_base (q_len) */
} mugen_attn_mla_absorb_args;
int mugen_attn_mla_absorb(const mugen_attn_mla_absorb_args* args, void* stream);

/*
 * out_h = out_comp x v_b^T (transformer.cpp:2610-2620):
 *   o      [rows][n_heads][kv_rank]         F32 (mugen_attn_mla_decode's out)
 *   w_vb   attn_v_b: n_heads*v_head_dim rows of kv_rank values (w_type)
 *   out    [rows][n_heads][v_head_dim]      F16 (the reference's output) or F32
 *   out[r][h][j] = sum_d o[r][h][d] * v_b[h*v_head_dim + j][d]
 * Supported: kv_rank 512, v_head_dim 128.
 */
typedef struct mugen_attn_mla_project_args {
    const void* o;
    const void* w_vb;
    void* out;
    int32_t rows;
    int32_t n_heads;
    int32_t kv_rank;
    int32_t v_head_dim;
    int32_t w_type;    /* mugen_attn_wtype */
    int32_t out_dtype; /* F16 or F32 */
} mugen_attn_mla_project_args;
int mugen_attn_mla_project(const mugen_attn_mla_project_args* args, void* stream);

/*
 * Latent-cache writer (transformer.cpp:3930-3987): for each new token r,
 *   c_kv = RMSNorm(kv_a[r][0:kv_rank]) * norm_w   (1/sqrt(mean(x^2) + eps))
 *   k_rope = RoPE(kv_a[r][kv_rank:], positions[r])
 * and [c_kv | k_rope] is written to row positions[r] of sequence
 * r / rows_per_seq of the latent cache, replacing the reference's host
 * round trip (read kv_a, normalise and rotate on the CPU, scatter_kv).
 *   kv_a      [rows][kv_rank + rope_dim] F16 (the kv_a_mqa projection)
 *   norm_w    [kv_rank] F16 (attn_kv_a_norm)
 *   positions [rows] device int32; rows outside [0, max_seq_len) are skipped;
 *             or null with seq_base (device int32 [n_seq]): row r goes to
 *             seq_base[r / rows_per_seq] + r % rows_per_seq
 *   latent    [n_seq][max_seq_len][kv_rank + rope_dim], seq_stride elements
 *             apart; F16 (the reference's rounding) or BF16
 * Supported: kv_rank 512, rope_dim 64.
 */
typedef struct mugen_attn_mla_latent_write_args {
    const void* kv_a;
    const void* norm_w;
    const int32_t* positions;
    void* latent;
    int32_t rows;
    int32_t rows_per_seq;
    int32_t max_seq_len;
    int32_t kv_rank;
    int32_t rope_dim;
    int32_t latent_dtype;
    int64_t seq_stride;
    float eps;
    mugen_attn_rope_params rope;
    const int32_t* seq_base; /* used when positions is null */
} mugen_attn_mla_latent_write_args;
int mugen_attn_mla_latent_write(const mugen_attn_mla_latent_write_args* args, void* stream);

/*
 * The two independent stages that precede the latent core in one call:
 * the latent write of the step's new tokens (as mugen_attn_mla_latent_write,
 * transformer.cpp:3930-3987) and the absorption of their queries (as
 * mugen_attn_mla_absorb, transformer.cpp:2563-2573 with the q RoPE of
 * :3882-3921).  Results are identical to the two calls.  At decode sizes
 * (absorb rows < 64) both run in ONE kernel launch, which removes a launch
 * from the layer step; at prompt sizes they run as the two launches.  The
 * absorption must not read the latent rows being written (it does not: it
 * reads q and W_UK only).  Either args' rows may be 0.
 */
int mugen_attn_mla_prepare(const mugen_attn_mla_latent_write_args* latent_write,
                           const mugen_attn_mla_absorb_args* absorb, void* stream);

/*
 * Decode-step helpers for captured HIP graphs.  The reference caches its
 * whole decode step as one dispatch chain ("mega-chain",
 * transformer.cpp:3734-3833) and patches pos / kv_offset / seq_len into the
 * cached constants before each step.  Here those values live in device
 * memory, so a captured graph of a step's calls replays unchanged:
 *
 * kv_append replaces the two scatter_kv dispatches of a step
 * (transformer.cpp:3749-3754): row j of sequence b's new K and V goes to
 * position seq_lens[b] + j of its cache (rows past max_seq_len are dropped).
 *   k_new, v_new      [n_seq][n_new][n_kv_heads*head_dim] (16-bit)
 *   k_cache, v_cache  [n_seq][max_seq_len][n_kv_heads*head_dim],
 *                     seq_stride elements apart
 *   seq_lens          device [n_seq]: tokens held before the append
 */
typedef struct mugen_attn_kv_append_args {
    const void* k_new;
    const void* v_new;
    void* k_cache;
    void* v_cache;
    const int32_t* seq_lens;
    int64_t seq_stride;
    int32_t n_seq;
    int32_t n_new;
    int32_t row;           /* n_kv_heads * head_dim, a multiple of 8 */
    int32_t max_seq_len;
} mugen_attn_kv_append_args;
int mugen_attn_kv_append(const mugen_attn_kv_append_args* args, void* stream);

/*
 * seq_lens[b] = min(seq_lens[b] + n, max_seq_len) for b < count, on the
 * device (KVCache::advance_seq_len, kv_cache.cpp:355-357); with n_q4
 * non-null also n_q4[b] = n_q4_next[b] (commits a 4-bit store append).
 * Run once per step after every layer's calls.
 */
int mugen_attn_seq_advance(int32_t* seq_lens, int32_t n, int32_t count, int32_t max_seq_len, int32_t* n_q4,
                           const int32_t* n_q4_next, void* stream);

/*
 * scatter_kv: dst[offset + i] = src[i], i < count, 16-bit elements.
 * Replaces scatter_kv (kernel_sources.h:3018-3028) / make_scatter_kv_dp
 * (transformer.cpp:872-886): the per-token append of K/V rows or latent
 * rows into the per-layer cache.
 */
int mugen_attn_scatter_kv(const void* src, void* dst, uint64_t offset, uint64_t count,
                          void* stream);

/* last error message of the calling thread ("" if none) */
const char* mugen_attn_last_error(void);
/* library version string */
const char* mugen_attn_version(void);

/*
 * Optional kernel timing (for benchmarks): when enabled, every compute call
 * launches its kernels with a start / stop HIP event pair that the runtime
 * stamps at each kernel's own start and end (hipExtLaunchKernelGGL), on the
 * call's stream.  mugen_attn_timing_read synchronises on the recorded
 * events and returns the summed milliseconds and launch count of the kernel
 * named `kernel` ("gqa_decode", "gqa_decode_combine", "gqa_prefill",
 * "mla_decode", "mla_decode_combine", "mla_absorb", "mla_project",
 * "mla_latent_write", "kv_q4_append", "kv_append", "seq_advance",
 * "scatter_kv").
 */
int mugen_attn_timing_enable(int enable);
int mugen_attn_timing_read(const char* kernel, double* total_ms, int64_t* launches);
void mugen_attn_timing_reset(void);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* MUGEN_ATTN_H */
