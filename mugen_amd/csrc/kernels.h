// kernels.h -- internal kernel parameter blocks and launchers (not ABI).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mugen_attn {

// YaRN frequencies of the 64 rope dims' 32 pairs, computed on the host
// (yarn_rope_freq, transformer.cpp:41-70) and passed by value.
struct RopeFreqs {
    float f[32];
};

struct KernelTimer;  // defined in capi.hip
// Per-kernel timing (mugen_attn_timing_*): when enabled, launches go through
// hipExtLaunchKernelGGL with a start / stop event pair that the runtime
// stamps at the kernel's own start and end (no launch gap included).
bool timer_pair(KernelTimer* t, hipEvent_t* start, hipEvent_t* stop);
void timer_push(KernelTimer* t, const char* name, hipEvent_t start, hipEvent_t stop);

template <typename... KArgs, typename... Args>
hipError_t launch_k(KernelTimer* t, const char* name, void (*kernel)(KArgs...), dim3 grid, dim3 block,
                    hipStream_t st, Args... args) {
    hipEvent_t a = nullptr, b = nullptr;
    if (timer_pair(t, &a, &b)) {
        hipExtLaunchKernelGGL(kernel, grid, block, 0, st, a, b, 0, args...);
        timer_push(t, name, a, b);
    } else {
        hipLaunchKernelGGL(kernel, grid, block, 0, st, args...);
    }
    return hipGetLastError();
}

struct GqaDecodeParams {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const int32_t* seq_lens;
    void* out;
    float* ws_o;   // [B][H][splits][D]   unnormalised partial outputs (D = padded head_dim)
    float* ws_ml;  // [B][H][splits][2]   (max in log2 units, sum)
    int B;
    int Hk;
    int H;
    int G;           // query heads per kv head
    int row_stride;  // elements between consecutive tokens (Hk * hd)
    int chunk;       // tokens per split
    int num_splits;
    int64_t seq_stride;
    float scale_log2;  // softmax scale * log2(e)
    // 4-bit group store (gqa_decode_q4): tokens [0, n_q4[b]) come from the
    // 20-byte groups of q4k / q4v, the others from the f16 ring in k / v
    // (token t at slot t % ring; seq_stride and row_stride describe the ring)
    const uint8_t* q4k;
    const uint8_t* q4v;
    const int32_t* n_q4;
    int64_t q4_seq_stride;  // bytes between sequences' Q4 stores
    int q4_row_bytes;       // bytes per token (Hk * D / 32 groups of 20)
    int ring;
    int per_xcd;            // 4-bit store: work items per XCD (0: blockIdx order)
    int max_T;              // device lengths are clamped to [0, max_T] (the caches' size)
    int hd;                 // head_dim of the caches, q and out (<= D, a multiple of 8)
    // prompt mode (the PF instantiation, head_dim above 128): item b is
    // query token b of one prompt over a single cache (seq_stride 0, one
    // split); it sees pf_start + b + 1 keys if pf_causal, else max_T
    int pf_start;
    int pf_causal;
};

// nwg: workgroups of the compact work list (exact, or an upper bound)
hipError_t launch_gqa_decode(const GqaDecodeParams& p, int nwg, int D, int kv_dt, int out_dt, hipStream_t st,
                             KernelTimer* t);
hipError_t launch_gqa_decode_q4(const GqaDecodeParams& p, int nwg, int D, int out_dt, hipStream_t st, KernelTimer* t);
// a prompt at head_dim 129..256 through the decode kernel's prompt mode
// (p.B = query tokens, one split, p.pf_start / p.pf_causal set)
hipError_t launch_gqa_prefill_wide(const GqaDecodeParams& p, int kv_dt, int out_dt, hipStream_t st, KernelTimer* t);

// 4-bit group store append (kv_q4.hip)
struct KvQ4AppendParams {
    const uint16_t* k_new;   // [n_seq][n_new][vpt]
    const uint16_t* v_new;
    uint8_t* q4k;
    uint8_t* q4v;
    uint16_t* ring_k;
    uint16_t* ring_v;
    const int32_t* seq_lens;
    const int32_t* n_q4;
    int32_t* n_q4_out;
    int64_t q4_seq_stride;
    int64_t ring_seq_stride;
    int n_new;
    int vpt;
    int ring;
    int preserve;
    int max_seq_len;
};
hipError_t launch_kv_q4_append(const KvQ4AppendParams& p, int n_seq, hipStream_t st, KernelTimer* t);

struct GqaPrefillParams {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    void* out;
    int N;
    int H;
    int G;
    int row_stride;  // Hk * hd
    int kv_len;
    int start_pos;
    int causal;
    float scale_log2;
    int hd;          // head_dim of q, the caches and out (<= D, a multiple of 8)
    // key splits (warp-specialised kernel; 1 = none): workgroup split s takes
    // keys [s kchunk, (s+1) kchunk) of its query block and writes the rows'
    // normalised partial O (O_s / l_s, fp16) to ws_o [N][H][ksplit][hd] and
    // (reference max in log2 units, weight sum l_s) to ws_ml
    // [N][H][ksplit][2]; the gqa_prefill_combine kernel then merges them
    // into out
    int ksplit;
    int kchunk;
    uint16_t* ws_o;
    float* ws_ml;
};

// kernel 1 (MUGEN_ATTN_PREFILL_KERNEL_BLOCK): one (query block, kv head) per
// workgroup, every wave doing S, softmax and PV; 2 (_WS): warp-specialised
// S / PV waves
hipError_t launch_gqa_prefill(const GqaPrefillParams& p, int Hk, int D, int dt, int out_dt, int kernel,
                              hipStream_t st, KernelTimer* t);
// kernel 3 (MUGEN_ATTN_PREFILL_KERNEL_SHORT): every key a query block sees
// held in LDS; serves head_dim 64 (unpadded), at most 4 heads per kv head
// and a kv range (start_pos + N causal, kv_len otherwise) of at most 512
bool gqa_prefill_short_fits(const GqaPrefillParams& p, int D);
// key steps of the warp-specialised kernel (32 or 64 keys) and its
// workgroups per CU, for the split planner (dt as for launch_gqa_prefill)
int gqa_prefill_ws_step_keys(int G, int dt);
int gqa_prefill_ws_blocks_per_cu(int G, int D);
int gqa_prefill_ws_slices(int G);
// most key splits the planner gives a prefill call (the merge unrolls to it)
constexpr int kPrefillMaxSplits = 32;
// dt code for launch_gqa_prefill: bf16 q / K with V already converted to fp16
constexpr int kDtBf16V16 = 100;
// fp16 copy of n bf16 values (n a multiple of 8, 16-byte aligned buffers)
hipError_t launch_v_to_f16(const uint16_t* v, uint16_t* dst, int64_t n, hipStream_t st, KernelTimer* t);

struct MlaParams {
    const void* q;         // [B][q_len*H][576], f32 or the latent dtype
    const uint16_t* lat;   // latent cache
    const int32_t* seq_lens;
    void* out;             // [B][q_len*H][512]
    float* ws_o;           // [B][splits][nq][16][64] 16-byte pairs of fp16x4 fragments of o/l (see blob_pair)
    float* ws_ml;          // [B][splits][R][2]
    int B;
    int q_len;
    int H;
    int R;                 // q_len * H rows per sequence
    int nrb;               // row blocks per sequence (ceil(R / rows per block))
    int nq;                // 16-row blocks per sequence (ceil(R / 16))
    int units;             // (sequence, split, row block) work units the grid covers (upper bound)
    int chunk;
    int num_splits;
    int max_T;             // device lengths are clamped to [0, max_T] (the cache's size)
    int64_t seq_stride;
    float scale_log2;
};

// every kernel reads a sequence's length through this clamp: a device value
// past the cache (or negative) never indexes outside the cache or the
// workspace that the host sized from max_T
__device__ __forceinline__ int clamp_len(int t, int max_T) { return min(max(t, 0), max_T); }

// query rows of one MLA workgroup, and tokens per LDS tile, of a kernel
// (MUGEN_ATTN_MLA_KERNEL_ROWS or _WS)
int mla_rows_per_block(int kernel);
int mla_tile_tokens(int kernel);
hipError_t launch_mla_decode(const MlaParams& p, int kernel, int q_dt, int lat_dt, int out_dt,
                             hipStream_t st, KernelTimer* t);

// MLA absorption / up-projection (mla_proj.hip)
enum { W_F16 = MUGEN_ATTN_W_F16, W_Q4_0 = MUGEN_ATTN_W_Q4_0, W_Q8_0 = MUGEN_ATTN_W_Q8_0 };
struct MlaProjParams {
    const void* in;   // absorb: q f16 [rows][H][nope+rope]; project: o f32 [rows][H][kv_rank]
    const void* w;    // weight rows in the GGML block encoding
    void* out;        // absorb: q_abs [rows][H][kv_rank+rope]; project: [rows][H][v_head]
    int rows;
    int H;
    const int32_t* positions;  // absorb: RoPE position of each row (null: see seq_base)
    RopeFreqs freqs;
    const int32_t* seq_base;   // absorb, positions null: row r at seq_base[r / rows_per_seq] + r % rows_per_seq
    int rows_per_seq;
};
hipError_t launch_mla_absorb(const MlaProjParams& p, int w_type, int out_dt, hipStream_t st, KernelTimer* t);
hipError_t launch_mla_project(const MlaProjParams& p, int w_type, int out_dt, hipStream_t st, KernelTimer* t);

// MLA latent-cache writer (mla_cache.hip)
struct LatentWriteParams {
    const uint16_t* kv_a;      // [rows][576] f16
    const uint16_t* norm_w;    // [512] f16
    const int32_t* positions;  // [rows], or null: seq_base[r / rows_per_seq] + r % rows_per_seq
    const int32_t* seq_base;
    uint16_t* latent;          // [n_seq][max_seq_len][576]
    int rows;
    int rows_per_seq;
    int max_seq_len;
    int64_t seq_stride;
    float eps;
    RopeFreqs freqs;
};
hipError_t launch_mla_latent_write(const LatentWriteParams& p, int latent_dt, hipStream_t st, KernelTimer* t);
// latent write + absorption in one launch at decode sizes (mla_proj.hip)
hipError_t launch_mla_prepare(const MlaProjParams& pa, const LatentWriteParams& pl, int w_type, int out_dt,
                              int lat_dt, hipStream_t st, KernelTimer* t);

// decode-step helpers (engine.hip)
struct KvAppendParams {
    const uint16_t* k_new;  // [n_seq][n_new][row]
    const uint16_t* v_new;
    uint16_t* k_cache;      // [n_seq][max_seq_len][row], seq_stride elements apart
    uint16_t* v_cache;
    const int32_t* seq_lens;
    int64_t seq_stride;
    int row;                // Hk * D
    int n_new;
    int max_seq_len;
};
hipError_t launch_kv_append(const KvAppendParams& p, int n_seq, hipStream_t st, KernelTimer* t);
hipError_t launch_seq_advance(int32_t* seq_lens, int n, int count, int max_seq_len, int32_t* n_q4,
                              const int32_t* n_q4_next, hipStream_t st, KernelTimer* t);

hipError_t launch_scatter_kv(const uint16_t* src, uint16_t* dst, uint64_t offset, uint64_t count,
                             hipStream_t st, KernelTimer* t);

}  // namespace mugen_attn
