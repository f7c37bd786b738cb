// engine.hip -- the two small kernels that make a decode step's attention
// calls replayable as one captured HIP graph (the equivalent of the
// reference's cached "mega-chain", transformer.cpp:3734-3833, which patches
// pos / kv_offset / seq_len into its cached dispatch constants before every
// step): every per-step value lives in device memory instead, so a captured
// graph needs no patching.
//
//  * kv_append: K and V rows of the new tokens written at the sequence's
//    current length (device seq_lens), replacing the two scatter_kv
//    dispatches with a host offset (transformer.cpp:3749-3754);
//  * seq_advance: seq_lens += n on the device (KVCache::advance_seq_len,
//    kv_cache.cpp:355-357), optionally committing the 4-bit store's n_q4.
#include "common.h"
#include "kernels.h"

namespace mugen_attn {

// grid (n_new, n_seq): one token row of K and V per workgroup
__global__ __launch_bounds__(256) void kv_append_kernel(KvAppendParams p) {
    const int j = blockIdx.x, b = blockIdx.y;
    const int t = p.seq_lens[b] + j;
    if (t < 0 || t >= p.max_seq_len) return;  // past the cache: dropped
    const int64_t src = ((int64_t)b * p.n_new + j) * p.row;
    const int64_t dst = (int64_t)b * p.seq_stride + (int64_t)t * p.row;
    for (int i = 8 * threadIdx.x; i < p.row; i += 8 * 256) {
        *reinterpret_cast<u32x4_t*>(p.k_cache + dst + i) = load16(p.k_new + src + i);
        *reinterpret_cast<u32x4_t*>(p.v_cache + dst + i) = load16(p.v_new + src + i);
    }
}

__global__ __launch_bounds__(256) void seq_advance_kernel(int32_t* seq_lens, int n, int count, int max_seq_len,
                                                          int32_t* n_q4, const int32_t* n_q4_next) {
    const int b = blockIdx.x * 256 + threadIdx.x;
    if (b >= count) return;
    seq_lens[b] = min(seq_lens[b] + n, max_seq_len);
    if (n_q4) n_q4[b] = n_q4_next[b];
}

hipError_t launch_kv_append(const KvAppendParams& p, int n_seq, hipStream_t st, KernelTimer* t) {
    return launch_k(t, "kv_append", kv_append_kernel, dim3(p.n_new, n_seq), dim3(256), st, p);
}

hipError_t launch_seq_advance(int32_t* seq_lens, int n, int count, int max_seq_len, int32_t* n_q4,
                              const int32_t* n_q4_next, hipStream_t st, KernelTimer* t) {
    return launch_k(t, "seq_advance", seq_advance_kernel, dim3((count + 255) / 256), dim3(256), st, seq_lens, n,
                    count, max_seq_len, n_q4, n_q4_next);
}

}  // namespace mugen_attn
