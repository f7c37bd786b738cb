// kv_q4.hip -- append to the 4-bit group KV store (KVCache::append,
// src/core/memory/kv_cache.cpp:163-216).
//
// Layout per sequence: Q4 groups of every quantised token at its absolute
// position ([max_seq_len][vpt/32][20 B]) and an f16 ring of `ring` token
// rows (a power of two) holding the newest ones (token t at slot
// t % ring).  Appending n_new
// tokens to a sequence holding T tokens of which n_q4 are quantised leaves
// the newest fp16_preserve_last in f16 and quantises the ones that age out:
// positions n_q4 .. n_q4 + q - 1 with q = max(0, T - n_q4 + n_new -
// preserve), exactly the tokens the reference's one-token appends quantise.
// With ring >= preserve + n_new, the ring slots read by those quantisations
// and the slots written by the new tokens are distinct, so one launch does
// both.
//
// Grid (2 * n_new, n_seq), one wave per job: job j < n_new writes new token
// j to its ring slot (unless it is quantised right away), job n_new + j
// quantises aged token n_q4 + j (from the ring, or from the new tokens when
// preserve < n_new), one lane per 32-value group:
//   quantize_group (kv_cache.cpp:21-56): min / max over the 32 f16 values,
//   scale = f16(range / 15) (0 for a constant group), nibble =
//   min(15, roundf((v - min) / scale)), value 2i in the low nibble of byte i.
#include "common.h"
#include "kernels.h"

namespace mugen_attn {

__device__ __forceinline__ void quantize_group32(const uint16_t* src, uint8_t* dst) {
#pragma clang fp contract(off)
    uint32_t w[16];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(src + 8 * i);
        w[4 * i] = v[0];
        w[4 * i + 1] = v[1];
        w[4 * i + 2] = v[2];
        w[4 * i + 3] = v[3];
    }
    float x[32];
#pragma unroll
    for (int i = 0; i < 16; i++) {
        x[2 * i] = lo_f32<DT_F16>(w[i]);
        x[2 * i + 1] = hi_f32<DT_F16>(w[i]);
    }
    float lo = x[0], hi = x[0];
    uint32_t lo_bits = w[0] & 0xffffu;
#pragma unroll
    for (int i = 1; i < 32; i++) {  // first occurrence wins, as the reference's strict compares
        if (x[i] < lo) {
            lo = x[i];
            lo_bits = (i & 1) ? (w[i >> 1] >> 16) : (w[i >> 1] & 0xffffu);
        }
        hi = x[i] > hi ? x[i] : hi;
    }
    const float range = hi - lo;
    const uint32_t sbits = range == 0.0f ? 0u : uint32_t(from_f32<DT_F16>(range / 15.0f));
    const float sf = to_f32<DT_F16>(uint16_t(sbits)), mf = to_f32<DT_F16>(uint16_t(lo_bits));
    uint32_t packed[4] = {0u, 0u, 0u, 0u};
    if (sf > 0.0f) {
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float a = fminf(15.0f, roundf((x[2 * i] - mf) / sf));
            const float c = fminf(15.0f, roundf((x[2 * i + 1] - mf) / sf));
            packed[i >> 2] |= ((uint32_t(c) << 4) | uint32_t(a)) << (8 * (i & 3));
        }
    }
    // 20 bytes at a 4-byte aligned address: five dword stores
    uint32_t* d = reinterpret_cast<uint32_t*>(dst);
    d[0] = sbits | (lo_bits << 16);
    d[1] = packed[0];
    d[2] = packed[1];
    d[3] = packed[2];
    d[4] = packed[3];
}

__global__ __launch_bounds__(64) void kv_q4_append_kernel(KvQ4AppendParams p) {
    const int b = blockIdx.y, job = blockIdx.x, lane = threadIdx.x;
    // lengths clamped to the store: a device value past max_seq_len (or
    // negative) never indexes outside it
    const int T = clamp_len(p.seq_lens[b], p.max_seq_len), nq = clamp_len(p.n_q4[b], T);
    const int q = max(0, T - nq + p.n_new - p.preserve);
    // tokens at positions >= max_seq_len are dropped, so they are not counted
    if (job == 0 && lane == 0) p.n_q4_out[b] = min(nq + q, p.max_seq_len);
    const uint16_t* knew = p.k_new + (int64_t)b * p.n_new * p.vpt;
    const uint16_t* vnew = p.v_new + (int64_t)b * p.n_new * p.vpt;
    uint16_t* rk = p.ring_k + (int64_t)b * p.ring_seq_stride;
    uint16_t* rv = p.ring_v + (int64_t)b * p.ring_seq_stride;
    if (job < p.n_new) {
        const int t = T + job;
        if (t < nq + q || t >= p.max_seq_len) return;  // quantised right away / past the cache
        const int64_t slot = (int64_t)(t & (p.ring - 1)) * p.vpt;
        for (int i = 8 * lane; i < p.vpt; i += 8 * 64) {
            *reinterpret_cast<u32x4_t*>(rk + slot + i) = load16(knew + (int64_t)job * p.vpt + i);
            *reinterpret_cast<u32x4_t*>(rv + slot + i) = load16(vnew + (int64_t)job * p.vpt + i);
        }
        return;
    }
    const int j = job - p.n_new;
    if (j >= q) return;
    const int t = nq + j;
    if (t >= p.max_seq_len) return;
    const uint16_t* ks = t < T ? rk + (int64_t)(t & (p.ring - 1)) * p.vpt : knew + (int64_t)(t - T) * p.vpt;
    const uint16_t* vs = t < T ? rv + (int64_t)(t & (p.ring - 1)) * p.vpt : vnew + (int64_t)(t - T) * p.vpt;
    const int groups = p.vpt / 32;
    const int64_t row = (int64_t)b * p.q4_seq_stride + (int64_t)t * groups * 20;
    for (int g = lane; g < groups; g += 64) {
        quantize_group32(ks + 32 * g, p.q4k + row + 20 * g);
        quantize_group32(vs + 32 * g, p.q4v + row + 20 * g);
    }
}

hipError_t launch_kv_q4_append(const KvQ4AppendParams& p, int n_seq, hipStream_t st, KernelTimer* t) {
    return launch_k(t, "kv_q4_append", kv_q4_append_kernel, dim3(2 * p.n_new, n_seq), dim3(64), st, p);
}

}  // namespace mugen_attn
