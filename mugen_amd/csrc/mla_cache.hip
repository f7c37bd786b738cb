// mla_cache.hip -- the MLA latent-cache writer: for each new token, RMSNorm
// of the compressed KV c_kv (512 dims, weight attn_kv_a_norm), NeoX RoPE of
// k_rope (64 dims, YaRN frequencies) and the append of the 576-dim latent
// row at its position in the sequence's cache (transformer.cpp:3930-3987,
// where the reference reads kv_a back to the host, normalises and rotates it
// there and scatters it with a third dispatch).
//
// One wave per token: lane l holds c_kv dims 8l..8l+7 (one 16-byte load),
// the sum of squares is a wave reduction, and lanes 0-31 rotate the 32 rope
// pairs.  The result goes straight to the cache row (16-byte stores), so a
// token costs 1152 bytes in and 1152 out.  Arithmetic follows the
// reference's float code: scale = 1 / sqrt(ss / 512 + eps) with IEEE sqrt
// and division, c_kv[i] = round((x_i * scale) * w_i), products rounded
// separately (no contraction).
#include "common.h"
#include "kernels.h"

namespace mugen_attn {

template <int LDT>
__global__ __launch_bounds__(64) void mla_latent_write_kernel(LatentWriteParams p) {
#pragma clang fp contract(off)
    constexpr int KR = 512, ROPE = 64, C = KR + ROPE;
    const int r = blockIdx.x, lane = threadIdx.x;
    const int pos = row_position(p.positions, p.seq_base, p.rows_per_seq, r);
    if (pos < 0 || pos >= p.max_seq_len) return;  // outside the cache: not written
    const uint16_t* src = p.kv_a + (int64_t)r * C;
    uint16_t* dst = p.latent + (int64_t)(r / p.rows_per_seq) * p.seq_stride + (int64_t)pos * C;
    const u32x4_t raw = *reinterpret_cast<const u32x4_t*>(src + 8 * lane);
    const u32x4_t wr = *reinterpret_cast<const u32x4_t*>(p.norm_w + 8 * lane);
    float x[8], w[8];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        x[2 * e] = lo_f32<DT_F16>(raw[e]);
        x[2 * e + 1] = hi_f32<DT_F16>(raw[e]);
        w[2 * e] = lo_f32<DT_F16>(wr[e]);
        w[2 * e + 1] = hi_f32<DT_F16>(wr[e]);
    }
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) ss += x[e] * x[e];
    ss = wave_sum(ss);
    const float scale = 1.0f / sqrtf(ss / (float)KR + p.eps);
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float a = (x[2 * e] * scale) * w[2 * e];
        const float b = (x[2 * e + 1] * scale) * w[2 * e + 1];
        if constexpr (LDT == DT_F16) {
            o[e] = uint32_t(from_f32<DT_F16>(a)) | (uint32_t(from_f32<DT_F16>(b)) << 16);
        } else {  // a bf16 cache keeps the float result rounded to bf16
            o[e] = uint32_t(from_f32<DT_BF16>(a)) | (uint32_t(from_f32<DT_BF16>(b)) << 16);
        }
    }
    *reinterpret_cast<u32x4_t*>(dst + 8 * lane) = u32x4_t{o[0], o[1], o[2], o[3]};
    if (lane < ROPE / 2) {
        const float x0 = to_f32<DT_F16>(src[KR + lane]), x1 = to_f32<DT_F16>(src[KR + lane + ROPE / 2]);
        uint16_t y0, y1;
        if constexpr (LDT == DT_F16) {
            rope_pair_f16(x0, x1, pos, p.freqs.f[lane], y0, y1);
        } else {
            const float angle = (float)pos * p.freqs.f[lane];
            const float cv = cosf(angle), sv = sinf(angle);
            y0 = from_f32<DT_BF16>(x0 * cv - x1 * sv);
            y1 = from_f32<DT_BF16>(x1 * cv + x0 * sv);
        }
        dst[KR + lane] = y0;
        dst[KR + lane + ROPE / 2] = y1;
    }
}

hipError_t launch_mla_latent_write(const LatentWriteParams& p, int latent_dt, hipStream_t st, KernelTimer* t) {
    if (latent_dt == DT_BF16)
        return launch_k(t, "mla_latent_write", mla_latent_write_kernel<DT_BF16>, dim3(p.rows), dim3(64), st, p);
    return launch_k(t, "mla_latent_write", mla_latent_write_kernel<DT_F16>, dim3(p.rows), dim3(64), st, p);
}

}  // namespace mugen_attn
