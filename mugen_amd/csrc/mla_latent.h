// mla_latent.h -- one token's latent-cache write (RMSNorm of c_kv, NeoX RoPE
// of k_rope, the 576-dim row appended at its position), for one wave:
// shared by the writer kernel (mla_cache.hip) and the one-launch
// latent-write + absorption kernel (mla_proj.hip).
#pragma once
#include "common.h"
#include "kernels.h"

namespace mugen_attn {

// row r of p.kv_a, lane = lane of the wave handling it.  Arithmetic
// follows the reference's float code (transformer.cpp:3930-3987): scale =
// 1 / sqrt(ss / 512 + eps) with IEEE sqrt and division, c_kv[i] =
// round((x_i * scale) * w_i), products rounded separately (no contraction).
template <int LDT>
__device__ __forceinline__ void latent_write_row(const LatentWriteParams& p, int r, int lane) {
#pragma clang fp contract(off)
    constexpr int KR = 512, ROPE = 64, C = KR + ROPE;
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

}  // namespace mugen_attn
