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
// token costs 1152 bytes in and 1152 out (latent_write_row, mla_latent.h).
#include "common.h"
#include "kernels.h"
#include "mla_latent.h"

namespace mugen_attn {

template <int LDT>
__global__ __launch_bounds__(64) void mla_latent_write_kernel(LatentWriteParams p) {
    latent_write_row<LDT>(p, blockIdx.x, threadIdx.x);
}

hipError_t launch_mla_latent_write(const LatentWriteParams& p, int latent_dt, hipStream_t st, KernelTimer* t) {
    if (latent_dt == DT_BF16)
        return launch_k(t, "mla_latent_write", mla_latent_write_kernel<DT_BF16>, dim3(p.rows), dim3(64), st, p);
    return launch_k(t, "mla_latent_write", mla_latent_write_kernel<DT_F16>, dim3(p.rows), dim3(64), st, p);
}

}  // namespace mugen_attn
