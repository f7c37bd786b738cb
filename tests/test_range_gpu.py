"""BF16 values at the edge of the f16 range (include/mugen_attn.h: BF16 V in
prefill and a BF16 MLA latent must lie within +-65504).  The prefill copies
BF16 V to f16 on chip and the MLA split partials are f16, so the contract's
whole range has to come through both paths unchanged.

Attention is linear in V: scaling V by 2^13 scales the output by 2^13, and a
power-of-two scale is exact in every float format on the way.  So the GPU
output with V scaled up to the range's edge (|v| up to 65280, the largest
bf16 value below 65504, planted in every case), divided by 2^13, must match
the oracle on the unscaled inputs to the path's usual tolerance.  For MLA the
latent is also the key, so the fp32 q is scaled by 2^-13 to keep the scores.
"""
import numpy as np
import pytest
import torch

import mugen_amd
from oracle import oracle as O
from tests import cases as C

pytestmark = pytest.mark.gpu

SCALE = 8192.0                # 2^13
EDGE = 65280.0 / SCALE        # 7.96875: bf16-exact, and 65280 after scaling


def plant(x, seed, n=64):
    """Set n entries of x (in place) to +-EDGE, a bf16-exact value."""
    rng = np.random.default_rng(seed)
    idx = rng.choice(x.size, size=min(n, x.size), replace=False)
    # index the view itself (a sliced view's reshape would be a copy)
    x[np.unravel_index(idx, x.shape)] = np.where(rng.random(idx.size) < 0.5, -EDGE, EDGE).astype(np.float32)
    return x


@pytest.mark.parametrize("N,H,Hk,D,start", [
    (100, 32, 8, 64, 0),       # short-prompt kernel
    (1100, 28, 4, 128, 0),     # warp-specialised kernel, BF16 V through the f16 copy
    (256, 28, 4, 128, 3840),   # a prompt chunk over a long context: key splits, f16 partials
])
def test_prefill_bf16_v_at_f16_edge(device, N, H, Hk, D, start):
    c = C.prefill_case(90 + N, N, H, Hk, D, start, C.BF16)
    v = plant(c["v"].copy(), 7 + N)
    ref = O.gqa_prefill(c["q"], c["k"], v, N, H, Hk, D, c["kv_len"], start, 0.0, nthreads=8)
    vs, vsb = O.round_to(v * np.float32(SCALE), C.BF16)
    assert np.array_equal(vs, v * np.float32(SCALE)) and np.abs(vs).max() == 65280.0
    C.say(f"prefill edge N={N} H={H} Hk={Hk} D={D} start={start}")
    out = mugen_amd.flash_prefill_attention(C.to_dev(c["qb"], C.BF16, device), C.to_dev(c["kb"], C.BF16, device),
                                            C.to_dev(vsb, C.BF16, device), start, out_dtype=torch.float32)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    C.assert_close(got / SCALE, ref, f"prefill bf16 V at the f16 edge N={N} start={start}")


@pytest.mark.parametrize("B,q_len,H,lens", [
    (2, 1, 16, [3000, 1500]),  # decode, many splits
    (1, 4, 128, [2048]),       # verify with DeepSeek-V3 heads
])
def test_mla_bf16_latent_at_f16_edge(device, B, q_len, H, lens):
    c = C.mla_case(95 + H, B, q_len, H, lens, q_dtype=C.F32, lat_dtype=C.BF16)
    lat = c["lat"].copy()
    plant(lat[..., :512], 11 + H)   # the value part, which the f16 partials carry
    c = dict(c, lat=lat)
    ref = C.mla_ref(c, nthreads=8)
    ls, lsb = O.round_to(lat * np.float32(SCALE), C.BF16)
    assert np.array_equal(ls, lat * np.float32(SCALE)) and np.abs(ls).max() == 65280.0
    C.say(f"mla edge B={B} q_len={q_len} H={H} lens={lens}")
    q = torch.from_numpy(c["q"] / np.float32(SCALE)).to(device)
    sl = torch.tensor(c["seq_lens"], dtype=torch.int32, device=device)
    out = mugen_amd.mla_attention(q, C.to_dev(lsb, C.BF16, device), sl, c["max_T"], scale=C.MLA_SCALE)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    C.assert_close(got / SCALE, ref, f"mla bf16 latent at the f16 edge q_len={q_len} H={H}")
