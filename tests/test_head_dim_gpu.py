"""head_dim other than 64 / 128 (multiples of 8 up to 256: the reference's
cpu_attention takes any head_dim, transformer.cpp:2441-2485; its unit-test
model uses 16).  The kernels run on the next supported width with the extra
dims masked, so these check both the results (against the oracle) and that
nothing is written past the head_dim-wide output rows (canary guard bands
around the outputs)."""
import numpy as np
import pytest
import torch

import mugen_amd
from mugen_amd import _capi
from tests import cases as C
from tests.test_bounds_gpu import Guarded

pytestmark = pytest.mark.gpu

HEAD_DIMS = [8, 16, 32, 48, 80, 96, 120]


@pytest.mark.parametrize("D", HEAD_DIMS)
def test_decode_head_dim(device, D):
    lens = [1, 700, 0, 333]
    for dt in (C.F16, C.BF16):
        c = C.gqa_decode_case(900 + D, 4, 8, 2, D, lens, max_T=1024, dtype=dt)
        ref = C.gqa_decode_ref(c)
        q = C.to_dev(c["qb"], dt, device)
        k = C.to_dev(c["kb"], dt, device)
        v = C.to_dev(c["vb"], dt, device)
        sl = torch.from_numpy(c["seq_lens"]).to(device)
        for splits in (0, 1, 5):
            C.say(f"gqa_decode head_dim={D} dtype={dt} splits={splits}")
            out = Guarded((4, 8, D), torch.float32, device)
            mugen_amd.attention_decode(q, k, v, sl, 1024, out=out.t, num_splits=splits)
            assert out.intact(), f"guard band overwritten (D={D}, splits={splits})"
            C.assert_close(out.t.cpu().numpy(), ref, f"decode head_dim={D} dtype={dt} splits={splits}")


@pytest.mark.parametrize("D", HEAD_DIMS)
def test_prefill_head_dim(device, D):
    N, start = 150, 40
    for dt in (C.BF16, C.F16):
        c = C.prefill_case(950 + D, N, 12, 3, D, start, dt)
        ref = C.prefill_ref(c)
        q = C.to_dev(c["qb"], dt, device)
        k = C.to_dev(c["kb"], dt, device)
        v = C.to_dev(c["vb"], dt, device)
        for kernel in (_capi.PREFILL_KERNEL_BLOCK, _capi.PREFILL_KERNEL_WS):
            C.say(f"gqa_prefill head_dim={D} dtype={dt} kernel={kernel}")
            out = Guarded((N, 12, D), torch.float32, device)
            mugen_amd.flash_prefill_attention(q, k, v, start, out=out.t, kernel=kernel)
            assert out.intact(), f"guard band overwritten (D={D}, kernel={kernel})"
            C.assert_close(out.t.cpu().numpy(), ref, f"prefill head_dim={D} dtype={dt} kernel={kernel}")


def test_reference_unit_test_model(device):
    # the reference's test model: 4 heads, 2 KV heads, head_dim 16
    c = C.gqa_decode_case(977, 1, 4, 2, 16, [37], dtype=C.F16)
    out = mugen_amd.attention_decode(C.to_dev(c["qb"], C.F16, device), C.to_dev(c["kb"], C.F16, device),
                                     C.to_dev(c["vb"], C.F16, device), torch.from_numpy(c["seq_lens"]).to(device),
                                     c["max_T"], out_dtype=torch.float32)
    torch.cuda.synchronize()
    C.assert_close(out.cpu().numpy(), C.gqa_decode_ref(c), "head_dim 16 model")
    p = C.prefill_case(978, 37, 4, 2, 16, 0, C.F16)
    got = mugen_amd.flash_prefill_attention(C.to_dev(p["qb"], C.F16, device), C.to_dev(p["kb"], C.F16, device),
                                            C.to_dev(p["vb"], C.F16, device), 0, out_dtype=torch.float32)
    torch.cuda.synchronize()
    C.assert_close(got.cpu().numpy(), C.prefill_ref(p), "head_dim 16 prompt")
    assert np.isfinite(got.cpu().numpy()).all()


WIDE = [256, 160, 136, 200]  # the 256-wide builds: native, and padded


@pytest.mark.parametrize("D", WIDE)
def test_decode_wide_head_dim(device, D):
    # head_dim 129..256: one wave per SIMD; ragged lengths, an empty
    # sequence, automatic and forced split counts
    lens = [1, 900, 0, 2500]
    for dt in (C.F16, C.BF16):
        c = C.gqa_decode_case(910 + D, 4, 16, 4, D, lens, max_T=2560, dtype=dt)
        ref = C.gqa_decode_ref(c, nthreads=8)
        q = C.to_dev(c["qb"], dt, device)
        k = C.to_dev(c["kb"], dt, device)
        v = C.to_dev(c["vb"], dt, device)
        sl = torch.from_numpy(c["seq_lens"]).to(device)
        for splits in (0, 1, 7):
            C.say(f"gqa_decode wide head_dim={D} dtype={dt} splits={splits}")
            out = Guarded((4, 16, D), torch.float32, device)
            mugen_amd.attention_decode(q, k, v, sl, 2560, out=out.t, num_splits=splits)
            assert out.intact(), f"guard band overwritten (D={D}, splits={splits})"
            C.assert_close(out.t.cpu().numpy(), ref, f"decode head_dim={D} dtype={dt} splits={splits}")


@pytest.mark.parametrize("D", [256, 200])
@pytest.mark.parametrize("N,start,causal", [(150, 40, True), (1, 0, True), (70, 0, False)])
def test_prefill_wide_head_dim(device, D, N, start, causal):
    # head_dim above 128: the per-token rule (query i over start + i + 1
    # keys), each token in its own workgroup; non-causal: every key
    H, Hk = 8, 2
    for dt in (C.BF16, C.F16):
        c = C.prefill_case(960 + D + N, N, H, Hk, D, start, dt)
        if causal:
            ref = C.prefill_ref(c, nthreads=8)
        else:
            kv = c["kv_len"]
            ref = C.O.gqa_attention(c["q"], c["k"].reshape(1, kv, Hk, D).repeat(N, 0),
                                    c["v"].reshape(1, kv, Hk, D).repeat(N, 0), [kv] * N, H, Hk, D, kv * Hk * D)
        q = C.to_dev(c["qb"], dt, device)
        k = C.to_dev(c["kb"], dt, device)
        v = C.to_dev(c["vb"], dt, device)
        C.say(f"gqa_prefill wide head_dim={D} N={N} start={start} causal={causal} dtype={dt}")
        out = Guarded((N, H, D), torch.float32, device)
        mugen_amd.flash_prefill_attention(q, k, v, start, causal=causal, out=out.t)
        assert out.intact(), f"guard band overwritten (D={D})"
        C.assert_close(out.t.cpu().numpy(), ref, f"prefill head_dim={D} N={N} causal={causal} dtype={dt}")
        with pytest.raises(_capi.MugenAttnError):  # one kernel above 128
            mugen_amd.flash_prefill_attention(q, k, v, start, causal=causal, kernel=_capi.PREFILL_KERNEL_WS)


@pytest.mark.parametrize("n", [130, 300])
def test_q4_store_head_dim_256(device, n):
    # the 4-bit group store at head_dim 256 (8 groups per head, two per lane
    # in the K contraction): appended on the GPU in chunks, decoded from the
    # store, against KVCache::read_k / read_v (the newest 32 tokens f16)
    from oracle import oracle as O
    kv = mugen_amd.KVCacheQ4(1, 2, 2, 256, max_seq_len=512, fp16_preserve_last=32, max_new=64, device=device)
    k = O.round_to(O.randn(931 + n, (2, n, 512)), C.F16)[1]
    v = O.round_to(O.randn(932 + n, (2, n, 512)), C.F16)[1]
    C.say(f"gqa_decode_q4 head_dim 256, {n} tokens")
    for t in range(0, n, 50):
        m = min(50, n - t)
        kv.append(0, C.to_dev(k[:, t:t + m], C.F16, device), C.to_dev(v[:, t:t + m], C.F16, device))
        kv.advance()
    q = O.round_to(O.randn(933, (2, 8, 256)), C.F16)[1]
    out = kv.attention_decode(0, C.to_dev(q, C.F16, device), out_dtype=torch.float32)
    fv = lambda x: x.view(np.float16).astype(np.float32)
    kk = np.stack([O.kvq4_read(k[b], n - 32) for b in range(2)])
    vv = np.stack([O.kvq4_read(v[b], n - 32) for b in range(2)])
    ref = O.gqa_attention(fv(q), fv(kk), fv(vv), [n, n], 8, 2, 256, n * 512)
    C.assert_close(out.cpu().numpy(), ref, f"q4 store head_dim 256, {n} tokens")
