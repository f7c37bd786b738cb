"""The benchmark's own timed inputs, checked against the oracle: every
bench.py workload (headline MLA V3 decode, V2-Lite, verify, GQA decode,
4-bit store decode, prefill, the fallback-cost workloads, both MLA layer
workloads) is built exactly
as bench.py builds it (seeded torch draws, its context lengths), run once,
and compared with the CPU oracle on the same bytes.  So the numbers bench.py
reports come from inputs whose results are parity-checked.  (The two longest
prefill workloads are checked on their first 1024 query tokens, which the
causal mask makes independent of the rest, and on their last 128 query
tokens, which see every key.)"""
import numpy as np
import pytest
import torch

import bench
from oracle import oracle as O
from tests import cases as C

pytestmark = pytest.mark.gpu


def _bits(t):
    """device 16-bit tensor -> numpy uint16 bits; fp32 stays float32."""
    t = t.detach().contiguous().cpu()
    if t.dtype == torch.float32:
        return t.numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


def _f32(t):
    return t.detach().float().cpu().numpy()


def _run(case):
    C.say(f"bench workload {case.name}")
    case.step()
    torch.cuda.synchronize()


@pytest.mark.parametrize("name", ["mla_decode_v3", "mla_decode_v2lite", "mla_verify_v3", "mla_prefill_v2lite_n512",
                                  "mla_decode_v3_fallback_1pct", "mla_decode_v3_fallback_10pct"])
def test_mla_workloads(device, name):
    lens45 = bench.seeded_lens(45, 8, 1024, 8192)
    make = {
        "mla_decode_v3": lambda: bench.MlaDecode(device, 8, 128, 1, lens45, 8192, torch.bfloat16, torch.bfloat16,
                                                 45, name),
        "mla_decode_v2lite": lambda: bench.MlaDecode(device, 1, 16, 1, [1024], 1024, torch.float32, torch.float16,
                                                     42, name),
        "mla_verify_v3": lambda: bench.MlaDecode(device, 4, 128, 5, [32768] * 4, 32768, torch.bfloat16,
                                                 torch.bfloat16, 47, name),
        "mla_prefill_v2lite_n512": lambda: bench.MlaDecode(device, 1, 16, 512, [512], 512, torch.float32,
                                                           torch.float16, 51, name),
        "mla_decode_v3_fallback_1pct": lambda: bench.MlaDecode(device, 8, 128, 1, lens45, 8192, torch.bfloat16,
                                                               torch.bfloat16, 45, name, fallback_rows=1),
        "mla_decode_v3_fallback_10pct": lambda: bench.MlaDecode(device, 8, 128, 1, lens45, 8192, torch.bfloat16,
                                                                torch.bfloat16, 45, name, fallback_rows=13),
    }[name]
    c = make()
    _run(c)
    ref = O.mla_attention(_f32(c.q), _f32(c.lat), c.lens, c.q_len, c.H, bench.MLA_SCALE,
                          seq_stride=c.lat.shape[1] * 576, nthreads=16)
    C.assert_close(_f32(c.out), ref, name)


@pytest.mark.parametrize("name,B,lens_seed", [("gqa_decode_qwen7b_b1", 1, None), ("gqa_decode_qwen7b_b16", 16, 44)])
def test_gqa_decode_workloads(device, name, B, lens_seed):
    lens = [4096] if lens_seed is None else bench.seeded_lens(lens_seed, 16, 256, 4096)
    c = bench.GqaDecode(device, B, 28, 4, 128, lens, 4096, 43 if B == 1 else 44, name)
    _run(c)
    ref = O.gqa_attention(_f32(c.q), _f32(c.k), _f32(c.v), c.lens, 28, 4, 128, 4096 * 4 * 128, nthreads=16)
    C.assert_close(_f32(c.out), ref, name)


def test_gqa_decode_q4_workload(device):
    c = bench.GqaDecodeQ4(device, 16, 28, 4, 128, bench.seeded_lens(44, 16, 256, 4096), 4096, 44,
                          "gqa_decode_q4_qwen7b_b16")
    _run(c)
    st = c.cache
    # the K / V the store represents (KVCache::read_k / read_v): quantised
    # groups below n_q4, the f16 ring above
    nq = np.maximum(c.lens - 256, 0)
    ks, vs = [], []
    for b in range(16):
        T = int(c.lens[b])
        for q4, ring, out in ((st.q4_k[0], st.ring_k[0], ks), (st.q4_v[0], st.ring_v[0], vs)):
            deq = O.q4_dequantize_tokens(q4[b].cpu().numpy()[:T], st.vpt)
            rows = _bits(ring[b])[np.arange(T) % st.ring]
            full = np.where((np.arange(T) < nq[b])[:, None], deq, rows)
            pad = np.zeros((4096, st.vpt), np.uint16)
            pad[:T] = full
            out.append(pad)
    k = O.bits_to_f32(np.stack(ks), C.F16)
    v = O.bits_to_f32(np.stack(vs), C.F16)
    ref = O.gqa_attention(_f32(c.q), k, v, c.lens, 28, 4, 128, 4096 * st.vpt, nthreads=16)
    C.assert_close(_f32(c.out), ref, "gqa_decode_q4_qwen7b_b16")


@pytest.mark.parametrize("name,N,H,Hk,D,seed", [
    ("gqa_prefill_llama1b", 512, 32, 8, 64, 46),
    ("gqa_prefill_qwen7b_n2048", 2048, 28, 4, 128, 50),
    ("gqa_prefill_qwen7b_n8192", 8192, 28, 4, 128, 49),
])
def test_prefill_workloads(device, name, N, H, Hk, D, seed):
    c = bench.Prefill(device, N, H, Hk, D, seed, name)
    _run(c)
    n = min(N, 1024)  # causal: the first n rows depend on the first n keys only
    ref = O.gqa_prefill(_f32(c.q[:n]), _f32(c.k[:n]), _f32(c.v[:n]), n, H, Hk, D, n, 0, nthreads=16)
    C.assert_close(_f32(c.out[:n]), ref, name)
    if N > n:
        # the last 128 rows see every key: the start-offset form of the oracle
        # (row i of the tail is query N-128+i over keys [0, N-128+i])
        t = 128
        ref = O.gqa_prefill(_f32(c.q[N - t:]), _f32(c.k[:N]), _f32(c.v[:N]), t, H, Hk, D, N, N - t, nthreads=16)
        C.assert_close(_f32(c.out[N - t:]), ref, name + " last 128 rows")


@pytest.mark.parametrize("name,N,start,seed", [("gqa_prefill_qwen7b_chunk256_at7936", 256, 7936, 53),
                                               ("gqa_prefill_qwen7b_verify5_at8000", 5, 8000, 54)])
def test_prefill_chunk_workload(device, name, N, start, seed):
    # the bench's chunks over a long context: every row against the oracle's
    # start-offset form (the key ranges are split, then merged)
    H, Hk, D = 28, 4, 128
    c = bench.Prefill(device, N, H, Hk, D, seed, name, start=start)
    assert c.ws.numel() > 0
    _run(c)
    ref = O.gqa_prefill(_f32(c.q), _f32(c.k), _f32(c.v), N, H, Hk, D, start + N, start, nthreads=16)
    C.assert_close(_f32(c.out), ref, name)


@pytest.mark.parametrize("name", ["mla_layer_v3_q8_0", "mla_layer_prefill_v2lite_n512"])
def test_mla_layer_workload(device, name):
    from tests.test_mla_cache_gpu import assert_f16_match
    if name == "mla_layer_v3_q8_0":
        c = bench.MlaFull(device, 8, 128, bench.seeded_lens(45, 8, 1024, 8192), 8192, "q8_0", 48, name)
    else:
        c = bench.MlaFull(device, 1, 16, [512], 512, "q8_0", 52, name, q_len=512)
    B, q_len, H = c.q.shape[0], c.q_len, c.q.shape[2]
    lat0 = _bits(c.lat).copy()  # the latent before the step writes the new tokens' rows
    _run(c)
    freqs = O.yarn_freqs(64, c.rope[1], c.rope[2], c.rope[0])
    pos = c.pos.cpu().numpy().astype(np.int32)
    lat_ref = O.mla_latent_write(_bits(c.kv_a), _bits(c.norm_w), pos, lat0, q_len, c.max_T, freqs, 1e-6)
    got = _bits(c.lat)
    seq = np.repeat(np.arange(B), q_len)
    assert_f16_match(got[seq, pos], lat_ref[seq, pos], "latent rows written by the step")
    q = O.rope_q_f16(_bits(c.q).reshape(B * q_len, H, 192), pos, freqs).reshape(B, q_len, H, 192)
    ref = O.mla_full(O.bits_to_f32(q, C.F16), c.w_kb.cpu().numpy(), c.w_vb.cpu().numpy(), O.W_Q8_0,
                     O.bits_to_f32(lat_ref, C.F16), c.lens, q_len, H, bench.MLA_SCALE, nthreads=16)
    C.assert_close(_f32(c.out), ref, name)
