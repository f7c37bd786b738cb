"""4-bit group KV store (src/core/memory/kv_cache.cpp) on the GPU: appends
quantise bit for bit like quantize_group, and GQA decode straight from the
store equals cpu_attention over KVCache::read_k / read_v (the CPU oracle's
kvq4_read + gqa_attention) within the path's tolerance."""
import ctypes

import numpy as np
import pytest
import torch

import mugen_amd
from mugen_amd import _capi
from oracle import oracle as O
from tests import cases as C

pytestmark = pytest.mark.gpu


def tokens(seed, n_seq, T, vpt, std=1.0):
    return O.round_to(O.randn(seed, (n_seq, T, vpt), 0.0, std), C.F16)[1]   # f16 bits


def dev16(bits, device):
    return C.to_dev(bits, C.F16, device)


@pytest.mark.parametrize("preserve,steps", [(32, [1, 5, 8, 3, 8, 8, 8, 8, 8, 8, 8, 8, 8, 8, 1, 1]),
                                            (0, [4, 1, 7]),
                                            (256, [64] * 5)])
def test_append_bytes_and_ring(device, preserve, steps):
    n_seq, Hk, D = 3, 4, 64
    vpt = Hk * D
    T = sum(steps)
    k = tokens(71, n_seq, T, vpt)
    v = tokens(72, n_seq, T, vpt, 0.5)
    cache = mugen_amd.KVCacheQ4(2, n_seq, Hk, D, max_seq_len=512, fp16_preserve_last=preserve,
                                max_new=max(steps), device=device)
    C.say(f"kv_q4 append preserve={preserve} steps={steps}")
    t = 0
    for n in steps:
        for layer in range(2):
            cache.append(layer, dev16(k[:, t:t + n], device), dev16(v[:, t:t + n], device))
        cache.advance()
        t += n
    torch.cuda.synchronize()
    nq = max(0, T - preserve)
    assert cache.n_q4.cpu().tolist() == [nq] * n_seq and cache.seq_lens.cpu().tolist() == [T] * n_seq
    for layer in range(2):
        for b in range(n_seq):
            for src, q4, ring in ((k, cache.q4_k, cache.ring_k), (v, cache.q4_v, cache.ring_v)):
                want = O.q4_quantize_tokens(src[b, :nq])
                got = q4[layer][b, :nq].cpu().numpy()
                assert np.array_equal(got, want), f"layer {layer} seq {b}: Q4 bytes differ"
                r = ring[layer][b].cpu().view(torch.int16).numpy().view(np.uint16)
                for tt in range(nq, T):
                    assert np.array_equal(r[tt % cache.ring], src[b, tt]), f"ring row of token {tt}"


def build_store(k, v, lens, n_q4, ring, device):
    """A store filled on the host: Q4 bytes of tokens < n_q4[b] (oracle
    quantize_token), f16 ring rows of the others up to lens[b]."""
    n_seq, T, vpt = k.shape
    rb = vpt // 32 * 20
    q4k = np.zeros((n_seq, T, rb), np.uint8)
    q4v = np.zeros_like(q4k)
    rk = np.zeros((n_seq, ring, vpt), np.uint16)
    rv = np.zeros_like(rk)
    for b in range(n_seq):
        nq = int(n_q4[b])
        q4k[b, :nq] = O.q4_quantize_tokens(k[b, :nq])
        q4v[b, :nq] = O.q4_quantize_tokens(v[b, :nq])
        for t in range(nq, int(lens[b])):
            rk[b, t % ring] = k[b, t]
            rv[b, t % ring] = v[b, t]
    return [torch.from_numpy(q4k).to(device), torch.from_numpy(q4v).to(device), dev16(rk, device), dev16(rv, device)]


def run_q4_decode(q_bits, store_t, seq_lens, n_q4, ring, preserve, Hk, D, max_T, device, num_splits=0):
    st = _capi.KvQ4Store()
    st.q4_k, st.q4_v, st.ring_k, st.ring_v = [t.data_ptr() for t in store_t]
    st.q4_seq_stride = store_t[0][0].numel()
    st.ring_seq_stride = store_t[2][0].numel()
    st.ring, st.fp16_preserve_last = ring, preserve
    B, H, _ = q_bits.shape
    q = dev16(q_bits, device)
    sl = torch.from_numpy(np.asarray(seq_lens, np.int32)).to(device)
    nq = torch.from_numpy(np.asarray(n_q4, np.int32)).to(device)
    out = torch.empty((B, H, D), dtype=torch.float32, device=device)
    a = _capi.GqaDecodeQ4Args()
    a.q, a.store, a.seq_lens, a.n_q4, a.out = q.data_ptr(), st, sl.data_ptr(), nq.data_ptr(), out.data_ptr()
    a.batch, a.n_heads, a.n_kv_heads, a.head_dim, a.max_seq_len = B, H, Hk, D, max_T
    a.num_splits, a.scale, a.out_dtype = num_splits, 0.0, _capi.F32
    L = _capi.lib()
    need = L.mugen_attn_gqa_decode_q4_workspace_size(ctypes.byref(a))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=device)
    _capi.check(L.mugen_attn_gqa_decode_q4(ctypes.byref(a), ctypes.c_void_p(ws.data_ptr()), need, None))
    torch.cuda.synchronize()
    return out.cpu().numpy()


def oracle_decode(q_bits, k, v, seq_lens, n_q4, H, Hk, D):
    n_seq, T, vpt = k.shape
    kr = np.stack([O.kvq4_read(k[b], n_q4[b]) for b in range(n_seq)])
    vr = np.stack([O.kvq4_read(v[b], n_q4[b]) for b in range(n_seq)])
    f = lambda x: x.view(np.float16).astype(np.float32)
    return O.gqa_attention(f(q_bits), f(kr).reshape(n_seq, T, Hk, D), f(vr).reshape(n_seq, T, Hk, D),
                           np.asarray(seq_lens, np.int32), H, Hk, D, T * vpt, nthreads=8)


@pytest.mark.parametrize("H,Hk,D", [(28, 4, 128), (32, 8, 64)])
@pytest.mark.parametrize("splits", [0, 1, 3])
def test_decode_from_store_ragged(device, H, Hk, D, splits):
    # sequences entirely f16, entirely Q4, and mixed with the boundary
    # inside a 32-token block; one empty sequence
    T, ring, preserve = 700, 512, 256
    lens = [700, 333, 1, 0, 450]
    n_q4 = [700 - 256, 333, 0, 0, 450 - 17]
    B = len(lens)
    k = tokens(81 + D, B, T, Hk * D)
    v = tokens(82 + D, B, T, Hk * D)
    q = tokens(83 + D, B, H, D)
    store = build_store(k, v, lens, n_q4, ring, device)
    C.say(f"gqa_decode_q4 H={H} Hk={Hk} D={D} lens={lens} n_q4={n_q4} splits={splits}")
    got = run_q4_decode(q, store, lens, n_q4, ring, preserve, Hk, D, T, device, splits)
    C.assert_close(got, oracle_decode(q, k, v, lens, n_q4, H, Hk, D), f"q4 decode splits={splits}")


def test_cache_class_end_to_end(device):
    # appends through KVCacheQ4 (Qwen-7B kv shape, preserve 256), then decode
    n_seq, H, Hk, D = 2, 28, 4, 128
    steps = [64] * 12 + [1, 1]
    T = sum(steps)
    k = tokens(91, n_seq, T, Hk * D)
    v = tokens(92, n_seq, T, Hk * D)
    cache = mugen_amd.KVCacheQ4(1, n_seq, Hk, D, max_seq_len=1024, fp16_preserve_last=256, max_new=64, device=device)
    t = 0
    for n in steps:
        cache.append(0, dev16(k[:, t:t + n], device), dev16(v[:, t:t + n], device))
        cache.advance()
        t += n
    q = tokens(93, n_seq, H, D)
    C.say(f"KVCacheQ4 end to end T={T}")
    got = cache.attention_decode(0, dev16(q, device), out_dtype=torch.float32).cpu().numpy()
    C.assert_close(got, oracle_decode(q, k, v, [T] * n_seq, [T - 256] * n_seq, H, Hk, D), "KVCacheQ4 decode")
