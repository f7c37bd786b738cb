"""Python binding of the CPU oracle (oracle/attn_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  The product package
``mugen_amd`` never imports this module.

Each function restates one reference routine; the citations live in
attn_oracle.c's header and in the docstrings below.  An fp64 numpy
brute-force (``*_np64``) is provided as an independent second formulation
(vectorised, different summation order) for cross-checking the C code.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_attn.so")
_lib = None

F32, F16, BF16 = 0, 1, 2


def build() -> str:
    """Compile the oracle with gcc (make); returns the .so path."""
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle_attn.so"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        # MUGEN_ORACLE_LIB: another build of this same file (the sanitizer
        # run of the oracle's tests loads an UBSan-instrumented one)
        path = os.environ.get("MUGEN_ORACLE_LIB", _LIB_PATH)
        if path == _LIB_PATH and not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(path)
        P = ctypes.c_void_p
        i32, i64, f32 = ctypes.c_int, ctypes.c_int64, ctypes.c_float
        L.oracle_randn.argtypes = [ctypes.c_uint64, i64, f32, f32, P]
        L.oracle_randint.argtypes = [ctypes.c_uint64, i64, ctypes.c_int32, ctypes.c_int32, P]
        L.oracle_mt64_first.argtypes = [ctypes.c_uint64, i64]
        L.oracle_mt64_first.restype = ctypes.c_uint64
        L.oracle_round_to_dtype.argtypes = [P, P, i64, i32]
        L.oracle_gqa_attention_f32.argtypes = [P, P, P, P, P, i32, i32, i32, i32, i64, f32, i32]
        L.oracle_gqa_attention_f64.argtypes = [P, P, P, P, P, i32, i32, i32, i32, i64, f32]
        L.oracle_gqa_prefill_f32.argtypes = [P, P, P, P, i32, i32, i32, i32, i32, i32, f32, i32]
        L.oracle_gqa_prefill_f64.argtypes = [P, P, P, P, i32, i32, i32, i32, i32, i32, f32]
        L.oracle_mla_attention_f32.argtypes = [P, P, P, P, i32, i32, i32, i32, i32, i64, f32, i32]
        L.oracle_mla_attention_f64.argtypes = [P, P, P, P, i32, i32, i32, i32, i32, i64, f32]
        L.oracle_scatter_kv.argtypes = [P, P, i64, i64]
        L.oracle_dequant_row.argtypes = [P, i32, i64, i32, P]
        L.oracle_mla_absorb.argtypes = [P, P, i32, P, i32, i32, i32, i32, i32]
        L.oracle_mla_project.argtypes = [P, P, i32, P, i32, i32, i32, i32]
        L.oracle_q4_quantize_group.argtypes = [P, P, i32]
        L.oracle_q4_dequantize_group.argtypes = [P, P]
        L.oracle_q4_quantize_token.argtypes = [P, P, i32]
        L.oracle_q4_dequantize_token.argtypes = [P, P, i32]
        L.oracle_kvq4_read.argtypes = [P, P, i32, i32, i32]
        L.oracle_yarn_rope_freq.argtypes = [i32, i32, f32, i32, f32]
        L.oracle_yarn_rope_freq.restype = f32
        L.oracle_rope_neox_f16.argtypes = [P, i32, i32, P]
        L.oracle_mla_kv_prepare.argtypes = [P, P, i32, i32, f32, i32, P]
        L.oracle_mla_latent_write.argtypes = [P, P, P, P, i32, i32, i64, i32, i32, i32, f32, P]
        L.oracle_num_threads.restype = ctypes.c_int
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------- inputs

def randn(seed: int, shape, mean=0.0, std=1.0) -> np.ndarray:
    """mt19937_64(seed) + Box-Muller normal draws, float32."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    lib().oracle_randn(seed, n, mean, std, _p(out))
    return out.reshape(shape)


def randint(seed: int, n: int, lo: int, hi: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    lib().oracle_randint(seed, n, lo, hi, _p(out))
    return out


def round_to(x: np.ndarray, dtype: int):
    """Round float32 array to fp16/bf16 values. Returns (values_f32, bits_u16)."""
    v = np.ascontiguousarray(x, dtype=np.float32).copy()
    bits = np.zeros(v.shape, dtype=np.uint16)
    lib().oracle_round_to_dtype(_p(v), _p(bits), v.size, dtype)
    return v, bits


def bits_to_f32(bits: np.ndarray, dtype: int) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    if dtype == BF16:
        return (b.astype(np.uint32) << 16).view(np.float32)
    if dtype == F16:
        return b.view(np.float16).astype(np.float32)
    raise ValueError(dtype)


# ---------------------------------------------------------------- oracles

def gqa_attention(q, k, v, seq_lens, H, Hk, D, seq_stride, scale=0.0, f64=False, nthreads=1):
    """cpu_attention (transformer.cpp:2441-2485), batched over sequences.

    q [B,H,D] f32 values; k/v flat f32 arrays, sequence b at b*seq_stride,
    token-major [T][Hk*D]; seq_lens int32 [B].  Returns [B,H,D] (f32 or f64).
    """
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    sl = np.ascontiguousarray(seq_lens, np.int32)
    B = sl.size
    out = np.empty((B, H, D), np.float64 if f64 else np.float32)
    if f64:
        lib().oracle_gqa_attention_f64(_p(q), _p(k), _p(v), _p(sl), _p(out), B, H, Hk, D, seq_stride, scale)
    else:
        lib().oracle_gqa_attention_f32(_p(q), _p(k), _p(v), _p(sl), _p(out), B, H, Hk, D, seq_stride, scale, nthreads)
    return out


def gqa_prefill(q, k, v, N, H, Hk, D, kv_len, start, scale=0.0, f64=False, nthreads=1):
    """flash_prefill_attention semantics (kernel_sources.h:2769-2896):
    token i sees keys [0, start+i].  q [N,H,D]; k/v [kv_len, Hk*D]."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    out = np.empty((N, H, D), np.float64 if f64 else np.float32)
    if f64:
        lib().oracle_gqa_prefill_f64(_p(q), _p(k), _p(v), _p(out), N, H, Hk, D, kv_len, start, scale)
    else:
        lib().oracle_gqa_prefill_f32(_p(q), _p(k), _p(v), _p(out), N, H, Hk, D, kv_len, start, scale, nthreads)
    return out


def mla_attention(q, latent, seq_lens, q_len, H, scale, kv_rank=512, rope=64, seq_stride=None,
                  f64=False, nthreads=1):
    """Latent core of cpu_mla_attention (transformer.cpp:2576-2608).

    q [B,q_len,H,kv_rank+rope]; latent flat, sequence b at b*seq_stride,
    token rows of kv_rank+rope; query i sees seq_len-q_len+i+1 tokens
    (transformer.cpp:1325-1337).  Returns [B,q_len,H,kv_rank].
    """
    q = np.ascontiguousarray(q, np.float32)
    lat = np.ascontiguousarray(latent, np.float32)
    sl = np.ascontiguousarray(seq_lens, np.int32)
    B = sl.size
    if seq_stride is None:
        seq_stride = lat.size // B
    out = np.empty((B, q_len, H, kv_rank), np.float64 if f64 else np.float32)
    if f64:
        lib().oracle_mla_attention_f64(_p(q), _p(lat), _p(sl), _p(out), B, q_len, H, kv_rank, rope,
                                       seq_stride, scale)
    else:
        lib().oracle_mla_attention_f32(_p(q), _p(lat), _p(sl), _p(out), B, q_len, H, kv_rank, rope,
                                       seq_stride, scale, nthreads)
    return out


# GGML weight type ids (src/model/ggml_types.h:12-20) accepted by the MLA
# absorption / up-projection
W_F16, W_Q4_0, W_Q8_0 = 1, 2, 8


def wrow_bytes(w_type: int, K: int) -> int:
    return {W_F16: 2 * K, W_Q8_0: K // 32 * 34, W_Q4_0: K // 32 * 18}[w_type]


def dequant_rows(w: np.ndarray, w_type: int, K: int) -> np.ndarray:
    """dequant_weight_row (transformer.cpp:2488-2534) applied to every row
    of a [rows, row_bytes] uint8 buffer; returns [rows, K] fp32."""
    w = np.ascontiguousarray(w, np.uint8)
    rows = w.shape[0]
    out = np.empty((rows, K), np.float32)
    for r in range(rows):
        lib().oracle_dequant_row(_p(w), w_type, r, K, _p(out[r]))
    return out


def mla_absorb(q, w_kb, w_type, H, nope=128, rope=64, kv_rank=512):
    """q_absorbed = q_nope x k_b (transformer.cpp:2563-2573) ++ q_rope.
    q [..., H, nope+rope] (f16 values as float32); w_kb [H*nope, row_bytes]
    uint8.  Returns [..., H, kv_rank+rope] fp32."""
    q = np.ascontiguousarray(q, np.float32)
    lead = q.shape[:-2]
    rows = int(np.prod(lead)) if lead else 1
    out = np.empty(lead + (H, kv_rank + rope), np.float32)
    lib().oracle_mla_absorb(_p(q), _p(np.ascontiguousarray(w_kb, np.uint8)), w_type, _p(out), rows, H, nope, rope,
                            kv_rank)
    return out


def mla_project(o, w_vb, w_type, H, kv_rank=512, v_head=128):
    """out_h = out_comp x v_b^T rounded to f16 (transformer.cpp:2610-2620).
    o [..., H, kv_rank] fp32; w_vb [H*v_head, row_bytes] uint8.  Returns
    [..., H, v_head] fp32 holding f16 values."""
    o = np.ascontiguousarray(o, np.float32)
    lead = o.shape[:-2]
    rows = int(np.prod(lead)) if lead else 1
    out = np.empty(lead + (H, v_head), np.float32)
    lib().oracle_mla_project(_p(o), _p(np.ascontiguousarray(w_vb, np.uint8)), w_type, _p(out), rows, H, kv_rank,
                             v_head)
    return out


def yarn_freqs(rope_dim=64, factor=0.0, original_ctx=0, theta=10000.0):
    """yarn_rope_freq (transformer.cpp:41-70) for i < rope_dim/2, float32."""
    return np.array([lib().oracle_yarn_rope_freq(i, rope_dim, factor, original_ctx, theta)
                     for i in range(rope_dim // 2)], np.float32)


def rope_neox_f16(x_bits, pos, freqs):
    """NeoX RoPE of one f16 vector (transformer.cpp:3903-3917); uint16 bits in/out."""
    x = np.ascontiguousarray(x_bits, np.uint16).copy()
    lib().oracle_rope_neox_f16(_p(x), x.size, int(pos), _p(np.ascontiguousarray(freqs, np.float32)))
    return x


def rope_q_f16(q_bits, positions, freqs, nope=128):
    """q rope stage (transformer.cpp:3882-3921): q [rows, H, nope+rope]
    uint16 f16 bits; the rope part of every head of row r rotated by
    positions[r]."""
    q = np.ascontiguousarray(q_bits, np.uint16).copy()
    rows = q.shape[0]
    for r in range(rows):
        for h in range(q.shape[1]):
            q[r, h, nope:] = rope_neox_f16(q[r, h, nope:], positions[r], freqs)
    return q


def mla_kv_prepare(kva_bits, norm_w_bits, pos, freqs, eps, kv_rank=512, rope=64):
    """c_kv RMSNorm + k_rope RoPE of one token (transformer.cpp:3935-3981)."""
    x = np.ascontiguousarray(kva_bits, np.uint16).copy()
    lib().oracle_mla_kv_prepare(_p(x), _p(np.ascontiguousarray(norm_w_bits, np.uint16)), kv_rank, rope,
                                float(eps), int(pos), _p(np.ascontiguousarray(freqs, np.float32)))
    return x


def mla_latent_write(kv_a_bits, norm_w_bits, positions, cache_bits, rows_per_seq, max_seq_len, freqs, eps,
                     kv_rank=512, rope=64):
    """Latent-cache writer (transformer.cpp:3930-3987) for every row of
    kv_a [rows, kv_rank+rope]; cache [n_seq, max_T, kv_rank+rope] uint16,
    returned updated (a copy)."""
    kv = np.ascontiguousarray(kv_a_bits, np.uint16)
    cache = np.ascontiguousarray(cache_bits, np.uint16).copy()
    pos = np.ascontiguousarray(positions, np.int32)
    lib().oracle_mla_latent_write(_p(kv), _p(np.ascontiguousarray(norm_w_bits, np.uint16)), _p(pos), _p(cache),
                                  kv.shape[0], rows_per_seq, cache[0].size, max_seq_len, kv_rank, rope, float(eps),
                                  _p(np.ascontiguousarray(freqs, np.float32)))
    return cache


def q4_quantize_group(bits, count=None):
    """quantize_group (kv_cache.cpp:21-56): up to 32 f16 bit patterns -> 20 bytes."""
    src = np.zeros(32, np.uint16)
    bits = np.asarray(bits, np.uint16)
    src[:bits.size] = bits
    out = np.zeros(20, np.uint8)
    lib().oracle_q4_quantize_group(_p(src), _p(out), bits.size if count is None else count)
    return out


def q4_dequantize_group(group):
    out = np.zeros(32, np.uint16)
    lib().oracle_q4_dequantize_group(_p(np.ascontiguousarray(group, np.uint8)), _p(out))
    return out


def q4_quantize_tokens(bits):
    """quantize_token for each row of [T, vpt] f16 bits -> [T, groups*20] bytes."""
    x = np.ascontiguousarray(bits, np.uint16)
    T, vpt = x.shape
    out = np.zeros((T, (vpt + 31) // 32 * 20), np.uint8)
    for t in range(T):
        lib().oracle_q4_quantize_token(_p(x[t]), _p(out[t]), vpt)
    return out


def q4_dequantize_tokens(q, vpt):
    q = np.ascontiguousarray(q, np.uint8)
    out = np.zeros((q.shape[0], vpt), np.uint16)
    for t in range(q.shape[0]):
        lib().oracle_q4_dequantize_token(_p(q[t]), _p(out[t]), vpt)
    return out


def kvq4_read(bits, n_q4):
    """KVCache::read_k / read_v of [T, vpt] f16 bits whose first n_q4 tokens
    were quantised (kv_cache.cpp:163-278)."""
    x = np.ascontiguousarray(bits, np.uint16)
    T, vpt = x.shape
    out = np.empty_like(x)
    lib().oracle_kvq4_read(_p(x), _p(out), T, vpt, int(n_q4))
    return out


def mla_full(q, w_kb, w_vb, w_type, latent, seq_lens, q_len, H, scale, nope=128, rope=64, kv_rank=512,
             v_head=128, seq_stride=None, nthreads=1):
    """cpu_mla_attention (transformer.cpp:2539-2623): absorb, latent core,
    up-project.  q [B,q_len,H,nope+rope]; returns [B,q_len,H,v_head] (f16
    values as float32)."""
    qa = mla_absorb(q, w_kb, w_type, H, nope, rope, kv_rank)
    o = mla_attention(qa, latent, seq_lens, q_len, H, scale, kv_rank, rope, seq_stride, nthreads=nthreads)
    return mla_project(o, w_vb, w_type, H, kv_rank, v_head)


def scatter_kv(src_bits, dst_bits, offset, count):
    """scatter_kv (kernel_sources.h:3018-3028) on uint16 element arrays."""
    src = np.ascontiguousarray(src_bits, np.uint16)
    dst = np.ascontiguousarray(dst_bits, np.uint16).copy()
    lib().oracle_scatter_kv(_p(src), _p(dst), offset, count)
    return dst


# ------------------------------------------- independent fp64 brute force

def _softmax_rows64(s):
    s = s - s.max(axis=-1, keepdims=True)
    e = np.exp(s)
    return e / e.sum(axis=-1, keepdims=True)


def gqa_attention_np64(q, k, v, seq_lens, H, Hk, D, seq_stride, scale=0.0):
    """Vectorised fp64 restatement (small shapes only)."""
    B = len(seq_lens)
    G = H // Hk
    sc = float(np.float32(scale)) if scale > 0 else float(np.float32(1.0) / np.sqrt(np.float32(D)))
    out = np.zeros((B, H, D))
    for b in range(B):
        T = int(seq_lens[b])
        if T <= 0:
            continue
        kb = np.asarray(k, np.float64).ravel()[b * seq_stride: b * seq_stride + T * Hk * D].reshape(T, Hk, D)
        vb = np.asarray(v, np.float64).ravel()[b * seq_stride: b * seq_stride + T * Hk * D].reshape(T, Hk, D)
        for h in range(H):
            s = kb[:, h // G, :] @ np.asarray(q[b, h], np.float64) * sc
            out[b, h] = _softmax_rows64(s) @ vb[:, h // G, :]
    return out


def mla_attention_np64(q, latent, seq_lens, q_len, H, scale, kv_rank=512, rope=64, seq_stride=None):
    B = len(seq_lens)
    C = kv_rank + rope
    lat = np.asarray(latent, np.float64).ravel()
    if seq_stride is None:
        seq_stride = lat.size // B
    out = np.zeros((B, q_len, H, kv_rank))
    for b in range(B):
        for i in range(q_len):
            T = int(seq_lens[b]) - q_len + i + 1
            if T <= 0:
                continue
            c = lat[b * seq_stride: b * seq_stride + T * C].reshape(T, C)
            s = np.asarray(q[b, i], np.float64) @ c.T * float(np.float32(scale))  # [H, T]
            out[b, i] = _softmax_rows64(s) @ c[:, :kv_rank]
    return out


def gqa_prefill_np64(q, k, v, N, H, Hk, D, kv_len, start, scale=0.0):
    G = H // Hk
    sc = float(np.float32(scale)) if scale > 0 else float(np.float32(1.0) / np.sqrt(np.float32(D)))
    k3 = np.asarray(k, np.float64).reshape(kv_len, Hk, D)
    v3 = np.asarray(v, np.float64).reshape(kv_len, Hk, D)
    out = np.zeros((N, H, D))
    for h in range(H):
        s = np.asarray(q[:, h, :], np.float64) @ k3[:, h // G, :].T * sc  # [N, kv_len]
        keys = np.arange(kv_len)[None, :]
        lim = (start + np.arange(N))[:, None]
        s = np.where(keys <= lim, s, -np.inf)
        out[:, h, :] = _softmax_rows64(s) @ v3[:, h // G, :]
    return out


def num_threads() -> int:
    return lib().oracle_num_threads()
