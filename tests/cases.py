"""Seeded test cases shared by the CPU and GPU tests.

Inputs come from the oracle's mt19937_64 + Box-Muller generator and are
rounded to the storage dtype before either side sees them, so the CPU
oracle and the HIP kernels consume bit-identical values.
"""
from __future__ import annotations

import math

import numpy as np

from oracle import oracle as O

ATOL = 2e-3   # max-abs tolerance stated for this path
RTOL = 1e-2   # relative tolerance stated for this path

F32, F16, BF16 = O.F32, O.F16, O.BF16
MLA_SCALE = 1.0 / math.sqrt(192.0)


def within_tol(got, ref, atol=ATOL, rtol=RTOL):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    ok = bool(np.all(np.isfinite(got)) and np.all(err <= atol + rtol * np.abs(ref)))
    return ok, float(err.max(initial=0.0))


def assert_close(got, ref, what="", atol=ATOL, rtol=RTOL):
    ok, mx = within_tol(got, ref, atol, rtol)
    print(f"  {what}: max-abs err {mx:.3e}", flush=True)
    assert ok, f"{what}: max-abs err {mx:.3e} exceeds atol {atol} + rtol {rtol}*|ref|"
    return mx


def gqa_decode_case(seed, B, H, Hk, D, seq_lens, max_T=None, dtype=F16, q_std=1.0, kv_std=1.0):
    seq_lens = np.asarray(seq_lens, np.int32)
    if max_T is None:
        max_T = int(seq_lens.max()) if seq_lens.size else 1
    max_T = max(max_T, 1)
    q, qb = O.round_to(O.randn(seed, (B, H, D), 0.0, q_std), dtype)
    k, kb = O.round_to(O.randn(seed + 1000, (B, max_T, Hk, D), 0.0, kv_std), dtype)
    v, vb = O.round_to(O.randn(seed + 2000, (B, max_T, Hk, D), 0.0, kv_std), dtype)
    return dict(B=B, H=H, Hk=Hk, D=D, max_T=max_T, seq_lens=seq_lens, dtype=dtype,
                q=q, k=k, v=v, qb=qb, kb=kb, vb=vb, seq_stride=max_T * Hk * D)


def gqa_decode_ref(c, f64=False, nthreads=0):
    return O.gqa_attention(c["q"], c["k"], c["v"], c["seq_lens"], c["H"], c["Hk"], c["D"],
                           c["seq_stride"], 0.0, f64=f64, nthreads=nthreads)


def prefill_case(seed, N, H, Hk, D, start=0, dtype=BF16):
    kv_len = start + N
    q, qb = O.round_to(O.randn(seed, (N, H, D)), dtype)
    k, kb = O.round_to(O.randn(seed + 1000, (kv_len, Hk, D)), dtype)
    v, vb = O.round_to(O.randn(seed + 2000, (kv_len, Hk, D)), dtype)
    return dict(N=N, H=H, Hk=Hk, D=D, start=start, kv_len=kv_len, dtype=dtype,
                q=q, k=k, v=v, qb=qb, kb=kb, vb=vb)


def prefill_ref(c, f64=False, nthreads=0):
    return O.gqa_prefill(c["q"], c["k"], c["v"], c["N"], c["H"], c["Hk"], c["D"], c["kv_len"],
                         c["start"], 0.0, f64=f64, nthreads=nthreads)


def mla_case(seed, B, q_len, H, seq_lens, max_T=None, q_dtype=BF16, lat_dtype=BF16,
             q_std=1.0, lat_std=0.5):
    seq_lens = np.asarray(seq_lens, np.int32)
    if max_T is None:
        max_T = int(seq_lens.max())
    max_T = max(max_T, 1)
    q = O.randn(seed, (B, q_len, H, 576), 0.0, q_std)
    qb = None
    if q_dtype != F32:
        q, qb = O.round_to(q, q_dtype)
    lat, latb = O.round_to(O.randn(seed + 1000, (B, max_T, 576), 0.0, lat_std), lat_dtype)
    return dict(B=B, q_len=q_len, H=H, max_T=max_T, seq_lens=seq_lens, q_dtype=q_dtype,
                lat_dtype=lat_dtype, q=q, qb=qb, lat=lat, latb=latb)


def mla_ref(c, f64=False, nthreads=0, heads=None):
    q = c["q"]
    H = c["H"]
    if heads is not None:
        q = np.ascontiguousarray(q[:, :, heads, :])
        H = len(heads)
    return O.mla_attention(q, c["lat"], c["seq_lens"], c["q_len"], H, MLA_SCALE,
                           seq_stride=c["max_T"] * 576, f64=f64, nthreads=nthreads)


# ------------------------------------------------------------ device helpers

def to_dev(bits_or_f32, dtype, device):
    """numpy (uint16 bits for F16/BF16, float32 for F32) -> torch device tensor."""
    import torch
    if dtype == F32:
        return torch.from_numpy(np.ascontiguousarray(bits_or_f32, np.float32)).to(device)
    t = torch.from_numpy(np.ascontiguousarray(bits_or_f32, np.uint16).view(np.int16))
    t = t.view(torch.float16 if dtype == F16 else torch.bfloat16)
    return t.to(device)


def torch_dtype(dtype):
    import torch
    return {F32: torch.float32, F16: torch.float16, BF16: torch.bfloat16}[dtype]


def say(msg):
    """Print + flush the case name before a GPU step (survives a box loss)."""
    print(msg, flush=True)


def golden_path(name):
    import os
    return os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", name)


def make_weights(seed, rows, K, w_type, std=0.05):
    """A [rows, row_bytes] uint8 weight buffer in a GGML encoding (F16, Q8_0,
    Q4_0; transformer.cpp:2488-2534), seeded, with dequantised weights of
    rms ~std as a quantiser would produce from N(0, std) weights: block
    scales std/rms(quants) times a factor in [0.5, 1.5), rounded to f16,
    quants uniform over their range (Q8_0 rms ~74, Q4_0 rms ~4.6)."""
    if w_type == O.W_F16:
        _, bits = O.round_to(O.randn(seed, (rows, K), 0.0, std), F16)
        return np.ascontiguousarray(bits.view(np.uint8).reshape(rows, 2 * K))
    nb = K // 32
    qrms = 73.9 if w_type == O.W_Q8_0 else 4.61
    jit = O.randint(seed, rows * nb, 0, 1023).astype(np.float32).reshape(rows, nb) / 1024 + 0.5
    _, sbits = O.round_to(jit * np.float32(std / qrms), F16)
    blk = 34 if w_type == O.W_Q8_0 else 18
    out = np.zeros((rows, nb, blk), np.uint8)
    out[:, :, 0:2] = sbits.reshape(rows, nb, 1).view(np.uint8).reshape(rows, nb, 2)
    if w_type == O.W_Q8_0:
        qs = O.randint(seed + 1, rows * nb * 32, -128, 127).astype(np.int8)
        out[:, :, 2:] = qs.view(np.uint8).reshape(rows, nb, 32)
    else:
        qs = O.randint(seed + 1, rows * nb * 16, 0, 255).astype(np.uint8)
        out[:, :, 2:] = qs.reshape(rows, nb, 16)
    return np.ascontiguousarray(out.reshape(rows, nb * blk))


def mla_full_case(seed, B, q_len, H, seq_lens, w_type, max_T=None, nope=128, rope=64, kv_rank=512, v_head=128):
    """cpu_mla_attention inputs: f16 q [B,q_len,H,nope+rope], f16 latent,
    k_b [H*nope, row], v_b [H*v_head, row] in w_type."""
    seq_lens = np.asarray(seq_lens, np.int32)
    if max_T is None:
        max_T = int(seq_lens.max()) if seq_lens.size else 1
    max_T = max(max_T, 1)
    q, qb = O.round_to(O.randn(seed, (B, q_len, H, nope + rope)), F16)
    lat, latb = O.round_to(O.randn(seed + 1000, (B, max_T, kv_rank + rope), 0.0, 0.5), F16)
    return dict(B=B, q_len=q_len, H=H, max_T=max_T, seq_lens=seq_lens, w_type=w_type, q=q, qb=qb, lat=lat,
                latb=latb, w_kb=make_weights(seed + 2000, H * nope, kv_rank, w_type),
                w_vb=make_weights(seed + 3000, H * v_head, kv_rank, w_type))


def mla_full_ref(c, nthreads=0):
    return O.mla_full(c["q"], c["w_kb"], c["w_vb"], c["w_type"], c["lat"], c["seq_lens"], c["q_len"], c["H"],
                      MLA_SCALE, nthreads=nthreads)
