"""Pins of the CPU oracle (CPU only).

The reference ships no golden vectors or attention tests for this path, so
each oracle function is pinned by checks chosen so that a plausible
mistake (dropped term, wrong head map, wrong causal bound, transposed
operand, missing normalisation) fails at least one of them:
  * known answers: the C++ standard's mt19937_64 outputs; IEEE rounding
    against numpy/torch conversions;
  * an independent fp64 numpy formulation (vectorised, masked softmax);
  * closed forms: T=1 -> V_0; q=0 or identical keys -> mean(V); a dominant
    score -> V of the argmax; T=0 -> 0;
  * invariants: KV permutation, GQA head map, prefill row == decode at
    seq_len start+t+1, MLA verify row == decode at seq_len T-q_len+i+1,
    MLA == MQA with one 576-dim kv head and V = latent[:, :512].
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests import cases as C


# ------------------------------------------------------------ generator / dtypes

def test_mt19937_64_known_answers():
    # std::mt19937_64 default seed 5489: first output and the 10000th
    # ([rand.predef] requires 9981545732273789042 for the latter)
    assert O.lib().oracle_mt64_first(5489, 0) == 14514284786278117030
    assert O.lib().oracle_mt64_first(5489, 9999) == 9981545732273789042


def test_randn_moments_and_determinism():
    x = O.randn(42, (200_000,))
    assert abs(float(x.mean())) < 0.01 and abs(float(x.std()) - 1.0) < 0.01
    np.testing.assert_array_equal(x, O.randn(42, (200_000,)))
    y = O.randn(7, (1001,), 3.0, 0.5)
    assert abs(float(y.mean()) - 3.0) < 0.1


def test_randint_range():
    r = O.randint(43, 10000, 256, 4096)
    assert r.min() >= 256 and r.max() <= 4096 and len(np.unique(r)) > 3000


def test_f16_rounding_matches_numpy():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * s for s in (1e-6, 1e-3, 1, 100, 3e4)])
    x = np.concatenate([x, np.array([0.0, -0.0, 65504, 65520, 1e9, 5.96e-8, 2.98e-8, 6.1e-5], np.float32)])
    v, bits = O.round_to(x, O.F16)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16)
    np.testing.assert_array_equal(bits, ref.view(np.uint16))
    np.testing.assert_array_equal(v, ref.astype(np.float32))


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(50000).astype(np.float32) * s for s in (1e-30, 1, 1e30)])
    v, bits = O.round_to(x, O.BF16)
    ref = torch.from_numpy(x).to(torch.bfloat16)
    np.testing.assert_array_equal(bits, ref.view(torch.int16).numpy().view(np.uint16))
    np.testing.assert_array_equal(v, ref.float().numpy())


# ------------------------------------------------------------ GQA decode

@pytest.mark.parametrize("B,H,Hk,D,lens", [
    (1, 4, 4, 64, [37]),
    (3, 28, 4, 128, [1, 130, 77]),
    (2, 8, 1, 64, [200, 5]),
    (2, 16, 2, 128, [0, 33]),
])
def test_gqa_oracle_vs_fp64_bruteforce(B, H, Hk, D, lens):
    c = C.gqa_decode_case(11, B, H, Hk, D, lens)
    ref = O.gqa_attention_np64(c["q"], c["k"], c["v"], c["seq_lens"], H, Hk, D, c["seq_stride"])
    got32 = C.gqa_decode_ref(c)
    got64 = C.gqa_decode_ref(c, f64=True)
    np.testing.assert_allclose(got64, ref, atol=1e-12, rtol=1e-10)
    np.testing.assert_allclose(got32, ref, atol=2e-6, rtol=1e-4)


def test_gqa_closed_forms():
    H, Hk, D, T = 8, 2, 64, 50
    c = C.gqa_decode_case(3, 1, H, Hk, D, [T])
    G = H // Hk
    # T = 1 -> out = V_0 of the head's kv group (exact in fp32)
    out1 = O.gqa_attention(c["q"], c["k"], c["v"], [1], H, Hk, D, c["seq_stride"])
    for h in range(H):
        np.testing.assert_array_equal(out1[0, h], c["v"][0, 0, h // G])
    # q = 0 -> uniform weights -> mean of V rows
    out0 = O.gqa_attention(np.zeros_like(c["q"]), c["k"], c["v"], [T], H, Hk, D, c["seq_stride"], f64=True)
    for h in range(H):
        np.testing.assert_allclose(out0[0, h], c["v"][0, :T, h // G].astype(np.float64).mean(0), atol=1e-12)
    # identical keys -> mean of V rows
    k_same = np.repeat(c["k"][:, :1], c["max_T"], axis=1).copy()
    outk = O.gqa_attention(c["q"], k_same, c["v"], [T], H, Hk, D, c["seq_stride"], f64=True)
    np.testing.assert_allclose(outk[0], out0[0], atol=1e-12)
    # one dominant score -> that row's V
    k_dom = c["k"].copy()
    k_dom[0, 17] = 0.0
    q_dom = np.zeros_like(c["q"])
    q_dom[0, :, 0] = 1.0
    k_dom[0, :, :, 0] = 0.0
    k_dom[0, 17, :, 0] = 1000.0
    outd = O.gqa_attention(q_dom, k_dom, c["v"], [T], H, Hk, D, c["seq_stride"], f64=True)
    for h in range(H):
        np.testing.assert_allclose(outd[0, h], c["v"][0, 17, h // G], atol=1e-12)
    # T = 0 -> zeros (documented departure: reference is undefined)
    assert np.all(O.gqa_attention(c["q"], c["k"], c["v"], [0], H, Hk, D, c["seq_stride"]) == 0)


def test_gqa_permutation_and_head_map():
    H, Hk, D, T = 12, 3, 64, 40
    c = C.gqa_decode_case(5, 1, H, Hk, D, [T])
    perm = np.random.default_rng(0).permutation(T)
    kp = c["k"].copy()
    vp = c["v"].copy()
    kp[0, :T] = c["k"][0, perm]
    vp[0, :T] = c["v"][0, perm]
    a = O.gqa_attention(c["q"], c["k"], c["v"], [T], H, Hk, D, c["seq_stride"], f64=True)
    b = O.gqa_attention(c["q"], kp, vp, [T], H, Hk, D, c["seq_stride"], f64=True)
    np.testing.assert_allclose(a, b, atol=1e-12)
    # head h reads kv head h // (H/Hk): moving one kv head changes exactly its G query heads
    k2 = c["k"].copy()
    k2[0, :, 1] += np.random.default_rng(1).standard_normal(k2[0, :, 1].shape).astype(np.float32)
    b2 = O.gqa_attention(c["q"], k2, c["v"], [T], H, Hk, D, c["seq_stride"], f64=True)
    changed = np.abs(b2 - a).max(axis=-1)[0] > 1e-9
    assert list(np.nonzero(changed)[0]) == [4, 5, 6, 7]


# ------------------------------------------------------------ prefill

@pytest.mark.parametrize("N,H,Hk,D,start", [(9, 4, 2, 64, 0), (20, 8, 8, 128, 13), (33, 6, 2, 64, 3)])
def test_prefill_oracle_vs_fp64_bruteforce(N, H, Hk, D, start):
    c = C.prefill_case(21, N, H, Hk, D, start)
    ref = O.gqa_prefill_np64(c["q"], c["k"], c["v"], N, H, Hk, D, c["kv_len"], start)
    np.testing.assert_allclose(C.prefill_ref(c, f64=True), ref, atol=1e-12, rtol=1e-10)
    np.testing.assert_allclose(C.prefill_ref(c), ref, atol=2e-6, rtol=1e-4)


def test_prefill_row_equals_decode_at_causal_len():
    N, H, Hk, D, start = 12, 8, 2, 64, 5
    c = C.prefill_case(22, N, H, Hk, D, start)
    pre = C.prefill_ref(c, f64=True)
    kv = c["kv_len"]
    for t in range(N):
        dec = O.gqa_attention(c["q"][t][None], c["k"].reshape(1, kv, Hk, D), c["v"].reshape(1, kv, Hk, D),
                              [start + t + 1], H, Hk, D, kv * Hk * D, f64=True)
        np.testing.assert_array_equal(pre[t], dec[0])


# ------------------------------------------------------------ MLA

@pytest.mark.parametrize("B,q_len,H,lens", [(1, 1, 4, [70]), (2, 3, 5, [40, 3]), (2, 1, 2, [0, 9])])
def test_mla_oracle_vs_fp64_bruteforce(B, q_len, H, lens):
    c = C.mla_case(31, B, q_len, H, lens, q_dtype=O.F32, lat_dtype=O.F16)
    ref = O.mla_attention_np64(c["q"], c["lat"], c["seq_lens"], q_len, H, C.MLA_SCALE)
    np.testing.assert_allclose(C.mla_ref(c, f64=True), ref, atol=1e-12, rtol=1e-10)
    np.testing.assert_allclose(C.mla_ref(c), ref, atol=2e-6, rtol=1e-4)


def test_mla_equals_mqa_with_one_576_dim_head():
    # MLA latent core == MQA with Hk=1, d_qk=576 and V = latent[:, :512]
    T, H = 60, 6
    c = C.mla_case(32, 1, 1, H, [T], q_dtype=O.F32, lat_dtype=O.BF16)
    mla = C.mla_ref(c, f64=True)[0, 0]
    k = c["lat"].reshape(1, T, 1, 576)
    v = k.copy()
    v[..., 512:] = 0.0
    mqa = O.gqa_attention(c["q"].reshape(1, H, 576), k, v, [T], H, 1, 576, T * 576, C.MLA_SCALE, f64=True)[0]
    np.testing.assert_array_equal(mla, mqa[:, :512])
    np.testing.assert_array_equal(mqa[:, 512:], 0.0)


def test_mla_closed_forms():
    H = 3
    c = C.mla_case(33, 1, 1, H, [1], max_T=8, q_dtype=O.F32, lat_dtype=O.F16)
    out = C.mla_ref(c)
    for h in range(H):  # T = 1 -> c_0[0:512]
        np.testing.assert_array_equal(out[0, 0, h], c["lat"][0, 0, :512])
    q0 = dict(c, q=np.zeros_like(c["q"]), seq_lens=np.array([8], np.int32))
    out0 = C.mla_ref(q0, f64=True)
    np.testing.assert_allclose(out0[0, 0, 0], c["lat"][0, :8, :512].astype(np.float64).mean(0), atol=1e-12)
    # the rope part of the score matters: q_rope . k_rope alone selects a token
    qr = np.zeros_like(c["q"])
    lat = c["lat"].copy()
    lat[0, :, 512:] = 0.0
    lat[0, 5, 512] = 1.0
    qr[0, 0, :, 512] = 4000.0
    outr = O.mla_attention(qr, lat, [8], 1, H, C.MLA_SCALE, seq_stride=8 * 576, f64=True)
    np.testing.assert_allclose(outr[0, 0, 1], lat[0, 5, :512], atol=1e-12)


def test_mla_verify_row_equals_decode_at_causal_len():
    B, q_len, H, T = 2, 5, 4, 50
    c = C.mla_case(34, B, q_len, H, [T, 7], max_T=T, q_dtype=O.F32, lat_dtype=O.BF16)
    ver = C.mla_ref(c, f64=True)
    for b in range(B):
        for i in range(q_len):
            Ti = int(c["seq_lens"][b]) - q_len + i + 1
            dec = O.mla_attention(c["q"][b:b + 1, i:i + 1].copy(), c["lat"][b:b + 1].copy(), [Ti], 1, H,
                                  C.MLA_SCALE, seq_stride=T * 576, f64=True)
            np.testing.assert_array_equal(ver[b, i], dec[0, 0])


# ------------------------------------------------------------ scatter_kv

def test_scatter_kv_oracle():
    src = np.arange(100, dtype=np.uint16)
    dst = np.full(1000, 7, np.uint16)
    out = O.scatter_kv(src, dst, 321, 100)
    np.testing.assert_array_equal(out[321:421], src)
    assert np.all(out[:321] == 7) and np.all(out[421:] == 7)


# ------------------------------------------------------------ committed fixtures

def test_golden_fixtures_reproduce():
    fx = np.load(C.golden_path("gqa_decode_small.npz"))
    q, k, v = (O.bits_to_f32(fx[n], int(fx["dtype"])) for n in ("qb", "kb", "vb"))
    out = O.gqa_attention(q, k, v, fx["seq_lens"], int(fx["H"]), int(fx["Hk"]), int(fx["D"]),
                          int(fx["max_T"]) * int(fx["Hk"]) * int(fx["D"]))
    np.testing.assert_array_equal(out, fx["out_f32"])
    fx = np.load(C.golden_path("prefill_small.npz"))
    q, k, v = (O.bits_to_f32(fx[n], int(fx["dtype"])) for n in ("qb", "kb", "vb"))
    N, kv = int(fx["N"]), int(fx["N"]) + int(fx["start"])
    out = O.gqa_prefill(q, k, v, N, int(fx["H"]), int(fx["Hk"]), int(fx["D"]), kv, int(fx["start"]))
    np.testing.assert_array_equal(out, fx["out_f32"])
    fx = np.load(C.golden_path("mla_verify_small.npz"))
    lat = O.bits_to_f32(fx["latb"], int(fx["lat_dtype"]))
    out = O.mla_attention(fx["q"], lat, fx["seq_lens"], int(fx["q_len"]), int(fx["H"]), C.MLA_SCALE,
                          seq_stride=int(fx["max_T"]) * 576)
    np.testing.assert_array_equal(out, fx["out_f32"])


def test_dequant_known_answers():
    # F16: the row's halfs widened exactly
    vals = np.array([1.0, -2.5, 0.000123, 65504.0] * 8, np.float16)
    out = O.dequant_rows(vals.view(np.uint8).reshape(1, -1), O.W_F16, 32)
    np.testing.assert_array_equal(out[0], vals.astype(np.float32))
    # Q8_0: scale 0.5 (f16 0x3800) times the int8 quants
    blk = np.zeros(34, np.uint8)
    blk[0:2] = np.array([0x3800], np.uint16).view(np.uint8)
    q = np.arange(-16, 16, dtype=np.int8) * 4
    blk[2:] = q.view(np.uint8)
    out = O.dequant_rows(blk.reshape(1, 34), O.W_Q8_0, 32)
    np.testing.assert_array_equal(out[0], 0.5 * q.astype(np.float32))
    # Q4_0: scale 2 (0x4000); byte j = (15 - j) << 4 | j -> element j is the
    # low nibble (j - 8) * 2, element j + 16 the high nibble (7 - j) * 2
    blk = np.zeros(18, np.uint8)
    blk[0:2] = np.array([0x4000], np.uint16).view(np.uint8)
    j = np.arange(16)
    blk[2:] = ((15 - j) << 4 | j).astype(np.uint8)
    out = O.dequant_rows(blk.reshape(1, 18), O.W_Q4_0, 32)
    np.testing.assert_array_equal(out[0, :16], ((j - 8) * 2).astype(np.float32))
    np.testing.assert_array_equal(out[0, 16:], ((7 - j) * 2).astype(np.float32))
    # an unsupported type zero-fills (transformer.cpp:2530-2533)
    np.testing.assert_array_equal(O.dequant_rows(blk.reshape(1, 18), 12, 32), np.zeros((1, 32), np.float32))


@pytest.mark.parametrize("w_type", [O.W_F16, O.W_Q8_0, O.W_Q4_0])
def test_absorb_and_project_vs_numpy(w_type):
    H, nope, rope, kr, vh, rows = 3, 128, 64, 512, 128, 2
    q, _ = O.round_to(O.randn(5, (rows, H, nope + rope)), C.F16)
    q[0, 1, 7] = 0.0  # a skipped term
    wkb = C.make_weights(6, H * nope, kr, w_type)
    wvb = C.make_weights(7, H * vh, kr, w_type)
    Wk = O.dequant_rows(wkb, w_type, kr).reshape(H, nope, kr).astype(np.float64)
    Wv = O.dequant_rows(wvb, w_type, kr).reshape(H, vh, kr).astype(np.float64)
    qa = O.mla_absorb(q, wkb, w_type, H)
    ref = np.einsum("rhi,hid->rhd", q[..., :nope].astype(np.float64), Wk)
    np.testing.assert_allclose(qa[..., :kr], ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())
    np.testing.assert_array_equal(qa[..., kr:], q[..., nope:])
    o = O.randn(8, (rows, H, kr), 0.0, 0.3)
    out = O.mla_project(o, wvb, w_type, H)
    refo = np.einsum("rhd,hjd->rhj", o.astype(np.float64), Wv)
    assert np.all(out == out.astype(np.float16).astype(np.float32))  # f16 values
    np.testing.assert_allclose(out, refo, rtol=2e-3, atol=2e-3 * np.abs(refo).max())


def test_mla_full_is_absorb_core_project():
    # the composition against an fp64 brute force of the whole operator
    c = C.mla_full_case(9, 2, 2, 4, [40, 17], O.W_Q8_0)
    got = C.mla_full_ref(c)
    Wk = O.dequant_rows(c["w_kb"], O.W_Q8_0, 512).reshape(4, 128, 512).astype(np.float64)
    Wv = O.dequant_rows(c["w_vb"], O.W_Q8_0, 512).reshape(4, 128, 512).astype(np.float64)
    q = c["q"].astype(np.float64)
    qa = np.concatenate([np.einsum("bthi,hid->bthd", q[..., :128], Wk), q[..., 128:]], -1)
    o = O.mla_attention_np64(qa, c["lat"], c["seq_lens"], 2, 4, C.MLA_SCALE)
    ref = np.einsum("bthd,hjd->bthj", o, Wv)
    np.testing.assert_allclose(got, ref, rtol=2e-3, atol=2e-3 * np.abs(ref).max())


# ------------------------------------------------------------ latent-cache writer

def _f16(x):
    return np.asarray(x, np.float32).astype(np.float16)


def _bits(x):
    return _f16(x).view(np.uint16)


def _vals(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float64)


def test_yarn_freqs_closed_form_and_deepseek_v3_correction_range():
    base = O.yarn_freqs(64, 0.0, 0, 10000.0)  # factor <= 1: theta^(-2i/d)
    np.testing.assert_allclose(base, 10000.0 ** (-2.0 * np.arange(32) / 64), rtol=2e-6)
    assert np.array_equal(O.yarn_freqs(64, 1.0, 4096, 10000.0), base)
    # DeepSeek-V3 (theta 1e4, factor 40, original ctx 4096, beta 32 / 1): the
    # YaRN correction range is dims [10, 23] -- below it the base frequency,
    # above it base / 40, a linear ramp over 13 steps in between
    v3 = O.yarn_freqs(64, 40.0, 4096, 10000.0)
    ratio = v3.astype(np.float64) / base
    i = np.arange(32)
    expect = np.where(i <= 10, 1.0, np.where(i >= 23, 1 / 40, 1 - (i - 10) / 13 * (1 - 1 / 40)))
    np.testing.assert_allclose(ratio, expect, rtol=1e-5)


def test_rope_neox_known_rotation_pairing_and_identity():
    freqs = O.yarn_freqs(64, 0.0, 0, 10000.0)   # freqs[0] = 1
    x = np.zeros(64, np.float32)
    x[0] = 1.0
    for pos in (1, 2, 7):
        y = _vals(O.rope_neox_f16(_bits(x), pos, freqs))
        # NeoX pairs (i, i + 32): e_0 -> (cos p, sin p) in dims 0 and 32
        assert abs(y[0] - np.cos(pos)) <= 2 ** -11 and abs(y[32] - np.sin(pos)) <= 2 ** -11
        assert np.count_nonzero(y) == 2
    r = np.asarray(O.randn(3, (64,)), np.float32)
    assert np.array_equal(O.rope_neox_f16(_bits(r), 0, freqs), _bits(r))   # pos 0: identity


def test_rope_neox_preserves_pair_norms_and_composes():
    freqs = O.yarn_freqs(64, 40.0, 4096, 10000.0)
    x = _bits(O.randn(4, (64,)))
    xv = _vals(x)
    y = _vals(O.rope_neox_f16(x, 1000, freqs))
    n0 = np.hypot(xv[:32], xv[32:])
    n1 = np.hypot(y[:32], y[32:])
    np.testing.assert_allclose(n1, n0, rtol=2e-3, atol=1e-3)
    # rotating by a then by b == rotating by a + b (up to f16 roundings)
    ab = _vals(O.rope_neox_f16(O.rope_neox_f16(x, 300, freqs), 200, freqs))
    np.testing.assert_allclose(ab, _vals(O.rope_neox_f16(x, 500, freqs)), atol=4e-3)
    # against an fp64 rotation
    ang = 1000.0 * freqs.astype(np.float64)
    ref0 = xv[:32] * np.cos(ang) - xv[32:] * np.sin(ang)
    ref1 = xv[32:] * np.cos(ang) + xv[:32] * np.sin(ang)
    np.testing.assert_allclose(y, np.concatenate([ref0, ref1]), atol=3e-3)


def test_kv_prepare_rmsnorm_closed_forms():
    freqs = O.yarn_freqs(64, 0.0, 0, 10000.0)
    kva = np.full(576, 2.0, np.float32)
    w = np.full(512, 0.5, np.float32)
    out = _vals(O.mla_kv_prepare(_bits(kva), _bits(w), 0, freqs, 1e-6))
    np.testing.assert_allclose(out[:512], 0.5, rtol=1e-3)          # 2 / rms(2) * 0.5
    assert np.all(out[512:] == 2.0)                                 # pos 0: k_rope unrotated
    # random vector against an fp64 RMSNorm, weights applied per dim
    v = _f16(O.randn(5, (576,))).astype(np.float32)
    wv = _f16(np.linspace(0.5, 1.5, 512)).astype(np.float32)
    out = _vals(O.mla_kv_prepare(_bits(v), _bits(wv), 37, freqs, 1e-6))
    v64 = v[:512].astype(np.float64)
    ref = v64 / np.sqrt(np.mean(v64 * v64) + 1e-6) * wv
    np.testing.assert_allclose(out[:512], ref, rtol=2e-3, atol=1e-4)
    np.testing.assert_array_equal(out[512:], _vals(O.rope_neox_f16(_bits(v[512:]), 37, freqs)))


def test_latent_write_rows_sequences_and_bounds():
    freqs = O.yarn_freqs(64, 40.0, 4096, 10000.0)
    kv = _bits(O.randn(6, (6, 576)))
    w = _bits(O.randn(7, (512,), 1.0, 0.1))
    cache = np.zeros((3, 16, 576), np.uint16)
    pos = np.array([3, 4, 0, 15, 16, -1], np.int32)     # 2 rows per sequence; the last two out of range
    out = O.mla_latent_write(kv, w, pos, cache, 2, 16, freqs, 1e-6)
    for r, p in enumerate(pos[:4]):
        np.testing.assert_array_equal(out[r // 2, p], O.mla_kv_prepare(kv[r], w, p, freqs, 1e-6))
    written = {(0, 3), (0, 4), (1, 0), (1, 15)}
    for b in range(3):
        for t in range(16):
            if (b, t) not in written:
                assert not out[b, t].any()


# ------------------------------------------------------------ 4-bit group KV store

def test_q4_group_known_answers():
    # values 0..15 twice: min 0, range 15 -> scale exactly 1, nibbles = values;
    # value 2i in the low nibble of byte i, 2i+1 in the high one
    v = np.concatenate([np.arange(16), np.arange(16)]).astype(np.float16)
    g = O.q4_quantize_group(v.view(np.uint16))
    assert g[0:2].view(np.float16)[0] == 1.0 and g[2:4].view(np.float16)[0] == 0.0
    expect = [(int(v[2 * i + 1]) << 4) | int(v[2 * i]) for i in range(16)]
    assert list(g[4:]) == expect
    assert np.array_equal(O.q4_dequantize_group(g), v.view(np.uint16))     # exact round trip
    # a constant group: scale 0, nibbles 0, every value comes back as the min
    c = np.full(32, -3.25, np.float16)
    gc = O.q4_quantize_group(c.view(np.uint16))
    assert gc[0:2].view(np.float16)[0] == 0.0 and not gc[4:].any()
    assert np.all(O.q4_dequantize_group(gc).view(np.float16) == -3.25)
    # a short group: the zero padding takes part in min / max (all-positive
    # values get min 0), round-half-away: (v - 0) / (30/15) = 2.5 -> 3
    s = np.array([5.0, 30.0], np.float16)
    gs = O.q4_quantize_group(s.view(np.uint16))
    assert gs[0:2].view(np.float16)[0] == 2.0 and gs[2:4].view(np.float16)[0] == 0.0
    assert gs[4] == (15 << 4) | 3 and not gs[5:].any()


def _fill_token(vpt, base):
    # the reference test's fill_token: f16(base + 0.01 i)
    return (base + np.float32(0.01) * np.arange(vpt, dtype=np.float32)).astype(np.float16).view(np.uint16)


def test_q4_store_reference_test_properties():
    # test_kv_cache.cpp:128-177 (4 heads x 64, preserve 32, 128 tokens):
    # quantised tokens within 10% relative, the fp16 tail exact
    vpt, T, keep = 256, 128, 32
    k = np.stack([_fill_token(vpt, 1.0 + 0.05 * t) for t in range(T)])
    got = O.kvq4_read(k, T - keep)
    kv, gv = k.view(np.float16).astype(np.float32), got.view(np.float16).astype(np.float32)
    rel = np.abs(kv - gv) / np.maximum(np.abs(kv), 1e-6)
    assert rel[:T - keep].max() < 0.10 and rel[:T - keep].max() > 0
    assert np.array_equal(got[T - keep:], k[T - keep:])
    # test_compression_ratio: 64 / 20 bytes per group of 32
    assert O.q4_quantize_tokens(k[:1]).nbytes * 3.2 == vpt * 2


def test_q4_error_bound_and_extremes():
    # |x - deq(q(x))| <= scale / 2 (+ f16 rounding) per value; in every
    # group the minimum gets nibble 0 and the maximum nibble 15
    x = O.round_to(O.randn(61, (64, 512), 0.0, 2.0), C.F16)[1]
    q = O.q4_quantize_tokens(x)
    d = O.q4_dequantize_tokens(q, 512)
    sc = q.reshape(64, 16, 20)[:, :, 0:2].copy().view(np.float16).astype(np.float32)[..., 0]
    err = np.abs(x.view(np.float16).astype(np.float32) - d.view(np.float16).astype(np.float32)).reshape(64, 16, 32)
    assert np.all(err <= sc[..., None] * 0.5 + 4e-3)
    nib = q.reshape(64, 16, 20)[:, :, 4:]
    nib = np.stack([nib & 15, nib >> 4], -1).reshape(64, 16, 32)
    xv = x.view(np.float16).astype(np.float32).reshape(64, 16, 32)
    rows = np.arange(64)[:, None]
    grps = np.arange(16)[None, :]
    assert np.all(nib[rows, grps, xv.argmin(-1)] == 0)
    assert np.all(nib[rows, grps, xv.argmax(-1)] == 15)
