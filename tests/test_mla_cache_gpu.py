"""MLA latent-cache writer (c_kv RMSNorm + k_rope RoPE + append,
transformer.cpp:3930-3987) and the q RoPE stage fused into absorption
(transformer.cpp:3882-3921) on the GPU vs the CPU oracle.

Bar: the f16 results equal the oracle's bit for bit except where the two
sides' float rounding differs in the last place before the f16 rounding (the
GPU sums the 512 squares as a tree, and its cosf / sinf are not glibc's):
every element within 1 f16 ulp, and at most 1 in 1000 elements off at all."""
import numpy as np
import pytest
import torch

import mugen_amd
from oracle import oracle as O
from tests import cases as C

pytestmark = pytest.mark.gpu

V3_ROPE = (10000.0, 40.0, 4096)
PLAIN_ROPE = (10000.0, 0.0, 0)


def f16_bits_dev(x, device):
    return C.to_dev(np.asarray(x, np.float32).astype(np.float16).view(np.uint16), C.F16, device)


def assert_f16_match(got_bits, ref_bits, what):
    g = np.asarray(got_bits, np.uint16).view(np.int16).astype(np.int32)
    r = np.asarray(ref_bits, np.uint16).view(np.int16).astype(np.int32)
    # ulp distance on the sign-magnitude f16 encoding
    gi = np.where(g < 0, -(g & 0x7fff), g)
    ri = np.where(r < 0, -(r & 0x7fff), r)
    d = np.abs(gi - ri)
    n_off = int(np.count_nonzero(d))
    print(f"  {what}: {n_off} of {d.size} elements differ (max {int(d.max(initial=0))} ulp)", flush=True)
    assert d.max(initial=0) <= 1, f"{what}: {int(d.max())} ulp"
    assert n_off <= max(1, d.size // 1000), f"{what}: {n_off} elements off by 1 ulp"


def run_write(kv, w, pos, cache, rows_per_seq, rope, device, eps=1e-6, dtype=torch.float16):
    C.say(f"latent_write rows={len(pos)} per_seq={rows_per_seq} rope={rope} pos={list(pos)[:8]} {dtype}")
    lat = C.to_dev(cache, C.F16, device)
    if dtype == torch.bfloat16:
        lat = lat.float().to(torch.bfloat16)
    mugen_amd.mla_latent_write(f16_bits_dev(kv, device), f16_bits_dev(w, device),
                               torch.from_numpy(np.asarray(pos, np.int32)).to(device), lat,
                               rows_per_seq=rows_per_seq, eps=eps, rope=rope)
    torch.cuda.synchronize()
    return lat


@pytest.mark.parametrize("rope", [V3_ROPE, PLAIN_ROPE])
def test_decode_rows(device, rope):
    # one new token per sequence (B = 8), positions across a long context
    B, T = 8, 40000
    kv = O.randn(11, (B, 576), 0.0, 2.0)
    w = O.randn(12, (512,), 1.0, 0.2)
    pos = O.randint(13, B, 0, T - 1)
    _, cache = O.round_to(O.randn(14, (B, T, 576), 0.0, 0.5), C.F16)
    ref = O.mla_latent_write(kv.astype(np.float16).view(np.uint16), w.astype(np.float16).view(np.uint16), pos,
                             cache, 1, T, O.yarn_freqs(64, rope[1], rope[2], rope[0]), 1e-6)
    got = run_write(kv, w, pos, cache, 1, rope, device).cpu().view(torch.int16).numpy().view(np.uint16)
    assert_f16_match(got, ref, "decode rows")  # also: every other cache row untouched


def test_verify_rows_and_out_of_range_positions(device):
    # q_len = 5 tokens per sequence at consecutive positions; the last
    # sequence's tokens run past the cache end and are not written
    B, q_len, T = 3, 5, 64
    kv = O.randn(21, (B * q_len, 576), 0.0, 1.0)
    w = O.randn(22, (512,), 1.0, 0.1)
    pos = np.concatenate([np.arange(10, 15), np.arange(0, 5), np.arange(61, 66)]).astype(np.int32)
    pos[1] = -1
    _, cache = O.round_to(O.randn(23, (B, T, 576), 0.0, 0.5), C.F16)
    ref = O.mla_latent_write(kv.astype(np.float16).view(np.uint16), w.astype(np.float16).view(np.uint16), pos,
                             cache, q_len, T, O.yarn_freqs(64, 40.0, 4096, 10000.0), 1e-6)
    got = run_write(kv, w, pos, cache, q_len, V3_ROPE, device).cpu().view(torch.int16).numpy().view(np.uint16)
    assert_f16_match(got, ref, "verify rows")


def test_bf16_cache(device):
    B, T = 4, 256
    kv = O.randn(31, (B, 576), 0.0, 1.0)
    w = O.randn(32, (512,), 1.0, 0.1)
    pos = np.array([0, 17, 255, 100], np.int32)
    cache = np.zeros((B, T, 576), np.uint16)
    ref = O.mla_latent_write(kv.astype(np.float16).view(np.uint16), w.astype(np.float16).view(np.uint16), pos,
                             cache, 1, T, O.yarn_freqs(64, 40.0, 4096, 10000.0), 1e-6)
    got = run_write(kv, w, pos, cache, 1, V3_ROPE, device, dtype=torch.bfloat16).float().cpu().numpy()
    refv = ref.view(np.float16).astype(np.float32)
    # bf16 keeps 8 significant bits: within 2^-8 relative of the f16 result
    np.testing.assert_allclose(got, refv, rtol=2 ** -8, atol=1e-6)


@pytest.mark.parametrize("w_type", [O.W_F16, O.W_Q4_0])
def test_absorb_with_q_rope(device, w_type):
    rows, H = 6, 16
    q, qb = O.round_to(O.randn(41, (rows, H, 192)), C.F16)
    pos = O.randint(42, rows, 0, 160000)
    freqs = O.yarn_freqs(64, 40.0, 4096, 10000.0)
    w = C.make_weights(43, H * 128, 512, w_type)
    name = {O.W_F16: "f16", O.W_Q4_0: "q4_0"}[w_type]
    wt = torch.from_numpy(w).to(device)
    if w_type == O.W_F16:
        wt = wt.view(torch.float16)
    C.say(f"absorb + q rope rows={rows} H={H} w={name}")
    got = mugen_amd.mla_absorb(C.to_dev(qb, C.F16, device), wt, name,
                               positions=torch.from_numpy(pos).to(device), rope=V3_ROPE)
    torch.cuda.synchronize()
    qr = O.rope_q_f16(qb, pos, freqs)
    ref = O.mla_absorb(qr.view(np.float16).astype(np.float32), w, w_type, H)
    got = got.cpu().numpy()
    C.assert_close(got[..., :512], ref[..., :512], "absorb (nope part)")
    assert_f16_match(got[..., 512:].astype(np.float16).view(np.uint16), qr[..., 128:], "q rope")


def test_writer_then_full_operator(device):
    # an engine step: append the new tokens' latent rows, then attend with
    # the rotated, absorbed queries (one decode token per sequence)
    B, H, T = 2, 16, 300
    rope = V3_ROPE
    freqs = O.yarn_freqs(64, rope[1], rope[2], rope[0])
    lens = np.array([300, 129], np.int32)
    c = C.mla_full_case(51, B, 1, H, lens, O.W_Q8_0, max_T=T)
    kv = O.randn(52, (B, 576), 0.0, 1.0)
    w = O.randn(53, (512,), 1.0, 0.1)
    pos = lens - 1
    kvb, wb = kv.astype(np.float16).view(np.uint16), w.astype(np.float16).view(np.uint16)
    cache_ref = O.mla_latent_write(kvb, wb, pos, c["latb"], 1, T, freqs, 1e-6)
    qr = O.rope_q_f16(c["qb"].reshape(B, H, 192), pos, freqs).reshape(B, 1, H, 192)
    ref = O.mla_full(qr.view(np.float16).astype(np.float32), c["w_kb"], c["w_vb"], O.W_Q8_0,
                     cache_ref.view(np.float16).astype(np.float32), lens, 1, H, C.MLA_SCALE)
    lat = run_write(kv, w, pos, c["latb"], 1, rope, device)
    posd = torch.from_numpy(pos).to(device)
    wk = torch.from_numpy(c["w_kb"]).to(device)
    wv = torch.from_numpy(c["w_vb"]).to(device)
    qa = mugen_amd.mla_absorb(C.to_dev(c["qb"], C.F16, device), wk, "q8_0", positions=posd, rope=rope)
    o = mugen_amd.mla_attention(qa, lat, torch.from_numpy(lens).to(device), T, scale=C.MLA_SCALE)
    out = mugen_amd.mla_project(o, wv, "q8_0")
    torch.cuda.synchronize()
    C.assert_close(out.float().cpu().numpy(), ref, "writer + full operator")


def test_seq_base_positions_match_explicit_positions(device):
    # rows_per_seq tokens per sequence at seq_base[b] + j: the same bytes as
    # passing those positions explicitly (writer and absorb's q RoPE)
    B, q_len, H, T = 3, 4, 16, 128
    base = np.array([10, 0, 120], np.int32)          # the last sequence runs past the cache
    pos = (base[:, None] + np.arange(q_len)[None, :]).reshape(-1).astype(np.int32)
    kv = O.randn(91, (B * q_len, 576))
    w = O.randn(92, (512,), 1.0, 0.1)
    _, cache = O.round_to(O.randn(93, (B, T, 576), 0.0, 0.5), C.F16)
    C.say("seq_base positions")
    a = C.to_dev(cache, C.F16, device)
    b = C.to_dev(cache, C.F16, device)
    kvd, wd = f16_bits_dev(kv, device), f16_bits_dev(w, device)
    mugen_amd.mla_latent_write(kvd, wd, torch.from_numpy(pos).to(device), a, rows_per_seq=q_len, rope=V3_ROPE)
    mugen_amd.mla_latent_write(kvd, wd, None, b, rows_per_seq=q_len, rope=V3_ROPE,
                               seq_base=torch.from_numpy(base).to(device))
    q = f16_bits_dev(O.randn(94, (B * q_len, H, 192)), device)
    wk = torch.from_numpy(C.make_weights(95, H * 128, 512, O.W_F16)).to(device).view(torch.float16)
    qa = mugen_amd.mla_absorb(q, wk, "f16", positions=torch.from_numpy(pos).to(device), rope=V3_ROPE)
    qb = mugen_amd.mla_absorb(q, wk, "f16", seq_base=torch.from_numpy(base).to(device), rows_per_seq=q_len,
                              rope=V3_ROPE)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert torch.equal(qa, qb)


@pytest.mark.parametrize("ldt", [C.F16, C.BF16])
@pytest.mark.parametrize("B,q_len,H", [(8, 1, 128), (2, 3, 16), (1, 100, 16), (3, 67, 16)])
def test_prepare_equals_separate_calls(device, ldt, B, q_len, H):
    """mla_prepare (one launch: the VALU absorb at decode sizes, the MFMA
    absorb at prompt sizes, with the latent rows beside it) writes the same
    latent rows and q_abs as mla_latent_write + mla_absorb (201 rows: four
    row groups and a last latent workgroup with one row)."""
    rows = B * q_len
    g = torch.Generator(device=device).manual_seed(70 + rows)
    kv_a = torch.randn((rows, 576), generator=g, device=device).half()
    norm_w = (torch.randn((512,), generator=g, device=device) * 0.1 + 1.0).half()
    q = torch.randn((B, q_len, H, 192), generator=g, device=device).half()
    w = torch.from_numpy(C.make_weights(71, H * 128, 512, O.W_Q8_0)).to(device)
    pos = torch.tensor([[100 * b + 7 + i for i in range(q_len)] for b in range(B)], dtype=torch.int32,
                       device=device).reshape(-1)
    rope = (10000.0, 40.0, 4096)
    C.say(f"mla_prepare B={B} q_len={q_len} H={H} latent={ldt}")
    lat1 = torch.zeros((B, 512, 576), dtype=C.torch_dtype(ldt), device=device)
    lat2 = lat1.clone()
    mugen_amd.mla_latent_write(kv_a, norm_w, pos, lat1, rows_per_seq=q_len, rope=rope)
    qa1 = mugen_amd.mla_absorb(q, w, "q8_0", positions=pos, rope=rope)
    qa2 = mugen_amd.mla_prepare(kv_a, norm_w, pos, lat2, q, w, "q8_0", rows_per_seq=q_len, rope=rope)
    torch.cuda.synchronize()
    assert torch.equal(lat1.view(torch.int16), lat2.view(torch.int16))
    assert torch.equal(qa1.view(torch.int32), qa2.view(torch.int32))

