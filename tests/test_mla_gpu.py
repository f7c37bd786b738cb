"""MLA absorbed decode / verify on the GPU vs the CPU oracle
(latent core of cpu_mla_attention)."""
import numpy as np
import pytest
import torch

import mugen_amd
from mugen_amd import _capi
from oracle import oracle as O
from tests import cases as C

pytestmark = pytest.mark.gpu


def run_gpu(c, device, out_dtype=C.F32, num_splits=0, seq_lens=None, q=None, kernel=0):
    sl_np = c["seq_lens"] if seq_lens is None else np.asarray(seq_lens, np.int32)
    C.say(f"mla B={c['B']} q_len={c['q_len']} H={c['H']} maxT={c['max_T']} q={c['q_dtype']} "
          f"lat={c['lat_dtype']} out={out_dtype} splits={num_splits} kernel={kernel} lens={list(sl_np)[:8]}")
    if q is None:
        q = C.to_dev(c["q"] if c["q_dtype"] == C.F32 else c["qb"], c["q_dtype"], device)
    lat = C.to_dev(c["latb"], c["lat_dtype"], device)
    sl = torch.from_numpy(sl_np).to(device)
    out = mugen_amd.mla_attention(q, lat, sl, c["max_T"], scale=C.MLA_SCALE,
                                  out_dtype=C.torch_dtype(out_dtype), num_splits=num_splits, kernel=kernel)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def test_v2lite_decode_config(device):
    # B=1, H=16, q f32 ~N(0,1), latent fp16 [1024x576] ~N(0,0.5)
    c = C.mla_case(42, 1, 1, 16, [1024], q_dtype=C.F32, lat_dtype=C.F16)
    ref = C.mla_ref(c)
    for splits in (0, 1):
        C.assert_close(run_gpu(c, device, C.F32, splits), ref, f"v2-lite splits={splits}")


def test_v3_decode_config(device):
    # B=8, H=128, bf16, T ~ U[1024, 8192]
    lens = O.randint(45, 8, 1024, 8192)
    c = C.mla_case(45, 8, 1, 128, lens, max_T=8192, q_dtype=C.BF16, lat_dtype=C.BF16)
    ref = C.mla_ref(c, nthreads=8)
    C.assert_close(run_gpu(c, device), ref, "v3 decode")


def test_v3_verify_config_and_causal_consistency(device):
    # B=4, q_len=5, H=128, T=32768; the oracle checks every head,
    # and every verify row must equal a decode call at seq_len T-5+i+1
    T = 32768
    c = C.mla_case(46, 4, 5, 128, [T] * 4, q_dtype=C.BF16, lat_dtype=C.BF16)
    got = run_gpu(c, device)
    ref = C.mla_ref(c, nthreads=16)  # all 128 heads (~180 GFLOP in the oracle)
    C.assert_close(got, ref, "v3 verify (all heads)")
    qdev = C.to_dev(c["qb"], C.BF16, device)
    for i in range(5):
        qi = qdev[:, i:i + 1].contiguous()
        dec = run_gpu(dict(c, q_len=1), device, seq_lens=[T - 5 + i + 1] * 4, q=qi)
        np.testing.assert_allclose(got[:, i:i + 1], dec, atol=5e-4, rtol=1e-3)


@pytest.mark.parametrize("q_len,start", [(64, 0), (64, 300), (512, 0), (512, 300)])
def test_v2lite_prompt_prefill(device, q_len, start):
    # a prompt of q_len tokens in one verify-shaped call: the reference runs
    # cpu_mla_attention once per prompt token at seq_len = start + t + 1
    # (transformer.cpp:1325-1337).  V2-Lite heads, fp32 absorbed q, f16 latent
    c = C.mla_case(300 + q_len + start, 1, q_len, 16, [start + q_len], q_dtype=C.F32, lat_dtype=C.F16)
    C.assert_close(run_gpu(c, device), C.mla_ref(c, nthreads=16), f"v2-lite prompt {q_len} at {start}")


@pytest.mark.parametrize("B,q_len,H,lens,qdt,ldt", [
    (3, 1, 16, [1, 31, 33], C.F32, C.F16),
    (2, 1, 20, [64, 0], C.BF16, C.BF16),
    (2, 3, 7, [3, 100], C.F32, C.BF16),
    (1, 5, 128, [4], C.BF16, C.BF16),      # q_len > visible tokens for the first rows
    (2, 2, 64, [700, 129], C.F16, C.F16),
])
def test_edges(device, B, q_len, H, lens, qdt, ldt):
    c = C.mla_case(47 + H, B, q_len, H, lens, q_dtype=qdt, lat_dtype=ldt)
    ref = C.mla_ref(c)
    for splits in (0, 1, 4):
        C.assert_close(run_gpu(c, device, C.F32, splits), ref, f"mla edge splits={splits}")


@pytest.mark.parametrize("od", [C.F16, C.BF16])
def test_16bit_outputs(device, od):
    c = C.mla_case(48, 2, 1, 32, [500, 900], q_dtype=C.BF16, lat_dtype=C.BF16)
    C.assert_close(run_gpu(c, device, od), C.mla_ref(c), f"out dtype {od}")


def test_split_count_invariance(device):
    c = C.mla_case(49, 2, 1, 128, [5000, 2100], q_dtype=C.BF16, lat_dtype=C.BF16)
    outs = [run_gpu(c, device, C.F32, s) for s in (1, 0, 9, 100)]
    # bf16 softmax weights: each split rounds its own P (relative 2^-9)
    for o in outs[1:]:
        np.testing.assert_allclose(o, outs[0], atol=5e-4, rtol=1e-3)


def test_golden_fixture(device):
    fx = np.load(C.golden_path("mla_verify_small.npz"))
    c = dict(B=int(fx["B"]), q_len=int(fx["q_len"]), H=int(fx["H"]), max_T=int(fx["max_T"]),
             q_dtype=int(fx["q_dtype"]), lat_dtype=int(fx["lat_dtype"]), q=fx["q"], qb=fx["qb"],
             latb=fx["latb"], seq_lens=fx["seq_lens"])
    C.assert_close(run_gpu(c, device), fx["out_f64"], "golden mla_verify_small")


@pytest.mark.parametrize("ldt,big", [(C.F16, 300.0), (C.BF16, 1000.0)])
@pytest.mark.parametrize("splits", [0, 1])
def test_late_score_overshoot_rebases(device, ldt, big, splits):
    # a token far into the context scores far above every token of the first
    # tile (beyond the weights' headroom): the rows re-base in the kernel
    c = C.mla_case(60, 2, 2, 16, [900, 300], q_dtype=ldt, lat_dtype=ldt)
    lat = c["lat"].copy()
    lat[0, 700, :] = 0.0
    lat[0, 700, 0] = big
    lat[1, 250, 3] = -big
    lat, latb = O.round_to(lat, ldt)
    q = c["q"].copy()
    q[:, :, :, 0] = np.abs(q[:, :, :, 0]) + 1.0
    q[:, :, :, 3] = -np.abs(q[:, :, :, 3]) - 1.0
    q, qb = O.round_to(q, ldt)
    c2 = dict(c, lat=lat, latb=latb, q=q, qb=qb)
    C.assert_close(run_gpu(c2, device, C.F32, splits), C.mla_ref(c2), f"overshoot fallback splits={splits}")


def test_host_length_hint_matches_no_hint(device):
    # the hint only plans the grid: equal results with and without it
    lens = O.randint(70, 5, 100, 3000)
    c = C.mla_case(70, 5, 1, 128, lens, max_T=3000, q_dtype=C.BF16, lat_dtype=C.BF16)
    q = C.to_dev(c["qb"], C.BF16, device)
    lat = C.to_dev(c["latb"], C.BF16, device)
    sl = torch.from_numpy(c["seq_lens"]).to(device)
    C.say("mla hint vs no hint")
    a = mugen_amd.mla_attention(q, lat, sl, 3000, scale=C.MLA_SCALE).cpu().numpy()
    bb = mugen_amd.mla_attention(q, lat, sl, 3000, scale=C.MLA_SCALE, seq_lens_host=c["seq_lens"]).cpu().numpy()
    torch.cuda.synchronize()
    C.assert_close(a, C.mla_ref(c, nthreads=8), "no hint")
    C.assert_close(bb, C.mla_ref(c, nthreads=8), "hint")


@pytest.mark.parametrize("kernel", [_capi.MLA_KERNEL_ROWS, _capi.MLA_KERNEL_WS])
@pytest.mark.parametrize("B,q_len,H,lens", [
    (2, 1, 128, [700, 33]),
    (1, 5, 128, [4]),
    (2, 2, 64, [700, 129]),
    (3, 1, 96, [1, 300, 2050]),
])
def test_kernel_variants(device, kernel, B, q_len, H, lens):
    # both 16-bit-q kernels, whichever one the planner would pick
    c = C.mla_case(80 + H, B, q_len, H, lens, q_dtype=C.BF16, lat_dtype=C.BF16)
    ref = C.mla_ref(c)
    for splits in (0, 1, 4):
        C.assert_close(run_gpu(c, device, C.F32, splits, kernel=kernel), ref, f"kernel {kernel} splits={splits}")


@pytest.mark.parametrize("kernel", [_capi.MLA_KERNEL_ROWS, _capi.MLA_KERNEL_WS])
@pytest.mark.parametrize("B,q_len,H,lens,ldt", [
    (2, 1, 128, [700, 33], C.BF16),
    (2, 3, 128, [3, 100], C.F16),
    (3, 1, 96, [1, 300, 2050], C.F16),
    (1, 1, 16, [1024], C.F16),
])
def test_fp32_q_variants(device, kernel, B, q_len, H, lens, ldt):
    # fp32 q (the absorbed q of the full operator): the hi + lo split in the
    # 4-wave and the warp-specialised kernels
    c = C.mla_case(90 + H, B, q_len, H, lens, q_dtype=C.F32, lat_dtype=ldt)
    ref = C.mla_ref(c)
    for splits in (0, 1, 4):
        C.assert_close(run_gpu(c, device, C.F32, splits, kernel=kernel), ref, f"fp32 q kernel {kernel} splits={splits}")


def test_fp32_q_overshoot_rebases(device):
    # the re-base path with fp32 q in the warp-specialised kernel
    c = C.mla_case(62, 2, 1, 128, [900, 300], q_dtype=C.F32, lat_dtype=C.F16)
    lat = c["lat"].copy()
    lat[0, 700, :] = 0.0
    lat[0, 700, 0] = 300.0
    lat, latb = O.round_to(lat, C.F16)
    q = c["q"].copy()
    q[:, :, :, 0] = np.abs(q[:, :, :, 0]) + 1.0
    c2 = dict(c, lat=lat, latb=latb, q=q)
    C.assert_close(run_gpu(c2, device, C.F32, 0, kernel=_capi.MLA_KERNEL_WS), C.mla_ref(c2), "fp32 q overshoot")


@pytest.mark.parametrize("kernel", [_capi.MLA_KERNEL_ROWS, _capi.MLA_KERNEL_WS])
def test_kernel_overshoot_rebases(device, kernel):
    # the re-base path of both 16-bit-q kernels (R = 128 rows)
    c = C.mla_case(61, 2, 1, 128, [900, 300], q_dtype=C.BF16, lat_dtype=C.BF16)
    lat = c["lat"].copy()
    lat[0, 700, :] = 0.0
    lat[0, 700, 0] = 1000.0
    lat, latb = O.round_to(lat, C.BF16)
    q = c["q"].copy()
    q[:, :, :, 0] = np.abs(q[:, :, :, 0]) + 1.0
    q, qb = O.round_to(q, C.BF16)
    c2 = dict(c, lat=lat, latb=latb, q=q, qb=qb)
    C.assert_close(run_gpu(c2, device, C.F32, 0, kernel=kernel), C.mla_ref(c2), f"kernel {kernel} overshoot")


@pytest.mark.parametrize("kernel", [_capi.MLA_KERNEL_ROWS, _capi.MLA_KERNEL_WS])
@pytest.mark.parametrize("q_len", [1, 3])
def test_climbing_scores_rebase_every_tile(device, kernel, q_len):
    # latent dim 0 grows 5 per token, so a row's scores climb ~11.5 nats per
    # 32-token tile: past the f16 weights' headroom every tile, the rows
    # re-base again and again (the last tokens dominate)
    c = C.mla_case(63, 2, q_len, 16, [1000, 333], q_dtype=C.F16, lat_dtype=C.F16)
    lat = c["lat"].copy()
    lat[:, :, 0] = 5.0 * np.arange(lat.shape[1])[None, :]
    lat, latb = O.round_to(lat, C.F16)
    q = c["q"].copy()
    q[:, :, :, 0] = 1.0
    q, qb = O.round_to(q, C.F16)
    c2 = dict(c, lat=lat, latb=latb, q=q, qb=qb)
    ref = C.mla_ref(c2)
    for splits in (0, 1, 5):
        C.assert_close(run_gpu(c2, device, C.F32, splits, kernel=kernel), ref, f"climbing kernel {kernel} splits={splits}")
