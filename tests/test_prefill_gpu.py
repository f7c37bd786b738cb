"""GQA causal prefill on the GPU vs the CPU oracle (flash_prefill_attention
semantics)."""
import numpy as np
import pytest
import torch

import mugen_amd
from mugen_amd import _capi
from tests import cases as C

pytestmark = pytest.mark.gpu


def run_gpu(c, device, out_dtype=None, causal=True, kernel=0):
    out_dtype = c["dtype"] if out_dtype is None else out_dtype
    C.say(f"prefill N={c['N']} H={c['H']} Hk={c['Hk']} D={c['D']} start={c['start']} dtype={c['dtype']} "
          f"out={out_dtype} causal={causal} kernel={kernel}")
    q = C.to_dev(c["qb"], c["dtype"], device)
    k = C.to_dev(c["kb"], c["dtype"], device)
    v = C.to_dev(c["vb"], c["dtype"], device)
    out = mugen_amd.flash_prefill_attention(q, k, v, c["start"], causal=causal,
                                            out_dtype=C.torch_dtype(out_dtype), kernel=kernel)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def test_llama1b_config(device):
    # N=512, H=32, Hk=8, D=64, bf16, causal
    c = C.prefill_case(44, 512, 32, 8, 64, 0, C.BF16)
    ref = C.prefill_ref(c, nthreads=8)
    C.assert_close(run_gpu(c, device), ref, "llama-1b prefill bf16 out")
    C.assert_close(run_gpu(c, device, C.F32), ref, "llama-1b prefill f32 out")


@pytest.mark.parametrize("N,H,Hk,D,start,dtype", [
    (1, 8, 2, 64, 0, C.F16), (17, 4, 4, 128, 0, C.BF16), (40, 28, 4, 128, 100, C.F16),
    (100, 16, 2, 64, 7, C.BF16), (65, 12, 3, 64, 0, C.F16), (200, 8, 1, 128, 300, C.BF16),
    (1100, 8, 2, 128, 50, C.BF16),  # a length the planner gives the warp-specialised kernel
])
def test_shapes_and_offsets(device, N, H, Hk, D, start, dtype):
    c = C.prefill_case(50 + N, N, H, Hk, D, start, dtype)
    C.assert_close(run_gpu(c, device, C.F32), C.prefill_ref(c), f"prefill N={N} start={start}")


@pytest.mark.parametrize("dtype", [C.F16, C.BF16])
def test_default_routed_ws_16bit_out(device, dtype):
    # 1024..4096 tokens route to the warp-specialised kernel by default; G = 7
    # (Qwen2.5-7B heads) and the 16-bit output store
    c = C.prefill_case(57, 1100, 28, 4, 128, 0, dtype)
    C.assert_close(run_gpu(c, device, dtype), C.prefill_ref(c, nthreads=8), f"default-routed ws out={dtype}")


def test_non_causal(device):
    c = C.prefill_case(51, 33, 8, 2, 64, 0, C.F16)
    from oracle import oracle as O
    # non-causal == every row sees all kv_len keys == decode over the whole cache
    ref = O.gqa_attention(c["q"], c["k"].reshape(1, c["kv_len"], 2, 64).repeat(33, 0),
                          c["v"].reshape(1, c["kv_len"], 2, 64).repeat(33, 0), [c["kv_len"]] * 33, 8, 2, 64,
                          c["kv_len"] * 2 * 64)
    C.assert_close(run_gpu(c, device, C.F32, causal=False), ref, "non-causal")


def test_golden_fixture(device):
    fx = np.load(C.golden_path("prefill_small.npz"))
    c = dict(N=int(fx["N"]), H=int(fx["H"]), Hk=int(fx["Hk"]), D=int(fx["D"]), start=int(fx["start"]),
             dtype=int(fx["dtype"]), qb=fx["qb"], kb=fx["kb"], vb=fx["vb"])
    C.assert_close(run_gpu(c, device, C.F32), fx["out_f64"], "golden prefill_small")


@pytest.mark.parametrize("N,H,Hk,D,start,dtype", [
    (512, 32, 8, 64, 0, C.BF16), (40, 28, 4, 128, 100, C.F16), (200, 8, 1, 128, 300, C.BF16),
    (65, 12, 3, 64, 0, C.F16), (300, 28, 4, 128, 0, C.BF16), (33, 16, 2, 64, 5, C.BF16),
])
def test_warp_specialised_variant(device, N, H, Hk, D, start, dtype):  # forced on short prompts
    # the S / PV warp-specialised kernel (4 or 8 heads per block, G = 1, 4, 7,
    # 8), against the same oracle, with fp32 and 16-bit outputs
    c = C.prefill_case(70 + N, N, H, Hk, D, start, dtype)
    ref = C.prefill_ref(c)
    for odt in (C.F32, dtype):
        C.assert_close(run_gpu(c, device, odt, kernel=_capi.PREFILL_KERNEL_WS), ref,
                       f"ws prefill N={N} start={start} out={odt}")


def test_warp_specialised_non_causal(device):
    c = C.prefill_case(52, 33, 14, 2, 128, 0, C.BF16)
    from oracle import oracle as O
    ref = O.gqa_attention(c["q"], c["k"].reshape(1, c["kv_len"], 2, 128).repeat(33, 0),
                          c["v"].reshape(1, c["kv_len"], 2, 128).repeat(33, 0), [c["kv_len"]] * 33, 14, 2, 128,
                          c["kv_len"] * 2 * 128)
    C.assert_close(run_gpu(c, device, C.F32, causal=False, kernel=_capi.PREFILL_KERNEL_WS), ref, "ws non-causal")


@pytest.mark.parametrize("N,H,Hk,D,start,dtype", [(300, 32, 2, 128, 40, C.BF16), (129, 24, 2, 64, 0, C.F16),
                                                  (70, 16, 1, 128, 5, C.F16)])
def test_more_than_8_heads_per_kv_head(device, N, H, Hk, D, start, dtype):
    # 12 / 16 query heads per kv head: the warp-specialised kernel in slices of 8
    c = C.prefill_case(60 + H, N, H, Hk, D, start, dtype)
    ref = C.prefill_ref(c, nthreads=8)
    C.assert_close(run_gpu(c, device, C.F32), ref, f"prefill G={H // Hk}")
    C.assert_close(run_gpu(c, device, C.F32, kernel=_capi.PREFILL_KERNEL_WS), ref, f"prefill G={H // Hk} forced")
    with pytest.raises(_capi.MugenAttnError):
        run_gpu(c, device, C.F32, kernel=_capi.PREFILL_KERNEL_BLOCK)



@pytest.mark.parametrize("v_scale", [1e-3, 300.0])
def test_bf16_value_range(device, v_scale):
    # bf16 prompts run P.V in fp16 (V converted in LDS): values far below
    # and far above 1 (inside the f16 range) keep the tolerance
    c = C.prefill_case(71, 300, 28, 4, 128, 20, C.BF16)
    v = c["v"] * v_scale
    v, vb = C.O.round_to(v, C.BF16)
    c["v"], c["vb"] = v, vb
    ref = C.prefill_ref(c)
    got = run_gpu(c, device, C.F32, kernel=_capi.PREFILL_KERNEL_BLOCK)
    C.assert_close(got, ref, f"bf16 prefill V x {v_scale}", atol=2e-3 * v_scale)


@pytest.mark.parametrize("kernel", [_capi.PREFILL_KERNEL_BLOCK, _capi.PREFILL_KERNEL_WS])
def test_bf16_v_prepass(device, kernel):
    # a bf16 prompt long enough for the optional fp16 copy of V: the result
    # with the workspace equals the oracle, and the call without it
    c = C.prefill_case(72, 2100, 28, 4, 128, 0, C.BF16)
    q = C.to_dev(c["qb"], C.BF16, device)
    k = C.to_dev(c["kb"], C.BF16, device)
    v = C.to_dev(c["vb"], C.BF16, device)
    ws = mugen_amd.prefill_workspace(q, k, v, 0)
    assert ws.numel() == 2100 * 4 * 128 * 2 + 256
    C.say(f"prefill bf16 V pre-pass N=2100 kernel={kernel}")
    with_ws = mugen_amd.flash_prefill_attention(q, k, v, 0, out_dtype=torch.float32, kernel=kernel, workspace=ws)
    without = mugen_amd.flash_prefill_attention(q, k, v, 0, out_dtype=torch.float32, kernel=kernel,
                                                workspace=torch.empty(0, dtype=torch.uint8, device=device))
    torch.cuda.synchronize()
    n = 1024  # causal: the first rows depend on the first keys only
    c1 = C.prefill_case(72, 2100, 28, 4, 128, 0, C.BF16)
    ref = C.O.gqa_prefill(c1["q"][:n], c1["k"][:n], c1["v"][:n], n, 28, 4, 128, n, 0, nthreads=16)
    C.assert_close(with_ws.cpu().numpy()[:n], ref, "bf16 prefill with the fp16 V copy")
    C.assert_close(without.cpu().numpy()[:n], ref, "bf16 prefill converting V on chip")
    if kernel == _capi.PREFILL_KERNEL_BLOCK:
        # same tiles either way: only where V is converted differs
        assert torch.allclose(with_ws, without, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("N,H,Hk,start,dtype,causal", [
    (512, 32, 8, 0, C.BF16, True),    # configs[2], the largest causal range
    (300, 32, 8, 212, C.F16, True),   # a continued prompt ending at key 512
    (1, 8, 2, 0, C.BF16, True), (17, 8, 2, 3, C.F16, True), (77, 12, 3, 0, C.BF16, True),
    (130, 16, 8, 40, C.BF16, True), (33, 4, 4, 0, C.F16, True), (45, 8, 8, 450, C.BF16, True),
    (200, 32, 8, 312, C.BF16, False),  # non-causal: every row sees all 512 keys
])
def test_short_kernel(device, N, H, Hk, start, dtype, causal):
    # the short-prompt kernel (whole kv range on chip, 4 key ranges merged),
    # G = 1..4, ranges that leave key ranges empty, all output types
    c = C.prefill_case(90 + N + start, N, H, Hk, 64, start, dtype)
    if not causal:
        from oracle import oracle as O
        kv = c["kv_len"]
        ref = O.gqa_attention(c["q"], c["k"].reshape(1, kv, Hk, 64).repeat(N, 0),
                              c["v"].reshape(1, kv, Hk, 64).repeat(N, 0), [kv] * N, H, Hk, 64, kv * Hk * 64)
    else:
        ref = C.prefill_ref(c, nthreads=8)
    for odt in (C.F32, C.F16, C.BF16):
        C.assert_close(run_gpu(c, device, odt, causal=causal, kernel=_capi.PREFILL_KERNEL_SHORT), ref,
                       f"short kernel N={N} H={H} Hk={Hk} start={start} out={odt}")


def test_short_kernel_is_the_default_where_it_fits(device):
    # the automatic choice for a Llama-3.2-1B prompt of >= 384 visible keys
    # equals the forced short kernel bit for bit
    c = C.prefill_case(93, 400, 32, 8, 64, 10, C.BF16)
    assert np.array_equal(run_gpu(c, device, C.F32), run_gpu(c, device, C.F32, kernel=_capi.PREFILL_KERNEL_SHORT))


@pytest.mark.parametrize("kernel,D", [
    (_capi.PREFILL_KERNEL_BLOCK, 64), (_capi.PREFILL_KERNEL_BLOCK, 128), (_capi.PREFILL_KERNEL_WS, 64),
    (_capi.PREFILL_KERNEL_WS, 128), (_capi.PREFILL_KERNEL_SHORT, 64),  # (the short kernel: head_dim 64 only)
])
def test_climbing_scores_rebase(device, kernel, D):
    # scores that climb by > 15 log2 units per 64-key tile (key dim 0 grows
    # with the key index, q dim 0 is large), so every row's running max moves
    # on every tile and the kernels' re-base paths run throughout
    N, H, Hk = (300, 32, 8) if D == 64 else (300, 28, 4)
    c = C.prefill_case(97 + D, N, H, Hk, D, 20, C.BF16)
    q, k = c["q"].copy(), c["k"].copy()
    q[:, :, 0] = 8.0
    k[:, :, 0] = 0.5 * np.arange(c["kv_len"], dtype=np.float32)[:, None]
    c["q"], c["qb"] = C.O.round_to(q, C.BF16)
    c["k"], c["kb"] = C.O.round_to(k, C.BF16)
    C.assert_close(run_gpu(c, device, C.F32, kernel=kernel), C.prefill_ref(c), f"climbing scores D={D} kernel={kernel}")


@pytest.mark.parametrize("N", [2048, 8192])
@pytest.mark.parametrize("kernel", [_capi.PREFILL_KERNEL_AUTO, _capi.PREFILL_KERNEL_BLOCK, _capi.PREFILL_KERNEL_WS])
def test_long_range_tail(device, N, kernel):
    # the 7B prompt lengths: the last 128 query rows see all N keys, so ring
    # slots, offsets and re-base accumulation over N/64 key tiles are compared
    # with the oracle's start-offset form (query N-128+i over keys [0, N-128+i])
    H, Hk, D, t = 28, 4, 128, 128
    c = C.prefill_case(80 + N // 1024, N, H, Hk, D, 0, C.BF16)
    got = run_gpu(c, device, C.F32, kernel=kernel)
    ref = C.O.gqa_prefill(c["q"][N - t:], c["k"], c["v"], t, H, Hk, D, N, N - t, nthreads=16)
    C.assert_close(got[N - t:], ref, f"prefill tail N={N} kernel={kernel}")
    head = C.O.gqa_prefill(c["q"][:64], c["k"][:64], c["v"][:64], 64, H, Hk, D, 64, 0, nthreads=16)
    C.assert_close(got[:64], head, f"prefill head N={N} kernel={kernel}")
