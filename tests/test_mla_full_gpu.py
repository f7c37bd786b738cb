"""MLA absorption, up-projection and the whole cpu_mla_attention operator
(transformer.cpp:2539-2623) on the GPU vs the CPU oracle, for each weight
encoding the reference dequantises (F16, Q8_0, Q4_0).

Tolerance: the path's stated atol 2e-3 + rtol 1e-2 (fp32 arithmetic on both
sides; the kernels sum in a different order and the operator's output is
rounded to f16, one f16 ulp being 2^-11 relative)."""
import numpy as np
import pytest
import torch

import mugen_amd
from oracle import oracle as O
from tests import cases as C

pytestmark = pytest.mark.gpu

WTYPES = [O.W_F16, O.W_Q8_0, O.W_Q4_0]
WNAME = {O.W_F16: "f16", O.W_Q8_0: "q8_0", O.W_Q4_0: "q4_0"}


def wdev(w, w_type, device):
    t = torch.from_numpy(np.ascontiguousarray(w)).to(device)
    return t.view(torch.float16) if w_type == O.W_F16 else t


def qdev(qb, device):
    return C.to_dev(qb, C.F16, device)


# rows >= 64 take the MFMA forms (bf16 hi / lo splits), fewer the VALU kernels
ROWS_H = [(1, 16), (8, 128), (37, 3), (64, 16), (77, 3), (512, 16)]


@pytest.mark.parametrize("w_type", WTYPES)
@pytest.mark.parametrize("rows,H", ROWS_H)
def test_absorb(device, w_type, rows, H):
    q, qb = O.round_to(O.randn(100 + rows, (rows, H, 192)), C.F16)
    q[0, 0, :40] = 0.0          # zero terms, skipped by the reference
    q, qb = O.round_to(q, C.F16)
    w = C.make_weights(200 + H, H * 128, 512, w_type)
    C.say(f"absorb rows={rows} H={H} w={WNAME[w_type]}")
    got = mugen_amd.mla_absorb(qdev(qb, device), wdev(w, w_type, device), WNAME[w_type])
    torch.cuda.synchronize()
    ref = O.mla_absorb(q, w, w_type, H)
    C.assert_close(got.cpu().numpy(), ref, f"absorb {WNAME[w_type]}")
    np.testing.assert_array_equal(got[..., 512:].cpu().numpy(), q[..., 128:])  # q_rope passes unchanged
    gb = mugen_amd.mla_absorb(qdev(qb, device), wdev(w, w_type, device), WNAME[w_type], out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    C.assert_close(gb.float().cpu().numpy(), ref, f"absorb bf16 out {WNAME[w_type]}", rtol=1e-2, atol=2e-2)


@pytest.mark.parametrize("w_type", WTYPES)
@pytest.mark.parametrize("rows,H", ROWS_H)
def test_project(device, w_type, rows, H):
    o = O.randn(300 + rows, (rows, H, 512), 0.0, 0.3)
    w = C.make_weights(400 + H, H * 128, 512, w_type)
    C.say(f"project rows={rows} H={H} w={WNAME[w_type]}")
    od = torch.from_numpy(o).to(device)
    got = mugen_amd.mla_project(od, wdev(w, w_type, device), WNAME[w_type])
    got32 = mugen_amd.mla_project(od, wdev(w, w_type, device), WNAME[w_type], out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = O.mla_project(o, w, w_type, H)  # f16-rounded, as the reference's output
    C.assert_close(got.float().cpu().numpy(), ref, f"project {WNAME[w_type]}")
    C.assert_close(got32.cpu().numpy(), ref, f"project f32 out {WNAME[w_type]}")


@pytest.mark.parametrize("w_type", WTYPES)
@pytest.mark.parametrize("B,q_len,H,lens", [
    (1, 1, 16, [1024]),          # configs[0] shape (V2-Lite heads) end to end
    (3, 2, 20, [2, 700, 129]),
    (2, 5, 128, [1500, 5]),      # verify rows, V3 heads
    (1, 64, 16, [300]),          # a prompt chunk: absorb / project on MFMA
])
def test_full_operator(device, w_type, B, q_len, H, lens):
    c = C.mla_full_case(500 + H + q_len, B, q_len, H, lens, w_type)
    C.say(f"mla full B={B} q_len={q_len} H={H} lens={lens} w={WNAME[w_type]}")
    got = mugen_amd.mla_attention_full(qdev(c["qb"], device), wdev(c["w_kb"], w_type, device),
                                       wdev(c["w_vb"], w_type, device), C.to_dev(c["latb"], C.F16, device),
                                       torch.from_numpy(c["seq_lens"]).to(device), c["max_T"], WNAME[w_type],
                                       scale=C.MLA_SCALE)
    torch.cuda.synchronize()
    assert got.dtype == torch.float16 and got.shape == (B, q_len, H, 128)
    C.assert_close(got.float().cpu().numpy(), C.mla_full_ref(c, nthreads=8), f"mla full {WNAME[w_type]}")


def test_absorb_rope_matches_across_forms(device):
    """The q RoPE stage of the MFMA form (100 rows) equals the VALU form's
    (the same rows absorbed 8 at a time) bit for bit, and q_abs agrees."""
    rows, H = 100, 16
    q, qb = O.round_to(O.randn(77, (rows, H, 192)), C.F16)
    w = C.make_weights(78, H * 128, 512, O.W_Q8_0)
    pos = torch.arange(900, 900 + rows, dtype=torch.int32, device=device)
    rope = (10000.0, 40.0, 4096)
    C.say("absorb rope MFMA vs VALU forms")
    qd, wd = qdev(qb, device), wdev(w, O.W_Q8_0, device)
    big = mugen_amd.mla_absorb(qd, wd, "q8_0", positions=pos, rope=rope)
    parts = [mugen_amd.mla_absorb(qd[i:i + 8], wd, "q8_0", positions=pos[i:i + 8], rope=rope)
             for i in range(0, rows, 8)]
    small = torch.cat(parts)
    torch.cuda.synchronize()
    assert torch.equal(big[..., 512:], small[..., 512:])
    C.assert_close(big[..., :512].cpu().numpy(), small[..., :512].cpu().numpy(), "q_abs MFMA vs VALU")


@pytest.mark.parametrize("w_type", [O.W_Q8_0, O.W_Q4_0])
def test_two_byte_aligned_weights(device, w_type):
    """Block-encoded weights need only 2-byte alignment, also in the MFMA
    forms (96 rows)."""
    rows, H = 96, 4
    q, qb = O.round_to(O.randn(91, (rows, H, 192)), C.F16)
    w = C.make_weights(92, H * 128, 512, w_type)
    buf = torch.zeros(w.size + 2, dtype=torch.uint8, device=device)
    buf[2:] = torch.from_numpy(w.reshape(-1)).to(device)
    wd = buf[2:].view(w.shape)
    assert wd.data_ptr() % 4 == 2
    C.say(f"absorb / project with 2-byte aligned {WNAME[w_type]} weights")
    got = mugen_amd.mla_absorb(qdev(qb, device), wd, WNAME[w_type])
    o = O.randn(93, (rows, H, 512), 0.0, 0.3)
    gp = mugen_amd.mla_project(torch.from_numpy(o).to(device), wd, WNAME[w_type], out_dtype=torch.float32)
    torch.cuda.synchronize()
    C.assert_close(got.cpu().numpy(), O.mla_absorb(q, w, w_type, H), "absorb, 2-byte aligned weights")
    C.assert_close(gp.cpu().numpy(), O.mla_project(o, w, w_type, H), "project, 2-byte aligned weights")


def test_zero_rows_is_a_no_op(device):
    q = torch.empty((0, 4, 192), dtype=torch.float16, device=device)
    w = torch.zeros((4 * 128, 512), dtype=torch.float16, device=device)
    assert mugen_amd.mla_absorb(q, w).shape == (0, 4, 576)
    o = torch.empty((0, 4, 512), dtype=torch.float32, device=device)
    assert mugen_amd.mla_project(o, w).shape == (0, 4, 128)
