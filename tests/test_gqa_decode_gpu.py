"""GQA decode on the GPU vs the CPU oracle (cpu_attention restatement)."""
import numpy as np
import pytest
import torch

import mugen_amd
from oracle import oracle as O
from tests import cases as C

pytestmark = pytest.mark.gpu


def run_gpu(c, device, out_dtype=C.F32, num_splits=0):
    C.say(f"gqa_decode B={c['B']} H={c['H']} Hk={c['Hk']} D={c['D']} maxT={c['max_T']} "
          f"dtype={c['dtype']} out={out_dtype} splits={num_splits}")
    q = C.to_dev(c["qb"], c["dtype"], device)
    k = C.to_dev(c["kb"], c["dtype"], device)
    v = C.to_dev(c["vb"], c["dtype"], device)
    sl = torch.from_numpy(c["seq_lens"]).to(device)
    out = mugen_amd.attention_decode(q, k, v, sl, c["max_T"], out_dtype=C.torch_dtype(out_dtype),
                                     num_splits=num_splits)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def test_qwen7b_b1_ctx4096(device):
    c = C.gqa_decode_case(43, 1, 28, 4, 128, [4096], dtype=C.F16)
    ref = C.gqa_decode_ref(c, nthreads=8)
    for od in (C.F16, C.F32):
        C.assert_close(run_gpu(c, device, od), ref, f"qwen7b b1 out={od}")


def test_qwen7b_b16_ragged(device):
    lens = O.randint(44, 16, 256, 4096)
    c = C.gqa_decode_case(44, 16, 28, 4, 128, lens, max_T=4096, dtype=C.F16)
    ref = C.gqa_decode_ref(c, nthreads=8)
    C.assert_close(run_gpu(c, device, C.F32), ref, "qwen7b b16 ragged")


@pytest.mark.parametrize("H,Hk,D,dtype", [
    (4, 4, 64, C.F16), (8, 4, 128, C.BF16), (32, 8, 64, C.BF16), (28, 4, 64, C.F16),
    (16, 2, 128, C.F16), (16, 1, 128, C.BF16), (12, 4, 128, C.F16), (20, 4, 64, C.BF16),
])
def test_head_groups_and_edges(device, H, Hk, D, dtype):
    lens = [0, 1, 15, 16, 17, 63, 64, 65, 100, 257]
    c = C.gqa_decode_case(45 + H, len(lens), H, Hk, D, lens, dtype=dtype)
    ref = C.gqa_decode_ref(c)
    for splits in (0, 1, 3):
        got = run_gpu(c, device, C.F32, splits)
        C.assert_close(got, ref, f"H={H} Hk={Hk} D={D} splits={splits}")
    assert np.all(got[0] == 0.0)  # seq_len 0 -> zeros


def test_split_count_invariance(device):
    c = C.gqa_decode_case(46, 2, 28, 4, 128, [3000, 1777], dtype=C.F16)
    outs = [run_gpu(c, device, C.F32, s) for s in (1, 0, 7, 40)]
    # fp16 softmax weights on MFMA: each split rounds its own P (relative 2^-12)
    for o in outs[1:]:
        C.say(f"split invariance max diff {np.abs(o - outs[0]).max():.2e}")
        np.testing.assert_allclose(o, outs[0], atol=1e-4, rtol=1e-3)


def test_golden_fixture(device):
    fx = np.load(C.golden_path("gqa_decode_small.npz"))
    c = dict(B=int(fx["B"]), H=int(fx["H"]), Hk=int(fx["Hk"]), D=int(fx["D"]), max_T=int(fx["max_T"]),
             dtype=int(fx["dtype"]), qb=fx["qb"], kb=fx["kb"], vb=fx["vb"], seq_lens=fx["seq_lens"])
    C.assert_close(run_gpu(c, device, C.F32), fx["out_f64"], "golden gqa_decode_small")


@pytest.mark.parametrize("D", [64, 128])
def test_more_than_64_splits(device, D):
    # 64-token splits over 8192 and 5000 tokens: 128 and 79 splits, past the
    # combine's one-load-per-lane weights (<= 64), so the block-wide
    # log-sum-exp weights run
    c = C.gqa_decode_case(47 + D, 2, 28, 4, D, [8192, 5000], dtype=C.F16)
    ref = C.gqa_decode_ref(c, nthreads=8)
    C.assert_close(run_gpu(c, device, C.F32, 200), ref, f"gqa decode D={D} 128 / 79 splits")
