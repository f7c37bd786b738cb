"""head_dim other than 64 / 128 (multiples of 8 up to 128: the reference's
cpu_attention takes any head_dim, transformer.cpp:2441-2485; its unit-test
model uses 16).  The kernels run on the next supported width with the extra
dims masked, so these check both the results (against the oracle) and that
nothing is written past the head_dim-wide output rows (canary guard bands
around the outputs)."""
import numpy as np
import pytest
import torch

import mugen_amd
from mugen_amd import _capi
from tests import cases as C
from tests.test_bounds_gpu import Guarded

pytestmark = pytest.mark.gpu

HEAD_DIMS = [8, 16, 32, 48, 80, 96, 120]


@pytest.mark.parametrize("D", HEAD_DIMS)
def test_decode_head_dim(device, D):
    lens = [1, 700, 0, 333]
    for dt in (C.F16, C.BF16):
        c = C.gqa_decode_case(900 + D, 4, 8, 2, D, lens, max_T=1024, dtype=dt)
        ref = C.gqa_decode_ref(c)
        q = C.to_dev(c["qb"], dt, device)
        k = C.to_dev(c["kb"], dt, device)
        v = C.to_dev(c["vb"], dt, device)
        sl = torch.from_numpy(c["seq_lens"]).to(device)
        for splits in (0, 1, 5):
            C.say(f"gqa_decode head_dim={D} dtype={dt} splits={splits}")
            out = Guarded((4, 8, D), torch.float32, device)
            mugen_amd.attention_decode(q, k, v, sl, 1024, out=out.t, num_splits=splits)
            assert out.intact(), f"guard band overwritten (D={D}, splits={splits})"
            C.assert_close(out.t.cpu().numpy(), ref, f"decode head_dim={D} dtype={dt} splits={splits}")


@pytest.mark.parametrize("D", HEAD_DIMS)
def test_prefill_head_dim(device, D):
    N, start = 150, 40
    for dt in (C.BF16, C.F16):
        c = C.prefill_case(950 + D, N, 12, 3, D, start, dt)
        ref = C.prefill_ref(c)
        q = C.to_dev(c["qb"], dt, device)
        k = C.to_dev(c["kb"], dt, device)
        v = C.to_dev(c["vb"], dt, device)
        for kernel in (_capi.PREFILL_KERNEL_BLOCK, _capi.PREFILL_KERNEL_WS):
            C.say(f"gqa_prefill head_dim={D} dtype={dt} kernel={kernel}")
            out = Guarded((N, 12, D), torch.float32, device)
            mugen_amd.flash_prefill_attention(q, k, v, start, out=out.t, kernel=kernel)
            assert out.intact(), f"guard band overwritten (D={D}, kernel={kernel})"
            C.assert_close(out.t.cpu().numpy(), ref, f"prefill head_dim={D} dtype={dt} kernel={kernel}")


def test_reference_unit_test_model(device):
    # the reference's test model: 4 heads, 2 KV heads, head_dim 16
    c = C.gqa_decode_case(977, 1, 4, 2, 16, [37], dtype=C.F16)
    out = mugen_amd.attention_decode(C.to_dev(c["qb"], C.F16, device), C.to_dev(c["kb"], C.F16, device),
                                     C.to_dev(c["vb"], C.F16, device), torch.from_numpy(c["seq_lens"]).to(device),
                                     c["max_T"], out_dtype=torch.float32)
    torch.cuda.synchronize()
    C.assert_close(out.cpu().numpy(), C.gqa_decode_ref(c), "head_dim 16 model")
    p = C.prefill_case(978, 37, 4, 2, 16, 0, C.F16)
    got = mugen_amd.flash_prefill_attention(C.to_dev(p["qb"], C.F16, device), C.to_dev(p["kb"], C.F16, device),
                                            C.to_dev(p["vb"], C.F16, device), 0, out_dtype=torch.float32)
    torch.cuda.synchronize()
    C.assert_close(got.cpu().numpy(), C.prefill_ref(p), "head_dim 16 prompt")
    assert np.isfinite(got.cpu().numpy()).all()
