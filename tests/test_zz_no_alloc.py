"""mugen_attn_mla_decode_noalloc, called through the C ABI: the same
results as mugen_attn_mla_decode with a caller workspace, on two calls in a
row (the second smaller, so stale scratch contents from the first must not
leak into it), and a clear error for a call that needs more than the fixed
scratch.  The fixed scratch is shared by every call on the GPU."""
import ctypes

import numpy as np
import pytest
import torch

from mugen_amd import _capi
from mugen_amd import attention as A
from tests import cases as C

pytestmark = pytest.mark.gpu


def _call(c, device, noalloc):
    q = C.to_dev(c["q"] if c["q_dtype"] == C.F32 else c["qb"], c["q_dtype"], device)
    lat = C.to_dev(c["latb"], c["lat_dtype"], device)
    sl = torch.from_numpy(c["seq_lens"]).to(device)
    out = torch.full((c["B"], c["q_len"], c["H"], 512), float("nan"), dtype=torch.float32, device=device)
    a = A.mla_args(q, lat, sl, out, c["max_T"], C.MLA_SCALE)
    L = _capi.lib()
    if noalloc:
        rc = L.mugen_attn_mla_decode_noalloc(ctypes.byref(a), A._stream(device))
    else:
        need = L.mugen_attn_mla_decode_workspace_size(ctypes.byref(a))
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=device)
        rc = L.mugen_attn_mla_decode(ctypes.byref(a), ctypes.c_void_p(ws.data_ptr()), need, A._stream(device))
    _capi.check(rc)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_noalloc_matches_workspace_entry_point(device):
    big = C.mla_case(601, 8, 1, 128, np.array([7651, 5132, 6268, 4812, 4836, 6498, 6085, 6843]), max_T=8192,
                     q_dtype=C.BF16, lat_dtype=C.BF16)
    small = C.mla_case(602, 2, 3, 16, [900, 40], q_dtype=C.F32, lat_dtype=C.F16)
    for name, c in (("v3 decode", big), ("smaller second call", small)):
        C.say(f"noalloc {name}: B={c['B']} q_len={c['q_len']} H={c['H']}")
        ref = _call(c, device, noalloc=False)
        got = _call(c, device, noalloc=True)
        # same kernels, same plan: bit-identical to the workspace entry point
        assert np.array_equal(got, ref), f"{name}: max diff {np.nanmax(np.abs(got - ref))}"
        C.assert_close(got, C.mla_ref(c, nthreads=16), f"noalloc {name} vs oracle")


def test_noalloc_rejects_calls_beyond_the_scratch(device):
    # 64 sequences of 32768 tokens in 64 splits each need more partial space
    # than the scratch
    B, T, H = 64, 32768, 128
    q = torch.zeros((B, 1, H, 576), dtype=torch.bfloat16, device=device)
    lat = torch.zeros((1, 576), dtype=torch.bfloat16, device=device)  # never read: the call is refused
    sl = torch.full((B,), T, dtype=torch.int32, device=device)
    out = torch.empty((B, 1, H, 512), dtype=torch.float32, device=device)
    a = A.mla_args(q, lat, sl, out, T, C.MLA_SCALE)
    a.seq_stride = T * 576  # a valid layout; the buffer is never read
    a.num_splits = 64
    assert _capi.lib().mugen_attn_mla_decode_workspace_size(ctypes.byref(a)) > _capi.MLA_SCRATCH_BYTES
    rc = _capi.lib().mugen_attn_mla_decode_noalloc(ctypes.byref(a), A._stream(device))
    assert rc == -3 and "fixed scratch" in _capi.lib().mugen_attn_last_error().decode()
